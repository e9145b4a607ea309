"""The Swift seam (ltx-2.5-swift_amd/swift/): what can be checked without a Swift toolchain.

* The SwiftPM C target CLTXHip compiles against the library's header and the HIP runtime
  headers, with warnings as errors.
* Every C function, type and constant the Swift sources use is declared by ltx_attn.h or
  CLTXHip.h, and every CLTXHip function is defined by cltx_hip.c.
* The patches to the reference's sources only add lines (no reference source is carried in
  them) and, where the reference checkout is present, apply cleanly with `git apply
  --unidiff-zero`. After patching:
  - every `switch` that gained a `case .hip:` switches over a value whose enum declares
    `case hip` (the value's type is resolved from its declaration: a stored property, a
    parameter, or a function's return type), and so does every `return .hip`;
  - Machine.swift, read for a host without Darwin (an MI355X's Linux host), keeps no Darwin-
    only call, and read for Darwin is the reference's code unchanged;
  - the renderer admits the HIP path's memory plan before it loads the transformer, and
    selects the text encoder's .hip path with the DiT's;
  - the text encoder's .hip route is taken before its MLX arithmetic and hands the kernel the
    layer's own weights.
* HIPMemoryPlan's six calls are the block's six attentions (DiTBlock.swift:343-438) with the
  shapes and rotary tables the model gives them.
"""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWIFT = os.path.join(ROOT, "ltx-2.5-swift_amd", "swift")
CTARGET = os.path.join(SWIFT, "Sources", "CLTXHip")
HEADER = os.path.join(ROOT, "include", "ltx_attn.h")
PATCHES = os.path.join(SWIFT, "patches")
REFERENCE = "/root/reference"
PATCHED_FILES = ("Sources/LTXModules/DiTAttention.swift",
                 "Sources/LTXModules/GemmaTextEncoder.swift",
                 "Sources/LTXPipeline/Renderer.swift", "Sources/ltx/BenchForward.swift")


def _swift_sources():
    out = []
    for d, _, files in os.walk(os.path.join(SWIFT, "Sources")):
        out += [os.path.join(d, f) for f in files if f.endswith(".swift")]
    return sorted(out)


def test_c_target_compiles(tmp_path):
    src = os.path.join(CTARGET, "cltx_hip.c")
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", "-I" + os.path.dirname(HEADER),
                    "-I" + os.path.join(CTARGET, "include"), "-c", src,
                    "-o", str(tmp_path / "cltx_hip.o")], check=True)


def test_modulemap_exports_the_umbrella_header_and_links_the_library():
    text = open(os.path.join(CTARGET, "include", "module.modulemap")).read()
    assert re.search(r"module\s+CLTXHip\s*\{", text)
    assert 'umbrella header "CLTXHip.h"' in text
    assert 'link "ltx_attn"' in text


def test_swift_uses_only_declared_c_symbols():
    decl = open(HEADER).read() + open(os.path.join(CTARGET, "include", "CLTXHip.h")).read()
    impl = open(os.path.join(CTARGET, "cltx_hip.c")).read()
    used = set()
    for path in _swift_sources():
        used |= set(re.findall(r"\b((?:ltx|cltx)_\w+|LTX_ATTN_\w+)\b", open(path).read()))
    assert {"ltx_attn_fwd", "ltx_attn_workspace_bytes", "ltx_device_query", "cltx_alloc",
            "ltx_gemma_attn_fwd", "cltx_host_alloc", "cltx_mem_info"} <= used
    for name in sorted(used):
        assert re.search(rf"\b{name}\b", decl), f"{name} is not declared"
        if name.startswith("cltx_"):
            assert re.search(rf"\b{name}\s*\(", impl), f"{name} is not defined"


def test_no_per_call_allocation_in_the_model_paths():
    """The .hip paths take their operands through the context's arenas and workspace (grown
    only when a call is larger than any before it), never a fresh buffer per call."""
    for name in ("DiTAttention+HIP.swift", "GemmaTextEncoder+HIP.swift"):
        text = open(os.path.join(SWIFT, "Sources", "LTXModules", name)).read()
        assert "ctx.arenas(" in text and "ctx.upload(" in text and "ctx.download(" in text
        assert "HIPBuffer(" not in text and "cltx_alloc" not in text, name


def test_patches_only_add_lines():
    names = sorted(f for f in os.listdir(PATCHES) if f.endswith(".patch"))
    assert len(names) == 6
    for n in names:
        for line in open(os.path.join(PATCHES, n)).read().splitlines():
            if line.startswith(("---", "+++", "@@", "+")):
                continue
            raise AssertionError(f"{n}: non-additive line {line!r}")


# ---------------------------------------------------------------------------------------
# Light Swift reading: enums, declarations, #if branches
# ---------------------------------------------------------------------------------------

def _enum_cases(tree, qualified):
    """Cases of enum `Outer.Name` (or `Name` searched everywhere) in the patched tree."""
    outer, _, name = qualified.rpartition(".")
    found = []
    for d, _, files in os.walk(tree / "Sources"):
        for f in files:
            if not f.endswith(".swift"):
                continue
            text = open(os.path.join(d, f)).read()
            if outer and not re.search(rf"\b(?:struct|class|enum|extension)\s+{outer}\b", text):
                continue
            for m in re.finditer(rf"\benum\s+{name}\b[^{{]*\{{", text):
                depth, i = 1, m.end()
                while depth:
                    depth += {"{": 1, "}": -1}.get(text[i], 0)
                    i += 1
                found.append(re.findall(r"^\s*case\s+(\w+)", text[m.end():i], re.M))
    assert len(found) == 1, (qualified, len(found))
    return found[0]


def _enclosing_type(text, pos):
    """Name of the innermost struct/class/enum whose body contains `pos`."""
    best = None
    for m in re.finditer(r"\b(?:struct|class|enum|actor)\s+(\w+)[^{]*\{", text):
        if m.start() > pos:
            break
        depth, i = 1, m.end()
        while depth and i < len(text):
            depth += {"{": 1, "}": -1}.get(text[i], 0)
            i += 1
        if i > pos:
            best = m.group(1)
    return best


def _type_of(text, var, pos):
    """The declared type of `var` as seen at `pos`: the nearest preceding declaration
    (`var/let var: T`, or a parameter `var: T` / `_ var: T`)."""
    decls = [m for m in re.finditer(rf"(?:\b(?:var|let)\s+|[(,]\s*(?:_\s+)?){var}\s*:\s*"
                                    r"([\w.]+)", text) if m.start() < pos]
    assert decls, (var, pos)
    return decls[-1].group(1)


def _qualify(text, typ, pos):
    if "." in typ:
        return typ
    owner = _enclosing_type(text, pos)
    if re.search(rf"\benum\s+{typ}\b", text) and owner:
        return f"{owner}.{typ}"
    return typ


def _resolved_hip_uses(tree):
    """(file, what, enum) for every `switch v {` with a `case .hip:` and every `return .hip`."""
    out = []
    for rel in PATCHED_FILES:
        text = (tree / rel).read_text()
        for m in re.finditer(r"\bswitch\s+(\w+)\s*\{", text):
            depth, i = 1, m.end()
            while depth:
                depth += {"{": 1, "}": -1}.get(text[i], 0)
                i += 1
            if "case .hip:" not in text[m.end():i]:
                continue
            typ = _qualify(text, _type_of(text, m.group(1), m.start()), m.start())
            out.append((rel, f"switch {m.group(1)}", typ))
        for m in re.finditer(r"return\s+\.hip\b", text):
            sig = [f for f in re.finditer(r"func\s+\w+\([^)]*\)[^{]*->\s*([\w.]+)", text)
                   if f.start() < m.start()][-1]
            out.append((rel, "return .hip", _qualify(text, sig.group(1), m.start())))
    return out


def _if_branch(text, darwin):
    """`text` with every `#if canImport(Darwin)` block resolved for a Darwin (or not) host."""
    out, stack = [], []
    for line in text.splitlines():
        s = line.strip()
        if s.startswith("#if "):
            assert s == "#if canImport(Darwin)", s
            stack.append(darwin)
            continue
        if s == "#else":
            stack[-1] = not stack[-1]
            continue
        if s == "#endif":
            stack.pop()
            continue
        if all(stack):
            out.append(line)
    assert not stack
    return "\n".join(out)


def _patched(tmp_path):
    for rel in ("Sources", "Package.swift"):
        src = os.path.join(REFERENCE, rel)
        (shutil.copytree if os.path.isdir(src) else shutil.copy)(src, tmp_path / rel)
    for n in sorted(os.listdir(PATCHES)):
        subprocess.run(["git", "apply", "--unidiff-zero", os.path.join(PATCHES, n)],
                       cwd=tmp_path, check=True)
    # the package's own Swift sources, as a maintainer adds them
    for d, _, files in os.walk(os.path.join(SWIFT, "Sources")):
        for f in files:
            if f.endswith(".swift"):
                rel = os.path.relpath(os.path.join(d, f), SWIFT)
                shutil.copy(os.path.join(d, f), tmp_path / rel)
    return tmp_path


needs_reference = pytest.mark.skipif(not os.path.isdir(REFERENCE),
                                     reason="reference checkout not present")


@needs_reference
def test_every_hip_case_names_a_hip_enum_case(tmp_path):
    tree = _patched(tmp_path)
    uses = _resolved_hip_uses(tree)
    # DiTAttention's switch over its path, the renderer's provenance, the text encoder's
    # switch, the bench's option parser
    assert {(rel, typ) for rel, _, typ in uses} == {
        ("Sources/LTXModules/DiTAttention.swift", "DiTAttention.AttentionPath"),
        ("Sources/LTXModules/GemmaTextEncoder.swift", "GemmaTextEncoder.AttentionPath"),
        ("Sources/LTXPipeline/Renderer.swift", "DiTAttention.AttentionPath"),
        ("Sources/ltx/BenchForward.swift", "DiTAttention.AttentionPath"),
    }, uses
    for rel, what, typ in uses:
        assert "hip" in _enum_cases(tree, typ), (rel, what, typ)
    assert _enum_cases(tree, "DiTAttention.AttentionPath") == ["fused", "explicit", "hip"]
    assert _enum_cases(tree, "GemmaTextEncoder.AttentionPath") == ["fused", "explicit", "hip"]


@needs_reference
def test_the_enum_check_fails_without_the_gemma_enum_case(tmp_path):
    """The check above can fail: with the text encoder's enum case taken out of the patched
    tree (as a patch that only adds the switch case would leave it), the switch's enum has no
    `hip`."""
    tree = _patched(tmp_path)
    path = tree / "Sources/LTXModules/GemmaTextEncoder.swift"
    text = path.read_text()
    i = text.index("case hip")
    path.write_text(text[:i] + "// (removed)" + text[i + len("case hip"):])
    uses = [u for u in _resolved_hip_uses(tree) if "Gemma" in u[0]]
    assert uses and all("hip" not in _enum_cases(tree, typ) for _, _, typ in uses)


@needs_reference
def test_machine_builds_without_darwin(tmp_path):
    tree = _patched(tmp_path)
    text = (tree / "Sources/LTXHardware/Machine.swift").read_text()
    linux = _if_branch(text, darwin=False)
    code = re.sub(r"//.*", "", linux)                      # calls, not comments
    for darwin_only in ("import Darwin", "sysctlbyname", "host_statistics64", "mach_host_self",
                        "vm_statistics64", "HOST_VM_INFO64", "KERN_SUCCESS", "integer_t"):
        assert darwin_only not in code, darwin_only
    for api in ("static func detect()", "static func availableBytes()", "MemAvailable"):
        assert api in linux, api
    # on Darwin the reference's own code, unchanged
    ref = open(os.path.join(REFERENCE, "Sources/LTXHardware/Machine.swift")).read()
    assert _if_branch(text, darwin=True).strip() == ref.strip()
    # nothing else in the targets below the MLX line imports Darwin
    for target in ("LTXFoundation", "LTXHardware", "LTXCatalog", "LTXRecipes"):
        for d, _, files in os.walk(tree / "Sources" / target):
            for f in files:
                if f.endswith(".swift"):
                    body = _if_branch(open(os.path.join(d, f)).read(), darwin=False)
                    assert "import Darwin" not in body, (target, f)


@needs_reference
def test_renderer_selects_and_admits_before_loading(tmp_path):
    tree = _patched(tmp_path)
    text = (tree / "Sources/LTXPipeline/Renderer.swift").read_text()
    render = text[text.index("public static func render(spec:"):]
    admit, load = render.index("HIPMemoryPlan.admit("), render.index("MLX.loadArrays(")
    assert admit < load
    assert "videoTokensWithReference" in render[admit:load]
    cond = text[text.index("public static func conditioning(spec:"):]
    sel = cond.index("text.encoder.attentionPath = .hip")
    assert cond.index("TextConditioningPipeline(") < sel < cond.index("text(prompt:")
    pkg = (tree / "Package.swift").read_text()
    assert '"CLTXHip"' in pkg and 'target.name == "LTXPipeline"' in pkg


@needs_reference
def test_text_encoder_route(tmp_path):
    tree = _patched(tmp_path)
    text = (tree / "Sources/LTXModules/GemmaTextEncoder.swift").read_text()
    body = text[text.index("private func attention("):text.index("private func feedForward(")]
    route = body.index("if attentionPath == .hip")
    assert route < body.index("// Q: project -> q_norm -> RoPE.")
    for w in ("q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj"):
        assert f'"{w}.weight"' in body[route:route + 900], w
    states = text[text.index("public func hiddenStates("):]
    assert states.index("HIPGemmaCore.leftPadding(tokenWeights)") < states.index("for layer in")


def test_memory_plan_calls_are_the_block_calls():
    """HIPMemoryPlan.blockCalls lists the six attentions in block order with the model's
    head dims and tables: attn1 / audio_attn1 rotate their queries (and keys with the same
    tables), the text calls take none, the cross-modal calls take both."""
    text = open(os.path.join(SWIFT, "Sources", "LTXHardware", "HIPMemoryPlan.swift")).read()
    text = re.sub(r"\s+", " ", text)
    calls = re.findall(r'Call\(name: "(\w+)", batch: batch, heads: 32, headDim: (\d+), '
                       r'queryTokens: (\w+), keyTokens: (\w+), queryRotary: (\w+), '
                       r'keyRotary: (\w+)\)', text)
    assert calls == [
        ("attn1", "128", "videoTokens", "videoTokens", "true", "false"),
        ("audio_attn1", "64", "audioTokens", "audioTokens", "true", "false"),
        ("attn2", "128", "videoTokens", "textTokens", "false", "false"),
        ("audio_attn2", "64", "audioTokens", "textTokens", "false", "false"),
        ("audio_to_video_attn", "64", "videoTokens", "audioTokens", "true", "true"),
        ("video_to_audio_attn", "64", "audioTokens", "videoTokens", "true", "true"),
    ]
