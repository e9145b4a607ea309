#!/usr/bin/env python3
"""Build-time check of the hand-placed MFMA hazard padding in fmha_dma.hip.

The S products of the LDS-DMA kernel are inline assembly (`; mfma_s <dst> src <srcC>`), so
the compiler's hazard recognizer does not see them as MFMAs. The source pads them itself;
this script verifies, on the compiler's output, that the padding holds wherever the
register allocator and scheduler put things:

  * after an S product, no instruction touches its result registers for RESULT_WAIT wait
    states, except the next product of the same chain (an MFMA whose SrcC is exactly that
    result, which the hardware forwards);
  * after an S product whose SrcC is not its own result, no VALU instruction writes that
    SrcC for RESULT_WAIT wait states (the MFMA reads SrcC over its passes; loads write their
    VGPRs only when the data returns, tens of cycles later, so they are not restricted);
  * no VALU instruction writes an input of an S product (A, B or SrcC register) fewer than
    INPUT_WAIT wait states before it (a label counts as a write of every register);
  * no result is still inside its window at a label or a branch (the padding never relies
    on one particular path).

It also rejects any kernel of the file that spills to scratch memory (`.private_seg_size`
above 0): the kernels are laid out to fit the register file, and a spill would otherwise
only show as a slowdown.

Wait states: each instruction counts one, `s_nop N` counts N + 1.

    python check_mfma_hazards.py <device assembly .s>     (exit status 1 on a violation)
"""
import re
import sys

RESULT_WAIT = 20   # XDL result -> any other access; the padding provides 8 + 8 + 4
INPUT_WAIT = 2     # VALU write of an input -> MFMA read

REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")


def regs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(1):
            out.update((m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def check(lines, name):
    errors = []
    pending = []           # [registers, remaining wait states, what, line]
    tag = None             # registers named by the most recent `; mfma_s` comment
    since = {}             # register -> wait states since its last VALU write
    fresh = 0              # wait states since the last label (a write of every register)
    for no, raw in enumerate(lines, 1):
        line = raw.strip()
        m = re.match(r";\s*mfma_s\s+(\S+)\s+src\s+(\S+)", line)
        if m:
            tag = (regs(m.group(1)), regs(m.group(2)))
            continue
        if not line or line.startswith(";") or line.startswith("."):
            continue
        if line.endswith(":"):                      # a label: nothing may be pending
            for p in pending:
                errors.append(f"{name}:{p[3]}: {p[2]} still within its window at label line {no}")
            pending = []
            since = {}
            fresh = 0
            continue
        op = line.split()[0]
        body = line[len(op):].split(";")[0]
        waits = int(body.strip() or 0) + 1 if op == "s_nop" else 1
        touched = regs(body)
        if op.startswith("s_cbranch") or op == "s_branch" or op == "s_setpc_b64":
            for p in pending:
                errors.append(f"{name}:{p[3]}: {p[2]} still within its window at branch line {no}")
            pending = []
        if op.startswith("v_mfma") and tag is not None:
            dst, src = tag
            inputs = regs(",".join(body.split(",")[1:]))
            near = [r for r in inputs if min(since.get(r, 1 << 30), fresh) < INPUT_WAIT]
            if near:
                errors.append(f"{name}:{no}: input {near[0]} written by VALU fewer than "
                              f"{INPUT_WAIT} wait states before an S product")
            keep = []
            for p in pending:
                if p[2].startswith("result") and p[0] == dst and src == dst:
                    continue                          # chain: forwarded SrcC
                if p[2].startswith("srcC"):
                    keep.append(p)                    # another product reading it is fine
                    continue
                if p[0] & touched:
                    errors.append(f"{name}:{no}: S product touches {p[2]} of line {p[3]}")
                keep.append(p)
            pending = keep
            pending.append([dst, RESULT_WAIT, f"result {sorted(dst)[0]}..", no])
            if src != dst:
                pending.append([src, RESULT_WAIT, f"srcC {sorted(src)[0]}..", no])
            tag = None
            waits = 1
        else:
            dest = regs(body.split(",")[0]) if op.startswith("v_") else set()
            for p in pending:
                hit = (p[0] & dest) if p[2].startswith("srcC") else (p[0] & touched)
                if hit:
                    errors.append(f"{name}:{no}: `{line}` touches {p[2]} of line {p[3]} "
                                  f"({RESULT_WAIT - p[1]} wait states later)")
            for r in dest:
                since[r] = -waits
        for p in pending:
            p[1] -= waits
        pending = [p for p in pending if p[1] > 0]
        for r in since:
            since[r] += waits
        fresh += waits
    return errors


def main(path, allow=()):
    """`allow`: (name substring, bytes) pairs -- a kernel whose symbol contains the substring
    may use up to that many bytes of scratch (a known, reviewed spill); any other spill, or a
    larger one, is an error."""
    text = open(path).read().split("\n")
    # one function at a time: a function starts at a global label and ends at s_endpgm
    errors, start, count = [], None, 0
    for i, line in enumerate(text):
        if re.match(r"^_Z\S+:", line):
            start = i
        elif start is not None and line.strip().startswith("s_endpgm"):
            fn = text[start].rstrip(":")
            body = text[start + 1:i + 1]
            count += sum(1 for l in body if re.match(r"\s*;\s*mfma_s\s", l))
            errors += check(body, fn[:60])
            start = None
    for m in re.finditer(r"\.set (\S+)\.private_seg_size, (\d+)", "\n".join(text)):
        limit = max([b for sub, b in allow if sub in m.group(1)], default=0)
        if int(m.group(2)) > limit:
            errors.append(f"{m.group(1)[:60]}: {m.group(2)} bytes of scratch (register spills)"
                          + (f", above the {limit} allowed" if limit else ""))
    for e in errors:
        print(e)
    print(f"check_mfma_hazards: {count} S products checked, {len(errors)} violations")
    return 1 if errors else 0


if __name__ == "__main__":
    # check_mfma_hazards.py FILE.s [--allow-spill SUBSTRING:BYTES ...]
    args, allowed = sys.argv[1:], []
    while "--allow-spill" in args:
        i = args.index("--allow-spill")
        sub, nbytes = args[i + 1].rsplit(":", 1)
        allowed.append((sub, int(nbytes)))
        del args[i:i + 2]
    sys.exit(main(args[0], allowed))
