"""The build-time MFMA hazard check (ltx-2.5-swift_amd/csrc/check_mfma_hazards.py) rejects the
mistakes it exists for, on small hand-written assembly, and passes the built kernel."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ltx-2.5-swift_amd", "csrc")
_spec = importlib.util.spec_from_file_location("check_mfma_hazards",
                                               os.path.join(CSRC, "check_mfma_hazards.py"))
H = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(H)

# A chain of two S products, then the 20-wait-state fence, then a use.
GOOD = """\
\t; mfma_s v[100:115] src v[20:35]
\ts_nop 2
\tv_mfma_f32_32x32x16_bf16 v[100:115], v[6:9], a[128:131], v[20:35]
\t; mfma_s v[100:115] src v[100:115]
\ts_nop 2
\tv_mfma_f32_32x32x16_bf16 v[100:115], v[10:13], a[132:135], v[100:115]
\t; s_ready v[100:115] v[84:99]
\ts_nop 7
\ts_nop 7
\ts_nop 3
\tv_exp_f32_e32 v40, v100
"""


def _errors(text):
    return H.check(text.split("\n"), "t")


def test_good_sequence_passes():
    assert _errors(GOOD) == []


def test_copy_right_after_product_is_caught():
    bad = GOOD.replace("\t; s_ready", "\tv_accvgpr_write_b32 a143, v115\n\t; s_ready")
    errs = _errors(bad)
    assert errs and "result" in errs[0]


def test_short_fence_is_caught():
    bad = GOOD.replace("\ts_nop 3\n", "")
    assert any("result" in e for e in _errors(bad))


def test_input_written_just_before_is_caught():
    bad = GOOD.replace("\ts_nop 2\n\tv_mfma_f32_32x32x16_bf16 v[100:115], v[6:9]",
                       "\ts_nop 2\n\tv_mov_b32_e32 v7, 0\n"
                       "\tv_mfma_f32_32x32x16_bf16 v[100:115], v[6:9]")
    assert any("wait states before" in e for e in _errors(bad))
    ok = GOOD.replace("\ts_nop 2\n\tv_mfma_f32_32x32x16_bf16 v[100:115], v[6:9]",
                      "\tv_mov_b32_e32 v7, 0\n\ts_nop 1\n"
                      "\tv_mfma_f32_32x32x16_bf16 v[100:115], v[6:9]")
    assert _errors(ok) == []


def test_valu_write_of_untied_srcc_is_caught_but_a_load_is_not():
    bad = GOOD.replace("\t; mfma_s v[100:115] src v[100:115]",
                       "\tv_mov_b32_e32 v20, 0\n\t; mfma_s v[100:115] src v[100:115]")
    assert any("srcC" in e for e in _errors(bad))
    ok = GOOD.replace("\t; mfma_s v[100:115] src v[100:115]",
                      "\tds_read_b128 v[20:23], v214 offset:64\n"
                      "\t; mfma_s v[100:115] src v[100:115]")
    assert _errors(ok) == []


def test_window_open_at_branch_is_caught():
    bad = GOOD.replace("\t; s_ready", "\ts_cbranch_scc1 .LBB0_7\n\t; s_ready")
    assert any("branch" in e for e in _errors(bad))


def test_built_kernel_passes():
    s = os.path.join(ROOT, "ltx-2.5-swift_amd", "_build", "fmha_dma.s")
    if not os.path.exists(s):
        pytest.skip("device assembly not built (make -C ltx-2.5-swift_amd/csrc)")
    assert H.main(s) == 0


def test_scratch_spill_is_caught(tmp_path):
    text = ("_Zkernel:\n\ts_endpgm\n"
            "\t.set _Zkernel.private_seg_size, 316\n")
    f = tmp_path / "k.s"
    f.write_text(text)
    assert H.main(str(f)) == 1
    f.write_text(text.replace("316", "0"))
    assert H.main(str(f)) == 0


def test_allowed_spill_is_bounded_by_its_size(tmp_path):
    """--allow-spill SUBSTRING:BYTES admits one reviewed spill at its size, and nothing more:
    a larger spill of that kernel or any spill of another kernel still fails."""
    f = tmp_path / "k.s"
    f.write_text("_Zknown:\n\ts_endpgm\n\t.set _Zknown.private_seg_size, 28\n"
                 "_Zother:\n\ts_endpgm\n\t.set _Zother.private_seg_size, 0\n")
    assert H.main(str(f)) == 1
    assert H.main(str(f), [("known", 28)]) == 0
    f.write_text("_Zknown:\n\ts_endpgm\n\t.set _Zknown.private_seg_size, 32\n")
    assert H.main(str(f), [("known", 28)]) == 1
    f.write_text("_Zother:\n\ts_endpgm\n\t.set _Zother.private_seg_size, 4\n")
    assert H.main(str(f), [("known", 28)]) == 1
