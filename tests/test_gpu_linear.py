"""GPU parity of the projection GEMM (``ltx_linear``) and of the RMS statistic it hands the
attention's norm, through the C ABI, against the CPU oracle.

Bar for y (bf16): the oracle's ``mode="reference"`` bits come from the exact sum rounded to
fp32 and then bf16 (plus the bias add's second bf16 rounding). The kernel accumulates in fp32
in its own order, so an element may differ from those bits by at most what fp32 summation can
move it -- the textbook bound gamma_K * sum_k |x_k w_k| (gamma_K = K u / (1 - K u), u = 2^-24)
-- plus one bf16 rounding step at the output's magnitude, and with a bias one more at the
magnitude of x . w^T (the matmul's own rounding comes before the add). Beyond that, at most 1% of
the elements may differ at all, and the relative RMS error against the exact float64 product
stays at bf16 rounding level (<= 3e-3).

Bar for the statistic: each fp32 partial equals the float64 sum of squares of the kernel's own
bf16 outputs over its 256 columns to fp32 summation accuracy (relative 2e-5 >= 258 u).
"""

import os

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

from test_gpu_parity import REL_RMS, MAX_ABS, check, dev, host_bits, host_f32

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def _say(msg):
    print(msg, flush=True)


def _ulp_bf16(a):
    """Spacing of bf16 values at |a| (the step of one rounding)."""
    a = np.maximum(np.abs(a), np.float64(2.0 ** -126))
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def check_linear(y_bits, x_bits, w_bits, b_bits, label):
    ref = O.linear(x_bits, w_bits, b_bits, "reference")
    exact = O.linear(x_bits, w_bits, b_bits, "exact")
    got = O.bf16_bits_to_f32(y_bits).astype(np.float64)
    K = x_bits.shape[-1]
    xa = np.abs(O.bf16_bits_to_f32(x_bits).astype(np.float64))
    wa = np.abs(O.bf16_bits_to_f32(w_bits).astype(np.float64))
    gamma = K * U32 / (1 - K * U32)
    acc = gamma * (xa @ wa.T) * 1.001              # fp32 summation in any order (+ fp32 I/O)
    bound = acc + _ulp_bf16(np.maximum(np.abs(got), np.abs(ref)))
    if b_bits is not None:
        # the matmul's own rounding happens at the magnitude of x.w^T, before the bias
        mm = np.abs(O.linear(x_bits, w_bits, None, "exact")) + acc
        bound = bound + _ulp_bf16(mm)
    diff = np.abs(got - ref)
    off = np.count_nonzero(diff) / diff.size
    c = O.compare(got, exact)
    _say(f"  {label}: {off:.2e} of elements off the reference bits, max diff/bound "
         f"{float(np.max(diff / bound)):.3f}, relRMS {c['rel_rms']:.2e}")
    assert np.all(diff <= bound), label
    assert off <= 0.01, label
    assert c["rel_rms"] <= 3e-3, label


def check_partials(parts, y_bits, label):
    want = O.sumsq_partials(O.bf16_bits_to_f32(y_bits))
    got = np.asarray(parts, dtype=np.float64)
    rel = np.abs(got - want) / np.maximum(want, 1e-30)
    _say(f"  {label}: statistic partials max rel err {float(rel.max()):.2e}")
    assert got.shape == want.shape, label
    assert np.all(rel <= 2e-5), label


@pytest.mark.parametrize("M,N,K,bias", [
    (256, 256, 64, False),      # one tile, one k step
    (256, 264, 128, True),      # two k steps (the first issues the second's later copies)
    (300, 520, 192, True),      # ragged rows and columns, three k steps
    (1000, 4096, 2048, True),   # audio-width projection rows of a stage-1 video
    (77, 32, 4096, True),       # to_gate_logits: 32 heads
    (600, 2048, 4096, False),   # the cross-modal to_q width (4096 -> 2048)
])
def test_linear_matches_oracle(device, M, N, K, bias):
    import torch

    x = O.randn_bf16_bits((M, K), 100 + M)
    w = O.randn_bf16_bits((N, K), 200 + N, std=K ** -0.5)
    b = O.randn_bf16_bits((N,), 300 + N, std=0.5) if bias else None
    _say(f"linear M={M} N={N} K={K} bias={bias}")
    y, parts = L.linear(dev(x, device), dev(w, device), None if b is None else dev(b, device),
                        sumsq=True)
    torch.cuda.synchronize()
    yb = host_bits(y)
    check_linear(yb, x, w, b, f"{M}x{N}x{K}")
    check_partials(parts.cpu().numpy(), yb, f"{M}x{N}x{K}")


def test_linear_strided_views_and_zero_rows(device):
    """x is a column slice of a wider buffer, y a column slice of a fused output buffer (its
    other columns untouched); without sumsq no partials are written; M = 0 is a no-op."""
    import torch

    M, N, K = 321, 264, 256
    xw = O.randn_bf16_bits((M, K + 64), 7)
    w = O.randn_bf16_bits((N, K), 8, std=K ** -0.5)
    big = torch.full((M, N + 136), 3.0, dtype=torch.bfloat16, device=device)
    xt = dev(xw, device)[:, 32:32 + K]
    y = L.linear(xt, dev(w, device), out=big[:, 64:64 + N])
    torch.cuda.synchronize()
    check_linear(host_bits(y), np.ascontiguousarray(xw[:, 32:32 + K]), w, None, "strided")
    rest = torch.cat([big[:, :64], big[:, 64 + N:]], dim=1).float().cpu().numpy()
    assert np.all(rest == 3.0)
    empty = L.linear(torch.empty((0, K), dtype=torch.bfloat16, device=device), dev(w, device))
    torch.cuda.synchronize()
    assert tuple(empty.shape) == (0, N)


def test_fused_projection_equals_separate_ones(device):
    """With every tile whole (no tail split), one GEMM over [to_q; to_k; to_v] weights writes
    the same bits, and the same statistic partials for the q and k column ranges (which start
    at multiples of 256), as three separate projections: each 256 x 256 tile depends only on
    its own rows of x and w. With the tail split (36 and 12 tiles: 3 and 4 k ranges) the
    summation order differs, so the two agree within the fp32 bound of check_linear."""
    import torch

    M, inner, K = 700, 1024, 2048
    xb = O.randn_bf16_bits((M, K), 41)
    x = dev(xb, device)
    wb = [O.randn_bf16_bits((inner, K), 42 + i, std=K ** -0.5) for i in range(3)]
    bb = [O.randn_bf16_bits((inner,), 45 + i, std=0.3) for i in range(3)]
    ws = [dev(w, device) for w in wb]
    bs = [dev(b, device) for b in bb]
    fused_w = torch.cat(ws, dim=0).contiguous()
    fused_b = torch.cat(bs, dim=0).contiguous()
    y, parts = L.linear(x, fused_w, fused_b, sumsq=True, workspace=False)
    sep = [L.linear(x, ws[i], bs[i], sumsq=True, workspace=False) for i in range(3)]
    ys, ps = L.linear(x, fused_w, fused_b, sumsq=True)
    sep_s = [L.linear(x, ws[i], bs[i], sumsq=True) for i in range(3)]
    torch.cuda.synchronize()
    nb = inner // 256
    for i, (yi, pi) in enumerate(sep):
        assert torch.equal(y[:, i * inner:(i + 1) * inner], yi), i
        assert torch.equal(parts[:, i * nb:(i + 1) * nb], pi), i
    check_linear(host_bits(ys), xb, np.concatenate(wb), np.concatenate(bb), "fused, split")
    for i, (yi, pi) in enumerate(sep_s):
        check_linear(host_bits(yi), xb, wb[i], bb[i], f"separate {i}, split")
        check_partials(pi.cpu().numpy(), host_bits(yi), f"separate {i}, split")


def test_projection_rows_of_the_video_stage2_call(device):
    """to_q of the 12480-token video call (12480 x 4096 x 4096): every tile runs, and a sample
    of 96 rows spread over all row tiles (first, last and ragged last tile included) is checked
    against the oracle, with their statistic partials."""
    import torch

    M, N, K = 12480, 4096, 4096
    g = torch.Generator(device="cpu").manual_seed(5)
    x = (torch.randn((M, K), generator=g) ).to(torch.bfloat16).to(device)
    w = (torch.randn((N, K), generator=g) * K ** -0.5).to(torch.bfloat16).to(device)
    b = (torch.randn((N,), generator=g) * 0.2).to(torch.bfloat16).to(device)
    y, parts = L.linear(x, w, b, sumsq=True)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1, M - 2, 12287, 12288],
                                     np.random.default_rng(3).integers(0, M, 89)]))
    xb = host_bits(x[torch.as_tensor(rows, device=device)])
    check_linear(host_bits(y[torch.as_tensor(rows, device=device)]), xb, host_bits(w),
                 host_bits(b), "12480x4096x4096 rows")
    check_partials(parts[torch.as_tensor(rows, device=device)].cpu().numpy(),
                   host_bits(y[torch.as_tensor(rows, device=device)]), "12480 rows")


@pytest.mark.parametrize("Lq,Lk", [(700, 700), (200, 200), (600, 152)])
def test_attention_takes_the_projection_statistic(device, Lq, Lk):
    """q and k from ltx_linear with their partials: the attention with q_sumsq / k_sumsq (no
    statistic pass over q and k) meets the tolerance against the oracle of the whole chain and
    agrees with the attention that computes the statistic itself. 700 queries take the LDS-DMA
    kernel (the K prologue reads the partials), 200 the register kernel (the statistic kernel
    feeds its fused K norm); 600 x 152 is a cross-modal shape with its own key tables."""
    import torch

    H, D, K = 16, 128, 1024
    inner = H * D
    xq = O.randn_bf16_bits((1, Lq, K), 51)
    xk = O.randn_bf16_bits((1, Lk, K), 52)
    wq = O.randn_bf16_bits((inner, K), 53, std=K ** -0.5)
    wk = O.randn_bf16_bits((inner, K), 54, std=K ** -0.5)
    wv = O.randn_bf16_bits((inner, K), 55, std=K ** -0.5)
    qn = O.randn_bf16_bits((inner,), 56, mean=1.0, std=0.2)
    kn = O.randn_bf16_bits((inner,), 57, mean=1.0, std=0.2)
    rng = np.random.default_rng(58)
    ang_q = rng.uniform(-3, 3, (H, Lq, D // 2))
    ang_k = rng.uniform(-3, 3, (H, Lk, D // 2))
    qc, qs = (O.f32_to_bf16_bits(f(ang_q).astype(np.float32)) for f in (np.cos, np.sin))
    kc, ks = (O.f32_to_bf16_bits(f(ang_k).astype(np.float32)) for f in (np.cos, np.sin))
    _say(f"attention with projection statistic Lq={Lq} Lk={Lk}")
    q, q_parts = L.linear(dev(xq, device), dev(wq, device), sumsq=True)
    k, k_parts = L.linear(dev(xk, device), dev(wk, device), sumsq=True)
    v = L.linear(dev(xk, device), dev(wv, device))
    rot = L.Rotary(dev(qc, device), dev(qs, device))
    krot = L.Rotary(dev(kc, device), dev(ks, device))
    kw = dict(heads=H, q_norm_w=dev(qn, device), k_norm_w=dev(kn, device), rotary=rot,
              key_rotary=krot)
    given = L.attention_fwd(q, k, v, q_sumsq=q_parts.view(Lq, -1),
                            k_sumsq=k_parts.view(Lk, -1), **kw)
    computed = L.attention_fwd(q, k, v, **kw)
    torch.cuda.synchronize()
    qb, kb, vb = host_bits(q), host_bits(k), host_bits(v)
    truth = O.attention(qb, kb, vb, H, q_norm_w=qn, k_norm_w=kn, q_cos=qc, q_sin=qs,
                        k_cos=kc, k_sin=ks)
    ref = O.attention(qb, kb, vb, H, q_norm_w=qn, k_norm_w=kn, q_cos=qc, q_sin=qs,
                      k_cos=kc, k_sin=ks, mode="reference")
    check(host_f32(given), truth, ref, f"statistic given {Lq}x{Lk}")
    c = O.compare(host_f32(given), host_f32(computed))
    _say(f"  given vs computed statistic: relRMS {c['rel_rms']:.2e} maxAbs {c['max_abs']:.2e}")
    assert c["rel_rms"] <= 1e-3 and c["max_abs"] <= MAX_ABS


@pytest.mark.parametrize("M,N,K", [
    (12480, 4096, 4096),    # to_q at 12480 tokens: 784 tiles = 3 rounds + 16 tiles in 8 ranges
    (12480, 32, 4096),      # to_gate_logits: 49 tiles in 4 ranges each
])
def test_tail_split_matches_whole_tiles(device, M, N, K):
    """The tiles past the last whole round of 256, cut along K into ranges whose fp32 partials
    the fixup kernel sums, against the same call with every tile whole (workspace=False):
    each element within twice the fp32 summation bound plus one bf16 step; rows of a whole
    tile and of the split tile row against the oracle; the statistic partials of every row."""
    import torch

    need = L.linear_workspace_bytes(M, N, K)
    assert need > 0
    x = O.randn_bf16_bits((M, K), 500 + N)
    w = O.randn_bf16_bits((N, K), 600 + N, std=K ** -0.5)
    b = O.randn_bf16_bits((N,), 700 + N, std=0.5)
    xt, wt, bt = dev(x, device), dev(w, device), dev(b, device)
    _say(f"linear tail split M={M} N={N} K={K}: {need >> 20} MiB of partials")
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    y_split, p_split = L.linear(xt, wt, bt, sumsq=True, workspace=ws)
    y_whole, _ = L.linear(xt, wt, bt, sumsq=True, workspace=False)
    torch.cuda.synchronize()
    ys, yw = host_f32(y_split).astype(np.float64), host_f32(y_whole).astype(np.float64)
    xa = np.abs(O.bf16_bits_to_f32(x)).astype(np.float32)
    wa = np.abs(O.bf16_bits_to_f32(w)).astype(np.float32)
    gamma = K * U32 / (1 - K * U32)
    acc = 2 * gamma * (xa @ wa.T).astype(np.float64) * 1.01
    mm = np.abs(yw) + acc
    bound = acc + _ulp_bf16(np.maximum(np.abs(ys), np.abs(yw))) + _ulp_bf16(mm)
    diff = np.abs(ys - yw)
    _say(f"  split vs whole: {np.count_nonzero(diff) / diff.size:.2e} of elements differ, "
         f"max diff/bound {float(np.max(diff / bound)):.3f}")
    assert np.all(diff <= bound)
    ysb = host_bits(y_split)
    rows = np.r_[0:64, M - 64:M]                  # a whole tile's rows, the split tile row's
    check_linear(ysb[rows], np.ascontiguousarray(x[rows]), w, b, f"{M}x{N}x{K} split rows")
    check_partials(p_split.cpu().numpy(), ysb, f"{M}x{N}x{K} split")


@pytest.mark.parametrize("groups", [32, 100])
def test_tail_split_for_other_part_sizes(device, groups):
    """ltx_linear splits its tail for the device's CU count (the resident_groups argument
    stands in for it) when the workspace sized for 256 CUs covers that split: 3000 x 1024 x 512 is 48
    tiles; 32 groups split the 16 past one round two ways, 100 split all 48 two ways (as the
    split sized for 256 does). The oracle on the rows of a whole tile and of a split one, and the
    statistic partials of every row."""
    import torch

    M, N, K = 3000, 1024, 512
    need = L.linear_workspace_bytes(M, N, K)
    assert need > 0
    x = O.randn_bf16_bits((M, K), 800 + groups)
    w = O.randn_bf16_bits((N, K), 900 + groups, std=K ** -0.5)
    b = O.randn_bf16_bits((N,), 1000 + groups, std=0.5)
    _say(f"linear {M}x{N}x{K}, tail split for {groups} resident groups")
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    y, parts = L.linear(dev(x, device), dev(w, device), dev(b, device), sumsq=True, workspace=ws,
                        resident_groups=groups)
    torch.cuda.synchronize()
    yb = host_bits(y)
    rows = np.r_[0:64, 1024:1088, M - 64:M]
    check_linear(yb[rows], np.ascontiguousarray(x[rows]), w, b, f"groups {groups} rows")
    check_partials(parts.cpu().numpy(), yb, f"groups {groups}")


@pytest.mark.parametrize("K,groups", [(64, 3), (128, 8), (192, 3), (1024, 8)])
def test_persistent_grid_walks_many_tiles(device, K, groups):
    """A few resident groups leave each workgroup of the persistent grid many whole tiles
    (1800 x 1000: 32 tiles on 3 or 8 workgroups). At K = 64 each tile restarts from its own
    prologue; from K = 128 on, the next tile's first copies and operands are issued during the
    current tile's last two k steps. A tile's sum order does not depend on the workgroup that
    runs it, so y and the statistic equal the default grid's (one tile per workgroup) bit for
    bit; the oracle on rows of the first and last row tiles."""
    import torch

    M, N = 1800, 1000
    x = O.randn_bf16_bits((M, K), 1100 + K)
    w = O.randn_bf16_bits((N, K), 1200 + K, std=K ** -0.5)
    b = O.randn_bf16_bits((N,), 1300 + K, std=0.5)
    xt, wt, bt = dev(x, device), dev(w, device), dev(b, device)
    _say(f"linear {M}x{N}x{K} on {groups} workgroups")
    y_few, p_few = L.linear(xt, wt, bt, sumsq=True, workspace=False, resident_groups=groups)
    y_all, p_all = L.linear(xt, wt, bt, sumsq=True, workspace=False)
    torch.cuda.synchronize()
    yb = host_bits(y_few)
    assert np.array_equal(yb, host_bits(y_all))
    assert np.array_equal(p_few.cpu().numpy(), p_all.cpu().numpy())
    rows = np.r_[0:64, M - 64:M]
    check_linear(yb[rows], np.ascontiguousarray(x[rows]), w, b, f"K {K} on {groups} groups")
    check_partials(p_few.cpu().numpy(), yb, f"K {K} on {groups} groups")


def _random_linear_case(i):
    """Seeded draws of M (any), N (a multiple of 8), K (a multiple of 64), bias, statistic,
    the part size the tail split is planned for, and whether a workspace allows the split."""
    rng = np.random.default_rng(0x5EED + 8000 + i)
    M = int(np.exp(rng.uniform(np.log(1), np.log(3000))))
    N = 8 * max(1, int(np.exp(rng.uniform(np.log(8), np.log(3000)))) // 8)
    K = 64 * int(rng.integers(1, 65))
    while M * N * K > 2_000_000_000:                 # the float64 oracle finishes in seconds
        M = max(1, M // 2)
    return dict(M=M, N=N, K=K, bias=bool(rng.random() < 0.5), sumsq=bool(rng.random() < 0.5),
                groups=int(rng.choice([0, 0, 32, 100])), split=bool(rng.random() < 0.7),
                seed=int(rng.integers(1, 1 << 30)))


# 12 cases by default; LTX_LINEAR_RANDOM_CASES=n runs the first n seeds of the same sequence.
@pytest.mark.parametrize("i", range(int(os.environ.get("LTX_LINEAR_RANDOM_CASES", "12"))))
def test_linear_random_shapes(device, i):
    import torch

    c = _random_linear_case(i)
    M, N, K, seed = c["M"], c["N"], c["K"], c["seed"]
    _say(f"linear random {i}: {c}")
    x = O.randn_bf16_bits((M, K), seed)
    w = O.randn_bf16_bits((N, K), seed + 1, std=K ** -0.5)
    b = O.randn_bf16_bits((N,), seed + 2, std=0.5) if c["bias"] else None
    out = L.linear(dev(x, device), dev(w, device), None if b is None else dev(b, device),
                   sumsq=c["sumsq"], workspace=None if c["split"] else False,
                   resident_groups=c["groups"])
    torch.cuda.synchronize()
    y, parts = out if c["sumsq"] else (out, None)
    yb = host_bits(y)
    check_linear(yb, x, w, b, f"random {i}")
    if parts is not None:
        check_partials(parts.cpu().numpy(), yb, f"random {i}")
