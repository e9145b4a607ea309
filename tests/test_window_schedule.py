"""The LDS-DMA kernel's window schedule (ltx-2.5-swift_amd/csrc/fmha_dma.hip, main loop),
restated step by step and checked on the CPU over split ranges and ragged key lengths:
every pipeline step runs exactly once, every operand read finds its tile in the buffer it
reads, no copy overwrites a buffer its own window reads, and the steady-state windows (no
edge handling, buffers fixed at compile time) have every step complete. A steady-state
window's copy of a tile past the range fetches the range's last tile instead (no branch);
the model tracks what each buffer then holds, so a later read of such a buffer would fail."""
import pytest

KT = 64


def schedule(t_begin, t_end, n_valid):
    blk_begin = 2 * t_begin
    blk_end = min(2 * t_end, (n_valid + 31) // 32)
    slots_k, slots_v = {}, {}
    if t_begin < t_end:
        slots_k[0] = t_begin
        if t_begin + 1 < t_end:
            slots_k[1] = t_begin + 1
        slots_v[0] = t_begin
    nwin = (blk_end - blk_begin + 2 + 3) // 4 if t_begin < t_end else 0
    lim_s = blk_end - blk_begin - 3
    wf0 = 1
    wf1 = min(nwin, (lim_s + 3) // 4 if lim_s > 0 else 0)
    order, w = [], 0
    while w < min(wf0, nwin):
        order.append((w, False)); w += 1
    if wf0 < wf1:
        assert w == wf0
        while w < wf1:
            order.append((w, True)); w += 1
    while w < nwin:
        order.append((w, False)); w += 1
    steps = []
    for w, fast in order:
        a, T0 = 2 * (w & 1), t_begin + 2 * w
        for k in range(4):
            s = 2 * T0 - 1 + k
            do_sm = blk_begin <= s < blk_end
            do_s = blk_begin <= s + 1 < blk_end
            do_pv = blk_begin <= s - 1 < blk_end
            if fast or (w == 0 and lim_s > 0 and k >= 2):   # steady, or window 0's last two
                assert do_sm and do_s and do_pv and s not in (blk_begin, blk_end - 1)
            if do_s:
                assert slots_k.get((a + (k >> 1)) & 3) == (s + 1) // 2
            if do_pv:
                assert slots_v.get((a + 3 + (k >> 1)) & 3) == (s - 1) // 2
            steps.append(s)
        reads_k = {(a + (k >> 1)) & 3 for k in range(4)}
        reads_v = {(a + 3 + (k >> 1)) & 3 for k in range(4)}
        copies = [("k", T0 + 2, (a + 2) & 3), ("k", T0 + 3, (a + 3) & 3),
                  ("v", T0 + 1, (a + 1) & 3), ("v", T0 + 2, (a + 2) & 3)]
        for kind, tile, slot in copies:
            if tile >= t_end:
                if not fast:
                    continue                      # edge windows skip it
                tile = ("past the range", min(tile, t_end - 1))
            if kind == "k":
                assert slot not in reads_k
                slots_k[slot] = tile
            else:
                assert slot not in reads_v
                slots_v[slot] = tile
    if t_begin < t_end:
        assert set(range(blk_begin - 1, blk_end + 1)) <= set(steps)
        assert len(steps) == len(set(steps))
    return len(order), sum(1 for _, f in order if f)


@pytest.mark.parametrize("t_begin", range(6))
def test_schedule_invariants(t_begin):
    for t_end in range(t_begin, t_begin + 40):
        for short in (0, 1, 31, 32, 33, 63):
            n_valid = max(1, t_end * KT - short) if t_end else 1
            if (n_valid + KT - 1) // KT >= t_end:
                schedule(t_begin, t_end, n_valid)


def test_benchmark_shapes():
    # 12480 keys, one whole item: 98 windows, 96 in the steady state
    assert schedule(0, 195, 12480) == (98, 96)
    # a tail item's key range of 28 tiles, and the last (ragged-free, shorter) one
    assert schedule(28, 56, 12480) == (15, 13)
    assert schedule(168, 195, 12480) == (14, 12)
