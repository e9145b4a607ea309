// Projection GEMM of the attention modules, y = x . w^T (+ bias), following
// Sources/LTXModules/DiTAttention.swift:178-188 (`linear`: matmul in the weight's dtype, then
// the bias add), with the RMS-norm statistic of the result emitted by the epilogue: for every
// row of y, the sum of squares of its bf16 values over each 256-column tile, so the q_norm /
// k_norm that follow (:202-204) need no pass of their own over q and k.
//
// Layout: x [M][K] and w [N][K] (the checkpoint's [out, in] layout) are both K-contiguous;
// y [M][N] row-major. One workgroup of four waves computes a 256 x 256 tile of y; wave (wm, wn)
// owns rows wm*128.. and columns wn*128.. as 4 x 4 products of v_mfma_f32_32x32x16_bf16 in
// which w is the A operand and x the B operand, so each lane's accumulators hold one row of y
// and runs of four consecutive columns (8-byte stores, and the row's sum of squares stays in
// the lane).
//
// Staging: every k step's 256 x BK tiles of x and w are copied HBM -> LDS by the
// buffer-load-to-LDS path, rows of BK elements with their 16-byte units XOR-swizzled so the
// operand reads (32 rows, one unit per half-wave) are free of bank conflicts. Rows past M (N)
// read as zeros through the buffer resource's bound. LDS holds three w tiles and two x tiles
// (160 KiB): k step g reads w buffer g % 3 and x buffer g % 2. The step loop is arranged
// around its one barrier, which sits in the last reduction chunk of each step, after that
// chunk's operands have been read into registers and before its products:
//   * the barrier certifies that every wave's copies for step g + 1 have landed (each wave
//     waits for its own first: the copies are untracked assembly, counted by vmcnt) and that
//     every wave has finished reading step g's buffers. Step g + 2's w tile, issued during
//     step g's first chunk into the third w buffer, stays in flight across it: a copy-only
//     run of this tile stream (30720 x 4096 x 4096) takes 0.53 ms when each step waits for
//     all its copies and 0.38 ms with half a step's copies always outstanding;
//   * right after it, the wave issues step g + 2's x tile into the x buffer just freed, one
//     copy after every other product of the chunk, and reads step g + 1's first operands
//     between the same products, so the matrix cores have the chunk's products to run while
//     the reads return. Half a step's copies per chunk keeps the texture address unit's queues
//     from filling (all sixteen in one chunk stalled the wave's issue).
// Within a step, the operands of chunk c + 1 are read while the products of chunk c run, one
// before every other product (all eight at the chunk's start left the LDS reads of the four
// waves bunched: the fused 12480 x 12288 x 4096 projection 1.075 -> 1.049 ms).
//
// Rounding follows the reference's two operations: the fp32 accumulator is rounded to bf16
// (the matmul's output), then the bias is added in fp32 and the sum rounded to bf16 again.
//
// Tail split: one workgroup runs per CU, so a tile count just past a multiple of 256 costs a
// whole extra round (12480 x 4096: 784 tiles = 3 rounds + 16 tiles). The host cuts the tiles
// past the last whole round into k ranges, at most as many as fill the CUs, the count weighing
// a range's k steps against its partials' round trip (16 tiles -> 8 ranges of 8 k steps
// each); a range stores its fp32 accumulators, in register order, to the
// workspace, and linear_fixup_kernel sums a tile's ranges in order and runs the same epilogue
// (eight workgroups per tile).
#include <type_traits>

#include "lds_copy.hpp"

namespace ltx {
namespace {

constexpr int LT = kLinearTile;       // 256 rows and columns of y per workgroup

template <int BK>
struct LinTile {
    static constexpr int U = BK / 8;              // 16-byte units per LDS row
    static constexpr int ELEMS = LT * BK;         // one operand's tile of one k step
    static constexpr int CPT = LT * U / 64 / 4;   // copies per wave per operand tile
    static constexpr int NCH = BK / 16;           // MFMA reduction chunks per k step
    static_assert(BK == 64, "k step: the copy schedule places CPT = 8 copies in each of two chunks");
    static_assert((3 + 2) * ELEMS * 2 <= 160 * 1024, "LDS budget: three w and two x buffers");
};

// Unit swizzle: the 16 lanes a 16-byte LDS read serves together read 16 consecutive rows at
// one logical unit; XOR-ing the unit with bits of the row puts them in 16 distinct 16-byte
// bank slots of a 256-byte window (rows of 8 units: 2 rows per window; of 4 units: 4).
template <int U>
__device__ __forceinline__ int lswz(int row, int u) {
    return U == 8 ? (u ^ ((row >> 1) & 7)) : (u ^ ((row >> 2) & 3));
}

// Tile t of the tile order -> (row tile, column tile): groups of 8 row tiles, walked column
// tile by column tile.
__device__ __forceinline__ void tile_coords(const LinearParams &p, int t, int &tm, int &tn) {
    constexpr int GRP = 8;
    const int group = t / (GRP * p.tiles_n);
    const int first_m = group * GRP;
    const int rows_g = min(GRP, p.tiles_m - first_m);
    const int within = t - group * GRP * p.tiles_n;
    tm = first_m + within % rows_g;
    tn = within / rows_g;
}

// Epilogue of NMB 32-row blocks of a wave: round to bf16, add the bias, store, and the rows'
// sums of squares (the two column halves' sums meet in red, 2 x 256 floats of LDS). Lane
// (r, g) of product (nb, mb) holds y[m][n + e] for
// m = mrow + 32*mb + r, n = ncol + 32*nb + 8*qd + 4*g (qd = 0..3), e = 0..3 in accumulator
// 4*qd + e; the wave covers columns [ncol, ncol + 128) of column tile tn, the workgroup's two
// waves of one row range (wn = 0, 1) all 256. The workgroup's rows are the `rows` rows from
// mrow - red_off, in which the wave's blocks start at red_off. Every thread calls it.
typedef __attribute__((address_space(3))) float lds_float;

template <int NMB>
__device__ __forceinline__ void store_rows(const LinearParams &p, const f32x16 (&acc)[4][NMB],
                                           int mrow, int ncol, int tn, int wn, int red_off,
                                           int rows, lds_float *red) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int r = lane & 31, g = lane >> 5;
    u32x2 bias[4][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const int n = ncol + 32 * nb + 8 * qd + 4 * g;
            bias[nb][qd] = (p.bias && n < p.N) ? *(const u32x2 *)((const bf16 *)p.bias + n)
                                               : u32x2{0u, 0u};
        }
    float ss[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
        const int m = mrow + 32 * mb + r;
        bf16 *yrow = (bf16 *)p.y + (int64_t)m * p.y_rs;
        float sum = 0.f;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int n = ncol + 32 * nb + 8 * qd + 4 * g;
                const f32x16 &c = acc[nb][mb];
                u32x2 w;
                w[0] = pack_bf2(c[4 * qd + 0], c[4 * qd + 1]);
                w[1] = pack_bf2(c[4 * qd + 2], c[4 * qd + 3]);
                if (p.bias) {
                    w[0] = pack_bf2(bf_lo(w[0]) + bf_lo(bias[nb][qd][0]),
                                    bf_hi(w[0]) + bf_hi(bias[nb][qd][0]));
                    w[1] = pack_bf2(bf_lo(w[1]) + bf_lo(bias[nb][qd][1]),
                                    bf_hi(w[1]) + bf_hi(bias[nb][qd][1]));
                }
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float lo = bf_lo(w[e]), hi = bf_hi(w[e]);
                    sum += lo * lo;
                    sum += hi * hi;
                }
                if (m < p.M && n < p.N) *(u32x2 *)(yrow + n) = w;
            }
        ss[mb] = sum + xlane32(sum);   // the wave's 128 columns (columns past N are zeros)
    }
    if (!p.sumsq) return;
    if (g == 0) {
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) red[wn * LT + red_off + 32 * mb + r] = ss[mb];
    }
    __syncthreads();
    const int m = mrow - red_off + tid;
    if (tid < rows && m < p.M) p.sumsq[(int64_t)m * p.ss_rs + tn] = red[tid] + red[LT + tid];
}

template <int BK>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void linear_kernel(const LinearParams p) {
    using T = LinTile<BK>;
    constexpr int U = T::U, CPT = T::CPT, NCH = T::NCH, ELEMS = T::ELEMS;
    // Three buffers of w tiles and two of x tiles (160 KiB): k step g of a run reads w buffer
    // g % 3 and x buffer g % 2, so half of step g + 2's copies (its w tile) can be in flight
    // before step g's barrier frees anything.
    __shared__ __attribute__((aligned(16))) bf16 sW[3 * ELEMS];
    __shared__ __attribute__((aligned(16))) bf16 sX[2 * ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, g = lane >> 5;

    // Work of this workgroup. The grid is persistent: workgroup g runs the whole tiles
    // g, g + G, g + 2G, ... of the tile order (G workgroups), then tail range g if there is
    // one. Workgroups go to the 8 XCDs round-robin and G is a multiple of 8 on a whole part, so
    // in every round each XCD runs a contiguous range of the tile order, which walks groups of
    // 8 row tiles column tile by column tile: the ~32 workgroups an XCD runs at once share 8 row
    // tiles of x and 4 column tiles of w in its L2, and the ranges of one tail tile share all
    // of it. From one whole tile to the next a workgroup does not stop: the next tile's first
    // copies are issued during the current tile's last two k steps, as within a tile, so its
    // epilogue runs while they land instead of after a round's worth of workgroups restarts.
    const int bid = blockIdx.x;
    const int G = gridDim.x;
    const int nsteps = p.K / BK;
    const int xrow = (int)(p.x_rs * 2), wrow = (int)(p.w_rs * 2);    // row bytes
    // Copy j of this wave's share of a tile: LDS unit q = (wave*CPT + j)*64 + lane holds row
    // q / U, logical unit lswz(row, q % U); its source offset is fixed for every tile, the tile
    // and the k step move the resource's base.
    int xl[CPT], wl[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int q = (wave * CPT + j) * 64 + lane;
        const int row = q / U, u = lswz<U>(row, q % U);
        xl[j] = row * xrow + 16 * u;
        wl[j] = row * wrow + 16 * u;
    }
    // Copy j (0 .. CPT-1) of this wave's share of a w (x) tile into w (x) buffer bf.
    auto copy_w = [&](const u32x4 &rw, int bf, int j) __attribute__((always_inline)) {
        copy_all(rw, (uint32_t)(uintptr_t)((lds_bf16 *)sW + bf * ELEMS + (wave * CPT + j) * 512), wl[j]);
    };
    auto copy_x = [&](const u32x4 &rx, int bf, int j) __attribute__((always_inline)) {
        copy_all(rx, (uint32_t)(uintptr_t)((lds_bf16 *)sX + bf * ELEMS + (wave * CPT + j) * 512), xl[j]);
    };
    // A tile's operand rows: x rows m0.., w rows n0.. (rows past M, N read as zeros through the
    // resources' bounds).
    struct TileSrc {
        const char *X0, *W0;
        int64_t xbytes, wbytes;
        int m0, n0, tn;
    };
    auto tile_src = [&](int t) __attribute__((always_inline)) {
        int tm, tn;
        tile_coords(p, t, tm, tn);
        TileSrc ts;
        ts.m0 = tm * LT;
        ts.n0 = tn * LT;
        ts.tn = tn;
        ts.X0 = (const char *)p.x + (int64_t)ts.m0 * xrow;
        ts.W0 = (const char *)p.w + (int64_t)ts.n0 * wrow;
        ts.xbytes = (int64_t)min(LT, p.M - ts.m0) * xrow;
        ts.wbytes = (int64_t)min(LT, p.N - ts.n0) * wrow;
        return ts;
    };
    // Operand of rows row0 + 0..31, reduction chunk c: lane (r, g) reads row row0 + r, unit 2c + g.
    auto frag = [&](const lds_bf16 *S, int row0, int c) __attribute__((always_inline)) {
        const int row = row0 + r;
        return *(const __attribute__((address_space(3))) bf16x8 *)(S + row * BK + 8 * lswz<U>(row, 2 * c + g));
    };
    bf16x8 a[2][4], b[2][4];           // operands of the current and the next chunk
    auto read_chunk = [&](int ws, int xs, int c, int buf) __attribute__((always_inline)) {
        const lds_bf16 *Ws = (const lds_bf16 *)sW + ws * ELEMS;
        const lds_bf16 *Xs = (const lds_bf16 *)sX + xs * ELEMS;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[buf][i] = frag(Ws, wn * 128 + 32 * i, c);
            b[buf][i] = frag(Xs, wm * 128 + 32 * i, c);
        }
    };
    // Prologue of a run of k steps: its first two steps' tiles into buffers 0 and 1, then the
    // first operands.
    auto prologue = [&](const TileSrc &ts, int k0, bool two) __attribute__((always_inline)) {
        const int kb = k0 * BK * 2;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            copy_w(rsrc_words(ts.W0 + kb, ts.wbytes), 0, j);
            copy_x(rsrc_words(ts.X0 + kb, ts.xbytes), 0, j);
        }
        if (two) {
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                copy_w(rsrc_words(ts.W0 + kb + BK * 2, ts.wbytes), 1, j);
                copy_x(rsrc_words(ts.X0 + kb + BK * 2, ts.xbytes), 1, j);
            }
            wait_copies_but<2 * CPT>();
        } else {
            wait_copies();
        }
        __syncthreads();
        read_chunk(0, 0, 0, 0);
    };

    // One k step g on w buffer ws, x buffer xs. has1: there is a step g + 1 (in this tile or
    // the next), whose first operands are read in the last chunk. has2: there is a step g + 2:
    // its w tile (resource rw2) is copied during the first chunk into w buffer (g + 2) % 3,
    // free since step g - 1's barrier, and its x tile (rx2) during the last chunk into x buffer
    // xs, which this step's barrier frees (a step's copies over two chunks keeps the address
    // unit's queue from filling). The barrier waits for step g + 1's tiles only: step g + 2's
    // w tile, the wave's CPT most recent copies, stays in flight. A1, A2: has1, has2 hold
    // whatever the run-time flags say (the inner steps of a run, without branches).
    auto step = [&](auto A1, auto A2, bool h1, bool h2, int ws, int xs, f32x16(&acc)[4][4],
                    const u32x4 &rw2, const u32x4 &rx2) __attribute__((always_inline)) {
        const bool has1 = decltype(A1)::value || h1, has2 = decltype(A2)::value || h2;
        const int ws1 = ws == 2 ? 0 : ws + 1, ws2 = ws == 0 ? 2 : ws - 1;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int cb = c & 1;          // NCH is even: chunk 0 of every step is in buffer 0
            // The next chunk's operands -- of this step, or after the barrier the next step's
            // first -- are read one before every other product of this chunk (all eight at the
            // chunk's start left the LDS reads of the four waves bunched).
            const bool rd = c < NCH - 1 || has1;
            const int rws = c < NCH - 1 ? ws : ws1, rxs = c < NCH - 1 ? xs : xs ^ 1;
            const int rc = c < NCH - 1 ? c + 1 : 0;
            if (c == NCH - 1) {
                // Step g + 1's tiles have landed for this wave; after the barrier they have for
                // every wave, and every wave's reads of this step's buffers are done. The
                // scheduling fences keep the earlier chunks' products ahead of the wait.
                __builtin_amdgcn_sched_barrier(0);
                if (has2) wait_copies_but<CPT>();
                else wait_copies();
                __syncthreads();
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    const int pr = 4 * nb + mb;                // product of the chunk
                    if (rd && (pr & 1) == 0) {
                        // operand pr / 2 of the next chunk: a[0], b[0], a[1], b[1], ...
                        const int j = pr >> 1;
                        const lds_bf16 *Ws = (const lds_bf16 *)sW + rws * ELEMS;
                        const lds_bf16 *Xs = (const lds_bf16 *)sX + rxs * ELEMS;
                        if ((j & 1) == 0) a[cb ^ 1][j >> 1] = frag(Ws, wn * 128 + 32 * (j >> 1), rc);
                        else b[cb ^ 1][j >> 1] = frag(Xs, wm * 128 + 32 * (j >> 1), rc);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    acc[nb][mb] = mfma32(a[cb][nb], b[cb][mb], acc[nb][mb]);
                    if (has2 && c == 0 && (pr & 1) == 0) {
                        copy_w(rw2, ws2, pr / 2);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    if (has2 && c == NCH - 1 && (pr & 1) == 0) {
                        copy_x(rx2, xs, pr / 2);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
        }
    };
    auto zero = [&](f32x16(&acc)[4][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = splat16(0.f);
    };
    // k steps [k0, k1) of tile cur (the prologue or the previous run issued the first two
    // steps' tiles). chain: the stream goes on into steps 0, 1, ... of tile nxt, whose first
    // tiles and operands this run issues and reads. ws, xs: the buffers of the run's first
    // step, on return those of the step after its last.
    using yes = std::true_type;
    using rt = std::false_type;
    auto run = [&](const TileSrc &cur, int k0, int k1, bool chain, const TileSrc &nxt, int &ws,
                   int &xs, f32x16(&acc)[4][4]) __attribute__((always_inline)) {
        auto res = [&](int s, u32x4 &rw, u32x4 &rx) __attribute__((always_inline)) {
            const bool in = s < k1;
            const TileSrc &t = in ? cur : nxt;
            const int kb = (in ? s : s - k1) * BK * 2;
            rw = rsrc_words(t.W0 + kb, t.wbytes);
            rx = rsrc_words(t.X0 + kb, t.xbytes);
        };
        auto advance = [&]() __attribute__((always_inline)) {
            ws = ws == 2 ? 0 : ws + 1;
            xs ^= 1;
        };
        u32x4 rw2, rx2;
        int s = k0;
        for (; s + 2 < k1; ++s) {
            res(s + 2, rw2, rx2);
            step(yes{}, yes{}, true, true, ws, xs, acc, rw2, rx2);
            advance();
        }
        if (s + 1 < k1) {              // step k1 - 2: the step after next is nxt's first
            res(s + 2, rw2, rx2);
            step(yes{}, rt{}, true, chain, ws, xs, acc, rw2, rx2);
            advance();
            ++s;
        }
        res(s + 2, rw2, rx2);          // step k1 - 1: next nxt's first, then its second
        step(rt{}, rt{}, chain, chain, ws, xs, acc, rw2, rx2);
        advance();
    };

    // ---- whole tiles: one stream of k steps over this workgroup's tiles ------------------
    if (bid < p.n_full) {
        f32x16 acc[4][4];              // [n block][m block]
        zero(acc);
        int i = bid;
        TileSrc cur = tile_src(xcd_major(i, p.n_full));
        prologue(cur, 0, nsteps > 1);
        int ws = 0, xs = 0;
        for (;;) {
            const bool more = i + G < p.n_full;
            // With one k step a tile's run cannot issue the tile after next's first copies:
            // such tiles restart from a prologue.
            const bool chain = more && nsteps > 1;
            const TileSrc nxt = more ? tile_src(xcd_major(i + G, p.n_full)) : cur;
            run(cur, 0, nsteps, chain, nxt, ws, xs, acc);
            // The tile's last w buffer is free until the next tile's second step copies into
            // it: the epilogue's row sums meet there.
            const int red_ws = ws == 0 ? 2 : ws - 1;
            store_rows<4>(p, acc, cur.m0 + wm * 128, cur.n0 + wn * 128, cur.tn, wn, wm * 128, LT,
                          (lds_float *)((lds_bf16 *)sW + red_ws * ELEMS));
            if (!more) break;
            zero(acc);
            i += G;
            cur = nxt;
            if (!chain) {
                __syncthreads();
                prologue(cur, 0, false);
                ws = xs = 0;
            } else if (p.sumsq) {
                __syncthreads();       // every wave's reads of the row sums are done
            }
        }
    }

    // ---- a tail range: k steps [k_begin, k_end) of a tail tile, its accumulators, in
    // register order, for the fixup --------------------------------------------------------
    const int n_ranges = (p.tiles_m * p.tiles_n - p.n_full) * p.splits;
    if (p.splits > 1 && bid < n_ranges) {
        const int range = xcd_major(bid, n_ranges);                // tile-major: (tile, split)
        const TileSrc ts = tile_src(p.n_full + range / p.splits);
        const int k_begin = (range % p.splits) * p.steps_per_split;
        const int k_end = min(k_begin + p.steps_per_split, nsteps);
        f32x16 acc[4][4];
        zero(acc);
        __syncthreads();               // the whole tiles' last reads of the LDS buffers are done
        prologue(ts, k_begin, k_end - k_begin > 1);
        int ws = 0, xs = 0;
        run(ts, k_begin, k_end, false, ts, ws, xs, acc);
        f32x16 *dst = (f32x16 *)(p.part + (int64_t)range * (LT * LT)) + wave * 16 * 64 + lane;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) dst[(4 * nb + mb) * 64] = acc[nb][mb];
    }
}

// Tail tiles: the sum of a tile's k ranges, then the epilogue. Eight workgroups per tile, one
// per 32-row block (wm, mb) of it, so the partials are read by as many CUs as a whole round
// of the tail had; the workgroup's two waves are the block's column halves (wn).
constexpr int kFixupThreads = 128;
__global__ __attribute__((amdgpu_flat_work_group_size(kFixupThreads, kFixupThreads)))
void linear_fixup_kernel(const LinearParams p) {
    const int lane = threadIdx.x & 63, wn = threadIdx.x >> 6;
    const int tt = blockIdx.x >> 3, wm = (blockIdx.x >> 2) & 1, mb = blockIdx.x & 3;
    int tm, tn;
    tile_coords(p, p.n_full + tt, tm, tn);
    // the range's accumulators of wave (wm, wn), products (nb, mb), in register order
    const f32x16 *src = (const f32x16 *)(p.part + (int64_t)tt * p.splits * (LT * LT)) +
                        (2 * wm + wn) * 16 * 64 + mb * 64 + lane;
    f32x16 acc[4][1];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb][0] = src[nb * 4 * 64];
    for (int sp = 1; sp < p.splits; ++sp) {
        src += LT * LT / 16;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[nb][0] += src[nb * 4 * 64];
    }
    __shared__ float red[2 * LT];
    store_rows<1>(p, acc, tm * LT + wm * 128 + 32 * mb, tn * LT + wn * 128, tn, wn, 0, 32,
                  (lds_float *)red);
}

}  // namespace

int64_t linear_part_bytes(int64_t tail_tiles, int splits) {
    return tail_tiles * splits * (int64_t)LT * LT * 4;
}

int launch_linear(const LinearParams &p, void *stream) {
    const int n_tail = p.tiles_m * p.tiles_n - p.n_full;
    const dim3 block(256);
    if (p.grid < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((linear_kernel<64>), dim3((unsigned)p.grid), block, 0, (hipStream_t)stream, p);
    if (n_tail > 0 && p.splits > 1)
        hipLaunchKernelGGL(linear_fixup_kernel, dim3((unsigned)n_tail * 8), dim3(kFixupThreads),
                           0, (hipStream_t)stream, p);
    return (int)hipGetLastError();
}

}  // namespace ltx
