/*
 * attn_oracle.c -- CPU restatement of the LTX 2.5 DiT attention path, in C.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (the parity reference) and by bench.py's cpu_baseline
 * leg (as the timed CPU baseline). The shipped library never links or calls it.
 *
 * It restates the reference's `.explicit` attention arithmetic with its rounding points:
 *   QK-RMSNorm over the inner dim, fp32 statistic, bf16 output
 *       Sources/LTXModules/DiTAttention.swift:190-204, :360-361; DiTBlock.swift:219-221
 *   head split [B,L,H*D] -> [B,H,L,D]                       DiTAttention.swift:346-349
 *   split RoPE, bf16 x bf16, each op rounded                 DiTAttention.swift:206-234
 *   SDPA: fp32 logits * scale, fp32 softmax, fp32 P.V, bf16 out   DiTAttention.swift:377-381
 *   key padding = SDPA over the first n keys                 TextConditioningLayout.swift:94-107
 * mode 0 keeps every intermediate in fp32 (no bf16 rounding after the inputs); mode 1 rounds
 * to bf16 where the reference does (after the norm, after each RoPE multiply/add).
 *
 * Pinned by tests/test_oracle.py against the float64 numpy restatement (oracle.py), closed
 * forms and invariants. Threads: OpenMP over (head, query block).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    int32_t B, H, Lq, Lk, D;
    const uint16_t *q, *k, *v;                 /* bf16 bits, [B][L][H*D] contiguous      */
    const uint16_t *q_norm_w, *k_norm_w;       /* [H*D] or NULL                          */
    float eps;
    const uint16_t *q_cos, *q_sin;             /* [H][Lq][D/2] or NULL                   */
    const uint16_t *k_cos, *k_sin;             /* [H][Lk][D/2] or NULL (then q's)        */
    const int32_t *k_valid_len;                /* [B] or NULL                            */
    float scale;
    int32_t mode;                              /* 0: fp32 throughout; 1: reference rounding */
    int32_t h_begin, h_end;                    /* head subset [h_begin, h_end)           */
    int32_t q_begin, q_end;                    /* query subset [q_begin, q_end)          */
    int32_t threads;                           /* <= 0: OpenMP default                   */
    float *out;                                /* [B][q_end-q_begin][h_end-h_begin][D]   */
} oracle_args;

static inline float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float rbf(float f) {               /* round to bf16 (RNE) and back */
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

/* One token row: norm (over all H*D channels) then RoPE for heads [h0, h1), written as
 * float [h1-h0][D] into dst. */
static void prep_row(const uint16_t *row, int H, int D, const uint16_t *w, float eps,
                     const uint16_t *cos_t, const uint16_t *sin_t, int L, int l, int h0,
                     int h1, int mode, float *dst) {
    const int inner = H * D;
    float rstd = 1.0f;
    if (w) {
        double ss = 0.0;
        for (int i = 0; i < inner; ++i) {
            const double x = bf2f(row[i]);
            ss += x * x;
        }
        const float ms = (float)(ss / inner);
        rstd = 1.0f / sqrtf(ms + eps);
    }
    const int half = D / 2;
    for (int h = h0; h < h1; ++h) {
        float *o = dst + (size_t)(h - h0) * D;
        for (int d = 0; d < D; ++d) {
            float x = bf2f(row[h * D + d]);
            if (w) {
                x = (x * rstd) * bf2f(w[h * D + d]);
                if (mode == 1) x = rbf(x);
            }
            o[d] = x;
        }
        if (cos_t) {
            const uint16_t *cs = cos_t + ((size_t)h * L + l) * half;
            const uint16_t *sn = sin_t + ((size_t)h * L + l) * half;
            for (int j = 0; j < half; ++j) {
                const float x1 = o[j], x2 = o[j + half], c = bf2f(cs[j]), s = bf2f(sn[j]);
                if (mode == 1) {
                    o[j] = rbf(rbf(x1 * c) - rbf(x2 * s));
                    o[j + half] = rbf(rbf(x2 * c) + rbf(x1 * s));
                } else {
                    o[j] = x1 * c - x2 * s;
                    o[j + half] = x2 * c + x1 * s;
                }
            }
        }
    }
}

int oracle_attention(const oracle_args *a) {
    if (!a || a->B < 1 || a->H < 1 || a->Lq < 1 || a->Lk < 1 || a->D < 2 || (a->D & 1))
        return -1;
    const int B = a->B, H = a->H, D = a->D, Lq = a->Lq, Lk = a->Lk;
    const int h0 = a->h_begin, h1 = a->h_end, qb0 = a->q_begin, qb1 = a->q_end;
    if (h0 < 0 || h1 > H || h0 >= h1 || qb0 < 0 || qb1 > Lq || qb0 >= qb1) return -1;
    const int nh = h1 - h0, nq = qb1 - qb0, inner = H * D;
    const uint16_t *kcos = a->k_cos ? a->k_cos : a->q_cos;
    const uint16_t *ksin = a->k_sin ? a->k_sin : a->q_sin;
    if (a->q_cos && !a->k_cos && Lq != Lk) return -1;
#ifdef _OPENMP
    if (a->threads > 0) omp_set_num_threads(a->threads);
#endif
    for (int b = 0; b < B; ++b) {
        const int n = a->k_valid_len ? a->k_valid_len[b] : Lk;
        if (n < 1 || n > Lk) return -1;
        /* K' transposed per head: kT[h][d][j]; V as float [h][j][d]; Q' [q][h][d] */
        float *kT = (float *)malloc(sizeof(float) * (size_t)nh * D * n);
        float *vf = (float *)malloc(sizeof(float) * (size_t)nh * n * D);
        float *qf = (float *)malloc(sizeof(float) * (size_t)nq * nh * D);
        if (!kT || !vf || !qf) {
            free(kT); free(vf); free(qf);
            return -2;
        }
#pragma omp parallel
        {
            float *tmp = (float *)malloc(sizeof(float) * (size_t)nh * D);
#pragma omp for schedule(static)
            for (int j = 0; j < n; ++j) {
                const uint16_t *krow = a->k + ((size_t)b * Lk + j) * inner;
                prep_row(krow, H, D, a->k_norm_w, a->eps, kcos, ksin, Lk, j, h0, h1, a->mode, tmp);
                for (int h = 0; h < nh; ++h)
                    for (int d = 0; d < D; ++d) kT[((size_t)h * D + d) * n + j] = tmp[h * D + d];
                const uint16_t *vrow = a->v + ((size_t)b * Lk + j) * inner;
                for (int h = 0; h < nh; ++h)
                    for (int d = 0; d < D; ++d)
                        vf[((size_t)h * n + j) * D + d] = bf2f(vrow[(h0 + h) * D + d]);
            }
#pragma omp for schedule(static)
            for (int i = 0; i < nq; ++i) {
                const int l = qb0 + i;
                const uint16_t *qrow = a->q + ((size_t)b * Lq + l) * inner;
                prep_row(qrow, H, D, a->q_norm_w, a->eps, a->q_cos, a->q_sin, Lq, l, h0, h1,
                         a->mode, qf + (size_t)i * nh * D);
            }
            free(tmp);
        }
        /* SDPA, 4 queries at a time per (head, block) */
        const int QB = 4;
        const int nblk = (nq + QB - 1) / QB;
#pragma omp parallel
        {
            float *lg = (float *)malloc(sizeof(float) * (size_t)QB * n);
            float acc[4][256];
#pragma omp for schedule(dynamic, 4) collapse(2)
            for (int h = 0; h < nh; ++h) {
                for (int blk = 0; blk < nblk; ++blk) {
                    const int i0 = blk * QB;
                    const int cnt = (nq - i0) < QB ? (nq - i0) : QB;
                    const float *kh = kT + (size_t)h * D * n;
                    const float *vh = vf + (size_t)h * n * D;
                    for (int t = 0; t < QB; ++t) memset(lg + (size_t)t * n, 0, sizeof(float) * n);
                    for (int d = 0; d < D; ++d) {
                        float qd[4];
                        for (int t = 0; t < QB; ++t)
                            qd[t] = t < cnt ? qf[((size_t)(i0 + t) * nh + h) * D + d] : 0.f;
                        const float *kr = kh + (size_t)d * n;
                        float *l0 = lg, *l1 = lg + n, *l2 = lg + 2 * (size_t)n, *l3 = lg + 3 * (size_t)n;
                        for (int j = 0; j < n; ++j) {
                            const float kv = kr[j];
                            l0[j] += qd[0] * kv;
                            l1[j] += qd[1] * kv;
                            l2[j] += qd[2] * kv;
                            l3[j] += qd[3] * kv;
                        }
                    }
                    for (int t = 0; t < cnt; ++t) {
                        float *lr = lg + (size_t)t * n;
                        float mx = -INFINITY;
                        for (int j = 0; j < n; ++j) {
                            lr[j] *= a->scale;
                            mx = lr[j] > mx ? lr[j] : mx;
                        }
                        double sum = 0.0;
                        for (int j = 0; j < n; ++j) {
                            lr[j] = expf(lr[j] - mx);
                            sum += lr[j];
                        }
                        const float inv = (float)(1.0 / sum);
                        for (int j = 0; j < n; ++j) lr[j] *= inv;
                        for (int d = 0; d < D; ++d) acc[t][d] = 0.f;
                    }
                    for (int j = 0; j < n; ++j) {
                        const float *vr = vh + (size_t)j * D;
                        const float p0 = lg[j], p1 = cnt > 1 ? lg[n + j] : 0.f;
                        const float p2 = cnt > 2 ? lg[2 * (size_t)n + j] : 0.f;
                        const float p3 = cnt > 3 ? lg[3 * (size_t)n + j] : 0.f;
                        for (int d = 0; d < D; ++d) {
                            const float vv = vr[d];
                            acc[0][d] += p0 * vv;
                            acc[1][d] += p1 * vv;
                            acc[2][d] += p2 * vv;
                            acc[3][d] += p3 * vv;
                        }
                    }
                    for (int t = 0; t < cnt; ++t) {
                        float *o = a->out + (((size_t)b * nq + i0 + t) * nh + h) * D;
                        memcpy(o, acc[t], sizeof(float) * D);
                    }
                }
            }
            free(lg);
        }
        free(kT); free(vf); free(qf);
    }
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
