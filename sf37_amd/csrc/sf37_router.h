// sf37_router.h - router logits row and top-k selection, shared by the
// staged kernels (k_router.hip) and the fused decode route kernel, so both
// paths produce identical logits and selections.
#pragma once

#include "sf37_dev.h"

typedef float sf37_f32x4 __attribute__((ext_vector_type(4), aligned(4)));

// Router logits of one expert row for NT tokens x[t0 .. t0+NT) by a
// 256-thread workgroup, accumulated in binary64 (sf37.c:1970-1976): thread i
// owns k in [c*i, c*(i+1)) with c = K / 256 and accumulates them in order
// (all loads of the row slice issued before the first fma), then a
// butterfly per wave, and the host combines (w0 + w1) + (w2 + w3).  K must be
// a multiple of 256.  part[t0 + t][wave] receives the wave sums.
template <int NT>
__device__ __forceinline__ void sf37_router_row(const float *wr, const float *x, uint32_t K, uint32_t t0,
                                                double (*part)[4]) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t c = K >> 8, k0 = threadIdx.x * c;
    double acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0;
    if ((c & 3u) == 0) {
        for (uint32_t kk = 0; kk < c; kk += 16u) {
            // up to 16 columns per pass: 4 weight + 4*NT activation float4s
            const uint32_t n4 = (c - kk) < 16u ? (c - kk) >> 2 : 4u;
            sf37_f32x4 wv[4], xv[NT][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if ((uint32_t)j < n4) {
                    wv[j] = *(const sf37_f32x4 *)(wr + k0 + kk + 4u * j);
#pragma unroll
                    for (int t = 0; t < NT; t++)
                        xv[t][j] = *(const sf37_f32x4 *)(x + (uint64_t)(t0 + t) * K + k0 + kk + 4u * j);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if ((uint32_t)j < n4) {
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int t = 0; t < NT; t++)
                            acc[t] = __builtin_fma((double)wv[j][q], (double)xv[t][j][q], acc[t]);
                }
            }
        }
    } else {
        for (uint32_t k = k0; k < k0 + c; k++) {
            const double wv = wr[k];
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t] = __builtin_fma(wv, (double)x[(uint64_t)(t0 + t) * K + k], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        double v = acc[t];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) part[t0 + t][wave] = v;
    }
}

// All tokens of a row in passes of at most 4 (register budget).
__device__ __forceinline__ void sf37_router_rows(const float *wr, const float *x, uint32_t K, uint32_t T,
                                                 double (*part)[4]) {
    for (uint32_t t0 = 0; t0 < T; t0 += 4u) {
        switch (T - t0 < 4u ? T - t0 : 4u) {
            case 1: sf37_router_row<1>(wr, x, K, t0, part); break;
            case 2: sf37_router_row<2>(wr, x, K, t0, part); break;
            case 3: sf37_router_row<3>(wr, x, K, t0, part); break;
            default: sf37_router_row<4>(wr, x, K, t0, part); break;
        }
    }
}

__device__ __forceinline__ float sf37_router_combine(const double *p4) {
    return (float)((p4[0] + p4[1]) + (p4[2] + p4[3]));
}

// Order-preserving key of a selection candidate: larger score first, then
// smaller expert index.  NaN scores never win (key 0 = no candidate), as in
// the reference's "score > best" scan.
__device__ __forceinline__ uint64_t sf37_topk_key(float score, uint32_t e) {
    if (score != score) return 0;
    const uint32_t b = __builtin_bit_cast(uint32_t, score);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - e);
}

// Top-k of NTOK tokens by one wave, interleaved so their latencies overlap
// (sf37.c:2144-2157, sf37_cuda.cu:4866-4997): p = sigmoid(logit), score =
// p + bias, k rounds of a wave arg-max under (score desc, index asc);
// weights = p / max(sum p, 1e-20) * scale with the sum in slot order.  Lane
// l owns experts l + 64j, j < NJ (E <= 64 * NJ); lane k keeps slot k, so
// nothing is written until the end.  load(t, e) reads token t's logit e.
template <int NTOK, int NJ, class LOAD>
__device__ __forceinline__ void sf37_wave_topk_n(LOAD load, const float *bias, uint32_t E, uint32_t topk,
                                                 float scale, const uint64_t *tab, int32_t *const *sel_out,
                                                 float *const *w_out, float *const *probs) {
    const uint32_t lane = threadIdx.x & 63u;
    float prob[NTOK][NJ];
    uint64_t key[NTOK][NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t e = lane + 64u * j;
        const bool ok = e < E;
        const uint32_t ec = ok ? e : 0u;                     // every lane reads a valid entry
        const float bj = bias[ec];
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            const float p = sf37_sigmoid_t(load(t, ec), tab);
            prob[t][j] = ok ? p : 0.0f;
            key[t][j] = ok ? sf37_topk_key(p + bj, e) : 0;
            if (ok && probs[t]) probs[t][e] = p;
        }
    }
    float sum[NTOK], my_p[NTOK];
    int32_t my_sel[NTOK];
#pragma unroll
    for (int t = 0; t < NTOK; t++) {
        sum[t] = 0.0f;
        my_p[t] = 0.0f;
        my_sel[t] = -1;
    }
    for (uint32_t k = 0; k < topk; k++) {
        uint64_t wk[NTOK];
        float bp[NTOK];
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            uint64_t bk = 0;
            bp[t] = 0.0f;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                if (key[t][j] > bk) {
                    bk = key[t][j];
                    bp[t] = prob[t][j];
                }
            }
            wk[t] = bk;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
            for (int t = 0; t < NTOK; t++) {
                const uint64_t o = __shfl_xor(wk[t], off, 64);
                wk[t] = o > wk[t] ? o : wk[t];
            }
        }
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            float pk = 0.0f;
            int32_t sk = -1;
            if (wk[t] != 0) {
                const uint32_t e = 0xffffffffu - (uint32_t)wk[t];
                pk = __shfl(bp[t], (int)(e & 63u), 64);
                sk = (int32_t)e;
                if ((e & 63u) == lane) {
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        if ((uint32_t)j == (e >> 6)) key[t][j] = 0;
                }
            }
            sum[t] += pk;                            // slot order, every lane identical
            if (lane == k) {
                my_p[t] = pk;
                my_sel[t] = sk;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NTOK; t++) {
        const float s = sum[t] < 1.0e-20f ? 1.0e-20f : sum[t];
        if (lane < topk) {
            sel_out[t][lane] = my_sel[t];
            w_out[t][lane] = my_p[t] / s * scale;
        }
    }
}

// Dispatch on the number of 64-expert columns (E <= 1024).
template <int NTOK, class LOAD>
__device__ __forceinline__ void sf37_wave_topk(LOAD load, const float *bias, uint32_t E, uint32_t topk, float scale,
                                               const uint64_t *tab, int32_t *const *sel_out, float *const *w_out,
                                               float *const *probs) {
    switch ((E + 63u) >> 6) {
#define SF37_TOPK_CASE(nj) \
    case nj: sf37_wave_topk_n<NTOK, nj>(load, bias, E, topk, scale, tab, sel_out, w_out, probs); break;
        SF37_TOPK_CASE(1) SF37_TOPK_CASE(2) SF37_TOPK_CASE(3) SF37_TOPK_CASE(4)
        SF37_TOPK_CASE(5) SF37_TOPK_CASE(6) SF37_TOPK_CASE(7) SF37_TOPK_CASE(8)
        SF37_TOPK_CASE(9) SF37_TOPK_CASE(10) SF37_TOPK_CASE(11) SF37_TOPK_CASE(12)
        SF37_TOPK_CASE(13) SF37_TOPK_CASE(14) SF37_TOPK_CASE(15) SF37_TOPK_CASE(16)
#undef SF37_TOPK_CASE
        default: break;
    }
}
