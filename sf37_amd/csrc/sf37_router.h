// sf37_router.h - router logits row and top-k selection, shared by the
// staged kernels (k_router.hip) and the fused decode route kernel, so both
// paths produce identical logits and selections.
#pragma once

#include "sf37_dev.h"

typedef float sf37_f32x4 __attribute__((ext_vector_type(4), aligned(4)));

// A 64-bit value moved between lanes by one DPP control (two 32-bit moves);
// lanes outside ROW_MASK or without a source keep their own value.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint64_t sf37_dpp64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xf, false);
    const uint32_t nhi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xf, false);
    return ((uint64_t)nhi << 32) | nlo;
}

__device__ __forceinline__ double sf37_readlane_f64(double v, uint32_t lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, (int)lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), (int)lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum over the 64 lanes of a wave, the same bits in every lane: pairs in
// each quad (lane ^ 1, then ^ 2), the two quads of each 8 (half mirror), the
// two halves of each row (mirror) - every lane adds the same two operands,
// so the row sum is identical across the row - then (r0 + r1) + (r2 + r3)
// over the four rows.
__device__ __forceinline__ double sf37_wave_sum_f64(double v) {
#define SF37_DPP_ADD(ctrl)                                                                                 \
    v = v + __builtin_bit_cast(double, sf37_dpp64<ctrl>(__builtin_bit_cast(uint64_t, v)))
    SF37_DPP_ADD(0xb1);   // quad_perm [1,0,3,2]
    SF37_DPP_ADD(0x4e);   // quad_perm [2,3,0,1]
    SF37_DPP_ADD(0x141);  // row_half_mirror
    SF37_DPP_ADD(0x140);  // row_mirror
#undef SF37_DPP_ADD
    return (sf37_readlane_f64(v, 0) + sf37_readlane_f64(v, 16)) + (sf37_readlane_f64(v, 32) + sf37_readlane_f64(v, 48));
}

// Router logits of NR consecutive expert rows (wr, row stride K; the
// first nr valid) for NT tokens x[t0 .. t0+NT) by a 256-thread workgroup,
// accumulated in binary64 (sf37.c:1970-1976): thread i owns k in
// [c*i, c*(i+1)) with c = K / 256 and accumulates them in order (the loads
// of up to 16 columns of every row and token issued before the first fma;
// the x slice is read once for all rows), then a DPP sum per wave
// (sf37_wave_sum_f64), and sf37_router_combine adds the four wave sums as
// (w0 + w1) + (w2 + w3).  K must be a multiple of 256.  store(r, t, wave, v)
// receives the wave sums; xf(t, k, v) maps each loaded x value (identity,
// or the row's normalisation).
struct sf37_x_identity {
    __device__ float operator()(uint32_t, uint32_t, float v) const { return v; }
};
struct sf37_no_pre {
    __device__ void operator()() const {}
};

template <int NR, int NT, class STORE, class XF = sf37_x_identity>
__device__ __forceinline__ void sf37_router_block(const float *wr, uint32_t nr, const float *x, uint32_t K,
                                                  uint32_t t0, STORE store, XF xf = XF()) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t c = K >> 8, k0 = threadIdx.x * c;
    double acc[NR][NT];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0;
    if ((c & 3u) == 0) {
        for (uint32_t kk = 0; kk < c; kk += 16u) {
            const uint32_t n4 = (c - kk) < 16u ? (c - kk) >> 2 : 4u;
            sf37_f32x4 wv[NR][4], xv[NT][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t jj = (uint32_t)j < n4 ? (uint32_t)j : 0u;     // loads stay in the pass
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const uint32_t rr = (uint32_t)r < nr ? (uint32_t)r : 0u;
                    wv[r][j] = *(const sf37_f32x4 *)(wr + (uint64_t)rr * K + k0 + kk + 4u * jj);
                }
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const uint32_t k = k0 + kk + 4u * jj;
                    xv[t][j] = *(const sf37_f32x4 *)(x + (uint64_t)(t0 + t) * K + k);
#pragma unroll
                    for (int q = 0; q < 4; q++) xv[t][j][q] = xf(t0 + (uint32_t)t, k + (uint32_t)q, xv[t][j][q]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if ((uint32_t)j < n4) {
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int r = 0; r < NR; r++)
#pragma unroll
                            for (int t = 0; t < NT; t++)
                                acc[r][t] = __builtin_fma((double)wv[r][j][q], (double)xv[t][j][q], acc[r][t]);
                }
            }
        }
    } else {
        for (uint32_t k = k0; k < k0 + c; k++) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const double wk = wr[(uint64_t)((uint32_t)r < nr ? r : 0) * K + k];
#pragma unroll
                for (int t = 0; t < NT; t++)
                    acc[r][t] = __builtin_fma(wk, (double)xf(t0 + (uint32_t)t, k, x[(uint64_t)(t0 + t) * K + k]),
                                              acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const double v = sf37_wave_sum_f64(acc[r][t]);
            if (lane == 0 && (uint32_t)r < nr) store((uint32_t)r, t0 + (uint32_t)t, wave, v);
        }
}

// NR rows, all T tokens, in passes of at most 8 tokens.
template <int NR, class STORE, class XF = sf37_x_identity>
__device__ __forceinline__ void sf37_router_rows_n(const float *wr, uint32_t nr, const float *x, uint32_t K, uint32_t T,
                                                   STORE store, XF xf = XF()) {
    for (uint32_t t0 = 0; t0 < T; t0 += 8u) {
        switch (T - t0 < 8u ? T - t0 : 8u) {
            case 1: sf37_router_block<NR, 1>(wr, nr, x, K, t0, store, xf); break;
            case 2: sf37_router_block<NR, 2>(wr, nr, x, K, t0, store, xf); break;
            case 3: sf37_router_block<NR, 3>(wr, nr, x, K, t0, store, xf); break;
            case 4: sf37_router_block<NR, 4>(wr, nr, x, K, t0, store, xf); break;
            case 5: sf37_router_block<NR, 5>(wr, nr, x, K, t0, store, xf); break;
            case 6: sf37_router_block<NR, 6>(wr, nr, x, K, t0, store, xf); break;
            case 7: sf37_router_block<NR, 7>(wr, nr, x, K, t0, store, xf); break;
            default: sf37_router_block<NR, 8>(wr, nr, x, K, t0, store, xf); break;
        }
    }
}

// One wave's share of NR router rows x NT tokens: the partials of chunk
// group cg (chunks 64 cg .. 64 cg + 63; chunk i owns k in [c i, c (i + 1)),
// c = K / 256, accumulated in order in binary64 as sf37_router_block does),
// each summed over the wave's 64 lanes by the balanced pairwise tree in
// lane order that sf37_wave_sum_f64 forms.  Here the tree is split through
// LDS: lane l writes its NR * NT partials to scr[v * 64 + l]; lane 8 v + g
// adds scr[v * 64 + 8 g .. + 7] as a balanced tree, and three DPP levels
// (lane ^ 1, lane ^ 2, the mirror within eight lanes) join the eight group
// sums of value v, so every value costs a few instructions instead of a DPP
// chain of its own.  store(r, t, v) receives value v = r * NT + t (from
// lane 8 v).  scr holds NR * NT * 64 doubles for this wave; NR * NT <= 8.
// pre() runs once after the first chunk's loads are issued and before xf is
// first applied (the fused norm forms its scales there while they load).
template <int NR, int NT, class STORE, class XF = sf37_x_identity, class PRE = sf37_no_pre>
__device__ __forceinline__ void sf37_router_wave(const float *wr, uint32_t nr, const float *x, uint32_t K,
                                                 uint32_t cg, uint32_t t0, double *scr, STORE store, XF xf = XF(),
                                                 PRE pre = PRE()) {
    static_assert(NR * NT <= 8, "eight values per wave at most");
    constexpr int NV = NR * NT;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = K >> 8, k0 = (cg * 64u + lane) * c;
    double acc[NR][NT];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0;
    if ((c & 3u) == 0) {
        for (uint32_t kk = 0; kk < c; kk += 16u) {
            const uint32_t n4 = (c - kk) < 16u ? (c - kk) >> 2 : 4u;
            sf37_f32x4 wv[NR][4], xv[NT][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t jj = (uint32_t)j < n4 ? (uint32_t)j : 0u;
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const uint32_t rr = (uint32_t)r < nr ? (uint32_t)r : 0u;
                    wv[r][j] = *(const sf37_f32x4 *)(wr + (uint64_t)rr * K + k0 + kk + 4u * jj);
                }
#pragma unroll
                for (int t = 0; t < NT; t++)
                    xv[t][j] = *(const sf37_f32x4 *)(x + (uint64_t)(t0 + t) * K + k0 + kk + 4u * jj);
            }
            if (kk == 0u) pre();
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if ((uint32_t)j < n4) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t k = k0 + kk + 4u * (uint32_t)j + (uint32_t)q;
#pragma unroll
                        for (int t = 0; t < NT; t++) {
                            const double xd = (double)xf(t0 + (uint32_t)t, k, xv[t][j][q]);
#pragma unroll
                            for (int r = 0; r < NR; r++)
                                acc[r][t] = __builtin_fma((double)wv[r][j][q], xd, acc[r][t]);
                        }
                    }
                }
            }
        }
    } else {
        pre();
        for (uint32_t k = k0; k < k0 + c; k++) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const double xd = (double)xf(t0 + (uint32_t)t, k, x[(uint64_t)(t0 + t) * K + k]);
#pragma unroll
                for (int r = 0; r < NR; r++)
                    acc[r][t] = __builtin_fma((double)wr[(uint64_t)((uint32_t)r < nr ? r : 0) * K + k], xd,
                                              acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) scr[(r * NT + t) * 64 + lane] = acc[r][t];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t v = lane >> 3 < (uint32_t)NV ? lane >> 3 : (uint32_t)NV - 1u;
    const double *g = scr + v * 64u + (lane & 7u) * 8u;
    double e[8];
#pragma unroll
    for (int i = 0; i < 8; i++) e[i] = g[i];
    double s = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    s = s + __builtin_bit_cast(double, sf37_dpp64<0xb1>(__builtin_bit_cast(uint64_t, s)));    // lane ^ 1
    s = s + __builtin_bit_cast(double, sf37_dpp64<0x4e>(__builtin_bit_cast(uint64_t, s)));    // lane ^ 2
    s = s + __builtin_bit_cast(double, sf37_dpp64<0x141>(__builtin_bit_cast(uint64_t, s)));   // 7 - lane in eight
    if ((lane & 7u) == 0 && (lane >> 3) < (uint32_t)NV) {
        const uint32_t vv = lane >> 3;
        store(vv / (uint32_t)NT, vv % (uint32_t)NT, s);
    }
}

// One row, all T tokens: part[t][wave] receives the wave sums.
__device__ __forceinline__ void sf37_router_rows(const float *wr, const float *x, uint32_t K, uint32_t T,
                                                 double (*part)[4]) {
    sf37_router_rows_n<1>(wr, 1u, x, K, T, [part](uint32_t, uint32_t t, uint32_t w, double v) { part[t][w] = v; });
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

// Selection candidate of expert e: p = sigmoid(logit), key of p + bias.
__device__ __forceinline__ uint64_t sf37_topk_candidate(float logit, float bias, uint32_t e, const uint64_t *tab,
                                                        float &p) {
    p = sf37_sigmoid_t(logit, tab);
    return sf37_topk_key(p + bias, e);
}

// Maximum of a 32-bit value over the wave, returned uniform: running maxima
// along each 16-lane row (row_shr 1, 2, 4, 8), row 0 into row 1 and row 2
// into row 3 (row_bcast:15), rows 0-1 into rows 2-3 (row_bcast:31); lane 63
// then holds the maximum.
__device__ __forceinline__ uint32_t sf37_wave_max_u32(uint32_t v) {
#define SF37_DPP_MAX32(ctrl, rows)                                                                     \
    do {                                                                                               \
        const uint32_t n_ = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, rows, 0xf, true);  \
        v = n_ > v ? n_ : v;                                                                           \
    } while (0)
    SF37_DPP_MAX32(0x111, 0xf);
    SF37_DPP_MAX32(0x112, 0xf);
    SF37_DPP_MAX32(0x114, 0xf);
    SF37_DPP_MAX32(0x118, 0xf);
    SF37_DPP_MAX32(0x142, 0xa);
    SF37_DPP_MAX32(0x143, 0xc);
#undef SF37_DPP_MAX32
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The k rounds of a wave arg-max over prepared candidates (sf37.c:2144-2157,
// sf37_cuda.cu:4866-4997): lane l holds experts l + 64j as keys (ordered
// score << 32 | ~e, 0 = none).  A lane keeps the score and expert of its
// best candidate (the smallest expert among equal scores); each round takes
// the wave maximum of the lanes' best scores, the lanes holding it by ballot
// - the smallest of their experts when several do - reads the winner's
// probability from its lane and removes it there, so ties go to the smaller
// expert index as in the reference's "score > best" scan.
// weights = p / max(sum p, 1e-20) * scale with the sum in slot order.  Lane
// k keeps slot k, so nothing is written until the end.  NTOK tokens are
// interleaved so their latencies overlap.
template <int NTOK, int NJ>
__device__ __forceinline__ void sf37_topk_rounds(uint64_t (&key)[NTOK][NJ], const float (&prob)[NTOK][NJ],
                                                 uint32_t topk, float scale, int32_t *const *sel_out,
                                                 float *const *w_out) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t sc[NTOK][NJ];
    uint32_t bs[NTOK], bj[NTOK];          // the lane's best score and its slot j
    float sum[NTOK], my_p[NTOK];
    int32_t my_sel[NTOK];
    auto lane_best = [&](int t) {
        uint32_t s = 0, jj = 0;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (sc[t][j] > s) {
                s = sc[t][j];
                jj = (uint32_t)j;
            }
        }
        bs[t] = s;
        bj[t] = jj;
    };
#pragma unroll
    for (int t = 0; t < NTOK; t++) {
#pragma unroll
        for (int j = 0; j < NJ; j++) sc[t][j] = (uint32_t)(key[t][j] >> 32);
        lane_best(t);
        sum[t] = 0.0f;
        my_p[t] = 0.0f;
        my_sel[t] = -1;
    }
    // kept rolled: this runs on one wave with a cold instruction cache, where
    // every extra line of code costs more than the loop
#pragma unroll 1
    for (uint32_t k = 0; k < topk; k++) {
        uint32_t m[NTOK];
#pragma unroll
        for (int t = 0; t < NTOK; t++) m[t] = sf37_wave_max_u32(bs[t]);
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            float pk = 0.0f;
            int32_t sk = -1;
            if (m[t] != 0) {
                const uint32_t be = lane + 64u * bj[t];
                uint64_t tied = __ballot(bs[t] == m[t]);
                uint32_t wl = (uint32_t)__builtin_ctzll(tied);
                uint32_t e = (uint32_t)__builtin_amdgcn_readlane((int)be, (int)wl);
                tied &= tied - 1u;
                while (tied) {                         // equal scores in several lanes
                    const uint32_t l2 = (uint32_t)__builtin_ctzll(tied);
                    const uint32_t e2 = (uint32_t)__builtin_amdgcn_readlane((int)be, (int)l2);
                    if (e2 < e) {
                        e = e2;
                        wl = l2;
                    }
                    tied &= tied - 1u;
                }
                float pb = 0.0f;
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    if ((uint32_t)j == bj[t]) pb = prob[t][j];
                pk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pb), (int)wl));
                sk = (int32_t)e;
                if (lane == wl) {
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        if ((uint32_t)j == bj[t]) sc[t][j] = 0;
                    lane_best(t);
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

// Top-k of NTOK tokens by one wave from logits: load(t, e) reads token t's
// logit e; the candidates are formed here (every load issued before the
// first is used), probs[t] (if not null) receives p.
template <int NTOK, int NJ, class LOAD>
__device__ __forceinline__ void sf37_wave_topk_n(LOAD load, const float *bias, uint32_t E, uint32_t topk,
                                                 float scale, const uint64_t *tab, int32_t *const *sel_out,
                                                 float *const *w_out, float *const *probs) {
    const uint32_t lane = threadIdx.x & 63u;
    float prob[NTOK][NJ];
    uint64_t key[NTOK][NJ];
    float lg[NTOK][NJ], bj[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t e = lane + 64u * j;
        const uint32_t ec = e < E ? e : 0u;                  // every lane reads a valid entry
        bj[j] = bias[ec];
#pragma unroll
        for (int t = 0; t < NTOK; t++) lg[t][j] = load(t, ec);
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t e = lane + 64u * j;
        const bool ok = e < E;
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            float p;
            const uint64_t kk = sf37_topk_candidate(lg[t][j], bj[j], e, tab, p);
            prob[t][j] = ok ? p : 0.0f;
            key[t][j] = ok ? kk : 0;
            if (ok && probs[t]) probs[t][e] = p;
        }
    }
    sf37_topk_rounds<NTOK, NJ>(key, prob, topk, scale, sel_out, w_out);
}

// Top-k of NTOK tokens by one wave from candidates formed elsewhere:
// cand(t, e, p) returns token t's key of expert e and sets p.
template <int NTOK, int NJ, class CAND>
__device__ __forceinline__ void sf37_wave_topk_cand_n(CAND cand, uint32_t E, uint32_t topk, float scale,
                                                      int32_t *const *sel_out, float *const *w_out) {
    const uint32_t lane = threadIdx.x & 63u;
    float prob[NTOK][NJ];
    uint64_t key[NTOK][NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t e = lane + 64u * j;
        const bool ok = e < E;
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
            key[t][j] = cand(t, ok ? e : 0u, prob[t][j]);
            if (!ok) {
                key[t][j] = 0;
                prob[t][j] = 0.0f;
            }
        }
    }
    sf37_topk_rounds<NTOK, NJ>(key, prob, topk, scale, sel_out, w_out);
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

template <int NTOK, class CAND>
__device__ __forceinline__ void sf37_wave_topk_cand(CAND cand, uint32_t E, uint32_t topk, float scale,
                                                    int32_t *const *sel_out, float *const *w_out) {
    switch ((E + 63u) >> 6) {
#define SF37_TOPK_CASE(nj) \
    case nj: sf37_wave_topk_cand_n<NTOK, nj>(cand, E, topk, scale, sel_out, w_out); break;
        SF37_TOPK_CASE(1) SF37_TOPK_CASE(2) SF37_TOPK_CASE(3) SF37_TOPK_CASE(4)
        SF37_TOPK_CASE(5) SF37_TOPK_CASE(6) SF37_TOPK_CASE(7) SF37_TOPK_CASE(8)
        SF37_TOPK_CASE(9) SF37_TOPK_CASE(10) SF37_TOPK_CASE(11) SF37_TOPK_CASE(12)
        SF37_TOPK_CASE(13) SF37_TOPK_CASE(14) SF37_TOPK_CASE(15) SF37_TOPK_CASE(16)
#undef SF37_TOPK_CASE
        default: break;
    }
}
