// k_decode.hip - the MoE layer for decode batches (up to 16 tokens) on
// gfx950, in six launches on one stream (five for a single token, where
// the up launch takes the select work):
//
//   route   : router GEMV (binary64 accumulation) and each expert's
//             selection candidate (sigmoid, key), the Q8_K / Q8_0
//             quantisation of x (optionally RMSNorm of x first); zeroes the
//             item queues.
//   select  : one workgroup runs top-k for every token and groups the
//             (token, slot) pairs by expert; the others compute the shared
//             expert's Q8_0 gate/up rows (LDS tiles).
//   up      : routed Q3 gate/up: a lane owns one 110-byte block, a wave two
//             rows of gate and up, and the canonical block-order chain runs
//             as a DPP scan; items come from atomic queues.
//   mid     : SwiGLU * routing weight and the Q8_K of the routed mid; SwiGLU
//             and Q8_0 of the shared mid.
//   down    : routed Q2 down, one row per pair and output row, then the
//             shared expert's down rows from atomic queues (they fill the
//             routed part's tail).
//   combine : out = shared + sum over slots in slot order (optionally added
//             to the hidden state).
//
// Nothing waits on another wave, so every wave always runs to completion;
// the up and down kernels' queues hand out each item once and every wave
// stops at its first request past the end of its queue.
//
// Arithmetic is the canonical order of the oracle (sf37_blocks.h), the
// reference CPU order for the Q8_0 shared expert (sf37_ops.c:92-108), and
// slot-order combines, so results equal the staged kernels bit for bit.
#include "sf37_blocks.h"
#include "sf37_router.h"
#include "sf37_norm.h"
#include "sf37_launch.h"

namespace {

constexpr uint32_t DEC_MAX_TOK = 16;
constexpr uint32_t DEC_TPC = 4;      // pairs per pass in the routed kernels
constexpr uint32_t SH_RS_UP = 2;     // shared gate/up rows per 256-thread workgroup of the select launch
constexpr uint32_t SH_RS_UPSEL = 4;  // ... in the up launch (one token: fewer shared workgroups, so
                                     // more routed ones start beside them; 2 and 8 measured slower)
constexpr uint32_t SH_RS_SEL = 4;    // ... in the select launch (512 threads)
constexpr uint32_t DN_MAX_NB = 5;    // down blocks per row held in registers (F <= 1280)
constexpr uint32_t DN_TPC = 2;       // pairs per pass in the routed down kernel
constexpr uint32_t DN_STAGE = 4;     // pairs whose activation blocks a down wave keeps in LDS
static_assert(DN_STAGE % DN_TPC == 0, "a down pass stays inside one staged chunk");
constexpr uint32_t SHD_CHUNK = 4;    // shared-down Q8_0 blocks per load batch (even)
constexpr uint32_t SHD_MAX_BPS = 12; // shared-down blocks per lane (a multiple of SHD_CHUNK)
constexpr uint32_t UP_QUEUES = 64;   // queues of the up kernel's dynamic items, one per 128 bytes
constexpr uint32_t DN_QUEUES = 64;   // queues of the down kernel's shared-down rows, one per 128 bytes

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ uint32_t clamp_expert(int32_t e, uint32_t n) {
    return (e < 0 || (uint32_t)e >= n) ? 0u : (uint32_t)e;
}

// Expert ids a grouping sees: the E routed experts, and with SH9 the shared
// expert as id E.
__device__ __forceinline__ uint32_t n_ids(const sf37_dec_params &p) {
    return p.E + ((p.flags & SF37_DEC_SH9) ? 1u : 0u);
}

// With SH9 the shared expert's pairs (one per token) form groups of at
// most SH9_PAIRS pairs, so no up or down item holds more pairs than a
// routed expert shared by two tokens.
constexpr uint32_t SH9_PAIRS = 2;
__device__ __forceinline__ uint32_t expert_groups(const sf37_dec_params &p, uint32_t e, uint32_t pairs) {
    return (p.flags & SF37_DEC_SH9) && e == p.E ? (pairs + SH9_PAIRS - 1u) / SH9_PAIRS : (pairs ? 1u : 0u);
}

// Weight bytes of expert e of a matrix (w: the routed experts, exp_bytes
// apart; sh: the shared expert, id E with SH9).
__device__ __forceinline__ const uint8_t *expert_base(const sf37_dec_params &p, const uint8_t *w, const uint8_t *sh,
                                                      uint32_t e, uint64_t exp_bytes) {
    return e < p.E ? w + (uint64_t)e * exp_bytes : sh;
}

}  // namespace

using dec_params = sf37_dec_params;

namespace {

// Counters: the up kernel's item queues, then the down kernel's, 32 words
// apart (zeroed by the route kernel's first workgroup).
__device__ __forceinline__ uint32_t *up_queue(const dec_params &p, uint32_t q) { return p.cnt + 32u * q; }
__device__ __forceinline__ uint32_t *dn_queue(const dec_params &p, uint32_t q) {
    return p.cnt + 32u * (UP_QUEUES + q);
}
// Arrivals of the select launch's top-k workgroups (the last one groups): a
// spare word of up queue 0's stripe (the two are used by different launches).
__device__ __forceinline__ uint32_t *sel_arrivals(const dec_params &p) { return p.cnt + 16u; }

// Shared-down lane layout: the Q8_0 blocks of a row are split into S slices
// (a power of two <= 16 with S * T <= 64, so one token's slices sit in one
// 16-lane DPP row); lane = (row, token, slice).
__host__ __device__ constexpr uint32_t shd_slices(uint32_t T) { return T <= 4u ? 16u : (T <= 8u ? 8u : 4u); }
// Blocks per shared-down slice: ceil(nb8 / S) rounded up to even, so every
// slice and every load batch starts on a 4-byte boundary (rows are 4-byte
// aligned: nb8 is even).
__host__ __device__ constexpr uint32_t shd_bps(uint32_t nb8, uint32_t S) { return ((nb8 + S - 1u) / S + 1u) & ~1u; }

// LDS layout sizes, shared by the kernels and the host-side launch plan.
// A weight tile buffer holds the tile plus the copy's leading offset.
__host__ __device__ constexpr uint32_t tile_buf(uint32_t bytes) { return (bytes + 31u + 15u) & ~15u; }
__host__ __device__ constexpr uint32_t up_shared_tile(uint32_t K, uint32_t rs) { return rs * (K / 32u) * SF37_Q8_0_BYTES; }
// up workgroup: x of every token, then group info and sorted pairs
// An activation block in the up kernel's LDS, padded to 304 bytes so the 16
// blocks a wave reads at once spread over the LDS banks (a 288-byte stride
// puts every fourth block on the same banks).
struct act_lds_t {
    act_t a;
    uint32_t pad[4];
};
static_assert(sizeof(act_lds_t) == 304, "act_lds_t is 304 bytes");
__host__ __device__ constexpr size_t lds_up_meta(uint32_t K, uint32_t T, uint32_t G, uint32_t P) {
    return (size_t)T * (K / SF37_QK) * sizeof(act_lds_t) + (size_t)(3u + 2u * G + 2u * P) * 4u;
}
// Rows of 4, 8 or 16 blocks can run on block pairs streamed through LDS.
__host__ __device__ constexpr bool up_pairs(uint32_t K) {
    return K / SF37_QK == 4u || K / SF37_QK == 8u || K / SF37_QK == 16u;
}
__host__ __device__ constexpr size_t tile_base(uint32_t K, uint32_t T, uint32_t G, uint32_t P) {
    return (lds_up_meta(K, T, G, P) + 15u) & ~(size_t)15u;
}
// LDS of a routed up workgroup on the block-pair path: a 14 KiB tile per
// wave after the activations and tables.
__host__ __device__ constexpr size_t lds_up_dma(uint32_t K, uint32_t T, uint32_t G, uint32_t P, uint32_t waves) {
    return tile_base(K, T, G, P) + (size_t)waves * 14336u;
}
// Row stride (floats) of the shared gate/up terms: K/32 terms plus 4, so the
// sums' lanes, one row each, read 16 distinct bank quads.
__host__ __device__ constexpr uint32_t sh_red_stride(uint32_t K) { return K / 32u + 4u; }
__host__ __device__ constexpr size_t lds_up_shared(uint32_t K, uint32_t T, uint32_t rs) {
    return 2u * (size_t)tile_buf(up_shared_tile(K, rs)) + (size_t)T * 2u * rs * sh_red_stride(K) * 4u;
}

// Q8_0 block (34 bytes) at LDS byte offset L of base: scale, eight i8x4 words.
__device__ __forceinline__ float q8_0_lds(const uint8_t *base, uint32_t L, uint32_t q[8]) {
    const uint32_t *wp = (const uint32_t *)(base + (L & ~3u));
    const uint32_t o = L & 3u;
    uint32_t raw[10], a[9];
#pragma unroll
    for (int k = 0; k < 10; k++) raw[k] = wp[k];
#pragma unroll
    for (int k = 0; k < 9; k++) a[k] = align_bytes(raw[k + 1], raw[k], o);
#pragma unroll
    for (int k = 0; k < 8; k++) q[k] = align_bytes(a[k + 1], a[k], 2);
    return sf37_f16(a[0]);
}

// ---------------------------------------------------------------------------
// route
// ---------------------------------------------------------------------------

// Route workgroups [0, n_rt): workgroup u takes router rows 2 (u / ntg),
// +1 and tokens 4 (u % ntg) .. + 3 (ntg = ceil(T / 4)); with ROUTER, wave
// w forms the partial sums of quarter w (columns 1024 w .. + 1023) of those
// rows and tokens (sf37_router_wave, the order of the reference's
// 256-thread binary64 GEMV, sf37.c:1970-1976) and the logits are
// (q0 + q1) + (q2 + q3).  Then each (row, token)'s selection candidate
// (SELECT): p = sigmoid of the selecting logit, the key of p + bias.
// Workgroups [n_rt, ...) quantise x (one 256-block of one token per wave)
// to Q8_K for the routed experts and Q8_0 for the shared expert.  With
// NORM, x is the hidden state: the waves first form the RMSNorm scales of
// the tokens they use (sf37_rms_scale_wave, one wave per token) and
// normalise x as they load it.
__host__ __device__ constexpr uint32_t route_wgs(uint32_t T, uint32_t E) { return (E + 1u) / 2u * ((T + 3u) / 4u); }

// The exponential table in LDS from immediates (no memory load on the
// launch's critical path): thread i < 32 writes entry i.
__device__ __forceinline__ void stage_exp_tab_imm(uint64_t *tab) {
    if (threadIdx.x < 32u) {
        uint64_t v = 0;
#pragma unroll
        for (uint32_t i = 0; i < 32u; i++) v = threadIdx.x == i ? sf37_exp2_tab(i) : v;
        tab[threadIdx.x] = v;
    }
}

__global__ void __launch_bounds__(256) dec_route_kernel(dec_params p, uint32_t n_rt) {
    __shared__ double scr[4][8 * 64];                  // per wave: the partials' transposition
    __shared__ double part[2][4][4];                   // [row][token][quarter]
    __shared__ float s_scale[4];
    __shared__ uint64_t tab[32];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nb = p.K / SF37_QK;
    const bool norm = (p.flags & SF37_DEC_NORM) != 0u;
    if (blockIdx.x == 0) {   // the up and down kernels' item queues, the select arrivals
        if (threadIdx.x < UP_QUEUES) *up_queue(p, threadIdx.x) = 0u;
        if (threadIdx.x < DN_QUEUES) *dn_queue(p, threadIdx.x) = 0u;
        if (threadIdx.x == 0) *sel_arrivals(p) = 0u;
    }
    if (blockIdx.x >= n_rt) {
        const uint32_t wq = (blockIdx.x - n_rt) * 4u + wave;
        if (wq >= p.T * nb) return;
        const uint32_t t = wq / nb, b = wq - t * nb;
        const float scale = norm ? sf37_rms_scale_wave(p.x + (uint64_t)t * p.K, p.K, p.eps) : 0.0f;
        const uint32_t k0 = b * SF37_QK + 4u * lane;
        const float *xb = p.x + (uint64_t)t * p.K + k0;
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = xb[k];
        if (norm) {
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = sf37_norm_w1_bf16(v[k], scale, p.norm_w[k0 + k]);
            if (p.xn) {
#pragma unroll
                for (int k = 0; k < 4; k++) p.xn[(uint64_t)t * p.K + k0 + k] = v[k];
            }
        }
        int8_t qk[4];
        int gsum;
        const float d = q8k_codes4(v, qk, gsum);
        act_t *y = (act_t *)p.xq + wq;
        uint8_t *qb = (uint8_t *)y->qs;
#pragma unroll
        for (int k = 0; k < 4; k++) qb[q3x_pos(4u * lane + k)] = (uint8_t)qk[k];
        if (lane == 0) y->d = d;
        if ((lane & 15u) == 0) y->gs[lane >> 4] = gsum;
        if (p.flags & SF37_DEC_SHARED) {
            // Q8_0 (sf37_ops.c:57-90): a 32-wide block is 8 lanes
            float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
            amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            float d8 = 0.0f;
            uint32_t packed = 0;
            if (amax != 0.0f) {
                d8 = amax / 127.0f;
                const float is = 1.0f / d8;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float r = fminf(fmaxf(__builtin_rintf(is * v[k]), -128.0f), 127.0f);
                    packed |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * k);
                }
            }
            ((uint32_t *)(p.xq8 + (uint64_t)t * p.K + (uint64_t)b * SF37_QK))[lane] = packed;
            if ((lane & 7u) == 0) p.xs8[(uint64_t)t * (p.K / 32u) + b * 8u + (lane >> 3)] = d8;
        }
        return;
    }
    const uint32_t ntg = (p.T + 3u) / 4u;
    const uint32_t t0 = 4u * (blockIdx.x % ntg), e0 = 2u * (blockIdx.x / ntg);
    const uint32_t nt = p.T - t0 < 4u ? p.T - t0 : 4u, nr = p.E - e0 < 2u ? p.E - e0 : 2u;
    // RMSNorm scales of the group's tokens (one wave per token), formed
    // inside the router pass once its first loads are in flight
    const auto scales = [&]() {
        if (wave < nt) {
            const float sc = sf37_rms_scale_wave(p.x + (uint64_t)(t0 + wave) * p.K, p.K, p.eps);
            if (lane == 0) s_scale[wave] = sc;
        }
        __syncthreads();
    };
    stage_exp_tab_imm(tab);
    if (p.flags & SF37_DEC_ROUTER) {
        const float *wr = p.router_w + (uint64_t)e0 * p.K;
        const uint32_t cg = wave;
        const auto store = [cg](uint32_t r, uint32_t t, double v) { part[r][t][cg] = v; };
        if (norm) {
            const uint16_t *nw16 = p.norm_w;
            const auto xf = [nw16, t0](uint32_t t, uint32_t k, float v) {
                return sf37_norm_w1_bf16(v, s_scale[t - t0], nw16[k]);
            };
            switch (nt) {
                case 1: sf37_router_wave<2, 1>(wr, nr, p.x, p.K, cg, t0, scr[wave], store, xf, scales); break;
                case 2: sf37_router_wave<2, 2>(wr, nr, p.x, p.K, cg, t0, scr[wave], store, xf, scales); break;
                case 3: sf37_router_wave<2, 3>(wr, nr, p.x, p.K, cg, t0, scr[wave], store, xf, scales); break;
                default: sf37_router_wave<2, 4>(wr, nr, p.x, p.K, cg, t0, scr[wave], store, xf, scales); break;
            }
        } else {
            switch (nt) {
                case 1: sf37_router_wave<2, 1>(wr, nr, p.x, p.K, cg, t0, scr[wave], store); break;
                case 2: sf37_router_wave<2, 2>(wr, nr, p.x, p.K, cg, t0, scr[wave], store); break;
                case 3: sf37_router_wave<2, 3>(wr, nr, p.x, p.K, cg, t0, scr[wave], store); break;
                default: sf37_router_wave<2, 4>(wr, nr, p.x, p.K, cg, t0, scr[wave], store); break;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < 2u * nt) {
        const uint32_t r = threadIdx.x / nt, t = threadIdx.x - r * nt, e = e0 + r;
        if (r < nr) {
            float l = 0.0f;
            if (p.flags & SF37_DEC_ROUTER) {
                l = sf37_router_combine(part[r][t]);
                p.logits[(uint64_t)(t0 + t) * p.E + e] = l;
            }
            if (p.flags & SF37_DEC_SELECT) {
                const bool own = (p.flags & SF37_DEC_ROUTER) && p.logits_sel == p.logits;
                const float ls = own ? l : p.logits_sel[(uint64_t)(t0 + t) * p.E + e];
                float pr;
                p.cand_key[(uint64_t)(t0 + t) * p.E + e] = sf37_topk_candidate(ls, p.router_bias[e], e, tab, pr);
                p.cand_p[(uint64_t)(t0 + t) * p.E + e] = pr;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// select + shared gate/up
// ---------------------------------------------------------------------------

// Token t's top-k by one wave from the candidates the route launch formed
// (sf37_wave_topk_cand: k rounds of a wave arg-max, sf37.c:2144-2157);
// sel_out / w_out receive the k slots.
__device__ void token_topk(const dec_params &p, uint32_t t, int32_t *sel_out, float *w_out) {
    const uint64_t *ck = p.cand_key + (uint64_t)t * p.E;
    const float *cp = p.cand_p + (uint64_t)t * p.E;
    int32_t *so[1] = {sel_out};
    float *wo[1] = {w_out};
    const uint32_t sh9 = (p.flags & SF37_DEC_SH9) ? 1u : 0u;
    sf37_wave_topk_cand<1>(
        [ck, cp](uint32_t, uint32_t e, float &pr) {
            pr = cp[e];
            return ck[e];
        },
        p.E, p.topk - sh9, p.scale, so, wo);
    if (sh9 && (threadIdx.x & 63u) == 0u) {   // the shared expert's slot: id E, weight 1
        sel_out[p.topk - 1u] = (int32_t)p.E;
        w_out[p.topk - 1u] = 1.0f;
    }
}

// Inclusive sum over the wave's lanes (DPP row shifts, then rows 0-1 into
// 1-3), broadcast from lane 63 by the caller as needed.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);   // row_shr 1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);   // row_shr 2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);   // row_shr 4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);   // row_shr 8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);   // row_bcast 15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);   // row_bcast 31
    return v;
}

constexpr uint32_t GROUP_MAX_E = 1024;   // experts the token-mask grouping handles

// The P = T * topk (token, slot) pairs grouped by expert, stably in pair
// order: gi ([0] groups n, [1 + g] first sorted position of group g,
// [1 + n] = P, [2 + G + g] its expert) and so (sorted position -> pair), in
// the caller's LDS; publish also writes ginfo and sorted.  s_sel holds the
// P selected ids (invalid ids act as expert 0).  When no token holds one
// expert twice, pair i = t * topk + s of expert e goes to start(e) + the
// number of earlier tokens holding e (per-expert token masks, one scan over
// the experts); otherwise every pair counts the pairs ordered before it.
// scr: GROUP_SCR words of LDS.  All threads of the workgroup take part;
// ends with a barrier.
constexpr uint32_t GROUP_SCR = 2u * GROUP_MAX_E + 2u * DEC_MAX_TOK * 16u + 2u + 16u;   // words of scratch
__device__ void group_pairs(const dec_params &p, const uint32_t *s_sel, uint32_t *gi, uint32_t *so, bool publish,
                            uint32_t *scr) {
    uint32_t *msk = scr, *st = msk + GROUP_MAX_E;
    uint32_t *s_e = st + GROUP_MAX_E, *s_se = s_e + DEC_MAX_TOK * 16u;
    uint32_t *s_tot = s_se + DEC_MAX_TOK * 16u, *s_wcnt = s_tot + 2u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, nthr = blockDim.x;
    const uint32_t P = p.T * p.topk, ne = n_ids(p);
    if (p.flags & SF37_DEC_SLOTS) {
        if (threadIdx.x < p.topk) {
            const uint32_t s = threadIdx.x, e = clamp_expert((int32_t)s_sel[s], ne);
            so[s] = s;
            gi[1u + s] = s;
            gi[2u + p.G + s] = e;
            if (publish) {
                p.sorted[s] = s;
                p.ginfo[1u + s] = s;
                p.ginfo[2u + p.G + s] = e;
            }
        }
        if (threadIdx.x == 0) {
            gi[0] = p.topk;
            gi[1u + p.topk] = p.topk;
            if (publish) {
                p.ginfo[0] = p.topk;
                p.ginfo[1u + p.topk] = p.topk;
            }
        }
        __syncthreads();
        return;
    }
    const bool masks = ne <= GROUP_MAX_E;
    if (masks) {
        for (uint32_t e = threadIdx.x; e < ne; e += nthr) msk[e] = 0u;
        __syncthreads();
        if (threadIdx.x < P)
            atomicOr(&msk[clamp_expert((int32_t)s_sel[threadIdx.x], ne)], 1u << (threadIdx.x / p.topk));
        __syncthreads();
        if (wave == 0) {
            // lane l: experts [c l, c l + c); exclusive scans of the pair
            // counts and of the non-empty experts
            const uint32_t c = (ne + 63u) >> 6, e0 = lane * c;
            uint32_t n = 0, g = 0;
            for (uint32_t i = 0; i < c; i++) {
                const uint32_t e = e0 + i;
                if (e < ne) {
                    const uint32_t m = msk[e], pc = (uint32_t)__builtin_popcount(m);
                    n += pc;
                    g += expert_groups(p, e, pc);
                }
            }
            const uint32_t ni = wave_incl_sum(n), gin = wave_incl_sum(g);
            uint32_t np = ni - n, ge = gin - g;
            if (lane == 63u) {
                s_tot[0] = ni;
                s_tot[1] = gin;
            }
            for (uint32_t i = 0; i < c; i++) {
                const uint32_t e = e0 + i;
                if (e < ne) {
                    const uint32_t m = msk[e], pc = (uint32_t)__builtin_popcount(m), ng_e = expert_groups(p, e, pc);
                    st[e] = np;
                    for (uint32_t k = 0; k < ng_e; k++) {   // one group, or the shared expert's pair chunks
                        gi[1u + ge] = np + SH9_PAIRS * k;
                        gi[2u + p.G + ge] = e;
                        if (publish) {
                            p.ginfo[1u + ge] = np + SH9_PAIRS * k;
                            p.ginfo[2u + p.G + ge] = e;
                        }
                        ge++;
                    }
                    np += pc;
                }
            }
        }
        __syncthreads();
    }
    if (masks && s_tot[0] == P) {
        if (threadIdx.x == 0) {
            const uint32_t ng = s_tot[1];
            gi[0] = ng;
            gi[1u + ng] = P;
            if (publish) {
                p.ginfo[0] = ng;
                p.ginfo[1u + ng] = P;
            }
        }
        if (threadIdx.x < P) {
            const uint32_t i = threadIdx.x, e = clamp_expert((int32_t)s_sel[i], ne), t = i / p.topk;
            const uint32_t pos = st[e] + (uint32_t)__builtin_popcount(msk[e] & ((1u << t) - 1u));
            so[pos] = i;
            if (publish) p.sorted[pos] = i;
        }
        __syncthreads();
        return;
    }
    // a token holds an expert twice: each pair counts the pairs before it
    if (threadIdx.x < P) s_e[threadIdx.x] = clamp_expert((int32_t)s_sel[threadIdx.x], ne);
    __syncthreads();
    if (threadIdx.x < P) {
        const uint32_t i = threadIdx.x, e = s_e[i];
        uint32_t pos = 0;
#pragma unroll 8
        for (uint32_t q = 0; q < P; q++) {
            const uint32_t f = s_e[q];
            pos += (uint32_t)(f < e) + ((uint32_t)(f == e) & (uint32_t)(q < i));
        }
        so[pos] = i;
        if (publish) p.sorted[pos] = i;
        s_se[pos] = e;
    }
    __syncthreads();
    // groups start where the expert changes along the sorted order; the
    // group index is the count of starts before (ballot prefix per wave)
    const uint32_t i = threadIdx.x;
    const bool act = i < P;
    const uint32_t e = act ? s_se[i] : 0u;
    // the shared expert (SH9, id E: the last run of the sorted order, one
    // pair per token) starts a group every SH9_PAIRS pairs
    const bool sh_chunk = (p.flags & SF37_DEC_SH9) && e == p.E && (i - (P - p.T)) % SH9_PAIRS == 0u;
    const bool start = act && (i == 0u || s_se[i - 1u] != e || sh_chunk);
    const uint64_t m = __ballot(start);
    const uint32_t below = (uint32_t)__builtin_popcountll(m & ((1ull << lane) - 1ull));
    if (lane == 0) s_wcnt[wave] = (uint32_t)__builtin_popcountll(m);
    __syncthreads();
    uint32_t base = 0;
    for (uint32_t w = 0; w < wave; w++) base += s_wcnt[w];
    if (start) {
        gi[1u + base + below] = i;
        gi[2u + p.G + base + below] = e;
        if (publish) {
            p.ginfo[1u + base + below] = i;
            p.ginfo[2u + p.G + base + below] = e;
        }
    }
    if (i == P - 1u) {
        const uint32_t ng = base + below + (start ? 1u : 0u);
        gi[0] = ng;
        gi[1u + ng] = P;
        if (publish) {
            p.ginfo[0] = ng;
            p.ginfo[1u + ng] = P;
        }
    }
    __syncthreads();
}

// Top-k of every token inside one workgroup (one wave per token, waves
// looping) into s_sel / s_wts, or the selections read from sel when they
// are inputs; then the grouping.  publish: this workgroup also writes sel
// and wts (SELECT), ginfo and sorted.  Used by the up launch when it runs
// the select step itself (UPSEL).
__device__ void select_and_group(const dec_params &p, uint32_t *gi, uint32_t *so, bool publish) {
    __shared__ int32_t s_sel[DEC_MAX_TOK * 16];
    __shared__ float s_wts[DEC_MAX_TOK * 16];
    __shared__ uint32_t scr[GROUP_SCR];
    const uint32_t wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t P = p.T * p.topk;
    if (p.flags & SF37_DEC_SELECT) {
        for (uint32_t t = wave; t < p.T; t += nw) token_topk(p, t, s_sel + t * p.topk, s_wts + t * p.topk);
    } else if (threadIdx.x < P) {
        s_sel[threadIdx.x] = p.sel[threadIdx.x];
    }
    __syncthreads();
    if (publish && (p.flags & SF37_DEC_SELECT) && threadIdx.x < P) {
        p.sel[threadIdx.x] = s_sel[threadIdx.x];
        p.wts[threadIdx.x] = s_wts[threadIdx.x];
    }
    group_pairs(p, (const uint32_t *)s_sel, gi, so, publish, scr);
}

// Shared gate/up workgroup wg (the leading workgroups of the up launch):
// rs shared gate/up rows - the weight tiles copied to LDS while the x
// blocks of the first 8 tokens load, the terms in LDS, then the
// reference's sequential block sum per (matrix, token, row)
// (sf37_ops.c:92-108) into sh_gu.
__device__ void shared_gate_up(const dec_params &p, uint32_t wg, unsigned char *smem, uint32_t rs) {
    const uint32_t nb8 = p.K / 32u;
    const uint32_t row0 = wg * rs;
    const uint32_t tbytes = up_shared_tile(p.K, rs), wbuf = tile_buf(tbytes);
    const uint64_t row_bytes = (uint64_t)nb8 * SF37_Q8_0_BYTES;
    uint8_t *wl = smem;                                             // gate tile | up tile
    float *red = (float *)(smem + 2u * wbuf);                       // [T][2][RS][rstr]
    const uint32_t rstr = sh_red_stride(p.K);
    const uint32_t og = lds_copy(wl, p.sh_gate + (uint64_t)row0 * row_bytes, tbytes);
    const uint32_t ou = wbuf + lds_copy(wl + wbuf, p.sh_up + (uint64_t)row0 * row_bytes, tbytes);
    // thread = (row, block) for both matrices; x blocks of 8 tokens at a time
    u32x4 xa[8], xb[8];
    float xs[8];
    auto load_x = [&](uint32_t b, uint32_t t0) {
#pragma unroll
        for (uint32_t j = 0; j < 8u; j++) {
            const uint32_t t = t0 + j < p.T ? t0 + j : p.T - 1u;
            const u32x4 *xp = (const u32x4 *)(p.xq8 + (uint64_t)t * p.K + (uint64_t)b * 32u);
            xa[j] = xp[0];
            xb[j] = xp[1];
            xs[j] = p.xs8[(uint64_t)t * nb8 + b];
        }
    };
    if (threadIdx.x < rs * nb8) load_x(threadIdx.x % nb8, 0);
    lds_copy_wait();
    for (uint32_t rb = threadIdx.x; rb < rs * nb8; rb += blockDim.x) {
        const uint32_t r = rb / nb8, b = rb - r * nb8;
        uint32_t qg[8], qu[8];
        const float wg = q8_0_lds(wl, og + rb * SF37_Q8_0_BYTES, qg);
        const float wu = q8_0_lds(wl, ou + rb * SF37_Q8_0_BYTES, qu);
        for (uint32_t t0 = 0; t0 < p.T; t0 += 8u) {
            if (rb != threadIdx.x || t0 != 0u) load_x(b, t0);
#pragma unroll
            for (uint32_t j = 0; j < 8u; j++) {
                if (t0 + j < p.T) {
                    const uint32_t t = t0 + j;
                    const uint32_t xv[8] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w, xb[j].x, xb[j].y, xb[j].z, xb[j].w};
                    int32_t ig = 0, iu = 0;
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        ig = sdot4(qg[k], xv[k], ig);
                        iu = sdot4(qu[k], xv[k], iu);
                    }
                    red[((t * 2u + 0u) * rs + r) * rstr + b] = (float)ig * wg * xs[j];
                    red[((t * 2u + 1u) * rs + r) * rstr + b] = (float)iu * wu * xs[j];
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < p.T * 2u * rs; i += blockDim.x) {
        const uint32_t t = i / (2u * rs), mr = i - t * 2u * rs;
        const uint32_t m = mr / rs, r = mr - m * rs;
        const float *rv = red + (uint64_t)i * rstr;
        float acc = 0.0f;
        if ((nb8 & 15u) == 0) {
            // the same sequential sum; 16 terms read per step so the LDS
            // latency is paid once per step, not once per term
            for (uint32_t b = 0; b < nb8; b += 16u) {
                float4 v[4];
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = *(const float4 *)(rv + b + 4u * j);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc = acc + v[j].x;
                    acc = acc + v[j].y;
                    acc = acc + v[j].z;
                    acc = acc + v[j].w;
                }
            }
        } else {
            for (uint32_t b = 0; b < nb8; b++) acc = acc + rv[b];
        }
        p.sh_gu[((uint64_t)m * p.T + t) * p.F + row0 + r] = acc;
    }
}

// ---------------------------------------------------------------------------
// routed gate/up
// ---------------------------------------------------------------------------

// 28 dwords of a Q3 block from the dword boundary at or below p, as seven
// 16-byte loads (dword alignment suffices on gfx950).
__device__ __forceinline__ void load_q3(uint32_t w[28], const uint8_t *p) {
    const u32x4a4 *q = (const u32x4a4 *)(p - ((uintptr_t)p & 3u));
#pragma unroll
    for (int i = 0; i < 7; i++) {
        const u32x4a4 v = q[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
}

// Block value blk = sum_g fma(s_g, I_g) of one realigned Q3 block (a[0..26])
// against NT activations (act_t in LDS, Q3 layout), in group order.
template <int NT>
__device__ __forceinline__ void q3_block_dots(const uint32_t *a, const act_t *const *x, float bs[4]) {
#pragma unroll
    for (int t = 0; t < NT; t++) bs[t] = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t c0[8], c1[8];
        q3_unpack32(a, 12 + 24 * g, c0);
        q3_unpack32(a, 24 + 24 * g, c1);
        const int32_t zp = (int32_t)((a[2] >> (8 * g)) & 7u);
        const float sc = sf37_f16(a[g >> 1] >> (16 * (g & 1)));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const u32x4 *xq = (const u32x4 *)&x[t]->qs[16 * g];
            int32_t acc = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const u32x4 v0 = xq[2 * h], v1 = xq[2 * h + 1];
                const uint32_t *c = h ? c1 : c0;
                acc = sdot4(c[0], v0.x, acc);
                acc = sdot4(c[1], v0.y, acc);
                acc = sdot4(c[2], v0.z, acc);
                acc = sdot4(c[3], v0.w, acc);
                acc = sdot4(c[4], v1.x, acc);
                acc = sdot4(c[5], v1.y, acc);
                acc = sdot4(c[6], v1.z, acc);
                acc = sdot4(c[7], v1.w, acc);
            }
            bs[t] = __builtin_fmaf(sc, (float)(acc - __mul24(zp, x[t]->gs[g])), bs[t]);
        }
    }
}

// acc = fma(d_b, bs_b, acc) over the blocks b = 0..nb-1 held by lanes 0..nb-1
// of each 16-lane row: a scan with row_shr:1, exact canonical order, for NT
// tokens at once (their steps interleave).  The row's total ends in lane
// nb-1.  Unrolled for 16 blocks (K = 4096).
template <int NT>
__device__ __forceinline__ void block_chains(const float *d, const float *bs, float *acc, uint32_t nb) {
    auto step = [&]() {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float prev = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc[t]), 0x111, 0xf, 0xf, true));
            acc[t] = __builtin_fmaf(d[t], bs[t], prev);
        }
    };
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = __builtin_fmaf(d[t], bs[t], 0.0f);
    if (nb == 16u) {
#pragma unroll
        for (int st = 1; st < 16; st++) step();
    } else {
        for (uint32_t st = 1; st < nb; st++) step();
    }
}

// Keeps the compiler from hoisting work on w out of a loop (an empty asm
// that may change the registers), so unpacked codes are not all kept live.
template <int N>
__device__ __forceinline__ void opaque(uint32_t *w) {
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(w[i]));
}

// Shared down: sh_out[t][row] = sum over Q8_0 blocks b in order of
// (isum_b * ws_b) * xs_b (sf37_ops.c:92-108) for R = 64 / (T * S) rows.
// Lane = (row, token, slice): the slice holds bps consecutive blocks, loaded
// in NB batches of SHD_CHUNK (up to two batches in registers at a time), and
// computes their terms; the sequential sum then walks the slices in order with
// row_shr:1 (each slice adds its terms to the previous slice's total).  The
// shared mid codes and scales of every token are in LDS (xq: T x F codes,
// xsc: T x F/32 scales).  store(t, row, v) takes each (row, token) total.
template <int NB, typename STORE>
__device__ void shared_down_pass(const dec_params &p, const int8_t *xq, const float *xsc, uint32_t r0,
                                 STORE &&store) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t S = shd_slices(p.T), TS = p.T * S, R = 64u / TS;
    const uint32_t nb8 = p.F / 32u, bps = shd_bps(nb8, S), ns = (nb8 + bps - 1u) / bps;
    const uint32_t nbat = (bps + SHD_CHUNK - 1u) / SHD_CHUNK;
    const uint32_t rsub = lane / TS, li = lane - rsub * TS, t = li / S, j = li - t * S;
    const bool lane_ok = rsub < R;
    const uint32_t tc = lane_ok ? t : 0u;
    const uint64_t row_bytes = (uint64_t)nb8 * SF37_Q8_0_BYTES;
    const uint32_t row = r0 + (lane_ok ? rsub : 0u);
    const uint32_t rowc = row < p.K ? row : p.K - 1u;
    (void)nbat;
    // batches in groups of GR, each group's loads issued before its first
    // block is used: all batches together when there are at most 2, one at
    // a time when 3 (registers)
    constexpr uint32_t GR = NB <= 2 ? (uint32_t)NB : 1u;
    float term[SHD_MAX_BPS];
#pragma unroll
    for (uint32_t c0 = 0; c0 < (uint32_t)NB; c0 += GR) {
        uint32_t w[GR][36];
#pragma unroll
        for (uint32_t cc = 0; cc < GR; cc++) {
            if (c0 + cc < (uint32_t)NB) {
                const uint32_t c = c0 + cc;
                // blocks [b0, b0 + nv) of this batch; nv = 0 past the slice or row
                const uint32_t b0 = j * bps + c * SHD_CHUNK;
                const uint32_t in_slice = bps > c * SHD_CHUNK ? bps - c * SHD_CHUNK : 0u;
                const uint32_t in_row = nb8 > b0 ? nb8 - b0 : 0u;
                uint32_t nv = in_slice < in_row ? in_slice : in_row;
                nv = nv < SHD_CHUNK ? nv : SHD_CHUNK;
                const u32x4a4 *q = (const u32x4a4 *)(p.sh_down + (uint64_t)rowc * row_bytes +
                                                     (uint64_t)(nv ? b0 : 0u) * SF37_Q8_0_BYTES);
#pragma unroll
                for (uint32_t i = 0; i < 9; i++) {
                    // dwords past the batch re-read its first 16 bytes: every load
                    // stays within the batch's blocks (+ < 16 bytes), unpredicated
                    const u32x4a4 v = q[16u * i < nv * SF37_Q8_0_BYTES ? i : 0u];
                    w[cc][4 * i] = v.x;
                    w[cc][4 * i + 1] = v.y;
                    w[cc][4 * i + 2] = v.z;
                    w[cc][4 * i + 3] = v.w;
                }
            }
        }
#pragma unroll
        for (uint32_t cc = 0; cc < GR; cc++) {
            if (c0 + cc < (uint32_t)NB) {
                const uint32_t c = c0 + cc, b0 = j * bps + c * SHD_CHUNK;
#pragma unroll
                for (uint32_t i = 0; i < SHD_CHUNK; i++) {
                    const uint32_t B = 34u * i, d0 = B / 4u;            // compile-time offset in the batch
                    const uint32_t bg = b0 + i;
                    const uint32_t b = bg < nb8 ? bg : 0u;
                    const u32x4 *xp = (const u32x4 *)(xq + (uint64_t)tc * p.F + (uint64_t)b * 32u);
                    const u32x4 x0 = xp[0], x1 = xp[1];
                    const uint32_t xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    int32_t isum = 0;
                    float ws;
                    if ((B & 3u) == 0u) {
                        ws = sf37_f16(w[cc][d0]);
#pragma unroll
                        for (int k = 0; k < 8; k++) isum = sdot4(align_bytes(w[cc][d0 + k + 1], w[cc][d0 + k], 2), xv[k], isum);
                    } else {
                        ws = sf37_f16(w[cc][d0] >> 16);
#pragma unroll
                        for (int k = 0; k < 8; k++) isum = sdot4(w[cc][d0 + 1 + k], xv[k], isum);
                    }
                    term[c * SHD_CHUNK + i] = (float)isum * ws * xsc[(uint64_t)tc * nb8 + b];
                }
            }
        }
        // the next group's loads are not hoisted above these terms
#pragma unroll
        for (uint32_t i = 0; i < GR * SHD_CHUNK; i++)
            if (c0 * SHD_CHUNK + i < (uint32_t)NB * SHD_CHUNK) asm volatile("" : "+v"(term[c0 * SHD_CHUNK + i]));
        __builtin_amdgcn_sched_barrier(0);
    }
    // sequential sum over the slices of each (row, token)
    float acc = 0.0f;
    for (uint32_t st = 0; st < ns; st++) {
        const float prev =
            __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x111, 0xf, 0xf, true));
        if (j == st) {
            float a2 = st == 0u ? 0.0f : prev;
#pragma unroll
            for (uint32_t i = 0; i < (uint32_t)NB * SHD_CHUNK; i++)
                if (i < bps && j * bps + i < nb8) a2 = a2 + term[i];
            acc = a2;
        }
    }
    if (lane_ok && j == ns - 1u && row < p.K) store(t, row, acc);
}

// ---------------------------------------------------------------------------
// routed gate/up on block pairs
// ---------------------------------------------------------------------------
// A lane owns the block pair (2j, 2j+1) of one weight row: 220 bytes that
// start on a 4-byte boundary (rows are 1760-byte multiples of 220 apart), read
// as 14 dwordx4 loads.  The even block sits at byte 0 and the odd one at byte
// 110 of the lane's registers, both compile-time offsets, so no lane
// realigns its data.  A wave owns 64 / NBP rows (NBP = K / 512 pairs per
// row) of one matrix of one group's expert; the chain over the row's blocks
// runs over the NBP lanes of the row, two blocks per step.
constexpr uint32_t PAIR_DW = 56;      // dwords of a lane's pair in registers (55 used)
constexpr uint32_t TILE_BYTES = 14080; // an item: 64 pairs of 220 bytes, contiguous in the matrix
constexpr uint32_t TILE_LOADS = 14;    // 16-byte loads per lane to move a tile (64 x 16 bytes each)
constexpr uint32_t TILE_LDS = TILE_LOADS * 1024u;   // a wave's LDS tile
static_assert(TILE_BYTES <= TILE_LDS, "tile fits its LDS slot");
static_assert(TILE_LDS == 14336u, "lds_up_dma sizes a wave's tile as 14336 bytes");
static_assert(64u * 55u * 4u <= TILE_BYTES, "a lane's pair (55 dwords at 220 * lane) lies inside the tile");

// Byte B / the f16 at even byte B of the dword array w (B folds to a constant).
__device__ __forceinline__ uint32_t w_byte(const uint32_t *w, int B) { return (w[B >> 2] >> (8 * (B & 3))) & 0xffu; }
__device__ __forceinline__ float w_f16(const uint32_t *w, int B) { return sf37_f16(w[B >> 2] >> (8 * (B & 3))); }

// bs[t] = sum_g fma(s_g, I_g) (group order) of the Q3 block at byte BB of w
// against NT activation blocks in LDS (Q3 act layout).
template <int NT, int BB>
__device__ __forceinline__ void q3_block_dots_at(const uint32_t *w, const act_t *const *x, float (&bs)[4]) {
#pragma unroll
    for (int t = 0; t < NT; t++) bs[t] = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t c0[8], c1[8];
        q3_unpack32(w, BB + 12 + 24 * g, c0);
        q3_unpack32(w, BB + 24 + 24 * g, c1);
        const int32_t zp = (int32_t)(w_byte(w, BB + 8 + g) & 7u);
        const float sc = w_f16(w, BB + 2 * g);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const u32x4 *xq = (const u32x4 *)&x[t]->qs[16 * g];
            int32_t acc = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const u32x4 v0 = xq[2 * h], v1 = xq[2 * h + 1];
                const uint32_t *c = h ? c1 : c0;
                acc = sdot4(c[0], v0.x, acc);
                acc = sdot4(c[1], v0.y, acc);
                acc = sdot4(c[2], v0.z, acc);
                acc = sdot4(c[3], v0.w, acc);
                acc = sdot4(c[4], v1.x, acc);
                acc = sdot4(c[5], v1.y, acc);
                acc = sdot4(c[6], v1.z, acc);
                acc = sdot4(c[7], v1.w, acc);
            }
            bs[t] = __builtin_fmaf(sc, (float)(acc - __mul24(zp, x[t]->gs[g])), bs[t]);
        }
    }
}

// acc = fma(d_b, blk_b, acc) over the row's blocks in order, two per lane:
// step s takes the previous lane's total (row_shr:1) and adds blocks 2s,
// 2s+1.  The row's segment of NBP lanes sits inside one 16-lane DPP row;
// after NBP - 1 steps its last lane holds the exact chain (a value that
// entered the segment from the previous one cannot reach its last lane).
template <int NT, int NBP>
__device__ __forceinline__ void pair_chains(const float (&dE)[4], const float (&bE)[4], const float (&dO)[4],
                                            const float (&bO)[4], float (&acc)[4]) {
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = __builtin_fmaf(dO[t], bO[t], __builtin_fmaf(dE[t], bE[t], 0.0f));
#pragma unroll
    for (int st = 1; st < NBP; st++) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float prev = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc[t]), 0x111, 0xf, 0xf, true));
            acc[t] = __builtin_fmaf(dO[t], bO[t], __builtin_fmaf(dE[t], bE[t], prev));
        }
    }
}

// LDS direct loads (global -> LDS, no registers), issued through inline asm
// so the compiler neither waits for them before unrelated LDS reads nor
// tracks them: the loop waits for them itself (s_waitcnt vmcnt).  Lane i of
// a dwordx4 load writes LDS bytes [m0 + 16 i, m0 + 16 i + 16); one wait
// state separates the M0 write from the load.  m0 cannot be named as a
// clobber; in the gfx950 assembly of this kernel every other m0 write sits
// right before the compiler's own LDS direct loads of the shared gate/up
// path (lds_copy), which never run in the same wave as these.
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, const uint8_t *base) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(
                     __builtin_amdgcn_readfirstlane(lds)),
                 "v"(voff), "s"(sb)
                 : "memory");
}

// The routed items of the up launch on block pairs (K = 512 * NBP).  An
// item is RPI = 64 / NBP rows of one matrix (gate or up) of one group's
// expert: 14080 contiguous bytes, moved by fully coalesced LDS direct loads
// (load i of lane l = bytes 16 (64 i + l)) into the wave's LDS tile one item
// ahead of the compute; each lane reads its block pair (220 bytes at 220 *
// lane) into registers, the tile is refilled with the next item, and the pair
// is computed while it loads.  xs holds each token's activation blocks with
// the even blocks first, then the odd ones (bank-conflict-free: the NBP lanes
// of a row read NBP distinct blocks 304 bytes apart).  Wave w takes items w,
// w + nw, ... up to 70% of them, then items from counters (the up queues),
// which evens out the waves' finishing times.
constexpr uint32_t ITEM_NONE = 0xffffffffu;
// Items of the DMA up launch dealt round-robin before the counters take
// over: 90 % up to 8 tokens, 80 % above, where fewer waves share a CU
// (measured best at 8 and 16 tokens); a multiple of the waves.
__device__ __forceinline__ uint32_t up_static_items(uint32_t n_items, uint32_t nw, uint32_t T) {
    return nw * ((n_items * (T <= 8u ? 9u : 8u) / 10u) / nw);
}
template <int NBP>
__device__ void up_items_pairs(const dec_params &p, const uint32_t *gi, const uint32_t *so, const uint32_t *xo,
                               const act_lds_t *xs, uint8_t *tile, uint32_t gw, uint32_t nw, bool prefilled) {
    constexpr uint32_t RPI = 64u / (uint32_t)NBP;           // rows per item
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r = lane / (uint32_t)NBP, j = lane % (uint32_t)NBP;
    const bool out_lane = j == (uint32_t)NBP - 1u;
    const uint32_t nbK = 2u * (uint32_t)NBP;
    const uint32_t ipm = p.F / RPI, ipg = 2u * ipm, n_items = gi[0] * ipg;
    const uint64_t row_bytes = (uint64_t)nbK * SF37_Q3_BYTES, exp_bytes = (uint64_t)p.F * row_bytes;
    // items [0, n_stat) round-robin (wave gw: gw, gw + nw, ...); the rest
    // from counters, each asked for after a compute while the next tile
    // loads
    const uint32_t n_stat = up_static_items(n_items, nw, p.T);
    // the dynamic items are split over UP_QUEUES counters, each owning a
    // contiguous share (one counter for every wave of the chip serialises
    // the requests); a queue's waves come from every XCD (workgroups are
    // dealt to the XCDs round-robin), so a slower XCD hands work to faster
    // ones
    const uint32_t qi = ((gw >> 6) * 8u + (gw & 7u)) % UP_QUEUES, n_dyn = n_items - n_stat;
    const uint32_t q0 = n_stat + (uint32_t)((uint64_t)n_dyn * qi / UP_QUEUES);
    const uint32_t q1 = n_stat + (uint32_t)((uint64_t)n_dyn * (qi + 1u) / UP_QUEUES);
    uint32_t *ctr = up_queue(p, qi);
    uint32_t pos = gw;
    bool more = n_dyn != 0u;
    // the wave's next item (ITEM_NONE at the end).  A dynamic one is lane 0's
    // atomic add on the counter, issued and awaited in one asm statement (the
    // wait also covers the tile in flight, which the loop needs next anyway),
    // so no register is read before the answer has arrived
    auto next = [&]() -> uint32_t {
        if (pos < n_stat) {
            const uint32_t v = pos;
            pos += nw;
            return v;
        }
        if (!more) return ITEM_NONE;
        uint32_t v = 0;
        if (lane == 0) {
            const uint32_t one = 1u;
            asm volatile("global_atomic_add %0, %1, %2, off sc0\n\ts_waitcnt vmcnt(0)"
                         : "=&v"(v) : "v"(ctr), "v"(one) : "memory");
        }
        v = q0 + (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
        if (v < q1) return v;
        more = false;
        return ITEM_NONE;
    };
    // an item's RPI rows are one contiguous 14080-byte span of the matrix
    auto tile_src = [&](uint32_t it) -> const uint8_t * {
        const uint32_t g = it / ipg, r2 = it - g * ipg;
        const uint32_t m = r2 >= ipm ? 1u : 0u, k = r2 - m * ipm;
        const uint8_t *W = expert_base(p, m ? p.up_w : p.gate_w, m ? p.sh_up : p.sh_gate, gi[2u + p.G + g], exp_bytes);
        return W + (uint64_t)(k * RPI) * row_bytes;
    };
    const uint32_t tile_lds = (uint32_t)(uintptr_t)tile;
    auto fill = [&](uint32_t it) {
        const uint8_t *src = tile_src(it);
        constexpr uint32_t last = TILE_BYTES / 16u - 1u;
#pragma unroll
        for (uint32_t i = 0; i < TILE_LOADS; i++) {
            const uint32_t c = i * 64u + lane;
            dma16(tile_lds + 1024u * i, 16u * (c < last ? c : last), src);
        }
    };
    auto compute = [&](uint32_t (&w)[PAIR_DW], uint32_t it) {
        const uint32_t g = it / ipg, r2 = it - g * ipg;
        const uint32_t m = r2 >= ipm ? 1u : 0u, k = r2 - m * ipm;
        float *const out_rows = m ? p.up_out : p.gate_out;
        const uint32_t row = k * RPI + r;
        const uint32_t p0 = gi[1u + g], p1 = gi[2u + g];
        for (uint32_t c0 = p0; c0 < p1; c0 += DEC_TPC) {
            const uint32_t nt = p1 - c0 < DEC_TPC ? p1 - c0 : DEC_TPC;
            opaque<PAIR_DW>(w);
            const act_t *xe[DEC_TPC], *xd[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) {
                const uint32_t base = xo[c0 + (t < nt ? t : 0u)];
                xe[t] = &xs[base + j].a;
                xd[t] = &xs[base + (uint32_t)NBP + j].a;
            }
            float bE[4], bO[4], dE[4], dO[4], acc[4];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) {
                dE[t] = xe[t]->d;
                dO[t] = xd[t]->d;
            }
#define SF37_UP_PASS(NTc)                                  \
    q3_block_dots_at<NTc, 0>(w, xe, bE);                   \
    q3_block_dots_at<NTc, SF37_Q3_BYTES>(w, xd, bO);       \
    pair_chains<NTc, NBP>(dE, bE, dO, bO, acc);
            switch (nt) {
                case 1: SF37_UP_PASS(1) break;
                case 2: SF37_UP_PASS(2) break;
                case 3: SF37_UP_PASS(3) break;
                default: SF37_UP_PASS(4) break;
            }
#undef SF37_UP_PASS
            if (out_lane) {
#pragma unroll
                for (uint32_t t = 0; t < DEC_TPC; t++)
                    if (t < nt) out_rows[(uint64_t)so[c0 + t] * p.F + row] = acc[t];
            }
        }
    };
    // one item: wait for its tile (and the stores before it), read the
    // lane's pair, refill the tile with the next item, compute
    const uint32_t *pl = (const uint32_t *)tile + lane * 55u;
    uint32_t it = next();                 // gw itself when the launch prologue already filled its tile
    if (it != ITEM_NONE && !prefilled) fill(it);
    uint32_t nx = it != ITEM_NONE ? next() : ITEM_NONE;
    while (it != ITEM_NONE) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");     // the tile (and the stores before it)
        uint32_t w[PAIR_DW];
#pragma unroll
        for (uint32_t i = 0; i < 55u; i++) w[i] = pl[i];
        w[55] = 0u;
        opaque<PAIR_DW>(w);                         // the reads are done before the tile is refilled
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (nx != ITEM_NONE) fill(nx);
        compute(w, it);
        const uint32_t nn = nx != ITEM_NONE ? next() : ITEM_NONE;   // a ticket waits for the tile too
        it = nx;
        nx = nn;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");       // no load into LDS outlives the wave
}

// Routed gate/up.  An item is 2 rows of one group's expert for both
// matrices: lane = matrix (gate/up) | row | block, so each wave reads two
// contiguous 2-row spans; the gate lane of each row stores gate and up.
// The first (100 - up_dyn_pct)% of the items are split into equal contiguous
// ranges, one per wave; the rest are handed out one at a time from
// UP_QUEUES queues (wave w asks queue w % UP_QUEUES, which owns a contiguous
// share), so waves that run faster - older waves win the issue arbitration -
// take more of them and all finish together.  A wave asks for its first
// dynamic item while computing its last static one; the next item's blocks
// are always loaded while the current one is computed.
// Select launch (batches of more tokens): workgroup 0 forms the top-k and
// the grouping; workgroups 1.. the shared gate/up rows.
// LDS of a top-k workgroup of the select launch: selections, weights,
// group table, sorted pairs, a flag and the grouping scratch.
__host__ __device__ constexpr size_t lds_select_topk() {
    return (2u * DEC_MAX_TOK * 16u + 3u + 2u * DEC_MAX_TOK * 16u + DEC_MAX_TOK * 16u + 1u + GROUP_SCR) * 4u;
}

// Select launch (512 threads up to 8 tokens, 256 above): workgroups
// [0, n_tk) - wave w of workgroup b takes token nw b + w (token_topk into
// LDS, then sel and wts); with one top-k workgroup it groups the pairs from
// LDS, otherwise the last top-k workgroup to arrive (a counter; each
// releases its writes before arriving) groups them from sel.  Both publish
// ginfo and sorted.  Workgroups [n_tk, ...) compute the shared gate/up rows
// (4 per workgroup of 512 threads, 2 of 256).
__global__ void __launch_bounds__(512) dec_select_kernel(dec_params p, uint32_t n_tk) {
    extern __shared__ __align__(16) unsigned char smem[];
    if (blockIdx.x >= n_tk) {
        shared_gate_up(p, blockIdx.x - n_tk, smem, blockDim.x == 512u ? SH_RS_SEL : SH_RS_UP);
        return;
    }
    // the top-k workgroups' tables live in the dynamic LDS the shared
    // workgroups use (no static LDS: it would count against every workgroup)
    int32_t *s_sel = (int32_t *)smem;
    float *s_wts = (float *)(s_sel + DEC_MAX_TOK * 16u);
    uint32_t *s_gi = (uint32_t *)(s_wts + DEC_MAX_TOK * 16u);
    uint32_t *s_so = s_gi + 3u + 2u * DEC_MAX_TOK * 16u;
    uint32_t *s_flag = s_so + DEC_MAX_TOK * 16u;
    uint32_t *scr = s_flag + 1u;
    const uint32_t wave = threadIdx.x >> 6, nw = blockDim.x >> 6, P = p.T * p.topk;
    const uint32_t t = blockIdx.x * nw + wave, t0 = blockIdx.x * nw;
    const uint32_t p0 = t0 * p.topk, p1 = (p.T < t0 + nw ? p.T : t0 + nw) * p.topk;
    if (p.flags & SF37_DEC_SELECT) {
        if (t < p.T) token_topk(p, t, s_sel + t * p.topk, s_wts + t * p.topk);
        __syncthreads();
        if (threadIdx.x >= p0 && threadIdx.x < p1) {
            p.sel[threadIdx.x] = s_sel[threadIdx.x];
            p.wts[threadIdx.x] = s_wts[threadIdx.x];
        }
    } else if (threadIdx.x < P) {
        s_sel[threadIdx.x] = p.sel[threadIdx.x];
    }
    if (n_tk > 1u) {
        __syncthreads();
        if (threadIdx.x == 0) {
            __threadfence();
            *s_flag = atomicAdd(sel_arrivals(p), 1u) == n_tk - 1u;
        }
        __syncthreads();
        if (!*s_flag) return;
        __threadfence();
        if (threadIdx.x < P && (threadIdx.x < p0 || threadIdx.x >= p1)) s_sel[threadIdx.x] = p.sel[threadIdx.x];
    }
    __syncthreads();
    group_pairs(p, (const uint32_t *)s_sel, s_gi, s_so, true, scr);
}

// The routed part of the up launch on the block-pair DMA path (rows of 4, 8
// or 16 blocks), after the launch prologue has staged each token's
// activation blocks (even blocks first, then odd ones) and, with prefilled,
// started the wave's first tile: the pairs' activation offsets, then the
// items.  A 14 KiB tile per wave sits after the activations.
__device__ void up_routed_dma(const dec_params &p, unsigned char *smem, act_lds_t *xs, const uint32_t *gi,
                              const uint32_t *so, uint32_t *xo, uint32_t gw, uint32_t nw, uint32_t wave,
                              bool prefilled) {
    const uint32_t nbK = p.K / SF37_QK, P = p.T * p.topk;
    for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) xo[i] = (so[i] / p.topk) * nbK;
    __syncthreads();
    uint8_t *tile = smem + tile_base(p.K, p.T, p.G, P) + wave * TILE_LDS;
    switch (nbK) {
        case 4: up_items_pairs<2>(p, gi, so, xo, xs, tile, gw, nw, prefilled); break;
        case 8: up_items_pairs<4>(p, gi, so, xo, xs, tile, gw, nw, prefilled); break;
        default: up_items_pairs<8>(p, gi, so, xo, xs, tile, gw, nw, prefilled); break;
    }
}

// LDS direct loads with a per-lane source address: lane i writes LDS bytes
// [m0 + 4 i, + 4) (dword) or [m0 + 16 i, + 16) (dwordx4); masked lanes write
// nothing.  Issued through inline asm, so the compiler neither tracks nor
// waits for them: the caller waits (s_waitcnt vmcnt) before reading.
__device__ __forceinline__ void dma4_lane(uint32_t lds, const void *src) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
                 "v"(src)
                 : "memory");
}
__device__ __forceinline__ void dma16_lane(uint32_t lds, const void *src) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
                 "v"(src)
                 : "memory");
}

// Batches with a select launch on the DMA path: workgroups of 8 waves (4-7
// where the activations of many tokens leave LDS for fewer tiles), one LDS
// tile each, the activations staged once per workgroup.
__global__ void __launch_bounds__(512) dec_up_dma_kernel(dec_params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nbK = p.K / SF37_QK, P = p.T * p.topk;
    act_lds_t *xs = (act_lds_t *)smem;
    uint32_t *gi = (uint32_t *)(xs + p.T * nbK);
    uint32_t *so = gi + 3u + 2u * p.G;
    uint32_t *xo = so + P;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nwg = blockDim.x >> 6;
    const uint32_t lane = threadIdx.x & 63u, gw = blockIdx.x * nwg + wave, nw = gridDim.x * nwg;
    // everything the workgroup stages goes by direct loads issued at once:
    // the group table and pair order (dwords), the activation blocks (even
    // blocks first, then odd; lane = destination 16-byte chunk, the pad
    // chunks of act_lds_t masked), then this wave's first tile (its static
    // item gw, whose expert is read from the table in memory), so the tile
    // is in flight while the rest arrives
    {
        const uint32_t n_gi = 3u + 2u * p.G;
        for (uint32_t c0 = wave * 64u; c0 < n_gi; c0 += nwg * 64u)
            if (c0 + lane < n_gi) dma4_lane((uint32_t)(uintptr_t)(gi + c0), p.ginfo + c0 + lane);
        for (uint32_t c0 = wave * 64u; c0 < P; c0 += nwg * 64u)
            if (c0 + lane < P) dma4_lane((uint32_t)(uintptr_t)(so + c0), p.sorted + c0 + lane);
        constexpr uint32_t A16 = sizeof(act_t) / 16u, L16 = sizeof(act_lds_t) / 16u;
        const uint32_t n_x = p.T * nbK * L16, half = nbK >> 1;
        for (uint32_t c0 = wave * 64u; c0 < n_x; c0 += nwg * 64u) {
            const uint32_t d = c0 + lane, bp = d / L16, c = d - bp * L16;
            const uint32_t t = bp / nbK, sl = bp - t * nbK;
            const uint32_t b = sl < half ? 2u * sl : 2u * (sl - half) + 1u;
            if (d < n_x && c < A16)
                dma16_lane((uint32_t)(uintptr_t)xs + 16u * c0, (const u32x4 *)p.xq + ((uint64_t)(t * nbK + b) * A16 + c));
        }
    }
    bool prefilled = false;
    {
        const uint32_t NBP = nbK / 2u, RPI = 64u / NBP, ipm = p.F / RPI, ipg = 2u * ipm;
        const uint32_t g0 = gw / ipg, g0c = g0 < p.G ? g0 : p.G - 1u;
        // the group count and this group's expert by scalar loads (the
        // compiler's vector loads would wait for the direct loads above)
        uint32_t n_grp, e0;
        {
            const uint64_t gp = (uint64_t)(uintptr_t)p.ginfo;
            const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)gp), hi = __builtin_amdgcn_readfirstlane((uint32_t)(gp >> 32));
            const uint64_t base = ((uint64_t)hi << 32) | lo;
            const uint32_t off = __builtin_amdgcn_readfirstlane(4u * (2u + p.G + g0c));
            asm volatile("s_load_dword %0, %2, 0x0\n\ts_load_dword %1, %2, %3\n\ts_waitcnt lgkmcnt(0)"
                         : "=&s"(n_grp), "=&s"(e0)
                         : "s"(base), "s"(off)
                         : "memory");
        }
        if (gw < up_static_items(n_grp * ipg, nw, p.T) && (nbK == 4u || nbK == 8u || nbK == 16u)) {
            const uint32_t r2 = gw - g0 * ipg, m = r2 >= ipm ? 1u : 0u, k = r2 - m * ipm;
            const uint64_t row_bytes = (uint64_t)nbK * SF37_Q3_BYTES, exp_bytes = (uint64_t)p.F * row_bytes;
            const uint8_t *src = expert_base(p, m ? p.up_w : p.gate_w, m ? p.sh_up : p.sh_gate, e0, exp_bytes) +
                                 (uint64_t)(k * RPI) * row_bytes;
            const uint32_t tile_lds = (uint32_t)(uintptr_t)(smem + tile_base(p.K, p.T, p.G, P) + wave * TILE_LDS);
            constexpr uint32_t last = TILE_BYTES / 16u - 1u;
#pragma unroll
            for (uint32_t i = 0; i < TILE_LOADS; i++) {
                const uint32_t c = i * 64u + lane;
                dma16(tile_lds + 1024u * i, 16u * (c < last ? c : last), src);
            }
            prefilled = true;
        }
    }
    if (prefilled) asm volatile("s_waitcnt vmcnt(14)" ::: "memory");      // all but the tile's TILE_LOADS
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    up_routed_dma(p, smem, xs, gi, so, xo, gw, nw, wave, prefilled);
}
static_assert(TILE_LOADS == 14u, "the prologue's wait leaves exactly one tile's loads in flight");

// With UPSEL (few tokens, no select launch): workgroups [0, n_sh) run the
// shared gate/up rows, the rest the routed items after each has formed the
// top-k and the grouping itself (the first one publishing them).  Without:
// the routed items, the grouping read from the select launch.
__global__ void __launch_bounds__(256) dec_up_kernel(dec_params p, uint32_t n_sh) {
    extern __shared__ __align__(16) unsigned char smem[];
    if (blockIdx.x < n_sh) {
        shared_gate_up(p, blockIdx.x, smem, SH_RS_UPSEL);
        return;
    }
    const uint32_t wg = blockIdx.x - n_sh, n_wg = gridDim.x - n_sh;
    const uint32_t nbK = p.K / SF37_QK, P = p.T * p.topk;
    act_lds_t *xs = (act_lds_t *)smem;
    uint32_t *gi = (uint32_t *)(xs + p.T * nbK);
    uint32_t *so = gi + 3u + 2u * p.G;
    uint32_t *xo = so + P;                                        // first x block of each sorted pair's token
    if (p.flags & SF37_DEC_UPSEL) {
        select_and_group(p, gi, so, wg == 0u);
    } else {
        for (uint32_t i = threadIdx.x; i < 3u + 2u * p.G; i += blockDim.x) gi[i] = p.ginfo[i];
        for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) so[i] = p.sorted[i];
    }
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = n_wg * (blockDim.x >> 6), gw = wg * (blockDim.x >> 6) + wave;
    const uint32_t m = lane >> 5, rr = (lane >> 4) & 1u, b = lane & 15u;
    const uint32_t bl = b < nbK ? b : nbK - 1u;                    // lanes past the row repeat its last block
    const bool out_lane = b == nbK - 1u;
    float *const out_rows = m ? p.up_out : p.gate_out;
    const uint32_t ipg = p.F / 2u, n_items = gi[0] * ipg;
    const uint32_t dyn_pct = p.up_dyn_pct < 100u ? p.up_dyn_pct : 100u;
    const uint32_t n_stat = n_items - (uint32_t)((uint64_t)n_items * dyn_pct / 100u);
    const uint32_t lo = (uint32_t)((uint64_t)n_stat * gw / nw), hi = (uint32_t)((uint64_t)n_stat * (gw + 1u) / nw);
    const uint32_t qi = gw % UP_QUEUES, n_dyn = n_items - n_stat;
    const uint32_t q0 = n_stat + (uint32_t)((uint64_t)n_dyn * qi / UP_QUEUES);
    const uint32_t q1 = n_stat + (uint32_t)((uint64_t)n_dyn * (qi + 1u) / UP_QUEUES);
    uint32_t *queue = up_queue(p, qi);
    const uint64_t row_bytes = (uint64_t)nbK * SF37_Q3_BYTES, exp_bytes = (uint64_t)p.F * row_bytes;
    const uint8_t *W = m ? p.up_w : p.gate_w, *Wsh = m ? p.sh_up : p.sh_gate;
    // an item is carried as (group, row pair): static successors step it,
    // dynamic answers divide once
    auto block_ptr = [&](uint32_t g, uint32_t rp) -> const uint8_t * {
        return expert_base(p, W, Wsh, gi[2u + p.G + g], exp_bytes) + (uint64_t)(2u * rp + rr) * row_bytes +
               (uint64_t)bl * SF37_Q3_BYTES;
    };
    // a dynamic request: lane 0's atomic; its index is read when needed
    auto request = [&]() -> uint32_t {
        uint32_t v = 0;
        if (lane == 0) v = atomicAdd(queue, 1u);
        return v;
    };
    auto answer = [&](uint32_t v) -> uint32_t { return q0 + (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
    // the first item and its loads are started before x is staged
    uint32_t pend = 0, cur;
    if (lo < hi) {
        cur = lo;
        if (lo + 1u == hi) pend = request();
    } else {
        cur = answer(request());
        if (cur < q1) pend = request();
    }
    uint32_t g = cur / ipg, rp = cur - g * ipg;
    uint32_t nxt[28];
    const uint8_t *curp = block_ptr(cur < q1 ? g : 0u, cur < q1 ? rp : 0u);
    if (cur < q1) load_q3(nxt, curp);
    constexpr uint32_t A16 = sizeof(act_t) / 16u, L16 = sizeof(act_lds_t) / 16u;
    for (uint32_t i = threadIdx.x; i < p.T * nbK * A16; i += blockDim.x) {
        const uint32_t blk = i / A16, c = i - blk * A16;
        ((u32x4 *)xs)[blk * L16 + c] = ((const u32x4 *)p.xq)[i];
    }
    for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) xo[i] = (so[i] / p.topk) * nbK;
    __syncthreads();
    if (cur >= q1) return;
    for (;;) {
        uint32_t raw[28], a[27];
#pragma unroll
        for (int k = 0; k < 28; k++) raw[k] = nxt[k];
        // the next item: the static successor, else the pending request's answer
        uint32_t nx, ng, nrp;
        if (cur + 1u < hi) {
            nx = cur + 1u;
            ng = rp + 1u == ipg ? g + 1u : g;
            nrp = rp + 1u == ipg ? 0u : rp + 1u;
            if (nx + 1u == hi) pend = request();
        } else {
            nx = answer(pend);
            ng = nx / ipg;
            nrp = nx - ng * ipg;
            if (nx < q1) pend = request();
        }
        const bool more = nx < hi || (nx >= q0 && nx < q1);
        const uint8_t *nxp = more ? block_ptr(ng, nrp) : curp;
        if (more) load_q3(nxt, nxp);
        q3_realign(a, raw, (uint32_t)((uintptr_t)curp & 3u));
        const uint32_t row = 2u * rp + rr;
        const uint32_t p0 = gi[1u + g], p1 = gi[2u + g];
        for (uint32_t c0 = p0; c0 < p1; c0 += DEC_TPC) {
            const uint32_t nt = p1 - c0 < DEC_TPC ? p1 - c0 : DEC_TPC;
            opaque<27>(a);
            const act_t *x[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) x[t] = &xs[xo[c0 + (t < nt ? t : 0u)] + bl].a;
            float bs[DEC_TPC], dd[DEC_TPC], acc[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) dd[t] = x[t]->d;
            switch (nt) {
                case 1: q3_block_dots<1>(a, x, bs); block_chains<1>(dd, bs, acc, nbK); break;
                case 2: q3_block_dots<2>(a, x, bs); block_chains<2>(dd, bs, acc, nbK); break;
                case 3: q3_block_dots<3>(a, x, bs); block_chains<3>(dd, bs, acc, nbK); break;
                default: q3_block_dots<4>(a, x, bs); block_chains<4>(dd, bs, acc, nbK); break;
            }
            // the last block's lane of each (matrix, row) stores its row
            if (out_lane) {
#pragma unroll
                for (uint32_t t = 0; t < DEC_TPC; t++)
                    if (t < nt) out_rows[(uint64_t)so[c0 + t] * p.F + row] = acc[t];
            }
        }
        if (!more) break;
        cur = nx;
        g = ng;
        rp = nrp;
        curp = nxp;
    }
}

// ---------------------------------------------------------------------------
// mid: SwiGLU * routing weight (sf37.c:2179-2186) and its Q8_K in the Q2
// activation layout, one wave per (pair, 256-row block), lane l owning rows
// 4l .. 4l + 3; then, with the shared expert, the shared mid
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dec_mid_kernel(dec_params p) {
    __shared__ uint64_t tab[32];
    stage_exp_tab_imm(tab);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, nbm = p.F / SF37_QK;
    const uint32_t w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), n_routed = p.T * p.topk * nbm;
    if (w >= n_routed) {
        if (!(p.flags & SF37_DEC_SHARED)) return;
        // shared mid: SwiGLU (clamp_shared) and Q8_0 (sf37_ops.c:57-90), one
        // half-wave per (token, 32-row block)
        const uint32_t nb32 = p.F / 32u;
        const uint32_t hw = 2u * (w - n_routed) + (lane >> 5), l = lane & 31u;
        if (hw >= p.T * nb32) return;
        const uint32_t t = hw / nb32, blk = hw - t * nb32;
        const uint64_t o = (uint64_t)t * p.F + (uint64_t)blk * 32u + l;
        const float v = sf37_swiglu_mid_t(p.sh_gu[o], p.sh_gu[(uint64_t)p.T * p.F + o], 1.0f, p.clamp_shared, tab);
        float amax = fabsf(v);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        int8_t qv = 0;
        float d = 0.0f;
        if (amax != 0.0f) {
            d = amax / 127.0f;
            const float is = 1.0f / d;
            qv = (int8_t)(int)fminf(fmaxf(__builtin_rintf(is * v), -128.0f), 127.0f);
        }
        p.sh_mq[o] = qv;
        if (l == 0) p.sh_ms[(uint64_t)t * nb32 + blk] = d;
        return;
    }
    const uint32_t pr = w / nbm, blk = w - pr * nbm;
    const uint64_t o = (uint64_t)pr * p.F + (uint64_t)blk * SF37_QK + 4u * lane;
    const float wt = p.wts[pr];
    // the shared expert's slot (SH9) takes the shared clamp
    const float clamp = (p.flags & SF37_DEC_SH9) && pr % p.topk == p.topk - 1u ? p.clamp_shared : p.clamp_routed;
    float gv[4], uv[4], v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        gv[k] = p.gate_out[o + k];
        uv[k] = p.up_out[o + k];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        v[k] = sf37_swiglu_mid_t(gv[k], uv[k], wt, clamp, tab);
        p.mid[o + k] = v[k];
    }
    int8_t qk[4];
    int gsum;
    const float d = q8k_codes4(v, qk, gsum);
    act_t *y = (act_t *)p.midq + w;
    uint8_t *qb = (uint8_t *)y->qs;
#pragma unroll
    for (int k = 0; k < 4; k++) qb[q2_perm_pos(4u * lane + k)] = (uint8_t)qk[k];
    if (lane == 0) y->d = d;
    if ((lane & 15u) == 0) y->gs[lane >> 4] = gsum;
}

// ---------------------------------------------------------------------------
// routed down
// ---------------------------------------------------------------------------

// 21 dwords of a Q2 block (dword aligned) as five 16-byte loads and one dword.
__device__ __forceinline__ void load_q2(uint32_t w[21], const uint8_t *p) {
    const u32x4a4 *q = (const u32x4a4 *)p;
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const u32x4a4 v = q[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
    w[20] = ((const uint32_t *)p)[20];
}

// Block values of one Q2 block (21 dwords in a) against NT activation blocks
// in LDS (Q2 act layout): bs[t] = sum_g fma(s_g, I_g).
template <int NT>
__device__ __forceinline__ void q2_block_dots_lds(const uint32_t *a, const act_t *const *x, float bs[4]) {
#pragma unroll
    for (int t = 0; t < NT; t++) bs[t] = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t c[16];
#pragma unroll
        for (int j = 0; j < 4; j++) q2_unpack16(a[3 + 4 * g + j], c[4 * j], c[4 * j + 1], c[4 * j + 2], c[4 * j + 3]);
        const int32_t zp = (int32_t)((a[2] >> (8 * g)) & 3u);
        const float sc = sf37_f16(a[g >> 1] >> (16 * (g & 1)));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const u32x4 *xq = (const u32x4 *)&x[t]->qs[16 * g];
            int32_t acc = 0;
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const u32x4 v = xq[h];
                acc = sdot4(c[4 * h], v.x, acc);
                acc = sdot4(c[4 * h + 1], v.y, acc);
                acc = sdot4(c[4 * h + 2], v.z, acc);
                acc = sdot4(c[4 * h + 3], v.w, acc);
            }
            bs[t] = __builtin_fmaf(sc, (float)(acc - __mul24(zp, x[t]->gs[g])), bs[t]);
        }
        __builtin_amdgcn_sched_barrier(0);            // one group's codes live at a time
    }
}

// acc = fma(d_b, bs_b, acc) along the nb lanes of each row segment (lane
// blocks 0..nb-1 of one row are consecutive lanes inside a 16-lane DPP
// row); the row's total ends in the lane of block nb-1.
// NT tokens at once (their steps interleave); unrolled for 5 blocks
// (F = 1280).
template <int NT>
__device__ __forceinline__ void seg_chains(const float *d, const float *bs, float *acc, uint32_t b, uint32_t nb) {
    auto step = [&]() {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float prev = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc[t]), 0x111, 0xf, 0xf, true));
            acc[t] = __builtin_fmaf(d[t], bs[t], b == 0u ? 0.0f : prev);
        }
    };
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = __builtin_fmaf(d[t], bs[t], 0.0f);
    if (nb == 5u) {
#pragma unroll
        for (int st = 1; st < 5; st++) step();
    } else {
        for (uint32_t st = 1; st < nb; st++) step();
    }
}

// Down.  Routed down: lane = (row, block): each 16-lane DPP row holds 16/nb rows
// with their nb blocks on consecutive lanes, so a wave reads 64/nb*4 rows
// (12 for F = 1280) as one contiguous span.  A wave owns a contiguous range
// of these sub-items (mostly inside one group); the group's activation
// blocks for up to four pairs sit in the wave's LDS slice.  The next
// sub-item's blocks are loaded while the current one is computed.
// Words [0, n) of src into LDS dst by direct global->LDS dword loads (lane
// i of an instruction writes dst word c0 + i; lanes past n masked off).  All
// threads of the workgroup call it; lds_copy_wait() must follow.
__device__ __forceinline__ void lds_copy_words(uint32_t *dst, const uint32_t *src, uint32_t n) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, nw = blockDim.x >> 6;
    for (uint32_t c0 = wave * 64u; c0 < n; c0 += nw * 64u) {
        const uint32_t c = c0 + lane;
        if (c < n) __builtin_amdgcn_global_load_lds((const void *)(src + c), dst + c0, 4, 0, 0);
    }
}

template <int SHNB>
__global__ void __launch_bounds__(256) dec_down_kernel(dec_params p) {
    extern __shared__ __align__(16) unsigned char smem[];        // shared mid codes, then scales
    __shared__ uint32_t meta[3u + 2u * 256u + 256u];
    __shared__ __align__(16) act_t xsl[4][DN_STAGE * DN_MAX_NB];
    const uint32_t P = p.T * p.topk;
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    uint32_t *gi = meta;
    uint32_t *so = gi + 3u + 2u * p.G;
    int8_t *shq = (int8_t *)smem;
    float *shs = (float *)(smem + p.T * p.F);
    // tables and the shared mid into LDS by direct loads, all in flight at once
    lds_copy_words(gi, p.ginfo, 3u + 2u * p.G);
    lds_copy_words(so, p.sorted, P);
    if (sh) {
        lds_copy_words((uint32_t *)shq, (const uint32_t *)p.sh_mq, p.T * p.F / 4u);
        lds_copy_words((uint32_t *)shs, (const uint32_t *)p.sh_ms, p.T * (p.F / 32u));
    }
    lds_copy_wait();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    act_t *xw = xsl[wave];
    const uint32_t nb = p.F / SF37_QK, rpd = 16u / nb, rpw = 4u * rpd;     // rows per DPP row / wave
    const uint32_t q = lane & 15u, r_in = q / nb, b = q - r_in * nb;
    const bool active = r_in < rpd;
    const uint32_t rl = (lane >> 4) * rpd + (active ? r_in : 0u);          // row within the sub-item
    const uint32_t spg = (p.K + rpw - 1u) / rpw, n_sub = gi[0] * spg;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6), gw = blockIdx.x * (blockDim.x >> 6) + wave;
    const uint32_t lo = (uint32_t)((uint64_t)n_sub * gw / nw), hi = (uint32_t)((uint64_t)n_sub * (gw + 1u) / nw);
    const uint64_t row_bytes = (uint64_t)nb * SF37_Q2_BYTES;
    // a sub-item is carried as (group, sub-item in group), stepped in order
    auto blk_ptr = [&](uint32_t g_, uint32_t sub_) -> const uint8_t * {
        uint32_t row = sub_ * rpw + rl;
        row = row < p.K ? row : p.K - 1u;                                    // keep tail lanes in bounds
        return expert_base(p, p.down_w, p.sh_down, gi[2u + p.G + g_], (uint64_t)p.K * row_bytes) + row * row_bytes +
               (uint64_t)b * SF37_Q2_BYTES;
    };
    uint32_t staged_g = 0xffffffffu, staged_c0 = 0xffffffffu;
    uint32_t g = lo / spg, sub = lo - g * spg;
    // The shared expert's down rows, handed out one row group at a time from
    // DN_QUEUES queues (wave w asks queue w % DN_QUEUES, which owns a
    // contiguous share): after the routed range, so waves that finish it
    // early take more - except at one token, where a wave has at most one
    // routed sub-item and takes its shared rows while that sub-item's weights
    // load.  The next request is issued before the current group is computed.
    auto shared_phase = [&]() {
        const uint32_t R = 64u / (p.T * shd_slices(p.T)), n_sp = (p.K + R - 1u) / R;
        const uint32_t qi = gw % DN_QUEUES;
        const uint32_t q0 = (uint32_t)((uint64_t)n_sp * qi / DN_QUEUES), q1 = (uint32_t)((uint64_t)n_sp * (qi + 1u) / DN_QUEUES);
        uint32_t *queue = dn_queue(p, qi);
        auto request = [&]() -> uint32_t {
            uint32_t v = 0;
            if (lane == 0) v = atomicAdd(queue, 1u);
            return v;
        };
        uint32_t pend = request();
        for (;;) {
            const uint32_t idx = q0 + (uint32_t)__builtin_amdgcn_readfirstlane((int)pend);
            if (idx >= q1) break;
            pend = request();
            shared_down_pass<SHNB>(p, shq, shs, idx * R,
                                   [&](uint32_t t, uint32_t row, float v) { p.sh_out[(uint64_t)t * p.K + row] = v; });
        }
    };
    const bool sh_first = p.T == 1u;
    uint32_t nxt[21];
    if (lo < hi) load_q2(nxt, blk_ptr(g, sub));
    if (sh && sh_first) shared_phase();
    for (uint32_t sidx = lo; sidx < hi; sidx++) {
        uint32_t w[21];
#pragma unroll
        for (int i = 0; i < 21; i++) w[i] = nxt[i];
        const uint32_t ng = sub + 1u == spg ? g + 1u : g, nsub = sub + 1u == spg ? 0u : sub + 1u;
        if (sidx + 1u < hi) load_q2(nxt, blk_ptr(ng, nsub));
        const uint32_t row = sub * rpw + rl;
        const bool out_lane = active && b == nb - 1u && row < p.K;
        const uint32_t p0 = gi[1u + g], p1 = gi[2u + g];
        for (uint32_t c0 = p0; c0 < p1; c0 += DN_TPC) {
            const uint32_t nt = p1 - c0 < DN_TPC ? p1 - c0 : DN_TPC;
            // the activation blocks of up to DN_STAGE pairs stay staged, so a
            // group of that many pairs is staged once for the wave's range
            const uint32_t cs = p0 + ((c0 - p0) / DN_STAGE) * DN_STAGE;
            if (g != staged_g || cs != staged_c0) {
                const uint32_t ns = p1 - cs < DN_STAGE ? p1 - cs : DN_STAGE;
                __builtin_amdgcn_wave_barrier();
                const uint32_t per = nb * (uint32_t)(sizeof(act_t) / 16u);
                for (uint32_t i = lane; i < ns * per; i += 64u) {
                    const uint32_t t = i / per, k = i - t * per;
                    ((u32x4 *)xw)[i] = ((const u32x4 *)((const act_t *)p.midq + (uint64_t)so[cs + t] * nb))[k];
                }
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_wave_barrier();
                staged_g = g;
                staged_c0 = cs;
            }
            opaque<21>(w);
            const act_t *x[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) x[t] = xw + (c0 - cs + (t < nt ? t : 0u)) * nb + b;
            float bs[DEC_TPC], dd[DN_TPC], acc[DN_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DN_TPC; t++) dd[t] = x[t]->d;
            if (nt == 1) {
                q2_block_dots_lds<1>(w, x, bs);
                seg_chains<1>(dd, bs, acc, b, nb);
            } else {
                q2_block_dots_lds<2>(w, x, bs);
                seg_chains<2>(dd, bs, acc, b, nb);
            }
            if (out_lane) {
#pragma unroll
                for (uint32_t t = 0; t < DN_TPC; t++)
                    if (t < nt) p.down_pair[(uint64_t)so[c0 + t] * p.K + row] = acc[t];
            }
        }
        g = ng;
        sub = nsub;
    }
    if (sh && !sh_first) shared_phase();
}

// ---------------------------------------------------------------------------
// One token, one group per slot (SF37_DEC_SLOTS): down and combine in one
// launch.  A workgroup owns the rpw output rows of one routed sub-item (12
// for F = 1280, lane = (row, block) as in dec_down_kernel): wave w computes
// slot w's rows of its expert (and slot w + 8's past eight slots, up to 16),
// waves 0 .. nsh-1 first the shared
// rows of the tile (R = 4 per wave), all into LDS; then one thread per row
// forms out = [shared +] (slots summed in slot order) [+ out], the
// arithmetic of dec_combine_kernel.  No per-pair rows reach memory.
// ---------------------------------------------------------------------------
constexpr uint32_t DN1_WAVES = 8;        // waves: slots (two each past eight) and shared passes (<= 8)
constexpr uint32_t DN1_MAX_RPW = 32;     // rows per tile (nb >= 2)

__host__ __device__ constexpr uint32_t dn1_rpw(uint32_t F) { return 4u * (16u / (F / SF37_QK)); }

template <int SHNB>
__global__ void __launch_bounds__(DN1_WAVES * 64, 2) dec_down1_kernel(dec_params p) {
    __shared__ __align__(16) int8_t shq[DN_MAX_NB * SF37_QK];
    __shared__ float shs[DN_MAX_NB * SF37_QK / 32u];
    __shared__ __align__(16) act_t xsl[SHNB == 1 ? 2 : 1][DN1_WAVES][DN_MAX_NB];
    __shared__ float res[(SHNB == 1 ? 2 : 1) * DN1_WAVES][DN1_MAX_RPW];
    __shared__ float shres[DN1_MAX_RPW];
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    const uint32_t nb = p.F / SF37_QK, rpd = 16u / nb, rpw = 4u * rpd, r0 = blockIdx.x * rpw;
    const uint32_t q = lane & 15u, r_in = q / nb, b = q - r_in * nb;
    const bool active = r_in < rpd;
    const uint32_t rl = (lane >> 4) * rpd + (active ? r_in : 0u);
    // wave w takes slot w and, past eight slots, slot w + 8 (the instance
    // without shared-down batches; the others take up to eight slots)
    constexpr uint32_t NJ = SHNB == 1 ? 2u : 1u;
    bool routed[NJ];
    uint32_t w[NJ][21];
#pragma unroll
    for (uint32_t j = 0; j < NJ; j++) {
        const uint32_t s = wave + DN1_WAVES * j;
        routed[j] = s < p.topk;
        if (routed[j]) {
            const uint32_t e = p.ginfo[2u + p.G + s];
            uint32_t row = r0 + rl;
            row = row < p.K ? row : p.K - 1u;                               // tail lanes stay in bounds
            const uint64_t rb = (uint64_t)nb * SF37_Q2_BYTES;
            load_q2(w[j], expert_base(p, p.down_w, p.sh_down, e, (uint64_t)p.K * rb) + (uint64_t)row * rb +
                              (uint64_t)b * SF37_Q2_BYTES);
        }
    }
    if (sh) {
        for (uint32_t i = threadIdx.x; i < p.F / 16u; i += blockDim.x) ((u32x4 *)shq)[i] = ((const u32x4 *)p.sh_mq)[i];
        for (uint32_t i = threadIdx.x; i < p.F / 32u; i += blockDim.x) shs[i] = p.sh_ms[i];
    }
#pragma unroll
    for (uint32_t j = 0; j < NJ; j++) {
        if (!routed[j]) continue;
        const uint32_t per = nb * (uint32_t)(sizeof(act_t) / 16u), s = wave + DN1_WAVES * j;
        for (uint32_t i = lane; i < per; i += 64u)
            ((u32x4 *)xsl[j][wave])[i] = ((const u32x4 *)((const act_t *)p.midq + (uint64_t)p.sorted[s] * nb))[i];
    }
    __syncthreads();
    const uint32_t R = 64u / shd_slices(1u), nsh = (rpw + R - 1u) / R;
    if (sh && wave < nsh)
        shared_down_pass<SHNB>(p, shq, shs, r0 + wave * R,
                               [&](uint32_t, uint32_t row, float v) { shres[row - r0] = v; });
#pragma unroll
    for (uint32_t j = 0; j < NJ; j++) {
        if (!routed[j]) continue;
        opaque<21>(w[j]);
        const act_t *x[DEC_TPC];
#pragma unroll
        for (uint32_t t = 0; t < DEC_TPC; t++) x[t] = xsl[j][wave] + b;
        float bs[DEC_TPC], dd[1] = {x[0]->d}, acc[1];
        q2_block_dots_lds<1>(w[j], x, bs);
        seg_chains<1>(dd, bs, acc, b, nb);
        if (active && b == nb - 1u && r0 + rl < p.K) res[wave + DN1_WAVES * j][rl] = acc[0];
    }
    __syncthreads();
    const uint32_t i = threadIdx.x;
    if (i < rpw && r0 + i < p.K) {
        const uint32_t r = r0 + i;
        float acc = 0.0f;
        for (uint32_t s2 = 0; s2 < p.topk; s2++) acc = acc + res[s2][i];
        const float y = sh ? shres[i] + acc : (p.flags & SF37_DEC_SHBASE) ? p.sh_out[r] + acc : acc;
        p.out[r] = (p.flags & SF37_DEC_RESID) ? p.out[r] + y : y;
    }
}

// ---------------------------------------------------------------------------
// combine: out = [shared +] sum over slots in slot order, one thread per
// output
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dec_combine_kernel(dec_params p) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= p.T * p.K) return;
    const uint32_t t = i / p.K, r = i - t * p.K;
    float v[16];
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const uint32_t sc = (uint32_t)s < p.topk ? (uint32_t)s : 0u;   // every read in bounds
        v[s] = p.down_pair[((uint64_t)t * p.topk + sc) * p.K + r];
    }
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; s++)
        if ((uint32_t)s < p.topk) acc = acc + v[s];
    const float y = (p.flags & (SF37_DEC_SHARED | SF37_DEC_SHBASE)) ? p.sh_out[i] + acc : acc;
    p.out[i] = (p.flags & SF37_DEC_RESID) ? p.out[i] + y : y;
}

}  // namespace

namespace {

struct dec_shape {
    bool up_wide;
    uint32_t n_rt, n_xq, n_tk, sel_threads, n_shup, sh_rs, up_waves, n_up, n_mid, n_dn, n_cb;
    size_t lds_up, lds_shup, lds_dn;
    size_t lds_sel_launch, lds_up_launch;   // dynamic LDS given to the select and up launches
    const void *dn_kernel;
};

// The LDS side of a launch plan, from the shapes and the device's LDS limit
// per workgroup alone (no device query): the routed up kernel's form and
// waves, the shared gate/up rows per workgroup, and the dynamic LDS of the
// select, up and down launches.  dec_plan and sf37k_decode_lds_check use it.
void dec_plan_lds(const dec_params &p, size_t ml, dec_shape &d) {
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    const bool upsel = (p.flags & SF37_DEC_UPSEL) != 0;
    d.sel_threads = p.T <= 8u ? 512u : 256u;
    // routed up: block-pair DMA workgroups when the batch has a select
    // launch and at least 4 waves' tiles fit beside the activations (up to
    // 8 waves), else the row-pair loop
    const uint32_t P = p.T * p.topk;
    const size_t tb = tile_base(p.K, p.T, p.G, P);
    const uint32_t fit = tb < ml ? (uint32_t)((ml - tb) / TILE_LDS) : 0u;
    d.up_waves = fit < 8u ? fit : 8u;
    d.up_wide = up_pairs(p.K) && !upsel && d.up_waves >= 4u;
    d.lds_up = d.up_wide ? lds_up_dma(p.K, p.T, p.G, P, d.up_waves) : lds_up_meta(p.K, p.T, p.G, P);
    // the select launch takes 4 shared rows per 512-thread workgroup up to 8
    // tokens; above that 2 per 256-thread workgroup (the terms of 16 tokens
    // x 4 rows would hold one workgroup per CU); the one-token up launch 4
    // per 256-thread workgroup
    d.sh_rs = upsel ? SH_RS_UPSEL : p.T > 8u ? SH_RS_UP : SH_RS_SEL;
    d.lds_shup = lds_up_shared(p.K, p.T, d.sh_rs);
    d.n_shup = sh ? p.F / d.sh_rs : 0u;                // shared gate/up workgroups (select or up launch)
    d.lds_sel_launch = d.n_shup && d.lds_shup > lds_select_topk() ? d.lds_shup : lds_select_topk();
    d.lds_up_launch = d.up_wide ? d.lds_up : (d.lds_up > d.lds_shup || !d.n_shup || !upsel ? d.lds_up : d.lds_shup);
    d.lds_dn = sh ? (size_t)p.T * p.F + (size_t)p.T * (p.F / 32u) * 4u : 0u;
}

uint32_t device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return (uint32_t)cus;
}

uint32_t device_max_lds() {
    static int lds = 0;
    if (!lds) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds <= 0)
            lds = 65536;
    }
    return (uint32_t)lds;
}

// Opts kernel fn into at least `bytes` of dynamic LDS (above 64 KiB).  The
// opt-in only ever rises: a batch needing less LDS never lowers what a
// larger batch of the same kernel was given.
int opt_in_lds(const void *fn, size_t bytes) {
    struct entry { const void *fn; size_t bytes; };
    static entry tab[16];
    static int used = 0;
    if (bytes <= 65536u) return 0;
    int i = 0;
    while (i < used && tab[i].fn != fn) i++;
    if (i < used && tab[i].bytes >= bytes) return 0;
    const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (err != hipSuccess) return (int)err;
    if (i < used) tab[i].bytes = bytes;
    else if (used < 16) tab[used++] = {fn, bytes};
    return 0;
}

// Workgroups of this kernel one CU holds at once (from the occupancy
// calculator, at least 1), cached per (kernel, block size, LDS bytes).
// Dynamic LDS above 64 KiB is opted into first.
uint32_t resident_wgs(const void *fn, int threads, size_t lds) {
    struct entry { const void *fn; int threads; size_t lds; uint32_t n; };
    static entry cache[16];
    static int used = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].fn == fn && cache[i].threads == threads && cache[i].lds == lds) return cache[i].n;
    (void)opt_in_lds(fn, lds);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess || n < 1) n = 1;
    (void)hipGetLastError();
    if (used < 16) cache[used++] = {fn, threads, lds, (uint32_t)n};
    return (uint32_t)n;
}

// One instance of the down kernel per shared-down batch count (registers:
// each instance stays at 3 waves per SIMD, a kernel holding all would not).
const void *down_kernel_for(const dec_params &p) {
    const uint32_t nbat = (shd_bps(p.F / 32u, shd_slices(p.T)) + SHD_CHUNK - 1u) / SHD_CHUNK;
    if ((p.flags & SF37_DEC_SHARED) == 0u || nbat <= 1u) return (const void *)dec_down_kernel<1>;
    return nbat == 2u ? (const void *)dec_down_kernel<2> : (const void *)dec_down_kernel<3>;
}

dec_shape dec_plan(const dec_params &p) {
    dec_shape d;
    const uint32_t nb = p.K / SF37_QK;
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    const uint32_t cus = device_cus();
    d.n_rt = (p.flags & (SF37_DEC_ROUTER | SF37_DEC_SELECT)) ? route_wgs(p.T, p.E) : 0u;
    d.n_xq = (p.T * nb + 3u) / 4u;
    dec_plan_lds(p, device_max_lds(), d);
    d.n_tk = (p.T + d.sel_threads / 64u - 1u) / (d.sel_threads / 64u);
    // persistent kernels: exactly as many workgroups as can be resident
    const uint32_t up_res = d.up_wide ? resident_wgs((const void *)dec_up_dma_kernel, 64 * (int)d.up_waves, d.lds_up)
                                      : resident_wgs((const void *)dec_up_kernel, 256, d.lds_up_launch);
    d.n_up = (p.up_wgs && p.up_wgs < up_res ? p.up_wgs : up_res) * cus;
    d.n_mid = (p.T * p.topk * (p.F / SF37_QK) + (sh ? (p.T * (p.F / 32u) + 1u) / 2u : 0u) + 3u) / 4u;
    d.dn_kernel = down_kernel_for(p);
    const uint32_t dn_res = resident_wgs(d.dn_kernel, 256, d.lds_dn);
    d.n_dn = (p.dn_wgs && p.dn_wgs < dn_res ? p.dn_wgs : dn_res) * cus;
    d.n_cb = (p.T * p.K + 255u) / 256u;
    return d;
}

}  // namespace

extern "C" int sf37k_decode_counters(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F) {
    (void)T; (void)topk; (void)E; (void)K; (void)F;
    return (int)(32u * (UP_QUEUES + DN_QUEUES));
}

// Scratch of the no-alloc decode entry point (sf37_hip_moe_layer_noalloc):
// device memory that exists from module load to process end, one copy per
// GPU.  The queues at its start are zeroed by every route launch.  In host
// code `scratch` names a host-side stand-in: only the address from
// hipGetSymbolAddress, looked up per device, is handed to kernels.
static_assert(32u * (UP_QUEUES + DN_QUEUES) * 4u <= SF37_NOALLOC_QUEUE_BYTES, "queues fit their region");
static __device__ __align__(256) uint8_t scratch[SF37_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
void *g_noalloc_ptr[NOALLOC_MAX_DEVICES];
}  // namespace

extern "C" int sf37k_noalloc_scratch_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (g_noalloc_ptr[dev]) return 0;
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    g_noalloc_ptr[dev] = ptr;
    return 0;
}

extern "C" void *sf37k_noalloc_scratch(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
    return g_noalloc_ptr[dev];
}

namespace {
int decode_supported_at(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F, int shared, size_t ml) {
    if (T == 0 || T > DEC_MAX_TOK || topk == 0 || K % SF37_QK || F % SF37_QK || K / SF37_QK > 16u ||
        F / SF37_QK > DN_MAX_NB)
        return 0;
    // shared down: the shared mid fits in the x area, a lane's slice in registers
    if (shared && shd_bps(F / 32u, shd_slices(T)) > SHD_MAX_BPS) return 0;
    const uint32_t P = T * topk, G = P < E ? P : E;
    if (lds_up_meta(K, T, G, P) > ml) return 0;
    if (shared && (lds_up_shared(K, T, SH_RS_UP) > ml || lds_up_shared(K, T, SH_RS_SEL) > ml ||
                   lds_up_shared(K, T, SH_RS_UPSEL) > ml))
        return 0;
    return 1;
}
}  // namespace

extern "C" int sf37k_decode_supported(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F, int shared) {
    return decode_supported_at(T, topk, E, K, F, shared, device_max_lds());
}

// Host-side check of the LDS direct loads of the decode launches for one
// shape and flag set at a per-workgroup LDS limit (no device needed).  A
// global_load_lds writes its 64 lanes' bytes at M0 + 16 * lane whatever the
// source, so every M0 a kernel forms must leave that whole span inside the
// region it targets, and every region must lie inside the LDS its launch is
// given.  ext[0..5]: end of the last routed up tile's loads, LDS of the up
// launch, end of the shared gate/up tile copies and terms, LDS of the launch
// running them, end of the up kernel's activation area, start of its tiles.
// Returns 0 when everything fits, -1 for a shape the library refuses before
// any launch at that limit, else the number of the first failed check.
extern "C" int sf37k_decode_lds_check(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F,
                                      uint32_t flags, uint32_t max_lds, uint64_t *ext) {
    for (int i = 0; i < 6; i++) ext[i] = 0;
    if (!decode_supported_at(T, topk, E, K, F, (flags & SF37_DEC_SHARED) != 0, max_lds)) return -1;
    dec_params p = {};
    p.T = T;
    p.topk = topk;
    p.E = E;
    p.K = K;
    p.F = F;
    p.flags = flags;
    const uint32_t P = T * topk;
    p.G = P < E ? P : E;
    dec_shape d = {};
    dec_plan_lds(p, max_lds, d);
    int fail = 0;
    auto check = [&](bool ok, int code) {
        if (!ok && !fail) fail = code;
    };
    if (d.up_wide) {
        // wave w's tile at tile_base + w * TILE_LDS; load i of the fill writes
        // [1024 i, 1024 i + 1024) of it (up_items_pairs)
        ext[4] = lds_up_meta(K, T, p.G, P);
        ext[5] = tile_base(K, T, p.G, P);
        ext[0] = ext[5] + (uint64_t)(d.up_waves - 1u) * TILE_LDS + 1024u * (TILE_LOADS - 1u) + 64u * 16u;
        ext[1] = d.lds_up_launch;
        check(ext[4] <= ext[5], 1);
        check(ext[0] <= ext[1], 2);
        check(ext[1] <= max_lds && 64u * d.up_waves <= 512u, 3);
    }
    if (d.n_shup) {
        // shared_gate_up: gate tile copy at 0, up tile copy at wbuf (lds_copy
        // writes 16 * ceil((off + n) / 16) bytes, off <= 15), terms after 2 wbuf
        const uint32_t tbytes = up_shared_tile(K, d.sh_rs), wbuf = tile_buf(tbytes);
        const uint64_t span = 16ull * ((15ull + tbytes + 15ull) / 16ull);
        const uint64_t terms_end = 2ull * wbuf + (uint64_t)T * 2u * d.sh_rs * sh_red_stride(K) * 4u;
        ext[2] = wbuf + span > terms_end ? wbuf + span : terms_end;
        ext[3] = (flags & SF37_DEC_UPSEL) ? d.lds_up_launch : d.lds_sel_launch;
        check(span <= wbuf, 4);
        check(terms_end <= ext[3], 5);
        check(ext[3] <= max_lds, 6);
    }
    return fail;
}

extern "C" int sf37k_decode_route(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_route_kernel, dim3(d.n_rt + d.n_xq), dim3(256), 0, (hipStream_t)s, *pp, d.n_rt);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_select(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    const size_t lds = d.lds_sel_launch;
    const int err = opt_in_lds((const void *)dec_select_kernel, lds);
    if (err) return err;
    hipLaunchKernelGGL(dec_select_kernel, dim3(d.n_tk + d.n_shup), dim3(d.sel_threads), lds, (hipStream_t)s, *pp,
                       d.n_tk);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_up(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    if (d.up_wide) {
        const int err = opt_in_lds((const void *)dec_up_dma_kernel, d.lds_up);
        if (err) return err;
        hipLaunchKernelGGL(dec_up_dma_kernel, dim3(d.n_up), dim3(64u * d.up_waves), d.lds_up, (hipStream_t)s, *pp);
        return (int)hipGetLastError();
    }
    const bool upsel = (pp->flags & SF37_DEC_UPSEL) != 0u;
    const uint32_t n_sh = upsel ? d.n_shup : 0u;
    const size_t lds = d.lds_up_launch;
    const int err = opt_in_lds((const void *)dec_up_kernel, lds);
    if (err) return err;
    sf37_dec_params p = *pp;
    hipLaunchKernelGGL(dec_up_kernel, dim3(n_sh + d.n_up), dim3(256), lds, (hipStream_t)s, p, n_sh);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_mid(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_mid_kernel, dim3(d.n_mid), dim3(256), 0, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_down(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    void *args[] = {(void *)pp};
    const int err = opt_in_lds(d.dn_kernel, d.lds_dn);
    if (err) return err;
    const hipError_t e = hipLaunchKernel(d.dn_kernel, dim3(d.n_dn), dim3(256), args, d.lds_dn, (hipStream_t)s);
    return (int)(e != hipSuccess ? e : hipGetLastError());
}

extern "C" int sf37k_decode_down_combine_supported(const sf37_dec_params *pp) {
    const sf37_dec_params &p = *pp;
    const uint32_t nb = p.F / SF37_QK;
    // slots: two per wave in the instance without shared-down batches
    const uint32_t nbat = (shd_bps(p.F / 32u, shd_slices(1u)) + SHD_CHUNK - 1u) / SHD_CHUNK;
    const uint32_t max_slots = (p.flags & SF37_DEC_SHARED) == 0u || nbat <= 1u ? 2u * DN1_WAVES : DN1_WAVES;
    return (p.flags & SF37_DEC_SLOTS) && p.T == 1u && p.topk <= max_slots && nb >= 2u && nb <= DN_MAX_NB &&
           dn1_rpw(p.F) <= DN1_MAX_RPW && (dn1_rpw(p.F) + 3u) / 4u <= DN1_WAVES && p.K > 0u;
}

extern "C" int sf37k_decode_down_combine(const sf37_dec_params *pp, sf37_stream_t s) {
    if (!sf37k_decode_down_combine_supported(pp)) return (int)hipErrorInvalidValue;
    const sf37_dec_params &p = *pp;
    const uint32_t nbat = (shd_bps(p.F / 32u, shd_slices(1u)) + SHD_CHUNK - 1u) / SHD_CHUNK;
    const void *fn = (p.flags & SF37_DEC_SHARED) == 0u || nbat <= 1u ? (const void *)dec_down1_kernel<1>
                     : nbat == 2u                                    ? (const void *)dec_down1_kernel<2>
                                                                     : (const void *)dec_down1_kernel<3>;
    const uint32_t rpw = dn1_rpw(p.F);
    void *args[] = {(void *)pp};
    const hipError_t e = hipLaunchKernel(fn, dim3((p.K + rpw - 1u) / rpw), dim3(DN1_WAVES * 64u), args, 0, (hipStream_t)s);
    return (int)(e != hipSuccess ? e : hipGetLastError());
}

extern "C" int sf37k_decode_combine(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_combine_kernel, dim3(d.n_cb), dim3(256), 0, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}
