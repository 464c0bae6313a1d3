// k_decode.hip - the MoE layer for decode batches (up to 16 tokens) on
// gfx950, in five launches on one stream:
//
//   route     : router GEMV (binary64 accumulation) and the Q8_K / Q8_0
//               quantisation of x; the last workgroup to finish runs top-k
//               for every token, groups the (token, slot) pairs by expert
//               and clears the down kernel's tile counters.
//   shared_up : the shared expert's Q8_0 gate/up rows (LDS tiles).
//   up        : routed Q3 gate/up with SwiGLU * routing weight; a lane owns
//               one 110-byte block, a wave two rows of gate and up, and the
//               canonical block-order chain runs as a DPP scan.
//   mid       : Q8_K of the routed mid, SwiGLU + Q8_0 of the shared mid.
//   down      : routed Q2 down (lane = row, activations through the scalar
//               cache) and the shared Q8_0 down; the last wave of each
//               64-row tile forms out = shared + sum over slots in slot order.
//
// Hand-offs inside a launch (logits to the top-k workgroup, per-pair down
// rows to the combining wave) use agent-coherent stores and loads and an
// atomic arrival counter; the workgroup or wave that completes a counter
// does the dependent work and resets it.  Nothing waits on another
// workgroup, so every wave always runs to completion.
//
// Arithmetic is the canonical order of the oracle (sf37_blocks.h), the
// reference CPU order for the Q8_0 shared expert (sf37_ops.c:92-108), and
// slot-order combines, so results equal the staged kernels bit for bit.
#include "sf37_blocks.h"
#include "sf37_router.h"
#include "sf37_launch.h"

namespace {

constexpr uint32_t DEC_MAX_TOK = 16;
constexpr uint32_t DEC_TPC = 4;      // pairs per pass in the routed kernels
constexpr uint32_t SH_RS = 2;        // shared gate/up rows per workgroup
constexpr uint32_t DN_TILE = 64;     // down rows per item (= combine tile)
constexpr uint32_t DN_MAX_NB = 5;    // down blocks per row held in registers (F <= 1280)
constexpr uint32_t DN_WG_WAVES = 2;  // waves per combine workgroup (one LDS tile each)
constexpr uint32_t DN_TPC = 2;       // pairs per pass in the routed down kernel

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
// Activation blocks read through the scalar cache (every lane of a wave
// reads the same block): constant address space, so loads become s_load.
typedef const __attribute__((address_space(4))) act_t c_act;

__device__ __forceinline__ uint32_t clamp_expert(int32_t e, uint32_t n) {
    return (e < 0 || (uint32_t)e >= n) ? 0u : (uint32_t)e;
}

// Data that one workgroup hands to another inside a launch is written and
// read with agent-scope accesses (global_store/load ... sc1): the store is
// acknowledged once it is coherent across all XCDs and the load bypasses the
// XCD-local caches, so no cache-wide writeback or invalidate is needed.
__device__ __forceinline__ void st_shared(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_shared(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival at a counter: every wave waits for its stores to be acknowledged,
// then thread 0 counts the workgroup.  Returns true in every thread of the
// workgroup that completed the count.  Loads after a true return that read
// other workgroups' data go through ld_shared.
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t target, int *flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = atomicAdd(counter, 1u);
        *flag = (old + 1u == target) ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

}  // namespace

using dec_params = sf37_dec_params;

namespace {

// counter layout: [0] route arrivals, [1..3) reserved
constexpr uint32_t CNT_FIXED = 3;

// LDS layout sizes, shared by the kernels and the host-side launch plan.
// A weight tile buffer holds the tile plus the copy's leading offset.
__host__ __device__ constexpr uint32_t tile_buf(uint32_t bytes) { return (bytes + 31u + 15u) & ~15u; }
__host__ __device__ constexpr uint32_t up_shared_tile(uint32_t K) { return SH_RS * (K / 32u) * SF37_Q8_0_BYTES; }
// down: per-wave tile buffer holding a routed 64-row tile; shared-down
// items take as many rows as fit (and as the 64 lanes allow for T tokens)
__host__ __device__ constexpr uint32_t dn_buf_bytes(uint32_t F) {
    return tile_buf(DN_TILE * (F / SF37_QK) * SF37_Q2_BYTES);
}
__host__ __device__ constexpr uint32_t sh_dn_rows(uint32_t F, uint32_t T) {
    return (64u / T) < (DN_TILE * (F / SF37_QK) * SF37_Q2_BYTES) / ((F / 32u) * SF37_Q8_0_BYTES)
               ? 64u / T
               : (DN_TILE * (F / SF37_QK) * SF37_Q2_BYTES) / ((F / 32u) * SF37_Q8_0_BYTES);
}
// up workgroup: x of every token, then group info, sorted pairs, weights
__host__ __device__ constexpr size_t lds_up_routed(uint32_t K, uint32_t T, uint32_t G, uint32_t P) {
    return (size_t)T * (K / SF37_QK) * sizeof(act_t) + (size_t)(3u + 2u * G + 2u * P) * 4u;
}
__host__ __device__ constexpr size_t lds_up_shared(uint32_t K, uint32_t T) {
    return 2u * (size_t)tile_buf(up_shared_tile(K)) + (size_t)T * 2u * SH_RS * (K / 32u) * 4u;
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

__global__ void __launch_bounds__(256) dec_route_kernel(dec_params p, uint32_t n_router) {
    __shared__ double part[DEC_MAX_TOK][4];
    __shared__ uint64_t tab[32];
    __shared__ uint32_t s_e[DEC_MAX_TOK * 16];
    __shared__ uint32_t s_less[DEC_MAX_TOK * 16];
    __shared__ uint32_t s_first[DEC_MAX_TOK * 16];
    __shared__ uint32_t s_ng;
    __shared__ int flag;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nb = p.K / SF37_QK;
    if (blockIdx.x < n_router) {
        const uint32_t e = blockIdx.x;
        sf37_router_rows(p.router_w + (uint64_t)e * p.K, p.x, p.K, p.T, part);
        __syncthreads();
        if (threadIdx.x < p.T) {
            const uint32_t t = threadIdx.x;
            st_shared(p.logits + (uint64_t)t * p.E + e, sf37_router_combine(part[t]));
        }
    } else {
        // Q8_K (and Q8_0) of one 256-block of one token per wave
        const uint32_t wq = (blockIdx.x - n_router) * 4u + wave;
        if (wq < p.T * nb) {
            const uint32_t t = wq / nb, b = wq - t * nb;
            const float *xb = p.x + (uint64_t)t * p.K + (uint64_t)b * SF37_QK + 4u * lane;
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = xb[k];
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
        }
    }
    if (!arrive_last(p.cnt, gridDim.x, &flag)) return;

    // ---- last workgroup: clear the next counters, top-k, groups ----------
    const uint32_t n_clear = CNT_FIXED - 1u;
    for (uint32_t i = threadIdx.x; i < n_clear; i += blockDim.x) p.cnt[1 + i] = 0u;
    sf37_stage_exp_tab(tab);
    __syncthreads();
    if (p.flags & SF37_DEC_SELECT) {
        // wave w: tokens w, w + 4, ... two at a time
        for (uint32_t t = wave; t < p.T; t += 8u) {
            const uint32_t t2 = t + 4u < p.T ? t + 4u : t;
            const float *lg0 = p.logits_sel + (uint64_t)t * p.E, *lg1 = p.logits_sel + (uint64_t)t2 * p.E;
            int32_t *so[2] = {p.sel + (uint64_t)t * p.topk, p.sel + (uint64_t)t2 * p.topk};
            float *wo[2] = {p.wts + (uint64_t)t * p.topk, p.wts + (uint64_t)t2 * p.topk};
            float *po[2] = {nullptr, nullptr};
            sf37_wave_topk<2>([lg0, lg1](uint32_t k, uint32_t e) { return ld_shared((k ? lg1 : lg0) + e); },
                              p.router_bias, p.E, p.topk, p.scale, tab, so, wo, po);
        }
    }
    __syncthreads();
    const uint32_t P = p.T * p.topk;
    if (threadIdx.x < P) s_e[threadIdx.x] = clamp_expert(p.sel[threadIdx.x], p.E);
    if (threadIdx.x == 0) s_ng = 0u;
    __syncthreads();
    if (p.flags & SF37_DEC_SLOTS) {
        if (threadIdx.x < p.topk) {
            const uint32_t s = threadIdx.x;
            p.sorted[s] = s;
            p.ginfo[1u + s] = s;
            p.ginfo[2u + p.G + s] = s_e[s];
        }
        if (threadIdx.x == 0) {
            p.ginfo[0] = p.topk;
            p.ginfo[1u + p.topk] = p.topk;
        }
    } else {
        // stable grouping: pairs ordered by (expert, pair id); a group starts
        // at the first pair of each expert
        if (threadIdx.x < P) {
            const uint32_t i = threadIdx.x, e = s_e[i];
            uint32_t less = 0, eq_before = 0;
#pragma unroll 8
            for (uint32_t q = 0; q < P; q++) {
                const uint32_t f = s_e[q];
                less += f < e ? 1u : 0u;
                eq_before += (f == e && q < i) ? 1u : 0u;
            }
            p.sorted[less + eq_before] = i;
            s_less[i] = less;
            s_first[i] = eq_before == 0u ? 1u : 0u;
        }
        __syncthreads();
        if (threadIdx.x < P && s_first[threadIdx.x]) {
            const uint32_t i = threadIdx.x, e = s_e[i];
            uint32_t gi = 0;
#pragma unroll 8
            for (uint32_t q = 0; q < P; q++) gi += (s_first[q] && s_e[q] < e) ? 1u : 0u;
            p.ginfo[1u + gi] = s_less[i];
            p.ginfo[2u + p.G + gi] = e;
            atomicAdd(&s_ng, 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            p.ginfo[0] = s_ng;
            p.ginfo[1u + s_ng] = P;
        }
    }
    if (threadIdx.x == 0) p.cnt[0] = 0u;
}

// ---------------------------------------------------------------------------
// shared gate/up: one workgroup per SH_RS rows, terms in LDS, then the
// reference's sequential block sum per (matrix, token, row)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dec_shup_kernel(dec_params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nb8 = p.K / 32u;
    const uint32_t row0 = blockIdx.x * SH_RS;
    const uint32_t tbytes = up_shared_tile(p.K), wbuf = tile_buf(tbytes);
    const uint64_t row_bytes = (uint64_t)nb8 * SF37_Q8_0_BYTES;
    uint8_t *wl = smem;                                             // gate tile | up tile
    float *red = (float *)(smem + 2u * wbuf);                       // [T][2][RS][nb8]
    const uint32_t og = lds_copy(wl, p.sh_gate + (uint64_t)row0 * row_bytes, tbytes);
    const uint32_t ou = wbuf + lds_copy(wl + wbuf, p.sh_up + (uint64_t)row0 * row_bytes, tbytes);
    lds_copy_wait();
    const uint32_t units = 2u * SH_RS * nb8;
    for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
        const uint32_t m = u / (SH_RS * nb8);
        const uint32_t rb = u - m * SH_RS * nb8;
        const uint32_t r = rb / nb8, b = rb - r * nb8;
        uint32_t q[8];
        const float wsc = q8_0_lds(wl, (m ? ou : og) + (r * nb8 + b) * SF37_Q8_0_BYTES, q);
        for (uint32_t t = 0; t < p.T; t++) {
            const uint32_t *xv = (const uint32_t *)(p.xq8 + (uint64_t)t * p.K + (uint64_t)b * 32u);
            int32_t isum = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) isum = sdot4(q[k], xv[k], isum);
            red[((t * 2u + m) * SH_RS + r) * nb8 + b] = (float)isum * wsc * p.xs8[(uint64_t)t * nb8 + b];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < p.T * 2u * SH_RS; i += blockDim.x) {
        const uint32_t t = i / (2u * SH_RS), mr = i - t * 2u * SH_RS;
        const uint32_t m = mr / SH_RS, r = mr - m * SH_RS;
        const float *rv = red + (uint64_t)i * nb8;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nb8; b++) acc = acc + rv[b];
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
// of each 16-lane row: a scan with row_shr:1, exact canonical order.  The
// row's total ends in lane nb-1.
__device__ __forceinline__ float block_chain(float d, float bs, uint32_t nb) {
    float acc = __builtin_fmaf(d, bs, 0.0f);
    for (uint32_t st = 1; st < nb; st++) {
        const float prev =
            __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x111, 0xf, 0xf, true));
        acc = __builtin_fmaf(d, bs, prev);
    }
    return acc;
}

// Keeps the compiler from hoisting work on w out of a loop (an empty asm
// that may change the registers), so unpacked codes are not all kept live.
template <int N>
__device__ __forceinline__ void opaque(uint32_t *w) {
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(w[i]));
}

// An item is 2 rows of one group's expert for both matrices: lane = matrix
// (gate/up) | row | block, so each wave reads two contiguous 2-row spans.
// Waves stride over the items (adjacent waves, adjacent rows) and load the
// next item's blocks while computing the current one.  The x of every token
// sits in LDS; the gate lane of each row applies SwiGLU * routing weight.
__global__ void __launch_bounds__(256) dec_up_kernel(dec_params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ uint64_t tab[32];
    const uint32_t nbK = p.K / SF37_QK, P = p.T * p.topk;
    act_t *xs = (act_t *)smem;
    uint32_t *gi = (uint32_t *)(xs + p.T * nbK);
    uint32_t *so = gi + 3u + 2u * p.G;
    float *wt = (float *)(so + P);
    sf37_stage_exp_tab(tab);
    const uint32_t n_x = p.T * nbK * (uint32_t)(sizeof(act_t) / 16u);
    for (uint32_t i = threadIdx.x; i < n_x; i += blockDim.x) ((u32x4 *)xs)[i] = ((const u32x4 *)p.xq)[i];
    for (uint32_t i = threadIdx.x; i < 3u + 2u * p.G; i += blockDim.x) gi[i] = p.ginfo[i];
    for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) {
        so[i] = p.sorted[i];
        wt[i] = p.wts[i];
    }
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t m = lane >> 5, rr = (lane >> 4) & 1u, b = lane & 15u;
    const uint32_t bl = b < nbK ? b : nbK - 1u;                    // lanes past the row repeat its last block
    const bool out_lane = m == 0u && b == nbK - 1u;
    const uint32_t ipg = p.F / 2u, n_items = gi[0] * ipg;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6);
    const uint64_t row_bytes = (uint64_t)nbK * SF37_Q3_BYTES, exp_bytes = (uint64_t)p.F * row_bytes;
    const uint8_t *W = m ? p.up_w : p.gate_w;
    auto block_ptr = [&](uint32_t item) -> const uint8_t * {
        const uint32_t g = item / ipg, rp = item - g * ipg;
        return W + (uint64_t)gi[2u + p.G + g] * exp_bytes + (uint64_t)(2u * rp + rr) * row_bytes +
               (uint64_t)bl * SF37_Q3_BYTES;
    };
    uint32_t item = blockIdx.x * (blockDim.x >> 6) + wave;
    if (item >= n_items) return;
    uint32_t nxt[28];
    load_q3(nxt, block_ptr(item));
    for (; item < n_items; item += nw) {
        uint32_t raw[28], a[27];
#pragma unroll
        for (int k = 0; k < 28; k++) raw[k] = nxt[k];
        const uint8_t *cur = block_ptr(item);
        if (item + nw < n_items) load_q3(nxt, block_ptr(item + nw));
        q3_realign(a, raw, (uint32_t)((uintptr_t)cur & 3u));
        const uint32_t g = item / ipg, row = 2u * (item - g * ipg) + rr;
        const uint32_t p0 = gi[1u + g], p1 = gi[2u + g];
        for (uint32_t c0 = p0; c0 < p1; c0 += DEC_TPC) {
            const uint32_t nt = p1 - c0 < DEC_TPC ? p1 - c0 : DEC_TPC;
            opaque<27>(a);
            const act_t *x[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) x[t] = xs + (so[c0 + (t < nt ? t : 0u)] / p.topk) * nbK + bl;
            float bs[DEC_TPC];
            switch (nt) {
                case 1: q3_block_dots<1>(a, x, bs); break;
                case 2: q3_block_dots<2>(a, x, bs); break;
                case 3: q3_block_dots<3>(a, x, bs); break;
                default: q3_block_dots<4>(a, x, bs); break;
            }
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) {
                if (t < nt) {
                    const float acc = block_chain(x[t]->d, bs[t], nbK);
                    const float up = __shfl_xor(acc, 32, 64);
                    if (out_lane) {
                        const uint32_t pr = so[c0 + t];
                        const uint64_t o = (uint64_t)pr * p.F + row;
                        if (p.gate_out) {
                            p.gate_out[o] = acc;
                            p.up_out[o] = up;
                        }
                        p.mid[o] = sf37_swiglu_mid_t(acc, up, wt[pr], p.clamp_routed, tab);
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// mid: Q8_K of the routed mid (one wave per pair and 256-row block, Q2 act
// layout) and, for the shared expert, SwiGLU + Q8_0 (one half-wave per token
// and 32-row block)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dec_mid_kernel(dec_params p) {
    __shared__ uint64_t tab[32];
    sf37_stage_exp_tab(tab);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nbm = p.F / SF37_QK, n_routed = p.T * p.topk * nbm;
    if (w < n_routed) {
        const uint32_t pr = w / nbm, blk = w - pr * nbm;
        const float *mv = p.mid + (uint64_t)pr * p.F + (uint64_t)blk * SF37_QK + 4u * lane;
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = mv[k];
        int8_t qk[4];
        int gsum;
        const float d = q8k_codes4(v, qk, gsum);
        act_t *y = (act_t *)p.midq + w;
        uint8_t *qb = (uint8_t *)y->qs;
#pragma unroll
        for (int k = 0; k < 4; k++) qb[q2_perm_pos(4u * lane + k)] = (uint8_t)qk[k];
        if (lane == 0) y->d = d;
        if ((lane & 15u) == 0) y->gs[lane >> 4] = gsum;
        return;
    }
    if (!(p.flags & SF37_DEC_SHARED)) return;
    const uint32_t nb8 = p.F / 32u;
    const uint32_t hw = 2u * (w - n_routed) + (lane >> 5), l = lane & 31u;
    if (hw >= p.T * nb8) return;
    const uint32_t t = hw / nb8, blk = hw - t * nb8;
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
    if (l == 0) p.sh_ms[(uint64_t)t * nb8 + blk] = d;
}

// ---------------------------------------------------------------------------
// down + combine
// ---------------------------------------------------------------------------

// Per-wave LDS tile copy: bytes [src, src + n) with direct global->LDS
// dwordx4 loads (one contiguous KiB per instruction), starting at the
// 16-byte boundary at or below src.  Returns the offset of src in dst; the
// caller waits with wave_lds_wait() before reading.
__device__ __forceinline__ uint32_t wave_lds_copy(uint8_t *dst, const uint8_t *src, uint32_t n) {
    const uintptr_t a0 = (uintptr_t)src & ~(uintptr_t)15;
    const uint32_t off = (uint32_t)((uintptr_t)src - a0);
    const uint32_t chunks = (off + n + 15u) >> 4, lane = threadIdx.x & 63u;
    for (uint32_t c0 = 0; c0 < chunks; c0 += 64u) {
        if (c0 + lane < chunks)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + 16u * (uintptr_t)(c0 + lane)), dst + 16u * c0, 16, 0, 0);
    }
    return off;
}

__device__ __forceinline__ void wave_lds_wait() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// Block values of one Q2 block (21 dwords in a) against NT activation blocks
// read through the scalar cache: bs[t] = sum_g fma(s_g, I_g).
template <int NT>
__device__ __forceinline__ void q2_block_dots(const uint32_t *a, c_act *const *x, float bs[4]) {
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
            int32_t acc = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) acc = sdot4(c[k], x[t]->qs[16 * g + k], acc);
            bs[t] = __builtin_fmaf(sc, (float)(acc - __mul24(zp, x[t]->gs[g])), bs[t]);
        }
        __builtin_amdgcn_sched_barrier(0);            // one group's codes live at a time
    }
}

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
__device__ __forceinline__ float seg_chain(float d, float bs, uint32_t b, uint32_t nb) {
    float acc = __builtin_fmaf(d, bs, 0.0f);
    for (uint32_t st = 1; st < nb; st++) {
        const float prev =
            __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x111, 0xf, 0xf, true));
        acc = __builtin_fmaf(d, bs, b == 0u ? 0.0f : prev);
    }
    return acc;
}

// Routed down.  Lane = (row, block): each 16-lane DPP row holds 16/nb rows
// with their nb blocks on consecutive lanes, so a wave reads 64/nb*4 rows
// (12 for F = 1280) as one contiguous span.  A wave owns a contiguous range
// of these sub-items (mostly inside one group); the group's activation
// blocks for up to four pairs sit in the wave's LDS slice.  The next
// sub-item's blocks are loaded while the current one is computed.
__global__ void __launch_bounds__(256) dec_down_kernel(dec_params p) {
    __shared__ uint32_t meta[3u + 2u * 256u + 256u];
    __shared__ __align__(16) act_t xsl[4][DN_TPC * DN_MAX_NB];
    const uint32_t P = p.T * p.topk;
    uint32_t *gi = meta;
    uint32_t *so = gi + 3u + 2u * p.G;
    for (uint32_t i = threadIdx.x; i < 3u + 2u * p.G; i += blockDim.x) gi[i] = p.ginfo[i];
    for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) so[i] = p.sorted[i];
    __syncthreads();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    act_t *xw = xsl[wave];
    const uint32_t nb = p.F / SF37_QK, rpd = 16u / nb, rpw = 4u * rpd;     // rows per DPP row / wave
    const uint32_t q = lane & 15u, r_in = q / nb, b = q - r_in * nb;
    const bool active = r_in < rpd;
    const uint32_t rl = (lane >> 4) * rpd + (active ? r_in : 0u);          // row within the sub-item
    const uint32_t spg = (p.K + rpw - 1u) / rpw, n_sub = gi[0] * spg;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6), gw = blockIdx.x * (blockDim.x >> 6) + wave;
    const uint32_t lo = (uint32_t)((uint64_t)n_sub * gw / nw), hi = (uint32_t)((uint64_t)n_sub * (gw + 1u) / nw);
    if (lo >= hi) return;
    const uint64_t row_bytes = (uint64_t)nb * SF37_Q2_BYTES;
    auto blk_ptr = [&](uint32_t sidx) -> const uint8_t * {
        const uint32_t g = sidx / spg, sub = sidx - g * spg;
        uint32_t row = sub * rpw + rl;
        row = row < p.K ? row : p.K - 1u;                                    // keep tail lanes in bounds
        return p.down_w + ((uint64_t)gi[2u + p.G + g] * p.K + row) * row_bytes + (uint64_t)b * SF37_Q2_BYTES;
    };
    uint32_t staged_g = 0xffffffffu, staged_c0 = 0xffffffffu;
    uint32_t nxt[21];
    load_q2(nxt, blk_ptr(lo));
    for (uint32_t sidx = lo; sidx < hi; sidx++) {
        uint32_t w[21];
#pragma unroll
        for (int i = 0; i < 21; i++) w[i] = nxt[i];
        if (sidx + 1u < hi) load_q2(nxt, blk_ptr(sidx + 1u));
        const uint32_t g = sidx / spg, sub = sidx - g * spg;
        const uint32_t row = sub * rpw + rl;
        const bool out_lane = active && b == nb - 1u && row < p.K;
        const uint32_t p0 = gi[1u + g], p1 = gi[2u + g];
        for (uint32_t c0 = p0; c0 < p1; c0 += DN_TPC) {
            const uint32_t nt = p1 - c0 < DN_TPC ? p1 - c0 : DN_TPC;
            if (g != staged_g || c0 != staged_c0) {
                // stage this pass's activation blocks (nt pairs x nb blocks)
                __builtin_amdgcn_wave_barrier();
                const uint32_t words = nt * nb * (uint32_t)(sizeof(act_t) / 16u);
                for (uint32_t i = lane; i < words; i += 64u) {
                    const uint32_t per = nb * (uint32_t)(sizeof(act_t) / 16u);
                    const uint32_t t = i / per, k = i - t * per;
                    ((u32x4 *)xw)[i] = ((const u32x4 *)((const act_t *)p.midq + (uint64_t)so[c0 + t] * nb))[k];
                }
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_wave_barrier();
                staged_g = g;
                staged_c0 = c0;
            }
            opaque<21>(w);
            const act_t *x[DEC_TPC];
#pragma unroll
            for (uint32_t t = 0; t < DEC_TPC; t++) x[t] = xw + (t < nt ? t : 0u) * nb + b;
            float bs[DEC_TPC];
            if (nt == 1) q2_block_dots_lds<1>(w, x, bs);
            else q2_block_dots_lds<2>(w, x, bs);
#pragma unroll
            for (uint32_t t = 0; t < DN_TPC; t++) {
                if (t < nt) {
                    const float acc = seg_chain(x[t]->d, bs[t], b, nb);
                    if (out_lane) p.down_pair[(uint64_t)so[c0 + t] * p.K + row] = acc;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// combine: out = shared + sum over slots (slot order); lane = (row, token).
// With the shared expert the lane first runs its shared-down row: the span's
// rows are copied to the wave's LDS buffer and the reference's block order
// acc = acc + (isum * ws) * xs is followed (sf37_ops.c:92-108).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(DN_WG_WAVES * 64) dec_combine_kernel(dec_params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    uint8_t *buf = smem + wave * dn_buf_bytes(p.F);
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    const uint32_t rpw = sh_dn_rows(p.F, p.T);
    const uint32_t n_items = (p.K + rpw - 1u) / rpw;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6);
    const uint32_t t = lane % p.T, rl = lane / p.T;
    const uint32_t nb8 = p.F / 32u, row_bytes = nb8 * SF37_Q8_0_BYTES;
    for (uint32_t item = blockIdx.x * (blockDim.x >> 6) + wave; item < n_items; item += nw) {
        const uint32_t r0 = item * rpw, nrows = p.K - r0 < rpw ? p.K - r0 : rpw;
        const uint32_t rc = rl < nrows ? rl : 0u, row = r0 + rc;
        // slot values first (independent loads, issued together)
        float v[16];
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const uint32_t sc = (uint32_t)s < p.topk ? (uint32_t)s : 0u;   // every read in bounds
            v[s] = p.down_pair[((uint64_t)t * p.topk + sc) * p.K + row];
        }
        float acc = 0.0f;
        if (sh) {
            const uint32_t off = wave_lds_copy(buf, p.sh_down + (uint64_t)r0 * row_bytes, nrows * row_bytes);
            wave_lds_wait();
            const int8_t *xq = p.sh_mq + (uint64_t)t * p.F;
            const float *xs = p.sh_ms + (uint64_t)t * nb8;
            const uint32_t base = off + rc * row_bytes;
            for (uint32_t b0 = 0; b0 < nb8; b0 += 8u) {
                uint32_t xv[8][8];
                float xsc[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t b = b0 + j < nb8 ? b0 + j : nb8 - 1u;
                    const u32x4 *xp = (const u32x4 *)(xq + (uint64_t)b * 32u);
                    const u32x4 x0 = xp[0], x1 = xp[1];
                    xv[j][0] = x0.x; xv[j][1] = x0.y; xv[j][2] = x0.z; xv[j][3] = x0.w;
                    xv[j][4] = x1.x; xv[j][5] = x1.y; xv[j][6] = x1.z; xv[j][7] = x1.w;
                    xsc[j] = xs[b];
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (b0 + j < nb8) {
                        uint32_t q[8];
                        const float wsc = q8_0_lds(buf, base + (b0 + j) * SF37_Q8_0_BYTES, q);
                        int32_t isum = 0;
#pragma unroll
                        for (int k = 0; k < 8; k++) isum = sdot4(q[k], xv[j][k], isum);
                        acc = acc + (float)isum * wsc * xsc[j];
                    }
                }
            }
            // the next item's copy must not overwrite rows still being read
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_wave_barrier();
        }
        float r = 0.0f;
#pragma unroll
        for (int s = 0; s < 16; s++)
            if ((uint32_t)s < p.topk) r = r + v[s];
        if (rl < nrows) p.out[(uint64_t)t * p.K + row] = sh ? acc + r : r;
    }
}

}  // namespace

namespace {

struct dec_shape {
    uint32_t n_router, n_xq, n_shup, n_up, n_mid, n_dn, n_cb;
    size_t lds_up, lds_shup, lds_dn;
};

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

// Workgroups of this kernel one CU holds at once (from the occupancy
// calculator, at least 1), cached per (kernel, block size, LDS bytes).
// Dynamic LDS above 64 KiB is opted into first.
uint32_t resident_wgs(const void *fn, int threads, size_t lds) {
    struct entry { const void *fn; int threads; size_t lds; uint32_t n; };
    static entry cache[16];
    static int used = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].fn == fn && cache[i].threads == threads && cache[i].lds == lds) return cache[i].n;
    if (lds > 65536u) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess || n < 1) n = 1;
    (void)hipGetLastError();
    if (used < 16) cache[used++] = {fn, threads, lds, (uint32_t)n};
    return (uint32_t)n;
}

dec_shape dec_plan(const dec_params &p) {
    dec_shape d;
    const uint32_t nb = p.K / SF37_QK;
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    const uint32_t cus = device_cus();
    d.n_router = (p.flags & SF37_DEC_ROUTER) ? p.E : 0u;
    d.n_xq = (p.T * nb + 3u) / 4u;
    d.lds_up = lds_up_routed(p.K, p.T, p.G, p.T * p.topk);
    d.lds_shup = lds_up_shared(p.K, p.T);
    d.n_shup = sh ? p.F / SH_RS : 0u;
    // every up workgroup resident at once: at most 3 per CU, fewer if LDS-bound
    // persistent kernels: exactly as many workgroups as can be resident
    d.n_up = resident_wgs((const void *)dec_up_kernel, 256, d.lds_up) * cus;
    const uint32_t n_mid_waves = p.T * p.topk * (p.F / SF37_QK) + (sh ? (p.T * (p.F / 32u) + 1u) / 2u : 0u);
    d.n_mid = (n_mid_waves + 3u) / 4u;
    d.lds_dn = 0;
    d.n_dn = resident_wgs((const void *)dec_down_kernel, 256, 0) * cus;
    const uint32_t cb_items = (p.K + sh_dn_rows(p.F, p.T) - 1u) / sh_dn_rows(p.F, p.T);
    d.n_cb = (cb_items + DN_WG_WAVES - 1u) / DN_WG_WAVES;
    return d;
}

}  // namespace

extern "C" int sf37k_decode_counters(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F) {
    (void)T; (void)topk; (void)E; (void)F; (void)K;
    return (int)CNT_FIXED;
}

extern "C" int sf37k_decode_supported(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F, int shared) {
    if (T == 0 || T > DEC_MAX_TOK || topk == 0 || K % SF37_QK || F % SF37_QK || K / SF37_QK > 16u ||
        F / SF37_QK > DN_MAX_NB || K % DN_TILE)
        return 0;
    const uint32_t P = T * topk, G = P < E ? P : E;
    if (lds_up_routed(K, T, G, P) > device_max_lds()) return 0;
    if (shared && lds_up_shared(K, T) > device_max_lds()) return 0;
    return 1;
}

namespace {
int set_lds(const void *fn, size_t bytes, size_t *opted) {
    if (bytes <= *opted) return 0;
    const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (err != hipSuccess) return (int)err;
    *opted = bytes;
    return 0;
}
}  // namespace

extern "C" int sf37k_decode_route(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_route_kernel, dim3(d.n_router + d.n_xq), dim3(256), 0, (hipStream_t)s, *pp, d.n_router);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_shared_up(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    if (!d.n_shup) return 0;
    static size_t opted = 65536;
    const int err = set_lds((const void *)dec_shup_kernel, d.lds_shup, &opted);
    if (err) return err;
    hipLaunchKernelGGL(dec_shup_kernel, dim3(d.n_shup), dim3(256), d.lds_shup, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_up(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    static size_t opted = 65536;
    const int err = set_lds((const void *)dec_up_kernel, d.lds_up, &opted);
    if (err) return err;
    hipLaunchKernelGGL(dec_up_kernel, dim3(d.n_up), dim3(256), d.lds_up, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_mid(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_mid_kernel, dim3(d.n_mid), dim3(256), 0, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_down(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_down_kernel, dim3(d.n_dn), dim3(256), 0, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_combine(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    const size_t lds = (pp->flags & SF37_DEC_SHARED) ? (size_t)DN_WG_WAVES * dn_buf_bytes(pp->F) : 0u;
    static size_t opted = 65536;
    const int err = set_lds((const void *)dec_combine_kernel, lds, &opted);
    if (err) return err;
    hipLaunchKernelGGL(dec_combine_kernel, dim3(d.n_cb), dim3(DN_WG_WAVES * 64), lds, (hipStream_t)s, *pp);
    return (int)hipGetLastError();
}
