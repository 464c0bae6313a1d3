// k_decode.hip - the MoE layer for decode batches (up to 16 tokens) in three
// launches on gfx950.
//
//   route : router GEMV (binary64 accumulation) and the Q8_K / Q8_0
//           quantisation of x; the last workgroup to finish runs top-k for
//           every token, groups the (token, slot) pairs by expert and clears
//           the counters of the next two launches.
//   up    : routed gate/up (Q3 x Q8_K) with SwiGLU * routing weight, and the
//           shared expert's gate/up (Q8_0).  The last workgroup of each
//           256-row block quantises that block of mid to Q8_K; the last of
//           each 32-row shared block applies SwiGLU and quantises to Q8_0.
//   down  : routed down (Q2 x Q8_K) per pair and the shared down (Q8_0); the
//           last workgroup of each 64-row tile forms out = shared + sum over
//           slots in slot order.
//
// Hand-offs between workgroups use agent-coherent stores and loads and an atomic
// arrival counter; the workgroup that brings a counter to its target does
// the dependent work and resets the counter.  Nothing waits on another
// workgroup, so every wave always runs to completion.
//
// Arithmetic is the canonical order of the oracle (sf37_blocks.h), the
// reference CPU order for the Q8_0 shared expert (sf37_ops.c:92-108), and
// slot-order combines, so results equal the separate-kernel path bit for bit.
#include "sf37_blocks.h"
#include "sf37_launch.h"

namespace {

constexpr uint32_t DEC_MAX_TOK = 16;
constexpr uint32_t DEC_TPC = 4;      // pairs per pass in the routed kernels
constexpr uint32_t UP_RT = 8;        // routed gate/up rows per workgroup
constexpr uint32_t SH_RS = 2;        // shared gate/up rows per workgroup
constexpr uint32_t DN_TILE = 64;     // down rows per workgroup (= combine tile)
constexpr uint32_t SH_SUB = 16;      // shared down rows per pass

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

// One token's top-k by a full wave (sf37.c:2144-2157): lane l owns experts
// l + 64j.  Ties go to the lower index; weights = p / max(sum p, 1e-20) * scale.
__device__ void wave_topk(const float *lg, const float *bias, uint32_t E, uint32_t topk, float scale,
                          const uint64_t *tab, int32_t *sel_out, float *w_out) {
    const uint32_t lane = threadIdx.x & 63u;
    float prob[16], score[16];
    uint32_t taken = 0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t e = lane + 64u * j;
        prob[j] = 0.0f;
        score[j] = -__builtin_inff();
        if (e < E) {
            const float p = sf37_sigmoid_t(ld_shared(lg + e), tab);
            prob[j] = p;
            score[j] = p + bias[e];
        } else {
            taken |= 1u << j;
        }
    }
    float sum = 0.0f;
    for (uint32_t k = 0; k < topk; k++) {
        float bs = -__builtin_inff(), bp = 0.0f;
        uint32_t bi = 0xffffffffu;
        int bj = -1;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t e = lane + 64u * j;
            const bool better = score[j] > bs || (score[j] == bs && e < bi);
            if (!((taken >> j) & 1u) && better) {
                bs = score[j];
                bp = prob[j];
                bi = e;
                bj = j;
            }
        }
        float ws = bs, wp = bp;
        uint32_t wi = bi;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float os = __shfl_xor(ws, off, 64);
            const float op = __shfl_xor(wp, off, 64);
            const uint32_t oi = __shfl_xor(wi, off, 64);
            if (os > ws || (os == ws && oi < wi)) {
                ws = os;
                wp = op;
                wi = oi;
            }
        }
        if (wi != 0xffffffffu && bi == wi && bj >= 0) taken |= 1u << bj;
        const float pk = wi == 0xffffffffu ? 0.0f : wp;
        sum += pk;                                   // slot order, every lane identical
        if (lane == 0) {
            sel_out[k] = wi == 0xffffffffu ? -1 : (int32_t)wi;
            w_out[k] = pk;
        }
    }
    if (sum < 1.0e-20f) sum = 1.0e-20f;
    if (lane == 0)
        for (uint32_t k = 0; k < topk; k++) w_out[k] = w_out[k] / sum * scale;
}

}  // namespace

using dec_params = sf37_dec_params;

namespace {

// counter layout: [0] route, then routed mid blocks G*(F/256), shared mid
// blocks F/32, down tiles K/64
__device__ __forceinline__ uint32_t *cnt_up(const dec_params &p) { return p.cnt + 1; }
__device__ __forceinline__ uint32_t *cnt_sh(const dec_params &p) { return p.cnt + 1 + p.G * (p.F / SF37_QK); }
__device__ __forceinline__ uint32_t *cnt_dn(const dec_params &p) {
    return p.cnt + 1 + p.G * (p.F / SF37_QK) + p.F / 32u;
}

// LDS layout sizes, shared by the kernels and the host-side launch plan.
// A weight tile buffer holds the tile plus the copy's leading offset.
__host__ __device__ constexpr uint32_t tile_buf(uint32_t bytes) { return (bytes + 31u + 15u) & ~15u; }
__host__ __device__ constexpr uint32_t up_routed_tile(uint32_t K) { return UP_RT * (K / SF37_QK) * SF37_Q3_BYTES; }
__host__ __device__ constexpr uint32_t up_shared_tile(uint32_t K) { return SH_RS * (K / 32u) * SF37_Q8_0_BYTES; }
__host__ __device__ constexpr uint32_t dn_routed_tile(uint32_t F) { return DN_TILE * (F / SF37_QK) * SF37_Q2_BYTES; }
__host__ __device__ constexpr uint32_t dn_shared_tile(uint32_t F) { return SH_SUB * (F / 32u) * SF37_Q8_0_BYTES; }
__host__ __device__ constexpr size_t lds_up_routed(uint32_t K) {
    return 2u * (size_t)tile_buf(up_routed_tile(K)) + (size_t)DEC_TPC * (K / SF37_QK) * sizeof(act_block) +
           (size_t)DEC_TPC * 2u * UP_RT * (K / SF37_QK) * 4u + (size_t)DEC_TPC * 2u * UP_RT * 4u;
}
__host__ __device__ constexpr size_t lds_up_shared(uint32_t K, uint32_t T) {
    return 2u * (size_t)tile_buf(up_shared_tile(K)) + (size_t)T * 2u * SH_RS * (K / 32u) * 4u;
}
__host__ __device__ constexpr size_t lds_dn_routed(uint32_t F) {
    return (size_t)tile_buf(dn_routed_tile(F)) + (size_t)DEC_TPC * (F / SF37_QK) * sizeof(act_block) +
           (size_t)DEC_TPC * DN_TILE * (F / SF37_QK) * 4u;
}
__host__ __device__ constexpr size_t lds_dn_shared(uint32_t F, uint32_t T) {
    return (size_t)tile_buf(dn_shared_tile(F)) + (size_t)T * SH_SUB * (F / 32u) * 4u;
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

// Router logits of expert e for NT tokens: thread i accumulates k = i,
// i + 256, ... in binary64 (the order of the separate router GEMV kernel),
// then a butterfly per wave and (w0 + w1) + (w2 + w3).  All loads of a
// 1024-wide slice are issued before the first fma.
template <int NT>
__device__ void router_row(const dec_params &p, uint32_t e, uint32_t t0, double (*part)[4]) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const float *wr = p.router_w + (uint64_t)e * p.K;
    double acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0;
    for (uint32_t k0 = 0; k0 < p.K; k0 += 256u * 4u) {
        float wv[4], xv[NT][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t k = k0 + 256u * j + threadIdx.x;
            wv[j] = k < p.K ? wr[k] : 0.0f;
#pragma unroll
            for (int t = 0; t < NT; t++) xv[t][j] = k < p.K ? p.x[(uint64_t)(t0 + t) * p.K + k] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (k0 + 256u * j + threadIdx.x < p.K) {
#pragma unroll
                for (int t = 0; t < NT; t++) acc[t] = __builtin_fma((double)wv[j], (double)xv[t][j], acc[t]);
            }
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
        // tokens in passes of at most 8 (register budget); the weight row
        // is re-read from cache by the second pass
        for (uint32_t t0 = 0; t0 < p.T; t0 += 8u) {
            switch (p.T - t0 < 8u ? p.T - t0 : 8u) {
#define SF37_ROUTER_CASE(n) \
    case n: router_row<n>(p, e, t0, part); break;
                SF37_ROUTER_CASE(1) SF37_ROUTER_CASE(2) SF37_ROUTER_CASE(3) SF37_ROUTER_CASE(4)
                SF37_ROUTER_CASE(5) SF37_ROUTER_CASE(6) SF37_ROUTER_CASE(7) SF37_ROUTER_CASE(8)
#undef SF37_ROUTER_CASE
                default: break;
            }
        }
        __syncthreads();
        if (threadIdx.x < p.T) {
            const uint32_t t = threadIdx.x;
            st_shared(p.logits + (uint64_t)t * p.E + e, (float)((part[t][0] + part[t][1]) + (part[t][2] + part[t][3])));
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
            q8k_block *y = (q8k_block *)p.xq + wq;
            ((uint32_t *)y->qs)[lane] = (uint32_t)(uint8_t)qk[0] | ((uint32_t)(uint8_t)qk[1] << 8) |
                                        ((uint32_t)(uint8_t)qk[2] << 16) | ((uint32_t)(uint8_t)qk[3] << 24);
            if (lane == 0) y->d = d;
            if ((lane & 15u) == 0) y->gsums[lane >> 4] = (int16_t)gsum;
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
    const uint32_t n_clear = p.G * (p.F / SF37_QK) + p.F / 32u + p.K / DN_TILE;
    for (uint32_t i = threadIdx.x; i < n_clear; i += blockDim.x) p.cnt[1 + i] = 0u;
    sf37_stage_exp_tab(tab);
    __syncthreads();
    if (p.flags & SF37_DEC_SELECT) {
        for (uint32_t t = wave; t < p.T; t += 4u)
            wave_topk(p.logits_sel + (uint64_t)t * p.E, p.router_bias, p.E, p.topk, p.scale, tab,
                      p.sel + (uint64_t)t * p.topk, p.wts + (uint64_t)t * p.topk);
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
// up
// ---------------------------------------------------------------------------
__device__ void up_routed(const dec_params &p, uint32_t wg, unsigned char *smem, const uint64_t *tab,
                          int *flag) {
    const uint32_t nblk = p.K / SF37_QK;
    const uint32_t tiles = p.F / UP_RT;
    const uint32_t g = wg / tiles, tile = wg - g * tiles;
    const uint32_t ng = p.ginfo[0];
    if (g >= ng) return;
    const uint32_t p0 = p.ginfo[1 + g], p1 = p.ginfo[2 + g];
    const uint32_t e = p.ginfo[2 + p.G + g];
    const uint32_t row0 = tile * UP_RT;
    const uint32_t tbytes = up_routed_tile(p.K), wbuf = tile_buf(tbytes);
    uint8_t *wl = smem;                                             // gate tile | up tile
    act_block *xs = (act_block *)(smem + 2u * wbuf);                // [TPC][nblk]
    float *red = (float *)(xs + DEC_TPC * nblk);                    // [TPC][2R][nblk]
    float *res = red + DEC_TPC * 2u * UP_RT * nblk;                 // [TPC][2R]
    const uint64_t row_bytes = (uint64_t)nblk * SF37_Q3_BYTES;
    const uint64_t src = (uint64_t)e * p.F * row_bytes + (uint64_t)row0 * row_bytes;
    const uint32_t og = lds_copy(wl, p.gate_w + src, tbytes);
    const uint32_t ou = wbuf + lds_copy(wl + wbuf, p.up_w + src, tbytes);
    const uint32_t units = 2u * UP_RT * nblk;
    for (uint32_t c0 = p0; c0 < p1; c0 += DEC_TPC) {
        const uint32_t nt = p1 - c0 < DEC_TPC ? p1 - c0 : DEC_TPC;
        for (uint32_t t = 0; t < nt; t++)
            stage_act<true>(xs + t * nblk, (const q8k_block *)p.xq + (uint64_t)(p.sorted[c0 + t] / p.topk) * nblk, nblk);
        lds_copy_wait();
        for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
            const uint32_t m = u / (UP_RT * nblk);
            const uint32_t rb = u - m * UP_RT * nblk;
            const uint32_t r = rb / nblk, b = rb - r * nblk;
            float bs[DEC_TPC] = {0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t L = (m ? ou : og) + (r * nblk + b) * SF37_Q3_BYTES;
            const uint32_t *wp = (const uint32_t *)(wl + (L & ~3u));
            uint32_t raw[28], a[27];
#pragma unroll
            for (int k = 0; k < 28; k++) raw[k] = wp[k];
            q3_realign(a, raw, L & 3u);
#pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                const uint32_t d0 = a[3 + 6 * gg], d1 = a[4 + 6 * gg], d2 = a[5 + 6 * gg];
                const uint32_t d3 = a[6 + 6 * gg], d4 = a[7 + 6 * gg], d5 = a[8 + 6 * gg];
                const uint32_t c[8] = {d0, align_bits(d1, d0, 24), align_bits(d2, d1, 16), d2 >> 8,
                                       d3, align_bits(d4, d3, 24), align_bits(d5, d4, 16), d5 >> 8};
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int k = 0; k < 8; k++) q3_unpack8(c[k], lo[k], hi[k]);
                const int32_t zp = (int32_t)((a[2] >> (8 * gg)) & 7u);
                const float sc = sf37_f16(a[gg >> 1] >> (16 * (gg & 1)));
#pragma unroll
                for (uint32_t t = 0; t < DEC_TPC; t++) {
                    if (t < nt) {
                        const act_block &x = xs[t * nblk + b];
                        int32_t acc = 0;
#pragma unroll
                        for (int k = 0; k < 8; k++) {
                            acc = sdot4(lo[k], x.qs[16 * gg + 2 * k], acc);
                            acc = sdot4(hi[k], x.qs[16 * gg + 2 * k + 1], acc);
                        }
                        bs[t] = __builtin_fmaf(sc, (float)(acc - zp * x.gs[gg]), bs[t]);
                    }
                }
            }
            for (uint32_t t = 0; t < nt; t++) red[(t * 2u * UP_RT + m * UP_RT + r) * nblk + b] = bs[t];
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * 2u * UP_RT; i += blockDim.x) {
            const uint32_t t = i / (2u * UP_RT), mr = i - t * 2u * UP_RT;
            const float *rv = red + (t * 2u * UP_RT + mr) * nblk;
            float acc = 0.0f;
            for (uint32_t b = 0; b < nblk; b++) acc = __builtin_fmaf(xs[t * nblk + b].d, rv[b], acc);
            res[t * 2u * UP_RT + mr] = acc;
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * UP_RT; i += blockDim.x) {
            const uint32_t t = i / UP_RT, r = i - t * UP_RT;
            const uint32_t pr = p.sorted[c0 + t];
            const float gv = res[t * 2u * UP_RT + r], uv = res[t * 2u * UP_RT + UP_RT + r];
            const uint64_t o = (uint64_t)pr * p.F + row0 + r;
            if (p.gate_out) {
                p.gate_out[o] = gv;
                p.up_out[o] = uv;
            }
            st_shared(p.mid + o, sf37_swiglu_mid_t(gv, uv, p.wts[pr], p.clamp_routed, tab));
        }
        __syncthreads();
    }
    // last of the 256/UP_RT tiles of this 256-row block quantises it for every pair
    const uint32_t nbm = p.F / SF37_QK, blk = row0 / SF37_QK;
    if (!arrive_last(cnt_up(p) + g * nbm + blk, SF37_QK / UP_RT, flag)) return;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    for (uint32_t i = p0 + wave; i < p1; i += blockDim.x >> 6) {
        const uint32_t pr = p.sorted[i];
        const float *mv = p.mid + (uint64_t)pr * p.F + (uint64_t)blk * SF37_QK + 4u * lane;
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = ld_shared(mv + k);
        int8_t qk[4];
        int gsum;
        const float d = q8k_codes4(v, qk, gsum);
        q8k_block *y = (q8k_block *)p.midq + (uint64_t)pr * nbm + blk;
        ((uint32_t *)y->qs)[lane] = (uint32_t)(uint8_t)qk[0] | ((uint32_t)(uint8_t)qk[1] << 8) |
                                    ((uint32_t)(uint8_t)qk[2] << 16) | ((uint32_t)(uint8_t)qk[3] << 24);
        if (lane == 0) y->d = d;
        if ((lane & 15u) == 0) y->gsums[lane >> 4] = (int16_t)gsum;
    }
    if (threadIdx.x == 0) cnt_up(p)[g * nbm + blk] = 0u;
}

__device__ void up_shared(const dec_params &p, uint32_t ws, unsigned char *smem, const uint64_t *tab, int *flag) {
    const uint32_t nb8 = p.K / 32u;
    const uint32_t row0 = ws * SH_RS;
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
        st_shared(p.sh_gu + ((uint64_t)m * p.T + t) * p.F + row0 + r, acc);
    }
    // last of the 32/RS workgroups of a 32-row block: SwiGLU and Q8_0 of mid
    const uint32_t blk = row0 / 32u;
    if (!arrive_last(cnt_sh(p) + blk, 32u / SH_RS, flag)) return;
    const uint32_t hw = threadIdx.x >> 5, l = threadIdx.x & 31u;
    for (uint32_t t = hw; t < p.T; t += blockDim.x >> 5) {
        const uint64_t o = (uint64_t)t * p.F + (uint64_t)blk * 32u + l;
        const float v = sf37_swiglu_mid_t(ld_shared(p.sh_gu + o), ld_shared(p.sh_gu + (uint64_t)p.T * p.F + o), 1.0f,
                                          p.clamp_shared, tab);
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
        if (l == 0) p.sh_ms[(uint64_t)t * (p.F / 32u) + blk] = d;
    }
    if (threadIdx.x == 0) cnt_sh(p)[blk] = 0u;
}

__global__ void __launch_bounds__(256) dec_up_kernel(dec_params p, uint32_t n_routed) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ uint64_t tab[32];
    __shared__ int flag;
    sf37_stage_exp_tab(tab);
    __syncthreads();
    if (blockIdx.x < n_routed) up_routed(p, blockIdx.x, smem, tab, &flag);
    else up_shared(p, blockIdx.x - n_routed, smem, tab, &flag);
}

// ---------------------------------------------------------------------------
// down + combine
// ---------------------------------------------------------------------------
__device__ void down_combine(const dec_params &p, uint32_t tile) {
    const uint32_t row0 = tile * DN_TILE;
    const uint32_t n = p.T * DN_TILE;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t t = i / DN_TILE, r = row0 + (i - t * DN_TILE);
        float acc = 0.0f;
        for (uint32_t s = 0; s < p.topk; s++) acc = acc + ld_shared(p.down_pair + ((uint64_t)t * p.topk + s) * p.K + r);
        const uint64_t o = (uint64_t)t * p.K + r;
        p.out[o] = (p.flags & SF37_DEC_SHARED) ? ld_shared(p.sh_out + o) + acc : acc;
    }
}

__device__ void down_routed(const dec_params &p, uint32_t wg, unsigned char *smem) {
    const uint32_t nblk = p.F / SF37_QK;
    const uint32_t tiles = p.K / DN_TILE;
    const uint32_t g = wg / tiles, tile = wg - g * tiles;
    const uint32_t p0 = p.ginfo[1 + g], p1 = p.ginfo[2 + g];
    const uint32_t e = p.ginfo[2 + p.G + g];
    const uint32_t tbytes = dn_routed_tile(p.F), wbuf = tile_buf(tbytes);
    uint8_t *wl = smem;
    act_block *xs = (act_block *)(smem + wbuf);                     // [TPC][nblk]
    float *red = (float *)(xs + DEC_TPC * nblk);                    // [TPC][TILE][nblk]
    const uint32_t row0 = tile * DN_TILE;
    const uint64_t row_bytes = (uint64_t)nblk * SF37_Q2_BYTES;
    const uint32_t od = lds_copy(wl, p.down_w + (uint64_t)e * p.K * row_bytes + (uint64_t)row0 * row_bytes, tbytes);
    const uint32_t units = DN_TILE * nblk;
    for (uint32_t c0 = p0; c0 < p1; c0 += DEC_TPC) {
        const uint32_t nt = p1 - c0 < DEC_TPC ? p1 - c0 : DEC_TPC;
        for (uint32_t t = 0; t < nt; t++)
            stage_act<false>(xs + t * nblk, (const q8k_block *)p.midq + (uint64_t)p.sorted[c0 + t] * nblk, nblk);
        lds_copy_wait();
        for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
            const uint32_t r = u / nblk, b = u - r * nblk;
            float bs[DEC_TPC] = {0.0f, 0.0f, 0.0f, 0.0f};
            uint32_t a[21];
            const uint32_t *wp = (const uint32_t *)(wl + ((od + (r * nblk + b) * SF37_Q2_BYTES) & ~3u));
#pragma unroll
            for (int k = 0; k < 21; k++) a[k] = wp[k];
#pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                uint32_t cw[16];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    q2_unpack16(a[3 + 4 * gg + j], cw[4 * j], cw[4 * j + 1], cw[4 * j + 2], cw[4 * j + 3]);
                const int32_t zp = (int32_t)((a[2] >> (8 * gg)) & 3u);
                const float sc = sf37_f16(a[gg >> 1] >> (16 * (gg & 1)));
#pragma unroll
                for (uint32_t t = 0; t < DEC_TPC; t++) {
                    if (t < nt) {
                        const act_block &x = xs[t * nblk + b];
                        int32_t acc = 0;
#pragma unroll
                        for (int k = 0; k < 16; k++) acc = sdot4(cw[k], x.qs[16 * gg + k], acc);
                        bs[t] = __builtin_fmaf(sc, (float)(acc - zp * x.gs[gg]), bs[t]);
                    }
                }
            }
            for (uint32_t t = 0; t < nt; t++) red[(t * DN_TILE + r) * nblk + b] = bs[t];
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * DN_TILE; i += blockDim.x) {
            const uint32_t t = i / DN_TILE, r = i - t * DN_TILE;
            const float *rv = red + (t * DN_TILE + r) * nblk;
            float acc = 0.0f;
            for (uint32_t b = 0; b < nblk; b++) acc = __builtin_fmaf(xs[t * nblk + b].d, rv[b], acc);
            st_shared(p.down_pair + (uint64_t)p.sorted[c0 + t] * p.K + row0 + r, acc);
        }
        __syncthreads();
    }
}

// Shared down rows [row0, row0 + SH_SUB) for every token.
__device__ void down_shared(const dec_params &p, uint32_t row0, unsigned char *smem) {
    const uint32_t nb8 = p.F / 32u;
    const uint32_t tbytes = dn_shared_tile(p.F), wbuf = tile_buf(tbytes);
    const uint64_t row_bytes = (uint64_t)nb8 * SF37_Q8_0_BYTES;
    uint8_t *wl = smem;
    float *red = (float *)(smem + wbuf);                            // [T][SUB][nb8]
    const uint32_t ow = lds_copy(wl, p.sh_down + (uint64_t)row0 * row_bytes, tbytes);
    lds_copy_wait();
    for (uint32_t u = threadIdx.x; u < SH_SUB * nb8; u += blockDim.x) {
        const uint32_t r = u / nb8, b = u - r * nb8;
        uint32_t q[8];
        const float wsc = q8_0_lds(wl, ow + (r * nb8 + b) * SF37_Q8_0_BYTES, q);
        for (uint32_t t = 0; t < p.T; t++) {
            const uint32_t *xv = (const uint32_t *)(p.sh_mq + (uint64_t)t * p.F + (uint64_t)b * 32u);
            int32_t isum = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) isum = sdot4(q[k], xv[k], isum);
            red[((uint64_t)t * SH_SUB + r) * nb8 + b] = (float)isum * wsc * p.sh_ms[(uint64_t)t * nb8 + b];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < p.T * SH_SUB; i += blockDim.x) {
        const uint32_t t = i / SH_SUB, r = i - t * SH_SUB;
        const float *rv = red + (uint64_t)i * nb8;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nb8; b++) acc = acc + rv[b];
        st_shared(p.sh_out + (uint64_t)t * p.K + row0 + r, acc);
    }
}

__global__ void __launch_bounds__(320) dec_down_kernel(dec_params p, uint32_t n_routed) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int flag;
    const uint32_t tiles = p.K / DN_TILE;
    uint32_t tile;
    if (blockIdx.x < n_routed) {
        const uint32_t g = blockIdx.x / tiles;
        tile = blockIdx.x - g * tiles;
        if (g >= p.ginfo[0]) return;
        down_routed(p, blockIdx.x, smem);
    } else {
        const uint32_t s = blockIdx.x - n_routed;
        tile = s / (DN_TILE / SH_SUB);
        down_shared(p, s * SH_SUB, smem);
    }
    const uint32_t target = p.ginfo[0] + ((p.flags & SF37_DEC_SHARED) ? DN_TILE / SH_SUB : 0u);
    if (!arrive_last(cnt_dn(p) + tile, target, &flag)) return;
    down_combine(p, tile);
    if (threadIdx.x == 0) cnt_dn(p)[tile] = 0u;
}

}  // namespace

namespace {

struct dec_shape {
    uint32_t n_router, n_xq, n_up_routed, n_up_shared, n_dn_routed, n_dn_shared;
    size_t lds_up, lds_dn;
};

dec_shape dec_plan(const dec_params &p) {
    dec_shape d;
    const uint32_t nb = p.K / SF37_QK;
    const bool sh = (p.flags & SF37_DEC_SHARED) != 0;
    d.n_router = (p.flags & SF37_DEC_ROUTER) ? p.E : 0u;
    d.n_xq = (p.T * nb + 3u) / 4u;
    const size_t up_r = lds_up_routed(p.K), up_s = sh ? lds_up_shared(p.K, p.T) : 0u;
    d.lds_up = up_r > up_s ? up_r : up_s;
    const size_t dn_r = lds_dn_routed(p.F), dn_s = sh ? lds_dn_shared(p.F, p.T) : 0u;
    d.lds_dn = dn_r > dn_s ? dn_r : dn_s;
    d.n_up_routed = p.G * (p.F / UP_RT);
    d.n_up_shared = sh ? p.F / SH_RS : 0u;
    d.n_dn_routed = p.G * (p.K / DN_TILE);
    d.n_dn_shared = sh ? p.K / SH_SUB : 0u;
    return d;
}

}  // namespace

extern "C" int sf37k_decode_counters(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F) {
    const uint32_t P = T * topk, G = P < E ? P : E;
    return (int)(1u + G * (F / SF37_QK) + F / 32u + K / DN_TILE);
}

extern "C" uint64_t sf37k_decode_lds(const sf37_dec_params *pp) {
    const dec_shape d = dec_plan(*pp);
    return d.lds_up > d.lds_dn ? d.lds_up : d.lds_dn;
}

extern "C" int sf37k_decode_route(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_route_kernel, dim3(d.n_router + d.n_xq), dim3(256), 0, (hipStream_t)s, *pp, d.n_router);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_up(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_up_kernel, dim3(d.n_up_routed + d.n_up_shared), dim3(256), d.lds_up, (hipStream_t)s, *pp,
                       d.n_up_routed);
    return (int)hipGetLastError();
}

extern "C" int sf37k_decode_down(const sf37_dec_params *pp, sf37_stream_t s) {
    const dec_shape d = dec_plan(*pp);
    hipLaunchKernelGGL(dec_down_kernel, dim3(d.n_dn_routed + d.n_dn_shared), dim3(320), d.lds_dn, (hipStream_t)s,
                       *pp, d.n_dn_routed);
    return (int)hipGetLastError();
}
