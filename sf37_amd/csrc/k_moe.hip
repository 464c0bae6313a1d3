// k_moe.hip - routed experts (Q8_K path) for gfx950: dispatch, grouped
// gate/up with fused SwiGLU * routing weight, grouped down, slot-order combine.
//
// Work is organised in expert groups: group g holds the pairs
// sorted[off[g] .. off[g+1]) that share expert[g] (pair p = token*topk+slot,
// sf37_cuda.cu:4601-4602).  A workgroup owns (group, row tile) and streams
// each weight block once for all pairs of the group, so a decode batch in
// which several tokens picked the same expert reads that expert once.
//
// Arithmetic per pair equals the one-token reference path
// (sf37_cuda.cu:4407-4503): Q8_K integer dots with zero-point correction,
// the canonical float chain (sf37_blocks.h), ((g*sig(g))*u)*w, and
// out = sum over slots in slot order (sf37_cuda.cu:4850-4864).  No float
// atomics anywhere, so results are deterministic run to run.
#include "sf37_blocks.h"
#include "sf37_launch.h"

namespace {

constexpr uint32_t MOE_TPC = 4;          // pairs per workgroup pass
constexpr uint32_t DISP_WAVES = 16;
constexpr uint32_t DISP_MAX_E = 512;
constexpr uint32_t DISP_UNROLL = 8;     // 64-pair chunks whose expert ids are loaded together

__device__ __forceinline__ uint32_t clamp_expert(int32_t e, uint32_t n) {
    return (e < 0 || (uint32_t)e >= n) ? 0u : (uint32_t)e;   // sf37_cuda.cu:4428-4429
}

// ---------------------------------------------------------------------------
// Dispatch: stable counting sort of pairs by expert in one workgroup.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024) dispatch_kernel(uint32_t *__restrict__ group_info,
                                                        uint32_t *__restrict__ sorted,
                                                        uint32_t *__restrict__ counts,
                                                        uint32_t *__restrict__ offsets,
                                                        const int32_t *__restrict__ selected,
                                                        uint32_t n_pairs, uint32_t n_expert) {
    __shared__ uint32_t cnt[DISP_WAVES][DISP_MAX_E];
    __shared__ uint32_t off[DISP_MAX_E];
    __shared__ uint32_t gidx[DISP_MAX_E];
    __shared__ uint32_t wsum[2][DISP_WAVES];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    for (uint32_t i = tid; i < DISP_WAVES * DISP_MAX_E; i += 1024u) (&cnt[0][0])[i] = 0u;
    __syncthreads();
    uint32_t span = (n_pairs + DISP_WAVES - 1) / DISP_WAVES;
    span = (span + 63u) & ~63u;
    const uint32_t beg = wave * span;
    const uint32_t end = beg + span < n_pairs ? beg + span : n_pairs;
    // DISP_UNROLL loads in flight per lane before their counts are added
    for (uint32_t p0 = beg + lane; p0 < end; p0 += 64u * DISP_UNROLL) {
        uint32_t ev[DISP_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < DISP_UNROLL; u++) {
            const uint32_t p = p0 + 64u * u;
            ev[u] = p < end ? clamp_expert(selected[p], n_expert) : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < DISP_UNROLL; u++)
            if (p0 + 64u * u < end) atomicAdd(&cnt[wave][ev[u]], 1u);
    }
    __syncthreads();
    // per expert: totals and exclusive offsets of each wave's share
    uint32_t tot = 0u, nz = 0u;
    if (tid < n_expert) {
        for (uint32_t w = 0; w < DISP_WAVES; w++) {
            const uint32_t c = cnt[w][tid];
            cnt[w][tid] = tot;
            tot += c;
        }
        nz = tot ? 1u : 0u;
    }
    // block-wide exclusive scans of tot and nz (tid < 1024 covers E <= 512)
    uint32_t st = tot, sn = nz;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t a = __shfl_up(st, o, 64), b = __shfl_up(sn, o, 64);
        if (lane >= (uint32_t)o) {
            st += a;
            sn += b;
        }
    }
    if (lane == 63u) {
        wsum[0][wave] = st;
        wsum[1][wave] = sn;
    }
    __syncthreads();
    uint32_t bt = 0u, bn = 0u, all_n = 0u;
    for (uint32_t w = 0; w < DISP_WAVES; w++) {
        if (w < wave) {
            bt += wsum[0][w];
            bn += wsum[1][w];
        }
        all_n += wsum[1][w];
    }
    if (tid < n_expert) {
        const uint32_t ex = bt + st - tot, gx = bn + sn - nz;
        off[tid] = ex;
        gidx[tid] = gx;
        counts[tid] = tot;
        offsets[tid] = ex;
        if (nz) {
            group_info[1u + gx] = ex;
            group_info[2u + n_expert + gx] = tid;
        }
    }
    if (tid == 0) {
        offsets[n_expert] = n_pairs;
        group_info[0] = all_n;
        group_info[1u + all_n] = n_pairs;
    }
    __syncthreads();
    // ordered scatter: each wave walks its own range in pair order
    uint32_t nbits = 1;
    while ((1u << nbits) < n_expert) nbits++;
    // chunks of 64 pairs in order; the experts of DISP_UNROLL chunks are
    // loaded before the first of them is ranked
    for (uint32_t base0 = beg; base0 < end; base0 += 64u * DISP_UNROLL) {
        uint32_t ev[DISP_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < DISP_UNROLL; u++) {
            const uint32_t p = base0 + 64u * u + lane;
            ev[u] = p < end ? clamp_expert(selected[p], n_expert) : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < DISP_UNROLL; u++) {
            const uint32_t base = base0 + 64u * u;
            if (base >= end) break;                       // wave-uniform
            const uint32_t p = base + lane;
            const bool act = p < end;
            const uint32_t e = ev[u];
            uint64_t peers = __ballot(act);
            for (uint32_t b = 0; b < nbits; b++) {
                const uint64_t m = __ballot(act && ((e >> b) & 1u));
                peers &= ((e >> b) & 1u) ? m : ~m;
            }
            if (act) {
                const uint64_t lt = lane ? (~0ull >> (64u - lane)) : 0ull;
                const uint32_t rank = (uint32_t)__popcll(peers & lt);
                sorted[off[e] + cnt[wave][e] + rank] = p;
                if ((peers & lt) == 0ull) cnt[wave][e] += (uint32_t)__popcll(peers);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Dispatch of large batches over many workgroups, same order as
// dispatch_kernel: chunk c of DC_CHUNK pairs goes to workgroup c.
// dispatch_count_kernel: per-chunk expert histograms hist[c][e].
// dispatch_scatter_kernel: every workgroup sums the histograms (expert
// totals, and the counts of the chunks before its own), scans the totals
// over the experts, and scatters its chunk in pair order: its waves take
// consecutive quarters, each ranks 64 pairs at a time by ballot.  Workgroup
// 0 writes the counts, offsets and group table.
// ---------------------------------------------------------------------------
constexpr uint32_t DC_CHUNK = 1024;   // pairs per workgroup
constexpr uint32_t DC_THREADS = 256;
constexpr uint32_t DC_WAVES = DC_THREADS / 64u;
constexpr uint32_t DC_PER_LANE = DC_CHUNK / DC_THREADS;   // pairs per lane (a wave's quarter: 4 x 64)
constexpr uint32_t DC_MIN_PAIRS = 8192;   // smaller batches: dispatch_kernel (one launch)
constexpr uint32_t DC_HB = 16;            // histogram rows loaded together

__global__ void __launch_bounds__(DC_THREADS) dispatch_count_kernel(uint32_t *__restrict__ hist,
                                                                    const int32_t *__restrict__ selected,
                                                                    uint32_t n_pairs, uint32_t n_expert) {
    __shared__ uint32_t h[DISP_MAX_E];
    for (uint32_t e = threadIdx.x; e < n_expert; e += DC_THREADS) h[e] = 0u;
    __syncthreads();
    const uint32_t c0 = blockIdx.x * DC_CHUNK;
    const uint32_t c1 = c0 + DC_CHUNK < n_pairs ? c0 + DC_CHUNK : n_pairs;
    uint32_t ev[DC_PER_LANE];
#pragma unroll
    for (uint32_t u = 0; u < DC_PER_LANE; u++) {   // every load issued before the first count
        const uint32_t p = c0 + threadIdx.x + u * DC_THREADS;
        ev[u] = p < c1 ? clamp_expert(selected[p], n_expert) : 0u;
    }
#pragma unroll
    for (uint32_t u = 0; u < DC_PER_LANE; u++)
        if (c0 + threadIdx.x + u * DC_THREADS < c1) atomicAdd(&h[ev[u]], 1u);
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < n_expert; e += DC_THREADS) hist[(uint64_t)blockIdx.x * n_expert + e] = h[e];
}

__global__ void __launch_bounds__(DC_THREADS) dispatch_scatter_kernel(uint32_t *__restrict__ group_info,
                                                                      uint32_t *__restrict__ sorted,
                                                                      uint32_t *__restrict__ counts,
                                                                      uint32_t *__restrict__ offsets,
                                                                      const uint32_t *__restrict__ hist,
                                                                      const int32_t *__restrict__ selected,
                                                                      uint32_t n_pairs, uint32_t n_expert) {
    __shared__ uint32_t tot[DISP_MAX_E], bef[DISP_MAX_E];
    __shared__ uint32_t cnt[DC_WAVES][DISP_MAX_E];
    __shared__ uint32_t wsum[2][DC_WAVES];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u, nc = gridDim.x, c = blockIdx.x;
    for (uint32_t e = tid; e < n_expert; e += DC_THREADS) {
        uint32_t t = 0u, b = 0u;
        for (uint32_t w0 = 0; w0 < nc; w0 += DC_HB) {   // DC_HB loads in flight
            uint32_t v[DC_HB];
#pragma unroll
            for (uint32_t k = 0; k < DC_HB; k++) v[k] = w0 + k < nc ? hist[(uint64_t)(w0 + k) * n_expert + e] : 0u;
#pragma unroll
            for (uint32_t k = 0; k < DC_HB; k++) {
                t += v[k];
                b += w0 + k < c ? v[k] : 0u;
            }
        }
        tot[e] = t;
        bef[e] = b;
    }
    for (uint32_t i = tid; i < DC_WAVES * DISP_MAX_E; i += DC_THREADS) (&cnt[0][0])[i] = 0u;
    __syncthreads();
    // exclusive scans over the experts of the totals and of the non-empty
    // flags: thread t owns experts 2t and 2t + 1 (n_expert <= 512)
    const uint32_t e0 = 2u * tid, e1 = e0 + 1u;
    const uint32_t t0 = e0 < n_expert ? tot[e0] : 0u, t1 = e1 < n_expert ? tot[e1] : 0u;
    const uint32_t z0 = t0 ? 1u : 0u, z1 = t1 ? 1u : 0u;
    uint32_t st = t0 + t1, sn = z0 + z1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t a = __shfl_up(st, o, 64), b = __shfl_up(sn, o, 64);
        if (lane >= (uint32_t)o) {
            st += a;
            sn += b;
        }
    }
    if (lane == 63u) {
        wsum[0][wave] = st;
        wsum[1][wave] = sn;
    }
    __syncthreads();
    uint32_t bt = 0u, bn = 0u, all_n = 0u;
    for (uint32_t w = 0; w < DC_WAVES; w++) {
        if (w < wave) {
            bt += wsum[0][w];
            bn += wsum[1][w];
        }
        all_n += wsum[1][w];
    }
    const uint32_t x0 = bt + st - t0 - t1, g0 = bn + sn - z0 - z1;   // exclusive prefix at e0
    const uint32_t xs[2] = {x0, x0 + t0}, gs[2] = {g0, g0 + z0}, ts[2] = {t0, t1};
    // the chunk's quarters: per-wave counts, then running offsets per expert
    const uint32_t c0 = c * DC_CHUNK, c1 = c0 + DC_CHUNK < n_pairs ? c0 + DC_CHUNK : n_pairs;
    const uint32_t span = DC_CHUNK / DC_WAVES;
    const uint32_t beg = c0 + wave * span < c1 ? c0 + wave * span : c1;
    const uint32_t end = beg + span < c1 ? beg + span : c1;
    uint32_t ev[DC_PER_LANE];
#pragma unroll
    for (uint32_t u = 0; u < DC_PER_LANE; u++) {
        const uint32_t p = beg + 64u * u + lane;
        ev[u] = p < end ? clamp_expert(selected[p], n_expert) : 0u;
    }
#pragma unroll
    for (uint32_t u = 0; u < DC_PER_LANE; u++)
        if (beg + 64u * u + lane < end) atomicAdd(&cnt[wave][ev[u]], 1u);
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < 2u; k++) {
        const uint32_t e = e0 + k;
        if (e >= n_expert) continue;
        uint32_t run = xs[k] + bef[e];
        for (uint32_t w = 0; w < DC_WAVES; w++) {
            const uint32_t v = cnt[w][e];
            cnt[w][e] = run;
            run += v;
        }
        if (c == 0) {
            counts[e] = ts[k];
            offsets[e] = xs[k];
            if (ts[k]) {
                group_info[1u + gs[k]] = xs[k];
                group_info[2u + n_expert + gs[k]] = e;
            }
        }
    }
    if (c == 0 && tid == 0) {
        offsets[n_expert] = n_pairs;
        group_info[0] = all_n;
        group_info[1u + all_n] = n_pairs;
    }
    __syncthreads();
    uint32_t nbits = 1;
    while ((1u << nbits) < n_expert) nbits++;
#pragma unroll
    for (uint32_t u = 0; u < DC_PER_LANE; u++) {
        const uint32_t p = beg + 64u * u + lane;
        const bool act = p < end;
        const uint32_t e = ev[u];
        uint64_t peers = __ballot(act);
        for (uint32_t b = 0; b < nbits; b++) {
            const uint64_t m = __ballot(act && ((e >> b) & 1u));
            peers &= ((e >> b) & 1u) ? m : ~m;
        }
        if (act) {
            const uint64_t lt = lane ? (~0ull >> (64u - lane)) : 0ull;
            const uint32_t rank = (uint32_t)__popcll(peers & lt);
            sorted[cnt[wave][e] + rank] = p;
            if ((peers & lt) == 0ull) cnt[wave][e] += (uint32_t)__popcll(peers);
        }
    }
}

// One group per slot of a single token (routed_moe_one): no sort needed.
__global__ void slots_kernel(uint32_t *__restrict__ group_info, uint32_t *__restrict__ sorted,
                             const int32_t *__restrict__ selected, uint32_t topk, uint32_t n_expert) {
    for (uint32_t s = threadIdx.x; s < topk; s += blockDim.x) {
        sorted[s] = s;
        group_info[1u + s] = s;
        group_info[2u + topk + s] = clamp_expert(selected[s], n_expert);
    }
    if (threadIdx.x == 0) {
        group_info[0] = topk;
        group_info[1u + topk] = topk;
    }
}

// ---------------------------------------------------------------------------
// Gate/up: rows [row0, row0+R) of gate and of up for one expert group.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) gate_up_kernel(float *__restrict__ mid,
                                                      float *__restrict__ gate_out,
                                                      float *__restrict__ up_out,
                                                      const uint8_t *__restrict__ gate_w,
                                                      const uint8_t *__restrict__ up_w,
                                                      const q8k_block *__restrict__ xq,
                                                      const uint32_t *__restrict__ ginfo,
                                                      const uint32_t *__restrict__ sorted,
                                                      const float *__restrict__ weights,
                                                      uint32_t max_groups, uint32_t topk,
                                                      uint32_t nblk, uint32_t mid_dim,
                                                      uint32_t R, float clamp) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t g = blockIdx.y;
    if (g >= ginfo[0]) return;
    const uint32_t p0 = ginfo[1 + g], p1 = ginfo[2 + g];
    const uint32_t e = ginfo[2 + max_groups + g];
    act_block *xs = (act_block *)smem;                                  // [TPC][nblk]
    float *red = (float *)(xs + MOE_TPC * nblk);                        // [TPC][2R][nblk]
    float *res = red + MOE_TPC * 2u * R * nblk;                         // [TPC][2][R]
    const uint32_t row0 = blockIdx.x * R;
    const uint64_t row_bytes = (uint64_t)nblk * SF37_Q3_BYTES;
    const uint64_t expert_bytes = (uint64_t)mid_dim * row_bytes;
    const uint32_t units = 2u * R * nblk;
    for (uint32_t c0 = p0; c0 < p1; c0 += MOE_TPC) {
        const uint32_t nt = p1 - c0 < MOE_TPC ? p1 - c0 : MOE_TPC;
        for (uint32_t t = 0; t < nt; t++)
            stage_act<true>(xs + t * nblk, xq + (uint64_t)(sorted[c0 + t] / topk) * nblk, nblk);
        __syncthreads();
        for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
            const uint32_t m = u / (R * nblk);
            const uint32_t rb = u - m * R * nblk;
            const uint32_t r = rb / nblk, b = rb - r * nblk;
            float bs[MOE_TPC] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row0 + r < mid_dim) {
                const uint8_t *blk = (m ? up_w : gate_w) + (uint64_t)e * expert_bytes +
                                     (uint64_t)(row0 + r) * row_bytes + (uint64_t)b * SF37_Q3_BYTES;
                uint32_t raw[28], a[27];
                q3_realign(a, raw, q3_load(raw, blk));
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
                    for (uint32_t t = 0; t < MOE_TPC; t++) {
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
            }
            for (uint32_t t = 0; t < nt; t++) red[(t * 2u * R + m * R + r) * nblk + b] = bs[t];
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * 2u * R; i += blockDim.x) {
            const uint32_t t = i / (2u * R), mr = i - t * 2u * R;
            const float *rv = red + (t * 2u * R + mr) * nblk;
            float acc = 0.0f;
            for (uint32_t b = 0; b < nblk; b++) acc = __builtin_fmaf(xs[t * nblk + b].d, rv[b], acc);
            res[t * 2u * R + mr] = acc;
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * R; i += blockDim.x) {
            const uint32_t t = i / R, r = i - t * R;
            if (row0 + r >= mid_dim) continue;
            const uint32_t p = sorted[c0 + t];
            const float gv = res[t * 2u * R + r], uv = res[t * 2u * R + R + r];
            const uint64_t o = (uint64_t)p * mid_dim + row0 + r;
            if (gate_out) {
                gate_out[o] = gv;
                up_out[o] = uv;
            }
            mid[o] = sf37_swiglu_mid(gv, uv, weights[p], clamp);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Down: rows [row0, row0+R) of the Q2 down matrix for one expert group;
// writes one fp32 output row per pair.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) down_kernel(float *__restrict__ down_pair,
                                                   const uint8_t *__restrict__ down_w,
                                                   const q8k_block *__restrict__ midq,
                                                   const uint32_t *__restrict__ ginfo,
                                                   const uint32_t *__restrict__ sorted,
                                                   uint32_t max_groups, uint32_t nblk,
                                                   uint32_t out_dim, uint32_t R) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t g = blockIdx.y;
    if (g >= ginfo[0]) return;
    const uint32_t p0 = ginfo[1 + g], p1 = ginfo[2 + g];
    const uint32_t e = ginfo[2 + max_groups + g];
    act_block *xs = (act_block *)smem;                                  // [TPC][nblk]
    float *red = (float *)(xs + MOE_TPC * nblk);                        // [TPC][R][nblk]
    const uint32_t row0 = blockIdx.x * R;
    const uint64_t row_bytes = (uint64_t)nblk * SF37_Q2_BYTES;
    const uint64_t expert_bytes = (uint64_t)out_dim * row_bytes;
    const uint32_t units = R * nblk;
    for (uint32_t c0 = p0; c0 < p1; c0 += MOE_TPC) {
        const uint32_t nt = p1 - c0 < MOE_TPC ? p1 - c0 : MOE_TPC;
        for (uint32_t t = 0; t < nt; t++)
            stage_act<false>(xs + t * nblk, midq + (uint64_t)sorted[c0 + t] * nblk, nblk);
        __syncthreads();
        for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
            const uint32_t r = u / nblk, b = u - r * nblk;
            float bs[MOE_TPC] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row0 + r < out_dim) {
                uint32_t a[21];
                ld_dwords(a, down_w + (uint64_t)e * expert_bytes + (uint64_t)(row0 + r) * row_bytes +
                                 (uint64_t)b * SF37_Q2_BYTES, 21);
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    uint32_t cw[16];
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        q2_unpack16(a[3 + 4 * gg + j], cw[4 * j], cw[4 * j + 1], cw[4 * j + 2], cw[4 * j + 3]);
                    const int32_t zp = (int32_t)((a[2] >> (8 * gg)) & 3u);
                    const float sc = sf37_f16(a[gg >> 1] >> (16 * (gg & 1)));
#pragma unroll
                    for (uint32_t t = 0; t < MOE_TPC; t++) {
                        if (t < nt) {
                            const act_block &x = xs[t * nblk + b];
                            int32_t acc = 0;
#pragma unroll
                            for (int k = 0; k < 16; k++) acc = sdot4(cw[k], x.qs[16 * gg + k], acc);
                            bs[t] = __builtin_fmaf(sc, (float)(acc - zp * x.gs[gg]), bs[t]);
                        }
                    }
                }
            }
            for (uint32_t t = 0; t < nt; t++) red[(t * R + r) * nblk + b] = bs[t];
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < nt * R; i += blockDim.x) {
            const uint32_t t = i / R, r = i - t * R;
            if (row0 + r >= out_dim) continue;
            const float *rv = red + (t * R + r) * nblk;
            float acc = 0.0f;
            for (uint32_t b = 0; b < nblk; b++) acc = __builtin_fmaf(xs[t * nblk + b].d, rv[b], acc);
            down_pair[(uint64_t)sorted[c0 + t] * out_dim + row0 + r] = acc;
        }
        __syncthreads();
    }
}

// out = [base +] sum over slots in slot order; with resid (MODE 2):
// resid = resid + (base + sum).  MODE 0: plain sum, 1: base +, 2: resid.
template <int MODE>
__device__ __forceinline__ void combine_store(float *out, const float *base, float *resid, uint64_t i, float v) {
    if constexpr (MODE == 0) out[i] = v;
    else if constexpr (MODE == 1) out[i] = base[i] + v;
    else resid[i] = resid[i] + (base[i] + v);
}

template <int MODE>
__global__ void __launch_bounds__(256) combine_kernel(float *out, const float *__restrict__ down_pair,
                                                      const float *base, float *resid, uint32_t topk,
                                                      uint32_t out_dim, uint32_t n_tok) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= (uint64_t)out_dim * n_tok) return;
    const uint64_t t = i / out_dim, r = i - t * out_dim;
    float acc = 0.0f;
    for (uint32_t s = 0; s < topk; s++) acc = acc + down_pair[(t * topk + s) * out_dim + r];
    combine_store<MODE>(out, base, resid, i, acc);
}

// The same, four outputs per thread (out_dim % 4 == 0, 1 <= topk <= 16, the
// row pointers 16-byte aligned): every slot's float4 is loaded before the
// first add; TK = 8 loads exactly the eight slots (0: topk at run time, 16
// loads of which those past topk repeat slot 0).  base and resid move as
// float4; each component gets the scalar kernel's operations.
template <int MODE, int TK>
__global__ void __launch_bounds__(256) combine4_kernel(float *out, const float *__restrict__ down_pair,
                                                       const float *base, float *resid, uint32_t topk,
                                                       uint32_t out_dim, uint32_t n_tok) {
    constexpr uint32_t NS = TK ? (uint32_t)TK : 16u;
    const uint32_t tk = TK ? (uint32_t)TK : topk;
    const uint64_t i = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * 4u;
    if (i >= (uint64_t)out_dim * n_tok) return;
    const uint64_t t = i / out_dim, r = i - t * out_dim;
    float4 v[NS];
#pragma unroll
    for (uint32_t s = 0; s < NS; s++) {
        const uint32_t sc = s < tk ? s : 0u;   // every load in bounds
        v[s] = *(const float4 *)(down_pair + (t * tk + sc) * out_dim + r);
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t s = 0; s < NS; s++) {
        if (s < tk) {
            acc.x = acc.x + v[s].x;
            acc.y = acc.y + v[s].y;
            acc.z = acc.z + v[s].z;
            acc.w = acc.w + v[s].w;
        }
    }
    if constexpr (MODE == 0) {
        *(float4 *)(out + i) = acc;
    } else if constexpr (MODE == 1) {
        const float4 bv = *(const float4 *)(base + i);
        *(float4 *)(out + i) = make_float4(bv.x + acc.x, bv.y + acc.y, bv.z + acc.z, bv.w + acc.w);
    } else {
        const float4 bv = *(const float4 *)(base + i), rv = *(const float4 *)(resid + i);
        *(float4 *)(resid + i) = make_float4(rv.x + (bv.x + acc.x), rv.y + (bv.y + acc.y), rv.z + (bv.z + acc.z),
                                             rv.w + (bv.w + acc.w));
    }
}

// ---------------------------------------------------------------------------
// fp32-activation path (sf37_cuda.cu:5089-5267): one workgroup per
// (row, slot); lanes stride over the elements, tree reduction in LDS.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float q3_weight(const uint8_t *blk, uint32_t j) {
    const uint32_t g = j >> 6, gi = j & 63u;
    const float s = sf37_f16((uint32_t)blk[2 * g] | ((uint32_t)blk[2 * g + 1] << 8));
    const uint8_t *pl = blk + 12 + 24 * g;
    const uint32_t bit = 3u * gi;
    uint32_t v = pl[bit >> 3];
    if ((bit & 7u) > 5u) v |= (uint32_t)pl[(bit >> 3) + 1] << 8;
    return ((float)((v >> (bit & 7u)) & 7u) - (float)(blk[8 + g] & 7u)) * s;
}

__device__ __forceinline__ float q2_weight(const uint8_t *blk, uint32_t j) {
    const uint32_t g = j >> 6, gi = j & 63u;
    const float s = sf37_f16((uint32_t)blk[2 * g] | ((uint32_t)blk[2 * g + 1] << 8));
    const uint32_t q = (blk[12 + 16 * g + (gi >> 2)] >> ((gi & 3u) * 2u)) & 3u;
    return ((float)q - (float)(blk[8 + g] & 3u)) * s;
}

__device__ __forceinline__ float block_sum256(float v, float *part) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = (part[0] + part[1]) + (part[2] + part[3]);
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(256) gate_up_f32_kernel(float *__restrict__ mid,
                                                          float *__restrict__ gate_out,
                                                          float *__restrict__ up_out,
                                                          const uint8_t *__restrict__ gate_w,
                                                          const uint8_t *__restrict__ up_w,
                                                          const float *__restrict__ x,
                                                          const int32_t *__restrict__ selected,
                                                          const float *__restrict__ weights,
                                                          uint32_t in_dim, uint32_t mid_dim,
                                                          uint32_t n_expert, float clamp) {
    __shared__ float part[4];
    const uint32_t row = blockIdx.x, slot = blockIdx.y;
    const uint32_t e = clamp_expert(selected[slot], n_expert);
    const uint64_t row_bytes = (uint64_t)(in_dim / SF37_QK) * SF37_Q3_BYTES;
    const uint8_t *gr = gate_w + ((uint64_t)e * mid_dim + row) * row_bytes;
    const uint8_t *ur = up_w + ((uint64_t)e * mid_dim + row) * row_bytes;
    float ga = 0.0f, ua = 0.0f;
    for (uint32_t i = threadIdx.x; i < in_dim; i += 256u) {
        const uint32_t b = i / SF37_QK, j = i - b * SF37_QK;
        ga += q3_weight(gr + (uint64_t)b * SF37_Q3_BYTES, j) * x[i];
        ua += q3_weight(ur + (uint64_t)b * SF37_Q3_BYTES, j) * x[i];
    }
    const float gv = block_sum256(ga, part);
    const float uv = block_sum256(ua, part);
    if (threadIdx.x == 0) {
        const uint64_t o = (uint64_t)slot * mid_dim + row;
        if (gate_out) {
            gate_out[o] = gv;
            up_out[o] = uv;
        }
        mid[o] = sf37_swiglu_mid(gv, uv, weights[slot], clamp);
    }
}

__global__ void __launch_bounds__(256) down_f32_kernel(float *__restrict__ down_slot,
                                                       const uint8_t *__restrict__ down_w,
                                                       const float *__restrict__ mid,
                                                       const int32_t *__restrict__ selected,
                                                       uint32_t mid_dim, uint32_t out_dim,
                                                       uint32_t n_expert) {
    __shared__ float part[4];
    const uint32_t row = blockIdx.x, slot = blockIdx.y;
    const uint32_t e = clamp_expert(selected[slot], n_expert);
    const uint64_t row_bytes = (uint64_t)(mid_dim / SF37_QK) * SF37_Q2_BYTES;
    const uint8_t *wr = down_w + ((uint64_t)e * out_dim + row) * row_bytes;
    const float *xr = mid + (uint64_t)slot * mid_dim;
    float acc = 0.0f;
    for (uint32_t i = threadIdx.x; i < mid_dim; i += 256u) {
        const uint32_t b = i / SF37_QK, j = i - b * SF37_QK;
        acc += q2_weight(wr + (uint64_t)b * SF37_Q2_BYTES, j) * xr[i];
    }
    const float v = block_sum256(acc, part);
    if (threadIdx.x == 0) down_slot[(uint64_t)slot * out_dim + row] = v;
}

}  // namespace

extern "C" uint64_t sf37k_moe_dispatch_scratch_bytes(uint32_t n_pairs, uint32_t n_expert) {
    return n_pairs > DC_MIN_PAIRS ? (uint64_t)((n_pairs + DC_CHUNK - 1u) / DC_CHUNK) * n_expert * 4u : 0u;
}

extern "C" int sf37k_moe_dispatch(uint32_t *group_info, uint32_t *sorted_pairs, uint32_t *counts,
                                  uint32_t *offsets, const int32_t *selected, uint32_t n_pairs,
                                  uint32_t n_expert, uint32_t *hist, sf37_stream_t s) {
    if (n_expert == 0 || n_expert > DISP_MAX_E) return (int)hipErrorInvalidValue;
    if (n_pairs <= DC_MIN_PAIRS) {
        hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, (hipStream_t)s, group_info,
                           sorted_pairs, counts, offsets, selected, n_pairs, n_expert);
        return (int)hipGetLastError();
    }
    if (!hist) return (int)hipErrorInvalidValue;
    const uint32_t nc = (n_pairs + DC_CHUNK - 1u) / DC_CHUNK;
    hipLaunchKernelGGL(dispatch_count_kernel, dim3(nc), dim3(DC_THREADS), 0, (hipStream_t)s, hist, selected, n_pairs,
                       n_expert);
    hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nc), dim3(DC_THREADS), 0, (hipStream_t)s, group_info,
                       sorted_pairs, counts, offsets, hist, selected, n_pairs, n_expert);
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_slots(uint32_t *group_info, uint32_t *sorted_pairs, const int32_t *selected,
                               uint32_t topk, uint32_t n_expert, sf37_stream_t s) {
    hipLaunchKernelGGL(slots_kernel, dim3(1), dim3(64), 0, (hipStream_t)s, group_info, sorted_pairs,
                       selected, topk, n_expert);
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_gate_up(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                                 const uint8_t *up_w, const void *xq, const uint32_t *group_info,
                                 const uint32_t *sorted_pairs, const float *weights,
                                 uint32_t max_groups, uint32_t max_group_pairs, uint32_t topk,
                                 uint32_t in_dim, uint32_t mid_dim, float clamp, sf37_stream_t s) {
    (void)max_group_pairs;
    const uint32_t nblk = in_dim / SF37_QK;
    uint32_t R = 128u / nblk;
    if (R < 1u) R = 1u;
    const size_t lds = (size_t)MOE_TPC * nblk * sizeof(act_block) +
                       (size_t)MOE_TPC * 2u * R * nblk * sizeof(float) +
                       (size_t)MOE_TPC * 2u * R * sizeof(float);
    if (lds > 64u * 1024u) return (int)hipErrorInvalidValue;
    const dim3 grid((mid_dim + R - 1) / R, max_groups);
    hipLaunchKernelGGL(gate_up_kernel, grid, dim3(256), lds, (hipStream_t)s, mid, gate_out, up_out,
                       gate_w, up_w, (const q8k_block *)xq, group_info, sorted_pairs, weights,
                       max_groups, topk, nblk, mid_dim, R, clamp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_down(float *down_pair, const uint8_t *down_w, const void *midq,
                              const uint32_t *group_info, const uint32_t *sorted_pairs,
                              uint32_t max_groups, uint32_t max_group_pairs, uint32_t mid_dim,
                              uint32_t out_dim, sf37_stream_t s) {
    (void)max_group_pairs;
    const uint32_t nblk = mid_dim / SF37_QK;
    uint32_t R = 256u / nblk;
    if (R < 1u) R = 1u;
    const size_t lds = (size_t)MOE_TPC * nblk * sizeof(act_block) +
                       (size_t)MOE_TPC * R * nblk * sizeof(float);
    if (lds > 64u * 1024u) return (int)hipErrorInvalidValue;
    const dim3 grid((out_dim + R - 1) / R, max_groups);
    hipLaunchKernelGGL(down_kernel, grid, dim3(256), lds, (hipStream_t)s, down_pair, down_w,
                       (const q8k_block *)midq, group_info, sorted_pairs, max_groups, nblk, out_dim, R);
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_combine(float *out, const float *down_pair, const float *base, float *resid,
                                 uint32_t topk, uint32_t out_dim, uint32_t n_tok, sf37_stream_t s) {
    const uint64_t n = (uint64_t)out_dim * n_tok;
    if (n == 0) return 0;
    const int mode = resid ? 2 : (base ? 1 : 0);
    if ((resid || base) && !base) return (int)hipErrorInvalidValue;
    const bool vec = out_dim % 4u == 0 && topk >= 1u && topk <= 16u &&
                     (((uintptr_t)down_pair | (uintptr_t)out | (uintptr_t)base | (uintptr_t)resid) & 15u) == 0;
    const dim3 grid((unsigned)(((vec ? n / 4u : n) + 255) / 256));
    if (vec) {
#define SF37_COMBINE4(M)                                                                                    \
    do {                                                                                                      \
        if (topk == 8u)                                                                                       \
            hipLaunchKernelGGL((combine4_kernel<M, 8>), grid, dim3(256), 0, (hipStream_t)s, out, down_pair, base, \
                               resid, topk, out_dim, n_tok);                                                  \
        else                                                                                                  \
            hipLaunchKernelGGL((combine4_kernel<M, 0>), grid, dim3(256), 0, (hipStream_t)s, out, down_pair, base, \
                               resid, topk, out_dim, n_tok);                                                  \
    } while (0)
        if (mode == 0) SF37_COMBINE4(0);
        else if (mode == 1) SF37_COMBINE4(1);
        else SF37_COMBINE4(2);
#undef SF37_COMBINE4
    } else {
        if (mode == 0) hipLaunchKernelGGL(combine_kernel<0>, grid, dim3(256), 0, (hipStream_t)s, out, down_pair, base, resid, topk, out_dim, n_tok);
        else if (mode == 1) hipLaunchKernelGGL(combine_kernel<1>, grid, dim3(256), 0, (hipStream_t)s, out, down_pair, base, resid, topk, out_dim, n_tok);
        else hipLaunchKernelGGL(combine_kernel<2>, grid, dim3(256), 0, (hipStream_t)s, out, down_pair, base, resid, topk, out_dim, n_tok);
    }
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_gate_up_f32(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                                     const uint8_t *up_w, const float *x, const int32_t *selected,
                                     const float *weights, uint32_t topk, uint32_t in_dim,
                                     uint32_t mid_dim, uint32_t n_expert, float clamp, sf37_stream_t s) {
    hipLaunchKernelGGL(gate_up_f32_kernel, dim3(mid_dim, topk), dim3(256), 0, (hipStream_t)s, mid,
                       gate_out, up_out, gate_w, up_w, x, selected, weights, in_dim, mid_dim, n_expert,
                       clamp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_moe_down_f32(float *down_slot, const uint8_t *down_w, const float *mid,
                                  const int32_t *selected, uint32_t topk, uint32_t mid_dim,
                                  uint32_t out_dim, uint32_t n_expert, sf37_stream_t s) {
    hipLaunchKernelGGL(down_f32_kernel, dim3(out_dim, topk), dim3(256), 0, (hipStream_t)s, down_slot,
                       down_w, mid, selected, mid_dim, out_dim, n_expert);
    return (int)hipGetLastError();
}
