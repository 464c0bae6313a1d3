// k_q8k.hip - Q8_K activations and single-matrix Q3/Q2 GEMVs for gfx950.
//
// Q8_K (sf37_cuda.cu:4162-4205): one wave per 256-block, 4 values per lane,
// wave-wide amax, IEEE division, round-half-even codes and 64-wide sums.
//
// Q3/Q2 x Q8_K GEMV (sf37_cuda.cu:4369-4405 computes the same dots): one
// lane per 256-weight block.  The lane loads its block with dword loads,
// expands the 3- or 2-bit codes into int8x4 words (sf37_dev.h) and runs
// v_dot4_i32_i8 against activations that were staged in LDS in the matching
// permuted order.  The float epilogue is the canonical order
//   blk = fma(s3,I3, fma(s2,I2, fma(s1,I1, fma(s0,I0,0))));  acc = fma(d_b, blk, acc)
// with the block chain done by one lane per row after an LDS exchange.
#include "sf37_blocks.h"
#include "sf37_launch.h"

namespace {

__global__ void __launch_bounds__(256) q8k_quantize_kernel(q8k_block *__restrict__ out,
                                                           const float *__restrict__ x,
                                                           uint32_t nblk, uint32_t n_rows) {
    const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    if (wave >= nblk * n_rows) return;
    const float *xb = x + (uint64_t)wave * SF37_QK + 4u * lane;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = xb[k];
    int8_t q[4];
    int gsum;
    const float d = q8k_codes4(v, q, gsum);
    q8k_block *y = out + wave;
    const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                            ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
    ((uint32_t *)y->qs)[lane] = packed;
    if (lane == 0) y->d = d;
    if ((lane & 15u) == 0) y->gsums[lane >> 4] = (int16_t)gsum;
}

}  // namespace

namespace {

// Generic Q3/Q2 x Q8_K GEMV: rows_per_wg rows, one lane per (row, block).
template <bool Q3>
__global__ void __launch_bounds__(256) qlow_q8k_matvec_kernel(float *__restrict__ out,
                                                              const uint8_t *__restrict__ w,
                                                              const q8k_block *__restrict__ xq,
                                                              uint32_t nblk, uint64_t out_dim,
                                                              uint32_t rows_per_wg) {
    extern __shared__ __align__(16) unsigned char smem[];
    act_block *xs = (act_block *)smem;
    float *red = (float *)(xs + nblk);
    stage_act<Q3>(xs, xq, nblk);
    __syncthreads();
    const uint64_t row0 = (uint64_t)blockIdx.x * rows_per_wg;
    const uint32_t bytes = Q3 ? SF37_Q3_BYTES : SF37_Q2_BYTES;
    const uint64_t row_bytes = (uint64_t)nblk * bytes;
    for (uint32_t u = threadIdx.x; u < rows_per_wg * nblk; u += blockDim.x) {
        const uint32_t r = u / nblk, b = u - r * nblk;
        float v = 0.0f;
        if (row0 + r < out_dim) {
            const uint8_t *blk = w + (row0 + r) * row_bytes + (uint64_t)b * bytes;
            int32_t I[4];
            if (Q3) {
                uint32_t raw[28], a[27];
                const uint32_t o = q3_load(raw, blk);
                q3_realign(a, raw, o);
                q3_block_idots(a, xs[b], I);
                v = q3_block_value(a, I);
            } else {
                uint32_t a[21];
                ld_dwords(a, blk, 21);
                q2_block_idots(a, xs[b], I);
                v = q2_block_value(a, I);
            }
        }
        red[u] = v;
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < rows_per_wg; r += blockDim.x) {
        if (row0 + r >= out_dim) break;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nblk; b++) acc = __builtin_fmaf(xs[b].d, red[r * nblk + b], acc);
        out[row0 + r] = acc;
    }
}

// fp32-activation GEMV (sf37_cuda.cu:5035-5087 computes the same sums): one
// wave per row, lanes stride over the elements, wave-wide float reduction.
template <bool Q3>
__global__ void __launch_bounds__(256) qlow_f32_matvec_kernel(float *__restrict__ out,
                                                              const uint8_t *__restrict__ w,
                                                              const float *__restrict__ x,
                                                              uint64_t in_dim, uint64_t out_dim) {
    const uint64_t row = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    if (row >= out_dim) return;
    const uint32_t bytes = Q3 ? SF37_Q3_BYTES : SF37_Q2_BYTES;
    const uint8_t *wr = w + row * (in_dim / SF37_QK) * bytes;
    float acc = 0.0f;
    for (uint64_t i = lane; i < in_dim; i += 64u) {
        const uint64_t b = i / SF37_QK;
        const uint32_t j = (uint32_t)(i - b * SF37_QK), g = j >> 6, gi = j & 63u;
        const uint8_t *blk = wr + b * bytes;
        const float s = sf37_f16((uint32_t)blk[2 * g] | ((uint32_t)blk[2 * g + 1] << 8));
        uint32_t q;
        float zp;
        if (Q3) {
            const uint8_t *pl = blk + 12 + 24 * g;
            const uint32_t bit = 3u * gi;
            uint32_t v = pl[bit >> 3];
            if ((bit & 7u) > 5u) v |= (uint32_t)pl[(bit >> 3) + 1] << 8;
            q = (v >> (bit & 7u)) & 7u;
            zp = (float)(blk[8 + g] & 7u);
        } else {
            q = (blk[12 + 16 * g + (gi >> 2)] >> ((gi & 3u) * 2u)) & 3u;
            zp = (float)(blk[8 + g] & 3u);
        }
        acc += ((float)q - zp) * s * x[i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) out[row] = acc;
}

}  // namespace

extern "C" int sf37k_q8k_quantize(void *out, const float *x, uint32_t in_dim, uint32_t n_rows,
                                  sf37_stream_t s) {
    const uint32_t nblk = in_dim / SF37_QK;
    const uint64_t waves = (uint64_t)nblk * n_rows;
    if (waves == 0) return 0;
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       (hipStream_t)s, (q8k_block *)out, x, nblk, n_rows);
    return (int)hipGetLastError();
}

static int qlow_matvec(bool q3, float *out, const uint8_t *w, const void *xq, uint32_t nblk,
                       uint64_t out_dim, sf37_stream_t s) {
    if (out_dim == 0) return 0;
    uint32_t rows = nblk >= 256u ? 1u : 256u / nblk;
    if (rows > 64u) rows = 64u;
    const size_t lds = (size_t)nblk * sizeof(act_block) + (size_t)rows * nblk * sizeof(float);
    const unsigned grid = (unsigned)((out_dim + rows - 1) / rows);
    if (q3)
        hipLaunchKernelGGL(qlow_q8k_matvec_kernel<true>, dim3(grid), dim3(256), lds, (hipStream_t)s,
                           out, w, (const q8k_block *)xq, nblk, out_dim, rows);
    else
        hipLaunchKernelGGL(qlow_q8k_matvec_kernel<false>, dim3(grid), dim3(256), lds, (hipStream_t)s,
                           out, w, (const q8k_block *)xq, nblk, out_dim, rows);
    return (int)hipGetLastError();
}

extern "C" int sf37k_q3_q8k_matvec(float *out, const uint8_t *w, const void *xq, uint32_t nblk,
                                   uint64_t out_dim, sf37_stream_t s) {
    return qlow_matvec(true, out, w, xq, nblk, out_dim, s);
}

extern "C" int sf37k_q2_q8k_matvec(float *out, const uint8_t *w, const void *xq, uint32_t nblk,
                                   uint64_t out_dim, sf37_stream_t s) {
    return qlow_matvec(false, out, w, xq, nblk, out_dim, s);
}

extern "C" int sf37k_q3_f32_matvec(float *out, const uint8_t *w, const float *x, uint64_t in_dim,
                                   uint64_t out_dim, sf37_stream_t s) {
    if (out_dim == 0) return 0;
    hipLaunchKernelGGL(qlow_f32_matvec_kernel<true>, dim3((unsigned)((out_dim + 3) / 4)), dim3(256),
                       0, (hipStream_t)s, out, w, x, in_dim, out_dim);
    return (int)hipGetLastError();
}

extern "C" int sf37k_q2_f32_matvec(float *out, const uint8_t *w, const float *x, uint64_t in_dim,
                                   uint64_t out_dim, sf37_stream_t s) {
    if (out_dim == 0) return 0;
    hipLaunchKernelGGL(qlow_f32_matvec_kernel<false>, dim3((unsigned)((out_dim + 3) / 4)), dim3(256),
                       0, (hipStream_t)s, out, w, x, in_dim, out_dim);
    return (int)hipGetLastError();
}
