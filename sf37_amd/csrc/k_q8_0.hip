// k_q8_0.hip - shared-expert Q8_0 path for gfx950.
//
// Activations (sf37_ops.c:57-90): per 32 values d = amax/127, codes
// round-half-even of x * (1/d) clamped to int8, zero block -> d = 0.
//
// Rows (sf37_ops.c:92-108): acc = sum_b ((float)isum_b * wscale_b) * xscale_b
// in block order.  One lane per (row, block): the lane loads its 34-byte
// block with dword loads, realigns it, forms isum with eight v_dot4_i32_i8
// per token and its term; one lane per (row, token) then adds the terms in
// block order, so every result equals the CPU function bit for bit.
#include "sf37_dev.h"
#include "sf37_launch.h"

namespace {

constexpr uint32_t Q8_TPC_MAX = 8;   // tokens per workgroup pass (at most)

__global__ void __launch_bounds__(256) q8_0_quantize_kernel(int8_t *__restrict__ xq,
                                                            float *__restrict__ xscale,
                                                            const float *__restrict__ x,
                                                            uint64_t in_dim, uint64_t nb,
                                                            uint64_t n_tok) {
    // one 32-lane half-wave per block
    const uint64_t hw = (uint64_t)blockIdx.x * 8u + (threadIdx.x >> 5);
    const uint32_t l = threadIdx.x & 31u;
    if (hw >= nb * n_tok) return;
    const uint64_t t = hw / nb, b = hw - t * nb;
    const uint64_t i = b * 32u + l;
    const float v = i < in_dim ? x[t * in_dim + i] : 0.0f;
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    int8_t q = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        d = amax / 127.0f;
        const float iscale = 1.0f / d;
        q = (int8_t)(int)fminf(fmaxf(__builtin_rintf(iscale * v), -128.0f), 127.0f);
        if (i >= in_dim) q = 0;
    }
    xq[(t * nb + b) * 32u + l] = q;
    if (l == 0) xscale[t * nb + b] = d;
}

// out[t][row] for rows of one matrix (blockIdx.z picks w0/out0 or w1/out1).
__global__ void __launch_bounds__(256) q8_0_matmul_kernel(float *__restrict__ out0,
                                                          float *__restrict__ out1,
                                                          const uint8_t *__restrict__ w0,
                                                          const uint8_t *__restrict__ w1,
                                                          const int8_t *__restrict__ xq,
                                                          const float *__restrict__ xscale,
                                                          uint32_t nb, uint64_t out_dim,
                                                          uint64_t n_tok, uint32_t rows_per_wg,
                                                          uint32_t tpc) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint32_t *xs = (uint32_t *)smem;                                   // [tpc][nb*8] i8x4
    float *sc = (float *)(xs + tpc * nb * 8u);                         // [tpc][nb]
    float *red = sc + tpc * nb;                                        // [tpc][rows][nb]
    const uint8_t *w = blockIdx.z ? w1 : w0;
    float *out = blockIdx.z ? out1 : out0;
    const uint64_t t0 = (uint64_t)blockIdx.y * tpc;
    const uint32_t nt = (uint32_t)(n_tok - t0 < tpc ? n_tok - t0 : tpc);
    for (uint32_t i = threadIdx.x; i < nt * nb * 8u; i += blockDim.x)
        xs[i] = ((const uint32_t *)(xq + t0 * nb * 32u))[i];
    for (uint32_t i = threadIdx.x; i < nt * nb; i += blockDim.x) sc[i] = xscale[t0 * nb + i];
    __syncthreads();
    const uint64_t row0 = (uint64_t)blockIdx.x * rows_per_wg;
    const uint64_t row_bytes = (uint64_t)nb * SF37_Q8_0_BYTES;
    const uint32_t units = rows_per_wg * nb;
    for (uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
        const uint32_t r = u / nb, b = u - r * nb;
        if (row0 + r >= out_dim) continue;
        const uint8_t *p = w + (row0 + r) * row_bytes + (uint64_t)b * SF37_Q8_0_BYTES;
        const uintptr_t addr = (uintptr_t)p;
        const uint32_t o = (uint32_t)(addr & 3u);
        const uint32_t *wp = (const uint32_t *)(addr & ~(uintptr_t)3);
        uint32_t raw[10], a[9], q[8];
#pragma unroll
        for (int k = 0; k < 10; k++) raw[k] = wp[k];
#pragma unroll
        for (int k = 0; k < 9; k++) a[k] = align_bytes(raw[k + 1], raw[k], o);
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = align_bytes(a[k + 1], a[k], 2);
        const float ws = sf37_f16(a[0]);
        for (uint32_t t = 0; t < nt; t++) {
            const uint32_t *xv = xs + ((uint64_t)t * nb + b) * 8u;
            int32_t isum = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) isum = sdot4(q[k], xv[k], isum);
            red[((uint64_t)t * rows_per_wg + r) * nb + b] = (float)isum * ws * sc[t * nb + b];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nt * rows_per_wg; i += blockDim.x) {
        const uint32_t t = i / rows_per_wg, r = i - t * rows_per_wg;
        if (row0 + r >= out_dim) continue;
        const float *rv = red + ((uint64_t)t * rows_per_wg + r) * nb;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nb; b++) acc = acc + rv[b];
        out[(t0 + t) * out_dim + row0 + r] = acc;
    }
}

}  // namespace

extern "C" int sf37k_q8_0_quantize(int8_t *xq, float *xscale, const float *x, uint64_t in_dim,
                                   uint64_t n_tok, sf37_stream_t s) {
    const uint64_t nb = (in_dim + 31u) / 32u;
    const uint64_t hw = nb * n_tok;
    if (hw == 0) return 0;
    hipLaunchKernelGGL(q8_0_quantize_kernel, dim3((unsigned)((hw + 7) / 8)), dim3(256), 0,
                       (hipStream_t)s, xq, xscale, x, in_dim, nb, n_tok);
    return (int)hipGetLastError();
}

extern "C" int sf37k_q8_0_matmul(float *out0, float *out1, const uint8_t *w0, const uint8_t *w1,
                                 const int8_t *xq, const float *xscale, uint64_t in_dim,
                                 uint64_t out_dim, uint64_t n_tok, sf37_stream_t s) {
    if (out_dim == 0 || n_tok == 0) return 0;
    const uint32_t nb = (uint32_t)((in_dim + 31u) / 32u);
    uint32_t rows = nb >= 256u ? 1u : 256u / nb;
    if (rows > 32u) rows = 32u;
    const size_t per_tok = (size_t)nb * 36u + (size_t)rows * nb * 4u;
    uint32_t tpc = (uint32_t)((48u << 10) / per_tok);
    if (tpc > Q8_TPC_MAX) tpc = Q8_TPC_MAX;
    if (tpc < 1u) return (int)hipErrorInvalidValue;   /* row too long for LDS staging */
    const size_t lds = per_tok * tpc;
    const dim3 grid((unsigned)((out_dim + rows - 1) / rows), (unsigned)((n_tok + tpc - 1) / tpc),
                    out1 ? 2u : 1u);
    hipLaunchKernelGGL(q8_0_matmul_kernel, grid, dim3(256), lds, (hipStream_t)s, out0, out1, w0, w1,
                       xq, xscale, nb, out_dim, n_tok, rows, tpc);
    return (int)hipGetLastError();
}
