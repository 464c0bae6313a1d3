// k_elem.hip - elementwise ops for gfx950: SwiGLU with clamp (sf37_ops.c:30-42),
// in-place add (sf37_cuda.cu:2137-2151), RMSNorm with (w + 1) weights
// (sf37_ops.c:22-28, computed by sf37_norm.h) and the exact bf16 -> f32
// widening of dense weights (sf37_quant.h bf16 decode: the 16 bits become the
// high half of the float).
#include "sf37_dev.h"
#include "sf37_norm.h"
#include "sf37_launch.h"

namespace {

__global__ void __launch_bounds__(256) swiglu_kernel(float *__restrict__ out,
                                                     const float *__restrict__ gate,
                                                     const float *__restrict__ up, uint64_t n,
                                                     float clamp) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    out[i] = sf37_swiglu_mid(gate[i], up[i], 1.0f, clamp);
}

__global__ void __launch_bounds__(256) add_kernel(float *__restrict__ dst,
                                                  const float *__restrict__ src, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) dst[i] = dst[i] + src[i];
}

__global__ void __launch_bounds__(256) add2_kernel(float *__restrict__ dst, const float *__restrict__ a,
                                                   const float *__restrict__ b, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) dst[i] = dst[i] + (a[i] + b[i]);
}

// One wave per row (four rows per workgroup): sf37_rms_scale_wave, then
// the weighted scale of every element.  Rows of 256..4096 elements (a
// multiple of 256) stay in registers between the two passes; the sum of
// squares runs in sf37_rms_scale_wave's order.
__global__ void __launch_bounds__(256) rms_norm_kernel(float *__restrict__ out,
                                                       const float *__restrict__ x,
                                                       const void *__restrict__ w, int bf16,
                                                       uint32_t n, uint32_t n_rows, float eps) {
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (row >= n_rows) return;
    const float *xr = x + (uint64_t)row * n;
    float *orow = out + (uint64_t)row * n;
    if (bf16 && (n & 255u) == 0 && n <= 4096u && ((uintptr_t)w & 7u) == 0) {
        // the row and its weights in registers (16-byte x loads, 8-byte
        // weight loads of four bf16 each, all issued before the sum)
        constexpr uint32_t MAXJ = 16;
        const uint32_t nj = n >> 8;
        sf37_f32x4 v[MAXJ];
        uint2 wv[MAXJ];
#pragma unroll
        for (uint32_t j = 0; j < MAXJ; j++)
            if (j < nj) {
                v[j] = *(const sf37_f32x4 *)(xr + 4u * lane + 256u * j);
                wv[j] = *(const uint2 *)((const uint16_t *)w + 4u * lane + 256u * j);
            }
        double ss = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < MAXJ; j++)
            if (j < nj) {
#pragma unroll
                for (int q = 0; q < 4; q++) ss = __builtin_fma((double)v[j][q], (double)v[j][q], ss);
            }
        const double tot = sf37_wave_sum_f64(ss);
        const float scale = 1.0f / __builtin_sqrtf((float)(tot / (double)n) + eps);
#pragma unroll
        for (uint32_t j = 0; j < MAXJ; j++)
            if (j < nj) {
                const uint32_t k = 4u * lane + 256u * j;
                const uint16_t wq[4] = {(uint16_t)wv[j].x, (uint16_t)(wv[j].x >> 16), (uint16_t)wv[j].y,
                                        (uint16_t)(wv[j].y >> 16)};
                sf37_f32x4 o;
#pragma unroll
                for (int q = 0; q < 4; q++) o[q] = sf37_norm_w1_bf16(v[j][q], scale, wq[q]);
                *(sf37_f32x4 *)(orow + k) = o;
            }
        return;
    }
    const float scale = sf37_rms_scale_wave(xr, n, eps);
    for (uint32_t i = lane; i < n; i += 64u) {
        orow[i] = bf16 ? sf37_norm_w1_bf16(xr[i], scale, ((const uint16_t *)w)[i])
                       : xr[i] * scale * (((const float *)w)[i] + 1.0f);
    }
}

// Four bf16 values per thread (one 8-byte load, one 16-byte store).
__global__ void __launch_bounds__(256) bf16_widen_kernel(float *__restrict__ out, const uint16_t *__restrict__ in,
                                                         uint64_t n) {
    const uint64_t i = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * 4u;
    if (i + 4u <= n && ((uintptr_t)(in + i) & 7u) == 0) {
        const uint2 v = *(const uint2 *)(in + i);
        float4 o;
        o.x = __builtin_bit_cast(float, v.x << 16);
        o.y = __builtin_bit_cast(float, v.x & 0xffff0000u);
        o.z = __builtin_bit_cast(float, v.y << 16);
        o.w = __builtin_bit_cast(float, v.y & 0xffff0000u);
        *(float4 *)(out + i) = o;
        return;
    }
    for (uint64_t k = i; k < i + 4u && k < n; k++) out[k] = __builtin_bit_cast(float, (uint32_t)in[k] << 16);
}

}  // namespace

extern "C" int sf37k_bf16_widen(float *out, const uint16_t *in, uint64_t n, sf37_stream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(bf16_widen_kernel, dim3((unsigned)((n + 1023u) / 1024u)), dim3(256), 0, (hipStream_t)s, out,
                       in, n);
    return (int)hipGetLastError();
}

extern "C" int sf37k_swiglu(float *out, const float *gate, const float *up, uint64_t n, float clamp,
                            sf37_stream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s,
                       out, gate, up, n, clamp);
    return (int)hipGetLastError();
}

extern "C" int sf37k_add_inplace(float *dst, const float *src, uint64_t n, sf37_stream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s,
                       dst, src, n);
    return (int)hipGetLastError();
}

extern "C" int sf37k_add2_inplace(float *dst, const float *a, const float *b, uint64_t n, sf37_stream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(add2_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s, dst, a, b, n);
    return (int)hipGetLastError();
}

extern "C" int sf37k_rms_norm(float *out, const float *x, const void *w, int w_is_bf16, uint32_t n,
                              uint32_t n_tok, float eps, sf37_stream_t s) {
    if (n_tok == 0) return 0;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((n_tok + 3u) / 4u), dim3(256), 0, (hipStream_t)s, out, x, w,
                       w_is_bf16, n, n_tok, eps);
    return (int)hipGetLastError();
}
