// k_synth.hip - synthetic inputs generated on the device (harness).
//
// N(0, sigma) values come from a counter-based splitmix64 stream keyed by
// (seed, stream) and a Box-Muller transform built only from IEEE +,-,*,/,
// sqrt and fixed polynomials, so they match the CPU generator bit for bit.
// Quantised weight rows apply the reference weight quantizer
// (gguf-tools/quants.c:341-421, 574-609) to rows generated in registers, so
// a full 288-expert layer never exists in fp32.
#include "sf37_dev.h"
#include "sf37_launch.h"

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ull;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebull;
    z ^= z >> 31;
    return z;
}

__device__ __forceinline__ float synth_ln(float u) {
    const uint32_t b = __float_as_uint(u);
    int e = (int)((b >> 23) & 0xffu) - 127;
    float m = __uint_as_float((b & 0x7fffffu) | 0x3f800000u);
    if (m > 0x1.6a09e6p+0f) {
        m = m * 0.5f;
        e += 1;
    }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 0x1.745d18p-4f;
    p = __builtin_fmaf(p, s2, 0x1.c71c72p-4f);
    p = __builtin_fmaf(p, s2, 0x1.24924ap-3f);
    p = __builtin_fmaf(p, s2, 0x1.99999ap-3f);
    p = __builtin_fmaf(p, s2, 0x1.555556p-2f);
    p = __builtin_fmaf(p, s2, 1.0f);
    return __builtin_fmaf((float)e, 0x1.62e430p-1f, (2.0f * s) * p);
}

__device__ __forceinline__ float synth_cos2pi(float t) {
    const float y = t * t;
    float p = 0x1.ef6e30p-9f;
    p = __builtin_fmaf(p, y, -0x1.2a0c5ap-5f);
    p = __builtin_fmaf(p, y, 0x1.20c62cp-2f);
    p = __builtin_fmaf(p, y, -0x1.b6e250p+0f);
    p = __builtin_fmaf(p, y, 0x1.f9d38ap+2f);
    p = __builtin_fmaf(p, y, -0x1.a6d1f2p+4f);
    p = __builtin_fmaf(p, y, 0x1.e1f506p+5f);
    p = __builtin_fmaf(p, y, -0x1.55d3c8p+6f);
    p = __builtin_fmaf(p, y, 0x1.03c1f0p+6f);
    p = __builtin_fmaf(p, y, -0x1.3bd3ccp+4f);
    return __builtin_fmaf(p, y, 1.0f);
}

__device__ __forceinline__ float synth_normal(uint64_t key, uint64_t index) {
    const uint64_t z = mix64(key + (index + 1u) * 0x9e3779b97f4a7c15ull);
    const float u1 = ((float)(uint32_t)(z >> 40) + 0.5f) * 0x1p-24f;
    const float u2 = (float)(uint32_t)((z >> 16) & 0xffffffu) * 0x1p-24f;
    const float r = __builtin_sqrtf(-2.0f * synth_ln(u1));
    return r * -synth_cos2pi(u2 - 0.5f);
}

__global__ void __launch_bounds__(256) normal_kernel(float *__restrict__ dst, uint64_t n,
                                                     uint64_t key, uint64_t index0, float sigma) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) dst[i] = sigma * synth_normal(key, index0 + i);
}

__device__ __forceinline__ uint16_t f16_bits(float f) {
    return __builtin_bit_cast(unsigned short, (_Float16)f);
}

// Scale and zero-point of a 64-wide asymmetric group (gguf-tools/quants.c:386-406).
__device__ __forceinline__ void asym_group(const float *v, int qmax, float &scale, int &zp) {
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int i = 1; i < 64; i++) {
        if (v[i] < lo) lo = v[i];
        if (v[i] > hi) hi = v[i];
    }
    scale = 1.0f;
    zp = 0;
    if (hi != lo) {
        scale = (hi - lo) / (float)qmax;
        zp = (int)__builtin_rintf(-lo / scale);
        zp = zp < 0 ? 0 : (zp > qmax ? qmax : zp);
    } else if (hi != 0.0f) {
        scale = fabsf(hi) / (float)qmax;
        zp = hi > 0.0f ? 0 : qmax;
    }
}

__device__ __forceinline__ int asym_code(float x, float inv, int zp, int qmax) {
    const int q = (int)__builtin_rintf(x * inv + (float)zp);
    return q < 0 ? 0 : (q > qmax ? qmax : q);
}

// One thread per output block; type 3 = Q3 (110 B), 2 = Q2 (84 B), 0 = Q8_0 (34 B).
template <int TYPE>
__global__ void __launch_bounds__(256) gen_quant_kernel(uint8_t *__restrict__ dst, uint64_t row0,
                                                        uint64_t nrows, uint64_t ncols, uint64_t key,
                                                        float sigma) {
    constexpr int QK = TYPE == 0 ? 32 : 256;
    constexpr int BS = TYPE == 0 ? SF37_Q8_0_BYTES : (TYPE == 3 ? SF37_Q3_BYTES : SF37_Q2_BYTES);
    const uint64_t nb = ncols / QK;
    const uint64_t blk = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (blk >= nrows * nb) return;
    const uint64_t r = blk / nb, b = blk - r * nb;
    const uint64_t idx0 = (row0 + r) * ncols + b * QK;
    uint8_t *y = dst + blk * BS;
    if (TYPE == 0) {
        float v[32];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            v[j] = sigma * synth_normal(key, idx0 + j);
            const float a = fabsf(v[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t hd = f16_bits(d);
        y[0] = (uint8_t)(hd & 0xffu);
        y[1] = (uint8_t)(hd >> 8);
#pragma unroll
        for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)__builtin_roundf(v[j] * id);
        return;
    }
    constexpr int QMAX = TYPE == 3 ? 7 : 3;
    uint8_t out[BS];
#pragma unroll
    for (int i = 0; i < BS; i++) out[i] = 0;
    for (int g = 0; g < 4; g++) {
        float v[64];
#pragma unroll
        for (int j = 0; j < 64; j++) v[j] = sigma * synth_normal(key, idx0 + 64 * g + j);
        float scale;
        int zp;
        asym_group(v, QMAX, scale, zp);
        const uint16_t hs = f16_bits(scale);
        out[2 * g] = (uint8_t)(hs & 0xffu);
        out[2 * g + 1] = (uint8_t)(hs >> 8);
        out[8 + g] = (uint8_t)zp;
        const float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        if (TYPE == 3) {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                uint32_t bits = 0;
#pragma unroll
                for (int j = 0; j < 8; j++) bits |= (uint32_t)asym_code(v[8 * c + j], inv, zp, 7) << (3 * j);
                out[12 + 24 * g + 3 * c] = (uint8_t)bits;
                out[12 + 24 * g + 3 * c + 1] = (uint8_t)(bits >> 8);
                out[12 + 24 * g + 3 * c + 2] = (uint8_t)(bits >> 16);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; c++) {
                uint32_t bits = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) bits |= (uint32_t)asym_code(v[4 * c + j], inv, zp, 3) << (2 * j);
                out[12 + 16 * g + c] = (uint8_t)bits;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < BS; i++) y[i] = out[i];
}

__global__ void __launch_bounds__(256) sigmoid_array_kernel(float *__restrict__ out,
                                                            const float *__restrict__ x, uint64_t n,
                                                            int mode) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = mode ? sf37_sigmoid(x[i]) : sf37_expf(x[i]);
}

}  // namespace

extern "C" int sf37k_synth_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                                  uint64_t index0, float sigma, sf37_stream_t s) {
    if (n == 0) return 0;
    uint64_t key;
    {
        // host copy of stream_key()
        auto mix = [](uint64_t z) {
            z ^= z >> 30;
            z *= 0xbf58476d1ce4e5b9ull;
            z ^= z >> 27;
            z *= 0x94d049bb133111ebull;
            z ^= z >> 31;
            return z;
        };
        key = mix(seed ^ mix(stream + 0x9e3779b97f4a7c15ull));
    }
    hipLaunchKernelGGL(normal_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s,
                       dst, n, key, index0, sigma);
    return (int)hipGetLastError();
}

extern "C" int sf37k_synth_quant_rows(int type, uint8_t *dst, uint64_t row0, uint64_t nrows,
                                      uint64_t ncols, uint64_t seed, uint64_t stream, float sigma,
                                      sf37_stream_t s) {
    auto mix = [](uint64_t z) {
        z ^= z >> 30;
        z *= 0xbf58476d1ce4e5b9ull;
        z ^= z >> 27;
        z *= 0x94d049bb133111ebull;
        z ^= z >> 31;
        return z;
    };
    const uint64_t key = mix(seed ^ mix(stream + 0x9e3779b97f4a7c15ull));
    const uint64_t qk = type == 0 ? 32u : 256u;
    const uint64_t blocks = nrows * (ncols / qk);
    if (blocks == 0) return 0;
    const dim3 grid((unsigned)((blocks + 255) / 256));
    if (type == 3)
        hipLaunchKernelGGL(gen_quant_kernel<3>, grid, dim3(256), 0, (hipStream_t)s, dst, row0, nrows, ncols, key, sigma);
    else if (type == 2)
        hipLaunchKernelGGL(gen_quant_kernel<2>, grid, dim3(256), 0, (hipStream_t)s, dst, row0, nrows, ncols, key, sigma);
    else if (type == 0)
        hipLaunchKernelGGL(gen_quant_kernel<0>, grid, dim3(256), 0, (hipStream_t)s, dst, row0, nrows, ncols, key, sigma);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

extern "C" int sf37k_sigmoid_array(float *out, const float *x, uint64_t n, int mode, sf37_stream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(sigmoid_array_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)s, out, x, n, mode);
    return (int)hipGetLastError();
}
