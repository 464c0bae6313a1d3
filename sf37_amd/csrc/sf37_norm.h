// sf37_norm.h - RMSNorm with (w + 1) weights (sf37_ops.c:22-28:
// y = x * (1 / sqrtf(mean(x^2) + eps)) * (w + 1), the sum of squares in
// binary64), shared by the standalone kernel (k_elem.hip) and the decode
// route kernel that normalises its input rows itself, so both give the same
// bits.
#pragma once

#include "sf37_router.h"

// Scale 1 / sqrtf(mean(x^2) + eps) of one row of n floats, computed by one
// wave and returned in every lane.  Lane l accumulates its elements in
// order in binary64 (each square is exact in binary64): for n a multiple of
// 256 the float4 groups at 4l + 256j, j ascending, else the elements
// l + 64j; then the lane sums are added by sf37_wave_sum_f64.
__device__ __forceinline__ float sf37_rms_scale_wave(const float *row, uint32_t n, float eps) {
    const uint32_t lane = threadIdx.x & 63u;
    double ss = 0.0;
    if ((n & 255u) == 0) {
#pragma unroll 4
        for (uint32_t k = 4u * lane; k < n; k += 256u) {
            const sf37_f32x4 v = *(const sf37_f32x4 *)(row + k);
#pragma unroll
            for (int q = 0; q < 4; q++) ss = __builtin_fma((double)v[q], (double)v[q], ss);
        }
    } else {
        for (uint32_t k = lane; k < n; k += 64u) {
            const double v = row[k];
            ss = __builtin_fma(v, v, ss);
        }
    }
    const double tot = sf37_wave_sum_f64(ss);
    return 1.0f / __builtin_sqrtf((float)(tot / (double)n) + eps);
}

// One normalised element: x * scale * (w + 1), w a bf16 weight.
__device__ __forceinline__ float sf37_norm_w1_bf16(float x, float scale, uint16_t w) {
    return x * scale * (__uint_as_float((uint32_t)w << 16) + 1.0f);
}
