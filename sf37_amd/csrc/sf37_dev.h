// sf37_dev.h - device helpers shared by the gfx950 kernels.
//
// All float arithmetic here is written in a fixed order with explicit fma;
// the library is compiled with -ffp-contract=off so nothing else is fused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SF37_QK 256
#define SF37_Q3_BYTES 110
#define SF37_Q2_BYTES 84
#define SF37_Q8_0_BYTES 34
#define SF37_Q8K_BYTES 268

// Q8_K activation block: byte layout of the reference (sf37_cuda.cu:4162-4166).
struct __attribute__((packed, aligned(4))) q8k_block {
    float d;
    int8_t qs[SF37_QK];
    int16_t gsums[4];
};
static_assert(sizeof(q8k_block) == SF37_Q8K_BYTES, "Q8_K block is 268 bytes");

// ---------------------------------------------------------------------------
// expf: the table-driven exp2 reduction with N = 32 entries and a cubic
// polynomial (the published method of ARM's optimized-routines, which glibc
// 2.28+ ships), evaluated in binary64 with the argument reduction fused.
// Verified bit-identical to the host glibc expf for every binary32 input.
// ---------------------------------------------------------------------------
__host__ __device__ inline uint64_t sf37_exp2_tab(uint32_t i) {
    // 2^(i/32) rounded to binary64, minus i << 47 (exponent bits added back below)
    constexpr uint64_t tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    return tab[i & 31u];
}

// LDS_TAB: the 32 table words (sf37_exp2_tab) are read from tab, a copy the
// caller staged in LDS; otherwise from the constant table.  Branch-free: the
// reduction runs for every input and the special cases (|x| >= 88 that
// overflow or underflow, infinities, NaN) are selected at the end, so
// unrolled calls stay straight-line code on the GPU.
template <bool LDS_TAB>
__host__ __device__ inline float sf37_expf_impl(float x, const uint64_t *tab) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;   // 32 / ln 2
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd = kd - shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = LDS_TAB ? tab[ki & 31u] : sf37_exp2_tab((uint32_t)(ki & 31u));
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    float res = (float)y;
    if (abstop >= 0x42bu) {                       // |x| >= 88 or nan (selects)
        res = x < -0x1.9fe368p6f ? 0.0f : res;
        res = x > 0x1.62e42ep6f ? __builtin_inff() : res;
        res = abstop >= 0x7f8u ? x + x : res;
        res = ux == 0xff800000u ? 0.0f : res;
    }
    return res;
}

__host__ __device__ inline float sf37_expf(float x) { return sf37_expf_impl<false>(x, nullptr); }

// sf37_ops.c:9-16: x >= 0 ? 1 / (1 + e^-x) : e^x / (1 + e^x), branch-free.
template <bool LDS_TAB>
__host__ __device__ inline float sf37_sigmoid_impl(float x, const uint64_t *tab) {
    const bool pos = x >= 0.0f;
    const float z = sf37_expf_impl<LDS_TAB>(pos ? -x : x, tab);
    return (pos ? 1.0f : z) / (1.0f + z);
}

__host__ __device__ inline float sf37_sigmoid(float x) { return sf37_sigmoid_impl<false>(x, nullptr); }
// tab: the table staged in LDS (sf37_stage_exp_tab), never null
__host__ __device__ inline float sf37_sigmoid_t(float x, const uint64_t *tab) { return sf37_sigmoid_impl<true>(x, tab); }

// Stage the exp table into LDS (all threads may call; caller syncs).
__device__ inline void sf37_stage_exp_tab(uint64_t *lds_tab) {
    for (uint32_t i = threadIdx.x; i < 32u; i += blockDim.x) lds_tab[i] = sf37_exp2_tab(i);
}

// ((g * sigmoid(g)) * u) * w with the routed/shared clamp (sf37_cuda.cu:4444-4456).
template <bool LDS_TAB>
__device__ __forceinline__ float sf37_swiglu_mid_impl(float g, float u, float w, float clamp, const uint64_t *tab) {
    if (clamp > 1.0e-6f) {
        if (g > clamp) g = clamp;
        if (u > clamp) u = clamp;
        if (u < -clamp) u = -clamp;
    }
    return g * sf37_sigmoid_impl<LDS_TAB>(g, tab) * u * w;
}

// tab: the table staged in LDS, never null
__device__ __forceinline__ float sf37_swiglu_mid_t(float g, float u, float w, float clamp, const uint64_t *tab) {
    return sf37_swiglu_mid_impl<true>(g, u, w, clamp, tab);
}

__device__ __forceinline__ float sf37_swiglu_mid(float g, float u, float w, float clamp) {
    return sf37_swiglu_mid_impl<false>(g, u, w, clamp, nullptr);
}

__device__ __forceinline__ float sf37_f16(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h16 & 0xffffu));
}

__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t nbytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, nbytes);
}

__device__ __forceinline__ uint32_t align_bits(uint32_t hi, uint32_t lo, uint32_t nbits) {
    return __builtin_amdgcn_alignbit(hi, lo, nbits);
}

// Eight 3-bit codes (bits [0,24) of c, upper bits ignored) -> two i8x4 words:
// a = codes {0,2,4,6}, b = codes {1,3,5,7}.  The activations are permuted
// to the same order, so no byte shuffles are needed.
__device__ __forceinline__ void q3_unpack8(uint32_t c, uint32_t &a, uint32_t &b) {
    const uint32_t t = (c & 0xfffu) | ((c << 4) & 0xfffff000u);          // codes 4..7 -> bit 16
    const uint32_t t2 = (t & 0x003f003fu) | ((t << 2) & 0xffc0ffc0u);     // codes 2,3 / 6,7 -> +8
    a = t2 & 0x07070707u;
    b = (t2 >> 3) & 0x07070707u;
}

// Sixteen 2-bit codes in w -> four i8x4 words holding codes {j, j+4, j+8, j+12}.
__device__ __forceinline__ void q2_unpack16(uint32_t w, uint32_t &a, uint32_t &b, uint32_t &c,
                                            uint32_t &d) {
    a = w & 0x03030303u;
    b = (w >> 2) & 0x03030303u;
    c = (w >> 4) & 0x03030303u;
    d = (w >> 6) & 0x03030303u;
}

__device__ __forceinline__ int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Position of element i (0..255) of a Q8_K block in the permuted order used
// by the Q3 kernels: within each run of 8, even elements first then odd.
__device__ __forceinline__ uint32_t q3_perm_pos(uint32_t i) {
    const uint32_t j = i & 7u;
    return (i & ~7u) | ((j & 1u) << 2) | (j >> 1);
}

// Position of element i in the order used by the Q2 kernels: within each
// run of 16, element 4k+s goes to 4s+k.
__device__ __forceinline__ uint32_t q2_perm_pos(uint32_t i) {
    const uint32_t j = i & 15u;
    return (i & ~15u) | ((j & 3u) << 2) | (j >> 2);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int wave_sum_i32_width(int v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Q8_K quantisation of one 256-block held by a full wave, 4 values per lane
// (lane l holds elements 4l..4l+3).  Writes codes with the given position
// map into qs_out (LDS or global) and returns d; gsum of group g is
// returned in lanes with (lane >> 4) == g.  Arithmetic of sf37_cuda.cu:4168-4205
// with IEEE division, clamp in float (identical for finite products).
__device__ __forceinline__ float q8k_codes4(const float v[4], int8_t q[4], int &gsum) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = wave_max(amax);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float r = fminf(fmaxf(__builtin_rintf(v[k] * id), -128.0f), 127.0f);
        q[k] = (int8_t)(int)r;
        s += q[k];
    }
    gsum = wave_sum_i32_width(s, 16);
    return d;
}
