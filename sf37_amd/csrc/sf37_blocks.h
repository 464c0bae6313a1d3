// sf37_blocks.h - per-block integer dots of Q3/Q2 weights against staged
// Q8_K activations, shared by the GEMV and MoE kernels.
//
// A lane owns one 256-weight block: it loads the block with dword loads,
// expands the 3- or 2-bit codes into int8x4 words (sf37_dev.h) and runs
// v_dot4_i32_i8 against activations staged in LDS in the matching permuted
// order.  Device buffers handed to these loads carry >= 4 bytes of slack
// past their end (the library pads every allocation), because a Q3 block
// that starts on a dword boundary is read as 112 bytes.
#pragma once

#include "sf37_dev.h"

__device__ __forceinline__ void ld_dwords(uint32_t *dst, const uint8_t *p, int n) {
    const uint32_t *q = (const uint32_t *)p;
#pragma unroll
    for (int i = 0; i < n; i++) dst[i] = q[i];
}

// Staged activation for one 256-block: codes permuted for the Q3 (or Q2)
// unpack, as 64 dwords, plus d and the four 64-wide code sums.
struct act_block {
    uint32_t qs[64];
    float d;
    int32_t gs[4];
};

// Copy n Q8_K blocks from global into LDS in permuted order.  All threads
// of the workgroup participate; caller synchronises afterwards.
template <bool Q3>
__device__ __forceinline__ void stage_act(act_block *dst, const q8k_block *src, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n * 64u; i += blockDim.x) {
        const uint32_t b = i >> 6, w = i & 63u;
        const uint32_t v = ((const uint32_t *)src[b].qs)[w];
        uint8_t *qd = (uint8_t *)dst[b].qs;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t e = 4u * w + k;
            qd[Q3 ? q3_perm_pos(e) : q2_perm_pos(e)] = (uint8_t)(v >> (8 * k));
        }
        if (w < 4u) dst[b].gs[w] = src[b].gsums[w];
        if (w == 4u) dst[b].d = src[b].d;
    }
}

// Realign a Q3 block that starts at byte offset o (0 or 2) of w[0..27] so
// that a[0..26] hold bytes 0..107 of the block.
__device__ __forceinline__ void q3_realign(uint32_t *a, const uint32_t *w, uint32_t o) {
#pragma unroll
    for (int i = 0; i < 27; i++) a[i] = align_bytes(w[i + 1], w[i], o);
}

// Integer part of the four groups of a Q3 block against one activation.
__device__ __forceinline__ void q3_block_idots(const uint32_t *a, const act_block &x, int32_t I[4]) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t d0 = a[3 + 6 * g], d1 = a[4 + 6 * g], d2 = a[5 + 6 * g];
        const uint32_t d3 = a[6 + 6 * g], d4 = a[7 + 6 * g], d5 = a[8 + 6 * g];
        const uint32_t c[8] = {d0, align_bits(d1, d0, 24), align_bits(d2, d1, 16), d2 >> 8,
                               d3, align_bits(d4, d3, 24), align_bits(d5, d4, 16), d5 >> 8};
        int32_t acc = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t lo, hi;
            q3_unpack8(c[k], lo, hi);
            acc = sdot4(lo, x.qs[16 * g + 2 * k], acc);
            acc = sdot4(hi, x.qs[16 * g + 2 * k + 1], acc);
        }
        const int32_t zp = (int32_t)((a[2] >> (8 * g)) & 7u);
        I[g] = acc - zp * x.gs[g];
    }
}

__device__ __forceinline__ float q3_block_value(const uint32_t *a, const int32_t I[4]) {
    float bs = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float s = sf37_f16(a[g >> 1] >> (16 * (g & 1)));
        bs = __builtin_fmaf(s, (float)I[g], bs);
    }
    return bs;
}

// Q2 block (21 dwords, always dword aligned in a row of 84-byte blocks).
__device__ __forceinline__ void q2_block_idots(const uint32_t *a, const act_block &x, int32_t I[4]) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        int32_t acc = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t c0, c1, c2, c3;
            q2_unpack16(a[3 + 4 * g + j], c0, c1, c2, c3);
            const uint32_t *xs = &x.qs[16 * g + 4 * j];
            acc = sdot4(c0, xs[0], acc);
            acc = sdot4(c1, xs[1], acc);
            acc = sdot4(c2, xs[2], acc);
            acc = sdot4(c3, xs[3], acc);
        }
        const int32_t zp = (int32_t)((a[2] >> (8 * g)) & 3u);
        I[g] = acc - zp * x.gs[g];
    }
}

__device__ __forceinline__ float q2_block_value(const uint32_t *a, const int32_t I[4]) {
    float bs = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float s = sf37_f16(a[g >> 1] >> (16 * (g & 1)));
        bs = __builtin_fmaf(s, (float)I[g], bs);
    }
    return bs;
}

// Load a Q3 block at byte address p (2-byte aligned) into 28 raw dwords
// from the enclosing dword boundary; returns the byte offset (0 or 2).
__device__ __forceinline__ uint32_t q3_load(uint32_t *w, const uint8_t *p) {
    const uintptr_t addr = (uintptr_t)p;
    ld_dwords(w, (const uint8_t *)(addr & ~(uintptr_t)3), 28);
    return (uint32_t)(addr & 3u);
}


// Copy the bytes [src, src + n) of global memory into LDS with direct
// global->LDS dwordx4 loads: each wave instruction moves 64 x 16 contiguous
// bytes, so weight tiles are read fully coalesced whatever their block size.
// The copy starts at the 16-byte boundary at or below src, so dst (16-byte
// aligned) must hold n + 31 bytes; returns the offset of src inside dst.
// Reads up to 15 bytes past src + n, inside the slack every library
// allocation carries.  All threads of the workgroup call it; lds_copy_wait()
// must follow before dst is read.
__device__ __forceinline__ uint32_t lds_copy(uint8_t *dst, const uint8_t *src, uint32_t n) {
    const uintptr_t a = (uintptr_t)src, a0 = a & ~(uintptr_t)15;
    const uint32_t off = (uint32_t)(a - a0);
    const uint32_t chunks = (off + n + 15u) >> 4;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, nw = blockDim.x >> 6;
    for (uint32_t c0 = wave * 64u; c0 < chunks; c0 += nw * 64u) {
        const uint32_t c = c0 + lane;
        if (c < chunks)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + 16u * (uintptr_t)c), dst + 16u * c0, 16, 0, 0);
    }
    return off;
}

__device__ __forceinline__ void lds_copy_wait() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Activation blocks for the fused decode kernels: 256 Q8_K codes in the
// order the weight unpack produces (Q3: q3x_pos, Q2: q2_perm_pos), the
// scale d and the four 64-wide code sums, padded to 288 bytes so a block
// is a whole number of 16-byte chunks.
// ---------------------------------------------------------------------------
struct __attribute__((aligned(16))) act_t {
    uint32_t qs[64];
    float d;
    int32_t gs[4];
    uint32_t pad[3];
};
static_assert(sizeof(act_t) == 288, "act_t is 288 bytes");

// Byte position of element i (0..255) of a block in the Q3 act layout: chunk
// c = i / 32 (12 payload bytes), code j = i % 32 sits in dword 8c + j % 8,
// byte j / 8 -- the order q3_unpack32 produces.
__host__ __device__ inline uint32_t q3x_pos(uint32_t i) {
    const uint32_t c = i >> 5, j = i & 31u;
    return ((c << 3) + (j & 7u)) * 4u + (j >> 3);
}

__device__ __forceinline__ uint32_t vperm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Bytes S, S+3, S+6, S+9 of the dword array w -> bytes 0..3 (S is a
// compile-time constant after inlining, so the selectors fold).
__device__ __forceinline__ uint32_t gather_every3(const uint32_t *w, int S) {
    const int d0 = S >> 2;
    uint32_t sel = 0;
    for (int k = 0; k < 4; k++) {
        const int pos = S + 3 * k, d = (pos >> 2) - d0, b = pos & 3;
        sel |= (uint32_t)(d <= 1 ? d * 4 + b : 0x0c) << (8 * k);
    }
    uint32_t t = vperm(w[d0 + 1], w[d0], sel);
    const int d3 = ((S + 9) >> 2) - d0;
    if (d3 >= 2) {
        uint32_t sel2 = 0;
        for (int k = 0; k < 4; k++) {
            const int pos = S + 3 * k, d = (pos >> 2) - d0, b = pos & 3;
            sel2 |= (uint32_t)(d <= 1 ? k : d == 2 ? 4 + b : 0x0c) << (8 * k);
        }
        t = vperm(w[d0 + 2], t, sel2);
    }
    if (d3 >= 3) {
        uint32_t sel3 = 0;
        for (int k = 0; k < 4; k++) {
            const int pos = S + 3 * k, d = (pos >> 2) - d0, b = pos & 3;
            sel3 |= (uint32_t)(d <= 2 ? k : 4 + b) << (8 * k);
        }
        t = vperm(w[d0 + 3], t, sel3);
    }
    return t;
}

// 32 three-bit codes (LSB-first) in the 12 bytes at byte S of w -> eight
// i8x4 words, word r byte a = code 8a + r.  Gathering bytes 3a, 3a+1, 3a+2
// puts code 8a + r at bit 3r of a 24-bit lane, so each word is one or two
// shifts and masks.
__device__ __forceinline__ void q3_unpack32(const uint32_t *w, int S, uint32_t c[8]) {
    const uint32_t D0 = gather_every3(w, S), D1 = gather_every3(w, S + 1), D2 = gather_every3(w, S + 2);
    c[0] = D0 & 0x07070707u;
    c[1] = (D0 >> 3) & 0x07070707u;
    c[2] = ((D0 >> 6) & 0x03030303u) | ((D1 << 2) & 0x04040404u);
    c[3] = (D1 >> 1) & 0x07070707u;
    c[4] = (D1 >> 4) & 0x07070707u;
    c[5] = ((D1 >> 7) & 0x01010101u) | ((D2 << 1) & 0x06060606u);
    c[6] = (D2 >> 2) & 0x07070707u;
    c[7] = (D2 >> 5) & 0x07070707u;
}
