/*
 * sf37_oracle.c - CPU restatement of the SF37 MoE FFN hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see sf37_oracle.h).  Built with
 *   -O2 -std=c11 -ffp-contract=off  (no fast-math)
 * so every float operation is a single IEEE-754 rounding in source order.
 * Citations are file:line in the ZephinueCode/sf37 reference repository.
 */
#include "sf37_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ===================================================================== */
/* Scalar formats                                                         */
/* ===================================================================== */

/* IEEE binary16 -> binary32, exact.  Restates sf37_quant.c:5-30. */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u;
    uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0u) {
        bits = sign;
    } else {
        /* subnormal half: m * 2^-24; normalise the 10-bit mantissa */
        uint32_t sh = 0;
        while (!(m & 0x400u)) { m <<= 1; sh++; }
        bits = sign | ((113u - sh) << 23) | ((m & 1023u) << 13);
    }
    return u2f(bits);
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN to the
 * quiet pattern 0x7e00.  Same results as ds4q_f32_to_f16
 * (gguf-tools/quants.c:92-109) for every input. */
uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (ax < 0x38800000u) {                                    /* < 2^-14 */
        /* subnormal half: count of 2^-24 units, rounded half-even */
        const float units = u2f(ax) * 0x1p24f;                 /* exact */
        return (uint16_t)(sign | (uint16_t)rintf(units));
    }
    const uint32_t m = ax & 0x7fffffu;
    uint32_t h = (((ax >> 23) - 112u) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* sf37_quant.c:32-37 */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round half to even for |v| <= 4194303.  gguf-tools/quants.c:111-117 adds
 * 1.5*2^23 so the float add performs the rounding; rintf performs the same
 * rounding in the default mode. */
int orc_nearest_int(float v) { return (int)rintf(v); }

/* ===================================================================== */
/* Block decode and fp32 dots (sf37_quant.c:45-124)                        */
/* ===================================================================== */

/* 3-bit value i of a 24-byte payload, LSB-first.  sf37_quant.c:45-52. */
uint32_t orc_q3_get(const uint8_t *p, int i) {
    const int bit = 3 * i;
    uint32_t w = p[bit >> 3];
    if ((bit & 7) > 5) w |= (uint32_t)p[(bit >> 3) + 1] << 8;
    return (w >> (bit & 7)) & 7u;
}

static uint32_t q2_get(const uint8_t *p, int i) {
    return (p[i >> 2] >> ((i & 3) * 2)) & 3u;
}

/* sf37_quant.c:54-58 */
void orc_q8_0_block_decode(const uint8_t *blk, float *dst32) {
    const float s = orc_f16_to_f32(rd16(blk));
    for (int i = 0; i < 32; i++) dst32[i] = (float)(int8_t)blk[2 + i] * s;
}

/* sf37_quant.c:60-66: sum += (q * s) * x, sequential. */
float orc_q8_0_block_dot(const uint8_t *blk, const float *x32) {
    const float s = orc_f16_to_f32(rd16(blk));
    float sum = 0.0f;
    for (int i = 0; i < 32; i++) sum += (float)(int8_t)blk[2 + i] * s * x32[i];
    return sum;
}

/* sf37_quant.c:68-79: w = (q - zp) * scale, zp masked to 3 bits. */
void orc_q3_block_decode(const uint8_t *blk, float *dst256) {
    for (int g = 0; g < 4; g++) {
        const float s = orc_f16_to_f32(rd16(blk + 2 * g));
        const float zp = (float)(blk[8 + g] & 7u);
        const uint8_t *pl = blk + 12 + 24 * g;
        for (int i = 0; i < 64; i++) dst256[64 * g + i] = ((float)orc_q3_get(pl, i) - zp) * s;
    }
}

/* sf37_quant.c:81-93 */
void orc_q2_block_decode(const uint8_t *blk, float *dst256) {
    for (int g = 0; g < 4; g++) {
        const float s = orc_f16_to_f32(rd16(blk + 2 * g));
        const float zp = (float)(blk[8 + g] & 3u);
        const uint8_t *pl = blk + 12 + 16 * g;
        for (int i = 0; i < 64; i++) dst256[64 * g + i] = ((float)q2_get(pl, i) - zp) * s;
    }
}

/* sf37_quant.c:95-108: sum += ((q - zp) * s) * x, groups then elements. */
float orc_q3_block_dot(const uint8_t *blk, const float *x256) {
    float sum = 0.0f;
    for (int g = 0; g < 4; g++) {
        const float s = orc_f16_to_f32(rd16(blk + 2 * g));
        const float zp = (float)(blk[8 + g] & 7u);
        const uint8_t *pl = blk + 12 + 24 * g;
        for (int i = 0; i < 64; i++) sum += ((float)orc_q3_get(pl, i) - zp) * s * x256[64 * g + i];
    }
    return sum;
}

/* sf37_quant.c:110-124 */
float orc_q2_block_dot(const uint8_t *blk, const float *x256) {
    float sum = 0.0f;
    for (int g = 0; g < 4; g++) {
        const float s = orc_f16_to_f32(rd16(blk + 2 * g));
        const float zp = (float)(blk[8 + g] & 3u);
        const uint8_t *pl = blk + 12 + 16 * g;
        for (int i = 0; i < 64; i++) sum += ((float)q2_get(pl, i) - zp) * s * x256[64 * g + i];
    }
    return sum;
}

/* ===================================================================== */
/* Reference weight quantizer (gguf-tools/quants.c)                       */
/* ===================================================================== */

/* Asymmetric 64-wide group: scale/zero-point choice of
 * gguf-tools/quants.c:386-406 (Q3, qmax 7) and :579-593 (Q2, qmax 3). */
static void asym_group(const float *gx, int qmax, float *scale_out, int *zp_out) {
    float lo = gx[0], hi = gx[0];
    for (int i = 1; i < 64; i++) {
        if (gx[i] < lo) lo = gx[i];
        if (gx[i] > hi) hi = gx[i];
    }
    float scale = 1.0f;
    int zp = 0;
    if (hi != lo) {
        scale = (hi - lo) / (float)qmax;
        zp = orc_nearest_int(-lo / scale);
        if (zp < 0) zp = 0;
        if (zp > qmax) zp = qmax;
    } else if (hi != 0.0f) {
        scale = fabsf(hi) / (float)qmax;
        zp = hi > 0.0f ? 0 : qmax;
    }
    *scale_out = scale;
    *zp_out = zp;
}

static int asym_code(float x, float inv, int zp, int qmax) {
    int q = orc_nearest_int(x * inv + (float)zp);
    return q < 0 ? 0 : (q > qmax ? qmax : q);
}

/* Q3 "Q3GU" block writer, gguf-tools/quants.c:381-421.  Layout:
 * [0,8) 4 x f16 scale, [8,12) 4 x u8 zp, [12,108) 4 x 24-byte 3-bit
 * payloads (value i at bits [3i,3i+3) LSB-first), [108,110) zero. */
void orc_quantize_q3_block(const float *x, uint8_t *y) {
    memset(y, 0, ORC_Q3_BLOCK);
    for (int g = 0; g < 4; g++) {
        float scale;
        int zp;
        asym_group(x + 64 * g, 7, &scale, &zp);
        const uint16_t hs = orc_f32_to_f16(scale);
        y[2 * g] = (uint8_t)(hs & 0xff);
        y[2 * g + 1] = (uint8_t)(hs >> 8);
        y[8 + g] = (uint8_t)zp;
        const float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        uint8_t *pl = y + 12 + 24 * g;
        /* eight 3-bit codes make three bytes */
        for (int c = 0; c < 8; c++) {
            uint32_t bits = 0;
            for (int j = 0; j < 8; j++)
                bits |= (uint32_t)asym_code(x[64 * g + 8 * c + j], inv, zp, 7) << (3 * j);
            pl[3 * c] = (uint8_t)bits;
            pl[3 * c + 1] = (uint8_t)(bits >> 8);
            pl[3 * c + 2] = (uint8_t)(bits >> 16);
        }
    }
}

/* Q2 "Q2D" block writer, gguf-tools/quants.c:574-609.  Layout:
 * [0,8) scales, [8,12) zp, [12,76) 4 x 16-byte 2-bit payloads (value i at
 * bits 2*(i&3) of byte i>>2), [76,84) zero. */
void orc_quantize_q2_block(const float *x, uint8_t *y) {
    memset(y, 0, ORC_Q2_BLOCK);
    for (int g = 0; g < 4; g++) {
        float scale;
        int zp;
        asym_group(x + 64 * g, 3, &scale, &zp);
        const uint16_t hs = orc_f32_to_f16(scale);
        y[2 * g] = (uint8_t)(hs & 0xff);
        y[2 * g + 1] = (uint8_t)(hs >> 8);
        y[8 + g] = (uint8_t)zp;
        const float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        uint8_t *pl = y + 12 + 16 * g;
        for (int b = 0; b < 16; b++) {
            uint32_t v = 0;
            for (int j = 0; j < 4; j++)
                v |= (uint32_t)asym_code(x[64 * g + 4 * b + j], inv, zp, 3) << (2 * j);
            pl[b] = (uint8_t)v;
        }
    }
}

/* Q8_0 weight block, gguf-tools/quants.c:349-365: d = amax/127, codes use
 * roundf (half away from zero). */
void orc_quantize_q8_0_block(const float *x, uint8_t *y) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(x[j]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t hd = orc_f32_to_f16(d);
    y[0] = (uint8_t)(hd & 0xff);
    y[1] = (uint8_t)(hd >> 8);
    for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

/* Row driver in the spirit of ds4q_quantize_chunk (gguf-tools/quants.c:1351-1378). */
void orc_quantize_rows(int type, const float *src, uint8_t *dst, int64_t nrows,
                       int64_t ncols) {
    const int64_t qk = type == 0 ? 32 : ORC_QK_K;
    const int64_t bs = type == 0 ? ORC_Q8_0_BLOCK : (type == 3 ? ORC_Q3_BLOCK : ORC_Q2_BLOCK);
    const int64_t nb = ncols / qk;
    for (int64_t r = 0; r < nrows; r++) {
        for (int64_t b = 0; b < nb; b++) {
            const float *x = src + r * ncols + b * qk;
            uint8_t *y = dst + (r * nb + b) * bs;
            if (type == 0) orc_quantize_q8_0_block(x, y);
            else if (type == 3) orc_quantize_q3_block(x, y);
            else orc_quantize_q2_block(x, y);
        }
    }
}

/* ===================================================================== */
/* CPU ops (sf37_ops.c)                                                   */
/* ===================================================================== */

/* sf37_ops.c:9-16, libm expf (the reference's own function). */
float orc_sigmoid(float x) {
    if (x >= 0.0f) {
        const float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = expf(x);
    return z / (1.0f + z);
}

/* sf37_ops.c:18-20 */
float orc_silu(float x) { return x * orc_sigmoid(x); }

/* sf37_ops.c:22-28: double sum of squares, scale = 1/sqrtf(mean + eps). */
void orc_rms_norm_weight1(float *out, const float *x, const float *w, uint64_t n,
                          float eps) {
    double ss = 0.0;
    for (uint64_t i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float scale = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * scale * (w[i] + 1.0f);
}

/* Same with bf16 weights (sf37.c:2211-2212 converts the bf16 norm weight). */
void orc_rms_norm_weight1_bf16(float *out, const float *x, const uint16_t *w,
                               uint64_t n, float eps) {
    double ss = 0.0;
    for (uint64_t i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float scale = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * scale * (orc_bf16_to_f32(w[i]) + 1.0f);
}

/* sf37_ops.c:30-42 */
void orc_swiglu(float *out, const float *gate, const float *up, uint64_t n,
                float clamp) {
    for (uint64_t i = 0; i < n; i++) {
        float g = gate[i], u = up[i];
        if (clamp > 1.0e-6f) {
            if (g > clamp) g = clamp;
            if (u > clamp) u = clamp;
            if (u < -clamp) u = -clamp;
        }
        out[i] = orc_silu(g) * u;
    }
}

/* sf37_ops.c:44-55: insertion top-k, strict '>' so ties keep the lower index. */
void orc_topk_desc(const float *score, int n, int k, int *idx) {
    for (int i = 0; i < k; i++) idx[i] = -1;
    for (int i = 0; i < n; i++) {
        for (int j = 0; j < k; j++) {
            if (idx[j] < 0 || score[i] > score[idx[j]]) {
                for (int m = k - 1; m > j; m--) idx[m] = idx[m - 1];
                idx[j] = i;
                break;
            }
        }
    }
}

/* sf37_ops.c:57-90: per 32 values d = amax/127, iscale = 1/d,
 * q = clamp(lrintf(iscale * x)); an all-zero block gets d = 0. */
void orc_q8_0_quantize_activation(const float *x, int8_t *xq, float *scale,
                                  uint64_t n) {
    const uint64_t blocks = (n + 31u) / 32u;
    for (uint64_t b = 0; b < blocks; b++) {
        const uint64_t off = b * 32u;
        uint64_t len = n - off;
        if (len > 32u) len = 32u;
        float amax = 0.0f;
        for (uint64_t i = 0; i < len; i++) {
            const float a = fabsf(x[off + i]);
            if (a > amax) amax = a;
        }
        if (amax == 0.0f) {
            scale[b] = 0.0f;
            memset(xq + off, 0, 32);
            continue;
        }
        const float d = amax / 127.0f;
        const float iscale = 1.0f / d;
        scale[b] = d;
        for (uint64_t i = 0; i < len; i++) {
            long v = lrintf(iscale * x[off + i]);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            xq[off + i] = (int8_t)v;
        }
        for (uint64_t i = len; i < 32u; i++) xq[off + i] = 0;
    }
}

/* sf37_ops.c:92-108: acc += ((float)isum * wscale) * xscale, sequential. */
float orc_q8_0_row_dot_prequant(const uint8_t *row, const int8_t *xq,
                                const float *xscale, uint64_t in_dim) {
    const uint64_t blocks = (in_dim + 31u) / 32u;
    float acc = 0.0f;
    for (uint64_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * ORC_Q8_0_BLOCK;
        const float ws = orc_f16_to_f32(rd16(blk));
        uint64_t len = in_dim - b * 32u;
        if (len > 32u) len = 32u;
        int isum = 0;
        for (uint64_t i = 0; i < len; i++) isum += (int)(int8_t)blk[2 + i] * (int)xq[b * 32u + i];
        acc += (float)isum * ws * xscale[b];
    }
    return acc;
}

/* sf37_ops.c:110-125 */
void orc_q8_0_matvec(float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim,
                     const float *x) {
    const uint64_t blocks = (in_dim + 31u) / 32u;
    int8_t *xq = malloc(blocks * 32u);
    float *xs = malloc(blocks * sizeof(float));
    if (!xq || !xs) abort();
    orc_q8_0_quantize_activation(x, xq, xs, in_dim);
    for (uint64_t r = 0; r < out_dim; r++)
        out[r] = orc_q8_0_row_dot_prequant(w + r * blocks * ORC_Q8_0_BLOCK, xq, xs, in_dim);
    free(xs);
    free(xq);
}

/* sf37_ops.c:127-141 */
void orc_q8_0_matvec_pair(float *out0, float *out1, const uint8_t *w0,
                          const uint8_t *w1, uint64_t in_dim, uint64_t out_dim,
                          const float *x) {
    const uint64_t blocks = (in_dim + 31u) / 32u;
    int8_t *xq = malloc(blocks * 32u);
    float *xs = malloc(blocks * sizeof(float));
    if (!xq || !xs) abort();
    orc_q8_0_quantize_activation(x, xq, xs, in_dim);
    for (uint64_t r = 0; r < out_dim; r++) {
        out0[r] = orc_q8_0_row_dot_prequant(w0 + r * blocks * ORC_Q8_0_BLOCK, xq, xs, in_dim);
        out1[r] = orc_q8_0_row_dot_prequant(w1 + r * blocks * ORC_Q8_0_BLOCK, xq, xs, in_dim);
    }
    free(xs);
    free(xq);
}

/* sf37_ops.c:143-151 */
void orc_bf16_matvec(float *out, const uint16_t *w, uint64_t in_dim, uint64_t out_dim,
                     const float *x) {
    for (uint64_t r = 0; r < out_dim; r++) {
        double acc = 0.0;
        for (uint64_t i = 0; i < in_dim; i++) acc += (double)orc_bf16_to_f32(w[r * in_dim + i]) * x[i];
        out[r] = (float)acc;
    }
}

/* sf37_ops.c:153-165 */
void orc_q3_matvec(float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim,
                   const float *x) {
    const uint64_t nb = in_dim / ORC_QK_K;
    for (uint64_t r = 0; r < out_dim; r++) {
        float acc = 0.0f;
        for (uint64_t b = 0; b < nb; b++)
            acc += orc_q3_block_dot(w + (r * nb + b) * ORC_Q3_BLOCK, x + b * ORC_QK_K);
        out[r] = acc;
    }
}

/* sf37_ops.c:167-179 */
void orc_q2_matvec(float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim,
                   const float *x) {
    const uint64_t nb = in_dim / ORC_QK_K;
    for (uint64_t r = 0; r < out_dim; r++) {
        float acc = 0.0f;
        for (uint64_t b = 0; b < nb; b++)
            acc += orc_q2_block_dot(w + (r * nb + b) * ORC_Q2_BLOCK, x + b * ORC_QK_K);
        out[r] = acc;
    }
}

/* F32 dense matvec with a double accumulator, sf37.c:1970-1976. */
void orc_f32_matvec_double(float *out, const float *w, uint64_t in_dim,
                           uint64_t out_dim, const float *x) {
    for (uint64_t r = 0; r < out_dim; r++) {
        double acc = 0.0;
        for (uint64_t i = 0; i < in_dim; i++) acc += (double)w[r * in_dim + i] * x[i];
        out[r] = (float)acc;
    }
}

/* ===================================================================== */
/* Q8_K activation path (sf37_cuda.cu:4149-4503)                          */
/* ===================================================================== */

/* sf37_cuda.cu:4168-4205 with IEEE division: per 256 values d = amax/127,
 * id = d != 0 ? 1/d : 0, qs = clamp(lrintf(x*id)), gsums[g] = sum of the
 * g-th 64 codes.  (When amax < 2^-121 the reciprocal overflows and the
 * reference's lrintf(inf) is undefined; the clamp-in-float form used here
 * gives the saturated code instead.) */
void orc_q8k_quantize(orc_q8k *out, const float *x, uint32_t in_dim, uint32_t n_rows) {
    const uint32_t nb = in_dim / ORC_QK_K;
    for (uint32_t r = 0; r < n_rows; r++) {
        for (uint32_t b = 0; b < nb; b++) {
            const float *xb = x + (uint64_t)r * in_dim + (uint64_t)b * ORC_QK_K;
            orc_q8k *y = out + (uint64_t)r * nb + b;
            float amax = 0.0f;
            for (int i = 0; i < ORC_QK_K; i++) amax = fmaxf(amax, fabsf(xb[i]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            y->d = d;
            for (int i = 0; i < ORC_QK_K; i++) {
                /* round half-even, clamp in float: equal to clamp(lrintf(.)) for
                 * every finite product; defined (127/-128) when 1/d overflowed */
                const float q = fminf(fmaxf(rintf(xb[i] * id), -128.0f), 127.0f);
                y->qs[i] = (int8_t)(int)q;
            }
            for (int g = 0; g < 4; g++) {
                int s = 0;
                for (int i = 0; i < 64; i++) s += y->qs[64 * g + i];
                y->gsums[g] = (int16_t)s;
            }
        }
    }
}

/* Exact integer part of one 64-wide group: sum(q * qs) - zp * gsum, the
 * dp4a loop plus correction of sf37_cuda.cu:4226-4249 (Q3, zp & 7). */
int32_t orc_q3_group_idot(const uint8_t *blk, int g, const orc_q8k *xq) {
    const uint8_t *pl = blk + 12 + 24 * g;
    int32_t dot = 0;
    for (int i = 0; i < 64; i++) dot += (int32_t)orc_q3_get(pl, i) * xq->qs[64 * g + i];
    return dot - (int32_t)(blk[8 + g] & 7u) * xq->gsums[g];
}

/* sf37_cuda.cu:4251-4274 (Q2, zp & 3). */
int32_t orc_q2_group_idot(const uint8_t *blk, int g, const orc_q8k *xq) {
    const uint8_t *pl = blk + 12 + 16 * g;
    int32_t dot = 0;
    for (int i = 0; i < 64; i++) dot += (int32_t)q2_get(pl, i) * xq->qs[64 * g + i];
    return dot - (int32_t)(blk[8 + g] & 3u) * xq->gsums[g];
}

/*
 * Canonical float order of a Q3/Q2 x Q8_K row dot.  The reference kernel
 * (sf37_cuda.cu:4226-4274, 4369-4405) sums scale*d*I per group and then
 * reduces across lanes, an order that differs per kernel.  This build fixes
 * one order that every HIP kernel (decode GEMV and prefill MFMA) reproduces:
 *   blk_b = fma(s3, I3, fma(s2, I2, fma(s1, I1, fma(s0, I0, 0))))
 *   acc   = fma(d_b, blk_b, acc)      for b = 0, 1, ..., nblk-1
 * The integers I_g are exact, so results are bit-identical across kernels.
 */
float orc_q3_q8k_row_dot(const uint8_t *row, const orc_q8k *xq, uint32_t nblk) {
    float acc = 0.0f;
    for (uint32_t b = 0; b < nblk; b++) {
        const uint8_t *blk = row + (uint64_t)b * ORC_Q3_BLOCK;
        float bs = 0.0f;
        for (int g = 0; g < 4; g++)
            bs = fmaf(orc_f16_to_f32(rd16(blk + 2 * g)), (float)orc_q3_group_idot(blk, g, &xq[b]), bs);
        acc = fmaf(xq[b].d, bs, acc);
    }
    return acc;
}

float orc_q2_q8k_row_dot(const uint8_t *row, const orc_q8k *xq, uint32_t nblk) {
    float acc = 0.0f;
    for (uint32_t b = 0; b < nblk; b++) {
        const uint8_t *blk = row + (uint64_t)b * ORC_Q2_BLOCK;
        float bs = 0.0f;
        for (int g = 0; g < 4; g++)
            bs = fmaf(orc_f16_to_f32(rd16(blk + 2 * g)), (float)orc_q2_group_idot(blk, g, &xq[b]), bs);
        acc = fmaf(xq[b].d, bs, acc);
    }
    return acc;
}

/* Q8_K GEMVs, sf37_cuda.cu:5783-5841 (q8k branch). */
void orc_q3_q8k_matvec(float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim,
                       const float *x) {
    const uint32_t nb = (uint32_t)(in_dim / ORC_QK_K);
    orc_q8k *xq = malloc(sizeof(orc_q8k) * nb);
    if (!xq) abort();
    orc_q8k_quantize(xq, x, (uint32_t)in_dim, 1);
    for (uint64_t r = 0; r < out_dim; r++) out[r] = orc_q3_q8k_row_dot(w + r * nb * ORC_Q3_BLOCK, xq, nb);
    free(xq);
}

void orc_q2_q8k_matvec(float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim,
                       const float *x) {
    const uint32_t nb = (uint32_t)(in_dim / ORC_QK_K);
    orc_q8k *xq = malloc(sizeof(orc_q8k) * nb);
    if (!xq) abort();
    orc_q8k_quantize(xq, x, (uint32_t)in_dim, 1);
    for (uint64_t r = 0; r < out_dim; r++) out[r] = orc_q2_q8k_row_dot(w + r * nb * ORC_Q2_BLOCK, xq, nb);
    free(xq);
}

/* SwiGLU with clamp times the routing weight, sf37_cuda.cu:4444-4456:
 * ((g * sigmoid(g)) * u) * w, left to right. */
float orc_swiglu_mid(float gate, float up, float w, float clamp) {
    if (clamp > 1.0e-6f) {
        if (gate > clamp) gate = clamp;
        if (up > clamp) up = clamp;
        if (up < -clamp) up = -clamp;
    }
    return gate * orc_sigmoid(gate) * up * w;
}

/* ===================================================================== */
/* Router (sf37.c:2144-2157, sf37_cuda.cu:4866-4910)                      */
/* ===================================================================== */

void orc_router_select(int32_t *selected, float *weights, float *probs,
                       const float *logits, const float *bias, uint32_t n_experts,
                       uint32_t topk, float scale) {
    int32_t idx[64];
    float bscore[64], bprob[64];
    for (uint32_t j = 0; j < topk; j++) { idx[j] = -1; bscore[j] = -INFINITY; bprob[j] = 0.0f; }
    for (uint32_t e = 0; e < n_experts; e++) {
        const float p = orc_sigmoid(logits[e]);
        if (probs) probs[e] = p;
        const float s = p + bias[e];
        for (uint32_t j = 0; j < topk; j++) {
            if (idx[j] < 0 || s > bscore[j]) {
                for (uint32_t m = topk - 1; m > j; m--) {
                    idx[m] = idx[m - 1];
                    bscore[m] = bscore[m - 1];
                    bprob[m] = bprob[m - 1];
                }
                idx[j] = (int32_t)e;
                bscore[j] = s;
                bprob[j] = p;
                break;
            }
        }
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < topk; j++) sum += bprob[j];
    if (sum < 1.0e-20f) sum = 1.0e-20f;
    for (uint32_t j = 0; j < topk; j++) {
        selected[j] = idx[j];
        weights[j] = bprob[j] / sum * scale;
    }
}

/* sf37_cuda.cu:7803-7889 / 7891-7966: one token per row. */
void orc_router_select_batch(int32_t *selected, float *weights, float *probs,
                             const float *logits, const float *bias, uint32_t n_experts,
                             uint32_t topk, float scale, uint32_t n_tok) {
    for (uint32_t t = 0; t < n_tok; t++)
        orc_router_select(selected + (uint64_t)t * topk, weights + (uint64_t)t * topk,
                          probs ? probs + (uint64_t)t * n_experts : NULL,
                          logits + (uint64_t)t * n_experts, bias, n_experts, topk, scale);
}

/* ===================================================================== */
/* Routed experts                                                         */
/* ===================================================================== */

static uint32_t clamp_expert(int32_t e, uint32_t n) {
    return (e < 0 || (uint32_t)e >= n) ? 0u : (uint32_t)e; /* sf37_cuda.cu:4428-4429 */
}

void orc_routed_moe_one_q8k(float *out, float *mid_out, orc_q8k *midq_out,
                            const uint8_t *gate_w, const uint8_t *up_w,
                            const uint8_t *down_w, const int32_t *selected,
                            const float *weights, uint32_t n_total_expert,
                            uint32_t topk, uint32_t in_dim, uint32_t mid_dim,
                            uint32_t out_dim, float clamp, const float *x) {
    const uint32_t xb = in_dim / ORC_QK_K, mb = mid_dim / ORC_QK_K;
    const uint64_t g_row = (uint64_t)xb * ORC_Q3_BLOCK, d_row = (uint64_t)mb * ORC_Q2_BLOCK;
    orc_q8k *xq = malloc(sizeof(orc_q8k) * xb);
    orc_q8k *mq = malloc(sizeof(orc_q8k) * (uint64_t)mb * topk);
    float *mid = malloc(sizeof(float) * (uint64_t)mid_dim * topk);
    if (!xq || !mq || !mid) abort();
    orc_q8k_quantize(xq, x, in_dim, 1);
    for (uint32_t s = 0; s < topk; s++) {
        const uint32_t e = clamp_expert(selected[s], n_total_expert);
        const uint8_t *ge = gate_w + (uint64_t)e * mid_dim * g_row;
        const uint8_t *ue = up_w + (uint64_t)e * mid_dim * g_row;
        for (uint32_t r = 0; r < mid_dim; r++) {
            const float g = orc_q3_q8k_row_dot(ge + r * g_row, xq, xb);
            const float u = orc_q3_q8k_row_dot(ue + r * g_row, xq, xb);
            mid[(uint64_t)s * mid_dim + r] = orc_swiglu_mid(g, u, weights[s], clamp);
        }
    }
    orc_q8k_quantize(mq, mid, mid_dim, topk);
    for (uint32_t r = 0; r < out_dim; r++) {
        float total = 0.0f;
        for (uint32_t s = 0; s < topk; s++) {
            const uint32_t e = clamp_expert(selected[s], n_total_expert);
            const uint8_t *row = down_w + ((uint64_t)e * out_dim + r) * d_row;
            total = total + orc_q2_q8k_row_dot(row, mq + (uint64_t)s * mb, mb);
        }
        out[r] = total;
    }
    if (mid_out) memcpy(mid_out, mid, sizeof(float) * (uint64_t)mid_dim * topk);
    if (midq_out) memcpy(midq_out, mq, sizeof(orc_q8k) * (uint64_t)mb * topk);
    free(mid);
    free(mq);
    free(xq);
}

void orc_routed_moe_one_f32(float *out, float *mid_out, const uint8_t *gate_w,
                            const uint8_t *up_w, const uint8_t *down_w,
                            const int32_t *selected, const float *weights,
                            uint32_t n_total_expert, uint32_t topk, uint32_t in_dim,
                            uint32_t mid_dim, uint32_t out_dim, float clamp,
                            const float *x) {
    const uint64_t g_row = (uint64_t)(in_dim / ORC_QK_K) * ORC_Q3_BLOCK;
    const uint64_t d_row = (uint64_t)(mid_dim / ORC_QK_K) * ORC_Q2_BLOCK;
    float *g = malloc(sizeof(float) * mid_dim), *u = malloc(sizeof(float) * mid_dim);
    float *mid = malloc(sizeof(float) * mid_dim), *down = malloc(sizeof(float) * out_dim);
    if (!g || !u || !mid || !down) abort();
    for (uint32_t r = 0; r < out_dim; r++) out[r] = 0.0f;
    for (uint32_t s = 0; s < topk; s++) {
        const uint32_t e = clamp_expert(selected[s], n_total_expert);
        orc_q3_matvec(g, gate_w + (uint64_t)e * mid_dim * g_row, in_dim, mid_dim, x);
        orc_q3_matvec(u, up_w + (uint64_t)e * mid_dim * g_row, in_dim, mid_dim, x);
        orc_swiglu(mid, g, u, mid_dim, clamp);
        for (uint32_t i = 0; i < mid_dim; i++) mid[i] *= weights[s];
        if (mid_out) memcpy(mid_out + (uint64_t)s * mid_dim, mid, sizeof(float) * mid_dim);
        orc_q2_matvec(down, down_w + (uint64_t)e * out_dim * d_row, mid_dim, out_dim, mid);
        for (uint32_t r = 0; r < out_dim; r++) out[r] += down[r];
    }
    free(down);
    free(mid);
    free(u);
    free(g);
}

/* Counting sort of pairs by expert; within an expert pairs keep ascending
 * pair id (pair = tok * topk + slot, sf37_cuda.cu:4601-4602). */
void orc_moe_dispatch(const int32_t *selected, uint32_t n_pairs, uint32_t n_total_expert,
                      uint32_t *counts, uint32_t *offsets, uint32_t *sorted_pairs) {
    for (uint32_t e = 0; e < n_total_expert; e++) counts[e] = 0;
    for (uint32_t p = 0; p < n_pairs; p++) counts[clamp_expert(selected[p], n_total_expert)]++;
    uint32_t sum = 0;
    for (uint32_t e = 0; e < n_total_expert; e++) { offsets[e] = sum; sum += counts[e]; }
    offsets[n_total_expert] = sum;
    uint32_t *cur = malloc(sizeof(uint32_t) * (n_total_expert ? n_total_expert : 1));
    if (!cur) abort();
    for (uint32_t e = 0; e < n_total_expert; e++) cur[e] = offsets[e];
    for (uint32_t p = 0; p < n_pairs; p++) sorted_pairs[cur[clamp_expert(selected[p], n_total_expert)]++] = p;
    free(cur);
}

/* Batch path: identical per-pair arithmetic to the one-token path and a
 * slot-order combine per token (sf37_cuda.cu:4850-4864). */
void orc_routed_moe_batch_q8k(float *out, float *mid_out, const uint8_t *gate_w,
                              const uint8_t *up_w, const uint8_t *down_w,
                              const int32_t *selected, const float *weights,
                              uint32_t n_total_expert, uint32_t topk, uint32_t in_dim,
                              uint32_t mid_dim, uint32_t out_dim, float clamp,
                              const float *x, uint32_t n_tok) {
    for (uint32_t t = 0; t < n_tok; t++)
        orc_routed_moe_one_q8k(out + (uint64_t)t * out_dim,
                               mid_out ? mid_out + (uint64_t)t * topk * mid_dim : NULL, NULL,
                               gate_w, up_w, down_w, selected + (uint64_t)t * topk,
                               weights + (uint64_t)t * topk, n_total_expert, topk, in_dim,
                               mid_dim, out_dim, clamp, x + (uint64_t)t * in_dim);
}

/* ===================================================================== */
/* Shared expert and layer composition                                    */
/* ===================================================================== */

/* sf37.c:2159-2167 */
void orc_shared_expert_q8_0(float *out, float *mid_out, const uint8_t *gate_w,
                            const uint8_t *up_w, const uint8_t *down_w, uint32_t in_dim,
                            uint32_t mid_dim, uint32_t out_dim, float clamp,
                            const float *x) {
    float *g = malloc(sizeof(float) * mid_dim), *u = malloc(sizeof(float) * mid_dim);
    float *mid = malloc(sizeof(float) * mid_dim);
    if (!g || !u || !mid) abort();
    orc_q8_0_matvec_pair(g, u, gate_w, up_w, in_dim, mid_dim, x);
    orc_swiglu(mid, g, u, mid_dim, clamp);
    orc_q8_0_matvec(out, down_w, mid_dim, out_dim, mid);
    if (mid_out) memcpy(mid_out, mid, sizeof(float) * mid_dim);
    free(mid);
    free(u);
    free(g);
}

void orc_moe_layer_q8k(float *out, int32_t *selected_out, float *weights_out,
                       const float *router_w, const float *router_bias,
                       const float *logits_in, const uint8_t *gate_w,
                       const uint8_t *up_w, const uint8_t *down_w,
                       const uint8_t *sh_gate, const uint8_t *sh_up,
                       const uint8_t *sh_down, uint32_t n_expert, uint32_t topk,
                       uint32_t in_dim, uint32_t mid_dim, float clamp_routed,
                       float clamp_shared, float scale, const float *x,
                       uint32_t n_tok) {
    float *logits = malloc(sizeof(float) * n_expert);
    float *routed = malloc(sizeof(float) * in_dim);
    int32_t *sel = malloc(sizeof(int32_t) * topk);
    float *w = malloc(sizeof(float) * topk);
    if (!logits || !routed || !sel || !w) abort();
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *xt = x + (uint64_t)t * in_dim;
        float *ot = out + (uint64_t)t * in_dim;
        if (logits_in) memcpy(logits, logits_in + (uint64_t)t * n_expert, sizeof(float) * n_expert);
        else orc_f32_matvec_double(logits, router_w, in_dim, n_expert, xt);
        orc_router_select(sel, w, NULL, logits, router_bias, n_expert, topk, scale);
        orc_shared_expert_q8_0(ot, NULL, sh_gate, sh_up, sh_down, in_dim, mid_dim, in_dim,
                               clamp_shared, xt);
        orc_routed_moe_one_q8k(routed, NULL, NULL, gate_w, up_w, down_w, sel, w, n_expert,
                               topk, in_dim, mid_dim, in_dim, clamp_routed, xt);
        for (uint32_t i = 0; i < in_dim; i++) ot[i] = ot[i] + routed[i]; /* sf37.c:3428 */
        if (selected_out) memcpy(selected_out + (uint64_t)t * topk, sel, sizeof(int32_t) * topk);
        if (weights_out) memcpy(weights_out + (uint64_t)t * topk, w, sizeof(float) * topk);
    }
    free(w);
    free(sel);
    free(routed);
    free(logits);
}

/* ===================================================================== */
/* Synthetic inputs (harness)                                             */
/* ===================================================================== */

static uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}

/* Counter-based generator: a splitmix64 sequence keyed by (seed, stream),
 * evaluated at position index, so any element can be drawn independently. */
uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t key = mix64(seed ^ mix64(stream + 0x9e3779b97f4a7c15ULL));
    return mix64(key + (index + 1u) * 0x9e3779b97f4a7c15ULL);
}

/* ln(u) for u in (0,1): u = m * 2^e with m in [sqrt(1/2), sqrt(2)),
 * ln m = 2s(1 + s^2/3 + ... + s^10/11), s = (m-1)/(m+1). */
static float synth_ln(float u) {
    uint32_t b = f2u(u);
    int e = (int)((b >> 23) & 0xff) - 127;
    float m = u2f((b & 0x7fffffu) | 0x3f800000u);
    if (m > 0x1.6a09e6p+0f) { m = m * 0.5f; e += 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 0x1.745d18p-4f;
    p = fmaf(p, s2, 0x1.c71c72p-4f);
    p = fmaf(p, s2, 0x1.24924ap-3f);
    p = fmaf(p, s2, 0x1.99999ap-3f);
    p = fmaf(p, s2, 0x1.555556p-2f);
    p = fmaf(p, s2, 1.0f);
    return fmaf((float)e, 0x1.62e430p-1f, (2.0f * s) * p);
}

/* cos(2*pi*t) for t in [-1/2, 1/2): Taylor series in y = t^2. */
static float synth_cos2pi(float t) {
    const float y = t * t;
    float p = 0x1.ef6e30p-9f;
    p = fmaf(p, y, -0x1.2a0c5ap-5f);
    p = fmaf(p, y, 0x1.20c62cp-2f);
    p = fmaf(p, y, -0x1.b6e250p+0f);
    p = fmaf(p, y, 0x1.f9d38ap+2f);
    p = fmaf(p, y, -0x1.a6d1f2p+4f);
    p = fmaf(p, y, 0x1.e1f506p+5f);
    p = fmaf(p, y, -0x1.55d3c8p+6f);
    p = fmaf(p, y, 0x1.03c1f0p+6f);
    p = fmaf(p, y, -0x1.3bd3ccp+4f);
    return fmaf(p, y, 1.0f);
}

/* Box-Muller from one 64-bit draw with only IEEE +,-,*,/,sqrt and the
 * polynomials above, so the HIP generator reproduces it bit-for-bit. */
float orc_rng_normal(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t z = orc_rng_u64(seed, stream, index);
    const float u1 = ((float)(uint32_t)(z >> 40) + 0.5f) * 0x1p-24f;
    const float u2 = (float)(uint32_t)((z >> 16) & 0xffffffu) * 0x1p-24f;
    const float r = sqrtf(-2.0f * synth_ln(u1));
    return r * -synth_cos2pi(u2 - 0.5f);
}

void orc_fill_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                     uint64_t index0, float sigma) {
    for (uint64_t i = 0; i < n; i++) dst[i] = sigma * orc_rng_normal(seed, stream, index0 + i);
}

void orc_gen_quant_rows(int type, uint8_t *dst, uint64_t row0, uint64_t nrows,
                        uint64_t ncols, uint64_t seed, uint64_t stream, float sigma) {
    const uint64_t qk = type == 0 ? 32 : ORC_QK_K;
    const uint64_t bs = type == 0 ? ORC_Q8_0_BLOCK : (type == 3 ? ORC_Q3_BLOCK : ORC_Q2_BLOCK);
    float *row = malloc(sizeof(float) * ncols);
    if (!row) abort();
    for (uint64_t r = 0; r < nrows; r++) {
        orc_fill_normal(row, ncols, seed, stream, (row0 + r) * ncols, sigma);
        orc_quantize_rows(type, row, dst + r * (ncols / qk) * bs, 1, (int64_t)ncols);
    }
    free(row);
}

/* Host libm expf / the engine sigmoid over an array (checker for the
 * device exp; sf37_ops.c:9-16). */
void orc_expf_array(float *out, const float *x, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = expf(x[i]);
}

void orc_sigmoid_array(float *out, const float *x, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_sigmoid(x[i]);
}
