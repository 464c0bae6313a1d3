/*
 * cpu_baseline.c - the reference CPU MoE layer for one token, for timing.
 *
 * TEST / BENCH INFRASTRUCTURE ONLY.  Composes the reference's own CPU ops
 * (sf37_ops.h / sf37_quant.h, compiled from /root/reference with the
 * reference `make cpu` flags) exactly as layer_moe_ffn does
 * (sf37.c:2127-2194), plus the F32 router matvec with a double accumulator
 * of matvec_dense_tensor (sf37.c:1970-1976), which is static in sf37.c and
 * therefore restated here.  Single-threaded, like the reference.
 *
 * Built by oracle/Makefile against the reference sources ("reference" kind)
 * or, with -DSF37CPU_PORT, against this build's restatement in
 * sf37_oracle.c ("port" kind).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef SF37CPU_PORT
#include "sf37_oracle.h"
#define OP_SIGMOID orc_sigmoid
#define OP_TOPK orc_topk_desc
#define OP_SWIGLU orc_swiglu
#define OP_Q8_PAIR orc_q8_0_matvec_pair
#define OP_Q8 orc_q8_0_matvec
#define OP_Q3 orc_q3_matvec
#define OP_Q2 orc_q2_matvec
#define Q3_BLOCK ORC_Q3_BLOCK
#define Q2_BLOCK ORC_Q2_BLOCK
#define QK ORC_QK_K
#else
#include "sf37_ops.h"
#include "sf37_quant.h"
#define OP_SIGMOID sf37_sigmoid
#define OP_TOPK sf37_topk_desc
#define OP_SWIGLU sf37_swiglu
#define OP_Q8_PAIR sf37_q8_0_matvec_pair
#define OP_Q8 sf37_q8_0_matvec
#define OP_Q3 sf37_q3_asym_matvec
#define OP_Q2 sf37_q2_asym_matvec
#define Q3_BLOCK SF37_Q3_BLOCK_SIZE
#define Q2_BLOCK SF37_Q2_BLOCK_SIZE
#define QK SF37_QK_K
#endif

/* out[in_dim] = shared + sum over the top-k experts, for one token x. */
void sf37cpu_moe_ffn_token(float *out, int32_t *sel_out, const float *router_w,
                           const float *router_bias, const uint8_t *gate_w,
                           const uint8_t *up_w, const uint8_t *down_w,
                           const uint8_t *sh_gate, const uint8_t *sh_up,
                           const uint8_t *sh_down, uint32_t n_expert, uint32_t topk,
                           uint32_t in_dim, uint32_t mid_dim, float clamp_routed,
                           float clamp_shared, const float *x) {
    float *logits = malloc(sizeof(float) * n_expert);
    float *prob = malloc(sizeof(float) * n_expert);
    float *score = malloc(sizeof(float) * n_expert);
    float *g = malloc(sizeof(float) * mid_dim);
    float *u = malloc(sizeof(float) * mid_dim);
    float *mid = malloc(sizeof(float) * mid_dim);
    float *down = malloc(sizeof(float) * in_dim);
    int sel[64];
    float w[64];
    if (!logits || !prob || !score || !g || !u || !mid || !down || topk > 64) abort();

    for (uint32_t r = 0; r < n_expert; r++) {
        double acc = 0.0;
        for (uint32_t i = 0; i < in_dim; i++) acc += (double)router_w[(uint64_t)r * in_dim + i] * x[i];
        logits[r] = (float)acc;
    }
    for (uint32_t i = 0; i < n_expert; i++) {
        prob[i] = OP_SIGMOID(logits[i]);
        score[i] = prob[i] + router_bias[i];
    }
    OP_TOPK(score, (int)n_expert, (int)topk, sel);
    float sum = 0.0f;
    for (uint32_t i = 0; i < topk; i++) {
        w[i] = prob[sel[i]];
        sum += w[i];
    }
    if (sum < 1.0e-20f) sum = 1.0e-20f;
    for (uint32_t i = 0; i < topk; i++) w[i] = w[i] / sum * 3.0f;

    OP_Q8_PAIR(g, u, sh_gate, sh_up, in_dim, mid_dim, x);
    OP_SWIGLU(mid, g, u, mid_dim, clamp_shared);
    OP_Q8(out, sh_down, mid_dim, in_dim, mid);

    const uint64_t g_bytes = (uint64_t)mid_dim * (in_dim / QK) * Q3_BLOCK;
    const uint64_t d_bytes = (uint64_t)in_dim * (mid_dim / QK) * Q2_BLOCK;
    for (uint32_t i = 0; i < topk; i++) {
        const uint64_t e = (uint64_t)sel[i];
        OP_Q3(g, gate_w + e * g_bytes, in_dim, mid_dim, x);
        OP_Q3(u, up_w + e * g_bytes, in_dim, mid_dim, x);
        OP_SWIGLU(mid, g, u, mid_dim, clamp_routed);
        for (uint32_t j = 0; j < mid_dim; j++) mid[j] *= w[i];
        OP_Q2(down, down_w + e * d_bytes, mid_dim, in_dim, mid);
        for (uint32_t j = 0; j < in_dim; j++) out[j] += down[j];
        if (sel_out) sel_out[i] = sel[i];
    }
    free(down);
    free(mid);
    free(u);
    free(g);
    free(score);
    free(prob);
    free(logits);
}
