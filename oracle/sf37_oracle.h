/*
 * sf37_oracle.h - CPU restatement of the SF37 MoE feed-forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in sf37_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the ZephinueCode/sf37 repository root).  Arithmetic is IEEE-754 binary32 /
 * binary64 with no floating-point contraction (the file is built with
 * -ffp-contract=off and no fast-math); where a fused multiply-add is part of
 * the canonical order it is written explicitly as fmaf()/fma().
 *
 * Two families of semantics live here:
 *   - "fp32" : the CPU engine path (sf37_ops.c / sf37_quant.c / sf37.c) that
 *              feeds fp32 activations to the Q3/Q2 dot products;
 *   - "q8k"  : the accelerator path (sf37_cuda.cu) that first quantizes the
 *              activations to 256-wide Q8_K blocks and runs integer dots with
 *              a zero-point correction.  Its float epilogue is fixed here to
 *              one canonical order (orc_q3_q8k_row_dot) that the HIP kernels
 *              reproduce bit-for-bit.
 */
#ifndef SF37_ORACLE_H
#define SF37_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_Q8_0_BLOCK 34
#define ORC_Q3_BLOCK 110
#define ORC_Q2_BLOCK 84

/* Q8_K activation block, byte layout of sf37_cuda.cu:4162-4166 (268 bytes). */
typedef struct {
    float d;
    int8_t qs[ORC_QK_K];
    int16_t gsums[4];
} orc_q8k;

/* ---- scalar formats ---------------------------------------------------- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
int orc_nearest_int(float v);

/* ---- block decode / fp32 dot (sf37_quant.c) ---------------------------- */
void orc_q8_0_block_decode(const uint8_t *blk, float *dst32);
float orc_q8_0_block_dot(const uint8_t *blk, const float *x32);
void orc_q3_block_decode(const uint8_t *blk, float *dst256);
void orc_q2_block_decode(const uint8_t *blk, float *dst256);
float orc_q3_block_dot(const uint8_t *blk, const float *x256);
float orc_q2_block_dot(const uint8_t *blk, const float *x256);
uint32_t orc_q3_get(const uint8_t *payload, int i);

/* ---- reference weight quantizer (gguf-tools/quants.c) ------------------ */
void orc_quantize_q3_block(const float *x256, uint8_t *out110);
void orc_quantize_q2_block(const float *x256, uint8_t *out84);
void orc_quantize_q8_0_block(const float *x32, uint8_t *out34);
/* type: 0 = Q8_0, 2 = Q2 asym, 3 = Q3 asym; rows of ncols floats. */
void orc_quantize_rows(int type, const float *src, uint8_t *dst,
                       int64_t nrows, int64_t ncols);

/* ---- CPU ops (sf37_ops.c) ---------------------------------------------- */
float orc_sigmoid(float x);
float orc_silu(float x);
void orc_rms_norm_weight1(float *out, const float *x, const float *w,
                          uint64_t n, float eps);
void orc_rms_norm_weight1_bf16(float *out, const float *x, const uint16_t *w,
                               uint64_t n, float eps);
void orc_swiglu(float *out, const float *gate, const float *up, uint64_t n,
                float clamp);
void orc_topk_desc(const float *score, int n, int k, int *idx);
void orc_q8_0_quantize_activation(const float *x, int8_t *xq, float *scale,
                                  uint64_t n);
float orc_q8_0_row_dot_prequant(const uint8_t *row, const int8_t *xq,
                                const float *xscale, uint64_t in_dim);
void orc_q8_0_matvec(float *out, const uint8_t *w, uint64_t in_dim,
                     uint64_t out_dim, const float *x);
void orc_q8_0_matvec_pair(float *out0, float *out1, const uint8_t *w0,
                          const uint8_t *w1, uint64_t in_dim, uint64_t out_dim,
                          const float *x);
void orc_bf16_matvec(float *out, const uint16_t *w, uint64_t in_dim,
                     uint64_t out_dim, const float *x);
void orc_q3_matvec(float *out, const uint8_t *w, uint64_t in_dim,
                   uint64_t out_dim, const float *x);
void orc_q2_matvec(float *out, const uint8_t *w, uint64_t in_dim,
                   uint64_t out_dim, const float *x);
void orc_f32_matvec_double(float *out, const float *w, uint64_t in_dim,
                           uint64_t out_dim, const float *x);

/* ---- Q8_K activation path (sf37_cuda.cu) ------------------------------- */
void orc_q8k_quantize(orc_q8k *out, const float *x, uint32_t in_dim,
                      uint32_t n_rows);
int32_t orc_q3_group_idot(const uint8_t *blk, int g, const orc_q8k *xq);
int32_t orc_q2_group_idot(const uint8_t *blk, int g, const orc_q8k *xq);
float orc_q3_q8k_row_dot(const uint8_t *row, const orc_q8k *xq, uint32_t nblk);
float orc_q2_q8k_row_dot(const uint8_t *row, const orc_q8k *xq, uint32_t nblk);
void orc_q3_q8k_matvec(float *out, const uint8_t *w, uint64_t in_dim,
                       uint64_t out_dim, const float *x);
void orc_q2_q8k_matvec(float *out, const uint8_t *w, uint64_t in_dim,
                       uint64_t out_dim, const float *x);
float orc_swiglu_mid(float gate, float up, float w, float clamp);

/* ---- router (sf37.c:2144-2157, sf37_cuda.cu:4866-4997) ----------------- */
void orc_router_select(int32_t *selected, float *weights, float *probs,
                       const float *logits, const float *bias,
                       uint32_t n_experts, uint32_t topk, float scale);
void orc_router_select_batch(int32_t *selected, float *weights, float *probs,
                             const float *logits, const float *bias,
                             uint32_t n_experts, uint32_t topk, float scale,
                             uint32_t n_tok);

/* ---- routed experts ----------------------------------------------------- */
/* Q8_K path, one token (sf37_cuda.cu:5313-5380).  mid_out: [topk][mid_dim],
 * midq_out: [topk][mid_dim/256] (either may be NULL). */
void orc_routed_moe_one_q8k(float *out, float *mid_out, orc_q8k *midq_out,
                            const uint8_t *gate_w, const uint8_t *up_w,
                            const uint8_t *down_w, const int32_t *selected,
                            const float *weights, uint32_t n_total_expert,
                            uint32_t topk, uint32_t in_dim,
                            uint32_t expert_mid_dim, uint32_t out_dim,
                            float clamp, const float *x);
/* fp32-activation path, one token (sf37_cuda.cu:5382-5446 == sf37.c:2169-2181). */
void orc_routed_moe_one_f32(float *out, float *mid_out, const uint8_t *gate_w,
                            const uint8_t *up_w, const uint8_t *down_w,
                            const int32_t *selected, const float *weights,
                            uint32_t n_total_expert, uint32_t topk,
                            uint32_t in_dim, uint32_t expert_mid_dim,
                            uint32_t out_dim, float clamp, const float *x);
/* Stable per-expert dispatch (sf37_cuda.cu:4505-4544, order pinned to
 * (expert asc, pair id asc)).  counts[E], offsets[E+1], sorted[P]. */
void orc_moe_dispatch(const int32_t *selected, uint32_t n_pairs,
                      uint32_t n_total_expert, uint32_t *counts,
                      uint32_t *offsets, uint32_t *sorted_pairs);
/* Q8_K batch path (sf37_cuda.cu:5449-5733).  mid_out: [n_tok*topk][mid]. */
void orc_routed_moe_batch_q8k(float *out, float *mid_out,
                              const uint8_t *gate_w, const uint8_t *up_w,
                              const uint8_t *down_w, const int32_t *selected,
                              const float *weights, uint32_t n_total_expert,
                              uint32_t topk, uint32_t in_dim,
                              uint32_t expert_mid_dim, uint32_t out_dim,
                              float clamp, const float *x, uint32_t n_tok);

/* ---- shared expert (sf37.c:2159-2167) and whole layer ------------------- */
void orc_shared_expert_q8_0(float *out, float *mid_out, const uint8_t *gate_w,
                            const uint8_t *up_w, const uint8_t *down_w,
                            uint32_t in_dim, uint32_t mid_dim,
                            uint32_t out_dim, float clamp, const float *x);
/* One MoE layer for n_tok tokens, composed as the accelerator engine does
 * (sf37.c:3392-3430 decode, 5959-6071 prefill):
 *   logits = router . x   (skipped when logits_in != NULL: "same logits")
 *   select top-k; shared = Q8_0 shared expert; routed = Q8_K experts;
 *   out = shared + routed.
 * selected/weights may be NULL. */
void orc_moe_layer_q8k(float *out, int32_t *selected_out, float *weights_out,
                       const float *router_w, const float *router_bias,
                       const float *logits_in, const uint8_t *gate_w,
                       const uint8_t *up_w, const uint8_t *down_w,
                       const uint8_t *sh_gate, const uint8_t *sh_up,
                       const uint8_t *sh_down, uint32_t n_expert,
                       uint32_t topk, uint32_t in_dim, uint32_t mid_dim,
                       float clamp_routed, float clamp_shared, float scale,
                       const float *x, uint32_t n_tok);

void orc_expf_array(float *out, const float *x, uint64_t n);
void orc_sigmoid_array(float *out, const float *x, uint64_t n);

/* ---- synthetic inputs (harness; no reference counterpart) --------------- */
uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t index);
float orc_rng_normal(uint64_t seed, uint64_t stream, uint64_t index);
void orc_fill_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                     uint64_t index0, float sigma);
/* Quantized weight rows generated from N(0, sigma) fp32 rows:
 * element (row r, col k) of tensor (seed, stream) has counter r*ncols+k. */
void orc_gen_quant_rows(int type, uint8_t *dst, uint64_t row0, uint64_t nrows,
                        uint64_t ncols, uint64_t seed, uint64_t stream,
                        float sigma);

#ifdef __cplusplus
}
#endif

#endif
