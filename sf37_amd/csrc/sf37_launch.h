/*
 * sf37_launch.h - C-linkage kernel launchers shared by sf37_hip.c (host C)
 * and the .hip kernel files.  Plain pointers and sizes only; every launcher
 * enqueues on the given stream and returns a hipError_t as int (0 = ok).
 * Shapes are validated by the callers in sf37_hip.c before any launch.
 */
#ifndef SF37_LAUNCH_H
#define SF37_LAUNCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *sf37_stream_t;

/* Q8_K activations (268-byte blocks, natural element order). */
int sf37k_q8k_quantize(void *out, const float *x, uint32_t in_dim, uint32_t n_rows,
                       sf37_stream_t s);
/* Q3/Q2 x Q8_K GEMV (canonical order) from a pre-quantized activation. */
int sf37k_q3_q8k_matvec(float *out, const uint8_t *w, const void *xq, uint32_t nblk,
                        uint64_t out_dim, sf37_stream_t s);
int sf37k_q2_q8k_matvec(float *out, const uint8_t *w, const void *xq, uint32_t nblk,
                        uint64_t out_dim, sf37_stream_t s);
/* fp32-activation Q3/Q2 GEMV (the reference's small-shape path). */
int sf37k_q3_f32_matvec(float *out, const uint8_t *w, const float *x, uint64_t in_dim,
                        uint64_t out_dim, sf37_stream_t s);
int sf37k_q2_f32_matvec(float *out, const uint8_t *w, const float *x, uint64_t in_dim,
                        uint64_t out_dim, sf37_stream_t s);

/* fp32 dense GEMV/GEMM with binary64 accumulation (router logits).  Above
 * 16 tokens the product may be split over K: part (at least
 * sf37k_f32_matmul_part_bytes bytes) then holds the slices' binary64 partial
 * sums; with part NULL or smaller the product runs unsplit.  With
 * slices_left non-NULL a split product leaves its slices in part (count in
 * *slices_left, out not written) for sf37k_router_select_part to add. */
uint64_t sf37k_f32_matmul_part_bytes(uint64_t in_dim, uint64_t out_dim, uint64_t n_tok);
int sf37k_f32_matmul(float *out, const float *w, const float *x, uint64_t in_dim,
                     uint64_t out_dim, uint64_t n_tok, double *part, uint64_t part_bytes,
                     uint32_t *slices_left, sf37_stream_t s);
/* Router: sigmoid, +bias, top-k (score desc, index asc), renormalise. */
int sf37k_router_select(int32_t *selected, float *weights, float *probs,
                        const float *logits, const float *bias, uint32_t n_experts,
                        uint32_t topk, float scale, uint32_t n_tok, sf37_stream_t s);
/* The same from slices > 1 binary64 slices in part ([slices][n_tok][n_experts],
 * added in slice order), or from logits when slices is 1. */
int sf37k_router_select_part(int32_t *selected, float *weights, float *probs, const float *logits,
                             const double *part, uint32_t slices, const float *bias, uint32_t n_experts,
                             uint32_t topk, float scale, uint32_t n_tok, sf37_stream_t s);

/* Q8_0 activations (32-wide) and Q8_0 GEMV / pair / batch. */
int sf37k_q8_0_quantize(int8_t *xq, float *xscale, const float *x, uint64_t in_dim,
                        uint64_t n_tok, sf37_stream_t s);
int sf37k_q8_0_matmul(float *out0, float *out1, const uint8_t *w0, const uint8_t *w1,
                      const int8_t *xq, const float *xscale, uint64_t in_dim,
                      uint64_t out_dim, uint64_t n_tok, sf37_stream_t s);

/* Elementwise. */
int sf37k_swiglu(float *out, const float *gate, const float *up, uint64_t n, float clamp,
                 sf37_stream_t s);
int sf37k_add_inplace(float *dst, const float *src, uint64_t n, sf37_stream_t s);
/* dst = dst + (a + b): a layer's output (shared + routed) added to the hidden state. */
int sf37k_add2_inplace(float *dst, const float *a, const float *b, uint64_t n, sf37_stream_t s);
int sf37k_rms_norm(float *out, const float *x, const void *w, int w_is_bf16, uint32_t n,
                   uint32_t n_tok, float eps, sf37_stream_t s);
/* out[i] = bf16 in[i] as float (exact), out 16-byte aligned. */
int sf37k_bf16_widen(float *out, const uint16_t *in, uint64_t n, sf37_stream_t s);

/* Routed experts, Q8_K path.  Work is organised in groups: group g covers
 * pairs sorted[pair_off[g] .. pair_off[g+1]) that all use expert
 * group_expert[g]; a pair p is token p / topk, slot p % topk. */
int sf37k_moe_gate_up(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                      const uint8_t *up_w, const void *xq, const uint32_t *group_info,
                      const uint32_t *sorted_pairs, const float *weights, uint32_t max_groups,
                      uint32_t max_group_pairs, uint32_t topk, uint32_t in_dim,
                      uint32_t mid_dim, float clamp, sf37_stream_t s);
int sf37k_moe_down(float *down_pair, const uint8_t *down_w, const void *midq,
                   const uint32_t *group_info, const uint32_t *sorted_pairs,
                   uint32_t max_groups, uint32_t max_group_pairs, uint32_t mid_dim,
                   uint32_t out_dim, sf37_stream_t s);
/* Slot-order sum of the per-pair rows: out = [base +] sum (base may be out);
 * with resid, resid = resid + (base + sum) instead and out is not written. */
int sf37k_moe_combine(float *out, const float *down_pair, const float *base, float *resid, uint32_t topk,
                      uint32_t out_dim, uint32_t n_tok, sf37_stream_t s);
/* Build the groups from selected experts: stable counting sort of pairs by
 * expert.  group_info layout: [0] = n_groups, [1 .. 1+E] = group pair
 * offsets, [2+E .. 2+2E) = group experts; counts/offsets per expert also.
 * hist: device scratch of sf37k_moe_dispatch_scratch_bytes (per-chunk
 * histograms of batches sorted by many workgroups; NULL when that is 0). */
uint64_t sf37k_moe_dispatch_scratch_bytes(uint32_t n_pairs, uint32_t n_expert);
int sf37k_moe_dispatch(uint32_t *group_info, uint32_t *sorted_pairs, uint32_t *counts,
                       uint32_t *offsets, const int32_t *selected, uint32_t n_pairs,
                       uint32_t n_expert, uint32_t *hist, sf37_stream_t s);
/* One group per slot for a single token (no sort), as routed_moe_one. */
int sf37k_moe_slots(uint32_t *group_info, uint32_t *sorted_pairs, const int32_t *selected,
                    uint32_t topk, uint32_t n_expert, sf37_stream_t s);

/* fp32-activation routed experts (the reference's small-shape path). */
int sf37k_moe_gate_up_f32(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                          const uint8_t *up_w, const float *x, const int32_t *selected,
                          const float *weights, uint32_t topk, uint32_t in_dim,
                          uint32_t mid_dim, uint32_t n_expert, float clamp, sf37_stream_t s);
int sf37k_moe_down_f32(float *down_slot, const uint8_t *down_w, const float *mid,
                       const int32_t *selected, uint32_t topk, uint32_t mid_dim,
                       uint32_t out_dim, uint32_t n_expert, sf37_stream_t s);

/* Synthetic inputs (harness): N(0, sigma) fp32 fill and generate+quantize
 * rows in the Q8_0 (type 0), Q2 (type 2) or Q3 (type 3) layouts. */
int sf37k_synth_normal(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                       uint64_t index0, float sigma, sf37_stream_t s);
int sf37k_synth_quant_rows(int type, uint8_t *dst, uint64_t row0, uint64_t nrows,
                           uint64_t ncols, uint64_t seed, uint64_t stream, float sigma,
                           sf37_stream_t s);
/* Elementwise exp/sigmoid of a float array (for exhaustive parity tests). */
int sf37k_sigmoid_array(float *out, const float *x, uint64_t n, int mode, sf37_stream_t s);

/* Routed experts on the matrix cores for many pairs per expert
 * (k_prefill.hip).  Activations are re-quantised to Q8_K and written as fp16
 * codes in the MFMA operand order of the weight format (q3 = 1: Q3 gate/up,
 * 0: Q2 down) with a table of 8 floats per (row, 256-block); groups are cut
 * into tiles of <= 128 pairs; gate/up and down read them.  codes: rows x dim
 * halves; tab: rows x dim/256 x 8 floats; tiles: (max_tiles + 1) x 4 words. */
uint32_t sf37k_pf_max_tiles(uint32_t n_pairs, uint32_t max_groups);
int sf37k_pf_supported(uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim);
int sf37k_pf_act(int q3, void *codes, float *tab, const float *x, uint32_t dim, uint32_t n_rows,
                 sf37_stream_t s);
int sf37k_pf_tiles(uint32_t *tiles, const uint32_t *group_info, uint32_t max_groups, sf37_stream_t s);
/* The per-block tables gathered into dispatch order (floats:
 * dim/256 x 5 x sf37k_pf_tab_stride(n_pairs)); row = pair / div. */
uint32_t sf37k_pf_tab_stride(uint32_t n_pairs);
int sf37k_pf_tab_sort(float *tabs, const float *tab, const uint32_t *sorted_pairs, uint32_t n_pairs, uint32_t dim,
                      uint32_t div, sf37_stream_t s);
int sf37k_pf_gate_up(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                     const uint8_t *up_w, const void *act, const float *tab, const uint32_t *tiles,
                     const uint32_t *sorted_pairs, const float *weights, uint32_t max_tiles,
                     uint32_t tab_stride, uint32_t topk, uint32_t in_dim, uint32_t mid_dim, float clamp,
                     sf37_stream_t s);
int sf37k_pf_down(float *down_pair, const uint8_t *down_w, const void *act, const float *tab,
                  const uint32_t *tiles, const uint32_t *sorted_pairs, uint32_t max_tiles,
                  uint32_t tab_stride, uint32_t mid_dim, uint32_t out_dim, sf37_stream_t s);

/* Shared expert (Q8_0) on the int8 matrix cores for many tokens
 * (k_prefill.hip): Q8_0 activations (a8: n_tok x dim int8 codes, xs: n_tok x
 * dim/32 float scales), gate/up straight from the Q8_0 weight tensors with
 * the shared SwiGLU into mid, down into out.  Results equal q8_0_matmul +
 * swiglu bit for bit. */
int sf37k_sh_supported(uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim);
int sf37k_sh_act(void *a8, float *xs, const float *x, uint32_t dim, uint32_t n_tok, sf37_stream_t s);
int sf37k_sh_gate_up(float *mid, const uint8_t *gate_w, const uint8_t *up_w, const void *a8, const float *xs,
                     uint32_t n_tok, uint32_t in_dim, uint32_t mid_dim, float clamp, sf37_stream_t s);
int sf37k_sh_down(float *out, const uint8_t *down_w, const void *a8, const float *xs, uint32_t n_tok,
                  uint32_t mid_dim, uint32_t out_dim, sf37_stream_t s);

/* Fused decode layer (up to 16 tokens): route, select, up, mid, down,
 * combine (k_decode.hip).  Pointers are device addresses; flags select the parts
 * that run.  cnt holds sf37k_decode_counters(...) zero-initialised words
 * that the kernels leave zero again when they finish. */
#define SF37_DEC_MAX_TOK 16u
#define SF37_DEC_ROUTER 1u   /* router GEMV of x into logits */
#define SF37_DEC_SELECT 2u   /* top-k from logits_sel (else sel/wts are inputs) */
#define SF37_DEC_SHARED 4u   /* shared expert, out = shared + routed */
#define SF37_DEC_SLOTS 8u    /* one group per slot of a single token */
#define SF37_DEC_NORM 16u    /* x is the hidden state: RMSNorm(w + 1) by the route kernel */
#define SF37_DEC_RESID 32u   /* out += layer output (out is the hidden state) */
#define SF37_DEC_UPSEL 64u   /* no select launch: the up launch forms the top-k and runs the shared gate/up */
#define SF37_DEC_SHBASE 128u /* out = sh_out (computed before) + routed; no shared expert here */
#define SF37_DEC_SH9 256u    /* the shared expert in the routed formats (Q3GU gate/up, Q2D down at sh_gate,
                                sh_up, sh_down) as expert id E in the last of topk slots per token: the
                                top-k fills topk - 1 slots, the last is (E, weight 1.0, clamp_shared) */
#define SF37_DEC_ACT_BYTES 288u  /* activation block: 256 codes, d, 4 sums, pad */
typedef struct sf37_dec_params {
    uint32_t T, E, K, F, topk, G;
    float scale, clamp_routed, clamp_shared;
    uint32_t flags;
    const float *x, *router_w, *router_bias, *logits_sel;
    const uint8_t *gate_w, *up_w, *down_w, *sh_gate, *sh_up, *sh_down;
    float *logits;       /* T x E router logits (ROUTER) */
    uint64_t *cand_key;  /* T x E selection keys (SELECT) */
    float *cand_p;       /* T x E sigmoid of the selecting logits (SELECT) */
    int32_t *sel;
    float *wts;
    void *xq;            /* T x K/256 activation blocks (Q3 order) */
    int8_t *xq8;         /* T x K Q8_0 codes */
    float *xs8;          /* T x K/32 Q8_0 scales */
    uint32_t *ginfo;     /* [0] groups, [1..G+1] pair offsets, [G+2..2G+2) experts */
    uint32_t *sorted;    /* pairs ordered by (expert, pair) */
    float *mid;          /* pairs x F SwiGLU * weight */
    void *midq;          /* pairs x F/256 activation blocks (Q2 order) */
    float *gate_out, *up_out;   /* pairs x F gate / up rows */
    float *sh_gu;        /* 2 x T x F shared gate | up */
    int8_t *sh_mq;       /* T x F Q8_0 codes of the shared mid */
    float *sh_ms;        /* T x F/32 scales */
    float *sh_out;       /* T x K shared expert output */
    float *down_pair;    /* pairs x K */
    float *out;          /* T x K */
    uint32_t *cnt;
    const uint16_t *norm_w;  /* K bf16 norm weights (NORM) */
    float eps;               /* RMSNorm epsilon (NORM) */
    float *xn;               /* T x K normalised rows, or NULL (NORM) */
    uint32_t up_dyn_pct;     /* share of the up items handed out dynamically (percent) */
    uint32_t up_wgs, dn_wgs; /* up / down workgroups per CU (0 = as many as fit) */
} sf37_dec_params;
int sf37k_decode_counters(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F);
/* The no-alloc decode entry point's scratch: a static device array of
 * SF37_NOALLOC_SCRATCH_BYTES per GPU, the item queues in its first
 * SF37_NOALLOC_QUEUE_BYTES.  _init (once per device, that device current)
 * looks its address up; _scratch returns the current device's address
 * (NULL before _init). */
#define SF37_NOALLOC_SCRATCH_BYTES (10u << 20)
#define SF37_NOALLOC_QUEUE_BYTES (16u << 10)
int sf37k_noalloc_scratch_init(void);
void *sf37k_noalloc_scratch(void);
/* 1 if the fused kernels take this shape (token count, dims, LDS). */
int sf37k_decode_supported(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F, int shared);
int sf37k_decode_lds_check(uint32_t T, uint32_t topk, uint32_t E, uint32_t K, uint32_t F, uint32_t flags,
                           uint32_t max_lds, uint64_t *ext);
/* The launches, in this order on one stream. */
int sf37k_decode_route(const sf37_dec_params *p, sf37_stream_t s);
int sf37k_decode_select(const sf37_dec_params *p, sf37_stream_t s);   /* skipped with UPSEL */
int sf37k_decode_up(const sf37_dec_params *p, sf37_stream_t s);
int sf37k_decode_mid(const sf37_dec_params *p, sf37_stream_t s);
int sf37k_decode_down(const sf37_dec_params *p, sf37_stream_t s);
int sf37k_decode_combine(const sf37_dec_params *p, sf37_stream_t s);
/* One token with SLOTS: down and combine as one launch (in place of the
 * last two), when _supported says the shape fits. */
int sf37k_decode_down_combine_supported(const sf37_dec_params *p);
int sf37k_decode_down_combine(const sf37_dec_params *p, sf37_stream_t s);

#ifdef __cplusplus
}
#endif

#endif
