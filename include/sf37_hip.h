/*
 * sf37_hip.h - C ABI of the MI355X (gfx950) MoE feed-forward backend.
 *
 * Drop-in for the MoE hot-path subset of the reference backend interface
 * sf37_cuda.h (ZephinueCode/sf37): every sf37_hip_X below takes the same
 * arguments with the same meaning as sf37_cuda_X at the cited line, and
 * follows its conventions:
 *   - int results: 1 = success, 0 = failure (a line "sf37: HIP <what>
 *     failed: <error>" goes to stderr); pointer results: NULL on failure;
 *   - sizes and shapes are checked before anything is launched; tensors too
 *     small for the stated shapes are rejected;
 *   - out-of-range expert ids in `selected` are treated as expert 0;
 *   - work is enqueued in order on one stream (the null stream unless
 *     sf37_hip_set_stream was called); results are visible after
 *     sf37_hip_synchronize or a tensor read;
 *   - one host thread drives the library at a time (not reentrant).
 *
 * Numerics: routed experts with in/mid rows >= 512 (option "q8k_min_rows")
 * run the Q8_K activation path (256-wide int8 activations, integer dots with
 * zero-point correction, sf37_cuda.cu:4162-4503); smaller shapes run the
 * fp32-activation path (sf37_cuda.cu:5035-5267), as the reference does.
 * Every float result of the Q8_K path follows one canonical operation order
 * and is bit-identical between the decode and batch kernels; the sigmoid is
 * bit-identical to the engine's CPU sigmoid (sf37_ops.c:9-16).
 *
 * Block layouts are the reference's, unchanged: Q3 "Q3GU" 110-byte blocks,
 * Q2 "Q2D" 84-byte blocks, Q8_0 34-byte blocks (sf37_quant.h:10-13,
 * gguf-tools/quants.c:369-380, 564-573).
 */
#ifndef SF37_HIP_H
#define SF37_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF37_HIP_QK_K 256
#define SF37_HIP_Q8_0_BLOCK_SIZE 34
#define SF37_HIP_Q3_BLOCK_SIZE 110
#define SF37_HIP_Q2_BLOCK_SIZE 84
#define SF37_HIP_Q8K_BLOCK_SIZE 268   /* {float d; int8 qs[256]; int16 gsums[4]} */

/* Opaque device buffer {device pointer, byte size} (sf37_cuda.cu:32-35). */
typedef struct sf37_hip_tensor sf37_hip_tensor;

/* ---- runtime (sf37_cuda.h:12-19) ------------------------------------- */
int sf37_hip_device_count(void);                                   /* sf37_cuda.h:12 */
void sf37_hip_print_devices(void);                                 /* sf37_cuda.h:13 */
int sf37_hip_init(void);                                           /* sf37_cuda.h:14 */
void sf37_hip_cleanup(void);                                       /* sf37_cuda.h:15 */
int sf37_hip_synchronize(void);                                    /* sf37_cuda.h:16 */
int sf37_hip_memory_info(uint64_t *free_bytes, uint64_t *total_bytes); /* sf37_cuda.h:17 */
int sf37_hip_begin_layer(uint32_t layer);                          /* sf37_cuda.h:18 */
void sf37_hip_end_layer(void);                                     /* sf37_cuda.h:19 */

/* ---- model map: weights resident in HBM (sf37_cuda.h:21-33) ---------- */
/* A registered range of the host model map is copied to the device once;
 * _mapped calls resolve (model_map, offset) to that resident copy, or copy
 * an unregistered range on first use and keep it until evicted. */
int sf37_hip_set_model_fd(int fd);                                 /* sf37_cuda.h:21 */
int sf37_hip_set_model_map_range(const void *model_map, uint64_t model_size,
                                 uint64_t map_offset, uint64_t map_size,
                                 uint64_t max_tensor_bytes);       /* sf37_cuda.h:22-24 */
int sf37_hip_set_model_map_spans(const void *model_map, uint64_t model_size,
                                 const uint64_t *offsets, const uint64_t *sizes,
                                 uint32_t count, uint64_t max_tensor_bytes); /* :25-29 */
int sf37_hip_cache_model_range(const void *model_map, uint64_t model_size,
                               uint64_t offset, uint64_t bytes,
                               const char *label);                 /* sf37_cuda.h:30-32 */
void sf37_hip_evict_model_cache(const char *reason);               /* sf37_cuda.h:33 */

/* ---- tensors (sf37_cuda.h:39-50) -------------------------------------- */
sf37_hip_tensor *sf37_hip_tensor_alloc(uint64_t bytes);            /* sf37_cuda.h:39 */
sf37_hip_tensor *sf37_hip_tensor_alloc_managed(uint64_t bytes);    /* sf37_cuda.h:40 */
void sf37_hip_tensor_free(sf37_hip_tensor *tensor);                /* sf37_cuda.h:41 */
uint64_t sf37_hip_tensor_bytes(const sf37_hip_tensor *tensor);     /* sf37_cuda.h:42 */
int sf37_hip_tensor_write(sf37_hip_tensor *tensor, uint64_t offset,
                          const void *data, uint64_t bytes);       /* sf37_cuda.h:43-44 */
int sf37_hip_tensor_read(const sf37_hip_tensor *tensor, uint64_t offset,
                         void *data, uint64_t bytes);              /* sf37_cuda.h:45-46 */
int sf37_hip_tensor_copy(sf37_hip_tensor *dst, uint64_t dst_offset,
                         const sf37_hip_tensor *src, uint64_t src_offset,
                         uint64_t bytes);                          /* sf37_cuda.h:47-49 */
int sf37_hip_tensor_fill_f32(sf37_hip_tensor *tensor, float value,
                             uint64_t count);                      /* sf37_cuda.h:50 */

/* ---- norm / elementwise (sf37_cuda.h:75-89) --------------------------- */
int sf37_hip_rms_norm_weight1_f32(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                  const sf37_hip_tensor *weight, uint32_t n,
                                  float eps);                      /* sf37_cuda.h:75-78 */
int sf37_hip_rms_norm_weight1_bf16(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                   const sf37_hip_tensor *weight, uint32_t n,
                                   float eps);                     /* sf37_cuda.h:79-82 */
int sf37_hip_add_inplace_f32(sf37_hip_tensor *dst, const sf37_hip_tensor *src,
                             uint64_t n);                          /* sf37_cuda.h:83-85 */
int sf37_hip_swiglu_f32(sf37_hip_tensor *out, const sf37_hip_tensor *gate,
                        const sf37_hip_tensor *up, uint64_t n,
                        float clamp);                              /* sf37_cuda.h:86-89 */

/* ---- dense and quantised GEMV (sf37_cuda.h:134-163) -------------------- */
int sf37_hip_matvec_q8_0(sf37_hip_tensor *out, const sf37_hip_tensor *weights,
                         uint64_t in_dim, uint64_t out_dim,
                         const sf37_hip_tensor *x);                /* sf37_cuda.h:134-137 */
int sf37_hip_matvec_q8_0_pair(sf37_hip_tensor *out0, sf37_hip_tensor *out1,
                              const sf37_hip_tensor *weights0,
                              const sf37_hip_tensor *weights1,
                              uint64_t in_dim, uint64_t out_dim,
                              const sf37_hip_tensor *x);           /* sf37_cuda.h:138-143 */
int sf37_hip_matvec_f32(sf37_hip_tensor *out, const sf37_hip_tensor *weights,
                        uint64_t in_dim, uint64_t out_dim,
                        const sf37_hip_tensor *x);                 /* sf37_cuda.h:152-155 */
/* bf16 weights, binary64 accumulation as the CPU engine (sf37_ops.c:143-151) */
int sf37_hip_matvec_bf16(sf37_hip_tensor *out, const sf37_hip_tensor *weights,
                         uint64_t in_dim, uint64_t out_dim,
                         const sf37_hip_tensor *x);                /* sf37_cuda.h:144-147 */
int sf37_hip_matvec_q3_asym(sf37_hip_tensor *out, const sf37_hip_tensor *weights,
                            uint64_t in_dim, uint64_t out_dim,
                            const sf37_hip_tensor *x);             /* sf37_cuda.h:156-159 */
int sf37_hip_matvec_q2_asym(sf37_hip_tensor *out, const sf37_hip_tensor *weights,
                            uint64_t in_dim, uint64_t out_dim,
                            const sf37_hip_tensor *x);             /* sf37_cuda.h:160-163 */

/* ---- router and routed experts (sf37_cuda.h:164-188) ------------------ */
int sf37_hip_router_select(sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                           sf37_hip_tensor *probs, const sf37_hip_tensor *logits,
                           const sf37_hip_tensor *bias, uint32_t n_experts,
                           uint32_t topk, float scale);            /* sf37_cuda.h:164-171 */
int sf37_hip_routed_moe_one(sf37_hip_tensor *out, sf37_hip_tensor *gate,
                            sf37_hip_tensor *up, sf37_hip_tensor *mid,
                            sf37_hip_tensor *down, const sf37_hip_tensor *moe_gate,
                            const sf37_hip_tensor *moe_up, const sf37_hip_tensor *moe_down,
                            const sf37_hip_tensor *selected, const sf37_hip_tensor *weights,
                            uint32_t n_total_expert, uint32_t topk, uint32_t in_dim,
                            uint32_t expert_mid_dim, uint32_t out_dim, float clamp,
                            const sf37_hip_tensor *x);             /* sf37_cuda.h:172-188 */

/* ---- mapped variants (sf37_cuda.h:190-203, 262-431) ------------------- */
int sf37_hip_rms_norm_weight1_bf16_mapped(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                          const void *model_map, uint64_t model_size,
                                          uint64_t weight_offset, uint32_t n,
                                          float eps);              /* sf37_cuda.h:190-195 */
int sf37_hip_rms_norm_weight1_bf16_batch_mapped(sf37_hip_tensor *out,
                                                const sf37_hip_tensor *x,
                                                const void *model_map, uint64_t model_size,
                                                uint64_t weight_offset, uint32_t n,
                                                uint32_t n_tok, float eps); /* :196-203 */
int sf37_hip_matvec_q8_0_mapped(sf37_hip_tensor *out, const void *model_map,
                                uint64_t model_size, uint64_t weight_offset,
                                uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x);         /* sf37_cuda.h:262-267 */
int sf37_hip_matmul_q8_0_mapped(sf37_hip_tensor *out, const void *model_map,
                                uint64_t model_size, uint64_t weight_offset,
                                uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x, uint64_t n_tok); /* :299-305 */
int sf37_hip_matmul_q8_0_pair_mapped(sf37_hip_tensor *out0, sf37_hip_tensor *out1,
                                     const void *model_map, uint64_t model_size,
                                     uint64_t weight0_offset, uint64_t weight1_offset,
                                     uint64_t in_dim, uint64_t out_dim,
                                     const sf37_hip_tensor *x, uint64_t n_tok); /* :306-315 */
int sf37_hip_matvec_q8_0_pair_mapped(sf37_hip_tensor *out0, sf37_hip_tensor *out1,
                                     const void *model_map, uint64_t model_size,
                                     uint64_t weight0_offset, uint64_t weight1_offset,
                                     uint64_t in_dim, uint64_t out_dim,
                                     const sf37_hip_tensor *x);    /* sf37_cuda.h:316-323 */
int sf37_hip_matvec_bf16_mapped(sf37_hip_tensor *out, const void *model_map,
                                uint64_t model_size, uint64_t weight_offset,
                                uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x);         /* sf37_cuda.h:324-329 */
int sf37_hip_matmul_bf16_mapped(sf37_hip_tensor *out, const void *model_map,
                                uint64_t model_size, uint64_t weight_offset,
                                uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x, uint64_t n_tok); /* :338-345 */
int sf37_hip_matvec_f32_mapped(sf37_hip_tensor *out, const void *model_map,
                               uint64_t model_size, uint64_t weight_offset,
                               uint64_t in_dim, uint64_t out_dim,
                               const sf37_hip_tensor *x);          /* sf37_cuda.h:346-351 */
int sf37_hip_matmul_f32_mapped(sf37_hip_tensor *out, const void *model_map,
                               uint64_t model_size, uint64_t weight_offset,
                               uint64_t in_dim, uint64_t out_dim,
                               const sf37_hip_tensor *x, uint64_t n_tok); /* :352-359 */
int sf37_hip_matvec_q3_asym_mapped(sf37_hip_tensor *out, const void *model_map,
                                   uint64_t model_size, uint64_t weight_offset,
                                   uint64_t in_dim, uint64_t out_dim,
                                   const sf37_hip_tensor *x);      /* sf37_cuda.h:360-365 */
int sf37_hip_matvec_q2_asym_mapped(sf37_hip_tensor *out, const void *model_map,
                                   uint64_t model_size, uint64_t weight_offset,
                                   uint64_t in_dim, uint64_t out_dim,
                                   const sf37_hip_tensor *x);      /* sf37_cuda.h:366-371 */
int sf37_hip_router_select_mapped(sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                                  sf37_hip_tensor *probs, const sf37_hip_tensor *logits,
                                  const void *model_map, uint64_t model_size,
                                  uint64_t bias_offset, uint32_t n_experts,
                                  uint32_t topk, float scale);     /* sf37_cuda.h:372-381 */
int sf37_hip_router_select_batch_mapped(sf37_hip_tensor *selected,
                                        sf37_hip_tensor *weights,
                                        sf37_hip_tensor *probs,
                                        const sf37_hip_tensor *logits,
                                        const void *model_map, uint64_t model_size,
                                        uint64_t bias_offset, uint32_t n_experts,
                                        uint32_t topk, float scale,
                                        uint32_t n_tok);           /* sf37_cuda.h:382-392 */
int sf37_hip_routed_moe_one_mapped(sf37_hip_tensor *out, sf37_hip_tensor *gate,
                                   sf37_hip_tensor *up, sf37_hip_tensor *mid,
                                   sf37_hip_tensor *down, const void *model_map,
                                   uint64_t model_size, uint64_t gate_offset,
                                   uint64_t up_offset, uint64_t down_offset,
                                   const sf37_hip_tensor *selected,
                                   const sf37_hip_tensor *weights,
                                   uint32_t n_total_expert, uint32_t topk,
                                   uint32_t in_dim, uint32_t expert_mid_dim,
                                   uint32_t out_dim, float clamp,
                                   const sf37_hip_tensor *x);      /* sf37_cuda.h:393-411 */
/* `mid` receives the per-pair SwiGLU output [n_tok*topk][expert_mid_dim]
 * when it is large enough (sf37_cuda.cu:5665-5674); pairs are token*topk+slot. */
int sf37_hip_routed_moe_batch_mapped(sf37_hip_tensor *out, sf37_hip_tensor *gate,
                                     sf37_hip_tensor *up, sf37_hip_tensor *mid,
                                     sf37_hip_tensor *down, const void *model_map,
                                     uint64_t model_size, uint64_t gate_offset,
                                     uint64_t up_offset, uint64_t down_offset,
                                     const sf37_hip_tensor *selected,
                                     const sf37_hip_tensor *weights,
                                     uint32_t n_total_expert, uint32_t topk,
                                     uint32_t in_dim, uint32_t expert_mid_dim,
                                     uint32_t out_dim, float clamp,
                                     const sf37_hip_tensor *x, uint32_t n_tok); /* :412-431 */

/* ======================================================================
 * Extensions (no counterpart in sf37_cuda.h).
 * ====================================================================== */

/* Launch stream for all work (a hipStream_t; NULL = null stream). */
int sf37_hip_set_stream(void *stream);
void *sf37_hip_get_stream(void);
/* Options, replacing the reference's SF37_CUDA_* environment toggles:
 *   "q8k_min_rows"      rows from which the Q8_K path is used (default 512,
 *                       as SF37_CUDA_QLOW_Q8K_MIN_ROWS, sf37_cuda.cu:200-214)
 *   "q8k"               0 disables the Q8_K path (SF37_CUDA_NO_QLOW_Q8K)
 *   "moe_write_gate_up" 1 also writes gate/up outputs in routed_moe_one
 *                       (SF37_CUDA_MOE_WRITE_GATE_UP)
 *   "decode_fused"      1 (default): batches of up to 16 tokens on the Q8_K
 *                       path run as the fused decode launches (route,
 *                       select, up, mid, down, combine; fewer for one
 *                       token); 0 uses the staged kernels.  Results are
 *                       identical either way.
 *   "decode_down_combine" 1 (default): one token's down and combine run as
 *                       one launch; the per-slot `down` tensor of
 *                       routed_moe_one is then scratch holding no rows (as
 *                       the reference's direct down-sum path,
 *                       sf37_cuda.cu:5366-5371); 0 writes them.
 *   "decode_select_in_up_max_tokens", "decode_up_dyn_pct", "decode_up_wgs",
 *   "decode_down_wgs"   decode tuning (results unchanged)
 *   "prefill_mfma"      1 (default): grouped batches run on the matrix cores;
 *   "prefill_min_pairs", "shared_min_tokens" the smallest batches that do
 *   "shared_stream"     1 (default): a prefill batch's Q8_0 shared expert
 *                       runs on a second stream of the library (default
 *                       priority), forked after its input rows and joined
 *                       before the routed combine; 0: in order
 *   "decode_shared_slot" 1 (default): a decode batch's Q3GU/Q2D shared
 *                       expert runs as one more slot of every token inside
 *                       the routed decode launches (slot topk, weight 1, the
 *                       shared clamp); 0: as launches of its own
 *   "router_with_logits" 1: sf37_hip_moe_layer computes the router GEMV even
 *                       when logits_in is given (its result is unused; for
 *                       benchmarks that inject routing but keep the cost)
 * Returns 1 for a known name. */
int sf37_hip_set_option(const char *name, int64_t value);
int64_t sf37_hip_get_option(const char *name);

/* Device address of a tensor (for interop) and non-owning views. */
void *sf37_hip_tensor_device_ptr(const sf37_hip_tensor *tensor);
sf37_hip_tensor *sf37_hip_tensor_view(const sf37_hip_tensor *base, uint64_t offset,
                                      uint64_t bytes);
/* Register existing device memory as the resident copy of a model-map range,
 * so _mapped calls can use weights that were produced on the device. */
int sf37_hip_register_device_range(const void *model_map, uint64_t model_size,
                                   uint64_t map_offset, uint64_t bytes,
                                   const sf37_hip_tensor *device);
/* Registry query (no reference counterpart; for tests and tools): -1 when no
 * registered range covers map[offset, offset+bytes), 0 when a range the
 * caller registered covers it, else the number of open GGUF handles holding
 * the range the layer binder made for it (freed when that reaches 0). */
int sf37_hip_model_range_holds(const void *model_map, uint64_t offset, uint64_t bytes);
/* Requests for device memory the library has served so far (its scratch,
 * counters, layer buffers, model-range copies, widened weights and tensor
 * allocations), counted whether or not a buffer had to grow.  No reference
 * counterpart; tests use it to show that an entry point allocates nothing. */
uint64_t sf37_hip_device_memory_requests(void);

/* Q8_K activations of n_rows rows (the reference's 268-byte block layout). */
int sf37_hip_q8k_quantize(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                          uint32_t in_dim, uint32_t n_rows);
/* Stable dispatch of n_pairs = n_tok*topk pairs: counts[E], offsets[E+1] and
 * pair ids sorted by (expert, pair id) (sf37_cuda.cu:4505-4544). */
int sf37_hip_moe_dispatch(sf37_hip_tensor *counts, sf37_hip_tensor *offsets,
                          sf37_hip_tensor *sorted_pairs, const sf37_hip_tensor *selected,
                          uint32_t n_pairs, uint32_t n_expert);

/* Whole MoE layer for n_tok tokens, composed as the engine does
 * (sf37.c:3392-3430 decode, 5959-6071 prefill): router logits, top-k,
 * shared expert, routed experts, out = shared + routed.  Weight pointers
 * are device tensors whose contents stay fixed while they are in use.
 * selected/weights may be NULL.
 *
 * router_type (GGUF type id of the router weights, any of the engine's
 * dense types, sf37.c:1775, 1960-1978): 0 F32 (binary64 sums), 30 BF16
 * (widened exactly, binary64 sums), 8 Q8_0 (the Q8_0 GEMV with Q8_0
 * activations, sf37_ops.c:110-141).
 * shared_type: 0 = Q8_0 gate/up/down (the engine's format, sf37.c:1780-1782);
 * 11 = Q3GU gate/up + Q2D down (the benchmark configurations' "same formats"
 * option), run on the Q8_K path as one more expert with routing weight 1.0
 * and the shared clamp. */
#define SF37_HIP_TYPE_F32 0u
#define SF37_HIP_TYPE_Q8_0 8u
#define SF37_HIP_TYPE_Q3GU 11u
#define SF37_HIP_TYPE_BF16 30u
typedef struct {
    const sf37_hip_tensor *router;        /* [n_expert][in_dim] of router_type */
    const sf37_hip_tensor *router_bias;   /* f32 [n_expert] */
    const sf37_hip_tensor *gate, *up;     /* Q3 [n_expert][mid][in/256 blocks] */
    const sf37_hip_tensor *down;          /* Q2 [n_expert][in][mid/256 blocks] */
    const sf37_hip_tensor *sh_gate, *sh_up, *sh_down;  /* shared expert of shared_type */
    uint32_t n_expert, topk, in_dim, mid_dim;
    float scale, clamp_routed, clamp_shared;
    uint32_t router_type, shared_type;
} sf37_hip_moe_layer_weights;
int sf37_hip_moe_layer(sf37_hip_tensor *out, sf37_hip_tensor *selected,
                       sf37_hip_tensor *weights, const sf37_hip_moe_layer_weights *w,
                       const sf37_hip_tensor *logits_in, const sf37_hip_tensor *x,
                       uint32_t n_tok);

/* sf37_hip_moe_layer without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * takes decode batches of 1..16 tokens on the fused decode path (an F32
 * router or injected logits, the Q8_0 shared expert, in/mid dims multiples of
 * 256 of at least q8k_min_rows) and keeps all of its scratch in one static
 * device array of 10 MiB per GPU (held until the process ends); a batch whose
 * scratch would not fit is refused with a message (288 experts x 4096 x 1280
 * at top-8 take 5 MiB at 16 tokens).  Results equal sf37_hip_moe_layer's bit
 * for bit.  Every call on a GPU uses that GPU's one array, whose address is
 * looked up on the first call with that device current: calls that overlap
 * on one GPU (other streams, other threads) race. */
int sf37_hip_moe_layer_noalloc(sf37_hip_tensor *out, sf37_hip_tensor *selected,
                               sf37_hip_tensor *weights, const sf37_hip_moe_layer_weights *w,
                               const sf37_hip_tensor *logits_in, const sf37_hip_tensor *x,
                               uint32_t n_tok);

/* The FFN block of an MoE decoder layer as the engine runs it
 * (sf37.c:2243-2250): hidden += moe_layer(rms_norm_weight1_bf16(hidden)),
 * the bf16 norm weights (in_dim of them) at norm_offset of a registered
 * model map, eps as sf37_hip_rms_norm_weight1_bf16_mapped.  Up to 16 tokens
 * the fused decode launches normalise and add the residual themselves (six
 * launches per block); larger batches run rms_norm, the layer and the add.
 * normed (optional) receives the normalised rows.  Same bits either way. */
int sf37_hip_moe_block(sf37_hip_tensor *hidden, sf37_hip_tensor *normed,
                       sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                       const sf37_hip_moe_layer_weights *w, const void *model_map,
                       uint64_t model_size, uint64_t norm_offset, float eps,
                       const sf37_hip_tensor *logits_in, uint32_t n_tok);

/* n_layers consecutive blocks (the engine's layer loop, sf37.c:2243-2250 per
 * layer) in one call: layers[l], norm weights at norm_offsets[l], injected
 * logits logits[l] and selection outputs selected[l] when those arrays are
 * given (entries may be NULL). */
int sf37_hip_moe_stack(sf37_hip_tensor *hidden, uint32_t n_layers,
                       const sf37_hip_moe_layer_weights *layers, const void *model_map,
                       uint64_t model_size, const uint64_t *norm_offsets, float eps,
                       const sf37_hip_tensor *const *logits,
                       sf37_hip_tensor *const *selected, uint32_t n_tok);

/* GGUF weight residency (the engine's reader, sf37.c:506-604, and MoE
 * tensor contract, sf37.c:1760-1782).  sf37_hip_gguf_open maps a GGUF v3
 * file read-only; sf37_hip_gguf_from_map parses a mapping the engine already
 * holds (the map pointer is then the model map of the _mapped calls).  Both
 * return NULL (with a stderr line) for a file that is not GGUF v3, a
 * truncated or malformed header, or a tensor outside the file.  Parsing
 * needs no GPU.  sf37_hip_gguf_tensor gives a tensor's absolute map offset,
 * bytes (0 for types the MoE path does not read), GGUF type id and up to 4
 * dims (unused dims 1).  sf37_hip_gguf_bind_moe_layer makes layer il's MoE
 * tensors device-resident and fills w for sf37_hip_moe_layer /
 * sf37_hip_moe_block (shapes read from the file and cross-checked; top-k 8,
 * scale 3.0, the layer's SwiGLU clamps) and the offset of its
 * post_attention_layernorm weights; the handles in w stay valid until
 * sf37_hip_gguf_close, which (for a handle from sf37_hip_gguf_open) also
 * drops the device copies of that mapping before unmapping it. */
typedef struct sf37_hip_gguf sf37_hip_gguf;
sf37_hip_gguf *sf37_hip_gguf_open(const char *path);
sf37_hip_gguf *sf37_hip_gguf_from_map(const void *map, uint64_t size);
void sf37_hip_gguf_close(sf37_hip_gguf *gguf);
const void *sf37_hip_gguf_map(const sf37_hip_gguf *gguf, uint64_t *size);
int sf37_hip_gguf_tensor(const sf37_hip_gguf *gguf, const char *name, uint64_t *offset,
                         uint64_t *bytes, uint32_t *type, uint32_t *ndim, uint64_t *dims);
int sf37_hip_gguf_bind_moe_layer(sf37_hip_gguf *gguf, uint32_t il,
                                 sf37_hip_moe_layer_weights *w, uint64_t *post_norm_offset);

/* Stage timing with HIP events, the counterpart of the reference's
 * SF37_CUDA_MOE_PROFILE (sf37_cuda.cu:345-449).  While enabled, every kernel
 * the library launches is bracketed by events on the launch stream;
 * sf37_hip_profile_read waits for them, fills total milliseconds and launch
 * counts per stage (index = enum order below) and resets the counters. */
enum {
    SF37_HIP_STAGE_ROUTER = 0, SF37_HIP_STAGE_SELECT, SF37_HIP_STAGE_Q8_0_ACT, SF37_HIP_STAGE_Q8_0_GEMM,
    SF37_HIP_STAGE_SWIGLU, SF37_HIP_STAGE_Q8K_X, SF37_HIP_STAGE_DISPATCH, SF37_HIP_STAGE_GATE_UP,
    SF37_HIP_STAGE_Q8K_MID, SF37_HIP_STAGE_DOWN, SF37_HIP_STAGE_COMBINE, SF37_HIP_STAGE_ADD,
    SF37_HIP_STAGE_OTHER,
    /* the fused decode layer (up to 16 tokens): route = router GEMV +
     * selection candidates + x quantisation, select = top-k + grouping and
     * the shared gate/up, up = routed gate/up, mid = SwiGLU + Q8_K of the
     * routed mid, down = Q8_0 of the shared mid + routed down, combine =
     * shared down + slot-order sum */
    SF37_HIP_STAGE_DEC_ROUTE, SF37_HIP_STAGE_DEC_UP, SF37_HIP_STAGE_DEC_DOWN,
    SF37_HIP_STAGE_DEC_SELECT, SF37_HIP_STAGE_DEC_COMBINE, SF37_HIP_STAGE_DEC_MID,
    /* the matrix-core prefill path (many pairs per expert): activations
     * re-quantised into the MFMA operand order (x, then the routed mid),
     * the per-expert tile list, gate/up + SwiGLU, down */
    SF37_HIP_STAGE_PF_ACT_X, SF37_HIP_STAGE_PF_TILES, SF37_HIP_STAGE_PF_GATE_UP,
    SF37_HIP_STAGE_PF_ACT_MID, SF37_HIP_STAGE_PF_DOWN,
    /* the shared expert on the matrix cores (prefill batches): Q8_0 weights
     * repacked to fp16 codes, Q8_0 activations (x, then the shared mid),
     * gate/up + SwiGLU, down */
    SF37_HIP_STAGE_SH_REPACK, SF37_HIP_STAGE_SH_ACT, SF37_HIP_STAGE_SH_GATE_UP, SF37_HIP_STAGE_SH_DOWN,
    SF37_HIP_N_STAGES
};
int sf37_hip_profile_enable(int on);
int sf37_hip_profile_read(double *ms, uint64_t *count, uint32_t n_stages);
const char *sf37_hip_profile_stage_name(uint32_t stage);

/* Synthetic inputs generated on the device (harness).  N(0, sigma) floats
 * from stream (seed, stream) starting at element index0; quantised rows
 * (type 0 = Q8_0, 2 = Q2, 3 = Q3) of ncols generated values each, rows
 * [row0, row0+nrows) of that tensor. */
int sf37_hip_synth_normal(sf37_hip_tensor *dst, uint64_t n, uint64_t seed,
                          uint64_t stream, uint64_t index0, float sigma);
int sf37_hip_synth_quant_rows(int type, sf37_hip_tensor *dst, uint64_t row0,
                              uint64_t nrows, uint64_t ncols, uint64_t seed,
                              uint64_t stream, float sigma);
/* Elementwise expf (mode 0) or sigmoid (mode 1) of n floats. */
int sf37_hip_sigmoid_array(sf37_hip_tensor *out, const sf37_hip_tensor *x, uint64_t n,
                           int mode);

#ifdef __cplusplus
}
#endif

#endif
