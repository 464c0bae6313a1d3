/*
 * sf37_engine_moe.h - the engine's MoE feed-forward block on the HIP backend:
 * the SF37_USE_HIP branch of the reference engine's per-layer decode and
 * prefill steps (sf37.c:3371-3430 in cuda_decode_layer, sf37.c:5936-6071 in
 * cuda_prefill_layer), written against include/sf37_hip.h the way that
 * engine writes its CUDA branch against sf37_cuda.h.
 *
 * libsf37_engine_moe.so links libsf37_hip.so.  The caller holds the model
 * map (the mapped GGUF, registered with sf37_hip_set_model_map_range or
 * resolved on demand) and the session's device buffers, as the engine's
 * sf37_session does (sf37.c:2935-2960); the block reads the hidden state,
 * runs post-attention RMSNorm, router, top-8, shared expert, routed experts,
 * shared + routed, and adds the result back into the hidden state.
 *
 * Return: 1 on success, 0 on failure with a line "sf37: HIP decode|prefill
 * layer <il> failed at <step>" on stderr (CUDA_LAYER_CHECK, sf37.c:3299-3305,
 * and its prefill twin).
 *
 * Precondition: il >= SF37_FIRST_MOE_LAYER.  Layers 0-2 are dense: the
 * engine runs their Q8_0 FFN instead (sf37.c:3376-3390, sf37.c:2245-2249),
 * which is not part of this block; both calls refuse them (return 0 and a
 * "dense layer" line on stderr) before any launch.
 */
#ifndef SF37_ENGINE_MOE_H
#define SF37_ENGINE_MOE_H

#include <stdint.h>

#include "sf37_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SF37_FIRST_MOE_LAYER 3u   /* sf37.c:2245: il < 3 runs the dense FFN */

/* One MoE layer's tensors as absolute offsets into the model map (the
 * engine's sf37_tensor abs_offset, sf37.c:1760-1782). */
typedef struct {
    const void *map;          /* e->gguf.map */
    uint64_t size;            /* e->gguf.size */
    uint32_t il;              /* layer index: SwiGLU clamps of layers 43/44 (sf37.c:2103-2106) */
    uint32_t router_type;     /* GGUF type of moe.gate.weight: F32 0, Q8_0 8, BF16 30 (sf37.c:2894-2933) */
    uint64_t post_norm;       /* post_attention_layernorm.weight, BF16 [embd] */
    uint64_t router_gate;     /* moe.gate.weight [experts][embd] */
    uint64_t router_bias;     /* moe.router_bias, F32 [experts] */
    uint64_t share_gate, share_up, share_down;   /* share_expert.*_proj, Q8_0 */
    uint64_t moe_gate, moe_up, moe_down;         /* moe.*_proj, Q3GU / Q3GU / Q2D */
    uint32_t n_expert, topk, embd, expert_ff;    /* 288, 8, 4096, 1280 in SF37 */
} sf37_engine_moe_layer;

/* The session buffers the block uses (sf37.c:2935-2960 decode, the prefill
 * batch buffers alongside): decode sizes are for one token; prefill sizes
 * for n_tok tokens (routed_mid may be smaller than n_tok x topk x ff, then
 * the per-pair mid is not exported). */
typedef struct {
    sf37_hip_tensor *hidden;           /* [n_tok][embd], updated in place */
    sf37_hip_tensor *ffn_norm;         /* [n_tok][embd] */
    sf37_hip_tensor *gate, *up, *mid;  /* shared expert [n_tok][ff] (decode: also routed scratch [topk][ff]) */
    sf37_hip_tensor *ffn_out;          /* [n_tok][embd] */
    sf37_hip_tensor *router_logits;    /* [n_tok][experts] */
    sf37_hip_tensor *router_probs;     /* [n_tok][experts] */
    sf37_hip_tensor *router_selected;  /* int32 [n_tok][topk] */
    sf37_hip_tensor *router_weights;   /* f32 [n_tok][topk] */
    sf37_hip_tensor *routed_gate, *routed_up, *routed_mid;   /* prefill: [n_tok*topk][ff] */
    sf37_hip_tensor *routed_down;      /* decode: [topk][embd] */
    sf37_hip_tensor *routed_out;       /* [n_tok][embd] */
} sf37_engine_moe_bufs;

/* hidden += MoE(RMSNorm(hidden)) for one token, cuda_decode_layer's call
 * sequence (sf37.c:3371-3430). */
int sf37_engine_moe_decode(const sf37_engine_moe_layer *l, sf37_engine_moe_bufs *s);

/* The same for an n_tok chunk, cuda_prefill_layer's call sequence
 * (sf37.c:5936-6071, the batched routed path). */
int sf37_engine_moe_prefill(const sf37_engine_moe_layer *l, sf37_engine_moe_bufs *p, uint32_t n_tok);

#ifdef __cplusplus
}
#endif

#endif
