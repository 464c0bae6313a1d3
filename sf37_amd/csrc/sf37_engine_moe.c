/*
 * sf37_engine_moe.c - the SF37_USE_HIP branch of the reference engine's MoE
 * feed-forward block (declared in include/sf37_engine_moe.h).
 *
 * The engine selects its GPU backend at compile time (#ifdef SF37_USE_CUDA,
 * sf37.c:6-8); this translation unit is the HIP side of that choice for the
 * MoE layers, compiled with -DSF37_USE_HIP.  Every step is one sf37_hip_*
 * call with the arguments cuda_decode_layer / cuda_prefill_layer pass to its
 * sf37_cuda_* twin, in the same order, through the _mapped entry points over
 * the engine's model map.
 */
#include <stdio.h>

#include "../../include/sf37_engine_moe.h"

#ifndef SF37_USE_HIP
#error "sf37_engine_moe.c is the SF37_USE_HIP engine branch: build it with -DSF37_USE_HIP"
#endif

#define SF37_RMS_EPS 1.0e-5f   /* sf37.c:61 */

/* sf37.c:2103-2106 */
static float layer_swiglu_limit(uint32_t il, int shared) {
    if (il == 43u || il == 44u) return shared ? 16.0f : 7.0f;
    return 0.0f;
}

/* cuda_matvec_dense_mapped / cuda_matmul_dense_mapped (sf37.c:2894-2933):
 * the router's own tensor type picks the GEMV. */
static int hip_matmul_dense_mapped(sf37_hip_tensor *out, const sf37_engine_moe_layer *l, const sf37_hip_tensor *x,
                                   uint32_t n_tok) {
    const uint64_t in = l->embd, outd = l->n_expert;
    switch (l->router_type) {
        case SF37_HIP_TYPE_Q8_0:
            return n_tok == 1u ? sf37_hip_matvec_q8_0_mapped(out, l->map, l->size, l->router_gate, in, outd, x)
                               : sf37_hip_matmul_q8_0_mapped(out, l->map, l->size, l->router_gate, in, outd, x, n_tok);
        case SF37_HIP_TYPE_BF16:
            return n_tok == 1u ? sf37_hip_matvec_bf16_mapped(out, l->map, l->size, l->router_gate, in, outd, x)
                               : sf37_hip_matmul_bf16_mapped(out, l->map, l->size, l->router_gate, in, outd, x, n_tok);
        case SF37_HIP_TYPE_F32:
            return n_tok == 1u ? sf37_hip_matvec_f32_mapped(out, l->map, l->size, l->router_gate, in, outd, x)
                               : sf37_hip_matmul_f32_mapped(out, l->map, l->size, l->router_gate, in, outd, x, n_tok);
        default:
            return 0;
    }
}

#define HIP_LAYER_CHECK(expr, label)                                                         \
    do {                                                                                     \
        if (!(expr)) {                                                                       \
            fprintf(stderr, "sf37: HIP %s layer %u failed at %s\n", mode, l->il, label);      \
            return 0;                                                                        \
        }                                                                                    \
    } while (0)

/* Layers 0-2 are dense (sf37.c:3376-3390 run their Q8_0 FFN instead); they
 * have no router or expert tensors, so the MoE block refuses them. */
static int moe_layer_ok(const sf37_engine_moe_layer *l, const char *mode) {
    if (l->il >= SF37_FIRST_MOE_LAYER) return 1;
    fprintf(stderr, "sf37: HIP %s layer %u is a dense layer (MoE layers start at %u)\n", mode, l->il,
            SF37_FIRST_MOE_LAYER);
    return 0;
}

int sf37_engine_moe_decode(const sf37_engine_moe_layer *l, sf37_engine_moe_bufs *s) {
    static const char mode[] = "decode";
    if (!l || !s || !moe_layer_ok(l, mode)) return 0;
    const uint32_t il = l->il;
    HIP_LAYER_CHECK(sf37_hip_begin_layer(il), "begin layer");
#ifdef SF37_USE_HIP
    HIP_LAYER_CHECK(sf37_hip_rms_norm_weight1_bf16_mapped(s->ffn_norm, s->hidden, l->map, l->size, l->post_norm,
                                                          l->embd, SF37_RMS_EPS),
                    "post rms");
    HIP_LAYER_CHECK(hip_matmul_dense_mapped(s->router_logits, l, s->ffn_norm, 1u), "router gate");
    HIP_LAYER_CHECK(sf37_hip_router_select_mapped(s->router_selected, s->router_weights, s->router_probs,
                                                  s->router_logits, l->map, l->size, l->router_bias, l->n_expert,
                                                  l->topk, 3.0f),
                    "router select");
    HIP_LAYER_CHECK(sf37_hip_matvec_q8_0_pair_mapped(s->gate, s->up, l->map, l->size, l->share_gate, l->share_up,
                                                     l->embd, l->expert_ff, s->ffn_norm),
                    "shared gate/up");
    HIP_LAYER_CHECK(sf37_hip_swiglu_f32(s->mid, s->gate, s->up, l->expert_ff, layer_swiglu_limit(il, 1)),
                    "shared swiglu");
    HIP_LAYER_CHECK(sf37_hip_matvec_q8_0_mapped(s->ffn_out, l->map, l->size, l->share_down, l->expert_ff, l->embd,
                                                s->mid),
                    "shared down");
    HIP_LAYER_CHECK(sf37_hip_routed_moe_one_mapped(s->routed_out, s->gate, s->up, s->mid, s->routed_down, l->map,
                                                   l->size, l->moe_gate, l->moe_up, l->moe_down, s->router_selected,
                                                   s->router_weights, l->n_expert, l->topk, l->embd, l->expert_ff,
                                                   l->embd, layer_swiglu_limit(il, 0), s->ffn_norm),
                    "routed moe");
    HIP_LAYER_CHECK(sf37_hip_add_inplace_f32(s->ffn_out, s->routed_out, l->embd), "shared+routed add");
    HIP_LAYER_CHECK(sf37_hip_add_inplace_f32(s->hidden, s->ffn_out, l->embd), "ffn residual");
#endif
    sf37_hip_end_layer();
    return 1;
}

int sf37_engine_moe_prefill(const sf37_engine_moe_layer *l, sf37_engine_moe_bufs *p, uint32_t n_tok) {
    static const char mode[] = "prefill";
    if (!l || !p || n_tok == 0 || !moe_layer_ok(l, mode)) return 0;
    const uint32_t il = l->il;
    const uint64_t n = (uint64_t)n_tok;
    HIP_LAYER_CHECK(sf37_hip_begin_layer(il), "begin layer");
#ifdef SF37_USE_HIP
    HIP_LAYER_CHECK(sf37_hip_rms_norm_weight1_bf16_batch_mapped(p->ffn_norm, p->hidden, l->map, l->size,
                                                                l->post_norm, l->embd, n_tok, SF37_RMS_EPS),
                    "post rms batch");
    HIP_LAYER_CHECK(hip_matmul_dense_mapped(p->router_logits, l, p->ffn_norm, n_tok), "router gate batch");
    HIP_LAYER_CHECK(sf37_hip_router_select_batch_mapped(p->router_selected, p->router_weights, p->router_probs,
                                                        p->router_logits, l->map, l->size, l->router_bias,
                                                        l->n_expert, l->topk, 3.0f, n_tok),
                    "router select batch");
    HIP_LAYER_CHECK(sf37_hip_matmul_q8_0_pair_mapped(p->gate, p->up, l->map, l->size, l->share_gate, l->share_up,
                                                     l->embd, l->expert_ff, p->ffn_norm, n),
                    "shared gate/up batch");
    HIP_LAYER_CHECK(sf37_hip_swiglu_f32(p->mid, p->gate, p->up, n * l->expert_ff, layer_swiglu_limit(il, 1)),
                    "shared swiglu batch");
    HIP_LAYER_CHECK(sf37_hip_matmul_q8_0_mapped(p->ffn_out, l->map, l->size, l->share_down, l->expert_ff, l->embd,
                                                p->mid, n),
                    "shared down batch");
    HIP_LAYER_CHECK(sf37_hip_routed_moe_batch_mapped(p->routed_out, p->routed_gate, p->routed_up, p->routed_mid,
                                                     p->routed_down, l->map, l->size, l->moe_gate, l->moe_up,
                                                     l->moe_down, p->router_selected, p->router_weights,
                                                     l->n_expert, l->topk, l->embd, l->expert_ff, l->embd,
                                                     layer_swiglu_limit(il, 0), p->ffn_norm, n_tok),
                    "routed moe batch");
    HIP_LAYER_CHECK(sf37_hip_add_inplace_f32(p->ffn_out, p->routed_out, n * l->embd), "shared+routed add batch");
    HIP_LAYER_CHECK(sf37_hip_add_inplace_f32(p->hidden, p->ffn_out, n * l->embd), "ffn residual batch");
#endif
    sf37_hip_end_layer();
    return 1;
}
