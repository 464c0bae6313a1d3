"""A GGUF-resident MoE layer (sf37_hip_gguf_bind_moe_layer) runs the same
bits as the same layer from device tensors: reduced-shape layers 43 (F32
router) and 44 (BF16 router, widened exactly), written by the engine's
tensor contract (sf37.c:1760-1782), through sf37_hip_moe_block at 3 tokens
(fused decode) and 40 tokens (matrix-core prefill), against the block on
the SynthLayer tensors and the layer's own norm weights."""
import ctypes as C

import numpy as np
import pytest

from gguf_writer import T_BF16, T_F32, gguf_bytes, moe_layer_tensors

pytestmark = pytest.mark.gpu

E, D, F = 16, 512, 256


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
    yield hip
    for k, v in (("q8k_min_rows", 512), ("prefill_min_pairs", 256), ("shared_min_tokens", 64)):
        hip.set_option(k, v)
    hip.synchronize()


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got, np.float32).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want, np.float32).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ"


@pytest.mark.parametrize("il,router_type", [(43, T_F32), (44, T_BF16)])
def test_gguf_layer_equals_device_layer(H, tmp_path, il, router_type):
    from sf37_amd import configs
    from sf37_amd.moe import SynthLayer, bf16_bits
    L = H.lib()
    for k in ("q8k_min_rows", "prefill_min_pairs", "shared_min_tokens"):
        H.set_option(k, 0)
    lay = SynthLayer(seed=500 + il, n_expert=E, in_dim=D, mid_dim=F, topk=8, il=il)
    rng = np.random.default_rng(il)
    norm = bf16_bits((rng.standard_normal(D) * 0.02).astype(np.float32))
    router = lay.router.read(np.float32)
    if router_type == T_BF16:
        rbits = bf16_bits(router)
        lay.router.write((rbits.astype(np.uint32) << 16).view(np.float32))   # the exact widening
        router = rbits
    dense = lay.host_dense()
    ex = lay.host_experts(np.arange(E))
    tensors = moe_layer_tensors(il, router, router_type, dense["router_bias"], ex["gate"].tobytes(),
                                ex["up"].tobytes(), ex["down"].tobytes(), dense["sh_gate"].tobytes(),
                                dense["sh_up"].tobytes(), dense["sh_down"].tobytes(), norm, E, D, F)
    data, _, _ = gguf_bytes([("general.architecture", "str", "sf37")], tensors)
    path = tmp_path / "layer.gguf"
    path.write_bytes(data)
    g = L.sf37_hip_gguf_open(str(path).encode())
    assert g
    try:
        w = H.LayerWeights()
        pn = C.c_uint64()
        assert L.sf37_hip_gguf_bind_moe_layer(g, il, C.byref(w), C.byref(pn))
        assert (w.n_expert, w.in_dim, w.mid_dim, w.topk) == (E, D, F, 8)
        assert w.clamp_routed == 7.0 and w.clamp_shared == 16.0
        size = C.c_uint64()
        gmap = L.sf37_hip_gguf_map(g, C.byref(size))
        # reference: the same layer from its device tensors, norm weights registered under a key
        key = np.zeros(64, np.uint8)
        nt = H.Tensor.from_array(norm)
        H.check(L.sf37_hip_register_device_range(key.ctypes.data, nt.nbytes, 0, nt.nbytes, nt), "register")
        ref_w = lay.weights_struct()
        for n_tok in (3, 40):
            h0 = (rng.standard_normal((n_tok, D)) * 2).astype(np.float32)
            lg = H.Tensor.from_array(configs.logits_for(4, il * 10 + n_tok, n_tok, n_expert=E))
            outs = []
            for ww, mp, ms, off in ((w, gmap, size.value, pn.value), (ref_w, key.ctypes.data, nt.nbytes, 0)):
                h = H.Tensor.from_array(h0)
                H.check(L.sf37_hip_moe_block(h, None, None, None, C.byref(ww), mp, ms, off, 1e-5, lg, n_tok),
                        "moe_block")
                outs.append(h.read(np.float32))
            assert_bitexact(outs[0], outs[1], f"layer {il}, {n_tok} tokens")
    finally:
        L.sf37_hip_gguf_close(g)
        lay.free()
