"""GGUF-resident MoE layers (sf37_hip_gguf_bind_moe_layer) against the CPU
oracle and against the same layers from device tensors.

Reduced-shape layers written by the engine's tensor contract
(sf37.c:1760-1782) run through sf37_hip_moe_block at 3 tokens (fused decode)
and 40 tokens (matrix-core prefill): layer 43 with an F32 router, layer 44
with a BF16 router, a Q8_0 router (logits computed by the block) and a
Q3GU/Q2D shared expert.  Also: binding all 42 MoE layers of a file on one
handle, eviction of the on-demand cache after binding (bound layers are
registered ranges, not cache entries), and undersized weight tensors
refused before any launch.
"""
import ctypes as C

import numpy as np
import pytest

from gguf_writer import T_BF16, T_F32, T_Q8_0, gguf_bytes, moe_layer_tensors

pytestmark = pytest.mark.gpu

E, D, F = 16, 512, 256


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
    for k in ("q8k_min_rows", "prefill_min_pairs", "shared_min_tokens"):
        hip.set_option(k, 0)
    yield hip
    for k, v in (("q8k_min_rows", 512), ("prefill_min_pairs", 256), ("shared_min_tokens", 64)):
        hip.set_option(k, v)
    hip.synchronize()


@pytest.fixture(scope="module")
def O():
    import oracle
    oracle.lib()
    return oracle


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got, np.float32).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want, np.float32).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ"


fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))


def layer_file(O, lay, il, router_type, norm):
    """GGUF bytes of one SynthLayer by the engine's contract, plus the host
    weights dict for the oracle."""
    dense = lay.host_dense()
    ex = lay.host_experts(np.arange(E))
    router = dense["router"]
    if router_type == T_BF16:
        from sf37_amd.moe import bf16_bits
        rbits = bf16_bits(router)
        router_host = (rbits.astype(np.uint32) << 16).view(np.float32)
        rdata = rbits
    elif router_type == T_Q8_0:
        rdata = O.quantize_rows("q8_0", router.reshape(E, D))
        router_host = rdata
    else:
        rdata = router_host = router
    tensors = moe_layer_tensors(il, rdata, router_type, dense["router_bias"], ex["gate"].tobytes(),
                                ex["up"].tobytes(), ex["down"].tobytes(), dense["sh_gate"].tobytes(),
                                dense["sh_up"].tobytes(), dense["sh_down"].tobytes(), norm, E, D, F,
                                shared_q3q2=lay.shared == "q3q2")
    w = dict(ex, **dense, n_expert=E, mid_dim=F)
    w["router"] = router_host
    return tensors, w


def oracle_block(O, w, norm, h0, logits, il, router_type, shared):
    """h0 + layer(RMSNorm(h0)); logits None = the router computes them."""
    n_tok = h0.shape[0]
    xn = np.zeros_like(h0)
    nb = np.ascontiguousarray(norm)
    for t in range(n_tok):
        O.lib().orc_rms_norm_weight1_bf16(fp(xn[t]), fp(np.ascontiguousarray(h0[t])),
                                          nb.ctypes.data_as(C.POINTER(C.c_uint16)), D, 1e-5)
    if logits is None and router_type == T_Q8_0:
        logits = np.zeros((n_tok, E), np.float32)
        for t in range(n_tok):
            O.lib().orc_q8_0_matvec(fp(logits[t]), w["router"].ctypes.data_as(C.POINTER(C.c_uint8)), D, E,
                                    fp(np.ascontiguousarray(xn[t])))
    cl = (7.0, 16.0) if il in (43, 44) else (0.0, 0.0)
    y, _, _ = O.moe_layer_q8k(w, xn, logits=logits, clamp_routed=cl[0], clamp_shared=cl[1],
                              shared_format=shared)
    return (h0 + y).astype(np.float32)


CASES = [(43, T_F32, "q8_0", True), (44, T_BF16, "q8_0", True), (44, T_Q8_0, "q8_0", False),
         (43, T_F32, "q3q2", True)]


@pytest.mark.parametrize("il,router_type,shared,inject", CASES)
def test_gguf_layer_vs_oracle_and_device_layer(H, O, tmp_path, il, router_type, shared, inject):
    from sf37_amd import configs
    from sf37_amd.moe import SynthLayer, bf16_bits
    L = H.lib()
    lay = SynthLayer(seed=500 + il + router_type, n_expert=E, in_dim=D, mid_dim=F, topk=8, il=il, shared=shared)
    rng = np.random.default_rng(il)
    norm = bf16_bits((rng.standard_normal(D) * 0.02).astype(np.float32))
    tensors, w_host = layer_file(O, lay, il, router_type, norm)
    if router_type == T_BF16:
        lay.router.write(w_host["router"])          # the device layer gets the widened router
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
        assert w.router_type == (0 if router_type == T_F32 else router_type)
        assert w.shared_type == (H.TYPE_Q3GU if shared == "q3q2" else 0)
        size = C.c_uint64()
        gmap = L.sf37_hip_gguf_map(g, C.byref(size))
        key = np.zeros(64, np.uint8)
        nt = H.Tensor.from_array(norm)
        H.check(L.sf37_hip_register_device_range(key.ctypes.data, nt.nbytes, 0, nt.nbytes, nt), "register")
        ref_w = lay.weights_struct()
        for n_tok in (3, 40):
            h0 = (rng.standard_normal((n_tok, D)) * 2).astype(np.float32)
            lg_host = configs.logits_for(4, il * 10 + n_tok, n_tok, n_expert=E) if inject else None
            lg = H.Tensor.from_array(lg_host) if inject else None
            h = H.Tensor.from_array(h0)
            H.check(L.sf37_hip_moe_block(h, None, None, None, C.byref(w), gmap, size.value, pn.value, 1e-5, lg,
                                         n_tok), "moe_block (GGUF)")
            got = h.read(np.float32).reshape(n_tok, D)
            want = oracle_block(O, w_host, norm, h0, lg_host, il, router_type, shared)
            assert_bitexact(got, want, f"GGUF layer {il} vs oracle, {n_tok} tokens")
            if router_type != T_Q8_0:
                h2 = H.Tensor.from_array(h0)
                H.check(L.sf37_hip_moe_block(h2, None, None, None, C.byref(ref_w), key.ctypes.data, nt.nbytes, 0,
                                             1e-5, lg, n_tok), "moe_block (device)")
                assert_bitexact(got, h2.read(np.float32), f"GGUF layer {il} vs device layer, {n_tok} tokens")
    finally:
        L.sf37_hip_gguf_close(g)
        lay.free()


def test_gguf_all_layers_one_handle_and_evict(H, O, tmp_path):
    """42 MoE layers (3..44) of one file bound on one handle; the on-demand
    cache evicted after binding; layers 3 and 44 then run against the oracle."""
    from sf37_amd import configs
    from sf37_amd.moe import SynthLayer, bf16_bits
    L = H.lib()
    lay = SynthLayer(seed=900, n_expert=E, in_dim=D, mid_dim=F, topk=8, il=3)
    norm = bf16_bits((np.random.default_rng(9).standard_normal(D) * 0.02).astype(np.float32))
    tensors, w_host = [], None
    for il in range(3, 45):
        t, w_host = layer_file(O, lay, il, T_F32, norm)
        tensors += t
    data, _, _ = gguf_bytes([("general.architecture", "str", "sf37")], tensors)
    path = tmp_path / "layers.gguf"
    path.write_bytes(data)
    g = L.sf37_hip_gguf_open(str(path).encode())
    assert g
    try:
        ws, pns = {}, {}
        for il in range(3, 45):
            w, pn = H.LayerWeights(), C.c_uint64()
            assert L.sf37_hip_gguf_bind_moe_layer(g, il, C.byref(w), C.byref(pn)), f"bind layer {il}"
            ws[il], pns[il] = w, pn.value
        L.sf37_hip_evict_model_cache(b"after binding")
        size = C.c_uint64()
        gmap = L.sf37_hip_gguf_map(g, C.byref(size))
        rng = np.random.default_rng(44)
        for il in (3, 44):
            h0 = (rng.standard_normal((3, D)) * 2).astype(np.float32)
            lg_host = configs.logits_for(4, il, 3, n_expert=E)
            h = H.Tensor.from_array(h0)
            H.check(L.sf37_hip_moe_block(h, None, None, None, C.byref(ws[il]), gmap, size.value, pns[il], 1e-5,
                                         H.Tensor.from_array(lg_host), 3), f"moe_block layer {il}")
            want = oracle_block(O, w_host, norm, h0, lg_host, il, T_F32, "q8_0")
            assert_bitexact(h.read(np.float32).reshape(3, D), want, f"layer {il} after evict")
    finally:
        L.sf37_hip_gguf_close(g)
        lay.free()


def test_gguf_two_handles_share_ranges(H, O):
    """Two from_map handles on one caller map bind the same layer: the device
    ranges are shared and held twice (registry query, no kernel); closing one
    handle leaves the other's ranges registered and its layer exact against
    the oracle; closing the second frees them."""
    from sf37_amd import configs
    from sf37_amd.moe import SynthLayer, bf16_bits
    L = H.lib()
    il = 44
    lay = SynthLayer(seed=321, n_expert=E, in_dim=D, mid_dim=F, topk=8, il=il)
    norm = bf16_bits((np.random.default_rng(321).standard_normal(D) * 0.02).astype(np.float32))
    tensors, w_host = layer_file(O, lay, il, T_F32, norm)
    data, _, _ = gguf_bytes([("general.architecture", "str", "sf37")], tensors)
    buf = np.frombuffer(data, np.uint8).copy()          # the caller's map; outlives both handles
    ga = L.sf37_hip_gguf_from_map(buf.ctypes.data, buf.nbytes)
    gb = L.sf37_hip_gguf_from_map(buf.ctypes.data, buf.nbytes)
    assert ga and gb
    names = ["moe.gate_proj.weight", "moe.down_proj.weight", "share_expert.up_proj.weight", "moe.gate.weight"]
    ext = []
    for n in names:
        off, nb, ty, nd = C.c_uint64(), C.c_uint64(), C.c_uint32(), C.c_uint32()
        dims = (C.c_uint64 * 4)()
        assert L.sf37_hip_gguf_tensor(ga, f"model.layers.{il}.{n}".encode(), C.byref(off), C.byref(nb),
                                      C.byref(ty), C.byref(nd), dims)
        ext.append((off.value, nb.value))
    closed_b = False
    try:
        wa, wb, pa, pb = H.LayerWeights(), H.LayerWeights(), C.c_uint64(), C.c_uint64()
        assert L.sf37_hip_gguf_bind_moe_layer(ga, il, C.byref(wa), C.byref(pa))
        assert [L.sf37_hip_model_range_holds(buf.ctypes.data, o, b) for o, b in ext] == [1] * 4
        assert L.sf37_hip_gguf_bind_moe_layer(gb, il, C.byref(wb), C.byref(pb))
        assert [L.sf37_hip_model_range_holds(buf.ctypes.data, o, b) for o, b in ext] == [2] * 4
        H.synchronize()
        L.sf37_hip_gguf_close(ga)
        ga = None
        assert [L.sf37_hip_model_range_holds(buf.ctypes.data, o, b) for o, b in ext] == [1] * 4
        h0 = (np.random.default_rng(5).standard_normal((3, D)) * 2).astype(np.float32)
        lg_host = configs.logits_for(4, 4401, 3, n_expert=E)
        h = H.Tensor.from_array(h0)
        H.check(L.sf37_hip_moe_block(h, None, None, None, C.byref(wb), buf.ctypes.data, buf.nbytes, pb.value, 1e-5,
                                     H.Tensor.from_array(lg_host), 3), "moe_block on the handle left open")
        want = oracle_block(O, w_host, norm, h0, lg_host, il, T_F32, "q8_0")
        assert_bitexact(h.read(np.float32).reshape(3, D), want, "layer after the other handle closed")
        L.sf37_hip_gguf_close(gb)
        closed_b = True
        assert [L.sf37_hip_model_range_holds(buf.ctypes.data, o, b) for o, b in ext] == [-1] * 4
    finally:
        if ga:
            L.sf37_hip_gguf_close(ga)
        if not closed_b:
            L.sf37_hip_gguf_close(gb)
        lay.free()


def test_undersized_weights_refused(H):
    """A layer whose gate tensor is one byte short returns 0 with no launch."""
    from sf37_amd.moe import SynthLayer
    L = H.lib()
    lay = SynthLayer(seed=77, n_expert=E, in_dim=D, mid_dim=F, topk=8)
    try:
        short = lay.gate.view(0, lay.gate.nbytes - 1)
        w = lay.weights_struct()
        w.gate = short.h
        x = H.synth_normal(2 * D, 1, 2)
        out = H.Tensor.alloc(2 * D * 4)
        lg = H.Tensor.from_array(np.zeros((2, E), np.float32))
        assert L.sf37_hip_moe_layer(out, None, None, C.byref(w), lg, x, 2) == 0
        w = lay.weights_struct()
        w.router_type = 5                               # not a router type the layer reads
        assert L.sf37_hip_moe_layer(out, None, None, C.byref(w), lg, x, 2) == 0
        w = lay.weights_struct()
        assert L.sf37_hip_moe_layer(out, None, None, C.byref(w), lg, x, 2) == 1
        H.synchronize()
    finally:
        lay.free()
