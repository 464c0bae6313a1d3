"""The BASELINE configurations' shared expert "in the same formats": Q3GU
gate/up and Q2D down, run on the Q8_K path as one more expert with routing
weight 1.0 and the shared clamp (shared_type 11), against the oracle's
composition of the same (oracle.moe_layer_q8k(shared_format="q3q2")), bit for
bit, at the BASELINE shape: config 0 (one token, router logits computed on
the device and fed to the oracle), config 1 (8 tokens), config 3 (4096
tokens, uniform routing) on a token sample, and layer 43's clamps; and the
decode form that runs it as one more slot of every token inside the routed
launches against the form that runs it as launches of its own.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, K, F = 288, 4096, 1280
_KEEP = []


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
    yield hip
    hip.synchronize()


@pytest.fixture(scope="module")
def O():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="module", params=[3, 43])
def layer(H, request):
    from sf37_amd.moe import SynthLayer
    say(f"BASELINE-shape layer with a Q3GU/Q2D shared expert (layer {request.param})")
    L = SynthLayer(seed=3311 + request.param, il=request.param, shared="q3q2")
    H.synchronize()
    yield L
    L.free()


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got, np.float32).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want, np.float32).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"{np.ravel(got)[bad[0]]!r} vs {np.ravel(want)[bad[0]]!r}")


@pytest.mark.parametrize("config", [0, 1, 3])
def test_shared_q3q2_layer_vs_oracle(H, O, layer, config):
    from sf37_amd import configs, moe
    n_tok = configs.CONFIG_TOKENS[config]
    say(f"config {config}: {n_tok} tokens, layer {layer.il}")
    seed = 77 + config
    scale = 4.0 if layer.il == 43 else 1.0          # clamps 7 / 16 bind at layer 43
    x = (configs.x_device(config, seed, n_tok).read(np.float32) * np.float32(scale)).reshape(n_tok, K)
    logits = configs.logits_for(config, seed, n_tok)
    xt = H.Tensor.from_array(x)
    out, sel, w = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * 32), H.Tensor.alloc(n_tok * 32)
    moe.moe_layer(layer, xt, n_tok, out, sel, w, H.Tensor.from_array(logits) if logits is not None else None)
    out = out.read(np.float32).reshape(n_tok, K)
    sel = sel.read(np.int32).reshape(n_tok, 8)
    w = w.read(np.float32).reshape(n_tok, 8)
    if logits is None:
        lt = H.Tensor.alloc(n_tok * E * 4)
        H.check(H.lib().sf37_hip_matvec_f32(lt.h, layer.router.h, K, E, xt), "logits")
        logits = lt.read(np.float32).reshape(n_tok, E)
    idx = np.arange(n_tok) if n_tok <= 8 else np.random.default_rng(3).choice(n_tok, 6, replace=False)
    weights = dict(layer.host_experts(np.append(np.ravel(sel[idx]), 0)), **layer.host_dense(), n_expert=E,
                   mid_dim=F)
    want, wsel, ww = O.moe_layer_q8k(weights, x[idx], logits=logits[idx], clamp_routed=layer.clamp_routed,
                                     clamp_shared=layer.clamp_shared, shared_format="q3q2")
    assert np.array_equal(sel[idx], wsel)
    assert_bitexact(w[idx], ww, "routing weights")
    assert_bitexact(out[idx], want, f"config {config} layer {layer.il} output")


@pytest.mark.parametrize("n_tok", [1, 3, 8, 16])
def test_shared_slot_equals_separate_launches(H, layer, n_tok):
    """Decode batches run the Q3GU/Q2D shared expert as one more slot of
    every token inside the routed launches, its pairs grouped two at a time
    (option decode_shared_slot, on by default: one route launch per layer);
    with the option off it runs as launches of its own (two route
    launches).  Outputs, selections and routing weights agree bit for bit."""
    from sf37_amd import moe
    rng = np.random.default_rng(900 + n_tok)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    got = {}
    for slot in (1, 0):
        say(f"shared slot {slot}: {n_tok} tokens, layer {layer.il}")
        H.set_option("decode_shared_slot", slot)
        H.lib().sf37_hip_profile_enable(1)
        H.profile_read()
        try:
            out, sel, w = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * 32), H.Tensor.alloc(n_tok * 32)
            moe.moe_layer(layer, H.Tensor.from_array(x), n_tok, out, sel, w, H.Tensor.from_array(logits))
            prof = H.profile_read()
            got[slot] = (out.read(np.float32), sel.read(np.int32), w.read(np.float32))
        finally:
            H.lib().sf37_hip_profile_enable(0)
            H.set_option("decode_shared_slot", 1)
        assert prof["dec_route"][1] == (1 if slot else 2), prof["dec_route"]
        if slot and n_tok == 1:   # nine slots: down and combine still one launch
            assert prof["dec_down"][1] == 1 and prof["dec_combine"][1] == 0, prof
    assert np.array_equal(got[1][1], got[0][1])
    assert_bitexact(got[1][2], got[0][2], "routing weights")
    assert_bitexact(got[1][0], got[0][0], f"output, {n_tok} tokens")


@pytest.mark.parametrize("n_tok", [1, 8])
def test_shared_slot_in_ffn_block(H, layer, n_tok):
    """sf37_hip_moe_block (RMSNorm(w+1) of the hidden rows, the layer, the
    residual) with the Q3GU/Q2D shared expert as a decode slot equals the
    same block with the shared expert's own launches, bit for bit, and the
    normalised rows it returns equal the standalone RMSNorm's."""
    import ctypes as C
    from sf37_amd import moe
    rng = np.random.default_rng(1300 + n_tok)
    norm = H.Tensor.from_array(moe.bf16_bits((rng.standard_normal(K) * 0.02).astype(np.float32)))
    key = np.zeros(64, np.uint8)                 # host address used as the map key
    _KEEP.append((key, norm))                    # registered for the session: no later key reuses it
    H.check(H.lib().sf37_hip_register_device_range(key.ctypes.data, norm.nbytes, 0, norm.nbytes, norm.h),
            "register norm weights")
    h0 = (rng.standard_normal((n_tok, K)) * 3).astype(np.float32)
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    got = {}
    try:
        for slot in (1, 0):
            say(f"FFN block, shared slot {slot}: {n_tok} tokens, layer {layer.il}")
            H.set_option("decode_shared_slot", slot)
            h, normed = H.Tensor.from_array(h0), H.Tensor.alloc(n_tok * K * 4)
            H.check(H.lib().sf37_hip_moe_block(h, normed, None, None, C.byref(layer.weights_struct()),
                                               key.ctypes.data, norm.nbytes, 0, 1e-5,
                                               H.Tensor.from_array(logits), n_tok), "moe_block")
            got[slot] = (h.read(np.float32), normed.read(np.float32))
    finally:
        H.set_option("decode_shared_slot", 1)
    assert_bitexact(got[1][1], got[0][1], "normalised rows")
    assert_bitexact(got[1][0], got[0][0], f"hidden rows, {n_tok} tokens")
