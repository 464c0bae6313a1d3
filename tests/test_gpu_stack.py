"""GPU parity of the layer stack: h <- h + MoE_l(RMSNorm_l(h))
over independently seeded layers, against the CPU oracle run layer by layer
(orc_rms_norm_weight1_bf16, moe_layer_q8k, float add), bit for bit.

Cases: a reduced-shape stack over layers 42..44 (the SwiGLU clamps of layers
43/44) at 3 tokens (fused decode path) and 40 tokens (matrix-core prefill
path for both the routed and the shared expert); the BASELINE shape over
layers 43/44 at one token.  Router logits are injected per layer (Zipf
skewed, as config 4) so routing is compared for the same logits.
"""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
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
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"{np.ravel(got)[bad[0]]!r} vs {np.ravel(want)[bad[0]]!r}")


def oracle_stack(O, stack, h, logits):
    """The stack on the CPU, layer by layer."""
    K = stack.in_dim
    h = np.array(h, np.float32, copy=True)
    n_tok = h.shape[0]
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    for l, lay in enumerate(stack.layers):
        xn = np.zeros_like(h)
        w = np.ascontiguousarray(stack.norm_bits[l])
        for t in range(n_tok):
            row = np.ascontiguousarray(h[t])
            out = np.zeros(K, np.float32)
            O.lib().orc_rms_norm_weight1_bf16(fp(out), fp(row), w.ctypes.data_as(C.POINTER(C.c_uint16)), K,
                                              stack.EPS)
            xn[t] = out
        sel, _, _ = O.router_select(logits[l], np.zeros(lay.n_expert, np.float32), lay.topk, 3.0)
        weights = dict(lay.host_experts(np.append(np.ravel(sel), 0)), **lay.host_dense(), n_expert=lay.n_expert,
                       mid_dim=lay.mid_dim)
        y, _, _ = O.moe_layer_q8k(weights, xn, logits=logits[l], topk=lay.topk, clamp_routed=lay.clamp_routed,
                                  clamp_shared=lay.clamp_shared)
        h = (h + y).astype(np.float32)
    return h


def run_stack(H, stack, h0, logits, native=True):
    n_tok, K = h0.shape
    h = H.Tensor.from_array(h0)
    xn, y = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * K * 4)
    lts = [H.Tensor.from_array(lg) for lg in logits]
    stack.forward(h, n_tok, xn, y, None, None, lts, native=native)
    return h.read(np.float32).reshape(n_tok, K)


@pytest.fixture(scope="module")
def small_stack(H):
    from sf37_amd.moe import SynthStack
    say("reduced-shape stack, layers 42..44")
    S = SynthStack(master=11, n_layers=3, il0=42, n_expert=16, in_dim=512, mid_dim=256, topk=4)
    H.synchronize()
    yield S
    S.free()


@pytest.mark.parametrize("n_tok", [1, 3, 16, 17, 40])
def test_small_stack_vs_oracle(H, O, small_stack, n_tok):
    """sf37_hip_moe_stack (fused norm + residual up to 16 tokens, the
    single-token variant at 1, rms_norm + layer + one residual add above) and
    the per-layer entry points, both against the oracle."""
    from sf37_amd import configs
    S = small_stack
    for k in ("q8k_min_rows", "prefill_min_pairs", "shared_min_tokens"):
        H.set_option(k, 0)
    rng = np.random.default_rng(40 + n_tok)
    h0 = rng.standard_normal((n_tok, S.in_dim)).astype(np.float32)
    logits = [configs.logits_for(4, 700 + l, n_tok, n_expert=16) for l in range(S.n_layers)]
    got = {}
    for native in (True, False):
        H.lib().sf37_hip_profile_enable(1)
        H.profile_read()
        try:
            got[native] = run_stack(H, S, h0, logits, native)
            prof = H.profile_read()
        finally:
            H.lib().sf37_hip_profile_enable(0)
        if n_tok > 16:
            assert prof["pf_gate_up"][1] == S.n_layers and prof["sh_gate_up"][1] == S.n_layers
            # the routed combine adds the shared rows (and, in the stack call, the residual)
            assert prof["add"][1] == (0 if native else S.n_layers), prof["add"]
        else:
            assert prof["dec_up"][1] == S.n_layers
            # the stack call's decode launches take the norm and the residual
            assert prof["other"][1] == (0 if native else S.n_layers), prof["other"]
    say(f"oracle: {S.n_layers} layers x {n_tok} tokens")
    want = oracle_stack(O, S, h0, logits)
    assert_bitexact(got[True], want, f"stack call output, {n_tok} tokens")
    assert_bitexact(got[False], want, f"per-layer calls output, {n_tok} tokens")


def test_block_normed_rows(H, small_stack):
    """sf37_hip_moe_block's optional normalised rows equal the standalone
    rms_norm entry point's, on the fused (5 tokens) and staged (20) paths."""
    import ctypes as C
    S = small_stack
    H.set_option("q8k_min_rows", 0)
    for n_tok in (5, 20):
        rng = np.random.default_rng(n_tok)
        h0 = (rng.standard_normal((n_tok, S.in_dim)) * 3).astype(np.float32)
        h, normed = H.Tensor.from_array(h0), H.Tensor.alloc(n_tok * S.in_dim * 4)
        ref = H.Tensor.alloc(n_tok * S.in_dim * 4)
        S.rms_norm(ref, H.Tensor.from_array(h0), 1, n_tok)
        H.check(H.lib().sf37_hip_moe_block(h, normed, None, None, C.byref(S._structs[1]), S._key.ctypes.data,
                                           S.norm.nbytes, S._offsets[1], S.EPS, None, n_tok), "moe_block")
        assert_bitexact(normed.read(np.float32), ref.read(np.float32), f"normed rows, {n_tok} tokens")


def test_baseline_shape_stack_layers_43_44(H, O):
    """Layers 43 and 44 at the BASELINE shape (clamps 7 / 16), one token."""
    from sf37_amd import configs
    from sf37_amd.moe import SynthStack
    say("BASELINE-shape stack, layers 43..44")
    S = SynthStack(master=12, n_layers=2, il0=43)
    try:
        rng = np.random.default_rng(4344)
        h0 = (rng.standard_normal((1, S.in_dim)) * 4).astype(np.float32)
        logits = [configs.logits_for(4, 800 + l, 1) for l in range(S.n_layers)]
        got = run_stack(H, S, h0, logits)
        want = oracle_stack(O, S, h0, logits)
        assert_bitexact(got, want, "stack output, 1 token")
    finally:
        S.free()
