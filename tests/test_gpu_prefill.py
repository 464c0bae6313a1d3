"""GPU parity of the matrix-core prefill path (k_prefill.hip).

The MFMA kernels form the same exact integer group sums as the dot-product
kernels and run the canonical float epilogue, so every output must equal the
staged path (option prefill_mfma=0) and the CPU oracle bit for bit.  Cases:
a small layer with an odd number of 256-blocks per row, a group larger than
one 128-pair tile, an invalid expert id and an expert repeated inside a
token; the BASELINE layer at config 2 (Zipf routing, idle experts, groups
of hundreds of pairs) and skewed batches (eight experts taken by all or half
of the tokens) against the staged path; config 3 (4096 tokens) on a sample
of tokens against the oracle.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, K, F, TOPK = 288, 4096, 1280, 8


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
    yield hip
    hip.set_option("prefill_mfma", 1)
    hip.synchronize()


@pytest.fixture(scope="module")
def O():
    import oracle
    oracle.lib()
    return oracle


_KEYS = []


def map_key():
    k = np.zeros(64, np.uint8)
    _KEYS.append(k)
    return k.ctypes.data


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got, np.float32).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want, np.float32).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"{np.ravel(got)[bad[0]]!r} vs {np.ravel(want)[bad[0]]!r}")


def batch_run(H, layer, sel, w, x, mfma):
    """routed_moe_batch_mapped over the layer's experts; returns out, per-pair mid
    and the launch counts of the matrix-core stages."""
    n_tok, topk = sel.shape
    gb, db = layer.gate.nbytes, layer.down.nbytes
    total = 2 * gb + db
    key = map_key()
    L = H.lib()
    for off, t in ((0, layer.gate), (gb, layer.up), (2 * gb, layer.down)):
        H.check(L.sf37_hip_register_device_range(key, total, off, t.nbytes, t), "register")
    D, Fm = layer.in_dim, layer.mid_dim
    st, wt, xt = H.Tensor.from_array(sel), H.Tensor.from_array(w), H.Tensor.from_array(x)
    out, g, u, d = H.Tensor.alloc(n_tok * D * 4), H.Tensor.alloc(topk * Fm * 4), \
        H.Tensor.alloc(topk * Fm * 4), H.Tensor.alloc(topk * D * 4)
    m = H.Tensor.alloc(n_tok * topk * Fm * 4)
    H.set_option("prefill_mfma", 1 if mfma else 0)
    L.sf37_hip_profile_enable(1)
    H.profile_read()
    try:
        H.check(L.sf37_hip_routed_moe_batch_mapped(out, g, u, m, d, key, total, 0, gb, 2 * gb, st, wt,
                                                   layer.n_expert, topk, D, Fm, D, layer.clamp_routed, xt,
                                                   n_tok), "batch")
        prof = H.profile_read()
    finally:
        L.sf37_hip_profile_enable(0)
        H.set_option("prefill_mfma", 1)
    return (out.read(np.float32).reshape(n_tok, D), m.read(np.float32).reshape(n_tok * topk, Fm),
            prof["pf_gate_up"][1] + prof["pf_down"][1])


def test_small_layer_odd_blocks_vs_oracle(H, O):
    """6 experts, in 768 (3 blocks, odd), mid 256, 150 tokens x top-4: expert 2
    in every token (150 pairs = two tiles), an invalid id, a repeated expert."""
    from sf37_amd.moe import SynthLayer
    n_exp, D, Fm, n_tok, topk = 6, 768, 256, 150, 4
    L = SynthLayer(seed=31, n_expert=n_exp, in_dim=D, mid_dim=Fm)
    rng = np.random.default_rng(7)
    sel = np.stack([rng.permutation([0, 1, 3, 4, 5])[:topk] for _ in range(n_tok)]).astype(np.int32)
    sel[:, 1] = 2
    sel[10, 3] = -1
    sel[20, 2] = sel[20, 0]
    w = (rng.random((n_tok, topk)) * 0.5).astype(np.float32)
    x = rng.standard_normal((n_tok, D)).astype(np.float32)
    H.set_option("q8k_min_rows", 0)
    try:
        say("small layer: matrix-core path")
        a = batch_run(H, L, sel, w, x, True)
        say("small layer: staged path")
        b = batch_run(H, L, sel, w, x, False)
    finally:
        H.set_option("q8k_min_rows", 512)
    assert a[2] == 2 and b[2] == 0, "matrix-core kernels did not run as selected"
    assert_bitexact(a[1], b[1], "mid mfma vs staged")
    assert_bitexact(a[0], b[0], "out mfma vs staged")
    host = L.host_experts(np.arange(n_exp))
    want, want_mid = O.routed_moe_batch_q8k(host["gate"], host["up"], host["down"], sel, w, n_exp, D, Fm, D,
                                            L.clamp_routed, x)
    assert_bitexact(a[1], want_mid, "mid vs oracle")
    assert_bitexact(a[0], want, "out vs oracle")
    L.free()


@pytest.fixture(scope="module")
def layer(H):
    from sf37_amd.moe import SynthLayer
    say("generating BASELINE-shape layer (seed 91)")
    L = SynthLayer(seed=91)
    H.synchronize()
    yield L
    L.free()


def test_config2_batch_mfma_equals_staged(H, layer):
    """512 tokens, Zipf routing (config 2's logits): out and every pair's mid
    equal the staged path bit for bit."""
    from sf37_amd import configs
    import oracle as O
    n_tok = 512
    x = configs.x_device(2, 4321, n_tok).read(np.float32).reshape(n_tok, K)
    logits = configs.logits_for(2, 4321, n_tok)
    sel, w, _ = O.router_select(logits, np.zeros(E, np.float32), TOPK, 3.0)
    counts = np.bincount(sel.ravel(), minlength=E)
    assert counts.max() > 128 and (counts == 0).any()
    say(f"config 2 batch: largest group {counts.max()} pairs")
    a = batch_run(H, layer, sel, w, x, True)
    b = batch_run(H, layer, sel, w, x, False)
    assert a[2] == 2 and b[2] == 0
    assert_bitexact(a[1], b[1], "config 2 mid")
    assert_bitexact(a[0], b[0], "config 2 out")


@pytest.mark.parametrize("n_tok,hot_frac", [(200, 1.0), (700, 1.0), (700, 0.5)])
def test_batch_hot_experts_mfma_equals_staged(H, layer, n_tok, hot_frac):
    """Skewed batches: a share of the tokens (all, or every other one) select
    the same eight experts (boosted logits, distinct boosts so the slot
    order is fixed), the rest route at random: groups of hundreds of pairs
    cut into many 64-pair tiles, beside groups of a few pairs or (all hot)
    280 idle experts.  out and every pair's mid equal the staged path bit
    for bit."""
    import oracle as O
    rng = np.random.default_rng(8100 + n_tok + int(hot_frac * 10))
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    hot = rng.choice(E, size=TOPK, replace=False)
    rows = np.arange(n_tok) if hot_frac == 1.0 else np.arange(0, n_tok, 2)
    for k, e in enumerate(hot):
        logits[rows, e] += np.float32(12.0 + k)
    sel, w, _ = O.router_select(logits, np.zeros(E, np.float32), TOPK, 3.0)
    counts = np.bincount(sel.ravel(), minlength=E)
    assert counts[hot].min() >= len(rows)
    assert hot_frac < 1.0 or (counts == 0).sum() == E - TOPK
    say(f"hot batch: {n_tok} tokens, {len(rows)} on the hot experts, largest group {counts.max()} pairs")
    a = batch_run(H, layer, sel, w, x, True)
    b = batch_run(H, layer, sel, w, x, False)
    assert a[2] == 2 and b[2] == 0
    assert_bitexact(a[1], b[1], f"hot batch mid ({n_tok} tokens)")
    assert_bitexact(a[0], b[0], f"hot batch out ({n_tok} tokens)")


def test_config3_layer_sample_vs_oracle(H, O, layer):
    """4096 tokens, uniform routing, the whole layer (shared + routed) on the
    device; 6 tokens checked bit-exactly against the oracle."""
    from sf37_amd import configs, moe
    n_tok = 4096
    x = configs.x_device(3, 99, n_tok).read(np.float32).reshape(n_tok, K)
    logits = configs.logits_for(3, 99, n_tok)
    say("config 3 layer on the device")
    xt = H.Tensor.from_array(x)
    out, sel, w = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * 32), H.Tensor.alloc(n_tok * 32)
    H.lib().sf37_hip_profile_enable(1)
    H.profile_read()
    try:
        moe.moe_layer(layer, xt, n_tok, out, sel, w, H.Tensor.from_array(logits))
        prof = H.profile_read()
    finally:
        H.lib().sf37_hip_profile_enable(0)
    assert prof["pf_gate_up"][1] == 1 and prof["pf_down"][1] == 1
    out = out.read(np.float32).reshape(n_tok, K)
    sel = sel.read(np.int32).reshape(n_tok, TOPK)
    idx = np.array([0, 1, 777, 2048, 3000, 4095])
    dense = layer.host_dense()
    weights = dict(layer.host_experts(np.append(np.ravel(sel[idx]), 0)), **dense, n_expert=E, mid_dim=F)
    say("oracle on 6 tokens")
    want, wsel, _ = O.moe_layer_q8k(weights, x[idx], logits=logits[idx], clamp_routed=layer.clamp_routed,
                                    clamp_shared=layer.clamp_shared)
    assert np.array_equal(sel[idx], wsel)
    assert_bitexact(out[idx], want, "config 3 sample")


@pytest.mark.parametrize("n_tok", [77, 300, 1100])
def test_layer_mfma_equals_staged(H, layer, n_tok):
    """Whole layer (router on the device, shared expert and routed experts on
    the matrix cores) against the dot-product kernels (prefill_mfma=0), bit for
    bit; token counts that leave partial 32- and 64-token tiles (77 and 300:
    the shared GEMM's 64-column form with its batched chunk body, 1100: the
    same form over more than one round, with the other body).  The matrix-
    core layer runs with the shared expert on the side stream (joined before
    the routed combine) and in order on the library stream."""
    from sf37_amd import moe
    rng = np.random.default_rng(300 + n_tok)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    res = []
    for mfma, side in ((1, 1), (1, 0), (0, 1)):
        H.set_option("prefill_mfma", mfma)
        H.set_option("shared_stream", side)
        H.lib().sf37_hip_profile_enable(1)
        H.profile_read()
        try:
            xt = H.Tensor.from_array(x)
            out, sel, w = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * 32), H.Tensor.alloc(n_tok * 32)
            moe.moe_layer(layer, xt, n_tok, out, sel, w, None)
            prof = H.profile_read()
        finally:
            H.lib().sf37_hip_profile_enable(0)
            H.set_option("prefill_mfma", 1)
            H.set_option("shared_stream", 1)
        ran = prof["sh_gate_up"][1] + prof["pf_gate_up"][1]
        assert ran == (2 if mfma else 0), f"matrix-core kernels ran {ran} times with prefill_mfma={mfma}"
        res.append((out.read(np.float32), sel.read(np.int32)))
    for r, what in ((res[0], "side stream"), (res[1], "one stream")):
        assert np.array_equal(r[1], res[2][1])
        assert_bitexact(r[0], res[2][0], f"layer out ({what}), {n_tok} tokens")
