"""GPU parity of the fused decode path (three launches for up to 16 tokens).

The fused kernels and the staged kernels (one launch per stage, option
decode_fused=0) follow the same canonical operation order, so every output
must agree bit for bit; each shape is also checked against the CPU oracle on
a case the oracle finishes in seconds.  Cases cover token counts 1..16, odd
counts, experts shared by every token (groups larger than one pass of four
pairs), invalid expert ids, duplicate experts within a token, the layer-43
SwiGLU clamps and the router computed on the device.
"""
import ctypes as C
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
    hip.set_option("decode_fused", 1)
    hip.synchronize()


@pytest.fixture(scope="module")
def O():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="module")
def layer(H):
    from sf37_amd.moe import SynthLayer
    say("generating BASELINE-shape layer (seed 77)")
    L = SynthLayer(seed=77)
    H.synchronize()
    yield L
    L.free()


_KEYS = []


def map_key():
    """A host address used as a model-map key, kept alive for the session so
    no later key can reuse it."""
    k = np.zeros(64, np.uint8)
    _KEYS.append(k)
    return k.ctypes.data


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bitexact(got, want, what):
    g, w = np.ravel(bits(got)), np.ravel(bits(want))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"{np.ravel(got)[bad[0]]!r} vs {np.ravel(want)[bad[0]]!r}")


def skewed_logits(rng, n_tok, hot=(5, 6, 7, 8, 9)):
    """N(0,1) logits with a few experts every token picks (groups of n_tok pairs)."""
    lg = rng.standard_normal((n_tok, E)).astype(np.float32)
    lg[:, list(hot)] += 8.0
    return lg


def run_layer(H, layer, x, logits, fused, clamps=None, scale=3.0):
    n_tok = x.shape[0]
    H.set_option("decode_fused", 1 if fused else 0)
    try:
        w = layer.weights_struct(scale)
        if clamps is not None:
            w.clamp_routed, w.clamp_shared = clamps
        out, sel, wt = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * TOPK * 4), \
            H.Tensor.alloc(n_tok * TOPK * 4)
        xt = H.Tensor.from_array(x)
        lt = H.Tensor.from_array(logits) if logits is not None else None
        H.check(H.lib().sf37_hip_moe_layer(out, sel, wt, w, lt, xt, n_tok), "moe_layer")
        return (out.read(np.float32).reshape(n_tok, K), sel.read(np.int32).reshape(n_tok, TOPK),
                wt.read(np.float32).reshape(n_tok, TOPK))
    finally:
        H.set_option("decode_fused", 1)


@pytest.mark.parametrize("n_tok,routing", [(1, "uniform"), (3, "skewed"), (8, "uniform"), (8, "skewed"),
                                           (13, "uniform"), (16, "skewed")])
def test_fused_layer_equals_staged(H, layer, n_tok, routing):
    rng = np.random.default_rng(1000 + n_tok)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    logits = skewed_logits(rng, n_tok) if routing == "skewed" else rng.standard_normal((n_tok, E)).astype(np.float32)
    say(f"fused vs staged: {n_tok} tokens, {routing} routing")
    H.lib().sf37_hip_profile_enable(1)
    H.profile_read()
    try:
        a = run_layer(H, layer, x, logits, True)
        prof = H.profile_read()
    finally:
        H.lib().sf37_hip_profile_enable(0)
    assert prof["dec_up"][1] == 1 and prof["dec_down"][1] == 1, "fused kernels did not run"
    b = run_layer(H, layer, x, logits, False)
    assert np.array_equal(a[1], b[1])
    assert_bitexact(a[2], b[2], "weights")
    assert_bitexact(a[0], b[0], f"out ({n_tok} tokens, {routing})")


@pytest.mark.parametrize("n_tok", [2, 4, 5, 6, 7, 9, 10, 11, 12, 14, 15])
def test_fused_layer_every_batch_size(H, layer, n_tok):
    """The batch sizes the cases above skip (each launch plan of 1..16
    tokens: the DMA up launch with and without its first tiles started in
    the prologue, the select launch's top-k workgroup counts, the down
    kernel's shared-down batch instances), fused against staged."""
    rng = np.random.default_rng(2000 + n_tok)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    say(f"fused vs staged: {n_tok} tokens")
    a = run_layer(H, layer, x, logits, True)
    b = run_layer(H, layer, x, logits, False)
    assert np.array_equal(a[1], b[1])
    assert_bitexact(a[2], b[2], "weights")
    assert_bitexact(a[0], b[0], f"out ({n_tok} tokens)")


@pytest.mark.parametrize("seed", range(12))
def test_fused_layer_random_batches(H, layer, seed):
    """Seeded random batches (1..16 tokens, hot experts of random count and
    strength, so groups of 1..16 pairs and launch plans of every shape),
    fused against staged, bit for bit."""
    rng = np.random.default_rng(5000 + seed)
    n_tok = int(rng.integers(1, 17))
    hot = tuple(int(e) for e in rng.choice(E, size=int(rng.integers(0, 9)), replace=False))
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    if hot:
        logits[:, list(hot)] += np.float32(rng.uniform(0.5, 8.0))
    x = (rng.standard_normal((n_tok, K)) * rng.uniform(0.5, 4.0)).astype(np.float32)
    say(f"random batch {seed}: {n_tok} tokens, {len(hot)} hot experts")
    a = run_layer(H, layer, x, logits, True)
    b = run_layer(H, layer, x, logits, False)
    assert np.array_equal(a[1], b[1])
    assert_bitexact(a[2], b[2], "weights")
    assert_bitexact(a[0], b[0], f"out (seed {seed}, {n_tok} tokens)")


def test_fused_layer_after_smaller_batches(H, layer):
    """Batch sizes going down and up again in one process: each kernel's
    dynamic-LDS opt-in must stay at the largest size asked for (a 16-token
    launch after an 8-token one needs more LDS in the up and select launches
    than the 8-token launch set up)."""
    rng = np.random.default_rng(77)
    outs = {}
    for n_tok in (16, 8, 2, 16, 12, 16):
        x = rng.standard_normal((n_tok, K)).astype(np.float32) if n_tok not in outs else outs[n_tok][0]
        lg = rng.standard_normal((n_tok, E)).astype(np.float32) if n_tok not in outs else outs[n_tok][1]
        say(f"batch sequence: {n_tok} tokens")
        a = run_layer(H, layer, x, lg, True)
        if n_tok in outs:
            assert_bitexact(a[0], outs[n_tok][2], f"out ({n_tok} tokens, repeated)")
        else:
            b = run_layer(H, layer, x, lg, False)
            assert_bitexact(a[0], b[0], f"out ({n_tok} tokens)")
            outs[n_tok] = (x, lg, a[0])


def test_fused_layer_router_on_device_and_clamps(H, layer):
    """Router logits computed in the fused route kernel (no injected logits),
    with the layer-43 clamps (routed 7, shared 16)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((5, K)) * 3).astype(np.float32)
    for clamps in (None, (7.0, 16.0)):
        say(f"router on device, clamps {clamps}")
        a = run_layer(H, layer, x, None, True, clamps)
        b = run_layer(H, layer, x, None, False, clamps)
        assert np.array_equal(a[1], b[1])
        assert_bitexact(a[2], b[2], "weights")
        assert_bitexact(a[0], b[0], f"out clamps {clamps}")


def test_fused_layer_16_tokens_against_oracle(H, O, layer):
    """16 tokens, skewed routing, clamps on: bit-exact against the oracle."""
    rng = np.random.default_rng(16)
    x = rng.standard_normal((16, K)).astype(np.float32)
    logits = skewed_logits(rng, 16)
    say("fused 16 tokens vs oracle")
    out, sel, w = run_layer(H, layer, x, logits, True, (7.0, 16.0))
    dense = layer.host_dense()
    weights = dict(layer.host_experts(np.append(np.ravel(sel), 0)), **dense, n_expert=E, mid_dim=F)
    want, wsel, ww = O.moe_layer_q8k(weights, x, logits=logits, clamp_routed=7.0, clamp_shared=16.0)
    assert np.array_equal(sel, wsel)
    assert_bitexact(w, ww, "weights")
    assert_bitexact(out, want, "16-token layer")


def tied_logits(rng, n_tok, kind):
    """Router logits whose scores tie (router bias 0): rounded to integers,
    all equal, or ten equal hot experts spread over every 64-expert column
    (only the eight smallest positions may win)."""
    if kind == "rounded":
        return np.round(1.5 * rng.standard_normal((n_tok, E))).astype(np.float32)
    if kind == "equal":
        return np.zeros((n_tok, E), np.float32)
    lg = (rng.standard_normal((n_tok, E)) - 4.0).astype(np.float32)
    lg[:, [287, 250, 200, 130, 70, 64, 63, 31, 5, 1]] = 3.0
    return lg


@pytest.mark.parametrize("n_tok", [1, 3, 8])
@pytest.mark.parametrize("kind", ["rounded", "equal", "hot_ties"])
def test_fused_layer_tied_scores(H, O, layer, n_tok, kind):
    """Tied router scores: the fused and staged paths select, order and
    weight as the oracle does (equal scores go to the smaller expert)."""
    rng = np.random.default_rng(500 + n_tok)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    logits = tied_logits(rng, n_tok, kind)
    say(f"tied scores: {n_tok} tokens, {kind}")
    a = run_layer(H, layer, x, logits, True)
    b = run_layer(H, layer, x, logits, False)
    dense = layer.host_dense()
    weights = dict(layer.host_experts(np.append(np.ravel(a[1]), 0)), **dense, n_expert=E, mid_dim=F)
    want, wsel, ww = O.moe_layer_q8k(weights, x, logits=logits)
    assert np.array_equal(a[1], wsel), (a[1], wsel)
    assert np.array_equal(b[1], wsel)
    if kind == "hot_ties":
        assert np.array_equal(np.sort(a[1], axis=1), np.tile([1, 5, 31, 63, 64, 70, 130, 200], (n_tok, 1)))
    assert_bitexact(a[2], ww, "weights")
    assert_bitexact(b[2], ww, "staged weights")
    assert_bitexact(a[0], want, f"out ({n_tok} tokens, {kind})")
    assert_bitexact(b[0], want, f"staged out ({n_tok} tokens, {kind})")


def test_fused_routed_batch_mapped(H, O, layer):
    """routed_moe_batch_mapped for 5 tokens at the full shape, with an invalid
    id and an expert repeated inside one token: out and per-pair mid equal
    the staged path and the oracle."""
    n_tok = 5
    rng = np.random.default_rng(55)
    sel = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(n_tok)]).astype(np.int32)
    sel[1, 2] = -1
    sel[2, 5] = sel[2, 1]
    sel[3, :4] = sel[0, :4]
    w = (rng.random((n_tok, TOPK)) * 0.5).astype(np.float32)
    x = rng.standard_normal((n_tok, K)).astype(np.float32)
    gb, db = layer.gate.nbytes, layer.down.nbytes
    total = 2 * gb + db
    key = map_key()
    L = H.lib()
    for off, t in ((0, layer.gate), (gb, layer.up), (2 * gb, layer.down)):
        H.check(L.sf37_hip_register_device_range(key, total, off, t.nbytes, t), "register")
    st, wt, xt = H.Tensor.from_array(sel), H.Tensor.from_array(w), H.Tensor.from_array(x)
    res = []
    for fused in (True, False):
        H.set_option("decode_fused", 1 if fused else 0)
        try:
            out, g, u, d = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(TOPK * F * 4), \
                H.Tensor.alloc(TOPK * F * 4), H.Tensor.alloc(TOPK * K * 4)
            m = H.Tensor.alloc(n_tok * TOPK * F * 4)
            H.check(L.sf37_hip_routed_moe_batch_mapped(out, g, u, m, d, key, total, 0, gb, 2 * gb, st,
                                                       wt, E, TOPK, K, F, K, 0.0, xt, n_tok), "batch")
            res.append((out.read(np.float32).reshape(n_tok, K), m.read(np.float32).reshape(n_tok * TOPK, F)))
        finally:
            H.set_option("decode_fused", 1)
    assert_bitexact(res[0][0], res[1][0], "fused vs staged out")
    assert_bitexact(res[0][1], res[1][1], "fused vs staged mid")
    host = layer.host_experts(np.append(np.ravel(sel), 0))
    want, want_mid = O.routed_moe_batch_q8k(host["gate"], host["up"], host["down"], sel, w, E, K, F, K, 0.0, x)
    assert_bitexact(res[0][0], want, "batch out vs oracle")
    assert_bitexact(res[0][1], want_mid, "batch mid vs oracle")


def test_fused_routed_one_duplicates(H, O, layer):
    """routed_moe_one (one group per slot) with a repeated expert and the
    gate/up export option: out, gate, up and mid equal the staged path with
    the one-token down+combine launch and without it; the per-slot down rows
    (scratch, written only when down and combine are separate launches, as
    the reference's direct down-sum path leaves them unwritten,
    sf37_cuda.cu:5366-5371) equal the staged path's."""
    rng = np.random.default_rng(9)
    sel = rng.choice(E, TOPK, replace=False).astype(np.int32)
    sel[6] = sel[2]
    w = (rng.random(TOPK) * 0.6).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    st, wt, xt = H.Tensor.from_array(sel), H.Tensor.from_array(w), H.Tensor.from_array(x)
    res = []
    H.set_option("moe_write_gate_up", 1)
    try:
        for fused, down_combine in ((True, True), (True, False), (False, False)):
            H.set_option("decode_fused", 1 if fused else 0)
            H.set_option("decode_down_combine", 1 if down_combine else 0)
            out, g, u, m, d = (H.Tensor.alloc(K * 4), H.Tensor.alloc(TOPK * F * 4), H.Tensor.alloc(TOPK * F * 4),
                               H.Tensor.alloc(TOPK * F * 4), H.Tensor.alloc(TOPK * K * 4))
            H.check(H.lib().sf37_hip_routed_moe_one(out, g, u, m, d, layer.gate, layer.up, layer.down, st, wt, E,
                                                    TOPK, K, F, K, 0.0, xt), "routed_moe_one")
            res.append([t.read(np.float32) for t in (out, g, u, m, d)])
    finally:
        H.set_option("moe_write_gate_up", 0)
        H.set_option("decode_fused", 1)
        H.set_option("decode_down_combine", 1)
    for k in (0, 1):
        for name, a, b in zip(("out", "gate", "up", "mid"), res[k], res[2]):
            assert_bitexact(a, b, f"routed_moe_one {name} (run {k})")
    assert_bitexact(res[1][4], res[2][4], "routed_moe_one down rows")
    host = layer.host_experts(sel)
    want, want_mid, _ = O.routed_moe_one_q8k(host["gate"], host["up"], host["down"], sel, w, E, K, F, K, 0.0, x)
    assert_bitexact(res[0][0], want, "routed_moe_one vs oracle")
    assert_bitexact(res[0][3].reshape(TOPK, F), want_mid, "routed_moe_one mid vs oracle")


@pytest.mark.parametrize("E_, D_, F_, topk", [(16, 1024, 512, 4), (16, 512, 768, 8), (12, 1024, 1280, 3),
                                             (32, 1024, 1280, 12)])
def test_one_token_down_combine_shapes(H, O, E_, D_, F_, topk):
    """The one-token down+combine launch on shapes other than the BASELINE
    one: fewer slots than its 8 waves (top-3, top-4), more (top-12: waves
    0-3 take two slots), 32- and 20-row tiles (F = 512, 768: 8 and 5 shared
    passes), against the two-launch path, the staged kernels and the
    oracle, bit for bit."""
    from sf37_amd.moe import SynthLayer
    say(f"one-token down+combine: E {E_}, D {D_}, F {F_}, top-{topk}")
    lay = SynthLayer(seed=300 + topk, n_expert=E_, in_dim=D_, mid_dim=F_, topk=topk)
    rng = np.random.default_rng(40 + topk)
    x = rng.standard_normal((1, D_)).astype(np.float32)
    lg = rng.standard_normal((1, E_)).astype(np.float32)
    xt, lt = H.Tensor.from_array(x), H.Tensor.from_array(lg)
    outs, profs = [], []
    try:
        for fused, dc in ((True, True), (True, False), (False, False)):
            H.set_option("decode_fused", 1 if fused else 0)
            H.set_option("decode_down_combine", 1 if dc else 0)
            out, sel, wt = H.Tensor.alloc(D_ * 4), H.Tensor.alloc(topk * 4), H.Tensor.alloc(topk * 4)
            H.lib().sf37_hip_profile_enable(1)
            H.profile_read()
            H.check(H.lib().sf37_hip_moe_layer(out, sel, wt, lay.weights_struct(), lt, xt, 1), "moe_layer")
            profs.append(H.profile_read())
            H.lib().sf37_hip_profile_enable(0)
            outs.append((out.read(np.float32), sel.read(np.int32)))
    finally:
        H.lib().sf37_hip_profile_enable(0)
        H.set_option("decode_fused", 1)
        H.set_option("decode_down_combine", 1)
    # the first run is the one-launch down+combine, the second two launches
    assert profs[0]["dec_down"][1] == 1 and profs[0]["dec_combine"][1] == 0, profs[0]
    assert profs[1]["dec_down"][1] == 1 and profs[1]["dec_combine"][1] == 1, profs[1]
    for k in (1, 2):
        assert np.array_equal(outs[0][1], outs[k][1])
        assert_bitexact(outs[0][0], outs[k][0], f"out vs run {k}")
    weights = dict(lay.host_experts(np.arange(E_)), **lay.host_dense(), n_expert=E_, mid_dim=F_)
    want, want_sel, _ = O.moe_layer_q8k(weights, x, logits=lg, topk=topk)
    assert np.array_equal(outs[0][1].reshape(1, topk), want_sel)
    assert_bitexact(outs[0][0], want.reshape(-1), "out vs oracle")
    lay.free()
