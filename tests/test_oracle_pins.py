"""Pins of the oracle functions the per-op checks leave open.

* The whole layer (orc_moe_layer_q8k: router, top-8, Q8_0 shared expert,
  Q8_K routed experts, shared + routed) against the reference's CPU MoE layer
  compiled from its own sources (oracle/_ref/libsf37cpu_ref.so: sf37_ops.c
  and sf37_quant.c with the `make cpu` flags, composed as layer_moe_ffn,
  sf37.c:2127-2194) at the BASELINE shape (288 x 4096 x 1280, top-8): equal
  expert indices, outputs within the reference's own CUDA-vs-CPU tolerance
  5e-2 abs / 1e-1 rel (tests/test_sf37_cuda_ops.cu:814).  A shared expert
  dropped or a routing weight lost moves outputs far beyond that; the
  layer-43 clamps are pinned with activations large enough for them to bind.
* The Q8_K activation rounding: lrintf, round half to even
  (sf37_cuda.cu:4194), on blocks built so that every product x * (1/d) is an
  exact half-integer; round-half-away would fail them.  Also the Q8_0
  activation quantiser (sf37_ops.c:57-90, lrintf) on the same blocks.
* orc_swiglu_mid against the reference's sf37_swiglu (sf37_ops.c:30-42)
  followed by the routing-weight product (sf37.c:2175-2177), bit for bit,
  clamps 0, 7 and 16.
* orc_rms_norm_weight1_bf16 against the engine's own sequence (sf37.c:2243-
  2244: the reference's sf37_bf16_to_f32 widening, then its
  sf37_rms_norm_weight1), bit for bit, and the reference KAT with bf16
  weights; plausible mistakes are shown to change the bits.
* orc_f32_matvec_double (the F32 router, sf37.c:1970-1976) against a float64
  matrix product (within 1 ulp), exact integer sums, and rows on which a
  float accumulator or a transposed operand fails.
"""
import ctypes as C

import numpy as np
import pytest

import synth_host

fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
bp = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint8))


def zipf_bias(seed, n_expert=288, s=1.1):
    """ln(p(rank)/p(1)) for p(k) ~ k^-s over a seeded permutation of ranks."""
    ranks = np.random.default_rng([seed, 17]).permutation(n_expert) + 1
    return (-s * np.log(ranks.astype(np.float64))).astype(np.float32)


def layer_case(orc, seed, n_tok, xscale=1.0, bias="zero"):
    """Host weights (the selected experts filled), x and the oracle's top-8."""
    w = synth_host.host_layer(orc, seed)
    if bias == "zipf":
        w["router_bias"] = zipf_bias(seed)
    x = (orc.fill_normal(n_tok * 4096, seed, synth_host.X_STREAM) * np.float32(xscale)).reshape(n_tok, 4096)
    logits = synth_host.router_logits(orc, w, x)
    sel, wts, _ = orc.router_select(logits, w["router_bias"], 8, 3.0)
    synth_host.fill_experts(orc, w, sel)
    return w, x, sel, wts


def ref_cpu_layer(ref, w, x, clamp_r=0.0, clamp_s=0.0):
    n_tok, D = x.shape
    want = np.zeros((n_tok, D), np.float32)
    want_sel = np.zeros((n_tok, 8), np.int32)
    for t in range(n_tok):
        ref.sf37cpu_moe_ffn_token(fp(want[t]), want_sel[t].ctypes.data_as(C.POINTER(C.c_int32)), fp(w["router"]),
                                  fp(w["router_bias"]), bp(w["gate"]), bp(w["up"]), bp(w["down"]),
                                  bp(w["sh_gate"]), bp(w["sh_up"]), bp(w["sh_down"]), w["n_expert"], 8, D,
                                  w["mid_dim"], clamp_r, clamp_s, fp(np.ascontiguousarray(x[t])))
    return want, want_sel


@pytest.mark.parametrize("seed,bias", [(7001, "zero"), (7002, "zipf")])
def test_layer_matches_reference_cpu_layer_at_baseline_shape(orc, seed, bias):
    ref = orc.cpu_baseline_lib("reference")
    if ref is None:
        pytest.skip("oracle/_ref/libsf37cpu_ref.so is not built (needs /root/reference)")
    w, x, sel_pred, _ = layer_case(orc, seed, 4, bias=bias)
    got, sel, _ = orc.moe_layer_q8k(w, x)
    assert np.array_equal(sel, sel_pred)
    want, want_sel = ref_cpu_layer(ref, w, x)
    assert np.array_equal(sel, want_sel), f"top-8 differs\n{sel}\n{want_sel}"
    diff = np.abs(got.astype(np.float64) - want)
    ok = (diff <= 5e-2) | (diff <= 1e-1 * np.maximum(1.0, np.abs(want)))
    mar = orc.max_abs_rel(got, want)
    print(f"\nlayer seed {seed} bias {bias}: max|a-b|/max(|b|,1) = {mar:.3e}, max|b| = {np.abs(want).max():.3f}")
    assert ok.all(), f"{(~ok).sum()} outputs outside 5e-2 / 1e-1; max_abs_rel {mar:.3g}"
    # a layer without its shared expert is far outside the tolerance
    no_sh = dict(w, sh_down=np.zeros_like(w["sh_down"]))
    bad, _, _ = orc.moe_layer_q8k(no_sh, x)
    assert orc.max_abs_rel(bad, want) > 10 * max(mar, 5e-2)


def test_layer_clamps_match_reference_at_baseline_shape(orc):
    """Layer 43 (routed clamp 7, shared clamp 16) with x ~ N(0, 64), so both
    clamps bind.  The shared expert and the final add are pinned bit for bit
    against the reference's own ops (IEEE build): layer = shared + routed
    (sf37.c:2159-2167, 3428).  The Q8_K routed part against the reference's
    fp32-activation routed path (sf37_ops.c:153-179 composed as
    sf37.c:2169-2181) within 2 % of the output's largest magnitude (Q8_K
    noise grows with the activations, so the element-wise unit-scale
    tolerance does not apply here), and the same routed part without its
    clamp lies far outside that bound."""
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref/libsf37ref.so is not built (needs /root/reference)")
    D, F, E = 4096, 1280, 288
    w, x, sel, wts = layer_case(orc, 7003, 2, xscale=8.0)
    got, got_sel, got_w = orc.moe_layer_q8k(w, x, clamp_routed=7.0, clamp_shared=16.0)
    assert np.array_equal(got_sel, sel) and np.array_equal(got_w, wts)
    gb, db = F * 16 * 110, D * 5 * 84
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t])
        g, u, m = (np.zeros(F, np.float32) for _ in range(3))
        ref.sf37_q8_0_matvec_pair(fp(g), fp(u), bp(w["sh_gate"]), bp(w["sh_up"]), D, F, fp(xt))
        assert (g > 16).any() and (np.abs(u) > 16).any()         # the shared clamp binds
        ref.sf37_swiglu(fp(m), fp(g), fp(u), F, 16.0)
        shared = np.zeros(D, np.float32)
        ref.sf37_q8_0_matvec(fp(shared), bp(w["sh_down"]), F, D, fp(m))
        routed, _, _ = orc.routed_moe_one_q8k(w["gate"], w["up"], w["down"], sel[t], wts[t], E, D, F, D, 7.0, xt)
        assert np.array_equal((shared + routed).view(np.uint32), got[t].view(np.uint32))
        want = np.zeros(D, np.float32)
        down = np.zeros(D, np.float32)
        for s, e in enumerate(sel[t]):
            gw = np.ascontiguousarray(w["gate"][e * gb:(e + 1) * gb])
            uw = np.ascontiguousarray(w["up"][e * gb:(e + 1) * gb])
            dw = np.ascontiguousarray(w["down"][e * db:(e + 1) * db])
            ref.sf37_q3_asym_matvec(fp(g), bp(gw), D, F, fp(xt))
            ref.sf37_q3_asym_matvec(fp(u), bp(uw), D, F, fp(xt))
            ref.sf37_swiglu(fp(m), fp(g), fp(u), F, 7.0)
            m *= wts[t][s]
            ref.sf37_q2_asym_matvec(fp(down), bp(dw), F, D, fp(m))
            want += down
        scale = np.abs(want).max()
        err = np.abs(routed - want).max() / scale
        unclamped, _, _ = orc.routed_moe_one_q8k(w["gate"], w["up"], w["down"], sel[t], wts[t], E, D, F, D, 0.0, xt)
        err_nc = np.abs(unclamped - want).max() / scale
        print(f"\nclamped layer token {t}: routed max|a-b|/max|b| = {err:.3e} (without the clamp {err_nc:.3e})")
        assert err <= 2e-2 and err_nc > 5 * 2e-2


def half_way_blocks():
    """Blocks of 256 whose amax is 127 * 2^k, so d = 2^k, 1/d = 2^-k and each
    x * (1/d) is an exact half-integer (or the amax itself)."""
    halves = np.arange(-126.5, 127.0, 1.0)                 # 254 half-integers
    rows = []
    for k in (-4, 0, 3):
        s = 2.0 ** k
        v = np.concatenate([[127.0], halves, [0.5]]) * s    # 256 values
        rows.append(v)
        rows.append(-v[::-1])                               # amax first negative, reversed order
    return np.array(rows, np.float32)


def test_q8k_rounds_half_to_even(orc):
    x = half_way_blocks()
    q = orc.q8k_quantize(x)
    scale = np.abs(x).max(axis=1) / np.float32(127.0)
    assert np.array_equal(q["d"], scale.astype(np.float32))
    v = x.astype(np.float64) / scale[:, None]
    want = np.rint(v)                                       # numpy rint: half to even
    away = np.trunc(v + np.copysign(0.5, v))
    assert (want != away).sum() > 500                       # the blocks tell the two rules apart
    assert np.array_equal(q["qs"].astype(np.float64), want)
    assert np.array_equal(q["gsums"], q["qs"].reshape(-1, 4, 64).astype(np.int32).sum(axis=2))


def test_q8_0_activation_rounds_half_to_even(orc):
    # 32-wide blocks: amax 127 * 2^k at the first element, 31 half-integers
    xb = np.zeros((48, 32), np.float32)
    xb[:, 0] = np.where(np.arange(xb.shape[0]) % 2 == 0, 127.0, -127.0) * np.float32(0.5)
    xb[:, 1:] = np.resize(np.arange(-15.5, 15.6, 1.0), (xb.shape[0], 31)) * np.float32(0.5)
    x = np.ascontiguousarray(xb.ravel(), np.float32)
    n = x.size
    xq = np.zeros(n, np.int8)
    sc = np.zeros(n // 32, np.float32)
    orc.lib().orc_q8_0_quantize_activation(fp(x), xq.ctypes.data_as(C.POINTER(C.c_int8)), fp(sc), n)
    want = np.rint(xb.astype(np.float64) / 0.5)
    assert np.all(sc == np.float32(0.5))
    assert np.array_equal(xq.reshape(-1, 32).astype(np.float64), want)
    ref = orc.ref_lib()
    if ref is not None:
        rq = np.zeros(n, np.int8)
        rs = np.zeros(n // 32, np.float32)
        ref.sf37_q8_0_quantize_activation(fp(x), rq.ctypes.data_as(C.POINTER(C.c_int8)), fp(rs), n)
        assert np.array_equal(rq, xq) and np.array_equal(rs, sc)


@pytest.mark.parametrize("clamp", [0.0, 7.0, 16.0])
def test_swiglu_mid_matches_reference_swiglu_times_weight(orc, clamp):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref/libsf37ref.so is not built (needs /root/reference)")
    r = np.random.default_rng(int(clamp) + 5)
    n = 20000
    g = (r.standard_normal(n) * 12).astype(np.float32)
    u = (r.standard_normal(n) * 12).astype(np.float32)
    w = r.uniform(0.0, 3.0, n).astype(np.float32)
    g[:4] = [clamp, -clamp, 1e-30, -88.0]                   # clamp boundary, tiny, deep negative
    u[:4] = [clamp, -clamp, -1e-30, 100.0]
    sw = np.zeros(n, np.float32)
    ref.sf37_swiglu(fp(sw), fp(g), fp(u), n, clamp)
    want = (sw * w).astype(np.float32)
    L = orc.lib()
    got = np.array([L.orc_swiglu_mid(float(g[i]), float(u[i]), float(w[i]), clamp) for i in range(n)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if clamp:
        assert (np.abs(g) > clamp).any() and (np.abs(u) > clamp).any()


# --------------------------------------------------------------------------
# RMSNorm(w + 1) with bf16 weights, and the F32 router GEMV (binary64 sums)
# --------------------------------------------------------------------------

def bf16_bits(a):
    """bf16 codes of float32 values by truncation (any bf16 code is a valid weight)."""
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def ref_widened_rms(ref, x, wb, eps):
    """The engine's sequence (sf37.c:2243-2244): tensor_bf16_to_f32 of the
    norm weight through the reference's sf37_bf16_to_f32 (sf37_quant.c:32-37),
    then sf37_rms_norm_weight1 (sf37_ops.c:22-28), both compiled from the
    reference's sources."""
    wf = np.array([ref.sf37_bf16_to_f32(int(v)) for v in wb], np.float32)
    out = np.zeros(x.size, np.float32)
    ref.sf37_rms_norm_weight1(fp(out), fp(x), fp(wf), x.size, eps)
    return out, wf


def rms_bf16_weights(seed, n):
    """bf16 norm weights with ties (repeated codes), negatives, -1 (w + 1 = 0),
    zeros of both signs, values that round when 1 is added, and tiny and huge
    magnitudes."""
    r = np.random.default_rng(seed)
    w = (r.standard_normal(n) * 0.3).astype(np.float32)
    w[::7] = w[min(3, n - 1)]          # ties
    w[1::11] = -1.0                    # (w + 1) == 0
    w[2::13] = 0.0
    w[4::17] = -0.0
    w[5::19] = 2.0 ** -30              # vanishes in w + 1
    w[6::23] = 384.0
    w[8::29] = -3.0e-3
    return bf16_bits(w)


def test_rms_norm_bf16_matches_reference_sequence(orc):
    """orc_rms_norm_weight1_bf16 == reference widen + sf37_rms_norm_weight1,
    bit for bit, at the engine's width 4096 and at odd widths; the inputs are
    chosen so that a float sum of squares, another eps, a dropped +1, a
    weight read as f16 or the scale applied as x * ((w + 1) * scale) give
    other bits (each checked to differ, so the comparison has the power to
    see them)."""
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent")
    L = orc.lib()
    u16 = C.POINTER(C.c_uint16)
    caught = set()
    names = ("float sum of squares", "eps 1e-6", "no +1", "weight read as f16", "reassociated product")
    for seed, n, xs, big in [(501, 4096, 3.0, True), (502, 4096, 1e-3, False), (503, 70, 50.0, False),
                             (504, 1, 2.0, False), (505, 1280, 1.0, True), (506, 4096, 1.0, False)]:
        r = np.random.default_rng(seed)
        x = (r.standard_normal(n) * xs).astype(np.float32)
        if big:
            x[:4] = [1e4, -1e4, 3e-3, 0.0]      # large terms: a float sum of squares drifts
        wb = rms_bf16_weights(seed, n)
        for eps in (1e-5, 1e-6):
            want, wf = ref_widened_rms(ref, x, wb, eps)
            got = np.zeros(n, np.float32)
            L.orc_rms_norm_weight1_bf16(fp(got), fp(x), wb.ctypes.data_as(u16), n, eps)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, n, eps)
            # the f32 variant on the widened weights gives the same bits
            got32 = np.zeros(n, np.float32)
            L.orc_rms_norm_weight1(fp(got32), fp(x), fp(wf), n, eps)
            assert np.array_equal(got32.view(np.uint32), want.view(np.uint32))
        # power of the comparison: plausible mistakes give other bits
        want, wf = ref_widened_rms(ref, x, wb, 1e-5)
        x64 = x.astype(np.float64)
        ss32 = np.float32(0)
        for v in x:                                     # float accumulator
            ss32 = np.float32(ss32 + v * v)
        mean64 = np.float32((x64 * x64).sum() / n)
        good = np.float32(1) / np.sqrt(mean64 + np.float32(1e-5))
        wp1 = wf + np.float32(1)
        with np.errstate(over="ignore", invalid="ignore"):
            mutants = {
                "float sum of squares": (x * (np.float32(1) / np.sqrt(ss32 / np.float32(n) + np.float32(1e-5)))) * wp1,
                "eps 1e-6": (x * (np.float32(1) / np.sqrt(mean64 + np.float32(1e-6)))) * wp1,
                "no +1": (x * good) * wf,
                "weight read as f16": (x * good) * (wb.view(np.float16).astype(np.float32) + np.float32(1)),
                "reassociated product": x * (good * wp1),
            }
        assert np.array_equal(((x * good) * wp1).view(np.uint32), want.view(np.uint32))
        for name, bad in mutants.items():
            if not np.array_equal(bad.view(np.uint32), want.view(np.uint32)):
                caught.add(name)
    assert caught == set(names), set(names) - caught


def test_rms_norm_bf16_reference_kat(orc):
    """tests/test_sf37_ops.c:89-97 with the weights stored as bf16 (all four
    are exact in bf16): within 1e-6 of the closed form, and equal to the f32
    variant's bits."""
    L = orc.lib()
    x = np.array([1.0, -2.0, 3.0, -4.0], np.float32)
    w = np.array([0.0, 0.5, -0.25, 1.0], np.float32)
    wb = bf16_bits(w)
    assert np.array_equal((wb.astype(np.uint32) << 16).view(np.float32), w)
    out = np.zeros(4, np.float32)
    L.orc_rms_norm_weight1_bf16(fp(out), fp(x), wb.ctypes.data_as(C.POINTER(C.c_uint16)), 4, 1e-5)
    ss = float(np.sum(x.astype(np.float64) ** 2))
    s = np.float32(1.0) / np.sqrt(np.float32(ss / 4.0) + np.float32(1e-5))
    assert np.all(np.abs(out - x * s * (w + np.float32(1))) <= 1e-6)
    out32 = np.zeros(4, np.float32)
    L.orc_rms_norm_weight1(fp(out32), fp(x), fp(w), 4, 1e-5)
    assert np.array_equal(out.view(np.uint32), out32.view(np.uint32))


def f32_ulp_diff(a, b):
    """Distance in units in the last place between float32 arrays (same sign)."""
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = np.where(ib < 0, -(ib & 0x7fffffff), ib)
    return np.abs(ia - ib)


def oracle_router(L, W, x):
    E, D = W.shape
    out = np.zeros((x.shape[0], E), np.float32)
    Wc = np.ascontiguousarray(W)
    for t in range(x.shape[0]):
        L.orc_f32_matvec_double(fp(out[t]), fp(Wc), D, E, fp(np.ascontiguousarray(x[t])))
    return out


def test_f32_router_matvec_double_vs_float64_matmul(orc):
    """orc_f32_matvec_double (the static F32 router, sf37.c:1970-1976:
    binary64 products and sums, one rounding to float at the end) against
    numpy's float64 matrix product rounded to float32: 288 x 4096 router,
    16 token rows, within 1 ulp (the two sum the same exact products in other
    orders), >= 99 % identical; a transposed operand fails that check."""
    L = orc.lib()
    r = np.random.default_rng(601)
    E, D, T = 288, 4096, 16
    W = (r.standard_normal((E, D)) * 0.02).astype(np.float32)
    x = r.standard_normal((T, D)).astype(np.float32)
    got = oracle_router(L, W, x)
    want = (x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32)
    d = f32_ulp_diff(got, want)
    assert d.max() <= 1 and (d == 0).mean() >= 0.99, (d.max(), (d == 0).mean())
    # exact sums: integer operands whose every partial sum is exact in binary64
    Wi = r.integers(-64, 64, (E, D)).astype(np.float32)
    xi = r.integers(-64, 64, (T, D)).astype(np.float32)
    gi = oracle_router(L, Wi, xi)
    assert np.array_equal(gi, (xi.astype(np.int64) @ Wi.T.astype(np.int64)).astype(np.float32))
    # power: the same weights read transposed ([D][E] memory as [E][D]) miss
    Wt = np.ascontiguousarray(W.T).reshape(E, D)
    bad = oracle_router(L, Wt, x)
    assert f32_ulp_diff(bad, want).max() > 1000


def test_f32_router_matvec_double_accumulator(orc):
    """The binary64 accumulator of sf37.c:1974 against cases a float
    accumulator gets wrong: terms 2^30, 1, -2^30 sum to 1 in binary64 and to
    0 in binary32, and a long alternating row whose float sum drifts."""
    L = orc.lib()
    D = 4096
    W = np.zeros((3, D), np.float32)
    W[0, :3] = [2.0 ** 30, 1.0, -(2.0 ** 30)]
    W[1, :] = np.where(np.arange(D) % 2 == 0, np.float32(1e8), np.float32(-1e8))
    W[1, 5] += np.float32(8.0)
    W[2, :] = np.float32(0.1)
    x = np.ones((1, D), np.float32)
    got = oracle_router(L, W, x)[0]
    assert got[0] == 1.0
    want1 = np.float32(np.sum(W[1].astype(np.float64)))
    assert got[1] == want1
    want2 = np.float32(np.float64(np.float32(0.1)) * D)
    assert f32_ulp_diff(got[2:3], np.array([want2], np.float32)).max() <= 1
    f32_acc = np.float32(0)
    for v in W[0]:
        f32_acc = np.float32(f32_acc + v)
    assert f32_acc != got[0]       # a float accumulator would fail the first row
