"""Pins for the CPU oracle (oracle/sf37_oracle.c).

Each restated function is checked against at least one of: the reference's
own C code compiled in place (oracle/_ref, bit-exact, when present), the
committed golden vectors made from it (tests/golden), the reference's own
known-answer tests (restated in refvec.py), or what the mathematics fixes
(closed forms, invariants, brute force), chosen so that a dropped term, a
wrong index or a transposed operand fails.
"""
import ctypes as C
import os

import numpy as np
import pytest

import refvec

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def P(a, t=C.c_float):
    return a.ctypes.data_as(C.POINTER(t))


U8 = C.c_uint8


def rng(seed=0):
    return np.random.default_rng(seed)


def random_q3_blocks(n, seed):
    r = rng(seed)
    b = r.integers(0, 256, size=(n, 110), dtype=np.uint8)
    # finite scales in [2^-10, 2^0) so decode is well away from inf/nan
    s = (r.random((n, 4)) * 0.9 + 0.1).astype(np.float16).view(np.uint16)
    b[:, 0:8] = s.view(np.uint8).reshape(n, 8)
    b[:, 108:110] = 0
    return b


def random_q2_blocks(n, seed):
    r = rng(seed)
    b = r.integers(0, 256, size=(n, 84), dtype=np.uint8)
    s = (r.random((n, 4)) * 0.9 + 0.1).astype(np.float16).view(np.uint16)
    b[:, 0:8] = s.view(np.uint8).reshape(n, 8)
    b[:, 76:84] = 0
    return b


# --------------------------------------------------------------------------
# scalar formats
# --------------------------------------------------------------------------

def test_f16_decode_exhaustive(orc):
    L = orc.lib()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]) == np.isnan(want[~finite]))
    ref = orc.ref_lib()
    if ref is not None:
        got_ref = np.array([ref.sf37_f16_to_f32(int(v)) for v in h[:: 7]], dtype=np.float32)
        assert np.array_equal(np.nan_to_num(got_ref), np.nan_to_num(got[:: 7]))


def test_f16_encode_rne_at_every_boundary(orc):
    """Round-to-nearest-even of every binary16 value's neighbourhood:
    the value itself, the midpoints to its neighbours and one ulp either side."""
    L = orc.lib()
    h = np.arange(0, 0x7C00, dtype=np.uint16)              # finite non-negative halves
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65520.0)
    mid = ((v + nxt) / 2).astype(np.float32)               # exact in binary32
    cands = np.concatenate([v.astype(np.float32), mid,
                            np.nextafter(mid, np.float32(np.inf)),
                            np.nextafter(mid, np.float32(0))])
    cands = np.concatenate([cands, -cands, np.array([7e4, -7e4, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        want = cands.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_f16(float(c)) for c in cands], dtype=np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------------
# block decode / dot: reference KATs and the compiled reference
# --------------------------------------------------------------------------

def test_reference_block_kats(orc):
    """tests/test_sf37_quant.c:78-147: decode equals (q - zp) * scale."""
    L = orc.lib()
    i = np.arange(256)
    q3 = (i * 5 + 3) & 7
    blk = refvec.q3_block(q3, [0.125, 0.25, 0.5, 1.0], [0, 3, 5, 7])
    dec = np.zeros(256, np.float32)
    L.orc_q3_block_decode(P(blk, U8), P(dec))
    want = (q3 - np.repeat([0, 3, 5, 7], 64)) * np.repeat([0.125, 0.25, 0.5, 1.0], 64)
    assert np.array_equal(dec, want.astype(np.float32))
    x = ((i % 13) - 6).astype(np.float32) * np.float32(0.03125)
    dot = L.orc_q3_block_dot(P(blk, U8), P(x))
    assert abs(dot - float(np.dot(want, x))) <= 5e-4

    q2 = (i * 3 + 1) & 3
    blk2 = refvec.q2_block(q2, [0.125, 0.25, 0.5, 1.0], [0, 1, 2, 3])
    L.orc_q2_block_decode(P(blk2, U8), P(dec))
    want2 = (q2 - np.repeat([0, 1, 2, 3], 64)) * np.repeat([0.125, 0.25, 0.5, 1.0], 64)
    assert np.array_equal(dec, want2.astype(np.float32))

    q8 = np.arange(32, dtype=np.int8) - 16
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = np.array([refvec.f16_bits(0.25)], np.uint16).view(np.uint8)
    b8[2:] = q8.view(np.uint8)
    d8 = np.zeros(32, np.float32)
    L.orc_q8_0_block_decode(P(b8, U8), P(d8))
    assert np.array_equal(d8, q8.astype(np.float32) * np.float32(0.25))


def test_block_decode_dot_match_reference_bitwise(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent")
    L = orc.lib()
    r = rng(1)
    for name, blocks, orc_dec, ref_dec, orc_dot, ref_dot in [
        ("q3", random_q3_blocks(200, 2), L.orc_q3_block_decode, ref.sf37_q3_asym_block_decode,
         L.orc_q3_block_dot, ref.sf37_q3_asym_block_dot),
        ("q2", random_q2_blocks(200, 3), L.orc_q2_block_decode, ref.sf37_q2_asym_block_decode,
         L.orc_q2_block_dot, ref.sf37_q2_asym_block_dot),
    ]:
        for b in blocks:
            b = np.ascontiguousarray(b)
            a1 = np.zeros(256, np.float32)
            a2 = np.zeros(256, np.float32)
            orc_dec(P(b, U8), P(a1))
            ref_dec(P(b, U8), P(a2))
            assert np.array_equal(a1.view(np.uint32), a2.view(np.uint32)), name
            x = r.standard_normal(256).astype(np.float32)
            assert orc_dot(P(b, U8), P(x)) == ref_dot(P(b, U8), P(x)), name


# --------------------------------------------------------------------------
# weight quantizer (gguf-tools/quants.c)
# --------------------------------------------------------------------------

def quant_inputs():
    r = rng(7)
    w = (r.standard_normal((24, 512)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0                      # all-zero group
    w[1, :64] = 0.0125                   # constant positive group
    w[2, :64] = -0.5                     # constant negative group
    w[3, :64] = r.standard_normal(64).astype(np.float32) * 1e-30   # tiny scale
    w[4, :32] = 3.0                      # Q8_0 block with equal values
    w[5, 64:128] = np.linspace(-1, 1, 64, dtype=np.float32)       # exact half-way codes
    w[6, :] = 0.0
    return w


@pytest.mark.parametrize("kind,type_id", [("q8_0", 8), ("q3", 11), ("q2", 10)])
def test_quantizer_matches_reference_bitwise(orc, kind, type_id):
    w = quant_inputs()
    got = orc.quantize_rows(kind, w)
    ref = orc.ref_lib()
    gold = np.load(os.path.join(GOLDEN, "quantizer.npz"))
    assert np.array_equal(got, gold[kind]), "oracle vs committed reference vectors"
    if ref is not None:
        want = np.zeros_like(got)
        ref.ds4q_quantize_chunk(type_id, P(w), want.ctypes.data, 0, w.shape[0], w.shape[1], None)
        assert np.array_equal(got, want)


def test_quantizer_dequant_error_bound(orc):
    """Asymmetric codes reconstruct every weight to within half a step
    (plus the binary16 rounding of the stored scale)."""
    L = orc.lib()
    w = (rng(9).standard_normal((8, 256)) * 0.02).astype(np.float32)
    for kind, qmax, bs, dec in [("q3", 7, 110, L.orc_q3_block_decode), ("q2", 3, 84, L.orc_q2_block_decode)]:
        q = orc.quantize_rows(kind, w)
        for r in range(8):
            blk = np.ascontiguousarray(q[r * bs:(r + 1) * bs])
            d = np.zeros(256, np.float32)
            dec(P(blk, U8), P(d))
            for g in range(4):
                x = w[r, 64 * g:64 * g + 64]
                step = (x.max() - x.min()) / qmax
                err = np.abs(d[64 * g:64 * g + 64] - x)
                assert err.max() <= 0.5 * step * 1.002 + step * 2 ** -10 * qmax


# --------------------------------------------------------------------------
# CPU ops (sf37_ops.c)
# --------------------------------------------------------------------------

def test_ops_kats(orc):
    """tests/test_sf37_ops.c:89-113."""
    L = orc.lib()
    x = np.array([1.0, -2.0, 3.0, -4.0], np.float32)
    w = np.array([0.0, 0.5, -0.25, 1.0], np.float32)
    out = np.zeros(4, np.float32)
    L.orc_rms_norm_weight1(P(out), P(x), P(w), 4, 1e-5)
    s = np.float32(1.0) / np.sqrt(np.float32(np.sum(x.astype(np.float64) ** 2) / 4) + np.float32(1e-5))
    assert np.allclose(out, x * s * (w + 1), atol=1e-6)
    g = np.array([-2.0, 0.0, 10.0], np.float32)
    u = np.array([1.0, -2.0, 8.0], np.float32)
    o = np.zeros(3, np.float32)
    L.orc_swiglu(P(o), P(g), P(u), 3, 6.0)
    silu = lambda v: v / (1 + np.exp(-v))
    assert abs(o[0] - silu(-2.0)) < 1e-6 and abs(o[1]) < 1e-6 and abs(o[2] - silu(6.0) * 6.0) < 1e-5
    score = np.array([0.1, 9.0, 2.0, 9.0, -1.0, 4.0], np.float32)
    idx = np.zeros(3, np.int32)
    L.orc_topk_desc(P(score), 6, 3, P(idx, C.c_int32))
    assert list(idx) == [1, 3, 5]


def test_ops_match_reference_bitwise(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent")
    L = orc.lib()
    r = rng(11)
    # sigmoid over a wide sweep including subnormal results
    xs = np.concatenate([r.standard_normal(20000) * 8, np.linspace(-110, 90, 20000)]).astype(np.float32)
    assert all(L.orc_sigmoid(float(v)) == ref.sf37_sigmoid(float(v)) for v in xs)
    for n in (70, 256, 4096):
        x = (r.standard_normal(n) * 3).astype(np.float32)
        if n == 256:
            x[:32] = 0.0
        nb = (n + 31) // 32
        q1, q2 = np.zeros(nb * 32, np.int8), np.zeros(nb * 32, np.int8)
        s1, s2 = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
        L.orc_q8_0_quantize_activation(P(x), P(q1, C.c_int8), P(s1), n)
        ref.sf37_q8_0_quantize_activation(P(x), P(q2, C.c_int8), P(s2), n)
        assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
        out_dim = 7
        wq = r.integers(0, 256, (out_dim, nb, 34), dtype=np.uint8)
        wq[:, :, 0:2] = (r.random((out_dim, nb)) * 0.05 + 0.001).astype(np.float16).view(np.uint8).reshape(out_dim, nb, 2)
        wq = np.ascontiguousarray(wq.ravel())
        o1, o2 = np.zeros(out_dim, np.float32), np.zeros(out_dim, np.float32)
        L.orc_q8_0_matvec(P(o1), P(wq, U8), n, out_dim, P(x))
        ref.sf37_q8_0_matvec(P(o2), P(wq, U8), n, out_dim, P(x))
        assert np.array_equal(o1, o2)
        p1, p2 = np.zeros(out_dim, np.float32), np.zeros(out_dim, np.float32)
        L.orc_q8_0_matvec_pair(P(o1), P(p1), P(wq, U8), P(wq, U8), n, out_dim, P(x))
        ref.sf37_q8_0_matvec_pair(P(o2), P(p2), P(wq, U8), P(wq, U8), n, out_dim, P(x))
        assert np.array_equal(o1, o2) and np.array_equal(p1, p2)
    # q3 / q2 matvec over several blocks
    x = r.standard_normal(1024).astype(np.float32)
    w3 = np.ascontiguousarray(random_q3_blocks(5 * 4, 12).ravel())
    w2 = np.ascontiguousarray(random_q2_blocks(5 * 4, 13).ravel())
    for fo, fr, w in [(L.orc_q3_matvec, ref.sf37_q3_asym_matvec, w3), (L.orc_q2_matvec, ref.sf37_q2_asym_matvec, w2)]:
        o1, o2 = np.zeros(5, np.float32), np.zeros(5, np.float32)
        fo(P(o1), P(w, U8), 1024, 5, P(x))
        fr(P(o2), P(w, U8), 1024, 5, P(x))
        assert np.array_equal(o1, o2)
    # rms norm, swiglu with clamp, bf16 matvec
    x = (r.standard_normal(4096) * 2).astype(np.float32)
    w = (r.standard_normal(4096) * 0.1).astype(np.float32)
    o1, o2 = np.zeros(4096, np.float32), np.zeros(4096, np.float32)
    L.orc_rms_norm_weight1(P(o1), P(x), P(w), 4096, 1e-5)
    ref.sf37_rms_norm_weight1(P(o2), P(x), P(w), 4096, 1e-5)
    assert np.array_equal(o1, o2)
    g = (r.standard_normal(4096) * 10).astype(np.float32)
    L.orc_swiglu(P(o1), P(g), P(x), 4096, 7.0)
    ref.sf37_swiglu(P(o2), P(g), P(x), 4096, 7.0)
    assert np.array_equal(o1, o2)
    wb = (r.standard_normal((3, 4096)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    o1, o2 = np.zeros(3, np.float32), np.zeros(3, np.float32)
    L.orc_bf16_matvec(P(o1), P(wb, C.c_uint16), 4096, 3, P(x))
    ref.sf37_bf16_matvec(P(o2), P(wb, C.c_uint16), 4096, 3, P(x))
    assert np.array_equal(o1, o2)


# --------------------------------------------------------------------------
# Q8_K activations and the canonical integer-dot row
# --------------------------------------------------------------------------

def test_q8k_quantize_invariants(orc):
    r = rng(21)
    x = (r.standard_normal((6, 1024)) * r.uniform(0.01, 10, (6, 1))).astype(np.float32)
    x[1, 256:512] = 0.0                                   # zero block
    x[2, :256] = np.float32(1e-30)                        # tiny block
    x[3, 7] = 1e6                                         # outlier
    q = orc.q8k_quantize(x)
    xb = x.reshape(-1, 256).astype(np.float64)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(q["d"], (amax.astype(np.float32) / np.float32(127.0)))
    assert np.all(q["d"][1 * 4 + 1] == 0) and np.all(q["qs"][1 * 4 + 1] == 0)
    assert np.array_equal(q["gsums"], q["qs"].reshape(-1, 4, 64).astype(np.int32).sum(axis=2))
    nz = q["d"] > 0
    deq = q["qs"][nz].astype(np.float64) * q["d"][nz, None]
    # |q - x/d| <= 1/2 up to the rounding of x * (1/d) (a few ulps of 127)
    assert np.all(np.abs(deq - xb[nz]) <= q["d"][nz, None] * (0.5 + 1e-4))
    assert q["qs"].min() >= -127 and q["qs"].max() <= 127


def decode_codes(kind, blk):
    """(codes, zp, scale) of one block, decoded independently with numpy."""
    bits = np.unpackbits(blk, bitorder="little")
    if kind == "q3":
        codes = np.stack([bits[(12 + 24 * g) * 8:(36 + 24 * g) * 8].reshape(64, 3) @ np.array([1, 2, 4])
                          for g in range(4)])
        zp = blk[8:12] & 7
    else:
        codes = np.stack([bits[(12 + 16 * g) * 8:(28 + 16 * g) * 8].reshape(64, 2) @ np.array([1, 2])
                          for g in range(4)])
        zp = blk[8:12] & 3
    scale = blk[0:8].view(np.float16).astype(np.float64)
    return codes, zp.astype(np.int64), scale


@pytest.mark.parametrize("kind", ["q3", "q2"])
def test_group_idot_brute_force(orc, kind):
    """I_g = sum(q*qs) - zp*gsum equals sum((q - zp)*qs) computed directly."""
    L = orc.lib()
    fn = L.orc_q3_group_idot if kind == "q3" else L.orc_q2_group_idot
    blocks = random_q3_blocks(64, 31) if kind == "q3" else random_q2_blocks(64, 32)
    x = (rng(33).standard_normal((64, 256)) * 2).astype(np.float32)
    xq = orc.q8k_quantize(x)
    for i, b in enumerate(blocks):
        b = np.ascontiguousarray(b)
        codes, zp, _ = decode_codes(kind, b)
        qs = xq["qs"][i].astype(np.int64).reshape(4, 64)
        for g in range(4):
            want = int(((codes[g] - zp[g]) * qs[g]).sum())
            got = fn(P(b, U8), g, xq[i:i + 1].ctypes.data)
            assert got == want


@pytest.mark.parametrize("kind", ["q3", "q2"])
def test_canonical_row_dot_closed_form(orc, kind):
    """The canonical row dot equals sum_b d_b * sum_g s_g * I_g, to float rounding."""
    L = orc.lib()
    fn = L.orc_q3_q8k_row_dot if kind == "q3" else L.orc_q2_q8k_row_dot
    nblk = 16 if kind == "q3" else 5
    bs = 110 if kind == "q3" else 84
    mk = random_q3_blocks if kind == "q3" else random_q2_blocks
    x = (rng(41).standard_normal((1, 256 * nblk))).astype(np.float32)
    xq = orc.q8k_quantize(x)
    for row in range(20):
        blocks = mk(nblk, 100 + row)
        flat = np.ascontiguousarray(blocks.ravel())
        want = 0.0
        for b in range(nblk):
            codes, zp, scale = decode_codes(kind, blocks[b])
            qs = xq["qs"][b].astype(np.int64).reshape(4, 64)
            ig = ((codes - zp[:, None]) * qs).sum(axis=1)
            want += float(xq["d"][b]) * float((scale * ig).sum())
        got = fn(P(flat, U8), xq.ctypes.data, nblk)
        assert abs(got - want) <= 1e-5 * max(1.0, abs(want))


def test_q8k_matvec_close_to_fp32_path(orc):
    """Q8_K GEMV vs the fp32-activation GEMV at the reference's own tolerance
    (4e-3 abs, tests/test_sf37_cuda_ops.cu:589,613) on its row generators."""
    L = orc.lib()
    x = np.array([refvec.fm((i % 29) - 14, 0.02) for i in range(256)], np.float32)
    q3 = np.concatenate([refvec.make_q3_row(r) for r in range(5)])
    q2 = np.concatenate([refvec.make_q2_row(r) for r in range(5)])
    for fq, ff, w in [(L.orc_q3_q8k_matvec, L.orc_q3_matvec, q3), (L.orc_q2_q8k_matvec, L.orc_q2_matvec, q2)]:
        a, b = np.zeros(5, np.float32), np.zeros(5, np.float32)
        fq(P(a), P(w, U8), 256, 5, P(x))
        ff(P(b), P(w, U8), 256, 5, P(x))
        assert np.max(np.abs(a - b)) <= 4e-3


# --------------------------------------------------------------------------
# router, dispatch, routed experts
# --------------------------------------------------------------------------

def ref_router(ref, logits, bias, topk, scale):
    n = logits.size
    prob = np.array([ref.sf37_sigmoid(float(v)) for v in logits], np.float32)
    score = prob + bias
    idx = np.zeros(topk, np.int32)
    ref.sf37_topk_desc(P(score), n, topk, P(idx, C.c_int32))
    p = prob[idx]
    s = np.float32(0)
    for v in p:
        s = np.float32(s + v)
    s = max(s, np.float32(1e-20))
    return idx, (p / s * np.float32(scale)).astype(np.float32), prob


def test_router_reference_cases(orc):
    logits, bias = refvec.router_top8_case()
    sel, w, probs = orc.router_select(logits, bias, 8, 3.0)
    assert sel[0, 0] == 40 and sel[0, 1] == 41                 # tie -> lower index first
    assert sorted(sel[0].tolist()) == sorted([40, 41, 7, 280, 13, 120, 121, 200])
    lb, bb = refvec.router_batch_case()
    sel_b, _, _ = orc.router_select(lb, bb, 8, 3.0)
    assert np.all(sel_b[:, 0] == 40) and np.all(sel_b[:, 1] == 41)
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent")
    for lg, bs in [(logits, bias)] + [(lb[t], bb) for t in range(3)]:
        idx, wr, pr = ref_router(ref, lg, bs, 8, 3.0)
        s, ww, pp = orc.router_select(lg, bs, 8, 3.0)
        assert np.array_equal(s[0], idx)
        assert np.array_equal(ww[0].view(np.uint32), wr.view(np.uint32))
        assert np.array_equal(pp[0].view(np.uint32), pr.view(np.uint32))


def test_router_random_match_reference(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent")
    r = rng(51)
    for t in range(40):
        lg = (r.standard_normal(288) * 2).astype(np.float32)
        bs = (r.standard_normal(288) * 0.05).astype(np.float32)
        idx, wr, _ = ref_router(ref, lg, bs, 8, 3.0)
        s, ww, _ = orc.router_select(lg, bs, 8, 3.0)
        assert np.array_equal(s[0], idx) and np.array_equal(ww[0], wr)


def test_dispatch_is_stable_counting_sort(orc):
    r = rng(61)
    for n_tok, n_exp in [(1, 288), (7, 4), (512, 288), (3, 4)]:
        sel = r.integers(-1, n_exp + 1, size=(n_tok, 8)).astype(np.int32)   # includes invalid ids
        counts, offsets, order = orc.dispatch(sel, n_exp)
        e = sel.ravel().copy()
        e[(e < 0) | (e >= n_exp)] = 0
        want = np.argsort(e, kind="stable")
        assert np.array_equal(order, want.astype(np.uint32))
        assert np.array_equal(counts, np.bincount(e, minlength=n_exp).astype(np.uint32))
        assert offsets[-1] == e.size and np.array_equal(np.diff(offsets), counts)


def test_routed_moe_reference_case(orc):
    """test_router_moe (tests/test_sf37_cuda_ops.cu:698-857): q8k path vs the
    fp32 path at the reference tolerance 5e-2 abs / 1e-1 rel; fp32 path vs the
    reference CPU composition bit-exactly."""
    c = refvec.router_moe_case()
    sel, w, _ = orc.router_select(c["logits"], c["bias"], c["topk"], 3.0)
    sel, w = sel[0], w[0]
    args = (c["gate"], c["up"], c["down"], sel, w, c["n_expert"], c["in_dim"], c["mid_dim"],
            c["out_dim"], 0.0, c["x"])
    out_q, _, _ = orc.routed_moe_one_q8k(*args)
    out_f, _ = orc.routed_moe_one_f32(*args)
    diff = np.abs(out_q - out_f)
    assert np.all((diff <= 5e-2) | (diff <= 1e-1 * np.maximum(1, np.abs(out_f))))
    ref = orc.ref_lib()
    if ref is None:
        return
    want = np.zeros(c["out_dim"], np.float32)
    g = np.zeros(c["mid_dim"], np.float32)
    u = np.zeros_like(g)
    mid = np.zeros_like(g)
    down = np.zeros(c["out_dim"], np.float32)
    gb = c["mid_dim"] * 110
    db = c["out_dim"] * 84
    for s, e in enumerate(sel):
        gw = np.ascontiguousarray(c["gate"][e * gb:(e + 1) * gb])
        uw = np.ascontiguousarray(c["up"][e * gb:(e + 1) * gb])
        dw = np.ascontiguousarray(c["down"][e * db:(e + 1) * db])
        ref.sf37_q3_asym_matvec(P(g), P(gw, U8), 256, 256, P(c["x"]))
        ref.sf37_q3_asym_matvec(P(u), P(uw, U8), 256, 256, P(c["x"]))
        ref.sf37_swiglu(P(mid), P(g), P(u), 256, 0.0)
        mid *= w[s]
        ref.sf37_q2_asym_matvec(P(down), P(dw, U8), 256, c["out_dim"], P(mid))
        want += down
    assert np.array_equal(out_f, want)


def test_batch_moe_equals_per_token_and_clamps_invalid(orc):
    c = refvec.batch_moe_case()
    out, mid = orc.routed_moe_batch_q8k(c["gate"], c["up"], c["down"], c["selected"], c["weights"],
                                        c["n_expert"], c["in_dim"], c["mid_dim"], c["out_dim"], 0.0, c["x"])
    for t in range(c["n_tok"]):
        sel = c["selected"][t].copy()
        o1, _, _ = orc.routed_moe_one_q8k(c["gate"], c["up"], c["down"], sel, c["weights"][t],
                                          c["n_expert"], 256, 256, 6, 0.0, c["x"][t])
        assert np.array_equal(out[t], o1)
    # -1 behaves as expert 0
    sel = c["selected"].copy()
    sel[1, 1] = 0
    out0, _ = orc.routed_moe_batch_q8k(c["gate"], c["up"], c["down"], sel, c["weights"],
                                       c["n_expert"], 256, 256, 6, 0.0, c["x"])
    assert np.array_equal(out, out0)
    out_f = np.stack([orc.routed_moe_one_f32(c["gate"], c["up"], c["down"], c["selected"][t],
                                             c["weights"][t], 4, 256, 256, 6, 0.0, c["x"][t])[0]
                      for t in range(3)])
    diff = np.abs(out - out_f)
    assert np.all((diff <= 7e-2) | (diff <= 1.5e-1 * np.maximum(1, np.abs(out_f))))


def test_swiglu_mid_order_and_clamp(orc):
    L = orc.lib()
    # clamp 7: gate capped above only, up both sides (sf37_cuda.cu:4444-4449)
    g, u, w = 9.0, -8.0, 0.5
    got = L.orc_swiglu_mid(g, u, w, 7.0)
    s = np.float32(L.orc_sigmoid(7.0))
    want = np.float32(np.float32(np.float32(np.float32(7.0) * s) * np.float32(-7.0)) * np.float32(0.5))
    assert np.float32(got) == want
    assert L.orc_swiglu_mid(-9.0, 1.0, 1.0, 7.0) == np.float32(np.float32(-9.0) * np.float32(L.orc_sigmoid(-9.0)))
    assert L.orc_swiglu_mid(20.0, 1.0, 1.0, 0.0) == np.float32(np.float32(20.0) * np.float32(L.orc_sigmoid(20.0)))


def test_shared_expert_matches_reference(orc):
    ref = orc.ref_lib()
    r = rng(71)
    in_dim, mid_dim = 512, 256
    x = r.standard_normal(in_dim).astype(np.float32)
    wg = orc.quantize_rows("q8_0", (r.standard_normal((mid_dim, in_dim)) * 0.02).astype(np.float32))
    wu = orc.quantize_rows("q8_0", (r.standard_normal((mid_dim, in_dim)) * 0.02).astype(np.float32))
    wd = orc.quantize_rows("q8_0", (r.standard_normal((in_dim, mid_dim)) * 0.02).astype(np.float32))
    out, mid = orc.shared_expert_q8_0(wg, wu, wd, in_dim, mid_dim, in_dim, 16.0, x)
    # closed form in float64 within quantization noise
    xq = x.copy()
    assert np.all(np.isfinite(out))
    if ref is None:
        return
    g, u, m = (np.zeros(mid_dim, np.float32) for _ in range(3))
    ref.sf37_q8_0_matvec_pair(P(g), P(u), P(wg, U8), P(wu, U8), in_dim, mid_dim, P(xq))
    ref.sf37_swiglu(P(m), P(g), P(u), mid_dim, 16.0)
    want = np.zeros(in_dim, np.float32)
    ref.sf37_q8_0_matvec(P(want), P(wd, U8), mid_dim, in_dim, P(m))
    assert np.array_equal(out, want) and np.array_equal(mid, m)


# --------------------------------------------------------------------------
# synthetic generator (harness)
# --------------------------------------------------------------------------

def test_generator_statistics_and_determinism(orc):
    a = orc.fill_normal(1 << 20, seed=5, stream=3)
    b = orc.fill_normal(1 << 20, seed=5, stream=3)
    c = orc.fill_normal(1 << 20, seed=5, stream=4)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1.0) < 5e-3
    # fourth moment of a normal is 3; tails exist beyond 4 sigma
    assert abs(np.mean(a.astype(np.float64) ** 4) - 3.0) < 0.05
    assert 0 < np.sum(np.abs(a) > 4.0) < 200
    # offset windows are consistent (counter-based)
    d = orc.fill_normal(1000, seed=5, stream=3, index0=12345)
    assert np.array_equal(d, a[12345:13345])


def test_gen_quant_rows_is_quantize_of_generated(orc):
    rows, cols = 3, 512
    w = orc.fill_normal(rows * cols, seed=9, stream=7, index0=10 * cols, sigma=0.02).reshape(rows, cols)
    for kind in ("q3", "q2", "q8_0"):
        assert np.array_equal(orc.gen_quant(kind, rows, cols, 9, 7, row0=10), orc.quantize_rows(kind, w))


def test_oracle_matches_committed_reference_vectors(orc):
    """tests/golden/ops.npz holds outputs of the reference's own C code."""
    L = orc.lib()
    g = np.load(os.path.join(GOLDEN, "ops.npz"))
    sig = np.array([L.orc_sigmoid(float(v)) for v in g["sig_x"]], np.float32)
    assert np.array_equal(sig.view(np.uint32), g["sig_y"].view(np.uint32))
    q, s = np.zeros(96, np.int8), np.zeros(3, np.float32)
    L.orc_q8_0_quantize_activation(P(g["x70"]), P(q, C.c_int8), P(s), 70)
    assert np.array_equal(q, g["q70"]) and np.array_equal(s, g["s70"])
    sel, _, _ = orc.router_select(g["logits"], g["bias"], 8, 3.0)
    assert np.array_equal(sel, g["sel"])
    for i in range(g["blocks3"].shape[0]):
        b = np.ascontiguousarray(g["blocks3"][i])
        x = np.ascontiguousarray(g["x256"][i])
        assert np.float32(L.orc_q3_block_dot(P(b, U8), P(x))) == g["dot3"][i]
