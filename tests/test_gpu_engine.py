"""The engine's MoE block through the reference-ABI _mapped entry points.

libsf37_engine_moe.so (sf37_amd/csrc/sf37_engine_moe.c) is the SF37_USE_HIP
branch of the engine's per-layer step: post-attention RMSNorm, router
(F32, BF16 or Q8_0, the engine's dense dispatch), router_select, the Q8_0
shared expert, routed experts, shared + routed, residual - the call
sequences of cuda_decode_layer (sf37.c:3371-3430) and cuda_prefill_layer
(sf37.c:5936-6071), issued from C.  The model map is a host byte buffer
laid out like a mapped GGUF (one BASELINE-shape layer), uploaded with
sf37_hip_set_model_map_range, or registered as spans, or resolved on demand
and evicted.

Checked against the CPU oracle (hidden + MoE(RMSNorm(hidden)) with the Q8_K
routed path), bit for bit, at 1 and 40 tokens; router logits within 1 ulp of
the CPU's binary64 sums (F32 / BF16) or bit-exact (Q8_0), routing compared
for the GPU's logits.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, D, F, TOPK = 288, 4096, 1280, 8
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class EngineLayer(C.Structure):
    _fields_ = [("map", C.c_void_p), ("size", C.c_uint64), ("il", C.c_uint32), ("router_type", C.c_uint32),
                ("post_norm", C.c_uint64), ("router_gate", C.c_uint64), ("router_bias", C.c_uint64),
                ("share_gate", C.c_uint64), ("share_up", C.c_uint64), ("share_down", C.c_uint64),
                ("moe_gate", C.c_uint64), ("moe_up", C.c_uint64), ("moe_down", C.c_uint64),
                ("n_expert", C.c_uint32), ("topk", C.c_uint32), ("embd", C.c_uint32), ("expert_ff", C.c_uint32)]


BUF_FIELDS = ["hidden", "ffn_norm", "gate", "up", "mid", "ffn_out", "router_logits", "router_probs",
              "router_selected", "router_weights", "routed_gate", "routed_up", "routed_mid", "routed_down",
              "routed_out"]


class EngineBufs(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in BUF_FIELDS]


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


@pytest.fixture(scope="module")
def ENG(H):
    L = C.CDLL(os.path.join(ROOT, "sf37_amd", "libsf37_engine_moe.so"))
    for name, extra in (("sf37_engine_moe_decode", []), ("sf37_engine_moe_prefill", [C.c_uint32])):
        fn = getattr(L, name)
        fn.restype = C.c_int
        fn.argtypes = [C.POINTER(EngineLayer), C.POINTER(EngineBufs)] + extra
    return L


class ModelMap:
    """One BASELINE-shape MoE layer laid out in a host byte buffer the way a
    mapped GGUF holds it (tensors at 256-aligned offsets), with the router
    in F32, BF16 and Q8_0."""

    def __init__(self, H, O, seed, il):
        from sf37_amd.moe import SynthLayer, bf16_bits
        lay = SynthLayer(seed=seed, il=il)
        H.synchronize()
        rng = np.random.default_rng(seed)
        router = lay.router.read(np.float32)
        parts = {
            "post_norm": bf16_bits((rng.standard_normal(D) * 0.02).astype(np.float32)).view(np.uint8),
            "router_f32": router.view(np.uint8),
            "router_bf16": bf16_bits(router).view(np.uint8),
            "router_q8_0": O.quantize_rows("q8_0", router.reshape(E, D)),
            "router_bias": (rng.standard_normal(E) * 0.05).astype(np.float32).view(np.uint8),
            "share_gate": lay.sh_gate.read(np.uint8), "share_up": lay.sh_up.read(np.uint8),
            "share_down": lay.sh_down.read(np.uint8),
            "moe_gate": lay.gate.read(np.uint8), "moe_up": lay.up.read(np.uint8), "moe_down": lay.down.read(np.uint8),
        }
        lay.free()
        self.off, pos = {}, 1024                 # a header-sized gap before the data
        for k, v in parts.items():
            self.off[k] = pos
            pos = (pos + v.nbytes + 255) // 256 * 256
        self.buf = np.zeros(pos, np.uint8)
        for k, v in parts.items():
            self.buf[self.off[k]:self.off[k] + v.nbytes] = v
        self.nbytes = {k: v.nbytes for k, v in parts.items()}
        self.il = il

    def view(self, name, dtype=np.uint8):
        o = self.off[name]
        return self.buf[o:o + self.nbytes[name]].view(dtype)

    def layer(self, router="f32", buf=None):
        b = self.buf if buf is None else buf
        t = {"f32": 0, "q8_0": 8, "bf16": 30}[router]
        o = self.off
        return EngineLayer(b.ctypes.data, b.nbytes, self.il, t, o["post_norm"], o["router_" + router],
                           o["router_bias"], o["share_gate"], o["share_up"], o["share_down"], o["moe_gate"],
                           o["moe_up"], o["moe_down"], E, TOPK, D, F)

    def oracle_weights(self):
        return {"gate": self.view("moe_gate"), "up": self.view("moe_up"), "down": self.view("moe_down"),
                "router": self.view("router_f32", np.float32), "router_bias": self.view("router_bias", np.float32),
                "sh_gate": self.view("share_gate"), "sh_up": self.view("share_up"),
                "sh_down": self.view("share_down"), "n_expert": E, "mid_dim": F}


@pytest.fixture(scope="module")
def mm(H, O):
    say("building a BASELINE-shape model map (layer 43, clamps 7 / 16)")
    m = ModelMap(H, O, seed=4301, il=43)
    assert H.lib().sf37_hip_set_model_map_range(m.buf.ctypes.data, m.buf.nbytes, 0, m.buf.nbytes, 0)
    return m


def make_bufs(H, n_tok):
    sizes = {"hidden": n_tok * D * 4, "ffn_norm": n_tok * D * 4, "gate": max(n_tok, TOPK) * F * 4,
             "up": max(n_tok, TOPK) * F * 4, "mid": max(n_tok, TOPK) * F * 4, "ffn_out": n_tok * D * 4,
             "router_logits": n_tok * E * 4, "router_probs": n_tok * E * 4, "router_selected": n_tok * TOPK * 4,
             "router_weights": n_tok * TOPK * 4, "routed_gate": n_tok * TOPK * F * 4,
             "routed_up": n_tok * TOPK * F * 4, "routed_mid": n_tok * TOPK * F * 4, "routed_down": TOPK * D * 4,
             "routed_out": n_tok * D * 4}
    t = {k: H.Tensor.alloc(v) for k, v in sizes.items()}
    return t, EngineBufs(*[t[k].h for k in BUF_FIELDS])


def run_block(H, ENG, m, h0, router="f32", buf=None):
    n_tok = h0.shape[0]
    t, b = make_bufs(H, n_tok)
    t["hidden"].write(h0)
    lay = m.layer(router, buf)
    ok = ENG.sf37_engine_moe_decode(C.byref(lay), C.byref(b)) if n_tok == 1 else \
        ENG.sf37_engine_moe_prefill(C.byref(lay), C.byref(b), n_tok)
    assert ok, "engine MoE block failed"
    r = {k: t[k].read(np.float32) for k in ("hidden", "ffn_norm", "router_logits", "router_weights")}
    r["selected"] = t["router_selected"].read(np.int32).reshape(n_tok, TOPK)
    r["routed_mid"] = t["routed_mid"].read(np.float32)
    return r


def oracle_block(O, m, h0, logits):
    """h0 + moe_layer_q8k(RMSNorm(h0)) for the GPU's router logits."""
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    n_tok = h0.shape[0]
    xn = np.zeros_like(h0)
    nw = np.ascontiguousarray(m.view("post_norm", np.uint16))
    for t in range(n_tok):
        O.lib().orc_rms_norm_weight1_bf16(fp(xn[t]), fp(np.ascontiguousarray(h0[t])),
                                          nw.ctypes.data_as(C.POINTER(C.c_uint16)), D, 1e-5)
    y, sel, wts = O.moe_layer_q8k(m.oracle_weights(), xn, logits=logits.reshape(n_tok, E), clamp_routed=7.0,
                                  clamp_shared=16.0)
    return (h0 + y).astype(np.float32), xn, sel, wts


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got, np.float32).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want, np.float32).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[0]}: "
                           f"{np.ravel(got)[bad[0]]!r} vs {np.ravel(want)[bad[0]]!r}")


def host_logits(O, m, xn, router):
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    out = np.zeros((xn.shape[0], E), np.float32)
    L = O.lib()
    for t in range(xn.shape[0]):
        x = np.ascontiguousarray(xn[t])
        if router == "f32":
            L.orc_f32_matvec_double(fp(out[t]), fp(m.view("router_f32", np.float32)), D, E, fp(x))
        elif router == "bf16":
            w = np.ascontiguousarray(m.view("router_bf16", np.uint16))
            L.orc_bf16_matvec(fp(out[t]), w.ctypes.data_as(C.POINTER(C.c_uint16)), D, E, fp(x))
        else:
            w = np.ascontiguousarray(m.view("router_q8_0"))
            L.orc_q8_0_matvec(fp(out[t]), w.ctypes.data_as(C.POINTER(C.c_uint8)), D, E, fp(x))
    return out


@pytest.mark.parametrize("n_tok,router", [(1, "f32"), (40, "f32"), (1, "bf16"), (40, "bf16"), (1, "q8_0"),
                                          (40, "q8_0")])
def test_engine_block_vs_oracle(H, O, ENG, mm, n_tok, router):
    say(f"engine MoE block: {n_tok} tokens, {router} router")
    rng = np.random.default_rng(100 + n_tok)
    h0 = (rng.standard_normal((n_tok, D)) * 2).astype(np.float32)
    r = run_block(H, ENG, mm, h0, router)
    want, xn, sel, wts = oracle_block(O, mm, h0, r["router_logits"])
    assert_bitexact(r["ffn_norm"], xn, "post-attention RMSNorm rows")
    lg = r["router_logits"].reshape(n_tok, E)
    ref = host_logits(O, mm, xn, router)
    if router == "q8_0":
        assert_bitexact(lg, ref, "Q8_0 router logits")
    else:
        assert np.all(np.abs(lg - ref) <= np.spacing(np.abs(ref))), "router logits beyond 1 ulp"
    assert np.array_equal(r["selected"], sel), "top-8 differs from the oracle's for the same logits"
    assert_bitexact(r["router_weights"], wts, "routing weights")
    assert_bitexact(r["hidden"], want, f"hidden after the block, {n_tok} tokens")
    if n_tok > 1:
        # the per-pair SwiGLU rows exported through routed_mid (sf37_cuda.cu:5665-5674)
        pairs = n_tok * TOPK
        w = mm.oracle_weights()
        _, mid = O.routed_moe_batch_q8k(w["gate"], w["up"], w["down"], sel, wts, E, D, F, D, 7.0, xn)
        assert_bitexact(r["routed_mid"][:pairs * F], mid, "exported routed mid")


def test_engine_block_spans_cache_evict(H, O, ENG, mm):
    """The same layer through a map registered as per-tensor spans, and
    through a map never registered (ranges copied on first use), before and
    after cache_model_range + evict_model_cache: the same bits as the map
    registered whole."""
    L = H.lib()
    rng = np.random.default_rng(7)
    h0 = (rng.standard_normal((1, D)) * 2).astype(np.float32)
    base = run_block(H, ENG, mm, h0)["hidden"]
    spans = mm.buf.copy()
    names = list(mm.off)
    offs = (C.c_uint64 * len(names))(*[mm.off[k] for k in names])
    sizes = (C.c_uint64 * len(names))(*[mm.nbytes[k] for k in names])
    assert L.sf37_hip_set_model_map_spans(spans.ctypes.data, spans.nbytes, offs, sizes, len(names), 0)
    assert_bitexact(run_block(H, ENG, mm, h0, buf=spans)["hidden"], base, "map registered as spans")
    lazy = mm.buf.copy()
    assert_bitexact(run_block(H, ENG, mm, h0, buf=lazy)["hidden"], base, "unregistered map, on-demand copies")
    assert L.sf37_hip_cache_model_range(lazy.ctypes.data, lazy.nbytes, mm.off["router_f32"],
                                        mm.nbytes["router_f32"], b"router")
    L.sf37_hip_evict_model_cache(b"test")
    assert_bitexact(run_block(H, ENG, mm, h0, buf=lazy)["hidden"], base, "after evict_model_cache")
    # a range outside the map is refused before any launch
    out = H.Tensor.alloc(E * 4)
    x = H.Tensor.alloc(D * 4)
    assert not L.sf37_hip_matvec_f32_mapped(out, lazy.ctypes.data, lazy.nbytes, lazy.nbytes - 16, D, E, x)
