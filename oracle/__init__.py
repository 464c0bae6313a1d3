"""CPU oracle for the SF37 MoE FFN hot path.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py load this package as the checker; the product (sf37_amd/)
never imports it.  liborc.so is this build's C restatement of the reference
(sf37_oracle.c, each function citing the reference file:line it follows);
_ref/ holds the reference's own C sources compiled in place (oracle/Makefile)
and is used to pin the restatement where it is present.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
QK_K = 256
Q8_0_BLOCK = 34
Q3_BLOCK = 110
Q2_BLOCK = 84
Q8K_BYTES = 268

Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("gsums", "<i2", (4,))])
assert Q8K_DTYPE.itemsize == Q8K_BYTES

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_i8 = C.POINTER(C.c_int8)
_i32 = C.POINTER(C.c_int32)
_u32 = C.POINTER(C.c_uint32)
_u16 = C.POINTER(C.c_uint16)
_vp = C.c_void_p
_u64 = C.c_uint64
_u32v = C.c_uint32


def build(with_ref: bool | None = None) -> None:
    """Compile liborc (always) and the _ref libraries when the reference is present."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if with_ref is None:
        with_ref = os.path.isdir("/root/reference")
    if with_ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


_LIB = None
_REF = None
_CPU = {}


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liborc.so")
        if not os.path.exists(path):
            build(with_ref=False)
        L = C.CDLL(path)
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_sigmoid": (C.c_float, [C.c_float]),
            "orc_q8k_quantize": (None, [_vp, _f, _u32v, _u32v]),
            "orc_q3_q8k_row_dot": (C.c_float, [_u8, _vp, _u32v]),
            "orc_q2_q8k_row_dot": (C.c_float, [_u8, _vp, _u32v]),
            "orc_q3_group_idot": (C.c_int32, [_u8, C.c_int, _vp]),
            "orc_q2_group_idot": (C.c_int32, [_u8, C.c_int, _vp]),
            "orc_quantize_rows": (None, [C.c_int, _f, _u8, C.c_int64, C.c_int64]),
            "orc_q3_block_decode": (None, [_u8, _f]),
            "orc_q2_block_decode": (None, [_u8, _f]),
            "orc_q8_0_block_decode": (None, [_u8, _f]),
            "orc_q3_block_dot": (C.c_float, [_u8, _f]),
            "orc_q2_block_dot": (C.c_float, [_u8, _f]),
            "orc_q8_0_block_dot": (C.c_float, [_u8, _f]),
            "orc_rms_norm_weight1": (None, [_f, _f, _f, _u64, C.c_float]),
            "orc_rms_norm_weight1_bf16": (None, [_f, _f, _u16, _u64, C.c_float]),
            "orc_swiglu": (None, [_f, _f, _f, _u64, C.c_float]),
            "orc_topk_desc": (None, [_f, C.c_int, C.c_int, _i32]),
            "orc_q8_0_quantize_activation": (None, [_f, _i8, _f, _u64]),
            "orc_q8_0_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "orc_q8_0_matvec_pair": (None, [_f, _f, _u8, _u8, _u64, _u64, _f]),
            "orc_bf16_matvec": (None, [_f, _u16, _u64, _u64, _f]),
            "orc_q3_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "orc_q2_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "orc_q3_q8k_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "orc_q2_q8k_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "orc_f32_matvec_double": (None, [_f, _f, _u64, _u64, _f]),
            "orc_swiglu_mid": (C.c_float, [C.c_float, C.c_float, C.c_float, C.c_float]),
            "orc_router_select": (None, [_i32, _f, _f, _f, _f, _u32v, _u32v, C.c_float]),
            "orc_router_select_batch": (None, [_i32, _f, _f, _f, _f, _u32v, _u32v, C.c_float, _u32v]),
            "orc_routed_moe_one_q8k": (None, [_f, _f, _vp, _u8, _u8, _u8, _i32, _f, _u32v, _u32v,
                                              _u32v, _u32v, _u32v, C.c_float, _f]),
            "orc_routed_moe_one_f32": (None, [_f, _f, _u8, _u8, _u8, _i32, _f, _u32v, _u32v,
                                              _u32v, _u32v, _u32v, C.c_float, _f]),
            "orc_moe_dispatch": (None, [_i32, _u32v, _u32v, _u32, _u32, _u32]),
            "orc_routed_moe_batch_q8k": (None, [_f, _f, _u8, _u8, _u8, _i32, _f, _u32v, _u32v,
                                                _u32v, _u32v, _u32v, C.c_float, _f, _u32v]),
            "orc_shared_expert_q8_0": (None, [_f, _f, _u8, _u8, _u8, _u32v, _u32v, _u32v,
                                              C.c_float, _f]),
            "orc_moe_layer_q8k": (None, [_f, _i32, _f, _f, _f, _f, _u8, _u8, _u8, _u8, _u8, _u8,
                                         _u32v, _u32v, _u32v, _u32v, C.c_float, C.c_float,
                                         C.c_float, _f, _u32v]),
            "orc_expf_array": (None, [_f, _f, _u64]),
            "orc_sigmoid_array": (None, [_f, _f, _u64]),
            "orc_rng_u64": (C.c_uint64, [_u64, _u64, _u64]),
            "orc_rng_normal": (C.c_float, [_u64, _u64, _u64]),
            "orc_fill_normal": (None, [_f, _u64, _u64, _u64, _u64, C.c_float]),
            "orc_gen_quant_rows": (None, [C.c_int, _u8, _u64, _u64, _u64, _u64, _u64, C.c_float]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def ref_lib():
    """The reference's own sf37_quant.c/sf37_ops.c/quants.c (IEEE build), or None."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libsf37ref.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        sig = {
            "sf37_f16_to_f32": (C.c_float, [C.c_uint16]),
            "sf37_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "sf37_q3_asym_block_decode": (None, [_u8, _f]),
            "sf37_q2_asym_block_decode": (None, [_u8, _f]),
            "sf37_q8_0_block_decode": (None, [_u8, _f]),
            "sf37_q3_asym_block_dot": (C.c_float, [_u8, _f]),
            "sf37_q2_asym_block_dot": (C.c_float, [_u8, _f]),
            "sf37_q8_0_block_dot": (C.c_float, [_u8, _f]),
            "sf37_sigmoid": (C.c_float, [C.c_float]),
            "sf37_rms_norm_weight1": (None, [_f, _f, _f, _u64, C.c_float]),
            "sf37_swiglu": (None, [_f, _f, _f, _u64, C.c_float]),
            "sf37_topk_desc": (None, [_f, C.c_int, C.c_int, _i32]),
            "sf37_q8_0_quantize_activation": (None, [_f, _i8, _f, _u64]),
            "sf37_q8_0_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "sf37_q8_0_matvec_pair": (None, [_f, _f, _u8, _u8, _u64, _u64, _f]),
            "sf37_bf16_matvec": (None, [_f, _u16, _u64, _u64, _f]),
            "sf37_q3_asym_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "sf37_q2_asym_matvec": (None, [_f, _u8, _u64, _u64, _f]),
            "ds4q_quantize_chunk": (C.c_size_t, [C.c_int, _f, _vp, C.c_int64, C.c_int64, C.c_int64, _f]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _REF = L
    return _REF


def cpu_baseline_lib(kind: str = "reference"):
    """CPU MoE layer per token: 'reference' (reference sources, make-cpu flags) or 'port'."""
    if kind not in _CPU:
        path = os.path.join(HERE, "_ref", "libsf37cpu_ref.so") if kind == "reference" \
            else os.path.join(HERE, "libsf37cpu_port.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        fn = L.sf37cpu_moe_ffn_token
        fn.restype = None
        fn.argtypes = [_f, _i32, _f, _f, _u8, _u8, _u8, _u8, _u8, _u8, _u32v, _u32v, _u32v,
                       _u32v, C.c_float, C.c_float, _f]
        _CPU[kind] = L
    return _CPU[kind]


# ---------------------------------------------------------------------------
# numpy conveniences
# ---------------------------------------------------------------------------

def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def q8k_quantize(x: np.ndarray) -> np.ndarray:
    """Q8_K blocks of each row of x (rows of a multiple of 256 floats)."""
    x = f32(np.atleast_2d(x))
    rows, n = x.shape
    out = np.zeros(rows * (n // QK_K), dtype=Q8K_DTYPE)
    lib().orc_q8k_quantize(out.ctypes.data, _p(x, _f), n, rows)
    return out


def quantize_rows(kind: str, w: np.ndarray) -> np.ndarray:
    """Quantize fp32 rows with the reference weight quantizer: kind in q8_0, q3, q2."""
    w = f32(np.atleast_2d(w))
    rows, n = w.shape
    t = {"q8_0": 0, "q3": 3, "q2": 2}[kind]
    qk, bs = (32, Q8_0_BLOCK) if t == 0 else (QK_K, Q3_BLOCK if t == 3 else Q2_BLOCK)
    out = np.zeros(rows * (n // qk) * bs, dtype=np.uint8)
    lib().orc_quantize_rows(t, _p(w, _f), _p(out, _u8), rows, n)
    return out


def row_bytes(kind: str, n: int) -> int:
    if kind == "q8_0":
        return (n + 31) // 32 * Q8_0_BLOCK
    return n // QK_K * (Q3_BLOCK if kind == "q3" else Q2_BLOCK)


def gen_quant(kind: str, rows: int, cols: int, seed: int, stream: int, row0: int = 0,
              sigma: float = 0.02) -> np.ndarray:
    t = {"q8_0": 0, "q3": 3, "q2": 2}[kind]
    out = np.zeros(rows * row_bytes(kind, cols), dtype=np.uint8)
    lib().orc_gen_quant_rows(t, _p(out, _u8), row0, rows, cols, seed, stream, sigma)
    return out


def fill_normal(n: int, seed: int, stream: int, index0: int = 0, sigma: float = 1.0):
    out = np.zeros(n, dtype=np.float32)
    lib().orc_fill_normal(_p(out, _f), n, seed, stream, index0, sigma)
    return out


def router_select(logits, bias, topk=8, scale=3.0):
    logits = f32(np.atleast_2d(logits))
    bias = f32(bias)
    n_tok, n_exp = logits.shape
    sel = np.zeros((n_tok, topk), dtype=np.int32)
    w = np.zeros((n_tok, topk), dtype=np.float32)
    probs = np.zeros((n_tok, n_exp), dtype=np.float32)
    lib().orc_router_select_batch(_p(sel, _i32), _p(w, _f), _p(probs, _f), _p(logits, _f),
                                  _p(bias, _f), n_exp, topk, scale, n_tok)
    return sel, w, probs


def dispatch(selected: np.ndarray, n_expert: int):
    sel = np.ascontiguousarray(selected, dtype=np.int32).ravel()
    counts = np.zeros(n_expert, dtype=np.uint32)
    offsets = np.zeros(n_expert + 1, dtype=np.uint32)
    sorted_pairs = np.zeros(sel.size, dtype=np.uint32)
    lib().orc_moe_dispatch(_p(sel, _i32), sel.size, n_expert, _p(counts, _u32),
                           _p(offsets, _u32), _p(sorted_pairs, _u32))
    return counts, offsets, sorted_pairs


def routed_moe_one_q8k(gate_w, up_w, down_w, selected, weights, n_expert, in_dim, mid_dim,
                       out_dim, clamp, x):
    topk = len(selected)
    out = np.zeros(out_dim, dtype=np.float32)
    mid = np.zeros(topk * mid_dim, dtype=np.float32)
    midq = np.zeros(topk * (mid_dim // QK_K), dtype=Q8K_DTYPE)
    sel = np.ascontiguousarray(selected, dtype=np.int32)
    w = f32(weights)
    x = f32(x)
    lib().orc_routed_moe_one_q8k(_p(out, _f), _p(mid, _f), midq.ctypes.data, _p(gate_w, _u8),
                                 _p(up_w, _u8), _p(down_w, _u8), _p(sel, _i32), _p(w, _f),
                                 n_expert, topk, in_dim, mid_dim, out_dim, clamp, _p(x, _f))
    return out, mid.reshape(topk, mid_dim), midq


def routed_moe_one_f32(gate_w, up_w, down_w, selected, weights, n_expert, in_dim, mid_dim,
                       out_dim, clamp, x):
    topk = len(selected)
    out = np.zeros(out_dim, dtype=np.float32)
    mid = np.zeros(topk * mid_dim, dtype=np.float32)
    sel = np.ascontiguousarray(selected, dtype=np.int32)
    lib().orc_routed_moe_one_f32(_p(out, _f), _p(mid, _f), _p(gate_w, _u8), _p(up_w, _u8),
                                 _p(down_w, _u8), _p(sel, _i32), _p(f32(weights), _f), n_expert,
                                 topk, in_dim, mid_dim, out_dim, clamp, _p(f32(x), _f))
    return out, mid.reshape(topk, mid_dim)


def routed_moe_batch_q8k(gate_w, up_w, down_w, selected, weights, n_expert, in_dim, mid_dim,
                         out_dim, clamp, x):
    sel = np.ascontiguousarray(selected, dtype=np.int32)
    n_tok, topk = sel.shape
    out = np.zeros((n_tok, out_dim), dtype=np.float32)
    mid = np.zeros((n_tok * topk, mid_dim), dtype=np.float32)
    lib().orc_routed_moe_batch_q8k(_p(out, _f), _p(mid, _f), _p(gate_w, _u8), _p(up_w, _u8),
                                   _p(down_w, _u8), _p(sel, _i32), _p(f32(weights), _f),
                                   n_expert, topk, in_dim, mid_dim, out_dim, clamp,
                                   _p(f32(x), _f), n_tok)
    return out, mid


def shared_expert_q8_0(gate_w, up_w, down_w, in_dim, mid_dim, out_dim, clamp, x):
    out = np.zeros(out_dim, dtype=np.float32)
    mid = np.zeros(mid_dim, dtype=np.float32)
    lib().orc_shared_expert_q8_0(_p(out, _f), _p(mid, _f), _p(gate_w, _u8), _p(up_w, _u8),
                                 _p(down_w, _u8), in_dim, mid_dim, out_dim, clamp, _p(f32(x), _f))
    return out, mid


def moe_layer_q8k(weights: dict, x, logits=None, topk=8, scale=3.0, clamp_routed=0.0,
                  clamp_shared=0.0, shared_format="q8_0"):
    """Whole MoE layer (router, shared, routed, add) for rows of x.

    shared_format "q8_0": the engine's Q8_0 shared expert (sf37.c:2159-2167).
    "q3q2": the benchmark configurations' shared expert in the routed formats
    (Q3GU gate/up, Q2D down), computed as one more routed expert on the Q8_K
    path with routing weight 1.0 and the shared clamp; out = shared + routed
    (sf37.c:3428)."""
    if shared_format == "q3q2":
        return _moe_layer_shared_q3q2(weights, x, logits, topk, scale, clamp_routed, clamp_shared)
    x = f32(np.atleast_2d(x))
    n_tok, in_dim = x.shape
    n_exp = weights["n_expert"]
    mid_dim = weights["mid_dim"]
    out = np.zeros((n_tok, in_dim), dtype=np.float32)
    sel = np.zeros((n_tok, topk), dtype=np.int32)
    w = np.zeros((n_tok, topk), dtype=np.float32)
    lg = None if logits is None else f32(logits)
    lib().orc_moe_layer_q8k(_p(out, _f), _p(sel, _i32), _p(w, _f), _p(weights["router"], _f),
                            _p(weights["router_bias"], _f), _p(lg, _f), _p(weights["gate"], _u8),
                            _p(weights["up"], _u8), _p(weights["down"], _u8),
                            _p(weights["sh_gate"], _u8), _p(weights["sh_up"], _u8),
                            _p(weights["sh_down"], _u8), n_exp, topk, in_dim, mid_dim,
                            clamp_routed, clamp_shared, scale, _p(x, _f), n_tok)
    return out, sel, w


def _moe_layer_shared_q3q2(weights, x, logits, topk, scale, clamp_routed, clamp_shared):
    x = f32(np.atleast_2d(x))
    n_tok, in_dim = x.shape
    n_exp, mid_dim = weights["n_expert"], weights["mid_dim"]
    if logits is None:
        logits = np.zeros((n_tok, n_exp), np.float32)
        for t in range(n_tok):
            lib().orc_f32_matvec_double(_p(logits[t], _f), _p(f32(weights["router"]), _f), in_dim, n_exp,
                                        _p(np.ascontiguousarray(x[t]), _f))
    sel, w, _ = router_select(logits, weights["router_bias"], topk, scale)
    shared, _ = routed_moe_batch_q8k(weights["sh_gate"], weights["sh_up"], weights["sh_down"],
                                     np.zeros((n_tok, 1), np.int32), np.ones((n_tok, 1), np.float32), 1,
                                     in_dim, mid_dim, in_dim, clamp_shared, x)
    routed, _ = routed_moe_batch_q8k(weights["gate"], weights["up"], weights["down"], sel, w, n_exp, in_dim,
                                     mid_dim, in_dim, clamp_routed, x)
    return (shared + routed).astype(np.float32), sel, w


def max_abs_rel(got, want) -> float:
    """max |a-b| / max(|b|, 1): the reference's assert_close_rel scale
    (tests/test_sf37_cuda_ops.cu:20-30)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    if got.size == 0:
        return 0.0
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)))
