"""ctypes binding of the C ABI in include/sf37_hip.h (libsf37_hip.so).

The library is the product: every call here goes straight to a C entry
point.  There is no fallback: if the shared library is missing or does not
load, importing functions from this module raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libsf37_hip.so")
HEADER = os.path.join(ROOT, "include", "sf37_hip.h")

QK_K = 256
Q8_0_BLOCK = 34
Q3_BLOCK = 110
Q2_BLOCK = 84
Q8K_BLOCK = 268

T = C.c_void_p          # sf37_hip_tensor *
u32, u64, i32, i64, f32 = C.c_uint32, C.c_uint64, C.c_int32, C.c_int64, C.c_float
vp = C.c_void_p


class LayerWeights(C.Structure):
    """sf37_hip_moe_layer_weights."""
    _fields_ = [("router", T), ("router_bias", T), ("gate", T), ("up", T), ("down", T),
                ("sh_gate", T), ("sh_up", T), ("sh_down", T),
                ("n_expert", u32), ("topk", u32), ("in_dim", u32), ("mid_dim", u32),
                ("scale", f32), ("clamp_routed", f32), ("clamp_shared", f32),
                ("router_type", u32), ("shared_type", u32)]

TYPE_F32, TYPE_Q8_0, TYPE_Q3GU, TYPE_BF16 = 0, 8, 11, 30


_SIGS = {
    "sf37_hip_device_count": (C.c_int, []),
    "sf37_hip_print_devices": (None, []),
    "sf37_hip_init": (C.c_int, []),
    "sf37_hip_cleanup": (None, []),
    "sf37_hip_synchronize": (C.c_int, []),
    "sf37_hip_memory_info": (C.c_int, [C.POINTER(u64), C.POINTER(u64)]),
    "sf37_hip_begin_layer": (C.c_int, [u32]),
    "sf37_hip_end_layer": (None, []),
    "sf37_hip_set_model_fd": (C.c_int, [C.c_int]),
    "sf37_hip_set_model_map_range": (C.c_int, [vp, u64, u64, u64, u64]),
    "sf37_hip_set_model_map_spans": (C.c_int, [vp, u64, C.POINTER(u64), C.POINTER(u64), u32, u64]),
    "sf37_hip_cache_model_range": (C.c_int, [vp, u64, u64, u64, C.c_char_p]),
    "sf37_hip_evict_model_cache": (None, [C.c_char_p]),
    "sf37_hip_tensor_alloc": (T, [u64]),
    "sf37_hip_tensor_alloc_managed": (T, [u64]),
    "sf37_hip_tensor_free": (None, [T]),
    "sf37_hip_tensor_bytes": (u64, [T]),
    "sf37_hip_tensor_write": (C.c_int, [T, u64, vp, u64]),
    "sf37_hip_tensor_read": (C.c_int, [T, u64, vp, u64]),
    "sf37_hip_tensor_copy": (C.c_int, [T, u64, T, u64, u64]),
    "sf37_hip_tensor_fill_f32": (C.c_int, [T, f32, u64]),
    "sf37_hip_rms_norm_weight1_f32": (C.c_int, [T, T, T, u32, f32]),
    "sf37_hip_rms_norm_weight1_bf16": (C.c_int, [T, T, T, u32, f32]),
    "sf37_hip_add_inplace_f32": (C.c_int, [T, T, u64]),
    "sf37_hip_swiglu_f32": (C.c_int, [T, T, T, u64, f32]),
    "sf37_hip_matvec_q8_0": (C.c_int, [T, T, u64, u64, T]),
    "sf37_hip_matvec_q8_0_pair": (C.c_int, [T, T, T, T, u64, u64, T]),
    "sf37_hip_matvec_f32": (C.c_int, [T, T, u64, u64, T]),
    "sf37_hip_matvec_bf16": (C.c_int, [T, T, u64, u64, T]),
    "sf37_hip_matvec_bf16_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T]),
    "sf37_hip_matmul_bf16_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T, u64]),
    "sf37_hip_matvec_q3_asym": (C.c_int, [T, T, u64, u64, T]),
    "sf37_hip_matvec_q2_asym": (C.c_int, [T, T, u64, u64, T]),
    "sf37_hip_router_select": (C.c_int, [T, T, T, T, T, u32, u32, f32]),
    "sf37_hip_routed_moe_one": (C.c_int, [T, T, T, T, T, T, T, T, T, T, u32, u32, u32, u32, u32, f32, T]),
    "sf37_hip_rms_norm_weight1_bf16_mapped": (C.c_int, [T, T, vp, u64, u64, u32, f32]),
    "sf37_hip_rms_norm_weight1_bf16_batch_mapped": (C.c_int, [T, T, vp, u64, u64, u32, u32, f32]),
    "sf37_hip_matvec_q8_0_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T]),
    "sf37_hip_matmul_q8_0_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T, u64]),
    "sf37_hip_matmul_q8_0_pair_mapped": (C.c_int, [T, T, vp, u64, u64, u64, u64, u64, T, u64]),
    "sf37_hip_matvec_q8_0_pair_mapped": (C.c_int, [T, T, vp, u64, u64, u64, u64, u64, T]),
    "sf37_hip_matvec_f32_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T]),
    "sf37_hip_matmul_f32_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T, u64]),
    "sf37_hip_matvec_q3_asym_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T]),
    "sf37_hip_matvec_q2_asym_mapped": (C.c_int, [T, vp, u64, u64, u64, u64, T]),
    "sf37_hip_router_select_mapped": (C.c_int, [T, T, T, T, vp, u64, u64, u32, u32, f32]),
    "sf37_hip_router_select_batch_mapped": (C.c_int, [T, T, T, T, vp, u64, u64, u32, u32, f32, u32]),
    "sf37_hip_routed_moe_one_mapped": (C.c_int, [T, T, T, T, T, vp, u64, u64, u64, u64, T, T, u32, u32,
                                                  u32, u32, u32, f32, T]),
    "sf37_hip_routed_moe_batch_mapped": (C.c_int, [T, T, T, T, T, vp, u64, u64, u64, u64, T, T, u32, u32,
                                                    u32, u32, u32, f32, T, u32]),
    "sf37_hip_set_stream": (C.c_int, [vp]),
    "sf37_hip_get_stream": (vp, []),
    "sf37_hip_set_option": (C.c_int, [C.c_char_p, i64]),
    "sf37_hip_get_option": (i64, [C.c_char_p]),
    "sf37_hip_tensor_device_ptr": (vp, [T]),
    "sf37_hip_tensor_view": (T, [T, u64, u64]),
    "sf37_hip_register_device_range": (C.c_int, [vp, u64, u64, u64, T]),
    "sf37_hip_model_range_holds": (C.c_int, [vp, u64, u64]),
    "sf37_hip_device_memory_requests": (u64, []),
    "sf37_hip_q8k_quantize": (C.c_int, [T, T, u32, u32]),
    "sf37_hip_moe_dispatch": (C.c_int, [T, T, T, T, u32, u32]),
    "sf37_hip_moe_layer": (C.c_int, [T, T, T, C.POINTER(LayerWeights), T, T, u32]),
    "sf37_hip_moe_layer_noalloc": (C.c_int, [T, T, T, C.POINTER(LayerWeights), T, T, u32]),
    "sf37_hip_gguf_open": (vp, [C.c_char_p]),
    "sf37_hip_gguf_from_map": (vp, [vp, u64]),
    "sf37_hip_gguf_close": (None, [vp]),
    "sf37_hip_gguf_map": (vp, [vp, C.POINTER(u64)]),
    "sf37_hip_gguf_tensor": (C.c_int, [vp, C.c_char_p, C.POINTER(u64), C.POINTER(u64), C.POINTER(u32),
                                       C.POINTER(u32), C.POINTER(u64)]),
    "sf37_hip_gguf_bind_moe_layer": (C.c_int, [vp, u32, C.POINTER(LayerWeights), C.POINTER(u64)]),
    "sf37_hip_moe_block": (C.c_int, [T, T, T, T, C.POINTER(LayerWeights), vp, u64, u64, f32, T, u32]),
    "sf37_hip_moe_stack": (C.c_int, [T, u32, C.POINTER(LayerWeights), vp, u64, C.POINTER(u64), f32, C.POINTER(T),
                                     C.POINTER(T), u32]),
    "sf37_hip_synth_normal": (C.c_int, [T, u64, u64, u64, u64, f32]),
    "sf37_hip_synth_quant_rows": (C.c_int, [C.c_int, T, u64, u64, u64, u64, u64, f32]),
    "sf37_hip_sigmoid_array": (C.c_int, [T, T, u64, C.c_int]),
    "sf37_hip_profile_enable": (C.c_int, [C.c_int]),
    "sf37_hip_profile_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(u64), u32]),
    "sf37_hip_profile_stage_name": (C.c_char_p, [u32]),
}

N_STAGES = 28


def profile_read() -> dict:
    """{stage: (total ms, launches)} since the last read (resets)."""
    ms = (C.c_double * N_STAGES)()
    cnt = (u64 * N_STAGES)()
    check(lib().sf37_hip_profile_read(ms, cnt, N_STAGES), "profile_read")
    return {lib().sf37_hip_profile_stage_name(i).decode(): (ms[i], cnt[i]) for i in range(N_STAGES)}

_LIB = None


def header_symbols(path: str = HEADER) -> list[str]:
    """Names of every function declared in include/sf37_hip.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf37_hip_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load libsf37_hip.so; raises if it is missing (no CPU fallback exists)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "or `make -C sf37_amd/csrc`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(ok: int, what: str) -> None:
    if not ok:
        raise RuntimeError(f"sf37_hip {what} failed")


class Tensor:
    """An sf37_hip_tensor handle owning device memory (or a view)."""

    def __init__(self, handle, nbytes: int, owned: bool = True):
        if not handle:
            raise RuntimeError("sf37_hip tensor allocation failed")
        self.h = handle
        self.nbytes = nbytes
        self.owned = owned

    @property
    def _as_parameter_(self):
        # ctypes passes the handle; the Tensor object stays referenced by the
        # call's argument tuple until the call returns (after the launch).
        return C.c_void_p(self.h)

    @classmethod
    def alloc(cls, nbytes: int) -> "Tensor":
        return cls(lib().sf37_hip_tensor_alloc(nbytes), nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "Tensor":
        a = np.ascontiguousarray(a)
        t = cls.alloc(a.nbytes)
        t.write(a)
        return t

    def write(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        check(lib().sf37_hip_tensor_write(self.h, offset, a.ctypes.data, a.nbytes), "tensor_write")

    def read(self, dtype, shape=None, offset: int = 0, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(count, dtype=dtype)
        check(lib().sf37_hip_tensor_read(self.h, offset, out.ctypes.data, out.nbytes), "tensor_read")
        return out.reshape(shape) if shape is not None else out

    def view(self, offset: int, nbytes: int) -> "Tensor":
        return Tensor(lib().sf37_hip_tensor_view(self.h, offset, nbytes), nbytes, owned=False)

    def device_ptr(self) -> int:
        return lib().sf37_hip_tensor_device_ptr(self.h)

    def free(self) -> None:
        if self.h:
            lib().sf37_hip_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def init() -> None:
    check(lib().sf37_hip_init(), "init")


def synchronize() -> None:
    check(lib().sf37_hip_synchronize(), "synchronize")


def set_option(name: str, value: int) -> None:
    check(lib().sf37_hip_set_option(name.encode(), value), f"set_option({name})")


def get_option(name: str) -> int:
    return lib().sf37_hip_get_option(name.encode())


def empty(shape, dtype) -> Tensor:
    return Tensor.alloc(int(np.prod(shape)) * np.dtype(dtype).itemsize)


def synth_quant(kind: str, rows: int, cols: int, seed: int, stream: int, row0: int = 0,
                sigma: float = 0.02, out: Tensor | None = None) -> Tensor:
    """Generate N(0, sigma) rows and quantize them on the device."""
    t = {"q8_0": 0, "q3": 3, "q2": 2}[kind]
    bs = {"q8_0": Q8_0_BLOCK, "q3": Q3_BLOCK, "q2": Q2_BLOCK}[kind]
    qk = 32 if t == 0 else QK_K
    nbytes = rows * (cols // qk) * bs
    if out is None:
        out = Tensor.alloc(nbytes)
    check(lib().sf37_hip_synth_quant_rows(t, out.h, row0, rows, cols, seed, stream, sigma), "synth_quant_rows")
    return out


def synth_normal(n: int, seed: int, stream: int, index0: int = 0, sigma: float = 1.0,
                 out: Tensor | None = None) -> Tensor:
    if out is None:
        out = Tensor.alloc(n * 4)
    check(lib().sf37_hip_synth_normal(out.h, n, seed, stream, index0, sigma), "synth_normal")
    return out
