"""Synthetic SF37 MoE layers resident in HBM, and thin wrappers over the
C ABI entry points that run them.

A layer is generated on the device from one seed: router
W_r ~ N(0, 0.02) fp32, router bias 0, 288 experts whose fp32 gate/up
[1280 x 4096] and down [4096 x 1280] rows ~ N(0, 0.02) are quantized to
Q3GU / Q2D by the reference quantizer, and a Q8_0 shared expert, all from
counter-based streams so any part can be regenerated bit-identically.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip
from .hip import Tensor, check, lib

EMBD = 4096          # sf37.c:36
EXPERTS = 288        # sf37.c:44
EXPERT_USED = 8      # sf37.c:45
EXPERT_FF = 1280     # sf37.c:46

STREAM = {"router": 1, "gate": 2, "up": 3, "down": 4, "sh_gate": 5, "sh_up": 6, "sh_down": 7, "norm": 8}


def layer_seed(master: int, layer: int) -> int:
    return master * 1000003 + layer


def swiglu_limit(il: int, shared: bool) -> float:
    """Per-layer SwiGLU clamp, sf37.c:2103-2106."""
    if il in (43, 44):
        return 16.0 if shared else 7.0
    return 0.0


class SynthLayer:
    """One MoE layer's weights on the device."""

    def __init__(self, seed: int, n_expert: int = EXPERTS, in_dim: int = EMBD, mid_dim: int = EXPERT_FF,
                 topk: int = EXPERT_USED, il: int = 3, sigma: float = 0.02, shared: str = "q8_0"):
        """shared: "q8_0" (the engine's shared expert) or "q3q2" (Q3GU gate/up
        and Q2D down, the BASELINE configurations' "same formats" option)."""
        self.seed, self.n_expert, self.in_dim, self.mid_dim, self.topk, self.il = \
            seed, n_expert, in_dim, mid_dim, topk, il
        self.shared = shared
        E, D, F = n_expert, in_dim, mid_dim
        self.g_row = D // 256 * hip.Q3_BLOCK
        self.d_row = F // 256 * hip.Q2_BLOCK
        self.router = hip.synth_normal(E * D, seed, STREAM["router"], sigma=sigma)
        self.router_bias = Tensor.from_array(np.zeros(E, np.float32))
        self.gate = hip.synth_quant("q3", E * F, D, seed, STREAM["gate"], sigma=sigma)
        self.up = hip.synth_quant("q3", E * F, D, seed, STREAM["up"], sigma=sigma)
        self.down = hip.synth_quant("q2", E * D, F, seed, STREAM["down"], sigma=sigma)
        gu, dn = ("q3", "q2") if shared == "q3q2" else ("q8_0", "q8_0")
        self.sh_gate = hip.synth_quant(gu, F, D, seed, STREAM["sh_gate"], sigma=sigma)
        self.sh_up = hip.synth_quant(gu, F, D, seed, STREAM["sh_up"], sigma=sigma)
        self.sh_down = hip.synth_quant(dn, D, F, seed, STREAM["sh_down"], sigma=sigma)
        self.clamp_routed = swiglu_limit(il, False)
        self.clamp_shared = swiglu_limit(il, True)

    # bytes moved by one pass over the routed experts in `experts`
    def expert_bytes(self) -> int:
        return self.mid_dim * self.g_row * 2 + self.in_dim * self.d_row

    def shared_bytes(self) -> int:
        return self.sh_gate.nbytes + self.sh_up.nbytes + self.sh_down.nbytes

    def router_bytes(self) -> int:
        return self.router.nbytes

    def weights_struct(self, scale: float = 3.0) -> hip.LayerWeights:
        return hip.LayerWeights(self.router.h, self.router_bias.h, self.gate.h, self.up.h, self.down.h,
                                self.sh_gate.h, self.sh_up.h, self.sh_down.h, self.n_expert, self.topk,
                                self.in_dim, self.mid_dim, scale, self.clamp_routed, self.clamp_shared,
                                hip.TYPE_F32, hip.TYPE_Q3GU if self.shared == "q3q2" else 0)

    def host_experts(self, experts) -> dict:
        """Host copies of the given experts' packed rows (for the CPU oracle),
        in an array with the full expert stride but only those experts filled."""
        E, F, D = self.n_expert, self.mid_dim, self.in_dim
        gate = np.zeros(E * F * self.g_row, np.uint8)
        up = np.zeros_like(gate)
        down = np.zeros(E * D * self.d_row, np.uint8)
        gb, db = F * self.g_row, D * self.d_row
        ids = {int(v) for v in np.ravel(experts)}
        for e in sorted({v if 0 <= v < E else 0 for v in ids}):      # invalid ids act as expert 0
            gate[e * gb:(e + 1) * gb] = self.gate.read(np.uint8, offset=e * gb, count=gb)
            up[e * gb:(e + 1) * gb] = self.up.read(np.uint8, offset=e * gb, count=gb)
            down[e * db:(e + 1) * db] = self.down.read(np.uint8, offset=e * db, count=db)
        return {"gate": gate, "up": up, "down": down}

    def host_dense(self) -> dict:
        return {"router": self.router.read(np.float32), "router_bias": self.router_bias.read(np.float32),
                "sh_gate": self.sh_gate.read(np.uint8), "sh_up": self.sh_up.read(np.uint8),
                "sh_down": self.sh_down.read(np.uint8)}

    def free(self) -> None:
        for t in (self.router, self.router_bias, self.gate, self.up, self.down, self.sh_gate, self.sh_up,
                  self.sh_down):
            t.free()


def moe_layer(layer: SynthLayer, x: Tensor, n_tok: int, out: Tensor, selected: Tensor | None = None,
              weights: Tensor | None = None, logits: Tensor | None = None, scale: float = 3.0) -> None:
    """out = shared(x) + routed(x) for n_tok tokens (sf37_hip_moe_layer)."""
    w = layer.weights_struct(scale)
    check(lib().sf37_hip_moe_layer(out.h, selected.h if selected else None, weights.h if weights else None,
                                   w, logits.h if logits else None, x.h, n_tok), "moe_layer")


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class SynthStack:
    """n_layers independently seeded layers (layer il
    has seed layer_seed(master, il) and the SwiGLU clamps of layer il), each
    preceded by RMSNorm with (w + 1) weights, bf16 w ~ N(0, 0.02), as the
    engine's h <- h + MoE_l(RMSNorm_l(h)) (sf37.c:2243-2250).  The norm
    weights of all layers sit in one device range registered under a model-map
    key, read by the batched bf16 RMSNorm entry point."""

    EPS = 1e-5       # sf37.c:61

    def __init__(self, master: int, n_layers: int = 45, il0: int = 0, **layer_kw):
        self.layers = [SynthLayer(seed=layer_seed(master, il0 + l), il=il0 + l, **layer_kw)
                       for l in range(n_layers)]
        K = self.layers[0].in_dim
        self.in_dim, self.n_layers = K, n_layers
        w = np.stack([hip.synth_normal(K, layer_seed(master, il0 + l), STREAM["norm"], sigma=0.02).read(np.float32)
                      for l in range(n_layers)])
        self.norm_bits = bf16_bits(w)                    # [n_layers][K] bf16
        self.norm = Tensor.from_array(self.norm_bits)
        self._key = np.zeros(64, np.uint8)               # host address used as the map key
        check(lib().sf37_hip_register_device_range(self._key.ctypes.data, self.norm.nbytes, 0, self.norm.nbytes,
                                                   self.norm.h), "register norm weights")
        self._structs = (hip.LayerWeights * n_layers)(*[lay.weights_struct() for lay in self.layers])
        self._offsets = (C.c_uint64 * n_layers)(*[l * K * 2 for l in range(n_layers)])

    def rms_norm(self, out: Tensor, x: Tensor, layer: int, n_tok: int) -> None:
        K = self.in_dim
        check(lib().sf37_hip_rms_norm_weight1_bf16_batch_mapped(out.h, x.h, self._key.ctypes.data, self.norm.nbytes,
                                                                layer * K * 2, K, n_tok, self.EPS), "rms_norm")

    def forward(self, h: Tensor, n_tok: int, xn: Tensor | None = None, y: Tensor | None = None, sel=None,
                wts: Tensor | None = None, logits=None, native: bool = True) -> None:
        """h <- h + MoE_l(RMSNorm_l(h)) for every layer; logits[l] (optional)
        are injected router logits of layer l; sel is one selection buffer or
        a list of one per layer.  native: one sf37_hip_moe_stack call (the
        decode launches normalise and add the residual themselves); else per
        layer the rms_norm, moe_layer and add entry points (xn, y needed)."""
        n = self.n_layers
        sels = list(sel) if isinstance(sel, (list, tuple)) else [sel] * n
        if native:
            Ta = C.c_void_p * n
            lg = Ta(*[t.h if t is not None else None for t in logits]) if logits is not None else None
            sl = Ta(*[t.h if t is not None else None for t in sels])
            check(lib().sf37_hip_moe_stack(h.h, n, self._structs, self._key.ctypes.data, self.norm.nbytes,
                                           self._offsets, self.EPS, lg, sl, n_tok), "moe_stack")
            return
        for l, lay in enumerate(self.layers):
            self.rms_norm(xn, h, l, n_tok)
            moe_layer(lay, xn, n_tok, y, sels[l], wts, logits[l] if logits is not None else None)
            check(lib().sf37_hip_add_inplace_f32(h.h, y.h, n_tok * self.in_dim), "add_inplace")

    def free(self) -> None:
        for lay in self.layers:
            lay.free()
        self.norm.free()
