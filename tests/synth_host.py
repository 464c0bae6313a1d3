"""Host copies of synthetic MoE layer weights (test infrastructure).

The device generator (sf37_amd.moe.SynthLayer, k_synth.hip) and the oracle's
orc_gen_quant_rows / orc_fill_normal draw the same counter-based streams, so
the rows made here equal the device layer's rows bit for bit.  Only the
experts a test needs are generated, into arrays with the full expert stride
(numpy's zero pages cost nothing until written), several experts at a time
on worker threads (the generator is C called through ctypes, which releases
the interpreter lock).
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

# streams of sf37_amd/moe.py STREAM
STREAM = {"router": 1, "gate": 2, "up": 3, "down": 4, "sh_gate": 5, "sh_up": 6, "sh_down": 7, "norm": 8}
X_STREAM = 100     # sf37_amd/configs.py X_STREAM


def workers() -> int:
    return max(1, min(8, os.cpu_count() or 1))


def host_layer(O, seed: int, n_expert: int = 288, in_dim: int = 4096, mid_dim: int = 1280,
               sigma: float = 0.02) -> dict:
    """Weights dict for oracle.moe_layer_q8k: router, zero bias, the Q8_0
    shared expert and expert arrays of full stride, no expert filled yet."""
    E, D, F = n_expert, in_dim, mid_dim
    g_row, d_row = D // 256 * 110, F // 256 * 84
    return {"gate": np.zeros(E * F * g_row, np.uint8), "up": np.zeros(E * F * g_row, np.uint8),
            "down": np.zeros(E * D * d_row, np.uint8), "n_expert": E, "in_dim": D, "mid_dim": F,
            "seed": seed, "sigma": sigma, "filled": set(),
            "router": O.fill_normal(E * D, seed, STREAM["router"], sigma=sigma),
            "router_bias": np.zeros(E, np.float32),
            "sh_gate": O.gen_quant("q8_0", F, D, seed, STREAM["sh_gate"], sigma=sigma),
            "sh_up": O.gen_quant("q8_0", F, D, seed, STREAM["sh_up"], sigma=sigma),
            "sh_down": O.gen_quant("q8_0", D, F, seed, STREAM["sh_down"], sigma=sigma)}


def fill_experts(O, w: dict, experts) -> None:
    """Generate the rows of the given experts (ids outside [0, n_expert) act
    as expert 0) that w does not hold yet."""
    E, D, F, seed, sigma = w["n_expert"], w["in_dim"], w["mid_dim"], w["seed"], w["sigma"]
    gb, db = F * (D // 256 * 110), D * (F // 256 * 84)
    ids = sorted({int(e) if 0 <= int(e) < E else 0 for e in np.ravel(experts)} - w["filled"])

    def one(e):
        w["gate"][e * gb:(e + 1) * gb] = O.gen_quant("q3", F, D, seed, STREAM["gate"], row0=e * F, sigma=sigma)
        w["up"][e * gb:(e + 1) * gb] = O.gen_quant("q3", F, D, seed, STREAM["up"], row0=e * F, sigma=sigma)
        w["down"][e * db:(e + 1) * db] = O.gen_quant("q2", D, F, seed, STREAM["down"], row0=e * D, sigma=sigma)

    with ThreadPoolExecutor(workers()) as ex:
        list(ex.map(one, ids))
    w["filled"].update(ids)


def router_logits(O, w: dict, x: np.ndarray) -> np.ndarray:
    """Router logits of rows x with the double-accumulated F32 router
    (sf37.c:1970-1976), as the oracle layer computes them."""
    import ctypes as C
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    E = w["n_expert"]
    out = np.zeros((x.shape[0], E), np.float32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    for t in range(x.shape[0]):
        row = np.zeros(E, np.float32)
        O.lib().orc_f32_matvec_double(fp(row), fp(w["router"]), x.shape[1], E, fp(np.ascontiguousarray(x[t])))
        out[t] = row
    return out
