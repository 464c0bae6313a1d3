"""Inputs of the BASELINE.json configurations (all drawn from one seed).

  0  decode, 1 token; logits = router . x
  1  decode, 8 tokens; router logits injected i.i.d. N(0,1) (uniform routing)
  2  prefill, 512 tokens; logits N(0,1) + per-expert Zipf(s=1.1) bias
  3  prefill, 4096 tokens; uniform logits
  4  45-layer stack; decode 1 token and a 2048-token Zipf prefill

x ~ N(0,1) is generated on the device by the counter-based generator
(bit-identical everywhere); injected logits come from numpy's PCG64 with
the same seed.  Zipf bias: expert e gets ln(p(rank_e) / p(1)) with
p(k) ~ k^-1.1 and ranks a seeded permutation, so the most popular expert's
bias is 0 and the least popular's is -1.1 ln 288 = -6.23.
"""
from __future__ import annotations

import numpy as np

from . import hip
from .moe import EMBD, EXPERTS

X_STREAM = 100
CONFIG_TOKENS = {0: 1, 1: 8, 2: 512, 3: 4096}


def zipf_bias(seed: int, n_expert: int = EXPERTS, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng([seed, 17])
    ranks = rng.permutation(n_expert) + 1
    return (-s * np.log(ranks.astype(np.float64))).astype(np.float32)


def logits_for(config: int, seed: int, n_tok: int, n_expert: int = EXPERTS):
    """Injected router logits of a config (None when computed from x)."""
    if config == 0:
        return None
    rng = np.random.default_rng([seed, config])
    lg = rng.standard_normal((n_tok, n_expert)).astype(np.float32)
    if config in (2, 4):
        lg = (lg + zipf_bias(seed, n_expert)[None, :]).astype(np.float32)
    return lg


def x_device(config: int, seed: int, n_tok: int, in_dim: int = EMBD) -> hip.Tensor:
    return hip.synth_normal(n_tok * in_dim, seed, X_STREAM + config)
