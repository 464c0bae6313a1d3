"""BASELINE configs[4] at its workload: 45 independently seeded BASELINE-shape
layers (81.65 GB of Q3GU/Q2D/Q8_0/F32 weights resident), h <- h +
MoE_l(RMSNorm_l(h)) through sf37_hip_moe_stack with Zipf-skewed injected
logits per layer, as bench.py runs it: a one-token decode and one 2048-token
prefill chunk.  Every token's path through the stack is independent of the
others (RMSNorm and the MoE FFN act per token), so the CPU oracle, run layer
by layer through all 45 layers, checks a sample of tokens bit for bit.
"""
import sys

import numpy as np
import pytest

from test_gpu_stack import assert_bitexact, oracle_stack

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


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
def stack(H):
    from sf37_amd import moe
    say("generating the 45-layer BASELINE-shape stack")
    S = moe.SynthStack(master=moe.layer_seed(1234, 4000), n_layers=45)
    H.synchronize()
    yield S
    S.free()


@pytest.mark.parametrize("n_tok,sample", [(1, [0]), (2048, [0, 777, 1500, 2047])])
def test_stack45_vs_oracle(H, O, stack, n_tok, sample):
    from sf37_amd import configs, moe
    S = stack
    x = configs.x_device(4, 4000 + n_tok, n_tok).read(np.float32).reshape(n_tok, S.in_dim)
    logits = [configs.logits_for(4, moe.layer_seed(4000 + n_tok, l), n_tok) for l in range(S.n_layers)]
    say(f"stack: {n_tok} tokens through 45 layers on the device")
    h = H.Tensor.from_array(x)
    lts = [H.Tensor.from_array(lg) for lg in logits]
    S.forward(h, n_tok, None, None, None, None, lts, native=True)
    got = h.read(np.float32).reshape(n_tok, S.in_dim)
    for t in lts:
        t.free()
    say(f"oracle: tokens {sample} through 45 layers")
    idx = np.array(sample)
    want = oracle_stack(O, S, x[idx], [lg[idx] for lg in logits])
    assert_bitexact(got[idx], want, f"45-layer stack, {n_tok} tokens, sampled rows {sample}")
