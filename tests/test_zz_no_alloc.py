"""sf37_hip_moe_layer_noalloc (the decode layer with its scratch in the
library's static device array) against sf37_hip_moe_layer, through the C
ABI, bit for bit: two calls in a row at the BASELINE shape, the second with
a smaller batch (8 tokens with injected logits, then 3 tokens routed by the
layer's own router), then one token, then 16 tokens (the largest scratch
layout); around every no-alloc call the library's count of device-memory
requests stays unchanged (no scratch, counter or buffer is asked for, not even
one that already exists); batches it does not take are refused with a
message."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E, K = 288, 4096


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def H():
    from sf37_amd import hip
    hip.init()
    yield hip
    hip.synchronize()


def assert_bitexact(got, want, what):
    g = np.ravel(np.ascontiguousarray(got).view(np.uint32))
    w = np.ravel(np.ascontiguousarray(want).view(np.uint32))
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ"


def run(H, fn, lay, x, n_tok, logits):
    """One call of fn with its outputs allocated beforehand; also returns how
    many device-memory requests the library served during the call."""
    L = H.lib()
    out, sel, wts = H.Tensor.alloc(n_tok * K * 4), H.Tensor.alloc(n_tok * 32), H.Tensor.alloc(n_tok * 32)
    w = lay.weights_struct()
    H.synchronize()
    before = L.sf37_hip_device_memory_requests()
    ok = fn(out, sel, wts, C.byref(w), logits, x, n_tok)
    H.synchronize()
    reqs = L.sf37_hip_device_memory_requests() - before
    return ok, out.read(np.float32), sel.read(np.int32), wts.read(np.float32), reqs


def test_noalloc_layer_equals_moe_layer(H):
    from sf37_amd import configs
    from sf37_amd.moe import SynthLayer
    L = H.lib()
    say("no-alloc decode layer: BASELINE-shape layer")
    lay = SynthLayer(seed=2024)
    try:
        for n_tok, config in ((8, 1), (3, 0), (1, 0), (16, 1)):
            say(f"no-alloc: {n_tok} tokens, config {config}")
            x = configs.x_device(config, 31 + n_tok, n_tok)
            lg_host = configs.logits_for(config, 31 + n_tok, n_tok)
            lg = H.Tensor.from_array(lg_host) if lg_host is not None else None
            ok_a, out_a, sel_a, w_a, reqs_a = run(H, L.sf37_hip_moe_layer_noalloc, lay, x, n_tok, lg)
            ok_b, out_b, sel_b, w_b, reqs_b = run(H, L.sf37_hip_moe_layer, lay, x, n_tok, lg)
            assert ok_a == 1 and ok_b == 1
            assert reqs_a == 0, f"no-alloc call asked for device memory {reqs_a} times"
            assert reqs_b > 0          # the counter does see the allocating entry point
            assert np.array_equal(sel_a, sel_b)
            assert_bitexact(w_a, w_b, f"routing weights, {n_tok} tokens")
            assert_bitexact(out_a, out_b, f"layer output, {n_tok} tokens")
        # batches outside the fused decode path are refused, nothing launched
        x = configs.x_device(2, 5, 17)
        out = H.Tensor.alloc(17 * K * 4)
        assert L.sf37_hip_moe_layer_noalloc(out, None, None, C.byref(lay.weights_struct()), None, x, 17) == 0
        H.synchronize()
    finally:
        lay.free()
