"""Host-side pieces that need no GPU: the bench contract's one-GPU rule and
the bf16 rounding used for the stack's norm weights."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_bf16_bits_round_to_nearest_even():
    """moe.bf16_bits against torch's float32 -> bfloat16 conversion (round to
    nearest even) on random values and on exact ties."""
    import torch
    from sf37_amd.moe import bf16_bits
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 0.02,
                        rng.standard_normal(4096).astype(np.float32) * 1e4])
    ties = (np.arange(1, 4097, dtype=np.uint32) << 16) | 0x8000     # halfway between two bf16 values
    x = np.concatenate([x, ties.view(np.float32), -ties.view(np.float32), np.float32([0.0, -0.0, 1.0, -2.5])])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_bits(x), want)
