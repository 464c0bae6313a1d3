"""Test vectors restated from the reference's own tests.

Row generators follow tests/test_sf37_cuda_ops.cu:87-111 (make_q3_row /
make_q2_row), whose scales are exact binary16 values; the block KAT patterns
follow tests/test_sf37_quant.c:78-147 and tests/test_sf37_ops.c:89-185.
"""
import numpy as np


def fm(i, c):
    """(float)i * c in binary32, as the C tests compute their inputs."""
    return np.float32(i) * np.float32(c)


def ctrunc_mod(a: int, m: int) -> int:
    """C99 '%' (truncating) for a possibly negative dividend."""
    return a - m * int(a / m)


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def put_q3(payload: np.ndarray, i: int, q: int) -> None:
    bit = 3 * i
    for k in range(3):
        if (q >> k) & 1:
            payload[(bit + k) >> 3] |= np.uint8(1 << ((bit + k) & 7))


def put_q2(payload: np.ndarray, i: int, q: int) -> None:
    payload[i >> 2] |= np.uint8((q & 3) << ((i & 3) * 2))


def q3_block(codes, scales, zps) -> np.ndarray:
    blk = np.zeros(110, dtype=np.uint8)
    for g in range(4):
        h = f16_bits(scales[g])
        blk[2 * g], blk[2 * g + 1] = h & 0xFF, h >> 8
        blk[8 + g] = zps[g]
        pl = blk[12 + 24 * g: 36 + 24 * g]
        for i in range(64):
            put_q3(pl, i, int(codes[64 * g + i]))
    return blk


def q2_block(codes, scales, zps) -> np.ndarray:
    blk = np.zeros(84, dtype=np.uint8)
    for g in range(4):
        h = f16_bits(scales[g])
        blk[2 * g], blk[2 * g + 1] = h & 0xFF, h >> 8
        blk[8 + g] = zps[g]
        pl = blk[12 + 16 * g: 28 + 16 * g]
        for i in range(64):
            put_q2(pl, i, int(codes[64 * g + i]))
    return blk


def make_q3_row(r: int, nblk: int = 1) -> np.ndarray:
    """tests/test_sf37_cuda_ops.cu:87-98 (one 256-block per call there)."""
    blocks = []
    for _ in range(nblk):
        codes = [(i + r + g) & 7 for g in range(4) for i in range(64)]
        scales = [0.015625 * (g + 1 + r) for g in range(4)]
        zps = [2 + ((r + g) & 3) for g in range(4)]
        blocks.append(q3_block(codes, scales, zps))
    return np.concatenate(blocks)


def make_q2_row(r: int, nblk: int = 1) -> np.ndarray:
    """tests/test_sf37_cuda_ops.cu:100-111."""
    blocks = []
    for _ in range(nblk):
        codes = [(i + r + g) & 3 for g in range(4) for i in range(64)]
        scales = [0.03125 * (g + 1 + r) for g in range(4)]
        zps = [1 + ((r + g) & 1) for g in range(4)]
        blocks.append(q2_block(codes, scales, zps))
    return np.concatenate(blocks)


def router_moe_case():
    """Shapes and inputs of test_router_moe, tests/test_sf37_cuda_ops.cu:698-748."""
    n_expert, topk, in_dim, mid_dim, out_dim = 4, 2, 256, 256, 6
    x = np.array([fm((i % 37) - 18, 0.015) for i in range(in_dim)], dtype=np.float32)
    logits = np.array([fm(e - 1, 0.375) for e in range(n_expert)], dtype=np.float32)
    bias = np.array([fm((e * 7) % 5 - 2, 0.025) for e in range(n_expert)], dtype=np.float32)
    gate = np.concatenate([make_q3_row(e * 13 + r) for e in range(n_expert) for r in range(mid_dim)])
    up = np.concatenate([make_q3_row(e * 17 + r + 3) for e in range(n_expert) for r in range(mid_dim)])
    down = np.concatenate([make_q2_row(e * 19 + r) for e in range(n_expert) for r in range(out_dim)])
    return dict(n_expert=n_expert, topk=topk, in_dim=in_dim, mid_dim=mid_dim, out_dim=out_dim,
                x=x, logits=logits, bias=bias, gate=gate, up=up, down=down)


def batch_moe_case():
    """Shapes and inputs of the batch routed-MoE test,
    tests/test_sf37_cuda_ops.cu:1214-1267 (an invalid id -1 clamps to 0)."""
    n_tok, n_expert, topk, in_dim, mid_dim, out_dim = 3, 4, 2, 256, 256, 6
    x = np.array([[fm(ctrunc_mod((t + 2) * (i % 41) - 33, 47), 0.011) for i in range(in_dim)]
                  for t in range(n_tok)], dtype=np.float32)
    selected = np.array([[3, 1], [2, -1], [1, 3]], dtype=np.int32)
    weights = np.array([[1.1, 0.7], [0.9, 1.3], [1.4, 0.6]], dtype=np.float32)
    gate = np.concatenate([make_q3_row(e * 23 + r + 1) for e in range(n_expert) for r in range(mid_dim)])
    up = np.concatenate([make_q3_row(e * 29 + r + 5) for e in range(n_expert) for r in range(mid_dim)])
    down = np.concatenate([make_q2_row(e * 31 + r + 7) for e in range(n_expert) for r in range(out_dim)])
    return dict(n_tok=n_tok, n_expert=n_expert, topk=topk, in_dim=in_dim, mid_dim=mid_dim,
                out_dim=out_dim, x=x, selected=selected, weights=weights, gate=gate, up=up,
                down=down)


def router_top8_case():
    """test_router_warp_top8, tests/test_sf37_cuda_ops.cu:620-640 (forced tie 40/41)."""
    n = 288
    logits = np.array([np.float32(-4.0) + fm((e * 17) % 53, 0.013) for e in range(n)], dtype=np.float32)
    bias = np.array([fm((e * 11) % 19 - 9, 0.002) for e in range(n)], dtype=np.float32)
    forced = [40, 41, 7, 280, 13, 120, 121, 200]
    for i, e in enumerate(forced):
        logits[e] = np.float32(4.0) - fm(i // 2, 0.25)
        bias[e] = np.float32(0.75) if i < 2 else np.float32(0.5) - fm(i, 0.01)
    logits[40] = logits[41]
    bias[40] = bias[41]
    return logits, bias


def router_batch_case():
    """Batch router test, tests/test_sf37_cuda_ops.cu:1151-1166."""
    n_tok, n = 3, 288
    bias = np.array([fm((e * 13) % 23 - 11, 0.003) for e in range(n)], dtype=np.float32)
    logits = np.zeros((n_tok, n), dtype=np.float32)
    for t in range(n_tok):
        for e in range(n):
            v = (t + 1) * e * 7
            logits[t, e] = fm((v % 61) - 30, 0.021)
        logits[t, 40] = 5.0
        logits[t, 41] = 5.0
    bias[40] = 0.5
    bias[41] = 0.5
    return logits, bias
