"""Write the golden vectors in this directory from the reference's own C code.

Run in a container where /root/reference exists:
    make -C oracle ref && python tests/golden/make_golden.py
It loads oracle/_ref/libsf37ref.so (the reference's sf37_quant.c, sf37_ops.c
and gguf-tools/quants.c compiled in place by oracle/Makefile with IEEE flags)
and stores inputs and the reference's outputs, so the oracle stays pinned on
machines where the reference sources are absent.  Data only.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def P(a, t=C.c_float):
    return a.ctypes.data_as(C.POINTER(t))


def quant_inputs():
    r = np.random.default_rng(7)
    w = (r.standard_normal((24, 512)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0
    w[1, :64] = 0.0125
    w[2, :64] = -0.5
    w[3, :64] = r.standard_normal(64).astype(np.float32) * 1e-30
    w[4, :32] = 3.0
    w[5, 64:128] = np.linspace(-1, 1, 64, dtype=np.float32)
    w[6, :] = 0.0
    return w


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libsf37ref.so missing: run `make -C oracle ref`")
    w = quant_inputs()
    out = {"w": w}
    for kind, t in [("q8_0", 8), ("q3", 11), ("q2", 10)]:
        n = w.shape[0] * oracle.row_bytes(kind, w.shape[1])
        dst = np.zeros(n, np.uint8)
        ref.ds4q_quantize_chunk(t, P(w), dst.ctypes.data, 0, w.shape[0], w.shape[1], None)
        out[kind] = dst
    np.savez_compressed(os.path.join(HERE, "quantizer.npz"), **out)

    r = np.random.default_rng(2024)
    xs = np.concatenate([r.standard_normal(4000) * 8, np.linspace(-110, 90, 4000)]).astype(np.float32)
    sig = np.array([ref.sf37_sigmoid(float(v)) for v in xs], np.float32)
    x70 = (r.standard_normal(70) * 3).astype(np.float32)
    q70 = np.zeros(96, np.int8)
    s70 = np.zeros(3, np.float32)
    ref.sf37_q8_0_quantize_activation(P(x70), P(q70, C.c_int8), P(s70), 70)
    logits = (r.standard_normal((16, 288)) * 2).astype(np.float32)
    bias = (r.standard_normal(288) * 0.05).astype(np.float32)
    sel = np.zeros((16, 8), np.int32)
    for t in range(16):
        prob = np.array([ref.sf37_sigmoid(float(v)) for v in logits[t]], np.float32)
        score = prob + bias
        ref.sf37_topk_desc(P(score), 288, 8, P(sel[t], C.c_int32))
    blocks3 = r.integers(0, 256, (32, 110), dtype=np.uint8)
    blocks3[:, 0:8] = (r.random((32, 4)) * 0.9 + 0.1).astype(np.float16).view(np.uint8).reshape(32, 8)
    x256 = r.standard_normal((32, 256)).astype(np.float32)
    dot3 = np.array([ref.sf37_q3_asym_block_dot(P(np.ascontiguousarray(blocks3[i]), C.c_uint8),
                                                 P(np.ascontiguousarray(x256[i]))) for i in range(32)], np.float32)
    np.savez_compressed(os.path.join(HERE, "ops.npz"), sig_x=xs, sig_y=sig, x70=x70, q70=q70, s70=s70,
                        logits=logits, bias=bias, sel=sel, blocks3=blocks3, x256=x256, dot3=dot3)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
