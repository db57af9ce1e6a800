"""Writes the dequant fixtures, computed by the reference's own dequant code
compiled from /root/reference/q36_dequant.cuh into oracle/_ref/ by
oracle/Makefile:
  tests/golden/mxfp4_dequant_ref.npz   MXFP4 blocks, q36_deq_mxfp4 values and
                                       q36_e8m0_half for every exponent byte;
  tests/golden/kquant_dequant_ref.npz  Q8_0 / Q5_K / Q6_K blocks (the formats
                                       of the release file's shared expert and
                                       fallback experts) and q36_deq_row values.

    make -C oracle && python tests/golden/make_golden.py

The fixture is data only (inputs and the reference's outputs)."""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import pyoracle  # noqa: E402


def main():
    ref = pyoracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_dequant.so missing: run `make -C oracle` with the reference tree present")
    rng = np.random.default_rng(20261201)
    n = 1024
    blocks = np.frombuffer(rng.bytes(n * 17), dtype=np.uint8).reshape(n, 17).copy()
    # exponent bytes over the whole finite E8M0 range, the benchmark range
    # [119, 127] and the denormal-handling edge e < 2 of q36_e8m0_half
    blocks[:, 0] = rng.integers(0, 255, size=n).astype(np.uint8)
    blocks[:64, 0] = np.arange(64) % 3            # 0, 1, 2
    blocks[64:256, 0] = 119 + rng.integers(0, 9, size=192)
    vals = np.empty((n, 32), dtype=np.float32)
    for i in range(n):
        ref.ref_deq_mxfp4(ctypes.c_void_p(blocks[i].ctypes.data),
                          ctypes.c_void_p(vals[i].ctypes.data))
    e8m0_half = np.array([ref.ref_e8m0_half(e) for e in range(256)], dtype=np.float32)
    np.savez_compressed(os.path.join(HERE, "mxfp4_dequant_ref.npz"), blocks=blocks, values=vals,
                        e8m0_half=e8m0_half)
    print("wrote", n, "blocks")
    # k-quants: random codes with finite f16 scales of several magnitudes
    # (including subnormal and negative d / dmin), 32 blocks per type
    out = {}
    for name, t, size, elems, f16_at in (("q8_0", 8, 34, 32, (0,)), ("q5_k", 13, 176, 256, (0, 2)),
                                         ("q6_k", 14, 210, 256, (208,))):
        nb = 32
        b = np.frombuffer(rng.bytes(nb * size), dtype=np.uint8).reshape(nb, size).copy()
        mags = np.array([3e-3, -1e-3, 6e-5, 2e-7, 0.25, 1.0, -0.5, 0.0], dtype=np.float16)
        for o in f16_at:
            b[:, o:o + 2] = np.frombuffer(np.resize(mags, nb).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
        v = np.empty(nb * elems, dtype=np.float32)
        ref.ref_deq_row(t, ctypes.c_void_p(b.ctypes.data), nb * elems, ctypes.c_void_p(v.ctypes.data))
        out[name + "_blocks"] = b
        out[name + "_values"] = v.reshape(nb, elems)
    np.savez_compressed(os.path.join(HERE, "kquant_dequant_ref.npz"), **out)
    print("wrote k-quant fixtures")


if __name__ == "__main__":
    main()
