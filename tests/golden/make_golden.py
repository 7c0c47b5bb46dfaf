"""Writes the small golden fixtures under tests/golden/ from the float64
oracle (the reference ships no numeric vectors: its tests compare against
mha_reference by tolerance only).  Run from the repo root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention, masks  # noqa: E402


def causal_fp32_b1h1s48d16():
    rng = np.random.default_rng(0)
    q, k, v, do = (rng.standard_normal((1, 1, 48, 16)).astype(np.float32) for _ in range(4))
    m = masks.dense(masks.causal, 48, 48)
    o, lse = attention.forward(q, k, v, mask=m)
    dq, dk, dv = attention.backward(q, k, v, do, mask=m)
    np.savez_compressed(os.path.join(HERE, "causal_fp32_b1h1s48d16.npz"), q=q, k=k, v=v, do=do,
                        o=o.astype(np.float32), lse=lse.astype(np.float32), dq=dq.astype(np.float32),
                        dk=dk.astype(np.float32), dv=dv.astype(np.float32))


if __name__ == "__main__":
    causal_fp32_b1h1s48d16()
