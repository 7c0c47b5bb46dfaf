"""Packed variable-length sequences (flex_attention_varlen, the
FlashAttention cu_seqlens convention) on the GPU: forward and backward
against the float64 oracle with the mask written out sequence by sequence
(bf16 atol = rtol = 2e-2, fp32 1e-5)."""
import zlib

import numpy as np
import pytest

from _cases import BF16_TOL, FP32_TOL, assert_close, inputs, oracle_fwd_bwd, to_np, to_torch

pytestmark = pytest.mark.gpu


def _oracle_mask(cu_q, cu_k, causal):
    tq, tk = cu_q[-1], cu_k[-1]
    m = np.zeros((tq, tk), bool)
    for s in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        for i in range(q0, q1):
            if causal:  # bottom-right aligned: the last query sees every key
                last = k1 - 1 - (q1 - 1 - i)
                m[i, k0:max(k0, last + 1)] = True
            else:
                m[i, k0:k1] = True
    return m[None, None]


CASES = [
    # name, dtype, Hq, Hkv, D, cu_q, cu_k, causal
    ("same-packing-causal-bf16", "bf16", 4, 2, 128, [0, 100, 420, 431, 700], None, True),
    ("same-packing-fp32", "fp32", 2, 2, 64, [0, 64, 65, 300], None, False),
    ("chunked-prefill-causal-bf16", "bf16", 4, 4, 128, [0, 30, 200, 264], [0, 150, 500, 700], True),
    ("cross-lengths-bf16", "bf16", 2, 1, 64, [0, 17, 140], [0, 300, 333], False),
    ("chunked-prefill-causal-fp32", "fp32", 2, 2, 32, [0, 20, 90], [0, 70, 260], True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_varlen_fwd_bwd(case):
    import torch
    import pallas_flexattn as pf
    name, dtype, Hq, Hkv, D, cu_q, cu_k, causal = case
    cu_k = cu_q if cu_k is None else cu_k
    print(f"[gpu varlen] {name}", flush=True)
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, 1, Hq, Hkv, cu_q[-1], cu_k[-1], D, dtype)
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention_varlen(tq, tk, tv, cu_q, cu_k, causal=causal, enable_gqa=Hq != Hkv, return_lse=True)
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    om = _oracle_mask(np.array(cu_q), np.array(cu_k), causal)
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    got_lse = to_np(lse)
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(wl))
    fin = np.isfinite(wl)
    assert_close(f"{name} LSE", got_lse[fin], wl[fin], tol)
    for nm, got, want in (("O", o, wo), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk), ("dV", tv.grad, wdv)):
        assert_close(f"{name} {nm}", to_np(got), want, tol)
