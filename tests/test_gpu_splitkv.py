"""Split-KV forward (C ABI fa_fwd_splitkv, pallas_flexattn.flex_decode) on the GPU.

The split kernels and their log-sum-exp merge must give the forward's
results: O and LSE within the bf16 tolerance of the oracle's float64
attention (atol = rtol = 2e-2, LSE to 1e-3), and close to the unsplit kernel
(the merge re-associates the softmax sum).  Decode shapes (one or a few
queries against thousands of keys), GQA, windows, document masks, score mods,
ragged lengths and explicit split counts, including splits left without a
tile by the mask."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, Sq, Skv, D, seed):
    import torch
    g = np.random.default_rng(seed)
    mk = lambda *s: torch.from_numpy(g.standard_normal(s, dtype=np.float32)).to("cuda", torch.bfloat16)
    return mk(B, Hq, Sq, D), mk(B, Hkv, Skv, D), mk(B, Hkv, Skv, D)


def _oracle(q, k, v, mask=None, slopes=None, cap=None):
    from oracle import attention
    to = lambda t: t.float().cpu().numpy()
    o, lse = attention.forward(to(q), to(k), to(v), mask=mask, alibi_slopes=slopes, softcap=cap)
    return o, lse


CASES = [
    # name, B, Hq, Hkv, Sq, Skv, D, mask, score, splits
    ("decode-1q", 2, 8, 8, 1, 4096, 128, None, None, None),
    ("decode-gqa", 2, 8, 2, 4, 3000, 128, None, None, None),
    ("decode-window", 1, 4, 4, 16, 5000, 128, "window", None, 7),
    ("short-q-alibi-cap", 1, 4, 4, 64, 2048, 64, None, "mods", 5),
    ("docs", 2, 2, 2, 300, 1200, 128, "docs", None, 3),
    ("splits-capped-by-keys", 1, 2, 2, 8, 200, 128, None, None, 64),
    ("causal-square", 1, 2, 2, 640, 640, 128, "causal", None, 4),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_split_kv_matches_oracle_and_forward(case):
    import torch
    import pallas_flexattn as pf
    name, B, Hq, Hkv, Sq, Skv, D, mname, sname, splits = case
    q, k, v = _case(B, Hq, Hkv, Sq, Skv, D, 7)
    mm, bm, omask = None, None, None
    if mname == "window":
        mm = pf.sliding_window_mask(700, 300)
    elif mname == "docs":
        mm = pf.document_mask([[200, 500, 500], [600, 600]])
    elif mname == "causal":
        mm = pf.causal_mask
    if mm is not None:
        bm = pf.create_block_mask(mm, B, Hq, Sq, Skv, 128)
        omask = mm
    score = slopes = cap = None
    if sname == "mods":
        score = pf.compose_score_mods(pf.alibi_score_mod(Hq), pf.softcap_score_mod(30.0))
        slopes, cap = pf.alibi_slopes(Hq), 30.0
    o, lse = pf.flex_decode(q, k, v, score_mod=score, block_mask=bm, enable_gqa=Hq != Hkv, num_splits=splits,
                            return_lse=True)
    o1, lse1 = pf.flex_attention(q, k, v, score_mod=score, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    torch.cuda.synchronize()
    # against the unsplit forward: the same attention up to bf16 rounding of O
    np.testing.assert_allclose(o.float().cpu().numpy(), o1.float().cpu().numpy(), atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), lse1.cpu().numpy(), atol=1e-4, rtol=1e-5)
    # against the oracle (mask descriptors take (b, h, q, kv) too)
    ro, rlse = _oracle(q, k, v, mask=omask, slopes=slopes, cap=cap)
    np.testing.assert_allclose(o.float().cpu().numpy(), ro, atol=2e-2, rtol=2e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), rlse, atol=1e-3, rtol=1e-3)


def test_split_kv_workspace_and_counts():
    import ctypes
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn import _lib
    from pallas_flexattn.flash_attn import _Plan
    q, k, v = _case(1, 4, 4, 1, 8192, 128, 3)
    plan = _Plan(q, k, None, None, None, None, (128, 64))
    lib = _lib.load()
    rows = 1 * 4 * 1
    assert lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), 8) == 8 * rows * (128 + 2) * 4
    assert lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), 1) == 0
    auto = lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), 0)
    assert auto > 0 and auto % (rows * (128 + 2) * 4) == 0
    assert lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), 65) == 0
    # too small a workspace is rejected before any launch
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device="cuda", dtype=torch.float32)
    ws = torch.empty(1024, device="cuda", dtype=torch.uint8)
    rc = lib.fa_fwd_splitkv(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), 8,
                            ws.data_ptr(), 1024, None)
    assert rc == -6
