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
    plan = _Plan(q, k, None, None, None, None, (128, 64, 128))
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


PACK_CASES = [
    # name, B, Hq, Hkv, Sq, Skv, D, mask, mods, splits: GQA groups packed into one query tile
    ("pack-1q-g8", 2, 16, 2, 1, 4100, 128, None, None, None),
    ("pack-16q-g4-window", 1, 8, 2, 16, 3000, 128, "window", None, 5),
    ("pack-4q-g4-alibi-cap", 2, 8, 2, 4, 2048, 64, None, "mods", None),
    ("pack-8q-g2-docs", 2, 4, 2, 8, 1200, 128, "docs-short", None, 3),
    # g * Sq = 32 rows: the one-wave split-KV instance at its limit; 36 rows: the 4-wave tiles
    ("pack-8q-g4-32rows", 1, 8, 2, 8, 2500, 128, None, None, 4),
    ("pack-9q-g4-36rows", 1, 8, 2, 9, 2500, 128, None, None, 4),
]


@pytest.mark.parametrize("case", PACK_CASES, ids=[c[0] for c in PACK_CASES])
def test_gqa_packed_decode(case):
    """Short query blocks with grouped-query attention run the group's heads
    as one tile (per-lane heads: ALiBi slopes, rows of several heads) --
    against the oracle and against the unsplit forward."""
    import torch
    import pallas_flexattn as pf
    name, B, Hq, Hkv, Sq, Skv, D, mname, sname, splits = case
    print(f"[gpu splitkv] {name}", flush=True)
    q, k, v = _case(B, Hq, Hkv, Sq, Skv, D, 11)
    mm, bm, omask = None, None, None
    if mname == "window":
        mm = pf.sliding_window_mask(700, 300)
    elif mname == "docs-short":
        mm = pf.sliding_window_mask(-1, 600)
    if mm is not None:
        bm = pf.create_block_mask(mm, B, Hq, Sq, Skv, 128)
        omask = mm
    score = slopes = cap = None
    if sname == "mods":
        score = pf.compose_score_mods(pf.alibi_score_mod(Hq), pf.softcap_score_mod(30.0))
        slopes, cap = pf.alibi_slopes(Hq), 30.0
    o, lse = pf.flex_decode(q, k, v, score_mod=score, block_mask=bm, enable_gqa=True, num_splits=splits,
                            return_lse=True)
    o1, lse1 = pf.flex_attention(q, k, v, score_mod=score, block_mask=bm, enable_gqa=True, return_lse=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(o.float().cpu().numpy(), o1.float().cpu().numpy(), atol=1e-2, rtol=1e-2)
    ro, rlse = _oracle(q, k, v, mask=omask, slopes=slopes, cap=cap)
    np.testing.assert_allclose(o.float().cpu().numpy(), ro, atol=2e-2, rtol=2e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), rlse, atol=1e-3, rtol=1e-3)
    np.testing.assert_allclose(o1.float().cpu().numpy(), ro, atol=2e-2, rtol=2e-2)


def test_gqa_packed_forward_with_backward():
    """The unsplit forward packs short GQA query blocks too; the backward
    (not packed) consumes its O and LSE."""
    import torch
    import pallas_flexattn as pf
    from _cases import BF16_TOL, assert_close, inputs, oracle_fwd_bwd, oracle_mask, to_np, to_torch
    B, Hq, Hkv, Sq, Skv, D = 2, 8, 2, 40, 600, 128
    q, k, v, do = inputs(5, B, Hq, Hkv, Sq, Skv, D, "bf16")
    bm = pf.create_block_mask(pf.sliding_window_mask(-1, 500), B, Hq, Sq, Skv, 128)
    tq, tk, tv = (to_torch(x, "bf16").requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, block_mask=bm, enable_gqa=True, return_lse=True)
    o.backward(to_torch(do, "bf16"))
    torch.cuda.synchronize()
    om = oracle_mask("window", Sq, Skv, 1, -1, 500)
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om)
    for nm, got, want in (("O", o, wo), ("LSE", lse, wl), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk),
                          ("dV", tv.grad, wdv)):
        assert_close(nm, to_np(got), want, BF16_TOL)


@pytest.mark.parametrize("paged", [False, True], ids=["contiguous", "paged"])
def test_kv_cache_lengths_and_pages(paged):
    """Per-batch key counts (kv_lens) and paged K / V caches (page_table):
    against the oracle with the keys past each row's length masked, and the
    paged run bit-identical to the contiguous one on the same keys."""
    import torch
    import pallas_flexattn as pf
    B, Hq, Hkv, Sq, D, ps = 3, 8, 2, 2, 128, 128
    max_pages = 24
    Skv = max_pages * ps
    q, k, v = _case(B, Hq, Hkv, Sq, Skv, D, 13)
    kv_lens = torch.tensor([Skv, 1000, 257], dtype=torch.int32)
    print(f"[gpu splitkv] kv cache paged={paged}", flush=True)
    o_c, lse_c = pf.flex_decode(q, k, v, enable_gqa=True, kv_lens=kv_lens, return_lse=True)
    mask = np.zeros((B, 1, Sq, Skv), bool)
    for b in range(B):
        mask[b, :, :, :int(kv_lens[b])] = True
    ro, rlse = _oracle(q, k, v, mask=mask)
    np.testing.assert_allclose(o_c.float().cpu().numpy(), ro, atol=2e-2, rtol=2e-2)
    np.testing.assert_allclose(lse_c.cpu().numpy(), rlse, atol=1e-3, rtol=1e-3)
    if not paged:
        return
    rng = np.random.default_rng(3)
    num_pages = B * max_pages + 5
    perm = rng.permutation(num_pages)[:B * max_pages].reshape(B, max_pages)
    kc = torch.zeros(num_pages, Hkv, ps, D, dtype=k.dtype, device=k.device)
    vc = torch.zeros_like(kc)
    for b in range(B):
        for j in range(max_pages):
            kc[perm[b, j]] = k[b, :, j * ps:(j + 1) * ps]
            vc[perm[b, j]] = v[b, :, j * ps:(j + 1) * ps]
    pt = torch.from_numpy(perm.astype(np.int32))
    for splits in (None, 1, 7):
        o_p, lse_p = pf.flex_decode(q, kc, vc, enable_gqa=True, kv_lens=kv_lens, page_table=pt, num_splits=splits,
                                    return_lse=True)
        o_r, lse_r = pf.flex_decode(q, k, v, enable_gqa=True, kv_lens=kv_lens, num_splits=splits, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(o_p, o_r) and torch.equal(lse_p, lse_r), f"paged != contiguous (splits={splits})"
