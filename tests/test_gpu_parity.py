"""GPU parity: the HIP kernels (through the C ABI) against the float64 oracle.

Tolerances: bf16 atol = rtol = 2e-2 on O, dQ, dK, dV (and LSE); fp32 atol =
rtol = 1e-5.  Inputs are seeded numpy normals (bf16 values rounded RNE)."""
import zlib

import numpy as np
import pytest

from _cases import (BF16_TOL, FP32_TOL, assert_as_accurate, assert_close, inputs, oracle_fwd_bwd, oracle_mask,
                    to_np, to_torch)

pytestmark = pytest.mark.gpu


def _pf():
    import pallas_flexattn as pf
    return pf


def _doc_lengths(rng, S):
    out, tot = [], 0
    while tot < S:
        n = int(rng.integers(24, 160))
        n = min(n, S - tot)
        out.append(n)
        tot += n
    return out


CASES = [
    # name, dtype, B, Hq, Hkv, S, D, mask, extras
    ("causal-bf16-d128", "bf16", 2, 4, 4, 256, 128, ("causal",), {}),
    ("causal-fp32-d64", "fp32", 1, 4, 4, 256, 64, ("causal",), {}),
    ("dense-bf16-d64-ragged", "bf16", 2, 2, 2, 192, 64, ("none",), {}),
    ("window-bf16-d128", "bf16", 1, 2, 2, 512, 128, ("window", 100, 0), {}),
    ("window-sym-bf16-d64", "bf16", 1, 2, 2, 384, 64, ("window", 32, 32), {}),
    ("doc-causal-bf16-d128", "bf16", 2, 2, 2, 512, 128, ("doc",), {}),
    ("gqa-alibi-softcap-bf16", "bf16", 1, 8, 2, 256, 128, ("causal",), {"alibi": True, "softcap": 50.0}),
    ("ragged-causal-bf16-d128", "bf16", 1, 2, 2, 300, 128, ("causal",), {}),
    ("dense-fp32-d32", "fp32", 1, 2, 2, 128, 32, ("none",), {}),
    ("causal-bf16-d32", "bf16", 1, 2, 2, 256, 32, ("causal",), {}),
    ("softcap-fp32-d128", "fp32", 1, 2, 1, 160, 128, ("causal",), {"softcap": 20.0, "alibi": True}),
    # each built-in score mod alone (the kernels' uncapped and capped branches)
    ("gqa-alibi-only-bf16", "bf16", 1, 4, 2, 320, 128, ("causal",), {"alibi": True}),
    ("softcap-only-window-bf16-d64", "bf16", 2, 2, 2, 384, 64, ("window", 96, 16), {"softcap": 30.0}),
    # full tiles of several q heads walked before the partial ones (GQA group of 4, no score mods)
    ("gqa-causal-bf16-d128", "bf16", 2, 8, 2, 384, 128, ("causal",), {}),
    # a window wide enough for fully-live tiles inside it
    ("window-wide-bf16-d128", "bf16", 1, 2, 2, 1024, 128, ("window", 300, 0), {}),
    # mask blocks of 2 and 3 kernel tiles per side (power-of-two and general sub-tile walks)
    ("causal-bf16-block256", "bf16", 1, 2, 2, 768, 128, ("causal",), {"block": 256}),
    ("causal-bf16-block384-d64", "bf16", 1, 2, 2, 768, 64, ("causal",), {"block": 384}),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_flex_attention_fwd_bwd(case):
    import torch
    pf = _pf()
    name, dtype, B, Hq, Hkv, S, D, mspec, extras = case
    print(f"[gpu parity] {name}", flush=True)
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, S, S, D, dtype)
    kind = mspec[0]
    doc_ids = None
    if kind == "causal":
        mm = pf.causal_mask
    elif kind == "window":
        mm = pf.sliding_window_mask(mspec[1], mspec[2])
    elif kind == "doc":
        rng = np.random.default_rng(7)
        lens = [_doc_lengths(rng, S) for _ in range(B)]
        dm = pf.document_mask(lens)
        doc_ids = dm.doc_ids
        mm = pf.and_masks(dm, pf.causal_mask)
    else:
        mm = None
    omask = oracle_mask("causal" if kind == "doc" else kind, S, S, B,
                        *(mspec[1:] if kind == "window" else ()), doc_ids=doc_ids)
    alibi = pf.alibi_slopes(Hq) if extras.get("alibi") else None
    softcap = extras.get("softcap")
    score = None
    if alibi is not None or softcap:
        parts = []
        if alibi is not None:
            parts.append(pf.alibi_score_mod(alibi))
        if softcap:
            parts.append(pf.softcap_score_mod(softcap))
        score = pf.compose_score_mods(*parts)
    bm = pf.create_block_mask(mm, B, Hq, S, S, extras.get("block", 128)) if mm is not None else None

    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    tdo = to_torch(do, dtype)
    o, lse = pf.flex_attention(tq, tk, tv, score_mod=score, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    o.backward(tdo)
    torch.cuda.synchronize()

    want_o, want_lse, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, omask, alibi=alibi, softcap=softcap)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    assert_close(f"{name} O", to_np(o), want_o, tol)
    assert_close(f"{name} LSE", to_np(lse), want_lse, tol)
    assert_close(f"{name} dQ", to_np(tq.grad), wdq, tol)
    assert_close(f"{name} dK", to_np(tk.grad), wdk, tol)
    assert_close(f"{name} dV", to_np(tv.grad), wdv, tol)


def test_flash_attention_autograd_fp32_block64():
    """flash_attention (custom backward) at the fp32 C1 shape: B1 H4 S256 D64, causal, block 64."""
    pf = _pf()
    B, H, S, D = 1, 4, 256, 64
    q, k, v, do = inputs(0, B, H, H, S, S, D, "fp32")
    tq, tk, tv = (to_torch(x, "fp32").requires_grad_() for x in (q, k, v))
    o = pf.flash_attention(tq, tk, tv, mask_mod=pf.causal_mask, block_r=64, block_c=64)
    o.backward(to_torch(do, "fp32"))
    wo, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, oracle_mask("causal", S, S))
    assert_close("O", to_np(o), wo, FP32_TOL)
    assert_close("dQ", to_np(tq.grad), wdq, FP32_TOL)
    assert_close("dK", to_np(tk.grad), wdk, FP32_TOL)
    assert_close("dV", to_np(tv.grad), wdv, FP32_TOL)


RESCALE_CASES = [
    # name, mask, q scale, key ramp (k row j scaled by 1 + ramp * j / S), check gradients
    # logits grow along the keys: the running maximum rises by more than 16 (log2 units) between
    # tiles, so the forward's speculative exponentials fail the 2^16 check mid-walk and the wave
    # takes the exact rescale path
    ("growing-dense", None, 2.0, 3.0, True),
    ("growing-causal", "causal", 2.0, 3.0, True),
    # logits with standard deviation 64: on ~40 rows the running maximum jumps by more than 128
    # (log2 units) from one 64-key tile to the next, so the speculative exponentials overflow to
    # inf before the exact path replaces them
    ("huge-logits-dense", None, 64.0, 0.0, False),
]


@pytest.mark.parametrize("case", RESCALE_CASES, ids=[c[0] for c in RESCALE_CASES])
def test_forward_rescale_paths(case):
    """bf16 inputs whose row maxima grow along the kv walk: O and LSE (and
    the gradients for the moderate cases) against the float64 oracle."""
    import torch
    pf = _pf()
    name, kind, qscale, ramp, grads = case
    B, H, S, D = 1, 2, 512, 128
    print(f"[gpu parity] rescale {name}", flush=True)
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, H, H, S, S, D, "fp32")
    from oracle.bf16 import round_bf16
    q = round_bf16(q * qscale)
    k = round_bf16(k * (1.0 + ramp * np.arange(S, dtype=np.float32) / S)[None, None, :, None])
    v, do = round_bf16(v), round_bf16(do)
    bm = pf.create_block_mask(pf.causal_mask, B, H, S, S, 128) if kind == "causal" else None
    tq, tk, tv = (to_torch(x, "bf16").requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, block_mask=bm, return_lse=True)
    if grads:
        o.backward(to_torch(do, "bf16"))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(lse).all())
    omask = oracle_mask(kind or "none", S, S)
    want_o, want_lse, g = oracle_fwd_bwd(q, k, v, do, omask, bwd=grads)
    assert_close(f"{name} O", to_np(o), want_o, BF16_TOL)
    assert_close(f"{name} LSE", to_np(lse), want_lse, BF16_TOL)
    if grads:
        # With keys up to 4x larger the bf16 roundings of P and dS before the backward products
        # set the gradient error (small dQ / dK values from large dS terms that cancel): the
        # oracle's C restatement of the reference's tiled algorithm (same cast points, float32
        # LSE / Delta) is itself off from float64 by up to 0.08 in dQ here, and two restatements
        # that differ only in where the softmax scale meets the dS rounding differ from each other
        # by as much.  So the kernels' gradients are held to the reference's own gradient
        # tolerance against float64 (tests/test_flash_attn.py:133-135) and to the accuracy of the
        # reference algorithm: max and RMS errors against float64 within 1.5x / 1.25x of its.
        from oracle import tiled
        win = (-1, 0) if kind == "causal" else None
        to, tl = tiled.fwd(q, k, v, 64, 64, window=win, bf16=True, stats_in_dtype=False)
        tg = tiled.bwd(q, k, v, to, tl, do, 64, 64, window=win, bf16=True, stats_in_dtype=False)
        for i, (nm, got) in enumerate((("dQ", tq.grad), ("dK", tk.grad), ("dV", tv.grad))):
            assert_close(f"{name} {nm} vs float64", to_np(got), g[i], dict(atol=1e-1, rtol=1e-2))
            assert_as_accurate(f"{name} {nm}", to_np(got), tg[i], g[i])


DOC_LABEL_CASES = [
    # name, dtype, B, Hq, Hkv, S, D, causal
    ("labels-bf16-d128-causal", "bf16", 2, 4, 2, 320, 128, True),
    ("labels-bf16-d64", "bf16", 1, 2, 2, 256, 64, False),
    ("labels-fp32-d64-causal", "fp32", 1, 2, 1, 200, 64, True),
]


@pytest.mark.parametrize("case", DOC_LABEL_CASES, ids=[c[0] for c in DOC_LABEL_CASES])
def test_document_labels_not_contiguous(case):
    """document_ids_mask with labels that recur along the sequence (tokens of
    one document interleaved with others): the kernels compare ids per element
    (the generic forward, dK/dV and dQ kernels), forward and backward."""
    import torch
    pf = _pf()
    name, dtype, B, Hq, Hkv, S, D, causal = case
    print(f"[gpu parity] {name}", flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    ids = rng.integers(0, 3, size=(B, S)).astype(np.int32)
    ids[:, ::7] = 5  # a label spread evenly over the whole row
    dm = pf.document_ids_mask(ids)
    mm = pf.and_masks(dm, pf.causal_mask) if causal else dm
    assert dm.doc_bounds() is None  # not contiguous runs: the id-comparing kernels run
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, S, S, D, dtype)
    bm = pf.create_block_mask(mm, B, Hq, S, S, 128)
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    omask = oracle_mask("causal" if causal else "none", S, S)
    same = ids[:, :, None] == ids[:, None, :]
    omask = (same if omask is None else (omask[0, 0][None] & same))[:, None]
    want_o, want_lse, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, omask)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    for nm, got, want in (("O", o, want_o), ("LSE", lse, want_lse), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk),
                          ("dV", tv.grad, wdv)):
        assert_close(f"{name} {nm}", to_np(got), want, tol)


SQ_SKV_CASES = [
    # name, dtype, B, Hq, Hkv, Sq, Skv, D, mask
    ("kv-longer-causal-bf16", "bf16", 1, 4, 2, 192, 448, 128, ("causal",)),
    ("kv-longer-window-bf16", "bf16", 2, 2, 2, 256, 640, 64, ("window", 200, 100)),
    ("q-longer-window-bf16", "bf16", 1, 2, 2, 384, 256, 128, ("window", 100, 0)),
    ("kv-longer-dense-fp32", "fp32", 1, 2, 1, 96, 300, 64, ("none",)),
]


@pytest.mark.parametrize("case", SQ_SKV_CASES, ids=[c[0] for c in SQ_SKV_CASES])
def test_query_and_key_lengths_differ(case):
    """Forward and backward with Sq != Skv (mask predicates on the raw query and
    key indices).  With the window and Sq > Skv some rows see no key at all:
    O = 0, LSE = -inf and zero gradients there, as in the oracle."""
    import torch
    pf = _pf()
    name, dtype, B, Hq, Hkv, Sq, Skv, D, mspec = case
    print(f"[gpu parity] {name}", flush=True)
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, Sq, Skv, D, dtype)
    if mspec[0] == "causal":
        mm, om = pf.causal_mask, oracle_mask("causal", Sq, Skv)
    elif mspec[0] == "window":
        mm, om = pf.sliding_window_mask(mspec[1], mspec[2]), oracle_mask("window", Sq, Skv, 1, mspec[1], mspec[2])
    else:
        mm, om = None, None
    bm = pf.create_block_mask(mm, B, Hq, Sq, Skv, 128) if mm is not None else None
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    want_o, want_lse, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    got_lse = to_np(lse)
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(want_lse)), "rows without a live key differ"
    fin = np.isfinite(want_lse)
    assert_close(f"{name} LSE", got_lse[fin], want_lse[fin], tol)
    for nm, got, want in (("O", o, want_o), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk), ("dV", tv.grad, wdv)):
        assert_close(f"{name} {nm}", to_np(got), want, tol)
