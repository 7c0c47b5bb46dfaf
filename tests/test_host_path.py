"""The host path (interpret=True), on the CPU: the reference-signature entry
points with ``interpret=True`` on CPU tensors run the library's host twins
(``fa_fwd_host`` / ``fa_bwd_*_host``), as the reference's interpret mode runs
its Pallas kernels on the CPU.  The reference's own test shapes
(``tests/test_flash_attn.py:26-191``), plus score mods, GQA, documents and
block tables through the host forward / backward cores, against the float64
oracle: float32 atol = rtol = 1e-5; bfloat16 atol = rtol = 2e-2 for O, and
gradients at 2e-2 against the oracle's C restatement of the reference's tiled
algorithm (P and dS rounded to bf16 before their products, as the host twins
do) with 5e-2 against float64 as a sanity bound."""
import math
import zlib

import numpy as np
import pytest

from _cases import BF16_TOL, FP32_TOL, assert_close, inputs, oracle_fwd_bwd, oracle_mask, to_np

torch = pytest.importorskip("torch")

import pallas_flexattn as pf  # noqa: E402

SANITY = dict(atol=5e-2, rtol=5e-2)


def cpu(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16 if dtype == "bf16" else torch.float32)


def _mask(name):
    return {"none": None, "causal": pf.causal_mask, "bidirectional": pf.bidirectional_mask,
            "sliding": pf.sliding_window_mask(32, 32)}[name]


def _omask(name, S):
    if name in ("none", "bidirectional"):
        return None
    if name == "causal":
        return oracle_mask("causal", S, S)
    return oracle_mask("window", S, S, 1, 32, 32)


def _window(name):
    return {"none": None, "bidirectional": None, "causal": (-1, 0), "sliding": (32, 32)}[name]


FWD_SHAPES = (
    [(b, 4, 64, 32, "none") for b in (1, 2, 4)]
    + [(2, 4, 64, d, "none") for d in (64, 128)]
    + [(2, 4, 128, 64, m) for m in ("none", "causal", "bidirectional", "sliding")]
    + [(1, 2, 512, 64, "none")]
)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("shape", FWD_SHAPES, ids=[f"B{b}H{h}T{t}D{d}-{m}" for b, h, t, d, m in FWD_SHAPES])
def test_forward_interpret(shape, dtype):
    B, H, T, D, mname = shape
    q, k, v, _ = inputs(zlib.crc32(repr(shape).encode()) % 997, B, H, H, T, T, D, dtype)
    o, lse = pf.flash_attention_fwd(cpu(q, dtype), cpu(k, dtype), cpu(v, dtype), mask_mod=_mask(mname),
                                    interpret=True)
    assert not o.is_cuda and o.shape == (B, H, T, D) and lse.dtype == o.dtype
    wo, wl, _ = oracle_fwd_bwd(q, k, v, None, _omask(mname, T), bwd=False)
    tol = FP32_TOL if dtype == "fp32" else BF16_TOL
    assert_close("O", to_np(o), wo, tol)
    assert_close("LSE", to_np(lse), wl, tol if dtype == "fp32" else dict(atol=2e-2, rtol=8e-3))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("mname", ["none", "causal", "sliding"])
def test_autograd_interpret(mname, dtype):
    """flash_attention(interpret=True) with autograd, B2 H4 T128 D64."""
    B, H, T, D = 2, 4, 128, 64
    q, k, v, do = inputs(zlib.crc32(mname.encode()), B, H, H, T, T, D, dtype)
    tq, tk, tv = (cpu(x, dtype).requires_grad_() for x in (q, k, v))
    o = pf.flash_attention(tq, tk, tv, mask_mod=_mask(mname), interpret=True)
    o.backward(cpu(do, dtype))
    wo, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, _omask(mname, T))
    got = {"dQ": to_np(tq.grad), "dK": to_np(tk.grad), "dV": to_np(tv.grad)}
    if dtype == "fp32":
        assert_close("O", to_np(o), wo, FP32_TOL)
        for n, w in (("dQ", wdq), ("dK", wdk), ("dV", wdv)):
            assert_close(n, got[n], w, FP32_TOL)
        return
    assert_close("O", to_np(o), wo, BF16_TOL)
    from oracle import tiled
    to, tl = tiled.fwd(q, k, v, 64, 64, window=_window(mname), bf16=True, stats_in_dtype=False)
    tg = tiled.bwd(q, k, v, to, tl, do, 64, 64, window=_window(mname), bf16=True, stats_in_dtype=False)
    for n, tw, w in zip(("dQ", "dK", "dV"), tg, (wdq, wdk, wdv)):
        assert_close(f"{n} vs tiled reference algorithm", got[n], tw, BF16_TOL)
        assert_close(f"{n} vs float64", got[n], w, SANITY)


@pytest.mark.parametrize("mname", ["none", "causal", "sliding"])
def test_backward_stages_interpret(mname):
    """The three backward stages with interpret=True on flattened arrays equal
    flash_attention_bwd(interpret=True) exactly and match the oracle."""
    B, H, T, D = 2, 2, 96, 32
    q, k, v, do = inputs(zlib.crc32(("st" + mname).encode()), B, H, H, T, T, D, "fp32")
    tq, tk, tv, tdo = (cpu(x, "fp32") for x in (q, k, v, do))
    mm = _mask(mname)
    o, lse = pf.flash_attention_fwd(tq, tk, tv, mask_mod=mm, interpret=True)
    flat = lambda t: t.reshape(B * H, T, *t.shape[3:])  # noqa: E731
    delta = pf.flash_attention_bwd_preprocess(flat(o), flat(tdo), interpret=True)
    assert_close("Delta", to_np(delta), to_np((o * tdo).sum(-1).reshape(B * H, T)), dict(atol=1e-5, rtol=1e-5))
    sc = 1.0 / math.sqrt(D)
    dk, dv = pf.flash_attention_bwd_dkv(flat(tq), flat(tk), flat(tv), flat(tdo), flat(lse), delta, sc, sc,
                                        mask_mod=mm, interpret=True)
    dq = pf.flash_attention_bwd_dq(flat(tq), flat(tk), flat(tv), flat(tdo), flat(lse), delta, sc, sc,
                                   mask_mod=mm, interpret=True)
    rdq, rdk, rdv = pf.flash_attention_bwd(tq, tk, tv, o, lse, tdo, mask_mod=mm, interpret=True)
    for n, a, b in (("dQ", dq, rdq), ("dK", dk, rdk), ("dV", dv, rdv)):
        assert torch.equal(a.reshape(b.shape), b), f"{n}: staged and whole backward differ"
    _, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, _omask(mname, T))
    for n, g, w in (("dQ", dq, wdq), ("dK", dk, wdk), ("dV", dv, wdv)):
        assert_close(n, to_np(g).reshape(w.shape), w, FP32_TOL)


HOST_CASES = [
    # name, dtype, B, Hq, Hkv, S, D, mask kind, alibi, softcap
    ("gqa-alibi-softcap-causal", "fp32", 1, 4, 2, 160, 64, "causal", True, 20.0),
    ("gqa-alibi-softcap-causal", "bf16", 1, 4, 2, 160, 64, "causal", True, 20.0),
    ("documents-contiguous", "fp32", 2, 2, 2, 200, 32, "docs", False, None),
    ("documents-labels", "fp32", 2, 2, 1, 150, 32, "labels", False, None),
    ("window-tables", "bf16", 1, 2, 2, 384, 64, "window", False, None),
]


@pytest.mark.parametrize("case", HOST_CASES, ids=[f"{c[0]}-{c[1]}" for c in HOST_CASES])
def test_host_cores_with_mods_documents_and_tables(case):
    """The host forward / backward cores with score mods, GQA, document masks
    (contiguous runs and recurring labels) and block tables, through the same
    plans (fa_params) the GPU path uses."""
    from pallas_flexattn.flash_attn import _bwd_core, _fwd_core
    name, dtype, B, Hq, Hkv, S, D, kind, alibi, softcap = case
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, S, S, D, dtype)
    rng = np.random.default_rng(3)
    doc_ids = None
    if kind == "causal":
        mask, om = pf.causal_mask, oracle_mask("causal", S, S)
    elif kind == "window":
        mask, om = pf.sliding_window_mask(90, 10), oracle_mask("window", S, S, 1, 90, 10)
    elif kind == "docs":
        lens = [[int(x) for x in np.diff(np.r_[0, np.sort(rng.choice(np.arange(1, S), 3, replace=False)), S])]
                for _ in range(B)]
        dm = pf.document_mask(lens)
        doc_ids = dm.doc_ids
        mask, om = pf.and_masks(dm, pf.causal_mask), oracle_mask("causal", S, S, B, doc_ids=doc_ids)
    else:
        ids = rng.integers(0, 3, size=(B, S)).astype(np.int32)
        mask = pf.document_ids_mask(ids)
        om = (ids[:, :, None] == ids[:, None, :])[:, None]
    slopes = pf.alibi_slopes(Hq) if alibi else None
    score = None
    if alibi:
        score = pf.compose_score_mods(pf.alibi_score_mod(slopes), pf.softcap_score_mod(softcap))
    bm = pf.create_block_mask(mask, B, Hq, S, S, 128)
    tq, tk, tv, tdo = (cpu(x, dtype) for x in (q, k, v, do))
    from pallas_flexattn.kernel_tuner import DEFAULT_TILES
    tiles = DEFAULT_TILES[dtype]
    o, lse, plan = _fwd_core(tq, tk, tv, mask, score, None, bm, tiles, None, True)
    dq, dk, dv = _bwd_core(tq, tk, tv, o, lse, tdo, mask, score, None, bm, tiles, None, True, plan=plan)
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om, alibi=slopes, softcap=softcap)
    tol = FP32_TOL if dtype == "fp32" else BF16_TOL
    assert_close(f"{name} O", to_np(o), wo, tol)
    assert_close(f"{name} LSE", to_np(lse), wl, tol)
    gtol = FP32_TOL if dtype == "fp32" else SANITY
    for n, g, w in (("dQ", dq, wdq), ("dK", dk, wdk), ("dV", dv, wdv)):
        assert_close(f"{name} {n}", to_np(g), w, gtol)


def test_host_path_refusals():
    x = torch.zeros(1, 1, 8, 32)
    with pytest.raises(ValueError, match="GPU tensors"):
        pf.flash_attention(x, x, x)  # CPU tensors without interpret
    with pytest.raises(NotImplementedError, match="interpret=True"):
        pf.flash_attention(x, x, x, mask_mod=lambda q, k: (q - k) % 2 == 0, interpret=True)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_empty_problems_interpret(dtype):
    """No queries: empty outputs and gradients.  No keys (Sq > 0): every row
    sees nothing, O = 0 and LSE = -inf (the fully-masked-row convention), zero
    gradients."""
    td = torch.float32 if dtype == "fp32" else torch.bfloat16
    x = torch.zeros(2, 2, 0, 32, dtype=td, requires_grad=True)
    o = pf.flash_attention(x, x, x, mask_mod=pf.causal_mask, interpret=True)
    o.sum().backward()
    assert o.shape == (2, 2, 0, 32) and x.grad.shape == x.shape
    o, lse = pf.flash_attention_fwd(x.detach(), x.detach(), x.detach(), interpret=True)
    assert o.shape == (2, 2, 0, 32) and lse.shape == (2, 2, 0)
    q = torch.randn(1, 2, 5, 32, dtype=td, requires_grad=True)
    kv = torch.zeros(1, 2, 0, 32, dtype=td, requires_grad=True)
    from pallas_flexattn.flash_attn import _bwd_core, _fwd_core
    o, lse, _ = _fwd_core(q.detach(), kv.detach(), kv.detach(), None, None, None, None, (128, 64, 128), None, True)
    assert torch.equal(o, torch.zeros_like(o)) and bool(torch.isneginf(lse).all())
    dq, dk, dv = _bwd_core(q.detach(), kv.detach(), kv.detach(), o, lse, torch.ones_like(o), None, None, None, None,
                           (128, 64, 128), None, True)
    assert not dq.any() and dk.shape == kv.shape and dv.shape == kv.shape
