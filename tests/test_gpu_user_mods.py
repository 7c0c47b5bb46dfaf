"""User mask_mod / score_mod callables on the GPU: traced, compiled at run time
into the tile kernels (C ABI fa_mods_*), forward and backward against the
float64 oracle (bf16 atol = rtol = 2e-2, fp32 1e-5).  The oracle's mask is
the materialised predicate written again in numpy, and its score mod is a
numpy function with a hand-derived derivative (pinned by finite differences
in tests/test_oracle.py), so nothing here checks the lowering against
itself."""
import zlib

import numpy as np
import pytest

from _cases import BF16_TOL, FP32_TOL, assert_close, inputs, oracle_fwd_bwd, to_np, to_torch

pytestmark = pytest.mark.gpu


def _pf():
    import pallas_flexattn as pf
    return pf


def _dense_mask(fn_np, B, H, Sq, Skv):
    q, k = np.arange(Sq)[:, None], np.arange(Skv)[None, :]
    return np.stack([np.stack([np.broadcast_to(fn_np(b, h, q, k), (Sq, Skv)) for h in range(H)])
                     for b in range(B)])


def _case_mods(name, Hq, S):
    """(mask callable for the kernels, its numpy twin, score callable, numpy score fn with derivative)."""
    import torch
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    if name == "prefix-lm":
        return (lambda q, kv: (kv < 96) | (q >= kv), lambda b, h, q, k: (k < 96) | (q >= k), None, None)
    if name == "parity":
        return (lambda q, kv: ((q - kv) % 2 == 0) & (q >= kv),
                lambda b, h, q, k: ((q - k) % 2 == 0) & (q >= k), None, None)
    if name == "head-bias-table":
        bias = rng.standard_normal((Hq, S)).astype(np.float32)
        tb = torch.from_numpy(bias)

        def np_score(s, b, h, q, k):
            return s + bias[h][np.broadcast_to(k, s.shape)], np.ones_like(s)
        return (None, None, lambda s, b, h, q, kv: s + tb[h, kv], np_score)
    if name == "custom-softcap-causal":
        def np_score(s, b, h, q, k):
            t = np.tanh(s / 7.0)
            return 7.0 * t + 0.5 * (h % 2), 1.0 - t * t
        return ("causal", None, lambda s, b, h, q, kv: 7.0 * torch.tanh(s / 7.0) + 0.5 * (h % 2), np_score)
    if name == "banded-per-head":
        widths = torch.tensor([16, 40, 100, 1000][:Hq] + [64] * max(0, Hq - 4), dtype=torch.int32)
        wn = widths.numpy()
        return (lambda b, h, q, kv: (q >= kv) & ((q - kv) < widths[h]),
                lambda b, h, q, k: (q >= k) & ((q - k) < wn[h]), None, None)
    if name == "quadratic-score-window":
        def np_score(s, b, h, q, k):
            return s - 0.05 * s * s, 1.0 - 0.1 * s
        return (lambda q, kv: (q - kv <= 70) & (kv - q <= 30), lambda b, h, q, k: (q - k <= 70) & (k - q <= 30),
                lambda s, b, h, q, kv: s - 0.05 * s * s, np_score)
    raise ValueError(name)


CASES = [
    # name, dtype, B, Hq, Hkv, S, D
    ("prefix-lm", "bf16", 2, 4, 4, 384, 128),
    ("prefix-lm", "fp32", 1, 2, 2, 256, 64),
    ("parity", "bf16", 1, 4, 2, 320, 128),
    ("head-bias-table", "bf16", 2, 4, 4, 256, 128),
    ("head-bias-table", "fp32", 1, 2, 1, 192, 64),
    ("custom-softcap-causal", "bf16", 1, 4, 4, 384, 64),
    ("banded-per-head", "bf16", 1, 4, 4, 512, 128),
    ("quadratic-score-window", "fp32", 1, 2, 2, 256, 32),
    ("quadratic-score-window", "bf16", 1, 2, 2, 256, 32),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}" for c in CASES])
def test_user_mods_fwd_bwd(case):
    import torch
    pf = _pf()
    name, dtype, B, Hq, Hkv, S, D = case
    print(f"[gpu user-mods] {name} {dtype}", flush=True)
    q, k, v, do = inputs(zlib.crc32(f"{name}{dtype}".encode()) % 1000, B, Hq, Hkv, S, S, D, dtype)
    mask_fn, mask_np, score_fn, score_np = _case_mods(name, Hq, S)
    if mask_fn == "causal":
        mask_fn, mask_np = pf.causal_mask, (lambda b, h, q, k: q >= k)
    bm = pf.create_block_mask(mask_fn, B, Hq, S, S, 128) if mask_fn is not None else None
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, score_mod=score_fn, block_mask=bm, enable_gqa=Hq != Hkv,
                               return_lse=True)
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    om = _dense_mask(mask_np, B, Hq, S, S) if mask_np is not None else None
    want_o, want_lse, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om, score_fn=score_np)
    tol = BF16_TOL if dtype == "bf16" else FP32_TOL
    for nm, got, want in (("O", o, want_o), ("LSE", lse, want_lse), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk),
                          ("dV", tv.grad, wdv)):
        assert_close(f"{name} {nm}", to_np(got), want, tol)


def test_reference_api_with_a_callable_mask():
    """flash_attention / flash_attention_fwd / the backward stages with a plain
    (q_idx, kv_idx) callable, as the reference takes mask_mod (flash_attn.py:85-88)."""
    import math
    import torch
    pf = _pf()
    B, H, T, D = 2, 2, 256, 64
    fn = lambda q, kv: (q >= kv) & ((q // 64) - (kv // 64) <= 1)  # noqa: E731
    fnp = lambda b, h, q, k: (q >= k) & ((q // 64) - (k // 64) <= 1)  # noqa: E731
    q, k, v, do = inputs(3, B, H, H, T, T, D, "fp32")
    tq, tk, tv = (to_torch(x, "fp32").requires_grad_() for x in (q, k, v))
    o = pf.flash_attention(tq, tk, tv, mask_mod=fn)
    o.backward(to_torch(do, "fp32"))
    om = _dense_mask(fnp, B, H, T, T)
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om)
    for nm, got, want in (("O", o, wo), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk), ("dV", tv.grad, wdv)):
        assert_close(nm, to_np(got), want, FP32_TOL)
    o2, lse2 = pf.flash_attention_fwd(tq.detach(), tk.detach(), tv.detach(), mask_mod=fn)
    assert_close("fwd LSE", to_np(lse2), wl, FP32_TOL)
    flat = lambda t: t.detach().reshape(B * H, T, D)  # noqa: E731
    delta = pf.flash_attention_bwd_preprocess(flat(o2), flat(to_torch(do, "fp32")))
    sc = 1.0 / math.sqrt(D)
    dk, dv = pf.flash_attention_bwd_dkv(flat(tq), flat(tk), flat(tv), flat(to_torch(do, "fp32")),
                                        lse2.reshape(B * H, T), delta, sc, sc, mask_mod=fn)
    dq = pf.flash_attention_bwd_dq(flat(tq), flat(tk), flat(tv), flat(to_torch(do, "fp32")),
                                   lse2.reshape(B * H, T), delta, sc, sc, mask_mod=fn)
    torch.cuda.synchronize()
    for nm, got, want in (("stage dQ", dq, wdq), ("stage dK", dk, wdk), ("stage dV", dv, wdv)):
        assert_close(nm, to_np(got).reshape(want.shape), want, FP32_TOL)


def test_callable_mask_with_builtin_score_and_document_labels():
    """A traced mask next to the built-in ALiBi + soft-cap, and a traced score
    next to a document-label mask (lowered with it: the bf16 tile kernels take
    documents only as intervals)."""
    import torch
    pf = _pf()
    B, Hq, Hkv, S, D = 2, 4, 2, 256, 128
    q, k, v, do = inputs(21, B, Hq, Hkv, S, S, D, "bf16")
    slopes = pf.alibi_slopes(Hq)
    sc = pf.compose_score_mods(pf.alibi_score_mod(slopes), pf.softcap_score_mod(30.0))
    fn = lambda q, kv: (q >= kv) & ((q - kv) % 3 != 2)  # noqa: E731
    bm = pf.create_block_mask(fn, B, Hq, S, S, 128)
    tq, tk, tv = (to_torch(x, "bf16").requires_grad_() for x in (q, k, v))
    o = pf.flex_attention(tq, tk, tv, score_mod=sc, block_mask=bm, enable_gqa=True)
    o.backward(to_torch(do, "bf16"))
    torch.cuda.synchronize()
    om = _dense_mask(lambda b, h, q, k: (q >= k) & ((q - k) % 3 != 2), B, Hq, S, S)
    wo, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om, alibi=slopes, softcap=30.0)
    for nm, got, want in (("O", o, wo), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk), ("dV", tv.grad, wdv)):
        assert_close(f"mask+alibi {nm}", to_np(got), want, BF16_TOL)

    rng = np.random.default_rng(4)
    ids = rng.integers(0, 3, size=(B, S)).astype(np.int32)
    dm = pf.and_masks(pf.document_ids_mask(ids), pf.causal_mask)
    bm2 = pf.create_block_mask(dm, B, Hq, S, S, 128)
    score = lambda s, b, h, q, kv: s * 0.75 + 0.1 * (h - 1)  # noqa: E731
    tq, tk, tv = (to_torch(x, "bf16").requires_grad_() for x in (q, k, v))
    o = pf.flex_attention(tq, tk, tv, score_mod=score, block_mask=bm2, enable_gqa=True)
    o.backward(to_torch(do, "bf16"))
    torch.cuda.synchronize()
    om2 = (ids[:, :, None] == ids[:, None, :]) & (np.arange(S)[:, None] >= np.arange(S)[None, :])
    wo, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om2[:, None],
                                            score_fn=lambda s, b, h, q, k: (s * 0.75 + 0.1 * (h - 1),
                                                                            np.full_like(s, 0.75)))
    for nm, got, want in (("O", o, wo), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk), ("dV", tv.grad, wdv)):
        assert_close(f"docs+score {nm}", to_np(got), want, BF16_TOL)


def test_builtin_score_params_need_a_blob_built_for_them():
    """A call whose params carry ALiBi slopes or a soft-cap runs the built-in
    score epilogue only in a blob compiled with FA_MODS_BUILTIN_SCORE; a
    mask-only blob refuses such params (FA_ERR_UNSUPPORTED) instead of
    silently dropping them, before any launch."""
    import ctypes
    import torch
    from pallas_flexattn import _lib, lowering as L
    from pallas_flexattn.flash_attn import _Plan, _as_score_spec, _stream
    pf = _pf()
    print("[gpu user mods] builtin-score params with a mask-only blob", flush=True)
    lib = _lib.load()
    B, H, S, D = 1, 2, 128, 64
    q, k, v = (torch.randn(B, H, S, D, device="cuda").to(torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda", dtype=torch.float32)
    mods = L.UserMods(L.lower_mask(lambda qi, kv: (qi - kv) % 3 != 1), None)
    blob = _lib.compile_mods(mods.source, _lib.DTYPE_BF16, D, mods.flags(False))
    h = ctypes.c_void_p()
    _lib.check(lib.fa_mods_load(blob, len(blob), ctypes.byref(h)))
    try:
        bufs = (ctypes.c_void_p * 1)()
        for score in (pf.alibi_score_mod(H), pf.softcap_score_mod(20.0)):
            plan = _Plan(q, k, None, _as_score_spec(score), None, None, (128, 64, 128))
            rc = lib.fa_mods_fwd(h, plan.ptr(), bufs, 0, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                 lse.data_ptr(), _stream())
            assert rc == -4, rc  # FA_ERR_UNSUPPORTED
        plan = _Plan(q, k, None, None, None, None, (128, 64, 128))  # no built-in score: runs
        _lib.check(lib.fa_mods_fwd(h, plan.ptr(), bufs, 0, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   lse.data_ptr(), _stream()))
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.fa_mods_unload(h))
