"""GPU parity of the reference-signature entry points with the reference's own
defaults and test shapes (``tests/test_flash_attn.py`` of the reference).

* forward at T=64 with D in {32, 64, 128} and B in {1, 2, 4}
  (``test_flash_attn.py:73-97``), B2 H4 T128 D64 with no mask, causal,
  bidirectional and sliding_window_mask(32, 32) (``:26-71``), and T=512
  (``:180-191``), through ``flash_attention_fwd`` with its default arguments
  (block_r = block_c = 64);
* forward + backward at B2 H4 T128 D64 through ``flash_attention`` (autograd)
  with no mask, causal and sliding(32, 32) (``:103-162``);
* ``flash_attention_fwd`` -> ``flash_attention_bwd`` with the LSE in q's
  dtype, as the reference passes it;
* the three exported backward stages run one at a time;
* ``mha_reference`` itself;
* the 64-row query tile (``kernel_options={"BLOCK_M": 64}``), including the
  forward's rescale path.

Every case runs in float32 and bfloat16.  Tolerances: float32 atol = rtol =
1e-5 against the float64 oracle; bfloat16 atol = rtol = 2e-2.  bfloat16
gradients are checked at 2e-2 against the oracle's C restatement of the
reference's tiled algorithm (``oracle.tiled``: P and dS rounded to bf16
before their products, as at ``flash_attn.py:94,244-245,349``), and against
the float64 oracle at 5e-2 as a sanity bound on that algorithm."""
import zlib

import numpy as np
import pytest

from _cases import (BF16_TOL, FP32_TOL, assert_as_accurate, assert_close, inputs, oracle_fwd_bwd, oracle_mask, to_np,
                    to_torch)

pytestmark = pytest.mark.gpu

SANITY = dict(atol=5e-2, rtol=5e-2)


def _pf():
    import pallas_flexattn as pf
    return pf


def _mask(pf, name):
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


def _tiled_grads(q, k, v, do, name, stats_in_dtype=False):
    """Gradients of the reference's tiled algorithm in bf16 (oracle C restatement)."""
    from oracle import tiled
    o, lse = tiled.fwd(q, k, v, 64, 64, window=_window(name), bf16=True, stats_in_dtype=stats_in_dtype)
    return tiled.bwd(q, k, v, o, lse, do, 64, 64, window=_window(name), bf16=True, stats_in_dtype=stats_in_dtype)


FWD_SHAPES = (
    # (B, H, T, D, mask): test_different_batch_sizes, test_different_head_dims, the small_attn_inputs
    # cases, test_large_sequence_length
    [(b, 4, 64, 32, "none") for b in (1, 2, 4)]
    + [(2, 4, 64, d, "none") for d in (64, 128)]
    + [(2, 4, 128, 64, m) for m in ("none", "causal", "bidirectional", "sliding")]
    + [(1, 2, 512, 64, "none")]
)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("shape", FWD_SHAPES, ids=[f"B{b}H{h}T{t}D{d}-{m}" for b, h, t, d, m in FWD_SHAPES])
def test_flash_attention_fwd_reference_defaults(shape, dtype):
    pf = _pf()
    B, H, T, D, mname = shape
    print(f"[gpu ref-api] fwd {shape} {dtype}", flush=True)
    q, k, v, _ = inputs(zlib.crc32(repr(shape).encode()) % 997, B, H, H, T, T, D, dtype)
    tq, tk, tv = (to_torch(x, dtype) for x in (q, k, v))
    o, lse = pf.flash_attention_fwd(tq, tk, tv, mask_mod=_mask(pf, mname))
    assert o.shape == tq.shape and lse.shape == (B, H, T) and lse.dtype == tq.dtype
    wo, wl, _ = oracle_fwd_bwd(q, k, v, None, _omask(mname, T), bwd=False)
    tol = FP32_TOL if dtype == "fp32" else BF16_TOL
    assert_close("O", to_np(o), wo, tol)
    # the LSE comes back in q's dtype (flash_attn.py:144): bf16 keeps 8 bits
    assert_close("LSE", to_np(lse), wl, tol if dtype == "fp32" else dict(atol=2e-2, rtol=8e-3))
    assert not bool(o.isnan().any()) and not bool(o.isinf().any())


BWD_MASKS = ["none", "causal", "sliding"]


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("mname", BWD_MASKS)
def test_flash_attention_autograd_reference_shape(mname, dtype):
    """flash_attention (custom backward), B2 H4 T128 D64, dO ~ N(0, 1)."""
    import torch
    pf = _pf()
    B, H, T, D = 2, 4, 128, 64
    print(f"[gpu ref-api] autograd {mname} {dtype}", flush=True)
    q, k, v, do = inputs(zlib.crc32(mname.encode()), B, H, H, T, T, D, dtype)
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o = pf.flash_attention(tq, tk, tv, mask_mod=_mask(pf, mname))
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    wo, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, _omask(mname, T))
    got = {"dQ": to_np(tq.grad), "dK": to_np(tk.grad), "dV": to_np(tv.grad)}
    if dtype == "fp32":
        assert_close("O", to_np(o), wo, FP32_TOL)
        for n, w in (("dQ", wdq), ("dK", wdk), ("dV", wdv)):
            assert_close(n, got[n], w, FP32_TOL)
    else:
        assert_close("O", to_np(o), wo, BF16_TOL)
        tdq, tdk, tdv = _tiled_grads(q, k, v, do, mname)
        for n, tw, w in (("dQ", tdq, wdq), ("dK", tdk, wdk), ("dV", tdv, wdv)):
            assert_close(f"{n} vs tiled reference algorithm", got[n], tw, BF16_TOL)
            assert_close(f"{n} vs float64", got[n], w, SANITY)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_fwd_then_bwd_with_lse_in_input_dtype(dtype):
    """flash_attention_fwd -> flash_attention_bwd, the LSE passed back in q's
    dtype (as the reference's custom_vjp residual is, flash_attn.py:487)."""
    pf = _pf()
    B, H, S, D = 2, 4, 256, 128
    q, k, v, do = inputs(11, B, H, H, S, S, D, dtype, scale=0.5)
    tq, tk, tv, tdo = (to_torch(x, dtype) for x in (q, k, v, do))
    o, lse = pf.flash_attention_fwd(tq, tk, tv, mask_mod=pf.causal_mask)
    assert lse.dtype == tq.dtype
    dq, dk, dv = pf.flash_attention_bwd(tq, tk, tv, o, lse, tdo, mask_mod=pf.causal_mask)
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, oracle_mask("causal", S, S))
    if dtype == "fp32":
        for n, g, w in (("O", o, wo), ("LSE", lse, wl), ("dQ", dq, wdq), ("dK", dk, wdk), ("dV", dv, wdv)):
            assert_close(n, to_np(g), w, FP32_TOL)
        return
    assert_close("O", to_np(o), wo, BF16_TOL)
    # the reference algorithm with its LSE (and Delta) stored in bf16 (flash_attn.py:144,190)
    tdq, tdk, tdv = _tiled_grads(q, k, v, do, "causal", stats_in_dtype=True)
    for n, g, tw, w in (("dQ", dq, tdq, wdq), ("dK", dk, tdk, wdk), ("dV", dv, tdv, wdv)):
        assert_close(f"{n} vs tiled reference algorithm (bf16 LSE)", to_np(g), tw, BF16_TOL)
        assert_close(f"{n} vs float64", to_np(g), w, SANITY)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("mname", ["none", "causal", "sliding"])
def test_backward_stages_one_at_a_time(mname, dtype):
    """flash_attention_bwd_preprocess / _dkv / _dq on flattened (B*H, T, D)
    arrays (flash_attn.py:176-407) give flash_attention_bwd's gradients and
    the oracle's."""
    import math
    import torch
    pf = _pf()
    B, H, T, D = 2, 2, 192, 64
    q, k, v, do = inputs(zlib.crc32(("stages" + mname).encode()), B, H, H, T, T, D, dtype)
    tq, tk, tv, tdo = (to_torch(x, dtype) for x in (q, k, v, do))
    mm = _mask(pf, mname)
    o, lse = pf.flash_attention_fwd(tq, tk, tv, mask_mod=mm)
    flat = lambda t: t.reshape(B * H, T, *t.shape[3:])
    delta = pf.flash_attention_bwd_preprocess(flat(o), flat(tdo))
    assert delta.shape == (B * H, T)
    want_delta = (o.float() * tdo.float()).sum(-1).reshape(B * H, T)
    assert_close("Delta", to_np(delta), to_np(want_delta), dict(atol=1e-4, rtol=1e-4))
    sc = 1.0 / math.sqrt(D)
    dk, dv = pf.flash_attention_bwd_dkv(flat(tq), flat(tk), flat(tv), flat(tdo), flat(lse), delta, sc, sc,
                                        mask_mod=mm)
    dq = pf.flash_attention_bwd_dq(flat(tq), flat(tk), flat(tv), flat(tdo), flat(lse), delta, sc, sc, mask_mod=mm)
    assert dq.shape == (B * H, T, D) and dk.shape == (B * H, T, D)
    rdq, rdk, rdv = pf.flash_attention_bwd(tq, tk, tv, o, lse, tdo, mask_mod=mm)
    torch.cuda.synchronize()
    for n, a, b in (("dQ", dq, rdq), ("dK", dk, rdk), ("dV", dv, rdv)):
        assert torch.equal(a.reshape(b.shape), b), f"{n}: staged and whole backward differ"
    _, _, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, _omask(mname, T))
    if dtype == "fp32":
        for n, g, w in (("dQ", dq, wdq), ("dK", dk, wdk), ("dV", dv, wdv)):
            assert_close(n, to_np(g).reshape(w.shape), w, FP32_TOL)
        return
    # bf16: at 2e-2 against the reference's tiled algorithm restated with the
    # kernels' own cast points (P and dS rounded to bf16, the softmax scale
    # applied after dS's rounding), float64 as the sanity bound
    from oracle import tiled
    to_, tl = tiled.fwd(q, k, v, 64, 64, window=_window(mname), bf16=True, stats_in_dtype=False)
    tg = tiled.bwd(q, k, v, to_, tl, do, 64, 64, window=_window(mname), bf16=True, stats_in_dtype=False,
                   ds_scale_after=True)
    for n, g, t, w in (("dQ", dq, tg[0], wdq), ("dK", dk, tg[1], wdk), ("dV", dv, tg[2], wdv)):
        assert_close(f"{n} vs tiled (kernel cast points)", to_np(g).reshape(w.shape), t, BF16_TOL)
        assert_close(f"{n} vs float64", to_np(g).reshape(w.shape), w, SANITY)


@pytest.mark.parametrize("mname", ["none", "causal", "sliding"])
def test_mha_reference_matches_oracle(mname):
    """pf.mha_reference (flash_attn.py:33-56) in float32 on the GPU, plus GQA
    inputs (repeated kv heads)."""
    pf = _pf()
    B, H, T, D = 2, 4, 128, 64
    q, k, v, _ = inputs(5, B, H, H, T, T, D, "fp32")
    o = pf.mha_reference(*(to_torch(x, "fp32") for x in (q, k, v)), mask_mod=_mask(pf, mname))
    wo, _, _ = oracle_fwd_bwd(q, k, v, None, _omask(mname, T), bwd=False)
    assert_close("mha_reference", to_np(o), wo, dict(atol=2e-5, rtol=2e-5))
    qg, kg, vg, _ = inputs(6, 1, 8, 2, T, T, D, "fp32")
    og = pf.mha_reference(*(to_torch(x, "fp32") for x in (qg, kg, vg)), mask_mod=_mask(pf, mname))
    wog, _, _ = oracle_fwd_bwd(qg, kg, vg, None, _omask(mname, T), bwd=False)
    assert_close("mha_reference GQA", to_np(og), wog, dict(atol=2e-5, rtol=2e-5))


BLOCK_M64_CASES = [
    # name, dtype, B, H, S, D, mask, q scale, key ramp
    ("causal-bf16-d128", "bf16", 2, 4, 256, 128, "causal", 1.0, 0.0),
    ("dense-bf16-d64-ragged", "bf16", 1, 2, 200, 64, "none", 1.0, 0.0),
    ("window-bf16-d128", "bf16", 1, 2, 512, 128, "window", 1.0, 0.0),
    ("rescale-causal-bf16-d128", "bf16", 1, 2, 512, 128, "causal", 2.0, 3.0),
    ("causal-fp32-d64", "fp32", 1, 2, 256, 64, "causal", 1.0, 0.0),
]


@pytest.mark.parametrize("case", BLOCK_M64_CASES, ids=[c[0] for c in BLOCK_M64_CASES])
def test_block_m64_tile(case):
    """The 64-query tile (two waves per workgroup) forward, dQ and dK/dV, including the forward's
    exact rescale path (row maxima rising along the kv walk)."""
    import torch
    pf = _pf()
    name, dtype, B, H, S, D, mname, qscale, ramp = case
    print(f"[gpu ref-api] BLOCK_M=64 {name}", flush=True)
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 991, B, H, H, S, S, D, "fp32")
    q = q * qscale
    k = k * (1.0 + ramp * np.arange(S, dtype=np.float32) / S)[None, None, :, None]
    if dtype == "bf16":
        from oracle.bf16 import round_bf16
        q, k, v, do = (round_bf16(x) for x in (q, k, v, do))
    mm = {"causal": pf.causal_mask, "none": None, "window": pf.sliding_window_mask(100, 0)}[mname]
    om = {"causal": oracle_mask("causal", S, S), "none": None,
          "window": oracle_mask("window", S, S, 1, 100, 0)}[mname]
    bm = pf.create_block_mask(mm, B, H, S, S, 128) if mm is not None else None
    tq, tk, tv = (to_torch(x, dtype).requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, block_mask=bm, return_lse=True, kernel_options={"BLOCK_M": 64})
    o.backward(to_torch(do, dtype))
    torch.cuda.synchronize()
    wo, wl, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, om)
    tol = FP32_TOL if dtype == "fp32" else BF16_TOL
    assert_close("O", to_np(o), wo, tol)
    assert_close("LSE", to_np(lse), wl, tol)
    got = {"dQ": to_np(tq.grad), "dK": to_np(tk.grad), "dV": to_np(tv.grad)}
    if dtype == "fp32":
        for n, w in (("dQ", wdq), ("dK", wdk), ("dV", wdv)):
            assert_close(n, got[n], w, tol)
        return
    from oracle import tiled
    win = {"causal": (-1, 0), "none": None, "window": (100, 0)}[mname]
    to, tl = tiled.fwd(q, k, v, 64, 64, window=win, bf16=True, stats_in_dtype=False)
    tdq, tdk, tdv = tiled.bwd(q, k, v, to, tl, do, 64, 64, window=win, bf16=True, stats_in_dtype=False)
    for n, tw, w in (("dQ", tdq, wdq), ("dK", tdk, wdk), ("dV", tdv, wdv)):
        if ramp == 0.0:
            assert_close(f"{n} vs tiled reference algorithm", got[n], tw, BF16_TOL)
            assert_close(f"{n} vs float64", got[n], w, SANITY)
        else:  # large logits: the algorithm's bf16 roundings set the error (see test_gpu_parity)
            assert_close(f"{n} vs float64", got[n], w, dict(atol=1e-1, rtol=1e-2))
            assert_as_accurate(n, got[n], tw, w)


def test_empty_problems_launch_nothing():
    """GPU tensors without queries give empty outputs and gradients; without
    keys every row sees nothing: O = 0, LSE = -inf, zero gradients."""
    import torch
    import pallas_flexattn as pf
    print("[gpu reference api] empty problems", flush=True)
    x = torch.zeros(2, 2, 0, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    o = pf.flash_attention(x, x, x, mask_mod=pf.causal_mask)
    o.sum().backward()
    assert o.shape == (2, 2, 0, 64) and x.grad.shape == x.shape
    q = torch.randn(1, 4, 7, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    kv = torch.zeros(1, 2, 0, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    o, lse = pf.flex_attention(q, kv, kv, enable_gqa=True, return_lse=True)
    o.sum().backward()
    torch.cuda.synchronize()
    assert not o.any() and bool(torch.isneginf(lse).all())
    assert not q.grad.any() and kv.grad.shape == kv.shape
