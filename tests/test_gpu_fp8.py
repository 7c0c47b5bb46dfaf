"""FP8 path on the GPU: the e4m3 block quantiser bit-exact against the
oracle's restatement (codes and scales), and the fp8 forward against float64
attention on the dequantised inputs (the same values the kernel multiplies).

The forward's only rounding beyond fp32 is P stored in e4m3 (3 mantissa
bits).  Every element of O is held to the worst case of that rounding
(``oracle.fp8.forward_model``'s bound: 2^-4 sum p |v| / l for normal values
plus the subnormal steps, whatever running maximum the kernel rounded
against) plus the bf16 rounding of O (2^-8 |O|) and 1e-4; the RMS error is
held within 1.3x of the model's (P rounded against the exact row maximum)
plus 1e-3.  S is exact (fp8 products, fp32 sums) and l sums the unrounded P,
so LSE is held to atol = rtol = 1e-4."""
import zlib

import numpy as np
import pytest

from _cases import inputs, oracle_mask, to_np, to_torch
from oracle import attention, fp8 as ofp8

pytestmark = pytest.mark.gpu


def _quant_np(x, transpose=False):
    B, H, S, D = x.shape
    codes, sc = ofp8.quantize_blocks(x.reshape(B * H, S, D), transpose)
    return codes.reshape((B, H) + codes.shape[1:]), sc.reshape(B, H, -1)


@pytest.mark.parametrize("S,D", [(300, 64), (128, 128), (1000, 128), (77, 32)])
def test_quantizer_bit_exact(S, D):
    import torch
    import pallas_flexattn as pf
    print(f"[gpu fp8] quantize S{S} D{D}", flush=True)
    rng = np.random.default_rng(S + D)
    x = rng.standard_normal((2, 3, S, D)).astype(np.float32)
    x[0, 1] *= 1e-4          # small magnitudes: negative exponents
    x[1, 2] *= 3000.0        # large ones
    x[1, 0, : min(S, 128)] = 0.0  # an all-zero block
    xb = to_torch(x, "bf16")
    xv = xb.float().cpu().numpy()  # the bf16 values the kernel reads
    for transpose in (False, True):
        t = pf.quantize_fp8(xb, transpose=transpose)
        torch.cuda.synchronize()
        codes, sc = _quant_np(xv, transpose)
        np.testing.assert_array_equal(t.scale.cpu().numpy(), sc)
        np.testing.assert_array_equal(t.data.cpu().numpy(), codes)


CASES = [
    # name, B, Hq, Hkv, Sq, Skv, D, mask, extras
    ("dense-ragged-d128", 1, 2, 2, 300, 300, 128, ("none",), {}),
    ("causal-d128", 2, 4, 4, 512, 512, 128, ("causal",), {}),
    ("causal-d64", 1, 4, 4, 384, 384, 64, ("causal",), {}),
    ("window-d128", 1, 2, 2, 640, 640, 128, ("window", 100, 20), {}),
    ("doc-causal-d128", 2, 2, 2, 512, 512, 128, ("doc",), {}),
    ("gqa-alibi-softcap-d128", 1, 8, 2, 384, 384, 128, ("causal",), {"alibi": True, "softcap": 30.0}),
    ("gqa-alibi-softcap-window-d64", 2, 4, 2, 320, 320, 64, ("window", 64, 0), {"alibi": True, "softcap": 20.0}),
    ("alibi-only-d128", 1, 4, 4, 256, 256, 128, ("causal",), {"alibi": True}),
    ("cross-d128", 1, 2, 2, 256, 704, 128, ("none",), {}),
]


def _doc_lengths(rng, S):
    out, tot = [], 0
    while tot < S:
        n = min(int(rng.integers(40, 200)), S - tot)
        out.append(n)
        tot += n
    return out


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fp8_forward(case):
    import torch
    import pallas_flexattn as pf
    name, B, Hq, Hkv, Sq, Skv, D, mspec, extras = case
    print(f"[gpu fp8] forward {name}", flush=True)
    q, k, v, _ = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, Sq, Skv, D, "bf16")
    kind = mspec[0]
    doc_ids = None
    if kind == "causal":
        mm = pf.causal_mask
    elif kind == "window":
        mm = pf.sliding_window_mask(mspec[1], mspec[2])
    elif kind == "doc":
        dm = pf.document_mask([_doc_lengths(np.random.default_rng(5 + b), Sq) for b in range(B)])
        doc_ids = dm.doc_ids
        mm = pf.and_masks(dm, pf.causal_mask)
    else:
        mm = None
    omask = oracle_mask("causal" if kind == "doc" else kind, Sq, Skv, B,
                        *(mspec[1:] if kind == "window" else ()), doc_ids=doc_ids)
    alibi = pf.alibi_slopes(Hq) if extras.get("alibi") else None
    softcap = extras.get("softcap")
    score = None
    if alibi is not None:
        score = pf.compose_score_mods(pf.alibi_score_mod(alibi), pf.softcap_score_mod(softcap))
    bm = pf.create_block_mask(mm, B, Hq, Sq, Skv, 128) if mm is not None else None
    tq, tk, tv = (to_torch(x, "bf16") for x in (q, k, v))
    q8, k8, v8 = pf.quantize_fp8(tq), pf.quantize_fp8(tk), pf.quantize_fp8(tv, transpose=True)
    o, lse = pf.flex_attention_fp8(q8, k8, v8, score_mod=score, block_mask=bm, enable_gqa=Hq != Hkv,
                                   return_lse=True)
    torch.cuda.synchronize()
    # the dequantised inputs: what the kernel multiplies
    qd, kd, vd = (to_np(pf.dequantize_fp8(t)) for t in (q8, k8, v8))
    want_o, want_lse = attention.forward(qd, kd, vd, mask=omask, alibi_slopes=alibi, softcap=softcap)
    model_o, _, bound = ofp8.forward_model(qd, kd, vd, omask, alibi_slopes=alibi, softcap=softcap, with_bound=True)
    _check_o(name, to_np(o), want_o, model_o, bound)
    np.testing.assert_allclose(to_np(lse), want_lse, atol=1e-4, rtol=1e-4)


def _check_o(name, got, want, model, bound):
    eg, em = np.abs(got - want), np.abs(model - want)
    lim = bound + 2.0 ** -8 * np.abs(want) + 1e-4
    bad = eg > lim
    rg, rm = np.sqrt((eg ** 2).mean()), np.sqrt((em ** 2).mean())
    assert not bad.any(), (f"{name}: {bad.sum()} O elements beyond the P-rounding bound; worst excess "
                           f"{(eg - lim).max():.3g} (error {eg.max():.3g})")
    assert rg <= 1.3 * rm + 1e-3, f"{name}: O RMS error {rg:.3g}, the P-rounding model's {rm:.3g}"


def test_fp8_forward_rescale_path():
    """Logits growing along the keys (the running maximum jumps between
    tiles, so tile sums exceed 448 and the exact path rescales) and logits
    with standard deviation ~30."""
    import torch
    import pallas_flexattn as pf
    from oracle.bf16 import round_bf16
    B, H, S, D = 1, 2, 512, 128
    for name, qs, ramp in (("growing", 2.0, 3.0), ("large", 30.0, 0.0)):
        print(f"[gpu fp8] rescale {name}", flush=True)
        q, k, v, _ = inputs(zlib.crc32(name.encode()) % 1000, B, H, H, S, S, D, "fp32")
        q = round_bf16(q * qs)
        k = round_bf16(k * (1.0 + ramp * np.arange(S, dtype=np.float32) / S)[None, None, :, None])
        v = round_bf16(v)
        q8, k8, v8 = (pf.quantize_fp8(to_torch(q, "bf16")), pf.quantize_fp8(to_torch(k, "bf16")),
                      pf.quantize_fp8(to_torch(v, "bf16"), transpose=True))
        bm = pf.create_block_mask(pf.causal_mask, B, H, S, S, 128)
        o, lse = pf.flex_attention_fp8(q8, k8, v8, block_mask=bm, return_lse=True)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(lse).all())
        qd, kd, vd = (to_np(pf.dequantize_fp8(t)) for t in (q8, k8, v8))
        om = oracle_mask("causal", S, S)
        want_o, want_lse = attention.forward(qd, kd, vd, mask=om)
        model_o, _, bound = ofp8.forward_model(qd, kd, vd, om, with_bound=True)
        _check_o(name, to_np(o), want_o, model_o, bound)
        # logits reach a few hundred here: the fp32 sums of 128 products carry
        # absolute errors of ~1e-4, so LSE gets atol 1e-3
        np.testing.assert_allclose(to_np(lse), want_lse, atol=1e-3, rtol=1e-4)


def test_fp8_rejections():
    """The fp8 dtype is refused by the bf16 / fp32 entry points, and the
    fp8 forward refuses head dim 32 and arbitrary document labels."""
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn import _lib
    x = torch.randn(1, 2, 128, 32, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pf.flex_attention_fp8(x, x, x)
    ids = np.random.default_rng(0).integers(0, 3, size=(1, 128)).astype(np.int32)
    x = torch.randn(1, 2, 128, 64, device="cuda", dtype=torch.bfloat16)
    bm = pf.create_block_mask(pf.document_ids_mask(ids), 1, 2, 128, 128, 128)
    with pytest.raises(_lib.FlexAttnError):
        pf.flex_attention_fp8(x, x, x, block_mask=bm)


def test_fp8_scales_must_be_powers_of_two():
    """The kernel reads only the exponent field of each block scale, so the
    binding refuses Fp8Tensor scales that are not powers of two in
    [2^-126, 2^127] (not powers of two, zero, subnormal, negative, inf),
    and accepts them again once fixed (the check follows in-place changes)."""
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn.fp8 import Fp8Tensor
    print("[gpu fp8] scale validation", flush=True)
    x = torch.randn(1, 2, 256, 64, device="cuda", dtype=torch.bfloat16)
    q8, k8, v8 = pf.quantize_fp8(x), pf.quantize_fp8(x), pf.quantize_fp8(x, transpose=True)
    pf.flex_attention_fp8(q8, k8, v8)
    for bad in (0.75, 0.0, 2.0 ** -130, -1.0, float("inf")):
        sc = k8.scale.clone()
        sc[0, 1, 1] = bad
        with pytest.raises(ValueError, match="powers of two"):
            pf.flex_attention_fp8(q8, Fp8Tensor(k8.data, sc, k8.seq_len, False), v8)
    sc = k8.scale.clone()
    sc[0, 0, 0] = 3.0
    kb = Fp8Tensor(k8.data, sc, k8.seq_len, False)
    with pytest.raises(ValueError, match="powers of two"):
        pf.flex_attention_fp8(q8, kb, v8)
    sc[0, 0, 0] = 4.0  # fixed in place: checked again, accepted
    pf.flex_attention_fp8(q8, kb, v8)
    torch.cuda.synchronize()
