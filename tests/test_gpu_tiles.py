"""Every tile configuration the tuner can pick (BLOCK_M x BLOCK_N x BLOCK_KV x
BLOCK_Q x NUM_STAGES of the bf16 kernels: 2, 4 or 8 waves per forward / dQ
workgroup, 32, 64 or 128 keys per LDS tile, 1, 2 or 3 K / V tiles in LDS,
2 or 4 waves per dK/dV workgroup, 64 or 128 queries per dK/dV tile) on the
GPU, forward and backward through flex_attention's kernel_options, against the float64
oracle at bf16 atol = rtol = 2e-2.  The masks rotate over the tile sets so
each set meets a different one (causal, window, contiguous documents, none
with ragged lengths, Sq != Skv), with GQA and ALiBi + soft-cap on some; the
forward's rescale path runs once per forward tile."""
import zlib

import numpy as np
import pytest

from _cases import BF16_TOL, assert_close, inputs, oracle_fwd_bwd, oracle_mask, to_np, to_torch

pytestmark = pytest.mark.gpu


def _tile_sets():
    from pallas_flexattn.kernel_tuner import candidate_tiles
    return [(d, t) for d in (128, 64) for t in candidate_tiles("bf16", d)]


MASKS = ["causal", "window", "doc", "none", "causal-gqa-mods", "cross"]


def _case(i, D, tiles):
    return (f"d{D}-{'x'.join(map(str, tiles))}-{MASKS[i % len(MASKS)]}", D, tiles, MASKS[i % len(MASKS)])


CASES = [_case(i, d, t) for i, (d, t) in enumerate(_tile_sets())]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_tiles_fwd_bwd(case):
    import torch
    import pallas_flexattn as pf
    name, D, tiles, kind = case
    print(f"[gpu tiles] {name}", flush=True)
    B, Hq, Hkv, Sq, Skv = 1, 4, 4, 640, 640
    if kind == "causal-gqa-mods":
        Hq, Hkv, Sq, Skv = 8, 2, 512, 512
    if kind == "none":
        Sq = Skv = 600  # ragged: the last q and kv tiles are partial
    if kind == "cross":
        Sq, Skv = 384, 704
    q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, Sq, Skv, D, "bf16")
    doc_ids = None
    alibi = softcap = score = None
    if kind in ("causal", "causal-gqa-mods"):
        mm, omask = pf.causal_mask, oracle_mask("causal", Sq, Skv)
    elif kind == "window":
        mm, omask = pf.sliding_window_mask(100, 20), oracle_mask("window", Sq, Skv, 1, 100, 20)
    elif kind == "doc":
        rng = np.random.default_rng(3)
        lens, tot = [], 0
        while tot < Sq:
            n = min(int(rng.integers(40, 200)), Sq - tot)
            lens.append(n)
            tot += n
        dm = pf.document_mask([lens])
        doc_ids = dm.doc_ids
        mm = pf.and_masks(dm, pf.causal_mask)
        omask = oracle_mask("causal", Sq, Skv, B, doc_ids=doc_ids)
    else:
        mm, omask = None, oracle_mask("none", Sq, Skv)
    if kind == "causal-gqa-mods":
        alibi, softcap = pf.alibi_slopes(Hq), 30.0
        score = pf.compose_score_mods(pf.alibi_score_mod(alibi), pf.softcap_score_mod(softcap))
    bm = pf.create_block_mask(mm, B, Hq, Sq, Skv, 128) if mm is not None else None
    from pallas_flexattn.kernel_tuner import TILE_NAMES
    opts = dict(zip(TILE_NAMES, tiles))
    tq, tk, tv = (to_torch(x, "bf16").requires_grad_() for x in (q, k, v))
    o, lse = pf.flex_attention(tq, tk, tv, score_mod=score, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True,
                               kernel_options=opts)
    o.backward(to_torch(do, "bf16"))
    torch.cuda.synchronize()
    want_o, want_lse, (wdq, wdk, wdv) = oracle_fwd_bwd(q, k, v, do, omask, alibi=alibi, softcap=softcap)
    for nm, got, want in (("O", o, want_o), ("LSE", lse, want_lse), ("dQ", tq.grad, wdq), ("dK", tk.grad, wdk),
                          ("dV", tv.grad, wdv)):
        assert_close(f"{name} {nm}", to_np(got), want, BF16_TOL)


FWD_TILES = [(128, 32, 2), (128, 32, 3), (128, 128, 2), (128, 128, 1), (256, 64, 2), (64, 64, 2)]


@pytest.mark.parametrize("fwd_tiles", FWD_TILES, ids=[f"{a}x{b}s{c}" for a, b, c in FWD_TILES])
def test_tiles_forward_rescale_path(fwd_tiles):
    """Logits growing along the keys (the running maximum rises by more than
    16 in log2 units between tiles) and huge logits (exponentials overflow
    before the exact path replaces them): O and LSE against float64."""
    import torch
    import pallas_flexattn as pf
    from oracle.bf16 import round_bf16
    B, H, S, D = 1, 2, 512, 128
    opts = {"BLOCK_M": fwd_tiles[0], "BLOCK_N": fwd_tiles[1], "NUM_STAGES": fwd_tiles[2]}
    for name, kind, qscale, ramp in (("growing-causal", "causal", 2.0, 3.0), ("huge-dense", None, 64.0, 0.0)):
        print(f"[gpu tiles] rescale {name} {fwd_tiles}", flush=True)
        q, k, v, do = inputs(zlib.crc32(name.encode()) % 1000, B, H, H, S, S, D, "fp32")
        q = round_bf16(q * qscale)
        k = round_bf16(k * (1.0 + ramp * np.arange(S, dtype=np.float32) / S)[None, None, :, None])
        v = round_bf16(v)
        bm = pf.create_block_mask(pf.causal_mask, B, H, S, S, 128) if kind == "causal" else None
        with torch.no_grad():
            o, lse = pf.flex_attention(to_torch(q, "bf16"), to_torch(k, "bf16"), to_torch(v, "bf16"), block_mask=bm,
                                       return_lse=True, kernel_options=opts)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(lse).all())
        want_o, want_lse, _ = oracle_fwd_bwd(q, k, v, do, oracle_mask(kind or "none", S, S), bwd=False)
        assert_close(f"{name} O", to_np(o), want_o, BF16_TOL)
        assert_close(f"{name} LSE", to_np(lse), want_lse, BF16_TOL)


def test_tiles_reach_the_c_abi():
    """kernel_options reach fa_params (a tile with no kernel is refused by
    the library, not silently replaced), and tables built at 128 are
    re-derived at 256 for 256-row query tiles."""
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn import _lib
    q = torch.randn(1, 2, 256, 32, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(_lib.FlexAttnError):
        pf.flex_attention(q, q, q, kernel_options={"BLOCK_M": 128, "BLOCK_N": 128})  # D = 32: 64-key tiles only
    x = torch.randn(1, 2, 256, 64, device="cuda", dtype=torch.bfloat16)
    for bad in ({"NUM_STAGES": 3}, {"BLOCK_N": 128, "NUM_STAGES": 3}, {"BLOCK_N": 32, "NUM_STAGES": 1},
                {"BLOCK_Q": 96}):
        with pytest.raises(_lib.FlexAttnError):  # stage counts / q tiles without an instantiation
            pf.flex_attention(x, x, x, kernel_options=bad)
    xr = x.detach().requires_grad_()
    with pytest.raises(_lib.FlexAttnError):  # 128-query dK/dV tiles need 128-key dK/dV workgroups
        pf.flex_attention(xr, xr, xr, kernel_options={"BLOCK_KV": 64, "BLOCK_Q": 128}).sum().backward()
    q = torch.randn(1, 2, 512, 128, device="cuda", dtype=torch.bfloat16)
    bm = pf.create_block_mask(pf.causal_mask, 1, 2, 512, 512, 128)
    a = pf.flex_attention(q, q, q, block_mask=bm, kernel_options={"BLOCK_M": 256})
    b = pf.flex_attention(q, q, q, block_mask=bm)
    torch.cuda.synchronize()
    assert float((a.float() - b.float()).abs().max()) < 2e-2
