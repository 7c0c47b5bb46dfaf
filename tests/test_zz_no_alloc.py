"""fa_bwd_noalloc (C ABI): the backward with its Delta scratch in a fixed
device array instead of a caller workspace.  Its outputs must equal
fa_bwd's bit for bit (same kernels, same Delta), on two calls in a row, the
second with a smaller problem (the array keeps the first call's contents),
and sizes beyond the array are rejected before any launch."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(B, Hq, Hkv, S, D, seed, mask):
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn import _lib
    from pallas_flexattn.flash_attn import _fwd_core, _stream
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    do = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
    bm = pf.create_block_mask(mask, B, Hq, S, S, 128) if mask is not None else None
    o, lse, plan = _fwd_core(q, k, v, mask, None, None, bm, (128, 64, 128))
    lib = _lib.load()
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ptrs = [t.data_ptr() for t in (q, k, v, o, lse, do, dq, dk, dv)]
        if noalloc:
            rc = lib.fa_bwd_noalloc(plan.ptr(), *ptrs, _stream())
        else:
            ws = torch.empty(lib.fa_bwd_workspace_bytes(plan.ptr()), device="cuda", dtype=torch.uint8)
            rc = lib.fa_bwd(plan.ptr(), *ptrs, ws.data_ptr(), ws.numel(), _stream())
        assert rc == 0, lib.fa_strerror(rc)
        outs.append((dq, dk, dv))
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), *outs):
        assert torch.equal(a, b), f"{name}: fa_bwd_noalloc differs from fa_bwd"
        assert bool(torch.isfinite(b).all())


def test_noalloc_matches_fa_bwd_two_calls():
    import pallas_flexattn as pf
    print("[gpu noalloc] B2 H8/4 S1024 D128 causal, then B1 H2 S320 D64 window", flush=True)
    _run(2, 8, 4, 1024, 128, 1, pf.causal_mask)
    _run(1, 2, 2, 320, 64, 2, pf.sliding_window_mask(100, 0))


def test_noalloc_rejects_oversize_before_launch():
    from pallas_flexattn import _lib
    lib = _lib.load()
    p = _lib.FaParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _lib.DTYPE_BF16
    limit = lib.fa_bwd_noalloc_max_rows()
    assert limit == 8 << 20
    p.B, p.Hq, p.Hkv, p.Sq, p.Skv, p.D = 1, 64, 64, limit // 64 + 128, 128, 128
    p.window_left = p.window_right = -1
    fake = [256] * 9  # never dereferenced: the size check comes first
    assert lib.fa_bwd_noalloc(ctypes.byref(p), *fake, None) == -9
    assert b"fa_bwd_noalloc_max_rows" in lib.fa_strerror(-9)
