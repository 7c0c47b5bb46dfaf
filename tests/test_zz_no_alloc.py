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


_CAPTURE_CHILD = r"""
import sys
import torch
sys.path[:0] = sys.argv[1:3]
import pallas_flexattn as pf
from pallas_flexattn import _lib
from pallas_flexattn.flash_attn import _fwd_core, _stream
B, Hq, Hkv, S, D = 2, 4, 2, 512, 128
g = torch.Generator(device="cuda").manual_seed(11)
q = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
k = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
v = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
do = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
bm = pf.create_block_mask(pf.causal_mask, B, Hq, S, S, 128)
# the first launching call of the process: the forward, eagerly
o, lse, plan = _fwd_core(q, k, v, pf.causal_mask, None, None, bm, (128, 64, 128))
lib = _lib.load()
ws = torch.empty(lib.fa_bwd_workspace_bytes(plan.ptr()), device="cuda", dtype=torch.uint8)
ref = [torch.empty_like(t) for t in (q, k, v)]
ptrs = lambda outs: [t.data_ptr() for t in (q, k, v, o, lse, do, *outs)]
assert lib.fa_bwd(plan.ptr(), *ptrs(ref), ws.data_ptr(), ws.numel(), _stream()) == 0
torch.cuda.synchronize()
got = [torch.zeros_like(t) for t in (q, k, v)]
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = lib.fa_bwd_noalloc(plan.ptr(), *ptrs(got), _stream())
assert rc == 0, rc
for rep in range(3):
    for t in got:
        t.zero_()
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager fa_bwd"
    # eager work between the replays: another backward through fa_bwd_noalloc
    # itself (same array) and through fa_bwd
    other = [torch.empty_like(t) for t in (q, k, v)]
    assert lib.fa_bwd_noalloc(plan.ptr(), *ptrs(other), _stream()) == 0
    assert lib.fa_bwd(plan.ptr(), *ptrs(other), ws.data_ptr(), ws.numel(), _stream()) == 0
    torch.cuda.synchronize()
print("capture ok")
"""


def test_noalloc_captured_in_a_graph_fresh_process():
    """In a fresh process whose first library call is the eager forward,
    fa_bwd_noalloc captured into a torch.cuda.graph replays bit-identical to
    the eager fa_bwd, three times, with eager backward calls (sharing the
    fixed array) between the replays."""
    import os
    import subprocess
    import sys
    print("[gpu noalloc] graph capture in a fresh process, B2 H4/2 S512 D128 causal", flush=True)
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root, os.path.join(root, "pallas-flexattn_amd")],
                         capture_output=True, text=True, timeout=100)
    assert res.returncode == 0 and "capture ok" in res.stdout, res.stderr[-4000:]
