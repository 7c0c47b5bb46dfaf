"""GPU checks at the benchmark workloads' full sizes (C2 causal S=2048, C3 sliding window S=8192,
C4 GQA + ALiBi + soft-cap S=4096, C5 packed documents S=16384, causal S=8192).

The kernels run over every (batch, head); two (batch, kv-head) groups are then
recomputed whole by a float32 PyTorch attention (chunked over query rows, on
the GPU) and compared on O, LSE, dQ, dK, dV to the bf16 tolerance (atol = rtol
= 2e-2).  Over all heads, two identities that hold for any inputs are checked:
sum_k dV[k] = sum_q dO[q] over a kv head's group (rows of P sum to 1), and
sum_k dK[k] = 0 without a soft-cap (rows of dS sum to 0: sum_k P (dP - Delta)
= Delta - Delta), both relative to the magnitude of the summed terms."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


def _reference_group(cfg, q, k, v, do, b, hk, slopes, cap):
    """float32 attention forward + backward for the q heads of kv head hk of
    batch row b: returns O, LSE (per q head), dQ (per q head), dK, dV (summed
    over the group)."""
    import torch
    S, D = cfg["S"], cfg["D"]
    g = cfg["Hq"] // cfg["Hkv"]
    scale = 1.0 / np.sqrt(D)
    left, right = cfg["window"]
    docs = None if cfg["docs"] is None else torch.as_tensor(cfg["docs"][b], device="cuda")
    kk = k[b, hk].float().contiguous()
    vv = v[b, hk].float().contiguous()
    kidx = torch.arange(S, device="cuda")
    outs, lses, dqs = [], [], []
    dk = torch.zeros(S, D, device="cuda")
    dv = torch.zeros(S, D, device="cuda")
    chunk = 1024
    for h in range(hk * g, (hk + 1) * g):
        qq = q[b, h].float().contiguous()
        dd = do[b, h].float().contiguous()
        o_h, l_h, dq_h = [], [], []
        for r0 in range(0, S, chunk):
            qi = torch.arange(r0, min(r0 + chunk, S), device="cuda")
            s = (qq[qi] @ kk.t()) * scale
            if slopes is not None:
                s = s + float(slopes[h]) * (kidx[None, :] - qi[:, None]).float()
            dsdx = None
            if cap:
                t = torch.tanh(s / cap)
                s = cap * t
                dsdx = 1.0 - t * t
            delta = qi[:, None] - kidx[None, :]
            live = torch.ones_like(s, dtype=torch.bool)
            if left >= 0:
                live &= delta <= left
            if right >= 0:
                live &= -delta <= right
            if docs is not None:
                live &= docs[qi][:, None] == docs[None, :]
            s = s.masked_fill(~live, float("-inf"))
            lse = torch.logsumexp(s, dim=1)
            p = torch.exp(s - lse[:, None])
            o = p @ vv
            dp = dd[qi] @ vv.t()
            dl = (dd[qi] * o).sum(1)
            ds = p * (dp - dl[:, None])
            if dsdx is not None:
                ds = ds * dsdx
            dq_h.append((ds @ kk) * scale)
            dk += (ds.t() @ qq[qi]) * scale
            dv += p.t() @ dd[qi]
            o_h.append(o)
            l_h.append(lse)
        outs.append(torch.cat(o_h))
        lses.append(torch.cat(l_h))
        dqs.append(torch.cat(dq_h))
    return outs, lses, dqs, dk, dv


def _close(name, got, want):
    got = got.float()
    want = want.float()
    err = (got - want).abs()
    bound = TOL["atol"] + TOL["rtol"] * want.abs()
    bad = err > bound
    assert not bool(bad.any()), (f"{name}: {int(bad.sum())} of {bad.numel()} outside atol/rtol 2e-2, "
                                 f"max err {float(err.max()):.3g}")


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "ns"])
def test_fullsize_workload(name):
    import torch
    import bench
    import pallas_flexattn as pf
    print(f"[gpu fullsize] {name}", flush=True)
    cfg = bench.make_config(name)
    B, Hq, Hkv, S, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    arrays = bench.gen_inputs(cfg)
    q, k, v, do = (torch.from_numpy(a).to("cuda", torch.bfloat16) for a in arrays)
    del arrays
    bm = pf.create_block_mask(cfg["mask"], B, Hq, S, S, 128)
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()
    o, lse = pf.flex_attention(q, k, v, score_mod=cfg["score"], block_mask=bm, enable_gqa=Hq != Hkv,
                               return_lse=True)
    o.backward(do)
    torch.cuda.synchronize()
    dq, dk, dv = q.grad, k.grad, v.grad
    assert all(bool(torch.isfinite(t).all()) for t in (o, lse, dq, dk, dv))

    # identities over every head
    g = Hq // Hkv
    sum_do = do.float().view(B, Hkv, g, S, D).sum(dim=(2, 3))
    sum_dv = dv.float().sum(dim=2)
    scale_dv = do.float().abs().view(B, Hkv, g, S, D).sum(dim=(2, 3))
    rel_dv = float(((sum_dv - sum_do).abs() / scale_dv.clamp_min(1.0)).max())
    assert rel_dv < 2e-2, f"sum_k dV != sum_q dO (max relative {rel_dv:.3g})"
    if cfg["score"] is None or not cfg["score"].softcap:  # the soft-cap's chain factor breaks it
        sum_dk = dk.float().sum(dim=2)
        scale_dk = dk.float().abs().sum(dim=2)
        rel_dk = float((sum_dk.abs() / scale_dk.clamp_min(1e-3)).max())
        assert rel_dk < 2e-2, f"sum_k dK != 0 (max relative {rel_dk:.3g})"

    # two (batch, kv head) groups recomputed whole
    slopes = None
    cap = None
    if cfg["score"] is not None:
        slopes = cfg["score"].alibi
        cap = cfg["score"].softcap or None
    for b, hk in ((0, 0), (B - 1, Hkv - 1)):
        outs, lses, dqs, rdk, rdv = _reference_group(cfg, q.detach(), k.detach(), v.detach(), do, b, hk, slopes, cap)
        for i, h in enumerate(range(hk * g, (hk + 1) * g)):
            _close(f"{name} O[{b},{h}]", o[b, h], outs[i])
            _close(f"{name} LSE[{b},{h}]", lse[b, h], lses[i])
            _close(f"{name} dQ[{b},{h}]", dq[b, h], dqs[i])
        _close(f"{name} dK[{b},{hk}]", dk[b, hk], rdk)
        _close(f"{name} dV[{b},{hk}]", dv[b, hk], rdv)
