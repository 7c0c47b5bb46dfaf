"""Shared helpers for the parity tests: seeded inputs, oracle evaluation and
tolerance checks.  The oracle is the float64 materialised attention in
``oracle/attention.py``; masks are materialised with the oracle's own
predicates (``oracle/masks.py``)."""
import numpy as np

from oracle import attention, masks as omasks
from oracle.bf16 import round_bf16

BF16_TOL = dict(atol=2e-2, rtol=2e-2)
FP32_TOL = dict(atol=1e-5, rtol=1e-5)


def inputs(seed, B, Hq, Hkv, Sq, Skv, D, dtype, scale=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, D), dtype=np.float32) * scale
    k = rng.standard_normal((B, Hkv, Skv, D), dtype=np.float32) * scale
    v = rng.standard_normal((B, Hkv, Skv, D), dtype=np.float32) * scale
    do = rng.standard_normal((B, Hq, Sq, D), dtype=np.float32)
    if dtype == "bf16":
        q, k, v, do = (round_bf16(x) for x in (q, k, v, do))
    return q, k, v, do


def oracle_mask(kind, Sq, Skv, B=1, left=-1, right=-1, doc_ids=None):
    """Dense (B, 1, Sq, Skv) boolean mask from the oracle's predicates."""
    if kind == "none":
        return None
    if kind == "causal":
        fn = omasks.causal
    elif kind == "window":
        fn = omasks.sliding_window(left, right)
    else:
        raise ValueError(kind)
    m = omasks.dense(fn, Sq, Skv)
    if doc_ids is not None:
        docs = np.asarray(doc_ids).reshape(-1, np.shape(doc_ids)[-1])
        out = np.stack([m & omasks.dense(omasks.same_document(docs[b]), Sq, Skv) for b in range(docs.shape[0])])
        return out[:, None]
    return m[None, None]


def to_torch(x, dtype, device="cuda"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(device=device, dtype=torch.bfloat16 if dtype == "bf16" else torch.float32)


def to_np(t):
    return t.detach().float().cpu().numpy()


def assert_close(name, got, want, tol):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    bound = tol["atol"] + tol["rtol"] * np.abs(want)
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - bound, -np.inf)), err.shape)
        raise AssertionError(f"{name}: {bad.sum()} / {bad.size} elements out of tolerance {tol}; "
                             f"worst at {i}: got {got[i]!r} want {want[i]!r} (max abs err {err.max():.3g})")


def oracle_fwd_bwd(q, k, v, do, mask, scale=None, alibi=None, softcap=None, bwd=True, score_fn=None):
    o, lse = attention.forward(q, k, v, mask=mask, scale=scale, alibi_slopes=alibi, softcap=softcap,
                               score_fn=score_fn)
    if not bwd:
        return o, lse, None
    return o, lse, attention.backward(q, k, v, do, mask=mask, scale=scale, alibi_slopes=alibi, softcap=softcap,
                                      score_fn=score_fn)


def assert_as_accurate(name, got, alg, exact, max_ratio=1.5, rms_ratio=1.25):
    """`got` is no further from `exact` than `alg` (the reference's algorithm
    restated with its bf16 cast points) is: max and RMS errors against the
    float64 result within the given ratios of the algorithm's own.  For inputs
    where the algorithm's bf16 roundings, not the implementation, set the
    error (large logits: dS values that cancel in the dQ / dK sums)."""
    got, alg, exact = (np.asarray(x, dtype=np.float64) for x in (got, alg, exact))
    eg, ea = np.abs(got - exact), np.abs(alg - exact)
    rg, ra = np.sqrt((eg ** 2).mean()), np.sqrt((ea ** 2).mean())
    if not (eg.max() <= max_ratio * ea.max() and rg <= rms_ratio * ra):
        raise AssertionError(f"{name}: error against float64 max {eg.max():.3g} / rms {rg:.3g}, the reference "
                             f"algorithm's max {ea.max():.3g} / rms {ra:.3g} (allowed x{max_ratio} / x{rms_ratio})")
