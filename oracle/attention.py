"""Materialised attention in float64 — the numerical oracle.

``forward`` restates ``mha_reference`` (``flash_attn.py:33-56``):
``softmax(where(mask, q k^T / sqrt(d), -inf)) v``, extended with the pieces
the MI355X build adds on top of the reference:

* an explicit ``scale`` (default ``1/sqrt(D)`` as at ``flash_attn.py:46``),
* score modifications applied after scaling and before masking, in the order
  ALiBi bias ``s += slope[h] * (kv - q)`` then tanh soft-cap
  ``s = cap * tanh(s / cap)``,
* grouped-query attention: query head ``h`` reads kv head ``h // (Hq // Hkv)``.

``backward`` is the analytic gradient of ``sum(forward(...) * do)``; it is
pinned by finite differences in the tests, not by the reference (whose own
gradient comes from ``jax.grad`` of ``mha_reference``, ``tests/test_flash_attn.py:117-135``).

Rows whose every key is masked produce output 0 and log-sum-exp -inf.

Arrays are processed one (b, h) head at a time to bound memory.
"""
import numpy as np


def _as64(x):
    return np.asarray(x, dtype=np.float64)


def _scores(qh, kh, scale, h, Hq, alibi_slopes, softcap, score_fn=None, b=0):
    """Return (s_final, d s_final / d s or None) for one head, float64 (Sq, Skv)."""
    s = (qh @ kh.T) * scale
    sq, skv = s.shape
    if score_fn is not None:
        return score_fn(s, b, h, np.arange(sq)[:, None], np.arange(skv)[None, :])
    if alibi_slopes is not None:
        s = s + float(alibi_slopes[h]) * (np.arange(skv)[None, :] - np.arange(sq)[:, None]).astype(np.float64)
    th = None
    if softcap is not None and softcap > 0:
        th = np.tanh(s / softcap)
        s = softcap * th
    return s, (None if th is None else 1.0 - th * th)


def _mask_for(mask, b, h, sq, skv):
    if mask is None:
        return None
    if callable(mask):
        return np.broadcast_to(mask(b, h, np.arange(sq)[:, None], np.arange(skv)[None, :]), (sq, skv))
    m = np.asarray(mask, dtype=bool)
    if m.ndim == 2:
        return m
    return m[b if m.shape[0] > 1 else 0, h if m.shape[1] > 1 else 0]


def _softmax_rows(s):
    m = np.max(s, axis=-1, keepdims=True)
    dead = ~np.isfinite(m)
    m = np.where(dead, 0.0, m)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    p = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)
    lse = np.where(l[:, 0] > 0, m[:, 0] + np.log(np.where(l[:, 0] > 0, l[:, 0], 1.0)), -np.inf)
    return p, lse


def forward(q, k, v, mask=None, scale=None, alibi_slopes=None, softcap=None, score_fn=None):
    """q (B,Hq,Sq,D), k/v (B,Hkv,Skv,D) -> (o float64 (B,Hq,Sq,D), lse float64 (B,Hq,Sq)).

    ``mask`` is None, a boolean array (Sq,Skv) or (B|1,H|1,Sq,Skv), or a
    callable ``mask(b, h, q_idx, kv_idx) -> bool``.  ``score_fn(s, b, h,
    q_idx, kv_idx) -> (s', d s' / d s)`` (float64 arrays) replaces ALiBi /
    soft-cap with an arbitrary score modification of s = scale * q.k.
    """
    q, k, v = _as64(q), _as64(k), _as64(v)
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    g = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else float(scale)
    o = np.zeros((B, Hq, Sq, v.shape[-1]))
    lse = np.zeros((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            s, _ = _scores(q[b, h], k[b, h // g], scale, h, Hq, alibi_slopes, softcap, score_fn, b)
            m = _mask_for(mask, b, h, Sq, Skv)
            if m is not None:
                s = np.where(m, s, -np.inf)
            p, lse[b, h] = _softmax_rows(s)
            o[b, h] = p @ v[b, h // g]
    return o, lse


def backward(q, k, v, do, mask=None, scale=None, alibi_slopes=None, softcap=None, score_fn=None):
    """Gradients of sum(forward(q,k,v) * do) w.r.t. q, k, v (float64)."""
    q, k, v, do = _as64(q), _as64(k), _as64(v), _as64(do)
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    g = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else float(scale)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        for h in range(Hq):
            kh, vh = k[b, h // g], v[b, h // g]
            s, dsds = _scores(q[b, h], kh, scale, h, Hq, alibi_slopes, softcap, score_fn, b)
            m = _mask_for(mask, b, h, Sq, Skv)
            if m is not None:
                s = np.where(m, s, -np.inf)
            p, _ = _softmax_rows(s)
            o = p @ vh
            dv[b, h // g] += p.T @ do[b, h]
            dp = do[b, h] @ vh.T
            delta = np.sum(o * do[b, h], axis=-1, keepdims=True)
            ds = p * (dp - delta)
            if dsds is not None:
                ds = np.where(p > 0, ds * dsds, 0.0)
            ds = ds * scale
            dq[b, h] = ds @ kh
            dk[b, h // g] += ds.T @ q[b, h]
    return dq, dk, dv


def repeat_kv(x, n_rep):
    """(B,Hkv,S,D) -> (B,Hkv*n_rep,S,D), kv head j serving query heads j*n_rep .. j*n_rep+n_rep-1."""
    return np.repeat(np.asarray(x), n_rep, axis=1)
