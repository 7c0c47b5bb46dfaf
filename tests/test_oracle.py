"""Pins for the oracle itself (CPU only): each check is independent of the
formula it tests — closed forms, invariants, finite differences, a second
implementation (the C tiled restatement), or torch's own bf16 conversion."""
import numpy as np
import pytest

from oracle import attention, masks, tiled
from oracle.bf16 import from_bf16_bits, round_bf16, to_bf16_bits


# ---------------------------------------------------------------- bf16 ----
def test_round_bf16_known_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 spacing at 1.0
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, 0.0, np.inf], np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2 * ulp, 1.0 + ulp, -2.5, 0.0, np.inf], np.float32)
    np.testing.assert_array_equal(round_bf16(vals), want)  # ties go to even
    assert np.isnan(round_bf16(np.array([np.nan], np.float32)))[0]
    assert one == round_bf16(one)


def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 10
    t = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_bf16(x), t)
    np.testing.assert_array_equal(from_bf16_bits(to_bf16_bits(x)), t)


# ------------------------------------------------------------ forward -----
def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_constant_v_gives_constant_output():
    q, k = _rand((1, 2, 33, 16), 0), _rand((1, 2, 33, 16), 1)
    v = np.full((1, 2, 33, 16), 3.25)
    o, _ = attention.forward(q, k, v, mask=masks.dense(masks.causal, 33, 33))
    np.testing.assert_allclose(o, 3.25, rtol=0, atol=1e-12)


def test_causal_first_query_sees_only_first_key():
    q, k, v = (_rand((2, 3, 20, 8), s) for s in range(3))
    o, lse = attention.forward(q, k, v, mask=masks.dense(masks.causal, 20, 20))
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], atol=1e-12)
    np.testing.assert_allclose(lse[:, :, 0], np.einsum("bhd,bhd->bh", q[:, :, 0], k[:, :, 0]) / np.sqrt(8),
                               atol=1e-12)


def test_one_hot_key_dominates():
    q = np.zeros((1, 1, 4, 8))
    q[..., 0] = 100.0
    k = np.zeros((1, 1, 6, 8))
    k[0, 0, 3, 0] = 10.0
    v = _rand((1, 1, 6, 8), 5)
    o, _ = attention.forward(q, k, v)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0, 3], (4, 8)), atol=1e-12)


def test_lse_matches_logsumexp_and_batch_head_permutation():
    from scipy.special import logsumexp
    q, k, v = (_rand((2, 3, 17, 8), s) for s in range(3))
    m = masks.dense(masks.sliding_window(4, 2), 17, 17)
    o, lse = attention.forward(q, k, v, mask=m)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) / np.sqrt(8)
    np.testing.assert_allclose(lse, logsumexp(np.where(m, s, -np.inf), axis=-1), atol=1e-12)
    perm_b, perm_h = [1, 0], [2, 0, 1]
    o2, _ = attention.forward(q[perm_b][:, perm_h], k[perm_b][:, perm_h], v[perm_b][:, perm_h], mask=m)
    np.testing.assert_allclose(o2, o[perm_b][:, perm_h], atol=1e-12)


def test_fully_masked_row_is_zero():
    q, k, v = (_rand((1, 1, 4, 8), s) for s in range(3))
    m = np.ones((4, 4), bool)
    m[2] = False
    o, lse = attention.forward(q, k, v, mask=m)
    assert np.all(o[0, 0, 2] == 0) and lse[0, 0, 2] == -np.inf


def test_gqa_equals_repeated_kv():
    q = _rand((2, 6, 12, 8), 0)
    k, v, do = _rand((2, 2, 12, 8), 1), _rand((2, 2, 12, 8), 2), _rand((2, 6, 12, 8), 3)
    m = masks.dense(masks.causal, 12, 12)
    o, lse = attention.forward(q, k, v, mask=m)
    kr, vr = attention.repeat_kv(k, 3), attention.repeat_kv(v, 3)
    o2, lse2 = attention.forward(q, kr, vr, mask=m)
    np.testing.assert_allclose(o, o2, atol=1e-12)
    dq, dk, dv = attention.backward(q, k, v, do, mask=m)
    dq2, dk2, dv2 = attention.backward(q, kr, vr, do, mask=m)
    np.testing.assert_allclose(dq, dq2, atol=1e-12)
    np.testing.assert_allclose(dk, dk2.reshape(2, 2, 3, 12, 8).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv, dv2.reshape(2, 2, 3, 12, 8).sum(2), atol=1e-12)


def test_score_fn_reduces_to_alibi_and_softcap():
    """score_fn with the ALiBi + soft-cap formula gives the built-in mods' results exactly."""
    q, k, v, do = (_rand((1, 2, 9, 4), s) for s in range(4))
    slopes = np.array([1.0, 0.25])

    def fn(s, b, h, qi, ki):
        t = np.tanh((s + slopes[h] * (ki - qi)) / 5.0)
        return 5.0 * t, 1.0 - t * t
    a = attention.forward(q, k, v, alibi_slopes=slopes, softcap=5.0)
    c = attention.forward(q, k, v, score_fn=fn)
    np.testing.assert_allclose(a[0], c[0], atol=1e-13)
    ga = attention.backward(q, k, v, do, alibi_slopes=slopes, softcap=5.0)
    gc = attention.backward(q, k, v, do, score_fn=fn)
    for x, y in zip(ga, gc):
        np.testing.assert_allclose(x, y, atol=1e-13)


def test_score_mods_match_direct_formula():
    q, k, v = (_rand((1, 2, 9, 4), s) for s in range(3))
    slopes = np.array([1.0, 0.25])
    o, _ = attention.forward(q, k, v, alibi_slopes=slopes, softcap=5.0)
    for h in range(2):
        s = q[0, h] @ k[0, h].T / 2.0
        s = s + slopes[h] * (np.arange(9)[None, :] - np.arange(9)[:, None])
        s = 5.0 * np.tanh(s / 5.0)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        np.testing.assert_allclose(o[0, h], p @ v[0, h], atol=1e-12)


# ----------------------------------------------------------- backward -----
def _capped_bias(s, b, h, q, kv):
    t = np.tanh(s / 3.0)
    return 3.0 * t + 0.05 * h * (kv - q), 1.0 - t * t


def _quadratic(s, b, h, q, kv):
    return 0.1 * s * s + s + 0.01 * (q % 3), 0.2 * s + 1.0


@pytest.mark.parametrize("mods", [dict(), dict(alibi_slopes=np.array([0.5, 0.125, 1.0, 2.0]), softcap=3.0),
                                  dict(score_fn=_capped_bias), dict(score_fn=_quadratic)])
def test_backward_matches_finite_differences(mods):
    B, Hq, Hkv, S, D = 1, 4, 2, 7, 5
    q, do = _rand((B, Hq, S, D), 0), _rand((B, Hq, S, D), 3)
    k, v = _rand((B, Hkv, S, D), 1), _rand((B, Hkv, S, D), 2)
    m = masks.dense(masks.sliding_window(3, 1), S, S)

    def loss(q_, k_, v_):
        return np.sum(attention.forward(q_, k_, v_, mask=m, **mods)[0] * do)

    grads = attention.backward(q, k, v, do, mask=m, **mods)
    eps = 1e-6
    rng = np.random.default_rng(9)
    for gi, (x, g) in enumerate(zip((q, k, v), grads)):
        for _ in range(12):
            idx = tuple(rng.integers(0, n) for n in x.shape)
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[gi], args_m[gi] = xp, xm
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - g[idx]) < 1e-6 * max(1.0, abs(fd)), (gi, idx, fd, g[idx])


# ------------------------------------------------- C tiled restatement ----
@pytest.mark.parametrize("window,doc", [((-1, 0), False), ((32, 32), False), (None, False), ((-1, 0), True)])
def test_tiled_restatement_matches_naive_fp32(window, doc):
    B, H, T, D = 2, 2, 200, 32
    q, k, v, do = (np.random.default_rng(s).standard_normal((B, H, T, D)).astype(np.float32) for s in range(4))
    docs = np.repeat(np.arange(4), 50)[None].repeat(B, 0).astype(np.int32) if doc else None
    m = np.ones((T, T), bool) if window is None else masks.dense(masks.sliding_window(*window), T, T)
    full = np.stack([m & (docs[b][:, None] == docs[b][None, :]) if doc else m for b in range(B)])[:, None]
    o, lse = tiled.fwd(q, k, v, 64, 32, window=window, doc_ids=docs)
    wo, wl = attention.forward(q, k, v, mask=full)
    np.testing.assert_allclose(o, wo, atol=2e-6)
    np.testing.assert_allclose(lse, wl, atol=2e-6)
    grads = tiled.bwd(q, k, v, o, lse, do, 64, 32, window=window, doc_ids=docs)
    for g, w in zip(grads, attention.backward(q, k, v, do, mask=full)):
        np.testing.assert_allclose(g, w, atol=2e-5)


def test_tiled_restatement_bf16_cast_points_within_bf16_tolerance():
    B, H, T, D = 1, 2, 256, 64
    q, k, v, do = (round_bf16(np.random.default_rng(s).standard_normal((B, H, T, D)).astype(np.float32))
                   for s in range(4))
    o, lse = tiled.fwd(q, k, v, 64, 64, window=(-1, 0), bf16=True, stats_in_dtype=False)
    m = masks.dense(masks.causal, T, T)
    wo, wl = attention.forward(q, k, v, mask=m)
    np.testing.assert_allclose(o, wo, atol=2e-2, rtol=2e-2)
    assert np.all(o == round_bf16(o))  # output stored in bf16
    grads = tiled.bwd(q, k, v, o, lse, do, 64, 64, window=(-1, 0), bf16=True, stats_in_dtype=False)
    for g, w in zip(grads, attention.backward(q, k, v, do, mask=m)):
        np.testing.assert_allclose(g, w, atol=5e-2, rtol=5e-2)


def test_tiled_ds_scale_after_cast_point():
    """ds_scale_after moves only the softmax scale across the dS rounding: in
    float32 (no rounding) the gradients are identical, in bf16 dV (which never
    sees dS) is identical and dQ / dK stay within the bf16 tolerance of the
    reference's cast point, and the cast itself is exercised (dQ changes; D = 128
    makes the scale 2^-3.5, which is not exact in bf16 rounding)."""
    B, H, T, D = 1, 2, 192, 128
    q, k, v, do = (round_bf16(np.random.default_rng(10 + s).standard_normal((B, H, T, D)).astype(np.float32))
                   for s in range(4))
    for bf16 in (False, True):
        o, lse = tiled.fwd(q, k, v, 64, 64, window=(-1, 0), bf16=bf16, stats_in_dtype=False)
        a = tiled.bwd(q, k, v, o, lse, do, 64, 64, window=(-1, 0), bf16=bf16, stats_in_dtype=False)
        b = tiled.bwd(q, k, v, o, lse, do, 64, 64, window=(-1, 0), bf16=bf16, stats_in_dtype=False,
                      ds_scale_after=True)
        if not bf16:
            for x, y in zip(a, b):
                np.testing.assert_allclose(x, y, rtol=1e-6, atol=1e-7)
        else:
            assert np.array_equal(a[2], b[2])
            assert not np.array_equal(a[0], b[0])
            for x, y in zip(a[:2], b[:2]):
                np.testing.assert_allclose(x, y, atol=2e-2, rtol=2e-2)


# --------------------------------------------------------- golden data ----
def test_golden_fixture_reproduces():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "causal_fp32_b1h1s48d16.npz")
    g = np.load(path)
    o, lse = attention.forward(g["q"], g["k"], g["v"], mask=masks.dense(masks.causal, 48, 48))
    dq, dk, dv = attention.backward(g["q"], g["k"], g["v"], g["do"], mask=masks.dense(masks.causal, 48, 48))
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        np.testing.assert_allclose(got, g[name], atol=1e-6, err_msg=name)
