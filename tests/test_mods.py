"""Mask and score descriptors (CPU): their host evaluation against the
oracle's restatement of the reference predicates and closed forms."""
import numpy as np
import pytest

import pallas_flexattn as pf
from oracle import masks as om

Q = np.arange(40)[:, None]
K = np.arange(40)[None, :]


@pytest.mark.parametrize("mm,omm", [
    (pf.causal_mask, om.causal), (pf.bidirectional_mask, om.bidirectional),
    (pf.sliding_window_mask(3, 5), om.sliding_window(3, 5)), (pf.sliding_window_mask(-1, 2), om.sliding_window(-1, 2)),
    (pf.sliding_window_mask(7, -1), om.sliding_window(7, -1)), (pf.sliding_window_mask(0, 0), om.sliding_window(0, 0)),
])
def test_mask_specs_match_reference_predicates(mm, omm):
    np.testing.assert_array_equal(np.broadcast_to(mm(Q, K), (40, 40)), np.broadcast_to(omm(Q, K), (40, 40)))
    np.testing.assert_array_equal(np.broadcast_to(mm(0, 0, Q, K), (40, 40)), np.broadcast_to(omm(Q, K), (40, 40)))


def test_mask_specs_on_torch_tensors():
    torch = pytest.importorskip("torch")
    tq, tk = torch.arange(40)[:, None], torch.arange(40)[None, :]
    for mm in (pf.causal_mask, pf.sliding_window_mask(3, 1), pf.document_mask([10, 30])):
        got = mm(tq, tk).numpy()
        np.testing.assert_array_equal(got, np.broadcast_to(mm(Q, K), (40, 40)))


def test_document_mask_and_causal():
    dm = pf.document_mask([5, 20, 15])
    ids = np.repeat([0, 1, 2], [5, 20, 15])
    both = pf.and_masks(dm, pf.causal_mask)
    want = om.dense(om.both(om.causal, om.same_document(ids)), 40, 40)
    np.testing.assert_array_equal(np.broadcast_to(both(Q, K), (40, 40)), want)
    assert isinstance(both, pf.MaskSpec) and both.left == -1 and both.right == 0
    np.testing.assert_array_equal(both.doc_ids[0], ids)


def test_batched_document_mask_needs_batch_index():
    dm = pf.document_mask([[10, 30], [25, 15]])
    assert dm.batch_dependent and dm.doc_ids.shape == (2, 40)
    with pytest.raises(ValueError):
        dm(Q, K)
    np.testing.assert_array_equal(dm(1, 0, Q, K), om.dense(om.same_document(np.repeat([0, 1], [25, 15])), 40, 40))


def test_and_masks_intersects_windows():
    m = pf.and_masks(pf.sliding_window_mask(10, 4), pf.sliding_window_mask(6, -1), pf.causal_mask)
    assert (m.left, m.right) == (6, 0)
    want = om.dense(om.both(om.sliding_window(6, -1), om.both(om.sliding_window(10, 4), om.causal)), 40, 40)
    np.testing.assert_array_equal(np.broadcast_to(m(Q, K), (40, 40)), want)


def test_and_masks_with_callable_is_host_only():
    m = pf.and_masks(pf.causal_mask, lambda q, k: (q - k) % 2 == 0)
    assert not isinstance(m, pf.MaskSpec)
    np.testing.assert_array_equal(m(Q, K), (Q >= K) & ((Q - K) % 2 == 0))


def test_reference_document_mask_stub_replaced():
    # the reference raised NotImplementedError (mask_mod.py:58-59); here it builds ids
    assert pf.document_mask([3, 4]).doc_ids.tolist() == [[0, 0, 0, 1, 1, 1, 1]]


def test_alibi_slopes_closed_form():
    s = pf.alibi_slopes(32)
    np.testing.assert_allclose(s, [2.0 ** (-8 * h / 32) for h in range(32)], rtol=1e-7)
    assert s[0] == 1.0 and s.dtype == np.float32


def test_score_spec_matches_formula():
    sc = pf.compose_score_mods(pf.alibi_score_mod(4), pf.softcap_score_mod(50.0))
    s = np.random.default_rng(0).standard_normal((40, 40)) * 30
    for h in range(4):
        want = 50.0 * np.tanh((s + pf.alibi_slopes(4)[h] * (K - Q)) / 50.0)
        np.testing.assert_allclose(sc(s, 0, h, Q, K), want, rtol=1e-6)
    with pytest.raises(NotImplementedError):
        pf.compose_score_mods(pf.softcap_score_mod(5.0), pf.alibi_score_mod(4))


def test_untraceable_callables_raise():
    torch = pytest.importorskip("torch")
    x = torch.zeros(1, 1, 8, 32)
    from pallas_flexattn.flash_attn import _resolve
    # callables are traced and lowered; Python control flow on traced indices cannot be
    with pytest.raises(NotImplementedError, match="control flow"):
        _resolve(lambda q, k: (q >= k) if q > 0 else (q < k), None)
    with pytest.raises(NotImplementedError, match="cannot be lowered"):
        _resolve(None, lambda s, b, h, q, k: torch.erf(s))
    mask, score, mods = _resolve(lambda q, k: q >= k, lambda s, b, h, q, k: s * 2.0)
    assert mask is None and score is None and mods.mask is not None and mods.score is not None
    with pytest.raises(ValueError):  # host tensors are rejected, never computed on the CPU
        pf.flash_attention_fwd(x, x, x)