"""Mask predicates of the reference, restated for the oracle.

Each returns a boolean numpy array broadcast over ``q_idx`` and ``kv_idx``.
"""
import numpy as np


def causal(q_idx, kv_idx):
    """``mask_mod.py:15-17``: a query sees keys at the same or earlier positions."""
    return np.asarray(q_idx) >= np.asarray(kv_idx)


def bidirectional(q_idx, kv_idx):
    """``mask_mod.py:20-22``: everything is visible."""
    return np.ones(np.broadcast(np.asarray(q_idx), np.asarray(kv_idx)).shape, dtype=bool)


def sliding_window(left, right):
    """``mask_mod.py:25-43``: delta = q - kv; delta <= left if left >= 0; -delta <= right if right >= 0."""
    def mask(q_idx, kv_idx):
        delta = np.asarray(q_idx) - np.asarray(kv_idx)
        m = np.ones(delta.shape, dtype=bool)
        if left >= 0:
            m = m & (delta <= left)
        if right >= 0:
            m = m & (-delta <= right)
        return m
    return mask


def same_document(doc_ids_row):
    """Packed-document predicate (the reference leaves it as a stub, ``mask_mod.py:46-59``):
    ``doc[q] == doc[kv]`` for one batch row of document ids."""
    d = np.asarray(doc_ids_row)

    def mask(q_idx, kv_idx):
        return d[np.asarray(q_idx)] == d[np.asarray(kv_idx)]
    return mask


def both(m1, m2):
    def mask(q_idx, kv_idx):
        return m1(q_idx, kv_idx) & m2(q_idx, kv_idx)
    return mask


def dense(mask_fn, sq, skv):
    """Materialise a predicate over the full (sq, skv) grid, like ``flash_attn.py:50-52``."""
    return np.broadcast_to(mask_fn(np.arange(sq)[:, None], np.arange(skv)[None, :]), (sq, skv)).copy()
