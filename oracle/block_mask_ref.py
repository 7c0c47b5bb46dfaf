"""Block-mask construction of the reference, restated with plain Python loops.

Returns ``(num_blocks_in_row, col_indices)`` as int32 numpy arrays, the two
array fields of the reference's ``BlockMask`` (``block_mask.py:16-51``).
"""
import math

import numpy as np


def _pad_rows(rows):
    # block_mask.py:115-121 — pad every row with -1 up to the longest row.
    width = max((len(r) for r in rows), default=0)
    nb = np.array([len(r) for r in rows], dtype=np.int32)
    ci = np.array([r + [-1] * (width - len(r)) for r in rows], dtype=np.int32)
    if ci.size == 0:
        ci = ci.reshape(len(rows), width)
    return nb, ci


def sampled(mask_fn, q_len, kv_len, block_size):
    """``block_mask.py:54-129``: a (q-block, kv-block) pair is kept iff the
    predicate holds on any of the 3x3 samples {start, (start+end)//2, end-1}."""
    nq = math.ceil(q_len / block_size)
    nk = math.ceil(kv_len / block_size)
    rows = []
    for i in range(nq):
        qs = i * block_size
        qe = min(qs + block_size, q_len)
        valid = []
        for j in range(nk):
            ks = j * block_size
            ke = min(ks + block_size, kv_len)
            q_sample = np.array([qs, (qs + qe) // 2, qe - 1])
            kv_sample = np.array([ks, (ks + ke) // 2, ke - 1])
            if np.any(mask_fn(q_sample[:, None], kv_sample[None, :])):
                valid.append(j)
        rows.append(valid)
    return _pad_rows(rows)


def causal_closed_form(seq_len, block_size):
    """``block_mask.py:132-172``: row i holds blocks 0..i."""
    n = math.ceil(seq_len / block_size)
    return _pad_rows([list(range(i + 1)) for i in range(n)])


def sliding_closed_form(seq_len, window_size, block_size):
    """``block_mask.py:175-218``: row i holds max(0, i-wb) .. min(n, i+wb+1)-1, wb = ceil(w/bs)."""
    n = math.ceil(seq_len / block_size)
    wb = math.ceil(window_size / block_size)
    return _pad_rows([list(range(max(0, i - wb), min(n, i + wb + 1))) for i in range(n)])


def sparsity(num_blocks_in_row, q_len, kv_len, block_size):
    """``block_mask.py:46-51``."""
    total = math.ceil(q_len / block_size) * math.ceil(kv_len / block_size)
    return 1.0 - float(np.sum(num_blocks_in_row)) / total


def exact_tiles(dense_mask, bq, bk):
    """Brute-force tile classification of a materialised (Sq, Skv) mask:
    returns (live, full) boolean (nq, nk) arrays; a tile that runs past the end
    of either sequence is never full."""
    sq, skv = dense_mask.shape
    nq, nk = math.ceil(sq / bq), math.ceil(skv / bk)
    live = np.zeros((nq, nk), dtype=bool)
    full = np.zeros((nq, nk), dtype=bool)
    for i in range(nq):
        for j in range(nk):
            t = dense_mask[i * bq:(i + 1) * bq, j * bk:(j + 1) * bk]
            live[i, j] = bool(t.any())
            full[i, j] = bool(t.all()) and t.shape == (bq, bk)
    return live, full
