"""Block masks (CPU).  The first classes port the reference's own assertions
(``tests/test_block_mask.py``); the rest pin bit-exactness of the reference
fields against the oracle's pure-Python restatement of the sampling rule, and
the exact kernel tables against brute-force tile classification."""
import math

import numpy as np
import pytest

import pallas_flexattn as pf
from pallas_flexattn.block_mask import BlockMask, create_block_mask, create_causal_block_mask, \
    create_sliding_window_block_mask
from pallas_flexattn.mask_mod import bidirectional_mask, causal_mask, sliding_window_mask

from oracle import block_mask_ref as ref
from oracle import masks as om


class TestBlockMaskCreation:
    def test_create_causal_block_mask(self):
        bm = create_causal_block_mask(256, 64)
        assert bm.block_size == 64 and bm.q_len == 256 and bm.kv_len == 256
        assert bm.num_q_blocks == 4
        assert [int(x) for x in bm.num_blocks_in_row] == [1, 2, 3, 4]

    def test_create_sliding_window_block_mask(self):
        bm = create_sliding_window_block_mask(256, 64, 64)
        assert bm.block_size == 64 and bm.q_len == 256
        assert bm.num_blocks_in_row[1] == 3
        assert bm.num_blocks_in_row[2] == 3

    def test_create_block_mask_from_mask_mod(self):
        bm = create_block_mask(mask_mod=causal_mask, B=2, H=4, Q_LEN=256, KV_LEN=256, block_size=64)
        assert bm.block_size == 64 and bm.q_len == 256 and bm.num_q_blocks == 4
        assert 0.3 < bm.sparsity < 0.5

    def test_block_mask_sparsity_dense(self):
        bm = create_block_mask(mask_mod=bidirectional_mask, B=1, H=1, Q_LEN=256, KV_LEN=256, block_size=64)
        assert bm.sparsity == 0.0

    def test_block_mask_sparsity_causal(self):
        bm = create_causal_block_mask(1024, 128)
        n = 1024 // 128
        assert abs(bm.sparsity - (1.0 - (n * (n + 1) / 2) / (n * n))) < 0.01


class TestBlockMaskStructure:
    def test_col_indices_shape(self):
        bm = create_causal_block_mask(256, 64)
        assert bm.col_indices.shape == (4, 4)

    def test_col_indices_values_causal(self):
        ci = create_causal_block_mask(256, 64).col_indices
        assert ci[0, 0] == 0 and ci[0, 1] == -1
        assert list(ci[2]) == [0, 1, 2, -1]

    def test_num_blocks_in_row_dtype(self):
        bm = create_causal_block_mask(128, 64)
        assert bm.num_blocks_in_row.dtype == np.int32
        assert bm.col_indices.dtype == np.int32


class TestBlockMaskEdgeCases:
    def test_non_power_of_two_seq_len(self):
        assert create_causal_block_mask(300, 64).num_q_blocks == 5

    def test_very_small_block_size(self):
        assert create_causal_block_mask(64, 16).num_q_blocks == 4

    def test_single_block(self):
        bm = create_causal_block_mask(64, 128)
        assert bm.num_q_blocks == 1 and bm.num_blocks_in_row[0] == 1


# ---------------------------------------------------------- bit-exactness --
MASK_PAIRS = [
    ("causal", causal_mask, om.causal),
    ("bidirectional", bidirectional_mask, om.bidirectional),
    ("window(100,0)", sliding_window_mask(100, 0), om.sliding_window(100, 0)),
    ("window(32,32)", sliding_window_mask(32, 32), om.sliding_window(32, 32)),
    ("window(-1,5)", sliding_window_mask(-1, 5), om.sliding_window(-1, 5)),
    ("window(0,0)", sliding_window_mask(0, 0), om.sliding_window(0, 0)),
    ("q-k==100 (lambda)", lambda q, k: (q - k) == 100, lambda q, k: (np.asarray(q) - np.asarray(k)) == 100),
]


@pytest.mark.parametrize("name,mm,omm", MASK_PAIRS, ids=[m[0] for m in MASK_PAIRS])
@pytest.mark.parametrize("q_len,kv_len,bs", [(256, 256, 64), (300, 300, 64), (1000, 1000, 128), (64, 64, 16),
                                             (64, 64, 128), (513, 200, 32)])
def test_reference_fields_bit_exact(name, mm, omm, q_len, kv_len, bs):
    with _no_fail():
        bm = create_block_mask(mm, 1, 1, q_len, kv_len, bs)
    n, c = ref.sampled(omm, q_len, kv_len, bs)
    assert bm.num_blocks_in_row.dtype == np.int32 and bm.col_indices.dtype == np.int32
    np.testing.assert_array_equal(bm.num_blocks_in_row, n)
    np.testing.assert_array_equal(bm.col_indices, c)
    assert bm.sparsity == ref.sparsity(n, q_len, kv_len, bs)


class _no_fail:
    def __enter__(self):
        import warnings
        self._w = warnings.catch_warnings()
        self._w.__enter__()
        warnings.simplefilter("ignore")

    def __exit__(self, *a):
        self._w.__exit__(*a)


@pytest.mark.parametrize("seq,bs", [(256, 64), (300, 64), (1024, 128), (64, 16), (64, 128)])
def test_closed_forms_match_reference(seq, bs):
    bm = create_causal_block_mask(seq, bs)
    n, c = ref.causal_closed_form(seq, bs)
    np.testing.assert_array_equal(bm.num_blocks_in_row, n)
    np.testing.assert_array_equal(bm.col_indices, c)
    for w in (0, 10, 64, 65, 200):
        bm = create_sliding_window_block_mask(seq, w, bs)
        n, c = ref.sliding_closed_form(seq, w, bs)
        np.testing.assert_array_equal(bm.num_blocks_in_row, n)
        np.testing.assert_array_equal(bm.col_indices, c)


def test_sampling_misses_exotic_tiles_but_tables_are_exact():
    """The 3x3 sampling rule (reference) misses q-k==100 tiles; the kernel tables do not."""
    with pytest.warns(UserWarning):
        bm = create_block_mask(lambda q, k: (q - k) == 100, 1, 1, 512, 512, 64)
    live, full = ref.exact_tiles(om.dense(lambda q, k: (q - k) == 100, 512, 512), 64, 64)
    np.testing.assert_array_equal(bm.kv_num_blocks[0, 0] + bm.full_kv_num_blocks[0, 0], live.sum(1))


# ------------------------------------------------------------ exact tables --
def _check_tables(bm, live, full):
    """live/full: (nq, nk) brute-force classification for table row (0, 0)."""
    nq, nk = live.shape
    partial = live & ~full
    for i in range(nq):
        n = bm.kv_num_blocks[0, 0, i]
        nf = bm.full_kv_num_blocks[0, 0, i]
        assert list(bm.kv_indices[0, 0, i, :n]) == list(np.flatnonzero(partial[i]))
        assert list(bm.full_kv_indices[0, 0, i, :nf]) == list(np.flatnonzero(full[i]))
        assert np.all(bm.kv_indices[0, 0, i, n:] == -1) and np.all(bm.full_kv_indices[0, 0, i, nf:] == -1)
    for j in range(nk):  # transposed q-side tables
        n = bm.q_num_blocks[0, 0, j]
        nf = bm.full_q_num_blocks[0, 0, j]
        assert list(bm.q_indices[0, 0, j, :n]) == list(np.flatnonzero(partial[:, j]))
        assert list(bm.full_q_indices[0, 0, j, :nf]) == list(np.flatnonzero(full[:, j]))
    assert bm.kv_indices.shape[-1] == bm.full_kv_indices.shape[-1]
    assert bm.q_indices.shape[-1] == bm.full_q_indices.shape[-1]


@pytest.mark.parametrize("name,mm,omm", MASK_PAIRS[:6], ids=[m[0] for m in MASK_PAIRS[:6]])
@pytest.mark.parametrize("q_len,kv_len,bs", [(256, 256, 64), (300, 300, 64), (520, 390, 128)])
def test_exact_tables_match_brute_force(name, mm, omm, q_len, kv_len, bs):
    with _no_fail():
        bm = create_block_mask(mm, 1, 1, q_len, kv_len, bs)
    live, full = ref.exact_tiles(om.dense(omm, q_len, kv_len), bs, bs)
    _check_tables(bm, live, full)


def test_document_tables_match_brute_force():
    rng = np.random.default_rng(3)
    S, bs = 700, 64
    rows = []
    for _ in range(2):
        lens, tot = [], 0
        while tot < S:
            n = min(int(rng.integers(20, 200)), S - tot)
            lens.append(n)
            tot += n
        rows.append(lens)
    dm = pf.document_mask(rows)
    for window in ((-1, 0), (50, 0), (-1, -1)):
        mm = pf.and_masks(dm, sliding_window_mask(*window))
        bm = create_block_mask(mm, 2, 3, S, S, bs)
        assert bm.kv_num_blocks.shape[:2] == (2, 1)
        for b in range(2):
            dense = om.dense(om.both(om.sliding_window(*window), om.same_document(dm.doc_ids[b])), S, S)
            live, full = ref.exact_tiles(dense, bs, bs)
            sub = BlockMask(bm.num_blocks_in_row, bm.col_indices, bs, S, S, mm,
                            **{k: getattr(bm, k)[b:b + 1] for k in (
                                "kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                                "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")})
            _check_tables(sub, live, full)


def test_document_ids_with_repeated_labels():
    ids = np.array([0] * 70 + [1] * 90 + [0] * 60 + [2] * 36)
    mm = pf.document_ids_mask(ids)
    bm = create_block_mask(mm, 1, 1, 256, 256, 32)
    live, full = ref.exact_tiles(om.dense(om.same_document(ids), 256, 256), 32, 32)
    _check_tables(bm, live, full)


def test_arity4_callable_gives_per_head_tables():
    def mm(b, h, q, k):
        return (q >= k) | (h == 1)
    bm = create_block_mask(mm, 2, 2, 128, 128, 32)
    assert bm.kv_num_blocks.shape == (2, 2, 4)
    assert list(bm.full_kv_num_blocks[0, 1]) == [4, 4, 4, 4]
    assert bm.num_blocks_in_row.shape == (2, 2, 4)


@pytest.mark.parametrize("S,mm,live", [(2048, causal_mask, 136), (8192, sliding_window_mask(1023, 0), 540),
                                      (4096, causal_mask, 528), (8192, causal_mask, 2080)])
def test_live_tile_counts_of_benchmark_configs(S, mm, live):
    bm = create_block_mask(mm, 1, 1, S, S, 128)
    assert bm.live_tiles() == live
    assert int(bm.num_blocks_in_row.sum()) == live  # sampling agrees with exact for these masks


def test_sliding_window_1024_split_into_full_and_partial():
    bm = create_block_mask(sliding_window_mask(1023, 0), 1, 1, 8192, 8192, 128)
    assert int(bm.full_kv_num_blocks.sum()) == 420 and int(bm.kv_num_blocks.sum()) == 120
