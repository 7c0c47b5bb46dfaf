"""Kernel tuner (CPU): the reference's invariants (``tests/test_kernel_tuner.py``)
plus the exact threshold table of ``kernel_tuner.py:28-63`` and the mapping
onto the MI355X tiles."""
import pytest

from pallas_flexattn import get_kernel_config, get_optimal_params
from pallas_flexattn.kernel_tuner import SUPPORTED_BLOCK_M, kernel_tiles


class TestKernelTuner:
    def test_get_optimal_params_short_sequence(self):
        block_r, block_c, num_warps, num_stages = get_optimal_params(256, 64)
        assert block_r <= 64 and block_c <= 64 and num_warps >= 4

    def test_get_optimal_params_long_sequence(self):
        block_r, block_c, num_warps, num_stages = get_optimal_params(4096, 64)
        assert block_r >= 128 and block_c >= 64 and num_warps >= 8

    def test_get_optimal_params_large_head_dim(self):
        block_r, block_c, _, _ = get_optimal_params(2048, 256)
        assert block_r <= 64 and block_c <= 64

    def test_get_optimal_params_cached(self):
        assert get_optimal_params(1024, 64) == get_optimal_params(1024, 64)
        assert get_optimal_params.cache_info().hits >= 1

    def test_get_kernel_config(self):
        config = get_kernel_config(2, 8, 2048, 64, 'causal')
        assert config['batch_size'] == 2 and config['num_heads'] == 8
        assert config['seq_len'] == 2048 and config['head_dim'] == 64
        for key in ('block_r', 'block_c', 'num_warps', 'num_stages'):
            assert key in config

    def test_sparsity_optimization(self):
        assert get_kernel_config(2, 8, 1024, 64, 'causal')['block_r'] <= get_kernel_config(2, 8, 1024, 64, None)['block_r']


# the reference's table, restated as literal rows (kernel_tuner.py:28-63)
@pytest.mark.parametrize("seq,d,sparse,want", [
    (256, 64, False, (32, 32, 4, 2)), (512, 64, False, (64, 64, 4, 3)), (2048, 64, False, (128, 64, 4, 3)),
    (4096, 64, False, (128, 128, 8, 4)), (8192, 64, False, (128, 128, 8, 5)),
    (2048, 256, False, (64, 64, 4, 3)), (8192, 256, False, (64, 64, 8, 3)),
    (256, 32, False, (32, 32, 4, 4)), (8192, 32, False, (128, 128, 8, 5)),
    (2048, 128, True, (64, 64, 4, 3)), (8192, 128, True, (64, 64, 8, 5)), (4096, 128, True, (64, 64, 8, 4)),
])
def test_threshold_table(seq, d, sparse, want):
    assert get_optimal_params(seq, d, sparse) == want


def test_kernel_tile_mapping():
    """The reference's block_r / block_c are Triton hints: without a tuned entry
    every hint maps to the default gfx950 tiles; with one, the tuned tiles."""
    for br, bc in ((128, 64), (64, 64), (32, 32), (256, 128)):
        assert kernel_tiles(br, bc, "bf16") == (128, 64, 128, 0, 0)
        assert kernel_tiles(br, bc, "fp32") == (128, 32, 128, 0, 0)
    assert kernel_tiles(64, 64, "bf16", 12345, 128, True) == (128, 64, 128, 0, 0)  # no entry for this shape


def test_resolved_tiles_and_mask_classes():
    import pallas_flexattn as pf
    import pallas_flexattn.kernel_tuner as kt
    assert kt.resolved_tiles((128, 64, 128), "bf16", 128) == (128, 64, 128, 128, 2)
    assert kt.resolved_tiles((128, 64, 64), "bf16", 128) == (128, 64, 64, 64, 2)
    assert kt.resolved_tiles((128, 64, 128), "bf16", 32) == (128, 64, 128, 64, 2)
    assert kt.resolved_tiles((128, 32, 128, 0, 3), "bf16", 64) == (128, 32, 128, 64, 3)
    assert kt.resolved_tiles((128, 32, 128, 128, 3), "bf16", 64) == (128, 32, 128, 128, 3)
    assert kt.resolved_tiles(kt.DEFAULT_TILES["fp32"], "fp32", 64) == (128, 32, 128, 32, 2)
    assert kt.mask_class(None) == "dense"
    assert kt.mask_class(pf.causal_mask) == "causal"
    assert kt.mask_class(pf.bidirectional_mask) == "dense"
    assert kt.mask_class(pf.sliding_window_mask(1023, 0)) == "window"
    dm = pf.document_mask([[100, 28]])
    assert kt.mask_class(pf.and_masks(dm, pf.causal_mask)) == "document"
    assert kt.table_key(8192, 128, "bf16", "window") == "bf16/D128/S8192/window"
    assert kt.table_key(8192, 128, "bf16", True) == "bf16/D128/S8192/causal"
    assert kt.table_key(8192, 128, "bf16", False) == "bf16/D128/S8192/dense"
    with pytest.raises(ValueError):
        kt.table_key(8192, 128, "bf16", "diagonal")
    assert kt.tile_name((128, 32, 128, 64, 3)) == "128x32x128q64s3"


def test_kernel_tiles_follow_the_tune_table(tmp_path, monkeypatch):
    import json
    import pallas_flexattn.kernel_tuner as kt
    path = tmp_path / "table.json"
    path.write_text(json.dumps({
        # an entry from before the mask classes and the last two axes
        "bf16/D64/S1024/sparse": {"block_m": 64, "block_n": 64},
        kt.table_key(2048, 128, "bf16", "causal"): {"block_m": 256, "block_n": 64, "block_kv": 64,
                                                    "block_q": 64, "num_stages": 2},
        kt.table_key(2048, 128, "bf16", "window"): {"block_m": 128, "block_n": 32, "block_kv": 128,
                                                    "block_q": 128, "num_stages": 3}}))
    monkeypatch.setattr(kt, "TUNE_TABLE", str(path))
    monkeypatch.setattr(kt.load_tune_table, "__defaults__", (str(path),))
    assert kt.kernel_tiles(128, 128, "bf16", 1024, 64, True) == (64, 64, 128, 0, 0)  # defaults for the rest
    assert kt.kernel_tiles(128, 128, "bf16", 1024, 64, False) == (128, 64, 128, 0, 0)
    assert kt.tuned_tiles(1024, 64, "bf16", "window") == (64, 64, 128, 0, 0)  # falls back to the causal entry
    assert kt.tuned_tiles(2048, 128, "bf16", "causal") == (256, 64, 64, 64, 2)
    assert kt.tuned_tiles(2048, 128, "bf16", "window") == (128, 32, 128, 128, 3)
    assert kt.tuned_tiles(2048, 128, "bf16", "document") == (256, 64, 64, 64, 2)
    assert kt.tuned_tiles(2048, 128, "bf16", "dense") is None
    # parsed once per modification time
    assert kt.load_tune_table(str(path)) is kt.load_tune_table(str(path))


def test_committed_tune_table_is_consistent():
    """The measured table shipped with the package: every entry names an
    instantiated tile choice and is the fastest fwd + bwd of its candidates
    (or the default tiles when none beats them by the margin)."""
    from pallas_flexattn.kernel_tuner import (DEFAULT_TILES, candidate_tiles, load_tune_table, resolved_tiles,
                                              tile_name, TUNE_TABLE)
    import os
    if not os.path.exists(TUNE_TABLE):
        pytest.skip("no tune table")
    table = load_tune_table()
    assert table
    for key, e in table.items():
        dtype, d, _, cls = key.split("/")
        assert cls in ("dense", "causal", "window", "document")
        tiles = (e["block_m"], e["block_n"], e["block_kv"], e["block_q"], e["num_stages"])
        assert tiles in candidate_tiles(dtype, int(d[1:]))
        chosen = e["candidates"][tile_name(tiles)]
        fastest = min(e["candidates"].values(), key=lambda c: c["ms_fwd_bwd"])
        default = e["candidates"].get(tile_name(resolved_tiles(DEFAULT_TILES[dtype], dtype, int(d[1:]))))
        assert chosen is fastest or (chosen is default and
                                     fastest["ms_fwd_bwd"] > chosen["ms_fwd_bwd"] * (1 - e["margin"]))
        for c in e["candidates"].values():
            assert c["waves"] * 32 in SUPPORTED_BLOCK_M and c["ms_fwd"] < c["ms_fwd_bwd"]


def test_candidate_tiles_cover_the_instantiated_axes():
    from pallas_flexattn.kernel_tuner import (SUPPORTED_BLOCK_KV, SUPPORTED_BLOCK_N, SUPPORTED_BLOCK_Q,
                                              SUPPORTED_NUM_STAGES, candidate_tiles)
    c = candidate_tiles("bf16", 128)
    assert {t[0] for t in c} == set(SUPPORTED_BLOCK_M)
    assert {t[1] for t in c} == set(SUPPORTED_BLOCK_N["bf16"])
    assert {t[2] for t in c} == set(SUPPORTED_BLOCK_KV["bf16"])
    assert {t[3] for t in c} == set(SUPPORTED_BLOCK_Q["bf16"])
    assert {t[4] for t in c} == set(SUPPORTED_NUM_STAGES["bf16"])
    assert len(c) == len(set(c)) == 21 and c[0] == (128, 64, 128, 128, 2)
    # stage counts only where an instantiation exists: 3 with 32-key tiles, 1 with 128-key tiles
    assert {(t[1], t[4]) for t in c} == {(64, 2), (32, 2), (32, 3), (128, 2), (128, 1)}
    # 128-query dK/dV tiles only with 128-key dK/dV workgroups
    assert {(t[2], t[3]) for t in c} == {(128, 128), (128, 64), (64, 64)}
    # D = 32: the DMA split needs at least 1 KiB per wave and tile
    assert candidate_tiles("bf16", 32) == ((128, 64, 128, 64, 2), (64, 64, 128, 64, 2))
    assert candidate_tiles("fp32", 128) == ((128, 32, 128, 32, 2), (64, 32, 128, 32, 2))
