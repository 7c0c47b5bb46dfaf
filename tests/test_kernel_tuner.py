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
    every hint maps to the default gfx950 tile; with one, the tuned tile."""
    import json
    import pallas_flexattn.kernel_tuner as kt
    for br, bc in ((128, 64), (64, 64), (32, 32), (256, 128)):
        assert kernel_tiles(br, bc, "bf16") == (128, 64, 128)
        assert kernel_tiles(br, bc, "fp32") == (128, 32, 128)
    assert kernel_tiles(64, 64, "bf16", 12345, 128, True) == (128, 64, 128)  # no entry for this shape


def test_kernel_tiles_follow_the_tune_table(tmp_path, monkeypatch):
    import json
    import pallas_flexattn.kernel_tuner as kt
    path = tmp_path / "table.json"
    path.write_text(json.dumps({kt.table_key(1024, 64, "bf16", True): {"block_m": 64, "block_n": 64},
                                kt.table_key(2048, 128, "bf16", True): {"block_m": 256, "block_n": 64,
                                                                        "block_kv": 64}}))
    monkeypatch.setattr(kt, "TUNE_TABLE", str(path))
    monkeypatch.setattr(kt.load_tune_table, "__defaults__", (str(path),))
    assert kt.kernel_tiles(128, 128, "bf16", 1024, 64, True) == (64, 64, 128)  # entries without block_kv
    assert kt.kernel_tiles(128, 128, "bf16", 1024, 64, False) == (128, 64, 128)
    assert kt.tuned_tiles(1024, 64, "bf16", True) == (64, 64, 128)
    assert kt.tuned_tiles(2048, 128, "bf16", True) == (256, 64, 64)
    # parsed once per modification time
    assert kt.load_tune_table(str(path)) is kt.load_tune_table(str(path))


def test_committed_tune_table_is_consistent():
    """The measured table shipped with the package: every entry names an
    instantiated tile pair and is the fastest fwd + bwd of its candidates."""
    from pallas_flexattn.kernel_tuner import candidate_tiles, load_tune_table, TUNE_TABLE
    import os
    if not os.path.exists(TUNE_TABLE):
        pytest.skip("no tune table")
    table = load_tune_table()
    assert table
    for key, e in table.items():
        dtype, d = key.split("/")[:2]
        tiles = (e["block_m"], e["block_n"], e.get("block_kv", 128))
        assert tiles in candidate_tiles(dtype, int(d[1:]))
        best, fastest = min(e["candidates"].items(), key=lambda kv: kv[1]["ms_fwd_bwd"])
        chosen = e["candidates"].get("x".join(map(str, tiles))) or e["candidates"][f"{tiles[0]}x{tiles[1]}"]
        # the fastest candidate, or the default tiles when none beats them by the margin
        assert chosen is fastest or fastest["ms_fwd_bwd"] > chosen["ms_fwd_bwd"] * (1 - e.get("margin", 0.0))
        for c in e["candidates"].values():
            assert c["waves"] * 32 in SUPPORTED_BLOCK_M and c["ms_fwd"] < c["ms_fwd_bwd"]


def test_candidate_tiles_cover_the_instantiated_axes():
    from pallas_flexattn.kernel_tuner import SUPPORTED_BLOCK_KV, SUPPORTED_BLOCK_N, candidate_tiles
    c = candidate_tiles("bf16", 128)
    assert {t[0] for t in c} == set(SUPPORTED_BLOCK_M)
    assert {t[1] for t in c} == set(SUPPORTED_BLOCK_N["bf16"])
    assert {t[2] for t in c} == set(SUPPORTED_BLOCK_KV["bf16"])
    assert len(c) == len(set(c)) == 10 and c[0] == (128, 64, 128)
    # D = 32: the DMA split needs at least 1 KiB per wave and tile
    assert candidate_tiles("bf16", 32) == ((128, 64, 128), (64, 64, 128))
    assert candidate_tiles("fp32", 128) == ((128, 32, 128), (64, 32, 128))
