"""Block masks built on the GPU (C ABI fa_build_block_mask) against the host
construction and the oracle (create_block_mask, block_mask.py:54-129).

Every field must be bit-identical to the host path: the reference's sampled
num_blocks_in_row / col_indices and the eight kernel tables, for windows,
causal, bidirectional, packed documents (contiguous and repeated labels,
per-batch rows), ragged lengths, Q_LEN != KV_LEN and the benchmark sizes (C3
sliding window S=8192, C5 packed documents S=16384).  Small cases are also
checked against the oracle's brute force (the 3x3 sampling rule on the mask
function, and the live / full state of every tile of the dense mask)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

pytestmark = pytest.mark.gpu

FIELDS = ("num_blocks_in_row", "col_indices", "kv_num_blocks", "kv_indices", "full_kv_num_blocks",
          "full_kv_indices", "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")


def _cases():
    import pallas_flexattn as pf
    rng = np.random.default_rng(11)
    labels = np.repeat(rng.integers(0, 3, size=20), 50).astype(np.int32)  # repeated, non-contiguous labels
    return [
        ("causal-ragged", pf.causal_mask, 1000, 1000, 128),
        ("causal-q300-kv500", pf.causal_mask, 300, 500, 64),
        ("causal-q500-kv300", pf.causal_mask, 500, 300, 64),
        ("window-100-0", pf.sliding_window_mask(100, 0), 1000, 1000, 64),
        ("window-64-32", pf.sliding_window_mask(64, 32), 777, 777, 32),
        ("window-0-200", pf.sliding_window_mask(0, 200), 640, 640, 128),
        ("bidirectional", pf.bidirectional_mask, 500, 700, 128),
        ("docs-causal", pf.and_masks(pf.document_mask([300, 200, 500]), pf.causal_mask), 1000, 1000, 128),
        ("docs-only", pf.document_mask([100, 28, 250, 134]), 512, 512, 64),
        ("docs-repeated-labels", pf.document_ids_mask(labels), 1000, 1000, 64),
        ("docs-batch-rows", pf.and_masks(pf.document_mask([[300, 700], [500, 500]]), pf.causal_mask),
         1000, 1000, 128),
        ("docs-window", pf.and_masks(pf.document_mask([400, 600]), pf.sliding_window_mask(150, 0)), 1000, 1000, 64),
        ("single-block", pf.causal_mask, 50, 50, 128),
        ("block-256", pf.causal_mask, 1280, 1280, 256),
    ]


@pytest.mark.parametrize("idx", range(14))
def test_device_block_mask_matches_host(idx):
    import pallas_flexattn as pf
    name, mm, q_len, kv_len, bs = _cases()[idx]
    host = pf.create_block_mask(mm, 2, 3, q_len, kv_len, bs)
    dev = pf.create_block_mask(mm, 2, 3, q_len, kv_len, bs, device="cuda")
    for f in FIELDS:
        a, b = getattr(host, f), getattr(dev, f)
        assert a.shape == b.shape and a.dtype == b.dtype, (name, f, a.shape, b.shape)
        assert np.array_equal(a, b), (name, f)
    assert dev.sparsity == host.sparsity
    # the cached device tables are the host tables
    tabs = dev.device_tables("cuda")
    for f in FIELDS[2:]:
        assert np.array_equal(tabs[f].cpu().numpy(), getattr(host, f)), (name, f)


@pytest.mark.parametrize("idx", [0, 1, 3, 4, 7, 9, 11])
def test_device_block_mask_matches_oracle_brute_force(idx):
    import pallas_flexattn as pf
    from oracle import block_mask_ref as ref
    name, mm, q_len, kv_len, bs = _cases()[idx]
    dev = pf.create_block_mask(mm, 1, 1, q_len, kv_len, bs, device="cuda")
    # sampled fields: the reference's rule evaluated point by point
    num, col = ref.sampled(mm, q_len, kv_len, bs)
    assert np.array_equal(dev.num_blocks_in_row, num) and np.array_equal(dev.col_indices, col), name
    # exact tables: every element of the dense mask
    dense = np.asarray(mm(np.arange(q_len)[:, None], np.arange(kv_len)[None, :]), dtype=bool)
    live, full = ref.exact_tiles(dense, bs, bs)
    part = live & ~full
    for side, (p, fu) in (("kv", (part, full)), ("q", (part.T, full.T))):
        for prefix, sel in (("", p), ("full_", fu)):
            n = getattr(dev, f"{prefix}{side}_num_blocks")[0, 0]
            idxs = getattr(dev, f"{prefix}{side}_indices")[0, 0]
            assert np.array_equal(n, sel.sum(axis=1)), (name, prefix, side)
            for r in range(sel.shape[0]):
                assert np.array_equal(idxs[r, :n[r]], np.flatnonzero(sel[r])), (name, prefix, side, r)
                assert np.all(idxs[r, n[r]:] == -1)


@pytest.mark.parametrize("cfg_name", ["c3", "c5"])
def test_device_block_mask_benchmark_sizes(cfg_name):
    import bench
    import pallas_flexattn as pf
    cfg = bench.make_config(cfg_name)
    S = cfg["S"]
    host = pf.create_block_mask(cfg["mask"], cfg["B"], cfg["Hq"], S, S, 128)
    dev = pf.create_block_mask(cfg["mask"], cfg["B"], cfg["Hq"], S, S, 128, device="cuda")
    for f in FIELDS:
        assert np.array_equal(getattr(host, f), getattr(dev, f)), (cfg_name, f)
    if cfg_name == "c3":
        assert dev.live_tiles() == 540


def test_flex_attention_builds_its_tables_on_the_device():
    """A mask given without a BlockMask gets its tables from the GPU builder;
    they equal the host tables, and flex_attention over a device-built
    BlockMask returns exactly what it returns over the host-built one."""
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn.block_mask import _finish
    from pallas_flexattn.flash_attn import _internal_block_mask
    torch.manual_seed(0)
    B, H, S, D = 2, 2, 640, 64
    mm = pf.and_masks(pf.document_mask([[200, 440], [320, 320]]), pf.causal_mask)
    internal = _internal_block_mask(mm, B, S, S, torch.device("cuda"))
    host = _finish(None, None, mm, B, 1, S, S, 128)
    for f in FIELDS[2:]:
        assert np.array_equal(getattr(internal, f), getattr(host, f)), f
    q, k, v = (torch.randn(B, H, S, D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    o_dev = pf.flex_attention(q, k, v, block_mask=pf.create_block_mask(mm, B, H, S, S, 128, device="cuda"))
    o_host = pf.flex_attention(q, k, v, block_mask=pf.create_block_mask(mm, B, H, S, S, 128))
    torch.cuda.synchronize()
    assert torch.equal(o_dev, o_host)
