"""The bf16 tile kernels' index arithmetic under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU).  tests/native/kernel_index_check.cpp
compiles the kernels' index functions (csrc/index.h) and the C ABI's host
set-up (csrc/problem.h) for the host and walks every workgroup of the
forward (plain, split-KV, GQA-packed, paged), dQ and dK/dV launches through
them, checking every table read, buffer-resource range, LDS offset and store
against its buffer.  The cases: the benchmark configurations (causal S = 2048
and 8192, sliding window, GQA, packed documents), ragged lengths (S = 300,
192, 200), Sq != Skv, head dims 32 / 64 / 128, per-head tables, tables with
out-of-range entries and over-long counts, and a paged decode cache with
invalid page ids and per-batch lengths; each at the default tiles and, for
the small ones, every tile set the tuner can pick."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import pallas_flexattn as pf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pallas-flexattn_amd", "csrc")
MAGIC = 0x46414958


def _tables(bm, per_head=0, corrupt=False):
    """int32 tables of a BlockMask as the C ABI takes them: (TB, TH, rows[, width])."""
    out = {}
    for n in ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
              "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"):
        a = np.asarray(getattr(bm, n), dtype=np.int32)
        if per_head:
            a = np.broadcast_to(a, (a.shape[0], per_head) + a.shape[2:])
        out[n] = np.ascontiguousarray(a)
    if corrupt:  # entries outside the block range and counts past the width
        rng = np.random.default_rng(7)
        for n in ("kv_indices", "q_indices", "full_kv_indices", "full_q_indices"):
            a = out[n].reshape(-1)
            idx = rng.choice(a.size, size=max(1, a.size // 7), replace=False)
            a[idx] = rng.choice(np.array([-5, -1, 99999, 1 << 30], dtype=np.int32), size=idx.size)
        for n, w in (("kv_num_blocks", "kv_indices"), ("q_num_blocks", "q_indices"),
                     ("full_kv_num_blocks", "full_kv_indices"), ("full_q_num_blocks", "full_q_indices")):
            a = out[n].reshape(-1)
            a[::3] = out[w].shape[-1] + 3
            a[-1] = out[w].shape[-1] + 3  # the last row too: a count past the width would leave the array
            a[1::5] = -2
    return out


def _case(B, Hq, Hkv, Sq, Skv, D, mask=None, per_head=0, corrupt=False, all_tiles=True):
    hdr_win = (-1, -1)
    docs = None
    tabs = None
    if mask is not None:
        hdr_win = (mask.left, mask.right)
        bm = pf.create_block_mask(mask, 1, 1, Sq, Skv, 128)
        tabs = _tables(bm, per_head, corrupt)
        if mask.doc_ids is not None:
            ids = np.ascontiguousarray(np.broadcast_to(mask.doc_ids, (B, Sq)), dtype=np.int32)
            start, end = (np.ascontiguousarray(np.broadcast_to(x, (B, Sq)), dtype=np.int32) for x in mask.doc_bounds())
            docs = (ids, ids, start, end)
    hdr = [B, Hq, Hkv, Sq, Skv, D, hdr_win[0], hdr_win[1], int(docs is not None), int(tabs is not None), 128,
           tabs["kv_num_blocks"].shape[0] if tabs else 0, tabs["kv_num_blocks"].shape[1] if tabs else 0,
           tabs["kv_indices"].shape[-1] if tabs else 0, tabs["q_indices"].shape[-1] if tabs else 0,
           0, 0, 0, 0, 0, int(all_tiles), MAGIC]
    parts = [np.asarray(hdr, np.int32)]
    if docs is not None:
        parts += list(docs)
    if tabs is not None:
        parts += [tabs[n] for n in ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                                    "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")]
    return b"".join(np.ascontiguousarray(p, np.int32).tobytes() for p in parts)


def _paged(B, Hq, Hkv, Skv, D, page_size, max_pages, num_pages):
    hdr = [B, Hq, Hkv, 1, Skv, D, -1, -1, 0, 0, 128, 0, 0, 0, 0, 1, page_size, max_pages, num_pages, 1, 0, MAGIC]
    return np.asarray(hdr, np.int32).tobytes()


def _doc_mask(S, seed):
    rng = np.random.default_rng(seed)
    lens, tot = [], 0
    while tot < S:
        n = min(int(rng.integers(256, 4097)), S - tot)
        lens.append(n)
        tot += n
    return pf.and_masks(pf.document_mask([lens]), pf.causal_mask)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_kernel_index_arithmetic_stays_in_bounds(tmp_path):
    exe = tmp_path / "kernel_index_check"
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-Wall", "-Wno-unknown-pragmas", "-I", CSRC, os.path.join(ROOT, "tests", "native", "kernel_index_check.cpp"),
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    cases = [
        # the benchmark configurations (default tiles and two alternatives)
        _case(8, 16, 16, 2048, 2048, 128, pf.causal_mask, all_tiles=False),
        _case(4, 32, 32, 8192, 8192, 128, pf.causal_mask, all_tiles=False),
        _case(4, 32, 32, 8192, 8192, 128, pf.sliding_window_mask(1023, 0), all_tiles=False),
        _case(4, 32, 8, 4096, 4096, 128, pf.causal_mask, all_tiles=False),
        _case(2, 16, 16, 16384, 16384, 128, _doc_mask(16384, 4), all_tiles=False),
        # small problems at every tile set
        _case(1, 4, 4, 256, 256, 64, pf.causal_mask),
        _case(2, 4, 2, 300, 300, 128, pf.causal_mask),
        _case(1, 2, 2, 192, 192, 64, None),
        _case(1, 3, 3, 200, 200, 32, pf.sliding_window_mask(100, 20)),
        _case(2, 4, 4, 384, 704, 128, None),
        _case(2, 4, 4, 384, 704, 64, pf.causal_mask),
        _case(2, 8, 2, 640, 640, 128, _doc_mask(640, 3)),
        _case(2, 4, 4, 512, 512, 128, pf.causal_mask, per_head=4),
        _case(2, 4, 2, 520, 520, 128, pf.sliding_window_mask(200, 30), per_head=4, corrupt=True),
        _case(1, 2, 2, 1000, 1000, 64, pf.causal_mask, corrupt=True),
        # paged decode: shuffled pages with invalid ids, per-batch key counts
        _paged(8, 32, 8, 32768, 128, 512, 64, 600),
        _paged(3, 8, 2, 5000, 64, 128, 40, 100),
    ]
    path = tmp_path / "cases.bin"
    path.write_bytes(b"".join(cases))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([str(exe), str(path)], capture_output=True, text=True, env=env, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr[-4000:]
    ok, ncases, launches, checks = res.stdout.split()
    assert ok == "ok" and int(ncases) == len(cases)
    assert int(launches) > 60 and int(checks) > 10 ** 6, res.stdout
