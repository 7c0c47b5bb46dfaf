"""Kernel tuner (``kernel_tuner.py`` of the reference).

``get_optimal_params`` / ``get_kernel_config`` / ``print_kernel_config`` keep
the reference's static table and signatures (``kernel_tuner.py:11-148``).
Their four numbers are the reference's Triton knobs; :func:`kernel_tiles`
takes them as hints only: the gfx950 tiles of a call are the ones
:func:`tune` measured fastest for the shape class, else the defaults.  The
tiles are (BLOCK_M, BLOCK_N, BLOCK_KV, BLOCK_Q, NUM_STAGES): BLOCK_M query
rows per forward / dQ workgroup (32 per wave, so it sets the wave count: 2, 4
or 8), BLOCK_N keys per LDS tile, BLOCK_KV keys per dK/dV workgroup (32 per
wave), BLOCK_Q queries per dK/dV tile (64 or 128) and NUM_STAGES the K / V
tiles the forward holds in LDS at once (2; 3 with 32-key tiles, 1 with
128-key tiles).  The reference's ``num_warps`` maps onto the waves of
BLOCK_M / BLOCK_KV and its ``num_stages`` (software-pipelining depth) onto
NUM_STAGES.  Shape classes: dtype, head dim, sequence length and mask class
(dense, causal, sliding window, packed documents).

:func:`tune` measures the available instantiations on the current GPU and
stores the winners in a JSON table that ``flex_attention`` consults.
"""
import functools
import json
import os
from typing import Dict, Optional, Tuple

DEFAULT_BLOCK_R = 64
DEFAULT_BLOCK_C = 64
DEFAULT_NUM_WARPS = 4
DEFAULT_NUM_STAGES = 3


@functools.lru_cache(maxsize=128)
def get_optimal_params(
    seq_len: int,
    head_dim: int = 64,
    use_block_sparsity: bool = False,
) -> Tuple[int, int, int, int]:
    """(block_r, block_c, num_warps, num_stages) for a sequence length
    (the reference's thresholds, ``kernel_tuner.py:28-63``)."""
    if seq_len <= 256:
        block_r, block_c, num_warps, num_stages = 32, 32, 4, 2
    elif seq_len <= 512:
        block_r, block_c, num_warps, num_stages = 64, 64, 4, 3
    elif seq_len <= 2048:
        block_r, block_c, num_warps, num_stages = 128, 64, 4, 3
    elif seq_len <= 4096:
        block_r, block_c, num_warps, num_stages = 128, 128, 8, 4
    else:
        block_r, block_c, num_warps, num_stages = 128, 128, 8, 5

    if head_dim > 128:
        block_r = min(block_r, 64)
        block_c = min(block_c, 64)
        num_stages = min(num_stages, 3)
    elif head_dim <= 32:
        num_stages = max(num_stages, 4)

    if use_block_sparsity:
        block_r = min(block_r, 64)
        block_c = min(block_c, 64)

    return block_r, block_c, num_warps, num_stages


def get_kernel_config(
    batch_size: int,
    num_heads: int,
    seq_len: int,
    head_dim: int,
    mask_type: Optional[str] = None,
) -> Dict[str, int]:
    """Configuration dictionary (``kernel_tuner.py:68-101``)."""
    use_block_sparsity = mask_type in ('causal', 'sliding_window')
    block_r, block_c, num_warps, num_stages = get_optimal_params(seq_len, head_dim, use_block_sparsity)
    return {
        'batch_size': batch_size,
        'num_heads': num_heads,
        'seq_len': seq_len,
        'head_dim': head_dim,
        'block_r': block_r,
        'block_c': block_c,
        'num_warps': num_warps,
        'num_stages': num_stages,
    }


def print_kernel_config(
    batch_size: int,
    num_heads: int,
    seq_len: int,
    head_dim: int,
    mask_type: Optional[str] = None,
):
    """Print the configuration (``kernel_tuner.py:104-148``) plus the MI355X tiles it maps to."""
    config = get_kernel_config(batch_size, num_heads, seq_len, head_dim, mask_type)
    cls = {"causal": "causal", "sliding_window": "window", "document": "document"}.get(mask_type, "dense")
    bm, bn, bkv, bq, ns = resolved_tiles(kernel_tiles(config['block_r'], config['block_c'], "bf16", seq_len,
                                                      head_dim, cls), "bf16", head_dim)
    print("=" * 70)
    print("MI355X FlexAttention Kernel Configuration")
    print("=" * 70)
    print("Input Configuration:")
    print(f"  Batch size (B):   {config['batch_size']}")
    print(f"  Num heads (H):    {config['num_heads']}")
    print(f"  Seq length (T):   {config['seq_len']}")
    print(f"  Head dim (D):     {config['head_dim']}")
    if mask_type:
        print(f"  Mask type:        {mask_type}")
    print()
    print("Kernel Parameters:")
    print(f"  BLOCK_R (block_r):      {config['block_r']}")
    print(f"  BLOCK_C (block_c):      {config['block_c']}")
    print(f"  NUM_WARPS:              {config['num_warps']}")
    print(f"  NUM_STAGES:             {config['num_stages']}")
    print(f"  gfx950 tiles (bf16):    BLOCK_M={bm} ({bm // 32} waves), BLOCK_N={bn}, NUM_STAGES={ns}, "
          f"BLOCK_KV={bkv} ({bkv // 32} waves), BLOCK_Q={bq}")
    print()
    print("Usage:")
    print("  from pallas_flexattn import flash_attention")
    print("  out = flash_attention(")
    print("      q, k, v,")
    print(f"      block_r={config['block_r']},")
    print(f"      block_c={config['block_c']},")
    print(f"      num_warps={config['num_warps']},")
    print(f"      num_stages={config['num_stages']},")
    print("  )")
    print("=" * 70)


# -- MI355X tile selection ----------------------------------------------------
# A tile choice is (BLOCK_M, BLOCK_N, BLOCK_KV, BLOCK_Q, NUM_STAGES), the
# kernel_options keys of flex_attention; 0 in the last two = automatic.
TILE_NAMES = ("BLOCK_M", "BLOCK_N", "BLOCK_KV", "BLOCK_Q", "NUM_STAGES")
SUPPORTED_BLOCK_M = (64, 128, 256)
SUPPORTED_BLOCK_N = {"bf16": (32, 64, 128), "fp32": (32,)}
SUPPORTED_BLOCK_KV = {"bf16": (64, 128), "fp32": (128,)}
SUPPORTED_BLOCK_Q = {"bf16": (64, 128), "fp32": (32,)}
SUPPORTED_NUM_STAGES = {"bf16": (1, 2, 3), "fp32": (2,)}
DEFAULT_TILES = {"bf16": (128, 64, 128, 0, 0), "fp32": (128, 32, 128, 0, 0), "fp8": (128, 64, 128, 0, 0)}
MASK_CLASSES = ("dense", "causal", "window", "document")


def full_tiles(tiles, dtype: str) -> Tuple[int, int, int, int, int]:
    """A tile tuple of 3 to 5 entries completed with the defaults."""
    t = tuple(int(x) for x in tiles)
    return t + DEFAULT_TILES[dtype][len(t):]


def resolved_tiles(tiles, dtype: str, head_dim: int) -> Tuple[int, int, int, int, int]:
    """The tiles a call runs (automatic entries made explicit): BLOCK_Q 128
    for bf16 with D = 128 and BLOCK_KV 128 (the C ABI's choice under window /
    document masks and 128-row tables), else 64 (fp32: 32); 2 LDS stages."""
    bm, bn, bkv, bq, ns = full_tiles(tiles, dtype)
    if not bq:
        bq = (128 if head_dim >= 128 and bkv == 128 else 64) if dtype == "bf16" else 32
    return bm, bn, bkv, bq, ns or 2


def candidate_tiles(dtype: str, head_dim: int) -> Tuple[Tuple[int, int, int, int, int], ...]:
    """Every tile choice the library has kernels for, in resolved form.
    bf16: forward / dQ (BLOCK_M, BLOCK_N, NUM_STAGES) in 128 x 64 x 2 and
    64 x 64 x 2, for head dims >= 64 also 128 x 32 x 2, 128 x 32 x 3 (K / V
    copied two tiles ahead), 128 x 128 x 2, 128 x 128 x 1 (a single LDS buffer:
    two workgroups per CU) and 256 x 64 x 2; each with dK/dV (BLOCK_KV,
    BLOCK_Q) in 128 x 128, 128 x 64 and 64 x 64 (for D = 32 only 128 x 64: the
    DMA split needs 1 KiB per wave and tile).  fp32: 128 x 32 and 64 x 32 with
    128-key dK/dV tiles of 32 queries."""
    if dtype == "fp32":
        return ((128, 32, 128, 32, 2), (64, 32, 128, 32, 2))
    fwd = [(128, 64, 2), (64, 64, 2)]
    bwd = [(128, 64)]
    if head_dim >= 64:
        fwd += [(128, 32, 2), (128, 32, 3), (128, 128, 2), (128, 128, 1), (256, 64, 2)]
        bwd = [(128, 128), (128, 64), (64, 64)]
    return tuple((bm, bn, bkv, bq, ns) for bm, bn, ns in fwd for bkv, bq in bwd)


def tile_name(tiles) -> str:
    """Key of a candidate in the table: BLOCK_M x BLOCK_N x BLOCK_KV, then
    q BLOCK_Q and s NUM_STAGES."""
    bm, bn, bkv, bq, ns = tiles
    return f"{bm}x{bn}x{bkv}q{bq}s{ns}"


def mask_class(mask) -> str:
    """Tune-table class of a mask descriptor (None: dense): "document" with
    document ids, "window" with a left window, "causal" for q >= kv alone,
    else "dense" (bidirectional masks have no masked element)."""
    if mask is None:
        return "dense"
    if getattr(mask, "doc_ids", None) is not None:
        return "document"
    left, right = getattr(mask, "left", -1), getattr(mask, "right", -1)
    if left >= 0:
        return "window"
    if right == 0:
        return "causal"
    return "dense" if right < 0 else "window"


def kernel_tiles(block_r: int, block_c: int, dtype: str, seq_len: Optional[int] = None,
                 head_dim: Optional[int] = None, sparse=False) -> Tuple[int, int, int, int, int]:
    """Tiles for a call that came with the reference's Triton tile hints
    ``block_r`` / ``block_c``.  The hints describe a Triton schedule on
    another GPU, so they do not pick the gfx950 tiles: the tiles recorded by
    :func:`tune` for this shape class are used when there are some, else the
    defaults (bf16: 128 queries x 64 keys, 128-key dK/dV workgroups with
    automatic q tiles, two LDS stages; fp32: 128 x 32, 128).  ``sparse`` is
    a mask class (:data:`MASK_CLASSES`) or a bool (True: causal)."""
    if seq_len is not None and head_dim is not None:
        t = tuned_tiles(seq_len, head_dim, dtype, sparse)
        if t is not None:
            return t
    return DEFAULT_TILES[dtype]


TUNE_TABLE = os.environ.get(
    "FLEXATTN_TUNE_TABLE", os.path.join(os.path.dirname(os.path.abspath(__file__)), "tune_table.json"))

_TABLE_CACHE: Dict[str, Tuple[float, Dict]] = {}


def load_tune_table(path: str = TUNE_TABLE) -> Dict[str, Dict[str, int]]:
    """The tuner's JSON table (empty if absent), parsed once per file
    modification time."""
    try:
        mtime = os.path.getmtime(path)
    except OSError:
        return {}
    hit = _TABLE_CACHE.get(path)
    if hit is not None and hit[0] == mtime:
        return hit[1]
    with open(path) as f:
        table = json.load(f)
    _TABLE_CACHE[path] = (mtime, table)
    return table


def _class_of(sparse) -> str:
    if isinstance(sparse, str):
        if sparse not in MASK_CLASSES + ("sparse",):
            raise ValueError(f"unknown mask class {sparse!r} (one of {MASK_CLASSES})")
        return "causal" if sparse == "sparse" else sparse
    return "causal" if sparse else "dense"


def table_key(seq_len: int, head_dim: int, dtype: str, sparse) -> str:
    """Key of a shape class: dtype, head dim, sequence length and mask class
    (``sparse``: a class of :data:`MASK_CLASSES`, or a bool: True = causal)."""
    return f"{dtype}/D{head_dim}/S{seq_len}/{_class_of(sparse)}"


def tuned_tiles(seq_len: int, head_dim: int, dtype: str, sparse) -> Optional[Tuple[int, int, int, int, int]]:
    """Tiles recorded by :func:`tune` for this shape class, if any.  A window
    or document class without an entry of its own takes the causal entry of
    the shape (the closest measured class: a block-sparse lower triangle)."""
    cls = _class_of(sparse)
    table = load_tune_table()
    e = table.get(table_key(seq_len, head_dim, dtype, cls))
    if e is None and cls in ("window", "document"):
        e = table.get(table_key(seq_len, head_dim, dtype, "causal"))
    if e is None and cls != "dense":  # entries from before the mask classes
        e = table.get(f"{dtype}/D{head_dim}/S{seq_len}/sparse")
    if not e:
        return None
    d = DEFAULT_TILES[dtype]
    return (e["block_m"], e["block_n"], e.get("block_kv", d[2]), e.get("block_q", d[3]), e.get("num_stages", d[4]))


def _doc_lengths(seq_len: int, seed: int = 4):
    """Packed document lengths ~ Uniform[256, 4096] (the last one truncated)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out, tot = [], 0
    while tot < seq_len:
        n = min(int(rng.integers(256, 4097)), seq_len - tot)
        out.append(n)
        tot += n
    return out


def _class_mask(cls: str, seq_len: int, window: int):
    """(mask descriptor, unmasked (q, kv) pairs per (batch, head)) of a class:
    causal, causal sliding window of ``window`` keys, causal packed documents
    (lengths ~ Uniform[256, 4096], seeded), or no mask."""
    from .mask_mod import and_masks, causal_mask, document_mask, sliding_window_mask
    S = seq_len
    if cls == "causal":
        return causal_mask, S * (S + 1) / 2
    if cls == "window":
        w = min(window, S)
        return sliding_window_mask(w - 1, 0), w * (w + 1) / 2 + (S - w) * w
    if cls == "document":
        lens = _doc_lengths(S)
        return and_masks(document_mask([lens]), causal_mask), sum(n * (n + 1) / 2 for n in lens)
    return None, float(S) * S


def _tune_inputs(batch, heads, seq_len, head_dim, cls, dtype, window=1024):
    import torch
    from .block_mask import create_block_mask
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn(batch, heads, seq_len, head_dim, device=dev, dtype=dt, generator=g) for _ in range(4))
    mask, pairs = _class_mask(cls, seq_len, window)
    bm_mask = create_block_mask(mask, 1, 1, seq_len, seq_len, 128) if mask is not None else None
    return q, k, v, do, bm_mask, pairs


def run_candidate(block_m: int, block_n: int = 64, batch: int = 4, heads: int = 32, seq_len: int = 4096,
                  head_dim: int = 128, causal=True, dtype: str = "bf16", iters: int = 3,
                  backward: bool = False, block_kv: int = 128, block_q: int = 0, num_stages: int = 0,
                  window: int = 1024) -> None:
    """Run one tile candidate ``iters`` times (forward, or forward + backward)
    and nothing else: the program rocprofv3 counter passes are taken over
    (MFMA busy cycles, HBM bytes) to compare candidates.  ``causal``: a mask
    class or a bool."""
    import torch
    from .flash_attn import flex_attention
    q, k, v, do, bm_mask, _ = _tune_inputs(batch, heads, seq_len, head_dim, _class_of(causal), dtype, window)
    opts = dict(zip(TILE_NAMES, (block_m, block_n, block_kv, block_q, num_stages)))
    qq, kk, vv = (t.detach().requires_grad_(backward) for t in (q, k, v))
    for _ in range(iters):
        o = flex_attention(qq, kk, vv, block_mask=bm_mask, kernel_options=opts)
        if backward:
            o.backward(do)
    torch.cuda.synchronize()


def tune(batch: int = 4, heads: int = 32, seq_len: int = 4096, head_dim: int = 128, causal=True,
         dtype: str = "bf16", iters: int = 20, rounds: int = 3, margin: float = 0.01,
         path: str = TUNE_TABLE, window: int = 1024) -> Dict[str, int]:
    """Time every instantiated tile choice for this shape (:func:`candidate_tiles`)
    on the current GPU with hipEvents and record the fastest forward +
    backward in the JSON table under the shape class (``causal``: a class of
    :data:`MASK_CLASSES` -- the window class with ``window`` keys, the
    document class with packed documents of 256-4096 tokens -- or a bool),
    with each candidate's forward and fwd + bwd time and TFLOP/s on the
    unmasked pairs (fwd 4 D P, fwd + bwd 14 D P per head).  The axes: waves
    per forward / dQ workgroup (BLOCK_M / 32: 2, 4, 8), keys per LDS tile
    (BLOCK_N: 32, 64, 128), K / V tiles the forward holds in LDS
    (NUM_STAGES: 1 with 128-key tiles, 2, 3 with 32-key tiles; the
    reference's num_stages), waves per dK/dV workgroup (BLOCK_KV / 32: 2, 4)
    and queries per dK/dV tile (BLOCK_Q: 64, 128).  Each time is the best of
    ``rounds`` passes over all candidates in turn (``iters`` calls each), so
    clock and thermal drift does not favour one candidate.  A candidate
    replaces the default tiles only when it is faster by more than ``margin``
    (run-to-run spread on one GPU is about 1 %)."""
    import torch
    from .flash_attn import flex_attention
    cls = _class_of(causal)
    q, k, v, do, bm_mask, pairs = _tune_inputs(batch, heads, seq_len, head_dim, cls, dtype, window)
    flops_fwd = 4.0 * head_dim * pairs * batch * heads
    peak = 2516.6 if dtype == "bf16" else 157.3

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters

    # every candidate's output is checked against the default tile's before it
    # can be recorded: a tile whose kernel disagrees is skipped, not chosen
    default = resolved_tiles(DEFAULT_TILES[dtype], dtype, head_dim)
    ref = _candidate_outputs(q, k, v, do, bm_mask, dict(zip(TILE_NAMES, default)))
    tol = 2e-2 if dtype == "bf16" else 1e-5
    runs, rejected = {}, {}
    for tiles in candidate_tiles(dtype, head_dim):
        opts = dict(zip(TILE_NAMES, tiles))
        bad = _mismatch(ref, _candidate_outputs(q, k, v, do, bm_mask, opts), tol)
        if bad:
            rejected[tile_name(tiles)] = bad
            continue
        qq, kk, vv = (t.detach().requires_grad_() for t in (q, k, v))

        def fwd_only(opts=opts):
            with torch.no_grad():
                flex_attention(q, k, v, block_mask=bm_mask, kernel_options=opts)

        def fwd_bwd(opts=opts, qq=qq, kk=kk, vv=vv):
            o = flex_attention(qq, kk, vv, block_mask=bm_mask, kernel_options=opts)
            o.backward(do)

        runs[tiles] = (fwd_only, fwd_bwd)
    best_f = {t: float("inf") for t in runs}
    best_fb = dict(best_f)
    for _ in range(rounds):
        for tiles, (fwd_only, fwd_bwd) in runs.items():
            best_f[tiles] = min(best_f[tiles], timed(fwd_only))
            best_fb[tiles] = min(best_fb[tiles], timed(fwd_bwd))
    results = {}
    for tiles in runs:
        bm, bn, bkv, bq, ns = tiles
        t_f, t_fb = best_f[tiles], best_fb[tiles]
        results[tiles] = {"waves": bm // 32, "dkdv_waves": bkv // 32, "dkdv_q_tile": bq, "lds_buffers": ns,
                          "ms_fwd": round(t_f, 4), "ms_fwd_bwd": round(t_fb, 4),
                          "tflops_fwd": round(flops_fwd / t_f / 1e9, 1),
                          "tflops_fwd_bwd": round(3.5 * flops_fwd / t_fb / 1e9, 1),
                          "pct_peak_fwd_bwd": round(100 * 3.5 * flops_fwd / t_fb / 1e9 / peak, 2)}
    if not results:
        raise RuntimeError(f"tune: every candidate disagreed with the default tiles: {rejected}")
    best_tiles, best = min(results.items(), key=lambda kv: kv[1]["ms_fwd_bwd"])
    if default in results and best["ms_fwd_bwd"] > results[default]["ms_fwd_bwd"] * (1.0 - margin):
        best_tiles, best = default, results[default]
    bm, bn, bkv, bq, ns = best_tiles
    table = load_tune_table(path)
    key = table_key(seq_len, head_dim, dtype, cls)
    shape = f"B{batch} H{heads} S{seq_len} D{head_dim} {cls}" + (f" {window}" if cls == "window" else "")
    table[key] = {"block_m": bm, "block_n": bn, "block_kv": bkv, "block_q": bq, "num_stages": ns,
                  "ms_fwd_bwd": best["ms_fwd_bwd"], "margin": margin, "shape": shape,
                  "candidates": {tile_name(t): r for t, r in results.items()}}
    if rejected:
        table[key]["rejected"] = rejected
    with open(path, "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
    return table[key]


def _candidate_outputs(q, k, v, do, bm_mask, opts):
    """O, LSE, dQ, dK, dV of one candidate on the first (batch, head) slice
    of the tuning inputs (float32 copies)."""
    from .flash_attn import flex_attention
    sl = [t[:1, :1].detach().clone().requires_grad_() for t in (q, k, v)]
    o, lse = flex_attention(*sl, block_mask=bm_mask, kernel_options=opts, return_lse=True)
    o.backward(do[:1, :1])
    return [t.detach().float() for t in (o, lse, sl[0].grad, sl[1].grad, sl[2].grad)]


def _mismatch(ref, got, tol):
    """Names of the outputs outside atol = rtol = tol of the reference ones."""
    names = ("O", "LSE", "dQ", "dK", "dV")
    return [n for n, a, b in zip(names, ref, got) if not bool(((a - b).abs() <= tol + tol * a.abs()).all())]


if __name__ == "__main__":
    import argparse

    parser = argparse.ArgumentParser(description="Kernel parameters for MI355X FlexAttention")
    parser.add_argument("--batch-size", type=int, default=2)
    parser.add_argument("--num-heads", type=int, default=8)
    parser.add_argument("--seq-len", type=int, default=2048)
    parser.add_argument("--head-dim", type=int, default=64)
    parser.add_argument("--mask-type", type=str, default=None,
                        choices=['causal', 'sliding_window', 'bidirectional', 'document'])
    parser.add_argument("--window", type=int, default=1024, help="keys per sliding window (tuning)")
    parser.add_argument("--tune", action="store_true", help="measure tiles on this GPU and record them")
    parser.add_argument("--run-candidate", type=int, nargs=5, default=None,
                        metavar=("BLOCK_M", "BLOCK_N", "BLOCK_KV", "BLOCK_Q", "NUM_STAGES"),
                        help="only run these tiles (for rocprofv3 counter passes)")
    parser.add_argument("--backward", action="store_true", help="--run-candidate: forward + backward")
    parser.add_argument("--iters", type=int, default=None, help="calls per measurement (3 / 20 with --tune)")
    args = parser.parse_args()
    cls = {"causal": "causal", "sliding_window": "window", "document": "document"}.get(args.mask_type, "dense")
    if args.run_candidate is not None:
        bm, bn, bkv, bq, ns = args.run_candidate
        run_candidate(bm, bn, args.batch_size, args.num_heads, args.seq_len, args.head_dim, cls,
                      iters=args.iters or 3, backward=args.backward, block_kv=bkv, block_q=bq, num_stages=ns,
                      window=args.window)
    elif args.tune:
        print(tune(args.batch_size, args.num_heads, args.seq_len, args.head_dim, cls, iters=args.iters or 20,
                   window=args.window))
    else:
        print_kernel_config(args.batch_size, args.num_heads, args.seq_len, args.head_dim, args.mask_type)
