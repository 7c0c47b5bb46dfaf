"""Block-sparse attention masks (``block_mask.py`` of the reference).

A :class:`BlockMask` records, for each query block, which key blocks contain
at least one live (query, key) pair.  Two views are kept:

* the reference's fields ``num_blocks_in_row`` / ``col_indices`` built by the
  reference's sampling rule (bit-exact, ``block_mask.py:54-129``): a block pair
  is kept iff the mask holds at one of 3x3 sample points
  ``{start, (start+end)//2, end-1}``;
* the tables the MI355X kernels consume, classified exactly (every element
  considered): ``kv_num_blocks / kv_indices`` list the *partial* key blocks of
  each query block (element mask applied), ``full_kv_num_blocks /
  full_kv_indices`` the fully-live ones (no mask work), and the transposed
  query-side tables ``q_* / full_q_*`` drive the dK/dV kernel.  Blocks in
  neither list are skipped.

Tables are int32 numpy arrays shaped (TB, TH, rows[, width]) with TB in
{1, B}, TH in {1, H}; rows are ascending and padded with -1.
"""
import math
from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Tuple
import inspect
import warnings

import numpy as np

from .lowering import LoweredMask, LoweringError, lower_mask
from .mask_mod import MaskMod, MaskSpec


@dataclass(frozen=True)
class BlockMask:
    """Block-sparse mask (``block_mask.py:16-51`` fields, plus kernel tables).

    Attributes (reference): ``num_blocks_in_row`` (Q_BLOCKS,) and
    ``col_indices`` (Q_BLOCKS, max_blocks_per_row) int32 (with a leading
    (TB, TH) for batch/head-dependent masks), ``block_size``, ``q_len``,
    ``kv_len``."""
    num_blocks_in_row: np.ndarray
    col_indices: np.ndarray
    block_size: int
    q_len: int
    kv_len: int
    mask_mod: Optional[Callable] = None
    kv_num_blocks: Optional[np.ndarray] = None
    kv_indices: Optional[np.ndarray] = None
    full_kv_num_blocks: Optional[np.ndarray] = None
    full_kv_indices: Optional[np.ndarray] = None
    q_num_blocks: Optional[np.ndarray] = None
    q_indices: Optional[np.ndarray] = None
    full_q_num_blocks: Optional[np.ndarray] = None
    full_q_indices: Optional[np.ndarray] = None
    _device_cache: Dict = field(default_factory=dict, compare=False, repr=False)

    @property
    def num_q_blocks(self) -> int:
        """Number of query blocks (``block_mask.py:36-39``)."""
        return int(math.ceil(self.q_len / self.block_size))

    @property
    def num_kv_blocks(self) -> int:
        """Number of key/value blocks (``block_mask.py:41-44``)."""
        return int(math.ceil(self.kv_len / self.block_size))

    @property
    def sparsity(self) -> float:
        """1 - kept / possible block pairs (``block_mask.py:46-51``)."""
        nb = np.asarray(self.num_blocks_in_row)
        rows = nb.size // max(self.num_q_blocks, 1) if nb.ndim > 1 else 1
        total_possible = self.num_q_blocks * self.num_kv_blocks * rows
        actual_blocks = int(np.sum(nb))
        return 1.0 - (float(actual_blocks) / total_possible)

    # -- kernel-facing helpers ----------------------------------------------
    @property
    def has_tables(self) -> bool:
        return self.kv_num_blocks is not None

    @property
    def table_shape(self) -> Tuple[int, int]:
        return tuple(self.kv_num_blocks.shape[:2])

    def live_tiles(self) -> int:
        """Number of live (partial + full) block pairs over all table rows."""
        return int(self.kv_num_blocks.sum() + self.full_kv_num_blocks.sum())

    def device_tables(self, device):
        """The eight kernel tables as contiguous int32 torch tensors on ``device`` (cached)."""
        key = str(device)
        if key not in self._device_cache:
            import torch
            names = ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                     "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")
            self._device_cache[key] = {
                n: torch.from_numpy(np.ascontiguousarray(getattr(self, n), dtype=np.int32)).to(device)
                for n in names}
        return self._device_cache[key]


# ---------------------------------------------------------------------------
def _arity(fn) -> int:
    if isinstance(fn, MaskSpec):
        return 2
    if isinstance(fn, LoweredMask):
        return 4
    try:
        params = [p for p in inspect.signature(fn).parameters.values()
                  if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD, p.VAR_POSITIONAL)]
    except (TypeError, ValueError):
        return 2
    if any(p.kind == p.VAR_POSITIONAL for p in params):
        return 2
    return 4 if len(params) >= 4 else 2


def _call(fn, b, h, q, kv):
    if isinstance(fn, MaskSpec):
        return fn(b, h, q, kv) if fn.doc_ids is not None else fn(q, kv)
    return fn(b, h, q, kv) if _arity(fn) == 4 else fn(q, kv)


def _mask_dims(mask_mod, B: int, H: int) -> Tuple[int, int]:
    """(TB, TH): how many distinct table rows the mask needs."""
    if isinstance(mask_mod, MaskSpec):
        return (mask_mod.doc_ids.shape[0] if mask_mod.batch_dependent else 1), 1
    if isinstance(mask_mod, LoweredMask):  # tables per (b, h) for (b, h, q_idx, kv_idx) callables
        return (B, H) if mask_mod.arity == 4 else (1, 1)
    if _arity(mask_mod) == 4:
        return B, H
    return 1, 1


def _pad_rows(live: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Boolean (..., n, m) -> (counts (..., n) int32, ascending indices padded with -1)."""
    counts = live.sum(axis=-1).astype(np.int32)
    width = int(counts.max()) if counts.size else 0
    order = np.argsort(~live, axis=-1, kind="stable")[..., :width]
    idx = np.where(np.take_along_axis(live, order, axis=-1), order, -1).astype(np.int32)
    return counts, idx


def _samples(n_blocks: int, length: int, bs: int) -> np.ndarray:
    starts = np.arange(n_blocks, dtype=np.int64) * bs
    ends = np.minimum(starts + bs, length)
    return np.stack([starts, (starts + ends) // 2, ends - 1], axis=1)


def _sampled_live(mask_mod, b, h, q_len, kv_len, bs) -> np.ndarray:
    """Reference sampling rule (``block_mask.py:85-109``), vectorised: the mask is
    evaluated once on the (3*nq) x (3*nk) grid of sample points."""
    nq, nk = math.ceil(q_len / bs), math.ceil(kv_len / bs)
    qs = _samples(nq, q_len, bs).reshape(nq, 3, 1, 1)
    ks = _samples(nk, kv_len, bs).reshape(1, 1, nk, 3)
    m = np.asarray(_call(mask_mod, b, h, qs, ks), dtype=bool)
    m = np.broadcast_to(m, (nq, 3, nk, 3))
    return m.any(axis=(1, 3))


# -- exact tile classification ----------------------------------------------
def _window_classify(qa, qb, ka, kb, left, right):
    """Live / full for rectangles [qa,qb] x [ka,kb] (inclusive) under the window."""
    lo = -right if right >= 0 else -np.inf
    hi = left if left >= 0 else np.inf
    dmin, dmax = qa - kb, qb - ka
    live = np.maximum(dmin, lo) <= np.minimum(dmax, hi)
    full = (dmin >= lo) & (dmax <= hi)
    return live, full


def _runs(ids: np.ndarray):
    change = np.flatnonzero(np.diff(ids)) + 1
    starts = np.concatenate([[0], change])
    ends = np.concatenate([change, [len(ids)]])
    return starts, ends, ids[starts]


def _spec_tiles(spec: MaskSpec, row: int, q_len, kv_len, bq, bk):
    nq, nk = math.ceil(q_len / bq), math.ceil(kv_len / bk)
    qa = (np.arange(nq) * bq)[:, None]
    qb = (np.minimum((np.arange(nq) + 1) * bq, q_len) - 1)[:, None]
    ka = (np.arange(nk) * bk)[None, :]
    kb = (np.minimum((np.arange(nk) + 1) * bk, kv_len) - 1)[None, :]
    complete = (((np.arange(nq) + 1) * bq <= q_len)[:, None]) & (((np.arange(nk) + 1) * bk <= kv_len)[None, :])
    wlive, wfull = _window_classify(qa, qb, ka, kb, spec.left, spec.right)
    if spec.doc_ids is None:
        return wlive, wfull & complete
    docs = spec.doc_ids[row]
    if docs.shape[0] < max(q_len, kv_len):
        raise ValueError("doc_ids shorter than the sequence")
    qd, kd = docs[:q_len], docs[:kv_len]
    live = np.zeros((nq, nk), dtype=bool)
    qs, qe, ql = _runs(qd)
    ks, ke, kl = _runs(kd)
    for r in range(len(qs)):
        for t in np.flatnonzero(kl == ql[r]):
            i0, i1 = qs[r] // bq, (qe[r] - 1) // bq
            j0, j1 = ks[t] // bk, (ke[t] - 1) // bk
            sqa = np.maximum(qa[i0:i1 + 1], qs[r])
            sqb = np.minimum(qb[i0:i1 + 1], qe[r] - 1)
            ska = np.maximum(ka[:, j0:j1 + 1], ks[t])
            skb = np.minimum(kb[:, j0:j1 + 1], ke[t] - 1)
            l, _ = _window_classify(sqa, sqb, ska, skb, spec.left, spec.right)
            live[i0:i1 + 1, j0:j1 + 1] |= l
    # a block lies inside one document run iff its first and last token do
    q_run = np.searchsorted(qs, np.arange(q_len), side="right") - 1
    k_run = np.searchsorted(ks, np.arange(kv_len), side="right") - 1
    q_single = q_run[qa[:, 0]] == q_run[qb[:, 0]]
    k_single = k_run[ka[0]] == k_run[kb[0]]
    same = ql[q_run[qa[:, 0]]][:, None] == kl[k_run[ka[0]]][None, :]
    full = wfull & complete & q_single[:, None] & k_single[None, :] & same & live
    return live, full


def _elementwise_tiles(mask_mod, b, h, q_len, kv_len, bq, bk):
    nq, nk = math.ceil(q_len / bq), math.ceil(kv_len / bk)
    live = np.zeros((nq, nk), dtype=bool)
    full = np.zeros((nq, nk), dtype=bool)
    kv = np.arange(nk * bk)
    kv_ok = kv < kv_len
    kv_c = np.minimum(kv, kv_len - 1)
    for i in range(nq):
        q = np.arange(i * bq, (i + 1) * bq)
        q_ok = q < q_len
        m = np.broadcast_to(np.asarray(_call(mask_mod, b, h, np.minimum(q, q_len - 1)[:, None], kv_c[None, :]),
                                       dtype=bool), (bq, nk * bk))
        m = m & q_ok[:, None] & kv_ok[None, :]
        t = m.reshape(bq, nk, bk)
        live[i] = t.any(axis=(0, 2))
        full[i] = t.all(axis=(0, 2))
    return live, full


def exact_tiles(mask_mod, B: int, H: int, q_len: int, kv_len: int, bq: int, bk: int):
    """Exact (live, full) boolean arrays of shape (TB, TH, nq, nk)."""
    tb, th = _mask_dims(mask_mod, B, H)
    nq, nk = math.ceil(q_len / bq), math.ceil(kv_len / bk)
    live = np.zeros((tb, th, nq, nk), dtype=bool)
    full = np.zeros((tb, th, nq, nk), dtype=bool)
    for b in range(tb):
        for h in range(th):
            if isinstance(mask_mod, MaskSpec):
                live[b, h], full[b, h] = _spec_tiles(mask_mod, b, q_len, kv_len, bq, bk)
            else:
                live[b, h], full[b, h] = _elementwise_tiles(mask_mod, b, h, q_len, kv_len, bq, bk)
    return live, full


def kernel_tables(live: np.ndarray, full: np.ndarray) -> Dict[str, np.ndarray]:
    """Partial / full kv-side tables and their transposed q-side twins.  The
    partial and full lists of one side share a row width (at least 1), as the
    C ABI has one width per side."""
    partial = live & ~full
    out = {}
    for side, (pa, fu) in (("kv", (partial, full)),
                           ("q", (np.swapaxes(partial, -1, -2), np.swapaxes(full, -1, -2)))):
        lists = [_pad_rows(pa), _pad_rows(fu)]
        width = max(1, max(idx.shape[-1] for _, idx in lists))
        for prefix, (n, idx) in zip(("", "full_"), lists):
            pad = np.full(idx.shape[:-1] + (width - idx.shape[-1],), -1, np.int32)
            out[f"{prefix}{side}_num_blocks"] = np.ascontiguousarray(n)
            out[f"{prefix}{side}_indices"] = np.ascontiguousarray(np.concatenate([idx, pad], axis=-1))
    return out


def _finish(num, col, mask_mod, B, H, Q_LEN, KV_LEN, block_size, kernel_block=None):
    bq = bk = block_size if kernel_block is None else kernel_block
    live, full = exact_tiles(mask_mod, B, H, Q_LEN, KV_LEN, bq, bk)
    return BlockMask(num_blocks_in_row=num, col_indices=col, block_size=block_size,
                     q_len=Q_LEN, kv_len=KV_LEN, mask_mod=mask_mod, **kernel_tables(live, full))


_TABLE_NAMES = ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")


def _build_on_device(spec: MaskSpec, q_len: int, kv_len: int, bs: int, device):
    """Evaluate the block mask of a mask descriptor on the GPU (C ABI
    ``fa_build_block_mask``).  Returns the sampled (num, col) fields shaped
    (rows, 1, ...), the kernel tables (host arrays) and their device copies.
    All outputs live in one device buffer, copied to the host at once."""
    import ctypes
    import torch
    from . import _lib
    lib = _lib.load()
    dev = torch.device(device)
    rows = spec.doc_ids.shape[0] if spec.doc_ids is not None else 1
    nq, nk = math.ceil(q_len / bs), math.ceil(kv_len / bs)
    docs = None
    if spec.doc_ids is not None:
        if spec.doc_ids.shape[1] < max(q_len, kv_len):
            raise ValueError("doc_ids shorter than the sequence")
        docs = torch.from_numpy(spec.doc_ids).to(dev)
    shapes = {"sampled_num": (rows, nq), "sampled_indices": (rows, nq, nk)}
    for side, n, m in (("kv", nq, nk), ("q", nk, nq)):
        for prefix in ("", "full_"):
            shapes[f"{prefix}{side}_num_blocks"] = (rows, n)
            shapes[f"{prefix}{side}_indices"] = (rows, n, m)
    shapes["max_counts"] = (5,)
    sizes = {k: int(np.prod(v)) for k, v in shapes.items()}
    buf = torch.empty(sum(sizes.values()), dtype=torch.int32, device=dev)
    views, off = {}, 0
    for k, v in shapes.items():
        views[k] = buf[off:off + sizes[k]].view(v)
        off += sizes[k]
    args = _lib.FaMaskBuild(abi_version=_lib.ABI_VERSION, rows=rows, q_len=q_len, kv_len=kv_len, block=bs,
                            window_left=spec.left, window_right=spec.right,
                            doc_ids=docs.data_ptr() if docs is not None else None,
                            doc_len=int(spec.doc_ids.shape[1]) if docs is not None else 0,
                            **{k: t.data_ptr() for k, t in views.items()})
    ws_bytes = lib.fa_mask_build_workspace_bytes(ctypes.byref(args))
    if ws_bytes == 0:
        raise ValueError("fa_build_block_mask: sizes out of range")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.fa_build_block_mask(ctypes.byref(args), ws.data_ptr(), ws_bytes, stream))
    host = buf.cpu().numpy()  # synchronizes
    hv, off = {}, 0
    for k, v in shapes.items():
        hv[k] = host[off:off + sizes[k]].reshape(v)
        off += sizes[k]
    mc = hv["max_counts"]
    wk, wq = max(1, int(mc[1]), int(mc[2])), max(1, int(mc[3]), int(mc[4]))
    tables, dev_tables = {}, {}
    for name in _TABLE_NAMES:
        t, h = views[name], hv[name]
        if t.dim() == 3:
            w = wk if name.endswith("kv_indices") else wq
            t, h = t[..., :w], h[..., :w]
        dev_tables[name] = t.unsqueeze(1).contiguous()
        tables[name] = np.ascontiguousarray(h[:, None])
    num = np.ascontiguousarray(hv["sampled_num"][:, None])
    col = np.ascontiguousarray(hv["sampled_indices"][..., :int(mc[0])][:, None])
    return num, col, tables, dev_tables


def create_block_mask(
    mask_mod: MaskMod,
    B: int,
    H: int,
    Q_LEN: int,
    KV_LEN: int,
    block_size: int = 128,
    device=None,
) -> BlockMask:
    """Create a BlockMask from a mask_mod (``block_mask.py:54-129``).

    The reference fields follow the reference's 3x3 sampling rule exactly.
    The kernel tables classify every element; if the sampled rule misses a
    block that has live elements, a warning is issued (the kernels use the
    exact tables).  With ``device`` (a GPU) and a mask descriptor
    (:class:`MaskSpec`), both are evaluated on the device by the HIP
    library, with identical results, and the tables stay cached there."""
    if not isinstance(mask_mod, (MaskSpec, LoweredMask)) and callable(mask_mod):
        # a callable is traced once: the tables come from the expression the
        # kernels will evaluate (callables that cannot be traced are called
        # directly on numpy index arrays)
        try:
            mask_mod = lower_mask(mask_mod)
        except LoweringError:
            pass
    if device is not None and isinstance(mask_mod, MaskSpec):
        num, col, tables, dev_tables = _build_on_device(mask_mod, Q_LEN, KV_LEN, block_size, device)
        if num.shape[0] == 1:
            num, col = num[0, 0], col[0, 0]
        bm = BlockMask(num_blocks_in_row=np.ascontiguousarray(num), col_indices=np.ascontiguousarray(col),
                       block_size=block_size, q_len=Q_LEN, kv_len=KV_LEN, mask_mod=mask_mod, **tables)
        bm._device_cache[str(device)] = dev_tables
        _warn_if_sampling_misses(int(np.sum(num)), bm)
        return bm
    tb, th = _mask_dims(mask_mod, B, H)
    sampled = np.stack([np.stack([_sampled_live(mask_mod, b, h, Q_LEN, KV_LEN, block_size)
                                  for h in range(th)]) for b in range(tb)])
    num, col = _pad_rows(sampled)
    if tb == 1 and th == 1:
        num, col = num[0, 0], col[0, 0]
    bm = _finish(np.ascontiguousarray(num), np.ascontiguousarray(col), mask_mod, B, H, Q_LEN, KV_LEN, block_size)
    _warn_if_sampling_misses(int(sampled.sum()), bm)
    return bm


def _warn_if_sampling_misses(sampled_live: int, bm: BlockMask) -> None:
    exact_live = int((bm.kv_num_blocks + bm.full_kv_num_blocks).sum())
    if exact_live != sampled_live:
        warnings.warn("create_block_mask: the 3x3 sampling rule and the exact classification disagree "
                      f"({sampled_live} vs {exact_live} live blocks); kernels use the exact tables",
                      stacklevel=3)


def _closed_form(rows, n):
    live = np.zeros((n, n), dtype=bool)
    for i, (a, b) in enumerate(rows):
        live[i, a:b] = True
    return _pad_rows(live)


def create_causal_block_mask(seq_len: int, block_size: int = 128) -> BlockMask:
    """Causal BlockMask (``block_mask.py:132-172``): query block i attends to key
    blocks 0..i."""
    from .mask_mod import causal_mask
    n = math.ceil(seq_len / block_size)
    num, col = _closed_form([(0, i + 1) for i in range(n)], n)
    return _finish(num, col, causal_mask, 1, 1, seq_len, seq_len, block_size)


def create_sliding_window_block_mask(seq_len: int, window_size: int, block_size: int = 128) -> BlockMask:
    """Sliding-window BlockMask (``block_mask.py:175-218``): query block i attends
    to key blocks ``max(0, i-wb) .. min(n, i+wb+1)-1`` with ``wb = ceil(window/block)``.
    The element mask is ``sliding_window_mask(window_size, window_size)``."""
    from .mask_mod import sliding_window_mask
    n = math.ceil(seq_len / block_size)
    wb = math.ceil(window_size / block_size)
    num, col = _closed_form([(max(0, i - wb), min(n, i + wb + 1)) for i in range(n)], n)
    return _finish(num, col, sliding_window_mask(window_size, window_size), 1, 1, seq_len, seq_len, block_size)
