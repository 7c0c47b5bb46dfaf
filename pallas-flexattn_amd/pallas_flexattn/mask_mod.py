"""Mask modification functions (``mask_mod.py`` of the reference).

A mask mod says which (query, key) pairs may attend.  The reference's mask
mods are plain ``(q_idx, kv_idx) -> bool`` callables (``mask_mod.py:12``); here
the built-in ones are :class:`MaskSpec` descriptors, which are also callable
with those two arguments (or PyTorch's ``(b, h, q_idx, kv_idx)``) on numpy
arrays or torch tensors, and which the MI355X kernels evaluate natively as a
fused epilogue: a window on ``delta = q - kv`` and/or equal document ids.
Arbitrary callables work everywhere too: :func:`create_block_mask` and
:func:`mha_reference` evaluate them directly, and the GPU kernels run them
after tracing (``lowering.py`` records the callable as an expression, which
is compiled into the same tile kernels at run time).
"""
from typing import Callable, Optional, Sequence, Union

import numpy as np

MaskMod = Callable  # (q_idx, kv_idx) -> bool array, or (b, h, q_idx, kv_idx) -> bool array


def _is_torch(x):
    return type(x).__module__.startswith("torch")


def _is_sym(x):
    return type(x).__name__ == "Sym" and type(x).__module__.endswith("lowering")


def _ones_like_bool(delta):
    if _is_torch(delta):
        import torch
        return torch.ones_like(delta, dtype=torch.bool)
    return np.ones(np.shape(delta), dtype=bool)


class MaskSpec:
    """Mask kept iff ``(left < 0 or q - kv <= left) and (right < 0 or kv - q <= right)
    and (doc_ids is None or doc[b, q] == doc[b, kv])``.

    ``doc_ids`` is an int array of shape (B, S) (or (S,) for one row)."""

    def __init__(self, left: int = -1, right: int = -1, doc_ids=None, name: Optional[str] = None):
        self.left = -1 if left is None or left < 0 else int(left)
        self.right = -1 if right is None or right < 0 else int(right)
        if doc_ids is not None:
            d = np.asarray(doc_ids, dtype=np.int32)
            if d.ndim == 1:
                d = d[None, :]
            if d.ndim != 2:
                raise ValueError("doc_ids must have shape (S,) or (B, S)")
            doc_ids = np.ascontiguousarray(d)
        self.doc_ids = doc_ids
        self.name = name or self._default_name()
        self._torch_docs = {}
        self._device_docs = {}
        self._cpu_docs = None

    def _default_name(self):
        parts = []
        if self.left >= 0 or self.right >= 0:
            parts.append(f"window({self.left},{self.right})")
        if self.doc_ids is not None:
            parts.append("document")
        return "&".join(parts) or "bidirectional"

    # -- properties used by block-mask construction and the kernels --------
    @property
    def has_window(self) -> bool:
        return self.left >= 0 or self.right >= 0

    @property
    def is_trivial(self) -> bool:
        return not self.has_window and self.doc_ids is None

    @property
    def batch_dependent(self) -> bool:
        return self.doc_ids is not None and self.doc_ids.shape[0] > 1

    head_dependent = False

    def doc_bounds(self):
        """(start, end) int32 arrays shaped like ``doc_ids``: token t's document
        spans [start[t], end[t]).  None unless every document is one contiguous
        run in every row (then masks are intervals for the kernels)."""
        if self.doc_ids is None:
            return None
        if not hasattr(self, "_bounds"):
            starts, ends = [], []
            ok = True
            for row in self.doc_ids:
                change = np.flatnonzero(np.diff(row)) + 1
                s = np.concatenate([[0], change])
                e = np.concatenate([change, [len(row)]])
                if len(np.unique(row[s])) != len(s):
                    ok = False
                    break
                run = np.repeat(np.arange(len(s)), e - s)
                starts.append(s[run].astype(np.int32))
                ends.append(e[run].astype(np.int32))
            self._bounds = (np.stack(starts), np.stack(ends)) if ok else None
        return self._bounds

    def key(self):
        """Hashable identity (used for caching block masks and kernel plans);
        computed once, the descriptor is immutable."""
        k = self.__dict__.get("_key")
        if k is None:
            docs = None if self.doc_ids is None else (self.doc_ids.shape, hash(self.doc_ids.tobytes()))
            k = self._key = ("MaskSpec", self.left, self.right, docs)
        return k

    def device_doc_arrays(self, device, B: int, Sq: int, Skv: int):
        """int32 device arrays the kernels read for a document mask, cached per
        (device, B, Sq, Skv): "q" (B, Sq) and "kv" (B, Skv) ids, plus "start" /
        "end" (B, Sq) run bounds when documents are contiguous runs of one
        self-attention sequence (masks are then intervals for the kernels)."""
        ck = (str(device), B, Sq, Skv)
        arrs = self._device_docs.get(ck)
        if arrs is not None:
            return arrs
        import torch
        docs = self.doc_ids
        if docs.shape[1] < max(Sq, Skv):
            raise ValueError("document ids are shorter than the sequence")
        if docs.shape[0] not in (1, B):
            raise ValueError("document ids must have 1 or B rows")
        arrs = {"q": torch.from_numpy(np.array(np.broadcast_to(docs[:, :Sq], (B, Sq)), dtype=np.int32)).to(device),
                "kv": torch.from_numpy(np.array(np.broadcast_to(docs[:, :Skv], (B, Skv)), dtype=np.int32)).to(device)}
        bounds = self.doc_bounds()
        if bounds is not None and Sq == Skv and docs.shape[1] == Sq:
            arrs["start"], arrs["end"] = (
                torch.from_numpy(np.array(np.broadcast_to(x, (B, Sq)), dtype=np.int32)).to(device) for x in bounds)
        self._device_docs[ck] = arrs
        return arrs

    def __eq__(self, other):
        return isinstance(other, MaskSpec) and self.key() == other.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return f"MaskSpec({self.name})"

    # -- evaluation ----------------------------------------------------------
    def __call__(self, *args):
        if len(args) == 2:
            b, (q_idx, kv_idx) = None, args
        elif len(args) == 4:
            b, _h, q_idx, kv_idx = args
        else:
            raise TypeError("mask mod takes (q_idx, kv_idx) or (b, h, q_idx, kv_idx)")
        if _is_sym(q_idx) or _is_sym(kv_idx):
            return self._traced(b, q_idx, kv_idx)
        delta = q_idx - kv_idx
        m = _ones_like_bool(delta)
        if self.left >= 0:
            m = m & (delta <= self.left)
        if self.right >= 0:
            m = m & (-delta <= self.right)
        if self.doc_ids is not None:
            m = m & self._same_doc(b, q_idx, kv_idx)
        return m

    def _traced(self, b, q_idx, kv_idx):
        """The mask as an expression of traced indices (when this descriptor is
        part of a callable lowered onto the kernels, e.g. and_masks(mask, fn))."""
        import torch
        delta = q_idx - kv_idx
        m = None
        if self.left >= 0:
            m = delta <= self.left
        if self.right >= 0:
            t = (-delta) <= self.right
            m = t if m is None else (m & t)
        if self.doc_ids is not None:
            if self._cpu_docs is None:
                self._cpu_docs = torch.from_numpy(self.doc_ids)
            row = 0 if b is None else b
            if b is None and self.doc_ids.shape[0] != 1:
                raise ValueError("a batch-dependent document mask needs (b, h, q_idx, kv_idx) arguments")
            t = self._cpu_docs[row, q_idx] == self._cpu_docs[row, kv_idx]
            m = t if m is None else (m & t)
        return True if m is None else m

    def _same_doc(self, b, q_idx, kv_idx):
        docs = self.doc_ids
        if b is None:
            if docs.shape[0] != 1:
                raise ValueError("a batch-dependent document mask needs (b, h, q_idx, kv_idx) arguments")
            b = 0
        if _is_torch(q_idx):
            import torch
            dev = q_idx.device
            if dev not in self._torch_docs:
                self._torch_docs[dev] = torch.as_tensor(docs, device=dev)
            t = self._torch_docs[dev]
            return t[b, q_idx.long()] == t[b, kv_idx.long()]
        return docs[b, q_idx] == docs[b, kv_idx]

    def __and__(self, other):
        return and_masks(self, other)


causal_mask = MaskSpec(-1, 0, name="causal")
"""Causal mask (``mask_mod.py:15-17``): ``q_idx >= kv_idx``."""

bidirectional_mask = MaskSpec(-1, -1, name="bidirectional")
"""Full attention (``mask_mod.py:20-22``)."""


def sliding_window_mask(left: int, right: int) -> MaskSpec:
    """Sliding window (``mask_mod.py:25-43``): with ``delta = q - kv``, keep
    ``delta <= left`` if ``left >= 0`` and ``-delta <= right`` if ``right >= 0``
    (-1 = unlimited on that side)."""
    return MaskSpec(left, right, name=f"sliding_window({left},{right})")


def _lengths_to_ids(lengths) -> np.ndarray:
    lengths = np.asarray(lengths, dtype=np.int64).reshape(-1)
    if np.any(lengths < 0):
        raise ValueError("document lengths must be non-negative")
    return np.repeat(np.arange(len(lengths), dtype=np.int32), lengths)


def document_mask(seq_lengths: Union[Sequence[int], np.ndarray, Sequence[Sequence[int]]],
                  block_size: int = 128) -> MaskSpec:
    """Packed-document mask (the reference's ``document_mask`` is a stub that
    raises, ``mask_mod.py:46-59``): tokens attend only within their document.

    ``seq_lengths`` lists the document lengths of one packed row, or one such
    list per batch row (rows must have equal totals).  ``block_size`` is kept
    for signature compatibility; block granularity is chosen by
    :func:`create_block_mask`.  Combine with :data:`causal_mask` via ``&``."""
    if len(seq_lengths) and np.ndim(seq_lengths[0]) == 1:
        rows = [_lengths_to_ids(r) for r in seq_lengths]
        if len({len(r) for r in rows}) != 1:
            raise ValueError("every batch row must pack the same number of tokens")
        ids = np.stack(rows)
    else:
        ids = _lengths_to_ids(seq_lengths)[None, :]
    return MaskSpec(doc_ids=ids, name="document")


def document_ids_mask(doc_ids) -> MaskSpec:
    """Document mask from explicit per-token document ids, shape (S,) or (B, S)."""
    return MaskSpec(doc_ids=doc_ids, name="document")


def and_masks(*mods):
    """Logical AND of mask mods.  Descriptors combine into one descriptor
    (windows intersect; at most one document term); anything else yields a
    plain callable usable on the host only."""
    if all(isinstance(m, MaskSpec) for m in mods):
        left, right, docs = -1, -1, None
        for m in mods:
            if m.left >= 0:
                left = m.left if left < 0 else min(left, m.left)
            if m.right >= 0:
                right = m.right if right < 0 else min(right, m.right)
            if m.doc_ids is not None:
                if docs is not None and not np.array_equal(docs, m.doc_ids):
                    break
                docs = m.doc_ids
        else:
            return MaskSpec(left, right, docs, name="&".join(m.name for m in mods))

    def combined(*args):
        out = mods[0](*args)
        for m in mods[1:]:
            out = out & m(*args)
        return out
    return combined
