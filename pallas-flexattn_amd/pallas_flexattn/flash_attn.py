"""FlexAttention on MI355X: host side of ``flash_attn.py`` of the reference.

Input shapes: q (B, Hq, T, D); k, v (B, Hkv, T, D) with Hq % Hkv == 0
(grouped-query attention; the reference requires Hq == Hkv).  Tensors are
torch tensors on the GPU (bf16 or fp32); the kernels run through the C ABI of
libflexattn.so on the current torch stream.

Entry points keep the reference's signatures:

* :func:`flash_attention` (``flash_attn.py:464-504``): differentiable output
  (a ``torch.autograd.Function`` replaces ``jax.custom_vjp``; the residuals are
  ``(q, k, v, o, lse)`` as at ``:487``, with the LSE kept in fp32),
* :func:`flash_attention_fwd` (``:111-165``) -> ``(o, lse)``, LSE returned in q's
  dtype as the reference does (``:144``),
* :func:`flash_attention_bwd` (``:410-461``) -> ``(dq, dk, dv)``,
* :func:`mha_reference` (``:33-56``): materialised attention,

plus the FlexAttention front door :func:`flex_attention` (``score_mod``,
``block_mask``, ``scale``, ``enable_gqa``, ``return_lse``, ``kernel_options``).

``interpret=True`` selected the Pallas interpreter on the host in the
reference; here it runs the library's host twins (``fa_fwd_host`` /
``fa_bwd_*_host``) on CPU tensors.  Problems without queries or keys launch
nothing: empty outputs, or O = 0 and LSE = -inf when there are no keys.
"""
import math
import os
from typing import Optional, Tuple

import numpy as np

from . import _lib, lowering
from .block_mask import BlockMask, _finish, create_block_mask
from .kernel_tuner import (DEFAULT_BLOCK_C, DEFAULT_BLOCK_R, DEFAULT_NUM_STAGES, DEFAULT_NUM_WARPS, DEFAULT_TILES,
                           TILE_NAMES, full_tiles, kernel_tiles, mask_class, tuned_tiles)
from .mask_mod import MaskSpec, MaskMod, and_masks, causal_mask, document_ids_mask
from .score_mod import ScoreSpec

# Granularity of the block tables built internally: a multiple of every
# kernel tile up to 128 (64/128 queries, 32/64/128 keys, 64/128-key dK/dV
# tiles); 256-row query tiles get tables at 256.
TABLE_BLOCK = 128


def _torch():
    import torch
    return torch


def _dtype_code(t):
    torch = _torch()
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16, "bf16"
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32, "fp32"
    if t.dtype == torch.float8_e4m3fn:
        return _lib.DTYPE_FP8_E4M3, "fp8"
    raise TypeError(f"unsupported dtype {t.dtype}: the MI355X kernels take bfloat16 or float32")


def _check_interpret(interpret, t):
    """Whether a call runs on the host: interpret=True (the reference's Pallas
    interpreter on the CPU) runs the library's host twins (fa_*_host) on CPU
    tensors; the GPU path takes GPU tensors only (no fallback either way)."""
    if interpret and t.is_cuda:
        raise ValueError("interpret=True executes on the host: pass CPU tensors (GPU tensors run with "
                         "interpret=False)")
    return bool(interpret)


def _check_inputs(q, k, v, host=False):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (B, H, T, D)")
    if host:
        if q.is_cuda or k.is_cuda or v.is_cuda:
            raise ValueError("the host path (interpret=True) takes CPU tensors")
    elif not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be GPU tensors (CPU tensors run with interpret=True)")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, v must share a dtype")
    B, Hq, Sq, D = q.shape
    if k.shape[0] != B or v.shape[0] != B or k.shape[3] != D or v.shape[3] != D:
        raise ValueError("batch / head-dim mismatch between q, k, v")
    if k.shape[1] != v.shape[1] or k.shape[2] != v.shape[2]:
        raise ValueError("k and v must have the same shape")
    if Hq % k.shape[1] != 0:
        raise ValueError("number of q heads must be a multiple of the number of kv heads")


class _Plan:
    """Everything the C ABI needs besides the tensors: an fa_params struct
    plus the device arrays its pointers refer to (kept alive here).  Plans
    are cached (:func:`_get_plan`): a call with the same shapes, mask, score
    mod, scale, block mask and tiles reuses the struct and the device arrays,
    so repeated calls make no host-to-device copies."""

    def __init__(self, q, k, mask: Optional[MaskSpec], score: Optional[ScoreSpec], scale: Optional[float],
                 block_mask: Optional[BlockMask], tiles: Tuple[int, ...]):
        B, Hq, Sq, D = q.shape
        Hkv, Skv = k.shape[1], k.shape[2]
        code, dname = _dtype_code(q)
        p = _lib.FaParams()
        p.abi_version = _lib.ABI_VERSION
        p.dtype = code
        p.B, p.Hq, p.Hkv, p.Sq, p.Skv, p.D = B, Hq, Hkv, Sq, Skv, D
        p.block_m, p.block_n, p.block_kv = tiles[:3]
        p.block_q = tiles[3] if len(tiles) > 3 else 0
        p.lds_stages = tiles[4] if len(tiles) > 4 else 0
        p.scale = 0.0 if scale is None else float(scale)
        p.window_left = p.window_right = -1
        self.keep = []
        dev = q.device
        if mask is not None:
            p.window_left, p.window_right = mask.left, mask.right
            if mask.doc_ids is not None:
                arrs = mask.device_doc_arrays(dev, B, Sq, Skv)
                self.keep.append(arrs)
                p.q_doc_ids, p.kv_doc_ids = arrs["q"].data_ptr(), arrs["kv"].data_ptr()
                if "start" in arrs:
                    p.doc_start, p.doc_end = arrs["start"].data_ptr(), arrs["end"].data_ptr()
        if score is not None:
            if score.alibi is not None:
                if score.alibi.shape[0] != Hq:
                    raise ValueError(f"ALiBi needs one slope per q head ({Hq}), got {score.alibi.shape[0]}")
                ts = score.device_slopes(dev)
                self.keep.append(ts)
                p.alibi_slopes = ts.data_ptr()
            p.softcap = score.softcap
        if block_mask is not None:
            if block_mask.q_len != Sq or block_mask.kv_len != Skv:
                raise ValueError(f"block mask built for ({block_mask.q_len}, {block_mask.kv_len}), "
                                 f"inputs are ({Sq}, {Skv})")
            bs = block_mask.block_size
            if bs % tiles[0] or bs % tiles[1] or bs % tiles[2] or bs % 128:
                raise ValueError(f"block_size {bs} must be a multiple of 128 and of the kernel tiles {tiles}")
            tb, th = block_mask.table_shape
            if tb not in (1, B) or th not in (1, Hq):
                raise ValueError("block mask tables do not broadcast over (B, H)")
            t = block_mask.device_tables(dev)
            self.keep.append(t)
            p.mask_block_q = p.mask_block_kv = bs
            p.table_b, p.table_h = tb, th
            p.kv_width = t["kv_indices"].shape[-1]
            p.q_width = t["q_indices"].shape[-1]
            for name in t:
                setattr(p, name, t[name].data_ptr())
        self.params = p
        self.dname = dname
        import ctypes
        self._ref = ctypes.byref(self.params)

    def ptr(self):
        return self._ref


_PLAN_CACHE = {}
_PLAN_CACHE_MAX = 128


def _get_plan(q, k, mask, score, scale, block_mask, tiles) -> _Plan:
    """Cached :class:`_Plan` for this call.  Keyed on everything the struct
    depends on; a block mask is keyed by identity and the cache entry holds a
    reference to it, so the key stays unique while the entry lives."""
    key = (tuple(q.shape), tuple(k.shape), q.dtype, str(q.device),
           None if mask is None else mask.key(), None if score is None else score.key(),
           scale, None if block_mask is None else id(block_mask), tuple(tiles))
    hit = _PLAN_CACHE.get(key)
    if hit is not None and hit[1] is block_mask:
        return hit[0]
    plan = _Plan(q, k, mask, score, scale, block_mask, tiles)
    if len(_PLAN_CACHE) >= _PLAN_CACHE_MAX:
        _PLAN_CACHE.pop(next(iter(_PLAN_CACHE)))
    _PLAN_CACHE[key] = (plan, block_mask)
    return plan


_MASK_CACHE = {}


def _internal_block_mask(mask: MaskSpec, B: int, Sq: int, Skv: int, device=None,
                         block: int = TABLE_BLOCK) -> BlockMask:
    """Tables for a mask given without a BlockMask, built on ``device`` when it is a GPU."""
    on_gpu = device is not None and getattr(device, "type", str(device)) == "cuda"
    key = (mask.key(), B, Sq, Skv, str(device) if on_gpu else None, block)
    bm = _MASK_CACHE.get(key)
    if bm is None:
        if on_gpu:
            bm = create_block_mask(mask, B, 1, Sq, Skv, block, device=device)
        else:
            bm = _finish(None, None, mask, B, 1, Sq, Skv, block)
        if len(_MASK_CACHE) > 64:
            _MASK_CACHE.clear()
        _MASK_CACHE[key] = bm
    return bm


def _as_mask_spec(mask_mod) -> Optional[MaskSpec]:
    """The built-in descriptor of a mask mod (None for callables, which are lowered)."""
    mask, _, _ = _resolve(mask_mod, None)
    return mask


_LOWERED = {}


def _lowered(fn, kind):
    """The traced form of a callable, cached per callable object."""
    hit = _LOWERED.get((kind, id(fn)))
    if hit is not None and hit[0] is fn:
        return hit[1]
    try:
        low = lowering.lower_mask(fn) if kind == "mask" else lowering.lower_score(fn)
    except lowering.LoweringError as e:
        raise NotImplementedError(f"this {kind}_mod cannot be lowered onto the MI355X kernels: {e}") from e
    if len(_LOWERED) > 256:
        _LOWERED.clear()
    _LOWERED[(kind, id(fn))] = (fn, low)
    return low


_MODS = {}


def _resolve(mask_mod, score_mod):
    """(mask descriptor, score descriptor, user mods) for a call.  Built-in
    descriptors (MaskSpec, ScoreSpec) run as the kernels' fused epilogues;
    any other callable is traced and lowered onto the kernels (run-time
    compiled element policy).  A document-label mask next to a user score mod
    is lowered too (the bf16 tile kernels take documents only as intervals)."""
    mask = score = None
    lmask = lscore = None
    if mask_mod is not None:
        if isinstance(mask_mod, MaskSpec):
            mask = mask_mod
        else:
            lmask = _lowered(mask_mod, "mask")
            if lmask.is_trivial:
                lmask = None
    if score_mod is not None:
        if isinstance(score_mod, ScoreSpec):
            score = None if (score_mod.alibi is None and score_mod.softcap == 0) else score_mod
        else:
            lscore = _lowered(score_mod, "score")
    if lscore is not None and mask is not None and mask.doc_ids is not None and mask.doc_bounds() is None:
        lmask, mask = _lowered(mask, "mask"), None
    if lmask is None and lscore is None:
        return mask, score, None
    key = (id(lmask), id(lscore))
    hit = _MODS.get(key)
    if hit is None or hit[0] is not lmask or hit[1] is not lscore:
        if len(_MODS) > 256:
            _MODS.clear()
        hit = _MODS[key] = (lmask, lscore, lowering.UserMods(lmask, lscore))
    return mask, score, hit[2]


def _as_score_spec(score_mod) -> Optional[ScoreSpec]:
    _, score, _ = _resolve(None, score_mod)
    return score


_HANDLES = {}


def _lib_identity():
    """Identifies the kernel headers the library compiles user mods from (a
    blob built from other headers does not load): the ABI version and the
    library's hash of its embedded headers."""
    return f"abi{_lib.ABI_VERSION}-{_lib.load().fa_mods_source_hash():016x}"


def _mods_handle(mods, dtype_code, D, flags, device):
    """Loaded kernels (C ABI fa_mods) for a policy on a device: compiled once
    per process, the code blob kept in a disk cache across processes
    ($FLEXATTN_CACHE_DIR, default ~/.cache/pallas_flexattn)."""
    import ctypes
    import hashlib
    dev = _torch().device(device)
    idx = dev.index if dev.index is not None else _torch().cuda.current_device()
    key = (mods.digest, dtype_code, D, flags, idx)
    h = _HANDLES.get(key)
    if h is not None:
        return h
    lib = _lib.load()
    tag = hashlib.sha256(f"{mods.source}|{dtype_code}|{D}|{flags}|{_lib_identity()}".encode()).hexdigest()
    cache_dir = os.environ.get("FLEXATTN_CACHE_DIR") or os.path.join(os.path.expanduser("~"), ".cache",
                                                                     "pallas_flexattn")
    path = os.path.join(cache_dir, f"mods-{tag}.blob")
    blob = None
    if os.path.exists(path):
        with open(path, "rb") as f:
            blob = f.read()
    if blob is None:
        blob = _lib.compile_mods(mods.source, dtype_code, D, flags)
        try:
            os.makedirs(cache_dir, exist_ok=True)
            tmp = f"{path}.{os.getpid()}.tmp"
            with open(tmp, "wb") as f:
                f.write(blob)
            os.replace(tmp, path)
        except OSError:
            pass  # the cache is an optimisation only
    handle = ctypes.c_void_p()
    with _torch().cuda.device(idx):
        _lib.check(lib.fa_mods_load(blob, len(blob), ctypes.byref(handle)))
    _HANDLES[key] = handle
    return handle


def _mods_args(mods, plan, q, score):
    """(handle, buffer-pointer array, count) for a launch with user mods."""
    import ctypes
    bufs = mods.device_buffers(q.device)
    arr = (ctypes.c_void_p * max(1, len(bufs)))(*[b.data_ptr() for b in bufs])
    code, _ = _dtype_code(q)
    flags = mods.flags(builtin_score=score is not None)
    return _mods_handle(mods, code, q.shape[3], flags, q.device), arr, len(bufs)


def _user_block_mask(lmask, B, H, Sq, Skv, block: int = TABLE_BLOCK):
    """Exact tables of a lowered mask at the kernels' table granularity
    (evaluated on the host from the traced expression), cached."""
    key = ("user", id(lmask), B, H, Sq, Skv, block)
    hit = _MASK_CACHE.get(key)
    if hit is None or hit[0] is not lmask:
        if len(_MASK_CACHE) > 64:
            _MASK_CACHE.clear()
        hit = _MASK_CACHE[key] = (lmask, create_block_mask(lmask, B, H, Sq, Skv, block))
    return hit[1]


def _tables_for(mask, mods, block_mask, q, k, tiles):
    """(block mask, tiles) of a call: the caller's tables, or ones built for
    its mask, at a block size every kernel tile divides: 128, or the query
    tile when that is larger (256-row tiles).  A caller's tables at another
    size are re-derived where the mask is known; otherwise the query tile
    drops to 128 rows."""
    blk = max(TABLE_BLOCK, tiles[0])
    if block_mask is not None:
        if block_mask.block_size % blk == 0:
            return block_mask, tiles
        if mask is not None and not mask.is_trivial:
            return _internal_block_mask(mask, q.shape[0], q.shape[2], k.shape[2], q.device, blk), tiles
        if mods is not None and mods.mask is not None:
            return _user_block_mask(mods.mask, q.shape[0], q.shape[1], q.shape[2], k.shape[2], blk), tiles
        if tiles[0] > TABLE_BLOCK:
            return block_mask, (TABLE_BLOCK,) + tuple(tiles[1:])
        return block_mask, tiles  # the plan reports the mismatch
    if mask is not None and not mask.is_trivial:
        return _internal_block_mask(mask, q.shape[0], q.shape[2], k.shape[2], q.device, blk), tiles
    if mods is not None and mods.mask is not None:
        return _user_block_mask(mods.mask, q.shape[0], q.shape[1], q.shape[2], k.shape[2], blk), tiles
    return None, tiles


_RAW_STREAM = None


def _stream():
    """Handle of torch's current stream on the current device.  torch's
    current_stream() builds a Stream object per call (~20 us); the raw
    handle getters it wraps are used directly where present."""
    global _RAW_STREAM
    if _RAW_STREAM is None:
        c = _torch()._C
        if hasattr(c, "_cuda_getCurrentRawStream") and hasattr(c, "_cuda_getDevice"):
            get, dev = c._cuda_getCurrentRawStream, c._cuda_getDevice
            _RAW_STREAM = lambda: get(dev())  # noqa: E731
        else:
            _RAW_STREAM = lambda: _torch().cuda.current_stream().cuda_stream  # noqa: E731
    return _RAW_STREAM()


def _dense16(t):
    """Contiguous with a 16-byte aligned base (the kernels use 16-byte loads)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _host_mods(mods):
    if mods is not None:
        raise NotImplementedError("interpret=True runs the built-in mask / score descriptors on the host; "
                                  "traced callables run on the GPU (interpret=False)")


def _fwd_core(q, k, v, mask, score, scale, block_mask, tiles, mods=None, host=False):
    """Forward through fa_fwd (fa_mods_fwd with user mods; fa_fwd_host on the
    host path) -> (o, lse fp32, plan)."""
    torch = _torch()
    _check_inputs(q, k, v, host)
    if host:
        _host_mods(mods)
    if q.numel() == 0 or k.shape[2] == 0:
        # nothing to launch: no queries (empty outputs), or no keys (every
        # row sees none: O = 0, LSE = -inf, as for fully masked rows)
        o = torch.zeros_like(q)
        lse = torch.full(q.shape[:3], -math.inf, device=q.device, dtype=torch.float32)
        return o, lse, None
    q, k, v = _dense16(q), _dense16(k), _dense16(v)
    if mods is not None:
        tiles = _MODS_TILES[_dtype_code(q)[1]]
    block_mask, tiles = _tables_for(mask, mods, block_mask, q, k, tiles)
    plan = _get_plan(q, k, mask, score, scale, block_mask, tiles)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr())
    if host:
        _lib.check(lib.fa_fwd_host(plan.ptr(), *ptrs, 0))
    elif mods is None:
        _lib.check(lib.fa_fwd(plan.ptr(), *ptrs, _stream()))
    else:
        h, bufs, n = _mods_args(mods, plan, q, score)
        _lib.check(lib.fa_mods_fwd(h, plan.ptr(), bufs, n, *ptrs, _stream()))
    return o, lse, plan


def _bwd_core(q, k, v, o, lse, do, mask, score, scale, block_mask, tiles, mods=None, host=False, plan=None):
    """Backward through fa_bwd (fa_mods_bwd with user mods; fa_bwd_host on
    the host path) -> (dq, dk, dv).  ``plan`` is the forward's plan when the
    caller has it (same problem), else one is looked up."""
    torch = _torch()
    _check_inputs(q, k, v, host)
    if host:
        _host_mods(mods)
    if q.numel() == 0 or k.shape[2] == 0:  # no (query, key) pair: zero gradients
        return torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    q, k, v, o, do = (_dense16(t) for t in (q, k, v, o, do))
    if lse.dtype != torch.float32 or not lse.is_contiguous():
        lse = lse.to(torch.float32).contiguous()
    if o.shape != q.shape or do.shape != q.shape or lse.shape != q.shape[:3]:
        raise ValueError("o / do / lse shapes do not match q")
    if plan is None:
        if mods is not None:
            tiles = _MODS_TILES[_dtype_code(q)[1]]
        block_mask, tiles = _tables_for(mask, mods, block_mask, q, k, tiles)
        plan = _get_plan(q, k, mask, score, scale, block_mask, tiles)
    lib = _lib.load()
    if host:
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        _lib.check(lib.fa_bwd_host(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   lse.data_ptr(), do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), 0))
        return dq, dk, dv
    ws_bytes = lib.fa_bwd_workspace_bytes(plan.ptr())
    ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(), dq.data_ptr(),
            dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel())
    if mods is None:
        _lib.check(lib.fa_bwd(plan.ptr(), *ptrs, _stream()))
    else:
        h, bufs, n = _mods_args(mods, plan, q, score)
        _lib.check(lib.fa_mods_bwd(h, plan.ptr(), bufs, n, *ptrs, _stream()))
    return dq, dk, dv


# tiles of the run-time compiled kernels (fixed at compile time)
_MODS_TILES = {"bf16": (128, 64, 128), "fp32": (128, 32, 128)}


class _AnyMask:
    """Stands for a traced user mask when picking tiles (causal class)."""
    left, right, doc_ids = -1, 0, None


_ANY_MASK = _AnyMask()


def _ref_tiles(q, block_r, block_c, mask=None):
    """Kernel tiles of a reference-signature call: block_r / block_c are
    Triton hints; the tuned tiles for the shape class (or the defaults) run."""
    _, dname = _dtype_code(q)
    return kernel_tiles(block_r, block_c, dname, q.shape[2], q.shape[3], mask_class(mask))


def _as4d(t):
    """(B*H, T, C) flattened arrays of the reference's stage functions -> (B*H, 1, T, C)."""
    return t.unsqueeze(1) if t.dim() == 3 else t


def _stage_plan(q4, k4, mask_mod, block_r, block_c, scale=None):
    """(plan, user mods) of a reference-signature backward stage."""
    mask, _, mods = _resolve(mask_mod, None)
    tiles = _MODS_TILES[_dtype_code(q4)[1]] if mods is not None else \
        _ref_tiles(q4, block_r, block_c, mask if mods is None or mods.mask is None else _ANY_MASK)
    bm, tiles = _tables_for(mask, mods, None, q4, k4, tiles)
    return _get_plan(q4, k4, mask, None, scale, bm, tiles), mods


def flash_attention_bwd_preprocess(o_flat, do_flat, block_r: int = DEFAULT_BLOCK_R,
                                   num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                                   interpret: bool = False):
    """Delta = rowsum(O * dO) (``flash_attn.py:168-203``), shape o.shape[:-1].
    Returned in fp32 (the reference stores it in O's dtype)."""
    host = _check_interpret(interpret, o_flat)
    torch = _torch()
    o4, do4 = _dense16(_as4d(o_flat)), _dense16(_as4d(do_flat).to(o_flat.dtype))
    plan, _ = _stage_plan(o4, o4, None, block_r, DEFAULT_BLOCK_C)
    delta = torch.empty(o4.shape[:3], device=o4.device, dtype=torch.float32)
    if host:
        _lib.check(_lib.load().fa_bwd_preprocess_host(plan.ptr(), o4.data_ptr(), do4.data_ptr(),
                                                      delta.data_ptr(), 0))
    else:
        _lib.check(_lib.load().fa_bwd_preprocess(plan.ptr(), o4.data_ptr(), do4.data_ptr(), delta.data_ptr(),
                                                 _stream()))
    return delta.reshape(o_flat.shape[:-1])


def _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale, softmax_scale, host=False):
    torch = _torch()
    if abs(qk_scale - softmax_scale) > 1e-12 * max(abs(qk_scale), 1.0):
        raise NotImplementedError("the kernels apply one softmax scale to both S and dS")
    q4, k4, v4 = (_dense16(_as4d(t)) for t in (q_flat, k_flat, v_flat))
    _check_inputs(q4, k4, v4, host)
    do4 = _dense16(_as4d(do_flat).to(q4.dtype))
    lse = logsumexp_flat.to(torch.float32).reshape(q4.shape[:3]).contiguous()
    delta = d_flat.to(torch.float32).reshape(q4.shape[:3]).contiguous()
    return q4, k4, v4, do4, lse, delta


def flash_attention_bwd_dkv(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale: float,
                            softmax_scale: float, block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                            num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                            mask_mod: Optional[MaskMod] = None, interpret: bool = False):
    """dK, dV (``flash_attn.py:206-310``) from q, k, v, dO, LSE and Delta."""
    host = _check_interpret(interpret, q_flat)
    torch = _torch()
    q4, k4, v4, do4, lse, delta = _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat,
                                                qk_scale, softmax_scale, host)
    plan, mods = _stage_plan(q4, k4, mask_mod, block_r, block_c, qk_scale)
    dk, dv = torch.empty_like(k4), torch.empty_like(v4)
    ptrs = (q4.data_ptr(), k4.data_ptr(), v4.data_ptr(), do4.data_ptr(), lse.data_ptr(), delta.data_ptr(),
            dk.data_ptr(), dv.data_ptr())
    if host:
        _host_mods(mods)
        _lib.check(_lib.load().fa_bwd_dkdv_host(plan.ptr(), *ptrs, 0))
    elif mods is None:
        _lib.check(_lib.load().fa_bwd_dkdv(plan.ptr(), *ptrs, _stream()))
    else:
        h, bufs, n = _mods_args(mods, plan, q4, None)
        _lib.check(_lib.load().fa_mods_bwd_dkdv(h, plan.ptr(), bufs, n, *ptrs, _stream()))
    return dk.reshape(k_flat.shape), dv.reshape(v_flat.shape)


def flash_attention_bwd_dq(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale: float,
                           softmax_scale: float, block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                           num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                           mask_mod: Optional[MaskMod] = None, interpret: bool = False):
    """dQ (``flash_attn.py:313-407``) from q, k, v, dO, LSE and Delta."""
    host = _check_interpret(interpret, q_flat)
    torch = _torch()
    q4, k4, v4, do4, lse, delta = _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat,
                                                qk_scale, softmax_scale, host)
    plan, mods = _stage_plan(q4, k4, mask_mod, block_r, block_c, qk_scale)
    dq = torch.empty_like(q4)
    ptrs = (q4.data_ptr(), k4.data_ptr(), v4.data_ptr(), do4.data_ptr(), lse.data_ptr(), delta.data_ptr(),
            dq.data_ptr())
    if host:
        _host_mods(mods)
        _lib.check(_lib.load().fa_bwd_dq_host(plan.ptr(), *ptrs, 0))
    elif mods is None:
        _lib.check(_lib.load().fa_bwd_dq(plan.ptr(), *ptrs, _stream()))
    else:
        h, bufs, n = _mods_args(mods, plan, q4, None)
        _lib.check(_lib.load().fa_mods_bwd_dq(h, plan.ptr(), bufs, n, *ptrs, _stream()))
    return dq.reshape(q_flat.shape)


class Runner:
    """Pre-planned kernel launches for repeated calls on fixed shapes (used by
    the benchmark): the fa_params struct, block tables and outputs are built
    once; each call only enqueues kernels on the current stream."""

    def __init__(self, q, k, v, do, mask_mod=None, score_mod=None, block_mask=None, scale=None, tiles=None):
        torch = _torch()
        _check_inputs(q, k, v)
        self.q, self.k, self.v = _dense16(q), _dense16(k), _dense16(v)
        self.do = _dense16(do)
        mask, score, mods = _resolve(mask_mod if block_mask is None else block_mask.mask_mod, score_mod)
        if mods is not None:
            raise NotImplementedError("Runner takes the built-in mask / score descriptors; use flex_attention for "
                                      "user callables")
        _, dname = _dtype_code(q)
        if tiles is None:  # the tuned tiles of the shape class, as flex_attention picks them
            tiles = tuned_tiles(q.shape[2], q.shape[3], dname, mask_class(mask)) or DEFAULT_TILES[dname]
        tiles = full_tiles(tiles, dname)
        block_mask, tiles = _tables_for(mask, None, block_mask, self.q, self.k, tiles)
        self.plan = _Plan(self.q, self.k, mask, score, scale, block_mask, tiles)
        self.block_mask = block_mask
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        self.delta = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        self.dq, self.dk, self.dv = torch.empty_like(self.q), torch.empty_like(self.k), torch.empty_like(self.v)
        self.lib = _lib.load()
        # fa_bwd's workspace holds Delta (B, Hq, Sq) fp32
        self.ws = torch.empty(max(self.lib.fa_bwd_workspace_bytes(self.plan.ptr()), 256), device=q.device,
                              dtype=torch.uint8)

    def fwd(self):
        _lib.check(self.lib.fa_fwd(self.plan.ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                                   self.o.data_ptr(), self.lse.data_ptr(), _stream()))

    def preprocess(self):
        _lib.check(self.lib.fa_bwd_preprocess(self.plan.ptr(), self.o.data_ptr(), self.do.data_ptr(),
                                              self.delta.data_ptr(), _stream()))

    def dkdv(self):
        _lib.check(self.lib.fa_bwd_dkdv(self.plan.ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                                        self.do.data_ptr(), self.lse.data_ptr(), self.delta.data_ptr(),
                                        self.dk.data_ptr(), self.dv.data_ptr(), _stream()))

    def dq_(self):
        _lib.check(self.lib.fa_bwd_dq(self.plan.ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                                      self.do.data_ptr(), self.lse.data_ptr(), self.delta.data_ptr(),
                                      self.dq.data_ptr(), _stream()))

    def bwd(self):
        """The whole backward (fa_bwd): for bf16 interval masks the dQ kernel
        computes Delta, then dK/dV; otherwise Delta, dK/dV, dQ."""
        _lib.check(self.lib.fa_bwd(self.plan.ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                                   self.o.data_ptr(), self.lse.data_ptr(), self.do.data_ptr(), self.dq.data_ptr(),
                                   self.dk.data_ptr(), self.dv.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                                   _stream()))

    def step(self):
        """One forward + backward pass."""
        self.fwd()
        self.bwd()


# ------------------------------------------------------------ public API ----
def mha_reference(q, k, v, mask_mod: Optional[MaskMod] = None):
    """Materialised attention (``flash_attn.py:33-56``): ``softmax(where(mask,
    q k^T / sqrt(d), -inf)) v`` computed in the input dtype with torch ops.
    Accepts any mask mod callable (and GQA inputs)."""
    torch = _torch()
    d = q.shape[-1]
    g = q.shape[1] // k.shape[1]
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(d)
    T, S = q.shape[2], k.shape[2]
    if mask_mod is not None:
        q_idx = torch.arange(T, device=q.device)[:, None]
        kv_idx = torch.arange(S, device=q.device)[None, :]
        mask = mask_mod(q_idx, kv_idx)
        logits = torch.where(mask, logits, torch.tensor(float("-inf"), dtype=logits.dtype, device=q.device))
    probs = torch.softmax(logits, dim=-1)
    return torch.matmul(probs, v.contiguous())


def flash_attention_fwd(q, k, v, mask_mod: Optional[MaskMod] = None, block_r: int = DEFAULT_BLOCK_R,
                        block_c: int = DEFAULT_BLOCK_C, num_warps: int = DEFAULT_NUM_WARPS,
                        num_stages: int = DEFAULT_NUM_STAGES, interpret: bool = False):
    """Forward pass -> (o, logsumexp) with logsumexp in q's dtype (``flash_attn.py:111-165``)."""
    host = _check_interpret(interpret, q)
    mask, _, mods = _resolve(mask_mod, None)
    o, lse, _ = _fwd_core(q, k, v, mask, None, None, None, _ref_tiles(q, block_r, block_c, mask), mods,
                          host)
    return o, lse.to(q.dtype)


def flash_attention_bwd(q, k, v, o, logsumexp, do, mask_mod: Optional[MaskMod] = None,
                        block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                        num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                        interpret: bool = False):
    """Backward pass -> (dq, dk, dv) (``flash_attn.py:410-461``).  ``logsumexp``
    may be in q's dtype (as returned by :func:`flash_attention_fwd`) or fp32."""
    host = _check_interpret(interpret, q)
    mask, _, mods = _resolve(mask_mod, None)
    return _bwd_core(q, k, v, o, logsumexp, do, mask, None, None, None,
                     _ref_tiles(q, block_r, block_c, mask), mods, host)


class _FlexFn:
    """torch.autograd.Function wrapper (created lazily so that importing the
    package does not require torch)."""
    fn = None

    @classmethod
    def get(cls):
        if cls.fn is None:
            torch = _torch()

            class FlexAttnFunction(torch.autograd.Function):
                @staticmethod
                def forward(ctx, q, k, v, cfg):
                    # cfg: mask, score, scale, block mask, tiles, mods, host
                    o, lse, plan = _fwd_core(q, k, v, *cfg)
                    ctx.save_for_backward(q, k, v, o, lse)
                    ctx.cfg = cfg
                    ctx.plan = plan
                    ctx.mark_non_differentiable(lse)
                    return o, lse

                @staticmethod
                def backward(ctx, do, dlse):
                    q, k, v, o, lse = ctx.saved_tensors
                    dq, dk, dv = _bwd_core(q, k, v, o, lse, do, *ctx.cfg, plan=ctx.plan)
                    return dq, dk, dv, None

            cls.fn = FlexAttnFunction
        return cls.fn


def flash_attention(q, k, v, mask_mod: Optional[MaskMod] = None, block_r: int = DEFAULT_BLOCK_R,
                    block_c: int = DEFAULT_BLOCK_C, num_warps: int = DEFAULT_NUM_WARPS,
                    num_stages: int = DEFAULT_NUM_STAGES, interpret: bool = False):
    """Flash attention with a custom backward (``flash_attn.py:464-504``)."""
    host = _check_interpret(interpret, q)
    mask, _, mods = _resolve(mask_mod, None)
    cfg = (mask, None, None, None, _ref_tiles(q, block_r, block_c, mask), mods, host)
    o, _ = _FlexFn.get().apply(q, k, v, cfg)
    return o


def flex_decode(query, key, value, score_mod: Optional[ScoreSpec] = None, block_mask: Optional[BlockMask] = None,
                scale: Optional[float] = None, enable_gqa: bool = False, num_splits: Optional[int] = None,
                return_lse: bool = False, kv_lens=None, page_table=None, kv_len: Optional[int] = None):
    """Forward-only FlexAttention for short query blocks against long key
    sequences (decoding).  The keys of each query tile are split into
    ``num_splits`` ranges computed by separate workgroups and merged by their
    log-sum-exp (``None`` picks about two workgroups per CU); with grouped-query
    attention the query heads sharing a kv head run as one tile, so each K / V
    tile is read once per group.  Same results as :func:`flex_attention`'s
    forward; no gradient.  The reference has no decode kernel (it is on its
    roadmap).

    KV cache: ``kv_lens`` (B,) int gives each batch row's key count (keys past
    it are ignored).  With ``page_table`` (B, max_pages) int, ``key`` / ``value``
    are paged caches of shape (num_pages, Hkv, page_size, D): key t of batch row
    b is row t % page_size of page page_table[b, t // page_size] (page_size a
    multiple of 64); ``kv_len`` is the logical key capacity (default
    max_pages * page_size) that masks and block masks refer to."""
    torch = _torch()
    mask_mod = None
    if block_mask is not None:
        mask_mod = block_mask.mask_mod
        if not block_mask.has_tables:
            raise ValueError("block_mask has no kernel tables (build it with create_block_mask)")
    mask, score, mods = _resolve(mask_mod, score_mod)
    paged = page_table is not None
    if mods is not None:  # user mods: the run-time compiled forward, unsplit
        if paged or kv_lens is not None:
            raise NotImplementedError("user score / mask callables with a KV cache: pass contiguous keys")
        o, lse, _ = _fwd_core(query, key, value, mask, score, scale, block_mask, None, mods)
        return (o, lse) if return_lse else o
    q, k, v = _dense16(query), _dense16(key), _dense16(value)
    if paged:
        if k.dim() != 4 or k.shape != v.shape:
            raise ValueError("paged key / value caches must be (num_pages, Hkv, page_size, D)")
        num_pages, Hkv, page_size, D = k.shape
        pt = page_table.to(device=q.device, dtype=torch.int32).contiguous()
        if pt.dim() != 2 or pt.shape[0] != q.shape[0]:
            raise ValueError("page_table must be (B, max_pages)")
        Skv = int(kv_len) if kv_len is not None else pt.shape[1] * page_size
        if q.dim() != 4 or not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise ValueError("query must be (B, Hq, Sq, D) and all tensors on the GPU")
        if q.dtype != k.dtype or q.dtype != v.dtype:
            raise TypeError("query and caches must share a dtype")
        if q.shape[3] != D or q.shape[1] % Hkv:
            raise ValueError("head dim or head counts of query and caches do not match")
    else:
        _check_inputs(q, k, v)
        Skv = k.shape[2]
    if query.shape[1] != (k.shape[1] if paged else key.shape[1]) and not enable_gqa:
        raise ValueError("query and key head counts differ: pass enable_gqa=True for grouped-query attention")
    _, dname = _dtype_code(q)
    shape_k = _ShapeOnly((q.shape[0], k.shape[1], Skv, q.shape[3]), q.device, q.dtype) if paged else k
    plan = _get_plan(q, shape_k, mask, score, scale, block_mask, DEFAULT_TILES[dname])
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    lib = _lib.load()
    n = 0 if num_splits is None else int(num_splits)
    if paged or kv_lens is not None:
        import ctypes
        kvc = _lib.FaKvCache()
        keep = []
        if kv_lens is not None:
            kl = torch.as_tensor(kv_lens, device=q.device).to(torch.int32).contiguous()
            if kl.shape != (q.shape[0],):
                raise ValueError("kv_lens must have one entry per batch row")
            keep.append(kl)
            kvc.kv_lens = kl.data_ptr()
        if paged:
            keep.append(pt)
            kvc.page_table, kvc.page_size, kvc.max_pages, kvc.num_pages = pt.data_ptr(), page_size, pt.shape[1], \
                num_pages
        ws_bytes = lib.fa_fwd_kvcache_workspace_bytes(plan.ptr(), ctypes.byref(kvc), n)
        ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
        _lib.check(lib.fa_fwd_kvcache(plan.ptr(), ctypes.byref(kvc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      o.data_ptr(), lse.data_ptr(), n, ws.data_ptr(), ws_bytes, _stream()))
    else:
        ws_bytes = lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), n)
        ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
        _lib.check(lib.fa_fwd_splitkv(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                      lse.data_ptr(), n, ws.data_ptr(), ws_bytes, _stream()))
    return (o, lse) if return_lse else o


def _seq_tokens(cu):
    """Per-token (sequence index, sequence start, sequence length) of packed sequences."""
    cu = np.asarray(cu, dtype=np.int64).reshape(-1)
    if cu.size < 2 or cu[0] != 0 or np.any(np.diff(cu) < 0):
        raise ValueError("cu_seqlens must start at 0 and be non-decreasing")
    lens = np.diff(cu)
    seq = np.repeat(np.arange(lens.size), lens)
    return seq, cu[:-1][seq], lens[seq], cu


def varlen_mask(cu_seqlens_q, cu_seqlens_k, causal: bool = False):
    """Mask mod of packed variable-length sequences (the FlashAttention
    ``cu_seqlens`` convention): query i of sequence s sees the keys of sequence
    s, and with ``causal`` only those at most as far from the end of the
    sequence's keys as the query is from the end of its queries (bottom-right
    aligned, as in FlashAttention's varlen causal mask).  Equal query and key
    packings give a document mask (interval kernels); otherwise the mask is a
    traced callable over per-token index tables."""
    sq, stq, lq, cq = _seq_tokens(cu_seqlens_q)
    sk, stk, lk, ck = _seq_tokens(cu_seqlens_k)
    if cq.size != ck.size:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must describe the same number of sequences")
    if np.array_equal(cq, ck):
        docs = document_ids_mask(sq.astype(np.int32))
        return and_masks(docs, causal_mask) if causal else docs
    import torch
    seq_q, seq_k = torch.from_numpy(sq.astype(np.int32)), torch.from_numpy(sk.astype(np.int32))
    # causal reach of query i: its key-side position may be at most off_q[i]
    off_q = torch.from_numpy((np.arange(sq.size) - stq + (np.diff(ck)[sq] - lq)).astype(np.int32))
    pos_k = torch.from_numpy((np.arange(sk.size) - stk).astype(np.int32))

    def mask(q_idx, kv_idx):
        same = seq_q[q_idx] == seq_k[kv_idx]
        return same & (pos_k[kv_idx] <= off_q[q_idx]) if causal else same
    return mask


def flex_attention_varlen(query, key, value, cu_seqlens_q, cu_seqlens_k, causal: bool = False,
                          score_mod=None, scale: Optional[float] = None, enable_gqa: bool = False,
                          return_lse: bool = False):
    """Attention over packed variable-length sequences: query (1, Hq, total_q,
    D), key / value (1, Hkv, total_k, D), sequence s occupying rows
    [cu_seqlens_q[s], cu_seqlens_q[s+1]) of the queries and
    [cu_seqlens_k[s], cu_seqlens_k[s+1]) of the keys (see :func:`varlen_mask`).
    Differentiable; tokens of different sequences never attend to each other
    and their tile pairs are skipped."""
    if query.shape[0] != 1 or key.shape[0] != 1:
        raise ValueError("packed variable-length inputs have batch size 1: (1, H, total_tokens, D)")
    mm = varlen_mask(cu_seqlens_q, cu_seqlens_k, causal)
    bm = create_block_mask(mm, 1, query.shape[1], query.shape[2], key.shape[2], TABLE_BLOCK,
                           device=query.device if isinstance(mm, MaskSpec) else None)
    return flex_attention(query, key, value, score_mod=score_mod, block_mask=bm, scale=scale, enable_gqa=enable_gqa,
                          return_lse=return_lse)


class _ShapeOnly:
    """Stands in for a tensor where only its shape, device and dtype are read
    (the logical key shape of a paged cache, for the plan)."""

    def __init__(self, shape, device, dtype):
        self.shape, self.device, self.dtype = tuple(shape), device, dtype


def flex_attention(query, key, value, score_mod: Optional[ScoreSpec] = None,
                   block_mask: Optional[BlockMask] = None, scale: Optional[float] = None,
                   enable_gqa: bool = False, return_lse: bool = False, kernel_options: Optional[dict] = None):
    """FlexAttention: ``softmax(mask(score_mod(scale * q k^T))) v`` over the
    blocks of ``block_mask`` (all blocks when None).  Differentiable.

    ``kernel_options`` may set ``BLOCK_M`` (query rows per forward / dQ
    workgroup, 32 per wave), ``BLOCK_N`` (keys per LDS tile), ``BLOCK_KV``
    (keys per dK/dV workgroup), ``BLOCK_Q`` (queries per dK/dV tile, 64 or
    128) and ``NUM_STAGES`` (K / V tiles the forward holds in LDS: 2, 3 with
    ``BLOCK_N`` 32, 1 with ``BLOCK_N`` 128); otherwise the tuned table entry
    for the shape class (dtype, head dim, length, mask class) or the defaults
    (bf16: 128 x 64 / 128 with automatic q tiles, fp32: 128 x 32 / 128) run."""
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key head counts differ: pass enable_gqa=True for grouped-query attention")
    mask_mod = None
    if block_mask is not None:
        mask_mod = block_mask.mask_mod
        if not block_mask.has_tables:
            raise ValueError("block_mask has no kernel tables (build it with create_block_mask)")
    mask, score, mods = _resolve(mask_mod, score_mod)
    # tables at another block size are re-derived for the kernel tiles (_tables_for)
    _, dname = _dtype_code(query)
    opts = kernel_options or {}
    cls = mask_class(mask) if mods is None or mods.mask is None else "causal"
    tiles = tuned_tiles(query.shape[2], query.shape[3], dname, cls) or DEFAULT_TILES[dname]
    if any(o in opts for o in TILE_NAMES):
        tiles = tuple(int(opts.get(o, d)) for o, d in zip(TILE_NAMES, DEFAULT_TILES[dname]))
    cfg = (mask, score, scale, block_mask, tiles, mods, False)
    o, lse = _FlexFn.get().apply(query, key, value, cfg)
    return (o, lse) if return_lse else o
