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
reference; this build has no host execution path and raises.
"""
import math
from typing import Optional, Tuple

import numpy as np

from . import _lib
from .block_mask import BlockMask, _finish, create_block_mask
from .kernel_tuner import (DEFAULT_BLOCK_C, DEFAULT_BLOCK_R, DEFAULT_NUM_STAGES, DEFAULT_NUM_WARPS,
                           kernel_tiles, tuned_tiles)
from .mask_mod import MaskSpec, MaskMod
from .score_mod import ScoreSpec

# Granularity of the block tables built internally: a multiple of every
# kernel tile (64/128 queries, 32/64 keys, 128-key dK/dV tiles).
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
    raise TypeError(f"unsupported dtype {t.dtype}: the MI355X kernels take bfloat16 or float32")


def _check_interpret(interpret):
    if interpret:
        raise NotImplementedError(
            "interpret=True ran the Pallas interpreter on the host; this MI355X build only executes its "
            "HIP kernels on the GPU. Pass GPU tensors with interpret=False (mha_reference gives a "
            "materialised reference result).")


def _check_inputs(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (B, H, T, D)")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be GPU tensors")
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
                 block_mask: Optional[BlockMask], tiles: Tuple[int, int]):
        B, Hq, Sq, D = q.shape
        Hkv, Skv = k.shape[1], k.shape[2]
        code, dname = _dtype_code(q)
        p = _lib.FaParams()
        p.abi_version = _lib.ABI_VERSION
        p.dtype = code
        p.B, p.Hq, p.Hkv, p.Sq, p.Skv, p.D = B, Hq, Hkv, Sq, Skv, D
        p.block_m, p.block_n = tiles
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
            if bs % tiles[0] or bs % tiles[1] or bs % 128:
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


def _internal_block_mask(mask: MaskSpec, B: int, Sq: int, Skv: int, device=None) -> BlockMask:
    """Tables for a mask given without a BlockMask, built on ``device`` when it is a GPU."""
    on_gpu = device is not None and getattr(device, "type", str(device)) == "cuda"
    key = (mask.key(), B, Sq, Skv, str(device) if on_gpu else None)
    bm = _MASK_CACHE.get(key)
    if bm is None:
        if on_gpu:
            bm = create_block_mask(mask, B, 1, Sq, Skv, TABLE_BLOCK, device=device)
        else:
            bm = _finish(None, None, mask, B, 1, Sq, Skv, TABLE_BLOCK)
        if len(_MASK_CACHE) > 64:
            _MASK_CACHE.clear()
        _MASK_CACHE[key] = bm
    return bm


def _as_mask_spec(mask_mod) -> Optional[MaskSpec]:
    if mask_mod is None:
        return None
    if isinstance(mask_mod, MaskSpec):
        return mask_mod
    raise NotImplementedError(
        "the MI355X kernels evaluate mask mods as fused epilogues: use causal_mask, bidirectional_mask, "
        "sliding_window_mask, document_mask or and_masks of them (arbitrary callables work with "
        "create_block_mask and mha_reference only)")


def _as_score_spec(score_mod) -> Optional[ScoreSpec]:
    if score_mod is None:
        return None
    if isinstance(score_mod, ScoreSpec):
        return None if (score_mod.alibi is None and score_mod.softcap == 0) else score_mod
    raise NotImplementedError(
        "the MI355X kernels support the fused score mods alibi_score_mod, softcap_score_mod and their "
        "composition; arbitrary callables are not lowered")


def _stream():
    return _torch().cuda.current_stream().cuda_stream


def _dense16(t):
    """Contiguous with a 16-byte aligned base (the kernels use 16-byte loads)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _fwd_core(q, k, v, mask, score, scale, block_mask, tiles):
    """Forward through fa_fwd -> (o, lse fp32, plan)."""
    torch = _torch()
    _check_inputs(q, k, v)
    q, k, v = _dense16(q), _dense16(k), _dense16(v)
    if block_mask is None and mask is not None and not mask.is_trivial:
        block_mask = _internal_block_mask(mask, q.shape[0], q.shape[2], k.shape[2], q.device)
    plan = _get_plan(q, k, mask, score, scale, block_mask, tiles)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.fa_fwd(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          _stream()))
    return o, lse, plan


def _bwd_core(q, k, v, o, lse, do, mask, score, scale, block_mask, tiles, plan=None):
    """Backward through fa_bwd -> (dq, dk, dv).  ``plan`` is the forward's
    plan when the caller has it (same problem), else one is looked up."""
    torch = _torch()
    _check_inputs(q, k, v)
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    q, k, v, o, do = (_dense16(t) for t in (q, k, v, o, do))
    if lse.dtype != torch.float32 or not lse.is_contiguous():
        lse = lse.to(torch.float32).contiguous()
    if o.shape != q.shape or do.shape != q.shape or lse.shape != q.shape[:3]:
        raise ValueError("o / do / lse shapes do not match q")
    if plan is None:
        if block_mask is None and mask is not None and not mask.is_trivial:
            block_mask = _internal_block_mask(mask, q.shape[0], q.shape[2], k.shape[2], q.device)
        plan = _get_plan(q, k, mask, score, scale, block_mask, tiles)
    lib = _lib.load()
    ws_bytes = lib.fa_bwd_workspace_bytes(plan.ptr())
    ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    _lib.check(lib.fa_bwd(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                          ws.numel(), _stream()))
    return dq, dk, dv


def _sparse(mask) -> bool:
    return mask is not None and not mask.is_trivial


def _ref_tiles(q, block_r, block_c, sparse=False):
    """Kernel tile of a reference-signature call: block_r / block_c are
    Triton hints; the tuned tile for the shape class (or the default) runs."""
    _, dname = _dtype_code(q)
    return kernel_tiles(block_r, block_c, dname, q.shape[2], q.shape[3], sparse)


def _as4d(t):
    """(B*H, T, C) flattened arrays of the reference's stage functions -> (B*H, 1, T, C)."""
    return t.unsqueeze(1) if t.dim() == 3 else t


def _stage_plan(q4, k4, mask_mod, block_r, block_c, scale=None):
    mask = _as_mask_spec(mask_mod)
    bm = None
    if mask is not None and not mask.is_trivial:
        bm = _internal_block_mask(mask, q4.shape[0], q4.shape[2], k4.shape[2], q4.device)
    return _get_plan(q4, k4, mask, None, scale, bm, _ref_tiles(q4, block_r, block_c, bm is not None))


def flash_attention_bwd_preprocess(o_flat, do_flat, block_r: int = DEFAULT_BLOCK_R,
                                   num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                                   interpret: bool = False):
    """Delta = rowsum(O * dO) (``flash_attn.py:168-203``), shape o.shape[:-1].
    Returned in fp32 (the reference stores it in O's dtype)."""
    _check_interpret(interpret)
    torch = _torch()
    o4, do4 = _dense16(_as4d(o_flat)), _dense16(_as4d(do_flat).to(o_flat.dtype))
    plan = _stage_plan(o4, o4, None, block_r, DEFAULT_BLOCK_C)
    delta = torch.empty(o4.shape[:3], device=o4.device, dtype=torch.float32)
    _lib.check(_lib.load().fa_bwd_preprocess(plan.ptr(), o4.data_ptr(), do4.data_ptr(), delta.data_ptr(),
                                             _stream()))
    return delta.reshape(o_flat.shape[:-1])


def _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale, softmax_scale):
    torch = _torch()
    if abs(qk_scale - softmax_scale) > 1e-12 * max(abs(qk_scale), 1.0):
        raise NotImplementedError("the kernels apply one softmax scale to both S and dS")
    q4, k4, v4 = (_dense16(_as4d(t)) for t in (q_flat, k_flat, v_flat))
    _check_inputs(q4, k4, v4)
    do4 = _dense16(_as4d(do_flat).to(q4.dtype))
    lse = logsumexp_flat.to(torch.float32).reshape(q4.shape[:3]).contiguous()
    delta = d_flat.to(torch.float32).reshape(q4.shape[:3]).contiguous()
    return q4, k4, v4, do4, lse, delta


def flash_attention_bwd_dkv(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale: float,
                            softmax_scale: float, block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                            num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                            mask_mod: Optional[MaskMod] = None, interpret: bool = False):
    """dK, dV (``flash_attn.py:206-310``) from q, k, v, dO, LSE and Delta."""
    _check_interpret(interpret)
    torch = _torch()
    q4, k4, v4, do4, lse, delta = _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat,
                                                qk_scale, softmax_scale)
    plan = _stage_plan(q4, k4, mask_mod, block_r, block_c, qk_scale)
    dk, dv = torch.empty_like(k4), torch.empty_like(v4)
    _lib.check(_lib.load().fa_bwd_dkdv(plan.ptr(), q4.data_ptr(), k4.data_ptr(), v4.data_ptr(), do4.data_ptr(),
                                       lse.data_ptr(), delta.data_ptr(), dk.data_ptr(), dv.data_ptr(), _stream()))
    return dk.reshape(k_flat.shape), dv.reshape(v_flat.shape)


def flash_attention_bwd_dq(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat, qk_scale: float,
                           softmax_scale: float, block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                           num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                           mask_mod: Optional[MaskMod] = None, interpret: bool = False):
    """dQ (``flash_attn.py:313-407``) from q, k, v, dO, LSE and Delta."""
    _check_interpret(interpret)
    torch = _torch()
    q4, k4, v4, do4, lse, delta = _stage_inputs(q_flat, k_flat, v_flat, do_flat, logsumexp_flat, d_flat,
                                                qk_scale, softmax_scale)
    plan = _stage_plan(q4, k4, mask_mod, block_r, block_c, qk_scale)
    dq = torch.empty_like(q4)
    _lib.check(_lib.load().fa_bwd_dq(plan.ptr(), q4.data_ptr(), k4.data_ptr(), v4.data_ptr(), do4.data_ptr(),
                                     lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), _stream()))
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
        mask = _as_mask_spec(mask_mod if block_mask is None else block_mask.mask_mod)
        if block_mask is None and mask is not None and not mask.is_trivial:
            block_mask = _internal_block_mask(mask, q.shape[0], q.shape[2], k.shape[2], q.device)
        _, dname = _dtype_code(q)
        tiles = tiles or (128, 64 if dname == "bf16" else 32)
        self.plan = _Plan(self.q, self.k, mask, _as_score_spec(score_mod), scale, block_mask, tiles)
        self.block_mask = block_mask
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        self.delta = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        self.dq, self.dk, self.dv = torch.empty_like(self.q), torch.empty_like(self.k), torch.empty_like(self.v)
        self.lib = _lib.load()

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

    def step(self):
        """One forward + backward pass."""
        self.fwd()
        self.preprocess()
        self.dkdv()
        self.dq_()


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
    _check_interpret(interpret)
    mask = _as_mask_spec(mask_mod)
    o, lse, _ = _fwd_core(q, k, v, mask, None, None, None, _ref_tiles(q, block_r, block_c, _sparse(mask)))
    return o, lse.to(q.dtype)


def flash_attention_bwd(q, k, v, o, logsumexp, do, mask_mod: Optional[MaskMod] = None,
                        block_r: int = DEFAULT_BLOCK_R, block_c: int = DEFAULT_BLOCK_C,
                        num_warps: int = DEFAULT_NUM_WARPS, num_stages: int = DEFAULT_NUM_STAGES,
                        interpret: bool = False):
    """Backward pass -> (dq, dk, dv) (``flash_attn.py:410-461``).  ``logsumexp``
    may be in q's dtype (as returned by :func:`flash_attention_fwd`) or fp32."""
    _check_interpret(interpret)
    mask = _as_mask_spec(mask_mod)
    return _bwd_core(q, k, v, o, logsumexp, do, mask, None, None, None,
                     _ref_tiles(q, block_r, block_c, _sparse(mask)))


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
    _check_interpret(interpret)
    mask = _as_mask_spec(mask_mod)
    cfg = (mask, None, None, None, _ref_tiles(q, block_r, block_c, _sparse(mask)))
    o, _ = _FlexFn.get().apply(q, k, v, cfg)
    return o


def flex_decode(query, key, value, score_mod: Optional[ScoreSpec] = None, block_mask: Optional[BlockMask] = None,
                scale: Optional[float] = None, enable_gqa: bool = False, num_splits: Optional[int] = None,
                return_lse: bool = False):
    """Forward-only FlexAttention for short query blocks against long key
    sequences (decoding): the keys of each query tile are split into
    ``num_splits`` ranges computed by separate workgroups and merged by their
    log-sum-exp (C ABI ``fa_fwd_splitkv``; ``None`` picks about two workgroups
    per CU).  Same results as :func:`flex_attention`'s forward; no gradient.
    The reference has no decode kernel (it is on its roadmap)."""
    torch = _torch()
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key head counts differ: pass enable_gqa=True for grouped-query attention")
    mask = None
    if block_mask is not None:
        mask = _as_mask_spec(block_mask.mask_mod) if block_mask.mask_mod is not None else None
        if not block_mask.has_tables:
            raise ValueError("block_mask has no kernel tables (build it with create_block_mask)")
    q, k, v = _dense16(query), _dense16(key), _dense16(value)
    _check_inputs(q, k, v)
    _, dname = _dtype_code(q)
    plan = _get_plan(q, k, mask, _as_score_spec(score_mod), scale, block_mask, (128, 64 if dname == "bf16" else 32))
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    lib = _lib.load()
    n = 0 if num_splits is None else int(num_splits)
    ws_bytes = lib.fa_fwd_splitkv_workspace_bytes(plan.ptr(), n)
    ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
    _lib.check(lib.fa_fwd_splitkv(plan.ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                  lse.data_ptr(), n, ws.data_ptr(), ws_bytes, _stream()))
    return (o, lse) if return_lse else o


def flex_attention(query, key, value, score_mod: Optional[ScoreSpec] = None,
                   block_mask: Optional[BlockMask] = None, scale: Optional[float] = None,
                   enable_gqa: bool = False, return_lse: bool = False, kernel_options: Optional[dict] = None):
    """FlexAttention: ``softmax(mask(score_mod(scale * q k^T))) v`` over the
    blocks of ``block_mask`` (all blocks when None).  Differentiable.

    ``kernel_options`` may set ``BLOCK_M`` / ``BLOCK_N``; otherwise a tuned
    table entry or the defaults (bf16: 128 x 64, fp32: 128 x 32) are used."""
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key head counts differ: pass enable_gqa=True for grouped-query attention")
    mask = None
    if block_mask is not None:
        mask = _as_mask_spec(block_mask.mask_mod) if block_mask.mask_mod is not None else None
        if not block_mask.has_tables:
            raise ValueError("block_mask has no kernel tables (build it with create_block_mask)")
        if block_mask.block_size % TABLE_BLOCK and mask is not None:
            # the dK/dV kernel walks 128-key tiles: re-derive the exact tables at 128
            block_mask = _internal_block_mask(mask, query.shape[0], query.shape[2], key.shape[2], query.device)
    _, dname = _dtype_code(query)
    opts = kernel_options or {}
    tiles = None
    if "BLOCK_M" in opts or "BLOCK_N" in opts:
        tiles = (int(opts.get("BLOCK_M", 128)), int(opts.get("BLOCK_N", 64 if dname == "bf16" else 32)))
    else:
        tiles = tuned_tiles(query.shape[2], query.shape[3], dname, block_mask is not None) or \
            (128, 64 if dname == "bf16" else 32)
    cfg = (mask, _as_score_spec(score_mod), scale, block_mask, tiles)
    o, lse = _FlexFn.get().apply(query, key, value, cfg)
    return (o, lse) if return_lse else o
