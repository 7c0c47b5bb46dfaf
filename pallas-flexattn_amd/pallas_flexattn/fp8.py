"""FP8 forward (OCP e4m3) on gfx950's scaled fp8 MFMA.

Not in the reference (its kernels are bfloat16 / float32): the fp8 path
serves forward-only use (inference, prefill) of the same masks, block tables
and built-in score mods.  Tensors are quantised per 128-row block of each head
with a power-of-two scale (``quantize_fp8``, on the GPU through the C ABI's
``fa_quantize_fp8``); V is kept transposed (head dim major), the layout the
kernel's P V product reads.  ``flex_attention_fp8`` takes bf16 tensors (and
quantises them) or ``Fp8Tensor`` values from ``quantize_fp8``.
"""
from typing import NamedTuple, Optional

from . import _lib
from .block_mask import BlockMask
from .flash_attn import _stream
from .kernel_tuner import DEFAULT_TILES

SCALE_ROWS = 128  # rows per scale block


class Fp8Tensor(NamedTuple):
    """e4m3 codes plus one power-of-two scale per 128-row block of each head.

    ``data``: uint8 ``(B, H, S, D)``, or with ``transposed`` ``(B, H, D, ld)``
    (``ld`` = S rounded up to 128, keys past S zero); ``scale``: float32
    ``(B, H, ceil(S / 128))``; the value is ``code * scale``."""
    data: object
    scale: object
    seq_len: int
    transposed: bool

    @property
    def shape(self):
        """Logical (B, H, S, D) shape."""
        if self.transposed:
            B, H, D, _ = self.data.shape
            return (B, H, self.seq_len, D)
        return tuple(self.data.shape)


def quantize_fp8(x, transpose: bool = False) -> Fp8Tensor:
    """bf16 ``(B, H, S, D)`` GPU tensor -> :class:`Fp8Tensor`: per 128-row
    block scale = 2^e, e the smallest integer with 448 * 2^e >= max |x| of
    the block, elements RNE(x / scale) in e4m3 (``fa_quantize_fp8``)."""
    import torch
    if x.dim() != 4 or not x.is_cuda or x.dtype != torch.bfloat16:
        raise ValueError("quantize_fp8 takes a bf16 (B, H, S, D) GPU tensor")
    x = x.contiguous()
    B, H, S, D = x.shape
    nb = (S + SCALE_ROWS - 1) // SCALE_ROWS
    ld = nb * SCALE_ROWS
    out = torch.empty((B, H, D, ld) if transpose else (B, H, S, D), device=x.device, dtype=torch.uint8)
    scale = torch.empty((B, H, nb), device=x.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.fa_quantize_fp8(x.data_ptr(), B * H, S, D, int(transpose), out.data_ptr(), scale.data_ptr(),
                                   _stream()))
    scale._fa_scales_ok = scale._version  # powers of two in range by construction
    return Fp8Tensor(out, scale, S, bool(transpose))


def _check_scales(t: Fp8Tensor, name: str) -> None:
    """The kernels read a scale's exponent field only (it becomes the E8M0
    scale operand of the MFMA): every scale must be a power of two 2^e with
    e in [-126, 127].  A scale tensor carries the version it was checked at
    (quantize_fp8's outputs are valid by construction), so the check (one
    device sync) runs once per tensor and again after an in-place change."""
    import torch
    sc = t.scale
    if getattr(sc, "_fa_scales_ok", None) == sc._version:
        return
    m, e = torch.frexp(sc)
    ok = bool(((m == 0.5) & (e >= -125) & (e <= 128)).all())
    if not ok:
        raise ValueError(f"{name}: Fp8Tensor scales must be powers of two 2^e with -126 <= e <= 127 "
                         "(the kernels use only their exponent)")
    sc._fa_scales_ok = sc._version


def dequantize_fp8(t: Fp8Tensor):
    """float32 values of an :class:`Fp8Tensor` in its logical (B, H, S, D) layout."""
    import torch
    x = t.data.view(torch.float8_e4m3fn).float()
    B, H = x.shape[:2]
    if t.transposed:
        x = x.transpose(2, 3)[:, :, :t.seq_len]
    s = t.scale.repeat_interleave(SCALE_ROWS, dim=2)[:, :, :t.seq_len]
    return x * s[..., None]


def flex_attention_fp8(query, key, value, score_mod=None, block_mask: Optional[BlockMask] = None,
                       scale: Optional[float] = None, enable_gqa: bool = False, return_lse: bool = False):
    """Forward attention on fp8 inputs (no gradient): ``query`` / ``key`` bf16
    ``(B, H, S, D)`` tensors or row-major :class:`Fp8Tensor`, ``value`` bf16
    or a transposed :class:`Fp8Tensor`.  Masks, block tables and score mods
    as :func:`flex_attention` (built-in descriptors; document labels as
    contiguous runs).  Returns bf16 O (and float32 LSE)."""
    r = Fp8Runner(query, key, value, score_mod, block_mask, scale, enable_gqa)
    r.fwd()
    return (r.o, r.lse) if return_lse else r.o


class Fp8Runner:
    """One fp8 forward problem bound to its inputs and outputs: the plan,
    the fa_fp8_inputs struct and O / LSE are built once; ``fwd()`` only
    enqueues the kernel on the current stream (as ``flash_attn.Runner`` does
    for the bf16 path; used by the benchmark)."""

    def __init__(self, query, key, value, score_mod=None, block_mask: Optional[BlockMask] = None,
                 scale: Optional[float] = None, enable_gqa: bool = False):
        import torch
        from .flash_attn import _get_plan, _resolve, _ShapeOnly, _tables_for
        q8, k8, v8, mask, score, dims = _prepare(query, key, value, score_mod, block_mask, enable_gqa, _resolve)
        B, Hq, Sq, D, Hkv, Skv = dims
        dev = q8.data.device
        f8 = torch.float8_e4m3fn
        qs, ks = _ShapeOnly((B, Hq, Sq, D), dev, f8), _ShapeOnly((B, Hkv, Skv, D), dev, f8)
        block_mask, tiles = _tables_for(mask, None, block_mask, qs, ks, DEFAULT_TILES["fp8"])
        self.plan = _get_plan(qs, ks, mask, score, scale, block_mask, tiles)
        self.inputs = (q8, k8, v8, block_mask)  # kept alive with the struct's pointers
        self.o = torch.empty((B, Hq, Sq, D), device=dev, dtype=torch.bfloat16)
        self.lse = torch.empty((B, Hq, Sq), device=dev, dtype=torch.float32)
        self.args = _lib.FaFp8Inputs(q8.data.data_ptr(), k8.data.data_ptr(), v8.data.data_ptr(), v8.data.shape[3],
                                     q8.scale.data_ptr(), k8.scale.data_ptr(), v8.scale.data_ptr())
        self.lib = _lib.load()

    def fwd(self):
        _lib.check(self.lib.fa_fwd_fp8(self.plan.ptr(), _lib.ctypes.byref(self.args), self.o.data_ptr(),
                                       self.lse.data_ptr(), _stream()))


def _prepare(query, key, value, score_mod, block_mask, enable_gqa, resolve):
    """Quantised inputs (bf16 tensors are quantised here), the resolved mask /
    score descriptors and the dims (B, Hq, Sq, D, Hkv, Skv), validated."""
    import torch
    q8 = query if isinstance(query, Fp8Tensor) else quantize_fp8(query)
    k8 = key if isinstance(key, Fp8Tensor) else quantize_fp8(key)
    v8 = value if isinstance(value, Fp8Tensor) else quantize_fp8(value, transpose=True)
    if q8.transposed or k8.transposed or not v8.transposed:
        raise ValueError("query / key row-major, value transposed (quantize_fp8(v, transpose=True))")
    B, Hq, Sq, D = q8.shape
    _, Hkv, Skv, Dk = k8.shape
    if v8.shape != k8.shape or Dk != D or k8.shape[0] != B:
        raise ValueError("query / key / value shapes do not match")
    if Hq != Hkv and not enable_gqa:
        raise ValueError("query and key head counts differ: pass enable_gqa=True for grouped-query attention")
    if Hq % Hkv:
        raise ValueError("number of q heads must be a multiple of the number of kv heads")
    if D not in (64, 128):
        raise ValueError("the fp8 forward takes head dims 64 and 128")
    mask_mod = block_mask.mask_mod if block_mask is not None else None
    mask, score, mods = resolve(mask_mod, score_mod)
    if mods is not None:
        raise NotImplementedError("the fp8 forward takes the built-in mask / score descriptors")
    for t, name in ((q8, "query"), (k8, "key"), (v8, "value")):
        if not (t.data.is_contiguous() and t.scale.is_contiguous() and t.scale.dtype == torch.float32):
            raise ValueError("Fp8Tensor data and scales must be contiguous, scales float32")
        _check_scales(t, name)
    return q8, k8, v8, mask, score, (B, Hq, Sq, D, Hkv, Skv)
