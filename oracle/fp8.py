"""OCP FP8 e4m3 in numpy and the fp8 forward's quantisation — TEST
INFRASTRUCTURE ONLY (see the package docstring).

The reference has no fp8 path (its kernels are bfloat16 / float32); these
functions restate the MI355X build's own fp8 specification so that the
kernels can be checked against it, and the attention itself is checked
against ``attention.forward`` (float64) on the dequantised inputs.

* ``encode_e4m3`` / ``decode_e4m3`` — OCP e4m3 ("fn": no infinities, NaN =
  S.1111.111, max 448, min normal 2^-6, min subnormal 2^-9), round to nearest
  even, magnitudes above 464 (the midpoint past 448) to NaN.  Pinned against
  torch's float8_e4m3fn conversion (an independent implementation) over all
  256 codes and random / tie values, and by closed forms.
* ``block_scales`` / ``quantize_blocks`` — one power-of-two scale per 128-row
  block of each head: scale = 2^e, e the smallest integer with 448 2^e >= the
  block's max |x| (the ratio computed in float32, e clamped to [-126, 127],
  e = 0 for an all-zero block), codes = e4m3(x / scale).  Pinned by the
  invariants that define it (power of two, |x / scale| <= 448, e minimal) in
  the tests.
* ``forward_model`` — attention on dequantised inputs with P rounded to e4m3
  as p 2^3 against the exact row maximum (float64 otherwise): the error the
  fp8 forward's P rounding alone makes, the yardstick for its tolerance; and
  the worst case of that error per element whatever reference maximum the
  rounding is taken against (below the row maximum, as a running maximum
  is): |dO| <= 2^-4 sum_j p_j |v_j| / l (relative rounding of normal e4m3
  values) + n 2^-13 max_j |v_j| / l (absolute rounding of the subnormal
  ones, p 2^3 < 2^-6).  Pinned against ``attention.forward`` (equal when the
  rounding is removed) and by the bound holding for the model itself.
"""
import numpy as np

from . import attention

E4M3_MAX = 448.0
SCALE_ROWS = 128


def decode_e4m3(codes) -> np.ndarray:
    """uint8 e4m3 codes -> float32 values (NaN for S.1111.111)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (s * val).astype(np.float32)


def encode_e4m3(x) -> np.ndarray:
    """float values -> uint8 e4m3 codes, round to nearest even; |x| > 464 and
    NaN become NaN codes (0x7F with x's sign; 0x7F for NaN)."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int32)
    out = np.zeros(x.shape, np.int32)
    sub = a < 2.0 ** -6
    out = np.where(sub, np.rint(a / 2.0 ** -9).astype(np.int64), out)  # 8 = the smallest normal, code 0x08
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(sub | ~np.isfinite(a), 1.0, a)))
        mant = np.where(sub | ~np.isfinite(a), 1.0, a) / np.exp2(e)
    # log2 of values just below a power of two can round up: fix the binade
    lo = mant < 1.0
    e = np.where(lo, e - 1, e)
    mant = np.where(lo, mant * 2.0, mant)
    q = np.rint((mant - 1.0) * 8.0).astype(np.int64)
    carry = q == 8
    e = np.where(carry, e + 1, e)
    q = np.where(carry, 0, q)
    normal = ((e + 7).astype(np.int64) << 3) | q
    out = np.where(sub, out, normal)
    nan = np.isnan(x) | (a > 464.0) | (~sub & (out > 0x7E))
    out = np.where(nan, 0x7F, out) | np.where(np.isnan(x), 0, sign)
    return out.astype(np.uint8)


def block_scales(x, rows: int = SCALE_ROWS) -> np.ndarray:
    """(heads, S, D) values -> (heads, ceil(S / rows)) float32 power-of-two scales."""
    x = np.asarray(x, dtype=np.float32)
    H, S, _ = x.shape
    nb = (S + rows - 1) // rows
    out = np.ones((H, nb), np.float32)
    for h in range(H):
        for b in range(nb):
            amax = np.float32(np.abs(x[h, b * rows:(b + 1) * rows]).max())
            if amax > 0 and np.isfinite(amax):
                f, ex = np.frexp(np.float32(amax) / np.float32(E4M3_MAX))  # float32 ratio
                e = int(ex) - 1 if f == 0.5 else int(ex)
                out[h, b] = np.float32(2.0 ** min(max(e, -126), 127))
    return out


def quantize_blocks(x, transpose: bool = False, rows: int = SCALE_ROWS):
    """(heads, S, D) -> (codes, scales): codes (heads, S, D) uint8, or with
    ``transpose`` (heads, D, ld) with ld = S rounded up to ``rows`` and the
    keys past S zero."""
    x = np.asarray(x, dtype=np.float32)
    H, S, D = x.shape
    sc = block_scales(x, rows)
    per_row = np.repeat(sc, rows, axis=1)[:, :S]
    codes = encode_e4m3(x.astype(np.float64) / per_row[..., None].astype(np.float64))
    if not transpose:
        return codes, sc
    ld = sc.shape[1] * rows
    t = np.zeros((H, D, ld), np.uint8)
    t[:, :, :S] = codes.transpose(0, 2, 1)
    return t, sc


def dequantize(codes, scales, transposed: bool = False, seq_len=None, rows: int = SCALE_ROWS) -> np.ndarray:
    """Inverse view of ``quantize_blocks``: (heads, S, D) float32 values."""
    v = decode_e4m3(codes)
    if transposed:
        v = v.transpose(0, 2, 1)[:, :seq_len]
    S = v.shape[1]
    per_row = np.repeat(np.asarray(scales, np.float32), rows, axis=1)[:, :S]
    return (v * per_row[..., None]).astype(np.float32)


def forward_model(q, k, v, mask=None, scale=None, alibi_slopes=None, softcap=None, round_p: bool = True,
                  with_bound: bool = False):
    """(o, lse) of attention on (B, H, S, D) float inputs with P rounded to
    e4m3 as p 2^3 (p = exp(s - rowmax)) before the P V product, everything
    else float64 (scores and mods as ``attention.forward``); ``round_p=False``
    is plain attention.  ``with_bound`` adds the per-element worst case of
    the P rounding error (module docstring) as a third result."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    sc = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.zeros((B, Hq, Sq, D))
    bound = np.zeros((B, Hq, Sq, D))
    lse = np.full((B, Hq, Sq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            s, _ = attention._scores(q[b, h], k[b, h // g], sc, h, Hq, alibi_slopes, softcap)
            if mask is not None:
                mk = attention._mask_for(mask, b, h, Sq, k.shape[2])
                s = np.where(mk, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            live = np.isfinite(m[:, 0])
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.exp(s - m)
            l = p.sum(axis=1)
            pr = decode_e4m3(encode_e4m3(p * 8.0)).astype(np.float64) / 8.0 if round_p else p
            vh = v[b, h // g]
            with np.errstate(invalid="ignore", divide="ignore"):
                o[b, h] = np.where(live[:, None], (pr @ vh) / l[:, None], 0.0)
                lse[b, h] = np.where(live, m[:, 0] + np.log(l), -np.inf)
                n = (p > 0).sum(axis=1)
                bnd = (2.0 ** -4 * (p @ np.abs(vh)) + n[:, None] * 2.0 ** -13 * np.abs(vh).max(axis=0)[None, :])
                bound[b, h] = np.where(live[:, None], bnd / l[:, None], 0.0)
    if with_bound:
        return o.astype(np.float32), lse.astype(np.float32), bound
    return o.astype(np.float32), lse.astype(np.float32)
