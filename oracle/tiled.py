"""ctypes front end of ``tiled_ref.c`` (the C restatement of the reference's
tiled Pallas kernels).  Test infrastructure and CPU baseline only."""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_tiled.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle_tiled.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        ip = ctypes.POINTER(ctypes.c_int)
        i = ctypes.c_int
        lib.ref_fwd.argtypes = [fp, fp, fp, i, i, i, i, i, i, i, i, i, ip, i, i, fp, fp, i, i, i]
        lib.ref_fwd.restype = i
        lib.ref_bwd.argtypes = [fp, fp, fp, fp, fp, fp, i, i, i, i, i, i, i, i, i, ip, i, i, i, fp, fp, fp, i, i, i]
        lib.ref_bwd.restype = i
        _lib = lib
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(a, t=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(t))


def _mask_args(window, doc_ids):
    if window is None and doc_ids is None:
        return 0, -1, -1, None
    left, right = window if window is not None else (-1, -1)
    doc = None if doc_ids is None else np.ascontiguousarray(doc_ids, dtype=np.int32)
    return 1, int(left), int(right), doc


def fwd(q, k, v, block_r=64, block_c=64, window=None, doc_ids=None, bf16=False,
        stats_in_dtype=True, nthreads=0, bh_range=None):
    """Reference tiled forward.  q,k,v (B,H,T,D) float arrays (values already in
    the input dtype).  ``window=(left,right)`` (causal = (-1, 0)); ``doc_ids`` (B,T).
    ``bh_range=(begin, end)`` restricts the work to flattened heads [begin, end)
    (outputs of other heads are left as zero).  Returns (o, lse) float32."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, T, D = q.shape
    o = np.zeros_like(q)
    lse = np.zeros((B, H, T), np.float32)
    use, left, right, doc = _mask_args(window, doc_ids)
    b0, b1 = bh_range if bh_range else (0, B * H)
    rc = _load().ref_fwd(_ptr(q), _ptr(k), _ptr(v), B, H, T, D, block_r, block_c, use, left, right,
                         None if doc is None else _ptr(doc, ctypes.c_int), int(bf16), int(stats_in_dtype),
                         _ptr(o), _ptr(lse), nthreads, b0, b1)
    if rc != 0:
        raise ValueError("ref_fwd rejected its arguments")
    return o, lse


def bwd(q, k, v, o, lse, do, block_r=64, block_c=64, window=None, doc_ids=None, bf16=False,
        stats_in_dtype=True, nthreads=0, bh_range=None, ds_scale_after=False):
    """Reference three-kernel backward.  Returns (dq, dk, dv) float32.
    ``ds_scale_after`` rounds dS before the softmax scale is applied (the
    MI355X kernels' cast point) instead of after (the reference's,
    ``flash_attn.py:243-245,347-349``)."""
    q, k, v, o, lse, do = (_f32(a) for a in (q, k, v, o, lse, do))
    B, H, T, D = q.shape
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    use, left, right, doc = _mask_args(window, doc_ids)
    b0, b1 = bh_range if bh_range else (0, B * H)
    rc = _load().ref_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(do), B, H, T, D, block_r,
                         block_c, use, left, right, None if doc is None else _ptr(doc, ctypes.c_int),
                         int(bf16), int(stats_in_dtype), int(ds_scale_after), _ptr(dq), _ptr(dk), _ptr(dv),
                         nthreads, b0, b1)
    if rc != 0:
        raise ValueError("ref_bwd rejected its arguments")
    return dq, dk, dv
