"""ctypes binding of libflexattn.so (the C ABI declared in include/flexattn.h).

The library is built in-tree next to this file.  There is no fallback: if it
is missing or a GPU is absent, calls raise.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# FLEXATTN_LIB names another build of the same library (same ABI), e.g. to
# time two builds side by side in one process tree.
LIB_PATH = os.environ.get("FLEXATTN_LIB") or os.path.join(_HERE, "libflexattn.so")
ABI_VERSION = 1

DTYPE_BF16 = 0
DTYPE_F32 = 1

_i32 = ctypes.c_int32
_pi32 = ctypes.c_void_p
_pf = ctypes.c_void_p


class FaParams(ctypes.Structure):
    """Mirror of ``struct fa_params`` (include/flexattn.h)."""
    _fields_ = [
        ("abi_version", _i32), ("dtype", _i32),
        ("B", _i32), ("Hq", _i32), ("Hkv", _i32), ("Sq", _i32), ("Skv", _i32), ("D", _i32),
        ("block_m", _i32), ("block_n", _i32),
        ("scale", ctypes.c_float),
        ("window_left", _i32), ("window_right", _i32),
        ("q_doc_ids", _pi32), ("kv_doc_ids", _pi32),
        ("doc_start", _pi32), ("doc_end", _pi32),
        ("alibi_slopes", _pf),
        ("softcap", ctypes.c_float),
        ("mask_block_q", _i32), ("mask_block_kv", _i32),
        ("table_b", _i32), ("table_h", _i32),
        ("kv_width", _i32), ("q_width", _i32),
        ("kv_num_blocks", _pi32), ("kv_indices", _pi32),
        ("full_kv_num_blocks", _pi32), ("full_kv_indices", _pi32),
        ("q_num_blocks", _pi32), ("q_indices", _pi32),
        ("full_q_num_blocks", _pi32), ("full_q_indices", _pi32),
    ]


class FaMaskBuild(ctypes.Structure):
    """Mirror of ``struct fa_mask_build`` (include/flexattn.h)."""
    _fields_ = [
        ("abi_version", _i32), ("rows", _i32),
        ("q_len", _i32), ("kv_len", _i32), ("block", _i32),
        ("window_left", _i32), ("window_right", _i32),
        ("doc_ids", _pi32), ("doc_len", _i32),
        ("sampled_num", _pi32), ("sampled_indices", _pi32),
        ("kv_num_blocks", _pi32), ("kv_indices", _pi32),
        ("full_kv_num_blocks", _pi32), ("full_kv_indices", _pi32),
        ("q_num_blocks", _pi32), ("q_indices", _pi32),
        ("full_q_num_blocks", _pi32), ("full_q_indices", _pi32),
        ("max_counts", _pi32),
    ]


EXPORTED = ("fa_fwd", "fa_fwd_splitkv", "fa_fwd_splitkv_workspace_bytes", "fa_bwd", "fa_bwd_workspace_bytes",
            "fa_bwd_noalloc", "fa_bwd_noalloc_max_rows", "fa_bwd_preprocess", "fa_bwd_dkdv", "fa_bwd_dq",
            "fa_mask_build_workspace_bytes", "fa_build_block_mask", "fa_strerror", "fa_abi_version")

_lib = None


class FlexAttnError(RuntimeError):
    """A non-zero status returned by the C ABI."""


def load():
    """Load libflexattn.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FlexAttnError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()' or pallas-flexattn_amd/build.py)")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(FaParams)
    v = ctypes.c_void_p
    lib.fa_fwd.argtypes = [P, v, v, v, v, v, v]
    lib.fa_fwd.restype = ctypes.c_int
    lib.fa_fwd_splitkv.argtypes = [P, v, v, v, v, v, ctypes.c_int, v, ctypes.c_size_t, v]
    lib.fa_fwd_splitkv.restype = ctypes.c_int
    lib.fa_fwd_splitkv_workspace_bytes.argtypes = [P, ctypes.c_int]
    lib.fa_fwd_splitkv_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_bwd.argtypes = [P, v, v, v, v, v, v, v, v, v, v, ctypes.c_size_t, v]
    lib.fa_bwd.restype = ctypes.c_int
    lib.fa_bwd_noalloc.argtypes = [P, v, v, v, v, v, v, v, v, v, v]
    lib.fa_bwd_noalloc.restype = ctypes.c_int
    lib.fa_bwd_noalloc_max_rows.argtypes = []
    lib.fa_bwd_noalloc_max_rows.restype = ctypes.c_size_t
    lib.fa_bwd_preprocess.argtypes = [P, v, v, v, v]
    lib.fa_bwd_preprocess.restype = ctypes.c_int
    lib.fa_bwd_dkdv.argtypes = [P, v, v, v, v, v, v, v, v, v]
    lib.fa_bwd_dkdv.restype = ctypes.c_int
    lib.fa_bwd_dq.argtypes = [P, v, v, v, v, v, v, v, v]
    lib.fa_bwd_dq.restype = ctypes.c_int
    lib.fa_bwd_workspace_bytes.argtypes = [P]
    lib.fa_bwd_workspace_bytes.restype = ctypes.c_size_t
    M = ctypes.POINTER(FaMaskBuild)
    lib.fa_mask_build_workspace_bytes.argtypes = [M]
    lib.fa_mask_build_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_build_block_mask.argtypes = [M, v, ctypes.c_size_t, v]
    lib.fa_build_block_mask.restype = ctypes.c_int
    lib.fa_strerror.argtypes = [ctypes.c_int]
    lib.fa_strerror.restype = ctypes.c_char_p
    lib.fa_abi_version.argtypes = []
    lib.fa_abi_version.restype = ctypes.c_int
    if lib.fa_abi_version() != ABI_VERSION:
        raise FlexAttnError("libflexattn.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().fa_strerror(status).decode()
        raise FlexAttnError(f"flexattn C ABI error {status}: {msg}")
