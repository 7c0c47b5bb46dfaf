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
ABI_VERSION = 3

DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_FP8_E4M3 = 2

_i32 = ctypes.c_int32
_pi32 = ctypes.c_void_p
_pf = ctypes.c_void_p


class FaParams(ctypes.Structure):
    """Mirror of ``struct fa_params`` (include/flexattn.h)."""
    _fields_ = [
        ("abi_version", _i32), ("dtype", _i32),
        ("B", _i32), ("Hq", _i32), ("Hkv", _i32), ("Sq", _i32), ("Skv", _i32), ("D", _i32),
        ("block_m", _i32), ("block_n", _i32), ("block_kv", _i32),
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
        ("block_q", _i32), ("lds_stages", _i32),
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


class FaKvCache(ctypes.Structure):
    """Mirror of ``struct fa_kv_cache`` (include/flexattn.h)."""
    _fields_ = [("page_table", _pi32), ("page_size", _i32), ("max_pages", _i32), ("num_pages", _i32),
                ("kv_lens", _pi32)]


class FaFp8Inputs(ctypes.Structure):
    """Mirror of ``struct fa_fp8_inputs`` (include/flexattn.h)."""
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("vt", ctypes.c_void_p), ("v_ld", _i32),
                ("q_scale", _pf), ("k_scale", _pf), ("v_scale", _pf)]


EXPORTED = ("fa_fwd", "fa_fwd_fp8", "fa_quantize_fp8", "fa_fwd_host", "fa_bwd_preprocess_host", "fa_bwd_dkdv_host",
            "fa_bwd_dq_host", "fa_bwd_host", "fa_fwd_splitkv", "fa_fwd_splitkv_workspace_bytes", "fa_fwd_kvcache",
            "fa_fwd_kvcache_workspace_bytes", "fa_bwd", "fa_bwd_workspace_bytes",
            "fa_bwd_noalloc", "fa_bwd_noalloc_max_rows", "fa_bwd_preprocess", "fa_bwd_dkdv", "fa_bwd_dq",
            "fa_mask_build_workspace_bytes", "fa_build_block_mask", "fa_strerror", "fa_abi_version",
            "fa_mods_compile", "fa_mods_free_blob", "fa_mods_load", "fa_mods_unload", "fa_mods_fwd", "fa_mods_bwd",
            "fa_mods_bwd_dkdv", "fa_mods_bwd_dq", "fa_mods_source_hash")

MODS_MASK, MODS_SCORE, MODS_BUILTIN_SCORE = 1, 2, 4

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
    KV = ctypes.POINTER(FaKvCache)
    lib.fa_fwd_kvcache.argtypes = [P, KV, v, v, v, v, v, ctypes.c_int, v, ctypes.c_size_t, v]
    lib.fa_fwd_kvcache.restype = ctypes.c_int
    ci = ctypes.c_int
    lib.fa_fwd_host.argtypes = [P, v, v, v, v, v, ci]
    lib.fa_bwd_preprocess_host.argtypes = [P, v, v, v, ci]
    lib.fa_bwd_dkdv_host.argtypes = [P, v, v, v, v, v, v, v, v, ci]
    lib.fa_bwd_dq_host.argtypes = [P, v, v, v, v, v, v, v, ci]
    lib.fa_bwd_host.argtypes = [P, v, v, v, v, v, v, v, v, v, ci]
    for n in ("fa_fwd_host", "fa_bwd_preprocess_host", "fa_bwd_dkdv_host", "fa_bwd_dq_host", "fa_bwd_host"):
        getattr(lib, n).restype = ci
    lib.fa_fwd_fp8.argtypes = [P, ctypes.POINTER(FaFp8Inputs), v, v, v]
    lib.fa_fwd_fp8.restype = ctypes.c_int
    i32 = ctypes.c_int32
    lib.fa_quantize_fp8.argtypes = [v, i32, i32, i32, i32, v, v, v]
    lib.fa_quantize_fp8.restype = ctypes.c_int
    lib.fa_fwd_kvcache_workspace_bytes.argtypes = [P, KV, ctypes.c_int]
    lib.fa_fwd_kvcache_workspace_bytes.restype = ctypes.c_size_t
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
    i = ctypes.c_int
    lib.fa_mods_compile.argtypes = [ctypes.c_char_p, i, i, i, ctypes.POINTER(v), ctypes.POINTER(ctypes.c_size_t),
                                    ctypes.c_char_p, ctypes.c_size_t]
    lib.fa_mods_compile.restype = i
    lib.fa_mods_free_blob.argtypes = [v]
    lib.fa_mods_free_blob.restype = None
    lib.fa_mods_load.argtypes = [v, ctypes.c_size_t, ctypes.POINTER(v)]
    lib.fa_mods_load.restype = i
    lib.fa_mods_unload.argtypes = [v]
    lib.fa_mods_unload.restype = i
    lib.fa_mods_fwd.argtypes = [v, P, v, i, v, v, v, v, v, v]
    lib.fa_mods_fwd.restype = i
    lib.fa_mods_bwd.argtypes = [v, P, v, i, v, v, v, v, v, v, v, v, v, v, ctypes.c_size_t, v]
    lib.fa_mods_bwd.restype = i
    lib.fa_mods_bwd_dkdv.argtypes = [v, P, v, i, v, v, v, v, v, v, v, v, v]
    lib.fa_mods_bwd_dkdv.restype = i
    lib.fa_mods_bwd_dq.argtypes = [v, P, v, i, v, v, v, v, v, v, v, v]
    lib.fa_mods_bwd_dq.restype = i
    lib.fa_strerror.argtypes = [ctypes.c_int]
    lib.fa_strerror.restype = ctypes.c_char_p
    lib.fa_mods_source_hash.argtypes = []
    lib.fa_mods_source_hash.restype = ctypes.c_uint64
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


# Runs fa_mods_compile in a fresh interpreter.  torch ships its own copies of
# the HIP runtime, hipRTC and comgr (an older LLVM than the one libflexattn.so
# is built with); once torch is imported those copies serve the whole
# process, so an in-process compile would use a different compiler than the
# library's own kernels (and reject the library's compile options).  The child
# loads only libflexattn.so and the ROCm libraries it was linked against.
_CHILD = r"""
import ctypes, sys
lib = ctypes.CDLL(sys.argv[1])
lib.fa_mods_compile.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t),
                                ctypes.c_char_p, ctypes.c_size_t]
lib.fa_mods_free_blob.argtypes = [ctypes.c_void_p]
src = sys.stdin.buffer.read()
blob, size = ctypes.c_void_p(), ctypes.c_size_t()
log = ctypes.create_string_buffer(1 << 16)
rc = lib.fa_mods_compile(src, int(sys.argv[2]), int(sys.argv[3]), int(sys.argv[4]), ctypes.byref(blob),
                         ctypes.byref(size), log, len(log))
sys.stderr.write(log.value.decode(errors="replace"))
if rc == 0:
    with open(sys.argv[5], "wb") as f:
        f.write(ctypes.string_at(blob, size.value))
    lib.fa_mods_free_blob(blob)
sys.exit(0 if rc == 0 else 3)
"""


def compile_mods(source: str, dtype: int, head_dim: int, flags: int) -> bytes:
    """Compile a user-mods policy (C ABI fa_mods_compile, no GPU needed) in a
    child interpreter and return the code blob.  Raises FlexAttnError with
    the compiler log."""
    import subprocess
    import sys
    import tempfile
    if not os.path.exists(LIB_PATH):
        load()  # raises the missing-library error
    fd, out = tempfile.mkstemp(suffix=".blob")
    os.close(fd)
    try:
        res = subprocess.run([sys.executable, "-c", _CHILD, LIB_PATH, str(dtype), str(head_dim), str(flags), out],
                             input=source.encode(), capture_output=True, timeout=600)
        if res.returncode != 0:
            raise FlexAttnError(f"compiling the user mods failed (exit {res.returncode}):\n"
                                f"{res.stderr.decode(errors='replace')[-8000:]}\n--- policy source ---\n{source}")
        with open(out, "rb") as f:
            return f.read()
    finally:
        os.unlink(out)
