"""The C ABI library (CPU): it loads, exports every function include/flexattn.h
declares, and rejects bad arguments before touching the GPU."""
import ctypes
import os
import re

import pytest

from pallas_flexattn import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flexattn.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|uint64_t|void|const char \*)\s*(fa_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTED)
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_and_strerror():
    lib = _lib.load()
    assert lib.fa_abi_version() == _lib.ABI_VERSION
    assert lib.fa_strerror(0) == b"success"
    for code in range(-9, 0):
        assert lib.fa_strerror(code) != b"unknown status"


@pytest.mark.parametrize("cname,pyname", [("fa_params", "FaParams"), ("fa_mask_build", "FaMaskBuild"),
                                          ("fa_kv_cache", "FaKvCache")])
def test_struct_layouts_match_header(cname, pyname, tmp_path):
    """Every field offset and the size of the ctypes mirrors equal what a C
    compiler makes of include/flexattn.h."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    st = getattr(_lib, pyname)
    fields = [f[0] for f in st._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "flexattn.h"\nint main(void) {\n' +
                   "".join(f'  printf("%zu\\n", offsetof(struct {cname}, {f}));\n' for f in fields) +
                   f'  printf("%zu\\n", sizeof(struct {cname}));\n  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [getattr(st, f).offset for f in fields] + [ctypes.sizeof(st)]


def _params(**kw):
    p = _lib.FaParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _lib.DTYPE_BF16
    p.B, p.Hq, p.Hkv, p.Sq, p.Skv, p.D = 1, 2, 2, 128, 128, 128
    p.window_left = p.window_right = -1
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=99), -8), (dict(dtype=7), -3), (dict(D=48), -4), (dict(Hq=3, Hkv=2), -2),
    (dict(Sq=0), -2), (dict(block_m=96), -4), (dict(softcap=-1.0), -2), (dict(dtype=2), -3),
    (dict(block_n=128, D=32), -4), (dict(block_kv=64, D=32), -4), (dict(block_m=256, D=32), -4),
    (dict(q_doc_ids=1234), -1),
    (dict(kv_num_blocks=8, kv_indices=8, mask_block_q=0, mask_block_kv=128), -5),
    (dict(kv_num_blocks=8, kv_indices=8, mask_block_q=128, mask_block_kv=128, table_b=3, table_h=1), -5),
])
def test_fwd_rejects_bad_params_before_any_launch(kw, code):
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    p = _params(**kw)
    assert lib.fa_fwd(ctypes.byref(p), dummy, dummy, dummy, dummy, dummy, None) == code


def test_misaligned_tensors_rejected():
    lib = _lib.load()
    p = _params()
    ok, odd = ctypes.c_void_p(256), ctypes.c_void_p(264)
    assert lib.fa_fwd(ctypes.byref(p), ok, ok, ok, odd, ok, None) == -2
    assert lib.fa_bwd_dq(ctypes.byref(p), ok, ok, ok, ok, ok, ok, odd, None) == -2
    assert lib.fa_bwd_dkdv(ctypes.byref(p), ok, odd, ok, ok, ok, ok, ok, ok, None) == -2


def test_null_pointers_and_small_workspace_rejected():
    lib = _lib.load()
    p = _params()
    d = ctypes.c_void_p(16)
    assert lib.fa_fwd(ctypes.byref(p), None, d, d, d, d, None) == -1
    assert lib.fa_fwd(None, d, d, d, d, d, None) == -1
    need = lib.fa_bwd_workspace_bytes(ctypes.byref(p))
    assert need >= 2 * 128 * 4
    assert lib.fa_bwd(ctypes.byref(p), d, d, d, d, d, d, d, d, d, d, need - 1, None) == -6
    assert lib.fa_bwd_dq(ctypes.byref(p), d, d, d, d, d, None, d, None) == -1


def test_fp8_entry_points_validate_before_any_launch():
    lib = _lib.load()
    d = 16
    p = _params(dtype=_lib.DTYPE_FP8_E4M3)
    inp = _lib.FaFp8Inputs(d, d, d, 128, d, d, d)
    fwd = lambda p, inp: lib.fa_fwd_fp8(ctypes.byref(p), ctypes.byref(inp), d, d, None)  # noqa: E731
    assert fwd(_params(), inp) == -3                      # bf16 params
    assert fwd(_params(dtype=2, D=32), inp) == -4         # head dim 32
    assert fwd(_params(dtype=2, block_n=32), inp) == -4   # tiles other than 128 x 64
    assert fwd(p, _lib.FaFp8Inputs(d, d, d, 100, d, d, d)) == -2   # v_ld not a multiple of 128
    assert fwd(p, _lib.FaFp8Inputs(d, d, d, 0, d, d, d)) == -2     # v_ld < Skv
    assert fwd(p, _lib.FaFp8Inputs(d, d, None, 128, d, d, d)) == -1
    assert fwd(p, _lib.FaFp8Inputs(d, d, d, 128, d, None, d)) == -1
    # the bf16 / fp32 entry points refuse the fp8 dtype
    assert lib.fa_bwd_dq(ctypes.byref(p), d, d, d, d, d, d, d, None) == -3
    assert lib.fa_bwd_noalloc(ctypes.byref(p), d, d, d, d, d, d, d, d, d, None) == -3
    # quantiser
    assert lib.fa_quantize_fp8(d, 1, 128, 48, 0, d, d, None) == -4
    assert lib.fa_quantize_fp8(d, 0, 128, 64, 0, d, d, None) == -2
    assert lib.fa_quantize_fp8(d, 1, 128, 64, 2, d, d, None) == -2
    assert lib.fa_quantize_fp8(None, 1, 128, 64, 0, d, d, None) == -1
    assert lib.fa_quantize_fp8(24, 1, 128, 64, 0, d, d, None) == -2  # misaligned


def _mask_build(**kw):
    m = _lib.FaMaskBuild()
    m.abi_version = _lib.ABI_VERSION
    m.rows, m.q_len, m.kv_len, m.block = 1, 1000, 1000, 128
    m.window_left, m.window_right = -1, 0
    for name, _ in _lib.FaMaskBuild._fields_:
        if name.endswith(("_num", "_indices", "_blocks", "max_counts")):
            setattr(m, name, 16)
    for k, v in kw.items():
        setattr(m, k, v)
    return m


def test_mask_build_workspace_layout():
    lib = _lib.load()
    # flags (1 x 8 x 8 bytes), then the two block-document arrays, each rounded up to 256 bytes
    assert lib.fa_mask_build_workspace_bytes(ctypes.byref(_mask_build())) == 3 * 256
    m = _mask_build(rows=2, doc_ids=16, doc_len=1000, q_len=1000, kv_len=600, block=64)
    assert lib.fa_mask_build_workspace_bytes(ctypes.byref(m)) == 512 + 256 + 256
    assert lib.fa_mask_build_workspace_bytes(ctypes.byref(_mask_build(block=0))) == 0


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=99), -8), (dict(q_len=0), -2), (dict(block=0), -2), (dict(block=2048), -2),
    (dict(rows=2), -2),                                  # several table rows need document ids
    (dict(doc_ids=16, doc_len=999), -2),                 # ids shorter than the sequences
    (dict(q_len=64 * 65535, block=64), -2),              # too many blocks for one launch
    (dict(kv_indices=None), -1), (dict(max_counts=None), -1),
])
def test_mask_build_rejects_bad_arguments_before_any_launch(kw, code):
    lib = _lib.load()
    m = _mask_build(**kw)
    assert lib.fa_build_block_mask(ctypes.byref(m), ctypes.c_void_p(16), 1 << 20, None) == code


def test_mask_build_null_struct_and_small_workspace_rejected():
    lib = _lib.load()
    assert lib.fa_build_block_mask(None, ctypes.c_void_p(16), 1 << 20, None) == -1
    m = _mask_build()
    need = lib.fa_mask_build_workspace_bytes(ctypes.byref(m))
    assert lib.fa_build_block_mask(ctypes.byref(m), ctypes.c_void_p(16), need - 1, None) == -6
    assert lib.fa_build_block_mask(ctypes.byref(m), None, need, None) == -6


def test_mask_build_struct_layout_matches_header():
    m = _lib.FaMaskBuild
    # 7 int32, then the ids pointer (8-byte aligned), doc_len, then 11 pointers
    assert m.doc_ids.offset == 32 and m.doc_len.offset == 40 and m.sampled_num.offset == 48
    assert ctypes.sizeof(m) == m.max_counts.offset + 8 == 48 + 11 * 8
