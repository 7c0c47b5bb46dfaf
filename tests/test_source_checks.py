"""Static checks of the HIP sources (CPU).

`__builtin_bit_cast(T, v[k])` with `v` an ext-vector and `k` an index compiles, with this image's
hipcc (clang, ROCm 7.2), to a cast of element 0 whatever `k` is: four casts of `x[0]` .. `x[3]` of
a `u32x4` read one register, with no diagnostic, and the results are silently wrong.  The kernels
go through a scalar (`const uint32_t w = v[k]; __builtin_bit_cast(T, w)`); this test keeps any
subscripted operand out of `__builtin_bit_cast` in the library's HIP sources and the C header."""
import glob
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pallas-flexattn_amd", "csrc")


def _bit_cast_operands(text):
    """(line, second operand) of every __builtin_bit_cast(...) call in `text`."""
    out, key, i = [], "__builtin_bit_cast(", 0
    while True:
        i = text.find(key, i)
        if i < 0:
            return out
        j, depth, comma = i + len(key), 1, None
        while j < len(text) and depth:
            c = text[j]
            if c in "([{":
                depth += 1
            elif c in ")]}":
                depth -= 1
            elif c == "," and depth == 1 and comma is None:
                comma = j
            j += 1
        if comma is not None:
            out.append((text.count("\n", 0, i) + 1, text[comma + 1:j - 1].strip()))
        i = j


def _subscripted(operands):
    return [(ln, op) for ln, op in operands if op.endswith("]")]


def test_planted_subscript_is_found():
    text = "a = __builtin_bit_cast(bf16x2_t, pf[c][k]);\nb = __builtin_bit_cast(float, f(x[1], 2));\n"
    assert _subscripted(_bit_cast_operands(text)) == [(1, "pf[c][k]")]


def test_no_bit_cast_of_a_subscript():
    files = sorted(glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(CSRC, "*.hip")) +
                   glob.glob(os.path.join(CSRC, "*.cpp")) + glob.glob(os.path.join(ROOT, "include", "*.h")))
    assert files
    bad = []
    for f in files:
        with open(f) as fh:
            bad += [f"{os.path.relpath(f, ROOT)}:{ln}: {op}" for ln, op in _subscripted(_bit_cast_operands(fh.read()))]
    assert not bad, "bit cast of a subscripted operand (reads element 0):\n" + "\n".join(bad)

