"""Lowering of user ``mask_mod`` / ``score_mod`` callables onto the kernels.

The reference evaluates any ``mask_mod(q_idx, kv_idx)`` callable per element
inside its Pallas kernels (``flash_attn.py:85-88``, ``:236-239``,
``:341-344``).  Here a callable is traced once: it is called with symbolic
arguments whose operators record an expression (integer / float / boolean
arithmetic, comparisons, ``&`` ``|`` ``~``, ``torch.where``, ``tanh`` ``exp``
``log`` ``sqrt`` ``abs`` ``minimum`` ``maximum`` ...,  and reads of captured
torch tensors indexed by the symbolic indices, e.g. ``bias[h, q_idx, kv_idx]``).
The expression is

* emitted as the C++ element policy of the tile kernels (``struct UserMod``,
  compiled at run time through the C ABI ``fa_mods_compile``), with the
  derivative of a score mod with respect to the score taken symbolically for
  the backward;
* evaluated with numpy on the host, so block masks of traced masks are built
  from the very expression the kernels run.

Python control flow on symbolic values (``if q_idx > kv_idx:``, ``and``,
``or``) cannot be traced and raises :class:`LoweringError`; use ``&``, ``|``
and ``torch.where`` instead.  Tensor reads are clamped to the tensor's extent
(an out-of-range index reads the nearest element instead of faulting).
"""
import hashlib
import inspect
import math
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

VARS = ("b", "h", "q", "kv", "score")


class LoweringError(TypeError):
    """A callable that cannot be lowered onto the kernels."""


# --------------------------------------------------------------- the IR ----
class Expr:
    """Immutable expression node.  dtype: 'i' (int32), 'f' (float32), 'b' (bool)."""
    __slots__ = ("op", "args", "dtype", "value", "_h")

    def __init__(self, op, args=(), dtype="i", value=None):
        self.op, self.args, self.dtype, self.value = op, tuple(args), dtype, value
        self._h = None

    def key(self):
        if self._h is None:
            self._h = (self.op, self.dtype, self.value if self.op != "gather" else self.value[:1],
                       tuple(a.key() for a in self.args))
        return self._h

    def uses(self) -> set:
        if self.op == "var":
            return {self.value}
        out = set()
        for a in self.args:
            out |= a.uses()
        return out

    def gathers(self) -> list:
        out = [self] if self.op == "gather" else []
        for a in self.args:
            out += a.gathers()
        return out


def const(v) -> Expr:
    if isinstance(v, (bool, np.bool_)):
        return Expr("const", dtype="b", value=bool(v))
    if isinstance(v, (int, np.integer)):
        if not -2 ** 31 <= int(v) < 2 ** 31:
            raise LoweringError(f"integer constant {v} does not fit in int32")
        return Expr("const", dtype="i", value=int(v))
    if isinstance(v, (float, np.floating)):
        return Expr("const", dtype="f", value=float(v))
    raise LoweringError(f"cannot lower constant {v!r} of type {type(v).__name__}")


def _promote(a: Expr, b: Expr) -> str:
    if "f" in (a.dtype, b.dtype):
        return "f"
    return "i"


_BIN_NUMERIC = {"add", "sub", "mul", "truediv", "floordiv", "mod", "pow", "min", "max"}
_CMP = {"lt", "le", "gt", "ge", "eq", "ne"}
_LOGIC = {"and", "or", "xor"}
_UNARY_F = {"tanh", "exp", "log", "sqrt", "sigmoid", "exp2", "log2", "sin", "cos", "floor", "ceil"}


def binop(op, a: Expr, b: Expr) -> Expr:
    if op in _CMP:
        return Expr(op, (a, b), "b")
    if op in _LOGIC:
        if a.dtype == "b" and b.dtype == "b":
            return Expr(op, (a, b), "b")
        if a.dtype == "f" or b.dtype == "f":
            raise LoweringError(f"bitwise {op} of float values")
        return Expr(op, (a, b), "i")
    if op == "truediv":
        return Expr(op, (a, b), "f")
    if op == "pow":
        return Expr(op, (a, b), "f")
    return Expr(op, (a, b), _promote(a, b))


def unop(op, a: Expr) -> Expr:
    if op == "not":
        return Expr("not" if a.dtype == "b" else "bitnot", (a,), a.dtype if a.dtype != "f" else "i")
    if op in ("neg", "abs"):
        return Expr(op, (a,), "i" if a.dtype == "b" else a.dtype)
    if op in _UNARY_F:
        return Expr(op, (a,), "f")
    if op == "float":
        return Expr("float", (a,), "f")
    if op == "int":
        return Expr("int", (a,), "i")
    if op == "bool":
        return Expr("ne", (a, const(0)), "b")
    raise LoweringError(op)


def where(c: Expr, a: Expr, b: Expr) -> Expr:
    if c.dtype != "b":
        c = Expr("ne", (c, const(0)), "b")
    if a.dtype == "b" and b.dtype == "b":
        dt = "b"
    else:
        dt = _promote(a, b) if "b" not in (a.dtype, b.dtype) else ("f" if "f" in (a.dtype, b.dtype) else "i")
    return Expr("where", (c, a, b), dt)


# ------------------------------------------------------------- tracing ----
def _as_expr(x) -> Expr:
    if isinstance(x, Sym):
        return x.e
    if isinstance(x, Expr):
        return x
    if _is_torch_tensor(x):
        if x.dim() == 0:
            v = x.item()
            return const(v)
        raise LoweringError("a captured tensor must be indexed by the symbolic indices (e.g. t[h, q_idx]) "
                            "before it is combined with them")
    if isinstance(x, np.ndarray):
        if x.ndim == 0:
            return const(x.item())
        raise LoweringError("numpy arrays cannot be indexed by symbolic indices: capture a torch tensor")
    return const(x)


def _is_torch_tensor(x):
    return type(x).__module__.startswith("torch") and hasattr(x, "dim")


class _Capture:
    """Tensors read by the traced expression, in first-use order."""

    def __init__(self):
        self.tensors: List = []

    def slot(self, t) -> int:
        for i, u in enumerate(self.tensors):
            if u is t:
                return i
        if len(self.tensors) >= 8:
            raise LoweringError("at most 8 captured tensors per set of mods")
        self.tensors.append(t)
        return len(self.tensors) - 1


_ACTIVE: List[_Capture] = []


def _gather(t, idx) -> Expr:
    if not _ACTIVE:
        raise LoweringError("tensor read outside a trace")
    if not isinstance(idx, tuple):
        idx = (idx,)
    if len(idx) != t.dim():
        raise LoweringError(f"a captured tensor of shape {tuple(t.shape)} must be read with {t.dim()} indices "
                            f"(one element per (b, h, q_idx, kv_idx)), got {len(idx)}")
    ie = []
    for i in idx:
        if isinstance(i, slice) or i is None or i is Ellipsis:
            raise LoweringError("slices of captured tensors cannot be lowered; index every dimension")
        e = _as_expr(i)
        if e.dtype == "f":
            raise LoweringError("tensor index is a float expression")
        ie.append(e)
    import torch
    if t.dtype == torch.bool:
        kind = "b"
    elif t.is_floating_point():
        kind = "f"
    else:
        kind = "i"
    slot = _ACTIVE[-1].slot(t)
    return Expr("gather", ie, kind, (slot, tuple(int(s) for s in t.shape)))


def _torch_fns():
    import torch
    F = torch.Tensor
    return {
        torch.where: lambda c, a, b: Sym(where(_as_expr(c), _as_expr(a), _as_expr(b))),
        torch.tanh: lambda a: Sym(unop("tanh", _as_expr(a))),
        torch.exp: lambda a: Sym(unop("exp", _as_expr(a))),
        torch.exp2: lambda a: Sym(unop("exp2", _as_expr(a))),
        torch.log: lambda a: Sym(unop("log", _as_expr(a))),
        torch.log2: lambda a: Sym(unop("log2", _as_expr(a))),
        torch.sqrt: lambda a: Sym(unop("sqrt", _as_expr(a))),
        torch.sigmoid: lambda a: Sym(unop("sigmoid", _as_expr(a))),
        torch.sin: lambda a: Sym(unop("sin", _as_expr(a))),
        torch.cos: lambda a: Sym(unop("cos", _as_expr(a))),
        torch.floor: lambda a: Sym(unop("floor", _as_expr(a))),
        torch.ceil: lambda a: Sym(unop("ceil", _as_expr(a))),
        torch.abs: lambda a: Sym(unop("abs", _as_expr(a))),
        torch.neg: lambda a: Sym(unop("neg", _as_expr(a))),
        torch.logical_not: lambda a: Sym(unop("not", _bool(_as_expr(a)))),
        torch.logical_and: lambda a, b: Sym(binop("and", _bool(_as_expr(a)), _bool(_as_expr(b)))),
        torch.logical_or: lambda a, b: Sym(binop("or", _bool(_as_expr(a)), _bool(_as_expr(b)))),
        torch.logical_xor: lambda a, b: Sym(binop("xor", _bool(_as_expr(a)), _bool(_as_expr(b)))),
        torch.minimum: lambda a, b: Sym(binop("min", _as_expr(a), _as_expr(b))),
        torch.maximum: lambda a, b: Sym(binop("max", _as_expr(a), _as_expr(b))),
        torch.remainder: lambda a, b: Sym(binop("mod", _as_expr(a), _as_expr(b))),
        torch.floor_divide: lambda a, b: Sym(binop("floordiv", _as_expr(a), _as_expr(b))),
        torch.clamp: _clamp,
        torch.pow: lambda a, b: Sym(binop("pow", _as_expr(a), _as_expr(b))),
        F.__getitem__: lambda t, idx: Sym(_gather(t, idx)),
        F.abs: lambda a: Sym(unop("abs", _as_expr(a))),
        F.tanh: lambda a: Sym(unop("tanh", _as_expr(a))),
        F.exp: lambda a: Sym(unop("exp", _as_expr(a))),
        F.float: lambda a: Sym(unop("float", _as_expr(a))),
        F.int: lambda a: Sym(unop("int", _as_expr(a))),
        F.long: lambda a: Sym(unop("int", _as_expr(a))),
        F.bool: lambda a: Sym(unop("bool", _as_expr(a))),
    }


def _bool(e: Expr) -> Expr:
    return e if e.dtype == "b" else Expr("ne", (e, const(0)), "b")


def _clamp(a, min=None, max=None):
    e = _as_expr(a)
    if min is not None:
        e = binop("max", e, _as_expr(min))
    if max is not None:
        e = binop("min", e, _as_expr(max))
    return Sym(e)


_NP_UFUNCS = {
    "add": "add", "subtract": "sub", "multiply": "mul", "true_divide": "truediv", "divide": "truediv",
    "floor_divide": "floordiv", "remainder": "mod", "mod": "mod", "power": "pow", "minimum": "min",
    "maximum": "max", "fmin": "min", "fmax": "max", "less": "lt", "less_equal": "le", "greater": "gt",
    "greater_equal": "ge", "equal": "eq", "not_equal": "ne", "logical_and": "and", "logical_or": "or",
    "logical_xor": "xor", "bitwise_and": "and", "bitwise_or": "or", "bitwise_xor": "xor",
}
_NP_UNARY = {"tanh": "tanh", "exp": "exp", "exp2": "exp2", "log": "log", "log2": "log2", "sqrt": "sqrt",
             "sin": "sin", "cos": "cos", "floor": "floor", "ceil": "ceil", "absolute": "abs", "negative": "neg",
             "logical_not": "not", "invert": "not"}


class Sym:
    """A traced value.  Operators build :class:`Expr` nodes."""
    __slots__ = ("e",)
    __array_priority__ = 1000

    def __init__(self, e: Expr):
        self.e = e

    def _b(self, op, other, rev=False):
        o = _as_expr(other)
        return Sym(binop(op, o, self.e) if rev else binop(op, self.e, o))

    __add__ = lambda s, o: s._b("add", o)
    __radd__ = lambda s, o: s._b("add", o, True)
    __sub__ = lambda s, o: s._b("sub", o)
    __rsub__ = lambda s, o: s._b("sub", o, True)
    __mul__ = lambda s, o: s._b("mul", o)
    __rmul__ = lambda s, o: s._b("mul", o, True)
    __truediv__ = lambda s, o: s._b("truediv", o)
    __rtruediv__ = lambda s, o: s._b("truediv", o, True)
    __floordiv__ = lambda s, o: s._b("floordiv", o)
    __rfloordiv__ = lambda s, o: s._b("floordiv", o, True)
    __mod__ = lambda s, o: s._b("mod", o)
    __rmod__ = lambda s, o: s._b("mod", o, True)
    __pow__ = lambda s, o: s._b("pow", o)
    __lt__ = lambda s, o: s._b("lt", o)
    __le__ = lambda s, o: s._b("le", o)
    __gt__ = lambda s, o: s._b("gt", o)
    __ge__ = lambda s, o: s._b("ge", o)
    __eq__ = lambda s, o: s._b("eq", o)
    __ne__ = lambda s, o: s._b("ne", o)
    __and__ = lambda s, o: s._b("and", o)
    __rand__ = lambda s, o: s._b("and", o, True)
    __or__ = lambda s, o: s._b("or", o)
    __ror__ = lambda s, o: s._b("or", o, True)
    __xor__ = lambda s, o: s._b("xor", o)
    __rxor__ = lambda s, o: s._b("xor", o, True)
    __neg__ = lambda s: Sym(unop("neg", s.e))
    __pos__ = lambda s: s
    __abs__ = lambda s: Sym(unop("abs", s.e))
    __invert__ = lambda s: Sym(unop("not", s.e))
    __hash__ = None

    def __bool__(self):
        raise LoweringError("Python control flow (if / and / or / not) on a traced index or score cannot be "
                            "lowered onto the kernels: write it with &, |, ~ and torch.where")

    def __index__(self):
        raise LoweringError("a traced index was used where Python needs a concrete integer (e.g. to index a "
                            "list or numpy array): capture a torch tensor and index it instead")

    __int__ = __index__

    def __float__(self):
        raise LoweringError("a traced value was converted to a Python float")

    # torch and numpy entry points
    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        fn = _torch_fns().get(func)
        if fn is None:
            raise LoweringError(f"{getattr(func, '__name__', func)} cannot be lowered onto the kernels")
        return fn(*args, **kwargs)

    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        if method != "__call__" or kwargs:
            raise LoweringError(f"numpy {ufunc.__name__}.{method} cannot be lowered")
        if ufunc.__name__ in _NP_UNARY and len(inputs) == 1:
            return Sym(unop(_NP_UNARY[ufunc.__name__], _as_expr(inputs[0])))
        if ufunc.__name__ in _NP_UFUNCS and len(inputs) == 2:
            a, b = _as_expr(inputs[0]), _as_expr(inputs[1])
            op = _NP_UFUNCS[ufunc.__name__]
            if op in _LOGIC and ufunc.__name__.startswith("logical"):
                a, b = _bool(a), _bool(b)
            return Sym(binop(op, a, b))
        raise LoweringError(f"numpy {ufunc.__name__} cannot be lowered")

    def __array_function__(self, func, types, args, kwargs):
        if func is np.where and len(args) == 3 and not kwargs:
            return Sym(where(*(_as_expr(a) for a in args)))
        if func in (np.minimum, np.maximum, np.clip):
            pass
        raise LoweringError(f"numpy {func.__name__} cannot be lowered")


def _arity(fn) -> int:
    try:
        params = [p for p in inspect.signature(fn).parameters.values()
                  if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD, p.VAR_POSITIONAL)]
    except (TypeError, ValueError):
        return 2
    if any(p.kind == p.VAR_POSITIONAL for p in params):
        return 4
    return len(params)


def _trace(fn, args) -> Tuple[Expr, list]:
    cap = _Capture()
    _ACTIVE.append(cap)
    try:
        out = fn(*args)
    except LoweringError:
        raise
    except Exception as e:  # anything else the callable did with traced values
        raise LoweringError(f"tracing the callable raised {type(e).__name__}: {e}") from e
    finally:
        _ACTIVE.pop()
    return _as_expr(out), cap.tensors


def trace_mask(fn) -> Tuple[Expr, list]:
    """Expression of a mask mod ``(q_idx, kv_idx)`` or ``(b, h, q_idx, kv_idx)``."""
    b, h, q, kv = (Sym(Expr("var", dtype="i", value=v)) for v in ("b", "h", "q", "kv"))
    n = _arity(fn)
    e, tensors = _trace(fn, (q, kv) if n == 2 else (b, h, q, kv))
    return _bool(e), tensors


def trace_score(fn) -> Tuple[Expr, list]:
    """Expression of a score mod ``(score, b, h, q_idx, kv_idx)``."""
    s = Sym(Expr("var", dtype="f", value="score"))
    b, h, q, kv = (Sym(Expr("var", dtype="i", value=v)) for v in ("b", "h", "q", "kv"))
    e, tensors = _trace(fn, (s, b, h, q, kv))
    if e.dtype != "f":
        e = unop("float", e)
    return e, tensors


# ---------------------------------------------------------- derivative ----
ZERO = Expr("const", dtype="f", value=0.0)
ONE = Expr("const", dtype="f", value=1.0)


def _is(e, v):
    return e.op == "const" and e.value == v


def _add(a, b):
    if _is(a, 0.0) or _is(a, 0):
        return b
    if _is(b, 0.0) or _is(b, 0):
        return a
    return binop("add", a, b)


def _mul(a, b):
    if _is(a, 0.0) or _is(b, 0.0) or _is(a, 0) or _is(b, 0):
        return ZERO
    if _is(a, 1.0):
        return b
    if _is(b, 1.0):
        return a
    return binop("mul", a, b)


def _fconst(v):
    return Expr("const", dtype="f", value=float(v))


def derivative(e: Expr) -> Expr:
    """d e / d score (0 for integer and boolean parts)."""
    if e.dtype != "f" or "score" not in e.uses():
        return ZERO
    op, a = e.op, e.args
    if op == "var":
        return ONE
    if op in ("add", "sub"):
        da, db = derivative(a[0]), derivative(a[1])
        return _add(da, db) if op == "add" else _add(da, _mul(_fconst(-1), db))
    if op == "mul":
        return _add(_mul(derivative(a[0]), a[1]), _mul(a[0], derivative(a[1])))
    if op == "truediv":
        da, db = derivative(a[0]), derivative(a[1])
        num = _add(_mul(da, a[1]), _mul(_fconst(-1), _mul(a[0], db)))
        return binop("truediv", num, binop("mul", a[1], a[1])) if not _is(num, 0.0) else ZERO
    if op == "neg":
        return _mul(_fconst(-1), derivative(a[0]))
    if op == "pow":
        if a[1].op != "const":
            raise LoweringError("the derivative of x ** y needs a constant exponent")
        c = float(a[1].value)
        return _mul(_mul(_fconst(c), binop("pow", a[0], _fconst(c - 1))), derivative(a[0]))
    da = derivative(a[0]) if a else ZERO
    if op == "tanh":
        return _mul(binop("sub", ONE, binop("mul", e, e)), da)
    if op == "exp":
        return _mul(e, da)
    if op == "exp2":
        return _mul(_mul(e, _fconst(math.log(2))), da)
    if op == "log":
        return _mul(binop("truediv", ONE, a[0]), da)
    if op == "log2":
        return _mul(binop("truediv", _fconst(1 / math.log(2)), a[0]), da)
    if op == "sqrt":
        return _mul(binop("truediv", _fconst(0.5), e), da)
    if op == "sigmoid":
        return _mul(binop("mul", e, binop("sub", ONE, e)), da)
    if op == "sin":
        return _mul(unop("cos", a[0]), da)
    if op == "cos":
        return _mul(unop("neg", unop("sin", a[0])), da)
    if op == "abs":
        return _mul(where(binop("lt", a[0], ZERO), _fconst(-1), ONE), da)
    if op in ("floor", "ceil", "mod", "floordiv"):
        return ZERO
    if op in ("min", "max"):
        pick_a = binop("le" if op == "min" else "ge", a[0], a[1])
        return where(pick_a, derivative(a[0]), derivative(a[1]))
    if op == "where":
        return where(a[0], derivative(a[1]), derivative(a[2]))
    if op == "float":
        return derivative(a[0])
    if op == "gather":
        raise LoweringError("a tensor read whose index depends on the score has no derivative")
    raise LoweringError(f"no derivative rule for {op}")


# -------------------------------------------------------------- codegen ----
_CTYPE = {"i": "int", "f": "float", "b": "bool"}
_CBIN = {"add": "+", "sub": "-", "mul": "*", "lt": "<", "le": "<=", "gt": ">", "ge": ">=", "eq": "==", "ne": "!="}
_CFUN = {"tanh": "tanhf", "exp": "expf", "log": "logf", "sqrt": "sqrtf", "exp2": "exp2f", "log2": "log2f",
         "sin": "sinf", "cos": "cosf", "floor": "floorf", "ceil": "ceilf"}


def _cast(code: str, src: str, dst: str) -> str:
    if src == dst:
        return code
    return f"(({_CTYPE[dst]})({code}))"


def emit(e: Expr) -> str:
    """C++ expression for e (variables b, h, q, kv, s; tensors through p.mod_buf)."""
    op, a = e.op, e.args
    if op == "const":
        if e.dtype == "b":
            return "true" if e.value else "false"
        if e.dtype == "i":
            # -2^31 written as a literal would be the negation of a long
            return "(-2147483647 - 1)" if e.value == -2 ** 31 else f"({e.value})"
        v = e.value
        if math.isinf(v):
            return "(INFINITY)" if v > 0 else "(-INFINITY)"
        if math.isnan(v):
            return "(__builtin_nanf(\"\"))"
        return f"({v!r}f)" if "e" in repr(v) or "." in repr(v) else f"({v!r}.0f)"
    if op == "var":
        return "s" if e.value == "score" else e.value
    if op in _CBIN:
        dt = "f" if "f" in (a[0].dtype, a[1].dtype) and op in ("add", "sub", "mul") else None
        if op in ("add", "sub", "mul"):
            t = e.dtype
            return f"({_cast(emit(a[0]), a[0].dtype, t)} {_CBIN[op]} {_cast(emit(a[1]), a[1].dtype, t)})"
        t = "f" if "f" in (a[0].dtype, a[1].dtype) else "i"
        return f"({_cast(emit(a[0]), a[0].dtype, t)} {_CBIN[op]} {_cast(emit(a[1]), a[1].dtype, t)})"
    if op == "truediv":
        return f"({_cast(emit(a[0]), a[0].dtype, 'f')} / {_cast(emit(a[1]), a[1].dtype, 'f')})"
    if op in ("floordiv", "mod"):
        if e.dtype == "f":
            x, y = _cast(emit(a[0]), a[0].dtype, "f"), _cast(emit(a[1]), a[1].dtype, "f")
            return f"um_f{op}({x}, {y})"
        return f"um_i{op}({emit(a[0])}, {emit(a[1])})"
    if op == "pow":
        x, y = _cast(emit(a[0]), a[0].dtype, "f"), _cast(emit(a[1]), a[1].dtype, "f")
        if a[1].op == "const" and a[1].value == 2:
            return f"um_sq({x})"
        return f"powf({x}, {y})"
    if op in ("min", "max"):
        if e.dtype == "f":
            return f"f{op}f({_cast(emit(a[0]), a[0].dtype, 'f')}, {_cast(emit(a[1]), a[1].dtype, 'f')})"
        return f"{op}({_cast(emit(a[0]), a[0].dtype, 'i')}, {_cast(emit(a[1]), a[1].dtype, 'i')})"
    if op in ("and", "or", "xor"):
        if e.dtype == "b":
            c = {"and": "&&", "or": "||", "xor": "!="}[op]
        else:
            c = {"and": "&", "or": "|", "xor": "^"}[op]
        return f"({emit(a[0])} {c} {emit(a[1])})"
    if op == "not":
        return f"(!{emit(a[0])})"
    if op == "bitnot":
        return f"(~{_cast(emit(a[0]), a[0].dtype, 'i')})"
    if op == "neg":
        return f"(-{_cast(emit(a[0]), a[0].dtype, e.dtype)})"
    if op == "abs":
        return f"fabsf({emit(a[0])})" if e.dtype == "f" else f"abs({_cast(emit(a[0]), a[0].dtype, 'i')})"
    if op in _CFUN:
        return f"{_CFUN[op]}({_cast(emit(a[0]), a[0].dtype, 'f')})"
    if op == "sigmoid":
        return f"um_sigmoid({_cast(emit(a[0]), a[0].dtype, 'f')})"
    if op == "float":
        return _cast(emit(a[0]), a[0].dtype, "f")
    if op == "int":
        return _cast(emit(a[0]), a[0].dtype, "i")
    if op == "where":
        t = e.dtype
        return (f"({emit(a[0])} ? {_cast(emit(a[1]), a[1].dtype, t)} : "
                f"{_cast(emit(a[2]), a[2].dtype, t)})")
    if op == "gather":
        slot, shape = e.value
        off, stride = [], 1
        terms = []
        for i in reversed(range(len(shape))):
            idx = f"um_clamp({_cast(emit(a[i]), a[i].dtype, 'i')}, {shape[i]})"
            terms.append(f"(long)({idx}) * {stride}L" if stride != 1 else f"(long)({idx})")
            stride *= shape[i]
        ty = {"f": "float", "i": "int", "b": "int"}[e.dtype]
        code = f"static_cast<const {ty}*>(p.mod_buf[{slot}])[{' + '.join(terms) or '0'}]"
        return f"({code} != 0)" if e.dtype == "b" else code
    raise LoweringError(f"no code for {op}")


_PRELUDE = """
namespace um {
__device__ __forceinline__ int um_clamp(int i, int n) { return i < 0 ? 0 : (i >= n ? n - 1 : i); }
// Python's floor division and modulo (sign of the divisor)
__device__ __forceinline__ int um_ifloordiv(int a, int b) {
  const int q = a / b;
  return (q * b != a && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__device__ __forceinline__ int um_imod(int a, int b) {
  const int r = a % b;
  return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
__device__ __forceinline__ float um_ffloordiv(float a, float b) { return floorf(a / b); }
__device__ __forceinline__ float um_fmod(float a, float b) { return a - b * floorf(a / b); }
__device__ __forceinline__ float um_sq(float x) { return x * x; }
__device__ __forceinline__ float um_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
}  // namespace um
"""


def policy_source(mask: Optional[Expr], score: Optional[Expr]) -> str:
    """C++ source of ``struct UserMod`` for the kernels (see include/flexattn.h)."""
    lines = [_PRELUDE, "struct UserMod {",
             f"  static constexpr bool kMask = {'true' if mask is not None else 'false'};",
             f"  static constexpr bool kScore = {'true' if score is not None else 'false'};",
             "  __device__ static bool mask(const fa::Problem& p, int b, int h, int q, int kv) {",
             "    using namespace um;",
             f"    return {emit(mask) if mask is not None else 'true'};",
             "  }",
             "  __device__ static float score(const fa::Problem& p, float s, int b, int h, int q, int kv, "
             "float* dsds) {",
             "    using namespace um;"]
    if score is not None:
        d = derivative(score)
        lines += [f"    *dsds = {_cast(emit(d), d.dtype, 'f')};",
                  f"    return {_cast(emit(score), score.dtype, 'f')};"]
    else:
        lines += ["    *dsds = 1.0f;", "    return s;"]
    lines += ["  }", "};", ""]
    return "\n".join(lines)


# ----------------------------------------------------- host evaluation ----
def evaluate(e: Expr, env: Dict[str, object], tensors: List[np.ndarray]):
    """numpy value of e with the variables in env (arrays broadcast)."""
    op, a = e.op, e.args
    if op == "const":
        return {"b": np.bool_, "i": np.int64, "f": np.float32}[e.dtype](e.value)
    if op == "var":
        return env[e.value]
    if op == "gather":
        slot, shape = e.value
        idx = tuple(np.clip(np.asarray(evaluate(x, env, tensors), dtype=np.int64), 0, n - 1)
                    for x, n in zip(a, shape))
        v = tensors[slot][idx]
        return v != 0 if e.dtype == "b" else v
    vals = [evaluate(x, env, tensors) for x in a]
    f32 = lambda x: np.asarray(x, dtype=np.float32)
    if op in ("add", "sub", "mul"):
        x, y = (f32(v) for v in vals) if e.dtype == "f" else (np.asarray(v, np.int64) for v in vals)
        return {"add": np.add, "sub": np.subtract, "mul": np.multiply}[op](x, y)
    if op == "truediv":
        return f32(vals[0]) / f32(vals[1])
    if op == "floordiv":
        return np.floor_divide(f32(vals[0]), f32(vals[1])) if e.dtype == "f" else \
            np.floor_divide(np.asarray(vals[0], np.int64), np.asarray(vals[1], np.int64))
    if op == "mod":
        return np.mod(f32(vals[0]), f32(vals[1])) if e.dtype == "f" else \
            np.mod(np.asarray(vals[0], np.int64), np.asarray(vals[1], np.int64))
    if op == "pow":
        return np.power(f32(vals[0]), f32(vals[1]))
    if op in _CMP:
        fn = {"lt": np.less, "le": np.less_equal, "gt": np.greater, "ge": np.greater_equal, "eq": np.equal,
              "ne": np.not_equal}[op]
        return fn(*vals)
    if op in ("min", "max"):
        return (np.minimum if op == "min" else np.maximum)(*vals)
    if op in ("and", "or", "xor"):
        fn = {"and": np.logical_and, "or": np.logical_or, "xor": np.logical_xor} if e.dtype == "b" else \
            {"and": np.bitwise_and, "or": np.bitwise_or, "xor": np.bitwise_xor}
        return fn[op](*vals)
    if op == "not":
        return np.logical_not(vals[0])
    if op == "bitnot":
        return np.invert(np.asarray(vals[0], np.int64))
    if op == "neg":
        return np.negative(vals[0])
    if op == "abs":
        return np.abs(vals[0])
    if op in ("tanh", "exp", "log", "sqrt", "exp2", "log2", "sin", "cos", "floor", "ceil"):
        return getattr(np, op)(f32(vals[0]))
    if op == "sigmoid":
        return 1.0 / (1.0 + np.exp(-f32(vals[0])))
    if op == "float":
        return f32(vals[0])
    if op == "int":
        return np.asarray(vals[0]).astype(np.int64)
    if op == "where":
        return np.where(*vals)
    raise LoweringError(op)


# ---------------------------------------------------------- the result ----
class LoweredMask:
    """A traced mask mod: callable with ``(q_idx, kv_idx)`` or
    ``(b, h, q_idx, kv_idx)`` on numpy arrays (evaluating the traced
    expression), and carrying what the kernels need."""

    def __init__(self, fn: Callable):
        self.fn = fn
        self.arity = 4 if _arity(fn) >= 4 else 2
        self.expr, self.tensors = trace_mask(fn)
        uses = self.expr.uses()
        self.batch_dependent = "b" in uses
        self.head_dependent = "h" in uses
        self._host = None

    def host_tensors(self):
        if self._host is None:
            self._host = [t.detach().cpu().numpy() for t in self.tensors]
        return self._host

    def __call__(self, *args):
        if len(args) == 2:
            b, h, q, kv = 0, 0, args[0], args[1]
        else:
            b, h, q, kv = args
        env = {"b": np.asarray(b), "h": np.asarray(h), "q": np.asarray(q), "kv": np.asarray(kv)}
        out = evaluate(self.expr, env, self.host_tensors())
        return np.broadcast_to(np.asarray(out, dtype=bool), np.broadcast(env["q"], env["kv"]).shape)

    @property
    def is_trivial(self) -> bool:
        return self.expr.op == "const" and self.expr.value is True


def lower_mask(fn) -> LoweredMask:
    return fn if isinstance(fn, LoweredMask) else LoweredMask(fn)


class LoweredScore:
    """A traced score mod ``(score, b, h, q_idx, kv_idx) -> score``."""

    def __init__(self, fn: Callable):
        self.fn = fn
        self.expr, self.tensors = trace_score(fn)
        self.dexpr = derivative(self.expr)
        self._host = None

    def host_tensors(self):
        if self._host is None:
            self._host = [t.detach().cpu().numpy() for t in self.tensors]
        return self._host

    def __call__(self, score, b, h, q, kv):
        env = {"score": np.asarray(score, np.float32), "b": np.asarray(b), "h": np.asarray(h),
               "q": np.asarray(q), "kv": np.asarray(kv)}
        return evaluate(self.expr, env, self.host_tensors())

    def grad(self, score, b, h, q, kv):
        env = {"score": np.asarray(score, np.float32), "b": np.asarray(b), "h": np.asarray(h),
               "q": np.asarray(q), "kv": np.asarray(kv)}
        return evaluate(self.dexpr, env, self.host_tensors())


def lower_score(fn) -> LoweredScore:
    return fn if isinstance(fn, LoweredScore) else LoweredScore(fn)


class UserMods:
    """The element policy of one call: a lowered mask and / or score mod, the
    tensors they read (slots 0..7, mask's first) and the policy source."""

    def __init__(self, mask: Optional[LoweredMask], score: Optional[LoweredScore]):
        self.mask, self.score = mask, score
        tensors: List = []

        def remap(e: Expr, own: list) -> Expr:
            if e.op == "gather":
                t = own[e.value[0]]
                for i, u in enumerate(tensors):
                    if u is t:
                        slot = i
                        break
                else:
                    tensors.append(t)
                    slot = len(tensors) - 1
                return Expr("gather", [remap(x, own) for x in e.args], e.dtype, (slot, e.value[1]))
            if not e.args:
                return e
            return Expr(e.op, [remap(x, own) for x in e.args], e.dtype, e.value)

        me = remap(mask.expr, mask.tensors) if mask is not None else None
        se = remap(score.expr, score.tensors) if score is not None else None
        if len(tensors) > 8:
            raise LoweringError("at most 8 captured tensors per call")
        self.tensors = tensors
        self.source = policy_source(me, se)
        self.digest = hashlib.sha256(self.source.encode()).hexdigest()
        self._device = {}

    def flags(self, builtin_score: bool) -> int:
        f = 0
        if self.mask is not None:
            f |= 1
        if self.score is not None:
            f |= 2
        if builtin_score and self.score is None:
            f |= 4
        return f

    def device_buffers(self, device):
        """Device copies (float32 / int32, contiguous) of the captured tensors, cached per device."""
        import torch
        key = str(device)
        bufs = self._device.get(key)
        if bufs is None:
            bufs = []
            for t in self.tensors:
                dt = torch.float32 if t.is_floating_point() else torch.int32
                bufs.append(t.detach().to(device=device, dtype=dt).contiguous())
            self._device[key] = bufs
        return bufs

    def key(self):
        return ("UserMods", self.digest, tuple(id(t) for t in self.tensors))
