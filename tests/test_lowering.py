"""Lowering of user mask / score callables (CPU): the traced expression
evaluates like the callable itself, Python's integer semantics survive,
derivatives with respect to the score match finite differences, untraceable
callables are refused with a reason, and the generated policy compiles for
gfx950 through the C ABI (fa_mods_compile needs no GPU)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import pallas_flexattn as pf  # noqa: E402
from pallas_flexattn import lowering as L  # noqa: E402

Q = np.arange(-5, 40)[:, None]
K = np.arange(0, 37)[None, :]

MASKS = {
    "prefix_lm": lambda q, kv: (kv < 8) | (q >= kv),
    "parity": lambda q, kv: (q - kv) % 2 == 0,
    "floordiv_blocks": lambda q, kv: (q // 16) == (kv // 16),
    "where_window": lambda q, kv: torch.where(q > 20, (q - kv) < 4, kv <= q),
    "not_and": lambda q, kv: ~(kv > q) & (torch.abs(q - kv) <= 9),
    "numpy_ops": lambda q, kv: np.logical_and(q >= kv, np.remainder(q + kv, 3) != 1),
}


@pytest.mark.parametrize("name", list(MASKS))
def test_traced_mask_evaluates_like_the_callable(name):
    fn = MASKS[name]
    low = L.lower_mask(fn)
    want = fn(torch.from_numpy(Q), torch.from_numpy(K)) if name != "numpy_ops" else fn(Q, K)
    want = np.broadcast_to(np.asarray(want), (Q.shape[0], K.shape[1]))
    np.testing.assert_array_equal(low(Q, K), want)


def test_integer_semantics_follow_python():
    # floor division and modulo take the divisor's sign, as in Python / torch
    low = L.lower_mask(lambda q, kv: ((q - kv) // 7 == -2) | ((q - kv) % -5 == -3))
    d = Q - K
    np.testing.assert_array_equal(low(Q, K), ((d // 7) == -2) | ((d % -5) == -3))
    src = L.policy_source(low.expr, None)
    assert "um_ifloordiv" in src and "um_imod" in src
    # the smallest int32 stays an int literal in C++ (a bare -2147483648 is
    # the negation of a long)
    assert L.emit(L.const(-2 ** 31)) == "(-2147483647 - 1)"
    low = L.lower_mask(lambda q, kv: (q - kv) > -2 ** 31)
    np.testing.assert_array_equal(low(Q, K), np.broadcast_to(True, (Q.shape[0], K.shape[1])))


def test_captured_tensor_reads_and_batch_head_dependence():
    allowed = torch.rand(2, 3, 45, 37) > 0.5
    low = L.lower_mask(lambda b, h, q, kv: allowed[b, h, q, kv] | (q == kv))
    assert low.batch_dependent and low.head_dependent and len(low.tensors) == 1
    for b in range(2):
        for h in range(3):
            got = low(b, h, np.arange(45)[:, None], np.arange(37)[None, :])
            want = allowed[b, h].numpy() | (np.arange(45)[:, None] == np.arange(37)[None, :])
            np.testing.assert_array_equal(got, want)
    # reads are clamped into the tensor (no out-of-bounds access)
    np.testing.assert_array_equal(low(0, 0, np.array([[100]]), np.array([[-3]])),
                                  allowed[0, 0, 44, 0].numpy() | False)


SCORES = {
    "softcap": (lambda s, b, h, q, kv: 20.0 * torch.tanh(s / 20.0)),
    "alibi_like": (lambda s, b, h, q, kv: s - 0.25 * (h + 1) * torch.abs(q - kv)),
    "quadratic_exp": (lambda s, b, h, q, kv: 0.1 * s * s + torch.exp(s / 8.0) + (q % 3)),
    "clamp_where": (lambda s, b, h, q, kv: torch.where(s > 2.0, 2.0 + 0.5 * (s - 2.0), torch.clamp(s, min=-3.0))),
    "sigmoid_log": (lambda s, b, h, q, kv: torch.log(torch.sigmoid(s) + 1.0) + torch.sqrt(s * s + 1.0)),
}


@pytest.mark.parametrize("name", list(SCORES))
def test_score_derivative_matches_finite_differences(name):
    fn = SCORES[name]
    low = L.lower_score(fn)
    rng = np.random.default_rng(1)
    s = rng.standard_normal((45, 37)).astype(np.float64) * 4
    h = 2
    val = low(s.astype(np.float32), 0, h, Q, K)
    want = fn(torch.from_numpy(s), 0, h, torch.from_numpy(Q), torch.from_numpy(K)).numpy()
    np.testing.assert_allclose(val, want, rtol=2e-5, atol=2e-5)
    eps = 1e-3
    fd = (fn(torch.from_numpy(s + eps), 0, h, torch.from_numpy(Q), torch.from_numpy(K)).numpy()
          - fn(torch.from_numpy(s - eps), 0, h, torch.from_numpy(Q), torch.from_numpy(K)).numpy()) / (2 * eps)
    g = low.grad(s.astype(np.float32), 0, h, Q, K)
    near_kink = np.abs(s - 2.0) < 2 * eps if name == "clamp_where" else np.zeros_like(s, bool)
    near_kink |= np.abs(s + 3.0) < 2 * eps if name == "clamp_where" else False
    np.testing.assert_allclose(np.where(near_kink, fd, g), fd, rtol=1e-3, atol=1e-3)


def test_descriptors_trace_to_their_own_predicates():
    """MaskSpec / ScoreSpec inside a traced callable lower to the same values."""
    dm = pf.document_mask([[10, 20, 15], [30, 15]])
    both = L.lower_mask(lambda b, h, q, kv: dm(b, h, q, kv) & pf.causal_mask(q, kv) &
                        pf.sliding_window_mask(12, -1)(q, kv))
    q, k = np.arange(45)[:, None], np.arange(45)[None, :]
    for b in range(2):
        want = dm(b, 0, q, k) & (q >= k) & (q - k <= 12)
        np.testing.assert_array_equal(both(b, 0, q, k), want)
    sc = pf.compose_score_mods(pf.alibi_score_mod(4), pf.softcap_score_mod(30.0))
    low = L.lower_score(lambda s, b, h, qi, ki: sc(s, b, h, qi, ki))
    s = np.random.default_rng(2).standard_normal((45, 45)).astype(np.float32) * 20
    for h in range(4):
        np.testing.assert_allclose(low(s, 0, h, q, k), sc(s, 0, h, q, k), rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("fn,why", [
    (lambda q, kv: q >= kv if q > 3 else q < kv, "control flow"),
    (lambda q, kv: [1, 2, 3][q] > 0, "concrete integer"),
    (lambda q, kv: np.arange(10)[q] > kv, "tracing the callable raised IndexError"),
    (lambda q, kv: torch.erf(q) > 0, "cannot be lowered"),
])
def test_untraceable_callables_are_refused(fn, why):
    with pytest.raises(L.LoweringError, match=why):
        L.lower_mask(fn)


def test_policy_compiles_for_gfx950_without_a_gpu():
    from pallas_flexattn import _lib
    bias = torch.randn(4, 8)
    mods = L.UserMods(L.lower_mask(MASKS["prefix_lm"]),
                      L.lower_score(lambda s, b, h, q, kv: 30.0 * torch.tanh((s + bias[h, kv % 8]) / 30.0)))
    assert len(mods.tensors) == 1 and mods.flags(False) == 3
    for dtype in (_lib.DTYPE_BF16, _lib.DTYPE_F32):
        blob = _lib.compile_mods(mods.source, dtype, 128, mods.flags(False))
        assert len(blob) > 1000
    with pytest.raises(_lib.FlexAttnError, match="compiling the user mods failed"):
        _lib.compile_mods("struct UserMod { this is not C++ };", _lib.DTYPE_BF16, 64, 1)


def test_policy_must_match_its_flags():
    """fa_mods_compile refuses a policy whose kMask / kScore disagree with the
    flags it is compiled under (the launches set up the mask walk and the
    score epilogue from the flags), and a user score together with the
    built-in ALiBi / soft-cap (which only run without a user score)."""
    from pallas_flexattn import _lib
    mods = L.UserMods(L.lower_mask(MASKS["parity"]), None)
    assert mods.flags(False) == _lib.MODS_MASK
    with pytest.raises(_lib.FlexAttnError, match="kMask disagrees"):
        _lib.compile_mods(mods.source, _lib.DTYPE_BF16, 64, 0)
    with pytest.raises(_lib.FlexAttnError, match="kScore disagrees"):
        _lib.compile_mods(mods.source, _lib.DTYPE_BF16, 64, _lib.MODS_MASK | _lib.MODS_SCORE)
    smods = L.UserMods(None, L.lower_score(lambda s, b, h, q, kv: s * 0.5))
    with pytest.raises(_lib.FlexAttnError, match="exit 3"):
        _lib.compile_mods(smods.source, _lib.DTYPE_BF16, 64, _lib.MODS_SCORE | _lib.MODS_BUILTIN_SCORE)


def test_blob_from_other_kernel_headers_is_refused():
    """A code blob records the ABI version, the hash of the kernel headers it
    was compiled from and the kernel argument sizes; fa_mods_load refuses a
    blob that differs in any of them (FA_ERR_VERSION) before any GPU call,
    so a stale cached or stored blob is never launched with another argument
    layout.  Header layout: magic u32, abi_version u32, header hash u64,
    sizeof(FwdArgs) u32, sizeof(BwdArgs) u32."""
    import ctypes
    from pallas_flexattn import _lib
    lib = _lib.load()
    mods = L.UserMods(L.lower_mask(MASKS["parity"]), None)
    blob = _lib.compile_mods(mods.source, _lib.DTYPE_BF16, 64, mods.flags(False))
    assert int.from_bytes(blob[4:8], "little") == _lib.ABI_VERSION
    assert int.from_bytes(blob[8:16], "little") == lib.fa_mods_source_hash()
    fwd_bytes, bwd_bytes = int.from_bytes(blob[16:20], "little"), int.from_bytes(blob[20:24], "little")
    assert 0 < fwd_bytes < 4096 and bwd_bytes > fwd_bytes - 512

    def load(b):
        h = ctypes.c_void_p()
        return lib.fa_mods_load(bytes(b), len(b), ctypes.byref(h))

    FA_ERR_SHAPE, FA_ERR_VERSION = -2, -8
    for lo, hi, delta in ((4, 8, 1), (8, 16, 1), (16, 20, 8), (20, 24, 8)):
        bad = bytearray(blob)
        bad[lo:hi] = ((int.from_bytes(blob[lo:hi], "little") + delta) % (1 << (8 * (hi - lo)))).to_bytes(
            hi - lo, "little")
        assert load(bad) == FA_ERR_VERSION, (lo, hi)
    bad = bytearray(blob)
    bad[0] ^= 1  # not a blob
    assert load(bad) == FA_ERR_SHAPE
    assert load(blob[:-1]) == FA_ERR_SHAPE  # truncated code object
    assert load(blob[:20]) == FA_ERR_SHAPE  # shorter than the header
