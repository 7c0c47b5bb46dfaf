"""The oracle's fp8 pieces (CPU): the e4m3 codec against torch's
float8_e4m3fn (an independent implementation) and closed forms, the block
quantisation against the invariants that define it, and the P-rounding model
against plain attention."""
import numpy as np
import pytest

from oracle import attention, fp8

torch = pytest.importorskip("torch")


def _torch_codes(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_all_codes_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = fp8.decode_e4m3(codes)
    want = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_closed_forms():
    assert fp8.decode_e4m3(0x7E) == 448.0 and fp8.decode_e4m3(0xFE) == -448.0
    assert fp8.decode_e4m3(0x08) == 2.0 ** -6 and fp8.decode_e4m3(0x01) == 2.0 ** -9
    assert fp8.decode_e4m3(0x38) == 1.0 and np.isnan(fp8.decode_e4m3(0x7F))
    assert fp8.encode_e4m3(448.0) == 0x7E and fp8.encode_e4m3(464.0) == 0x7E  # tie to even (448)
    assert fp8.encode_e4m3(464.5) == 0x7F and fp8.encode_e4m3(1.0625) == 0x38  # tie 1 | 1.125 -> 1
    assert fp8.encode_e4m3(1.1875) == 0x3A  # tie 1.125 | 1.25 -> 1.25 (even mantissa)
    assert fp8.encode_e4m3(2.0 ** -10) == 0x00 and fp8.encode_e4m3(1.5 * 2.0 ** -10) == 0x01


def test_encode_matches_torch_on_random_values_and_ties():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000) * 10.0, rng.standard_normal(5000) * 1e-3,
                        rng.uniform(-460, 460, 5000)]).astype(np.float32)
    # exact midpoints between neighbouring codes
    vals = fp8.decode_e4m3(np.arange(0x7E, dtype=np.uint8)).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    np.testing.assert_array_equal(fp8.encode_e4m3(x), _torch_codes(x))


def test_quantize_blocks_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 300, 64)).astype(np.float32)
    x[1] *= 1e-3
    x[2, 128:256] = 0.0
    x[2, :128] *= 1000.0
    codes, sc = fp8.quantize_blocks(x)
    assert sc.shape == (3, 3)
    e = np.log2(sc)
    np.testing.assert_array_equal(e, np.round(e))  # powers of two
    assert sc[2, 1] == 1.0  # all-zero block
    for h in range(3):
        for b in range(3):
            blk = x[h, 128 * b:128 * (b + 1)]
            amax = np.abs(blk).max()
            if amax == 0:
                continue
            assert amax <= 448 * sc[h, b] and amax > 448 * sc[h, b] / 2  # the smallest such power of two
    y = fp8.dequantize(codes, sc)
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 for normal values
    big = np.abs(x) > 2.0 ** -6 * np.repeat(sc, 128, axis=1)[:, :300, None]
    assert np.all(np.abs(y - x)[big] <= np.abs(x)[big] * 2.0 ** -4 * 1.0001)
    # transposed layout: V^T with the keys past S zero
    t, sc2 = fp8.quantize_blocks(x, transpose=True)
    assert t.shape == (3, 64, 384) and not t[:, :, 300:].any()
    np.testing.assert_array_equal(sc2, sc)
    np.testing.assert_array_equal(t[:, :, :300], codes.transpose(0, 2, 1))
    np.testing.assert_array_equal(fp8.dequantize(t, sc, transposed=True, seq_len=300), y)


def test_forward_model_reduces_to_attention():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((1, 2, 96, 64)) for _ in range(3))
    mask = np.tril(np.ones((96, 96), bool))
    o, lse = fp8.forward_model(q, k, v, mask, round_p=False)
    wo, wl = attention.forward(q, k, v, mask)
    np.testing.assert_allclose(o, wo, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, wl, rtol=1e-6, atol=1e-6)
    o8, lse8, bound = fp8.forward_model(q, k, v, mask, with_bound=True)
    np.testing.assert_array_equal(lse8, lse)  # the row sums use the unrounded P
    err = np.abs(o8 - wo)
    assert 1e-3 < err.max() < 0.1  # rounding P to 3 mantissa bits is visible
    assert np.all(err <= bound * (1 + 1e-6) + 1e-7)  # and within its worst case
    # the bound is not vacuous: within a small factor of the observed error on average
    assert np.mean(bound) < 20 * np.mean(err)
