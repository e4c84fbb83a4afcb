"""The oracle's page write rule (oracle_write_pages / oracle_e4m3_encode), the
checker of dh_pool_write_pages_device, pinned without the library:

- E4M3 encoding against torch's float32 -> float8_e4m3fn cast (round to
  nearest even) on every bfloat16 value within +-448 and on every midpoint
  between adjacent codes (the ties), and against a brute-force nearest search
  over all 256 codes on random floats;
- saturation beyond 448 and the signed zero;
- bf16 / f16 conversion against torch's casts;
- the FP8 block scale (amax / 448, 1 for a zero block) and the MXFP8 group
  scale (amax / 2^e in [256, 512)) from their definitions, with the decoded
  values within half a code step of the inputs (MX values scaled above 448
  saturate, as OCP MX v1.0 specifies).
A planted mistake (a truncating encoder, a max taken over one plane only, an
MX exponent off by one) fails one of these.
"""
import numpy as np
import pytest
import torch

import oracle


def _enc(xs):
    return np.array([oracle.e4m3_encode(float(x)) for x in xs], dtype=np.uint8)


def _torch_e4m3(xs):
    return torch.tensor(np.asarray(xs, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _dec(codes):
    return np.array([oracle.e4m3_to_float(int(c)) for c in codes])


def test_e4m3_encode_matches_torch_on_bf16_values():
    bits = np.arange(0, 1 << 16, dtype=np.uint32) << 16
    xs = bits.view(np.float32)
    xs = xs[np.isfinite(xs) & (np.abs(xs) <= 448.0)]
    xs = xs[:: 3]   # every third pattern: ~21k values across all binades, both signs
    assert np.array_equal(_enc(xs), _torch_e4m3(xs))


def test_e4m3_ties_go_to_the_even_code():
    vals = _dec(range(0, 0x7F))
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    got = _enc(mids)
    assert np.array_equal(got, _torch_e4m3(mids))
    assert np.all(got % 2 == 0), "a midpoint rounded to an odd code"
    neg = _enc(-mids)
    assert np.array_equal(neg, got | 0x80)


def test_e4m3_encode_is_the_nearest_code():
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(2000) * 50, rng.uniform(-2e-3, 2e-3, 500)]).astype(np.float32)
    table = _dec(range(0, 0x7F))
    table = np.concatenate([table, -table])
    codes = _enc(xs)
    err = np.abs(_dec(codes) - xs.astype(np.float64))
    best = np.min(np.abs(table[None, :] - xs[:, None].astype(np.float64)), axis=1)
    assert np.array_equal(err, best)


def test_e4m3_saturates_and_keeps_the_sign_of_zero():
    assert list(_enc([448.0, 449.0, 464.0, 1e30])) == [0x7E] * 4
    assert list(_enc([-448.0, -1e30])) == [0xFE] * 2
    assert list(_enc([0.0, -0.0])) == [0x00, 0x80]


def _pages(rng, n, hkv, d, outliers=False):
    x = rng.standard_normal((n, 2, hkv, 16, d)).astype(np.float32)
    if outliers:
        m = rng.random(x.shape) < 0.01
        x[m] = np.where(x[m] < 0, -20.0, 20.0)
    return x


@pytest.mark.parametrize("fmt", [oracle.BF16, oracle.F16, oracle.F32])
def test_sixteen_and_thirty_two_bit_pages_are_the_torch_casts(fmt):
    rng = np.random.default_rng(4)
    x = _pages(rng, 3, 2, 64) * 1000
    data, scales = oracle.write_pages(fmt, 2, 64, x)
    assert scales is None
    want = {oracle.BF16: torch.bfloat16, oracle.F16: torch.float16, oracle.F32: torch.float32}[fmt]
    t = torch.from_numpy(x.reshape(3, -1)).to(want)
    ref = t.view(torch.int16 if fmt != oracle.F32 else torch.int32).numpy().view(np.uint8)
    assert np.array_equal(data, ref.reshape(3, -1))


def test_fp8_block_scale_is_amax_over_448():
    rng = np.random.default_rng(5)
    hkv, d = 2, 128
    x = _pages(rng, 2, hkv, d, outliers=True)
    x[1, 1, 0] = 0.0                                   # an all-zero (plane, head) block
    data, scales = oracle.write_pages(oracle.FP8, hkv, d, x)
    sc = scales.view(np.float32).reshape(2, 2, hkv)
    amax = np.abs(x).max(axis=(3, 4))
    want = np.where(amax > 0, (amax / np.float32(448.0)).astype(np.float32), np.float32(1.0))
    assert np.array_equal(sc, want)
    codes = data.reshape(x.shape)
    deq = _dec(codes.reshape(-1)).reshape(x.shape) * sc[..., None, None]
    # within half a code step: 2^-4 relative, 2^-10 * scale absolute (subnormals)
    tol = np.maximum(np.abs(x) * 2.0 ** -4, 2.0 ** -10 * sc[..., None, None]) * (1 + 1e-6)
    assert np.all(np.abs(deq - x) <= tol)
    assert np.all(codes[1, 1, 0] == 0)
    # the block's largest magnitude maps to +-448
    flat = np.abs(x).reshape(2, 2, hkv, -1)
    idx = flat.argmax(axis=-1)
    top = np.take_along_axis(codes.reshape(2, 2, hkv, -1), idx[..., None], axis=-1)[..., 0]
    assert np.all(((top & 0x7F) == 0x7E) | (amax == 0))


@pytest.mark.parametrize("d", [64, 128])
def test_mx_group_scale_is_the_power_of_two_below_amax_over_256(d):
    rng = np.random.default_rng(6)
    hkv = 2
    x = _pages(rng, 2, hkv, d, outliers=True)
    x[0, 0, 0, 3, :32] = 0.0                           # an all-zero group
    data, scales = oracle.write_pages(oracle.MX, hkv, d, x)
    se = scales.reshape(2, 2, hkv, 16, d // 32).astype(np.int64) - 127
    g = x.reshape(2, 2, hkv, 16, d // 32, 32)
    amax = np.abs(g).max(axis=-1)
    nz = amax > 0
    ratio = amax[nz] / np.ldexp(1.0, se[nz])
    assert np.all((ratio >= 256) & (ratio < 512))
    assert np.all(se[~nz] == -127)
    deq = _dec(data.reshape(-1)).reshape(g.shape) * np.ldexp(1.0, se)[..., None]
    # OCP MX: scaled values reach [256, 512); those above 448 saturate
    sat = np.abs(g) > 448.0 * np.ldexp(1.0, se)[..., None]
    assert np.all(np.abs(deq[sat]) == (448.0 * np.ldexp(1.0, se)[..., None] * np.ones_like(g))[sat])
    assert np.all(np.sign(deq[sat]) == np.sign(g[sat]))
    tol = np.maximum(np.abs(g) * 2.0 ** -4, np.ldexp(2.0 ** -10, se)[..., None]) * (1 + 1e-6)
    assert np.all((np.abs(deq - g) <= tol) | sat)
    assert sat.any(), "no group reached the saturating range"
