"""Pins the oracle's f16 conversions and fixture generator (CPU only).

f16: IEEE binary16 round-to-nearest-even, which the reference gets from the
`half` 2.7.1 crate (hier.rs, decode.rs; pinned in the reference only against
`half` itself, cpu.rs:197-218). numpy's float16 implements the same IEEE
rounding, so it is an independent implementation to compare against.
"""
import numpy as np


def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.f16_value(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_round_trip_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    back = orc.f16_bits(vals)
    keep = ~np.isnan(vals)
    assert np.array_equal(back[keep], bits[keep])
    assert np.all(np.isnan(orc.f16_value(back[~keep])))  # NaN stays NaN


def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(0)
    # every f32 exponent that lands in or near the f16 range, random mantissas,
    # plus the exact halfway points between adjacent f16 values
    u = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32)
    u = (u & np.uint32(0x807FFFFF)) | (rng.integers(96, 145, u.size).astype(np.uint32) << 23)
    x = u.view(np.float32)
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mid, -mid, np.float32([65504, 65519.99, 65520, 1e-8, 3e-8, np.inf,
                                                  -np.inf, 0.0, -0.0])])
    got = orc.f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_splitmix64_published_vectors(orc):
    """SplitMix64 (Steele, Lea, Flood 2014) from state 0: the first outputs of
    the reference generator are 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4."""
    g = 0x9E3779B97F4A7C15
    assert orc.lib().orc_splitmix64(0) == 0xE220A8397B1DCDAF
    assert orc.lib().orc_splitmix64(g) == 0x6E789E6AA1B965F4


def test_fixture_normal_is_integer_exact_with_unit_irwin_hall_variance(orc):
    std = 0.02
    unit = orc.fixture_normal(3, 7, 200_000, 1.0)
    n = unit.astype(np.float64) * 2**17  # 2 * the centred 16-bit sum
    assert np.array_equal(n, np.round(n))
    v = orc.fixture_normal(3, 7, 200_000, std)
    assert np.all(np.abs(n) <= 2 * 6 * 65536)
    z = v.astype(np.float64) / std
    assert abs(z.mean()) < 0.01
    assert abs(z.var() - 1.0) < 0.01
    assert abs(np.mean(z**4) - 2.9) < 0.05  # Irwin-Hall(12) kurtosis is 3 - 1/10
    # one rounding: std * (n * 2^-17)
    w = ((n * 2.0**-17).astype(np.float32) * np.float32(std)).astype(np.float32)
    assert np.array_equal(w, v)


def test_fixture_streams_and_offsets(orc):
    a = orc.fixture_normal(0, 5, 1000)
    b = orc.fixture_normal(0, 5, 500, index0=500)
    assert np.array_equal(a[500:], b)
    c = orc.fixture_normal(0, 6, 1000)
    d = orc.fixture_normal(1, 5, 1000)
    assert abs(np.corrcoef(a, c)[0, 1]) < 0.1 and abs(np.corrcoef(a, d)[0, 1]) < 0.1
