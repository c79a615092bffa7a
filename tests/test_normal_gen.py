"""The library's random-init generator (normal_gen.h on the device, orc_fill_normal in the oracle), pinned on the
CPU: the oracle's C restatement is checked bit for bit against a second restatement in numpy float32 (IEEE-rounded
+, −, ×, ÷ and sqrt, one operation at a time), and the math it spells out (ln by the atanh series, sin/cos by
Taylor series per octant) against float64 log/cos/sin over every one of the 2^24 values each uniform can take.
The device kernels are compared with orc_fill_normal bit for bit in test_normal_gen_gpu.py."""

import numpy as np

import oracle_lib as orc
from decide_amd import synth

F = np.float32
PHI = np.uint64(0x9E3779B97F4A7C15)


def _c(h: str) -> np.float32:
    return F(float.fromhex(h))


LN = [_c(h) for h in ("0x1.745d18p-4", "0x1.c71c72p-4", "0x1.24924ap-3", "0x1.99999ap-3", "0x1.555556p-2")]
SIN = [_c(h) for h in ("-0x1.e30750p-30", "0x1.507834p-22", "-0x1.32d2ccp-15", "0x1.466bc6p-9", "-0x1.4abbcep-4",
                       "0x1.921fb6p-1")]
COS = [_c(h) for h in ("0x1.f9d38ap-34", "-0x1.a6d1f2p-26", "0x1.e1f506p-19", "-0x1.55d3c8p-12", "0x1.03c1f0p-6",
                       "-0x1.3bd3ccp-2")]


def _bits(seed: int, j: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return (synth.mix64(np.uint64(seed) + PHI * j) >> np.uint64(40)).astype(np.uint32)


def _ln(u: np.ndarray) -> np.ndarray:
    bits = u.view(np.uint32)
    e = (bits >> np.uint32(23)).astype(np.int32) - 127
    m = ((bits & np.uint32(0x7FFFFF)) | np.uint32(0x3F800000)).view(F)
    big = m > _c("0x1.6a09e6p+0")
    m = np.where(big, m * F(0.5), m)
    e = e + big
    z = (m - F(1)) / (m + F(1))
    z2 = z * z
    p = np.full_like(z, LN[0])
    for c in LN[1:]:
        p = p * z2 + c
    p = p * z2 + F(1)
    return e.astype(F) * _c("0x1.62e430p-1") + (z + z) * p


def _sincos(t: np.ndarray):
    t2 = t * t
    ps = np.full_like(t, SIN[0])
    for c in SIN[1:]:
        ps = ps * t2 + c
    pc = np.full_like(t, COS[0])
    for c in COS[1:]:
        pc = pc * t2 + c
    return t * ps, pc * t2 + F(1)


def _trig(b: np.ndarray):
    """(cos θ, sin θ) for θ = 2π(b + ½)/2^24, folded per octant."""
    o = b >> np.uint32(21)
    t = ((b & np.uint32(0x1FFFFF)).astype(F) + F(0.5)) * F(2.0 ** -21)
    odd = (o & np.uint32(1)).astype(bool)
    sb, cb = _sincos(np.where(odd, F(1) - t, t))
    sb = np.where(odd, -sb, sb)
    k = ((o + np.uint32(1)) >> np.uint32(1)) & np.uint32(3)
    cth = np.select([k == 0, k == 1, k == 2], [cb, -sb, -cb], sb)
    sth = np.select([k == 0, k == 1, k == 2], [sb, cb, -sb], -cb)
    return cth, sth


def _normal_np(seed: int, i: np.ndarray, mean: float, sd: float) -> np.ndarray:
    i = i.astype(np.uint64)
    p = i >> np.uint64(1)
    a = _bits(seed, np.uint64(2) * p + np.uint64(1))
    b = _bits(seed, np.uint64(2) * p + np.uint64(2))
    r = np.sqrt(F(-2) * _ln((a.astype(F) + F(0.5)) * F(2.0 ** -24)))
    cth, sth = _trig(b)
    z = r * np.where((i & np.uint64(1)) == 1, sth, cth)
    return z * F(sd) + F(mean)


def test_oracle_generator_matches_a_numpy_restatement_bitwise():
    n = 1 << 20
    for seed, mean, sd in ((0xDEC1DE, 0.0, 1.0), (12345, 0.5, 0.5), (2**64 - 7, 1.0, 0.02), (0, 0.0, 0.3)):
        want = _normal_np(seed, np.arange(n), mean, sd)
        got = orc.fill_normal(n, seed, mean, sd, 2)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"seed {seed}")
        # fp16 / bf16 outputs are the fp32 values rounded to nearest even
        np.testing.assert_array_equal(orc.fill_normal(n, seed, mean, sd, 0).view(np.uint16),
                                      want.astype(np.float16).view(np.uint16))
        np.testing.assert_array_equal(orc.fill_normal(n, seed, mean, sd, 1), synth.bf16_bits(want))


def test_single_elements_match_the_stream():
    seed = 0xABCDEF
    stream = orc.fill_normal(4096, seed, 0.25, 2.0, 2)
    lib = orc.load()
    for i in (0, 1, 2, 3, 777, 4094, 4095):
        assert np.float32(lib.orc_normal_at(seed, i, 0.25, 2.0)) == stream[i]


def test_ln_over_every_uniform():
    """The atanh-series log against float64 log for all 2^24 values of u1 = (a + ½)·2^-24."""
    a = np.arange(1 << 24, dtype=np.uint32)
    u = (a.astype(F) + F(0.5)) * F(2.0 ** -24)
    got = _ln(u).astype(np.float64)
    want = np.log(u.astype(np.float64))
    err = np.abs(got - want)
    assert (err <= 4e-7 * np.maximum(np.abs(want), 1e-3)).all(), float((err / np.abs(want).clip(1e-3)).max())
    assert got[-1] == 0.0  # u1 rounds to 1 at the top of the range: radius 0, no NaN


def test_sincos_over_every_uniform():
    """The octant-folded Taylor sin/cos against float64 cos/sin for all 2^24 values of θ = 2π(b + ½)/2^24."""
    b = np.arange(1 << 24, dtype=np.uint32)
    cth, sth = _trig(b)
    th = 2 * np.pi * (b.astype(np.float64) + 0.5) / 2.0 ** 24
    assert np.abs(cth - np.cos(th)).max() <= 2.4e-7
    assert np.abs(sth - np.sin(th)).max() <= 2.4e-7
    assert np.abs(cth.astype(np.float64) ** 2 + sth.astype(np.float64) ** 2 - 1).max() <= 6e-7


def test_close_to_float64_box_muller_and_gaussian():
    """Within fp32 rounding of float64 Box–Muller on the same uniforms (u1 as the generator rounds it to fp32:
    (a + ½) needs 25 bits when a >= 2^23), near synth's float64 stream, and N(0, 1) by its moments."""
    n = 1 << 22
    seed = 0x5EED
    got = orc.fill_normal(n, seed, 0.0, 1.0, 2).astype(np.float64)
    i = np.arange(n, dtype=np.uint64)
    p = i >> np.uint64(1)
    a = _bits(seed, np.uint64(2) * p + np.uint64(1))
    b = _bits(seed, np.uint64(2) * p + np.uint64(2))
    u1 = ((a.astype(F) + F(0.5)) * F(2.0 ** -24)).astype(np.float64)
    th = 2 * np.pi * (b.astype(np.float64) + 0.5) / 2.0 ** 24
    r = np.sqrt(-2 * np.log(u1))
    want = np.where((i & np.uint64(1)) == 1, r * np.sin(th), r * np.cos(th))
    assert np.abs(got - want).max() <= 2e-6
    assert np.abs(got - synth.normal(seed, n)).max() <= 1e-4  # synth keeps u1 in float64
    assert abs(got.mean()) < 5 / np.sqrt(n)
    assert abs(got.var() - 1) < 5 * np.sqrt(2 / n)
    assert abs((got ** 4).mean() - 3) < 0.02
    assert np.abs(got).max() < 6.0  # r = sqrt(-2 ln u1) <= sqrt(2·ln(2^25)) ≈ 5.9
