"""Pins the oracle's binary64 exp_d / log_d and the SplitMix64 mixer.

* bit vectors held by the reference's own tests
  (crates/yskn-ref/src/portable_math.rs:487-587);
* the mathematics: every branch of the fdlibm method against the platform
  libm (correctly rounded or within 1 ulp), monotonicity, and identities;
* SplitMix64's published output sequence for seed 0.
"""
import math
import struct

import numpy as np
import pytest

import yskn_oracle as O


def bits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def from_bits(b: int) -> float:
    return struct.unpack("<d", struct.pack("<Q", b))[0]


def ulp_diff(a: float, b: float) -> int:
    ia, ib = bits(a), bits(b)
    # map to a monotone integer line
    ia = ia if ia < (1 << 63) else (1 << 63) - ia
    ib = ib if ib < (1 << 63) else (1 << 63) - ib
    return abs(ia - ib)


# portable_math.rs:563-581 -- exp_d / log_d bit vectors at 0.5, 1, 10
@pytest.mark.parametrize("x,e_bits,l_bits", [
    (0.5, 0x3FFA61298E1E069C, 0xBFE62E42FEFA39EF),
    (1.0, 0x4005BF0A8B14576A, 0x0),
    (10.0, 0x40D5829DCF950560, 0x40026BB1BBB55516),
])
def test_reference_bit_vectors(x, e_bits, l_bits):
    assert bits(O.exp_d(x)) == e_bits
    assert bits(O.log_d(x)) == l_bits


def test_reference_zero_endpoint_artifacts():
    # portable_math.rs:583-587
    assert bits(O.log_d(0.0)) == 0xC0875427F6ACAD6F
    assert bits(O.log_d(-0.0)) == 0xC0A0EC2B7D284853


def test_reference_identities_and_limits():
    # portable_math.rs:487-510
    assert bits(O.exp_d(0.0)) == bits(1.0)
    assert bits(O.log_d(1.0)) == bits(0.0)
    assert bits(O.exp_d(-746.0)) == 0
    assert O.exp_d(710.0) == math.inf
    assert O.exp_d(-math.inf) == 0.0
    assert O.exp_d(math.inf) == math.inf
    assert math.isnan(O.exp_d(math.nan))


def _exp_inputs():
    rng = np.random.default_rng(1234)
    xs = []
    xs += list(rng.uniform(-1e-9, 1e-9, 200))           # |x| < 2^-28: 1 + x
    xs += list(rng.uniform(-0.34, 0.34, 500))            # k = 0 branch
    xs += list(rng.uniform(0.35, 1.03, 300))             # k = +-1 branch
    xs += list(-rng.uniform(0.35, 1.03, 300))
    xs += list(rng.uniform(-40.0, 40.0, 2000))           # general reduction
    xs += list(rng.uniform(-745.0, 709.7, 1000))
    xs += list(rng.uniform(-745.1, -708.0, 300))         # subnormal results
    return xs


def test_exp_d_against_libm_every_branch():
    worst = 0
    for x in _exp_inputs():
        got, ref = O.exp_d(x), math.exp(x)
        if ref == 0.0:
            assert got == 0.0
            continue
        if ref < 2.2250738585072014e-308:
            # subnormal: both round to the same grid within one unit
            assert abs(got - ref) <= 5e-324 * 1.0001, x
            continue
        worst = max(worst, ulp_diff(got, ref))
    assert worst <= 1


def test_log_d_against_libm_every_branch():
    rng = np.random.default_rng(99)
    xs = list(rng.uniform(0.70, 1.42, 1000))          # k = 0
    xs += list(rng.uniform(1e-300, 1e300, 500))
    xs += list(10.0 ** rng.uniform(-300, 300, 2000))
    xs += [5e-324, 1e-310, 2.2250738585072014e-308]    # subnormal inputs
    xs += [1.0 + 2.0 ** -30, 1.0 - 2.0 ** -30, 2.0, 0.5, 4.0]
    xs += list(2.0 ** rng.integers(-1000, 1000, 200).astype(float))  # f == 0 branch
    worst = 0
    for x in xs:
        worst = max(worst, ulp_diff(O.log_d(x), math.log(x)))
    assert worst <= 1


def test_exp_log_monotone_on_adjacent_doubles():
    rng = np.random.default_rng(7)
    for x in rng.uniform(-40, 0, 400):
        y = np.nextafter(x, 1.0)
        assert O.exp_d(x) <= O.exp_d(y)
    for x in 10.0 ** rng.uniform(-20, 20, 400):
        y = np.nextafter(x, np.inf)
        assert O.log_d(x) <= O.log_d(y)


def test_splitmix64_published_sequence():
    # SplitMix64 with state 0: outputs of state += gamma, mix.
    gamma = 0x9E3779B97F4A7C15
    expected = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for i, e in enumerate(expected):
        assert O.mix64((i * gamma) & ((1 << 64) - 1)) == e


def test_gumbel_closed_form():
    # spec 06 section 6: h from three mixes, u = ((h >> 11) + 0.5) 2^-53,
    # g = -log(-log u); compared with libm logs (agree to a few ulps)
    M = (1 << 64) - 1
    rng = np.random.default_rng(5)
    for _ in range(300):
        seed, pos, tok = (int(rng.integers(0, 2**63)), int(rng.integers(0, 2**40)),
                          int(rng.integers(0, 2**32)))
        a = O.mix64(seed)
        b = O.mix64(a ^ pos)
        h = O.mix64(b ^ ((tok * 0xD6E8FEB86659FD93) & M))
        u = ((h >> 11) + 0.5) * 2.0 ** -53
        g = -math.log(-math.log(u))
        assert O.gumbel(seed, pos, tok) == pytest.approx(g, rel=1e-13, abs=1e-13)


def test_gumbel_upper_endpoint_is_finite():
    # spec 06 SMP-03: if h >> 11 == 2^53 - 1 then u rounds to 1.0 and the
    # log_d(-0) artefact keeps the draw finite. Direct check on the formula:
    u = ((2 ** 53 - 1) + 0.5) * 2.0 ** -53
    assert u == 1.0
    g = -O.log_d(-O.log_d(u))
    assert math.isfinite(g) and g > 2000.0
