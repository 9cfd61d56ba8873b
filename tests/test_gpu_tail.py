"""The truncation tail on many candidates: the block-parallel, exact form of
the reference's serial binary64 sums (output_head_sampler.rs:157-207).

The device scan (test hook fn 8) must return every prefix sum bit for bit
as a plain left-to-right binary64 loop does, on sequences built to hit its
hard cases: weights that tie exactly halfway between two units of the
running sum's binade, sums that land on or next to a binade boundary,
weights absorbed whole, zeros, and runs that cross many binades. Then the
sampler itself, through the compact and the dense path, against the oracle
on rows whose kept set is thousands of candidates, for both draw versions.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import oracle_select, pmap, to_u32
from yskn_smp import DeviceSampler, SamplingParameters, pm_test

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _serial(w):
    out = np.empty(len(w))
    s = 0.0
    for j, x in enumerate(w.tolist()):
        s = s + x
        out[j] = s
    return out


def _hard_weights(n, seed):
    """w[0] = 1, then weights in [0, 1] chosen against the running sum."""
    rng = np.random.default_rng(seed)
    kinds = rng.integers(0, 8, n)
    r1 = rng.random(n)
    r2 = rng.integers(0, 1 << 62, n, dtype=np.int64)
    w = np.empty(n)
    w[0] = 1.0
    s = 1.0
    for j in range(1, n):
        e = math.frexp(s)[1] - 1                 # s in [2^e, 2^(e+1))
        u = math.ldexp(1.0, e - 52)
        k = kinds[j]
        if k == 0:                               # a tie: (2q + 1) u / 2 <= 1
            qmax = int(min(1.0 / u, 2.0 ** 52))
            q = int(r2[j]) % max(qmax // 2, 1)
            x = (2 * q + 1) * u / 2
        elif k == 1:
            x = float(r1[j])
        elif k == 2:
            x = 0.0
        elif k == 3:
            x = math.ldexp(1.0, -int(r2[j] % 60))
        elif k == 4:                             # land on the next binade edge, or just short of it
            gap = math.ldexp(1.0, e + 1) - s
            x = gap - (u / 2 if r1[j] < 0.5 else 0.0) if gap <= 1.0 else float(r1[j])
        elif k == 5:                             # half a unit: a tie at q = 0, or absorbed
            x = u / 2 if r1[j] < 0.5 else u / 4
        elif k == 6:
            x = 1.0
        else:                                    # one bit above a tie
            x = (3 * u / 2) + u * 2.0 ** -40 if 3 * u / 2 <= 1 else float(r1[j])
        x = min(max(x, 0.0), 1.0)
        w[j] = x
        s = s + x
    return w


@pytest.mark.parametrize("n,seed", [(1, 1), (2, 2), (3, 3), (4095, 4), (4096, 5), (4097, 6),
                                    (8193, 7), (50_000, 8), (200_000, 9)])
def test_exact_prefix_matches_the_serial_sum(n, seed):
    w = _hard_weights(n, seed)
    got = pm_test(8, w).view(np.float64)
    ref = _serial(w)
    bad = np.nonzero(got.view(np.uint64) != ref.view(np.uint64))[0]
    assert bad.size == 0, (int(bad[0]), got[bad[0]], ref[bad[0]])


def test_exact_prefix_on_sampler_weights():
    # sorted exp(z) weights of a flat row: the common shape, many binades
    rng = np.random.default_rng(11)
    z = np.sort(-np.abs(rng.standard_normal(300_000)) * 2.0)[::-1]
    z[0] = 0.0
    w = np.exp(z)
    w[0] = 1.0
    got = pm_test(8, w).view(np.float64)
    assert np.array_equal(got.view(np.uint64), _serial(w).view(np.uint64))
    ones = np.ones(150_000)                      # 17 binade crossings, each inside a tile
    assert np.array_equal(pm_test(8, ones).view(np.float64), np.arange(1, 150_001, dtype=np.float64))


@pytest.mark.parametrize("version", [2, 3])
@pytest.mark.parametrize("dense", [False, True])
def test_large_kept_sets_match_the_oracle(version, dense):
    # flat rows: the top-p set holds thousands (to all) of the candidates
    V, rows = 60_000, 6
    rng = np.random.default_rng(40 + version)
    scale = np.array([[0.05], [0.3], [1.0], [0.02], [0.5], [2.0]])
    x = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
    x[3, ::7] = 0.0                              # many equal values
    d = DeviceSampler(rows, V, extended_top_k=True, force_dense=dense)
    sps = [SamplingParameters(temperature_milli=t, top_p_milli=p, top_k=k, min_p_milli=m, seed=5 + i,
                              version=version)
           for i, (t, p, k, m) in enumerate([(1000, 950, 0, 0), (1500, 999, 0, 0), (700, 900, 5000, 0),
                                             (1000, 1000, 0, 0), (1200, 800, 0, 1), (300, 950, 0, 0)])]
    d.set_params(sps)
    pos = torch.tensor([[3 + r, 1000 + r, 2**40 + r] for r in range(rows)], dtype=torch.int64, device=DEV)
    out = d.sample(torch.from_numpy(x).to(DEV), pos)
    d.sync()
    got = to_u32(out["ids"])
    for r in range(rows):
        for q in range(3):
            want = oracle_select(x[r], int(pos[r, q]), sps[r], extension=True)
            assert got[r, q] == want, (r, q)
    d.close()
