"""Shared helpers of the GPU parity tests: oracle evaluation per row (in a
thread pool: ctypes releases the GIL) and tolerance checks."""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

import yskn_oracle as O

# logprob / NLL tolerance: 1e-5 relative, with an absolute floor of 1e-10,
# above the reference's own worst-case rounding of its serial binary64 sum
# over V = 248,320 terms (V * 2^-53 ~ 2.8e-11).
LP_REL, LP_ABS = 1e-5, 1e-10

_POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))


def pmap(fn, items):
    return list(_POOL.map(fn, items))


def oracle_params(sp, extension=False):
    """Oracle params from a yskn_smp.SamplingParameters (thousandths)."""
    return O.params_from_thousandths(sp.temperature_milli, sp.top_p_milli, sp.min_p_milli,
                                     top_k=sp.top_k, seed=sp.seed, version=sp.version,
                                     extension=extension)


def oracle_select(row: np.ndarray, pos: int, sp, extension=False) -> int:
    if sp.temperature_milli == 0:
        return O.greedy(row)
    return O.sample(row, pos, oracle_params(sp, extension))


def assert_logprobs_close(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    lim = LP_REL * np.abs(ref) + LP_ABS
    bad = np.nonzero(err > lim)
    assert bad[0].size == 0, (got[bad][:5], ref[bad][:5])


def to_u32(t) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.int64).astype(np.uint32)


def is_finite(x: float) -> bool:
    return math.isfinite(x)
