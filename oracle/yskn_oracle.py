"""ctypes binding of the CPU oracle (oracle/yskn_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP sampler. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

OK, EINVAL, ENONFINITE = 0, -1, -2
GUMBEL, INVERSE_CDF = 3, 2


class Params(C.Structure):
    """yo_params: SamplingParameters (output_head_sampler.rs:21-41)."""

    _fields_ = [
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("top_k", C.c_uint64),
        ("min_p", C.c_double),
        ("seed", C.c_uint64),
        ("version", C.c_int),
        ("extension_top_k", C.c_int),
    ]


class Diag(C.Structure):
    _fields_ = [
        ("k", C.c_uint64),
        ("n_top_p", C.c_uint64),
        ("retained", C.c_uint64),
        ("pick", C.c_uint64),
        ("total", C.c_double),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        L.yo_exp_d.argtypes, L.yo_exp_d.restype = [C.c_double], C.c_double
        L.yo_log_d.argtypes, L.yo_log_d.restype = [C.c_double], C.c_double
        L.yo_mix64.argtypes, L.yo_mix64.restype = [C.c_uint64], C.c_uint64
        L.yo_gumbel.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.yo_gumbel.restype = C.c_double
        L.yo_uniform_v2.argtypes = [C.c_uint64, C.c_uint64]
        L.yo_uniform_v2.restype = C.c_double
        L.yo_default_params.argtypes = [C.POINTER(Params)]
        L.yo_params_from_thousandths.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32,
                                                 C.POINTER(Params)]
        L.yo_validate.argtypes = [C.POINTER(Params), C.c_uint64]
        L.yo_greedy.argtypes = [f32p, C.c_uint64, C.POINTER(C.c_uint32)]
        L.yo_top_tokens.argtypes = [f32p, C.c_uint64, C.c_uint64, u32p]
        L.yo_sample.argtypes = [f32p, C.c_uint64, C.c_uint64, C.POINTER(Params),
                                C.POINTER(C.c_uint32), C.POINTER(Diag)]
        L.yo_sample_positions.argtypes = [f32p, C.c_uint64, u64p, C.c_uint64,
                                          C.POINTER(Params), u32p]
        L.yo_nll.argtypes = [f32p, C.c_uint64, C.c_uint32, C.POINTER(C.c_double)]
        L.yo_mass.argtypes = [f32p, C.c_uint64, C.POINTER(C.c_double), C.POINTER(C.c_float)]
        L.yo_top_logprobs.argtypes = [f32p, C.c_uint64, C.c_uint64, u32p, f64p]
        L.yo_bf16_to_f32.argtypes = [u16p, f32p, C.c_uint64]
        L.yo_apply_penalties.argtypes = [f32p, C.c_uint64, u32p, C.c_uint64, C.c_float,
                                         C.c_float, C.c_float]
        L.yo_verify.argtypes = [f32p, C.c_uint64, C.c_uint64, C.c_uint64, u32p, C.c_uint64,
                                C.POINTER(Params), C.c_int, u32p, C.c_uint64, u32p,
                                C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_int)]
        L.yo_draft_choose.argtypes = [f32p, u32p, C.c_uint64, C.c_uint32, C.c_uint64,
                                      C.POINTER(C.c_uint32)]
        _lib = L
    return _lib


class OracleError(Exception):
    def __init__(self, status: int):
        super().__init__({EINVAL: "invalid input", ENONFINITE: "non-finite value"}.get(
            status, f"status {status}"))
        self.status = status


def _check(st: int) -> None:
    if st != OK:
        raise OracleError(st)


def params(temperature=1.0, top_p=0.95, top_k=20, min_p=0.0, seed=0, version=GUMBEL,
           extension=False) -> Params:
    return Params(temperature, top_p, top_k, min_p, seed, version, 1 if extension else 0)


def params_from_thousandths(t: int, tp: int, mp: int, top_k=20, seed=0, version=GUMBEL,
                            extension=False) -> Params:
    """SamplingParameters::from_thousandths (output_head_sampler.rs:43-54), then the
    product mapping's top_k / seed / version assignment (real_engine.rs:244-247)."""
    p = Params()
    lib().yo_default_params(C.byref(p))
    p.temperature = float(t) / 1000.0
    p.top_p = float(tp) / 1000.0
    p.min_p = float(mp) / 1000.0
    p.top_k, p.seed, p.version = top_k, seed, version
    p.extension_top_k = 1 if extension else 0
    return p


def exp_d(x: float) -> float:
    return lib().yo_exp_d(x)


def log_d(x: float) -> float:
    return lib().yo_log_d(x)


def mix64(x: int) -> int:
    return lib().yo_mix64(x)


def gumbel(seed: int, pos: int, tok: int) -> float:
    return lib().yo_gumbel(seed, pos, tok)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def greedy(logits) -> int:
    a = _f32(logits)
    out = C.c_uint32()
    _check(lib().yo_greedy(a, a.size, C.byref(out)))
    return out.value


def top_tokens(logits, count: int) -> np.ndarray:
    a = _f32(logits)
    out = np.zeros(count, np.uint32)
    _check(lib().yo_top_tokens(a, a.size, count, out))
    return out


def sample(logits, position: int, p: Params, diag: bool = False):
    a = _f32(logits)
    out = C.c_uint32()
    d = Diag()
    _check(lib().yo_sample(a, a.size, position, C.byref(p), C.byref(out), C.byref(d)))
    return (out.value, d) if diag else out.value


def sample_positions(logits, positions, p: Params) -> np.ndarray:
    a = _f32(logits)
    pos = np.ascontiguousarray(positions, dtype=np.uint64)
    out = np.zeros(pos.size, np.uint32)
    _check(lib().yo_sample_positions(a, a.size, pos, pos.size, C.byref(p), out))
    return out


def nll(logits, target: int) -> float:
    a = _f32(logits)
    out = C.c_double()
    _check(lib().yo_nll(a, a.size, target, C.byref(out)))
    return out.value


def top_logprobs(logits, n: int):
    a = _f32(logits)
    ids = np.zeros(n, np.uint32)
    lp = np.zeros(n, np.float64)
    _check(lib().yo_top_logprobs(a, a.size, n, ids, lp))
    return ids, lp


def bf16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.size, np.float32)
    lib().yo_bf16_to_f32(b, out, b.size)
    return out


def apply_penalties(logits, history, repetition: float, presence: float,
                    frequency: float) -> np.ndarray:
    a = _f32(logits).copy()
    h = np.ascontiguousarray(history, dtype=np.uint32)
    _check(lib().yo_apply_penalties(a, a.size, h, h.size, repetition, presence, frequency))
    return a


def verify(rows, guesses, base_position: int, p: Params | None, eos=()):
    """Acceptance loop (speculation.rs:483-523). Returns (selected, emitted,
    accepted, stop_eos); selected holds only the rows the reference samples."""
    r = _f32(rows)
    M, V = r.shape
    g = np.ascontiguousarray(guesses, dtype=np.uint32)
    if g.size == 0:
        g = np.zeros(1, np.uint32)
    e = np.ascontiguousarray(list(eos) or [0], dtype=np.uint32)
    sel = np.zeros(M, np.uint32)
    em, acc, st = C.c_uint64(), C.c_uint64(), C.c_int()
    pp = p if p is not None else params()
    _check(lib().yo_verify(r, M, V, V, g, base_position, C.byref(pp), 1 if p is None else 0,
                           e, len(eos), sel, C.byref(em), C.byref(acc), C.byref(st)))
    return sel[: em.value], em.value, acc.value, bool(st.value)


def draft_choose(scores, tokens, seed: int, temperature_thousandths: int, position: int) -> int:
    s = _f32(scores)
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = C.c_uint32()
    _check(lib().yo_draft_choose(s, t, seed, temperature_thousandths, position, C.byref(out)))
    return out.value
