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
        ("kept", C.c_double),
        ("uniform", C.c_double),
        ("threshold", C.c_double),
    ]


class DraftDiag(C.Structure):
    """yo_draft_diag: intermediates of one sampled draft choice."""

    _fields_ = [
        ("temperature", C.c_double),
        ("z", C.c_double * 16),
        ("w", C.c_double * 16),
        ("total", C.c_double),
        ("order", C.c_int * 16),
        ("member", C.c_int * 16),
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
        L.yo_draft_choose_ex.argtypes = [f32p, u32p, C.c_int, C.c_uint64, C.c_uint32, C.c_uint64,
                                         C.POINTER(C.c_uint32), C.POINTER(DraftDiag)]
        L.yo_shortlist.argtypes = [f32p, C.c_uint64, C.c_uint64, u32p]
        L.yo_top16.argtypes = [u32p, f32p, C.c_uint64, u32p, f32p]
        L.yo_sqrt_rn.argtypes, L.yo_sqrt_rn.restype = [C.c_float], C.c_float
        L.yo_rsqrt.argtypes, L.yo_rsqrt.restype = [C.c_float], C.c_float
        L.yo_inverse_rms.argtypes = [f32p, C.c_uint64, C.c_float, C.c_float, C.POINTER(C.c_float)]
        i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
        L.yo_head_logits.argtypes = [i64p, f32p, C.c_uint64, C.c_float, C.c_float, f32p]
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


def draft_choose_ex(scores, tokens, seed: int, temperature_thousandths: int, position: int,
                    greedy: bool = False):
    """DraftChoice::{Greedy, Sampled} (draft_head.rs:325-379); returns (token, diag)."""
    s = _f32(scores)
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = C.c_uint32()
    d = DraftDiag()
    _check(lib().yo_draft_choose_ex(s, t, 1 if greedy else 0, seed, temperature_thousandths, position,
                                    C.byref(out), C.byref(d)))
    return out.value, d


def shortlist(scores, count: int) -> np.ndarray:
    """draft_head.rs:239-282: two-stage histogram cutoff, ascending-id tie bucket."""
    s = _f32(scores)
    out = np.zeros(count, np.uint32)
    _check(lib().yo_shortlist(s, s.size, count, out))
    return out


def top16(tokens, scores):
    """draft_head.rs:284-300: the 16 best (score desc, token asc)."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    s = _f32(scores)
    ot = np.zeros(16, np.uint32)
    os_ = np.zeros(16, np.float32)
    _check(lib().yo_top16(t, s, t.size, ot, os_))
    return ot, os_


def sqrt_rn(x: float) -> float:
    return lib().yo_sqrt_rn(x)


def rsqrt(x: float) -> float:
    return lib().yo_rsqrt(x)


def inverse_rms(block_sums, width: float, epsilon: float) -> float:
    b = _f32(block_sums)
    out = C.c_float()
    _check(lib().yo_inverse_rms(b, b.size, width, epsilon, C.byref(out)))
    return out.value


def head_logits(acc, tau, unit_scale: float, inv_rms: float) -> np.ndarray:
    """Head scale restoration (compressed_linear.rs:329-340; spec 06 section 2)."""
    a = np.ascontiguousarray(acc, dtype=np.int64)
    t = _f32(tau)
    out = np.zeros(a.size, np.float32)
    _check(lib().yo_head_logits(a, t, a.size, unit_scale, inv_rms, out))
    return out
