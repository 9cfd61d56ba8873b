"""Python host binding of the MI355X sampling library (include/yskn_smp.h).

The names mirror the reference's sampling surface so that callers and tests
read like the reference's own:

* ``SamplingParameters`` / ``SamplingParameters.from_thousandths`` /
  ``validate``  -- crates/yskn-ref/src/output_head_sampler.rs:21-75
* ``Sampler`` with ``Greedy`` and ``Sampled(params)`` and ``sample(logits,
  prediction_position)`` -- output_head_sampler.rs:77-92
* ``greedy``, ``top_tokens``, ``negative_log_likelihood`` --
  output_head_sampler.rs:103-134,230-250
* ``select`` (the ``Selector`` trait, crates/yskn-ref/src/speculation.rs:123-139)
* ``verify`` -- the acceptance loop of speculation.rs:483-523

Errors are raised as ``InvalidInput`` / ``NonFinite`` (lib.rs:37-45).

Every call goes through the HIP library ``lib/libyskn_smp.so``; there is no
CPU fallback. If the library is missing the import of the binding fails.
PyTorch provides device memory and the stream only.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libyskn_smp.so")

OK, EINVAL, ENONFINITE, ERANGE, EDEVICE = 0, -1, -2, -3, -4
F32, BF16 = 0, 1
INVERSE_CUMULATIVE, GUMBEL = 2, 3
FLAG_EXTENDED_TOP_K, FLAG_FORCE_DENSE = 0x1, 0x2


class SamplerError(Exception):
    """Base error; ``code`` is the C-ABI status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class InvalidInput(SamplerError):
    pass


class NonFinite(SamplerError):
    pass


class DeviceError(SamplerError):
    pass


class CParams(C.Structure):
    _fields_ = [
        ("temperature_milli", C.c_uint32),
        ("top_p_milli", C.c_uint32),
        ("top_k", C.c_uint32),
        ("min_p_milli", C.c_uint32),
        ("seed", C.c_uint64),
        ("version", C.c_int32),
        ("repetition_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
    ]


class CParamsF64(C.Structure):
    _fields_ = [
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("min_p", C.c_double),
        ("top_k", C.c_uint32),
        ("greedy", C.c_int32),
        ("seed", C.c_uint64),
        ("version", C.c_int32),
        ("repetition_penalty", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
    ]


class CAux(C.Structure):
    _fields_ = [
        ("argmax", C.c_void_p),
        ("top8_ids", C.c_void_p),
        ("top8_vals", C.c_void_p),
        ("top20_ids", C.c_void_p),
        ("top20_vals", C.c_void_p),
        ("n_logprobs", C.c_int32),
        ("logprob_ids", C.c_void_p),
        ("logprobs", C.c_void_p),
        ("row_status", C.c_void_p),
        ("history", C.c_void_p),
        ("history_len", C.c_void_p),
        ("history_ld", C.c_int64),
    ]


class CDraftChoice(C.Structure):
    _fields_ = [("sampled", C.c_int32), ("temperature_thousandths", C.c_uint32), ("seed", C.c_uint64)]


class CHead(C.Structure):
    _fields_ = [
        ("acc", C.c_void_p), ("acc_ld", C.c_int64), ("unit_scale", C.c_void_p),
        ("block_sums", C.c_void_p), ("n_blocks", C.c_int32), ("width", C.c_float),
        ("epsilon", C.c_float), ("tau", C.c_void_p), ("logits_out", C.c_void_p),
        ("logits_ld", C.c_int64), ("clear_acc", C.c_int32),
    ]


class CAdvance(C.Structure):
    _fields_ = [("position", C.c_void_p), ("token", C.c_void_p)]


EXPORTED = [
    "yskn_smp_last_error", "yskn_smp_create", "yskn_smp_destroy", "yskn_smp_set_params",
    "yskn_smp_sample", "yskn_smp_argmax", "yskn_smp_top_tokens", "yskn_smp_nll",
    "yskn_smp_verify", "yskn_smp_sync", "yskn_smp_select_host", "yskn_smp_validate_params",
    "yskn_smp_version", "yskn_smp_get_stats", "yskn_smp_set_params_f64",
    "yskn_smp_validate_params_f64", "yskn_smp_sample_at", "yskn_smp_pm_test",
    "yskn_smp_sample_head", "yskn_smp_draft_shortlist", "yskn_smp_draft_top16", "yskn_smp_draft_choose",
]

_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load libyskn_smp.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    L = C.CDLL(path)
    vp, i32, i64, u32, u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64
    L.yskn_smp_last_error.restype = C.c_char_p
    L.yskn_smp_version.restype = C.c_char_p
    L.yskn_smp_create.argtypes = [i32, i32, u32, C.POINTER(vp)]
    L.yskn_smp_destroy.argtypes = [vp]
    L.yskn_smp_destroy.restype = None
    L.yskn_smp_set_params.argtypes = [vp, C.POINTER(CParams), i32]
    L.yskn_smp_sample.argtypes = [vp, vp, i32, i32, i32, i64, vp, i32, vp, C.POINTER(CAux), vp]
    L.yskn_smp_argmax.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp]
    L.yskn_smp_top_tokens.argtypes = [vp, vp, i32, i32, i32, i64, i32, vp, vp, vp]
    L.yskn_smp_nll.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, vp]
    L.yskn_smp_verify.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, vp, i32, vp, vp, C.POINTER(CAux),
                                  C.POINTER(CAdvance), vp]
    L.yskn_smp_sample_at.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, i32, vp, C.POINTER(CAux),
                                     C.POINTER(CAdvance), vp]
    L.yskn_smp_pm_test.argtypes = [i32, u64, vp, vp, i64]
    L.yskn_smp_sample_head.argtypes = [vp, C.POINTER(CHead), i32, i32, vp, i32, vp, C.POINTER(CAux), vp]
    L.yskn_smp_draft_shortlist.argtypes = [vp, vp, i32, i32, i64, i32, vp, i64, vp, vp]
    L.yskn_smp_draft_top16.argtypes = [vp, vp, vp, i32, i32, i64, vp, vp, vp, vp]
    L.yskn_smp_draft_choose.argtypes = [vp, vp, vp, i32, i64, C.POINTER(CDraftChoice), vp, vp, vp, vp, vp,
                                        vp, vp]
    L.yskn_smp_sync.argtypes = [vp, vp]
    L.yskn_smp_select_host.argtypes = [vp, vp, i32, u64, C.POINTER(u32)]
    L.yskn_smp_validate_params.argtypes = [C.POINTER(CParams), i32, u32]
    L.yskn_smp_set_params_f64.argtypes = [vp, C.POINTER(CParamsF64), i32]
    L.yskn_smp_validate_params_f64.argtypes = [C.POINTER(CParamsF64), i32, u32]
    L.yskn_smp_get_stats.argtypes = [vp, C.POINTER(C.c_uint64), i32]
    L.yskn_smp_get_stats.restype = C.c_int
    for name in ("yskn_smp_create", "yskn_smp_set_params", "yskn_smp_sample", "yskn_smp_argmax",
                 "yskn_smp_top_tokens", "yskn_smp_nll", "yskn_smp_verify", "yskn_smp_sync",
                 "yskn_smp_select_host", "yskn_smp_validate_params", "yskn_smp_sample_at",
                 "yskn_smp_pm_test", "yskn_smp_sample_head", "yskn_smp_draft_shortlist",
                 "yskn_smp_draft_top16", "yskn_smp_draft_choose"):
        L[name].restype = C.c_int
    _lib = L
    return L


def _raise(code: int) -> None:
    if code == OK:
        return
    msg = (_lib.yskn_smp_last_error() or b"").decode()
    if code == ENONFINITE:
        raise NonFinite(code, msg)
    if code in (EINVAL, ERANGE):
        raise InvalidInput(code, msg)
    raise DeviceError(code, msg)


@dataclass
class SamplingParameters:
    """Integer-thousandths sampling parameters (the native setter's units,
    src/engine35.cpp:946-959); the sampler stores binary64 value / 1000.0.
    temperature_milli = 0 selects greedy."""

    temperature_milli: int = 1000
    top_p_milli: int = 950
    top_k: int = 20
    min_p_milli: int = 0
    seed: int = 0
    version: int = GUMBEL
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    @classmethod
    def from_thousandths(cls, temperature: int, top_p: int, min_p: int) -> "SamplingParameters":
        p = cls(temperature_milli=temperature, top_p_milli=top_p, min_p_milli=min_p)
        p.validate(20)
        return p

    @property
    def temperature(self) -> float:
        return self.temperature_milli / 1000.0

    @property
    def top_p(self) -> float:
        return self.top_p_milli / 1000.0

    @property
    def min_p(self) -> float:
        return self.min_p_milli / 1000.0

    def to_c(self) -> CParams:
        return CParams(self.temperature_milli, self.top_p_milli, self.top_k, self.min_p_milli,
                       self.seed & 0xFFFFFFFFFFFFFFFF, self.version, self.repetition_penalty,
                       self.presence_penalty, self.frequency_penalty)

    def validate(self, vocabulary_size: int, flags: int = 0) -> None:
        L = load_library()
        c = self.to_c()
        _raise(L.yskn_smp_validate_params(C.byref(c), vocabulary_size, flags))


@dataclass
class SamplingParametersF64:
    """The Rust ``SamplingParameters`` fields as they are
    (output_head_sampler.rs:21-28): binary64 temperature, top_p and min_p.
    ``greedy=True`` stands for ``Sampler::Greedy``."""

    temperature: float = 1.0
    top_p: float = 0.95
    top_k: int = 20
    min_p: float = 0.0
    seed: int = 0
    version: int = GUMBEL
    greedy: bool = False
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def to_c(self) -> CParamsF64:
        return CParamsF64(self.temperature, self.top_p, self.min_p, self.top_k, int(self.greedy),
                          self.seed & 0xFFFFFFFFFFFFFFFF, self.version, self.repetition_penalty,
                          self.presence_penalty, self.frequency_penalty)

    def validate(self, vocabulary_size: int, flags: int = 0) -> None:
        L = load_library()
        c = self.to_c()
        _raise(L.yskn_smp_validate_params_f64(C.byref(c), vocabulary_size, flags))


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


class DeviceSampler:
    """Owns one native handle: scratch for up to ``max_rows`` rows of up to
    ``max_vocab`` logits. Calls are asynchronous on the current torch stream;
    ``sync()`` raises the first per-row error of the last call."""

    def __init__(self, max_rows: int, max_vocab: int, extended_top_k: bool = False,
                 force_dense: bool = False):
        import torch  # device memory and streams only

        self.torch = torch
        self.L = load_library()
        flags = (FLAG_EXTENDED_TOP_K if extended_top_k else 0) | (FLAG_FORCE_DENSE if force_dense else 0)
        self.flags = flags
        h = C.c_void_p()
        _raise(self.L.yskn_smp_create(max_rows, max_vocab, flags, C.byref(h)))
        self.h = h
        self.max_rows, self.max_vocab = max_rows, max_vocab
        self.device = torch.device("cuda", torch.cuda.current_device())

    def close(self) -> None:
        if getattr(self, "h", None):
            self.L.yskn_smp_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def set_params(self, params) -> None:
        """One set for every row, or one per row. Thousandths sets go
        through yskn_smp_set_params, binary64 sets through
        yskn_smp_set_params_f64 (a list must not mix the two)."""
        if isinstance(params, (SamplingParameters, SamplingParametersF64)):
            params = [params]
        if all(isinstance(p, SamplingParametersF64) for p in params):
            arr = (CParamsF64 * len(params))(*[p.to_c() for p in params])
            _raise(self.L.yskn_smp_set_params_f64(self.h, arr, len(params)))
            return
        arr = (CParams * len(params))(*[p.to_c() for p in params])
        _raise(self.L.yskn_smp_set_params(self.h, arr, len(params)))

    @staticmethod
    def _dtype(logits) -> int:
        import torch

        if logits.dtype == torch.float32:
            return F32
        if logits.dtype == torch.bfloat16:
            return BF16
        raise InvalidInput(EINVAL, "logits must be float32 or bfloat16")

    def _check_logits(self, logits):
        if not logits.is_cuda or logits.dim() != 2 or logits.stride(1) != 1:
            raise InvalidInput(EINVAL, "logits must be a 2-D CUDA tensor with unit column stride")
        return logits.shape[0], logits.shape[1], logits.stride(0)

    def _aux(self, rows, dev, out, argmax=False, top8=False, top20=False, n_logprobs=0,
             history=None, history_len=None, row_status=False) -> CAux:
        """Optional outputs (allocated into `out`) and the penalty history.
        A 1-D history is shared by every row (history_ld = 0); a 2-D history
        must have one row per logits row."""
        torch = self.torch
        aux = CAux()
        if argmax:
            out["argmax"] = torch.empty(rows, dtype=torch.int32, device=dev)
            aux.argmax = out["argmax"].data_ptr()
        if top8:
            out["top8_ids"] = torch.empty((rows, 8), dtype=torch.int32, device=dev)
            out["top8_vals"] = torch.empty((rows, 8), dtype=torch.float32, device=dev)
            aux.top8_ids, aux.top8_vals = out["top8_ids"].data_ptr(), out["top8_vals"].data_ptr()
        if top20:
            out["top20_ids"] = torch.empty((rows, 20), dtype=torch.int32, device=dev)
            out["top20_vals"] = torch.empty((rows, 20), dtype=torch.float32, device=dev)
            aux.top20_ids, aux.top20_vals = out["top20_ids"].data_ptr(), out["top20_vals"].data_ptr()
        if n_logprobs:
            out["logprob_ids"] = torch.empty((rows, n_logprobs), dtype=torch.int32, device=dev)
            out["logprobs"] = torch.empty((rows, n_logprobs), dtype=torch.float64, device=dev)
            aux.n_logprobs = n_logprobs
            aux.logprob_ids, aux.logprobs = out["logprob_ids"].data_ptr(), out["logprobs"].data_ptr()
        if row_status:
            out["status"] = torch.empty(rows, dtype=torch.int32, device=dev)
            aux.row_status = out["status"].data_ptr()
        if history is not None:
            hist = history.to(torch.int32).contiguous()
            if hist.dim() == 1:
                ld, width = 0, hist.shape[0]
            elif hist.dim() == 2 and hist.shape[0] == rows:
                ld, width = hist.stride(0), hist.shape[1]
            else:
                raise InvalidInput(EINVAL, "invalid input: history must be 1-D (shared) or have one row per logits row")
            hl = history_len
            if hl is None:
                hl = torch.full((rows,), width, dtype=torch.int32, device=dev)
            hl = hl.to(torch.int32).contiguous()
            if hl.numel() != rows:
                raise InvalidInput(EINVAL, "invalid input: history_len needs one entry per row")
            out["_hist"], out["_hl"] = hist, hl
            aux.history, aux.history_len, aux.history_ld = hist.data_ptr(), hl.data_ptr(), ld
        return aux

    def sample(self, logits, positions, *, argmax=False, top8=False, top20=False,
               n_logprobs=0, history=None, history_len=None, row_status=False):
        """Sample; positions is an int64 tensor [rows] or [rows, n_draws] of
        absolute prediction positions. Returns a dict of device tensors."""
        torch = self.torch
        rows, V, ld = self._check_logits(logits)
        pos = positions.to(torch.int64)
        if pos.dim() == 1:
            pos = pos.reshape(rows, 1)
        pos = pos.contiguous()
        n_draws = pos.shape[1]
        dev = logits.device
        out = {"ids": torch.empty((rows, n_draws), dtype=torch.int32, device=dev)}
        aux = self._aux(rows, dev, out, argmax, top8, top20, n_logprobs, history, history_len, row_status)
        out["_pos"] = pos
        _raise(self.L.yskn_smp_sample(self.h, logits.data_ptr(), self._dtype(logits), rows, V, ld,
                                      pos.data_ptr(), n_draws, out["ids"].data_ptr(),
                                      C.byref(aux), self._stream()))
        return out

    def sample_at(self, logits, base_position, *, row_depth=None, row0=0, advance=None,
                  argmax=False, top8=False, top20=False, n_logprobs=0, history=None,
                  history_len=None, row_status=False):
        """Sample at device positions *base_position + depth + 1 (depth from
        row_depth[row0 + r] or row0 + r). advance = (position int64 tensor [1],
        token int32 tensor [1]) advances them on the device (one row only)."""
        torch = self.torch
        rows, V, ld = self._check_logits(logits)
        dev = logits.device
        out = {"ids": torch.empty(rows, dtype=torch.int32, device=dev)}
        aux = self._aux(rows, dev, out, argmax, top8, top20, n_logprobs, history, history_len, row_status)
        adv = None
        if advance is not None:
            adv = CAdvance(advance[0].data_ptr(), advance[1].data_ptr())
        depth_ptr = None
        if row_depth is not None:
            out["_depth"] = row_depth.to(torch.uint8).contiguous()
            depth_ptr = out["_depth"].data_ptr()
        _raise(self.L.yskn_smp_sample_at(self.h, logits.data_ptr(), self._dtype(logits), rows, V, ld,
                                         base_position.data_ptr(), depth_ptr, row0, out["ids"].data_ptr(),
                                         C.byref(aux), C.byref(adv) if adv is not None else None,
                                         self._stream()))
        return out

    def sample_head(self, acc, unit_scale, block_sums, tau, positions, *, width=5120.0, epsilon=1e-6,
                    logits_out=None, clear_acc=False, argmax=False, top8=False, top20=False,
                    n_logprobs=0, history=None, history_len=None, row_status=False):
        """yskn_smp_sample_head: sample from the output head's int64
        accumulators (acc [rows, V] int64, unit_scale [rows] f32, block_sums
        [rows, n_blocks] f32, tau [V] f32), the logits formed in the sweep."""
        torch = self.torch
        if not acc.is_cuda or acc.dim() != 2 or acc.stride(1) != 1 or acc.dtype != torch.int64:
            raise InvalidInput(EINVAL, "acc must be a 2-D int64 CUDA tensor with unit column stride")
        rows, V, ld = acc.shape[0], acc.shape[1], acc.stride(0)
        dev = acc.device
        pos = positions.to(torch.int64)
        if pos.dim() == 1:
            pos = pos.reshape(rows, 1)
        pos = pos.contiguous()
        us = unit_scale.to(torch.float32).contiguous()
        sums = block_sums.to(torch.float32).contiguous()
        tt = tau.to(torch.float32).contiguous()
        out = {"ids": torch.empty((rows, pos.shape[1]), dtype=torch.int32, device=dev),
               "_keep": (pos, us, sums, tt)}
        aux = self._aux(rows, dev, out, argmax, top8, top20, n_logprobs, history, history_len, row_status)
        hd = CHead(acc.data_ptr(), ld, us.data_ptr(), sums.data_ptr(), sums.shape[1], width, epsilon,
                   tt.data_ptr(), _ptr(logits_out), logits_out.stride(0) if logits_out is not None else 0,
                   1 if clear_acc else 0)
        _raise(self.L.yskn_smp_sample_head(self.h, C.byref(hd), rows, V, pos.data_ptr(), pos.shape[1],
                                           out["ids"].data_ptr(), C.byref(aux), self._stream()))
        return out

    def argmax(self, logits):
        torch = self.torch
        rows, V, ld = self._check_logits(logits)
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
        _raise(self.L.yskn_smp_argmax(self.h, logits.data_ptr(), self._dtype(logits), rows, V, ld,
                                      out.data_ptr(), self._stream()))
        return out

    def top_tokens(self, logits, count: int):
        torch = self.torch
        rows, V, ld = self._check_logits(logits)
        ids = torch.empty((rows, count), dtype=torch.int32, device=logits.device)
        vals = torch.empty((rows, count), dtype=torch.float32, device=logits.device)
        _raise(self.L.yskn_smp_top_tokens(self.h, logits.data_ptr(), self._dtype(logits), rows, V,
                                          ld, count, ids.data_ptr(), vals.data_ptr(),
                                          self._stream()))
        return ids, vals

    def nll(self, logits, targets):
        torch = self.torch
        rows, V, ld = self._check_logits(logits)
        t = targets.to(torch.int32).contiguous()
        out = torch.empty(rows, dtype=torch.float64, device=logits.device)
        _raise(self.L.yskn_smp_nll(self.h, logits.data_ptr(), self._dtype(logits), rows, V, ld,
                                   t.data_ptr(), out.data_ptr(), self._stream()))
        return out

    def verify(self, logits, drafts, base_position, eos_ids: Sequence[int] = (), *, commit=None,
               argmax=False, top8=False, top20=False, n_logprobs=0, history=None,
               history_len=None, row_status=False):
        """One-launch verification of M rows; returns (ids[M], result[5], keep)
        with result = (accepted, emitted, token, stop_eos, status) as device
        int32 and `keep` holding the buffers (and the optional outputs, as a
        dict, in keep[-1]). commit = (position int64 [1], token int32 [1])
        advances them on the device when the pass succeeds."""
        torch = self.torch
        M, V, ld = self._check_logits(logits)
        dev = logits.device
        d = drafts.to(torch.int32).contiguous() if M > 1 else torch.zeros(1, dtype=torch.int32, device=dev)
        bp = base_position.to(torch.int64).reshape(1).contiguous() if base_position.dtype != torch.int64 \
            else base_position.reshape(1)
        eos = torch.tensor(list(eos_ids) or [0], dtype=torch.int32, device=dev)
        ids = torch.empty(M, dtype=torch.int32, device=dev)
        res = torch.empty(5, dtype=torch.int32, device=dev)
        outs = {}
        aux = self._aux(M, dev, outs, argmax, top8, top20, n_logprobs, history, history_len, row_status)
        adv = CAdvance(commit[0].data_ptr(), commit[1].data_ptr()) if commit is not None else None
        _raise(self.L.yskn_smp_verify(self.h, logits.data_ptr(), self._dtype(logits), M, V, ld,
                                      d.data_ptr(), bp.data_ptr(), eos.data_ptr(), len(eos_ids),
                                      ids.data_ptr(), res.data_ptr(), C.byref(aux),
                                      C.byref(adv) if adv is not None else None, self._stream()))
        return ids, res, (d, bp, eos, outs)

    # ---- draft-side selection (draft_head.rs:219-379) ----
    def _rows2d(self, t, dtype, what):
        torch = self.torch
        if not t.is_cuda or t.dim() != 2 or t.stride(1) != 1 or t.dtype != dtype:
            raise InvalidInput(EINVAL, f"{what} must be a 2-D {dtype} CUDA tensor with unit column stride")
        return t.shape[0], t.shape[1], t.stride(0)

    def draft_shortlist(self, scores, count: int, row_status=False):
        """shortlist() per row of scores [rows, V] f32: count ids [rows, count]."""
        torch = self.torch
        rows, V, ld = self._rows2d(scores, torch.float32, "scores")
        out = {"ids": torch.empty((rows, max(count, 1)), dtype=torch.int32, device=scores.device)}
        if row_status:
            out["status"] = torch.empty(rows, dtype=torch.int32, device=scores.device)
        _raise(self.L.yskn_smp_draft_shortlist(self.h, scores.data_ptr(), rows, V, ld, count,
                                               out["ids"].data_ptr(), out["ids"].stride(0),
                                               _ptr(out.get("status")), self._stream()))
        return out

    def draft_top16(self, tokens, scores, row_status=False):
        """top16() per row of (tokens [rows, n] int32, scores [rows, n] f32)."""
        torch = self.torch
        rows, n, ld = self._rows2d(scores, torch.float32, "scores")
        if tuple(tokens.shape) != (rows, n) or tokens.stride() != scores.stride() or tokens.dtype != torch.int32:
            raise InvalidInput(EINVAL, "tokens must be int32 and laid out like scores")
        out = {"tokens": torch.empty((rows, 16), dtype=torch.int32, device=scores.device),
               "scores": torch.empty((rows, 16), dtype=torch.float32, device=scores.device)}
        if row_status:
            out["status"] = torch.empty(rows, dtype=torch.int32, device=scores.device)
        _raise(self.L.yskn_smp_draft_top16(self.h, tokens.data_ptr(), scores.data_ptr(), rows, n, ld,
                                           out["tokens"].data_ptr(), out["scores"].data_ptr(),
                                           _ptr(out.get("status")), self._stream()))
        return out

    def draft_choose(self, scores, tokens, *, sampled=True, seed=0, temperature_thousandths=850,
                     positions=None, alternates=False, row_status=False):
        """choose() per row of 16 candidates (scores [rows, >=16] f32, tokens
        int32 alike); positions int64 [rows] for a sampled choice."""
        torch = self.torch
        rows, n, ld = self._rows2d(scores, torch.float32, "scores")
        if tuple(tokens.shape) != (rows, n) or tokens.stride() != scores.stride() or tokens.dtype != torch.int32:
            raise InvalidInput(EINVAL, "tokens must be int32 and laid out like scores")
        dev = scores.device
        out = {"token": torch.empty(rows, dtype=torch.int32, device=dev)}
        if alternates:
            out["alt"] = torch.empty(rows, dtype=torch.int32, device=dev)
            out["margin"] = torch.empty(rows, dtype=torch.float32, device=dev)
            out["alt3"] = torch.empty(rows, dtype=torch.int32, device=dev)
        if row_status:
            out["status"] = torch.empty(rows, dtype=torch.int32, device=dev)
        pos = None
        if positions is not None:
            pos = positions.to(device=dev, dtype=torch.int64).contiguous()
            out["_pos"] = pos
        ch = CDraftChoice(1 if sampled else 0, temperature_thousandths, seed & 0xFFFFFFFFFFFFFFFF)
        _raise(self.L.yskn_smp_draft_choose(self.h, scores.data_ptr(), tokens.data_ptr(), rows, ld, C.byref(ch),
                                            _ptr(pos), out["token"].data_ptr(), _ptr(out.get("alt")),
                                            _ptr(out.get("margin")), _ptr(out.get("alt3")),
                                            _ptr(out.get("status")), self._stream()))
        return out

    def sync(self) -> None:
        _raise(self.L.yskn_smp_sync(self.h, self._stream()))

    STAT_NAMES = ("rows", "dense_rows", "certified_rows", "candidates")

    def stats(self) -> dict:
        """Cumulative profiling counters of the handle (synchronises)."""
        buf = (C.c_uint64 * len(self.STAT_NAMES))()
        n = self.L.yskn_smp_get_stats(self.h, buf, len(self.STAT_NAMES))
        if n < 0:
            _raise(n)
        return {k: int(buf[i]) for i, k in enumerate(self.STAT_NAMES[:n])}

    def select(self, logits: np.ndarray, prediction_position: int) -> int:
        """Selector::select on a host slice (speculation.rs:123-139)."""
        a = np.ascontiguousarray(logits, dtype=np.float32)
        out = C.c_uint32()
        _raise(self.L.yskn_smp_select_host(self.h, a.ctypes.data, a.size, prediction_position,
                                           C.byref(out)))
        return out.value


@dataclass
class Sampler:
    """``Sampler::{Greedy, Sampled(params)}`` (output_head_sampler.rs:77-92)
    running on the device. ``sample`` takes a host slice, like the Rust API."""

    params: Optional[SamplingParameters] = None  # None = Greedy
    extended_top_k: bool = False
    _dev: Optional[DeviceSampler] = field(default=None, repr=False)

    @classmethod
    def greedy(cls) -> "Sampler":
        return cls(None)

    @classmethod
    def sampled(cls, params: SamplingParameters, extended_top_k: bool = False) -> "Sampler":
        return cls(params, extended_top_k)

    def _device(self, V: int) -> DeviceSampler:
        if self._dev is None or self._dev.max_vocab < V:
            self._dev = DeviceSampler(1, max(V, 1), extended_top_k=self.extended_top_k)
        self._dev.set_params(self.params if self.params is not None
                             else SamplingParameters(temperature_milli=0))
        return self._dev

    def sample(self, logits, prediction_position: int) -> int:
        a = np.ascontiguousarray(logits, dtype=np.float32)
        if a.size == 0:
            load_library()
            raise InvalidInput(EINVAL, "invalid input: logits must contain a nonempty u32-indexed vocabulary")
        return self._device(a.size).select(a, prediction_position)

    select = sample


def greedy(logits) -> int:
    return Sampler.greedy().sample(logits, 0)


def top_tokens(logits, count: int) -> np.ndarray:
    import torch

    a = np.ascontiguousarray(logits, dtype=np.float32)
    dev = DeviceSampler(1, max(a.size, 1))
    t = torch.from_numpy(a).reshape(1, -1).cuda()
    ids, _ = dev.top_tokens(t, count)
    dev.sync()
    return ids.cpu().numpy().astype(np.uint32).reshape(-1)


def negative_log_likelihood(logits, target: int) -> float:
    import torch

    a = np.ascontiguousarray(logits, dtype=np.float32)
    dev = DeviceSampler(1, max(a.size, 1))
    t = torch.from_numpy(a).reshape(1, -1).cuda()
    out = dev.nll(t, torch.tensor([target], dtype=torch.int32, device=t.device))
    dev.sync()
    return float(out.cpu()[0])


def version() -> str:
    return load_library().yskn_smp_version().decode()


def pm_test(fn: int, inputs=None, base: int = 0, n: int = 0) -> np.ndarray:
    """yskn_smp_pm_test: one device primitive on host inputs (see
    include/yskn_smp.h). fn 10/11/14/15 take u64 words (binary64 bits or
    integers), 12 takes (seed, position, token) rows, 16 (z binary32 bits,
    position key, token) rows, 13 (seed, position) rows, 6/7 the binary32
    bit patterns base .. base + n - 1."""
    L = load_library()
    if fn in (6, 7):
        out = np.zeros(n, np.uint32)
        _raise(L.yskn_smp_pm_test(fn, base, None, out.ctypes.data, n))
        return out
    a = np.ascontiguousarray(inputs)
    if a.dtype == np.float64:
        a = a.view(np.uint64)
    a = np.ascontiguousarray(a, dtype=np.uint64)
    n = a.shape[0]
    out = np.zeros(n, np.uint64)
    _raise(L.yskn_smp_pm_test(fn, 0, a.ctypes.data, out.ctypes.data, n))
    return out
