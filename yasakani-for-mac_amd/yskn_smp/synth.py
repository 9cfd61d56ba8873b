"""Seeded synthetic logits for the sampling workloads.

Every random number comes from a counter-based SplitMix64 stream: value i of
stream `key` is mix64(key + i * 0x9E3779B97F4A7C15) (the SplitMix64 sequence),
turned into a uniform in (0, 1) as ((h >> 11) + 0.5) * 2^-53 and into normals
by Box-Muller. The generator runs in torch on any device; the bytes it returns
are the input of both the device sampler and the CPU oracle.

Workloads (vocabulary sizes are the reference model's):
  single_row   1 x 151,936 f32, 2.5*N(0,1), 20 distinct ids spiked +8
  spec_verify  M x 248,320 f32, 3*N(0,1) + Zipf(1.1) bias; drafts from a
               0.5*N(0,1)-perturbed copy
  penalties    1 x 248,320 bf16 of 2*N(0,1); 8,192-token Zipf(1.2) history
  batched      64 x 248,320 f32, sigma_r*N(0,1), sigma_r ~ U[1,4]
  large_batch  256 x 248,320 f32, 2*t_3 (Student-t, nu = 3)
"""
from __future__ import annotations

import math

import torch

GAMMA = 0x9E3779B97F4A7C15
C1 = 0xBF58476D1CE4E5B9
C2 = 0x94D049BB133111EB
MASK64 = (1 << 64) - 1

V_SMALL = 151_936
V_LARGE = 248_320

# stream tags (the "config" part of each stream key)
TAG_SINGLE, TAG_SPEC, TAG_PEN, TAG_BATCH, TAG_LARGE = 1, 2, 3, 4, 5


def _s64(x: int) -> int:
    """Python int -> signed 64-bit value with the same bits."""
    x &= MASK64
    return x - (1 << 64) if x >= (1 << 63) else x


def _srl(z: torch.Tensor, k: int) -> torch.Tensor:
    """Logical right shift of int64 bit patterns."""
    return (z >> k) & ((1 << (64 - k)) - 1)


def mix64_t(z: torch.Tensor) -> torch.Tensor:
    z = z + _s64(GAMMA)
    z = (z ^ _srl(z, 30)) * _s64(C1)
    z = (z ^ _srl(z, 27)) * _s64(C2)
    return z ^ _srl(z, 31)


def mix64_int(z: int) -> int:
    z = (z + GAMMA) & MASK64
    z = ((z ^ (z >> 30)) * C1) & MASK64
    z = ((z ^ (z >> 27)) * C2) & MASK64
    return z ^ (z >> 31)


def stream_key(tag: int, row: int, sub: int = 0) -> int:
    return mix64_int((tag << 40) ^ (sub << 32) ^ row)


def raw64(key: int, n: int, offset: int = 0, device="cpu") -> torch.Tensor:
    i = torch.arange(offset, offset + n, dtype=torch.int64, device=device)
    return mix64_t(i * _s64(GAMMA) + _s64(key))


def uniform(key: int, n: int, offset: int = 0, device="cpu") -> torch.Tensor:
    h = raw64(key, n, offset, device)
    return (_srl(h, 11).to(torch.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(key: int, n: int, device="cpu") -> torch.Tensor:
    m = (n + 1) // 2
    u = uniform(key, 2 * m, 0, device)
    u1, u2 = u[0::2], u[1::2]
    r = torch.sqrt(-2.0 * torch.log(u1))
    z = torch.cat([r * torch.cos(2.0 * math.pi * u2), r * torch.sin(2.0 * math.pi * u2)])
    return z[:n]


def permutation(key: int, n: int, device="cpu") -> torch.Tensor:
    """A seeded permutation of 0..n-1 (argsort of random keys)."""
    h = raw64(key, n, 0, device)
    return torch.argsort(h, stable=True)


def single_row(device="cpu", V: int = V_SMALL) -> torch.Tensor:
    """1 x V f32, 2.5*N(0,1) with 20 distinct seeded ids spiked by +8."""
    x = 2.5 * normal(stream_key(TAG_SINGLE, 0), V, device)
    spikes = permutation(stream_key(TAG_SINGLE, 0, 1), V, device)[:20]
    x = x.to(torch.float32)
    x[spikes] = x[spikes] + 8.0
    return x.reshape(1, V)


def zipf_bias(key: int, V: int, s: float, device="cpu") -> torch.Tensor:
    """b_i = -s * ln(rank_i) for ranks 1..V assigned by a seeded permutation."""
    perm = permutation(key, V, device)
    rank = torch.empty(V, dtype=torch.float64, device=device)
    rank[perm] = torch.arange(1, V + 1, dtype=torch.float64, device=device)
    return -s * torch.log(rank)


def spec_verify(M: int = 8, device="cpu", V: int = V_LARGE):
    """Target logits [M, V] = 3*N(0,1) + Zipf(1.1) bias and a draft copy with
    0.5*N(0,1) noise. Returns (target, draft) float32 tensors."""
    bias = zipf_bias(stream_key(TAG_SPEC, 0, 7), V, 1.1, device)
    tgt = torch.empty((M, V), dtype=torch.float32, device=device)
    drf = torch.empty((M, V), dtype=torch.float32, device=device)
    for r in range(M):
        t = 3.0 * normal(stream_key(TAG_SPEC, r), V, device) + bias
        tgt[r] = t.to(torch.float32)
        drf[r] = (t + 0.5 * normal(stream_key(TAG_SPEC, r, 1), V, device)).to(torch.float32)
    return tgt, drf


def penalties(device="cpu", V: int = V_LARGE, n_hist: int = 8192):
    """1 x V bf16 of 2*N(0,1) and an n_hist-token history drawn Zipf(1.2) over
    ranks, mapped to ids by a seeded permutation. Returns (bf16 logits, int32 history)."""
    x = (2.0 * normal(stream_key(TAG_PEN, 0), V, device)).to(torch.float32).to(torch.bfloat16)
    k = torch.arange(1, V + 1, dtype=torch.float64, device=device)
    pmf = k.pow(-1.2)
    cdf = torch.cumsum(pmf, 0)
    cdf = cdf / cdf[-1]
    u = uniform(stream_key(TAG_PEN, 0, 2), n_hist, 0, device)
    ranks = torch.searchsorted(cdf, u).clamp_(max=V - 1)
    perm = permutation(stream_key(TAG_PEN, 0, 3), V, device)
    hist = perm[ranks].to(torch.int32)
    return x.reshape(1, V), hist


def batched(rows: int = 64, device="cpu", V: int = V_LARGE):
    """rows x V f32, row r = sigma_r * N(0,1) with sigma_r ~ U[1,4]."""
    out = torch.empty((rows, V), dtype=torch.float32, device=device)
    sig = 1.0 + 3.0 * uniform(stream_key(TAG_BATCH, 0, 9), rows, 0, device)
    for r in range(rows):
        out[r] = (sig[r] * normal(stream_key(TAG_BATCH, r), V, device)).to(torch.float32)
    return out


def batched_params(rows: int = 64):
    """Per-row parameters of the batched workload, quantised to thousandths:
    T in [0.3, 1.5], top-p in [0.8, 1.0], min-p in [0, 0.1], top-k cycling
    {1, 20, 50, disabled}, seed_r = mix64(base + r), positions 4096 + r."""
    u = uniform(stream_key(TAG_BATCH, 0, 10), 3 * rows, 0, "cpu").numpy()
    out = []
    ks = [1, 20, 50, 0]
    for r in range(rows):
        t = int(round((0.3 + 1.2 * u[3 * r]) * 1000))
        tp = int(round((0.8 + 0.2 * u[3 * r + 1]) * 1000))
        mp = int(round((0.1 * u[3 * r + 2]) * 1000))
        out.append(dict(temperature_milli=t, top_p_milli=max(1, min(1000, tp)),
                        min_p_milli=max(0, min(1000, mp)), top_k=ks[r % 4],
                        seed=mix64_int(0x5EED + r), position=4096 + r))
    return out


def large_batch(rows: int = 256, device="cpu", V: int = V_LARGE, row0: int = 0):
    """rows x V f32 of 2*t_3: N / sqrt(chi2_3 / 3)."""
    out = torch.empty((rows, V), dtype=torch.float32, device=device)
    for i in range(rows):
        r = row0 + i
        n0 = normal(stream_key(TAG_LARGE, r, 0), V, device)
        c = (normal(stream_key(TAG_LARGE, r, 1), V, device) ** 2
             + normal(stream_key(TAG_LARGE, r, 2), V, device) ** 2
             + normal(stream_key(TAG_LARGE, r, 3), V, device) ** 2)
        out[i] = (2.0 * n0 / torch.sqrt(c / 3.0)).to(torch.float32)
    return out


def large_batch_seeds(rows: int = 256):
    return [mix64_int(0x1A46E + r) for r in range(rows)]
