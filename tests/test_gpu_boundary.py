"""GPU checks of the boundary pieces around the sampler kernel, through the C ABI:

* device portable math, bit for bit against the oracle (the reference's
  yskn_pm_test hook, src/pm_test.cu:30-52): exp_d, log_d across every fdlibm
  branch, the Gumbel and version-2 uniforms, mix64, sqrt_rn and rsqrt;
* rows whose length is not a whole number of 16-byte groups on the vector
  path (padded ld, 16-byte aligned base, row maximum in the last group);
* the device position form and advance of launch_q35_smp
  (src/q35_sample.cu:180-181,206) through yskn_smp_sample_at;
* verify: rows after the first mismatch are never validated
  (speculation.rs:520-522), checked position overflow (:489-497), per-row
  argmax / top-8 outputs (include/yskn_abi.h:39,55), on-device commit
  (src/engine35.cpp:1319-1329), per-row parameters;
* the reference's NonFinite rule for z = (l - l_0) / T at tiny temperatures
  (output_head_sampler.rs:146-153);
* the penalty history layout (shared 1-D history, length above the row stride).
"""
import math
import struct

import numpy as np
import pytest
import torch

import yskn_oracle as O
from gpu_helpers import assert_logprobs_close, oracle_params, oracle_select, pmap, to_u32

pytestmark = pytest.mark.gpu

import yskn_smp
from yskn_smp import (GUMBEL, INVERSE_CUMULATIVE, DeviceSampler, InvalidInput, NonFinite,
                      SamplingParameters, SamplingParametersF64)

DEV = "cuda"


def _bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


# ---------------------------------------------------------------------------
# device math
# ---------------------------------------------------------------------------
def _exp_inputs(rng):
    parts = [
        rng.uniform(-745.2, 709.8, 400_000),                    # whole range
        rng.uniform(-0.35, 0.35, 100_000),                      # |x| <= 0.5 ln2: k = 0
        rng.uniform(0.34, 1.04, 100_000) * rng.choice([-1, 1], 100_000),  # k = +-1 branch
        rng.uniform(-745.2, -708.0, 100_000),                   # subnormal results
        rng.uniform(-1e-8, 1e-8, 50_000),                       # tiny: 1 + x
        np.ldexp(rng.uniform(0.5, 1.0, 50_000), rng.integers(-1074, -28, 50_000)),
        rng.uniform(709.0, 710.0, 50_000), rng.uniform(-746.0, -744.0, 50_000),  # limits
        rng.standard_normal(100_000) * 40.0,                    # the sampler's z range
        np.array([0.0, -0.0, 1.0, 0.5, 10.0, -746.0, 710.0, math.inf, -math.inf, math.nan,
                  709.782712893384, -745.1332191019411, 0.5 * math.log(2), 1.5 * math.log(2)]),
    ]
    return np.concatenate(parts)


def _log_inputs(rng):
    parts = [
        np.exp(rng.uniform(-740.0, 709.0, 500_000)),
        rng.uniform(0.70, 1.42, 100_000),                       # k = 0 around 1
        1.0 + rng.uniform(-1e-6, 1e-6, 50_000),                 # f near 0
        np.ldexp(1.0 + rng.integers(0, 4, 50_000) * 2.0**-52, rng.integers(-1000, 1000, 50_000)),
        np.ldexp(rng.uniform(0.5, 1.0, 100_000), rng.integers(-1074, -1022, 100_000)),  # subnormal
        rng.uniform(0.0, 1.0, 100_000),                         # Gumbel's log(u)
        -np.log(rng.uniform(1e-16, 1.0, 100_000)),              # Gumbel's log(-log u)
        np.array([0.0, -0.0, 1.0, 2.0, 0.5, 10.0, math.inf, 5e-324, 1.7976931348623157e308]),
    ]
    return np.concatenate(parts)


@pytest.mark.parametrize("fn,oracle_fn,gen", [(10, O.exp_d, _exp_inputs), (11, O.log_d, _log_inputs)])
def test_device_exp_log_bits_match_the_oracle(fn, oracle_fn, gen):
    x = gen(np.random.default_rng(fn))
    assert x.size >= 1_000_000
    got = yskn_smp.pm_test(fn, x.astype(np.float64))
    lib = O.lib()
    f = lib.yo_exp_d if fn == 10 else lib.yo_log_d
    want = np.array([f(float(v)) for v in x], np.float64)
    gv = got.view(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(gv), nan)
    bad = np.nonzero(got[~nan] != _bits(want)[~nan])[0]
    assert bad.size == 0, (x[~nan][bad[:5]], gv[~nan][bad[:5]], want[~nan][bad[:5]])


def test_device_log_zero_artefacts_and_reference_vectors():
    # portable_math.rs:563-587
    got = yskn_smp.pm_test(11, np.array([0.0, -0.0, 0.5, 1.0, 10.0]))
    assert [hex(int(v)) for v in got] == ["0xc0875427f6acad6f", "0xc0a0ec2b7d284853", "0xbfe62e42fefa39ef",
                                          "0x0", "0x40026bb1bbb55516"]
    got = yskn_smp.pm_test(10, np.array([0.5, 1.0, 10.0, 0.0]))
    assert [hex(int(v)) for v in got] == ["0x3ffa61298e1e069c", "0x4005bf0a8b14576a", "0x40d5829dcf950560",
                                          "0x3ff0000000000000"]


def test_device_hashes_and_uniforms_match_the_oracle():
    rng = np.random.default_rng(3)
    n = 200_000
    seeds = rng.integers(0, 2**64, n, dtype=np.uint64)
    pos = rng.integers(0, 2**64, n, dtype=np.uint64)
    pos[:10] = [0, 1, 2**63, 2**64 - 1, 2**32, 7, 2**53 + 1, 100, 1023, 4096]
    tok = rng.integers(0, 2**32, n, dtype=np.uint64)
    g = yskn_smp.pm_test(12, np.stack([seeds, pos, tok], 1).reshape(-1, 3)).view(np.float64)
    u = yskn_smp.pm_test(13, np.stack([seeds, pos], 1)).view(np.float64)
    m = yskn_smp.pm_test(14, seeds)
    sel = range(0, n, 7)
    assert all(_bits([O.gumbel(int(seeds[i]), int(pos[i]), int(tok[i]))])[0] == g.view(np.uint64)[i] for i in sel)
    lib = O.lib()
    assert all(_bits([lib.yo_uniform_v2(int(seeds[i]), int(pos[i]))])[0] == u.view(np.uint64)[i] for i in sel)
    assert all(O.mix64(int(seeds[i])) == int(m[i]) for i in sel)


def _mix64(x):
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def test_certified_tail_approximations_stay_within_their_bounds():
    """The certified dense tail rests on two bounded approximations, taken
    here from the device: its polynomial exp (within 2^-46 relative of e^z
    for z <= 0, against long double) and its binary32 version-3 score (within
    1e-4 of the binary64 z + g, z = (l - M) / T formed as the tail forms it,
    g the device Gumbel noise that matches the oracle bit for bit)."""
    rng = np.random.default_rng(8)
    z = np.concatenate([-40.0 * rng.random(300_000), -700.0 * rng.random(1000),
                        [0.0, -0.0, -1e-300, -37.5, -40.0, -0.34657359, -0.34657360, -700.0]])
    got = yskn_smp.pm_test(15, z.astype(np.float64)).view(np.float64)
    ref = np.exp(z.astype(np.longdouble))
    rel = np.abs((got.astype(np.longdouble) - ref) / ref)
    assert float(rel.max()) <= 2.0 ** -46, float(rel.max())
    n = 400_000
    seeds = rng.integers(0, 2**64, n, dtype=np.uint64)
    pos = rng.integers(0, 2**64, n, dtype=np.uint64)
    tok = rng.integers(0, 2**32, n, dtype=np.uint64)
    T = rng.uniform(0.2, 3.0, n)
    l = (8.0 * rng.standard_normal(n)).astype(np.float32)
    M = (l.astype(np.float64) + 37.5 * T * rng.random(n)).astype(np.float32)
    M = np.maximum(M, l)
    zf = (l - M) * (1.0 / T).astype(np.float32)  # binary32, as the tail forms it
    pk = _mix64(_mix64(seeds) ^ pos)
    s32 = yskn_smp.pm_test(16, np.stack([zf.view(np.uint32).astype(np.uint64), pk, tok], 1))
    s32 = s32.astype(np.uint32).view(np.float32).astype(np.float64)
    g = yskn_smp.pm_test(12, np.stack([seeds, pos, tok], 1)).view(np.float64)
    exact = (l.astype(np.float64) - M.astype(np.float64)) / T + g
    fin = np.isfinite(exact)
    err = np.abs(s32[fin] - exact[fin])
    assert float(err.max()) <= 1e-4, float(err.max())
    assert np.all(np.isposinf(s32[~fin]))


@pytest.mark.parametrize("fn", [6, 7])
def test_device_sqrt_rn_and_rsqrt_are_correctly_rounded(fn):
    for base, n in [(0, 1 << 22), (0x3F000000, 1 << 24), (0x7F000000, 0x7F800000 - 0x7F000000)]:
        got = yskn_smp.pm_test(fn, base=base, n=n)
        x = (np.arange(n, dtype=np.uint64) + base).astype(np.uint32).view(np.float32)
        s = np.sqrt(x)
        want = (np.float32(1.0) / s if fn == 6 else s).view(np.uint32)
        assert np.array_equal(got, want)


# ---------------------------------------------------------------------------
# vector path: rows that end inside a 16-byte group
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,V,ld", [("f32", 1537, 1540), ("f32", 33_333, 33_336),
                                        ("f32", 248_317, 248_320), ("bf16", 30_001, 30_008),
                                        ("bf16", 2049, 2056)])
def test_padded_rows_with_a_ragged_last_group(dtype, V, ld):
    rng = np.random.default_rng(V)
    rows = 4
    buf = torch.empty(rows * ld + 64, dtype=torch.float32 if dtype == "f32" else torch.bfloat16, device=DEV)
    off = (-buf.data_ptr() // buf.element_size()) % (16 // buf.element_size())
    base = buf[off: off + rows * ld].view(rows, ld)
    assert base.data_ptr() % 16 == 0
    x = (2.0 * rng.standard_normal((rows, V))).astype(np.float32)
    x[:, V - 1] = 50.0                       # the row maximum sits in the last group
    x[1, V - 2] = 60.0
    x[2, V - 3:] = 70.0                      # ties in the last group
    t = torch.from_numpy(x).to(DEV)
    base[:, :V] = t.to(base.dtype)
    base[:, V:] = 1e30                       # padding must never be read
    view = base[:, :V]
    xs = view.float().cpu().numpy()
    d = DeviceSampler(rows, V)
    sp = SamplingParameters(temperature_milli=800, top_p_milli=950, top_k=20, seed=V)
    d.set_params(sp)
    out = d.sample(view, torch.arange(rows, device=DEV) + 3, argmax=True, top20=True, n_logprobs=20)
    d.sync()
    assert list(to_u32(out["argmax"])) == [O.greedy(xs[r]) for r in range(rows)]
    for r in range(rows):
        ids, lp = O.top_logprobs(xs[r], 20)
        assert list(to_u32(out["logprob_ids"])[r]) == list(ids)
        assert_logprobs_close(out["logprobs"][r].cpu().numpy(), lp)
    for r in range(rows):
        tt = O.top_tokens(xs[r], 20)
        assert list(to_u32(out["top20_ids"])[r]) == list(tt)
        assert np.array_equal(out["top20_vals"][r].cpu().numpy().view(np.uint32), xs[r][tt].view(np.uint32))
    assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(xs[r], r + 3, sp) for r in range(rows)]
    d.close()


# ---------------------------------------------------------------------------
# device position form and advance
# ---------------------------------------------------------------------------
def test_sample_at_matches_explicit_positions_with_depth_table_and_row0():
    rng = np.random.default_rng(41)
    rows, V = 6, 20_000
    x = (2.0 * rng.standard_normal((rows, V))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    d = DeviceSampler(rows, V)
    sp = SamplingParameters(temperature_milli=900, top_p_milli=930, top_k=20, seed=12)
    d.set_params(sp)
    base = torch.tensor([1_000_000], dtype=torch.int64, device=DEV)
    depth = torch.tensor([0, 0, 3, 1, 2, 2, 1, 5, 4], dtype=torch.uint8, device=DEV)
    for row_depth, row0 in [(None, 0), (None, 3), (depth, 0), (depth, 2)]:
        out = d.sample_at(xt, base, row_depth=row_depth, row0=row0, argmax=True)
        d.sync()
        dep = [(int(depth[row0 + r]) if row_depth is not None else row0 + r) for r in range(rows)]
        pos = [1_000_000 + dp + 1 for dp in dep]
        assert list(to_u32(out["ids"])) == [oracle_select(x[r], pos[r], sp) for r in range(rows)]
        ref = d.sample(xt, torch.tensor(pos, device=DEV))
        d.sync()
        assert torch.equal(out["ids"], ref["ids"].reshape(-1))
    d.close()


def test_sample_at_advance_runs_a_decode_loop_on_the_device():
    rng = np.random.default_rng(42)
    V = 30_000
    x = (2.5 * rng.standard_normal((1, V))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    d = DeviceSampler(1, V)
    sp = SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, seed=77)
    d.set_params(sp)
    pos = torch.tensor([500], dtype=torch.int64, device=DEV)
    tok = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    got = []
    for step in range(12):
        # the position counter is both the base and the advance target
        d.sample_at(xt, pos, advance=(pos, tok))
        got.append(int(tok.cpu()[0]))
    d.sync()
    assert int(pos.cpu()[0]) == 512
    assert got == [oracle_select(x[0], 500 + s + 1, sp) for s in range(12)]
    with pytest.raises(InvalidInput):
        d2 = DeviceSampler(2, V)
        d2.sample_at(torch.zeros((2, V), device=DEV), pos, advance=(pos, tok))
    d.close()


def test_decode_step_replays_in_a_hip_graph():
    # the decode step (device position form, device advance, a row split in
    # segments) captured once in a HIP graph: the call allocates nothing and
    # records no memset, so every replay samples at the advanced position
    # exactly as an eager call does; eager work and synchronisation between
    # the replays
    rng = np.random.default_rng(43)
    V = 30_000
    x = (2.5 * rng.standard_normal((1, V))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    d = DeviceSampler(1, V)
    sp = SamplingParameters(temperature_milli=800, top_p_milli=950, top_k=20, seed=91)
    d.set_params(sp)
    pos = torch.tensor([900], dtype=torch.int64, device=DEV)
    tok = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = d.sample_at(xt, pos, advance=(pos, tok), top20=True)
    assert int(pos.cpu()[0]) == 900                 # capture runs nothing
    for r in range(6):
        g.replay()
        d.sync()
        p = 900 + r + 1
        assert int(pos.cpu()[0]) == p
        want = oracle_select(x[0], p, sp)
        assert int(tok.cpu()[0]) == want and int(out["ids"].cpu()[0]) == want
        assert list(to_u32(out["top20_ids"])[0]) == list(O.top_tokens(x[0], 20))
        # eager work between replays: a torch reduction and an eager call
        assert float((xt * 2.0).sum()) == pytest.approx(2.0 * float(xt.sum()), rel=1e-5)
        e = d.sample(xt, torch.tensor([[p]], dtype=torch.int64, device=DEV))
        d.sync()
        assert int(to_u32(e["ids"])[0, 0]) == want
    d.close()


def test_sample_at_position_overflow_fails_the_row():
    V = 1000
    x = torch.zeros((2, V), dtype=torch.float32, device=DEV)
    d = DeviceSampler(2, V)
    d.set_params(SamplingParameters(temperature_milli=0))
    base = torch.tensor([np.uint64(2**64 - 2).view(np.int64)], dtype=torch.int64, device=DEV)
    out = d.sample_at(x, base, row_status=True)       # row 0 at 2^64 - 1, row 1 past it
    with pytest.raises(InvalidInput):
        d.sync()
    assert out["status"].cpu().tolist() == [0, -1]
    assert to_u32(out["ids"])[1] == 0xFFFFFFFF
    d.close()


# ---------------------------------------------------------------------------
# verify
# ---------------------------------------------------------------------------
def _verify_rows(M, V, seed):
    rng = np.random.default_rng(seed)
    return (2.0 * rng.standard_normal((M, V))).astype(np.float32)


def test_verify_ignores_a_failed_row_after_the_first_mismatch():
    M, V = 5, 8000
    x = _verify_rows(M, V, 1)
    sp = SamplingParameters(top_k=20, seed=3)
    p = oracle_params(sp)
    truth = [O.sample(x[j], 100 + j + 1, p) for j in range(M)]
    bad = x.copy()
    bad[3, 17] = np.nan
    d = DeviceSampler(M, V)
    d.set_params(sp)
    drafts = list(truth[:M - 1])
    drafts[1] = (drafts[1] + 1) % V                 # mismatch at row 1: rows 2.. never reached
    ids, res, _ = d.verify(torch.from_numpy(bad).to(DEV), torch.tensor(drafts, device=DEV),
                           torch.tensor([100], device=DEV))
    d.sync()
    sel, em, acc, stop = O.verify(bad, drafts, 100, p)
    r = res.cpu().tolist()
    assert (r[0], r[1], r[2], r[4]) == (acc, em, sel[-1], 0)
    # all drafts right: the walk reaches row 3 and the pass fails
    ids, res, _ = d.verify(torch.from_numpy(bad).to(DEV), torch.tensor(truth[:M - 1], device=DEV),
                           torch.tensor([100], device=DEV))
    with pytest.raises(NonFinite):
        d.sync()
    with pytest.raises(O.OracleError):
        O.verify(bad, truth[:M - 1], 100, p)
    r = res.cpu().tolist()
    assert r[4] == -2 and r[1] == 0
    d.close()


def test_verify_position_overflow_matches_the_checked_accept_loop():
    x = np.array([[0.0, 1.0, 2.0], [2.0, 1.0, 0.0], [1.0, 2.0, 0.0]], np.float32)
    d = DeviceSampler(3, 3)
    d.set_params(SamplingParameters(temperature_milli=0))
    base = torch.tensor([np.uint64(2**64 - 3).view(np.int64)], dtype=torch.int64, device=DEV)
    xt = torch.from_numpy(x).to(DEV)
    ids, res, _ = d.verify(xt, torch.tensor([2, 1], device=DEV), base)
    d.sync()
    assert res.cpu().tolist()[:3] == [1, 2, 0]
    ids, res, _ = d.verify(xt, torch.tensor([2, 0], device=DEV), base)
    with pytest.raises(InvalidInput):
        d.sync()
    assert res.cpu().tolist()[4] == -1
    d.close()


def test_verify_per_row_outputs_commit_and_per_row_params():
    M, V = 8, 40_000
    x = _verify_rows(M, V, 7)
    xt = torch.from_numpy(x).to(DEV)
    sps = [SamplingParameters(temperature_milli=600 + 100 * j, top_p_milli=900, top_k=[20, 5, 1, 20][j % 4],
                              seed=9 + j, version=GUMBEL if j % 2 else INVERSE_CUMULATIVE) for j in range(M)]
    base = 4_000
    truth = [oracle_select(x[j], base + j + 1, sps[j]) for j in range(M)]
    d = DeviceSampler(M, V)
    d.set_params(sps)
    for depth_wrong in (None, 4):
        drafts = list(truth[:M - 1])
        if depth_wrong is not None:
            drafts[depth_wrong] = (drafts[depth_wrong] + 1) % V
        pos = torch.tensor([base], dtype=torch.int64, device=DEV)
        tok = torch.full((1,), -1, dtype=torch.int32, device=DEV)
        ids, res, keep = d.verify(xt, torch.tensor(drafts, device=DEV), pos, commit=(pos, tok),
                                  argmax=True, top8=True, top20=True, n_logprobs=8)
        d.sync()
        outs = keep[-1]
        r = res.cpu().tolist()
        emitted = M if depth_wrong is None else depth_wrong + 1
        assert r[1] == emitted and r[0] == (M - 1 if depth_wrong is None else depth_wrong)
        assert list(to_u32(ids)[:emitted]) == truth[:emitted]
        assert int(pos.cpu()[0]) == base + emitted and int(tok.cpu()[0]) == truth[emitted - 1]
        assert list(to_u32(outs["argmax"])) == [O.greedy(x[j]) for j in range(M)]
        for j in range(M):
            t8 = O.top_tokens(x[j], 8)
            assert list(to_u32(outs["top8_ids"])[j]) == list(t8)
            assert np.array_equal(outs["top8_vals"][j].cpu().numpy().view(np.uint32), x[j][t8].view(np.uint32))
            assert list(to_u32(outs["top20_ids"])[j]) == list(O.top_tokens(x[j], 20))
    d.close()


# ---------------------------------------------------------------------------
# NonFinite z at tiny temperatures
# ---------------------------------------------------------------------------
def test_tiny_temperature_follows_the_reference_nonfinite_rule():
    rng = np.random.default_rng(5)
    V = 5000
    wide = (1e4 * rng.standard_normal(V)).astype(np.float32)      # (l - l0) / 1e-305 overflows
    narrow = (1e-3 * rng.standard_normal(V)).astype(np.float32)   # stays finite
    equal = np.full(V, 0.5, np.float32)
    rows = np.stack([wide, narrow, equal])
    d = DeviceSampler(3, V, extended_top_k=True)
    for k in (20, 0):
        q = SamplingParametersF64(temperature=1e-305, top_p=0.95, min_p=0.0, top_k=k, seed=4)
        d.set_params(q)
        out = d.sample(torch.from_numpy(rows).to(DEV), torch.tensor([1, 2, 3], device=DEV), row_status=True)
        with pytest.raises(NonFinite):
            d.sync()
        st = out["status"].cpu().tolist()
        p = O.params(1e-305, 0.95, k, 0.0, 4, GUMBEL, extension=True)
        for r in range(3):
            try:
                want = O.sample(rows[r], r + 1, p)
                assert st[r] == 0 and to_u32(out["ids"])[r, 0] == want, r
            except O.OracleError as e:
                assert e.status == O.ENONFINITE and st[r] == -2, r
        assert st[0] == -2 and st[2] == 0
    d.close()


# ---------------------------------------------------------------------------
# penalty history layout
# ---------------------------------------------------------------------------
def test_shared_history_and_history_longer_than_its_row():
    rng = np.random.default_rng(12)
    rows, V = 3, 4000
    x = (2 * rng.standard_normal((rows, V))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    hist = rng.integers(0, 100, 300).astype(np.int32)
    sp = SamplingParameters(temperature_milli=700, top_p_milli=900, seed=8, top_k=20,
                            repetition_penalty=1.3, presence_penalty=0.7, frequency_penalty=0.2)
    d = DeviceSampler(rows, V)
    d.set_params(sp)
    out = d.sample(xt, torch.tensor([5, 6, 7], device=DEV), top20=True,
                   history=torch.from_numpy(hist).to(DEV))
    d.sync()
    for r in range(rows):
        y = O.apply_penalties(x[r], hist, 1.3, 0.7, 0.2)
        assert to_u32(out["ids"])[r, 0] == oracle_select(y, 5 + r, sp)
        assert list(to_u32(out["top20_ids"])[r]) == list(O.top_tokens(y, 20))
    h2 = torch.from_numpy(rng.integers(0, 100, (rows, 50)).astype(np.int32)).to(DEV)
    out = d.sample(xt, torch.tensor([5, 6, 7], device=DEV), history=h2, row_status=True,
                   history_len=torch.tensor([50, 51, 10], dtype=torch.int32, device=DEV))
    with pytest.raises(InvalidInput):
        d.sync()
    assert out["status"].cpu().tolist() == [0, -1, 0]
    with pytest.raises(InvalidInput):
        d.sample(xt, torch.tensor([5, 6, 7], device=DEV), history=h2[:2])
    d.close()
