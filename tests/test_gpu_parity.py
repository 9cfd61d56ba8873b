"""Parity of the HIP sampler (through the C ABI) with the CPU oracle.

Bit-exact: sampled token ids, argmax, top-8 / top-20 / top-N id lists and
values, verification counts. Logprobs and NLL: 1e-5 relative (absolute floor
1e-10). Inputs are seeded and identical for both sides.
"""
import math

import numpy as np
import pytest
import torch

import yskn_oracle as O
from gpu_helpers import assert_logprobs_close, oracle_params, oracle_select, pmap, to_u32

pytestmark = pytest.mark.gpu

from yskn_smp import (GUMBEL, INVERSE_CUMULATIVE, DeviceSampler, InvalidInput, NonFinite,
                      SamplingParameters)
from yskn_smp import synth

DEV = "cuda"


def _run(dev, x, positions, **kw):
    out = dev.sample(x, torch.as_tensor(positions, dtype=torch.int64, device=DEV), **kw)
    dev.sync()
    return out


@pytest.fixture(scope="module")
def small_dev():
    d = DeviceSampler(64, 70_000, extended_top_k=True)
    yield d
    d.close()


# ---------------------------------------------------------------------------
# edge cases on small rows
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("V", [1, 2, 3, 5, 8, 17, 64, 1000, 16383, 16384, 16385, 40000, 65537])
def test_small_rows_all_outputs(small_dev, V):
    rng = np.random.default_rng(V)
    rows = 6
    x = (2.0 * rng.standard_normal((rows, V))).astype(np.float32)
    x[1] = np.round(x[1])                      # heavy ties
    x[2, : V // 2] = -0.0                      # signed zeros
    x[2, V // 2:] = 0.0
    xt = torch.from_numpy(x).to(DEV)
    k = min(20, V)
    for version in (GUMBEL, INVERSE_CUMULATIVE):
        sp = SamplingParameters(temperature_milli=900, top_p_milli=950, top_k=k, seed=99 + V,
                                version=version)
        small_dev.set_params(sp)
        pos = rng.integers(0, 2 ** 40, rows)
        out = _run(small_dev, xt, pos, argmax=True, top8=V >= 8, top20=V >= 20)
        ids = to_u32(out["ids"]).reshape(-1)
        ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sp), range(rows))
        assert list(ids) == ref
        am = to_u32(out["argmax"])
        assert list(am) == [O.greedy(x[r]) for r in range(rows)]
        for n in (8, 20):
            if V >= n:
                got = to_u32(out[f"top{n}_ids"])
                vals = out[f"top{n}_vals"].cpu().numpy()
                for r in range(rows):
                    tt = O.top_tokens(x[r], n)
                    assert list(got[r]) == list(tt)
                    assert np.array_equal(vals[r].view(np.uint32), x[r][tt].view(np.uint32))


def test_all_equal_row_uses_smallest_ids(small_dev):
    V = 50_000
    x = torch.full((2, V), 0.25, dtype=torch.float32, device=DEV)
    sp = SamplingParameters(top_k=20, seed=3)
    small_dev.set_params(sp)
    out = _run(small_dev, x, [5, 6], argmax=True, top20=True)
    assert list(to_u32(out["argmax"])) == [0, 0]
    assert list(to_u32(out["top20_ids"])[0]) == list(range(20))
    xn = x.cpu().numpy()
    assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(xn[0], 5, sp),
                                                    oracle_select(xn[1], 6, sp)]


@pytest.mark.parametrize("bad", [math.nan, math.inf, -math.inf])
def test_nonfinite_rows_are_rejected(small_dev, bad):
    x = torch.zeros((3, 1000), dtype=torch.float32, device=DEV)
    x[1, 500] = bad
    small_dev.set_params(SamplingParameters())
    out = small_dev.sample(x, torch.tensor([1, 2, 3], device=DEV), row_status=True)
    with pytest.raises(NonFinite):
        small_dev.sync()
    st = out["status"].cpu().tolist()
    assert st == [0, -2, 0]
    assert to_u32(out["ids"])[1, 0] == 0xFFFFFFFF


def test_parameter_validation_mirrors_reference():
    d = DeviceSampler(1, 100)
    for kw in [dict(top_k=0), dict(top_k=21), dict(top_p_milli=0), dict(top_p_milli=1001),
               dict(min_p_milli=1001), dict(version=4)]:
        with pytest.raises(InvalidInput):
            d.set_params(SamplingParameters(**kw))
    x = torch.zeros((1, 10), dtype=torch.float32, device=DEV)
    d.set_params(SamplingParameters(top_k=20))
    with pytest.raises(InvalidInput):      # top_k > V
        d.sample(x, torch.tensor([0], device=DEV))
    with pytest.raises(InvalidInput):      # V over the handle's limit
        d.sample(torch.zeros((1, 101), device=DEV), torch.tensor([0], device=DEV))
    d.close()


def test_misaligned_rows_use_the_scalar_path(small_dev):
    rng = np.random.default_rng(77)
    V, ld = 33_333, 33_335
    base = torch.from_numpy((1.5 * rng.standard_normal(4 * ld + 1)).astype(np.float32)).to(DEV)
    x = base[1:1 + 4 * ld].view(4, ld)[:, :V]     # odd offset and stride
    sp = SamplingParameters(top_k=20, seed=5)
    small_dev.set_params(sp)
    out = _run(small_dev, x, [1, 2, 3, 4], top20=True)
    xn = x.cpu().numpy()
    assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(xn[r], r + 1, sp) for r in range(4)]
    for r in range(4):
        assert list(to_u32(out["top20_ids"])[r]) == list(O.top_tokens(xn[r], 20))


def test_many_draws_from_one_row(small_dev):
    rng = np.random.default_rng(1)
    x = (2.5 * rng.standard_normal((1, 30_000))).astype(np.float32)
    sp = SamplingParameters(top_k=20, seed=11)
    small_dev.set_params(sp)
    pos = np.arange(300, 812)
    out = _run(small_dev, torch.from_numpy(x).to(DEV), pos.reshape(1, -1))
    ref = O.sample_positions(x[0], pos.astype(np.uint64), oracle_params(sp))
    assert np.array_equal(to_u32(out["ids"]).reshape(-1), ref)


@pytest.mark.parametrize("T,tp,mp,k", [(1, 1000, 0, 20), (5000, 1000, 0, 20), (300, 500, 100, 7),
                                       (1000, 1000, 1000, 20), (2000, 10, 0, 20)])
def test_parameter_corners(small_dev, T, tp, mp, k):
    rng = np.random.default_rng(T + tp)
    x = (3.0 * rng.standard_normal((8, 20_000))).astype(np.float32)
    for version in (GUMBEL, INVERSE_CUMULATIVE):
        sp = SamplingParameters(temperature_milli=T, top_p_milli=tp, min_p_milli=mp, top_k=k,
                                seed=1234, version=version)
        small_dev.set_params(sp)
        pos = np.arange(8) * 1000 + 7
        out = _run(small_dev, torch.from_numpy(x).to(DEV), pos)
        assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(x[r], int(pos[r]), sp)
                                                        for r in range(8)]


@pytest.mark.parametrize("k", [0, 21, 64, 65, 500, 20_000])
def test_extended_top_k(small_dev, k):
    rng = np.random.default_rng(k + 1)
    x = (rng.standard_normal((6, 20_000)) * np.array([[0.5], [1], [2], [4], [8], [30]])).astype(np.float32)
    for version in (GUMBEL, INVERSE_CUMULATIVE):
        sp = SamplingParameters(temperature_milli=800, top_p_milli=930, min_p_milli=0, top_k=k,
                                seed=77, version=version)
        small_dev.set_params(sp)
        pos = np.arange(6) + 50
        out = _run(small_dev, torch.from_numpy(x).to(DEV), pos)
        ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sp, extension=True), range(6))
        assert list(to_u32(out["ids"]).reshape(-1)) == ref


def test_binary64_parameters(small_dev):
    """yskn_smp_set_params_f64: the Rust SamplingParameters fields as they are.
    Values that are thousandths give the thousandths path's ids; arbitrary
    binary64 values match the oracle run with the same binary64 values."""
    from yskn_smp import SamplingParametersF64
    rng = np.random.default_rng(64)
    x = (2.5 * rng.standard_normal((8, 30_000))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    pos = rng.integers(0, 10 ** 6, 8)
    for version in (GUMBEL, INVERSE_CUMULATIVE):
        sp = SamplingParameters(temperature_milli=700, top_p_milli=900, min_p_milli=50, top_k=20,
                                seed=99, version=version)
        small_dev.set_params(sp)
        a = to_u32(_run(small_dev, xt, pos)["ids"])
        small_dev.set_params(SamplingParametersF64(temperature=700 / 1000.0, top_p=900 / 1000.0,
                                                   min_p=50 / 1000.0, top_k=20, seed=99,
                                                   version=version))
        b = to_u32(_run(small_dev, xt, pos)["ids"])
        assert list(a) == list(b)
        odd = [SamplingParametersF64(temperature=0.3 + 0.1234567 * r, top_p=0.8 + 0.0246813 * r,
                                     min_p=0.0123457 * r, top_k=[1, 7, 20, 13][r % 4],
                                     seed=5000 + r, version=version, greedy=(r == 5))
               for r in range(8)]
        small_dev.set_params(odd)
        got = to_u32(_run(small_dev, xt, pos)["ids"])

        def ref(r):
            q = odd[r]
            if q.greedy:
                return O.greedy(x[r])
            return O.sample(x[r], int(pos[r]), O.params(q.temperature, q.top_p, q.top_k, q.min_p,
                                                        q.seed, q.version))
        assert list(got.reshape(-1)) == pmap(ref, range(8))


def test_per_row_parameters_and_greedy_rows(small_dev):
    rng = np.random.default_rng(9)
    rows = 12
    x = (2.0 * rng.standard_normal((rows, 25_000))).astype(np.float32)
    sps = [SamplingParameters(temperature_milli=(0 if r % 4 == 0 else 300 + 100 * r),
                              top_p_milli=800 + 15 * r, top_k=[1, 20, 50, 0][r % 4],
                              min_p_milli=5 * r, seed=1000 + r,
                              version=GUMBEL if r % 2 else INVERSE_CUMULATIVE) for r in range(rows)]
    small_dev.set_params(sps)
    pos = rng.integers(0, 10 ** 9, rows)
    out = _run(small_dev, torch.from_numpy(x).to(DEV), pos)
    ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sps[r], extension=True), range(rows))
    assert list(to_u32(out["ids"]).reshape(-1)) == ref


def test_bf16_rows(small_dev):
    rng = np.random.default_rng(10)
    x = torch.from_numpy((2 * rng.standard_normal((5, 30_001))).astype(np.float32)).to(torch.bfloat16)
    sp = SamplingParameters(temperature_milli=700, top_p_milli=900, min_p_milli=50, seed=4)
    small_dev.set_params(sp)
    out = _run(small_dev, x.to(DEV), [1, 2, 3, 4, 5], top20=True)
    xf = x.float().numpy()
    assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(xf[r], r + 1, sp) for r in range(5)]
    for r in range(5):
        assert list(to_u32(out["top20_ids"])[r]) == list(O.top_tokens(xf[r], 20))


def test_penalties_small(small_dev):
    rng = np.random.default_rng(12)
    V = 5000
    x = (2 * rng.standard_normal((3, V))).astype(np.float32)
    hist = rng.integers(0, 200, (3, 700)).astype(np.int32)   # concentrated history
    hl = np.array([700, 0, 333], np.int32)
    sp = SamplingParameters(temperature_milli=700, top_p_milli=900, min_p_milli=50, seed=8,
                            repetition_penalty=1.05, presence_penalty=0.5, frequency_penalty=0.3)
    small_dev.set_params(sp)
    out = _run(small_dev, torch.from_numpy(x).to(DEV), [10, 11, 12], top20=True,
               history=torch.from_numpy(hist).to(DEV), history_len=torch.from_numpy(hl).to(DEV))
    for r in range(3):
        y = O.apply_penalties(x[r], hist[r, :hl[r]], 1.05, 0.5, 0.3)
        assert to_u32(out["ids"])[r, 0] == oracle_select(y, 10 + r, sp)
        tt = O.top_tokens(y, 20)
        assert list(to_u32(out["top20_ids"])[r]) == list(tt)
        assert np.array_equal(out["top20_vals"][r].cpu().numpy().view(np.uint32), y[tt].view(np.uint32))


@pytest.mark.parametrize("V,count", [(5000, 65), (5000, 1000), (5000, 5000), (70_000, 4097), (70_000, 20_000)])
def test_top_tokens_beyond_64(small_dev, V, count):
    # counts above the waves' lists take the exact dense path: every id in
    # order, ties to the smaller id, raw values (the sign of zeros kept)
    rng = np.random.default_rng(count + V)
    x = (2 * rng.standard_normal((3, V))).astype(np.float32)
    x[1] = np.round(x[1])                                   # heavy ties
    x[2, : V // 2] = -0.0
    x[2, V // 2:] = 0.0
    x[2, 7] = 1.5
    xt = torch.from_numpy(x).to(DEV)
    ids, vals = small_dev.top_tokens(xt, count)
    small_dev.sync()
    got = to_u32(ids)
    gv = vals.cpu().numpy()
    for r in range(3):
        tt = O.top_tokens(x[r], count)
        assert np.array_equal(got[r], tt), r
        assert np.array_equal(gv[r].view(np.uint32), x[r][tt].view(np.uint32)), r
    with pytest.raises(InvalidInput):
        small_dev.top_tokens(xt, V + 1)


@pytest.mark.parametrize("n_lp,top_k", [(65, 20), (300, 0), (1000, 40)])
def test_logprobs_beyond_64_keep_the_draw(n_lp, top_k):
    rng = np.random.default_rng(n_lp)
    V, rows = 30_000, 4
    x = (rng.standard_normal((rows, V)) * np.array([[0.5], [1.0], [3.0], [8.0]])).astype(np.float32)
    sp = SamplingParameters(temperature_milli=900, top_p_milli=930, top_k=top_k, seed=4)
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sp)
    pos = np.arange(rows) + 11
    out = _run(d, torch.from_numpy(x).to(DEV), pos, n_logprobs=n_lp, top20=True)
    ids = to_u32(out["ids"]).reshape(-1)
    got_ids = to_u32(out["logprob_ids"])
    got_lp = out["logprobs"].cpu().numpy()
    for r in range(rows):
        assert ids[r] == oracle_select(x[r], int(pos[r]), sp, extension=True), r
        li, lv = O.top_logprobs(x[r], n_lp)
        assert list(got_ids[r]) == list(li), r
        assert_logprobs_close(got_lp[r], lv)
        assert list(to_u32(out["top20_ids"])[r]) == list(O.top_tokens(x[r], 20))
    d.close()


def test_penalties_across_vocabulary_windows():
    # the history's membership words are built 262,144 ids at a time: ids on
    # both sides of each window edge, the first and last id, one id repeated
    # thousands of times and a full 16,384-token history
    rng = np.random.default_rng(21)
    V, rows = 700_001, 3
    x = (2 * rng.standard_normal((rows, V))).astype(np.float32)
    edges = np.array([0, 31, 32, 262_143, 262_144, 262_145, 524_287, 524_288, V - 1], np.int64)
    hist = np.empty((rows, 16_384), np.int32)
    for r in range(rows):
        h = np.concatenate([np.repeat(edges, np.arange(1, len(edges) + 1) * (r + 1)),
                            np.full(5000, 400_000 + r),
                            rng.zipf(1.2, 16_384) % (V - 1000) + 1000])[:16_384]
        hist[r] = rng.permutation(h)
        x[r, edges] = 30.0 + rng.random(len(edges)).astype(np.float32)   # all in the top 20
    hl = np.array([16_384, 9_000, 16_384], np.int32)
    hist[2, 77] = V                                                      # invalid id
    sp = SamplingParameters(temperature_milli=900, top_p_milli=950, top_k=20, seed=3,
                            repetition_penalty=1.05, presence_penalty=0.5, frequency_penalty=0.3)
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sp)
    out = d.sample(torch.from_numpy(x).to(DEV), torch.tensor([[9], [10], [11]], device=DEV), top20=True,
                   row_status=True, history=torch.from_numpy(hist).to(DEV),
                   history_len=torch.from_numpy(hl).to(DEV))
    with pytest.raises(InvalidInput):
        d.sync()
    assert out["status"].cpu().tolist() == [0, 0, -1]
    for r in range(2):
        y = O.apply_penalties(x[r], hist[r, :hl[r]], 1.05, 0.5, 0.3)
        assert to_u32(out["ids"])[r, 0] == oracle_select(y, 9 + r, sp)
        tt = O.top_tokens(y, 20)
        assert set(edges) <= set(tt)
        assert list(to_u32(out["top20_ids"])[r]) == list(tt)
        assert np.array_equal(out["top20_vals"][r].cpu().numpy().view(np.uint32), y[tt].view(np.uint32))
    d.close()


def test_top_tokens_and_nll_apis(small_dev):
    rng = np.random.default_rng(13)
    x = (3 * rng.standard_normal((7, 12_345))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    for count in (1, 8, 33, 64):
        ids, vals = small_dev.top_tokens(xt, count)
        small_dev.sync()
        for r in range(7):
            assert list(to_u32(ids)[r]) == list(O.top_tokens(x[r], count))
    tg = rng.integers(0, 12_345, 7)
    nll = small_dev.nll(xt, torch.from_numpy(tg).to(DEV))
    small_dev.sync()
    assert_logprobs_close(nll.cpu().numpy(), [O.nll(x[r], int(tg[r])) for r in range(7)])


def test_dense_path_matches_compact_path():
    rng = np.random.default_rng(14)
    V = 40_000
    x = (rng.standard_normal((6, V)) * np.array([[0.3], [1], [2], [5], [20], [100]])).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    a = DeviceSampler(6, V, extended_top_k=True)
    b = DeviceSampler(6, V, extended_top_k=True, force_dense=True)
    for k in (20, 0):
        sp = SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=k, seed=21)
        a.set_params(sp)
        b.set_params(sp)
        pos = np.arange(6) + 3
        oa = _run(a, xt, pos, argmax=True, top20=True, n_logprobs=20)
        ob = _run(b, xt, pos, argmax=True, top20=True, n_logprobs=20)
        for key in ("ids", "argmax", "top20_ids", "logprob_ids"):
            assert torch.equal(oa[key], ob[key]), key
        ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sp, extension=True), range(6))
        assert list(to_u32(ob["ids"]).reshape(-1)) == ref
    a.close()
    b.close()


def _dense_rows(rng, rows, V, dtype=np.float32):
    scale = np.array([0.5, 1.0, 2.0, 3.0])[np.arange(rows) % 4].reshape(-1, 1)
    return (scale * rng.standard_normal((rows, V))).astype(dtype)


def _dense_params(rows, seed):
    """Top-k disabled; temperatures, top-p and min-p that put the cut before
    and after min-p's, at top-p 1 (no margin: the sorting path) and at
    min-p 0."""
    Ts = [300, 700, 1000, 1500]
    tps = [800, 900, 950, 990, 1000]
    mps = [0, 1, 20, 100, 0, 3]
    return [SamplingParameters(temperature_milli=Ts[r % 4], top_p_milli=tps[r % 5], min_p_milli=mps[r % 6],
                               top_k=0, seed=seed + r) for r in range(rows)]


def test_certified_dense_tail_matches_the_oracle_and_the_sorting_path():
    """Rows with tens of thousands of candidates (top-k disabled): the cut is
    certified from bucket sums without sorting the row, or the row falls back
    to the sort. Both give the oracle's ids; the forced sorting path agrees."""
    rng = np.random.default_rng(41)
    rows, V = 24, 50_000
    x = _dense_rows(rng, rows, V)
    sps = _dense_params(rows, 900)
    a = DeviceSampler(rows, V, extended_top_k=True)
    b = DeviceSampler(rows, V, extended_top_k=True, force_dense=True)
    a.set_params(sps)
    b.set_params(sps)
    pos = np.arange(rows) + 123
    xt = torch.from_numpy(x).to(DEV)
    oa = _run(a, xt, pos, argmax=True, top20=True, n_logprobs=8)
    ob = _run(b, xt, pos, argmax=True, top20=True, n_logprobs=8)
    ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sps[r], extension=True), range(rows))
    assert list(to_u32(oa["ids"]).reshape(-1)) == ref
    for key in ("ids", "argmax", "top20_ids", "logprob_ids"):
        assert torch.equal(oa[key], ob[key]), key
    st = a.stats()
    assert st["dense_rows"] == rows
    assert 0 < st["certified_rows"] < rows  # top-p 1 at min-p 0 has no margin: sorted
    a.close()
    b.close()


def test_certified_dense_tail_several_draws_and_ties():
    """Several positions per row, and bf16 rows whose values repeat (the cut
    falls inside a run of equal values: ids in ascending order decide)."""
    rng = np.random.default_rng(42)
    rows, V, nd = 8, 60_000, 5
    x = _dense_rows(rng, rows, V)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    xf = xb.float().numpy()
    sps = _dense_params(rows, 300)
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sps)
    pos = (np.arange(rows * nd).reshape(rows, nd) * 7 + 11).astype(np.int64)
    out = _run(d, xb.to(DEV), pos)
    got = to_u32(out["ids"]).reshape(rows, nd)
    for r in range(rows):
        ref = O.sample_positions(xf[r], pos[r].astype(np.uint64), oracle_params(sps[r], True))
        assert list(got[r]) == list(ref), r
    assert d.stats()["certified_rows"] > 0
    d.close()


def test_certified_dense_tail_with_penalties_and_coarse_values():
    """Penalised rows, and rows of a few distinct values (a cut bucket too
    large to collect: the sorting path)."""
    rng = np.random.default_rng(43)
    rows, V = 6, 40_000
    x = _dense_rows(rng, rows, V)
    x[3:] = np.round(x[3:] * 4) / 4
    hist = rng.integers(0, V, (rows, 3000)).astype(np.int32)
    sps = _dense_params(rows, 50)
    sps = [SamplingParameters(temperature_milli=s.temperature_milli, top_p_milli=s.top_p_milli,
                              min_p_milli=s.min_p_milli, top_k=0, seed=s.seed, repetition_penalty=1.1,
                              presence_penalty=0.2, frequency_penalty=0.05) for s in sps]
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sps)
    pos = np.arange(rows) + 5
    out = _run(d, torch.from_numpy(x).to(DEV), pos, history=torch.from_numpy(hist).to(DEV))
    for r in range(rows):
        y = O.apply_penalties(x[r], hist[r], 1.1, 0.2, 0.05)
        assert to_u32(out["ids"])[r, 0] == oracle_select(y, int(pos[r]), sps[r], extension=True), r
    d.close()


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_certified_dense_tail_randomised(seed):
    """Many dense rows with random shapes and parameters (scale, temperature,
    top-p including 1, min-p including 0, version 2 rows that take the
    sorting path, heavy tails, repeated values): every id is the oracle's,
    and most rows are served by the certified tail."""
    rng = np.random.default_rng(1000 + seed)
    rows, V = 40, 30_000
    x = np.empty((rows, V), np.float32)
    for r in range(rows):
        kind = r % 4
        sc = rng.uniform(0.3, 4.0)
        if kind == 0:
            x[r] = sc * rng.standard_normal(V)
        elif kind == 1:
            x[r] = sc * rng.standard_t(3, V)
        elif kind == 2:
            x[r] = np.round(sc * rng.standard_normal(V) * 64) / 64  # repeated values
        else:
            x[r] = sc * rng.uniform(-1, 1, V)
    sps = [SamplingParameters(temperature_milli=int(rng.integers(200, 3000)),
                              top_p_milli=int(rng.choice([500, 800, 900, 950, 990, 999, 1000])),
                              min_p_milli=int(rng.choice([0, 0, 1, 5, 50, 200])), top_k=0,
                              seed=int(rng.integers(0, 2**62)),
                              version=INVERSE_CUMULATIVE if r % 10 == 9 else GUMBEL) for r in range(rows)]
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sps)
    pos = rng.integers(0, 2**40, rows)
    out = _run(d, torch.from_numpy(x).to(DEV), pos, argmax=True, top8=True)
    ref = pmap(lambda r: oracle_select(x[r], int(pos[r]), sps[r], extension=True), range(rows))
    got = to_u32(out["ids"]).reshape(-1)
    bad = [r for r in range(rows) if got[r] != ref[r]]
    assert not bad, [(r, int(got[r]), ref[r], sps[r]) for r in bad]
    for r in range(rows):
        assert list(to_u32(out["top8_ids"])[r]) == list(O.top_tokens(x[r], 8)), r
    st = d.stats()
    print("path counters", st, flush=True)
    assert st["certified_rows"] >= rows // 2
    d.close()


def test_certified_dense_tail_in_verify():
    """Verify rows with top-k disabled: the certified tail draws the target
    row's token, the accept rule sees the oracle's."""
    rng = np.random.default_rng(77)
    M, V = 6, 40_000
    tgt = (1.5 * rng.standard_normal((M, V))).astype(np.float32)
    sp = SamplingParameters(temperature_milli=900, top_p_milli=930, min_p_milli=0, top_k=0, seed=0xC0FFEE)
    base = 5_000
    drafts = [oracle_select(tgt[j], base + j + 1, sp, extension=True) for j in range(M - 1)]
    d = DeviceSampler(M, V, extended_top_k=True)
    d.set_params(sp)
    ids, res, _keep = d.verify(torch.from_numpy(tgt).to(DEV), torch.tensor(drafts, device=DEV),
                               torch.tensor([base], device=DEV))
    d.sync()
    sel, em, acc, stop = O.verify(tgt, drafts, base, oracle_params(sp, True))
    r = res.cpu().numpy().astype(np.int64)
    assert (r[0], r[1], r[2]) == (acc, em, sel[-1])
    assert list(to_u32(ids)[:em]) == list(sel)
    assert d.stats()["certified_rows"] > 0
    d.close()


def test_large_launches_with_other_features():
    """Launches of 192 rows or more that go beyond plain sampling (several
    draws, logprob lists longer than 64, device positions, NLL, top lists)
    run the general kernel form; plain ones the large form. Both match the
    oracle."""
    rng = np.random.default_rng(55)
    rows, V = 200, 6_000
    x = (2.0 * rng.standard_normal((rows, V))).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    sp = SamplingParameters(temperature_milli=900, top_p_milli=950, top_k=0, seed=123)
    d = DeviceSampler(rows, V, extended_top_k=True)
    d.set_params(sp)
    # plain sampling with top-20 and 20 logprobs (the large form)
    pos = np.arange(rows) + 7
    out = _run(d, xt, pos, top20=True, n_logprobs=20)
    assert list(to_u32(out["ids"]).reshape(-1)) == pmap(
        lambda r: oracle_select(x[r], int(pos[r]), sp, extension=True), range(rows))
    # several draws per row
    pos3 = (np.arange(rows * 3).reshape(rows, 3) * 11 + 5).astype(np.int64)
    out = _run(d, xt, pos3)
    got = to_u32(out["ids"]).reshape(rows, 3)
    for r in range(0, rows, 17):
        assert list(got[r]) == list(O.sample_positions(x[r], pos3[r].astype(np.uint64), oracle_params(sp, True)))
    # 100 logprobs per row (lists past 64)
    out = _run(d, xt, pos, n_logprobs=100)
    for r in range(0, rows, 23):
        ids, lps = O.top_logprobs(x[r], 100)
        assert list(to_u32(out["logprob_ids"])[r]) == list(ids)
        assert_logprobs_close(out["logprobs"][r].cpu().numpy(), lps)
    assert list(to_u32(out["ids"]).reshape(-1))[:5] == [oracle_select(x[r], int(pos[r]), sp, extension=True)
                                                        for r in range(5)]
    # device positions: *base + row + 1
    base = torch.tensor([1000], dtype=torch.int64, device=DEV)
    out = d.sample_at(xt, base)
    d.sync()
    assert list(to_u32(out["ids"]).reshape(-1))[:40] == [oracle_select(x[r], 1000 + r + 1, sp, extension=True)
                                                         for r in range(40)]
    # NLL over the same launch shape
    tg = rng.integers(0, V, rows)
    nll = d.nll(xt, torch.from_numpy(tg).to(DEV))
    d.sync()
    assert_logprobs_close(nll.cpu().numpy(), [O.nll(x[r], int(tg[r])) for r in range(rows)])
    d.close()


@pytest.mark.parametrize("case", range(30))
def test_random_feature_combinations(case):
    """Deterministic random combinations of row shape (padded, ragged),
    element type, value distribution, per-row or shared parameters (top-k 1
    to disabled, both versions, top-p, min-p, temperature), draws per row,
    logprob and top lists, and penalties: ids, argmax, top-8 and logprob ids
    against the oracle."""
    rng = np.random.default_rng(5000 + case)
    rows = int(rng.integers(1, 25))
    V = int(rng.choice([1000, 4097, 20_000, 33_333, 60_000]))
    pad = int(rng.choice([0, 3, 16]))
    bf16 = bool(rng.random() < 0.3)
    kind = int(rng.integers(0, 3))
    sc = float(rng.uniform(0.5, 4.0))
    if kind == 0:
        x = sc * rng.standard_normal((rows, V))
    elif kind == 1:
        x = sc * rng.standard_t(3, (rows, V))
    else:
        x = np.round(sc * rng.standard_normal((rows, V)) * 16) / 16
    x = x.astype(np.float32)
    full = torch.zeros((rows, V + pad), dtype=torch.float32)
    full[:, :V] = torch.from_numpy(x)
    if bf16:
        full = full.to(torch.bfloat16)
        x = full[:, :V].float().numpy()
    xt = full.to(DEV)[:, :V]
    def params(r):
        return SamplingParameters(temperature_milli=int(rng.integers(100, 3000)),
                                  top_p_milli=int(rng.choice([300, 800, 950, 990, 1000])),
                                  min_p_milli=int(rng.choice([0, 0, 10, 100])),
                                  top_k=int(rng.choice([1, 5, 20, 64, 65, 300, 0])),
                                  seed=int(rng.integers(0, 2**62)),
                                  version=GUMBEL if rng.random() < 0.7 else INVERSE_CUMULATIVE)
    shared = bool(rng.random() < 0.5)
    sps = [params(0)] * rows if shared else [params(r) for r in range(rows)]
    nd = int(rng.choice([1, 1, 3]))
    n_lp = int(rng.choice([0, 8, 70]))
    pen = bool(rng.random() < 0.3)
    d = DeviceSampler(rows, V + pad, extended_top_k=True)
    d.set_params(sps[0] if shared else sps)
    pos = rng.integers(0, 2**40, (rows, nd)).astype(np.int64)
    kw = dict(argmax=True, top8=True, n_logprobs=n_lp)
    y = x
    if pen:
        hist = rng.integers(0, V, (rows, 1500)).astype(np.int32)
        hl = rng.integers(0, 1501, rows).astype(np.int32)
        sps = [SamplingParameters(temperature_milli=q.temperature_milli, top_p_milli=q.top_p_milli,
                                  min_p_milli=q.min_p_milli, top_k=q.top_k, seed=q.seed, version=q.version,
                                  repetition_penalty=1.1, presence_penalty=0.3, frequency_penalty=0.05)
               for q in sps]
        d.set_params(sps[0] if shared else sps)
        kw.update(history=torch.from_numpy(hist).to(DEV), history_len=torch.from_numpy(hl).to(DEV))
        y = np.stack([O.apply_penalties(x[r], hist[r, :hl[r]], 1.1, 0.3, 0.05) for r in range(rows)])
    out = _run(d, xt, pos, **kw)
    got = to_u32(out["ids"]).reshape(rows, nd)
    ref = pmap(lambda r: list(O.sample_positions(y[r], pos[r].astype(np.uint64), oracle_params(sps[r], True))),
               range(rows))
    for r in range(rows):
        assert list(got[r]) == ref[r], (case, r, sps[r])
        assert int(to_u32(out["argmax"])[r]) == O.greedy(y[r]), (case, r)
        assert list(to_u32(out["top8_ids"])[r]) == list(O.top_tokens(y[r], 8)), (case, r)
        if n_lp:
            assert list(to_u32(out["logprob_ids"])[r]) == list(O.top_logprobs(y[r], n_lp)[0]), (case, r)
    d.close()


@pytest.mark.parametrize("case", range(20))
def test_random_verify(case):
    """Deterministic random verify calls: row count, vocabulary, parameters
    (top-k 1 to disabled, both versions, min-p), drafts right up to a random
    depth then wrong or right to the end, EOS ids drawn from the selections:
    accepted, emitted, token and EOS flag against the oracle's accept loop."""
    rng = np.random.default_rng(7000 + case)
    M = int(rng.integers(1, 13))
    V = int(rng.choice([2000, 30_001, 70_000]))
    x = (float(rng.uniform(0.5, 3.0)) * rng.standard_normal((M, V))).astype(np.float32)
    sp = SamplingParameters(temperature_milli=int(rng.integers(200, 2000)),
                            top_p_milli=int(rng.choice([800, 950, 1000])),
                            min_p_milli=int(rng.choice([0, 20])),
                            top_k=int(rng.choice([1, 20, 64, 500, 0])), seed=int(rng.integers(0, 2**62)),
                            version=GUMBEL if rng.random() < 0.7 else INVERSE_CUMULATIVE)
    base = int(rng.integers(0, 2**40))
    sel = [oracle_select(x[j], base + j + 1, sp, extension=True) for j in range(M)]
    depth = int(rng.integers(0, M))
    drafts = [sel[j] if j < depth or rng.random() < 0.3 else (sel[j] + 1) % V for j in range(M - 1)]
    eos = [sel[int(rng.integers(0, M))]] if rng.random() < 0.3 else []
    d = DeviceSampler(M, V, extended_top_k=True)
    d.set_params(sp)
    dt = torch.tensor(drafts if drafts else [0], dtype=torch.int32, device=DEV)
    ids, res, _keep = d.verify(torch.from_numpy(x).to(DEV), dt, torch.tensor([base], device=DEV), eos)
    d.sync()
    osel, em, acc, stop = O.verify(x, drafts, base, oracle_params(sp, True), eos)
    r = res.cpu().numpy().astype(np.int64)
    assert (int(r[0]), int(r[1]), int(r[3])) == (acc, em, int(stop)), (case, M, depth)
    assert int(r[2]) == int(osel[-1]), case
    assert list(to_u32(ids)[:em]) == list(osel), case
    d.close()


# ---------------------------------------------------------------------------
# the five workloads at full size
# ---------------------------------------------------------------------------
def test_single_row_1024_draws():
    x = synth.single_row(DEV)
    d = DeviceSampler(1, synth.V_SMALL)
    sp = SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, min_p_milli=0, seed=0)
    d.set_params(sp)
    pos = np.arange(1024)
    out = _run(d, x, pos.reshape(1, -1), argmax=True, top20=True)
    xn = x.cpu().numpy()[0]
    assert to_u32(out["argmax"])[0] == O.greedy(xn)
    ref = O.sample_positions(xn, pos.astype(np.uint64), oracle_params(sp))
    assert np.array_equal(to_u32(out["ids"]).reshape(-1), ref)
    assert list(to_u32(out["top20_ids"])[0]) == list(O.top_tokens(xn, 20))
    d.close()


@pytest.mark.parametrize("M", [8, 9])
def test_spec_verify(M):
    tgt, drf = synth.spec_verify(M, DEV)
    sp = SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, seed=0x5EC)
    base = 10_000
    drn, tgn = drf.cpu().numpy(), tgt.cpu().numpy()
    drafts = [oracle_select(drn[j], base + j + 1, sp) for j in range(M - 1)]
    d = DeviceSampler(M, synth.V_LARGE)
    d.set_params(sp)
    ids, res, _keep = d.verify(tgt, torch.tensor(drafts, device=DEV), torch.tensor([base], device=DEV))
    d.sync()
    sel, em, acc, stop = O.verify(tgn, drafts, base, oracle_params(sp))
    r = res.cpu().numpy().astype(np.int64)
    assert (r[0], r[1], r[3]) == (acc, em, int(stop))
    assert r[2] == sel[-1]
    assert list(to_u32(ids)[:em]) == list(sel)
    # a wrong draft at depth 2 stops acceptance there
    bad = list(drafts)
    bad[2] = (bad[2] + 1) % synth.V_LARGE
    ids, res, _keep = d.verify(tgt, torch.tensor(bad, device=DEV), torch.tensor([base], device=DEV))
    d.sync()
    sel, em, acc, stop = O.verify(tgn, bad, base, oracle_params(sp))
    r = res.cpu().numpy().astype(np.int64)
    assert (r[0], r[1], r[2]) == (acc, em, sel[-1])
    d.close()


def test_penalties_workload():
    x, hist = synth.penalties(DEV)
    sp = SamplingParameters(temperature_milli=700, top_p_milli=900, min_p_milli=50, top_k=20,
                            seed=31, repetition_penalty=1.05, presence_penalty=0.5,
                            frequency_penalty=0.3)
    d = DeviceSampler(1, synth.V_LARGE)
    d.set_params(sp)
    pos = np.arange(1)
    out = _run(d, x, pos, top20=True, history=hist.reshape(1, -1))
    xf = x.float().cpu().numpy()[0]
    y = O.apply_penalties(xf, hist.cpu().numpy(), 1.05, 0.5, 0.3)
    assert to_u32(out["ids"])[0, 0] == oracle_select(y, 0, sp)
    assert list(to_u32(out["top20_ids"])[0]) == list(O.top_tokens(y, 20))
    d.close()


def test_batched_heterogeneous():
    x = synth.batched(64, DEV)
    pr = synth.batched_params(64)
    sps = [SamplingParameters(temperature_milli=p["temperature_milli"], top_p_milli=p["top_p_milli"],
                              min_p_milli=p["min_p_milli"], top_k=p["top_k"], seed=p["seed"])
           for p in pr]
    pos = np.array([p["position"] for p in pr])
    d = DeviceSampler(64, synth.V_LARGE, extended_top_k=True)
    d.set_params(sps)
    out = _run(d, x, pos, argmax=True)
    xn = x.cpu().numpy()
    ref = pmap(lambda r: oracle_select(xn[r], int(pos[r]), sps[r], extension=True), range(64))
    assert list(to_u32(out["ids"]).reshape(-1)) == ref
    assert list(to_u32(out["argmax"])) == [int(np.argmax(xn[r])) for r in range(64)]
    st = d.stats()
    print("path counters", st, flush=True)
    assert st["dense_rows"] == 16 and st["certified_rows"] == 16  # the top-k-disabled rows
    d.close()


def test_large_batch_top_p_with_logprobs():
    rows = 256
    x = synth.large_batch(rows, DEV)
    seeds = synth.large_batch_seeds(rows)
    sps = [SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=0, seed=s) for s in seeds]
    d = DeviceSampler(rows, synth.V_LARGE, extended_top_k=True)
    d.set_params(sps)
    pos = np.arange(rows) + 1
    out = _run(d, x, pos, n_logprobs=20)
    xn = x.cpu().numpy()
    ref = pmap(lambda r: oracle_select(xn[r], int(pos[r]), sps[r], extension=True), range(rows))
    assert list(to_u32(out["ids"]).reshape(-1)) == ref
    lps = pmap(lambda r: O.top_logprobs(xn[r], 20), range(rows))
    got_ids = to_u32(out["logprob_ids"])
    got_lp = out["logprobs"].cpu().numpy()
    for r in range(rows):
        assert list(got_ids[r]) == list(lps[r][0])
        assert_logprobs_close(got_lp[r], lps[r][1])
    d.close()
