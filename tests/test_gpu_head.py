"""The output head's epilogue fused into the sampler (yskn_smp_sample_head),
through the C ABI, against the oracle's restatement of the head scale
restoration (spec 06 section 2; compressed_linear.rs:329-340;
residual_norm_mlp.rs:37-46 with the portable rsqrt) followed by the oracle
sampler: sampled ids, argmax and top lists bit for bit, logprobs within 1e-5
relative, the written logits bit for bit, cleared accumulators, and the
reference's NonFinite rules for the inverse RMS and the logits."""
import numpy as np
import pytest
import torch

import yskn_oracle as O
from gpu_helpers import assert_logprobs_close, oracle_params, oracle_select, pmap, to_u32
from yskn_smp import DeviceSampler, NonFinite, InvalidInput, SamplingParameters

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _head_inputs(rows, V, seed, nblk=10):
    rng = np.random.default_rng(seed)
    acc = (rng.standard_normal((rows, V)) * 2.0**34).astype(np.int64)
    # conversion ties and exactly representable values
    acc[:, 0] = 2**24 + 1
    acc[:, 1] = -(2**24 + 3)
    acc[:, 2] = 2**53 + 2**29
    us = (rng.uniform(0.9, 1.1, rows) * 2.0**-33).astype(np.float32)
    sums = np.abs(rng.standard_normal((rows, nblk)) * 500.0).astype(np.float32)
    tau = rng.uniform(0.5, 1.5, V).astype(np.float32)
    return acc, us, sums, tau


def _oracle_logits(acc, us, sums, tau, width=5120.0, eps=1e-6):
    out = []
    for r in range(acc.shape[0]):
        ir = O.inverse_rms(sums[r], width, eps)
        out.append(O.head_logits(acc[r], tau, float(us[r]), ir))
    return np.stack(out)


def test_head_rows_with_top_k_disabled_take_the_certified_tail():
    """Flat head rows with top-k disabled: every value is relevant, so the
    finishing block re-forms the logits from the accumulators in its passes
    over the row (certified tail). Ids, argmax and top-8 against the oracle."""
    rows, V = 4, 60_000
    acc, us, sums, tau = _head_inputs(rows, V, 99)
    acc[:, :3] = acc[:, 3:6]  # no planted extreme values: a flat row
    x = _oracle_logits(acc, us, sums, tau)
    d = DeviceSampler(rows, V, extended_top_k=True)
    sp = SamplingParameters(temperature_milli=1200, top_p_milli=920, min_p_milli=0, top_k=0, seed=5)
    d.set_params(sp)
    pos = np.arange(rows) * 5 + 3
    t = lambda a: torch.from_numpy(a).to(DEV)
    out = d.sample_head(t(acc), t(us), t(sums), t(tau), torch.tensor(pos, device=DEV), argmax=True, top8=True)
    d.sync()
    assert list(to_u32(out["ids"]).reshape(-1)) == pmap(
        lambda r: oracle_select(x[r], int(pos[r]), sp, extension=True), range(rows))
    assert list(to_u32(out["argmax"])) == [O.greedy(x[r]) for r in range(rows)]
    for r in range(rows):
        assert list(to_u32(out["top8_ids"])[r]) == list(O.top_tokens(x[r], 8))
    assert d.stats()["certified_rows"] > 0
    d.close()


@pytest.mark.parametrize("rows,V", [(1, 151_936), (3, 1537), (8, 248_320), (16, 40_001)])
def test_head_sampling_matches_the_oracle(rows, V):
    acc, us, sums, tau = _head_inputs(rows, V, rows * 7 + V)
    x = _oracle_logits(acc, us, sums, tau)
    d = DeviceSampler(rows, V)
    sp = SamplingParameters(temperature_milli=900, top_p_milli=950, top_k=20, seed=rows)
    d.set_params(sp)
    pos = np.arange(rows) * 3 + 11
    t = lambda a: torch.from_numpy(a).to(DEV)
    out = d.sample_head(t(acc), t(us), t(sums), t(tau), torch.tensor(pos, device=DEV), argmax=True,
                        top8=True, top20=True, n_logprobs=20)
    d.sync()
    assert list(to_u32(out["ids"]).reshape(-1)) == pmap(lambda r: oracle_select(x[r], int(pos[r]), sp), range(rows))
    assert list(to_u32(out["argmax"])) == [O.greedy(x[r]) for r in range(rows)]
    for r in range(rows):
        tt = O.top_tokens(x[r], 20)
        assert list(to_u32(out["top20_ids"])[r]) == list(tt)
        assert np.array_equal(out["top20_vals"][r].cpu().numpy().view(np.uint32), x[r][tt].view(np.uint32))
        ids, lp = O.top_logprobs(x[r], 20)
        assert list(to_u32(out["logprob_ids"])[r]) == list(ids)
        assert_logprobs_close(out["logprobs"][r].cpu().numpy(), lp)
    # the same logits through the binary32 entry point give the same answers
    ref = d.sample(t(x), torch.tensor(pos, device=DEV), argmax=True, top20=True)
    d.sync()
    assert torch.equal(ref["ids"], out["ids"]) and torch.equal(ref["top20_ids"], out["top20_ids"])
    d.close()


def test_head_logits_written_out_and_accumulators_cleared():
    rows, V = 4, 70_001
    acc, us, sums, tau = _head_inputs(rows, V, 5)
    x = _oracle_logits(acc, us, sums, tau)
    d = DeviceSampler(rows, V)
    sp = SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, seed=9)
    d.set_params(sp)
    ta = torch.from_numpy(acc).to(DEV)
    lo = torch.full((rows, V + 3), 7.0, dtype=torch.float32, device=DEV)[:, :V]
    t = lambda a: torch.from_numpy(a).to(DEV)
    out = d.sample_head(ta, t(us), t(sums), t(tau), torch.arange(rows, device=DEV), logits_out=lo,
                        clear_acc=True, top20=True)
    d.sync()
    assert np.array_equal(lo.cpu().numpy().view(np.uint32), x.view(np.uint32))
    assert int(torch.count_nonzero(ta)) == 0
    assert list(to_u32(out["ids"]).reshape(-1)) == [oracle_select(x[r], r, sp) for r in range(rows)]
    for r in range(rows):
        assert list(to_u32(out["top20_ids"])[r]) == list(O.top_tokens(x[r], 20))
    with pytest.raises(InvalidInput):
        d.sample_head(ta, t(us), t(sums), t(tau), torch.arange(rows, device=DEV), clear_acc=True)
    d.close()


def test_head_nonfinite_inverse_rms_and_logits_fail_the_row():
    rows, V = 3, 5000
    acc, us, sums, tau = _head_inputs(rows, V, 17)
    sums[1, 4] = np.inf                    # the sum of squares is not finite
    tau[100] = 3e38                         # row 2 overflows at token 100
    acc[:2, 100] = 0
    acc[2, 100] = 2**62
    d = DeviceSampler(rows, V)
    d.set_params(SamplingParameters(temperature_milli=0))
    t = lambda a: torch.from_numpy(a).to(DEV)
    out = d.sample_head(t(acc), t(us), t(sums), t(tau), torch.arange(rows, device=DEV), row_status=True)
    with pytest.raises(NonFinite):
        d.sync()
    st = out["status"].cpu().tolist()
    with pytest.raises(O.OracleError):
        O.inverse_rms(sums[1], 5120.0, 1e-6)
    ir = O.inverse_rms(sums[2], 5120.0, 1e-6)
    with pytest.raises(O.OracleError):
        O.head_logits(acc[2], tau, float(us[2]), ir)
    assert st == [0, -2, -2]
    x0 = _oracle_logits(acc[:1], us[:1], sums[:1], tau)[0]
    assert to_u32(out["ids"])[0, 0] == O.greedy(x0)
    d.close()
