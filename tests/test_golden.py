"""Golden fixtures (tests/golden/): the reference's own known answers and the
frozen oracle outputs on seeded small inputs.

CPU tests: the oracle still reproduces every fixture bit for bit, and the
reference's vectors (portable_math.rs, output_head_sampler.rs unit tests)
hold for it. GPU tests: the HIP path, called through the C ABI, returns the
fixture's ids, argmax, top-20 and accept counts exactly, and its logprobs and
NLL within 1e-5 relative (absolute floor 1e-10).
"""
from __future__ import annotations

import base64
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

import yskn_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
LP_REL, LP_ABS = 1e-5, 1e-10


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


SMALL = _load("sampler_small.json")
REFV = _load("reference_vectors.json")
POSITIONS = [int(x) for x in SMALL["positions"]]
PARAMS = {p["name"]: p for p in SMALL["params"]}


def rows_of(entry) -> np.ndarray:
    return np.stack([np.frombuffer(base64.b64decode(s), np.float32) for s in entry["rows"]])


def bits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def oparams(name):
    p = PARAMS[name]
    return O.params_from_thousandths(p["temperature_milli"], p["top_p_milli"], p["min_p_milli"],
                                     top_k=p["top_k"], seed=p["seed"], version=p["version"],
                                     extension=p["extension"])


def close(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= LP_REL * np.abs(ref) + LP_ABS))


# --------------------------------------------------------------------------
# CPU: the reference's known answers
# --------------------------------------------------------------------------

def test_reference_exp_log_bits():
    for x, e, l in REFV["exp_d_log_d_bits"]["cases"]:
        assert bits(O.exp_d(x)) == int(e, 16)
        assert bits(O.log_d(x)) == int(l, 16)
    assert bits(O.exp_d(0.0)) == int(REFV["identity_points"]["exp_d(0)"], 16)
    assert bits(O.log_d(1.0)) == int(REFV["identity_points"]["log_d(1)"], 16)
    assert bits(O.exp_d(-746.0)) == int(REFV["underflow_overflow"]["exp_d(-746)"], 16)
    assert O.exp_d(710.0) == math.inf
    assert bits(O.log_d(0.0)) == int(REFV["log_zero_endpoints"]["log_d(+0)"], 16)
    assert bits(O.log_d(-0.0)) == int(REFV["log_zero_endpoints"]["log_d(-0)"], 16)


def test_splitmix64_published_outputs():
    gamma = 0x9E3779B97F4A7C15
    for k, want in enumerate(REFV["splitmix64_state0"]["mix64_of_k_times_golden"]):
        assert O.mix64((k * gamma) % 2**64) == int(want, 16)


def test_reference_sampler_unit_cases():
    t = REFV["tie_order"]
    assert O.greedy([-0.0, 0.0]) == t["greedy([-0.0, 0.0])"]
    assert list(O.top_tokens([2.0, 3.0, 3.0, -1.0], 3)) == t["top_tokens([2,3,3,-1], 3)"]
    for bad in (math.nan, -math.inf):
        with pytest.raises(O.OracleError):
            O.greedy([bad])
    tr = REFV["truncation"]
    for ver in (2, 3):
        p = O.params(top_k=tr["top_k"], min_p=tr["min_p"], version=ver)
        assert [O.sample(tr["logits"], pos, p) for pos in range(tr["positions"])] == [tr["expected"]] * 16
    ns = REFV["nll_shift"]
    assert bits(O.nll(ns["a"], ns["target"])) == bits(O.nll(ns["b"], ns["target"]))
    row, target, want = ns["single"]
    assert bits(O.nll(row, target)) == int(want, 16)


# --------------------------------------------------------------------------
# CPU: the oracle reproduces its frozen outputs
# --------------------------------------------------------------------------

@pytest.mark.parametrize("rs", SMALL["row_sets"], ids=lambda r: r["name"])
def test_oracle_reproduces_row_fixture(rs):
    rows = rows_of(rs)
    pos = np.array(POSITIONS, np.uint64)
    for i, r in enumerate(rows):
        n20 = min(20, rs["V"])
        assert O.greedy(r) == rs["argmax"][i]
        assert list(O.top_tokens(r, n20)) == rs["top20"][i]
        ids, lp = O.top_logprobs(r, n20)
        assert list(ids) == rs["logprob_ids"][i]
        assert [bits(x) for x in lp] == [bits(x) for x in rs["logprobs"][i]]
        assert [bits(O.nll(r, t)) for t in rs["nll_targets"][i]] == [bits(x) for x in rs["nll"][i]]
        for name, per_row in rs["ids"].items():
            want = per_row[i]
            if isinstance(want, dict):
                with pytest.raises(O.OracleError):
                    O.sample_positions(r, pos, oparams(name))
            else:
                assert list(O.sample_positions(r, pos, oparams(name))) == want, name


@pytest.mark.parametrize("case", range(len(SMALL["penalty_cases"])))
def test_oracle_reproduces_penalty_fixture(case):
    pc = SMALL["penalty_cases"][case]
    rows = rows_of(pc)
    for r in range(rows.shape[0]):
        pen = O.apply_penalties(rows[r], pc["history"][r], pc["repetition"], pc["presence"], pc["frequency"])
        assert hashlib.sha256(pen.tobytes()).hexdigest() == pc["penalised_sha256"][r]
        assert list(O.sample_positions(pen, np.array(POSITIONS, np.uint64), oparams(pc["params"]))) == pc["ids"][r]


@pytest.mark.parametrize("case", range(len(SMALL["verify_cases"])))
def test_oracle_reproduces_verify_fixture(case):
    vc = SMALL["verify_cases"][case]
    target = rows_of(SMALL["verify_rows"])
    p = None if vc["params"] == "greedy" else oparams(vc["params"])
    sel, emitted, accepted, stop = O.verify(target, vc["drafts"], vc["base_position"], p, vc["eos"])
    assert list(sel) == vc["selected"]
    assert (emitted, accepted, stop) == (vc["emitted"], vc["accepted"], vc["stop_eos"])


# --------------------------------------------------------------------------
# GPU: the HIP path through the C ABI against the fixtures
# --------------------------------------------------------------------------

def _device_params(name, penalties=(1.0, 0.0, 0.0)):
    import yskn_smp

    p = PARAMS[name]
    return yskn_smp.SamplingParameters(temperature_milli=p["temperature_milli"], top_p_milli=p["top_p_milli"],
                                       min_p_milli=p["min_p_milli"], top_k=p["top_k"], seed=p["seed"],
                                       version=p["version"], repetition_penalty=penalties[0],
                                       presence_penalty=penalties[1], frequency_penalty=penalties[2])


def _positions(torch, rows):
    pos = np.array(POSITIONS, dtype=np.uint64).view(np.int64)
    return torch.from_numpy(np.tile(pos, (rows, 1))).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("rs", SMALL["row_sets"], ids=lambda r: r["name"])
def test_device_matches_row_fixture(rs):
    import torch

    import yskn_smp

    rows = rows_of(rs)
    R, V = rows.shape
    n20 = min(20, V)
    x = torch.from_numpy(rows).cuda()
    pos = _positions(torch, R)
    for ext in (False, True):
        dev = yskn_smp.DeviceSampler(R, V, extended_top_k=ext)
        try:
            assert dev.argmax(x).cpu().tolist() == rs["argmax"]
            ids, _ = dev.top_tokens(x, n20)
            assert ids.cpu().tolist() == rs["top20"]
            for j in range(max(len(t) for t in rs["nll_targets"])):
                tgt = torch.tensor([t[min(j, len(t) - 1)] for t in rs["nll_targets"]], dtype=torch.int32).cuda()
                got = dev.nll(x, tgt).cpu().numpy()
                want = [n[min(j, len(n) - 1)] for n in rs["nll"]]
                assert close(got, want), (j, got, want)
            for name, per_row in rs["ids"].items():
                if PARAMS[name]["extension"] != ext:
                    continue
                if isinstance(per_row[0], dict):
                    with pytest.raises(yskn_smp.InvalidInput):
                        dev.set_params(_device_params(name))
                        dev.sample(x, pos)
                        dev.sync()
                    continue
                dev.set_params(_device_params(name))
                out = dev.sample(x, pos, n_logprobs=n20)
                dev.sync()
                got = out["ids"].cpu().numpy().astype(np.int64).tolist()
                assert got == per_row, name
                assert out["logprob_ids"].cpu().tolist() == rs["logprob_ids"], name
                assert close(out["logprobs"].cpu().numpy(), rs["logprobs"]), name
        finally:
            dev.close()


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(SMALL["penalty_cases"])))
def test_device_matches_penalty_fixture(case):
    import torch

    import yskn_smp

    pc = SMALL["penalty_cases"][case]
    rows = rows_of(pc)
    R, V = rows.shape
    dev = yskn_smp.DeviceSampler(R, V)
    try:
        dev.set_params(_device_params(pc["params"], (pc["repetition"], pc["presence"], pc["frequency"])))
        hist = torch.tensor(pc["history"], dtype=torch.int32).cuda()
        out = dev.sample(torch.from_numpy(rows).cuda(), _positions(torch, R), history=hist)
        dev.sync()
        assert out["ids"].cpu().numpy().astype(np.int64).tolist() == pc["ids"]
    finally:
        dev.close()


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(SMALL["verify_cases"])))
def test_device_matches_verify_fixture(case):
    import torch

    import yskn_smp

    vc = SMALL["verify_cases"][case]
    target = rows_of(SMALL["verify_rows"])
    M, V = target.shape
    dev = yskn_smp.DeviceSampler(M, V)
    try:
        if vc["params"] == "greedy":
            dev.set_params(yskn_smp.SamplingParameters(temperature_milli=0))
        else:
            dev.set_params(_device_params(vc["params"]))
        ids, res, _keep = dev.verify(torch.from_numpy(target).cuda(), torch.tensor(vc["drafts"]).cuda(),
                                     torch.tensor([vc["base_position"]]).cuda(), vc["eos"])
        dev.sync()
        accepted, emitted, token, stop, status = res.cpu().tolist()
        assert status == 0
        assert (accepted, emitted, bool(stop)) == (vc["accepted"], vc["emitted"], vc["stop_eos"])
        assert ids.cpu().tolist()[:emitted] == vc["selected"]
        assert token == vc["selected"][-1]
    finally:
        dev.close()
