"""Writes the golden fixtures of the sampling path (tests/golden/*.json).

reference_vectors.json
    Known answers held by the reference's own tests, transcribed as data with
    the file:line each comes from: the binary64 exp_d / log_d bit vectors
    (crates/yskn-ref/src/portable_math.rs:487-590), the sampler's unit-test
    cases (crates/yskn-ref/src/output_head_sampler.rs:256-310) and the
    published SplitMix64 outputs for state 0.

sampler_small.json
    Seeded small inputs (raw float32 bytes, base64) and the oracle's outputs on
    them: argmax, top-20, top-N logprobs, NLL, sampled ids for a grid of
    parameter sets and absolute positions (including positions past 2^32 and
    2^63), penalised rows (with the SHA-256 of the penalised logits) and
    speculative-verify blocks over one shared set of M target rows. The oracle is the
    C restatement under oracle/, itself pinned by reference_vectors.json and
    the mathematical checks in tests/test_oracle_*.py; freezing its outputs
    here lets the GPU tests compare against data and lets the CPU tests catch
    any drift of the oracle.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import base64
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import yskn_oracle as O  # noqa: E402

GUMBEL, INVERSE_CDF = 3, 2

# Absolute prediction positions: small, around 2^32 and near 2^64.
POSITIONS = [0, 1, 2, 3, 17, 100, 1023, 4096, 2**32 - 1, 2**32 + 5, 2**53 + 1, 2**63 + 7]

# (name, temperature, top_p, min_p in thousandths, top_k, seed, version, extension)
PARAMS = [
    ("default_v3", 1000, 950, 0, 20, 0, GUMBEL, False),
    ("default_v2", 1000, 950, 0, 20, 0x112345678, INVERSE_CDF, False),
    ("top_k_1", 1000, 950, 0, 1, 5, GUMBEL, False),
    ("cold_min_p", 700, 900, 50, 20, 77, GUMBEL, False),
    ("hot_v2", 1500, 800, 0, 20, 3, INVERSE_CDF, False),
    ("very_cold_full_p", 300, 1000, 0, 20, 9, GUMBEL, False),
    ("min_p_one_v2", 1000, 950, 1000, 20, 21, INVERSE_CDF, False),
    ("ext_top_k_disabled", 1000, 950, 0, 0, 11, GUMBEL, True),
    ("ext_top_k_50_v2", 1000, 900, 20, 50, 13, INVERSE_CDF, True),
    ("ext_disabled_hot", 2000, 990, 0, 0, 17, GUMBEL, True),
]


def b64(a: np.ndarray) -> str:
    return base64.b64encode(np.ascontiguousarray(a, np.float32).tobytes()).decode()


def splitmix_normals(seed: int, n: int) -> np.ndarray:
    """Box-Muller normals from a SplitMix64 counter stream (input generator
    only; its exact form does not matter, the bytes are stored)."""
    i = np.arange(2 * ((n + 1) // 2), dtype=np.uint64) + np.uint64(seed) * np.uint64(0x10000)
    with np.errstate(over="ignore"):
        z = i * np.uint64(0x9E3779B97F4A7C15) + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0**-53
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(u.size)
    out[0::2] = r * np.cos(2 * np.pi * u2)
    out[1::2] = r * np.sin(2 * np.pi * u2)
    return out[:n]


def row_sets():
    sets = []
    V = 1537  # ragged: not a multiple of 2, 4 or the device chunk
    r0 = 2.5 * splitmix_normals(1, V)
    boost = (splitmix_normals(2, 20) * 1e6).astype(np.int64) % V
    r0[np.abs(boost)] += 8.0
    r1 = np.round(2.0 * splitmix_normals(3, V)) / 2.0  # heavy ties
    r1[::97] = 0.0
    r1 = r1.astype(np.float32)
    r1[::194] = -0.0  # -0 and +0 tie; id breaks it
    t_den = np.sqrt((splitmix_normals(4, V) ** 2 + splitmix_normals(5, V) ** 2 + splitmix_normals(6, V) ** 2) / 3)
    r2 = 2.0 * splitmix_normals(7, V) / t_den  # Student-t, 3 degrees of freedom
    r3 = np.zeros(V)  # uniform
    r4 = splitmix_normals(8, V)
    r4[1234] = 50.0  # one dominant token
    r5 = splitmix_normals(9, V) * 1e30  # huge finite range
    sets.append(("v1537", np.stack([r0, r1, r2, r3, r4, r5]).astype(np.float32)))
    V = 5000  # spans several device chunks with a ragged tail
    a = 2.5 * splitmix_normals(10, V)
    b = np.round(splitmix_normals(11, V) * 4.0) / 4.0
    c = 2.0 * splitmix_normals(12, V) / np.sqrt((splitmix_normals(13, V) ** 2 + splitmix_normals(14, V) ** 2
                                                  + splitmix_normals(15, V) ** 2) / 3)
    sets.append(("v5000", np.stack([a, b, c]).astype(np.float32)))
    # the reference's unit-test inputs (output_head_sampler.rs:256-310)
    sets.append(("tiny_v1", np.array([[4.0]], np.float32)))
    sets.append(("tiny_v2", np.array([[-0.0, 0.0]], np.float32)))
    sets.append(("tiny_v3", np.array([[1.0, 3.0, 2.0], [1.0, 2.0, -1.0], [17.0, 18.0, 15.0]], np.float32)))
    sets.append(("tiny_v4", np.array([[2.0, 3.0, 3.0, -1.0]], np.float32)))
    sets.append(("v32", np.array([[(i % 7) / 8.0 for i in range(32)]], np.float32)))
    return sets


def oracle_params(p):
    _, t, tp, mp, k, seed, ver, ext = p
    return O.params_from_thousandths(t, tp, mp, top_k=k, seed=seed, version=ver, extension=ext)


def sample_or_error(row, p):
    try:
        return [int(x) for x in O.sample_positions(row, np.array(POSITIONS, np.uint64), oracle_params(p))]
    except O.OracleError as e:
        return {"error": int(e.status)}


def make_small():
    out = {"generator": "tests/golden/make_golden.py", "positions": [str(x) for x in POSITIONS],
           "params": [dict(zip(("name", "temperature_milli", "top_p_milli", "min_p_milli", "top_k", "seed",
                                "version", "extension"), p)) for p in PARAMS],
           "row_sets": [], "penalty_cases": [], "verify_cases": []}
    for name, rows in row_sets():
        R, V = rows.shape
        n20 = min(20, V)
        rs = {"name": name, "V": V, "rows": [b64(r) for r in rows], "argmax": [], "top20": [],
              "logprob_ids": [], "logprobs": [], "nll_targets": [], "nll": [], "ids": {}}
        for r in rows:
            rs["argmax"].append(O.greedy(r))
            rs["top20"].append([int(x) for x in O.top_tokens(r, n20)])
            ids, lp = O.top_logprobs(r, n20)
            rs["logprob_ids"].append([int(x) for x in ids])
            rs["logprobs"].append([float(x) for x in lp])
            targets = sorted({0, V - 1, O.greedy(r), V // 2})
            rs["nll_targets"].append(targets)
            rs["nll"].append([O.nll(r, t) for t in targets])
        for p in PARAMS:
            rs["ids"][p[0]] = [sample_or_error(r, p) for r in rows]
        out["row_sets"].append(rs)

    # penalised rows: history of ids, repetition / presence / frequency
    V = 1537
    logits = (2.0 * splitmix_normals(20, 2 * V)).reshape(2, V).astype(np.float32)
    hist = (np.abs(splitmix_normals(21, 2 * 300)) * 200).astype(np.int64).reshape(2, 300) % V
    for i, (rep, pres, freq) in enumerate([(1.05, 0.5, 0.3), (1.3, 0.0, 0.0)]):
        p = PARAMS[3] if i == 0 else PARAMS[0]
        pen = np.stack([O.apply_penalties(logits[r], hist[r], rep, pres, freq) for r in range(2)])
        out["penalty_cases"].append({
            "V": V, "rows": [b64(r) for r in logits], "history": hist.tolist(),
            "repetition": rep, "presence": pres, "frequency": freq, "params": p[0],
            "penalised_sha256": [hashlib.sha256(np.ascontiguousarray(r, np.float32).tobytes()).hexdigest()
                                 for r in pen],
            "ids": [[int(x) for x in O.sample_positions(pen[r], np.array(POSITIONS, np.uint64), oracle_params(p))]
                    for r in range(2)]})

    # speculative verification blocks of M = 8 rows
    V, M = 1537, 8
    target = (3.0 * splitmix_normals(30, M * V)).reshape(M, V).astype(np.float32)
    base = 4095
    out["verify_rows"] = {"V": V, "M": M, "rows": [b64(r) for r in target]}
    for case, (pname, agree, eos) in enumerate([("default_v3", 3, []), ("default_v3", 7, []),
                                                ("hot_v2", 0, []), ("default_v3", 7, "third"),
                                                ("greedy", 5, [])]):
        p = None if pname == "greedy" else oracle_params(next(q for q in PARAMS if q[0] == pname))
        sel_all = [O.greedy(target[j]) if p is None else O.sample(target[j], base + j + 1, p) for j in range(M)]
        drafts = [sel_all[j] if j < agree else (sel_all[j] + 1) % V for j in range(M - 1)]
        eos_ids = [sel_all[2]] if eos == "third" else []
        sel, emitted, accepted, stop = O.verify(target, drafts, base, p, eos_ids)
        out["verify_cases"].append({"params": pname, "drafts": drafts, "base_position": base, "eos": eos_ids,
                                    "selected": [int(x) for x in sel], "emitted": int(emitted),
                                    "accepted": int(accepted), "stop_eos": bool(stop)})
    return out


def make_reference_vectors():
    """Known answers from the reference's tests, as (input, expected bits)."""
    return {
        "source": "crates/yskn-ref/src/portable_math.rs and output_head_sampler.rs (unit tests)",
        "exp_d_log_d_bits": {
            "cite": "portable_math.rs:563-571",
            "cases": [[0.5, "3ffa61298e1e069c", "bfe62e42fefa39ef"],
                      [1.0, "4005bf0a8b14576a", "0000000000000000"],
                      [10.0, "40d5829dcf950560", "40026bb1bbb55516"]]},
        "identity_points": {"cite": "portable_math.rs:495-496",
                            "exp_d(0)": "3ff0000000000000", "log_d(1)": "0000000000000000"},
        "underflow_overflow": {"cite": "portable_math.rs:507-508",
                               "exp_d(-746)": "0000000000000000", "exp_d(710)": "inf"},
        "log_zero_endpoints": {"cite": "portable_math.rs:584-587",
                               "log_d(+0)": "c0875427f6acad6f", "log_d(-0)": "c0a0ec2b7d284853"},
        "splitmix64_state0": {
            "cite": "SplitMix64 (Steele, Lea, Flood 2014), published first outputs for state 0",
            "mix64_of_k_times_golden": ["e220a8397b1dcdaf", "6e789e6aa1b965f4", "06c45d188009454f"]},
        "tie_order": {"cite": "output_head_sampler.rs:256-262",
                      "greedy([-0.0, 0.0])": 0, "top_tokens([2,3,3,-1], 3)": [1, 2, 0],
                      "greedy([nan])": "NonFinite", "greedy([-inf])": "error"},
        "truncation": {"cite": "output_head_sampler.rs:286-299",
                       "logits": [1.0, 3.0, 2.0], "top_k": 3, "min_p": 1.0, "positions": 16, "expected": 1},
        "nll_shift": {"cite": "output_head_sampler.rs:301-310",
                      "a": [1.0, 2.0, -1.0], "b": [17.0, 18.0, 15.0], "target": 1,
                      "single": [[4.0], 0, "0000000000000000"]},
        "seed_position_only": {"cite": "output_head_sampler.rs:264-284",
                               "logits": "(i % 7) / 8 for i in 0..32", "seed": "112345678",
                               "positions": [100, 120]},
    }


def main():
    O.build() if not os.path.exists(os.path.join(ROOT, "oracle", "build", "liboracle.so")) else None
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(make_reference_vectors(), f, indent=1)
        f.write("\n")
    with open(os.path.join(HERE, "sampler_small.json"), "w") as f:
        json.dump(make_small(), f, separators=(",", ":"))
        f.write("\n")


if __name__ == "__main__":
    main()
