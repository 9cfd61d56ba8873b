"""Pins the oracle's sampler (output_head_sampler.rs:21-250), acceptance loop
(speculation.rs:483-523) and the build-defined extensions.

Pins used, so that a plausible mistake (a dropped term, a flipped comparison,
a wrong index) fails at least one test:
* the reference's unit tests (output_head_sampler.rs:252-311);
* an independent ordering (Python's sort on (-value, id)) on tiny rows;
* special cases with known answers: top_k = 1 is argmax; equal logits with
  top_p = 0.5 keep exactly the first candidate; min_p = 1 keeps the first;
* distributional checks: Gumbel-max (version 3) and inverse-CDF (version 2)
  draw frequencies match the truncated softmax;
* an independent numpy Gumbel argmax when nothing is truncated.
"""
import math

import numpy as np
import pytest
import torch

import yskn_oracle as O


# ---- output_head_sampler.rs:256-262 -----------------------------------------
def test_raw_order_ties_are_broken_by_token_id():
    assert O.greedy([-0.0, 0.0]) == 0
    assert list(O.top_tokens([2.0, 3.0, 3.0, -1.0], 3)) == [1, 2, 0]
    with pytest.raises(O.OracleError) as e:
        O.greedy([math.nan])
    assert e.value.status == O.ENONFINITE
    with pytest.raises(O.OracleError):
        O.greedy([-math.inf])


# ---- output_head_sampler.rs:264-284 -----------------------------------------
@pytest.mark.parametrize("version", [O.GUMBEL, O.INVERSE_CDF])
def test_seed_and_absolute_position_are_the_only_sampling_state(version):
    logits = np.array([(i % 7) / 8.0 for i in range(32)], np.float32)
    p = O.params(seed=0x1_1234_5678, version=version)
    expected = [O.sample(logits, pos, p) for pos in range(100, 120)]
    actual = [O.sample(logits, pos, p) for pos in reversed(range(100, 120))][::-1]
    assert actual == expected
    assert any(a != b for a, b in zip(expected, expected[1:]))


# ---- output_head_sampler.rs:286-299 -----------------------------------------
@pytest.mark.parametrize("version", [O.GUMBEL, O.INVERSE_CDF])
def test_truncation_retains_at_least_the_top_candidate(version):
    p = O.params(top_k=3, min_p=1.0, version=version)
    for pos in range(16):
        assert O.sample([1.0, 3.0, 2.0], pos, p) == 1


# ---- output_head_sampler.rs:301-310 -----------------------------------------
def test_loss_is_invariant_to_an_exact_constant_logit_shift():
    first = O.nll([1.0, 2.0, -1.0], 1)
    shifted = O.nll([17.0, 18.0, 15.0], 1)
    assert first == shifted
    assert O.nll([4.0], 0) == 0.0


# ---- independent checks -----------------------------------------------------
def test_top_tokens_matches_an_independent_sort_on_tiny_rows():
    rng = np.random.default_rng(3)
    for trial in range(200):
        V = int(rng.integers(1, 12))
        x = rng.integers(-3, 4, V).astype(np.float32)  # many ties
        x[rng.random(V) < 0.2] = -0.0
        ref = sorted(range(V), key=lambda i: (-float(x[i]), i))
        assert list(O.top_tokens(x, V)) == ref
        assert O.greedy(x) == ref[0]


def test_top_k_one_is_argmax():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(500).astype(np.float32)
    p = O.params(top_k=1, seed=7)
    for pos in range(50):
        assert O.sample(x, pos, p) == int(np.argmax(x))


def test_top_p_cut_on_equal_weights():
    # w = [1, 1]: total 2; top_p 0.5 -> threshold 1.0 is met by the first
    # candidate alone; top_p 0.6 needs both.
    x = np.array([5.0, 5.0], np.float32)
    only_first = {O.sample(x, pos, O.params(top_k=2, top_p=0.5)) for pos in range(64)}
    assert only_first == {0}
    both = {O.sample(x, pos, O.params(top_k=2, top_p=0.6)) for pos in range(64)}
    assert both == {0, 1}
    _, d = O.sample(x, 0, O.params(top_k=2, top_p=0.5), diag=True)
    assert (d.k, d.n_top_p, d.retained, d.total) == (2, 1, 1, 2.0)


def test_min_p_is_relative_to_the_top_weight():
    # weights exp(-0), exp(-1), exp(-2), exp(-3) = 1, .368, .135, .0498
    x = np.array([0.0, -1.0, -2.0, -3.0], np.float32)
    for mp, keep in [(0.3, 2), (0.1, 3), (0.04, 4), (0.5, 1)]:
        _, d = O.sample(x, 0, O.params(top_k=4, top_p=1.0, min_p=mp), diag=True)
        assert d.retained == keep, mp


def _truncated_softmax(x, T, k, top_p, min_p):
    order = sorted(range(len(x)), key=lambda i: (-float(x[i]), i))[:k]
    z = [(float(x[i]) - float(x[order[0]])) / T for i in order]
    w = [math.exp(v) for v in z]
    tot = sum(w)
    n = k
    pre = 0.0
    for j, v in enumerate(w):
        pre += v
        if pre >= top_p * tot:
            n = j + 1
            break
    if min_p > 0:
        m = 1
        while m < n and w[m] >= min_p:
            m += 1
        n = m
    ws = np.array(w[:n])
    return order[:n], ws / ws.sum()


@pytest.mark.parametrize("version", [O.GUMBEL, O.INVERSE_CDF])
def test_draw_frequencies_match_the_truncated_softmax(version):
    x = np.array([2.0, 1.5, 1.4, 0.3, -0.2, 0.9, 1.0, -1.0], np.float32)
    T, k, top_p, min_p = 0.8, 6, 0.9, 0.0
    ids, probs = _truncated_softmax(x, T, k, top_p, min_p)
    p = O.params(temperature=T, top_k=k, top_p=top_p, min_p=min_p, seed=42, version=version)
    n = 20000
    draws = O.sample_positions(x, np.arange(n, dtype=np.uint64), p)
    counts = np.array([(draws == i).sum() for i in ids], float)
    assert counts.sum() == n  # nothing outside the truncated set
    chi2 = ((counts - n * probs) ** 2 / (n * probs)).sum()
    # 5 dof; P(chi2 > 25) ~ 1.4e-4
    assert chi2 < 25.0, (counts, n * probs)


def test_gumbel_pick_equals_an_independent_argmax_without_truncation():
    rng = np.random.default_rng(21)
    x = (3.0 * rng.standard_normal(40)).astype(np.float32)
    T, seed = 1.3, 0xABCDEF
    order = sorted(range(40), key=lambda i: (-float(x[i]), i))[:20]
    p = O.params(temperature=T, top_k=20, top_p=1.0, seed=seed)
    M = (1 << 64) - 1
    for pos in range(200):
        b = O.mix64(O.mix64(seed) ^ pos)
        best, pick = -math.inf, None
        for i in order:
            h = O.mix64(b ^ ((i * 0xD6E8FEB86659FD93) & M))
            u = ((h >> 11) + 0.5) * 2.0 ** -53
            s = (float(x[i]) - float(x[order[0]])) / T - math.log(-math.log(u))
            if s > best:
                best, pick = s, i
        assert O.sample(x, pos, p) == pick


def test_from_thousandths_divides():
    p = O.params_from_thousandths(700, 900, 50)
    assert p.temperature == 700 / 1000.0 and p.top_p == 900 / 1000.0 and p.min_p == 50 / 1000.0
    # 0.001 * 700 differs from 700 / 1000 in the last bit for some values
    diffs = [t for t in range(1, 2000) if t / 1000.0 != 0.001 * t]
    assert diffs, "division and multiplication by 0.001 must differ somewhere"


def test_validation_rules():
    x = np.zeros(30, np.float32)
    bad = [dict(top_k=0), dict(top_k=21), dict(top_p=0.0), dict(top_p=1.01),
           dict(min_p=-0.1), dict(min_p=1.1), dict(temperature=0.0), dict(temperature=math.inf)]
    for kw in bad:
        with pytest.raises(O.OracleError):
            O.sample(x, 0, O.params(**kw))
    with pytest.raises(O.OracleError):
        O.sample(np.zeros(5, np.float32), 0, O.params(top_k=6))
    # extension: k = 0 disables top-k, k up to V
    O.sample(x, 0, O.params(top_k=0, extension=True))
    O.sample(x, 0, O.params(top_k=30, extension=True))
    with pytest.raises(O.OracleError):
        O.sample(x, 0, O.params(top_k=31, extension=True))
    with pytest.raises(O.OracleError):
        O.sample(np.zeros(0, np.float32), 0, O.params())


# ---- extensions --------------------------------------------------------------
def test_bf16_widening_matches_torch():
    rng = np.random.default_rng(8)
    bits16 = rng.integers(0, 2 ** 16, 5000).astype(np.uint16)
    bits16 = bits16[(bits16 & 0x7F80) != 0x7F80]  # finite only
    ref = torch.from_numpy(bits16.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = O.bf16_to_f32(bits16)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_penalties_hand_computed():
    x = np.array([2.0, -2.0, 1.0, 0.5, 3.0], np.float32)
    hist = [0, 0, 1, 3, 0]
    y = O.apply_penalties(x, hist, 1.25, 0.5, 0.25)
    f = np.float32
    exp0 = f(f(f(2.0) / f(1.25)) - f(f(0.25) * f(3.0))) - f(0.5)
    exp1 = f(f(f(-2.0) * f(1.25)) - f(f(0.25) * f(1.0))) - f(0.5)
    exp3 = f(f(f(0.5) / f(1.25)) - f(0.25)) - f(0.5)
    assert y[0] == exp0 and y[1] == exp1 and y[3] == exp3
    assert y[2] == x[2] and y[4] == x[4]
    with pytest.raises(O.OracleError):
        O.apply_penalties(x, [5], 1.0, 0.0, 0.0)


def test_penalty_identity_parameters_change_nothing():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(100).astype(np.float32)
    y = O.apply_penalties(x, rng.integers(0, 100, 50), 1.0, 0.0, 0.0)
    assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_top_logprobs_are_negated_nll():
    rng = np.random.default_rng(4)
    x = (2 * rng.standard_normal(300)).astype(np.float32)
    ids, lp = O.top_logprobs(x, 10)
    assert list(ids) == list(O.top_tokens(x, 10))
    for i, v in zip(ids, lp):
        assert v == -O.nll(x, int(i))
    m = float(x.max())
    lse = m + math.log(np.exp(x.astype(np.float64) - m).sum())
    assert lp[0] == pytest.approx(float(x[ids[0]]) - lse, rel=1e-12)


# ---- acceptance loop (speculation.rs:483-523; pattern of :880-1012) ----------
def _sequential(rows, guesses, base, p, eos=()):
    out = []
    acc = 0
    for j in range(rows.shape[0]):
        sel = O.sample(rows[j], base + j + 1, p) if p is not None else O.greedy(rows[j])
        out.append(sel)
        matched = j < len(guesses) and guesses[j] == sel
        acc += matched
        if sel in eos or not matched:
            return out, acc, sel in eos
    return out, acc, False


@pytest.mark.parametrize("p", [None, O.params(seed=17), O.params(seed=0xABCDEF, top_k=5)])
def test_verify_equals_token_at_a_time(p):
    rng = np.random.default_rng(6)
    for trial in range(30):
        M = int(rng.integers(1, 9))
        rows = (2.0 * rng.standard_normal((M, 64))).astype(np.float32)
        truth = [O.sample(rows[j], 100 + j + 1, p) if p is not None else O.greedy(rows[j])
                 for j in range(M)]
        # right, wrong at a random depth, or random proposer
        mode = trial % 3
        guesses = list(truth[:M - 1])
        if mode == 1 and M > 1:
            d = int(rng.integers(0, M - 1))
            guesses[d] = (guesses[d] + 1) % 64
        elif mode == 2:
            guesses = list(rng.integers(0, 64, M - 1))
        eos = (truth[int(rng.integers(0, M))],) if trial % 5 == 0 else ()
        sel, em, acc, stop = O.verify(rows, guesses, 100, p, eos)
        ref, racc, rstop = _sequential(rows, guesses, 100, p, eos)
        assert list(sel) == ref and em == len(ref) and acc == racc and stop == rstop


def test_draft_choose_greedy_part_and_determinism():
    rng = np.random.default_rng(12)
    scores = rng.standard_normal(16).astype(np.float32)
    tokens = rng.permutation(1000)[:16].astype(np.uint32)
    a = [O.draft_choose(scores, tokens, 5, 850, pos) for pos in range(50)]
    b = [O.draft_choose(scores, tokens, 5, 850, pos) for pos in range(50)]
    assert a == b and set(a) <= set(tokens.tolist())
    # very low temperature concentrates on the highest score
    top = tokens[int(np.argmax(scores))]
    assert all(O.draft_choose(scores, tokens, 5, 1, pos) == top for pos in range(20))
