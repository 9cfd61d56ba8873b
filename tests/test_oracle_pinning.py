"""Pins the oracle functions that the reference's own unit tests leave open:
the version-2 inverse-CDF draw (output_head_sampler.rs:192-209; spec 06
section 7), the draft-side coupled choice, shortlist and top 16
(draft_head.rs:219-379), the binary32 square root and the head scale
restoration (portable_math.rs:61-111; compressed_linear.rs:329-340), and the
acceptance loop's position overflow (speculation.rs:489-497).

Each check is an independent formulation (Python integers for the hash, an
independent sort, numpy binary32 arithmetic, a sort-based cutoff instead of
histograms), and each plausible mistake listed in the tests is planted in a
Python copy of the formulation to show that the comparison would catch it in
the oracle.
"""
import math
import struct

import numpy as np
import pytest

import yskn_oracle as O

MASK = (1 << 64) - 1
G, C1, C2 = 0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB


def mix64(z: int) -> int:
    z = (z + G) & MASK
    z = ((z ^ (z >> 30)) * C1) & MASK
    z = ((z ^ (z >> 27)) * C2) & MASK
    return z ^ (z >> 31)


def _unxorshift(y: int, s: int) -> int:
    x = y
    for _ in range(64 // s + 1):
        x = y ^ (x >> s)
    return x


def unmix64(h: int) -> int:
    """Inverse of the SplitMix64 finaliser (it is a bijection of 64-bit words)."""
    z = _unxorshift(h, 31)
    z = (z * pow(C2, -1, 1 << 64)) & MASK
    z = _unxorshift(z, 27)
    z = (z * pow(C1, -1, 1 << 64)) & MASK
    z = _unxorshift(z, 30)
    return (z - G) & MASK


def dbits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def f32(x) -> float:
    return float(np.float32(x))


# ---------------------------------------------------------------------------
# version 2: position-keyed inverse-CDF draw (spec 06 section 7)
# ---------------------------------------------------------------------------
def v2_closed_form(x, pos, T, top_k, top_p, min_p, seed, mutant=None):
    """Independent restatement: Python sort, Python integers for the hash,
    binary64 Python floats for the sums, exp_d from the pinned oracle."""
    order = sorted(range(len(x)), key=lambda i: (-float(x[i]), i))[:top_k]
    top = float(x[order[0]])
    w = [O.exp_d((float(x[i]) - top) / T) for i in order]
    total = 0.0
    for v in w:
        total += v
    n, prefix = len(order), 0.0
    for j, v in enumerate(w):
        prefix += v
        if prefix >= top_p * total:
            n = j + 1
            break
    if min_p > 0.0:
        m = 1
        while m < n and w[m] >= min_p:
            m += 1
        n = m
    kept = 0.0
    for v in w[:n]:
        kept += v
    h = mix64(seed ^ pos) if mutant == "no_inner_mix" else mix64(mix64(seed) ^ pos)
    u = float(h >> 11)
    if mutant == "plus_half":
        u = u + 0.5
    u = u * (1.0 / 9007199254740992.0)
    thr = u * kept
    pick, prefix = n - 1, 0.0
    for j in range(n):
        prefix += w[j]
        if (thr <= prefix) if mutant == "le" else (thr < prefix):
            pick = j
            break
    return order[pick], u, thr, kept


V2_CASES = [
    # (V, scale, T, top_k, top_p, min_p, seed)
    (40, 1.0, 1.0, 20, 0.95, 0.0, 0),
    (64, 2.5, 0.7, 20, 0.9, 0.05, 0x112345678),
    (300, 0.5, 1.5, 20, 1.0, 0.0, 77),
    (13, 3.0, 0.3, 13, 0.8, 0.0, 2**63 + 5),
]


@pytest.mark.parametrize("case", V2_CASES)
def test_v2_draw_matches_closed_form_over_many_positions(case):
    V, scale, T, k, tp, mp, seed = case
    rng = np.random.default_rng(V)
    x = (scale * rng.standard_normal(V)).astype(np.float32)
    p = O.params(temperature=T, top_k=k, top_p=tp, min_p=mp, seed=seed, version=O.INVERSE_CDF)
    positions = [int(v) for v in rng.integers(0, 2**63, 1500)] + [0, 1, 2**64 - 1, 2**32]
    for pos in positions:
        tok, d = O.sample(x, pos, p, diag=True)
        want, u, thr, kept = v2_closed_form(x, pos, T, k, tp, mp, seed)
        assert tok == want
        assert dbits(d.uniform) == dbits(u) and dbits(d.threshold) == dbits(thr)
        assert dbits(d.kept) == dbits(kept)


def _exact_half_position(seed: int) -> int:
    """A position whose uniform is exactly 0.5: h >> 11 == 2^52."""
    return unmix64(1 << 63) ^ mix64(seed)


def test_v2_threshold_equal_to_a_prefix_takes_the_next_candidate():
    # Two equal logits: weights [1, 1], kept = 2. At u = 0.5 the threshold is
    # exactly 1.0 = prefix_0, so the strict < skips candidate 0.
    x = np.array([5.0, 5.0], np.float32)
    for seed in (0, 9, 2**40 + 3):
        pos = _exact_half_position(seed)
        assert mix64(mix64(seed) ^ pos) >> 11 == 1 << 52
        p = O.params(top_k=2, top_p=1.0, seed=seed, version=O.INVERSE_CDF)
        tok, d = O.sample(x, pos, p, diag=True)
        assert d.uniform == 0.5 and d.threshold == 1.0
        assert tok == 1
        assert v2_closed_form(x, pos, 1.0, 2, 1.0, 0.0, seed)[0] == 1
        assert v2_closed_form(x, pos, 1.0, 2, 1.0, 0.0, seed, mutant="le")[0] == 0


@pytest.mark.parametrize("mutant", ["no_inner_mix", "plus_half", "le"])
def test_v2_planted_mistakes_are_caught(mutant):
    """Each mistake, planted in the closed form, disagrees with the oracle on
    the cases above: the comparison pins the oracle against it."""
    caught = False
    x2 = np.array([5.0, 5.0], np.float32)
    pos = _exact_half_position(0)
    p2 = O.params(top_k=2, top_p=1.0, seed=0, version=O.INVERSE_CDF)
    if v2_closed_form(x2, pos, 1.0, 2, 1.0, 0.0, 0, mutant)[0] != O.sample(x2, pos, p2):
        caught = True
    V, scale, T, k, tp, mp, seed = V2_CASES[0]
    x = (scale * np.random.default_rng(V).standard_normal(V)).astype(np.float32)
    p = O.params(temperature=T, top_k=k, top_p=tp, min_p=mp, seed=seed, version=O.INVERSE_CDF)
    for pos in range(400):
        tok, d = O.sample(x, pos, p, diag=True)
        m, u, thr, _ = v2_closed_form(x, pos, T, k, tp, mp, seed, mutant)
        if m != tok or dbits(u) != dbits(d.uniform):
            caught = True
            break
    assert caught


def test_version3_uses_plus_half_and_version2_does_not():
    for seed, pos in [(0, 0), (5, 17), (2**63, 2**40)]:
        h = mix64(mix64(seed) ^ pos)
        assert dbits(O.lib().yo_uniform_v2(seed, pos)) == dbits(float(h >> 11) * 2.0**-53)
        tok = 12345
        h3 = mix64(h ^ ((tok * 0xD6E8FEB86659FD93) & MASK))
        u3 = (float(h3 >> 11) + 0.5) * (1.0 / 9007199254740992.0)
        assert dbits(O.gumbel(seed, pos, tok)) == dbits(-O.log_d(-O.log_d(u3)))


# ---------------------------------------------------------------------------
# draft-side choice (draft_head.rs:325-379)
# ---------------------------------------------------------------------------
def choose_closed_form(scores, tokens, seed, t, pos, mutant=None):
    s = [float(np.float32(v)) for v in scores]
    best = 0
    for i in range(1, 16):
        if s[i] > s[best]:
            best = i
    order = sorted(range(16), key=lambda i: (-s[i], int(tokens[i])))
    T = (t / 1000.0) if mutant == "divide" else 0.001 * t
    z = [(s[i] - s[order[0]]) / T for i in range(16)]
    w = [O.exp_d(v) for v in z]
    total = 0.0
    for i in order:
        total += w[i]
    prefix, maximum = 0.0, -math.inf
    for i in order:
        if mutant == "after_add":
            prefix += w[i]
        if prefix < 0.95 * total:
            sc = z[i] + O.gumbel(seed, pos, int(tokens[i]))
            if sc > maximum:
                maximum, best = sc, i
        if mutant != "after_add":
            prefix += w[i]
    return int(tokens[best]), T, z, w, total


def _draft_case(rng, spread):
    scores = (spread * rng.standard_normal(16)).astype(np.float32)
    tokens = rng.permutation(248_320)[:16].astype(np.uint32)
    return scores, tokens


def test_draft_choice_matches_closed_form():
    rng = np.random.default_rng(31)
    for trial in range(300):
        scores, tokens = _draft_case(rng, [0.3, 1.0, 3.0][trial % 3])
        if trial % 7 == 0:
            scores[3] = scores[9]          # equal scores rank by token
        t = int(rng.integers(1, 2000))
        seed, pos = int(rng.integers(0, 2**64, dtype=np.uint64)), int(rng.integers(0, 2**40))
        tok, d = O.draft_choose_ex(scores, tokens, seed, t, pos)
        want, T, z, w, total = choose_closed_form(scores, tokens, seed, t, pos)
        assert tok == want
        assert dbits(d.temperature) == dbits(T)
        assert [dbits(d.z[i]) for i in range(16)] == [dbits(v) for v in z]
        assert [dbits(d.w[i]) for i in range(16)] == [dbits(v) for v in w]
        assert dbits(d.total) == dbits(total)


def test_draft_temperature_is_a_multiply_by_0_001():
    diff = []
    scores = np.linspace(1.0, -1.0, 16).astype(np.float32)
    tokens = np.arange(16, dtype=np.uint32)
    for t in range(1, 2001):
        _, d = O.draft_choose_ex(scores, tokens, 1, t, 0)
        assert dbits(d.temperature) == dbits(0.001 * t)
        if dbits(0.001 * t) != dbits(t / 1000.0):
            diff.append(t)
    assert diff, "the divide mutant must differ from the multiply for some thousandths"


def test_draft_membership_is_decided_before_the_weight_is_added():
    # Two live candidates (the rest far below): w = [1, w1] with w1 / (1 + w1)
    # about 0.09, so candidate 1 enters only if membership is tested before
    # its own weight is added (prefix 1 / (1 + w1) ~ 0.91 < 0.95).
    scores = np.full(16, -1000.0, np.float32)
    scores[0], scores[1] = 0.0, np.float32(-2.0 * 0.85)
    tokens = np.arange(100, 116, dtype=np.uint32)
    picks = {O.draft_choose(scores, tokens, 7, 850, pos) for pos in range(400)}
    assert picks == {100, 101}
    mutant = {choose_closed_form(scores, tokens, 7, 850, pos, "after_add")[0] for pos in range(400)}
    assert mutant == {100}
    _, d = O.draft_choose_ex(scores, tokens, 7, 850, 0)
    assert list(d.member)[:2] == [1, 1] and sum(d.member) == 2


def test_draft_choice_reference_known_answers():
    # crates/yskn-ref/tests/draft.rs:209-241
    ties_tokens = np.arange(15, -1, -1, dtype=np.uint32)  # (0..16).rev()
    ties = np.zeros(16, np.float32)
    assert O.draft_choose_ex(ties, ties_tokens, 0, 0, 8, greedy=True)[0] == 15
    dominant = ties.copy()
    dominant[7] = 100.0
    for seed in range(8):
        assert O.draft_choose(dominant, ties_tokens, seed, 850, 8) == int(ties_tokens[7])
    a = O.draft_choose(ties, ties_tokens, 314, 850, 8)
    assert O.draft_choose(ties[::-1].copy(), ties_tokens[::-1].copy(), 314, 850, 8) == a
    with pytest.raises(O.OracleError):
        O.draft_choose(ties, ties_tokens, 0, 0, 0)


# ---------------------------------------------------------------------------
# draft shortlist and top 16 (draft_head.rs:227-300)
# ---------------------------------------------------------------------------
def _key(x: float) -> int:
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    return (~u & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)


def shortlist_by_sort(scores, count):
    """The histogram cutoff finds the 21-bit key prefix of the count-th largest
    key; everything above it, then that prefix in ascending id order."""
    keys = [_key(float(s)) for s in np.asarray(scores, np.float32)]
    P = sorted(keys, reverse=True)[count - 1] >> 11
    above = [i for i, k in enumerate(keys) if (k >> 11) > P]
    bucket = [i for i, k in enumerate(keys) if (k >> 11) == P]
    return above + bucket[: count - len(above)]


def test_shortlist_reference_known_answers():
    # crates/yskn-ref/tests/draft.rs:169-192
    bits1 = struct.unpack("<I", struct.pack("<f", 1.0))[0]
    scores = np.array([struct.unpack("<f", struct.pack("<I", bits1 + i))[0] for i in range(31)] + [2.0],
                      np.float32)
    assert list(O.shortlist(scores, 16)) == [31] + list(range(15))
    scores[:16], scores[16:24], scores[24:] = -3.0, -2.0, -1.0
    assert list(O.shortlist(scores, 16)) == list(range(24, 32)) + list(range(16, 24))
    assert list(O.shortlist(np.zeros(32, np.float32), 24)) == list(range(24))
    with pytest.raises(O.OracleError):
        O.shortlist(np.zeros(32, np.float32), 17)
    with pytest.raises(O.OracleError):
        O.shortlist(np.full(32, np.nan, np.float32), 16)


@pytest.mark.parametrize("V,count", [(16, 16), (100, 24), (5000, 64), (70_000, 2048), (248_320, 256)])
def test_shortlist_equals_sort_based_cutoff(V, count):
    rng = np.random.default_rng(V + count)
    for trial in range(3):
        x = (rng.standard_normal(V) * [1.0, 1e-3, 50.0][trial]).astype(np.float32)
        if trial == 1:
            x[rng.integers(0, V, V // 3)] = x[0]      # a crowded cutoff bucket
        if trial == 2:
            x[: V // 4] = -0.0                        # -0 keys differ from +0 keys here
            x[V // 4: V // 2] = 0.0
        assert list(O.shortlist(x, count)) == shortlist_by_sort(x, count)


def test_top16_reference_known_answer_and_duplicates():
    # crates/yskn-ref/tests/draft.rs:195-208
    tokens = np.arange(31, -1, -1, dtype=np.uint32)
    scores = (tokens % 2).astype(np.float32)
    t, s = O.top16(tokens, scores)
    assert list(t) == [2 * i + 1 for i in range(16)]
    with pytest.raises(O.OracleError):
        O.top16(np.zeros(16, np.uint32), np.arange(16, dtype=np.float32))


# ---------------------------------------------------------------------------
# head epilogue arithmetic
# ---------------------------------------------------------------------------
def test_sqrt_rn_reference_vectors_and_correct_rounding():
    # portable_math.rs:468-485
    for a, e in [(0x00000000, 0x00000000), (0x80000000, 0x80000000), (0x3F800000, 0x3F800000),
                 (0x40000000, 0x3FB504F3), (0x40800000, 0x40000000), (0x00000001, 0x1A3504F3),
                 (0x00800000, 0x20000000), (0x7F7FFFFF, 0x5F7FFFFF)]:
        x = struct.unpack("<f", struct.pack("<I", a))[0]
        assert struct.unpack("<I", struct.pack("<f", O.sqrt_rn(x)))[0] == e
    assert O.rsqrt(4.0) == 0.5
    assert math.isnan(O.sqrt_rn(-1.0))
    # IEEE binary32 square root (numpy's is correctly rounded) on random bits,
    # subnormals included
    rng = np.random.default_rng(5)
    b = rng.integers(0, 0x7F800000, 20000, dtype=np.uint32)
    b[:2000] &= 0x007FFFFF
    xs = b.view(np.float32)
    want = np.sqrt(xs).view(np.uint32)
    got = np.array([O.sqrt_rn(float(v)) for v in xs], np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def test_inverse_rms_fold_order_and_rounding():
    rng = np.random.default_rng(8)
    for trial in range(200):
        sums = (np.abs(rng.standard_normal(10)) * 10.0 ** rng.integers(-3, 6)).astype(np.float32)
        if trial % 5 == 0:
            sums[0] = np.float32(3e7)                # later small terms are rounded against it
        tot = np.float32(0.0)
        for v in sums:
            tot = np.float32(tot + v)
        arg = np.float32(np.float32(tot / np.float32(5120.0)) + np.float32(1e-6))
        want = np.float32(np.float32(1.0) / np.sqrt(arg))
        assert O.inverse_rms(sums, 5120.0, 1e-6) == float(want)
    with pytest.raises(O.OracleError):
        O.inverse_rms(np.array([np.inf], np.float32), 5120.0, 1e-6)


def test_head_logits_conversion_and_scale_order():
    # int64 -> binary32 rounds to nearest, ties to even
    acc = np.array([2**24 + 1, 2**24 + 3, -(2**24 + 1), 2**53 + 2**29, 0, -1, 2**62], np.int64)
    tau = np.ones(acc.size, np.float32)
    got = O.head_logits(acc, tau, 1.0, 1.0)
    assert list(got[:3]) == [2.0**24, 2.0**24 + 4, -(2.0**24)]
    assert got[3] == np.float32(2.0**53)                   # tie, even significand kept
    rng = np.random.default_rng(2)
    acc = rng.integers(-(2**40), 2**40, 5000, dtype=np.int64)
    tau = (rng.random(5000) * 0.01).astype(np.float32)
    us, r = np.float32(3.1e-9), np.float32(0.37)
    got = O.head_logits(acc, tau, float(us), float(r))
    want = ((acc.astype(np.float32) * us) * r) * tau      # numpy: separately rounded binary32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # reassociating the three scales changes bits somewhere
    alt = acc.astype(np.float32) * ((us * r) * tau)
    assert not np.array_equal(alt.view(np.uint32), want.view(np.uint32))
    with pytest.raises(O.OracleError):
        O.head_logits(np.array([2**62], np.int64), np.array([1e30], np.float32), 1e10, 1.0)


# ---------------------------------------------------------------------------
# acceptance loop: checked position arithmetic (speculation.rs:489-497)
# ---------------------------------------------------------------------------
def test_verify_position_overflow_fails_only_when_reached():
    rows = np.array([[0.0, 1.0, 2.0], [2.0, 1.0, 0.0], [1.0, 2.0, 0.0]], np.float32)
    base = 2**64 - 3          # rows 0, 1 at 2^64 - 2, 2^64 - 1; row 2 would wrap
    sel, em, acc, _ = O.verify(rows, [2, 1], base, None)      # greedy; mismatch at row 1
    assert (list(sel), em, acc) == ([2, 0], 2, 1)
    with pytest.raises(O.OracleError) as e:
        O.verify(rows, [2, 0], base, None)                     # all match: row 2 is reached
    assert e.value.status == O.EINVAL
    # a non-finite row after the first mismatch is never sampled
    bad = rows.copy()
    bad[2, 1] = np.nan
    sel, em, acc, _ = O.verify(bad, [2, 1], 10, None)
    assert (list(sel), em) == ([2, 0], 2)
    with pytest.raises(O.OracleError):
        O.verify(bad, [2, 0], 10, None)
