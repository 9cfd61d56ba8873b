"""Draft-side selection through the C ABI (yskn_smp_draft_shortlist / _top16
/ _choose) against the oracle's restatement of draft_head.rs:219-379:
shortlist ids in their exact order, top-16 tokens and score bits, chosen
tokens (greedy and sampled) bit for bit, and the error rules. The runner-up
outputs follow the CUDA drafter's selection rule (q35_bdraft.cu:437-450),
restated here from the oracle's per-candidate z values and membership."""
import numpy as np
import pytest
import torch

import yskn_oracle as O
from gpu_helpers import to_u32
from yskn_smp import DeviceSampler, InvalidInput, NonFinite

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _shortlist_rows(V, seed):
    rng = np.random.default_rng(seed)
    rows = [
        (rng.standard_normal(V) * 3.0).astype(np.float32),                      # spread over binades
        np.round(rng.standard_normal(V) * 4.0).astype(np.float32) / 8,            # heavy ties
        np.full(V, 1.5, np.float32),                                             # one tie bucket
        np.where(rng.random(V) < 0.5, np.float32(-0.0), np.float32(0.0)).astype(np.float32),  # signed zeros
        (rng.standard_t(3, V) * 2.0).astype(np.float32),
    ]
    return np.stack(rows)


@pytest.mark.parametrize("V,count", [(248_320, 16), (248_320, 512), (248_320, 2048), (151_936, 64), (2048, 2048),
                                     (16, 16), (30_001, 1000)])
def test_shortlist_matches_the_oracle(V, count):
    x = _shortlist_rows(V, V + count)
    d = DeviceSampler(x.shape[0], 16)
    out = d.draft_shortlist(_t(x), count, row_status=True)
    d.sync()
    got = to_u32(out["ids"])
    for r in range(x.shape[0]):
        assert np.array_equal(got[r], O.shortlist(x[r], count)), r
    assert out["status"].cpu().tolist() == [0] * x.shape[0]
    d.close()


def test_shortlist_padded_rows_and_nonfinite():
    V, ld, count = 50_001, 50_048, 256
    rng = np.random.default_rng(3)
    buf = rng.standard_normal((3, ld)).astype(np.float32)
    buf[:, V:] = 1e30  # padding never read
    buf[1, 777] = np.nan
    xt = _t(buf)[:, :V]
    d = DeviceSampler(3, 16)
    out = d.draft_shortlist(xt, count, row_status=True)
    with pytest.raises(NonFinite):
        d.sync()
    assert out["status"].cpu().tolist() == [0, -2, 0]
    got = to_u32(out["ids"])
    assert np.array_equal(got[0], O.shortlist(buf[0, :V], count))
    assert np.array_equal(got[2], O.shortlist(buf[2, :V], count))
    assert (got[1] == 0xFFFFFFFF).all()
    with pytest.raises(O.OracleError):
        O.shortlist(buf[1, :V], count)
    for bad in (8, 15, 20, 2056):
        with pytest.raises(InvalidInput):
            d.draft_shortlist(xt, bad)
    with pytest.raises(InvalidInput):
        d.draft_shortlist(xt[:, :100], 104)
    d.close()


@pytest.mark.parametrize("n", [16, 17, 100, 2048, 4096])
def test_top16_matches_the_oracle(n):
    rows = 6
    rng = np.random.default_rng(n)
    tok = np.stack([rng.permutation(1 << 20)[:n] for _ in range(rows)]).astype(np.uint32)
    sc = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    sc[1] = np.round(sc[1] * 2) / 2                       # ties broken by token
    sc[2] = np.where(rng.random(n) < 0.5, np.float32(-0.0), np.float32(0.0))
    sc[3] = 7.0
    tok[4] = np.arange(n)[::-1] + 0xFFFFFFFF - n          # tokens near 2^32
    d = DeviceSampler(rows, 16)
    out = d.draft_top16(_t(tok.view(np.int32)), _t(sc), row_status=True)
    d.sync()
    gt, gs = to_u32(out["tokens"]), out["scores"].cpu().numpy()
    for r in range(rows):
        et, es = O.top16(tok[r], sc[r])
        assert np.array_equal(gt[r], et), r
        assert np.array_equal(gs[r].view(np.uint32), es.view(np.uint32)), r
    d.close()


def test_top16_rejects_duplicates_and_nonfinite():
    n = 300
    rng = np.random.default_rng(1)
    tok = np.stack([rng.permutation(5000)[:n] for _ in range(3)]).astype(np.uint32)
    sc = rng.standard_normal((3, n)).astype(np.float32)
    tok[0, 299] = tok[0, 3]          # duplicate token with a different score
    sc[2, 10] = np.inf
    d = DeviceSampler(3, 16)
    out = d.draft_top16(_t(tok.view(np.int32)), _t(sc), row_status=True)
    with pytest.raises(InvalidInput):
        d.sync()
    assert out["status"].cpu().tolist() == [-1, 0, -1]
    for r in (0, 2):
        with pytest.raises(O.OracleError):
            O.top16(tok[r], sc[r])
    assert np.array_equal(to_u32(out["tokens"])[1], O.top16(tok[1], sc[1])[0])
    with pytest.raises(InvalidInput):
        d.draft_top16(_t(tok[:, :15].view(np.int32)), _t(sc[:, :15]))
    d.close()


def _alternates(scores, tokens, seed, t, pos, greedy):
    """The CUDA drafter's runner-up rule (q35_bdraft.cu:437-450), restated:
    sampled -- member scores z + g in candidate order, the largest strictly;
    greedy -- raw scores in input order."""
    tok, diag = O.draft_choose_ex(scores, tokens, seed, t, pos, greedy=greedy)
    if greedy:
        b = int(np.argmax(scores))
        b2 = max((k for k in range(16) if k != b), key=lambda k: (scores[k], -k))
        b3 = max((k for k in range(16) if k not in (b, b2)), key=lambda k: (scores[k], -k))
        return tok, int(tokens[b2]), np.float32(scores[b] - scores[b2]), int(tokens[b3])
    order = [diag.order[i] for i in range(16)]
    val = {i: (diag.z[i] + O.gumbel(seed, pos, int(tokens[i]))) if diag.member[i] else -np.inf for i in range(16)}

    def first_best(excl):
        best, bi = -np.inf, -1
        for i in order:
            if i not in excl and val[i] > best:
                best, bi = val[i], i
        return best, bi

    vb, b = first_best(())
    assert int(tokens[b]) == tok
    v2, b2 = first_best((b,))
    if b2 < 0:
        return tok, -1, np.float32(1e30), -1
    v3, b3 = first_best((b, b2))
    return tok, int(tokens[b2]), np.float32(vb - v2), (int(tokens[b3]) if b3 >= 0 else -1)


@pytest.mark.parametrize("temp", [850, 1, 300, 1000, 5000, 60_000])
def test_choose_matches_the_oracle(temp):
    rows = 512
    rng = np.random.default_rng(temp)
    sc = (rng.standard_normal((rows, 16)) * 2).astype(np.float32)
    sc[::7] = np.round(sc[::7])                      # score ties, broken by token
    sc[::11, :4] = 3.0
    tok = rng.integers(0, 248_320, (rows, 16)).astype(np.uint32)
    tok[::13, 5] = tok[::13, 6]                      # a repeated token (allowed)
    pos = rng.integers(0, 2**63, rows, dtype=np.int64).astype(np.uint64)
    pos[0] = 2**64 - 1
    seed = int(rng.integers(0, 2**63)) * 2 + 1
    d = DeviceSampler(rows, 16)
    for greedy in (False, True):
        out = d.draft_choose(_t(sc), _t(tok.view(np.int32)), sampled=not greedy, seed=seed,
                             temperature_thousandths=temp, positions=torch.tensor(pos.view(np.int64)),
                             alternates=True)
        d.sync()
        got = to_u32(out["token"])
        alt, marg, alt3 = out["alt"].cpu().numpy(), out["margin"].cpu().numpy(), out["alt3"].cpu().numpy()
        for r in range(rows):
            et, ea, em, e3 = _alternates(sc[r], tok[r], seed, temp, int(pos[r]), greedy)
            assert got[r] == et, (greedy, r)
            assert alt[r] == ea and alt3[r] == e3, (greedy, r)
            assert marg[r].view(np.uint32) == em.view(np.uint32), (greedy, r, marg[r], em)
    d.close()


def test_choose_errors():
    rng = np.random.default_rng(5)
    sc = rng.standard_normal((3, 16)).astype(np.float32)
    tok = rng.integers(0, 1000, (3, 16)).astype(np.int32)
    sc[1, 15] = -np.inf
    d = DeviceSampler(3, 16)
    out = d.draft_choose(_t(sc), _t(tok), seed=1, positions=torch.arange(3), row_status=True)
    with pytest.raises(InvalidInput):
        d.sync()
    assert out["status"].cpu().tolist() == [0, -1, 0]
    with pytest.raises(InvalidInput):
        d.draft_choose(_t(sc), _t(tok), seed=1, temperature_thousandths=0, positions=torch.arange(3))
    with pytest.raises(InvalidInput):
        d.draft_choose(_t(sc[:, :15]), _t(tok[:, :15]), seed=1, positions=torch.arange(3))
    d.close()
