"""Pins the oracle's drafter-side selection (oracle/spec_ref.py pick, spec.py:151-159, and grow_dynamic, spec.py:183-204)
against the reference's own outputs (tests/golden/drafter_golden.npz, written by make_drafter_golden.py from
goethe_engine.spec.TreeDrafter on a toy model restated below) and against what the definitions fix: the stable
descending order with ties to the lowest id, the SALT_DRAFT uniform streams at the node's absolute index, and log q."""
import math
import os

import numpy as np
import pytest

from oracle import sampling_ref as ora
from oracle import spec_ref as spo

GOLD = os.path.join(os.path.dirname(__file__), "golden", "drafter_golden.npz")
M64 = (1 << 64) - 1


def _mix(seed, i):
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def toy_lp(seq, v):
    """The fixture's model: fp64 log-probabilities after seq, log_softmax(4 u), u splitmix64 uniforms of seq's hash."""
    h = 3
    for t in seq:
        h = _mix(h, int(t) + 1)
    u = np.array([(_mix(h, j) >> 11) / float(1 << 53) for j in range(v)])
    z = 4.0 * u
    return z - (z.max() + np.log(np.exp(z - z.max()).sum()))


def test_pick_matches_the_reference(gold):
    v = int(gold["V"])
    for c in range(len(gold["pick_n"])):
        seq = [int(t) for t in gold["pick_seq"][c]]
        n, t = int(gold["pick_n"][c]), float(gold["pick_t"][c])
        got = spo.pick(toy_lp(seq, v), n, t, int(gold["pick_seed"][c]), int(gold["pick_at"][c]))
        assert [g[0] for g in got] == [int(x) for x in gold["pick_tok"][c, :n]], c
        np.testing.assert_allclose([g[2] for g in got], gold["pick_lp"][c, :n], rtol=1e-13, atol=1e-13)


def test_grow_matches_the_reference(gold):
    v = int(gold["V"])
    for c in range(len(gold["grow_k"])):
        seq = [int(t) for t in gold["grow_seq"][c]]
        seed, k, t = int(gold["grow_seed"][c]), int(gold["grow_k"][c]), float(gold["grow_t"][c])
        n = int(gold["grow_len"][c])
        if gold["grow_dynamic"][c]:
            toks, par, _ = spo.grow_dynamic(lambda pt: toy_lp(seq + list(pt), v), seed, len(seq), k,
                                            int(gold["grow_topk"][c]), int(gold["grow_depth"][c]), t)
        else:
            toks = []
            for d in range(k):
                toks.append(spo.pick(toy_lp(seq + toks, v), 1, t, seed, len(seq) + d)[0][0])
            par = list(range(k))
        assert toks == [int(x) for x in gold["grow_tok"][c, :n]], c
        assert par == [int(x) for x in gold["grow_par"][c, :n]], c


def test_greedy_pick_is_the_stable_descending_order():
    """t == 0: the n best, ties to the lowest id (a sort of (-lp, id) pairs in plain Python)."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        lp = np.round(rng.normal(0, 1, 40), 1)  # many ties
        n = int(rng.integers(1, 12))
        want = sorted(range(40), key=lambda i: (-float(lp[i]), i))[:n]
        got = spo.pick(lp, n, 0.0, 5, 9)
        assert [g[0] for g in got] == want
        assert [g[2] for g in got] == [float(lp[i]) for i in want]


def test_sampled_pick_uses_the_drafter_streams_at_the_absolute_index():
    """t > 0 over four equal log-probabilities: q = 1/4 exactly, so draw r is the count of the exact prefixes
    {1/4, 1/2, 3/4, 1} below u_r, u_r = uniform(mix(seed, 2^42 + r), at) (a wrong salt or index changes it)."""
    lp = np.full(4, -math.log(4.0))
    for seed in (1, 77, 2 ** 40 + 5):
        for at in (0, 3, 1000):
            got = spo.pick(lp, 8, 1.0, seed, at)
            for r, (x, _, lq) in enumerate(got):
                u = (_mix(_mix(seed, (1 << 42) + r), at) >> 11) / float(1 << 53)
                assert x == sum(1 for c in (0.25, 0.5, 0.75, 1.0) if c < u), (seed, at, r)
                assert lq == math.log(0.25)


def test_sampled_pick_log_q_and_law():
    """log q[x] equals the log of the fp64 softmax in plain Python floats, and the draws follow q (chi-square)."""
    rng = np.random.default_rng(5)
    lp = rng.normal(0, 1.0, 12)
    t = 0.7
    zs = [float(x) / t for x in lp]
    m = max(zs)
    tot = math.fsum(math.exp(z - m) for z in zs)
    q = [math.exp(z - m) / tot for z in zs]
    counts = np.zeros(12)
    for seed in range(3000):
        for x, _, lq in spo.pick(lp, 2, t, seed, 4):
            assert abs(lq - math.log(q[x])) < 1e-12
            counts[x] += 1
    exp = 6000 * np.array(q)
    chi2 = float(((counts - exp) ** 2 / exp).sum())
    assert chi2 < 40.0, chi2  # 11 degrees of freedom: p < 1e-4 above 40
    assert ora.uniform(_mix(0, 1 << 42), 4) == (_mix(_mix(0, 1 << 42), 4) >> 11) / float(1 << 53)
