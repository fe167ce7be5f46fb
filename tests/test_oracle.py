"""Pins the CPU oracle (oracle/sampling_ref.py, oracle/spec_ref.py) before it is trusted as the parity checker:

  * golden vectors written by the reference's own sampling.py / spec.py (tests/golden/make_golden.py),
  * the independent C restatement (oracle/c/oracle.c) for splitmix64, the greedy masked argmax and the bit unpack,
  * known answers of the reference's tests (test_sampling.py:37-63) and hand-computed closed forms,
  * brute force in plain Python floats on tiny rows, distribution laws (4 sigma, chi-square) and invariances.
"""
import math
import random
from types import SimpleNamespace as NS

import numpy as np
import pytest

from oracle import cref
from oracle import sampling_ref as ora
from oracle import spec_ref as spo


def P(**kw):
    d = dict(temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, repetition_penalty=1.0, frequency_penalty=0.0,
             presence_penalty=0.0, logprobs=None)
    d.update(kw)
    return NS(**d)


# ---- golden vectors of the reference ----------------------------------------------------------------------------------

def test_mix_uniform_golden_and_c(golden):
    for a, s in enumerate(golden["mix_seed"]):
        for b, i in enumerate(golden["mix_idx"]):
            assert ora.mix(int(s), int(i)) == int(golden["mix_out"][a, b])
            assert ora.uniform(int(s), int(i)) == golden["uni_out"][a, b]
            assert cref.mix(int(s), int(i)) == int(golden["mix_out"][a, b])
            assert cref.uniform(int(s), int(i)) == golden["uni_out"][a, b]
    s = np.array([int(v) for v in golden["mix_seed"]], dtype=np.uint64)
    for b, i in enumerate(golden["mix_idx"]):
        got = np.array([ora.mix_np(int(x), int(i)) for x in s], dtype=np.uint64)
        assert (got == golden["mix_out"][:, b]).all()


def test_sample_tiny_golden(golden):
    x = golden["tiny_x"]
    for (t, k, p), want in zip(golden["tiny_params"], golden["tiny_tok"]):
        got = [ora.sample(x, [P(temperature=t, top_k=int(k), top_p=p)], [s], [0], [None])[0] for s in range(64)]
        assert got == list(want)


def _rows_params(g, prefix):
    return [P(temperature=float(t), top_k=int(k), top_p=float(p))
            for t, k, p in zip(g[prefix + "_T"], g[prefix + "_K"], g[prefix + "_TP"])]


def test_sample_rows_golden(golden):
    g = golden
    params = _rows_params(g, "rows")
    masks = [g["rows_mask"][r] if g["rows_has_mask"][r] else None for r in range(len(params))]
    for j in range(g["rows_seed"].shape[1]):
        got = ora.sample(g["rows_x"], params, [int(s) for s in g["rows_seed"][:, j]],
                         [int(i) for i in g["rows_idx"][:, j]], masks)
        assert got == list(g["rows_tok"][:, j])


def test_sample_edge_golden(golden):
    g = golden
    params = _rows_params(g, "edge")
    masks = [g["edge_mask"][r] if g["edge_has_mask"][r] else None for r in range(len(params))]
    with np.errstate(all="ignore"):
        for j in range(g["edge_tok"].shape[1]):
            got = ora.sample(g["edge_x"], params, [int(g["edge_seed"][j])] * len(params), [j] * len(params), masks)
            assert got == list(g["edge_tok"][:, j]), j


def test_dist_draw_mss_golden(golden):
    g = golden
    for r, (t, k, p) in enumerate(g["dist_params"]):
        m = g["dist_mask"][r] if g["dist_has_mask"][r] else None
        d = ora.dist(g["dist_x"][r], P(temperature=t, top_k=int(k), top_p=p), m)
        np.testing.assert_allclose(d, g["dist_out"][r], rtol=1e-15, atol=0)
    for r in range(g["draw_q"].shape[0]):
        for c, u in enumerate(g["draw_u"][r]):
            assert ora.draw(g["draw_q"][r], float(u)) == g["draw_out"][r, c]
    for n in range(g["mss_p"].shape[0]):
        kids = [(int(t), g["mss_q"][n, k] if g["mss_has_q"][n, k] else None)
                for k, t in enumerate(g["mss_tok"][n]) if t >= 0]
        t, r = spo.mss(g["mss_p"][n], kids, int(g["mss_seed"][n]), int(g["mss_i"][n]))
        assert (t, -1 if r is None else r) == (g["mss_out_tok"][n], g["mss_out_kid"][n])


# ---- independent restatement (C) ----------------------------------------------------------------------------------------

def test_greedy_matches_c_restatement():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, size=(40, 333)).astype(np.float32)
    x[1, 5] = np.nan
    x[2, :] = -np.inf
    x[3, 7] = np.inf
    x[4, 9] = np.inf
    x[4, 2] = np.inf
    x[5, :] = 1.25
    x[6, 100:] = np.float32(-3.4028235e38)
    x[7, 40] = np.nan
    m = rng.random((40, 333)) < 0.2
    m[8] = False
    m[7, 40] = False
    words = ora.pack_mask(m[0])
    assert (cref.unpack(words, 333) == m[0]).all() and (ora.unpack_mask(words, 333) == m[0]).all()
    wm = np.stack([ora.pack_mask(r) for r in m])
    for use_mask in (False, True):
        masks = [m[r] for r in range(40)] if use_mask else [None] * 40
        want = cref.greedy(x, wm if use_mask else None)
        got = ora.sample(x, [P()] * 40, [0] * 40, [0] * 40, masks)
        assert got == list(want)


# ---- reference test known answers and closed forms ------------------------------------------------------------------

def test_reference_known_answers():
    x = np.array([[5.0, 4.0, 3.0, 2.0, 1.0, 0.0]], np.float32)
    assert {ora.sample(x, [P(temperature=5.0, top_k=2)], [s], [0], [None])[0] for s in range(200)} == {0, 1}
    assert {ora.sample(x, [P(temperature=1.0, top_p=0.5)], [s], [0], [None])[0] for s in range(200)} == {0}
    assert {ora.sample(x, [P(temperature=1.0, top_k=1)], [s], [0], [None])[0] for s in range(50)} == {0}
    rng = np.random.default_rng(1)
    y = rng.normal(size=(3, 10)).astype(np.float32)
    m = np.zeros(10, bool)
    m[3] = True
    y[2, 4] = np.nan
    assert ora.sample(y, [P(), P(temperature=1.0), P()], [0, 1, 2], [0, 0, 0], [m, m, None]) == [3, 3, -1]
    assert ora.sample(y[:1], [P()], [0], [0], [np.zeros(10, bool)]) == [-1]


def _brute(x, t, k, p, u, minp=0.0):
    """Plain Python floats, written from sampling.py:59-83 semantics with an explicit sorted list (no numpy)."""
    z = [float(np.float32(v) / np.float32(t)) for v in x]
    order = sorted(range(len(z)), key=lambda i: (-z[i], i))
    e = [math.exp(z[i] - z[order[0]]) for i in order]
    s = math.fsum(e)
    q = [v / s for v in e]
    keep, acc = [], 0.0
    for r, v in enumerate(q):
        keep.append(r < (k or len(q)) and acc < p and v >= minp * q[0])
        acc += v
    c, tot = [], 0.0
    for v, kp in zip(q, keep):
        tot += v if kp else 0.0
        c.append(tot)
    j = max(min(sum(1 for v in c if v < u * c[-1]), sum(keep) - 1), 0)
    return order[j]


def test_brute_force_tiny_rows():
    rng = random.Random(3)
    for case in range(400):
        n = rng.randint(2, 9)
        x = [round(rng.gauss(0, 2), 1) for _ in range(n)]   # coarse values: ties happen
        t = rng.choice([0.3, 0.5, 1.0, 2.0])
        k = rng.choice([0, 1, 2, 3, 10])
        p = rng.choice([1.0, 0.9, 0.6, 0.3])
        mp = rng.choice([0.0, 0.0, 0.1, 0.5])
        u = rng.random()
        want = _brute(x, t, k, p, u, mp)
        got = ora.sample(np.array([x], np.float32), [P(temperature=t, top_k=k, top_p=p, min_p=mp)], [0], [0], [None],
                         uniforms=[u])[0]
        # a boundary within 1e-12 of u * c[-1] may round either way between math.fsum and numpy's pairwise sum
        if got != want:
            zz = np.array(x, np.float32) / np.float32(t)
            order, q = ora.sorted_p(np.array(x, np.float32), t)
            c = np.cumsum(q * ora.keep_mask(q, P(top_k=k, top_p=p, min_p=mp)))
            assert np.min(np.abs(c - u * c[-1])) < 1e-12, (case, x, t, k, p, mp, u, got, want, zz)


def test_draw_frequencies_follow_softmax():
    x = np.array([[1.0, 0.0, -1.0]], np.float32)
    n = 4000
    c = np.bincount([ora.sample(x, [P(temperature=1.0)], [7], [i], [None])[0] for i in range(n)], minlength=3)
    want = np.exp(x[0] - x[0].max())
    want = want / want.sum() * n
    assert (np.abs(c - want) < 4 * np.sqrt(want * (1 - want / n))).all()


def test_batch_and_permutation_invariance():
    rng = np.random.default_rng(5)
    x = rng.normal(size=(8, 64)).astype(np.float32)
    ps = [P(temperature=0.7 + i / 10, top_k=i % 4 * 5, top_p=1 - 0.1 * (i % 3), min_p=0.02 * (i % 2)) if i % 3 else P()
          for i in range(8)]
    seeds, idx = list(range(100, 108)), [i * 3 for i in range(8)]
    batch = ora.sample(x, ps, seeds, idx, [None] * 8)
    solo = [ora.sample(x[i:i + 1], ps[i:i + 1], seeds[i:i + 1], idx[i:i + 1], [None])[0] for i in range(8)]
    assert batch == solo
    perm = [5, 2, 7, 0, 1, 6, 3, 4]
    assert ora.sample(x[perm], [ps[i] for i in perm], [seeds[i] for i in perm], [idx[i] for i in perm],
                      [None] * 8) == [batch[i] for i in perm]


def test_penalties_known_answers():
    x = np.array([2.0, -2.0, 1.0, 0.0, 3.0], np.float32)
    y = ora.apply_penalties(x.copy(), [0, 1, 1, 3, 7, -1], rp=2.0, fp=0.5, pp=0.25)
    # t0: 2/2 - 0.5*1 - 0.25; t1: -2*2 - 0.5*2 - 0.25; t2, t4 untouched; t3: 0/2 - 0.5 - 0.25; ids 7, -1 ignored
    assert y.tolist() == [0.25, -5.25, 1.0, -0.75, 3.0]
    z = ora.apply_penalties(np.array([1.1, -1.1], np.float32), [0, 1], rp=1.1)
    assert z[0] == np.float32(1.1) / np.float32(1.1) and z[1] == np.float32(-1.1) * np.float32(1.1)
    # a penalised token changes the greedy choice
    row = np.array([[3.0, 2.9, 0.0]], np.float32)
    assert ora.sample(row, [P(frequency_penalty=0.2)], [0], [0], [None], history=[[0]]) == [1]
    assert ora.sample(row, [P()], [0], [0], [None], history=[[0]]) == [0]


def test_min_p_known_answer():
    # q proportional to [1, 0.5, 0.06, 0.04]: min_p 0.05 keeps ranks 0-2, so u near 1 draws token 2, never 3
    x = np.log(np.array([[1.0, 0.5, 0.06, 0.04]])).astype(np.float32)
    p = P(temperature=1.0, min_p=0.05)
    assert ora.sample(x, [p], [0], [0], [None], uniforms=[0.999999])[0] == 2
    assert ora.sample(x, [P(temperature=1.0)], [0], [0], [None], uniforms=[0.999999])[0] == 3
    d = ora.dist(x[0], p)
    assert d[3] == 0 and abs(d.sum() - 1) < 1e-15 and abs(d[0] / d[1] - 2.0) < 1e-6


def test_logprobs_match_torch_log_softmax():
    import torch
    rng = np.random.default_rng(9)
    x = rng.normal(0, 2, size=(4, 500)).astype(np.float32)
    res = ora.sample_full(x, [P(temperature=0.7, logprobs=20)] * 4, [0] * 4, [0] * 4, [None] * 4)
    for r in range(4):
        lp = torch.log_softmax(torch.from_numpy(x[r] / np.float32(0.7)).double(), 0)
        top = torch.sort(lp, descending=True, stable=True)
        assert res[r]["logprob_ids"].tolist() == top.indices[:20].tolist()
        np.testing.assert_allclose(res[r]["logprobs"], top.values[:20].float().numpy(), rtol=1e-6)


def test_dist_is_the_renormalised_kept_softmax():
    import torch
    rng = np.random.default_rng(11)
    x = rng.normal(0, 2, size=300).astype(np.float32)
    d = ora.dist(x, P(temperature=1.3, top_k=40, top_p=0.8))
    z = torch.from_numpy(x / np.float32(1.3)).double()
    q = torch.softmax(z, 0)
    order = torch.sort(z, descending=True, stable=True).indices
    qs = q[order]
    keep = (torch.arange(300) < 40) & (torch.cumsum(qs, 0) - qs < 0.8)
    want = torch.zeros(300, dtype=torch.float64)
    want[order[keep]] = qs[keep] / qs[keep].sum()
    np.testing.assert_allclose(d, want.numpy(), rtol=1e-12, atol=1e-300)


def test_mss_is_distribution_equal_to_the_target():
    """spec.py:88-103 law (SpecInfer): the accepted-or-resampled token is distributed as p (chi-square, 3 kids)."""
    v, n = 6, 12000
    rng = np.random.default_rng(2)
    p = rng.dirichlet(np.ones(v))
    q = rng.dirichlet(np.ones(v))
    counts = np.zeros(v)
    for s in range(n):
        kids = []
        for r in range(3):
            u = ora.uniform(s, 1 << 42 | r)
            kids.append((int(min(np.searchsorted(np.cumsum(q), u), v - 1)), q))
        t, _ = spo.mss(p, kids, s, 0)
        counts[t] += 1
    e = p * n
    stat = ((counts - e) ** 2 / e).sum()
    assert stat < (v - 1) + 6 * math.sqrt(2 * (v - 1)), stat


def test_chi2_has_power_against_a_residual_free_mss():
    v, n = 6, 6000
    rng = np.random.default_rng(2)
    p = rng.dirichlet(np.ones(v))
    q = rng.dirichlet(np.ones(v))
    counts = np.zeros(v)
    for s in range(n):
        u = ora.uniform(s, 1 << 42)
        counts[int(min(np.searchsorted(np.cumsum(q), u), v - 1))] += 1   # accept the draft always
    e = p * n
    assert ((counts - e) ** 2 / e).sum() > 10 * ((v - 1) + 6 * math.sqrt(2 * (v - 1)))


@pytest.mark.parametrize("seed", range(3))
def test_verify_tree_walk_follows_accepted_kids(seed):
    rng = np.random.default_rng(seed)
    v = 30
    parents = [0, 1, 2, 3, 0, 5, 6, 7]
    tgt = rng.normal(0, 1, size=(9, v)).astype(np.float32)
    qrows = {}
    toks = [0] * 8
    kids = spo.kids_of(parents)
    for u in range(9):
        if kids[u]:
            z = tgt[u].astype(np.float64) + rng.normal(0, 0.3, v)
            qrows[u] = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
            for k, c in enumerate(kids[u]):
                toks[c - 1] = int(rng.choice(v, p=qrows[u]))
    out, path, _ = spo.verify_tree(tgt, qrows, toks, parents, P(temperature=1.0, accept="rejection"), 1234 + seed)
    assert len(out) == len(path)
    for d in range(1, len(path)):
        assert toks[path[d] - 1] == out[d - 1] and parents[path[d] - 1] == path[d - 1]
