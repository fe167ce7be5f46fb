"""The drafter's proposal trees as the reference's scheduler and engine consume them (CPU).

The scheduler takes a drafter's proposals through as_tree, ok and fit (scheduler.py:128-133) and cuts them by budget
(scheduler.py:152); the engine walks kids() and hands tree.q[c - 1] to mss (engine.py:248-283). The oracle's Tree restates
that consumer side, spec.py:22-67 (pinned by the reference's known answers below), so that the drop-in's Tree and TreeDrafter are checked against what the reference's
own code would do with them. TreeDrafter's selection runs on the device; here it is replaced by the oracle's pick
(spec.py:151-159), so that the host logic that builds the trees is checked on the CPU."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora
from oracle import spec_ref as spo


RefTree, ref_as_tree = spo.Tree, spo.as_tree


def test_tree_known_answers(ge):
    """The reference's own known answers for Tree (tests/test_spec.py:21-27), on the oracle's Tree and the drop-in's."""
    V = 10
    for T in (RefTree, ge.spec.Tree):
        t = T([5, 6, 7, 8, 9], [0, 0, 1, 3, 2])
        assert t.kids() == [[1, 2], [3], [5], [4], [], []] and not t.is_chain and T.chain([1, 2]).is_chain
        f = t.fit(4, 2)
        assert f.tokens == [5, 6, 7, 9] and f.parents == [0, 0, 1, 2]
        assert not T([1], [1]).ok(V) and not T([V], [0]).ok(V) and t.ok(V)


def _random_tree(rng, n, v, with_q):
    parents = [int(rng.integers(0, j + 1)) for j in range(n)]
    tokens = [int(t) for t in rng.integers(0, v, size=n)]
    q = [object() for _ in range(n)] if with_q else None
    return tokens, parents, q


@pytest.mark.parametrize("seed", range(12))
def test_tree_methods_match_the_reference(ge, seed):
    rng = np.random.default_rng(seed)
    T = ge.spec.Tree
    for n in (0, 1, 5, 17):
        toks, par, q = _random_tree(rng, n, 100, seed % 2 == 1)
        a, b = T(list(toks), list(par), q), RefTree(list(toks), list(par), q)
        assert len(a) == len(b) and a.kids() == b.kids() and a.is_chain == b.is_chain
        assert a.ok(100) == b.ok(100) and a.ok(50) == b.ok(50)
        for m in (0, 1, 3, 20):
            ca, cb = a.cut(m), b.cut(m)
            assert (ca.tokens, ca.parents, ca.q) == (cb.tokens, cb.parents, cb.q)
            for depth in (0, 1, 2, 6):
                fa, fb = a.fit(m, depth), b.fit(m, depth)
                assert (fa.tokens, fa.parents, fa.q) == (fb.tokens, fb.parents, fb.q), (n, m, depth)
        c = ge.spec.as_tree(list(toks))
        assert (c.tokens, c.parents, c.q) == (list(toks), list(range(n)), None)
        assert ge.spec.as_tree(a) is a
    bad = T([1, 2], [0, 2])  # a parent after its node
    assert not bad.ok(10) and not RefTree([1, 2], [0, 2]).ok(10)


class _LM:
    """A tiny next-token model: log-probabilities of a hashed row (CPU tensor), with feed / release hooks."""

    def __init__(self, v):
        self.v, self.fed, self.released = v, [], []

    def dist(self, s, path):
        h = 3
        for t in list(s.tokens) + list(path):
            h = ora.mix(h, t + 1)
        u = ora.uniform_np(h, np.arange(self.v, dtype=np.uint64))
        z = (4.0 * u).astype(np.float32)
        return torch.from_numpy(z - np.float32(np.log(np.exp(z.astype(np.float64)).sum())))

    def feed(self, seq, pos, rows):
        self.fed.append((seq, pos, rows))

    def release(self, sid):
        self.released.append(sid)


def _oracle_pick_batch(x, n, t, seeds, ats):
    """pick_batch's contract on the CPU from the oracle's pick (spec.py:151-159)."""
    rows = x.shape[0]
    per = lambda v: list(v) if isinstance(v, (list, tuple, np.ndarray)) else [v] * rows
    nn, ss, aa = per(n), per(seeds), per(ats)
    nmax = max(int(k) for k in nn)
    toks = np.full((rows, nmax), -1, np.int32)
    vals = np.zeros((rows, nmax), np.float64)
    for r in range(rows):
        for k, (tok, _, lp) in enumerate(spo.pick(x[r].numpy().astype(np.float64), int(nn[r]), t, ss[r], aa[r])):
            toks[r, k], vals[r, k] = tok, lp
    return torch.from_numpy(toks), torch.from_numpy(vals)


@pytest.mark.parametrize("shape,t", [("chain", 0.0), ("chain", 1.0), ("dynamic", 0.0), ("dynamic", 0.8),
                                     ("static", 0.0), ("static", 1.0)])
def test_drafter_proposals_go_through_the_scheduler(ge, monkeypatch, shape, t):
    """propose() -> as_tree -> ok -> fit as scheduler.py:128-133 does, with the reference's Tree class injected and
    with the drop-in's own: the fitted trees hold the oracle's tokens and parents, and sampled children carry a q
    (QRef) per drafted token; static rank paths never sample (spec.py:171-181)."""
    from types import SimpleNamespace as NS
    monkeypatch.setattr(ge.spec, "pick_batch", _oracle_pick_batch)
    v, k = 3000, 6
    m = _LM(v)
    seqs = [NS(tokens=[5, 9, 2], seed=4242, sid=1), NS(tokens=[7], seed=77, sid=2)]
    choices = [(0,), (1,), (0, 0), (0, 1), (1, 0), (0, 0, 0)]
    for cls in (RefTree, None):
        d = ge.spec.TreeDrafter(m, shape, topk=3, depth=3, choices=choices, temperature=t, tree_cls=cls)
        for s, tr in zip(seqs, d.propose(seqs, k)):
            tr = ref_as_tree(tr)
            assert isinstance(tr, cls or ge.spec.Tree)
            assert tr.ok(v)
            fit = tr.fit(k, 3)
            at = len(s.tokens)
            lp = lambda pt: m.dist(s, pt).numpy().astype(np.float64)
            if shape == "chain":
                want_t = []
                for j in range(k):
                    want_t.append(spo.pick(lp(want_t), 1, t, s.seed, at + j)[0][0])
                want = (want_t[:3], [0, 1, 2])
            elif shape == "dynamic":
                wt, wp, _ = spo.grow_dynamic(lp, s.seed, at, k, 3, 3, t)
                want = RefTree(wt, wp).fit(k, 3)
                want = (want.tokens, want.parents)
            else:
                order = {}
                node, toks, par = {(): 0}, [], []
                for c in sorted(set(choices), key=lambda c: (len(c), c)):
                    if len(toks) == k or c[:-1] not in node:
                        continue
                    p = node[c[:-1]]
                    path, n = [], p
                    while n:
                        path.append(toks[n - 1])
                        n = par[n - 1]
                    if p not in order:
                        order[p] = list(np.argsort(-lp(path[::-1]), kind="stable"))
                    toks.append(int(order[p][c[-1]]))
                    par.append(p)
                    node[c] = len(toks)
                want = (toks, par)
            assert (fit.tokens, fit.parents) == want, (shape, t, cls)
            if t and shape != "static":
                assert fit.q is not None and all(isinstance(q, ge.spec.QRef) for q in fit.q)
                assert all(len(q) == v for q in fit.q)
            else:
                assert fit.q is None
        assert d.propose(seqs, 0)[0].tokens == []
    d.feed("seq", 3, "rows")
    d.release(9)
    assert m.fed == [("seq", 3, "rows")] and m.released == [9]
