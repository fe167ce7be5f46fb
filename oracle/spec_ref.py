"""Oracle: numpy restatement of goethe_engine/spec.py (mss, the drafter's selection) and the engine's tree-verify walk
(test infrastructure, never product code).

  SALT_ACC/RES/DRAFT  spec.py:19
  mss                 spec.py:88-103   SpecInfer VerifyStochastic at one node: kid r accepted iff q(x) > 0 and
                                       uniform(mix(seed, SALT_ACC + r), i) * q(x) < p(x); a rejected kid replaces p by
                                       max(p - q, 0) / sum (one-hot q: p[x] = 0) when that sum is > 0; after the last kid
                                       draw(p, uniform(mix(seed, SALT_RES), i)) in vocabulary order
  verify_tree         engine.py:262-298 one request's walk from the anchor: a strict request (accept == "rejection" and
                                       temperature > 0, scheduler.py:67-70) at a node with kids takes dist + mss; every
                                       other node takes sample() and the walk follows the first kid holding its token.
                                       The uniform index is the number of tokens emitted so far (nout, engine.py:272,282),
                                       one more per committed token; the node's grammar mask applies to dist and sample
                                       (engine.py:272,280); a stop reason after a token ends the walk (engine.py:218-229,
                                       290-292); a token -1 ends it as an error (engine.py:286-288)
  pick                spec.py:151-159  the drafter's children of one node: temperature 0 -> the n best tokens of the
                                       log-probabilities (stable descending order); temperature t > 0 -> q = softmax(lp /
                                       t) in fp64 and n draws draw(q, uniform(mix(seed, SALT_DRAFT + r), at)), each with
                                       log q[x]
  grow_dynamic        spec.py:183-204  EAGLE-2 expand + rerank of a proposal tree from pick()
  Tree / as_tree      spec.py:22-67    the proposal tree as the scheduler consumes it (scheduler.py:128-133: as_tree,
                                       ok, fit; cut at :152) and the engine walks it (kids, tokens, q)

The walk is pinned in tests/test_oracle_walk.py by the joint law of its emitted tokens (chi-square against the product
of the target's dist(), with power controls) and by known answers that fix which uniform index each depth uses. pick and
grow_dynamic are pinned in tests/test_oracle_drafter.py against the reference's own TreeDrafter outputs on a toy model
(tests/golden/drafter_golden.npz) and by the stable order, the SALT_DRAFT streams and log q in closed form. mss is
pinned by the golden vectors of tests/test_oracle.py. Tree is pinned by the known answers of the reference's
tests/test_spec.py:21-27 (kids, fit, ok) in tests/test_spec_tree.py.
"""
from dataclasses import dataclass

import numpy as np

from .sampling_ref import dist, draw, mix, sample, uniform

SALT_ACC, SALT_RES, SALT_DRAFT = 1 << 40, 1 << 41, 1 << 42


def mss(p, kids, seed, i):
    """spec.py:88-103. p: fp64 [V]; kids: [(token, q fp64 [V] or None for one-hot)] in draft order."""
    p = np.asarray(p, dtype=np.float64)
    for r, (x, q) in enumerate(kids):
        qx = 1.0 if q is None else float(q[x])
        if qx > 0 and uniform(mix(seed, SALT_ACC + r), i) * qx < float(p[x]):
            return x, r
        res = np.array(p, dtype=np.float64)
        if q is None:
            res[x] = 0
        else:
            res = np.maximum(p - np.asarray(q, dtype=np.float64), 0)
        if res.sum() > 0:
            p = res / res.sum()
    return draw(p, uniform(mix(seed, SALT_RES), i)), None


def kids_of(parents):
    """Children of every node (node 0 the anchor) in draft order; parents[j] is the parent node of node j + 1
    (spec.py:51-56)."""
    out = [[] for _ in range(len(parents) + 1)]
    for j, par in enumerate(parents):
        out[par].append(j + 1)
    return out


def depths(parents):
    """Depth of every node, node 0 (the anchor) at depth 0."""
    d = [0]
    for par in parents:
        d.append(d[par] + 1)
    return d


def is_strict(p):
    """scheduler.py:67-70: rejection acceptance at temperature > 0."""
    return getattr(p, "accept", "exact") == "rejection" and p.temperature > 0


def _kid_q(q, u, c):
    """The distribution kid c of node u was drawn from: q is a per-drafted-node list (Tree.q, spec.py:26: q[c - 1]) or
    a dict node -> the distribution shared by its kids; None: one-hot."""
    if q is None:
        return None
    if isinstance(q, dict):
        return q.get(u)
    return q[c - 1]


def verify_tree(target, q, tokens, parents, p, seed, nout0=0, masks=None, stop=None, history=None):
    """One request's acceptance walk (engine.py:262-298).

    target: fp32 [n_nodes + 1, V], row u the target logits after node u (0 = the anchor); q: the draft distributions
    (see _kid_q); tokens[j], parents[j]: node j + 1; masks: per node a bool [V] mask (the grammar's state after the path
    to that node) or None; history: per node the penalty history of that row or None; stop(emitted) -> a reason or None
    after each emitted token. Returns (emitted tokens, accepted path of nodes from the anchor, reason): reason is None
    when the walk ended at a node whose token no kid holds (or a leaf), "error" for a token -1 (not emitted), else what
    stop returned."""
    kids = kids_of(parents)
    strict = is_strict(p)
    u, nout, out, path = 0, nout0, [], [0]
    while True:
        m = masks[u] if masks is not None else None
        hist = history[u] if history is not None else None
        if strict and kids[u]:
            pd = dist(target[u], p, m, hist)
            t, r = mss(pd, [(tokens[c - 1], _kid_q(q, u, c)) for c in kids[u]], seed, nout)
            hit = kids[u][r] if r is not None else None
        else:
            t = sample(target[u:u + 1], [p], [seed], [nout], [m], [hist] if hist is not None else None)[0]
            hit = next((c for c in kids[u] if tokens[c - 1] == t), None) if t >= 0 else None
        if t < 0:
            return out, path, "error"
        out.append(t)
        nout += 1
        why = stop(out) if stop is not None else None
        if why:
            return out, path, why
        if hit is None:
            return out, path, None
        u = hit
        path.append(u)


def pick(lp, n, t, seed, at):
    """spec.py:151-159: n children of a node whose next token sits at absolute index at, as (token, q, log-prob)."""
    lp = np.asarray(lp, dtype=np.float64)
    if t == 0:
        top = np.argsort(-lp, kind="stable")[:n]
        return [(int(x), None, float(lp[x])) for x in top]
    z = lp / t
    e = np.exp(z - z.max())
    q = e / e.sum()
    xs = [draw(q, uniform(mix(seed, SALT_DRAFT + r), at)) for r in range(n)]
    return [(x, q, float(np.log(q[x]))) for x in xs]


def grow_dynamic(dist_fn, seed, at, k, topk, depth, t):
    """spec.py:183-204 (EAGLE-2): expand the topk best of each level by cumulative log-probability, rerank every
    candidate, keep the k best whose parent is kept. dist_fn(path) -> log-probabilities after the drafted path.
    Returns (tokens, parents, q list or None)."""
    cand = []  # (score, token, parent candidate index or -1, q)
    beam = [-1]
    for _ in range(depth):
        new = []
        for b in beam:
            pt = _cpath(cand, b)
            for x, qq, l in pick(dist_fn(pt), topk, t, seed, at + len(pt)):
                new.append((l + (cand[b][0] if b >= 0 else 0.0), x, b, qq))
        base = len(cand)
        cand += new
        beam = sorted(range(base, len(cand)), key=lambda i: (-cand[i][0], i))[:topk]
    keep, sel = {}, []
    for i in sorted(range(len(cand)), key=lambda i: (-cand[i][0], i)):
        if len(sel) == k:
            break
        if cand[i][2] < 0 or cand[i][2] in keep:
            keep[i] = None
            sel.append(i)
    sel.sort()
    idx = {i: j + 1 for j, i in enumerate(sel)}
    return ([cand[i][1] for i in sel], [idx.get(cand[i][2], 0) for i in sel],
            [cand[i][3] for i in sel] if t else None)


def _cpath(cand, b):
    out = []
    while b >= 0:
        out.append(cand[b][1])
        b = cand[b][2]
    return out[::-1]


@dataclass
class Tree:
    """spec.py:22-63: drafted tokens (node j + 1) with their parent nodes (0 the anchor) and the distribution each was
    drawn from (None: deterministic)."""
    tokens: list
    parents: list
    q: list | None = None

    @staticmethod
    def chain(tokens, q=None):
        return Tree(list(tokens), list(range(len(tokens))), q)

    def __len__(self):
        return len(self.tokens)

    def cut(self, n):
        return Tree(self.tokens[:n], self.parents[:n], self.q[:n] if self.q else None)

    def fit(self, n, depth):
        d, idx, toks, par, qs = [0], {0: 0}, [], [], []
        for i, (t, p) in enumerate(zip(self.tokens, self.parents)):
            d.append(d[p] + 1)
            if len(toks) < n and p in idx and d[-1] <= depth:
                idx[i + 1] = len(toks) + 1
                toks.append(t)
                par.append(idx[p])
                qs.append(self.q[i] if self.q else None)
        return Tree(toks, par, qs if self.q else None)

    @property
    def is_chain(self):
        return self.parents == list(range(len(self.parents)))

    def kids(self):
        return kids_of(self.parents)

    def ok(self, vocab):
        return (len(self.parents) == len(self.tokens) and all(0 <= p <= i for i, p in enumerate(self.parents))
                and all(0 <= t < vocab for t in self.tokens) and (self.q is None or len(self.q) == len(self.tokens)))


def as_tree(x):
    """spec.py:66-67: a Tree as is (any object with the Tree methods), a token list as a chain."""
    return x if hasattr(x, "fit") else Tree.chain(x)
