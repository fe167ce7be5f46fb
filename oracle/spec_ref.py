"""Oracle: numpy restatement of goethe_engine/spec.py mss and the engine's tree-verify walk (test infrastructure).

  SALT_ACC/RES/DRAFT  spec.py:19
  mss                 spec.py:88-103   SpecInfer VerifyStochastic at one node: kid r accepted iff q(x) > 0 and
                                       uniform(mix(seed, SALT_ACC + r), i) * q(x) < p(x); a rejected kid replaces p by
                                       max(p - q, 0) / sum (one-hot q: p[x] = 0) when that sum is > 0; after the last kid
                                       draw(p, uniform(mix(seed, SALT_RES), i)) in vocabulary order
  verify_tree         engine.py:262-298 one request's walk from the anchor: a node with kids takes dist + mss (strict
                                       rejection request), a leaf takes sample(); the walk follows the accepted kid and
                                       the uniform index advances by one per committed token (nout)
"""
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
    """Children of every node (node 0 the anchor) in draft order; parents[j] is the parent node of node j + 1."""
    out = [[] for _ in range(len(parents) + 1)]
    for j, par in enumerate(parents):
        out[par].append(j + 1)
    return out


def verify_tree(target, qrows, tokens, parents, p, seed, nout0=0):
    """One strict request's acceptance walk (engine.py:262-298).

    target: fp32 [n_nodes + 1, V] target logits, row u for node u (0 = anchor); qrows: dict node -> fp64 [V] draft
    distribution its kids were drawn from (None entries: one-hot); tokens[j], parents[j]: node j + 1.
    Returns (emitted tokens, accepted path of nodes from the anchor)."""
    kids = kids_of(parents)
    u, nout, out, path = 0, nout0, [], [0]
    while True:
        if kids[u]:
            pd = dist(target[u], p)
            t, r = mss(pd, [(tokens[c - 1], qrows.get(u)) for c in kids[u]], seed, nout)
            hit = kids[u][r] if r is not None else None
        else:
            t = sample(target[u:u + 1], [p], [seed], [nout], [None])[0]
            hit = None
        out.append(t)
        nout += 1
        if t < 0 or hit is None:
            return out, path
        u = hit
        path.append(u)
