"""MI355X drop-in for the acceptance step of goethe_engine/spec.py: SALT_* streams (spec.py:19) and mss (spec.py:88-103),
with the arithmetic in libgse.so (gse_mss), plus the batched form the engine's tree walk (engine.py:262-298) can use.

  mss(p, kids, seed, i)            one node: p the target distribution (fp64 [V]), kids [(token, q or None)] in draft
                                   order; returns (token, index of the accepted kid or None)
  mss_batch(p, kids, seeds, idxs)  many independent nodes in one launch
  verify_tree(...)                 strict-rejection acceptance walk of many requests' draft trees, level by level
"""
import ctypes as C

import numpy as np
import torch

from . import _lib
from .sampling import _device, dist_batch, sample_ex

SALT_ACC, SALT_RES, SALT_DRAFT = 1 << 40, 1 << 41, 1 << 42  # uniform streams: acceptance coins, residual, drafter


def _f64_rows(rows, dev):
    out = []
    for r in rows:
        t = r if isinstance(r, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(r, np.float64)))
        out.append(t.to(dev, torch.float64).reshape(-1))
    return torch.stack(out).contiguous() if out else None


def mss_batch(p, kids, seeds, idxs):
    """p: [n, V] target distributions (anything torch / numpy; copied, never modified); kids: per node a list of
    (token, q or None) in draft order; seeds, idxs: per node. Returns ([token], [kid index or None])."""
    dev = p.device if isinstance(p, torch.Tensor) and p.device.type == "cuda" else _device()
    pt = p if isinstance(p, torch.Tensor) else torch.from_numpy(np.asarray(p, np.float64))
    pt = pt.to(dev, torch.float64).reshape(len(kids), -1).clone()
    n, v = pt.shape
    kmax = max([len(k) for k in kids] + [1])
    ktok = np.full((n, kmax), -1, np.int32)
    kq = np.full((n, kmax), -1, np.int32)
    qs = []
    for a, ks in enumerate(kids):
        for r, (x, q) in enumerate(ks):
            ktok[a, r] = int(x)
            if q is not None:
                kq[a, r] = len(qs)
                qs.append(q)
    qt = _f64_rows(qs, dev)
    h = _lib.handle(dev.index, 1, v)
    ktok_d = torch.from_numpy(ktok).to(dev)
    kq_d = torch.from_numpy(kq).to(dev)
    seed_d = torch.from_numpy(np.array([int(s) & ((1 << 64) - 1) for s in seeds], np.uint64).view(np.int64)).to(dev)
    idx_d = torch.from_numpy(np.array([int(i) & ((1 << 64) - 1) for i in idxs], np.uint64).view(np.int64)).to(dev)
    otok = torch.empty(n, dtype=torch.int32, device=dev)
    okid = torch.empty(n, dtype=torch.int32, device=dev)
    b = _lib.MssBatch()
    b.size = C.sizeof(_lib.MssBatch)
    b.nodes, b.vocab, b.max_kids = n, v, kmax
    b.p, b.p_ld = pt.data_ptr(), pt.stride(0)
    b.q, b.q_ld = (qt.data_ptr(), qt.stride(0)) if qt is not None else (None, v)
    b.kid_tok, b.kid_q = ktok_d.data_ptr(), kq_d.data_ptr()
    b.seed, b.idx = seed_d.data_ptr(), idx_d.data_ptr()
    b.out_token, b.out_kid = otok.data_ptr(), okid.data_ptr()
    b.stream = torch.cuda.current_stream(dev).cuda_stream
    h.ck(h.L.gse_mss(h.h, C.byref(b)), "gse_mss")
    toks = otok.cpu().tolist()
    kid = [None if k < 0 else int(k) for k in okid.cpu().tolist()]
    return [int(t) for t in toks], kid


def mss(p, kids, seed, i):
    """Multi-step speculative sampling at one node (SpecInfer Algorithm 2 VerifyStochastic): p the target distribution,
    kids [(token, q or None: one-hot)] in draft order. Returns (token, index of the accepted kid or None)."""
    t, r = mss_batch(p if isinstance(p, torch.Tensor) else np.asarray(p, np.float64), [kids], [seed], [i])
    return t[0], r[0]


def kids_of(parents):
    """Children of every node (node 0 the anchor) in draft order; parents[j] is the parent node of node j + 1."""
    out = [[] for _ in range(len(parents) + 1)]
    for j, par in enumerate(parents):
        out[par].append(j + 1)
    return out


def verify_tree(reqs, nout0=0):
    """Acceptance walk of strict (rejection) requests, one tree level per round across all requests (engine.py:262-298).

    reqs: list of dict(target=[n_nodes + 1, V] logits (row u: the target after node u), q={node: draft distribution
    its kids were drawn from} (missing: one-hot), tokens, parents, params, seed). A node with kids takes dist + mss,
    a leaf takes sample() at the same uniform index (nout). Returns per request (emitted tokens, accepted node path)."""
    state = [dict(u=0, nout=nout0, out=[], path=[0], kids=kids_of(r["parents"])) for r in reqs]
    active = list(range(len(reqs)))
    while active:
        inner = [a for a in active if state[a]["kids"][state[a]["u"]]]
        leaf = [a for a in active if not state[a]["kids"][state[a]["u"]]]
        got = {}
        if inner:
            rows = torch.stack([_as_row(reqs[a]["target"], state[a]["u"]) for a in inner])
            pd = dist_batch(rows, [reqs[a]["params"] for a in inner])
            kids = []
            for a in inner:
                s = state[a]
                q = reqs[a].get("q", {}).get(s["u"])
                kids.append([(reqs[a]["tokens"][c - 1], q) for c in s["kids"][s["u"]]])
            toks, ks = mss_batch(pd, kids, [reqs[a]["seed"] for a in inner], [state[a]["nout"] for a in inner])
            for a, t, k in zip(inner, toks, ks):
                s = state[a]
                got[a] = (t, s["kids"][s["u"]][k] if k is not None else None)
        if leaf:
            rows = torch.stack([_as_row(reqs[a]["target"], state[a]["u"]) for a in leaf])
            sel = sample_ex(rows, [reqs[a]["params"] for a in leaf], [reqs[a]["seed"] for a in leaf],
                            [state[a]["nout"] for a in leaf], None).tolist()
            for a, t in zip(leaf, sel):
                got[a] = (t, None)
        nxt = []
        for a in active:
            t, hit = got[a]
            s = state[a]
            s["out"].append(t)
            s["nout"] += 1
            if t >= 0 and hit is not None:
                s["u"] = hit
                s["path"].append(hit)
                nxt.append(a)
        active = nxt
    return [(s["out"], s["path"]) for s in state]


def _as_row(x, u):
    t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float32)))
    if t.device.type != "cuda":
        t = t.to(_device())
    return t[u]
