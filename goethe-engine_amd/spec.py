"""MI355X drop-in for the speculative-decoding selection of goethe_engine/spec.py and engine.py: the SALT_* streams
(spec.py:19), mss (spec.py:88-103), the engine's acceptance walk (engine.py:262-298) and the drafter's child selection
(spec.py:151-159), with the arithmetic in libgse.so.

  mss(p, kids, seed, i)            one node (gse_mss): p the target distribution (fp64 [V]), kids [(token, q or None)]
                                   in draft order; returns (token, index of the accepted kid or None)
  mss_batch(p, kids, seeds, idxs)  many independent nodes in one launch
  verify_tree(reqs, ...)           one verify round of many requests' draft trees in one call (gse_verify_tree): every
                                   node decided on the device, the walk done there, one copy of the results back
  pick_batch(x, n, t, seeds, ats)  the drafter's children of many nodes in one call (gse_draft_pick)
  qprob(x, t)                      q = softmax(float64(x) / t) of drafter rows on the device (gse_qprob)
  Tree / as_tree                   spec.py:22-67: the proposal tree the scheduler fits and the engine walks
  TreeDrafter                      spec.py:125-216 with its selection on the device (chain / static / dynamic shapes);
                                   propose() returns Tree objects whose q entries (sampled children) are QRefs, which
                                   mss(), mss_batch() and numpy read
"""
from dataclasses import dataclass
import ctypes as C

import numpy as np
import torch

from . import _lib
from .sampling import M64, _device, _history, _logits, _masks, _rows, dist_batch, sample_ex  # noqa: F401

SALT_ACC, SALT_RES, SALT_DRAFT = 1 << 40, 1 << 41, 1 << 42  # uniform streams: acceptance coins, residual, drafter


def _f64_rows(rows, dev):
    out = []
    for r in rows:
        if isinstance(r, QRef):
            t = r.prob()
        else:
            t = r if isinstance(r, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(r, np.float64)))
        out.append(t.to(dev, torch.float64).reshape(-1))
    return torch.stack(out).contiguous() if out else None


def _u64(vals, dev):
    return torch.from_numpy(np.array([int(v) & M64 for v in vals], np.uint64).view(np.int64)).to(dev)


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
            if not 0 <= int(x) < v:
                raise ValueError(f"kid token {x} outside the vocabulary of {v}")
            ktok[a, r] = int(x)
            if q is not None:
                kq[a, r] = len(qs)
                qs.append(q)
    qt = _f64_rows(qs, dev)
    h = _lib.handle(dev.index, 1, v)
    ktok_d = torch.from_numpy(ktok).to(dev)
    kq_d = torch.from_numpy(kq).to(dev)
    seed_d, idx_d = _u64(seeds, dev), _u64(idxs, dev)
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
    h.call("gse_mss", C.byref(b))
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


def strict(p):
    """scheduler.py:67-70: rejection acceptance at temperature > 0 (such nodes with kids take dist + mss)."""
    return getattr(p, "accept", "exact") == "rejection" and p.temperature > 0


def qprob(x, t):
    """q = softmax(float64(x) / t) (spec.py:157) of drafter rows x [rows, V] (device tensor, fp32 or bf16, or anything
    torch / numpy) at per-row temperatures t > 0 (a list, or one value): an fp64 [rows, V] device tensor (gse_qprob)."""
    xt, code = _logits(x)
    rows, v = xt.shape
    dev = xt.device
    ts = [float(k) for k in (t if isinstance(t, (list, tuple, np.ndarray)) else [t] * rows)]
    if len(ts) != rows or not all(k > 0 for k in ts):
        raise ValueError("qprob needs one temperature > 0 per row")
    tt = torch.tensor(ts, dtype=torch.float64, device=dev)
    out = torch.empty((rows, v), dtype=torch.float64, device=dev)
    q = _lib.QRows()
    q.size = C.sizeof(_lib.QRows)
    q.kind = _lib.Q_LOGITS_BF16 if code == _lib.BF16 else _lib.Q_LOGITS_F32
    q.rows, q.q, q.ld, q.temperature = rows, xt.data_ptr(), xt.stride(0), tt.data_ptr()
    h = _lib.handle(dev.index, 1, v)
    h.call("gse_qprob", C.byref(q), v, out.data_ptr(), out.stride(0), _lib.stream_of(dev.index))
    return out


class QRef:
    """A draft distribution held as the drafter's logits row on the device: q = softmax(float64(x) / t) (spec.py:157).
    verify_tree reads it without materialising it; mss / mss_batch, q[i] and numpy (np.asarray(q), so the reference's
    mss and host() too) read the fp64 row, computed on the device once (gse_qprob). pick_batch's callers make these the
    q of the children they draw."""

    __slots__ = ("x", "t", "_q")

    def __init__(self, x, t):
        self.x, self.t, self._q = x, float(t), None

    def prob(self):
        """q as an fp64 [V] device tensor."""
        if self._q is None:
            self._q = qprob(self.x.reshape(1, -1), [self.t])[0]
        return self._q

    def __len__(self):
        return int(self.x.numel())

    def __getitem__(self, i):
        return float(self.prob()[i])

    def __array__(self, dtype=None, copy=None):
        a = self.prob().cpu().numpy()
        return a if dtype is None else a.astype(dtype)


@dataclass
class Tree:
    """The proposal tree of spec.py:22-67, with the same fields and methods, so that the reference's scheduler
    (scheduler.py:128-133: as_tree, ok, fit; cut at :152) and engine (engine.py:248-282: kids, tokens, q) take it: node 0
    is the anchor, tokens[j] is node j + 1 with parent node parents[j] < j + 1; q[j] is the distribution tokens[j] was
    drawn from (fp64 [V] or a QRef), None for a deterministic drafter."""

    tokens: list
    parents: list
    q: list | None = None

    @staticmethod
    def chain(tokens, q=None):
        return Tree(list(tokens), list(range(len(tokens))), q)

    def __len__(self):
        return len(self.tokens)

    def cut(self, n):
        """The first n drafted nodes (parents come before children, so it is still a tree)."""
        return type(self)(self.tokens[:n], self.parents[:n], self.q[:n] if self.q else None)

    def fit(self, n, depth):
        """At most n nodes no deeper than depth, in draft order, renumbered; a node is kept only with its parent."""
        depth_of, new_id = [0], {0: 0}
        toks, par, qs = [], [], []
        for j, (t, p) in enumerate(zip(self.tokens, self.parents)):
            depth_of.append(depth_of[p] + 1)
            if len(toks) < n and p in new_id and depth_of[-1] <= depth:
                new_id[j + 1] = len(toks) + 1
                toks.append(t)
                par.append(new_id[p])
                qs.append(self.q[j] if self.q else None)
        return type(self)(toks, par, qs if self.q else None)

    @property
    def is_chain(self):
        return list(self.parents) == list(range(len(self.parents)))

    def kids(self):
        """Children of every node (node 0 the anchor) in draft order."""
        return kids_of(self.parents)

    def ok(self, vocab):
        """Well formed over a vocabulary: one parent per token, each an earlier node, tokens in range, q per token."""
        return (len(self.parents) == len(self.tokens) and all(0 <= p <= j for j, p in enumerate(self.parents))
                and all(0 <= t < vocab for t in self.tokens) and (self.q is None or len(self.q) == len(self.tokens)))


def as_tree(x):
    """A Tree as is; a token list as a chain (spec.py:66-67)."""
    return x if isinstance(x, Tree) else Tree.chain(x)


def _per_node(v, n):
    """A per-node option given as a list (node u at index u), a dict {node: value} or one value for every node."""
    if v is None:
        return [None] * n
    if isinstance(v, dict):
        return [v.get(u) for u in range(n)]
    if isinstance(v, (list, tuple)) and len(v) == n:
        return list(v)
    return [v] * n


def _per_node_history(hv, n):
    """History per node: None; one id sequence for every node; or a dict / length-n list of per-node sequences."""
    if hv is None:
        return [None] * n
    if isinstance(hv, dict):
        return [hv.get(u) for u in range(n)]
    if isinstance(hv, (list, tuple)) and len(hv) == n and all(h is None or not np.isscalar(h) for h in hv):
        return list(hv)
    return [hv] * n


def verify_tree(reqs, nout0=0, stop=None, emit_ld=None):
    """One verify round (engine.py:262-298) of many requests, in one gse_verify_tree call.

    reqs: list of dict(target=[n_nodes + 1, V] target logits (row u: after node u; a device tensor is used in place
    when it is one contiguous block), tokens=[drafted token of node j + 1], parents=[parent node of node j + 1],
    params=SamplingParams, seed=int, and optionally q= the draft distributions (spec.py Tree.q: per drafted node an fp64
    [V] or None (one-hot), or a QRef; or a dict {node: distribution its kids were drawn from}), draft= [n_nodes + 1, V]
    drafter logits with draft_t= t (the kids of node u were drawn from softmax(draft[u] / t), SpecInfer), masks= per node
    grammar masks (bool [V] / packed int32; list or dict), history= penalty history (one list for every node, or per
    node), nout= this request's nout0).
    stop: optional stop(request index, emitted tokens) -> reason or None, applied after each emitted token as
    engine.py:218-229 does; the walk of that request ends there (the tokens before it do not depend on the rest).
    Returns per request (emitted tokens, accepted path of nodes from the anchor, reason): reason "error" when a node had
    no valid token (engine.py:286-288, the -1 is not emitted), what stop returned, or None."""
    if not reqs:
        return []
    call = VerifyCall(reqs, nout0, emit_ld)
    call.launch()
    return call.result(stop)


class VerifyCall:
    """verify_tree's device call with its inputs resident: built once from the requests (the same arguments as
    verify_tree), launch() enqueues gse_verify_tree on the current stream (as often as wanted: the inputs are left as
    they are), result(stop) copies the emitted tokens back (one copy) and applies the stop predicate."""

    def __init__(self, reqs, nout0=0, emit_ld=None):
        if not reqs:
            raise ValueError("no requests")
        self._build(reqs, nout0, emit_ld)

    def launch(self):
        self.b.stream = torch.cuda.current_stream(self.dev).cuda_stream
        h = _lib.handle(self.dev.index, self.nodes, self.vocab)  # (this stream's handle, grown by other calls or not)
        h.call("gse_verify_tree", C.byref(self.b), C.byref(self.t), C.byref(self.o))

    def result(self, stop=None):
        out = torch.cat([self.e_len[:, None], self.e_st[:, None], self.e_tok, self.e_node], 1).cpu().numpy()
        ld, anchors = self.ld, self.anchors
        res = []
        for a in range(self.n_req):
            n, stt = int(out[a, 0]), int(out[a, 1])
            tk = [int(v) for v in out[a, 2:2 + min(n, ld)]]
            nd = [int(v) - int(anchors[a]) for v in out[a, 2 + ld:2 + ld + min(n, ld)]]
            why = None
            if stt == _lib.WALK_KIDS:
                raise RuntimeError(f"gse_verify_tree: request {a} reached a node with more kids than max_kids")
            if stt == _lib.WALK_ERROR:  # the path also holds the node whose row had no valid token
                why = "error"
                if n < ld:
                    nd.append(int(out[a, 2 + ld + n]) - int(anchors[a]))
            if stop is not None:
                for d in range(len(tk)):
                    w = stop(a, tk[:d + 1])
                    if w:
                        tk, nd, why = tk[:d + 1], nd[:d + 1], w
                        break
            res.append((tk, nd, why))
        return res

    def _build(self, reqs, nout0, emit_ld):
        dev = _device()
        sizes = [len(r["tokens"]) + 1 for r in reqs]
        anchors = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int32)
        nodes = int(sum(sizes))
        parents = np.full(nodes, -1, np.int32)
        toks = np.zeros(nodes, np.int32)
        qrow = np.full(nodes, -1, np.int32)
        params, seeds, idxs, masks, hists = [], [], [], [], []
        qprob, qlog, qtemp, qkey = [], [], [], {}
        max_kids = 1
        for a, r in enumerate(reqs):
            n, base, p = sizes[a], int(anchors[a]), r["params"]
            par = list(r["parents"])
            if len(par) != n - 1 or not all(0 <= q <= j for j, q in enumerate(par)):
                raise ValueError(f"request {a}: parents must give node j + 1 a parent in [0, j]")
            kids = kids_of(par)
            max_kids = max(max_kids, max(len(k) for k in kids))
            depth = [0] * n
            for j, q in enumerate(par):
                depth[j + 1] = depth[q] + 1
                parents[base + j + 1] = base + q
            toks[base + 1:base + n] = r["tokens"]
            n0 = int(r.get("nout", nout0))
            qsrc = r.get("q")
            for u in range(n):
                params.append(p)
                seeds.append(r["seed"])
                idxs.append(n0 + depth[u])
            for j in range(1, n):
                c_parent = par[j - 1]
                qd = None
                if r.get("draft") is not None:
                    qd = ("draft", a, c_parent)
                elif isinstance(qsrc, dict):
                    qd = qsrc.get(c_parent)
                elif qsrc is not None:
                    qd = qsrc[j - 1]
                if qd is None:
                    continue
                if isinstance(qd, tuple):  # the request's drafter logits row of the parent
                    key = qd
                    if key not in qkey:
                        qkey[key] = len(qlog)
                        qlog.append(_as_row(r["draft"], c_parent, dev))
                        qtemp.append(float(r.get("draft_t", 1.0)))
                elif isinstance(qd, QRef):
                    key = ("ref", id(qd))
                    if key not in qkey:
                        qkey[key] = len(qlog)
                        qlog.append(qd.x.reshape(-1))
                        qtemp.append(qd.t)
                else:
                    key = ("prob", id(qd))
                    if key not in qkey:
                        qkey[key] = len(qprob)
                        qprob.append(qd)
                qrow[base + j] = qkey[key]
            masks += _per_node(r.get("masks"), n)
            hists += _per_node_history(r.get("history"), n)
        if qprob and qlog:
            raise ValueError("one verify call takes its draft distributions either as fp64 rows or as drafter logits")
        if max_kids > _lib.MAX_KIDS:
            raise ValueError(f"a node with {max_kids} kids; at most {_lib.MAX_KIDS}")
        x = _stack_targets([r["target"] for r in reqs], sizes, dev)
        x, code = _logits(x)
        v = x.shape[1]
        if np.any((toks < 0) | (toks >= v)):
            raise ValueError("drafted token outside the vocabulary")
        h = _lib.handle(dev.index, nodes, v)
        hist_dev, offs = _history(hists if any(hh is not None for hh in hists) else None, nodes, dev)
        rows = _rows(params, seeds, idxs, offs)
        for a, r in enumerate(reqs):
            if strict(r["params"]):
                base = int(anchors[a])
                for u, k in enumerate(kids_of(list(r["parents"]))):
                    if k:
                        rows["flags"][base + u] |= _lib.ROW_MSS
        mask_dev, mask_ld = _masks(h, masks if any(m is not None for m in masks) else None, nodes, v, dev, rows)
        rows_dev = torch.from_numpy(rows.view(np.uint8)).to(dev, non_blocking=True)
        b = _lib.Batch()
        b.size = C.sizeof(_lib.Batch)
        b.dtype, b.rows, b.vocab, b.ld = code, nodes, v, x.stride(0)
        b.logits, b.params = x.data_ptr(), rows_dev.data_ptr()
        b.mask = mask_dev.data_ptr() if mask_dev is not None else None
        b.mask_ld = mask_ld
        b.hist = hist_dev.data_ptr() if hist_dev is not None else None
        b.stream = torch.cuda.current_stream(dev).cuda_stream
        t = _lib.Tree()
        t.size = C.sizeof(_lib.Tree)
        t.requests = len(reqs)
        anc_d = torch.from_numpy(anchors).to(dev)
        par_d = torch.from_numpy(parents).to(dev)
        tok_d = torch.from_numpy(toks).to(dev)
        qrow_d = torch.from_numpy(qrow).to(dev)
        t.anchor, t.parent, t.token, t.qrow = anc_d.data_ptr(), par_d.data_ptr(), tok_d.data_ptr(), qrow_d.data_ptr()
        t.max_kids = max_kids
        keep = [anc_d, par_d, tok_d, qrow_d, rows_dev, mask_dev, hist_dev, x]
        t.qrows.size = C.sizeof(_lib.QRows)
        if qprob:
            qt = _f64_rows(qprob, dev)
            t.qrows.kind, t.qrows.rows, t.qrows.q, t.qrows.ld = _lib.Q_PROB, len(qprob), qt.data_ptr(), qt.stride(0)
            keep.append(qt)
        elif qlog:
            ql = torch.stack([q.to(dev) for q in qlog])
            if ql.dtype not in (torch.float32, torch.bfloat16):
                ql = ql.float()
            ql = ql.contiguous()
            tt = torch.tensor(qtemp, dtype=torch.float64, device=dev)
            t.qrows.kind = _lib.Q_LOGITS_BF16 if ql.dtype == torch.bfloat16 else _lib.Q_LOGITS_F32
            t.qrows.rows, t.qrows.q, t.qrows.ld, t.qrows.temperature = len(qlog), ql.data_ptr(), ql.stride(0), tt.data_ptr()
            keep += [ql, tt]
        ld = int(emit_ld or max(sizes))
        e_len = torch.empty(len(reqs), dtype=torch.int32, device=dev)
        e_tok = torch.empty((len(reqs), ld), dtype=torch.int32, device=dev)
        e_node = torch.empty((len(reqs), ld), dtype=torch.int32, device=dev)
        e_st = torch.empty(len(reqs), dtype=torch.int32, device=dev)
        o = _lib.TreeOut()
        o.size = C.sizeof(_lib.TreeOut)
        o.emit_len, o.emit_tokens, o.emit_nodes, o.emit_ld = e_len.data_ptr(), e_tok.data_ptr(), e_node.data_ptr(), ld
        o.status = e_st.data_ptr()
        self.dev, self.b, self.t, self.o, self.keep = dev, b, t, o, keep
        self.e_len, self.e_tok, self.e_node, self.e_st = e_len, e_tok, e_node, e_st
        self.ld, self.anchors, self.n_req, self.nodes, self.vocab = ld, anchors, len(reqs), nodes, v


def _as_row(x, u, dev):
    t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float32)))
    return t[u].to(dev)


def _stack_targets(ts, sizes, dev):
    """The requests' target rows as one [nodes, V] tensor: in place when they are consecutive rows of one device
    tensor, else copied."""
    if all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts):
        base = ts[0]
        if all(t.dim() == 2 and t.stride() == base.stride() and t.dtype == base.dtype for t in ts):
            rows = base.stride(0) * base.element_size()
            ok = all(t.data_ptr() == base.data_ptr() + rows * int(sum(sizes[:i])) for i, t in enumerate(ts))
            if ok:
                return torch.as_strided(base, (int(sum(sizes)), base.shape[1]), base.stride())
        return torch.cat([t.to(dev) for t in ts])
    return torch.cat([(t if isinstance(t, torch.Tensor) else torch.from_numpy(np.asarray(t))).to(dev) for t in ts])


# ---- the drafter's selection (spec.py:151-159) ---------------------------------------------------------------------

def pick_batch(x, n, t, seeds, ats):
    """Children of many nodes in one gse_draft_pick call. x: [rows, V] drafter logits or log-probabilities (device
    tensor used in place); n, t, seeds, ats: per row (or one value for all). temperature 0: the n best tokens in stable
    descending order, each with its input value; t > 0: n draws from q = softmax(float64(x) / t) with the SALT_DRAFT
    streams at index at, each with log q[x]. Returns (tokens int32 [rows, nmax], values fp64 [rows, nmax]) on the device;
    entries past a row's n are unset."""
    xt, code = _logits(x)
    rows, v = xt.shape
    dev = xt.device
    per = lambda val: list(val) if isinstance(val, (list, tuple, np.ndarray)) else [val] * rows
    nn, tt, ss, aa = per(n), per(t), per(seeds), per(ats)
    nmax = max([int(k) for k in nn] + [1])
    if nmax > _lib.MAX_KIDS:
        raise ValueError(f"at most {_lib.MAX_KIDS} children per node")
    h = _lib.handle(dev.index, rows, v)
    n_d = torch.tensor([int(k) for k in nn], dtype=torch.int32, device=dev)
    t_d = torch.tensor([float(k) for k in tt], dtype=torch.float64, device=dev)
    s_d, a_d = _u64(ss, dev), _u64(aa, dev)
    out_t = torch.full((rows, nmax), -1, dtype=torch.int32, device=dev)
    out_v = torch.empty((rows, nmax), dtype=torch.float64, device=dev)
    b = _lib.PickBatch()
    b.size = C.sizeof(_lib.PickBatch)
    b.dtype = _lib.BF16 if code == _lib.BF16 else _lib.F32
    b.rows, b.vocab, b.x, b.ld = rows, v, xt.data_ptr(), xt.stride(0)
    b.temperature, b.n, b.seed, b.at = t_d.data_ptr(), n_d.data_ptr(), s_d.data_ptr(), a_d.data_ptr()
    b.out_tokens, b.out_logq, b.out_ld = out_t.data_ptr(), out_v.data_ptr(), nmax
    b.stream = torch.cuda.current_stream(dev).cuda_stream
    h.call("gse_draft_pick", C.byref(b))
    out_t._keep = (xt, n_d, t_d, s_d, a_d)
    return out_t, out_v


class TreeDrafter:
    """spec.py:125-216 TreeDrafter over a next-token model m: m.dist(seq, path) -> log-probabilities (a device tensor
    [V]) of the token after seq.tokens + path; m.feed / m.release optional (passed through, as spec.py:146-152 does).
    Shapes: chain; static rank paths (Medusa, EAGLE-1); dynamic (EAGLE-2: expand the topk best of each level by
    cumulative log-probability, rerank every candidate, keep the k best). temperature > 0: chain and dynamic children are
    drawn from the model at that temperature and carry their q (a QRef) for rejection acceptance; static paths always
    take ranks. The selection of every node of one level runs in one gse_draft_pick call. propose() returns tree_cls
    objects (default: this module's Tree; the reference's Tree class may be passed instead, it takes the same
    arguments)."""

    def __init__(self, m, shape="chain", topk=4, depth=6, choices=None, temperature=0.0, tree_cls=None):
        assert shape in ("chain", "static", "dynamic") and (shape != "static" or choices)
        self.m, self.shape, self.topk, self.depth, self.t = m, shape, topk, depth, temperature
        self.choices = sorted({tuple(c) for c in choices or ()}, key=lambda c: (len(c), c))
        self.needs = dict(tree=shape != "chain", taps=tuple(getattr(m, "taps", ())))
        self.tree_cls = tree_cls or Tree

    def propose(self, seqs, k):
        return [self.grow(s, k) if k > 0 else self.tree_cls([], []) for s in seqs]

    def feed(self, seq, pos, rows):
        if hasattr(self.m, "feed"):
            self.m.feed(seq, pos, rows)

    def release(self, sid):
        if hasattr(self.m, "release"):
            self.m.release(sid)

    def _pick_level(self, s, lps, n, ats, t):
        """n children of each of a level's nodes (log-prob rows lps, absolute indices ats) at temperature t:
        [(token, q, log-prob)] per node."""
        x = torch.stack([lp.reshape(-1) for lp in lps]).float()  # (the drafter's row as fp32)
        toks, vals = pick_batch(x, n, t, s.seed, ats)
        toks, vals = toks.cpu().tolist(), vals.cpu().tolist()
        out = []
        for r in range(len(lps)):
            q = QRef(x[r], t) if t else None
            out.append([(int(toks[r][k]), q, float(lps[r][toks[r][k]]) if t == 0 else float(vals[r][k]))
                        for k in range(n)])
        return out

    def grow(self, s, k):
        """The proposal tree after s (spec.py:161-204), a tree_cls object."""
        m, at, T = self.m, len(s.tokens), self.tree_cls
        if self.shape == "chain":
            toks, qs = [], []
            for d in range(k):
                x, q, _ = self._pick_level(s, [m.dist(s, toks)], 1, [at + d], self.t)[0][0]
                toks.append(x)
                qs.append(q)
            return T(toks, list(range(len(toks))), qs if self.t else None)
        if self.shape == "static":
            node, toks, par, order = {(): 0}, [], [], {}
            for c in self.choices:
                if len(toks) == k or c[:-1] not in node:
                    continue
                p = node[c[:-1]]
                if p not in order:  # the node's tokens by rank (spec.py:176: a stable descending sort)
                    lp = m.dist(s, self._path(toks, par, p))
                    n = min(lp.numel(), max(cc[-1] for cc in self.choices) + 1)
                    order[p] = [x for x, _, _ in self._pick_level(s, [lp], n, [at], 0.0)[0]]
                toks.append(int(order[p][c[-1]]))
                par.append(p)
                node[c] = len(toks)
            return T(toks, par)
        cand = []  # (score, token, parent candidate index or -1, q)
        beam = [-1]
        for _ in range(self.depth):
            paths = [self._cpath(cand, b) for b in beam]
            got = self._pick_level(s, [m.dist(s, pt) for pt in paths], self.topk, [at + len(pt) for pt in paths],
                                   self.t)
            new = []
            for b, kids in zip(beam, got):
                for x, q, lp in kids:
                    new.append((lp + (cand[b][0] if b >= 0 else 0.0), x, b, q))
            base = len(cand)
            cand += new
            beam = sorted(range(base, len(cand)), key=lambda i: (-cand[i][0], i))[:self.topk]
        keep, sel = {}, []
        for i in sorted(range(len(cand)), key=lambda i: (-cand[i][0], i)):
            if len(sel) == k:
                break
            if cand[i][2] < 0 or cand[i][2] in keep:
                keep[i] = None
                sel.append(i)
        sel.sort()
        idx = {i: j + 1 for j, i in enumerate(sel)}
        return T([cand[i][1] for i in sel], [idx.get(cand[i][2], 0) for i in sel],
                 [cand[i][3] for i in sel] if self.t else None)

    @staticmethod
    def _path(toks, par, n):
        out = []
        while n:
            out.append(toks[n - 1])
            n = par[n - 1]
        return out[::-1]

    @staticmethod
    def _cpath(cand, b):
        out = []
        while b >= 0:
            out.append(cand[b][1])
            b = cand[b][2]
        return out[::-1]
