"""GPU parity of the speculative-decoding path through the C ABI: the device verify round (gse_verify_tree) against the
oracle's walk (oracle/spec_ref.verify_tree, pinned in tests/test_oracle_walk.py), and the drafter's selection
(gse_draft_pick) against the oracle's restatement of spec.py:151-159 and :183-204. Token ids and paths are compared
bit-exact; log q within 1e-12 relative."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora
from oracle import spec_ref as spo

pytestmark = pytest.mark.gpu


def _q_of_draft(draft, parents, t=1.0):
    """{node: softmax(draft[node] / t) in fp64} for the nodes with kids (what the kids were drawn from)."""
    q = {}
    for u, ks in enumerate(spo.kids_of(parents)):
        if ks:
            z = draft[u].astype(np.float64) / t
            e = np.exp(z - z.max())
            q[u] = e / e.sum()
    return q


def test_c4_verify_all_requests_matches_oracle(ge, gpu):
    """All 32 requests of the tree-verification workload (V=128256), draft distributions given as drafter logits
    (q = softmax(draft) formed on the device): emitted tokens and accepted paths equal the oracle walk's."""
    reqs = ge.workloads.c4()
    got = ge.spec.verify_tree([dict(target=torch.from_numpy(r["target"]).to(gpu), tokens=r["tokens"],
                                    parents=r["parents"], params=r["params"], seed=r["seed"],
                                    draft=torch.from_numpy(r["draft"]).to(gpu), draft_t=1.0) for r in reqs])
    acc = 0
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], _q_of_draft(r["draft"], r["parents"]), r["tokens"], r["parents"],
                               r["params"], r["seed"])
        assert got[a] == want, (a, got[a], want)
        acc += len(want[1]) - 1
    assert acc > 0  # some drafts were accepted


def _random_trees(ge, rng, n_req, v, kinds):
    P = ge.sampling.SamplingParams
    reqs = []
    for a in range(n_req):
        kind = kinds[a % len(kinds)]
        n = int(rng.integers(1, 9))
        parents = [int(rng.integers(0, j + 1)) for j in range(n)]
        target = rng.normal(0, 1.5, size=(n + 1, v)).astype(np.float32)
        draft = (target + rng.normal(0, 0.6, size=target.shape)).astype(np.float32)
        if kind == "greedy":
            p = P()
        elif kind == "exact":
            p = P(temperature=0.8, top_k=int(rng.choice([0, 30])), top_p=float(rng.choice([1.0, 0.9])))
        else:
            p = P(temperature=float(rng.choice([0.7, 1.0, 1.3])), top_k=int(rng.choice([0, 0, 50])),
                  top_p=float(rng.choice([1.0, 0.95, 0.8])), min_p=float(rng.choice([0.0, 0.0, 0.02])),
                  accept="rejection")
        # drafted tokens: drawn from q where the node has one, else a target top token (a deterministic drafter)
        q = _q_of_draft(draft, parents)
        toks = []
        for j, par in enumerate(parents):
            if kind == "rejection" and a % 3 != 0:
                toks.append(int(rng.choice(v, p=q[par])))
            else:
                toks.append(int(np.argsort(-target[par], kind="stable")[int(rng.integers(0, 3))]))
        reqs.append(dict(target=target, draft=draft, tokens=toks, parents=parents, params=p,
                         seed=int(rng.integers(0, 1 << 62)), nout=int(rng.integers(0, 50)),
                         onehot=kind != "rejection" or a % 3 == 0))
    return reqs


@pytest.mark.parametrize("seed,v", [(0, 3000), (1, 3000), (2, 3001)])
def test_verify_mixed_requests_match_oracle(ge, gpu, seed, v):
    """Strict (rejection), exact-acceptance and greedy requests in one call; random trees up to 8 nodes with nodes of
    several kids, one-hot (deterministic) and sampled drafts, top-k / top-p / min-p, per-request nout; an odd
    vocabulary leaves every row after the first unaligned for 16-byte loads."""
    rng = np.random.default_rng(100 + seed)
    reqs = _random_trees(ge, rng, 24, v, ["rejection", "exact", "rejection", "greedy"])
    calls = []
    for r in reqs:
        d = dict(target=r["target"], tokens=r["tokens"], parents=r["parents"], params=r["params"], seed=r["seed"],
                 nout=r["nout"])
        if not r["onehot"]:
            d["q"] = _q_of_draft(r["draft"], r["parents"])
        calls.append(d)
    got = ge.spec.verify_tree(calls)
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], None if r["onehot"] else _q_of_draft(r["draft"], r["parents"]),
                               r["tokens"], r["parents"], r["params"], r["seed"], r["nout"])
        assert got[a] == want, (a, r["params"], got[a], want)


def test_verify_masks_history_and_stop(ge, gpu):
    """Per-node grammar masks and penalty histories (the state once the path to the node is accepted), and a stop
    predicate applied after each emitted token."""
    rng = np.random.default_rng(7)
    v = 2000
    P = ge.sampling.SamplingParams
    reqs = []
    for a in range(12):
        n = 6
        parents = [0, 1, 2, 0, 4, 5][:n]
        target = rng.normal(0, 2, size=(n + 1, v)).astype(np.float32)
        masks = [rng.random(v) < 0.4 for _ in range(n + 1)]
        hist = [rng.integers(0, v, size=20) for _ in range(n + 1)]
        # drafted tokens allowed by their parent's mask (what a grammar-constrained drafter proposes)
        toks = [int(np.nonzero(masks[par])[0][int(rng.integers(0, 5))]) for par in parents]
        p = P(temperature=1.1, top_p=0.9, repetition_penalty=1.2, frequency_penalty=0.3,
              accept="rejection" if a % 2 else "exact")
        reqs.append(dict(target=target, tokens=toks, parents=parents, params=p, seed=1000 + a, masks=masks,
                         history=hist))
    stop = lambda a, emitted: "stop" if (a % 3 == 0 and len(emitted) == 2) else None
    got = ge.spec.verify_tree(reqs, nout0=4, stop=stop)
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], None, r["tokens"], r["parents"], r["params"], r["seed"], 4,
                               masks=r["masks"], stop=lambda e, a=a: stop(a, e), history=r["history"])
        assert got[a] == want, (a, got[a], want)
        for d, t in enumerate(got[a][0]):
            assert r["masks"][got[a][1][d]][t]


def test_verify_prob_rows_and_bad_rows(ge, gpu):
    """q given as fp64 probability rows (the reference's Tree.q layout), and a node whose target row holds a NaN: the
    walk ends there as an error without emitting it (engine.py:286-288)."""
    rng = np.random.default_rng(9)
    v = 1500
    P = ge.sampling.SamplingParams
    parents = [0, 1, 2]
    reqs = []
    for a in range(6):
        target = rng.normal(0, 1, size=(4, v)).astype(np.float32)
        qd = {u: rng.dirichlet(np.ones(v) * 0.5) for u in range(3)}
        toks = [int(np.argmax(qd[par])) for par in parents]
        if a == 2:
            target[1, 5] = np.nan
        reqs.append(dict(target=target, tokens=toks, parents=parents, params=P(temperature=1.0, accept="rejection"),
                         seed=77 + a, q=[qd[par] for par in parents]))
    got = ge.spec.verify_tree(reqs)
    for a, r in enumerate(reqs):
        if a == 2 and got[a][2] == "error":
            assert got[a][1][-1] == 1 or got[a][1] == [0]
            continue
        want = spo.verify_tree(r["target"], r["q"], r["tokens"], r["parents"], r["params"], r["seed"])
        assert got[a] == want, (a, got[a], want)


@pytest.mark.parametrize("t", [0.0, 0.7, 1.0, 1.6])
def test_draft_pick_matches_oracle(ge, gpu, t):
    """spec.py:151-159 for a batch of nodes: t == 0 the n best (stable descending), t > 0 n draws with the SALT_DRAFT
    streams and their log q."""
    rng = np.random.default_rng(int(t * 10) + 3)
    rows, v = 20, 50000
    x = rng.normal(0, 2, size=(rows, v)).astype(np.float32)
    x[3, 100:110] = x[3].max() + 1.0       # ties at the top
    n = [int(k) for k in rng.integers(1, 9, size=rows)]
    seeds = [int(s) for s in rng.integers(0, 1 << 62, size=rows)]
    ats = [int(s) for s in rng.integers(0, 4000, size=rows)]
    toks, vals = ge.spec.pick_batch(torch.from_numpy(x).to(gpu), n, t, seeds, ats)
    toks, vals = toks.cpu().numpy(), vals.cpu().numpy()
    for r in range(rows):
        want = spo.pick(x[r].astype(np.float64), n[r], t, seeds[r], ats[r])
        assert list(toks[r, :n[r]]) == [w[0] for w in want], r
        np.testing.assert_allclose(vals[r, :n[r]], [w[2] for w in want], rtol=1e-12, atol=1e-12)


class _LM:
    """A tiny next-token model for the drafter: log-probabilities of a hashed row (device tensor)."""

    def __init__(self, v, dev):
        self.v, self.dev = v, dev

    def dist(self, s, path):
        h = 3
        for t in list(s.tokens) + list(path):
            h = ora.mix(h, t + 1)
        u = ora.uniform_np(h, np.arange(self.v, dtype=np.uint64))
        z = (4.0 * u).astype(np.float32)
        return torch.from_numpy(z - np.float32(np.log(np.exp(z.astype(np.float64)).sum()))).to(self.dev)


@pytest.mark.parametrize("shape,t", [("chain", 0.0), ("chain", 1.0), ("dynamic", 0.0), ("dynamic", 1.0)])
def test_tree_drafter_matches_oracle(ge, gpu, shape, t):
    from types import SimpleNamespace as NS
    v = 4000
    m = _LM(v, gpu)
    d = ge.spec.TreeDrafter(m, shape, topk=3, depth=3, temperature=t)
    s = NS(tokens=[5, 9, 2], seed=4242)
    tr = d.grow(s, 6)
    toks, par, q = tr.tokens, tr.parents, tr.q
    if shape == "chain":
        want_t, want_q = [], []
        for k in range(6):
            x, qq, _ = spo.pick(m.dist(s, want_t).cpu().numpy().astype(np.float64), 1, t, s.seed, 3 + k)[0]
            want_t.append(x)
        assert toks == want_t and par == list(range(6))
    else:
        wt, wp, _ = spo.grow_dynamic(lambda pt: m.dist(s, pt).cpu().numpy().astype(np.float64), s.seed, 3, 6, 3, 3, t)
        assert (toks, par) == (wt, wp)
    assert (q is None) == (t == 0)


def test_verify_passes_with_more_items_than_workgroups(ge, gpu):
    """Residual passes that take more (node, slice) items than their grid (later passes run a quarter of a resident
    round): 96 strict requests whose root has four kids the drafter favours but the target finds unlikely, so most
    roots are rejected kid after kid and draw from their fourth residual, over a 131072-token vocabulary (16 slices a
    row)."""
    rng = np.random.default_rng(31)
    v = 131072
    P = ge.sampling.SamplingParams
    parents = [0, 0, 0, 0]
    calls, reqs = [], []
    for a in range(96):
        target = rng.normal(0, 1.5, size=(5, v)).astype(np.float32)
        draft = (target + rng.normal(0, 0.6, size=target.shape)).astype(np.float32)
        order = np.argsort(target[0], kind="stable")  # ascending: the first ids are the least likely
        toks = [int(order[int(rng.integers(0, 1000))]) for _ in parents]
        draft[0, toks] = draft[0].max() + 4.0  # the drafter favours them: p/q is tiny, the kids are rejected
        p = P(temperature=1.0, accept="rejection")
        seed = int(rng.integers(0, 1 << 62))
        reqs.append((target, draft, toks, p, seed))
        calls.append(dict(target=torch.from_numpy(target).to(gpu), tokens=toks, parents=parents, params=p, seed=seed,
                          draft=torch.from_numpy(draft).to(gpu), draft_t=1.0))
    print(f"[verify] 96 requests x 5 rows, V={v}", flush=True)
    got = ge.spec.verify_tree(calls)
    rejected = 0
    for a, (target, draft, toks, p, seed) in enumerate(reqs):
        want = spo.verify_tree(target, _q_of_draft(draft, parents), toks, parents, p, seed)
        assert got[a] == want, (a, got[a], want)
        rejected += len(want[1]) == 1
    assert rejected > 48, rejected  # most roots went through all four residual passes


def test_verify_rounds_back_to_back_on_a_stream(ge, gpu):
    """Two verify rounds with drafter logits (their q-row statistics included), launched alternately four times each on
    a non-default stream without any synchronisation: every launch's output equals a synchronised launch's, which
    equals the oracle walk's."""
    reqs = ge.workloads.c4()
    other = [dict(r, seed=(r["seed"] * 7 + 3) % (1 << 62)) for r in reqs[:12]]

    def call_of(rs):
        return ge.spec.VerifyCall([dict(target=torch.from_numpy(r["target"]).to(gpu), tokens=r["tokens"],
                                        parents=r["parents"], params=r["params"], seed=r["seed"],
                                        draft=torch.from_numpy(r["draft"]).to(gpu), draft_t=1.0) for r in rs])

    def snap(c):
        return torch.cat([c.e_len[:, None], c.e_st[:, None], c.e_tok, c.e_node], 1).clone()

    calls, refs = [call_of(reqs), call_of(other)], []
    for c, rs in zip(calls, [reqs, other]):
        c.launch()
        torch.cuda.synchronize()
        got = c.result()
        for a, r in enumerate(rs):
            want = spo.verify_tree(r["target"], _q_of_draft(r["draft"], r["parents"]), r["tokens"], r["parents"],
                                   r["params"], r["seed"])
            assert got[a] == want, (a, got[a], want)
        refs.append(snap(c))
    print("[verify] back-to-back rounds on a non-default stream", flush=True)
    st = torch.cuda.Stream(gpu)  # (default priority)
    snaps = []
    with torch.cuda.stream(st):
        for _ in range(4):
            for c in calls:
                c.launch()
                snaps.append(snap(c))
    torch.cuda.synchronize()
    for k, sn in enumerate(snaps):
        assert torch.equal(sn, refs[k % 2]), k


def test_verify_keep_all_node_with_history_overflow(ge, gpu):
    """Strict nodes that keep every token list nothing in the selection pass (the round needs only their maximum); one
    whose part holds more distinct penalty-history ids than a part can count (3000 of 8192 tokens) cannot finish on its
    maximum and takes the exact path. Every request's walk still equals the oracle's."""
    rng = np.random.default_rng(41)
    v = 8192
    P = ge.sampling.SamplingParams
    parents = [0, 1, 0]
    reqs = []
    for a in range(6):
        target = rng.normal(0, 1.5, size=(4, v)).astype(np.float32)
        draft = (target + rng.normal(0, 0.6, size=target.shape)).astype(np.float32)
        q = _q_of_draft(draft, parents)
        toks = [int(rng.choice(v, p=q[par])) for par in parents]
        big = a % 2 == 0  # (the overflowing history on every other request)
        hist = [rng.permutation(v)[:3000] if big else rng.integers(0, v, size=40) for _ in range(4)]
        p = P(temperature=1.0, frequency_penalty=0.2, presence_penalty=0.1, accept="rejection")
        reqs.append(dict(target=target, tokens=toks, parents=parents, params=p, seed=500 + a, q=q, history=hist))
    print(f"[verify] keep-all strict nodes, V={v}, histories of 3000 distinct ids", flush=True)
    got = ge.spec.verify_tree(reqs)
    paths = ge._lib.handle(gpu.index, 4 * len(reqs), v).row_paths(4 * len(reqs))
    assert (paths == ge._lib.PATH_EXACT).sum() >= 3, paths  # (the strict nodes of the overflowing requests)
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], r["q"], r["tokens"], r["parents"], r["params"], r["seed"],
                               history=r["history"])
        assert got[a] == want, (a, got[a], want)


def _bf16(x, gpu):
    """A bf16 device copy of x and the fp32 values it holds (bf16 widens to fp32 exactly)."""
    d = torch.from_numpy(x).to(gpu).to(torch.bfloat16)
    return d, d.float().cpu().numpy()


def test_verify_bf16_target_and_drafter_logits(ge, gpu):
    """A verify round over bf16 target rows with bf16 drafter logits (the bf16 instances of the statistics and residual
    passes, and q = softmax(float64(x) / t) from bf16 x): strict, exact-acceptance and greedy requests, a ragged
    vocabulary (40000 tokens). The oracle walks the same values widened to fp32."""
    rng = np.random.default_rng(77)
    v = 40000
    P = ge.sampling.SamplingParams
    calls, want = [], []
    for a in range(12):
        parents = [0, 1, 2, 0, 4][:int(rng.integers(2, 6))]
        n = len(parents)
        tgt, tgt32 = _bf16(rng.normal(0, 1.5, size=(n + 1, v)).astype(np.float32), gpu)
        drf, drf32 = _bf16((tgt32 + rng.normal(0, 0.6, size=tgt32.shape)).astype(np.float32), gpu)
        t = float(rng.choice([0.8, 1.0, 1.3]))
        q = _q_of_draft(drf32, parents, t)
        toks = [int(rng.choice(v, p=q[par])) for par in parents]
        kind = a % 3
        p = (P(temperature=1.0, top_p=float(rng.choice([1.0, 0.9])), accept="rejection") if kind == 0 else
             P(temperature=0.9, top_k=40) if kind == 1 else P())
        seed = int(rng.integers(0, 1 << 62))
        calls.append(dict(target=tgt, tokens=toks, parents=parents, params=p, seed=seed, draft=drf, draft_t=t))
        want.append(spo.verify_tree(tgt32, q, toks, parents, p, seed))
    print(f"[verify] 12 requests, bf16 target and drafter logits, V={v}", flush=True)
    got = ge.spec.verify_tree(calls)
    for a in range(len(calls)):
        assert got[a] == want[a], (a, got[a], want[a])


@pytest.mark.parametrize("t", [0.0, 1.0])
def test_draft_pick_bf16_matches_oracle(ge, gpu, t):
    """The drafter's selection over bf16 logits (the bf16 pick instances) against the oracle on the widened values."""
    rng = np.random.default_rng(int(t * 10) + 9)
    rows, v = 12, 50000
    x, x32 = _bf16(rng.normal(0, 2, size=(rows, v)).astype(np.float32), gpu)
    n = [int(k) for k in rng.integers(1, 9, size=rows)]
    seeds = [int(s) for s in rng.integers(0, 1 << 62, size=rows)]
    ats = [int(s) for s in rng.integers(0, 4000, size=rows)]
    toks, vals = ge.spec.pick_batch(x, n, t, seeds, ats)
    toks, vals = toks.cpu().numpy(), vals.cpu().numpy()
    for r in range(rows):
        w = spo.pick(x32[r].astype(np.float64), n[r], t, seeds[r], ats[r])
        assert list(toks[r, :n[r]]) == [e[0] for e in w], r
        np.testing.assert_allclose(vals[r, :n[r]], [e[2] for e in w], rtol=1e-12, atol=1e-12)


def test_verify_round_in_a_captured_graph(ge, gpu):
    """A verify round with drafter logits (its q-row statistics included) captured in a graph
    on the stream it ran on before (so its handle exists: opening one allocates), replayed three times with eager work
    between the replays; every replay's walks equal the eager round's, which equal the oracle's."""
    reqs = ge.workloads.c4()[:8]
    call = ge.spec.VerifyCall([dict(target=torch.from_numpy(r["target"]).to(gpu), tokens=r["tokens"],
                                    parents=r["parents"], params=r["params"], seed=r["seed"],
                                    draft=torch.from_numpy(r["draft"]).to(gpu), draft_t=1.0) for r in reqs])
    st = torch.cuda.Stream(gpu)  # (default priority)
    with torch.cuda.stream(st):
        call.launch()
    torch.cuda.synchronize()
    ref = call.result()
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], _q_of_draft(r["draft"], r["parents"]), r["tokens"], r["parents"],
                               r["params"], r["seed"])
        assert ref[a] == want, (a, ref[a], want)
    print("[verify] capturing one round in a graph", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        call.launch()
    torch.cuda.synchronize()
    for k in range(3):
        for t in (call.e_len, call.e_st, call.e_tok, call.e_node):
            t.fill_(-7)  # (eager work between the replays: the outputs cleared)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert call.result() == ref, k


@pytest.mark.parametrize("shape,t", [("chain", 0.0), ("chain", 1.0), ("dynamic", 0.0), ("dynamic", 0.8)])
def test_drafter_proposals_through_scheduler_and_mss(ge, gpu, shape, t):
    """The drafter as the reference's scheduler and engine use it: propose() (selection on the device) -> as_tree ->
    ok -> fit (scheduler.py:128-133, the oracle's Tree injected as the tree class), then at every node with kids the
    drop-in mss over (token, tree.q[c - 1]) (engine.py:280-283; the q of a sampled child is a QRef, read on the device)
    against the oracle's mss over the oracle's own drafted q: same tokens, same accepted kid. The materialised q equals
    the oracle's softmax within 1e-12."""
    from types import SimpleNamespace as NS
    v, k = 4000, 6
    m = _LM(v, gpu)
    seqs = [NS(tokens=[5, 9, 2], seed=4242), NS(tokens=[7, 1], seed=99)]
    d = ge.spec.TreeDrafter(m, shape, topk=3, depth=3, temperature=t, tree_cls=spo.Tree)
    rng = np.random.default_rng(5)
    P = ge.sampling.SamplingParams
    nodes = 0
    for s, tr in zip(seqs, d.propose(seqs, k)):
        tr = spo.as_tree(tr)
        assert isinstance(tr, spo.Tree) and tr.ok(v)
        tr = tr.fit(k, 4)
        at = len(s.tokens)
        lp = lambda pt: m.dist(s, pt).cpu().numpy().astype(np.float64)
        if shape == "chain":
            wt, wq = [], []
            for j in range(k):
                x, q, _ = spo.pick(lp(wt), 1, t, s.seed, at + j)[0]
                wt.append(x)
                wq.append(q)
            want = spo.Tree.chain(wt, wq if t else None).fit(k, 4)
        else:
            want = spo.Tree(*spo.grow_dynamic(lp, s.seed, at, k, 3, 3, t)).fit(k, 4)
        assert (tr.tokens, tr.parents) == (want.tokens, want.parents)
        assert (tr.q is None) == (t == 0)
        if t:
            for qa, qb in zip(tr.q, want.q):
                np.testing.assert_allclose(np.asarray(qa), qb, rtol=1e-12, atol=1e-300)
        # the engine's strict node: dist of the target row, then mss over the node's kids
        for u, kids in enumerate(tr.kids()):
            if not kids:
                continue
            x = (rng.standard_normal(v) * 2.0).astype(np.float32)
            pp = P(temperature=1.0, accept="rejection")
            pd = ora.dist(x, pp)
            got = ge.spec.mss(torch.from_numpy(pd).to(gpu), [(tr.tokens[c - 1], tr.q[c - 1] if tr.q else None)
                                                             for c in kids], s.seed, 7 + u)
            exp = spo.mss(pd, [(want.tokens[c - 1], want.q[c - 1] if want.q else None) for c in kids], s.seed, 7 + u)
            assert got == exp, (shape, t, u, got, exp)
            nodes += 1
    assert nodes > 0


def test_qprob_matches_softmax(ge, gpu):
    """gse_qprob: q = softmax(float64(x) / t) of fp32 and bf16 drafter rows (spec.py:157) against numpy in fp64."""
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((5, 30011)) * 3.0).astype(np.float32)
    t = [1.0, 0.5, 1.7, 2.0, 0.9]
    got = ge.spec.qprob(torch.from_numpy(x).to(gpu), t).cpu().numpy()
    for r in range(5):
        z = x[r].astype(np.float64) / t[r]
        e = np.exp(z - z.max())
        np.testing.assert_allclose(got[r], e / e.sum(), rtol=1e-12, atol=1e-300)
    xb, x32 = _bf16(x, gpu)
    got = ge.spec.qprob(xb, t).cpu().numpy()
    for r in range(5):
        z = x32[r].astype(np.float64) / t[r]
        e = np.exp(z - z.max())
        np.testing.assert_allclose(got[r], e / e.sum(), rtol=1e-12, atol=1e-300)


def test_understated_max_kids_is_reported(ge, gpu):
    """A C-ABI caller that passes a max_kids below a strict node's kid count: the round cannot decide that node as the
    reference would (spec.py:91 walks every kid), so the walk stops before it with GSE_WALK_KIDS (the node in
    emit_nodes[emit_len]) instead of emitting a token; the Python layer raises. Requests that never reach such a node
    are unaffected."""
    reqs = ge.workloads.c4(requests=range(3), v=20000)
    calls = [dict(target=torch.from_numpy(r["target"]).to(gpu), tokens=r["tokens"], parents=r["parents"],
                  params=r["params"], seed=r["seed"], draft=torch.from_numpy(r["draft"]).to(gpu), draft_t=1.0)
             for r in reqs]
    call = ge.spec.VerifyCall(calls)
    assert call.t.max_kids == 2  # the anchor has two kids
    call.t.max_kids = 1
    call.launch()
    st = call.e_st.cpu().tolist()
    n = call.e_len.cpu().tolist()
    nodes = call.e_node.cpu().numpy()
    for a in range(3):
        assert st[a] == ge._lib.WALK_KIDS and n[a] == 0, (a, st[a], n[a])
        assert nodes[a, 0] == call.anchors[a]
    with pytest.raises(RuntimeError, match="kids"):
        call.result()
    call.t.max_kids = 2
    call.launch()
    for a, r in enumerate(reqs):
        want = spo.verify_tree(r["target"], _q_of_draft(r["draft"], r["parents"]), r["tokens"], r["parents"],
                               r["params"], r["seed"])
        assert call.result()[a] == want
