"""GPU parity: the HIP path (through the C ABI) against the reference's golden vectors and the oracle, on seeded inputs
of every workload at sizes the oracle finishes in seconds. Token ids are compared bit-exact, probabilities and logprobs
within the stated tolerances, processed logits bit-exact."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora
from oracle import spec_ref as spo

pytestmark = pytest.mark.gpu

DIST_RTOL = 1e-12      # fp64 probabilities: GPU exp vs numpy exp, tree vs pairwise sums
LOGPROB_RTOL = 1e-5    # fp32 logprobs (the stated 1e-5 relative bar)


def _P(ge, **kw):
    return ge.sampling.SamplingParams(**kw)


def both_paths(ge, x, params, seeds, idxs, masks, history=None, uniforms=None):
    fast = ge.sampling.sample(x, params, seeds, idxs, masks, history=history, uniforms=uniforms)
    exact = ge.sampling.sample(x, params, seeds, idxs, masks, history=history, uniforms=uniforms, exact=True)
    return fast, exact


def test_golden_tiny(ge, gpu, golden):
    x = torch.from_numpy(golden["tiny_x"]).to(gpu)
    for (t, k, p), want in zip(golden["tiny_params"], golden["tiny_tok"]):
        params = [_P(ge, temperature=float(t), top_k=int(k), top_p=float(p))] * 64
        xs = x.expand(64, -1).contiguous()
        f, e = both_paths(ge, xs, params, list(range(64)), [0] * 64, None)
        assert f == list(want) and e == list(want), (t, k, p)


@pytest.mark.parametrize("prefix", ["rows", "edge"])
def test_golden_rows(ge, gpu, golden, prefix):
    g = golden
    n = len(g[prefix + "_T"])
    params = [_P(ge, temperature=float(t), top_k=int(k), top_p=float(p))
              for t, k, p in zip(g[prefix + "_T"], g[prefix + "_K"], g[prefix + "_TP"])]
    masks = [torch.from_numpy(g[prefix + "_mask"][r]) if g[prefix + "_has_mask"][r] else None for r in range(n)]
    x = torch.from_numpy(g[prefix + "_x"]).to(gpu)
    toks = g[prefix + "_tok"]
    for j in range(toks.shape[1]):
        if prefix == "rows":
            seeds, idxs = [int(s) for s in g["rows_seed"][:, j]], [int(i) for i in g["rows_idx"][:, j]]
        else:
            seeds, idxs = [int(g["edge_seed"][j])] * n, [j] * n
        f, e = both_paths(ge, x, params, seeds, idxs, masks)
        assert f == list(toks[:, j]), (prefix, j)
        assert e == list(toks[:, j]), (prefix, j, "exact")


def test_golden_dist_draw_mss(ge, gpu, golden):
    g = golden
    for r, (t, k, p) in enumerate(g["dist_params"]):
        m = torch.from_numpy(g["dist_mask"][r]) if g["dist_has_mask"][r] else None
        d = ge.sampling.dist(torch.from_numpy(g["dist_x"][r]).to(gpu), _P(ge, temperature=float(t), top_k=int(k),
                                                                           top_p=float(p)), m)
        np.testing.assert_allclose(d.cpu().numpy(), g["dist_out"][r], rtol=DIST_RTOL, atol=1e-300)
    for r in range(g["draw_q"].shape[0]):
        q = torch.from_numpy(g["draw_q"][r]).to(gpu)
        assert [ge.sampling.draw(q, float(u)) for u in g["draw_u"][r]] == list(g["draw_out"][r])
    kids = [[(int(t), g["mss_q"][n, k] if g["mss_has_q"][n, k] else None) for k, t in enumerate(g["mss_tok"][n])
             if t >= 0] for n in range(g["mss_p"].shape[0])]
    toks, ks = ge.spec.mss_batch(g["mss_p"], kids, [int(s) for s in g["mss_seed"]], [int(i) for i in g["mss_i"]])
    assert toks == list(g["mss_out_tok"])
    assert [-1 if k is None else k for k in ks] == list(g["mss_out_kid"])


def _run(ge, batch, gpu, exact=False, processed=False, flags=0):
    x = torch.from_numpy(batch.logits).to(gpu)
    if batch.bf16:
        x = x.view(torch.bfloat16)
    masks = None if batch.masks is None else [torch.from_numpy(m) for m in batch.masks]
    return ge.sampling.sample_ex(x, batch.params, None, None, masks, history=batch.history, uniforms=batch.uniforms,
                                 exact=exact, processed=processed, flags=flags)


def _oracle(batch):
    masks = None if batch.masks is None else [ora.unpack_mask(m, batch.vocab) for m in batch.masks]
    return ora.sample_full(batch.logits_f32(), batch.params, None, None, masks, batch.history, batch.uniforms)


def _check(ge, batch, gpu, check_processed=True):
    want = _oracle(batch)
    for exact in (False, True):
        sel = _run(ge, batch, gpu, exact=exact, processed=check_processed)
        toks = sel.tolist()
        assert toks == [w["token"] for w in want], (batch.name, exact)
        if check_processed and not exact:
            proc = sel.processed.cpu().numpy()
            for r, w in enumerate(want):
                assert np.array_equal(proc[r].view(np.uint32), w["processed"].view(np.uint32)), (batch.name, r)
        if sel.logprobs is not None:
            ids, lps = sel.logprob_ids.cpu().numpy(), sel.logprobs.cpu().numpy()
            for r, w in enumerate(want):
                n = len(w["logprob_ids"])
                assert list(ids[r, :n]) == list(w["logprob_ids"]), (batch.name, r)
                np.testing.assert_allclose(lps[r, :n], w["logprobs"], rtol=LOGPROB_RTOL)
    return want


def test_c1_cpu_sampler_workload(ge, gpu):
    _check(ge, ge.workloads.c1(), gpu)


def test_c2_masked_greedy(ge, gpu):
    b = ge.workloads.c2()
    want = _check(ge, b, gpu, check_processed=False)
    assert all(t >= 0 for t in (w["token"] for w in want))


@pytest.mark.parametrize("rows", [list(range(0, 16)), list(range(100, 116)), list(range(240, 256))])
def test_c3_full_stack_rows(ge, gpu, rows):
    _check(ge, ge.workloads.c3(rows=rows), gpu)


def test_c5_bf16_nucleus_logprobs(ge, gpu):
    _check(ge, ge.workloads.c5(rows=list(range(8))), gpu, check_processed=False)


def test_exact_head_branches(ge, gpu):
    """Rows chosen for each branch of the exact path's sorted head: keep sets that run below the head (top-p near 1,
    top-k 3000), a min-p threshold below the head's cut, a row whose one key fills every bin the head could cut at (no
    head: every query runs its own histogram levels, logprobs included), logprobs served from the head, a greedy row
    with logprobs. Fast and exact paths against the oracle, tokens and logprobs."""
    v = 151936
    rng = np.random.default_rng(11)
    x = rng.normal(0.0, 1.0, size=(8, v)).astype(np.float32)
    x[2] = 0.5
    x[3, :40] += 6.0
    P = ge.sampling.SamplingParams
    params = [P(temperature=1.0, top_p=0.999),
              P(temperature=1.2, top_k=3000, top_p=1.0),
              P(temperature=1.0, top_p=0.9, logprobs=5),
              P(temperature=0.8, top_p=0.95, min_p=0.05, logprobs=8),
              P(temperature=1.0, top_p=1.0, min_p=1e-6),
              P(temperature=0.0, logprobs=6),
              P(temperature=0.7, top_k=50, top_p=0.9),
              P(temperature=1.5, top_p=0.5, min_p=0.2)]
    u = np.array([ora.uniform(2000 + r, 1) for r in range(8)], np.float64)
    batch = ge.workloads.Batch("head", x, params, u)
    want = _oracle(batch)
    for exact in (False, True):
        sel = _run(ge, batch, gpu, exact=exact)
        assert sel.tolist() == [w["token"] for w in want], exact
        ids, lps = sel.logprob_ids.cpu().numpy(), sel.logprobs.cpu().numpy()
        for r, w in enumerate(want):
            if "logprob_ids" in w:
                n = len(w["logprob_ids"])
                assert list(ids[r, :n]) == list(w["logprob_ids"]), (exact, r)
                np.testing.assert_allclose(lps[r, :n], w["logprobs"], rtol=LOGPROB_RTOL)


def test_c4_tree_verify(ge, gpu):
    reqs = ge.workloads.c4(requests=range(4), v=128256)
    qrows = []
    for r in reqs:
        q = {}
        for u in range(9):
            if r["draft"][u].any():
                z = r["draft"][u].astype(np.float64)
                e = np.exp(z - z.max())
                q[u] = e / e.sum()
        qrows.append(q)
    got = ge.spec.verify_tree([dict(target=r["target"], q=q, tokens=r["tokens"], parents=r["parents"],
                                    params=r["params"], seed=r["seed"]) for r, q in zip(reqs, qrows)])
    for res, r, q in zip(got, reqs, qrows):
        assert res == spo.verify_tree(r["target"], q, r["tokens"], r["parents"], r["params"], r["seed"])


def _dev(x, gpu, dtype):
    """x (fp32 numpy) on the device as fp32 or bf16, and the fp32 values the device holds (bf16 widens exactly)."""
    d = torch.from_numpy(x).to(gpu)
    if dtype == "bf16":
        d = d.to(torch.bfloat16)
        return d, d.float().cpu().numpy()
    return d, x


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("v", [1, 7, 33, 8191, 8193, 20000])
def test_odd_vocab_sizes_and_strides(ge, gpu, v, dtype):
    """Odd vocabularies, a row stride of v + 5 and a start two elements in (rows not 16-byte aligned), with ties, masks,
    penalty histories, top-k, top-p and min-p; fp32 and bf16 logits (the bf16 rows against the oracle on the widened
    values); the fast and the exact path."""
    rng = np.random.default_rng(v)
    n = 12
    x = (rng.normal(0, 2, size=(n, v + 5)) ).astype(np.float32)
    x[3, : min(v, 4)] = 1.0   # ties
    xd, x = _dev(x, gpu, dtype)
    P = ge.sampling.SamplingParams
    params = [P(), P(temperature=0.9), P(temperature=1.0, top_k=3), P(temperature=1.4, top_p=0.7),
              P(temperature=0.6, min_p=0.1), P(temperature=1.0, repetition_penalty=1.3, frequency_penalty=0.4)] * 2
    hist = [rng.integers(0, v, size=9) for _ in range(n)]
    m = rng.random(v) < 0.5
    m[0] = True
    masks = [m if r % 4 == 1 else None for r in range(n)]
    seeds, idxs = list(range(n)), [5] * n
    xt = xd[:, 2:2 + v]                                   # row stride v + 5, misaligned start
    want = ora.sample(x[:, 2:2 + v], params, seeds, idxs, masks, history=hist)
    f, e = both_paths(ge, xt, params, seeds, idxs, masks, history=hist)
    assert f == want and e == want


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_masks_penalties_minp_logprobs(ge, gpu, dtype):
    """The full stack over one odd vocabulary in both dtypes: bool masks and packed masks in one call, a MaskBatch in
    another, penalty histories, min-p, top-k / top-p, logprobs, greedy rows with logprobs; rows aligned and rows
    starting one element in. Tokens, processed logits (bit-exact) and logprobs (1e-5) against the oracle on the
    device's values, on the fast and the exact path."""
    rng = np.random.default_rng(21 if dtype == "f32" else 22)
    n, v = 16, 50257
    P = ge.sampling.SamplingParams
    params = [P(temperature=[0.0, 0.7, 1.0, 1.3][r % 4], top_k=[0, 40, 0, 200][(r // 4) % 4],
                top_p=[1.0, 0.9, 0.95, 0.8][r % 4], min_p=[0.0, 0.05, 0.0, 0.1][(r + 1) % 4],
                repetition_penalty=[1.0, 1.1, 1.3, 1.05][(r + 2) % 4], frequency_penalty=[0.0, 0.5, 0.2, 1.0][r % 4],
                presence_penalty=[0.0, 0.3, 0.0, 0.7][(r + 3) % 4], logprobs=[None, 3, 20, 0][(r // 2) % 4])
              for r in range(n)]
    hist = [rng.integers(0, v, size=int(rng.integers(0, 400))) for _ in range(n)]
    hist[5] = None
    bools = [(rng.random(v) < [0.05, 0.5, 0.9][r % 3]) for r in range(n)]
    for m in bools:
        m[int(rng.integers(0, v))] = True
    masks_np = [bools[r] if r % 3 else None for r in range(n)]
    masks_in = [None if m is None else (torch.from_numpy(m) if r % 2 else ge.grammar.pack(m))
                for r, m in enumerate(masks_np)]
    seeds, idxs = [int(s) for s in rng.integers(0, 1 << 62, size=n)], list(range(n))
    for off in (0, 1):
        x = rng.normal(0, 2.5, size=(n, v + 8)).astype(np.float32)
        xd, x = _dev(x, gpu, dtype)
        xt, xn = xd[:, off:off + v], x[:, off:off + v]
        want = ora.sample_full(xn, params, seeds, idxs, masks_np, hist)
        mb = ge.grammar.MaskBatch(n, v)
        for r, m in enumerate(masks_np):
            if m is not None:
                mb.set(r, m)
        for exact in (False, True):
            for masks in (masks_in, mb):
                sel = ge.sampling.sample_ex(xt, params, seeds, idxs, masks, history=hist, exact=exact, processed=True)
                assert sel.tolist() == [w["token"] for w in want], (dtype, off, exact)
                proc = sel.processed.cpu().numpy()
                ids, lps = sel.logprob_ids.cpu().numpy(), sel.logprobs.cpu().numpy()
                for r, w in enumerate(want):
                    assert np.array_equal(proc[r].view(np.uint32), w["processed"].view(np.uint32)), (dtype, off, r)
                    if "logprob_ids" in w:
                        k = len(w["logprob_ids"])
                        assert list(ids[r, :k]) == list(w["logprob_ids"]), (dtype, off, exact, r)
                        np.testing.assert_allclose(lps[r, :k], w["logprobs"], rtol=LOGPROB_RTOL)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_dist_with_penalties_minp_masks(ge, gpu, dtype):
    """gse_dist (sampling.py:88-97 with the extensions) against the oracle's dist, row by row within 1e-12: penalty
    histories, min-p, masks, top-k, top-p, flat rows whose keep set runs deep, bf16 rows unaligned."""
    rng = np.random.default_rng(31 if dtype == "f32" else 32)
    n, v = 12, 100003
    P = ge.sampling.SamplingParams
    params = [P(temperature=[0.8, 1.0, 1.4][r % 3], top_k=[0, 50, 0, 0][r % 4], top_p=[0.9, 1.0, 0.99, 0.8][r % 4],
                min_p=[0.0, 0.05, 0.0, 0.02, 0.0, 0.2][r % 6], repetition_penalty=[1.0, 1.2][r % 2],
                frequency_penalty=[0.3, 0.0, 0.8][r % 3], presence_penalty=[0.0, 0.5][(r // 2) % 2])
              for r in range(n)]
    hist = [rng.integers(0, v, size=int(rng.integers(1, 300))) for _ in range(n)]
    masks = [(rng.random(v) < 0.6) if r % 3 == 1 else None for r in range(n)]
    x = rng.normal(0, 1.0, size=(n, v + 3)).astype(np.float32)
    x[::2] *= 2.5  # peaked rows between the flat ones
    xd, x = _dev(x, gpu, dtype)
    xt, xn = xd[:, 1:1 + v], x[:, 1:1 + v]
    d = ge.sampling.dist_batch(xt, params, [None if m is None else torch.from_numpy(m) for m in masks], hist)
    d = d.cpu().numpy()
    for r in range(n):
        np.testing.assert_allclose(d[r], ora.dist(xn[r], params[r], masks[r], hist[r]), rtol=DIST_RTOL,
                                   atol=1e-300, err_msg=f"{dtype} row {r}")


def test_bf16_deep_rows_unaligned(ge, gpu):
    """The split-row finish over bf16 rows that are not 16-byte aligned (its bf16 scalar-load instance), with masks and
    penalty histories: tokens against the oracle on the widened values, and the finish took part."""
    n, v = 16, 100003
    x, params = _flat_rows(ge, n, v + 3, 17)
    rng = np.random.default_rng(17)
    P = ge.sampling.SamplingParams
    params = [P(temperature=p.temperature, top_p=p.top_p, top_k=p.top_k, min_p=p.min_p, repetition_penalty=1.1,
                frequency_penalty=0.2) for p in params]
    masks = [rng.random(v) < 0.8 for _ in range(n)]
    hist = [rng.integers(0, v, size=200) for _ in range(n)]
    u = np.array([ora.uniform(4000 + r, 2) for r in range(n)], np.float64)
    xd, xw = _dev(x, gpu, "bf16")
    xt, xn = xd[:, 3:3 + v], xw[:, 3:3 + v]
    got = ge.sampling.sample_ex(xt, params, None, None, [torch.from_numpy(m) for m in masks], history=hist,
                                uniforms=u).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    print(f"[bf16 deep] paths {np.bincount(paths, minlength=3).tolist()}", flush=True)
    assert got == ora.sample(xn, params, None, None, masks, history=hist, uniforms=u)
    assert (paths == ge._lib.PATH_DEEP).sum() >= 1, paths


def test_determinism_and_batch_invariance_full_c3(ge, gpu):
    b = ge.workloads.c3()
    a1 = _run(ge, b, gpu).tolist()
    a2 = _run(ge, b, gpu).tolist()
    ax = _run(ge, b, gpu, exact=True).tolist()
    assert a1 == a2 == ax
    perm = np.random.default_rng(0).permutation(b.rows)
    pb = ge.workloads.Batch(b.name, b.logits[perm], [b.params[i] for i in perm], b.uniforms[perm], b.masks[perm],
                            [b.history[i] for i in perm])
    assert _run(ge, pb, gpu).tolist() == [a1[i] for i in perm]


def test_c3_full_batch_matches_oracle(ge, gpu):
    """The whole 256-row C3 batch: the main pass resolves most rows and the split-row finish the deep ones (30 or so
    flat, hot nucleus rows); every token equals the oracle's."""
    b = ge.workloads.c3()
    want = [w["token"] for w in _oracle(b)]
    got = _run(ge, b, gpu).tolist()
    assert got == want
    paths = ge._lib.handle(gpu.index, b.rows, b.vocab).row_paths(b.rows)
    assert (paths == ge._lib.PATH_DEEP).sum() > 0  # the split-row finish took part
    assert (paths == ge._lib.PATH_EXACT).sum() == 0


def _flat_rows(ge, n, v, seed):
    """Hot rows over a flat distribution: the keep prefix of top-p runs to thousands of elements."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 1.0, size=(n, v)).astype(np.float32)
    P = ge.sampling.SamplingParams
    tp = [0.8, 0.9, 0.95, 0.99, 0.999]
    params = [P(temperature=[1.0, 1.3, 1.7][r % 3], top_p=tp[r % 5], top_k=[0, 0, 0, 5000][r % 4],
                min_p=[0.0, 0.0, 0.0, 0.0, 0.01][r % 5]) for r in range(n)]
    return x, params


def test_deep_rows_sample_and_dist(ge, gpu):
    """Rows settled by the split-row finish: tokens against the oracle under shared uniforms, and the fp64
    distribution (which reads the finish's keep boundary and sums) against the oracle's dist."""
    n, v = 24, 151936
    x, params = _flat_rows(ge, n, v, 7)
    u = np.array([ora.uniform(1000 + r, 3) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    got = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    want = ora.sample(x, params, None, None, None, uniforms=u)
    assert got == want
    assert (paths == ge._lib.PATH_DEEP).sum() >= n // 2, paths
    d = ge.sampling.dist_batch(xt, params).cpu().numpy()
    for r in range(0, n, 5):
        np.testing.assert_allclose(d[r], ora.dist(x[r], params[r]), rtol=DIST_RTOL, atol=1e-300)


def test_deep_rows_subbin_finish(ge, gpu):
    """The split-row finish has two ways to the cut and the draw: one sort of the whole window list (lists of at most
    2048 entries, nearly every row) and the sub-bin walk (longer lists). GSE_BATCH_SUBBIN_FINISH sends every list to
    the walk: on the flat rows and on the whole C3 batch both give the oracle's tokens, on the split-row path."""
    n, v = 24, 151936
    x, params = _flat_rows(ge, n, v, 7)
    u = np.array([ora.uniform(1000 + r, 3) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    want = ora.sample(x, params, None, None, None, uniforms=u)
    for flags in (0, ge._lib.BATCH_SUBBIN_FINISH):
        got = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u, flags=flags).tolist()
        paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
        assert got == want, flags
        assert (paths == ge._lib.PATH_DEEP).sum() >= n // 2, (flags, paths)
    b = ge.workloads.c3()
    a0 = _run(ge, b, gpu).tolist()
    a1 = _run(ge, b, gpu, flags=ge._lib.BATCH_SUBBIN_FINISH).tolist()
    paths = ge._lib.handle(gpu.index, b.rows, b.vocab).row_paths(b.rows)
    assert a0 == a1 == [w["token"] for w in _oracle(b)]
    assert (paths == ge._lib.PATH_DEEP).sum() > 0 and (paths == ge._lib.PATH_EXACT).sum() == 0, paths


def test_deep_rows_odd_vocab_masks_history(ge, gpu):
    """The split-row finish over an odd vocabulary (rows unaligned for 16-byte loads: the finish's scalar-load
    instance) with grammar masks and penalty histories in its count and pick streams: tokens against the oracle."""
    n, v = 16, 100003
    x, params = _flat_rows(ge, n, v, 13)
    rng = np.random.default_rng(13)
    P = ge.sampling.SamplingParams
    params = [P(temperature=p.temperature, top_p=p.top_p, top_k=p.top_k, min_p=p.min_p, repetition_penalty=1.1,
                frequency_penalty=0.2, presence_penalty=0.1) for p in params]
    masks = [rng.random(v) < 0.7 for _ in range(n)]
    hist = [rng.integers(0, v, size=300) for _ in range(n)]
    u = np.array([ora.uniform(3000 + r, 7) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    got = ge.sampling.sample_ex(xt, params, None, None, [torch.from_numpy(m) for m in masks], history=hist,
                                uniforms=u).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    assert got == ora.sample(x, params, None, None, masks, history=hist, uniforms=u)
    assert (paths == ge._lib.PATH_DEEP).sum() >= n // 2, paths


def test_no_split_flag_sends_deep_rows_to_exact(ge, gpu):
    """GSE_BATCH_NO_SPLIT on rows that need the split-row finish: it is not launched, those rows take the exact path,
    and every token still equals the oracle's. (The drop-in sets the flag only when every row is greedy.)"""
    n, v = 8, 151936
    x, params = _flat_rows(ge, n, v, 7)
    u = np.array([ora.uniform(1000 + r, 3) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    got = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u, flags=ge._lib.BATCH_NO_SPLIT).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    assert got == ora.sample(x, params, None, None, None, uniforms=u)
    assert (paths == ge._lib.PATH_DEEP).sum() == 0 and (paths == ge._lib.PATH_EXACT).sum() >= 1, paths
    assert ge.sampling._sample_flags(params) == 0
    assert ge.sampling._sample_flags([ge.sampling.SamplingParams()] * 3) == ge._lib.BATCH_NO_SPLIT


@pytest.mark.gpu
def test_deep_rows_plan_wait_off(ge, gpu):
    """The split-row finish's bounded wait: with GSE_BATCH_NO_PLAN_WAIT a pick slice that finds its row's plan not yet
    out gives the row up (the forced form of a wait that ran out), and the exact path finishes it: same tokens."""
    n, v = 24, 151936
    x, params = _flat_rows(ge, n, v, 7)
    u = np.array([ora.uniform(1000 + r, 3) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    got = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u,
                                flags=ge._lib.BATCH_NO_PLAN_WAIT).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    assert got == ora.sample(x, params, None, None, None, uniforms=u)
    assert (paths == ge._lib.PATH_EXACT).sum() >= 1, paths
    again = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u).tolist()  # the slots were cleared
    assert again == got


@pytest.mark.gpu
def test_hard_rows_in_the_split_row_launch(ge, gpu):
    """With the split-row launch, it finishes every hard row itself (no exact launch follows it): rows whose part holds
    more distinct penalty-history ids than it can count (3000 of 8192; hard, not sent to the split-row finish) beside
    deep rows, such rows alone (the launch without deep rows), deep rows whose finish gives up (GSE_BATCH_NO_PLAN_WAIT)
    beside them, and deep rows alone, in turn on one handle, twice over: every token equals the oracle's, so each call
    left the counts it used cleared for the next."""
    n, v = 16, 8192
    rng = np.random.default_rng(5)
    x = rng.normal(0.0, 1.0, size=(n, v)).astype(np.float32)
    P = ge.sampling.SamplingParams
    params = [P(temperature=[1.0, 1.3][r % 2], top_p=[0.95, 0.99, 0.999][r % 3], frequency_penalty=0.05)
              for r in range(n)]
    big = [rng.permutation(v)[:3000] for _ in range(n)]
    small = [rng.integers(0, v, size=20) for _ in range(n)]
    mixed = [big[r] if r % 4 == 0 else small[r] for r in range(n)]
    u = np.array([ora.uniform(3000 + r, 2) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    lib = ge._lib
    cases = [("mixed", mixed, 0), ("overflow only", big, 0), ("no plan wait", mixed, lib.BATCH_NO_PLAN_WAIT),
             ("deep only", small, 0)]
    for rep in range(2):
        for name, hist, flags in cases:
            print(f"[hard rows] {name}, pass {rep}", flush=True)
            got = ge.sampling.sample_ex(xt, params, None, None, None, history=hist, uniforms=u, flags=flags).tolist()
            paths = lib.handle(gpu.index, n, v).row_paths(n)
            assert got == ora.sample(x, params, None, None, None, history=hist, uniforms=u), (rep, name)
            deep, exact = (paths == lib.PATH_DEEP).sum(), (paths == lib.PATH_EXACT).sum()
            if name == "mixed":
                assert deep >= 1 and exact >= n // 4, (name, paths)
            elif name == "overflow only":
                assert deep == 0 and exact >= n // 2, (name, paths)
            elif name == "no plan wait":
                assert exact >= n // 4 + 1, (name, paths)
            else:
                assert deep >= n // 2, (name, paths)


@pytest.mark.gpu
def test_deep_slots_overflow_to_exact(ge, gpu):
    """More deep rows than the split-row finish has slots (1024 per call at most): the rows past the slots take the
    exact path, and every token still equals the oracle's."""
    n, v = 1100, 8192
    x, params = _flat_rows(ge, n, v, 11)
    u = np.array([ora.uniform(2000 + r, 5) for r in range(n)], np.float64)
    xt = torch.from_numpy(x).to(gpu)
    got = ge.sampling.sample_ex(xt, params, None, None, None, uniforms=u).tolist()
    paths = ge._lib.handle(gpu.index, n, v).row_paths(n)
    assert got == ora.sample(x, params, None, None, None, uniforms=u)
    assert (paths == ge._lib.PATH_DEEP).sum() <= 1024, paths
    assert (paths == ge._lib.PATH_EXACT).sum() >= 1, paths


def test_mask_batch_one_copy_matches_oracle(ge, gpu):
    """Grammar masks straight to the device (one pinned buffer, one copy; engine.py:272-273 applies each row's mask
    before sampling, grammar.py:42-45 unpacks it): tokens and processed logits equal the oracle's on the same logits and
    masks; rows left unfilled sample unmasked; a buffer sized for more rows than the call serves its first rows."""
    rng = np.random.default_rng(11)
    n, v = 12, 20000
    xn = (rng.standard_normal((n, v)) * 2.0).astype(np.float32)
    x = torch.from_numpy(xn).to(gpu)
    params = [_P(ge, temperature=0.8 if i % 3 else 0.0, top_p=0.9, top_k=50 if i % 2 else 0) for i in range(n)]
    seeds, idxs = list(range(100, 100 + n)), [3] * n
    masks = [(rng.random(v) < 0.3) if i < 8 else None for i in range(n)]
    mb = ge.grammar.MaskBatch(n + 5, v)
    assert mb.host.is_pinned()
    for i in range(8):
        if i % 2:
            mb.set(i, masks[i])
        else:
            mb.set(i, ge.grammar.pack(masks[i]))
    mb.set(n + 2, np.zeros(v, dtype=bool))  # a row past the call's rows: not read
    got = ge.sampling.sample_ex(x, params, seeds, idxs, mb, processed=True)
    torch.cuda.synchronize()
    want = ora.sample_full(xn, params, seeds, idxs, masks)
    assert got.tolist() == [w["token"] for w in want]
    proc = got.processed.cpu().numpy()
    for i in range(n):
        assert np.array_equal(proc[i].view(np.uint32), want[i]["processed"].view(np.uint32)), i
        if i < 8:
            assert bool(masks[i][got.tolist()[i]])
    # the same buffer refilled for a second step with fewer rows filled and fewer rows sampled
    mb.reset()
    mb.set(1, masks[1])
    m2 = 6
    masks2 = [masks[1] if i == 1 else None for i in range(m2)]
    got2 = ge.sampling.sample(x[:m2], params[:m2], seeds[:m2], idxs[:m2], mb)
    assert got2 == ora.sample(xn[:m2], params[:m2], seeds[:m2], idxs[:m2], masks2)


def test_logits_borrowed_not_copied(ge, gpu, monkeypatch):
    """Device-resident logits hand-off: sample() reads the caller's device tensor in place (the pointer it passes is
    the tensor's own) and never brings logits to the host (sampling.py:54-56 host() is not on the path)."""
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.standard_normal((4, 5000)).astype(np.float32)).to(gpu)
    y, _ = ge.sampling._logits(x)
    assert y.data_ptr() == x.data_ptr()

    def no_host(*_):
        raise AssertionError("logits brought to the host")

    monkeypatch.setattr(ge.sampling, "host", no_host)
    params = [_P(ge, temperature=1.0, top_p=0.95) for _ in range(4)]
    toks = ge.sampling.sample(x, params, [1, 2, 3, 4], [0, 0, 0, 0], None)
    assert toks == ora.sample(x.cpu().numpy(), params, [1, 2, 3, 4], [0, 0, 0, 0], None)


def test_sample_in_a_captured_graph(ge, gpu):
    """One gse_sample call over the whole full-stack batch (256 rows, 23 of them settled by the split-row finish, the
    exact pass launched too) captured in a graph on the stream whose handle it used before, replayed three times with
    an eager call of the same handle and cleared outputs between the replays: every replay's tokens equal the eager
    call's, which equal the Python path's."""
    import ctypes as C
    lib = ge._lib
    b = ge.workloads.c3()
    x0 = torch.from_numpy(b.logits).to(gpu)
    masks = [torch.from_numpy(m) for m in b.masks]
    st = torch.cuda.Stream(gpu)  # (default priority)
    with torch.cuda.stream(st):
        h, x, code, _, b0, keep = ge.sampling._prepare(x0, b.params, None, None, masks, b.history, b.uniforms)
        bb = ge.sampling._batch(x, code, keep[1], keep[2], b0.mask_ld, keep[3], keep[4], gpu)
        toks = torch.empty(b.rows, dtype=torch.int32, device=gpu)
        o = lib.Out()
        o.size = C.sizeof(lib.Out)
        o.tokens = toks.data_ptr()
        h.ck(h.L.gse_sample(h.h, C.byref(bb), C.byref(o)), "gse_sample")
    torch.cuda.synchronize()
    ref = toks.cpu().tolist()
    want = ge.sampling.sample_ex(x0.clone(), b.params, None, None, masks, history=b.history,
                                 uniforms=b.uniforms).tolist()
    assert ref == want
    print("[sample] capturing one full-stack call in a graph", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        h.ck(h.L.gse_sample(h.h, C.byref(bb), C.byref(o)), "gse_sample")
    torch.cuda.synchronize()
    for k in range(3):
        with torch.cuda.stream(st):
            h.ck(h.L.gse_sample(h.h, C.byref(bb), C.byref(o)), "gse_sample")  # (eager, the same workspace)
        torch.cuda.synchronize()
        toks.fill_(-5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert toks.cpu().tolist() == ref, k
