"""Pins the oracle's tree-verify walk (oracle/spec_ref.verify_tree, restating engine.py:262-298) before the HIP walk is
compared with it.

  * Joint law: tokens decoded round after round (a drafted tree per round, then the walk) must follow the product of
    the target's per-step distributions dist(target(prefix)) (chi-square, bins with expectation < 5 pooled), as
    the reference's tests/test_spec.py:255-290 checks its engine. Power controls: the same statistic rejects a walk
    whose mss accepts every draft (no residual) and a walk that never advances the uniform index.
  * Known answers: chains where the acceptance at depth d is decided by uniform(mix(seed, 2^40), nout0 + d) alone and a
    rejection resamples one fixed token, so the emitted sequence follows from the uniform stream (the C restatement's
    splitmix64, oracle/c). A walk that does not advance nout, or that samples at inner nodes, fails them (checked).
  * Engine semantics: a token -1 ends the walk as an error and is not emitted, a stop reason ends it after the token,
    exact-acceptance requests follow the kid holding the sampled token, and a node's mask applies to its dist.
"""
import math
from types import SimpleNamespace as NS

import numpy as np
import pytest

from oracle import cref
from oracle import sampling_ref as ora
from oracle import spec_ref as spo

SALT_ACC, SALT_RES, SALT_DRAFT = 1 << 40, 1 << 41, 1 << 42


def P(**kw):
    d = dict(temperature=1.0, top_p=1.0, top_k=0, min_p=0.0, repetition_penalty=1.0, frequency_penalty=0.0,
             presence_penalty=0.0, logprobs=None, accept="rejection")
    d.update(kw)
    return NS(**d)


def _h(seq, salt):
    h = salt
    for t in seq:
        h = ora.mix(h, t + 1)
    return h


def target_logits(seq, v):
    """A target model: fp32 logits of the next token after seq (a hash of the whole sequence picks them)."""
    u = ora.uniform_np(_h(seq, 7), np.arange(v, dtype=np.uint64))
    return (3.0 * (u - 0.5)).astype(np.float32)


def draft_logp(seq, v):
    """A drafter unlike the target: log-probabilities of a different hash."""
    u = ora.uniform_np(_h(seq, 11), np.arange(v, dtype=np.uint64))
    z = 2.0 * u
    return z - np.log(np.exp(z).sum())


def tree_round(seq, seed, nout, v, shape, p, walk):
    """One engine round: draft a tree after seq (SpecInfer: kids drawn from q with SALT_DRAFT streams), target rows for
    every node, then the walk. Returns the emitted tokens."""
    parents = {"chain": [0, 1, 2], "tree": [0, 1, 0, 3]}[shape]
    kids = spo.kids_of(parents)
    toks, qs = [0] * len(parents), [None] * len(parents)
    path_of = {0: []}
    for u in range(len(parents) + 1):
        pu = path_of[u]
        lp = draft_logp(seq + pu, v)
        picked = spo.pick(lp, len(kids[u]), 1.0, seed, len(seq) + len(pu))
        for c, (x, q, _) in zip(kids[u], picked):
            toks[c - 1], qs[c - 1] = x, q
            path_of[c] = pu + [x]
    target = np.stack([target_logits(seq + path_of[u], v) for u in range(len(parents) + 1)])
    out, _, _ = walk(target, qs, toks, parents, p, seed, nout)
    return out


def decode(seed, n, v, shape, p, walk=spo.verify_tree):
    seq, out = [1, 2], []
    while len(out) < n:
        got = tree_round(seq + out, seed, len(out), v, shape, p, walk)
        out += got
    return tuple(out[:n])


def target_joint(n, v, p):
    out = {}
    for cell in np.ndindex(*([v] * n)):
        pr, seq = 1.0, [1, 2]
        for t in cell:
            pr *= float(ora.dist(target_logits(seq, v), p)[t])
            seq = seq + [t]
        out[tuple(int(c) for c in cell)] = pr
    return out


def chi2(counts, probs, runs):
    """Pearson statistic and degrees of freedom, bins with expectation < 5 pooled."""
    stat, df, pe, po = 0.0, -1, 0.0, 0
    for k, pr in probs.items():
        e = pr * runs
        if e < 5:
            pe, po = pe + e, po + counts.get(k, 0)
            continue
        stat, df = stat + (counts.get(k, 0) - e) ** 2 / e, df + 1
    if pe > 0:
        stat, df = stat + (po - pe) ** 2 / pe, df + 1
    return stat, df


def sampled_joint(n, v, p, shape, runs, walk=spo.verify_tree):
    c = {}
    for i in range(runs):
        k = decode(1000 + i, n, v, shape, p, walk)
        c[k] = c.get(k, 0) + 1
    return c


@pytest.mark.parametrize("shape,p", [("chain", P(temperature=1.0)), ("tree", P(temperature=1.0)),
                                     ("tree", P(temperature=1.0, top_p=0.8))])
def test_walk_joint_law_equals_the_target(shape, p):
    v, n, runs = 5, 3, 3000
    stat, df = chi2(sampled_joint(n, v, p, shape, runs), target_joint(n, v, p), runs)
    assert stat < df + 6 * math.sqrt(2 * df), (stat, df)


def _residual_free(target, q, tokens, parents, p, seed, nout0=0):
    """A broken walk: every draft is accepted (mss without its acceptance test and residual)."""
    kids = spo.kids_of(parents)
    u, out, path = 0, [], [0]
    while kids[u]:
        c = kids[u][0]
        out.append(tokens[c - 1])
        u = c
        path.append(u)
    out.append(ora.sample(target[u:u + 1], [p], [seed], [nout0 + len(out)], [None])[0])
    return out, path, None


def _stuck_index(target, q, tokens, parents, p, seed, nout0=0):
    """A broken walk: the uniform index never advances past nout0 inside the round."""
    kids = spo.kids_of(parents)
    u, out, path = 0, [], [0]
    while True:
        if kids[u]:
            pd = ora.dist(target[u], p)
            t, r = spo.mss(pd, [(tokens[c - 1], spo._kid_q(q, u, c)) for c in kids[u]], seed, nout0)
            hit = kids[u][r] if r is not None else None
        else:
            t, hit = ora.sample(target[u:u + 1], [p], [seed], [nout0], [None])[0], None
        out.append(t)
        if hit is None:
            return out, path, None
        u = hit
        path.append(u)


def test_chi2_has_power_against_a_residual_free_walk():
    v, n, runs, p = 5, 3, 1500, P(temperature=1.0)
    stat, df = chi2(sampled_joint(n, v, p, "chain", runs, _residual_free), target_joint(n, v, p), runs)
    assert stat > 10 * (df + 6 * math.sqrt(2 * df)), (stat, df)


def test_chi2_has_power_against_a_walk_that_reuses_the_uniform_index():
    v, n, runs, p = 5, 3, 3000, P(temperature=1.0)
    stat, df = chi2(sampled_joint(n, v, p, "chain", runs, _stuck_index), target_joint(n, v, p), runs)
    assert stat > df + 6 * math.sqrt(2 * df), (stat, df)


# ---- known answers: the uniform index of each depth ----------------------------------------------------------------

def _half_chain(depth, v=4):
    """A chain of `depth` drafted tokens 0 (one-hot q) over targets with dist = [1/2, 1/2, 0, ...] (logits 0, 0, -inf):
    the kid at depth d is accepted iff uniform(mix(seed, 2^40), nout0 + d) < 1/2; a rejection leaves p = [0, 1, 0, ..]
    and the residual draw returns token 1; the leaf samples [1/2, 1/2] with uniform(seed, nout0 + depth)."""
    x = np.full((depth + 1, v), -np.inf, np.float32)
    x[:, :2] = 0.0
    return x, [0] * depth, list(range(depth))


def _half_chain_answer(seed, nout0, depth):
    out = []
    for d in range(depth):
        if cref.uniform(cref.mix(seed, SALT_ACC), nout0 + d) < 0.5:
            out.append(0)
        else:
            return out + [1]
    u = cref.uniform(seed, nout0 + depth)
    return out + [0 if u <= 0.5 else 1]   # order [0, 1], c = [1/2, 1]: j = #{c < u}


@pytest.mark.parametrize("nout0", [0, 5, 1000])
def test_walk_known_answers_fix_the_uniform_index(nout0):
    depth = 4
    x, toks, parents = _half_chain(depth)
    for seed in range(60):
        out, path, why = spo.verify_tree(x, None, toks, parents, P(), seed, nout0)
        assert out == _half_chain_answer(seed, nout0, depth), seed
        assert why is None and path == list(range(len(out)))  # token d comes from node d of the chain


def test_known_answers_catch_a_stuck_index_and_sampling_at_inner_nodes():
    depth = 4
    x, toks, parents = _half_chain(depth)
    stuck = [seed for seed in range(60)
             if _stuck_index(x, None, toks, parents, P(), seed, 3)[0] != _half_chain_answer(seed, 3, depth)]
    assert len(stuck) >= 10

    def sample_inner(target, q, tokens, parents_, p, seed, nout0=0):
        kids = spo.kids_of(parents_)
        u, out, nout = 0, [], nout0
        while True:
            t = ora.sample(target[u:u + 1], [p], [seed], [nout], [None])[0]
            out.append(t)
            nout += 1
            hit = next((c for c in kids[u] if tokens[c - 1] == t), None)
            if hit is None:
                return out, None, None
            u = hit

    wrong = [seed for seed in range(60)
             if sample_inner(x, None, toks, parents, P(), seed, 3)[0] != _half_chain_answer(seed, 3, depth)]
    assert len(wrong) >= 10


def test_two_kids_second_is_tested_against_the_residual():
    """Root kids 0 then 1 (one-hot), target [1/2, 1/2, 0, 0]: kid 0 accepted iff coin_0 < 1/2; otherwise p becomes
    [0, 1, 0, 0] and kid 1 (token 1) is accepted iff coin_1 * 1 < 1, always."""
    x = np.full((3, 4), -np.inf, np.float32)
    x[:, :2] = 0.0
    for seed in range(40):
        out, path, _ = spo.verify_tree(x, None, [0, 1], [0, 0], P(), seed, 2)
        if cref.uniform(cref.mix(seed, SALT_ACC), 2) < 0.5:
            assert path == [0, 1] and out[0] == 0
        else:
            assert path == [0, 2] and out[0] == 1
        assert len(out) == 2   # the kid's own row (a leaf) samples the bonus token


# ---- engine semantics ------------------------------------------------------------------------------------------------

def test_error_token_ends_the_walk_unemitted():
    x = np.zeros((3, 6), np.float32)
    x[1, 2] = np.nan                       # node 1's row is bad: sample / dist give -1
    toks, parents = [0, 1], [0, 1]
    out, path, why = spo.verify_tree(x, None, toks, parents, P(temperature=0.0), 3, 0)
    # greedy (exact acceptance): the anchor's argmax is token 0 = node 1's token, node 1's row is bad
    assert out == [0] and path == [0, 1] and why == "error"


def test_stop_reason_ends_the_walk_after_its_token():
    x = np.full((4, 5), -np.inf, np.float32)
    x[:, 3] = 0.0                           # every node: token 3 with certainty
    out, path, why = spo.verify_tree(x, None, [3, 3, 3], [0, 1, 2], P(), 9, 0,
                                     stop=lambda emitted: "stop" if len(emitted) == 2 else None)
    assert out == [3, 3] and path == [0, 1] and why == "stop"


def test_exact_acceptance_follows_the_kid_with_the_sampled_token():
    rng = np.random.default_rng(5)
    v = 7
    x = rng.normal(0, 1, size=(5, v)).astype(np.float32)
    p = P(temperature=0.9, accept="exact")
    parents = [0, 0, 1, 2]
    for seed in range(30):
        t0 = ora.sample(x[0:1], [p], [seed], [4], [None])[0]
        toks = [t0, (t0 + 1) % v, 0, 0]     # kid 1 holds the anchor's sample
        out, path, _ = spo.verify_tree(x, None, toks, parents, p, seed, 4)
        assert out[0] == t0 and path[:2] == [0, 1]
        assert out[1] == ora.sample(x[1:2], [p], [seed], [5], [None])[0]


def test_node_masks_apply_to_dist_and_sample():
    rng = np.random.default_rng(8)
    v = 9
    x = rng.normal(0, 1, size=(4, v)).astype(np.float32)
    allowed = [np.arange(v) % 3 == k for k in range(3)] + [np.arange(v) % 3 == 0]
    for strict in ("rejection", "exact"):
        p = P(temperature=1.2, accept=strict)
        for seed in range(40):
            toks = [int(rng.integers(v)) for _ in range(3)]
            out, path, _ = spo.verify_tree(x, None, toks, [0, 1, 2], p, seed, 0, masks=allowed)
            assert len(path) == len(out)
            for d, t in enumerate(out):   # token d comes from node path[d], under that node's mask
                assert allowed[path[d]][t], (strict, seed, d)
