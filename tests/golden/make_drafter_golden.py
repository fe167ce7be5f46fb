"""Writes tests/golden/drafter_golden.npz: input/output vectors of the reference's drafter-side selection,
goethe_engine.spec.TreeDrafter (_pick, spec.py:151-159; grow with the chain and dynamic shapes, spec.py:161-204),
imported from /root/reference in the build container only.

Run from the repository root:  python tests/golden/make_drafter_golden.py [/root/reference]

The drafter's model is a deterministic toy defined here and restated in the tests (tests/test_oracle_drafter.py): the
fp64 log-probabilities after a sequence are log_softmax(4 u), u the splitmix64 uniforms of a hash of the sequence. The
fixture holds the model's parameters, every input and the reference's outputs; the tests never run the reference.
"""
import os
import sys

import numpy as np

M64 = (1 << 64) - 1
V = 48  # toy vocabulary


def mix(seed, i):
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def toy_lp(seq):
    """fp64 log-probabilities of the token after seq (a list of ints)."""
    h = 3
    for t in seq:
        h = mix(h, t + 1)
    u = np.array([(mix(h, j) >> 11) / float(1 << 53) for j in range(V)])
    z = 4.0 * u
    return z - (z.max() + np.log(np.exp(z - z.max()).sum()))


def main(ref):
    sys.path.insert(0, ref)
    import torch
    from goethe_engine import spec as SP

    class Toy:
        def dist(self, s, path):
            return torch.from_numpy(toy_lp(list(s.tokens) + list(path)))

    class Seq:
        def __init__(self, tokens, seed):
            self.tokens, self.seed = tokens, seed

    out = {"V": np.array(V)}
    # _pick on single rows: (row seq, n, t, seed, at) -> tokens, log-probs
    cases = []
    for c in range(40):
        seq = [c % 7, (3 * c) % 11, c]
        n = 1 + c % 5
        t = [0.0, 0.5, 1.0, 1.7][c % 4]
        seed = mix(99, c)
        at = 5 + (c * 37) % 1000
        d = SP.TreeDrafter(Toy(), "chain", temperature=t)
        got = d._pick(Seq(seq, seed), torch.from_numpy(toy_lp(seq)), n, at)
        cases.append((seq, n, t, seed, at, [g[0] for g in got], [g[2] for g in got]))
    out["pick_seq"] = np.array([cs[0] for cs in cases], np.int64)
    out["pick_n"] = np.array([cs[1] for cs in cases], np.int64)
    out["pick_t"] = np.array([cs[2] for cs in cases], np.float64)
    out["pick_seed"] = np.array([cs[3] for cs in cases], np.uint64)
    out["pick_at"] = np.array([cs[4] for cs in cases], np.int64)
    nmax = max(cs[1] for cs in cases)
    out["pick_tok"] = np.array([cs[5] + [-1] * (nmax - len(cs[5])) for cs in cases], np.int64)
    out["pick_lp"] = np.array([cs[6] + [0.0] * (nmax - len(cs[6])) for cs in cases], np.float64)

    # grow: (shape, t, anchor seq, seed, k, topk, depth) -> tokens, parents
    grows = []
    for c in range(24):
        shape = ["chain", "dynamic"][c % 2]
        t = [0.0, 0.0, 0.8, 1.0, 1.3, 0.0][c % 6]
        seq = [c, (5 * c) % 13]
        seed = mix(7, c)
        k = [4, 6, 8][c % 3]
        topk, depth = [2, 3, 4][(c // 2) % 3], [3, 4][c % 2]
        tree = SP.TreeDrafter(Toy(), shape, topk=topk, depth=depth, temperature=t).grow(Seq(seq, seed), k)
        grows.append((c % 2, t, seq, seed, k, topk, depth, list(tree.tokens), list(tree.parents)))
    kmax = max(len(g[7]) for g in grows)
    out["grow_dynamic"] = np.array([g[0] for g in grows], np.int64)
    out["grow_t"] = np.array([g[1] for g in grows], np.float64)
    out["grow_seq"] = np.array([g[2] for g in grows], np.int64)
    out["grow_seed"] = np.array([g[3] for g in grows], np.uint64)
    out["grow_k"] = np.array([g[4] for g in grows], np.int64)
    out["grow_topk"] = np.array([g[5] for g in grows], np.int64)
    out["grow_depth"] = np.array([g[6] for g in grows], np.int64)
    out["grow_len"] = np.array([len(g[7]) for g in grows], np.int64)
    out["grow_tok"] = np.array([g[7] + [-1] * (kmax - len(g[7])) for g in grows], np.int64)
    out["grow_par"] = np.array([g[8] + [-1] * (kmax - len(g[8])) for g in grows], np.int64)

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "drafter_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
