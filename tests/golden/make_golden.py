"""Writes tests/golden/sampling_golden.npz: input/output vectors of the reference's goethe_engine.sampling (sample, dist,
draw, mix, uniform) and goethe_engine.spec (mss), imported from /root/reference in the build container only.

Run from the repository root:  python tests/golden/make_golden.py [/root/reference]

Only the reference's pure-numpy functions are called (sampling.py imports dataclasses and numpy, spec.py numpy and
.sampling). Inputs come from a local splitmix64 + Box-Muller generator so the script needs nothing else; the inputs
are stored in the fixture next to the outputs, so the tests never regenerate them.
"""
import os
import sys

import numpy as np

M64 = (1 << 64) - 1


def mix_np(seed, idx):
    with np.errstate(over="ignore"):
        z = np.uint64(seed & M64) + (np.asarray(idx, np.uint64) + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def unif(seed, n, off=0):
    return (mix_np(seed, np.arange(off, off + n, dtype=np.uint64)) >> np.uint64(11)).astype(np.float64) / 2.0 ** 53


def normal(seed, n, off=0):
    u1 = 1.0 - unif(seed, n, 2 * off)[:n]
    u2 = unif(seed + 1, n, 2 * off)[:n]
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def main(ref):
    sys.path.insert(0, ref)
    from goethe_engine import sampling as S
    from goethe_engine import spec as SP
    P = S.SamplingParams
    out = {}

    # mix / uniform known answers
    seeds = np.array([0, 1, 5, 6, 77, 1000, 2 ** 40 + 3, 2 ** 63 - 1, M64], dtype=np.uint64)
    idxs = np.array([0, 1, 2, 63, 2 ** 41, 12345678901], dtype=np.uint64)
    out["mix_seed"], out["mix_idx"] = seeds, idxs
    out["mix_out"] = np.array([[S.mix(int(s), int(i)) for i in idxs] for s in seeds], dtype=np.uint64)
    out["uni_out"] = np.array([[S.uniform(int(s), int(i)) for i in idxs] for s in seeds], dtype=np.float64)

    # tiny support rows (test_sampling.py:37-44), many seeds
    tiny = np.array([[5.0, 4.0, 3.0, 2.0, 1.0, 0.0]], np.float32)
    tiny_p = [(5.0, 2, 1.0), (1.0, 0, 0.5), (1.0, 1, 1.0), (1.0, 0, 1.0), (0.5, 3, 0.9), (2.0, 0, 0.99)]
    out["tiny_x"] = tiny
    out["tiny_params"] = np.array(tiny_p, np.float64)
    out["tiny_tok"] = np.array([[S.sample(tiny, [P(temperature=t, top_k=int(k), top_p=p)], [s], [0], [None])[0]
                                 for s in range(64)] for t, k, p in tiny_p], np.int64)

    # random rows: B rows x V, mixed params, masks, several (seed, idx) per row
    B, V, R = 48, 1000, 12
    x = np.stack([(sig * normal(100 + r, V)).astype(np.float32) for r, sig in
                  zip(range(B), [0.5, 2.0, 5.0] * (B // 3))])
    uu = unif(7, B * 8).reshape(B, 8)
    T = np.where(uu[:, 0] < 0.2, 0.0, np.array([0.3, 0.7, 1.0, 1.5, 3.0])[(uu[:, 1] * 5).astype(int)])
    K = np.array([0, 0, 1, 5, 50, 2000])[(uu[:, 2] * 6).astype(int)]
    TP = np.array([1.0, 0.9, 0.5, 0.2, 0.999])[(uu[:, 3] * 5).astype(int)]
    msk = np.ones((B, V), bool)
    for r in range(B):
        if uu[r, 4] < 0.3:
            msk[r] = unif(900 + r, V) < 0.3
    has_mask = uu[:, 4] < 0.3
    rseeds = (mix_np(11, np.arange(B * R, dtype=np.uint64)) >> np.uint64(1)).reshape(B, R)
    ridx = (np.arange(B * R) % 17).reshape(B, R).astype(np.uint64)
    toks = np.zeros((B, R), np.int64)
    for j in range(R):
        params = [P(temperature=float(T[r]), top_k=int(K[r]), top_p=float(TP[r])) for r in range(B)]
        toks[:, j] = S.sample(x, params, [int(s) for s in rseeds[:, j]], [int(i) for i in ridx[:, j]],
                              [msk[r] if has_mask[r] else None for r in range(B)])
    out.update(rows_x=x, rows_T=T, rows_K=K, rows_TP=TP, rows_mask=msk, rows_has_mask=has_mask, rows_seed=rseeds,
               rows_idx=ridx, rows_tok=toks)

    # edge rows (sampling.py:70-84 corner cases)
    Ve = 16
    base = normal(300, Ve).astype(np.float32)
    edge = []
    def row(v=None, **kw):
        edge.append((base.copy() if v is None else np.asarray(v, np.float32), kw))
    r = base.copy(); r[3] = np.nan; row(r, T=1.0)                      # NaN -> -1
    row(T=1.0, mask=np.zeros(Ve, bool))                               # all masked -> -1
    r = base.copy(); r[5] = np.inf; r[9] = np.inf; row(r, T=1.0)      # +inf, T > 0 -> lowest +inf
    r = base.copy(); r[5] = np.inf; row(r, T=0.0)                     # +inf greedy
    r = base.copy(); r[2] = -np.inf; r[7] = -np.inf; row(r, T=0.9)
    row(np.full(Ve, 1.5), T=1.0)                                      # all ties
    row(np.full(Ve, 1.5), T=0.0)
    r = np.zeros(Ve, np.float32); r[4] = -0.0; r[6] = 2.0; r[10] = 2.0; row(r, T=0.5, K=2)
    row(T=1e-50)                                                      # float32(t) == 0
    row(T=1e30, P=0.5)
    row(T=1.0, K=100)                                                 # top_k > V
    m1 = np.zeros(Ve, bool); m1[11] = True; row(T=2.0, mask=m1)       # one allowed
    row(T=0.0, mask=m1)
    r = base.copy(); r[0] = np.nan; row(r, T=0.0, mask=m1)            # masked NaN still -1
    r = np.full(Ve, -np.inf, np.float32); r[6] = 1.0; row(r, T=1.0)
    r = np.full(Ve, -3.4028235e38, np.float32); row(r, T=0.0, mask=m1)  # -FLT_MAX ties with masked
    row(T=1.0, P=1e-9)
    row(T=0.25, K=3, P=0.6)
    ex, et, ek, ep, em, ehm = [], [], [], [], [], []
    for v, kw in edge:
        ex.append(v)
        et.append(kw.get("T", 1.0))
        ek.append(kw.get("K", 0))
        ep.append(kw.get("P", 1.0))
        m = kw.get("mask")
        ehm.append(m is not None)
        em.append(m if m is not None else np.ones(Ve, bool))
    ex = np.stack(ex)
    eseeds = np.arange(8, dtype=np.uint64) * np.uint64(7919)
    etok = np.zeros((len(edge), 8), np.int64)
    for j in range(8):
        etok[:, j] = S.sample(ex, [P(temperature=float(et[i]), top_k=int(ek[i]), top_p=float(ep[i]))
                                   for i in range(len(edge))], [int(eseeds[j])] * len(edge), [j] * len(edge),
                              [em[i] if ehm[i] else None for i in range(len(edge))])
    out.update(edge_x=ex, edge_T=np.array(et), edge_K=np.array(ek), edge_TP=np.array(ep), edge_mask=np.stack(em),
               edge_has_mask=np.array(ehm), edge_seed=eseeds, edge_tok=etok)

    # dist rows
    nd = 12
    dp = [(1.0, 0, 1.0), (0.7, 5, 1.0), (1.3, 0, 0.8), (0.5, 50, 0.9), (2.0, 0, 0.3), (1.0, 1, 1.0)] * 2
    dx = x[:nd]
    out["dist_x"], out["dist_params"] = dx, np.array(dp, np.float64)
    out["dist_mask"] = np.stack([msk[r] for r in range(nd)])
    out["dist_has_mask"] = np.array([r % 3 == 0 for r in range(nd)])
    out["dist_out"] = np.stack([S.dist(dx[r], P(temperature=t, top_k=int(k), top_p=p),
                                       out["dist_mask"][r] if out["dist_has_mask"][r] else None)
                                for r, (t, k, p) in enumerate(dp)])

    # draw rows
    qd = np.abs(normal(500, 8 * 300).reshape(8, 300)) ** 3
    qd[1, 250:] = 0
    qd[2, :100] = 0
    qd[3] = 0
    qd[3, 17] = 1.0
    qd = qd / qd.sum(1, keepdims=True)
    du = unif(501, 8 * 16).reshape(8, 16)
    du[:, 0] = 0.0
    du[:, 1] = 1.0 - 2.0 ** -53
    out["draw_q"], out["draw_u"] = qd, du
    out["draw_out"] = np.array([[S.draw(qd[r], float(u)) for u in du[r]] for r in range(8)], np.int64)

    # mss nodes (spec.py:88-103)
    Vm, nm = 20, 40
    ms_p, ms_tok, ms_q, ms_has_q, ms_seed, ms_i, ms_out_t, ms_out_r = [], [], [], [], [], [], [], []
    for n in range(nm):
        zp = normal(600 + n, Vm) * 1.5
        p = np.exp(zp - zp.max())
        p /= p.sum()
        nk = 1 + n % 3
        toks, qs, hq = [], [], []
        for k in range(nk):
            zq = zp + normal(700 + 10 * n + k, Vm) * (0.3 + n % 4)
            q = np.exp(zq - zq.max())
            q /= q.sum()
            toks.append(int(np.searchsorted(np.cumsum(q), unif(800 + n, 3)[k] * q.sum())) % Vm)
            one_hot = (n + k) % 5 == 0
            qs.append(np.zeros(Vm) if one_hot else q)
            hq.append(not one_hot)
        seed, i = int(mix_np(900, np.array([n], np.uint64))[0]), n % 7
        t, r = SP.mss(p, [(toks[k], qs[k] if hq[k] else None) for k in range(nk)], seed, i)
        ms_p.append(p)
        ms_tok.append(toks + [-1] * (3 - nk))
        ms_q.append(np.stack(qs + [np.zeros(Vm)] * (3 - nk)))
        ms_has_q.append(hq + [False] * (3 - nk))
        ms_seed.append(seed)
        ms_i.append(i)
        ms_out_t.append(t)
        ms_out_r.append(-1 if r is None else r)
    out.update(mss_p=np.stack(ms_p), mss_tok=np.array(ms_tok, np.int64), mss_q=np.stack(ms_q),
               mss_has_q=np.array(ms_has_q), mss_seed=np.array(ms_seed, np.uint64), mss_i=np.array(ms_i, np.int64),
               mss_out_tok=np.array(ms_out_t, np.int64), mss_out_kid=np.array(ms_out_r, np.int64))

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sampling_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {sorted(out)}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
