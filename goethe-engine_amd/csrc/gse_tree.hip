// Speculative decoding on the device: the acceptance walk of a verify round (goethe_engine/engine.py:262-298 with
// spec.py:88-103 mss at strict nodes) and the drafter's child selection (spec.py:151-159 TreeDrafter._pick).
//
// Verify. A node's outcome does not depend on the path that reaches it: its uniform index is nout0 + depth (one token
// is committed per level, engine.py:272,282) and its target row, mask and history are fixed by the path to it. So every
// node is decided in parallel and the walk only follows the decisions:
//   1. the selection pass (main / split-row / exact) over all node rows: the sampled token of every node, and for
//      GSE_ROW_MSS nodes the maximum of z and the keep boundary of dist() (sampling.py:88-97);
//   2. stats: per MSS node the exact kept mass C = sum(keep e), e = exp(z - M), so that p0 = keep e / C is dist();
//      per q row given as drafter logits the maximum and exact mass of softmax(x / t) (spec.py:157);
//   3. residual passes 1..max_kids: pass r computes res_r = max(p_{r-1} - q_{r-1}, 0) (one-hot q: p with p[x] = 0) over
//      the row in slices, exact fixed-point partial sums; the node's last slice (atomic ticket) forms the total,
//      p_r = res_r / total (unchanged when the total is 0, spec.py:101-102), tests kid r (accepted iff q(x) > 0 and
//      uniform(mix(seed, 2^40 + r), i) q(x) < p_r(x), spec.py:93-94) or, after the last kid, draws from p in vocabulary
//      order with uniform(mix(seed, 2^41), i) (spec.py:103, sampling.py:100-104); kid 0 is tested at the start of pass 1;
//   4. the walk: from each anchor, MSS nodes take their decision, the others their sampled token and the first kid
//      holding it (engine.py:284-285); a token -1 ends the walk as an error (engine.py:286-288).
// Every slice of a node computes the same values from the same partials, read in slice order, so the decisions are
// deterministic and identical in every workgroup.
//
// Pick. t == 0: the n largest tokens in stable descending order (ties to the lowest id), per slice then merged by the
// row's last slice. t > 0: the maximum of z = x / t, the exact mass E = sum(exp(z - M)) in fixed point per slice, then
// one workgroup per draw k finds the first index whose inclusive prefix reaches uniform(mix(seed, 2^42 + k), at) * E.
#include "gse_rowctx.h"

namespace gse {

namespace {

constexpr int TT = 256;          // threads per slice workgroup
constexpr int TS = CH;           // tokens per slice
constexpr int TK = TS / TT;      // tokens per thread (strided: token s0 + k * TT + tid)
constexpr int TSEG = TS / WAVE;  // 64-token segments of a slice
constexpr uint64_t SALT_ACC = 1ull << 40, SALT_RES = 1ull << 41, SALT_DRAFT = 1ull << 42;

// ---- fixed-point helpers -------------------------------------------------------------------------------------------

__device__ __forceinline__ Fx fx_zero() { return Fx{0ull, 0ull}; }

// Block sum of one Fx per thread (exact): every thread gets it.
__device__ __forceinline__ Fx block_fx_sum(Fx v, uint64_t *red) {
  const uint64_t hi = wave_sum_u64(v.hi), lo = wave_sum_u64(v.lo);
  __syncthreads();
  if (lane_id() == 0) {
    red[2 * (threadIdx.x >> 6)] = hi;
    red[2 * (threadIdx.x >> 6) + 1] = lo;
  }
  __syncthreads();
  Fx t = fx_zero();
#pragma unroll
  for (int w = 0; w < TT / WAVE; ++w) t = fx_add(t, Fx{red[2 * w], red[2 * w + 1]});
  __syncthreads();
  return t;
}

__device__ __forceinline__ int block_max_i32(int v, int *red) {
  v = (int)wave_max_u32((uint32_t)(v + 1)) - 1;  // (v >= -1)
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int m = red[0];
#pragma unroll
  for (int w = 1; w < TT / WAVE; ++w) m = max(m, red[w]);
  __syncthreads();
  return m;
}

__device__ __forceinline__ double block_max_f64(double v, double *red) {
  v = lane63(wave_scan(v, (double)-INFINITY, [](double x, double y) { return fmax(x, y); }));
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double m = red[0];
#pragma unroll
  for (int w = 1; w < TT / WAVE; ++w) m = fmax(m, red[w]);
  __syncthreads();
  return m;
}

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t *red) {
  v = wave_sum_u32(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t m = 0;
#pragma unroll
  for (int w = 0; w < TT / WAVE; ++w) m += red[w];
  __syncthreads();
  return m;
}

// ---- q rows: softmax(x / t) of drafter logits, or fp64 probability rows -------------------------------------------

struct QRow {
  int kind;
  const char *base;
  double t, M, E;  // logits: z = x / t, M = max z, E = sum exp(z - M) (exact fixed point)
};

__device__ __forceinline__ double qz(const QRow &q, int i) {
  const double x = q.kind == GSE_Q_LOGITS_BF16 ? (double)bf16_to_f32(((const uint16_t *)q.base)[i])
                                                : (double)((const float *)q.base)[i];
  return x / q.t;
}
__device__ __forceinline__ double q_at(const QRow &q, int i) {
  if (q.kind == GSE_Q_PROB) return ((const double *)q.base)[i];
  return exp(qz(q, i) - q.M) / q.E;
}

// ---- the dist() of a node's target row: p0_i = keep_i e_i / C -----------------------------------------------------

struct Tgt {
  RowCtx c;
  double M;        // maximum of z
  uint64_t kkeep;  // packed key of the last kept rank (0: every token with z > -inf is kept)
};

__device__ __forceinline__ double tgt_e(const Tgt &g, int t, uint32_t cnt) {
  bool fn = false, ff = false;
  float xm;
  const uint32_t k = elem_key(g.c, load_one(g.c, t), cnt, mask_bit(g.c, t), fn, ff, xm);
  if (k <= KEY_NEGINF || pack(k, (uint32_t)t) < g.kkeep) return 0.0;
  return exp((double)fkey_inv(k) - g.M);
}

// History count of token x in the row (every thread of the block calls it; all get the count).
__device__ __forceinline__ uint32_t hist_count(const RowCtx &c, const int32_t *hist, int x, uint32_t *red) {
  uint32_t n = 0;
  if (c.pen)
    for (int j = c.hb + (int)threadIdx.x; j < c.he; j += TT) n += hist[j] == x ? 1u : 0u;
  return block_sum_u32(n, red);
}

struct TreeShared {
  uint32_t cnt[TS];            // history counts of the slice's tokens
  uint64_t seg[2 * TSEG];      // segment sums (Fx hi, lo)
  uint64_t red[16];
  double redd[8];
  int redi[8];
  uint32_t redu[8];
  uint32_t ticket;
  int found;
};

// Kids of node u in draft order: rows j > u with parent[j] == u, up to the next anchor (parent -1).
struct Kids {
  int n;
  int row[GSE_MAX_KIDS];
  int tok[GSE_MAX_KIDS];
  int qs[GSE_MAX_KIDS];  // index into the node's distinct q rows, -1 one-hot
  int nq;
  int qrow[GSE_MAX_KIDS];
  bool over;             // more kids than GSE_MAX_KIDS / max_kids
};

struct TreeArgs {
  ScanArgs s;              // the target rows (params, logits, mask, history) and the selection's RowInfo
  const int32_t *parent, *token, *qrow;
  gse_qrows q;
  int nodes, max_kids, nsl;
  const int32_t *anchor;
  int requests;
  const int32_t *sampled;  // [nodes] tokens of the selection pass
  TreeNode *st;            // [nodes]
  Fx *npart;               // [nodes][GSE_MAX_KIDS + 1][nsl]
  int32_t *nlast;          // [nodes][GSE_MAX_KIDS + 1][nsl]
  double *qmax;            // [qrows][nsl]
  Fx *qpart;               // [qrows][nsl]
  QFin *qfin;              // [qrows]
  gse_tree_out out;
};

__device__ __forceinline__ void find_kids(const TreeArgs &a, int u, Kids &k) {
  k.n = 0;
  k.nq = 0;
  k.over = false;
  for (int j = u + 1; j < a.nodes; ++j) {
    const int pj = a.parent[j];
    if (pj < 0) break;
    if (pj != u) continue;
    if (k.n >= a.max_kids || k.n >= GSE_MAX_KIDS) {
      k.over = true;
      break;
    }
    k.row[k.n] = j;
    k.tok[k.n] = a.token[j];
    const int qr = a.qrow ? a.qrow[j] : -1;
    int qs = -1;
    if (qr >= 0 && qr < (int)a.q.rows) {
      for (int m = 0; m < k.nq; ++m)
        if (k.qrow[m] == qr) qs = m;
      if (qs < 0) {
        qs = k.nq++;
        k.qrow[qs] = qr;
      }
    }
    k.qs[k.n] = qs;
    ++k.n;
  }
}

__device__ __forceinline__ QRow qrow_of(const TreeArgs &a, int qr) {
  QRow q;
  q.kind = (int)a.q.kind;
  const size_t es = a.q.kind == GSE_Q_PROB ? 8 : a.q.kind == GSE_Q_LOGITS_BF16 ? 2 : 4;
  q.base = (const char *)a.q.q + (size_t)qr * (size_t)a.q.ld * es;
  q.t = a.q.kind == GSE_Q_PROB ? 1.0 : a.q.temperature[qr];
  q.M = a.qfin[qr].M;
  q.E = a.qfin[qr].E;
  return q;
}

// The chain of residuals at token i (spec.py:95-102): p_0 = p0; res_{r+1} = max(p_r - q_r, 0) (one-hot kid: p_r with
// the kid's token set to 0); p_{r+1} = res_{r+1} / sig[r + 1], or p_r when that total is 0. Returns res_d (norm false)
// or p_d (norm true); d == 0 returns p0. The kids' q values are formed as the chain needs them (kids that share a q row,
// as SpecInfer's do, share one evaluation).
__device__ __forceinline__ double chain(const Kids &k, const QRow *qr, double p0, int i, const double *sig, int d,
                                        bool norm) {
  double p = p0;
  int qid = -2;
  double qv = 0.0;
  for (int r = 0; r < d; ++r) {
    double res;
    if (k.qs[r] < 0) {
      res = i == k.tok[r] ? 0.0 : p;
    } else {
      if (k.qs[r] != qid) {
        qid = k.qs[r];
        qv = q_at(qr[qid], i);
      }
      res = fmax(p - qv, 0.0);
    }
    const double pn = sig[r + 1] > 0.0 ? res / sig[r + 1] : p;
    if (r == d - 1) return norm ? pn : res;
    p = pn;
  }
  return p;
}

// The node's p0 at one token (every thread calls; all get it).
__device__ __forceinline__ double p0_at(const TreeArgs &a, const Tgt &g, int x, double clast, TreeShared &sh) {
  const uint32_t cnt = hist_count(g.c, a.s.hist, x, sh.redu);
  return tgt_e(g, x, cnt) / clast;
}

// The first index of slice [s0, s1) whose inclusive prefix of the weights wfn (after `before`, the exact mass of the
// slices ahead) reaches thr; -1 if none. Exact fixed-point prefixes: 64-token segment sums (wave w takes segments w,
// w + 4, ...), the crossing segment, then its weights again and their scan. Every thread gets the result.
template <typename W>
__device__ int slice_find(int s0, int s1, Fx before, double thr, W wfn, TreeShared &sh) {
  const int tid = threadIdx.x;
  const int wv = tid >> 6, ln = lane_id();
  for (int g = wv; g < TSEG; g += TT / WAVE) {
    const int i = s0 + g * WAVE + ln;
    const Fx f = fx_of(i < s1 ? wfn(i) : 0.0);
    const uint64_t hi = wave_sum_u64(f.hi), lo = wave_sum_u64(f.lo);
    if (ln == 0) {
      sh.seg[2 * g] = hi;
      sh.seg[2 * g + 1] = lo;
    }
  }
  if (tid == 0) sh.found = -1;
  __syncthreads();
  if (wv == 0) {
    // the crossing segment: two segments per lane, inclusive prefixes
    const Fx a0 = Fx{sh.seg[4 * ln], sh.seg[4 * ln + 1]}, a1 = Fx{sh.seg[4 * ln + 2], sh.seg[4 * ln + 3]};
    const Fx pair = fx_add(a0, a1);
    const uint64_t ih = wave_incl_scan_u64(pair.hi), il = wave_incl_scan_u64(pair.lo);
    const Fx ex = fx_add(before, Fx{ih - pair.hi, il - pair.lo});
    const Fx i0 = fx_add(ex, a0), i1 = fx_add(i0, a1);
    const bool h0 = fx_val(i0) >= thr, h1 = fx_val(i1) >= thr;
    const uint64_t bl = ballot64(h0 || h1);
    if (bl) {
      const int l = __builtin_ctzll(bl);
      const bool first = __shfl(h0 ? 1 : 0, l, WAVE) != 0;
      const int g = 2 * l + (first ? 0 : 1);
      const Fx gb = first ? Fx{shfl_u64(ex.hi, l), shfl_u64(ex.lo, l)} : Fx{shfl_u64(i0.hi, l), shfl_u64(i0.lo, l)};
      const int i = s0 + g * WAVE + ln;
      const Fx f = fx_of(i < s1 ? wfn(i) : 0.0);
      const uint64_t ch = wave_incl_scan_u64(f.hi), cl = wave_incl_scan_u64(f.lo);
      const uint64_t hb = ballot64(fx_val(fx_add(gb, Fx{ch, cl})) >= thr);
      if (ln == 0) sh.found = hb ? s0 + g * WAVE + __builtin_ctzll(hb) : -1;
    }
  }
  __syncthreads();
  const int r = sh.found;
  __syncthreads();
  return r;
}

// ---- verify: stats --------------------------------------------------------------------------------------------------

__device__ __forceinline__ bool node_live(const TreeArgs &a, int u, const gse_row &P) {
  if (!(P.flags & GSE_ROW_MSS)) return false;
  const uint32_t f = a.s.info[u].flags;
  return (f & R_DONE) && !(f & (R_SPECIAL | R_BAD | R_GREEDY));
}

__device__ __forceinline__ Tgt tgt_of(const TreeArgs &a, int u, const gse_row &P) {
  Tgt g;
  g.c = make_ctx(a.s, u, P);
  const RowInfo &ri = a.s.info[u];
  g.M = (double)fkey_inv(pk_key(ri.cmax));
  g.kkeep = ri.kkeep;
  return g;
}

// Maximum of z = x / t over each slice of each logits q row.
__global__ __launch_bounds__(TT) void qmax_kernel(TreeArgs a) {
  __shared__ double red[8];
  const int s = blockIdx.x, qr = blockIdx.y;
  QRow q;
  q.kind = (int)a.q.kind;
  q.base = (const char *)a.q.q + (size_t)qr * (size_t)a.q.ld * (a.q.kind == GSE_Q_LOGITS_BF16 ? 2 : 4);
  q.t = a.q.temperature[qr];
  const int V = a.s.V, s0 = s * TS, s1 = min(V, s0 + TS);
  double m = -INFINITY;
  for (int i = s0 + (int)threadIdx.x; i < s1; i += TT) m = fmax(m, qz(q, i));
  m = block_max_f64(m, red);
  if (threadIdx.x == 0) a.qmax[(size_t)qr * a.nsl + s] = m;
}

// Per MSS node: the exact kept mass per slice (the last slice forms C); per logits q row: exp(z - M) per slice (the
// last slice forms E).
__global__ __launch_bounds__(TT) void tstats_kernel(TreeArgs a) {
  __shared__ TreeShared sh;
  const int s = blockIdx.x, y = blockIdx.y, tid = threadIdx.x;
  const int V = a.s.V, s0 = s * TS, s1 = min(V, s0 + TS);
  if (y < a.nodes) {
    const int u = y;
    const gse_row P = a.s.params[u];
    if (!node_live(a, u, P)) return;
    const Tgt g = tgt_of(a, u, P);
    if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);
    Fx f = fx_zero();
    int last = -1;
    for (int k = 0; k < TK; ++k) {
      const int i = s0 + k * TT + tid;
      if (i >= s1) break;
      const double e = tgt_e(g, i, g.c.pen ? sh.cnt[i - s0] : 0u);
      f = fx_add(f, fx_of(e));
      if (e > 0.0) last = i;
    }
    f = block_fx_sum(f, sh.red);
    last = block_max_i32(last, sh.redi);
    const size_t o = ((size_t)u * (GSE_MAX_KIDS + 1)) * a.nsl + s;
    if (tid == 0) {
      st_ag(&a.npart[o].hi, f.hi);
      st_ag(&a.npart[o].lo, f.lo);
      st_ag(&a.nlast[o], last);
    }
    store_wait();
    __syncthreads();
    if (tid == 0) sh.ticket = ticket_add(&a.st[u].ticket);
    __syncthreads();
    if (sh.ticket != (uint32_t)(a.nsl - 1)) return;
    if (tid == 0) {
      Fx t = fx_zero();
      for (int j = 0; j < a.nsl; ++j) t = fx_add(t, Fx{ld_ag(&a.npart[o - s + j].hi), ld_ag(&a.npart[o - s + j].lo)});
      TreeNode &nd = a.st[u];
      nd.clast = fx_val(t);
      nd.sig[0] = nd.clast;
      nd.next = 1;
      nd.token = -1;
      nd.kid = -1;
      nd.ticket = 0;
    }
    return;
  }
  const int qr = y - a.nodes;
  if (a.q.kind == GSE_Q_PROB) return;
  QRow q;
  q.kind = (int)a.q.kind;
  q.base = (const char *)a.q.q + (size_t)qr * (size_t)a.q.ld * (a.q.kind == GSE_Q_LOGITS_BF16 ? 2 : 4);
  q.t = a.q.temperature[qr];
  double M = -INFINITY;
  for (int j = 0; j < a.nsl; ++j) M = fmax(M, a.qmax[(size_t)qr * a.nsl + j]);
  Fx f = fx_zero();
  for (int k = 0; k < TK; ++k) {
    const int i = s0 + k * TT + tid;
    if (i >= s1) break;
    f = fx_add(f, fx_of(exp(qz(q, i) - M)));
  }
  f = block_fx_sum(f, sh.red);
  const size_t o = (size_t)qr * a.nsl + s;
  if (tid == 0) {
    st_ag(&a.qpart[o].hi, f.hi);
    st_ag(&a.qpart[o].lo, f.lo);
  }
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&a.qfin[qr].ticket);
  __syncthreads();
  if (sh.ticket != (uint32_t)(a.nsl - 1)) return;
  if (tid == 0) {
    Fx t = fx_zero();
    for (int j = 0; j < a.nsl; ++j)
      t = fx_add(t, Fx{ld_ag(&a.qpart[o - s + j].hi), ld_ag(&a.qpart[o - s + j].lo)});
    a.qfin[qr].M = M;
    a.qfin[qr].E = fx_val(t);
    a.qfin[qr].ticket = 0;
  }
}

// ---- verify: residual passes ----------------------------------------------------------------------------------------


// A node's uniform data for one workgroup, in LDS: its kids, their q rows, the residual totals.
struct NodeShared {
  Kids k;
  QRow qr[GSE_MAX_KIDS];
  double sig[GSE_MAX_KIDS + 1];
  double clast;
};

__device__ __forceinline__ void load_node(const TreeArgs &a, int u, NodeShared &ns) {
  if (threadIdx.x == 0) {
    find_kids(a, u, ns.k);
    for (int m = 0; m < ns.k.nq; ++m) ns.qr[m] = qrow_of(a, ns.k.qrow[m]);
    const TreeNode &nd = a.st[u];
    ns.clast = nd.clast;
    for (int r = 0; r <= GSE_MAX_KIDS; ++r) ns.sig[r] = nd.sig[r];
  }
  __syncthreads();
}

// The node's draw after its last kid was rejected (run by one workgroup): from p_d, d the deepest chain level with a
// positive total (sig[0] = C > 0 for a live node), in vocabulary order (sampling.py:100-104), with the uniform
// uniform(mix(seed, 2^41), i) (spec.py:103). The unnormalised weights (keep e for d = 0, res_d otherwise) give the same
// count(c < u c[-1]) as the normalised p_d.
__device__ int node_draw(const TreeArgs &a, int u, const gse_row &P, const Tgt &g, const NodeShared &ns, int kdone,
                         TreeShared &sh) {
  int d = kdone;
  while (d > 0 && !(ns.sig[d] > 0.0)) --d;
  const size_t o = ((size_t)u * (GSE_MAX_KIDS + 1) + d) * a.nsl;
  Fx tot = fx_zero();
  int last = -1;
  for (int j = 0; j < a.nsl; ++j) {
    tot = fx_add(tot, Fx{ld_ag(&a.npart[o + j].hi), ld_ag(&a.npart[o + j].lo)});
    last = max(last, ld_ag(&a.nlast[o + j]));
  }
  if (last < 0) return -1;
  const double thr = uniform64(mix64(P.seed, SALT_RES), P.idx) * fx_val(tot);
  Fx before = fx_zero();  // the crossing slice
  int sx = a.nsl - 1;
  for (int j = 0; j < a.nsl; ++j) {
    const Fx nxt = fx_add(before, Fx{ld_ag(&a.npart[o + j].hi), ld_ag(&a.npart[o + j].lo)});
    if (fx_val(nxt) >= thr) {
      sx = j;
      break;
    }
    before = nxt;
  }
  const int s0 = sx * TS, s1 = min(a.s.V, s0 + TS);
  if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);
  const int j = slice_find(s0, s1, before, thr, [&](int i) {
    const double e = tgt_e(g, i, g.c.pen ? sh.cnt[i - s0] : 0u);
    return d == 0 ? e : chain(ns.k, ns.qr, e / ns.clast, i, ns.sig, d, false);
  }, sh);
  const int jj = j < 0 ? last : j;
  return jj < last ? jj : last;
}

__device__ __forceinline__ bool kid_accepts(const gse_row &P, int r, double px, double qx) {
  return qx > 0.0 && uniform64(mix64(P.seed, SALT_ACC + (uint64_t)r), P.idx) * qx < px;
}

// Kid r's test (spec.py:93-94) against p_r; every thread calls it and gets the answer.
__device__ __forceinline__ bool test_kid(const TreeArgs &a, const gse_row &P, const Tgt &g, const NodeShared &ns, int r,
                                         TreeShared &sh) {
  const int x = ns.k.tok[r];
  if (x < 0 || x >= a.s.V) return false;  // (not a token of this vocabulary: never accepted)
  const double p0 = p0_at(a, g, x, ns.clast, sh);
  const double px = chain(ns.k, ns.qr, p0, x, ns.sig, r, true);
  const double qx = ns.k.qs[r] < 0 ? 1.0 : q_at(ns.qr[ns.k.qs[r]], x);
  return kid_accepts(P, r, px, qx);
}

// Pass r over slice blockIdx.x of node blockIdx.y (see the file comment).
__global__ __launch_bounds__(TT) void tpass_kernel(TreeArgs a, int r) {
  __shared__ TreeShared sh;
  __shared__ NodeShared ns;
  const int s = blockIdx.x, u = blockIdx.y, tid = threadIdx.x;
  const gse_row P = a.s.params[u];
  if (!node_live(a, u, P)) return;
  TreeNode &nd = a.st[u];
  if ((int)nd.next != r) return;
  load_node(a, u, ns);
  const Tgt g = tgt_of(a, u, P);
  const int V = a.s.V, s0 = s * TS, s1 = min(V, s0 + TS);
  if (r == 1) {
    if (ns.k.n == 0) {  // no kids: mss returns draw(p0, uniform(mix(seed, 2^41), i)) (spec.py:103)
      if (s == 0) {
        const int j = node_draw(a, u, P, g, ns, 0, sh);
        if (tid == 0) {
          nd.token = j;
          nd.kid = -1;
          nd.next = 0;
        }
      }
      return;
    }
    if (test_kid(a, P, g, ns, 0, sh)) {  // kid 0, tested alike by every slice
      if (s == 0 && tid == 0) {
        nd.token = ns.k.tok[0];
        nd.kid = ns.k.row[0];
        nd.next = 0;
      }
      return;
    }
  }
  // res_r over this slice: kid r - 1 was rejected
  if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);
  Fx f = fx_zero();
  int last = -1;
  for (int kk = 0; kk < TK; ++kk) {
    const int i = s0 + kk * TT + tid;
    if (i >= s1) break;
    const double e = tgt_e(g, i, g.c.pen ? sh.cnt[i - s0] : 0u);
    const double res = chain(ns.k, ns.qr, e / ns.clast, i, ns.sig, r, false);
    f = fx_add(f, fx_of(res));
    if (res > 0.0) last = i;
  }
  f = block_fx_sum(f, sh.red);
  last = block_max_i32(last, sh.redi);
  const size_t o = ((size_t)u * (GSE_MAX_KIDS + 1) + r) * a.nsl + s;
  if (tid == 0) {
    st_ag(&a.npart[o].hi, f.hi);
    st_ag(&a.npart[o].lo, f.lo);
    st_ag(&a.nlast[o], last);
  }
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&nd.ticket);
  __syncthreads();
  if (sh.ticket != (uint32_t)(a.nsl - 1)) return;
  // the node's last slice: the total of res_r, then kid r or the draw
  if (tid == 0) {
    Fx t = fx_zero();
    for (int j = 0; j < a.nsl; ++j) t = fx_add(t, Fx{ld_ag(&a.npart[o - s + j].hi), ld_ag(&a.npart[o - s + j].lo)});
    ns.sig[r] = fx_val(t);
    nd.sig[r] = ns.sig[r];
    nd.ticket = 0;
  }
  __syncthreads();
  if (r < ns.k.n) {
    const bool acc = test_kid(a, P, g, ns, r, sh);
    if (tid == 0) {
      if (acc) {
        nd.token = ns.k.tok[r];
        nd.kid = ns.k.row[r];
        nd.next = 0;
      } else {
        nd.next = r + 1;
      }
    }
    return;
  }
  const int j = node_draw(a, u, P, g, ns, r, sh);
  if (tid == 0) {
    nd.token = j;
    nd.kid = -1;
    nd.next = 0;
  }
}

// ---- verify: the walk ------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(64) void walk_kernel(TreeArgs a) {
  const int q = blockIdx.x * 64 + threadIdx.x;
  // node_token / node_kid of every node
  for (int u = q; u < a.nodes && (a.out.node_token || a.out.node_kid); u += gridDim.x * 64) {
    const gse_row &P = a.s.params[u];
    int tok, kid;
    if (P.flags & GSE_ROW_MSS) {
      const bool live = node_live(a, u, P);
      tok = live ? a.st[u].token : -1;
      kid = live ? a.st[u].kid : -1;
    } else {
      tok = a.sampled[u];
      kid = -1;
      if (tok >= 0)
        for (int j = u + 1; j < a.nodes && a.parent[j] >= 0; ++j)
          if (a.parent[j] == u && a.token[j] == tok) {
            kid = j;
            break;
          }
    }
    if (a.out.node_token) a.out.node_token[u] = tok;
    if (a.out.node_kid) a.out.node_kid[u] = kid;
  }
  if (q >= a.requests) return;
  int u = a.anchor[q];
  const int end = q + 1 < a.requests ? a.anchor[q + 1] : a.nodes;
  int n = 0;
  uint32_t status = GSE_WALK_OK;
  for (int step = 0; step <= end - a.anchor[q] && u >= 0 && u < end; ++step) {
    const gse_row &P = a.s.params[u];
    int tok, kid = -1;
    if (P.flags & GSE_ROW_MSS) {
      const bool live = node_live(a, u, P);
      tok = live ? a.st[u].token : -1;
      kid = live ? a.st[u].kid : -1;
    } else {
      tok = a.sampled[u];
      if (tok >= 0)
        for (int j = u + 1; j < end; ++j)
          if (a.parent[j] == u && a.token[j] == tok) {
            kid = j;
            break;
          }
    }
    if (tok < 0) {  // the path holds the node (engine.py:280-288 appends the kid before its row is decided)
      status = GSE_WALK_ERROR;
      if (n < a.out.emit_ld) a.out.emit_nodes[(int64_t)q * a.out.emit_ld + n] = u;
      break;
    }
    if (n < a.out.emit_ld) {
      a.out.emit_tokens[(int64_t)q * a.out.emit_ld + n] = tok;
      a.out.emit_nodes[(int64_t)q * a.out.emit_ld + n] = u;
    } else {
      status = GSE_WALK_TRUNCATED;
    }
    ++n;
    if (kid < 0) break;
    u = kid;
  }
  a.out.emit_len[q] = n;
  if (a.out.status) a.out.status[q] = status;
}

// ---- pick (spec.py:151-159) -----------------------------------------------------------------------------------------

struct PickArgs {
  gse_pick_batch b;
  int nsl;
  double *pmax;     // [rows][nsl]
  Fx *ppart;        // [rows][nsl]
  int32_t *plast;   // [rows][nsl]
  uint64_t *ptop;   // [rows][nsl][4 * GSE_MAX_KIDS] packed (key, id) top candidates per wave
  uint32_t *tick;   // [rows]
};

__device__ __forceinline__ float pick_x(const PickArgs &a, int row, int i) {
  const char *base = (const char *)a.b.x + (size_t)row * (size_t)a.b.ld * (a.b.dtype == GSE_BF16 ? 2 : 4);
  return a.b.dtype == GSE_BF16 ? bf16_to_f32(((const uint16_t *)base)[i]) : ((const float *)base)[i];
}

// t > 0: the maximum of z = x / t per slice. t == 0: the top-n packed (key(x), id) of each wave of the slice, then the
// row's last slice merges them (bitonic sort in LDS) and writes the n best.
__global__ __launch_bounds__(TT) void pick1_kernel(PickArgs a) {
  __shared__ double red[8];
  __shared__ uint64_t cand[TT / WAVE * GSE_MAX_KIDS * 32];
  __shared__ uint32_t ticket;
  const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int V = (int)a.b.vocab, s0 = s * TS, s1 = min(V, s0 + TS);
  const double t = a.b.temperature[row];
  const int n = min(max(a.b.n[row], 0), (int)min((int64_t)GSE_MAX_KIDS, a.b.out_ld));
  if (t > 0.0) {
    double m = -INFINITY;
    for (int i = s0 + tid; i < s1; i += TT) m = fmax(m, (double)pick_x(a, row, i) / t);
    m = block_max_f64(m, red);
    if (tid == 0) a.pmax[(size_t)row * a.nsl + s] = m;
    return;
  }
  if (n == 0) return;
  uint64_t v[TK];
  for (int k = 0; k < TK; ++k) {
    const int i = s0 + k * TT + tid;
    v[k] = i < s1 ? pack(fkey(pick_x(a, row, i)), (uint32_t)i) : 0ull;
  }
  // n rounds of the wave maximum, the winner removed
  uint64_t *wc = a.ptop + ((size_t)row * a.nsl + s) * (TT / WAVE) * GSE_MAX_KIDS + (tid >> 6) * GSE_MAX_KIDS;
  for (int r = 0; r < n; ++r) {
    uint64_t lm = 0;
    for (int k = 0; k < TK; ++k) lm = v[k] > lm ? v[k] : lm;
    const uint64_t wm = wave_max_u64(lm);
    for (int k = 0; k < TK; ++k)
      if (v[k] == wm) v[k] = 0ull;
    if (lane_id() == 0) st_ag(&wc[r], wm);
  }
  store_wait();
  __syncthreads();
  if (tid == 0) ticket = ticket_add(&a.tick[row]);
  __syncthreads();
  if (ticket != (uint32_t)(a.nsl - 1)) return;
  // merge the nsl * 4 lists of n in rounds of the LDS buffer, carrying the best n
  const int tot = a.nsl * (TT / WAVE) * GSE_MAX_KIDS;
  const uint64_t *all = a.ptop + (size_t)row * a.nsl * (TT / WAVE) * GSE_MAX_KIDS;
  uint64_t best[GSE_MAX_KIDS];
  for (int r = 0; r < GSE_MAX_KIDS; ++r) best[r] = 0ull;
  const int cap = TT / WAVE * GSE_MAX_KIDS * 32;
  for (int b0 = 0; b0 < tot; b0 += cap - GSE_MAX_KIDS) {
    // the buffer: the best so far, then the next entries
    const int nb = min(cap, GSE_MAX_KIDS + (tot - b0));
    const int np = pow2_ceil(nb);
    for (int i = tid; i < np; i += TT) {
      uint64_t x = 0ull;
      const int e = b0 + i - GSE_MAX_KIDS;  // entry of the lists: [slice][wave][GSE_MAX_KIDS], the first n filled
      if (i < GSE_MAX_KIDS) x = best[i];
      else if (i < nb && e % GSE_MAX_KIDS < n) x = ld_ag(&all[e]);
      cand[i] = x;
    }
    __syncthreads();
    block_sort_desc_u64(cand, np);
    for (int r = 0; r < GSE_MAX_KIDS; ++r) best[r] = r < n ? cand[r] : 0ull;
    __syncthreads();
  }
  if (tid < n) {
    const uint64_t pk = best[tid];
    const int id = pk ? (int)pk_id(pk) : -1;
    a.b.out_tokens[(int64_t)row * a.b.out_ld + tid] = id;
    a.b.out_logq[(int64_t)row * a.b.out_ld + tid] = id >= 0 ? (double)pick_x(a, row, id) : __builtin_nan("");
  }
  if (tid == 0) a.tick[row] = 0;
}

// t > 0: exact partial masses exp(z - M) per slice.
__global__ __launch_bounds__(TT) void pick2_kernel(PickArgs a) {
  __shared__ uint64_t red[16];
  __shared__ int redi[8];
  const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const double t = a.b.temperature[row];
  if (!(t > 0.0) || a.b.n[row] <= 0) return;
  const int V = (int)a.b.vocab, s0 = s * TS, s1 = min(V, s0 + TS);
  double M = -INFINITY;
  for (int j = 0; j < a.nsl; ++j) M = fmax(M, a.pmax[(size_t)row * a.nsl + j]);
  Fx f = fx_zero();
  int last = -1;
  for (int k = 0; k < TK; ++k) {
    const int i = s0 + k * TT + tid;
    if (i >= s1) break;
    const double e = exp((double)pick_x(a, row, i) / t - M);
    f = fx_add(f, fx_of(e));
    if (e > 0.0) last = i;
  }
  f = block_fx_sum(f, red);
  last = block_max_i32(last, redi);
  if (tid == 0) {
    a.ppart[(size_t)row * a.nsl + s] = f;
    a.plast[(size_t)row * a.nsl + s] = last;
  }
}

// t > 0: one workgroup per (row, draw k): draw(q, uniform(mix(seed, SALT_DRAFT + k), at)) in vocabulary order.
__global__ __launch_bounds__(TT) void pick3_kernel(PickArgs a) {
  __shared__ TreeShared sh;
  const int row = blockIdx.y, kd = blockIdx.x, tid = threadIdx.x;
  const double t = a.b.temperature[row];
  const int n = min(max(a.b.n[row], 0), (int)min((int64_t)GSE_MAX_KIDS, a.b.out_ld));
  if (!(t > 0.0) || kd >= n) return;
  const int V = (int)a.b.vocab;
  double M = -INFINITY;
  Fx tot = fx_zero();
  int last = -1;
  for (int j = 0; j < a.nsl; ++j) {
    M = fmax(M, a.pmax[(size_t)row * a.nsl + j]);
    tot = fx_add(tot, a.ppart[(size_t)row * a.nsl + j]);
    last = max(last, a.plast[(size_t)row * a.nsl + j]);
  }
  int tok = -1;
  double lq = __builtin_nan("");
  if (last >= 0) {
    const double E = fx_val(tot);
    const double thr = uniform64(mix64(a.b.seed[row], SALT_DRAFT + (uint64_t)kd), a.b.at[row]) * E;
    Fx before = fx_zero();
    int sx = a.nsl - 1;
    for (int j = 0; j < a.nsl; ++j) {
      const Fx nxt = fx_add(before, a.ppart[(size_t)row * a.nsl + j]);
      if (fx_val(nxt) >= thr) {
        sx = j;
        break;
      }
      before = nxt;
    }
    const int s0 = sx * TS, s1 = min(V, s0 + TS);
    const int j = slice_find(s0, s1, before, thr, [&](int i) { return exp((double)pick_x(a, row, i) / t - M); }, sh);
    tok = j < 0 ? last : min(j, last);
    lq = ((double)pick_x(a, row, tok) / t - M) - log(E);
  }
  if (tid == 0) {
    a.b.out_tokens[(int64_t)row * a.b.out_ld + kd] = tok;
    a.b.out_logq[(int64_t)row * a.b.out_ld + kd] = lq;
  }
}

}  // namespace

hipError_t launch_tree(const TreeLaunch &L, hipStream_t s) {
  TreeArgs a;
  a.s = L.s;
  a.parent = L.parent;
  a.token = L.token;
  a.qrow = L.qrow;
  a.q = L.q;
  a.nodes = L.s.rows;
  a.max_kids = L.max_kids;
  a.nsl = (L.s.V + TS - 1) / TS;
  a.anchor = L.anchor;
  a.requests = L.requests;
  a.sampled = L.sampled;
  a.st = L.st;
  a.npart = L.npart;
  a.nlast = L.nlast;
  a.qmax = L.qmax;
  a.qpart = L.qpart;
  a.qfin = L.qfin;
  a.out = L.out;
  const bool qlog = L.q.rows > 0 && L.q.kind != GSE_Q_PROB;
  if (qlog) hipLaunchKernelGGL(qmax_kernel, dim3(a.nsl, L.q.rows), dim3(TT), 0, s, a);
  hipLaunchKernelGGL(tstats_kernel, dim3(a.nsl, a.nodes + (qlog ? L.q.rows : 0)), dim3(TT), 0, s, a);
  // pass r: kid r - 1 rejected -> res_r; a node with k kids needs passes 1..k (one without kids draws in pass 1)
  for (int r = 1; r <= max(L.max_kids, 1); ++r) hipLaunchKernelGGL(tpass_kernel, dim3(a.nsl, a.nodes), dim3(TT), 0, s, a, r);
  hipLaunchKernelGGL(walk_kernel, dim3((max(a.requests, a.nodes) + 63) / 64), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_pick(const PickLaunch &L, hipStream_t s) {
  PickArgs a;
  a.b = L.b;
  a.nsl = ((int)L.b.vocab + TS - 1) / TS;
  a.pmax = L.pmax;
  a.ppart = L.ppart;
  a.plast = L.plast;
  a.ptop = L.ptop;
  a.tick = L.tick;
  const int nmax = (int)min((int64_t)GSE_MAX_KIDS, L.b.out_ld);
  hipLaunchKernelGGL(pick1_kernel, dim3(a.nsl, L.b.rows), dim3(TT), 0, s, a);
  hipLaunchKernelGGL(pick2_kernel, dim3(a.nsl, L.b.rows), dim3(TT), 0, s, a);
  hipLaunchKernelGGL(pick3_kernel, dim3(nmax, L.b.rows), dim3(TT), 0, s, a);
  return hipGetLastError();
}

}  // namespace gse
