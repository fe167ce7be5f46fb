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
#include <type_traits>

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

// ---- per-slice partials, read by one wave (lane l takes slices l, l + 64, ...: every load of a round at once) ------

// The exact total of the fixed-point partials p[0, n) (every lane gets it).
template <typename LD>
__device__ __forceinline__ Fx wave_fx_total(int n, LD ld) {
  Fx t = fx_zero();
  for (int j = lane_id(); j < n; j += WAVE) t = fx_add(t, ld(j));
  return Fx{wave_sum_u64(t.hi), wave_sum_u64(t.lo)};
}

// The first j whose inclusive prefix of the partials reaches thr, with the exact prefix before it (every lane gets
// them); when none does, n - 1 with the total of all n.
template <typename LD>
__device__ __forceinline__ int wave_fx_cross(int n, double thr, LD ld, Fx &before) {
  const int ln = lane_id();
  Fx run = fx_zero();
  for (int j0 = 0; j0 < n; j0 += WAVE) {
    const int j = j0 + ln;
    const Fx v = j < n ? ld(j) : fx_zero();
    const uint64_t ih = wave_incl_scan_u64(v.hi), il = wave_incl_scan_u64(v.lo);
    const Fx inc = fx_add(run, Fx{ih, il});
    const uint64_t hit = ballot64(j < n && fx_val(inc) >= thr);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      before = Fx{shfl_u64(inc.hi - v.hi, l), shfl_u64(inc.lo - v.lo, l)};
      return j0 + l;
    }
    run = fx_add(run, Fx{shfl_u64(ih, WAVE - 1), shfl_u64(il, WAVE - 1)});
  }
  before = run;
  return n - 1;
}

__device__ __forceinline__ double wave_max_f64(double v) {
  return lane63(wave_scan(v, (double)-INFINITY, [](double x, double y) { return fmax(x, y); }));
}

// ---- q rows: softmax(x / t) of drafter logits, or fp64 probability rows -------------------------------------------

struct QRow {
  int kind;
  const char *base;
  bool t1;                // t == 1: z = x
  double t, M, invE;      // logits: z = x / t, M = max z, invE = 1 / sum exp(z - M)
};

// The raw value of token i (the probability, or the logit widened to fp64).
__device__ __forceinline__ double q_raw(const QRow &q, int i) {
  if (q.kind == GSE_Q_PROB) return ((const double *)q.base)[i];
  if (q.kind == GSE_Q_LOGITS_BF16) return (double)bf16_to_f32(((const uint16_t *)q.base)[i]);
  return (double)((const float *)q.base)[i];
}
// q at a token from its raw value: the probability, or exp(z - M) / E (every evaluation of one row takes this same
// path, so the sums and the tests of a round see one set of values).
__device__ __forceinline__ double q_of_raw(const QRow &q, double r, const double *etab) {
  if (q.kind == GSE_Q_PROB) return r;
  const double z = q.t1 ? r : r / q.t;
  return exp_nonpos(z - q.M, etab) * q.invE;
}
__device__ __forceinline__ double q_at(const QRow &q, int i, const double *etab) {
  return q_of_raw(q, q_raw(q, i), etab);
}

// ---- the dist() of a node's target row: p0_i = keep_i e_i / C -----------------------------------------------------

struct Tgt {
  RowCtx c;
  double M;        // maximum of z
  uint64_t kkeep;  // packed key of the last kept rank (0: every token with z > -inf is kept)
};

// keep_i e_i of token t from its raw logit x, its mask word and its history count.
__device__ __forceinline__ double tgt_e(const Tgt &g, int t, float x, uint32_t mword, uint32_t cnt,
                                        const double *etab) {
  bool fn = false, ff = false;
  float xm;
  const uint32_t k = elem_key(g.c, x, cnt, (mword >> (t & 31)) & 1u, fn, ff, xm);
  if (k <= KEY_NEGINF || pack(k, (uint32_t)t) < g.kkeep) return 0.0;
  return exp_nonpos((double)fkey_inv(k) - g.M, etab);
}
__device__ __forceinline__ uint32_t mask_word(const RowCtx &c, int t) { return c.mw ? c.mw[t >> 5] : 0xFFFFFFFFu; }
__device__ __forceinline__ double tgt_e_at(const Tgt &g, int t, uint32_t cnt, const double *etab) {
  return tgt_e(g, t, load_one(g.c, t), mask_word(g.c, t), cnt, etab);
}

// The same weight for the streaming loops, with the division by the temperature chosen at compile time (a live node
// is never greedy, so z is x / T or x): the value tgt_e gives, with fewer instructions.
template <bool DIV>
__device__ __forceinline__ double tgt_w(const Tgt &g, int t, float x, uint32_t mword, uint32_t cnt,
                                        const double *etab) {
  if (cnt) x = penalize(x, cnt, g.c.rp, g.c.fp, g.c.pp);
  const float z = DIV ? div_rn(x, g.c.T, g.c.Td, g.c.Rd) : x;
  if (!((mword >> (t & 31)) & 1u) || !(z > -INFINITY)) return 0.0;
  if (g.kkeep && pack(fkey(z), (uint32_t)t) < g.kkeep) return 0.0;
  return exp_nonpos((double)z - g.M, etab);
}

// q from its raw value with its kind chosen at compile time: QK 0 probabilities, 1 logits with t == 1, 2 logits with
// another t (the value q_of_raw gives).
template <int QK>
__device__ __forceinline__ double q_w(const QRow &q, double r, const double *etab) {
  if constexpr (QK == 0) {
    return r;
  } else {
    const double z = QK == 1 ? r : r / q.t;
    return exp_nonpos(z - q.M, etab) * q.invE;
  }
}

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};
template <int N>
struct IntC {
  static constexpr int value = N;
};
template <typename F>
__device__ __forceinline__ void with_bool(bool d, F f) {
  if (d) f(BoolC<true>{});
  else f(BoolC<false>{});
}
template <typename F>
__device__ __forceinline__ void with_div(bool d, F f) {
  with_bool(d, f);
}

// ---- streaming a slice --------------------------------------------------------------------------------------------
// Thread tid takes the groups g < NG of its slice, group g holding the tokens t_e = s0 + g * 4 TT + e * TT + tid,
// e < 4 (each of the four loads of a group is one coalesced 256-token read per wave). The loop over the groups stays
// rolled (it is the kernel's hot code) and its loads run QD groups ahead. The loads go through buffer resources: no
// branch around a load (a load in a branch is waited for where the branch joins), and a token past the row reads 0.
constexpr int NG = TS / (4 * TT);  // groups per thread per slice
constexpr int Q_NONE = 3;          // q loader kind of a node whose kids are all one-hot (GSE_Q_* otherwise)

__device__ const uint32_t ALL_ALLOWED = 0xFFFFFFFFu;  // the mask word of a row without a mask

struct TBuf {                    // a target row's logits and mask words
  __amdgpu_buffer_rsrc_t x, m;
  int mstep;                     // bytes per 32 tokens in m: 4, or 0 (the one word ALL_ALLOWED)
};
__device__ __forceinline__ TBuf tbuf(const RowCtx &c) {
  constexpr int FMT = 0x00020000;  // raw 32-bit buffer (GFX9 resource word 3)
  TBuf b;
  b.x = __builtin_amdgcn_make_buffer_rsrc((void *)c.base, (short)0, c.V * (c.dtype == GSE_BF16 ? 2 : 4), FMT);
  b.m = __builtin_amdgcn_make_buffer_rsrc(c.mw ? (void *)c.mw : (void *)&ALL_ALLOWED, (short)0,
                                          c.mw ? (c.V + 31) / 32 * 4 : 4, FMT);
  b.mstep = c.mw ? 4 : 0;
  return b;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qbuf(const QRow &q, int V) {
  const int es = q.kind == GSE_Q_PROB ? 8 : q.kind == GSE_Q_LOGITS_BF16 ? 2 : 4;
  return __builtin_amdgcn_make_buffer_rsrc((void *)q.base, (short)0, V * es, 0x00020000);
}

template <int DT>
__device__ __forceinline__ float ld_x(const TBuf &b, int t) {
  if constexpr (DT == GSE_BF16) {
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(b.x, t * 2, 0, 0));
  } else {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(b.x, t * 4, 0, 0));
  }
}
__device__ __forceinline__ uint32_t ld_m(const TBuf &b, int t) {
  return __builtin_amdgcn_raw_buffer_load_b32(b.m, (t >> 5) * b.mstep, 0, 0);
}
// A q value as loaded: a probability (fp64), or a logit (f32, exact for bf16 too); widened by the caller.
template <int QL>
using QRaw = typename std::conditional<QL == GSE_Q_PROB, double, float>::type;
template <int QL>
__device__ __forceinline__ QRaw<QL> ld_q(__amdgpu_buffer_rsrc_t q, int t) {
  if constexpr (QL == GSE_Q_PROB) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(q, t * 8, 0, 0);
    return __longlong_as_double((long long)(((uint64_t)v[1] << 32) | v[0]));
  } else if constexpr (QL == GSE_Q_LOGITS_BF16) {
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(q, t * 2, 0, 0));
  } else if constexpr (QL == GSE_Q_LOGITS_F32) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(q, t * 4, 0, 0));
  } else {
    return 0.0f;
  }
}

template <int DT, int QL>
struct Grp {  // one group's loads: target logits and mask words, and q values (QL != Q_NONE)
  float x[4];
  uint32_t mw[4];
  QRaw<QL> q[QL == Q_NONE ? 1 : 4];
};
template <int DT, int QL>
__device__ __forceinline__ Grp<DT, QL> ld_grp(const TBuf &b, __amdgpu_buffer_rsrc_t qb, int t0) {
  Grp<DT, QL> r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = t0 + e * TT;
    r.x[e] = ld_x<DT>(b, t);
    r.mw[e] = ld_m(b, t);
    if constexpr (QL != Q_NONE) r.q[e] = ld_q<QL>(qb, t);
  }
  return r;
}
// q values only (the q rows' statistics)
template <int QL>
struct QGrp {
  QRaw<QL> q[4];
};
template <int QL>
__device__ __forceinline__ QGrp<QL> ld_qgrp(__amdgpu_buffer_rsrc_t qb, int t0) {
  QGrp<QL> r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r.q[e] = ld_q<QL>(qb, t0 + e * TT);
  return r;
}

// f(t0, group) for the thread's groups of slice s0 (token t0 + e TT is element e). RING groups are in registers: the
// loop is unrolled by RING so that each one is reloaded in place after its use (a copy of a register whose load is
// still in flight would wait for the load), so every group is loaded RING - 1 groups ahead of its use. Four suits the
// kernels that keep four waves per SIMD; two frees the registers a heavier per-token body needs for a third wave.
template <int RING = 4, typename Ld, typename F>
__device__ __forceinline__ void slice_groups(int s0, Ld ld, F f) {
  static_assert(NG % 4 == 0 && (RING == 2 || RING == 4), "");
  const int tid = threadIdx.x;
  auto t0_of = [&](int g) { return s0 + min(g, NG - 1) * 4 * TT + tid; };  // (past the end: the last group again)
  if constexpr (RING == 2) {
    auto b0 = ld(t0_of(0));
    __builtin_amdgcn_sched_barrier(0);
    auto b1 = ld(t0_of(1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
    for (int g = 0; g < NG; g += 2) {
      f(t0_of(g), b0);
      __builtin_amdgcn_sched_barrier(0);
      b0 = ld(t0_of(g + 2));
      __builtin_amdgcn_sched_barrier(0);
      f(t0_of(g + 1), b1);
      __builtin_amdgcn_sched_barrier(0);
      b1 = ld(t0_of(g + 3));
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  }
  // (the groups' loads go out in the loop's order before it too, and no step's code moves across another's loads: a
  // loop entered with its loads issued in another order waited for all of them in every round)
  auto b0 = ld(t0_of(0));
  __builtin_amdgcn_sched_barrier(0);
  auto b1 = ld(t0_of(1));
  __builtin_amdgcn_sched_barrier(0);
  auto b2 = ld(t0_of(2));
  __builtin_amdgcn_sched_barrier(0);
  auto b3 = ld(t0_of(3));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
  for (int g = 0; g < NG; g += 4) {
    f(t0_of(g), b0);
    __builtin_amdgcn_sched_barrier(0);
    b0 = ld(t0_of(g + 4));
    __builtin_amdgcn_sched_barrier(0);
    f(t0_of(g + 1), b1);
    __builtin_amdgcn_sched_barrier(0);
    b1 = ld(t0_of(g + 5));
    __builtin_amdgcn_sched_barrier(0);
    f(t0_of(g + 2), b2);
    __builtin_amdgcn_sched_barrier(0);
    b2 = ld(t0_of(g + 6));
    __builtin_amdgcn_sched_barrier(0);
    f(t0_of(g + 3), b3);
    __builtin_amdgcn_sched_barrier(0);
    b3 = ld(t0_of(g + 7));
    __builtin_amdgcn_sched_barrier(0);
  }
}

// tgt_w with the division chosen at run time (one uniform test per token).
__device__ __forceinline__ double tgt_wr(const Tgt &g, int t, float x, uint32_t mword, uint32_t cnt,
                                         const double *etab) {
  if (cnt) x = penalize(x, cnt, g.c.rp, g.c.fp, g.c.pp);
  float z = x;
  if (g.c.divide) z = div_rn(x, g.c.T, g.c.Td, g.c.Rd);
  if (!((mword >> (t & 31)) & 1u) || !(z > -INFINITY)) return 0.0;
  if (g.kkeep && pack(fkey(z), (uint32_t)t) < g.kkeep) return 0.0;
  return exp_nonpos((double)z - g.M, etab);
}

// A node's q variant: 0 no q row (every kid one-hot), 1 probabilities, 2 / 3 f32 logits with t == 1 / another t,
// 4 / 5 bf16 logits likewise; its loader kind and its q_w kind.
template <int QKK, typename F>
__device__ __forceinline__ void with_qv(bool has_q, bool t1, F f) {
  if (!has_q) {
    f(IntC<0>{});
  } else if constexpr (QKK == GSE_Q_PROB) {
    f(IntC<1>{});
  } else if constexpr (QKK == GSE_Q_LOGITS_F32) {
    if (t1) f(IntC<2>{});
    else f(IntC<3>{});
  } else if constexpr (QKK == GSE_Q_LOGITS_BF16) {
    if (t1) f(IntC<4>{});
    else f(IntC<5>{});
  } else {
    f(IntC<0>{});
  }
}
constexpr int ql_of(int qv) {
  return qv == 0 ? Q_NONE : qv == 1 ? (int)GSE_Q_PROB : qv <= 3 ? (int)GSE_Q_LOGITS_F32 : (int)GSE_Q_LOGITS_BF16;
}
constexpr int qk_of(int qv) { return qv == 0 ? 3 : qv == 1 ? 0 : (qv == 2 || qv == 4) ? 1 : 2; }

// The streaming kernels are compiled per logits type DTK and per q kind QKK of the call (GSE_Q_*, or Q_NONE when
// the call has no q rows): launch_tree picks the instance.

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
  double etab[64];             // 2^(k/64), the table of exp_nonpos
  int redi[8];
  uint32_t redu[8];
  uint32_t ticket;
  int found;
};

__device__ __forceinline__ void load_etab(TreeShared &sh) {
  if (threadIdx.x < 64) sh.etab[threadIdx.x] = EXP2_64[threadIdx.x];
}

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
  uint64_t *tseg;          // [nodes][nsl][2 TSEG]: segment sums {hi, lo} of the residual the node draws from
  uint32_t *plist;         // [GSE_MAX_KIDS + 1][nodes]: the nodes residual pass r takes (appended by the kernel before it)
  uint32_t *pcnt;          // [GSE_MAX_KIDS + 1]: their counts (cleared by the statistics pass)
  double *qmax;            // [qrows][nsl] slice maxima of z
  Fx *qpart;               // [qrows][nsl] slice masses exp(z - slice maximum)
  QFin *qfin;              // [qrows]
  gse_tree_out out;
};

// Node u takes residual pass r (thread 0 of its workgroup).
__device__ __forceinline__ void pass_add(const TreeArgs &a, int r, int u) {
  const uint32_t k = __hip_atomic_fetch_add(&a.pcnt[r], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  a.plist[(size_t)r * a.nodes + k] = (uint32_t)u;  // (a node enters each list once: k < nodes)
}

// Kids of node u found by one wave: lanes read 64 rows after u at a time, the kids (parent u) before the first row of
// another request (parent -1) are appended in row order by lane 0 of the wave.
__device__ __forceinline__ void find_kids(const TreeArgs &a, int u, Kids &k) {
  const int ln = lane_id();
  if (ln == 0) {
    k.n = 0;
    k.nq = 0;
    k.over = false;
  }
  for (int base = u + 1; base < a.nodes; base += WAVE) {
    const int j = base + ln;
    const int pj = j < a.nodes ? a.parent[j] : -1;
    const bool kid = pj == u;
    const int tok = kid ? a.token[j] : 0;
    const int qr = kid && a.qrow ? a.qrow[j] : -1;
    const uint64_t endm = ballot64(pj < 0);
    const uint64_t before_end = endm ? (endm & (0ull - endm)) - 1ull : ~0ull;
    uint64_t km = ballot64(kid) & before_end;
    while (km) {  // (uniform: every lane follows, lane 0 writes)
      const int l = __builtin_ctzll(km);
      km &= km - 1ull;
      const int tk = __shfl(tok, l, WAVE), q = __shfl(qr, l, WAVE);
      if (ln == 0) {
        if (k.n >= a.max_kids || k.n >= GSE_MAX_KIDS) {
          k.over = true;
        } else {
          int qs = -1;
          if (q >= 0 && q < (int)a.q.rows) {
            for (int m = 0; m < k.nq; ++m)
              if (k.qrow[m] == q) qs = m;
            if (qs < 0) {
              qs = k.nq++;
              k.qrow[qs] = q;
            }
          }
          k.row[k.n] = base + l;
          k.tok[k.n] = tk;
          k.qs[k.n] = qs;
          ++k.n;
        }
      }
    }
    if (endm) break;
  }
}

__device__ __forceinline__ const char *qbase(const TreeArgs &a, int qr) {
  const size_t es = a.q.kind == GSE_Q_PROB ? 8 : a.q.kind == GSE_Q_LOGITS_BF16 ? 2 : 4;
  return (const char *)a.q.q + (size_t)qr * (size_t)a.q.ld * es;
}

__device__ __forceinline__ QRow qrow_of(const TreeArgs &a, int qr) {
  QRow q;
  q.kind = (int)a.q.kind;
  q.base = qbase(a, qr);
  q.t = a.q.kind == GSE_Q_PROB ? 1.0 : a.q.temperature[qr];
  q.t1 = q.t == 1.0;
  q.M = a.qfin[qr].M;
  q.invE = 1.0 / a.qfin[qr].E;
  return q;
}

// The chain of residuals at one token (spec.py:95-102): p_0 = p0; res_{r+1} = max(p_r - q_r, 0) (one-hot kid: p_r with
// the kid's token set to 0); p_{r+1} = res_{r+1} / sig[r + 1] (a product by isig[r + 1] = 1 / sig[r + 1]), or p_r when
// that total is 0. Returns res_d (norm false) or p_d (norm true); d == 0 returns p0. qf(m) gives the node's distinct q
// row m at the token (called once per run of kids that share it, as SpecInfer's kids do).
template <typename QF>
__device__ __forceinline__ double chain(const Kids &k, QF qf, double p0, int i, const double *sig, const double *isig,
                                        int d, bool norm) {
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
        qv = qf(qid);
      }
      res = fmax(p - qv, 0.0);
    }
    const double pn = sig[r + 1] > 0.0 ? res * isig[r + 1] : p;
    if (r == d - 1) return norm ? pn : res;
    p = pn;
  }
  return p;
}

// The first two chain levels in registers, for nodes whose kids share at most one q row (the usual tree): chain_r<D>
// gives chain(...) for d = D <= 2 with qv the shared row's value at the token, in the same operations.
struct ChainR {
  int qs[2], tok[2];
  double sig[3], isig[3];
};
template <int D>
__device__ __forceinline__ double chain_r(const ChainR &c, double qv, double p0, int i, bool norm) {
  static_assert(D >= 1 && D <= 2, "");
  double p = p0;
#pragma unroll
  for (int r = 0; r < D; ++r) {
    const double res = c.qs[r] < 0 ? (i == c.tok[r] ? 0.0 : p) : fmax(p - qv, 0.0);
    const double pn = c.sig[r + 1] > 0.0 ? res * c.isig[r + 1] : p;
    if (r == D - 1) return norm ? pn : res;
    p = pn;
  }
  return p;
}

// A node's uniform data for one workgroup, in LDS: its kids, their q rows, the residual totals and their inverses.
struct NodeShared {
  Kids k;
  QRow qr[GSE_MAX_KIDS];
  double sig[GSE_MAX_KIDS + 1];
  double isig[GSE_MAX_KIDS + 1];
  double clast, iclast;
};

// chain_r for a chain depth d of 1 or 2 known at run time.
__device__ __forceinline__ double chain_rd(const ChainR &c, double qv, double p0, int i, int d, bool norm) {
  const double res1 = c.qs[0] < 0 ? (i == c.tok[0] ? 0.0 : p0) : fmax(p0 - qv, 0.0);
  const double p1 = c.sig[1] > 0.0 ? res1 * c.isig[1] : p0;
  if (d == 1) return norm ? p1 : res1;
  const double res2 = c.qs[1] < 0 ? (i == c.tok[1] ? 0.0 : p1) : fmax(p1 - qv, 0.0);
  const double p2 = c.sig[2] > 0.0 ? res2 * c.isig[2] : p1;
  return norm ? p2 : res2;
}

__device__ __forceinline__ ChainR chain_regs(const NodeShared &ns) {
  ChainR c;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    c.qs[r] = r < ns.k.n ? ns.k.qs[r] : -1;
    c.tok[r] = r < ns.k.n ? ns.k.tok[r] : -1;
  }
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    c.sig[r] = ns.sig[r];
    c.isig[r] = ns.isig[r];
  }
  return c;
}

// The node's p0 at one token (every thread calls; all get it).
__device__ __forceinline__ double p0_at(const TreeArgs &a, const Tgt &g, int x, const NodeShared &ns,
                                        TreeShared &sh) {
  const uint32_t cnt = hist_count(g.c, a.s.hist, x, sh.redu);
  return tgt_e_at(g, x, cnt, sh.etab) * ns.iclast;
}

// The 64-token segment sums of slice [s0, s1) into sh.seg (see slice_find).
template <typename LD, typename EV>
__device__ __forceinline__ void slice_segs(int s0, int s1, LD ld, EV ev, TreeShared &sh) {
  constexpr int NS = TSEG / (TT / WAVE);  // segments per wave
  const int tid = threadIdx.x;
  const int wv = tid >> 6, ln = lane_id();
  auto tok = [&](int j) { return s0 + (j * (TT / WAVE) + wv) * WAVE + ln; };  // this lane's token of segment j
  auto load = [&](int j) {
    const int i = tok(j);
    return ld(i < s1 ? i : s0);
  };
  auto seg = [&](int j, const auto &r) {
    const int i = tok(j), g = j * (TT / WAVE) + wv;
    const Fx f = fx_of(i < s1 ? ev(i, r) : 0.0);
    const uint64_t hi = wave_sum_u64(f.hi), lo = wave_sum_u64(f.lo);
    if (ln == 0) {
      sh.seg[2 * g] = hi;
      sh.seg[2 * g + 1] = lo;
    }
  };
  // four segments in registers, each reloaded in place after its use (see slice_groups)
  auto r0 = load(0);
  auto r1 = load(1);
  auto r2 = load(2);
  auto r3 = load(3);
#pragma unroll 1
  for (int j = 0; j < NS; j += 4) {
    seg(j, r0);
    r0 = load(min(j + 4, NS - 1));
    seg(j + 1, r1);
    r1 = load(min(j + 5, NS - 1));
    seg(j + 2, r2);
    r2 = load(min(j + 6, NS - 1));
    seg(j + 3, r3);
    r3 = load(min(j + 7, NS - 1));
  }
}

// The first index of slice [s0, s1) whose inclusive prefix of the weights (after `before`, the exact mass of the
// slices ahead) reaches thr; -1 if none. The weight of token i is ev(i, ld(i)): ld does the loads, which run three
// segments ahead of the weights. Exact fixed-point prefixes: 64-token segment sums (wave w takes segments w, w + 4,
// ...), the crossing segment, then its weights again and their scan. pre: the slice's segment sums when a pass kept
// them ({hi, lo} per segment), else null. Every thread gets the result.
template <typename LD, typename EV>
__device__ __forceinline__ int slice_find(int s0, int s1, Fx before, double thr, LD ld, EV ev, TreeShared &sh,
                                          const uint64_t *pre = nullptr) {
  constexpr int NS = TSEG / (TT / WAVE);  // segments per wave
  static_assert(NS % 4 == 0 && 2 * TSEG == TT, "");
  const int tid = threadIdx.x;
  const int wv = tid >> 6, ln = lane_id();
  if (pre) {
    sh.seg[tid] = ld_ag(&pre[tid]);
  } else {
    slice_segs(s0, s1, ld, ev, sh);
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
      const Fx f = fx_of(i < s1 ? ev(i, ld(i)) : 0.0);
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

// Per MSS node: the exact kept mass per slice (the last slice forms C). Per logits q row: the slice maximum m of z and
// the slice mass exp(z - m) (the last slice forms M = max m and E = sum over slices of mass * exp(m - M), in slice
// order: within a few ulp of the sum of exp(z - M) over the row). Row y = blockIdx.y: node y, or q row y - nodes.
template <int DTK, int QKK>
__global__ __launch_bounds__(TT) void tstats_kernel(TreeArgs a) {
  __shared__ TreeShared sh;
  const int s = blockIdx.x, y = (int)blockIdx.y, tid = threadIdx.x;
  if (s == 0 && y == 0 && tid <= GSE_MAX_KIDS) a.pcnt[tid] = 0u;  // (the residual passes' lists of this call)
  const int V = a.s.V, s0 = s * TS, s1 = min(V, s0 + TS);
  if (y < a.nodes) {
    const int u = y;
    const gse_row P = a.s.params[u];
    const uint32_t inf = a.s.info[u].flags;  // (node_live in place: one round of loads, as in tkid0_kernel)
    const Tgt g = tgt_of(a, u, P);
    if (!(P.flags & GSE_ROW_MSS) || !(inf & R_DONE) || (inf & (R_SPECIAL | R_BAD | R_GREEDY))) return;
    load_etab(sh);
    if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);  // (its barriers publish the table)
    else __syncthreads();
    const TBuf tb = tbuf(g.c);
    const uint32_t *cnt = g.c.pen ? sh.cnt : nullptr;
    Fx f = fx_zero();
    int last = -1;
    {
      with_div(g.c.divide, [&](auto dv) {
        constexpr int DT = DTK;
        constexpr bool DIV = decltype(dv)::value;
        slice_groups(s0, [&](int t0) { return ld_grp<DT, Q_NONE>(tb, tb.x, t0); },
                     [&](int t0, const Grp<DT, Q_NONE> &gr) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = t0 + e * TT;
            if (i < s1) {
              const double w = tgt_w<DIV>(g, i, gr.x[e], gr.mw[e], cnt ? cnt[i - s0] : 0u, sh.etab);
              f = fx_add(f, fx_of(w));
              if (w > 0.0) last = i;
            }
          }
        });
      });
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
    if (tid < WAVE) {
      const Fx *pp = a.npart + (o - s);
      const Fx t = wave_fx_total(a.nsl, [&](int j) { return Fx{ld_ag(&pp[j].hi), ld_ag(&pp[j].lo)}; });
      if (tid == 0) {
        TreeNode &nd = a.st[u];
        nd.clast = fx_val(t);
        nd.sig[0] = nd.clast;
        nd.next = 1;
        nd.token = -1;
        nd.kid = -1;
        nd.ticket = 0;
      }
    }
    return;
  }
  const int qr = y - a.nodes;
  if (a.q.kind == GSE_Q_PROB) return;
  QRow q;
  q.kind = (int)a.q.kind;
  q.base = qbase(a, qr);
  q.t = a.q.temperature[qr];
  q.t1 = q.t == 1.0;
  const auto qb = qbuf(q, V);
  // the slice maximum first (z = x / t is monotone in x for t > 0 and rounds once: the maximum of z is the maximum of x
  // divided once), then the masses (a second read of the slice, from the cache)
  double xm = -INFINITY;
  Fx f = fx_zero();
  load_etab(sh);
  {
    constexpr int QL = QKK;
    if constexpr (QL == GSE_Q_LOGITS_F32 || QL == GSE_Q_LOGITS_BF16) {
      slice_groups(s0, [&](int t0) { return ld_qgrp<QL>(qb, t0); }, [&](int t0, const QGrp<QL> &gr) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t0 + e * TT < s1) xm = fmax(xm, (double)gr.q[e]);
      });
      const double xmax = block_max_f64(xm, sh.redd);  // (its barriers publish the table)
      const double m = q.t1 ? xmax : xmax / q.t;
      xm = m;
      if (m > -INFINITY) {
        with_bool(q.t1, [&](auto t1c) {
          constexpr bool T1 = decltype(t1c)::value;
          slice_groups(s0, [&](int t0) { return ld_qgrp<QL>(qb, t0); }, [&](int t0, const QGrp<QL> &gr) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (t0 + e * TT < s1) {
                const double z = T1 ? (double)gr.q[e] : (double)gr.q[e] / q.t;
                f = fx_add(f, fx_of(exp_nonpos(z - m, sh.etab)));
              }
            }
          });
        });
      }
    }
  }
  const double m = xm;
  f = block_fx_sum(f, sh.red);
  const size_t o = (size_t)qr * a.nsl + s;
  if (tid == 0) {
    st_ag(&a.qmax[o], m);
    st_ag(&a.qpart[o].hi, f.hi);
    st_ag(&a.qpart[o].lo, f.lo);
  }
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&a.qfin[qr].ticket);
  __syncthreads();
  if (sh.ticket != (uint32_t)(a.nsl - 1)) return;
  if (tid < WAVE) {
    // M = max of the slice maxima; E = sum of mass_j exp(m_j - M), each lane its slices, then a wave sum in a fixed
    // order (the same E every call)
    const double *mq = a.qmax + (o - s);
    const Fx *pq = a.qpart + (o - s);
    double M = -INFINITY;
    for (int j = tid; j < a.nsl; j += WAVE) M = fmax(M, ld_ag(&mq[j]));
    M = wave_max_f64(M);
    double E = 0.0;
    for (int j = tid; j < a.nsl; j += WAVE) {
      const double mj = ld_ag(&mq[j]);
      if (mj > -INFINITY) E += fx_val(Fx{ld_ag(&pq[j].hi), ld_ag(&pq[j].lo)}) * exp_nonpos(mj - M, sh.etab);
    }
    E = wave_sum_f64(E);
    if (tid == 0) {
      a.qfin[qr].M = M;
      a.qfin[qr].E = E;
      a.qfin[qr].ticket = 0;
    }
  }
}

// ---- verify: residual passes ----------------------------------------------------------------------------------------

// The node's kids, q rows and totals into LDS, by wave 0 (every load of a round issued at once).
__device__ __forceinline__ void load_node(const TreeArgs &a, int u, NodeShared &ns) {
  if (threadIdx.x < WAVE) {
    const int ln = lane_id();
    const TreeNode &nd = a.st[u];
    if (ln <= GSE_MAX_KIDS) {
      const double sg = nd.sig[ln];
      ns.sig[ln] = sg;
      ns.isig[ln] = 1.0 / sg;
    }
    if (ln == 0) {
      ns.clast = nd.clast;
      ns.iclast = 1.0 / nd.clast;
    }
    find_kids(a, u, ns.k);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // (lane 0's LDS writes, then every lane reads them)
    if (ln < ns.k.nq) ns.qr[ln] = qrow_of(a, ns.k.qrow[ln]);
  }
  __syncthreads();
}

// The node's draw after its last kid was rejected (run by one workgroup): from p_d, d the deepest chain level with a
// positive total (sig[0] = C > 0 for a live node), in vocabulary order (sampling.py:100-104), with the uniform
// uniform(mix(seed, 2^41), i) (spec.py:103). The unnormalised weights (keep e for d = 0, res_d otherwise) give the same
// count(c < u c[-1]) as the normalised p_d.
template <int DTK, int QKK>
__device__ __forceinline__ int node_draw(const TreeArgs &a, int u, const gse_row &P, const Tgt &g, const NodeShared &ns,
                                         int kdone, TreeShared &sh, bool segs_kept = false) {
  int d = kdone;
  while (d > 0 && !(ns.sig[d] > 0.0)) --d;
  const size_t o = ((size_t)u * (GSE_MAX_KIDS + 1) + d) * a.nsl;
  const Fx *pp = a.npart + o;
  auto part = [&](int j) { return Fx{ld_ag(&pp[j].hi), ld_ag(&pp[j].lo)}; };
  const uint64_t *pre_all = segs_kept && d == kdone ? a.tseg + (size_t)u * a.nsl * 2 * TSEG : nullptr;
  const Fx tot = wave_fx_total(a.nsl, part);  // (every wave reads the partials itself)
  int lastl = -1;
  for (int j = lane_id(); j < a.nsl; j += WAVE) lastl = max(lastl, ld_ag(&a.nlast[o + j]));
  const int last = (int)wave_max_u32((uint32_t)(lastl + 1)) - 1;
  if (last < 0) return -1;
  const double thr = uniform64(mix64(P.seed, SALT_RES), P.idx) * fx_val(tot);
  Fx before;  // the crossing slice and the exact mass ahead of it
  const int sx = wave_fx_cross(a.nsl, thr, part, before);
  const int s0 = sx * TS, s1 = min(a.s.V, s0 + TS);
  if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);
  const TBuf tb = tbuf(g.c);
  const uint32_t *cnt = g.c.pen ? sh.cnt : nullptr;
  int j = -1;
  {
    constexpr int DT = DTK;
    if (ns.k.nq <= 1 && d <= 2) {
      const ChainR cr = chain_regs(ns);
      const QRow q = ns.qr[0];
      const auto qb = qbuf(q, a.s.V);
      const double iclast = ns.iclast;
      with_qv<QKK>(ns.k.nq > 0 && d > 0, q.t1, [&](auto qvc) {
        constexpr int QL = ql_of(decltype(qvc)::value), QK = qk_of(decltype(qvc)::value);
        struct El {
          float x;
          uint32_t mw;
          QRaw<QL> q;
        };
        j = slice_find(s0, s1, before, thr, [&](int i) {
          return El{ld_x<DT>(tb, i), ld_m(tb, i), ld_q<QL>(qb, i)};
        }, [&](int i, const El &w) {
          const double e = tgt_wr(g, i, w.x, w.mw, cnt ? cnt[i - s0] : 0u, sh.etab);
          if (d == 0) return e;
          double qx = 0.0;
          if constexpr (QL != Q_NONE) qx = q_w<QK>(q, w.q, sh.etab);
          return chain_rd(cr, qx, e * iclast, i, d, false);
        }, sh, pre_all ? pre_all + (size_t)sx * 2 * TSEG : nullptr);
      });
    } else {
      j = slice_find(s0, s1, before, thr, [&](int i) { return ld_x<DT>(tb, i); }, [&](int i, float x) {
        const double e = tgt_wr(g, i, x, ld_m(tb, i), cnt ? cnt[i - s0] : 0u, sh.etab);
        if (d == 0) return e;
        return chain(ns.k, [&](int m) { return q_at(ns.qr[m], i, sh.etab); }, e * ns.iclast, i, ns.sig, ns.isig, d,
                     false);
      }, sh);
    }
  }
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
  const double p0 = p0_at(a, g, x, ns, sh);
  const double px = chain(ns.k, [&](int m) { return q_at(ns.qr[m], x, sh.etab); }, p0, x, ns.sig, ns.isig, r, true);
  const double qx = ns.k.qs[r] < 0 ? 1.0 : q_at(ns.qr[ns.k.qs[r]], x, sh.etab);
  return kid_accepts(P, r, px, qx);
}

// Kid 0 of every live node with kids (spec.py:93-94 against p0), one workgroup per node, between the statistics and
// pass 1: an accepted node is decided here and pass 1 skips it.
__global__ __launch_bounds__(TT) void tkid0_kernel(TreeArgs a) {
  __shared__ TreeShared sh;
  __shared__ NodeShared ns;
  const int u = blockIdx.x;
  const gse_row P = a.s.params[u];
  TreeNode &nd = a.st[u];
  // the row's flags, its state and its target fields in one round of loads (a load behind a branch waits for the
  // branch's own): node_live in place
  const uint32_t inf = a.s.info[u].flags;
  const int next = (int)nd.next;
  const Tgt g = tgt_of(a, u, P);
  if (!(P.flags & GSE_ROW_MSS) || !(inf & R_DONE) || (inf & (R_SPECIAL | R_BAD | R_GREEDY)) || next != 1) return;
  load_etab(sh);
  load_node(a, u, ns);  // (its barrier publishes the table)
  if (ns.k.n == 0) {  // (no kids: pass 1 draws)
    if (threadIdx.x == 0) pass_add(a, 1, u);
    return;
  }
  const bool acc = test_kid(a, P, g, ns, 0, sh);
  if (threadIdx.x == 0) {
    if (acc) {
      nd.token = ns.k.tok[0];
      nd.kid = ns.k.row[0];
      nd.next = 0;
    } else {
      pass_add(a, 1, u);
    }
  }
}

// Pass r over slice s of node u (see the file comment).
template <int DTK, int QKK>
__device__ __forceinline__ void tpass_item(const TreeArgs &a, int r, int u, int s, TreeShared &sh, NodeShared &ns) {
  const int tid = threadIdx.x;
  const gse_row P = a.s.params[u];
  TreeNode &nd = a.st[u];
  const uint32_t inf = a.s.info[u].flags;  // (node_live in place: one round of loads, as in tkid0_kernel)
  const int next = (int)nd.next;
  const Tgt g = tgt_of(a, u, P);
  if (!(P.flags & GSE_ROW_MSS) || !(inf & R_DONE) || (inf & (R_SPECIAL | R_BAD | R_GREEDY)) || next != r) return;
  const int V = a.s.V, s0 = s * TS, s1 = min(V, s0 + TS);
  load_etab(sh);
  load_node(a, u, ns);  // (its barrier publishes the table)
  if (r == 1) {
    if (ns.k.n == 0) {  // no kids: mss returns draw(p0, uniform(mix(seed, 2^41), i)) (spec.py:103)
      if (s == 0) {
        const int j = node_draw<DTK, QKK>(a, u, P, g, ns, 0, sh);
        if (tid == 0) {
          nd.token = j;
          nd.kid = -1;
          nd.next = 0;
        }
      }
      return;
    }
    // (kid 0 was tested and rejected by tkid0_kernel)
  }
  // res_r over this slice: kid r - 1 was rejected
  if (g.c.pen) build_counts(g.c, a.s.hist, s0, sh.cnt);
  Fx f = fx_zero();
  int last = -1;
  const TBuf tb = tbuf(g.c);
  const uint32_t *cnt = g.c.pen ? sh.cnt : nullptr;
  const bool keep_seg = ns.k.nq <= 1 && r <= 2 && r == ns.k.n;
  {
    constexpr int DT = DTK;
    if (ns.k.nq <= 1 && r <= 2) {
      // the usual tree (kids sharing at most one q row, a chain of one or two levels): the chain in registers, the q
      // row streaming with the logits
      const ChainR cr = chain_regs(ns);
      const QRow q = ns.qr[0];
      const auto qb = qbuf(q, V);
      const double iclast = ns.iclast;
      // the pass after which the node draws (its last kid was rejected) keeps its 64-token segment sums for the draw
      uint64_t *sg = keep_seg ? a.tseg + ((size_t)u * a.nsl + s) * 2 * TSEG : nullptr;
      const int wv = tid >> 6;
      with_qv<QKK>(ns.k.nq > 0, q.t1, [&](auto qvc) {
        constexpr int QL = ql_of(decltype(qvc)::value), QK = qk_of(decltype(qvc)::value);
        slice_groups<2>(s0, [&](int t0) { return ld_grp<DT, QL>(tb, qb, t0); }, [&](int t0, const Grp<DT, QL> &gr) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = t0 + e * TT;
            Fx fe = fx_zero();
            if (i < s1) {
              const double w = tgt_wr(g, i, gr.x[e], gr.mw[e], cnt ? cnt[i - s0] : 0u, sh.etab);
              double qx = 0.0;
              if constexpr (QL != Q_NONE) qx = q_w<QK>(q, gr.q[e], sh.etab);
              const double res = chain_rd(cr, qx, w * iclast, i, r, false);
              fe = fx_of(res);
              f = fx_add(f, fe);
              if (res > 0.0) last = i;
            }
            if (sg) {  // (the wave's 64 tokens of this element form segment ((t0 - s0 - tid) / 4 TT) 16 + 4 e + wave)
              const uint64_t hi = wave_sum_u64(fe.hi), lo = wave_sum_u64(fe.lo);
              const int k = ((t0 - s0 - tid) >> 10) * 16 + 4 * e + wv;
              if (lane_id() == 0) {
                st_ag(&sg[2 * k], hi);
                st_ag(&sg[2 * k + 1], lo);
              }
            }
          }
        });
      });
    } else {
      // deeper chains or kids with several q rows: the q values read token by token
      slice_groups<2>(s0, [&](int t0) { return ld_grp<DT, Q_NONE>(tb, tb.x, t0); },
                      [&](int t0, const Grp<DT, Q_NONE> &gr) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = t0 + e * TT;
          if (i < s1) {
            const double w = tgt_wr(g, i, gr.x[e], gr.mw[e], cnt ? cnt[i - s0] : 0u, sh.etab);
            const double res = chain(ns.k, [&](int m) { return q_at(ns.qr[m], i, sh.etab); }, w * ns.iclast, i,
                                     ns.sig, ns.isig, r, false);
            f = fx_add(f, fx_of(res));
            if (res > 0.0) last = i;
          }
        }
      });
    }
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
  if (tid < WAVE) {
    const Fx *pp = a.npart + (o - s);
    const Fx t = wave_fx_total(a.nsl, [&](int j) { return Fx{ld_ag(&pp[j].hi), ld_ag(&pp[j].lo)}; });
    if (tid == 0) {
      ns.sig[r] = fx_val(t);
      ns.isig[r] = 1.0 / ns.sig[r];
      nd.sig[r] = ns.sig[r];
      nd.ticket = 0;
    }
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
        pass_add(a, r + 1, u);
      }
    }
    return;
  }
  const int j = node_draw<DTK, QKK>(a, u, P, g, ns, r, sh, keep_seg);
  if (tid == 0) {
    nd.token = j;
    nd.kid = -1;
    nd.next = 0;
  }
}

// Residual pass r: the (node, slice) items of the nodes listed for it, over a grid of at most one resident round (a
// grid over every node and slice spent most of its time dispatching workgroups of nodes the pass does not take). Three
// waves per SIMD where the f32 target's body fits them without spilling (the pass's items then take one round more
// often).
template <int DTK, int QKK>
__global__ __launch_bounds__(TT) __attribute__((amdgpu_waves_per_eu(DTK == GSE_F32 ? 3 : 2, 8))) void tpass_kernel(
    TreeArgs a, int r) {
  __shared__ TreeShared sh;
  __shared__ NodeShared ns;
  const int items = (int)a.pcnt[r] * a.nsl;  // (written by the kernels before this one)
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int u = (int)a.plist[(size_t)r * a.nodes + it / a.nsl];
    __syncthreads();  // (LDS of the previous item)
    tpass_item<DTK, QKK>(a, r, u, it % a.nsl, sh, ns);
  }
}

// ---- verify: the walk ------------------------------------------------------------------------------------------------

// One node as the walk reads it, every load issued at once with its index in range (a load behind a branch, or one
// whose address or loop bound is a loaded value, waits for what came before it: a chain of cache latencies per node):
// the row's flags, the strict decision, the sampled token and the eight rows after u (indexes clamped into rows
// [u, end); the scans stop on what they read).
struct WalkNode {
  uint32_t pf, inf;
  int stok, skid, samp;
  int p[8], t[8];
};

__device__ __forceinline__ void rows8(const TreeArgs &a, int j0, int end, int (&p)[8], int (&t)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int j = min(j0 + k, end - 1);
    p[k] = a.parent[j];
    t[k] = a.token[j];
  }
}

__device__ __forceinline__ WalkNode walk_node(const TreeArgs &a, int u, int end) {
  WalkNode w;
  w.pf = a.s.params[u].flags;
  w.inf = a.s.info[u].flags;
  w.stok = a.st[u].token;
  w.skid = a.st[u].kid;
  w.samp = a.sampled[u];
  rows8(a, u + 1, end, w.p, w.t);
  return w;
}

// node_live from the loaded flags
__device__ __forceinline__ bool walk_live(const WalkNode &w) {
  return (w.pf & GSE_ROW_MSS) && (w.inf & R_DONE) && !(w.inf & (R_SPECIAL | R_BAD | R_GREEDY));
}

// More kids than the round was given room for (max_kids, GSE_MAX_KIDS): find_kids dropped the later ones, so a strict
// node's decision would not be the reference's (spec.py:91 walks every kid). The kids are the rows after u with parent
// u, before the first root (parent < 0) or end.
__device__ __forceinline__ bool kids_over(const TreeArgs &a, int u, int end, WalkNode w) {
  int n = 0;
  bool go = true;
  for (int j0 = u + 1;;) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      go = go && j0 + k < end && w.p[k] >= 0;
      n += go && w.p[k] == u ? 1 : 0;
    }
    j0 += 8;
    if (!go || j0 >= end) break;
    rows8(a, j0, end, w.p, w.t);
  }
  return n > a.max_kids || n > GSE_MAX_KIDS;
}

// The first kid of u holding tok among the rows (u, end), or -1; ROOT: a root (parent < 0) also ends the rows.
template <bool ROOT>
__device__ __forceinline__ int kid_of(const TreeArgs &a, int u, int end, int tok, WalkNode w) {
  for (int j0 = u + 1;;) {
    int kid = -1;
    bool go = true;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      go = go && j0 + k < end && (!ROOT || w.p[k] >= 0);
      if (go && kid < 0 && w.p[k] == u && w.t[k] == tok) kid = j0 + k;
    }
    j0 += 8;
    if (kid >= 0 || !go || j0 >= end) return kid;
    rows8(a, j0, end, w.p, w.t);
  }
}

__global__ __launch_bounds__(64) void walk_kernel(TreeArgs a) {
  const int q = blockIdx.x * 64 + threadIdx.x;
  // node_token / node_kid of every node
  for (int u = q; u < a.nodes && (a.out.node_token || a.out.node_kid); u += gridDim.x * 64) {
    const WalkNode w = walk_node(a, u, a.nodes);
    int tok, kid;
    if (w.pf & GSE_ROW_MSS) {
      const bool live = walk_live(w) && !kids_over(a, u, a.nodes, w);
      tok = live ? w.stok : -1;
      kid = live ? w.skid : -1;
    } else {
      tok = w.samp;
      kid = tok >= 0 ? kid_of<true>(a, u, a.nodes, tok, w) : -1;
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
    const WalkNode w = walk_node(a, u, end);
    int tok, kid = -1;
    if (w.pf & GSE_ROW_MSS) {
      if (kids_over(a, u, end, w)) {  // (the node's decision is not the reference's: the walk stops before it)
        status = GSE_WALK_KIDS;
        if (n < a.out.emit_ld) a.out.emit_nodes[(int64_t)q * a.out.emit_ld + n] = u;
        break;
      }
      const bool live = walk_live(w);
      tok = live ? w.stok : -1;
      kid = live ? w.skid : -1;
    } else {
      tok = w.samp;
      if (tok >= 0) kid = kid_of<false>(a, u, end, tok, w);
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
  for (int j = lane_id(); j < a.nsl; j += WAVE) M = fmax(M, a.pmax[(size_t)row * a.nsl + j]);
  M = wave_max_f64(M);
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
  // (every wave reads the row's partials itself, a slice per lane)
  const double *pm = a.pmax + (size_t)row * a.nsl;
  const Fx *pp = a.ppart + (size_t)row * a.nsl;
  const int32_t *pl = a.plast + (size_t)row * a.nsl;
  double M = -INFINITY;
  int lastl = -1;
  for (int j = lane_id(); j < a.nsl; j += WAVE) {
    M = fmax(M, pm[j]);
    lastl = max(lastl, pl[j]);
  }
  M = wave_max_f64(M);
  const int last = (int)wave_max_u32((uint32_t)(lastl + 1)) - 1;
  auto part = [&](int j) { return pp[j]; };
  const Fx tot = wave_fx_total(a.nsl, part);
  int tok = -1;
  double lq = __builtin_nan("");
  if (last >= 0) {
    const double E = fx_val(tot);
    const double thr = uniform64(mix64(a.b.seed[row], SALT_DRAFT + (uint64_t)kd), a.b.at[row]) * E;
    Fx before;
    const int sx = wave_fx_cross(a.nsl, thr, part, before);
    const int s0 = sx * TS, s1 = min(V, s0 + TS);
    const int j = slice_find(s0, s1, before, thr, [&](int i) { return pick_x(a, row, i); },
                             [&](int, float x) { return exp((double)x / t - M); }, sh);
    tok = j < 0 ? last : min(j, last);
    lq = ((double)pick_x(a, row, tok) / t - M) - log(E);
  }
  if (tid == 0) {
    a.b.out_tokens[(int64_t)row * a.b.out_ld + kd] = tok;
    a.b.out_logq[(int64_t)row * a.b.out_ld + kd] = lq;
  }
}

}  // namespace

namespace {

TreeArgs tree_args(const TreeLaunch &L) {
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
  a.tseg = L.tseg;
  a.plist = L.plist;
  a.pcnt = L.pcnt;
  a.qmax = L.qmax;
  a.qpart = L.qpart;
  a.qfin = L.qfin;
  a.out = L.out;
  return a;
}

// f(IntC<logits type>, IntC<q kind>) for the call's instance
template <typename F>
void by_instance(const TreeLaunch &L, F f) {
  auto by_q = [&](auto dtc) {
    if (L.q.rows == 0) f(dtc, IntC<Q_NONE>{});
    else if (L.q.kind == GSE_Q_PROB) f(dtc, IntC<GSE_Q_PROB>{});
    else if (L.q.kind == GSE_Q_LOGITS_BF16) f(dtc, IntC<GSE_Q_LOGITS_BF16>{});
    else f(dtc, IntC<GSE_Q_LOGITS_F32>{});
  };
  if (L.s.dtype == GSE_BF16) by_q(IntC<GSE_BF16>{});
  else by_q(IntC<GSE_F32>{});
}

}  // namespace

hipError_t launch_tree(const TreeLaunch &L, hipStream_t s) {
  const TreeArgs a = tree_args(L);
  // the statistics of the q rows given as drafter logits in the same launch (grid rows past the nodes)
  const int yq = L.q.rows > 0 && L.q.kind != GSE_Q_PROB ? (int)L.q.rows : 0;
  // the instances for the call's logits type and q kind
  auto go = [&](auto dtc, auto qkc) {
    constexpr int DT = decltype(dtc)::value, QK = decltype(qkc)::value;
    hipLaunchKernelGGL((tstats_kernel<DT, QK>), dim3(a.nsl, a.nodes + yq), dim3(TT), 0, s, a);
    hipLaunchKernelGGL(tkid0_kernel, dim3(a.nodes), dim3(TT), 0, s, a);
    // pass r: kid r - 1 rejected -> res_r; a node with k kids needs passes 1..k (one without kids draws in pass 1)
    // pass 1 takes most live nodes: one resident round; later passes only nodes with more kids (a quarter round,
    // workgroups take several items if there are more)
    for (int r = 1; r <= max(L.max_kids, 1); ++r) {
      const int pg = max(1, min(a.nsl * a.nodes, r == 1 ? L.pgrid : max(L.pgrid / 4, a.nsl)));
      hipLaunchKernelGGL((tpass_kernel<DT, QK>), dim3(pg), dim3(TT), 0, s, a, r);
    }
  };
  by_instance(L, go);
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
