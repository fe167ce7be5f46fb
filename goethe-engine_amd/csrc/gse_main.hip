// The fused selection pass: one 256-thread workgroup per (row, 8192-token slice) holds its slice in registers after a
// single HBM read of the logits, the packed mask words and the row's history ids; the last workgroup of each row to
// finish (atomic ticket, nothing waits) resolves the row.
//
// Reference semantics (goethe_engine/sampling.py:59-85):
//   bad   = NaN anywhere before the mask, or no finite value after it        -> token -1            (sampling.py:71-75,84)
//   T = 0 -> first argmax of nan_to_num(masked x)                            (sampling.py:76)
//   T > 0 -> z = x / float32(T); stable descending order; fp64 softmax q; keep = rank < top_k AND cumsum(q) - q < top_p
//            (AND q >= min_p * q_0); c = cumsum(q * keep); token = order[count(c < u * c[-1])]   (sampling.py:59-83)
//
// Per slice, in registers: penalties (u16 history counts in LDS), the NaN test, the mask, z = RN(x / T) computed as
// RN32(x * RN64(1 / T)) (exact, see div_exact), the slice maximum, and the softmax sum of the elements the slice does
// not list, from v_exp_f32 with a rigorous error bound. Each wave takes the 16th largest of its 64 lane maxima (to 16
// key bits) as a threshold; the slice lists (exact key, id) of every element at or above the largest of its waves'
// thresholds, so the listed set certifies the slice's top elements down to that key.
//
// Row resolve: the union of the slices' lists cut at the largest certified key is the row's certified head: exactly its
// top elements, stable order included. The resolve sorts the top ~512 of the head (the whole head when the keep prefix
// runs past them), takes exact fp64 masses of it (and of every listed element for S), and decides the keep prefix and
// the draw. Top-k, min-p and the draw do not depend on S (they compare masses with masses); top-p uses the S bounds.
// A decision inside the bound, a keep prefix that runs past the head, or an overflow marks the row hard: the exact
// path (gse_exact.hip) finishes it.
#include "gse_rowctx.h"

namespace gse {

namespace {

constexpr int MT = 256;                // threads per slice workgroup
constexpr int NWV = MT / WAVE;         // waves
constexpr int EPT = CH / MT;           // 32 elements per thread
constexpr int KW = 16;                 // lane rank of a wave's candidate threshold
constexpr int NH = 2048;               // certified head capacity of the row resolve
constexpr int NSUB = 1024;             // sorted sub-head capacity
constexpr int SUBT = 512;              // sub-head target size
constexpr int HPT = 8;                 // history ids per thread per round
constexpr int GPT = 8;                 // listed entries per thread per gather round
constexpr int MAXSL = (1 << 21) / CH;  // slices of the largest vocabulary (= MT: one record per thread)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float FLTMAX = 3.402823466e+38f;
static_assert(MAXSL <= MT, "one slice record per resolve thread");

template <int DT>
struct Lay;
template <>
struct Lay<GSE_F32> {  // thread tid, vector v, lane element k: token c0 + v * 1024 + tid * 4 + k
  static constexpr int VEC = 4, NV = EPT / 4, STRIDE = MT * 4;
};
template <>
struct Lay<GSE_BF16> {  // token c0 + v * 2048 + tid * 8 + k
  static constexpr int VEC = 8, NV = EPT / 8, STRIDE = MT * 8;
};

struct Shared {
  union {
    uint32_t cnt[CH / 2];  // history counts of the slice's tokens, two u16 per word
    struct {
      uint64_t head[NH];   // listed elements at or above the certified key
      uint64_t sub[NSUB];  // the top of the head
    } r;
  };
  float wmax[NWV];
  uint32_t wtau[NWV];
  uint32_t wflags[NWV];
  double wred[NWV], wred2[NWV];
  uint32_t minid, ncand, ticket, hover;
  // resolve
  uint32_t loff[MAXSL];
  uint32_t bins[256];
  uint64_t rtop, rtopL;
  uint32_t rflags, rkappa, rmkey, ltot, nh, ns, mfail_sure, mfail_maybe, jcount, bsel;
  double rsc;
};

// z = RN32(x / T) as RN32(x * Rd), Rd = RN64(1 / T). |x * Rd - x / T| <= 2^-51 |x / T| (two fp64 roundings), while
// x / T lies at least 2^-49 |x / T| from every fp32 rounding midpoint (x and T have 24-bit significands, so x - m T
// for a midpoint m is a nonzero multiple of 2^-47 of the binade); the fp32 rounding of the fp64 product therefore
// equals the correctly rounded quotient, subnormal and overflowing results included.
__device__ __forceinline__ float div_exact(float x, double Rd) { return (float)((double)x * Rd); }

__device__ __forceinline__ int nlp_of(const ScanArgs &a, const gse_row &P) {
  return a.lp_ids ? min(min(P.logprobs, GSE_MAX_LOGPROBS), (int)a.lp_ld) : 0;
}

// u16 history counts of tokens [c0, c0 + CH) into sh.cnt; hid holds this thread's ids of the first round (loaded
// before the logits). Returns true (in every thread) when a token occurs more than 65535 times (its counter would
// carry): the row then takes the exact path. Ends with a barrier.
__device__ __forceinline__ bool build_counts16(const RowCtx &c, const int32_t *hist, const int (&hid)[HPT], int c0,
                                               Shared &sh) {
  for (int i = threadIdx.x; i < CH / 8; i += MT) reinterpret_cast<uint4 *>(sh.cnt)[i] = make_uint4(0, 0, 0, 0);
  if (threadIdx.x == 0) sh.hover = 0;
  __syncthreads();
  bool ov = false;
  auto add = [&](int t) {
    if (t >= c0 && t < c0 + CH && t < c.V) {
      const int o = t - c0, s = (o & 1) * 16;
      const uint32_t old = atomicAdd(&sh.cnt[o >> 1], 1u << s);
      ov |= ((old >> s) & 0xFFFFu) == 0xFFFFu;
    }
  };
#pragma unroll
  for (int k = 0; k < HPT; ++k) add(hid[k]);
  for (int j0 = c.hb + MT * HPT; j0 < c.he; j0 += MT * HPT) {
    int more[HPT];
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int j = j0 + k * MT + (int)threadIdx.x;
      more[k] = j < c.he ? hist[j] : -1;
    }
#pragma unroll
    for (int k = 0; k < HPT; ++k) add(more[k]);
  }
  if (ov) sh.hover = 1u;
  __syncthreads();
  return sh.hover != 0;
}

template <int DT, bool FULL>
__device__ __forceinline__ void load_slice(const RowCtx &c, int c0, float (&x)[EPT]) {
  using L = Lay<DT>;
  const int tid = threadIdx.x;
  if constexpr (DT == GSE_F32) {
    const float *p = (const float *)c.base + c0 + tid * 4;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      if (FULL) {
        const float4 f = *reinterpret_cast<const float4 *>(p + v * L::STRIDE);
        x[4 * v] = f.x;
        x[4 * v + 1] = f.y;
        x[4 * v + 2] = f.z;
        x[4 * v + 3] = f.w;
      } else {
        const int t0 = c0 + v * L::STRIDE + tid * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) x[4 * v + k] = 0.0f;
        if (t0 < c.V) {
          const float *q = p + v * L::STRIDE;
          x[4 * v] = q[0];
#pragma unroll
          for (int k = 1; k < 4; ++k)
            if (t0 + k < c.V) x[4 * v + k] = q[k];
        }
      }
    }
  } else {
    const uint16_t *p = (const uint16_t *)c.base + c0 + tid * 8;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      if (FULL) {
        const uint4 u = *reinterpret_cast<const uint4 *>(p + v * L::STRIDE);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[8 * v + 2 * i] = __uint_as_float(w[i] << 16);
          x[8 * v + 2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
      } else {
        const int t0 = c0 + v * L::STRIDE + tid * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k) x[8 * v + k] = 0.0f;
        if (t0 < c.V) {
          const uint16_t *q = p + v * L::STRIDE;
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (t0 + k < c.V) x[8 * v + k] = bf16_to_f32(q[k]);
        }
      }
    }
  }
}

// Block-wide sums over MT threads in a fixed order (wave trees, then waves in order): deterministic.
__device__ __forceinline__ double block_sum_f64(double v, double *red) {
  v = wave_sum_f64(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < NWV; ++w) r += red[w];
  __syncthreads();
  return r;
}

// Exclusive prefix over MT threads in thread order.
__device__ __forceinline__ double block_excl_scan_f64(double v, double *red) {
  const double inc = wave_incl_scan_f64(v);
  __syncthreads();
  if (lane_id() == WAVE - 1) red[threadIdx.x >> 6] = inc;
  __syncthreads();
  double pre = 0.0;
  const int w = threadIdx.x >> 6;
  for (int k = 0; k < w; ++k) pre += red[k];
  __syncthreads();
  return pre + inc - v;
}

// Descending bitonic sort of n (a power of two) packed keys in LDS, one compare-exchange pair per thread per step.
__device__ __forceinline__ void bitonic_desc(uint64_t *a, int n) {
  const int half = n >> 1;
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = threadIdx.x; p < half; p += MT) {
        const int lo = ((p & ~(j - 1)) << 1) | (p & (j - 1));
        const int hi = lo | j;
        const uint64_t x = a[lo], y = a[hi];
        const bool desc = (lo & k) == 0;
        if (desc ? (x < y) : (x > y)) {
          a[lo] = y;
          a[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ void lp_invalid(const ScanArgs &a, int row, int nlp) {
  for (int i = threadIdx.x; i < nlp; i += MT) {
    a.lp_ids[(int64_t)row * a.lp_ld + i] = -1;
    a.lps[(int64_t)row * a.lp_ld + i] = __builtin_nanf("");
  }
}

__device__ __forceinline__ void set_info(RowInfo *ri, uint64_t cmax, uint64_t kkeep, double S, double Z, uint32_t flags,
                                         int32_t token) {
  RowInfo r = {};
  r.cmax = cmax;
  r.kkeep = kkeep;
  r.S = S;
  r.Z = Z;
  r.flags = flags;
  r.token = token;
  *ri = r;
}

// ---------------------------------------------------------------------------------------------------------------------
// Row resolve, run by the last workgroup of the row.

enum { EV_DONE = 0, EV_MORE = 1, EV_HARD = 2 };

struct RowEval {
  const ScanArgs *a;
  int row, nlp, n;
  bool greedy, complete;
  double M, S, B;
  uint64_t gtop;  // greedy rows: packed argmax
  const gse_row *P;
};

// Keep prefix, draw and logprobs over the sorted top arr[0, ns) of the head (ns == n: the whole head).
template <int RPT>
__device__ __forceinline__ int evaluate(const RowEval &ev, const uint64_t *arr, int ns, Shared &sh) {
  const ScanArgs &a = *ev.a;
  const gse_row &P = *ev.P;
  const int tid = threadIdx.x;
  const bool all = ns == ev.n;
  if (ev.nlp > ns && !all) return EV_MORE;
  if (ev.nlp > ns) return EV_HARD;  // logprobs past the finite elements: -inf ranks in id order
  if (tid == 0) {
    sh.mfail_sure = 0xFFFFFFFFu;
    sh.mfail_maybe = 0xFFFFFFFFu;
    sh.jcount = 0;
  }
  // ranks [r0, r0 + RPT) per thread: exact masses e, exclusive prefixes A, inclusive prefixes I
  const int r0 = tid * RPT;
  const double M = ev.M, S = ev.S;
  double e[RPT], A[RPT], I[RPT];
  double loc = 0.0;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = r0 + i;
    e[i] = r < ns ? exp((double)fkey_inv(pk_key(arr[r])) - M) : 0.0;
    loc += e[i];
  }
  double run = block_excl_scan_f64(loc, sh.wred);
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    A[i] = run;
    run += e[i];
    I[i] = run;
  }
  if (ev.nlp > 0) {
    const double lS = log(S);
    for (int i = tid; i < ev.nlp; i += MT) {
      const uint64_t pk = arr[i];
      a.lp_ids[(int64_t)ev.row * a.lp_ld + i] = (int32_t)pk_id(pk);
      a.lps[(int64_t)ev.row * a.lp_ld + i] = (float)(((double)fkey_inv(pk_key(pk)) - M) - lS);
    }
  }
  RowInfo *ri = a.info + ev.row;
  if (ev.greedy) {
    if (tid == 0) set_info(ri, ev.gtop, 0, S, 0.0, R_DONE | R_GREEDY, (int32_t)pk_id(ev.gtop));
    return EV_DONE;
  }
  // keep_r = r < K AND A_r / S < top_p AND q_r >= min_p q_0 (sampling.py:80 plus min-p). A top-p decision is sure when
  // it holds for every S in [S - B, S + B]; the first rank that surely fails and the first that may fail must agree.
  const int64_t K = P.top_k > 0 ? (int64_t)P.top_k : (int64_t)0x7FFFFFFFFFFFll;
  const double topp = P.top_p, minp = P.min_p;
  const double q0 = 1.0 / S, Slo = S - ev.B, Shi = S + ev.B;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = r0 + i;
    if (r < ns) {
      const bool kk = (int64_t)r < K;
      const bool km = !(minp > 0.0) || (e[i] / S >= minp * q0);
      const bool fs = !kk || !km || (A[i] / Shi >= topp);
      const bool fm = !kk || !km || !(A[i] / Slo < topp);
      if (fs) atomicMin(&sh.mfail_sure, (uint32_t)r);
      if (fm) atomicMin(&sh.mfail_maybe, (uint32_t)r);
    }
  }
  __syncthreads();
  uint32_t m = sh.mfail_sure;
  if (m != sh.mfail_maybe) return EV_HARD;
  if (m == 0xFFFFFFFFu) {  // every sorted rank is kept
    if (!all) return EV_MORE;
    if (!ev.complete) return EV_HARD;  // the keep prefix runs past the certified head
    m = (uint32_t)ns;
  }
  // c_last = I_{m-1}; j = #{r < m : I_r < u c_last}, clamped to [0, m - 1] (sampling.py:81-83)
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    if ((uint32_t)(r0 + i) == m - 1) sh.rsc = I[i];
  __syncthreads();
  const double clast = sh.rsc;
  int32_t tok = -1;
  if (a.mode == MODE_SAMPLE) {
    const double u = a.uni ? a.uni[ev.row] : uniform64(P.seed, P.idx);
    const double thr = u * clast;
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      if ((uint32_t)(r0 + i) < m && I[i] < thr) ++cnt;
    if (cnt) atomicAdd(&sh.jcount, cnt);
    __syncthreads();
    tok = (int32_t)pk_id(arr[min(sh.jcount, m - 1u)]);
  }
  if (tid == 0) {
    set_info(ri, arr[0], arr[m - 1], S, clast / S, R_DONE, tok);
    if (a.mode == MODE_SAMPLE) a.tokens[ev.row] = tok;
  }
  return EV_DONE;
}

__device__ __forceinline__ void resolve_row(const ScanArgs &a, int row, const gse_row &P, Shared &sh) {
  const int tid = threadIdx.x;
  const SliceRec *rb = a.rec + (size_t)row * a.nch;
  const bool greedy = is_greedy(a.mode, P);
  RowInfo *ri = a.info + row;
  const int nlp = nlp_of(a, P);
  if (tid == 0) {
    sh.rtop = 0;
    sh.rtopL = 0;
    sh.rflags = 0;
    sh.rkappa = 0;
    sh.rmkey = 0;
    sh.nh = 0;
    sh.ns = 0;
  }
  // One round of record loads: thread s holds slice s's record.
  uint32_t r_nc = 0, r_mkey = 0, r_kap = 0, r_fl = 0;
  uint64_t r_top = 0;
  double r_s = 0.0, r_b = 0.0;
  if (tid < a.nch) {
    const SliceRec *r = rb + tid;
    r_top = ld_ag(&r->top);
    r_kap = ld_ag(&r->kappa);
    r_fl = ld_ag(&r->flags);
    r_nc = ld_ag(&r->ncand);
    r_mkey = ld_ag(&r->mkey);
    r_s = ld_ag(&r->s);
    r_b = ld_ag(&r->bnd);
  }
  __syncthreads();
  if (tid < a.nch) {
    atomicOr(&sh.rflags, r_fl);
    atomicMax((unsigned long long *)&sh.rtop, (unsigned long long)r_top);
    atomicMax(&sh.rkappa, r_kap);
    atomicMax(&sh.rmkey, r_mkey);
  }
  // exclusive prefix of the list lengths (one record per thread)
  {
    const uint32_t inc = wave_incl_scan_u32(r_nc);
    if (lane_id() == WAVE - 1) sh.wtau[tid >> 6] = inc;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      pre += w < (tid >> 6) ? sh.wtau[w] : 0u;
      tot += sh.wtau[w];
    }
    if (tid < a.nch) sh.loff[tid] = pre + inc - r_nc;
    if (tid == 0) sh.ltot = tot;
  }
  __syncthreads();
  const uint32_t flags = sh.rflags;
  const uint32_t mk = sh.rmkey;
  const uint64_t gtop = sh.rtop;  // greedy argmax; or, for a row without z > -inf, the lowest id of its -inf
  const bool bad = (flags & F_NAN) || !(flags & F_FINITE);

  if ((flags & F_OVERFLOW) && (greedy || bad)) {
    // a history counter carried: the exact path redoes the whole row (flags, argmax, logprobs)
    if (tid == 0) set_info(ri, gtop, 0, 0.0, 0.0, R_HARD | R_FULL | (greedy ? R_GREEDY : 0u), -1);
    return;
  }
  if (a.mode == MODE_SAMPLE && (greedy || bad)) {
    const int32_t tok = bad ? -1 : (int32_t)pk_id(gtop);
    if (tid == 0) a.tokens[row] = tok;
    const bool lp_head = greedy && !bad && nlp > 0 && mk > KEY_NEGINF && mk < KEY_POSINF;
    if (!lp_head) {
      if (tid == 0) set_info(ri, gtop, 0, 0.0, 0.0, (greedy ? R_GREEDY : 0u) | (bad ? R_BAD : 0u) | R_DONE, tok);
      lp_invalid(a, row, nlp);
      return;
    }
    // greedy row with logprobs: z = x, the head below gives them; the token stays the argmax
  } else if ((flags & F_NAN) || mk <= KEY_NEGINF) {
    // NaN in z (dist of a bad row) or no z > -inf: q is NaN, keep is empty and j clamps to 0 -> order[0]
    // (sampling.py:82); gtop is the lowest id holding -inf
    if (tid == 0) {
      set_info(ri, gtop, 0, 0.0, 0.0, R_DONE | R_SPECIAL, (int32_t)pk_id(gtop));
      if (a.mode == MODE_SAMPLE) a.tokens[row] = (int32_t)pk_id(gtop);
    }
    lp_invalid(a, row, nlp);
    return;
  }

  // Gather the listed elements: masses for S, the certified head, the packed maximum.
  const bool finite_max = mk < KEY_POSINF;
  const double M = finite_max ? (double)fkey_inv(mk) : 0.0;
  const uint32_t kappa = max(sh.rkappa, KEY_NEGINF + 1u);
  const bool complete = kappa <= KEY_NEGINF + 1u;
  double srest = 0.0, brest = 0.0;
  if (tid < a.nch && finite_max && r_mkey > KEY_NEGINF) {
    const double f = exp((double)fkey_inv(r_mkey) - M);
    srest = f * r_s;
    brest = f * r_b;
  }
  double scand = 0.0;
  const uint64_t *cl0 = a.cand + (size_t)row * a.nch * CAPC;
  const uint32_t ltot = sh.ltot;
  uint64_t bestL = 0;
  for (uint32_t f0 = 0; f0 < ltot; f0 += MT * GPT) {
    uint64_t pk[GPT];
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      const uint32_t f = f0 + g * MT + tid;
      pk[g] = 0;
      if (f < ltot) {
        int lo = 0, hi = a.nch - 1;  // the slice whose range [loff, loff + ncand) holds f
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (sh.loff[mid] <= f) lo = mid;
          else hi = mid - 1;
        }
        pk[g] = ld_ag(&cl0[(size_t)lo * CAPC + (f - sh.loff[lo])]);
      }
    }
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      if (!pk[g]) continue;
      const uint32_t k = pk_key(pk[g]);
      bestL = pk[g] > bestL ? pk[g] : bestL;
      if (finite_max && k > KEY_NEGINF) scand += exp((double)fkey_inv(k) - M);
      if (k >= kappa) {
        const uint32_t pos = atomicAdd(&sh.nh, 1u);
        if (pos < (uint32_t)NH) sh.r.head[pos] = pk[g];
      }
    }
  }
  bestL = wave_max_u64(bestL);
  if (lane_id() == 0) atomicMax((unsigned long long *)&sh.rtopL, (unsigned long long)bestL);
  if (!finite_max) {
    // z holds +inf: every +inf element is listed; token = the lowest id among them (sampling.py:82, order[0])
    __syncthreads();
    const uint64_t t = sh.rtopL;
    const bool hard = (flags & F_OVERFLOW) || a.force_exact;
    if (tid == 0) {
      if (hard) {
        set_info(ri, t, 0, 0.0, 0.0, R_HARD | (greedy ? R_GREEDY : 0u), -1);
      } else {
        set_info(ri, t, 0, 0.0, 0.0, R_DONE | R_SPECIAL | (greedy ? R_GREEDY : 0u), (int32_t)pk_id(t));
        if (a.mode == MODE_SAMPLE && !greedy) a.tokens[row] = (int32_t)pk_id(t);
      }
    }
    if (!hard) lp_invalid(a, row, nlp);
    return;
  }
  srest = block_sum_f64(srest, sh.wred);
  brest = block_sum_f64(brest, sh.wred);
  scand = block_sum_f64(scand, sh.wred);  // (its barriers order the head appends)
  RowEval ev;
  ev.a = &a;
  ev.row = row;
  ev.nlp = nlp;
  ev.greedy = greedy;
  ev.complete = complete;
  ev.M = M;
  ev.S = srest + scand;
  ev.B = brest + 2e-15 * ev.S;
  ev.gtop = gtop;
  ev.P = &P;
  const uint32_t nh_all = sh.nh;
  ev.n = (int)min(nh_all, (uint32_t)NH);
  const int n = ev.n;
  int st = EV_HARD;
  if (!((flags & F_OVERFLOW) || nh_all > (uint32_t)NH || a.force_exact)) {
    if (n <= NSUB) {
      const int np2 = pow2_ceil(max(n, 2));
      for (int i = n + tid; i < np2; i += MT) sh.r.head[i] = 0;
      __syncthreads();
      bitonic_desc(sh.r.head, np2);
      st = evaluate<NSUB / MT>(ev, sh.r.head, n, sh);
    } else {
      // The top of the head: a 256-bin count histogram of (max key - key) picks a key bound with >= SUBT elements
      // above it (<= NSUB when the bins allow); those are sorted first.
      const uint32_t span = mk - kappa;
      const int shift = span >> 8 ? 32 - __clz(span) - 8 : 0;
      sh.bins[tid] = 0;
      if (tid == 0) sh.bsel = 255;
      __syncthreads();
      for (int i = tid; i < n; i += MT) atomicAdd(&sh.bins[(mk - pk_key(sh.r.head[i])) >> shift], 1u);
      __syncthreads();
      const uint32_t cb = sh.bins[tid];
      const uint32_t inc = wave_incl_scan_u32(cb);
      if (lane_id() == WAVE - 1) sh.wtau[tid >> 6] = inc;
      __syncthreads();
      uint32_t pre = 0;
#pragma unroll
      for (int w = 0; w < NWV; ++w) pre += w < (tid >> 6) ? sh.wtau[w] : 0u;
      const uint32_t incl = pre + inc;
      if (incl >= (uint32_t)SUBT && incl - cb < (uint32_t)SUBT) {  // the bin that crosses the target
        atomicMin(&sh.bsel, incl <= (uint32_t)NSUB || tid == 0 ? (uint32_t)tid : (uint32_t)tid - 1u);
      }
      __syncthreads();
      const uint32_t bsel = sh.bsel;
      for (int i = tid; i < n; i += MT) {
        const uint64_t pk = sh.r.head[i];
        if (((mk - pk_key(pk)) >> shift) <= bsel) {
          const uint32_t pos = atomicAdd(&sh.ns, 1u);
          if (pos < (uint32_t)NSUB) sh.r.sub[pos] = pk;
        }
      }
      __syncthreads();
      const int ns = (int)min(sh.ns, (uint32_t)NSUB);
      if (sh.ns <= (uint32_t)NSUB) {
        const int np2 = pow2_ceil(max(ns, 2));
        for (int i = ns + tid; i < np2; i += MT) sh.r.sub[i] = 0;
        __syncthreads();
        bitonic_desc(sh.r.sub, np2);
        st = evaluate<NSUB / MT>(ev, sh.r.sub, ns, sh);
      } else {
        st = EV_MORE;
      }
      if (st == EV_MORE) {  // the keep prefix (or the logprobs) run past the sorted top: sort the whole head
        const int np2 = pow2_ceil(n);
        for (int i = n + tid; i < np2; i += MT) sh.r.head[i] = 0;
        __syncthreads();
        bitonic_desc(sh.r.head, np2);
        st = evaluate<NH / MT>(ev, sh.r.head, n, sh);
      }
    }
  }
  if (st != EV_DONE && tid == 0) {
    // the exact path finishes the row (for a greedy row: its logprobs; the token is already written)
    set_info(ri, gtop, 0, ev.S, 0.0, R_HARD | (greedy ? R_GREEDY : 0u), greedy ? (int32_t)pk_id(gtop) : -1);
  }
}

// ---------------------------------------------------------------------------------------------------------------------

// One slice. Returns true in the workgroup that finished the row last (it then resolves the row).
template <int DT, bool FULL>
__device__ __forceinline__ bool slice_body(const ScanArgs &a, const gse_row &P, const RowCtx &c, int row, int sl,
                                           Shared &sh) {
  using L = Lay<DT>;
  constexpr uint32_t VMASK = (1u << L::VEC) - 1u;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int c0 = sl * CH;
  const int nlp = nlp_of(a, P);
  const bool listing = !c.greedy || nlp > 0;  // candidates and the softmax sum are needed
  const bool divide = c.divide;
  const double Rd = c.Rd;

  // History ids first, then the logits and mask words: the counts build while the logits stream in.
  int hid[HPT];
  if (c.pen) {
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int j = c.hb + k * MT + tid;
      hid[k] = j < c.he ? a.hist[j] : -1;
    }
  }
  float xr[EPT];
  load_slice<DT, FULL>(c, c0, xr);
  uint32_t mw[L::NV];
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = c0 + v * L::STRIDE + tid * L::VEC;
    mw[v] = c.mw ? ((FULL || t0 < c.V) ? c.mw[t0 >> 5] : 0u) : 0xFFFFFFFFu;
  }
  if (tid == 0) {
    sh.minid = 0xFFFFFFFFu;
    sh.ncand = 0;
  }
  const bool hover = c.pen ? build_counts16(c, a.hist, hid, c0, sh) : false;
  float *proc = a.processed ? a.processed + (int64_t)row * a.processed_ld : nullptr;

  // Phase 1: penalties, NaN test (before the mask), mask, z; lane maximum and flags.
  bool fnan = false, ffin = false;
  float zmax = -INFINITY;
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = c0 + v * L::STRIDE + tid * L::VEC;
    uint32_t bits = (mw[v] >> ((tid * L::VEC) & 31)) & VMASK;
    if (!FULL) bits &= t0 >= c.V ? 0u : (c.V - t0 >= L::VEC ? VMASK : (1u << (c.V - t0)) - 1u);  // past the row end
    uint32_t cw[L::VEC / 2];
    bool anycnt = false;
    if (c.pen) {
      const int o = (v * L::STRIDE + tid * L::VEC) >> 1;
      if constexpr (L::VEC == 4) {
        const uint2 q = *reinterpret_cast<const uint2 *>(&sh.cnt[o]);
        cw[0] = q.x;
        cw[1] = q.y;
      } else {
        const uint4 q = *reinterpret_cast<const uint4 *>(&sh.cnt[o]);
        cw[0] = q.x;
        cw[1] = q.y;
        cw[2] = q.z;
        cw[3] = q.w;
      }
#pragma unroll
      for (int k = 0; k < L::VEC / 2; ++k) anycnt |= cw[k] != 0u;
    }
    if (anycnt) {
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const uint32_t ct = (cw[k >> 1] >> ((k & 1) * 16)) & 0xFFFFu;
        if (ct) xr[v * L::VEC + k] = penalize(xr[v * L::VEC + k], ct, c.rp, c.fp, c.pp);
      }
    }
    if (bits == VMASK) {  // every token of the vector allowed
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        const float x = xr[i];
        fnan |= (x != x);
        ffin |= fabsf(x) < INFINITY;
        if (proc) proc[t0 + k] = x;
        const float z = divide ? div_exact(x, Rd) : x;
        xr[i] = z;
        zmax = fmaxf(zmax, z);
      }
    } else {
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        const float x = xr[i];
        fnan |= (x != x);  // (a token past the row end loads 0)
        const bool al = (bits >> k) & 1u;
        const float xm = al ? x : -INFINITY;
        ffin |= fabsf(xm) < INFINITY;
        if (proc && (FULL || t0 + k < c.V)) proc[t0 + k] = xm;
        const float z = (divide && al) ? div_exact(x, Rd) : xm;
        xr[i] = z;
        zmax = fmaxf(zmax, z);
      }
    }
  }

  // Wave reductions: maximum, flags, the wave's candidate threshold (16th largest lane maximum, to 16 key bits).
  const float wmx = wave_max_f32(zmax);
  const uint64_t bn = ballot64(fnan), bf = ballot64(ffin);
  uint32_t tau = 0;
  if (listing) tau = wave_kth_largest_u16(fkey(zmax) >> 16, KW) << 16;
  if (lane == 0) {
    sh.wmax[w] = wmx;
    sh.wflags[w] = (bn ? F_NAN : 0u) | (bf ? F_FINITE : 0u);
    sh.wtau[w] = tau;
  }
  __syncthreads();
  float zw = sh.wmax[0];
  uint32_t flags = sh.wflags[0];
  tau = sh.wtau[0];
#pragma unroll
  for (int k = 1; k < NWV; ++k) {
    zw = fmaxf(zw, sh.wmax[k]);
    flags |= sh.wflags[k];
    tau = max(tau, sh.wtau[k]);
  }
  const bool badrow = (flags & F_NAN) != 0;

  // Lowest id holding the slice maximum: greedy rows (of nan_to_num(x), sampling.py:76), and slices without z > -inf
  // (of -inf: the row may have nothing else). Sampled rows otherwise take it from their listed elements.
  const bool want_id = c.greedy || !(zw > -INFINITY);
  if (want_id) {
    const float target = c.greedy ? fminf(fmaxf(zw, -FLTMAX), FLTMAX) : zw;
    uint32_t best = 0xFFFFFFFFu;
#pragma unroll
    for (int i = EPT - 1; i >= 0; --i) {
      const float g = c.greedy ? fminf(fmaxf(xr[i], -FLTMAX), FLTMAX) : xr[i];
      const int t = c0 + (i / L::VEC) * L::STRIDE + tid * L::VEC + (i % L::VEC);
      if (g == target && (FULL || t < c.V) && xr[i] == xr[i]) best = (uint32_t)t;  // NaN: bad row anyway
    }
    best = wave_min_u32(best);
    if (lane == 0 && best != 0xFFFFFFFFu) atomicMin(&sh.minid, best);
  }

  // Phase 2: listing and the softmax sum of the unlisted elements.
  const uint32_t kap = max(tau, KEY_NEGINF + 1u);
  const float tauf = fkey_inv(kap);
  double s64 = 0.0;
  float mom = 0.0f;
  uint32_t ncl = 0;
  if (listing && !badrow) {
    const bool dosum = fabsf(zw) < INFINITY;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      float ev[L::VEC];
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const float z = xr[v * L::VEC + k];
        const bool p = z >= tauf;
        ncl += p ? 1u : 0u;
        float e = 0.0f;
        if (dosum) {  // -inf (masked) gives t = -inf, e = 0, and 0 * 1e4 in the moment
          const float t = (z - zw) * LOG2E;
          const float ex = __builtin_amdgcn_exp2f(t);
          e = p ? 0.0f : ex;
          mom = fmaf(e, fminf(-t, 1.0e4f), mom);
        }
        ev[k] = e;
      }
      // fixed pairwise order inside the vector, fp64 across vectors
      if constexpr (L::VEC == 4) {
        s64 += (double)((ev[0] + ev[1]) + (ev[2] + ev[3]));
      } else {
        s64 += (double)(((ev[0] + ev[1]) + (ev[2] + ev[3])) + ((ev[4] + ev[5]) + (ev[6] + ev[7])));
      }
    }
  }
  // Candidate positions: wave prefix of the lane counts, one LDS atomic per wave.
  const uint32_t off = wave_incl_scan_u32(ncl) - ncl;
  const uint32_t wtot = (uint32_t)__shfl((int)(off + ncl), WAVE - 1, WAVE);
  uint32_t base = 0;
  if (lane == 0 && wtot) base = atomicAdd(&sh.ncand, wtot);
  base = (uint32_t)__shfl((int)base, 0, WAVE);
  uint64_t *cl = a.cand + ((size_t)row * a.nch + sl) * CAPC;
  if (ncl) {
    uint32_t pos = base + off;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float z = xr[i];
      if (z >= tauf) {
        const int t = c0 + (i / L::VEC) * L::STRIDE + tid * L::VEC + (i % L::VEC);
        if (pos < (uint32_t)CAPC) st_ag(&cl[pos], pack(fkey(z), (uint32_t)t));
        ++pos;
      }
    }
  }
  // error bound of the unlisted sum: v_exp_f32 (2 ulp), the argument's three roundings (2.6 ulp of |t|, times ln 2),
  // two fp32 pairwise additions; flushed subnormal results
  const double bnd = s64 * 4.2e-7 + (double)mom * 1.12e-7 + 1e-36;
  const double sw = wave_sum_f64(s64), bw = wave_sum_f64(bnd);
  if (lane == 0) {
    sh.wred[w] = sw;
    sh.wred2[w] = bw;
  }
  __syncthreads();
  if (tid == 0) {
    double s = 0.0, b = 0.0;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      s += sh.wred[k];
      b += sh.wred2[k];
    }
    const uint32_t nc = sh.ncand;
    const bool over = nc > (uint32_t)CAPC || hover;
    const uint32_t mkey = fkey(zw);
    const uint32_t topkey = c.greedy ? fkey(fminf(fmaxf(zw, -FLTMAX), FLTMAX)) : mkey;
    SliceRec *r = a.rec + (size_t)row * a.nch + sl;
    st_ag(&r->top, (want_id && sh.minid != 0xFFFFFFFFu) ? pack(topkey, sh.minid) : (uint64_t)0);
    st_ag(&r->kappa, listing ? kap : 0u);
    st_ag(&r->ncand, min(nc, (uint32_t)CAPC));
    st_ag(&r->flags, flags | (over ? F_OVERFLOW : 0u));
    st_ag(&r->mkey, mkey);
    st_ag(&r->s, s);
    st_ag(&r->bnd, b);
  }
  // Ticket: the last workgroup of the row resolves it.
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&a.done[row]);
  __syncthreads();
  return sh.ticket == (uint32_t)(a.nch - 1);
}

template <int DT>
__global__ __launch_bounds__(MT) void main_kernel(ScanArgs a) {
  __shared__ Shared sh;
  const int L = blockIdx.x;
  int row, sl;
  if (a.xcd_map) {  // the slices of a row on one XCD (workgroups go round-robin over the 8 XCDs): shared L2
    const int x = L & 7, i = L >> 3;
    row = x + 8 * (i / a.nch);
    sl = i % a.nch;
  } else {
    row = L / a.nch;
    sl = L % a.nch;
  }
  if (row >= a.rows) return;
  const gse_row P = a.params[row];
  const RowCtx c = make_ctx(a, row, P);
  const bool aligned = (((uintptr_t)c.base) & 15u) == 0;
  const bool last = (aligned && (sl + 1) * CH <= a.V) ? slice_body<DT, true>(a, P, c, row, sl, sh)
                                                        : slice_body<DT, false>(a, P, c, row, sl, sh);
  if (!last) return;
  resolve_row(a, row, P, sh);
  if (threadIdx.x == 0) a.done[row] = 0u;
}

}  // namespace

hipError_t launch_main(const ScanArgs &a, hipStream_t s) {
  const int rows = a.xcd_map ? (a.rows + 7) / 8 * 8 : a.rows;
  dim3 grid((unsigned)(rows * a.nch)), block(MT);
  if (a.dtype == GSE_BF16) {
    hipLaunchKernelGGL(main_kernel<GSE_BF16>, grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL(main_kernel<GSE_F32>, grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace gse
