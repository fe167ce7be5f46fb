// The exact path's body, compiled once per workgroup shape by its includer (gse_exact.hip: 1024 threads for the exact
// launch; gse_deep.hip: 256 threads inside the split-row launch). The includer defines, in the namespace it includes
// this in: XT (threads), NB (histogram bins, 4 per thread), LB (log2 NB: key bits per histogram level), CAPS
// (collected elements), CHX (tokens per chunk, 8 per thread), and afterwards xs(), the workgroup's ExactShared in LDS.
// (Included inside namespace gse, after gse_rowctx.h; no include guard: one inclusion per shape.)

constexpr int XW = XT / WAVE;    // waves
constexpr int PER = CHX / XT;    // tokens per thread per chunk (contiguous)
constexpr int HS = 32 - LB;      // level-0 bins (2^HS keys each) of the head's histogram, which the max pass counts
static_assert(NB == 4 * XT && (1 << LB) == NB && CAPS == 8 * XT && PER == 8, "the shape the body is written for");

constexpr int HIDC = 2048;                // history ids a row keeps in LDS for its chunks' count tables
constexpr uint32_t NHID_GLOBAL = 0xFFFFFFFFu;

struct ExactShared {
  uint32_t cnt[CHX];
  union {
    struct {
      uint32_t c[NB];
      uint64_t hi[NB];
      uint64_t lo[NB];
    } h;
    struct {
      uint64_t k[CAPS];
      uint64_t phi[XT];
      uint64_t plo[XT];
    } col;
  } u;
  uint64_t wred[XW];
  uint64_t wred2[XW];
  double dred[XW];
  uint64_t xs[4];
  uint32_t n, found;
  int32_t hid[HIDC];  // the row's history ids, when they fit (nhid of them; nhid = NHID_GLOBAL: read from memory)
  uint32_t nhid;
};

// Context of the row being finished.
struct XCtx {
  const int32_t *hist;
  RowCtx c;
  int row, nch;
  double M, S;
};

// The all-ones mask word that a run of a row without a mask reads (so that the mask word's load has no branch).
__device__ const uint32_t XONES[1] = {0xFFFFFFFFu};

// The logits of tokens t0 .. t0+PER-1 (a thread's run inside a chunk) as raw bits (bf16 zero-extended), loaded
// together so that the PER loads are in flight at once, and converted only where used (raw_logit), so that a
// prefetched run is not waited for early; indexes past the row end read its last element (the callers skip those
// tokens). Returns the mask word of the run (its PER tokens share one: PER divides 32), all ones without a mask.
// The pointers are global ones and no load sits behind a branch (the logits type is a template argument, the mask
// word's address a select): loads through generic pointers, or behind a branch, make later uses wait for every load
// in flight, the next runs' included.
template <int DT>
__device__ __forceinline__ uint32_t load_run(const RowCtx &c, int t0, uint32_t (&v)[PER]) {
  static_assert(32 % PER == 0, "a run shares one mask word");
  typedef const __attribute__((address_space(1))) uint16_t g16;
  typedef const __attribute__((address_space(1))) uint32_t g32;
  if constexpr (DT == GSE_BF16) {
    g16 *p = (g16 *)c.base;
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = p[min(t0 + i, c.V - 1)];
  } else {
    g32 *p = (g32 *)c.base;
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = p[min(t0 + i, c.V - 1)];
  }
  g32 *mp = c.mw ? (g32 *)c.mw : (g32 *)XONES;
  return mp[c.mw ? (min(t0, c.V - 1) >> 5) : 0];
}
__device__ __forceinline__ uint32_t load_run_any(const RowCtx &c, int t0, uint32_t (&v)[PER]) {
  return c.dtype == GSE_BF16 ? load_run<GSE_BF16>(c, t0, v) : load_run<GSE_F32>(c, t0, v);
}

__device__ __forceinline__ float raw_logit(const RowCtx &c, uint32_t r) {
  return __uint_as_float(c.dtype == GSE_BF16 ? r << 16 : r);
}

// The count table sh.cnt of the chunk [c0, c0 + CHX) from the row's history: from its LDS copy when the row's history
// fits, else from memory (a round trip per chunk). Ends with a barrier.
__device__ __forceinline__ void chunk_counts(const RowCtx &c, const int32_t *hist, int c0, ExactShared &sh) {
  const uint32_t nh = sh.nhid;
  if (nh == NHID_GLOBAL) {
    build_counts<CHX>(c, hist, c0, &sh.cnt[0]);
    return;
  }
  for (int i = threadIdx.x; i < CHX / 4; i += XT) reinterpret_cast<uint4 *>(sh.cnt)[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  for (int j = threadIdx.x; j < (int)nh; j += XT) {
    const int t = sh.hid[j];
    if (t >= c0 && t < c0 + CHX && t < c.V) atomicAdd(&sh.cnt[t - c0], 1u);
  }
  __syncthreads();
}

// Calls f(t, key) for every token of the row, thread-contiguous inside each chunk (ids increase with (tid, i)).
// The runs of the next two chunks are loading while the current one is processed (a pass is a chain of chunks, each
// waiting for its loads: with 256 threads a row is about 75 chunks of 2048 tokens). A load past the row reads its last
// chunk again, so every step issues the same loads.
template <int DT, typename F>
__device__ __forceinline__ void for_each_key(const RowCtx &c, const int32_t *hist, int nch, ExactShared &sh, F f) {
  const int tid = threadIdx.x;
  uint32_t v[PER], vn[PER];
  uint32_t mword = load_run<DT>(c, tid * PER, v);
  uint32_t mn = load_run<DT>(c, (nch > 1 ? CHX : 0) + tid * PER, vn);
  for (int ch = 0; ch < nch; ++ch) {
    const int c0 = ch * CHX;
    const int t0 = c0 + tid * PER;
    if (c.pen) chunk_counts(c, hist, c0, sh);
    uint32_t vm[PER];
    const uint32_t mm = load_run<DT>(c, ch + 2 < nch ? t0 + 2 * CHX : t0, vm);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int t = t0 + i;
      if (t < c.V) {
        const uint32_t ct = c.pen ? sh.cnt[t - c0] : 0u;
        bool fn = false, ff = false;
        float xm;
        const uint32_t k = elem_key(c, raw_logit(c, v[i]), ct, (mword >> (t & 31)) & 1u, fn, ff, xm);
        f(t, k);
      }
    }
    if (c.pen) __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = vn[i];
      vn[i] = vm[i];
    }
    mword = mn;
    mn = mm;
  }
}

// The workgroup's LDS: a file-scope __shared__ object of the includer (xs() returns it), so that the pass functions
// below address it as LDS without taking it as an argument (a pointer argument would be a generic one).
__device__ __forceinline__ ExactShared &xs();

// ---- whole-row passes -----------------------------------------------------------------------------------------------
// Each pass over the row is a function of its own, not inlined, taking the row context by value: its element loop is
// then register-allocated apart from the finishing code around it. Inlined, the loop reloaded values of that code
// from private memory (spill slots) inside every element, each reload waited for, at 150-700 us per pass over a
// 128k-token row.

enum { P_MAX = 0, P_SUM, P_COUNT, P_HIST, P_COLLECT, P_TOP, P_MAXH };

struct PassIn {
  double M;         // row maximum of z (P_SUM, P_HIST)
  uint32_t lo, hi;  // key window (P_HIST, P_COLLECT); lo alone: the smallest key counted (P_COUNT)
  int shift;        // bin width 2^shift keys (P_HIST, P_MAXH)
  uint64_t pk;      // smallest packed key collected (P_TOP)
};

struct PassOut {
  uint64_t u;  // P_MAX: the thread's largest packed key; P_COUNT: its count
  double d;    // P_SUM: the thread's sum of exp(z - M), in token order
};

// Every thread of the workgroup calls it. P_HIST adds counts and fixed-point masses to the histogram bins (P_MAXH:
// P_MAX that also counts every key into the bins, masses left alone), P_COLLECT
// and P_TOP append packed keys at xsh.n (the callers clear the bins and the count first and synchronise afterwards).
template <int OP, int DT>
__device__ __noinline__ PassOut row_pass(const RowCtx c, const int32_t *hist, int nch, const PassIn in) {
  ExactShared &sh = xs();
  uint64_t u = 0;
  double d = 0.0;
  for_each_key<DT>(c, hist, nch, sh, [&](int t, uint32_t k) {
    if constexpr (OP == P_MAX || OP == P_MAXH) {
      const uint64_t p = pack(k, (uint32_t)t);
      u = p > u ? p : u;
      if constexpr (OP == P_MAXH) atomicAdd(&sh.u.h.c[k >> in.shift], 1u);
    } else if constexpr (OP == P_SUM) {
      d += k > KEY_NEGINF ? exp((double)fkey_inv(k) - in.M) : 0.0;
    } else if constexpr (OP == P_COUNT) {
      u += k >= in.lo ? 1u : 0u;
    } else if constexpr (OP == P_HIST) {
      if (k >= in.lo && k <= in.hi) {
        const int b = (int)((k - in.lo) >> in.shift);
        atomicAdd(&sh.u.h.c[b], 1u);
        if (k > KEY_NEGINF) {
          const Fx f = fx_of(exp((double)fkey_inv(k) - in.M));
          if (f.hi) atomicAdd((unsigned long long *)&sh.u.h.hi[b], (unsigned long long)f.hi);
          if (f.lo) atomicAdd((unsigned long long *)&sh.u.h.lo[b], (unsigned long long)f.lo);
        }
      }
    } else if constexpr (OP == P_COLLECT) {
      if (k >= in.lo && k <= in.hi) {
        const uint32_t pos = atomicAdd(&sh.n, 1u);
        if (pos < (uint32_t)CAPS) sh.u.col.k[pos] = pack(k, (uint32_t)t);
      }
    } else {
      const uint64_t p = pack(k, (uint32_t)t);
      if (p >= in.pk) {
        const uint32_t pos = atomicAdd(&sh.n, 1u);
        if (pos < (uint32_t)CAPS) sh.u.col.k[pos] = p;
      }
    }
  });
  return PassOut{u, d};
}

template <int OP>
__device__ __forceinline__ PassOut pass(const XCtx &x, const PassIn &in) {
  return x.c.dtype == GSE_BF16 ? row_pass<OP, GSE_BF16>(x.c, x.hist, x.nch, in)
                               : row_pass<OP, GSE_F32>(x.c, x.hist, x.nch, in);
}

// ---- block reductions / scans (1024 threads) ------------------------------------------------------------------------

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, ExactShared &sh) {
  v = wave_max_u64(v);
  __syncthreads();
  if (lane_id() == 0) sh.wred[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int w = 0; w < XW; ++w) r = sh.wred[w] > r ? sh.wred[w] : r;
  __syncthreads();
  return r;
}


__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, ExactShared &sh) {
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane_id() == 0) sh.wred[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int w = 0; w < XW; ++w) r += sh.wred[w];
  __syncthreads();
  return r;
}

// Deterministic block sum: wave tree, then waves in order.
__device__ __forceinline__ double block_sum_f64(double v, ExactShared &sh) {
  v = wave_sum_f64(v);
  __syncthreads();
  if (lane_id() == 0) sh.dred[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
  for (int w = 0; w < XW; ++w) r += sh.dred[w];
  __syncthreads();
  return r;
}


// Exclusive block scan of two u64 values per thread (in thread order).
__device__ __forceinline__ void block_excl_scan2(uint64_t &a, uint64_t &b, ExactShared &sh) {
  const uint64_t ia = wave_incl_scan_u64(a), ib = wave_incl_scan_u64(b);
  __syncthreads();
  if (lane_id() == WAVE - 1) {
    sh.wred[threadIdx.x >> 6] = ia;
    sh.wred2[threadIdx.x >> 6] = ib;
  }
  __syncthreads();
  uint64_t pa = 0, pb = 0;
  const int w = threadIdx.x >> 6;
  for (int k = 0; k < w; ++k) {
    pa += sh.wred[k];
    pb += sh.wred2[k];
  }
  a = pa + ia - a;
  b = pb + ib - b;
  __syncthreads();
}

// ---- histogram over a key window --------------------------------------------------------------------------------------

struct Win {
  uint32_t lo, hi;   // key range of the window (inclusive)
  int shift;         // bin width 2^shift keys
  uint64_t above_n;  // elements with key above the window
  Fx above_m;        // their mass
};

// Builds counts and masses of the keys inside the window.
__device__ __noinline__ void build_hist(const XCtx &x, ExactShared &, const Win &w) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  for (int b = threadIdx.x; b < NB; b += XT) {
    sh.u.h.c[b] = 0;
    sh.u.h.hi[b] = 0;
    sh.u.h.lo[b] = 0;
  }
  __syncthreads();
  pass<P_HIST>(x, PassIn{x.M, w.lo, w.hi, w.shift, 0});
  __syncthreads();
}

// Query kinds: rank (0-based) / first rank whose exclusive mass >= target / first rank whose inclusive mass >= target.
enum { Q_RANK = 0, Q_EXCL = 1, Q_INCL = 2 };

struct Hit {
  int64_t rank;    // rank of the answer element (V when no element qualifies)
  uint64_t pk;     // its packed key (0 when none)
  Fx above;        // mass of all elements ranked before it
  Fx self;         // its own mass
};

__device__ __forceinline__ bool q_pred(int kind, uint64_t r, int64_t n_before, Fx m_before, Fx m_incl, double S,
                                       double tgt) {
  if (kind == Q_RANK) return (int64_t)r < n_before;
  if (kind == Q_EXCL) return fx_val(m_before) / S >= tgt;
  return fx_val(m_incl) / S >= tgt;
}

// Finds, in the current histogram (descending bins), the first bin whose inclusive prefix satisfies the query.
// Returns -1 when none does; fills the window-relative prefix before that bin.
__device__ __noinline__ int find_bin(ExactShared &, const Win &w, int kind, uint64_t r, double S, double tgt, uint64_t &nb_out,
                        Fx &mb_out) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  // thread t owns 4 consecutive bins in descending order: NB-1-4t ... NB-4-4t
  const int tid = threadIdx.x;
  uint64_t n4 = 0, h4 = 0, l4 = 0;
  for (int i = 0; i < 4; ++i) {
    const int b = NB - 1 - (4 * tid + i);
    n4 += sh.u.h.c[b];
    h4 += sh.u.h.hi[b];
    l4 += sh.u.h.lo[b];
  }
  uint64_t pn = n4, ph = h4;
  block_excl_scan2(pn, ph, sh);
  uint64_t pl = l4, dummy = 0;
  block_excl_scan2(pl, dummy, sh);
  if (tid == 0) sh.found = 0xFFFFFFFFu;
  __syncthreads();
  uint64_t n = w.above_n + pn;
  Fx m = fx_add(w.above_m, Fx{ph, pl});
  for (int i = 0; i < 4; ++i) {
    const int b = NB - 1 - (4 * tid + i);
    const uint64_t cb = sh.u.h.c[b];
    const Fx mb{sh.u.h.hi[b], sh.u.h.lo[b]};
    const Fx mi = fx_add(m, mb);
    bool hit;
    if (kind == Q_RANK) hit = r < n + cb;
    else if (kind == Q_EXCL) hit = cb > 0 && fx_val(mi) / S >= tgt;
    else hit = cb > 0 && fx_val(mi) / S >= tgt;
    if (hit) {
      atomicMin(&sh.found, (uint32_t)(4 * tid + i));
      break;
    }
    n += cb;
    m = mi;
  }
  __syncthreads();
  const uint32_t f = sh.found;
  __syncthreads();
  if (f == 0xFFFFFFFFu) return -1;
  // recompute the prefix before bin index f (descending index) on one thread and broadcast
  if (tid == (int)(f >> 2)) {
    uint64_t nn = w.above_n + pn;
    Fx mm = fx_add(w.above_m, Fx{ph, pl});
    for (uint32_t i = 0; i < (f & 3u); ++i) {
      const int b = NB - 1 - (int)(4 * (f >> 2) + i);
      nn += sh.u.h.c[b];
      mm = fx_add(mm, Fx{sh.u.h.hi[b], sh.u.h.lo[b]});
    }
    sh.xs[0] = nn;
    sh.xs[1] = mm.hi;
    sh.xs[2] = mm.lo;
  }
  __syncthreads();
  nb_out = sh.xs[0];
  mb_out = Fx{sh.xs[1], sh.xs[2]};
  __syncthreads();
  return NB - 1 - (int)f;
}

// Collects the packed keys of every element with key in [klo, khi] into LDS (sorted descending). Returns the count
// (possibly above CAPS: then the list is partial).
__device__ __noinline__ uint32_t collect(const XCtx &x, ExactShared &, uint32_t klo, uint32_t khi) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  if (threadIdx.x == 0) sh.n = 0;
  __syncthreads();
  pass<P_COLLECT>(x, PassIn{0.0, klo, khi, 0, 0});
  __syncthreads();
  const uint32_t n = sh.n;
  if (n <= (uint32_t)CAPS) {
    const int np2 = pow2_ceil(max((int)n, 2));
    for (int i = (int)n + threadIdx.x; i < np2; i += XT) sh.u.col.k[i] = 0;
    __syncthreads();
    block_sort_desc_u64(sh.u.col.k, np2);
  }
  return n;
}

// Walks a collected, sorted list (n <= CAPS) for the query, with n_before / m_before the prefix above the list.
// Returns the index inside the list (or n when no element qualifies) and fills the element's prefix mass.
__device__ __noinline__ int walk_list(const XCtx &x, ExactShared &, int n, int kind, uint64_t r, uint64_t n_before, Fx m_before,
                         double tgt, Fx &above, Fx &self) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  const int tid = threadIdx.x;
  constexpr int PT = CAPS / XT;  // 8 elements per thread, consecutive
  Fx ef[PT];
  const double M = x.M;
  uint64_t sh_hi = 0, sh_lo = 0;
  for (int i = 0; i < PT; ++i) {
    const int idx = tid * PT + i;
    ef[i] = Fx{0, 0};
    if (idx < n) {
      const uint32_t k = pk_key(sh.u.col.k[idx]);
      if (k > KEY_NEGINF) ef[i] = fx_of(exp((double)fkey_inv(k) - M));
    }
    sh_hi += ef[i].hi;
    sh_lo += ef[i].lo;
  }
  block_excl_scan2(sh_hi, sh_lo, sh);
  if (tid == 0) sh.found = 0xFFFFFFFFu;
  __syncthreads();
  Fx m = fx_add(m_before, Fx{sh_hi, sh_lo});
  for (int i = 0; i < PT; ++i) {
    const int idx = tid * PT + i;
    if (idx >= n) break;
    const Fx mi = fx_add(m, ef[i]);
    if (q_pred(kind, r, (int64_t)n_before + idx + 1, m, mi, x.S, tgt)) {
      atomicMin(&sh.found, (uint32_t)idx);
      break;
    }
    m = mi;
  }
  __syncthreads();
  const uint32_t f = sh.found;
  __syncthreads();
  if (f == 0xFFFFFFFFu) return n;
  if (tid == (int)(f / PT)) {
    Fx mm = fx_add(m_before, Fx{sh_hi, sh_lo});
    for (uint32_t i = 0; i < f % PT; ++i) mm = fx_add(mm, ef[i]);
    sh.xs[0] = mm.hi;
    sh.xs[1] = mm.lo;
    sh.xs[2] = ef[f % PT].hi;
    sh.xs[3] = ef[f % PT].lo;
  }
  __syncthreads();
  above = Fx{sh.xs[0], sh.xs[1]};
  self = Fx{sh.xs[2], sh.xs[3]};
  __syncthreads();
  return (int)f;
}

// Elements sharing one key, taken in token-id order: the token at position p (0-based) among them.
__device__ __noinline__ uint32_t nth_with_key(const XCtx &x, ExactShared &, uint32_t key, uint64_t p) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  const int tid = threadIdx.x;
  uint64_t base = 0;
  if (tid == 0) sh.found = 0xFFFFFFFFu;
  __syncthreads();
  const RowCtx c = x.c;
  const int32_t *hist = x.hist;
  const int nch = x.nch;
  for (int ch = 0; ch < nch; ++ch) {
    const int c0 = ch * CHX;
    if (c.pen) chunk_counts(c, hist, c0, sh);
    const int t0 = c0 + tid * PER;
    uint32_t v[PER];
    const uint32_t mword = load_run_any(c, t0, v);
    uint32_t match = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int t = t0 + i;
      if (t < c.V) {
        const uint32_t ct = c.pen ? sh.cnt[t - c0] : 0u;
        bool fn = false, ff = false;
        float xm;
        if (elem_key(c, raw_logit(c, v[i]), ct, (mword >> (t & 31)) & 1u, fn, ff, xm) == key) match |= 1u << i;
      }
    }
    uint64_t cntm = (uint64_t)__popc(match), d = 0;
    block_excl_scan2(cntm, d, sh);
    const uint64_t total = block_sum_u64((uint64_t)__popc(match), sh);
    const uint64_t mine = base + cntm;
    if (p >= mine && p < mine + (uint64_t)__popc(match)) {
      uint32_t left = (uint32_t)(p - mine), mm = match;
      for (int i = 0; i < PER; ++i) {
        if (mm & (1u << i)) {
          if (left == 0) {
            sh.found = (uint32_t)(t0 + i);
            break;
          }
          --left;
        }
      }
    }
    base += total;
    if (x.c.pen) __syncthreads();
    __syncthreads();
    if (sh.found != 0xFFFFFFFFu) break;
  }
  __syncthreads();
  return sh.found;
}

// Runs one query to its element: histogram levels, collection, walk.
__device__ __noinline__ Hit query(const XCtx &x, ExactShared &, int kind, uint64_t r, double tgt) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  Hit out;
  Win w{0u, 0xFFFFFFFFu, HS, 0, Fx{0, 0}};
  for (int level = 0; level < (32 + LB - 1) / LB; ++level) {
    build_hist(x, sh, w);
    uint64_t nb = 0;
    Fx mb{0, 0};
    const int b = find_bin(sh, w, kind, r, x.S, tgt, nb, mb);
    if (b < 0) {
      out.rank = -1;
      out.pk = 0;
      return out;
    }
    const uint64_t cb = sh.u.h.c[b];
    const uint32_t klo = w.lo + ((uint32_t)b << w.shift);
    const uint32_t khi = w.shift == 0 ? klo : klo + ((1u << w.shift) - 1u);
    __syncthreads();
    if (cb <= (uint64_t)CAPS) {
      const uint32_t n = collect(x, sh, klo, khi);
      Fx above, self;
      const int i = walk_list(x, sh, (int)n, kind, r, nb, mb, tgt, above, self);
      if (i >= (int)n) {  // no element of the bin qualifies (exclusive mass): the answer is the next bin's first
        out.rank = (int64_t)(nb + n);
        out.pk = 0;
        return out;
      }
      out.rank = (int64_t)(nb + i);
      out.pk = sh.u.col.k[i];
      out.above = above;
      out.self = self;
      __syncthreads();
      return out;
    }
    if (w.shift == 0) {
      // one key with more elements than fit: equal z, equal mass; the answer is positional in token-id order
      const uint32_t k = klo;
      const Fx e = k > KEY_NEGINF ? fx_of(exp((double)fkey_inv(k) - x.M)) : Fx{0, 0};
      uint64_t pos;
      if (kind == Q_RANK) {
        pos = r - nb;
      } else {
        // smallest p with (before + p * e (+ e)) / S >= tgt; the bin holds the answer so p < cb
        uint64_t lo = 0, hi = cb - 1;
        while (lo < hi) {
          const uint64_t mid = (lo + hi) / 2;
          const Fx mp = fx_add(mb, Fx{e.hi * (mid + (kind == Q_INCL)), e.lo * (mid + (kind == Q_INCL))});
          if (fx_val(mp) / x.S >= tgt) hi = mid;
          else lo = mid + 1;
        }
        pos = lo;
      }
      const uint32_t t = nth_with_key(x, sh, k, pos);
      out.rank = (int64_t)(nb + pos);
      out.pk = pack(k, t);
      out.above = fx_add(mb, Fx{e.hi * pos, e.lo * pos});
      out.self = e;
      return out;
    }
    w = Win{klo, khi, w.shift > LB ? w.shift - LB : 0, nb, mb};
  }
  out.rank = -1;
  out.pk = 0;
  return out;
}


// Elements of the head, at most: the cut is the level-0 bin that holds this rank. Smaller heads sort faster; a query
// whose answer ranks below the head runs its own levels (forced exact, 16 rows: 2048 measured 12% faster than 8192
// on C3 rows, 37% on C1 rows).
constexpr int HEADN = 2048;
static_assert(HEADN <= CAPS, "the head fits the list area");
static_assert((0xFFFFFFFFu >> HS) < (uint32_t)NB, "the level-0 bins cover every key");

// The head of the row: every element above the level-0 histogram bin that holds rank HEADN (every element when the row
// has at most HEADN), collected and sorted descending in the list area; kcut receives the smallest key it covers
// completely (every element with a key >= kcut is in the head). Returns its length, 0 when the top bin alone holds
// more than HEADN elements. Expects the level-0 counts of every key in the histogram (the max pass, P_MAXH), masses
// zero: the cut is a rank. A query answered inside the head is a walk of the list; query() reuses the LDS, after
// which the head is gone.
__device__ __noinline__ uint32_t collect_head(const XCtx &x, ExactShared &, uint32_t &kcut) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  const Win w{0u, 0xFFFFFFFFu, HS, 0, Fx{0, 0}};
  uint64_t nb = 0;
  Fx mb{0, 0};
  const int b = find_bin(sh, w, Q_RANK, (uint64_t)HEADN, x.S, 0.0, nb, mb);
  if (b == NB - 1) return 0;
  kcut = b < 0 ? 0u : (uint32_t)(b + 1) << w.shift;
  __syncthreads();
  return collect(x, sh, kcut, 0xFFFFFFFFu);
}

// A query answered from the head of n elements: false when no element of the head satisfies it (the answer, if any,
// ranks at n or below).
__device__ __noinline__ bool head_query(const XCtx &x, ExactShared &, uint32_t n, int kind, uint64_t r, double tgt, Hit &h) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  Fx above, self;
  const int i = walk_list(x, sh, (int)n, kind, r, 0, Fx{0, 0}, tgt, above, self);
  if (i >= (int)n) return false;
  h.rank = i;
  h.pk = sh.u.col.k[i];
  h.above = above;
  h.self = self;
  __syncthreads();
  return true;
}

__device__ __noinline__ uint64_t count_ge(const XCtx &x, ExactShared &, uint32_t kmin) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  return block_sum_u64(pass<P_COUNT>(x, PassIn{0.0, kmin, 0, 0, 0}).u, sh);
}

// Collects the elements with packed key >= pk (the top ranks) and sorts them.
__device__ __noinline__ uint32_t collect_top(const XCtx &x, ExactShared &, uint64_t pk) {
  ExactShared &sh = xs();  // (the LDS object itself: a reference argument is a generic pointer)
  if (threadIdx.x == 0) sh.n = 0;
  __syncthreads();
  pass<P_TOP>(x, PassIn{0.0, 0, 0, 0, pk});
  __syncthreads();
  const uint32_t n = min(sh.n, (uint32_t)CAPS);
  const int np2 = pow2_ceil(max((int)n, 2));
  for (int i = (int)n + threadIdx.x; i < np2; i += XT) sh.u.col.k[i] = 0;
  __syncthreads();
  block_sort_desc_u64(sh.u.col.k, np2);
  return n;
}

// Finishes one hard row (every thread of the workgroup calls it; its LDS is free again when it returns).
__device__ __forceinline__ void exact_row(const ScanArgs &a, int row, ExactShared &sh) {
  RowInfo *ri = a.info + row;
  const int tid = threadIdx.x;
  const gse_row P = a.params[row];
  const bool greedy = is_greedy(a.mode, P);
  XCtx x;
  x.hist = a.hist;
  x.row = row;
  x.nch = (a.V + CHX - 1) / CHX;
  x.c = make_ctx(a, row, P);
  {  // the row's history ids into LDS when they fit (every chunk of every pass counts its tokens from them)
    const int nh = x.c.pen ? x.c.he - x.c.hb : 0;
    const bool fits = nh <= HIDC;
    if (fits)
      for (int j = tid; j < nh; j += XT) sh.hid[j] = a.hist[x.c.hb + j];
    if (tid == 0) sh.nhid = fits ? (uint32_t)nh : NHID_GLOBAL;
    __syncthreads();
  }
  if (greedy) {  // logprobs of a greedy row are taken over z = x
    x.c.greedy = false;
    x.c.divide = false;
  }
  const int nlp = a.lp_ids ? min(min(P.logprobs, GSE_MAX_LOGPROBS), (int)a.lp_ld) : 0;
  if (ri->flags & R_FULL) {
    // the main pass could not count the history: recompute the row flags and, for a greedy row, the argmax
    // (first maximum of nan_to_num of the masked logits, sampling.py:70-76)
    RowCtx gc = make_ctx(a, row, P);
    bool fnan = false, ffin = false;
    uint64_t gb = 0;
    const int nch = (a.V + CHX - 1) / CHX;
    for (int ch = 0; ch < nch; ++ch) {
      const int c0 = ch * CHX;
      if (gc.pen) chunk_counts(gc, a.hist, c0, sh);
      const int t0 = c0 + tid * PER;
      uint32_t v[PER];
      const uint32_t mword = load_run_any(gc, t0, v);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int t = t0 + i;
        if (t < gc.V) {
          float xm;
          const uint32_t k =
              elem_key(gc, raw_logit(gc, v[i]), gc.pen ? sh.cnt[t - c0] : 0u, (mword >> (t & 31)) & 1u, fnan, ffin, xm);
          const uint64_t p = pack(k, (uint32_t)t);
          gb = p > gb ? p : gb;
        }
      }
      if (gc.pen) __syncthreads();
    }
    gb = block_max_u64(gb, sh);
    const bool anynan = block_sum_u64(fnan ? 1u : 0u, sh) != 0;
    const bool anyfin = block_sum_u64(ffin ? 1u : 0u, sh) != 0;
    const bool bad = anynan || !anyfin;
    if (a.mode == MODE_SAMPLE && (bad || greedy)) {
      const int32_t tok = bad ? -1 : (int32_t)pk_id(gb);
      if (tid == 0) a.tokens[row] = tok;
      if (bad || !nlp) {
        for (int i = tid; i < nlp; i += XT) {
          a.lp_ids[(int64_t)row * a.lp_ld + i] = -1;
          a.lps[(int64_t)row * a.lp_ld + i] = __builtin_nanf("");
        }
        if (tid == 0) ri->flags = R_DONE | R_BY_EXACT | (bad ? R_BAD : 0u) | (greedy ? R_GREEDY : 0u);
        return;
      }
    } else if (anynan) {  // dist of a NaN row is NaN everywhere
      if (tid == 0) ri->flags = R_DONE | R_BY_EXACT | R_SPECIAL;
      return;
    }
  }
  // pass 0: the row maximum of z
  // (with the level-0 counts of the head when a query will need it)
  const bool want_head = !greedy || nlp > 0;
  if (want_head) {
    for (int b = tid; b < NB; b += XT) {
      sh.u.h.c[b] = 0;
      sh.u.h.hi[b] = 0;
      sh.u.h.lo[b] = 0;
    }
    __syncthreads();
  }
  const PassIn pin{0.0, 0u, 0xFFFFFFFFu, HS, 0};
  uint64_t best = block_max_u64((want_head ? pass<P_MAXH>(x, pin) : pass<P_MAX>(x, pin)).u, sh);
  const uint32_t mk = pk_key(best);
  if (mk >= KEY_POSINF || mk <= KEY_NEGINF) {
    for (int i = tid; i < nlp; i += XT) {
      a.lp_ids[(int64_t)row * a.lp_ld + i] = -1;
      a.lps[(int64_t)row * a.lp_ld + i] = __builtin_nanf("");
    }
    if (tid == 0) {
      // z holds +inf or its maximum is -inf: token = order[0], the lowest id at the maximum key (sampling.py:82)
      ri->cmax = best;
      ri->flags = R_DONE | R_BY_EXACT | R_SPECIAL | (greedy ? R_GREEDY : 0u);
      if (a.mode == MODE_SAMPLE && !greedy) a.tokens[row] = (int32_t)pk_id(best);
    }
    return;
  }
  x.M = (double)fkey_inv(mk);
  // pass A: S (fixed thread order, deterministic)
  x.S = block_sum_f64(pass<P_SUM>(x, PassIn{x.M, 0, 0, 0, 0}).d, sh);
  const double S = x.S;
  const int64_t V = a.V;

  // The head serves the queries below whose answers rank inside it; nh = 0 once a query has run its own levels.
  uint32_t kcut = 0, nh = 0;
  if (want_head) nh = collect_head(x, sh, kcut);
  if (!greedy) {
    const double q0 = 1.0 / S;
    int64_t m = V;
    if (P.top_k > 0 && P.top_k < m) m = P.top_k;
    if (P.min_p > 0.0) {
      // smallest key whose q passes q >= min_p * q_0 (monotone in the key), then count the keys above it
      const double thr = P.min_p * q0;
      uint32_t lo = KEY_NEGINF + 1u, hi = mk;
      while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (exp((double)fkey_inv(mid) - x.M) / S >= thr) hi = mid;
        else lo = mid + 1;
      }
      int64_t mm;
      if (nh > 0 && lo >= kcut) {  // every key >= lo is in the head
        uint64_t c = 0;
        for (int i = tid; i < (int)nh; i += XT) c += pk_key(sh.u.col.k[i]) >= lo ? 1u : 0u;
        mm = (int64_t)block_sum_u64(c, sh);
      } else {
        mm = (int64_t)count_ge(x, sh, lo);
      }
      if (mm < m) m = mm;
    }
    {
      // An answer at rank m or below leaves m as it is: with m <= nh, one not in the head needs no search.
      Hit hp;
      if (nh > 0 && head_query(x, sh, nh, Q_EXCL, 0, P.top_p, hp)) {
        if (hp.rank < m) m = hp.rank;
      } else if (!(nh > 0 && m <= (int64_t)nh)) {
        nh = 0;
        hp = query(x, sh, Q_EXCL, 0, P.top_p);
        if (hp.rank >= 0 && hp.rank < m) m = hp.rank;
      }
    }
    if (m < 1) m = 1;
    Hit hl;
    if (!(m <= (int64_t)nh && head_query(x, sh, nh, Q_RANK, (uint64_t)(m - 1), 0.0, hl))) {
      nh = 0;
      hl = query(x, sh, Q_RANK, (uint64_t)(m - 1), 0.0);
    }
    const double clast = fx_val(fx_add(hl.above, hl.self)) / S;
    int32_t tok = -1;
    if (a.mode == MODE_SAMPLE) {
      const double u = a.uni ? a.uni[row] : uniform64(P.seed, P.idx);
      const double thr = u * clast;
      Hit hj;
      if (!(nh > 0 && head_query(x, sh, nh, Q_INCL, 0, thr, hj))) {
        nh = 0;
        hj = query(x, sh, Q_INCL, 0, thr);
      }
      if (hj.rank < 0 || hj.rank > m - 1) hj = hl;  // j = min(count, keep.sum() - 1)
      tok = (int32_t)pk_id(hj.pk);
    }
    if (tid == 0) {
      RowInfo r = {};
      r.cmax = best;
      r.kkeep = hl.pk;
      r.S = S;
      r.Z = clast;
      r.flags = R_DONE | R_BY_EXACT;
      r.token = tok;
      if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
      *ri = r;
    }
  } else if (tid == 0) {
    ri->flags = R_DONE | R_BY_EXACT | R_GREEDY;
  }
  if (nlp > 0) {
    const int n_top = (int)min((int64_t)nlp, V);
    uint32_t n = (uint32_t)n_top;  // the first n_top elements of the head, when it holds them
    if (n_top > (int)nh) {
      const Hit hn = query(x, sh, Q_RANK, (uint64_t)(n_top - 1), 0.0);
      n = collect_top(x, sh, hn.pk);
    }
    const double lS = log(S);
    for (int i = tid; i < nlp; i += XT) {
      int32_t id = -1;
      float lp = __builtin_nanf("");
      if (i < (int)n) {
        const uint64_t pk = sh.u.col.k[i];
        id = (int32_t)pk_id(pk);
        const uint32_t k = pk_key(pk);
        lp = k > KEY_NEGINF ? (float)(((double)fkey_inv(k) - x.M) - lS) : -INFINITY;
      }
      a.lp_ids[(int64_t)row * a.lp_ld + i] = id;
      a.lps[(int64_t)row * a.lp_ld + i] = lp;
    }
  }
}

