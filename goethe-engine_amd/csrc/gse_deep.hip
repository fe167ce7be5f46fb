// Split-row finish of the rows the main pass could not decide from its certified head: a keep prefix that runs past
// the listed elements (the nucleus of a flat, hot row), or a top-p decision that fell inside the main pass's bound on
// S. One launch; each deep row is spread over S slices (S and the slice length follow from the number of deep rows so
// that the grid is one round of resident workgroups, one slice each). Slices add their results into the row's record
// with integer atomics (the same sums in any order), and the last slice of a row to finish a phase (atomic ticket)
// carries on with the row. Every workgroup runs all its count items before any pick item.
//
//   count:  each slice recomputes z exactly as the main pass does and adds a 512-bin histogram of
//           d = z_max - z: counts and exact fixed-point masses (fp64 exp, whole multiples of 2^-40 and 2^-64; bins
//           1/32 wide, the last one open-ended). d is monotone in z, so the bins follow the stable order and ties share
//           a bin. The row's last slice plans: the bins that hold the last kept element (top-p, top-k and min-p cuts)
//           and the bins that may hold the draw, whether they hold at most DCAP elements, and the exact masses of the
//           regions before and between them; then it publishes the plan's status.
//   pick:   each slice builds its history table, waits for its row's plan (a bounded wait: past the limit the slice
//           spoils the row, which then takes the exact path), recomputes z and lists the window elements (no z is
//           written between the passes).
//           The row's last slice finishes: exact sub-bin counts and masses over the list locate the cut and the draw,
//           only the sub-bins holding them are sorted, and their exact prefixes (one scan) give the last kept element,
//           c_last and the token. A failed check leaves the row to the exact path (gse_exact.hip). It then clears the
//           row's records for the next call.
//
// Semantics (goethe_engine/sampling.py:77-83): keep_r = r < top_k AND cumsum(q)_r - q_r < top_p (AND q_r >= min_p q_0);
// c = cumsum(q keep); token = order[min(count(c < u c[-1]), m - 1)], m = keep.sum().
#include "gse_stream.h"

namespace gse {

namespace {

using namespace strm;

constexpr float BSC = 32.0f;    // bins per unit of d
constexpr int BPT = DNB / MT;   // planner: bins per thread (contiguous)
constexpr int WLC = 1024;       // window elements a slice gathers in LDS before one global reservation (the histogram's space)
static_assert(BPT * MT == DNB, "");

struct DeepShared {
  HistTab h;                    // the slice's history tables while streaming
  union {
    struct {
      uint64_t hi[DNB];         // count pass: the slice's histogram, mass in 2^-40 units
      uint64_t lo[DNB];         // mass in 2^-64 units (below 2^40), element count << 48
    } c;
    uint64_t wl[WLC];           // pick pass: the slice's window elements
  };
  uint64_t pplan;
  uint32_t hover, ticket, nwl, wbase;
  uint32_t wsum[NWV];
  uint64_t wred[NWV], wred2[NWV];
  double dred[NWV];
  uint32_t q[8];                // first-bin / first-index queries (atomicMin)
  double qd[2];
  uint64_t acc[DA_N];
  uint64_t pub[6];
};

// Bin of z (z > -inf, z <= M): monotone non-increasing in z.
__device__ __forceinline__ uint32_t dbin(float z, float M) {
  return (uint32_t)fminf((M - z) * BSC, (float)(DNB - 1));
}

__device__ __forceinline__ void atomic_add_ag(uint64_t *p, uint64_t v) {
  (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A slice's wave priority by its workgroup's dispatch quarter (later: higher). The workgroups sharing a CU are
// dispatched in order, and at equal priority the oldest wave wins issue arbitration, so the last quarter's slices used
// to end last; a row's plan waits for its slowest slice. (C3 split-row pass 49.6 -> 48.5 us.)
__device__ __forceinline__ void prio_by_quarter() {
  const uint32_t q = min(3u, (uint32_t)blockIdx.x * 4u / gridDim.x);
  if (q == 0) __builtin_amdgcn_s_setprio(0);
  else if (q == 1) __builtin_amdgcn_s_setprio(1);
  else if (q == 2) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(3);
}

// Streams the slice [p0, p1) of the row through the main pass's element pipeline. The full chunks go through a
// double-buffered loop whose loads are the same for every chunk (a chunk past the end reads the row's first one), so
// one chunk stays in flight while the wave works on another; the history ids and each wave's first chunks are loaded
// before the history tables are built. A partial last chunk is taken by wave 0 afterwards, with bounds checks.
// With keep, the history tables in LDS are already the slice's (built by the count item of the same slice) and are not
// built again. pre() runs (every thread) once the history tables are built, before the first chunk is used. f(z, token, valid) is
// called for every element slot of each chunk by every lane of the wave (valid false past the slice end), so f may use
// ballots. Ends with a barrier.
template <int DT, bool AL, typename Pre, typename F>
__device__ __forceinline__ void stream_slice(const ScanArgs &a, const RowCtx &c, int row, int p0, int p1,
                                             DeepShared &sh, bool keep, Pre pre, F f) {
  using L = Lay<DT>;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int nfull = (p1 - p0) / CHK;
  const bool build = c.pen && !keep;
  int hid[HPT];
  if (build) {
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int j = c.hb + k * MT + tid;
      hid[k] = j < c.he ? a.hist[j] : -1;
    }
  }
  float xa[EPL], xb[EPL];
  uint32_t ma[L::NV], mb[L::NV];
  const int wu = __builtin_amdgcn_readfirstlane(w);  // (the wave index as a scalar: the chunk loop stays uniform)
  int ck = wu, cn = wu + NWV;
  // both buffers' chunks go out before the history build (a slice of a few chunks per wave then loads at once)
  if (nfull > 0) {
    load_full<DT, AL>(c, p0 + ck * CHK, ck < nfull, xa, ma);
    load_full<DT, AL>(c, p0 + cn * CHK, cn < nfull, xb, mb);
  }
  if (build) {
    if (tid == 0) sh.hover = 0;
    build_history(c, a.hist, hid, p0, p1, sh.h, sh.wsum, sh.hover);
  } else {
    __syncthreads();
  }
  pre();
  Lane ln;
  ln.m = -INFINITY;
  ln.s = 0.0;
  ln.b = 0.0;
  ln.kap = 0;
  ln.woff = 0;
  ln.g = -INFINITY;
  ln.gid = 0xFFFFFFFFu;
  ln.fid = 0xFFFFFFFFu;
  ln.fnan = false;
  ln.ffin = false;
  int nxt = wu + 2 * NWV;  // wave w takes chunks w, w + 4, w + 8, ... (scalar arithmetic)
  auto grab = [&]() -> int {
    const int n = nxt;
    nxt += NWV;
    return n;
  };
  auto body = [&](int k, float(&x)[EPL], uint32_t(&mw)[L::NV]) __attribute__((always_inline)) {
    const int cb = p0 + k * CHK;
    // take the chunk's registers here, unconditionally: the waits for its loads then sit at this point (counted, with
    // the next chunk still in flight) rather than inside the rare per-element branches below
#pragma unroll
    for (int i = 0; i < EPL; ++i) asm volatile("" : "+v"(x[i]));
#pragma unroll
    for (int v = 0; v < L::NV; ++v) asm volatile("" : "+v"(mw[v]));
    (void)chunk_phase1<DT>(a, c, row, cb, p0, p1, x, mw, ln, sh.h);
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
#pragma unroll
      for (int e = 0; e < L::VEC; ++e) {
        const int t = cb + v * L::STRIDE + lane * L::VEC + e;
        f(x[v * L::VEC + e], t, t < p1);
      }
    }
  };
  if (nfull > 0) {
    while (true) {
      if (ck >= nfull) break;
      body(ck, xa, ma);
      ck = grab();
      load_full<DT, AL>(c, p0 + ck * CHK, ck < nfull, xa, ma);
      if (cn >= nfull) break;
      body(cn, xb, mb);
      cn = grab();
      load_full<DT, AL>(c, p0 + cn * CHK, cn < nfull, xb, mb);
    }
  }
  if (nfull * CHK < p1 - p0 && w == 0) {  // the partial last chunk (uniform in wave 0)
    load_chunk<DT, AL>(c, p0 + nfull * CHK, p1, xa, ma);
    body(nfull, xa, ma);
  }
  __syncthreads();
}

// Slices of the deep rows: as many per row as one round of the grid holds (the grid is resident at once), at most
// DSMAX, each a multiple of CHK long and at most PTOK. Item i is slice i % S of slot i / S, in both phases.
struct DGeom {
  int S, len;
};
__device__ __forceinline__ DGeom deep_geom(const ScanArgs &a, int nd) {
  int S = min(max(1, (int)gridDim.x / nd), DSMAX);
  S = max(S, (a.V + PTOK - 1) / PTOK);
  int len = ((a.V + S - 1) / S + CHK - 1) / CHK * CHK;
  len = min(len, PTOK);
  return DGeom{(a.V + len - 1) / len, len};
}

// ---------------------------------------------------------------------------------------------------------------------
// Pass 1: histogram and plan.

// The plan of a row from its histogram (added by every slice of this launch), into the row's slot: {w2lo, w2hi, w1lo,
// w1hi, status} and the element counts of the regions outside the windows. Run by the whole workgroup of the row's
// last count slice: thread t holds bins 2t and 2t + 1; inclusive prefixes by block scans (wave scans, then the wave
// totals in order), "first bin with" queries by LDS minima, and lookups at the window edges from LDS tables.
struct PlanShared {
  uint64_t ph[DNB], po[DNB];  // inclusive prefixes through each bin: masses in 2^-40 and 2^-64 units
  uint32_t pc[DNB];           // and element counts (a row has fewer than 2^32 elements)
  uint64_t wt[3][NWV];                 // wave totals
  uint32_t q[8];                       // queries: first / last bins
};

enum { PQ_B0, PQ_B1, PQ_B2, PQ_B5, PQ_B6, PQ_B3, PQ_B4, PQ_N };

__device__ __forceinline__ void plan_block(const uint64_t *gh, DeepSlot *ds, int mode, PlanShared &sh) {
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const gse_row &P = ds->P;
  const float M = ds->M;
  const uint64_t K = P.top_k > 0 ? (uint64_t)P.top_k : ~0ull;
  const double top_p = P.top_p, min_p = P.min_p, u = ds->u;
  uint64_t c[BPT], mh[BPT], mo[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    c[j] = ld_ag(&gh[tid * BPT + j]);
    mh[j] = ld_ag(&gh[DNB + tid * BPT + j]);
    mo[j] = ld_ag(&gh[2 * DNB + tid * BPT + j]);
  }
  // min-p keeps exp(z - M) >= min_p, i.e. d <= -ln(min_p): bins below bm - 1 are all kept, bins above bm + 1 all cut
  const bool mp = min_p > 0.0;
  uint32_t bm = 0;
  if (mp) {
    const double dm = -log(min_p) * (double)BSC;
    bm = dm >= (double)(DNB - 1) ? (uint32_t)(DNB - 1) : (uint32_t)dm;
  }
  // inclusive prefixes through each bin: counts, exact masses (2^-40 and 2^-64 parts) and their fp64 values
  uint64_t cl = 0, hl = 0, ol = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    cl += c[j];
    hl += mh[j];
    ol += mo[j];
  }
  const uint64_t ci = wave_incl_scan_u64(cl), hi = wave_incl_scan_u64(hl), oi = wave_incl_scan_u64(ol);
  if (lane == WAVE - 1) {
    sh.wt[0][w] = ci;
    sh.wt[1][w] = hi;
    sh.wt[2][w] = oi;
  }
  if (tid < PQ_N) sh.q[tid] = (tid == PQ_B5) ? 0u : (uint32_t)(DNB - 1);
  __syncthreads();
  uint64_t bc = 0, bh = 0, bo = 0, ctot = 0, htot = 0, otot = 0;
#pragma unroll
  for (int k = 0; k < NWV; ++k) {
    const uint64_t x0 = sh.wt[0][k], x1 = sh.wt[1][k], x2 = sh.wt[2][k];
    if (k < w) {
      bc += x0;
      bh += x1;
      bo += x2;
    }
    ctot += x0;
    htot += x1;
    otot += x2;
  }
  uint64_t pc[BPT];
  double pm[BPT];
  {
    uint64_t rc = bc + ci - cl, rh = bh + hi - hl, ro = bo + oi - ol;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      rc += c[j];
      rh += mh[j];
      ro += mo[j];
      pc[j] = rc;
      pm[j] = fx_val(Fx{rh, ro});
      sh.pc[tid * BPT + j] = (uint32_t)rc;
      sh.ph[tid * BPT + j] = rh;
      sh.po[tid * BPT + j] = ro;
    }
  }
  const double S = fx_val(Fx{htot, otot});
  // the masses are exact; the margin covers the fp64 roundings of their values here (the finish decides exactly)
  const double delta = 1e-12 * S;
  const double tS = top_p * S;
  // the windows of the cuts:
  //   b0, b1: first bins with inclusive mass >= tS - delta, >= tS + delta (top-p: the bin of the last kept element)
  //   b2:     first bin with inclusive count >= K (top-k: the bin of rank K - 1)
  //   b5 - 1: last non-empty bin below bm - 1 (min-p: holds a kept element, so the last kept one is at or after it)
  //   b6:     first non-empty bin above bm + 1 (min-p: holds a cut element)
  {
    uint32_t b0 = DNB - 1, b1 = DNB - 1, b2 = DNB - 1, b5 = 0, b6 = DNB - 1;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      const uint32_t b = tid * BPT + j;
      if (pm[j] >= tS - delta) b0 = b;
      if (pm[j] >= tS + delta) b1 = b;
      if (pc[j] >= K) b2 = b;
      if (mp && c[j] && b > bm + 1) b6 = b;
    }
    if (mp) {
#pragma unroll
      for (int j = 0; j < BPT; ++j) {
        const uint32_t b = tid * BPT + j;
        if (c[j] && b + 1 < bm) b5 = b + 1;
      }
    }
    b0 = wave_min_u32(b0);
    b1 = wave_min_u32(b1);
    b2 = wave_min_u32(b2);
    b5 = wave_max_u32(b5);
    b6 = wave_min_u32(b6);
    if (lane == 0) {
      atomicMin(&sh.q[PQ_B0], b0);
      atomicMin(&sh.q[PQ_B1], b1);
      atomicMin(&sh.q[PQ_B2], b2);
      atomicMax(&sh.q[PQ_B5], b5);
      atomicMin(&sh.q[PQ_B6], b6);
    }
  }
  __syncthreads();
  uint32_t w1lo = sh.q[PQ_B0], w1hi = sh.q[PQ_B1];
  if (K < ctot) {
    w1lo = min(w1lo, sh.q[PQ_B2]);
    w1hi = min(w1hi, sh.q[PQ_B2]);
  }
  if (mp) {
    const uint32_t b5 = sh.q[PQ_B5], lo = b5 ? b5 - 1u : 0u, hi = sh.q[PQ_B6];
    w1lo = min(w1lo, lo);
    // when min-p may bind, the window reaches its first cut element (the finish cannot test min-p unlisted)
    w1hi = lo <= w1hi ? max(w1hi, min(hi, (uint32_t)(DNB - 1))) : min(w1hi, hi);
  }
  auto at = [&](const auto *t, int b) { return b < 0 ? decltype(t[0])(0) : t[b]; };
  // masses before w1lo and through w1hi, then the windows of the draw
  uint32_t w2lo = w1lo, w2hi = w1hi;
  if (mode == MODE_SAMPLE) {
    const double qd0 = fx_val(Fx{at(sh.ph, (int)w1lo - 1), at(sh.po, (int)w1lo - 1)});  // (pm of those bins)
    const double qd1 = fx_val(Fx{at(sh.ph, (int)w1hi), at(sh.po, (int)w1hi)});
    const double tlo = u * (qd0 - delta) - delta, thi = u * (qd1 + delta) + delta;
    uint32_t b3 = DNB - 1, b4 = DNB - 1;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      if (pm[j] >= tlo) b3 = tid * BPT + j;
      if (pm[j] >= thi) b4 = tid * BPT + j;
    }
    b3 = wave_min_u32(b3);
    b4 = wave_min_u32(b4);
    if (lane == 0) {
      atomicMin(&sh.q[PQ_B3], b3);
      atomicMin(&sh.q[PQ_B4], b4);
    }
    __syncthreads();
    w2hi = min(sh.q[PQ_B4], w1hi);
    w2lo = min(sh.q[PQ_B3], w2hi);
  }
  if (w2hi + 1 >= w1lo) {  // touching or overlapping windows: one window
    w2lo = min(w2lo, w1lo);
    w2hi = max(w2hi, w1hi);
    w1lo = w2lo;
    w1hi = w2hi;
  }
  if (tid == 0) {
    // the regions outside the windows from the prefixes at their edges: before the draw window (0), between the
    // windows (1), after the cut window (counts), and the rest of the mass (2)
    const bool sep = w1lo > w2hi + 1;
    const uint64_t n0 = at(sh.pc, (int)w2lo - 1);
    const uint64_t n1 = sep ? (uint64_t)(at(sh.pc, (int)w1lo - 1) - at(sh.pc, (int)w2hi)) : 0ull;
    const uint64_t n2 = ctot - at(sh.pc, (int)w1hi);
    const uint64_t inw = ctot - n0 - n1 - n2;
    const uint64_t x0h = at(sh.ph, (int)w2lo - 1), x0o = at(sh.po, (int)w2lo - 1);
    const uint64_t x1h = sep ? at(sh.ph, (int)w1lo - 1) - at(sh.ph, (int)w2hi) : 0ull;
    const uint64_t x1o = sep ? at(sh.po, (int)w1lo - 1) - at(sh.po, (int)w2hi) : 0ull;
    const uint64_t xm[6] = {x0h, x0o, x1h, x1o, htot - x0h - x1h, otot - x0o - x1o};
    const uint32_t status =
        (inw > 0 && inw <= (uint64_t)DCAP && S > 0.0 && fabsf(M) < INFINITY) ? DS_PLANNED : DS_FAIL;
    // the region counts and sums (read by the finish, which comes after this workgroup's pick ticket and so after
    // these stores), then the status and windows in one word, which the row's pick slices wait for
    st_ag(&ds->acc[DA_C0], n0);  // (the element counts of the regions the pick pass sums without listing)
    st_ag(&ds->acc[DA_C1], n1);
    st_ag(&ds->acc[DA_C2], n2);
    for (int k = 0; k < 6; ++k) st_ag(&ds->acc[DA_X0HI + k], xm[k]);
    st_ag(&ds->plan, plan_word(status, w2lo, w2hi, w1lo, w1hi));
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// Pass 2: exact masses, window list, finish.

// ---- finish ---------------------------------------------------------------------------------------------------------
// The window entries are not sorted as a whole: an exact sub-histogram over their keys (per window, 128 sub-bins of
// equal key width; counts and fixed-point masses, order-independent) gives the rank and exclusive prefix at the head of
// every sub-bin. The keep cut lies in the last non-empty sub-bin before the first one whose head is cut (s0); the draw
// in the first sub-bin whose inclusive prefix reaches u * c_last (sj). Only the entries of those two sub-bins are
// sorted; their exact prefixes come from one scan of their fixed-point masses.

constexpr int NSB = 256;        // sub-bins (128 per window)
constexpr int SUBC = 2048;      // entries of one sub-bin that can be collected
constexpr int SW = SUBC / MT;   // sorted entries per thread in the walks
constexpr int LC = 2048;        // window entries the finish copies into LDS (the rest it reads from the list)
static_assert(LC <= DCAP && LC % MT == 0, "");
constexpr uint32_t NONE = 0xFFFFFFFFu;

struct FinShared {
  alignas(16) uint64_t lc[LC];  // the first LC window entries (16-byte aligned: pairs are read as one)
  uint64_t sub[SUBC];           // the collected entries of one sub-bin, sorted
  uint32_t scnt[NSB];           // sub-bin counts, then their exclusive prefix
  uint32_t stop[NSB];           // sub-bin head keys (largest key)
  uint64_t shi[NSB], slo[NSB];  // sub-bin masses
  uint32_t kmax[2], kmin[2];
  uint32_t q[4];
  uint32_t ns;
  uint64_t wred[NWV], wred2[NWV];
  uint32_t wsum[NWV];
  uint64_t pub[8];
  uint64_t acc[DA_N];           // the sorted finish: the plan's sums and counts
};

// Set by the finish's thread 0 when it has written the row's result (cleared by the same thread before the finish);
// a row without it goes to the exact path, in the same workgroup.
__shared__ uint32_t g_fin;

// Exclusive prefix of two u64 values per thread, in thread order; ta, tb receive the totals.
__device__ __forceinline__ void excl_scan2(uint64_t &a, uint64_t &b, uint64_t &ta, uint64_t &tb, FinShared &sh) {
  const uint64_t ia = wave_incl_scan_u64(a), ib = wave_incl_scan_u64(b);
  __syncthreads();
  if (lane_id() == WAVE - 1) {
    sh.wred[threadIdx.x >> 6] = ia;
    sh.wred2[threadIdx.x >> 6] = ib;
  }
  __syncthreads();
  uint64_t pa = 0, pb = 0, sa = 0, sb = 0;
  const int w = threadIdx.x >> 6;
  for (int k = 0; k < NWV; ++k) {
    pa += k < w ? sh.wred[k] : 0ull;
    pb += k < w ? sh.wred2[k] : 0ull;
    sa += sh.wred[k];
    sb += sh.wred2[k];
  }
  a = pa + ia - a;
  b = pb + ib - b;
  ta = sa;
  tb = sb;
  __syncthreads();
}

// Sorts sh.sub[0, n) descending (bitonic over the next power of two, zero padded). Rolled loops: it runs once per
// row, cold, so its code is kept small.
__device__ __forceinline__ void sort_sub(int n, FinShared &sh) {
  const int tid = threadIdx.x;
  int N = 2;
  while (N < n) N <<= 1;
  for (int i = n + tid; i < N; i += MT) sh.sub[i] = 0ull;
  __syncthreads();
#pragma unroll 1
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll 1
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll 1
      for (int i = tid; i < N / 2; i += MT) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1)), hi = lo + j;
        const uint64_t x = sh.sub[lo], y = sh.sub[hi];
        if ((lo & k) == 0 ? x < y : x > y) {
          sh.sub[lo] = y;
          sh.sub[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Sub-bin of a window entry.
__device__ __forceinline__ int sub_of(uint32_t k, const uint32_t (&shift)[2], bool sep, uint32_t w1lo, float Mf,
                                      const FinShared &sh) {
  const int g = (sep && dbin(fkey_inv(k), Mf) >= w1lo) ? 1 : 0;
  return g * (NSB / 2) + (int)min((sh.kmax[g] - k) >> shift[g], (uint32_t)(NSB / 2 - 1));
}

__device__ __forceinline__ Fx mass_of(uint32_t key, double M, const double *etab) {
  return fx_of(exp_nonpos((double)fkey_inv(key) - M, etab));
}

// What the finish uses of the launch arguments (by value: the kernel keeps its arguments in registers).
struct FinArgs {
  const uint64_t *lst;  // the row's window list
  RowInfo *info;
  int32_t *tokens;
  int mode;
};

// (not inlined: its registers are allocated apart from the streaming code of the pick pass)
__device__ __noinline__ void finish_row(const FinArgs a, DeepSlot *ds, FinShared &sh, const double *etab) {
  const int tid = threadIdx.x;
  const gse_row &P = ds->P;
  const int row = ds->row;
  const float Mf = ds->M;
  const double M = (double)Mf;
  const uint64_t pw = ld_ag(&ds->plan);
  const uint32_t w2hi = plan_win(pw, 1), w1lo = plan_win(pw, 2);
  const bool sep = w1lo > w2hi;  // an unlisted gap (region 1) between the draw window and the cut window
  const Fx X0{ld_ag(&ds->acc[DA_X0HI]), ld_ag(&ds->acc[DA_X0LO])}, X1{ld_ag(&ds->acc[DA_X1HI]), ld_ag(&ds->acc[DA_X1LO])};
  const Fx SF = fx_add(fx_add(X0, X1), Fx{ld_ag(&ds->acc[DA_RHI]), ld_ag(&ds->acc[DA_RLO])});
  const uint64_t c0 = ld_ag(&ds->acc[DA_C0]), c1 = ld_ag(&ds->acc[DA_C1]), tail = ld_ag(&ds->acc[DA_C2]);
  const uint32_t nraw = ld_ag(&ds->lcnt);
  const double Sd = fx_val(SF);
  const uint64_t K = P.top_k > 0 ? (uint64_t)P.top_k : ~0ull;
  const double topp = P.top_p, minp = P.min_p, q0 = 1.0 / Sd;
  const bool ok0 = nraw > 0 && nraw <= (uint32_t)DCAP && Sd > 0.0;
  const int n = ok0 ? (int)nraw : 0;
  const uint64_t *lst = a.lst;
  const uint64_t cmax = a.info[row].cmax;  // (written by the main pass; loaded now, used at the end)
  // the list's first LC entries into LDS, every load issued before the first is used (entries past n are stale and
  // never read)
  {
    uint64_t v[LC / MT];
#pragma unroll
    for (int j = 0; j < LC / MT; ++j) v[j] = ld_ag(&lst[j * MT + tid]);
#pragma unroll
    for (int j = 0; j < LC / MT; ++j) sh.lc[j * MT + tid] = v[j];
  }
  auto entry = [&](int i) -> uint64_t { return i < LC ? sh.lc[i] : ld_ag(&lst[i]); };
  // key ranges of the two windows
  if (tid < 2) {
    sh.kmax[tid] = 0;
    sh.kmin[tid] = NONE;
  }
  sh.scnt[tid] = 0;
  sh.stop[tid] = 0;
  sh.shi[tid] = 0;
  sh.slo[tid] = 0;
  __syncthreads();
  {
    uint32_t kx[2] = {0u, 0u}, kn[2] = {NONE, NONE};
    for (int i = tid; i < n; i += MT) {
      const uint32_t k = pk_key(entry(i));
      const int g = (sep && dbin(fkey_inv(k), Mf) >= w1lo) ? 1 : 0;
      kx[g] = max(kx[g], k);
      kn[g] = min(kn[g], k);
    }
    for (int g = 0; g < 2; ++g) {  // (one LDS atomic per wave)
      kx[g] = wave_max_u32(kx[g]);
      kn[g] = wave_min_u32(kn[g]);
      if (lane_id() == 0) {
        atomicMax(&sh.kmax[g], kx[g]);
        atomicMin(&sh.kmin[g], kn[g]);
      }
    }
  }
  __syncthreads();
  uint32_t shift[2];
  for (int g = 0; g < 2; ++g) {
    const uint32_t span = sh.kmax[g] >= sh.kmin[g] ? sh.kmax[g] - sh.kmin[g] : 0u;
    uint32_t sft = 0;
    while (sft < 31 && (span >> sft) >= (uint32_t)(NSB / 2)) ++sft;
    shift[g] = sft;
  }
  // exact sub-bin counts, masses and head keys
  for (int i = tid; i < n; i += MT) {
    const uint32_t k = pk_key(entry(i));
    const int b = sub_of(k, shift, sep, w1lo, Mf, sh);
    const Fx f = mass_of(k, M, etab);
    atomicAdd(&sh.scnt[b], 1u);
    atomicMax(&sh.stop[b], k);
    atomicAdd((unsigned long long *)&sh.shi[b], (unsigned long long)f.hi);
    atomicAdd((unsigned long long *)&sh.slo[b], (unsigned long long)f.lo);
  }
  __syncthreads();
  // exclusive prefix over sub-bins (thread t = sub-bin t, in key order): rank and mass at each sub-bin head
  const uint32_t mycnt = sh.scnt[tid], mytop = sh.stop[tid];
  const Fx mym{sh.shi[tid], sh.slo[tid]};
  uint64_t ph = mym.hi, pl = mym.lo;
  {
    uint64_t th, tl;
    const uint32_t ic = wave_incl_scan_u32(mycnt);
    if (lane_id() == WAVE - 1) sh.wsum[tid >> 6] = ic;
    excl_scan2(ph, pl, th, tl, sh);  // (its barriers publish wsum)
    uint32_t pc = 0;
    for (int k = 0; k < NWV; ++k) pc += k < (tid >> 6) ? sh.wsum[k] : 0u;
    sh.scnt[tid] = pc + ic - mycnt;  // (now the exclusive count prefix)
  }
  const bool seg1 = sep && tid >= NSB / 2;
  const Fx pbase = fx_add(fx_add(X0, Fx{ph, pl}), seg1 ? X1 : Fx{0, 0});
  const uint64_t rbase = c0 + sh.scnt[tid] + (seg1 ? c1 : 0ull);
  if (tid < 4) sh.q[tid] = tid == 1 ? 0u : NONE;
  __syncthreads();
  // s1: the first non-empty sub-bin whose head entry is cut
  if (ok0 && mycnt) {
    const Fx f0 = mass_of(mytop, M, etab);
    const bool cut = rbase >= K || (minp > 0.0 && !(fx_val(f0) / Sd >= minp * q0)) || fx_val(pbase) / Sd >= topp;
    if (cut) atomicMin(&sh.q[0], (uint32_t)tid);
  }
  __syncthreads();
  const uint32_t s1 = sh.q[0];
  // s0: the last non-empty sub-bin before s1 (it holds the last kept entry)
  if (ok0 && mycnt && (uint32_t)tid < s1) atomicMax(&sh.q[1], (uint32_t)tid + 1u);
  __syncthreads();
  const int s0 = (int)sh.q[1] - 1;
  if (ok0 && s0 >= 0 && tid == s0) {
    sh.pub[0] = rbase;
    sh.pub[1] = pbase.hi;
    sh.pub[2] = pbase.lo;
    sh.pub[3] = mycnt;
    sh.pub[4] = seg1 ? 1u : 0u;
  }
  if (ok0 && s1 != NONE && tid == (int)s1) sh.pub[5] = rbase;
  __syncthreads();
  bool ok = ok0 && s0 >= 0;
  const uint64_t r_s1 = sh.pub[5];
  const bool g0 = sh.pub[4] != 0;
  // Two walks over the sorted entries of one sub-bin, with exact prefixes: walk 0 finds the first cut entry of s0 (the
  // last kept entry is the one before it, c_last its inclusive prefix), walk 1 the first entry of sj whose inclusive
  // prefix reaches u * c_last (the token).
  uint64_t r0 = sh.pub[0];
  Fx base{sh.pub[1], sh.pub[2]};
  uint32_t cnt = (uint32_t)sh.pub[3];
  int sb = s0;
  double clast = 0.0, thr = 0.0;
  uint64_t kkeep = 0;
  int32_t tok = -1;
#pragma unroll 1
  for (int w = 0; w < 2 && ok; ++w) {
    if (w == 1) {
      if (a.mode != MODE_SAMPLE) break;
      // sj: the first non-empty sub-bin whose inclusive prefix reaches u * c_last; its head's exclusive prefix must be
      // below it (else the draw falls in an unlisted region)
      thr = ds->u * clast;
      if (mycnt && fx_val(fx_add(pbase, mym)) / Sd >= thr) atomicMin(&sh.q[2], (uint32_t)tid);
      __syncthreads();
      const uint32_t sj = sh.q[2];
      if (sj != NONE && tid == (int)sj) {
        sh.pub[0] = pbase.hi;
        sh.pub[1] = pbase.lo;
        sh.pub[3] = mycnt;
      }
      __syncthreads();
      base = Fx{sh.pub[0], sh.pub[1]};
      cnt = (uint32_t)sh.pub[3];
      ok = sj != NONE && !(fx_val(base) / Sd >= thr);
      if (!ok) break;
      sb = (int)sj;
    }
    // collect the sub-bin's entries (in list order) and sort them
    if (cnt > (uint32_t)SUBC) {
      ok = false;
      break;
    }
    if (tid == 0) sh.ns = 0;
    __syncthreads();
    for (int i = tid; i < n; i += MT) {
      const uint64_t pk = entry(i);
      if (sub_of(pk_key(pk), shift, sep, w1lo, Mf, sh) == sb) {
        const uint32_t pos = atomicAdd(&sh.ns, 1u);
        if (pos < (uint32_t)SUBC) sh.sub[pos] = pk;
      }
    }
    __syncthreads();
    if (sh.ns != cnt) {
      ok = false;
      break;
    }
    const int m = (int)cnt;
    sort_sub(m, sh);
    // exclusive prefix at entry tid * SW, then the first entry that meets the walk's test
    uint64_t hi = 0, lo = 0, thi, tlo;
#pragma unroll 1
    for (int i = 0; i < SW; ++i) {
      const int k = tid * SW + i;
      if (k < m) {
        const Fx f = mass_of(pk_key(sh.sub[k]), M, etab);
        hi += f.hi;
        lo += f.lo;
      }
    }
    excl_scan2(hi, lo, thi, tlo, sh);
    if (tid == 0) sh.q[3] = NONE;
    __syncthreads();
    Fx A = fx_add(base, Fx{hi, lo});
    uint32_t kc = NONE;
#pragma unroll 1
    for (int i = 0; i < SW; ++i) {
      const int k = tid * SW + i;
      if (k >= m) break;
      const Fx f = mass_of(pk_key(sh.sub[k]), M, etab);
      const Fx Ai = fx_add(A, f);
      const bool hit = w == 0 ? (r0 + (uint64_t)k >= K || (minp > 0.0 && !(fx_val(f) / Sd >= minp * q0)) ||
                                 fx_val(A) / Sd >= topp)
                              : fx_val(Ai) / Sd >= thr;
      if (hit) {
        kc = (uint32_t)k;
        break;
      }
      A = Ai;
    }
    kc = wave_min_u32(kc);
    if (lane_id() == 0 && kc != NONE) atomicMin(&sh.q[3], kc);
    __syncthreads();
    kc = sh.q[3];
    if (w == 1) {
      ok = kc != NONE;
      if (ok) tok = (int32_t)pk_id(sh.sub[kc]);
      break;
    }
    // walk 0: the last kept entry and its inclusive prefix (the exclusive prefix of the first cut entry, or the
    // sub-bin's total)
    const bool inside = kc != NONE;
    const int last = inside ? (int)kc - 1 : m - 1;
    if (inside && tid == (int)(kc / SW)) {
      sh.pub[6] = A.hi;  // (the thread stopped at kc: A is its exclusive prefix)
      sh.pub[7] = A.lo;
    }
    __syncthreads();
    const Fx Al = inside ? Fx{sh.pub[6], sh.pub[7]} : fx_add(base, Fx{thi, tlo});
    bool good = last >= 0;
    if (good && !inside) {
      // the next rank is s1's head (cut by definition) when directly adjacent, else past the list
      const uint64_t rl = r0 + (uint64_t)last;
      if (s1 != NONE) {
        good = r_s1 == rl + 1;
      } else {
        const uint64_t after = (!sep || g0) ? tail : c1 + tail;
        good = after == 0 || rl + 1 >= K || fx_val(Al) / Sd >= topp;
      }
    }
    ok = good;
    if (ok) {
      clast = fx_val(Al) / Sd;
      kkeep = sh.sub[last];
    }
    __syncthreads();  // (sh.pub, sh.sub before walk 1)
  }
  if (tid == 0 && ok) {
    RowInfo *ri = a.info + row;
    RowInfo r = {};
    r.cmax = cmax;
    r.kkeep = kkeep;
    r.S = Sd;
    r.Z = clast;
    r.flags = R_DONE | R_BY_DEEP;
    r.token = tok;
    *ri = r;
    g_fin = 1u;
    if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
  }
}

// The finish of a window list of at most LC entries, sorted whole. The entries stay in registers (SP per thread) and
// are ranked with a counting sort: FB key buckets per window (the draw window's entries rank above the cut window's),
// an atomic slot in its bucket for every entry, the buckets' starts, a scatter into bucket order, and the rank inside
// the bucket by counting its greater members (buckets hold a few entries). Every entry's exact mass then goes to its
// rank, one exclusive scan in rank order (thread t: ranks [SP t, SP t + SP)) gives every prefix, and the keep cut (the
// first entry not kept) and the draw (the first entry whose inclusive prefix reaches u c_last) are one test per rank
// and one block minimum each. The unlisted region between the windows (X1, c1 elements) counts before the cut
// window's entries. The tests and fixed-point sums are finish_row's; a failed check leaves the row to the exact path.
constexpr int FB = 1024;  // key buckets per window
static_assert(2 * 2 * FB * sizeof(uint32_t) <= SUBC * sizeof(uint64_t), "bucket counts and starts live in sub");
static_assert(SUBC >= LC, "masses by rank live in sub");

__device__ __forceinline__ uint64_t rl64(uint64_t x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
  return (uint64_t)hi << 32 | lo;
}

// The least x >= 0 with RN(x / S) >= t, for finite S > 0 and t >= 0: RN(x / S) is non-decreasing in x, so a test
// RN(x / S) >= t reads x >= that least x, one comparison in place of a division per element. It lies within an ulp or
// two of RN(t S): lane i of the wave (i < 16) tests RN(t S) + (i - 8) ulps, all at once, and the first lane whose
// test holds gives it. ok turns false when the 16 candidates do not bracket it (the row then goes to the exact path).
// Every lane of the wave must call it.
__device__ __forceinline__ double least_ge(double t, double S, bool &ok) {
  const double x0 = t * S;
  const int i = lane_id() & 15;
  const long long b0 = __double_as_longlong(x0) + (long long)(i - 8);
  const double x = b0 > 0 ? __longlong_as_double(b0) : 0.0;
  const uint64_t m = ballot64(lane_id() < 16 && x / S >= t);
  const bool fin = x0 >= 0.0 && x0 < INFINITY;
  // the first candidate that holds; candidate 0 only when it is 0 (nothing lies below)
  const int f = m ? (int)__builtin_ctzll(m) : 16;
  const double xf = __longlong_as_double((long long)rl64((uint64_t)__double_as_longlong(x), f & 15));
  ok = ok && fin && f < 16 && (f > 0 || xf == 0.0);
  return xf;
}

// The sorted finish of a list of at most 64 entries, by wave 0 alone (no barrier): lane l holds entry l; its rank is
// the count of greater entries (read back from LDS, wave-local), the entries return to LDS in rank order, and lane r
// takes rank r. The prefix sums are one wave scan, the cut and the draw one ballot each; the tests are finish_row's.
// acc: lane i holds the plan's acc[i].
__device__ __forceinline__ void finish_wave(const FinArgs a, DeepSlot *ds, FinShared &sh, const double *etab, int n,
                                         uint64_t e, uint64_t accv, int row, float Mf, double u, uint64_t K,
                                         double topp, double minp, bool sep, uint32_t w1lo) {
  const int l = lane_id();
  const bool val = l < n;
  const double M = (double)Mf;
  const bool g1o = val && sep && dbin(fkey_inv(pk_key(e)), Mf) >= w1lo;
  const uint32_t n0 = (uint32_t)__popcll(ballot64(val && !g1o));  // entries of the draw window (they rank first)
  if (val) sh.lc[l] = e;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint32_t r = 0;
  {
    int m = 0;
#pragma unroll 1
    for (; m + 2 <= n; m += 2) r += (sh.lc[m] > e ? 1u : 0u) + (sh.lc[m + 1] > e ? 1u : 0u);
    if (m < n) r += sh.lc[m] > e ? 1u : 0u;
  }
  if (val) sh.sub[r] = e;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint64_t es = val ? sh.sub[l] : 0ull;  // rank l
  const Fx f = val ? fx_of(exp_nonpos((double)fkey_inv(pk_key(es)) - M, etab)) : Fx{0, 0};
  const Fx X0{rl64(accv, DA_X0HI), rl64(accv, DA_X0LO)}, X1{rl64(accv, DA_X1HI), rl64(accv, DA_X1LO)};
  const Fx SF = fx_add(fx_add(X0, X1), Fx{rl64(accv, DA_RHI), rl64(accv, DA_RLO)});
  const uint64_t c0 = rl64(accv, DA_C0), c1 = rl64(accv, DA_C1), tail = rl64(accv, DA_C2);
  const double Sd = fx_val(SF), q0 = 1.0 / Sd;
  bool okd = Sd > 0.0 && Sd < INFINITY;  // (x / Sd >= t reads x >= least_ge(t, Sd))
  const double ap = least_ge(topp, Sd, okd), am = minp > 0.0 ? least_ge(minp * q0, Sd, okd) : 0.0;
  const uint64_t ih = wave_incl_scan_u64(f.hi), il = wave_incl_scan_u64(f.lo);
  const bool g1 = (uint32_t)l >= n0;
  const Fx Ar = fx_add(fx_add(X0, Fx{ih - f.hi, il - f.lo}), g1 ? X1 : Fx{0, 0});  // exclusive prefix of rank l
  // the first entry that is not kept (sampling.py:80, with min-p)
  const bool cut = val && ((c0 + (uint64_t)l + (g1 ? c1 : 0ull) >= K) | (minp > 0.0 && !(fx_val(f) >= am)) |
                           (fx_val(Ar) >= ap));
  const uint64_t cb = ballot64(cut);
  const int fc = cb ? (int)__builtin_ctzll(cb) : -1;
  const int last = fc >= 0 ? fc - 1 : n - 1;  // the last kept entry
  const bool glast = last >= 0 && (uint32_t)last >= n0;
  bool ok = n > 0 && okd && last >= 0;
  if (!ok) return;
  Fx Al;  // c_last, unnormalized
  if (fc >= 0) {
    Al = Fx{rl64(Ar.hi, fc), rl64(Ar.lo, fc)};
    ok = !((uint32_t)fc >= n0 && !glast && c1 > 0);  // (the first cut entry right after the gap: the cut may be inside it)
  } else {
    Al = fx_add(fx_add(X0, Fx{rl64(ih, n - 1), rl64(il, n - 1)}), glast ? X1 : Fx{0, 0});
    const uint64_t rl = c0 + (uint64_t)last + (glast ? c1 : 0ull);
    const uint64_t after = (!sep || glast) ? tail : c1 + tail;  // unlisted elements ranked after the list
    ok = after == 0 || rl + 1 >= K || fx_val(Al) / Sd >= topp;
  }
  const double clast = fx_val(Al) / Sd;
  int32_t tok = -1;
  if (ok && a.mode == MODE_SAMPLE) {
    // the draw: the first kept entry whose inclusive prefix reaches u c_last; its exclusive prefix must lie below it
    const double at = least_ge(u * clast, Sd, ok);
    const uint64_t hb = ballot64(l <= last && fx_val(fx_add(Ar, f)) >= at);
    const uint64_t bb = ballot64(!(fx_val(Ar) >= at));
    ok = ok && hb != 0;
    if (ok) {
      const int fj = (int)__builtin_ctzll(hb);
      ok = ((bb >> fj) & 1ull) != 0;
      tok = (int32_t)pk_id(rl64(es, fj));
    }
  }
  const uint64_t kkeep = rl64(es, last);
  if (l == 0 && ok) {  // (the main pass's cmax stays)
    RowInfo *ri = a.info + row;
    ri->kkeep = kkeep;
    ri->S = Sd;
    ri->Z = clast;
    ri->flags = R_DONE | R_BY_DEEP;
    ri->ncert = 0;
    ri->token = tok;
    if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
    g_fin = 1u;
  }
}

// Longest list the block finish takes (its ranking pass grows with the list; the bucketed finish below is as fast
// from about 200 entries on: C3 lists of 87-150 entries 8.7-10.8 -> 6.0-7.6 us, of about 230 entries 9-10 us either way).
constexpr int FBN = 192;
static_assert(FBN <= MT, "");

// The sorted finish of a list of at most FBN entries (finish_wave's steps, a workgroup wide): thread t holds entry t,
// ranks it by the count of greater entries (a pass over the list in LDS), and then holds rank t; one block scan of the
// fixed-point masses gives every rank's exclusive prefix, and the cut and the draw are block minima. Five barriers.
__device__ __forceinline__ void finish_block(const FinArgs a, DeepSlot *ds, FinShared &sh, const double *etab, int n,
                                          uint64_t e, int row, float Mf, double u, uint64_t K, double topp,
                                          double minp, bool sep, uint32_t w1lo) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6;
  const bool val = tid < n;
  const double M = (double)Mf;
  const bool g1o = val && sep && dbin(fkey_inv(pk_key(e)), Mf) >= w1lo;
  if (val) sh.lc[tid] = e;
  const uint64_t dw = ballot64(val && !g1o);  // (every lane takes part in the ballot)
  if (l == 0) sh.wsum[w] = (uint32_t)__popcll(dw);
  if (tid < 2) sh.q[tid] = NONE;
  __syncthreads();  // 1: the list, the draw window's counts
  uint32_t n0 = 0;
#pragma unroll
  for (int k = 0; k < NWV; ++k) n0 += sh.wsum[k];  // entries of the draw window (they rank first)
  if (val) {  // (entries past n in lc are stale: the pairs loop reads whole pairs below n only)
    uint32_t r = 0;
    int m = 0;
    const ulonglong2 *lp = reinterpret_cast<const ulonglong2 *>(sh.lc);
#pragma unroll 1
    for (; m + 4 <= n; m += 4) {
      const ulonglong2 p = lp[m >> 1], q = lp[(m >> 1) + 1];
      r += (p.x > e ? 1u : 0u) + (p.y > e ? 1u : 0u) + (q.x > e ? 1u : 0u) + (q.y > e ? 1u : 0u);
    }
#pragma unroll 1
    for (; m < n; ++m) r += sh.lc[m] > e ? 1u : 0u;
    sh.sub[r] = e;
  }
  __syncthreads();  // 2: the entries in rank order
  const uint64_t es = val ? sh.sub[tid] : 0ull;  // rank tid
  const Fx f = val ? fx_of(exp_nonpos((double)fkey_inv(pk_key(es)) - M, etab)) : Fx{0, 0};
  const Fx X0{sh.acc[DA_X0HI], sh.acc[DA_X0LO]}, X1{sh.acc[DA_X1HI], sh.acc[DA_X1LO]};
  const Fx SF = fx_add(fx_add(X0, X1), Fx{sh.acc[DA_RHI], sh.acc[DA_RLO]});
  const uint64_t c0 = sh.acc[DA_C0], c1 = sh.acc[DA_C1], tail = sh.acc[DA_C2];
  const double Sd = fx_val(SF), q0 = 1.0 / Sd;
  bool okd = Sd > 0.0 && Sd < INFINITY;  // (x / Sd >= t reads x >= least_ge(t, Sd))
  const double ap = least_ge(topp, Sd, okd), am = minp > 0.0 ? least_ge(minp * q0, Sd, okd) : 0.0;
  // exclusive prefix of rank tid: the wave scan, then the earlier waves' totals
  const uint64_t ih = wave_incl_scan_u64(f.hi), il = wave_incl_scan_u64(f.lo);
  if (l == WAVE - 1) {
    sh.wred[w] = ih;
    sh.wred2[w] = il;
  }
  __syncthreads();  // 3: the wave totals
  uint64_t ph = ih - f.hi, pl = il - f.lo, th = 0, tl = 0;
#pragma unroll
  for (int k = 0; k < NWV; ++k) {
    ph += k < w ? sh.wred[k] : 0ull;
    pl += k < w ? sh.wred2[k] : 0ull;
    th += sh.wred[k];
    tl += sh.wred2[k];
  }
  const bool g1 = (uint32_t)tid >= n0;
  const Fx Ar = fx_add(fx_add(X0, Fx{ph, pl}), g1 ? X1 : Fx{0, 0});
  // the first entry that is not kept (sampling.py:80, with min-p); it publishes its exclusive prefix
  const bool cut = val && ((c0 + (uint64_t)tid + (g1 ? c1 : 0ull) >= K) | (minp > 0.0 && !(fx_val(f) >= am)) |
                           (fx_val(Ar) >= ap));
  if (cut) {
    sh.shi[tid] = Ar.hi;
    sh.slo[tid] = Ar.lo;
  }
  {
    const uint64_t cb = ballot64(cut);
    if (l == 0 && cb) atomicMin(&sh.q[0], (uint32_t)(w * WAVE + (int)__builtin_ctzll(cb)));
  }
  __syncthreads();  // 4: the first cut
  const uint32_t fc = sh.q[0];
  const int last = fc == NONE ? n - 1 : (int)fc - 1;  // the last kept entry
  const bool glast = last >= 0 && (uint32_t)last >= n0;
  bool ok = n > 0 && okd && last >= 0;
  Fx Al{0, 0};  // c_last, unnormalized
  if (fc != NONE) {
    Al = Fx{sh.shi[fc], sh.slo[fc]};
    ok = ok && !(fc >= n0 && !glast && c1 > 0);  // (the first cut entry right after the gap: the cut may be inside it)
  } else {
    Al = fx_add(fx_add(X0, Fx{th, tl}), glast ? X1 : Fx{0, 0});
    const uint64_t rl = c0 + (uint64_t)last + (glast ? c1 : 0ull);
    const uint64_t after = (!sep || glast) ? tail : c1 + tail;  // unlisted elements ranked after the list
    ok = ok && (after == 0 || rl + 1 >= K || fx_val(Al) / Sd >= topp);
  }
  const double clast = fx_val(Al) / Sd;
  if (ok && a.mode == MODE_SAMPLE) {
    // the draw: the first kept entry whose inclusive prefix reaches u c_last; its exclusive prefix must lie below it.
    // Packed as rank << 1 | (not below).
    bool okt = true;
    const double at = least_ge(u * clast, Sd, okt);  // (the same value in every thread)
    const bool hit = tid <= last && fx_val(fx_add(Ar, f)) >= at, below = !(fx_val(Ar) >= at);
    uint32_t fj = hit ? (uint32_t)tid << 1 | (below ? 0u : 1u) : NONE;
    fj = wave_min_u32(fj);
    if (l == 0 && fj != NONE) atomicMin(&sh.q[1], fj);
    __syncthreads();  // 5: the draw
    fj = sh.q[1];
    ok = okt && fj != NONE && (fj & 1u) == 0u;
  }
  if (tid == 0 && ok) {  // (the main pass's cmax stays)
    const int32_t tok = a.mode == MODE_SAMPLE ? (int32_t)pk_id(sh.sub[sh.q[1] >> 1]) : -1;
    RowInfo *ri = a.info + row;
    ri->kkeep = sh.sub[last];
    ri->S = Sd;
    ri->Z = clast;
    ri->flags = R_DONE | R_BY_DEEP;
    ri->ncert = 0;
    ri->token = tok;
    if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
    g_fin = 1u;
  }
}

__device__ __noinline__ int finish_sorted(const FinArgs a, DeepSlot *ds, FinShared &sh, const double *etab) {
  constexpr int SP = LC / MT;  // entries (and ranks) per thread
  const int tid = threadIdx.x, w = tid >> 6;
  // every load the finish makes, issued together: the list's first LC entries (entries past its end are stale and
  // never used), the plan's windows, sums and counts (lanes of wave 0, into LDS), the row's parameters
  const uint32_t nraw = ld_ag(&ds->lcnt), spoil = ld_ag(&ds->spoil);
  const uint64_t pw = ld_ag(&ds->plan);
  const uint32_t w2hi = plan_win(pw, 1), w1lo = plan_win(pw, 2);
  uint64_t v[SP];
#pragma unroll
  for (int j = 0; j < SP; ++j) v[j] = ld_ag(&a.lst[j * MT + tid]);
  const uint64_t accv = tid < DA_N ? ld_ag(&ds->acc[tid]) : 0ull;  // (lane i of wave 0: acc[i])
  const int row = ds->row;
  const float Mf = ds->M;
  const double M = (double)Mf, u = ds->u;
  const uint64_t K = ds->P.top_k > 0 ? (uint64_t)ds->P.top_k : ~0ull;
  const double topp = ds->P.top_p, minp = ds->P.min_p;
  if (spoil != 0u) return 0;  // (a slice gave up waiting for the plan: the exact path takes the row)
  if (nraw > (uint32_t)LC) return 1;
  const int n = (int)nraw;
  const bool sep = w1lo > w2hi;
  if (n <= WAVE) {  // one wave does it all, without a barrier
    if (tid < WAVE) finish_wave(a, ds, sh, etab, n, v[0], accv, row, Mf, u, K, topp, minp, sep, w1lo);
    return 0;
  }
  if (tid < DA_N) sh.acc[tid] = accv;  // (published by the first barrier of either path)
  if (n <= FBN) {
    finish_block(a, ds, sh, etab, n, v[0], row, Mf, u, K, topp, minp, sep, w1lo);
    return 0;
  }
  uint32_t *bcnt = reinterpret_cast<uint32_t *>(sh.sub), *bofs = bcnt + 2 * FB;
  double *msr = reinterpret_cast<double *>(sh.sub);  // (after the ranks: the masses by rank)
  for (int b = tid; b < 2 * FB; b += MT) bcnt[b] = 0;
  if (tid < 2) sh.q[tid] = NONE;
  // each entry's window and the key range of each window (per-wave ranges in wred / wred2, no atomics)
  uint32_t gm = 0, kx0 = 0, kx1 = 0, kn0 = NONE, kn1 = NONE;
#pragma unroll
  for (int j = 0; j < SP; ++j) {
    if (j * MT + tid < n) {
      const uint32_t k = pk_key(v[j]);
      if (sep && dbin(fkey_inv(k), Mf) >= w1lo) {
        gm |= 1u << j;
        kx1 = max(kx1, k);
        kn1 = min(kn1, k);
      } else {
        kx0 = max(kx0, k);
        kn0 = min(kn0, k);
      }
    }
  }
  kx0 = wave_max_u32(kx0);
  kx1 = wave_max_u32(kx1);
  kn0 = wave_min_u32(kn0);
  kn1 = wave_min_u32(kn1);
  if (lane_id() == 0) {
    sh.wred[w] = (uint64_t)kx1 << 32 | kx0;
    sh.wred2[w] = (uint64_t)kn1 << 32 | kn0;
  }
  __syncthreads();
  uint32_t top[2] = {0u, 0u}, sft[2];
  {
    uint32_t lo[2] = {NONE, NONE};
    for (int k = 0; k < NWV; ++k) {
      top[0] = max(top[0], (uint32_t)sh.wred[k]);
      top[1] = max(top[1], (uint32_t)(sh.wred[k] >> 32));
      lo[0] = min(lo[0], (uint32_t)sh.wred2[k]);
      lo[1] = min(lo[1], (uint32_t)(sh.wred2[k] >> 32));
    }
    for (int g = 0; g < 2; ++g) {
      const uint32_t span = top[g] >= lo[g] ? top[g] - lo[g] : 0u, nb = sep ? (uint32_t)FB : 2u * FB;
      uint32_t s = 0;
      while (s < 31 && (span >> s) >= nb) ++s;
      sft[g] = s;
    }
  }
  const uint32_t nb0 = sep ? (uint32_t)FB : 2u * FB;  // buckets of the draw window (all of them when one window)
  // bucket of entry j (recomputed where used: fewer registers live across the phases) and its slot in the bucket
  auto bucket = [&](int j) __attribute__((always_inline)) {
    const uint32_t k = pk_key(v[j]);
    return ((gm >> j) & 1u) ? FB + min((top[1] - k) >> sft[1], (uint32_t)(FB - 1)) : min((top[0] - k) >> sft[0], nb0 - 1u);
  };
  uint32_t sl[SP];
#pragma unroll
  for (int j = 0; j < SP; ++j) sl[j] = j * MT + tid < n ? atomicAdd(&bcnt[bucket(j)], 1u) : 0u;
  __syncthreads();
  // bucket starts: thread t owns buckets [8 t, 8 t + 8)
  {
    constexpr int BT = 2 * FB / MT;
    uint32_t c[BT], loc = 0;
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      c[j] = bcnt[tid * BT + j];
      loc += c[j];
    }
    const uint32_t inc = wave_incl_scan_u32(loc);
    if (lane_id() == WAVE - 1) sh.wsum[w] = inc;
    __syncthreads();
    uint32_t run = inc - loc;
    for (int k = 0; k < NWV; ++k) run += k < w ? sh.wsum[k] : 0u;
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      bofs[tid * BT + j] = run;
      run += c[j];
    }
  }
  __syncthreads();
  const uint32_t n0 = sep ? bofs[FB] : (uint32_t)n;  // entries of the draw window (they rank first)
#pragma unroll
  for (int j = 0; j < SP; ++j)
    if (j * MT + tid < n) sh.lc[bofs[bucket(j)] + sl[j]] = v[j];
  __syncthreads();
  // rank = bucket start + greater members of the bucket
  uint32_t rk[SP];
#pragma unroll
  for (int j = 0; j < SP; ++j) {
    rk[j] = 0;
    if (j * MT + tid < n) {
      const uint32_t bj = bucket(j), b0 = bofs[bj], b1 = b0 + bcnt[bj];
      uint32_t r = b0, q = b0;
#pragma unroll 1
      for (; q + 4 <= b1; q += 4)
        r += (sh.lc[q] > v[j] ? 1u : 0u) + (sh.lc[q + 1] > v[j] ? 1u : 0u) + (sh.lc[q + 2] > v[j] ? 1u : 0u) +
             (sh.lc[q + 3] > v[j] ? 1u : 0u);
#pragma unroll 1
      for (; q < b1; ++q) r += sh.lc[q] > v[j] ? 1u : 0u;
      rk[j] = r;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < SP; ++j) {
    if (j * MT + tid < n) {
      sh.lc[rk[j]] = v[j];
      msr[rk[j]] = exp_nonpos((double)fkey_inv(pk_key(v[j])) - M, etab);  // (the entry's exact mass)
    }
  }
  __syncthreads();
  // exclusive prefix at rank SP t (one block scan of the fixed-point masses)
  const int r0 = tid * SP;
  uint64_t hi = 0, lo = 0;
#pragma unroll
  for (int s = 0; s < SP; ++s) {
    if (r0 + s < n) {
      const Fx f = fx_of(msr[r0 + s]);
      hi += f.hi;
      lo += f.lo;
    }
  }
  const Fx X0{sh.acc[DA_X0HI], sh.acc[DA_X0LO]}, X1{sh.acc[DA_X1HI], sh.acc[DA_X1LO]};
  const Fx SF = fx_add(fx_add(X0, X1), Fx{sh.acc[DA_RHI], sh.acc[DA_RLO]});
  const uint64_t c0 = sh.acc[DA_C0], c1 = sh.acc[DA_C1], tail = sh.acc[DA_C2];
  const double Sd = fx_val(SF), q0 = 1.0 / Sd;
  bool okd = Sd > 0.0 && Sd < INFINITY;  // (x / Sd >= t reads x >= least_ge(t, Sd))
  const double ap = least_ge(topp, Sd, okd), am = minp > 0.0 ? least_ge(minp * q0, Sd, okd) : 0.0;
  uint64_t th = 0, tl = 0;  // the list's total
  {
    const uint64_t ih = wave_incl_scan_u64(hi), il = wave_incl_scan_u64(lo);
    if (lane_id() == WAVE - 1) {
      sh.wred[w] = ih;
      sh.wred2[w] = il;
    }
    __syncthreads();
    uint64_t ph = ih - hi, pl = il - lo;
    for (int k = 0; k < NWV; ++k) {
      ph += k < w ? sh.wred[k] : 0ull;
      pl += k < w ? sh.wred2[k] : 0ull;
      th += sh.wred[k];
      tl += sh.wred2[k];
    }
    hi = ph;  // (now the exclusive prefix at rank r0)
    lo = pl;
  }
  // The first entry that is not kept (sampling.py:80, with min-p); the thread holding it publishes its exclusive
  // prefix (the inclusive prefix of the last kept entry). The thread's SP tests are independent (their prefixes are
  // integer sums), so they overlap.
  {
    Fx A = fx_add(X0, Fx{hi, lo}), Ah{0, 0};
    uint32_t fc = NONE;
#pragma unroll 4
    for (int s = 0; s < SP; ++s) {
      const uint32_t r = (uint32_t)(r0 + s);
      const bool g1 = r >= n0;
      const Fx Ar = g1 ? fx_add(A, X1) : A, f = fx_of(msr[r]);
      const bool cut = (c0 + r + (g1 ? c1 : 0ull) >= K) | (minp > 0.0 && !(fx_val(f) >= am)) | (fx_val(Ar) >= ap);
      if (r < (uint32_t)n && cut && fc == NONE) {
        fc = r;
        Ah = Ar;
      }
      A = fx_add(A, f);
    }
    if (fc != NONE) {
      sh.shi[tid] = Ah.hi;
      sh.slo[tid] = Ah.lo;
    }
    fc = wave_min_u32(fc);
    if (lane_id() == 0 && fc != NONE) atomicMin(&sh.q[0], fc);
  }
  __syncthreads();
  const uint32_t fc = sh.q[0];
  const int last = fc == NONE ? n - 1 : (int)fc - 1;  // the last kept entry
  const bool glast = last >= 0 && (uint32_t)last >= n0;
  bool ok = n > 0 && okd && last >= 0;
  Fx Al{0, 0};  // c_last, unnormalized
  if (fc != NONE) {
    Al = Fx{sh.shi[fc / SP], sh.slo[fc / SP]};
    ok = ok && !(fc >= n0 && !glast && c1 > 0);  // (the first cut entry right after the gap: the cut may be inside it)
  } else {
    Al = fx_add(fx_add(X0, Fx{th, tl}), glast ? X1 : Fx{0, 0});
    const uint64_t rl = c0 + (uint64_t)last + (glast ? c1 : 0ull);
    const uint64_t after = (!sep || glast) ? tail : c1 + tail;  // unlisted elements ranked after the list
    ok = ok && (after == 0 || rl + 1 >= K || fx_val(Al) / Sd >= topp);
  }
  const double clast = fx_val(Al) / Sd;
  if (ok && a.mode == MODE_SAMPLE) {
    // the draw: the first kept entry whose inclusive prefix reaches u c_last; its exclusive prefix must lie below it
    // (else the draw falls in an unlisted region: before the list, or in the gap). Packed as rank << 1 | (not below).
    bool okt = true;
    const double at = least_ge(u * clast, Sd, okt);  // (the same value in every thread)
    Fx A = fx_add(X0, Fx{hi, lo});
    uint32_t fj = NONE;
#pragma unroll 4
    for (int s = 0; s < SP; ++s) {
      const uint32_t r = (uint32_t)(r0 + s);
      const Fx Ar = r >= n0 ? fx_add(A, X1) : A, f = fx_of(msr[r]);
      const bool hit = fx_val(fx_add(Ar, f)) >= at, below = !(fx_val(Ar) >= at);
      if ((int)r <= last && hit && fj == NONE) fj = r << 1 | (below ? 0u : 1u);
      A = fx_add(A, f);
    }
    fj = wave_min_u32(fj);
    if (lane_id() == 0 && fj != NONE) atomicMin(&sh.q[1], fj);
    __syncthreads();
    fj = sh.q[1];
    ok = okt && fj != NONE && (fj & 1u) == 0u;
  }
  if (tid == 0 && ok) {  // (the main pass's cmax stays)
    const int32_t tok = a.mode == MODE_SAMPLE ? (int32_t)pk_id(sh.lc[sh.q[1] >> 1]) : -1;
    RowInfo *ri = a.info + row;
    ri->kkeep = sh.lc[last];
    ri->S = Sd;
    ri->Z = clast;
    ri->flags = R_DONE | R_BY_DEEP;
    ri->ncert = 0;
    ri->token = tok;
    if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
    g_fin = 1u;
  }
  return 0;
}

// The plan's tables lie past the history tables, so that the planning workgroup's pick item (the same slice) keeps
// them.
union PickShared {
  DeepShared d;
  struct {
    HistTab h;
    PlanShared pl;
  } p;
  FinShared f;
};

// ---- the exact path inside this launch ------------------------------------------------------------------------------
// The hard rows this launch does not finish by the window lists (a finish that failed, a row that was not planned, and
// the hard rows the main pass did not send here) are finished by the exact radix-select path, in this launch's
// workgroup shape, so that no second launch follows. Its LDS is the pick items' (a union).
namespace x256 {
constexpr int XT = MT;      // threads
constexpr int NB = 1024;    // histogram bins
constexpr int LB = 10;      // key bits per histogram level
constexpr int CAPS = 2048;  // collected elements
constexpr int CHX = 2048;   // tokens per chunk
#include "gse_exact_body.h"
}  // namespace x256

union DeepLds {
  PickShared p;
  x256::ExactShared x;
};
__shared__ DeepLds g_lds;
__shared__ ScanArgs g_args;               // the exact path's copy of the kernel's arguments
__shared__ uint64_t g_fail[DEEP_MAX / 64];  // slots whose finish failed in this workgroup (its exact rows)
__shared__ uint64_t g_hb[NWV];            // the hard-row scan: one ballot per wave
__shared__ uint32_t g_scan;               // hard rows that the main pass did not send to the split-row finish
__shared__ uint64_t g_pl[DEEP_MAX / 64];  // thread 0: slots planned by this workgroup whose rows-planned ticket is due
__shared__ uint32_t g_gs;                 // workgroups that share the hard-row scan (rows g, g + g_gs, ...)
__shared__ uint32_t g_nd;                 // thread 0: the call's deep rows (read after the items, not kept in a register)

// The call's counts (deep rows and other hard rows: one 64-bit word, read and cleared whole) and the rows-planned ticket
// are cleared for the next call once every row is planned: every workgroup with items has then read the counts (its
// first count item came before). A workgroup without items reads them before (deep rows, so it has no items) or after
// (nothing to do): either way it does nothing.
__device__ __forceinline__ void clear_counts(const ScanArgs &a) {
  st_ag(reinterpret_cast<uint64_t *>(a.dctl), (uint64_t)0);
  st_ag(&a.dctl[2], 0u);
}

namespace x256 {
__device__ __forceinline__ ExactShared &xs() { return g_lds.x; }
}  // namespace x256

// Finishes one hard row by the exact path (every thread of the workgroup calls it; the LDS is free again when it
// returns).
__device__ __noinline__ void exact_hard(int row) { x256::exact_row(g_args, row, g_lds.x); }

// The workgroup's exact rows, after its items: the rows whose finish failed here (their flags still read R_HARD |
// R_DEEP), then, when the main pass counted any (scan), the hard rows it did not send to the split-row finish (R_HARD
// without R_DEEP), workgroup g of the g_gs that scan taking rows g, g + g_gs, ... (A row that another workgroup is
// finishing reads R_DEEP, then R_DONE: skipped.) Not inlined, reading the arguments from their LDS copy, so that the
// kernel keeps nothing across it and its streaming code's registers are allocated apart from the exact path's.
__device__ __noinline__ void exact_rows(bool scan) {
  const ScanArgs &a = g_args;
  const int G = (int)g_gs, tid = threadIdx.x;
#pragma unroll 1
  for (int k = 0; k < DEEP_MAX / 64; ++k) {
    for (uint64_t m = g_fail[k]; m; m &= m - 1ull) {
      exact_hard(a.dslot[k * 64 + (int)__builtin_ctzll(m)].row);
      __syncthreads();  // (LDS of the row)
    }
  }
  if (!scan) return;
  for (int j0 = (int)blockIdx.x; j0 < a.rows; j0 += MT * G) {
    const int r = j0 + tid * G;
    const bool hard = r < a.rows && (a.info[r].flags & (R_HARD | R_DEEP)) == R_HARD;
    const uint64_t bl = ballot64(hard);
    if (lane_id() == 0) g_hb[tid / WAVE] = bl;
    __syncthreads();
    uint64_t hb[NWV];
#pragma unroll
    for (int k = 0; k < NWV; ++k) hb[k] = g_hb[k];
    __syncthreads();  // (every thread has read the ballots)
#pragma unroll 1
    for (int k = 0; k < NWV; ++k) {
      for (uint64_t m = hb[k]; m; m &= m - 1ull) {
        exact_hard(j0 + (k * WAVE + (int)__builtin_ctzll(m)) * G);
        __syncthreads();  // (LDS of the row)
      }
    }
  }
  // Without deep rows, every workgroup scans, and the last to end clears the count of other hard rows.
  if (tid == 0 && g_nd == 0u && ticket_add(&a.dctl[3]) == gridDim.x - 1u) {
    st_ag(reinterpret_cast<uint64_t *>(a.dctl), (uint64_t)0);
    st_ag(&a.dctl[3], 0u);
  }
}

template <int DT, bool AL>
__device__ __forceinline__ void count_item(const ScanArgs &a, int slot, int slice, const DGeom &g, PickShared &ps,
                                           const double *etab) {
  DeepShared &sh = ps.d;
  const int tid = threadIdx.x;
  DeepSlot *ds = a.dslot + slot;
  const int row = ds->row;
  const gse_row P = ds->P;
  const float M = ds->M;
  const double Md = (double)M;
  const RowCtx c = make_ctx(a, row, P);
  const int p0 = slice * g.len, p1 = min(a.V, p0 + g.len);
  __syncthreads();  // (LDS of the previous item)
  prio_by_quarter();
  for (int b = tid; b < DNB; b += MT) {
    sh.c.hi[b] = 0;
    sh.c.lo[b] = 0;
  }
  stream_slice<DT, AL>(a, c, row, p0, p1, sh, false, [] {}, [&](float z, int, bool ok) __attribute__((always_inline)) {
    if (ok && z > -INFINITY) {
      const uint32_t b = dbin(z, M);
      const Fx f = fx_of(exp_nonpos((double)z - Md, etab));
      atomicAdd((unsigned long long *)&sh.c.hi[b], (unsigned long long)f.hi);
      atomicAdd((unsigned long long *)&sh.c.lo[b], (unsigned long long)(f.lo | (1ull << 48)));
    }
  });
  uint64_t *gh = a.dhist + (size_t)slot * 3 * DNB;
  for (int b = tid; b < DNB; b += MT) {
    const uint64_t lo = sh.c.lo[b];
    if (lo) {
      atomic_add_ag(&gh[b], lo >> 48);
      atomic_add_ag(&gh[DNB + b], sh.c.hi[b]);
      atomic_add_ag(&gh[2 * DNB + b], lo & ((1ull << 48) - 1ull));
    }
  }
  // Ticket: the row's last slice plans it.
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&ds->cdone);
  __syncthreads();
  const bool lastc = sh.ticket == (uint32_t)(g.S - 1);
  __syncthreads();  // (every thread has read the ticket: the plan's tables reuse the slice's LDS)
  if (!lastc) return;
  __builtin_amdgcn_s_setprio(3);  // (the row's other slices wait for the plan)
  plan_block(gh, ds, a.mode, ps.p.pl);
  if (tid == 0) {
    ds->cdone = 0u;
    g_pl[slot >> 6] |= 1ull << (slot & 63);  // (its pick item takes the rows-planned ticket)
  }
}


// Returns the slot to finish when this slice was the row's last (-2 - slot when the row was not planned), else -1.
template <int DT, bool AL>
__device__ __forceinline__ int pick_item(const ScanArgs &a, int slot, int slice, const DGeom &g, PickShared &ps,
                                         const double *etab, bool keep) {
  DeepShared &sh = ps.d;
  const int tid = threadIdx.x;
  DeepSlot *ds = a.dslot + slot;
  const int row = ds->row;
  const gse_row P = ds->P;
  const float Mf = ds->M;
  const RowCtx c = make_ctx(a, row, P);
  const int p0 = slice * g.len, p1 = min(a.V, p0 + g.len);
  __syncthreads();  // (LDS of the previous item)
  prio_by_quarter();
  bool planned = false;
  uint32_t w2lo = 0, w2hi = 0, w1lo = 0, w1hi = 0;
  // The wait for the plan comes after this slice's history tables are built and its first chunks are loading, so that
  // both overlap it.
  auto wait_plan = [&]() __attribute__((always_inline)) {
    if (tid == 0) {
      sh.nwl = 0;
      uint64_t st = ld_ag(&ds->plan);
      if (plan_status(st) == DS_PENDING) {
        const uint64_t t0 = wall_clock64();
        while (plan_status(st = ld_ag(&ds->plan)) == DS_PENDING) {
          // (every slice of the grid is resident at once and a plan takes microseconds: the limit, a.plan_wait, only
          // ends the wait when the device could not hold the whole grid)
          if (wall_clock64() - t0 >= a.plan_wait) {
            (void)__hip_atomic_fetch_or(&ds->spoil, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            st = DS_FAIL;
            break;
          }
          __builtin_amdgcn_s_sleep(16);  // (about 1000 clocks between polls)
        }
      }
      sh.pplan = st;
    }
    __syncthreads();
    const uint64_t pw = sh.pplan;
    planned = plan_status(pw) == DS_PLANNED;
    if (planned) {
      w2lo = plan_win(pw, 0);
      w2hi = plan_win(pw, 1);
      w1lo = plan_win(pw, 2);
      w1hi = plan_win(pw, 3);
    }
  };
  stream_slice<DT, AL>(a, c, row, p0, p1, sh, keep, wait_plan, [&](float z, int t, bool ok) __attribute__((always_inline)) {
    if (planned && ok && z > -INFINITY) {
      const uint32_t b = dbin(z, Mf);
      if ((b >= w2lo && b <= w2hi) || (b >= w1lo && b <= w1hi)) {
        const uint32_t pos = atomicAdd(&sh.nwl, 1u);
        if (pos < (uint32_t)WLC) sh.wl[pos] = pack(fkey(z), (uint32_t)t);
      }
    }
  });
  if (planned) {  // the slice's window elements into the row list (stream_slice ends with a barrier: sh.nwl)
    const uint32_t nw = sh.nwl;
    if (tid == 0 && nw) {
      // a slice with more window elements than it can hold spoils the row's count (the row takes the exact path)
      const uint32_t add = nw <= (uint32_t)WLC ? nw : (uint32_t)DCAP + 1u;
      sh.wbase = __hip_atomic_fetch_add(&ds->lcnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (nw && nw <= (uint32_t)WLC) {
      uint64_t *lst = a.dlist + (size_t)slot * DCAP;
      for (uint32_t i = tid; i < nw; i += MT) {
        const uint32_t pos = sh.wbase + i;
        if (pos < (uint32_t)DCAP) st_ag(&lst[pos], sh.wl[i]);
      }
    }
  }
  // Ticket: the row's last slice finishes it (finish_item, called by the kernel's loop). With it, for a row this
  // workgroup planned, the rows-planned ticket (both in flight together).
  store_wait();
  __syncthreads();
  if (tid == 0) {
    uint32_t t = 0xFFFFFFFFu;
    const uint64_t pb = 1ull << (slot & 63);
    if (g_pl[slot >> 6] & pb) {
      g_pl[slot >> 6] &= ~pb;
      t = ticket_add(&a.dctl[2]);
    }
    sh.ticket = ticket_add(&ds->pdone);
    if (t == g_nd - 1u) clear_counts(a);
  }
  __syncthreads();
  if (sh.ticket != (uint32_t)(g.S - 1)) return -1;
  return planned ? slot : -2 - slot;
}

// The finish of the row in slot fs (fs < -1: the row was not planned; its records are cleared all the same), then the
// row's records cleared for the next call. Called at the kernel's top level, after the pick item: its registers are
// allocated apart from the streaming code's, with no call in between.
__device__ __forceinline__ void finish_item(const ScanArgs &a, int fs, PickShared &ps, const double *etab) {
  const int tid = threadIdx.x;
  const bool planned = fs >= 0;
  const int slot = planned ? fs : -2 - fs;
  DeepSlot *ds = a.dslot + slot;
  __builtin_amdgcn_s_setprio(3);  // (the finish is the row's critical path)
  if (tid == 0) g_fin = 0u;
  if (planned) {
    const FinArgs fa{a.dlist + (size_t)slot * DCAP, a.info, a.tokens, a.mode};
    if (a.fin_sorted ? finish_sorted(fa, ds, ps.f, etab) != 0 : ld_ag(&ds->spoil) == 0u) {
      finish_row(fa, ds, ps.f, etab);
    }
  }
  __syncthreads();  // (every thread has read the row's sums)
  uint64_t *gh = a.dhist + (size_t)slot * 3 * DNB;
  for (int b = tid; b < 3 * DNB; b += MT) gh[b] = 0;
  if (tid < DA_N) ds->acc[tid] = 0;
  if (tid == 0) {
    ds->lcnt = 0;
    ds->pdone = 0;
    ds->spoil = 0;
    if (g_fin == 0u) g_fail[slot >> 6] |= 1ull << (slot & 63);  // (the exact path takes the row after the items)
  }
}

// Four waves per SIMD: every workgroup of the grid resident at once. All count items of a workgroup come before its
// pick items, so a pick item only waits for count work that never waits itself.
template <int DT, bool AL>
__global__ __launch_bounds__(MT) __attribute__((amdgpu_waves_per_eu(4, 8))) void deep_kernel(ScanArgs a) {
  PickShared &sh = g_lds.p;
  __shared__ double etab[64];
  const int tid = threadIdx.x;
  const uint64_t cnt = *reinterpret_cast<const uint64_t *>(a.dctl);  // (one load: both counts of one moment)
  const int nd = __builtin_amdgcn_readfirstlane((int)min((uint32_t)cnt, (uint32_t)a.dslots));  // (uniform)
  if (tid < DEEP_MAX / 64) {
    g_fail[tid] = 0ull;
    g_pl[tid] = 0ull;
  }
  if (nd > 0) {
    if (tid < 64) etab[tid] = EXP2_64[tid];  // (published by the first barrier of an item)
    const DGeom g = deep_geom(a, nd);
    if (tid == 0) {  // (kept in LDS, not in registers across the items)
      g_nd = (uint32_t)nd;
      g_scan = (uint32_t)(cnt >> 32);
      g_gs = (uint32_t)min(nd * g.S, (int)gridDim.x);  // (the workgroups with items: every one of them reads the counts)
    }
    for (int i = blockIdx.x; i < nd * g.S; i += gridDim.x) count_item<DT, AL>(a, i / g.S, i % g.S, g, sh, etab);
    // one item per workgroup in each pass: the pick item is the count item's slice, whose history tables are still in
    // LDS
    const bool keep = nd * g.S <= (int)gridDim.x;
    for (int i = blockIdx.x; i < nd * g.S; i += gridDim.x) {
      const int fs = pick_item<DT, AL>(a, i / g.S, i % g.S, g, sh, etab, keep);
      if (fs != -1) finish_item(a, fs, sh, etab);
    }
  } else if (tid == 0) {
    g_nd = 0u;
    g_scan = (uint32_t)(cnt >> 32);
    g_gs = gridDim.x;
  }
  // the exact rows: the arguments copied into LDS first (the argument segment pointer is the launch's only here, in the
  // kernel; its one argument lies at the segment's start: a word per thread)
  __syncthreads();  // (g_fail; LDS of the last item)
  const bool scan = g_scan != 0u && (int)blockIdx.x < (int)g_gs;
  if (__syncthreads_or(tid < DEEP_MAX / 64 && g_fail[tid] != 0ull) || scan) {
    static_assert(sizeof(ScanArgs) % 4 == 0 && sizeof(ScanArgs) / 4 <= MT, "a word per thread");
    const uint32_t *src = (const uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();  // (an address space cast)
    if (tid < (int)(sizeof(ScanArgs) / 4)) reinterpret_cast<uint32_t *>(&g_args)[tid] = src[tid];
    __syncthreads();
    exact_rows(scan);
  }
}

template <int DT, bool AL>
void launch_all(const ScanArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((deep_kernel<DT, AL>), dim3((unsigned)a.dgrid), dim3(MT), 0, s, a);
}

}  // namespace

hipError_t launch_deep(const ScanArgs &a0, hipStream_t s) {
  ScanArgs a = a0;
  a.processed = nullptr;  // the main pass has written the processed logits
  // 16-byte vector loads when every row starts 16-byte aligned
  const bool al = ((((uintptr_t)a.logits) | ((uintptr_t)a.ld * (a.dtype == GSE_BF16 ? 2u : 4u))) & 15u) == 0;
  if (a.dtype == GSE_BF16) {
    if (al) launch_all<GSE_BF16, true>(a, s);
    else launch_all<GSE_BF16, false>(a, s);
  } else {
    if (al) launch_all<GSE_F32, true>(a, s);
    else launch_all<GSE_F32, false>(a, s);
  }
  return hipGetLastError();
}

}  // namespace gse
