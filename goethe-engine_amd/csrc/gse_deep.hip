// Split-row finish of the rows the main pass could not decide from its certified head: a keep prefix that runs past
// the listed elements (the nucleus of a flat, hot row), or a top-p decision that fell inside the main pass's bound on
// S. Three launches, back to back on the stream: two passes over each such row, each spread over dslices workgroups
// (slices of dlen tokens), then one workgroup per row. No workgroup waits for another: slices add their results into
// the row's record with integer atomics (the same sums in any order).
//
//   count:  each slice recomputes z exactly as the main pass does and adds a 512-bin histogram of d = z_max - z
//           (counts, and masses exp2 in fp32 summed as 2^-40 fixed point; bins 1/32 wide, the last one open-ended). d
//           is monotone in z, so the bins follow the stable order and ties share a bin.
//   pick:   each slice plans from the histogram (the same deterministic plan in every slice, overlapped with its first
//           loads): the bins that may hold the last kept element (top-p, top-k and min-p cuts, with a margin for the
//           fp32 masses), the bins that may hold the draw, and whether they hold at most DCAP elements. It then adds the
//           exact fixed-point mass of every element (fp64 exp, 2^-64 resolution) to S and to the regions before and
//           between the two windows, and lists the window elements.
//   finish: sorts the list, walks exact prefixes, and checks that the cut and the draw fall inside it at contiguous
//           ranks; then it writes the token and the row's dist data, and clears the row's records for the next call. A
//           failed check leaves the row to the exact path (gse_exact.hip).
//
// Semantics (goethe_engine/sampling.py:77-83): keep_r = r < top_k AND cumsum(q)_r - q_r < top_p (AND q_r >= min_p q_0);
// c = cumsum(q keep); token = order[min(count(c < u c[-1]), m - 1)], m = keep.sum().
#include "gse_stream.h"

namespace gse {

namespace {

using namespace strm;

constexpr float BSC = 32.0f;    // bins per unit of d
constexpr int BPT = DNB / MT;   // planner: bins per thread (contiguous)
constexpr int WLC = 512;        // window elements a slice gathers in LDS before one global reservation
static_assert(BPT * MT == DNB, "");

struct DeepShared {
  HistTab h;                    // the slice's history tables while streaming
  union {
    struct {
      uint32_t cnt[DNB];        // count pass: the slice's histogram
      uint64_t mass[DNB];
    } c;
    uint64_t wl[WLC];           // pick pass: the slice's window elements
  };
  uint32_t next, hover, ticket, nwl, wbase;
  uint32_t wsum[NWV];
  uint64_t wred[NWV], wred2[NWV];
  double dred[NWV];
  uint32_t q[8];                // first-bin / first-index queries (atomicMin)
  uint32_t plan[5];             // w2lo, w2hi, w1lo, w1hi, status
  double qd[2];
  uint64_t acc[DA_N];
  uint64_t pub[6];
};

// Bin of z (z > -inf, z <= M): monotone non-increasing in z.
__device__ __forceinline__ uint32_t dbin(float z, float M) {
  return (uint32_t)fminf((M - z) * BSC, (float)(DNB - 1));
}

// floor(e * 2^40) for an fp32 e in [0, 1], exact integer arithmetic on its bits.
__device__ __forceinline__ uint64_t q40(float e) {
  const uint32_t b = __float_as_uint(e);
  const int ex = (int)(b >> 23);
  if (ex == 0) return 0;  // zero (subnormals are flushed)
  const uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);
  const int sh = ex - 127 - 23 + 40;
  return sh >= 0 ? m << sh : (sh > -64 ? m >> -sh : 0ull);
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  for (int m = 32; m; m >>= 1) v += shfl_xor_u64(v, m);
  return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const int l = lane_id();
  for (int d = 1; d < WAVE; d <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, d, WAVE);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), d, WAVE);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    if (l >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ void atomic_add_ag(uint64_t *p, uint64_t v) {
  (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, DeepShared &sh) {
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane_id() == 0) sh.wred[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int w = 0; w < NWV; ++w) r += sh.wred[w];
  __syncthreads();
  return r;
}

// Exclusive prefix of two u64 values per thread, in thread order.
__device__ __forceinline__ void block_excl_scan2(uint64_t &a, uint64_t &b, DeepShared &sh) {
  const uint64_t ia = wave_incl_scan_u64(a), ib = wave_incl_scan_u64(b);
  __syncthreads();
  if (lane_id() == WAVE - 1) {
    sh.wred[threadIdx.x >> 6] = ia;
    sh.wred2[threadIdx.x >> 6] = ib;
  }
  __syncthreads();
  uint64_t pa = 0, pb = 0;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < NWV; ++k) {
    pa += k < w ? sh.wred[k] : 0ull;
    pb += k < w ? sh.wred2[k] : 0ull;
  }
  a = pa + ia - a;
  b = pb + ib - b;
  __syncthreads();
}

// Exclusive prefix of an fp64 value per thread in thread order (fixed association); tot receives the total.
__device__ __forceinline__ double block_excl_scan_f64(double v, double &tot, DeepShared &sh) {
  const double inc = wave_incl_scan_f64(v);
  __syncthreads();
  if (lane_id() == WAVE - 1) sh.dred[threadIdx.x >> 6] = inc;
  __syncthreads();
  double pre = 0.0, t = 0.0;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < NWV; ++k) {
    if (k < w) pre += sh.dred[k];
    t += sh.dred[k];
  }
  __syncthreads();
  tot = t;
  return pre + inc - v;
}

// Streams the slice [p0, p1) of the row through the main pass's element pipeline, double-buffered like the main pass:
// the history ids and each wave's first chunk are loaded before the history tables are built. f(z, token, valid) is
// called for every element slot of each chunk by every lane of the wave (valid false past the slice end), so f may use
// ballots. pre() runs (by the whole workgroup) once the first loads are in flight. Ends with a barrier.
template <int DT, bool AL, typename Pre, typename F>
__device__ __forceinline__ void stream_slice(const ScanArgs &a, const RowCtx &c, int row, int p0, int p1,
                                             DeepShared &sh, Pre pre, F f) {
  using L = Lay<DT>;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int nck = (p1 - p0 + CHK - 1) / CHK;
  int hid[HPT];
  if (c.pen) {
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int j = c.hb + k * MT + tid;
      hid[k] = j < c.he ? a.hist[j] : -1;
    }
  }
  float xa[EPL], xb[EPL];
  uint32_t ma[L::NV], mb[L::NV];
  int ck = w;
  if (ck < nck) load_chunk<DT, AL>(c, p0 + ck * CHK, p1, xa, ma);
  pre();
  if (tid == 0) {
    sh.next = NWV;
    sh.hover = 0;
  }
  if (c.pen) build_history(c, a.hist, hid, p0, p1, sh.h, sh.wsum, sh.hover);
  else __syncthreads();
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
  auto grab = [&]() -> int {
    uint32_t n = 0;
    if (lane == 0) n = atomicAdd(&sh.next, 1u);
    return __shfl((int)n, 0, WAVE);
  };
  auto body = [&](int k, float(&x)[EPL], const uint32_t(&mw)[L::NV]) __attribute__((always_inline)) {
    const int cb = p0 + k * CHK;
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
  while (ck < nck) {
    const int cn = grab();
    if (cn < nck) load_chunk<DT, AL>(c, p0 + cn * CHK, p1, xb, mb);
    body(ck, xa, ma);
    if (cn >= nck) break;
    const int cn2 = grab();
    if (cn2 < nck) load_chunk<DT, AL>(c, p0 + cn2 * CHK, p1, xa, ma);
    body(cn, xb, mb);
    ck = cn2;
  }
  __syncthreads();
}

// Work items (deep row slot, slice) of a pass: the slices of a slot on one XCD (workgroups go round-robin over the 8
// XCDs and the grid is a multiple of 8).
__device__ __forceinline__ bool item_of(const ScanArgs &a, int i, int nd, int &slot, int &slice) {
  slot = (i & 7) + 8 * ((i >> 3) / a.dslices);
  slice = (i >> 3) % a.dslices;
  return slot < nd;
}

__device__ __forceinline__ int items_of(const ScanArgs &a, int nd) { return (nd + 7) / 8 * 8 * a.dslices; }

// ---------------------------------------------------------------------------------------------------------------------
// Pass 1: histogram and plan.

// The plan of a row from its histogram (written by the previous launch): sh.plan = {w2lo, w2hi, w1lo, w1hi, status}.
// The slice that stores it (slice 0) also writes it into the row's slot for the finish launch.
__device__ __forceinline__ void plan_row(const ScanArgs &a, DeepSlot *ds, const gse_row &P, float M, bool store,
                                         DeepShared &sh) {
  const int tid = threadIdx.x;
  const uint64_t *gh = a.dhist + (size_t)(ds - a.dslot) * 2 * DNB;
  uint64_t c[BPT], q[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    c[j] = gh[tid * BPT + j];
    q[j] = gh[DNB + tid * BPT + j];
  }
  double m[BPT];
  uint64_t cl = 0, dummy = 0;
  double ml = 0.0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    m[j] = (double)q[j] * 9.094947017729282e-13;  // 2^-40
    cl += c[j];
    ml += m[j];
  }
  double S;
  const double mpre = block_excl_scan_f64(ml, S, sh);
  const uint64_t ctot = block_sum_u64(cl, sh);
  block_excl_scan2(cl, dummy, sh);
  double pin[BPT], pex[BPT];
  uint64_t cin[BPT];
  {
    double p = mpre;
    uint64_t n = cl;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      pex[j] = p;
      p += m[j];
      pin[j] = p;
      n += c[j];
      cin[j] = n;
    }
  }
  // the fp32 exp2 terms (2 ulp) and the 2^-40 floors stay far inside this margin
  const double delta = 1e-4 * S;
  const uint64_t K = P.top_k > 0 ? (uint64_t)P.top_k : ~0ull;
  const double tS = P.top_p * S;
  // min-p keeps exp(z - M) >= min_p, i.e. d <= -ln(min_p): bins below bm - 1 are all kept, bins above bm + 1 all cut
  const bool mp = P.min_p > 0.0;
  uint32_t bm = 0;
  if (mp) {
    const double dm = -log(P.min_p) * (double)BSC;
    bm = dm >= (double)(DNB - 1) ? (uint32_t)(DNB - 1) : (uint32_t)dm;
  }
  if (tid < 8) sh.q[tid] = tid == 5 ? 0u : DNB - 1;
  __syncthreads();
  // round 1: the windows of the cuts
  //   q[0], q[1]: first bins with Pincl >= tS - delta, >= tS + delta (top-p: the bin of the last kept element)
  //   q[2]:       first bin with Cincl >= K (top-k: the bin of rank K - 1)
  //   q[5] - 1:   last non-empty bin below bm - 1 (min-p: holds a kept element, so the last kept one is at or after it)
  //   q[6]:       first non-empty bin above bm + 1 (min-p: holds a cut element)
  {
    uint32_t b0 = DNB - 1, b1 = DNB - 1, b2 = DNB - 1, b5 = 0, b6 = DNB - 1;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      const uint32_t b = tid * BPT + j;
      if (pin[j] >= tS - delta) b0 = b;
      if (pin[j] >= tS + delta) b1 = b;
      if (cin[j] >= K) b2 = b;
      if (mp && c[j] && b + 1 < bm) b5 = max(b5, b + 1);
      if (mp && c[j] && b > bm + 1) b6 = b;
    }
    atomicMin(&sh.q[0], b0);
    atomicMin(&sh.q[1], b1);
    atomicMin(&sh.q[2], b2);
    atomicMax(&sh.q[5], b5);
    atomicMin(&sh.q[6], b6);
  }
  __syncthreads();
  uint32_t w1lo = sh.q[0], w1hi = sh.q[1];
  if (K < ctot) {
    w1lo = min(w1lo, sh.q[2]);
    w1hi = min(w1hi, sh.q[2]);
  }
  if (mp) {
    const uint32_t lo = sh.q[5] ? sh.q[5] - 1u : 0u, hi = sh.q[6];
    w1lo = min(w1lo, lo);
    // when min-p may bind, the window reaches its first cut element (the finish cannot test min-p unlisted)
    w1hi = lo <= w1hi ? max(w1hi, min(hi, (uint32_t)(DNB - 1))) : min(w1hi, hi);
  }
  // masses before w1lo and through w1hi (approximate)
  if (tid == (int)(w1lo / BPT)) sh.qd[0] = pex[w1lo % BPT];
  if (tid == (int)(w1hi / BPT)) sh.qd[1] = pin[w1hi % BPT];
  __syncthreads();
  uint32_t w2lo = w1lo, w2hi = w1hi;
  if (a.mode == MODE_SAMPLE) {
    const double u = ds->u;  // (P and u: the slot copy)
    const double tlo = u * (sh.qd[0] - delta) - delta, thi = u * (sh.qd[1] + delta) + delta;
    uint32_t b3 = DNB - 1, b4 = DNB - 1;
#pragma unroll
    for (int j = BPT - 1; j >= 0; --j) {
      const uint32_t b = tid * BPT + j;
      if (pin[j] >= tlo) b3 = b;
      if (pin[j] >= thi) b4 = b;
    }
    atomicMin(&sh.q[3], b3);
    atomicMin(&sh.q[4], b4);
    __syncthreads();
    w2hi = min(sh.q[4], w1hi);
    w2lo = min(sh.q[3], w2hi);
  }
  if (w2hi + 1 >= w1lo) {  // touching or overlapping windows: one window
    w2lo = min(w2lo, w1lo);
    w2hi = max(w2hi, w1hi);
    w1lo = w2lo;
    w1hi = w2hi;
  }
  uint64_t inw = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const uint32_t b = tid * BPT + j;
    if ((b >= w2lo && b <= w2hi) || (b >= w1lo && b <= w1hi)) inw += c[j];
  }
  inw = block_sum_u64(inw, sh);
  const uint32_t status = (inw > 0 && inw <= (uint64_t)DCAP && S > 0.0 && fabsf(M) < INFINITY) ? DS_PLANNED : DS_FAIL;
  if (tid == 0) {
    sh.plan[0] = w2lo;
    sh.plan[1] = w2hi;
    sh.plan[2] = w1lo;
    sh.plan[3] = w1hi;
    sh.plan[4] = status;
    if (store) {
      ds->w2lo = w2lo;
      ds->w2hi = w2hi;
      ds->w1lo = w1lo;
      ds->w1hi = w1hi;
      ds->status = status;
    }
  }
  __syncthreads();
}

template <int DT, bool AL>
__device__ __forceinline__ void count_item(const ScanArgs &a, int slot, int slice, DeepShared &sh) {
  const int tid = threadIdx.x;
  DeepSlot *ds = a.dslot + slot;
  const int row = ds->row;
  const gse_row P = ds->P;
  const float M = ds->M;
  const RowCtx c = make_ctx(a, row, P);
  const int p0 = slice * a.dlen, p1 = min(a.V, p0 + a.dlen);
  __syncthreads();  // (LDS of the previous item)
  for (int b = tid; b < DNB; b += MT) {
    sh.c.cnt[b] = 0;
    sh.c.mass[b] = 0;
  }
  stream_slice<DT, AL>(a, c, row, p0, p1, sh, []() {}, [&](float z, int, bool ok) __attribute__((always_inline)) {
    if (ok && z > -INFINITY) {
      const uint32_t b = dbin(z, M);
      atomicAdd(&sh.c.cnt[b], 1u);
      atomicAdd((unsigned long long *)&sh.c.mass[b], (unsigned long long)q40(__builtin_amdgcn_exp2f((z - M) * LOG2E)));
    }
  });
  uint64_t *gh = a.dhist + (size_t)slot * 2 * DNB;
  for (int b = tid; b < DNB; b += MT) {
    const uint32_t n = sh.c.cnt[b];
    if (n) {
      atomic_add_ag(&gh[b], (uint64_t)n);
      atomic_add_ag(&gh[DNB + b], sh.c.mass[b]);
    }
  }
}

// Four waves per SIMD: every workgroup of the grid resident at once.
template <int DT, bool AL>
__global__ __launch_bounds__(MT) __attribute__((amdgpu_waves_per_eu(4, 8))) void deep_count_kernel(ScanArgs a) {
  __shared__ DeepShared sh;
  const int nd = (int)min(a.dctl[0], (uint32_t)DEEP_MAX);
  const int ni = items_of(a, nd);
  for (int i = blockIdx.x; i < ni; i += gridDim.x) {
    int slot, slice;
    if (item_of(a, i, nd, slot, slice)) count_item<DT, AL>(a, slot, slice, sh);
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// Pass 2: exact masses, window list, finish.

// ---- finish ---------------------------------------------------------------------------------------------------------
// The window entries are not sorted as a whole: an exact sub-histogram over their keys (per window, 128 sub-bins of
// equal key width; counts and fixed-point masses, order-independent) gives the rank and exclusive prefix at the head of
// every sub-bin. The keep cut lies in the last non-empty sub-bin before the first one whose head is cut (s0); the draw
// in the first sub-bin whose inclusive prefix reaches u * c_last (sj). Only the entries of those two sub-bins are
// sorted and walked.

constexpr int NSB = 256;       // sub-bins (128 per window)
constexpr int SUBC = 2048;     // entries of one sub-bin that can be collected

struct FinShared {
  uint64_t list[DCAP];         // the window entries (unsorted)
  uint64_t sub[SUBC];          // the collected entries of one sub-bin, sorted
  uint32_t scnt[NSB];          // sub-bin counts, then their exclusive prefix
  uint32_t stop[NSB];          // sub-bin head keys (largest key)
  uint64_t shi[NSB], slo[NSB]; // sub-bin masses, then their exclusive prefix
  uint32_t kmax[2], kmin[2];
  uint32_t q[4];
  uint32_t ns;
  uint64_t wred[NWV], wred2[NWV];
  uint32_t wsum[NWV];
  uint64_t pub[8];
};

template <int S>
__device__ __forceinline__ void sort_sub(int n, FinShared &sh) {
  const int tid = threadIdx.x;
  uint64_t v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) v[s] = tid * S + s < n ? sh.sub[tid * S + s] : 0ull;
  __syncthreads();
  sort_regs<S>(v, sh.sub);
#pragma unroll
  for (int s = 0; s < S; ++s) sh.sub[tid * S + s] = v[s];
  __syncthreads();
}

// Collects the entries of sub-bin sb into sh.sub and sorts them (descending). Returns their number (0 when more than
// SUBC; the caller then gives up).
__device__ __forceinline__ int collect_sub(int n, int sb, uint32_t cnt, const uint32_t (&shift)[2], bool sep,
                                           uint32_t w1lo, float Mf, FinShared &sh) {
  const int tid = threadIdx.x;
  if (cnt > (uint32_t)SUBC) return 0;
  if (tid == 0) sh.ns = 0;
  __syncthreads();
  for (int i = tid; i < n; i += MT) {
    const uint64_t pk = sh.list[i];
    const uint32_t k = pk_key(pk);
    const int g = (sep && dbin(fkey_inv(k), Mf) >= w1lo) ? 1 : 0;
    const int b = g * (NSB / 2) + (int)min((sh.kmax[g] - k) >> shift[g], (uint32_t)(NSB / 2 - 1));
    if (b == sb) sh.sub[atomicAdd(&sh.ns, 1u)] = pk;
  }
  __syncthreads();
  const int m = (int)cnt;
  if (m <= MT) sort_sub<1>(m, sh);
  else sort_sub<SUBC / MT>(m, sh);
  return m;
}

__device__ __forceinline__ void finish_row(const ScanArgs &a, DeepSlot *ds, FinShared &sh) {
  const int tid = threadIdx.x;
  const gse_row &P = ds->P;
  const int row = ds->row;
  const float Mf = ds->M;
  const double M = (double)Mf;
  const uint32_t w2hi = ds->w2hi, w1lo = ds->w1lo;
  const bool sep = w1lo > w2hi;  // an unlisted gap (region 1) between the draw window and the cut window
  uint64_t acc[DA_N];
#pragma unroll
  for (int k = 0; k < DA_N; ++k) acc[k] = ds->acc[k];
  const uint32_t nraw = ds->lcnt;
  const Fx X0{acc[DA_X0HI], acc[DA_X0LO]}, X1{acc[DA_X1HI], acc[DA_X1LO]}, SF{acc[DA_SHI], acc[DA_SLO]};
  const uint64_t c0 = acc[DA_C0], c1 = acc[DA_C1], tail = acc[DA_C2];
  const double Sd = fx_val(SF);
  const uint64_t K = P.top_k > 0 ? (uint64_t)P.top_k : ~0ull;
  const double topp = P.top_p, minp = P.min_p, q0 = 1.0 / Sd;
  const bool ok0 = nraw > 0 && nraw <= (uint32_t)DCAP && Sd > 0.0;
  const int n = ok0 ? (int)nraw : 0;
  const uint64_t *lst = a.dlist + (size_t)(ds - a.dslot) * DCAP;
  // entries into LDS; key ranges of the two windows
  if (tid < 2) {
    sh.kmax[tid] = 0;
    sh.kmin[tid] = 0xFFFFFFFFu;
  }
  sh.scnt[tid] = 0;
  sh.stop[tid] = 0;
  sh.shi[tid] = 0;
  sh.slo[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += MT) {
    const uint64_t pk = lst[i];
    sh.list[i] = pk;
    const uint32_t k = pk_key(pk);
    const int g = (sep && dbin(fkey_inv(k), Mf) >= w1lo) ? 1 : 0;
    atomicMax(&sh.kmax[g], k);
    atomicMin(&sh.kmin[g], k);
  }
  __syncthreads();
  uint32_t shift[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint32_t span = sh.kmax[g] >= sh.kmin[g] ? sh.kmax[g] - sh.kmin[g] : 0u;
    uint32_t sft = 0;
    while (sft < 31 && (span >> sft) >= (uint32_t)(NSB / 2)) ++sft;
    shift[g] = sft;
  }
  // exact sub-bin counts, masses and head keys
  for (int i = tid; i < n; i += MT) {
    const uint64_t pk = sh.list[i];
    const uint32_t k = pk_key(pk);
    const float z = fkey_inv(k);
    const int g = (sep && dbin(z, Mf) >= w1lo) ? 1 : 0;
    const int b = g * (NSB / 2) + (int)min((sh.kmax[g] - k) >> shift[g], (uint32_t)(NSB / 2 - 1));
    const Fx f = fx_of(exp((double)z - M));
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
    const uint64_t ia = wave_incl_scan_u64(ph), ib = wave_incl_scan_u64(pl);
    const uint32_t ic = wave_incl_scan_u32(mycnt);
    __syncthreads();
    if (lane_id() == WAVE - 1) {
      sh.wred[tid >> 6] = ia;
      sh.wred2[tid >> 6] = ib;
      sh.wsum[tid >> 6] = ic;
    }
    __syncthreads();
    uint64_t pa = 0, pb = 0;
    uint32_t pc = 0;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      pa += k < (tid >> 6) ? sh.wred[k] : 0ull;
      pb += k < (tid >> 6) ? sh.wred2[k] : 0ull;
      pc += k < (tid >> 6) ? sh.wsum[k] : 0u;
    }
    ph = pa + ia - ph;
    pl = pb + ib - pl;
    sh.scnt[tid] = pc + ic - mycnt;  // (now the exclusive count prefix)
  }
  const bool seg1 = sep && tid >= NSB / 2;
  const Fx pbase = fx_add(fx_add(X0, Fx{ph, pl}), seg1 ? X1 : Fx{0, 0});
  const uint64_t rbase = c0 + sh.scnt[tid] + (seg1 ? c1 : 0ull);
  if (tid < 4) sh.q[tid] = tid == 1 ? 0u : 0xFFFFFFFFu;
  __syncthreads();
  // s1: the first non-empty sub-bin whose head entry is cut
  if (ok0 && mycnt) {
    const double e0 = exp((double)fkey_inv(mytop) - M);
    const bool cut = rbase >= K || (minp > 0.0 && !(fx_val(fx_of(e0)) / Sd >= minp * q0)) || fx_val(pbase) / Sd >= topp;
    if (cut) atomicMin(&sh.q[0], (uint32_t)tid);
  }
  __syncthreads();
  const uint32_t s1 = sh.q[0];
  // s0: the last non-empty sub-bin before s1 (it holds the last kept entry)
  if (ok0 && mycnt && (uint32_t)tid < s1) atomicMax(&sh.q[1], (uint32_t)tid + 1u);
  __syncthreads();
  const int s0 = (int)sh.q[1] - 1;
  bool ok = ok0 && s0 >= 0;
  if (ok && tid == s0) {
    sh.pub[0] = rbase;
    sh.pub[1] = pbase.hi;
    sh.pub[2] = pbase.lo;
    sh.pub[3] = mycnt;
    sh.pub[4] = seg1 ? 1u : 0u;
  }
  if (ok && s1 != 0xFFFFFFFFu && tid == (int)s1) sh.pub[5] = rbase;
  __syncthreads();
  // walk s0's sorted entries: the last kept entry and c_last
  double clast = 0.0;
  uint64_t kkeep = 0;
  if (ok) {
    const uint64_t r0 = sh.pub[0];
    const Fx b0{sh.pub[1], sh.pub[2]};
    const uint32_t cnt0 = (uint32_t)sh.pub[3];
    const bool g0 = sh.pub[4] != 0;
    const uint64_t r_s1 = sh.pub[5];
    const int m0 = collect_sub(n, s0, cnt0, shift, sep, w1lo, Mf, sh);
    ok = m0 == (int)cnt0;
    if (ok && tid == 0) {
      // sequential over the (few) entries of one sub-bin: exact prefixes in sorted order
      Fx A = b0;
      int last = m0 - 1;  // the last kept entry, unless a cut falls inside the sub-bin
      bool inside = false;
      for (int k = 0; k < m0; ++k) {
        const double e = exp((double)fkey_inv(pk_key(sh.sub[k])) - M);
        const Fx f = fx_of(e);
        const bool cut = r0 + (uint64_t)k >= K || (minp > 0.0 && !(fx_val(f) / Sd >= minp * q0)) ||
                         fx_val(A) / Sd >= topp;
        if (cut) {
          last = k - 1;
          inside = true;
          break;
        }
        A = fx_add(A, f);
        if (k == m0 - 1) break;
      }
      // A = exclusive prefix of entry last + 1 = inclusive prefix of entry last
      bool good = last >= 0;
      if (good && !inside) {
        // the next rank is s1's head (cut by definition) when directly adjacent, else past the list
        const uint64_t rl = r0 + (uint64_t)last;
        if (s1 != 0xFFFFFFFFu) {
          good = r_s1 == rl + 1;
        } else {
          const uint64_t after = (!sep || g0) ? tail : c1 + tail;
          good = after == 0 || rl + 1 >= K || fx_val(A) / Sd >= topp;
        }
      }
      sh.pub[6] = good ? 1u : 0u;
      sh.pub[1] = A.hi;
      sh.pub[2] = A.lo;
      sh.pub[7] = good ? sh.sub[last] : 0ull;
    }
    __syncthreads();
    ok = ok && sh.pub[6] != 0;
    if (ok) {
      clast = fx_val(Fx{sh.pub[1], sh.pub[2]}) / Sd;
      kkeep = sh.pub[7];
    }
  }
  __syncthreads();
  int32_t tok = -1;
  if (ok && a.mode == MODE_SAMPLE) {
    // sj: the first non-empty sub-bin whose last entry's inclusive prefix reaches u * c_last; its head's exclusive
    // prefix must be below it (else the draw falls in an unlisted region)
    const double thr = ds->u * clast;
    if (tid == 0) sh.q[2] = 0xFFFFFFFFu;
    __syncthreads();
    if (mycnt && fx_val(fx_add(pbase, mym)) / Sd >= thr) atomicMin(&sh.q[2], (uint32_t)tid);
    __syncthreads();
    const uint32_t sj = sh.q[2];
    if (sj != 0xFFFFFFFFu && tid == (int)sj) {
      sh.pub[0] = pbase.hi;
      sh.pub[1] = pbase.lo;
      sh.pub[3] = mycnt;
    }
    __syncthreads();
    ok = sj != 0xFFFFFFFFu && !(fx_val(Fx{sh.pub[0], sh.pub[1]}) / Sd >= thr);
    if (ok) {
      const uint32_t cj = (uint32_t)sh.pub[3];
      const Fx bj{sh.pub[0], sh.pub[1]};
      const int mj = collect_sub(n, (int)sj, cj, shift, sep, w1lo, Mf, sh);
      ok = mj == (int)cj;
      if (ok && tid == 0) {
        Fx A = bj;
        int j = -1;
        for (int k = 0; k < mj; ++k) {
          A = fx_add(A, fx_of(exp((double)fkey_inv(pk_key(sh.sub[k])) - M)));
          if (fx_val(A) / Sd >= thr) {
            j = k;
            break;
          }
        }
        sh.pub[5] = j >= 0 ? (uint64_t)pk_id(sh.sub[j]) : 0xFFFFFFFFFFFFFFFFull;
      }
      __syncthreads();
      ok = ok && sh.pub[5] != 0xFFFFFFFFFFFFFFFFull;
      if (ok) tok = (int32_t)sh.pub[5];
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (ok) {
      RowInfo *ri = a.info + row;
      RowInfo r = {};
      r.cmax = ri->cmax;
      r.kkeep = kkeep;
      r.S = Sd;
      r.Z = clast;
      r.flags = R_DONE | R_BY_DEEP;
      r.token = tok;
      *ri = r;
      if (a.mode == MODE_SAMPLE) a.tokens[row] = tok;
    }
  }
}

template <int DT, bool AL>
__device__ __forceinline__ void pick_item(const ScanArgs &a, int slot, int slice, DeepShared &sh) {
  const int tid = threadIdx.x;
  DeepSlot *ds = a.dslot + slot;
  const int row = ds->row;
  const gse_row P = ds->P;
  const float Mf = ds->M;
  const double M = (double)Mf;
  const RowCtx c = make_ctx(a, row, P);
  const int p0 = slice * a.dlen, p1 = min(a.V, p0 + a.dlen);
  __syncthreads();  // (LDS of the previous item)
  if (tid == 0) sh.nwl = 0;
  uint64_t acc[DA_N];
#pragma unroll
  for (int k = 0; k < DA_N; ++k) acc[k] = 0;
  uint32_t w2lo = 0, w2hi = 0, w1lo = 0, w1hi = 0;
  bool planned = false;
  auto pre = [&]() __attribute__((always_inline)) {
    plan_row(a, ds, P, Mf, slice == 0, sh);
    w2lo = sh.plan[0];
    w2hi = sh.plan[1];
    w1lo = sh.plan[2];
    w1hi = sh.plan[3];
    planned = sh.plan[4] == DS_PLANNED;
  };
  stream_slice<DT, AL>(a, c, row, p0, p1, sh, pre, [&](float z, int t, bool ok) __attribute__((always_inline)) {
    const bool live = planned && ok && z > -INFINITY;
    bool inw = false;
    if (live) {
      const uint32_t b = dbin(z, Mf);
      const Fx f = fx_of(exp((double)z - M));
      acc[DA_SHI] += f.hi;
      acc[DA_SLO] += f.lo;
      if (b < w2lo) {
        acc[DA_X0HI] += f.hi;
        acc[DA_X0LO] += f.lo;
        acc[DA_C0] += 1;
      } else if (b > w2hi && b < w1lo) {
        acc[DA_X1HI] += f.hi;
        acc[DA_X1LO] += f.lo;
        acc[DA_C1] += 1;
      } else if (b > w1hi) {
        acc[DA_C2] += 1;
      } else {
        inw = true;
      }
    }
    if (inw) {
      const uint32_t pos = atomicAdd(&sh.nwl, 1u);
      if (pos < (uint32_t)WLC) sh.wl[pos] = pack(fkey(z), (uint32_t)t);
    }
  });
  // the slice's sums into the row record (per wave; integer adds, any order), its window elements into the row list
#pragma unroll
  for (int k = 0; k < DA_N; ++k) {
    const uint64_t v = wave_sum_u64(acc[k]);
    if (lane_id() == 0 && v) atomic_add_ag(&ds->acc[k], v);
  }
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

template <int DT, bool AL>
__global__ __launch_bounds__(MT) __attribute__((amdgpu_waves_per_eu(4, 8))) void deep_pick_kernel(ScanArgs a) {
  __shared__ DeepShared sh;
  const int nd = (int)min(a.dctl[0], (uint32_t)DEEP_MAX);
  const int ni = items_of(a, nd);
  for (int i = blockIdx.x; i < ni; i += gridDim.x) {
    int slot, slice;
    if (item_of(a, i, nd, slot, slice)) pick_item<DT, AL>(a, slot, slice, sh);
  }
}

// One workgroup per deep row: the finish, and the row's histogram cleared for the next call.
__global__ __launch_bounds__(MT) void deep_finish_kernel(ScanArgs a) {
  __shared__ FinShared sh;
  const int nd = (int)min(a.dctl[0], (uint32_t)DEEP_MAX);
  const int slot = blockIdx.x;
  if (slot >= nd) return;
  DeepSlot *ds = a.dslot + slot;
  uint64_t *gh = a.dhist + (size_t)slot * 2 * DNB;
  for (int b = threadIdx.x; b < 2 * DNB; b += MT) gh[b] = 0;
  if (ds->status == DS_PLANNED) finish_row(a, ds, sh);
  __syncthreads();  // (every thread has read the row's sums)
  if (threadIdx.x < DA_N) ds->acc[threadIdx.x] = 0;
  if (threadIdx.x == 0) ds->lcnt = 0;
}

template <int DT, bool AL>
void launch_all(const ScanArgs &a, hipStream_t s) {
  dim3 grid((unsigned)a.dgrid), block(MT);
  hipLaunchKernelGGL((deep_count_kernel<DT, AL>), grid, block, 0, s, a);
  hipLaunchKernelGGL((deep_pick_kernel<DT, AL>), grid, block, 0, s, a);
  hipLaunchKernelGGL(deep_finish_kernel, dim3((unsigned)min(a.rows, DEEP_MAX)), block, 0, s, a);
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
