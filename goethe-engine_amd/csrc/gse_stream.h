// Streaming pieces shared by the selection kernels: the chunk layout of a 256-thread workgroup (four waves, 64 lanes x
// 16 tokens per chunk), the part history tables, the chunk loads, the per-element pipeline (penalties, NaN test, mask,
// temperature) and deterministic block reductions.
#pragma once
#include "gse_rowctx.h"

namespace gse {
namespace strm {

constexpr int MT = 256;                // threads per part workgroup
constexpr int NWV = MT / WAVE;         // waves
constexpr int EPL = 8;                 // tokens per lane per chunk
constexpr int CHK = WAVE * EPL;        // tokens per chunk
constexpr int PMAX = PTOK;             // tokens per part, at most
constexpr int PWORDS = PMAX / 32;      // history bitset words of a part
constexpr int HMAX = 2048;             // distinct history ids of a part (more: the row takes the exact path)
constexpr int HPT = 8;                 // history ids per thread per round
constexpr float LOG2E = 1.4426950408889634f;
constexpr float FLTMAX = 3.402823466e+38f;

template <int DT>
struct Lay;
template <>
struct Lay<GSE_F32> {  // chunk base cb, lane l, vector v, element k: token cb + v * 256 + l * 4 + k
  static constexpr int VEC = 4, NV = EPL / 4, STRIDE = WAVE * 4;
};
template <>
struct Lay<GSE_BF16> {  // token cb + v * 512 + l * 8 + k
  static constexpr int VEC = 8, NV = EPL / 8, STRIDE = WAVE * 8;
};

struct HistTab {  // history of a part's tokens: bitset, prefix popcounts of its words, counts and offsets by rank
  uint32_t bits[PWORDS];
  uint32_t pre[PWORDS];
  uint32_t cnt[HMAX];
  uint16_t off[HMAX];   // offset in the part of the token of each rank
  uint32_t nd;          // distinct tokens (ranks), at most HMAX
};

// z = RN32(x / T) as RN32(x * Rd), Rd = RN64(1 / T). |x * Rd - x / T| <= 2^-51 |x / T| (two fp64 roundings), while
// x / T lies at least 2^-49 |x / T| from every fp32 rounding midpoint (x and T have 24-bit significands, so x - m T
// for a midpoint m is a nonzero multiple of 2^-47 of the binade); the fp32 rounding of the fp64 product therefore
// equals the correctly rounded quotient, subnormal and overflowing results included.
__device__ __forceinline__ float div_exact(float x, double Rd) { return (float)((double)x * Rd); }

__device__ __forceinline__ int nlp_of(const ScanArgs &a, const gse_row &P) {
  return a.lp_ids ? min(min(P.logprobs, GSE_MAX_LOGPROBS), (int)a.lp_ld) : 0;
}

// The part's history [p0, p1): bitset of the tokens present, their prefix popcounts, and the count of each present
// token indexed by its rank among them. hid holds this thread's first ids (loaded before the logits). Ends with a
// barrier.
__device__ __forceinline__ void build_history(const RowCtx &c, const int32_t *hist, const int (&hid)[HPT], int p0,
                                              int p1, HistTab &h, uint32_t (&wsum)[NWV], uint32_t &hover) {
  const int tid = threadIdx.x;
  const int nw = (p1 - p0 + 31) >> 5;
  for (int i = tid; i < nw; i += MT) h.bits[i] = 0;
  __syncthreads();
  auto each = [&](auto f) {
#pragma unroll
    for (int k = 0; k < HPT; ++k)
      if (hid[k] >= p0 && hid[k] < p1) f(hid[k] - p0);
    for (int j0 = c.hb + MT * HPT; j0 < c.he; j0 += MT * HPT) {
      int more[HPT];
#pragma unroll
      for (int k = 0; k < HPT; ++k) {
        const int j = j0 + k * MT + tid;
        more[k] = j < c.he ? hist[j] : -1;
      }
#pragma unroll
      for (int k = 0; k < HPT; ++k)
        if (more[k] >= p0 && more[k] < p1) f(more[k] - p0);
    }
  };
  each([&](int o) { atomicOr(&h.bits[o >> 5], 1u << (o & 31)); });
  __syncthreads();
  // exclusive prefix of the word popcounts (words per thread contiguous)
  const int per = (nw + MT - 1) / MT, w0 = tid * per;
  uint32_t loc = 0;
  for (int i = 0; i < per; ++i)
    if (w0 + i < nw) loc += __popc(h.bits[w0 + i]);
  const uint32_t inc = wave_incl_scan_u32(loc);
  if (lane_id() == WAVE - 1) wsum[tid >> 6] = inc;
  __syncthreads();
  uint32_t run = inc - loc, tot = 0;
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    run += w < (tid >> 6) ? wsum[w] : 0u;
    tot += wsum[w];
  }
  for (int i = 0; i < per; ++i)
    if (w0 + i < nw) {
      h.pre[w0 + i] = run;
      run += __popc(h.bits[w0 + i]);
    }
  const uint32_t nd = min(tot, (uint32_t)HMAX);
  for (uint32_t i = tid; i < nd; i += MT) h.cnt[i] = 0;
  if (tid == 0) {
    h.nd = nd;
    if (tot > (uint32_t)HMAX) hover = 1;
  }
  __syncthreads();
  each([&](int o) {
    const uint32_t r = h.pre[o >> 5] + __popc(h.bits[o >> 5] & ((1u << (o & 31)) - 1u));
    if (r < (uint32_t)HMAX) {
      atomicAdd(&h.cnt[r], 1u);
      h.off[r] = (uint16_t)o;  // (a repeated id writes the same offset)
    }
  });
  __syncthreads();
}

// One chunk's logits into registers (fp32, or bf16 widened exactly) and its packed mask words; AL: the row start is
// 16-byte aligned, so a whole vector is one 16-byte load. A token past the part end loads 0.
template <int DT, bool AL>
__device__ __forceinline__ void load_chunk(const RowCtx &c, int cb, int p1, float (&x)[EPL],
                                           uint32_t (&mw)[Lay<DT>::NV]) {
  using L = Lay<DT>;
  const int l = lane_id();
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = cb + v * L::STRIDE + l * L::VEC;
    mw[v] = c.mw ? (t0 < p1 ? c.mw[t0 >> 5] : 0u) : 0xFFFFFFFFu;
  }
  if constexpr (DT == GSE_F32) {
    const float *p = (const float *)c.base + cb + l * 4;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int t0 = cb + v * L::STRIDE + l * 4;
      if (AL && t0 + 4 <= p1) {
        const float4 f = *reinterpret_cast<const float4 *>(p + v * L::STRIDE);
        x[4 * v] = f.x;
        x[4 * v + 1] = f.y;
        x[4 * v + 2] = f.z;
        x[4 * v + 3] = f.w;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[4 * v + k] = t0 + k < p1 ? p[v * L::STRIDE + k] : 0.0f;
      }
    }
  } else {
    const uint16_t *p = (const uint16_t *)c.base + cb + l * 8;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int t0 = cb + v * L::STRIDE + l * 8;
      if (AL && t0 + 8 <= p1) {
        const uint4 u = *reinterpret_cast<const uint4 *>(p + v * L::STRIDE);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[8 * v + 2 * i] = __uint_as_float(w[i] << 16);
          x[8 * v + 2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[8 * v + k] = t0 + k < p1 ? bf16_to_f32(p[v * L::STRIDE + k]) : 0.0f;
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

// Descending bitonic sort of MT * S packed keys held S per thread (element i = tid * S + s). Pairs closer than S are
// in one thread, closer than WAVE * S in one wave (lane shuffles); only the three widest steps go through LDS (buf,
// MT * S entries), each between two barriers.
template <int S>
__device__ __forceinline__ void sort_regs(uint64_t (&v)[S], uint64_t *buf) {
  constexpr int N = MT * S;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          if ((s ^ j) > s) {
            const bool desc = ((tid * S + s) & k) == 0;
            const uint64_t x = v[s], y = v[s ^ j];
            if (desc ? (x < y) : (x > y)) {
              v[s] = y;
              v[s ^ j] = x;
            }
          }
        }
      } else {
        uint64_t o[S];
        if (j < WAVE * S) {
#pragma unroll
          for (int s = 0; s < S; ++s) o[s] = shfl_xor_u64(v[s], j / S);
        } else {
#pragma unroll
          for (int s = 0; s < S; ++s) buf[tid * S + s] = v[s];
          __syncthreads();
#pragma unroll
          for (int s = 0; s < S; ++s) o[s] = buf[(tid * S + s) ^ j];
          __syncthreads();
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int i = tid * S + s;
          const bool keep_max = (((i & k) == 0) == ((i & j) == 0));  // lower of a descending pair, upper of an ascending
          v[s] = keep_max ? (o[s] > v[s] ? o[s] : v[s]) : (o[s] < v[s] ? o[s] : v[s]);
        }
      }
    }
  }
}

// a[0, n) (n <= MT * S, in LDS) sorted descending by sort_regs, tmp (MT * S entries) its buffer; zero pads sort last.
// Out of line: inlined, its unrolled network held the registers of the code around it (the main pass spilled).
template <int S>
__device__ __noinline__ void sort_lds_regs(uint64_t *a, uint64_t *tmp, int n) {
  const int tid = threadIdx.x;
  uint64_t v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) v[s] = tid * S + s < n ? a[tid * S + s] : 0ull;
  sort_regs<S>(v, tmp);
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (tid * S + s < n) a[tid * S + s] = v[s];
  __syncthreads();
}

// Sorts a[0, n) (packed keys, descending: key desc, then token id asc) in place, every key in [klo, khi], by the whole
// workgroup (MT threads): a counting sort over NB buckets of equal key width (count, scan, scatter into tmp), then each
// element's rank inside its bucket by counting; a bucket larger than BK (many equal or close keys: bf16 logits tie
// often) makes the whole array take a bitonic sort instead, in registers (sort_regs: four or eight elements a thread,
// only its three widest steps through LDS) for n <= 8 MT. a and tmp hold at least pow2_ceil(n) entries, bcnt and bofs
// NB; wsum NWV words, bmax one word of scratch. Rolled loops elsewhere: compact code (this runs once per row, from a
// cold instruction cache). Ends with a barrier.
template <int NB, int BK>
__device__ __forceinline__ void sort_desc_counting(uint64_t *a, uint64_t *tmp, uint32_t *bcnt, uint32_t *bofs,
                                                   uint32_t *wsum, uint32_t *bmax, int n, uint32_t khi, uint32_t klo) {
  static_assert(NB % MT == 0, "");
  const int tid = threadIdx.x;
  const uint32_t span = khi - klo;
  int shift = 0;
  while ((span >> shift) >= (uint32_t)NB) ++shift;
  for (int b = tid; b < NB; b += MT) bcnt[b] = 0;
  if (tid == 0) *bmax = 0;
  __syncthreads();
#pragma unroll 1
  for (int i = tid; i < n; i += MT) atomicAdd(&bcnt[(khi - pk_key(a[i])) >> shift], 1u);
  __syncthreads();
  // bucket starts: NB / MT buckets per thread, contiguous
  constexpr int BPT = NB / MT;
  uint32_t c[BPT], loc = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    c[j] = bcnt[tid * BPT + j];
    loc += c[j];
    mx = max(mx, c[j]);
  }
  const uint32_t inc = wave_incl_scan_u32(loc);
  mx = wave_max_u32(mx);
  if (lane_id() == WAVE - 1) wsum[tid >> 6] = inc;
  if (lane_id() == 0) atomicMax(bmax, mx);
  __syncthreads();
  uint32_t run = inc - loc;
  for (int w = 0; w < NWV; ++w) run += w < (tid >> 6) ? wsum[w] : 0u;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    bofs[tid * BPT + j] = run;
    bcnt[tid * BPT + j] = run;  // (the running end while scattering)
    run += c[j];
  }
  __syncthreads();
  if (*bmax <= (uint32_t)BK) {
#pragma unroll 1
    for (int i = tid; i < n; i += MT) {
      const uint64_t v = a[i];
      tmp[atomicAdd(&bcnt[(khi - pk_key(v)) >> shift], 1u)] = v;
    }
    __syncthreads();
#pragma unroll 1
    for (int i = tid; i < n; i += MT) {
      const uint64_t v = tmp[i];
      const uint32_t b = (khi - pk_key(v)) >> shift;
      const uint32_t b0 = bofs[b], b1 = bcnt[b];
      uint32_t r = b0, q = b0;
      // (eight reads in flight per round: a bucket of dozens of tied keys, common with bf16 logits, costs a few LDS
      // round trips instead of one per member)
#pragma unroll 1
      for (; q + 8 <= b1; q += 8) {
        uint64_t t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = tmp[q + k];
#pragma unroll
        for (int k = 0; k < 8; ++k) r += t[k] > v ? 1u : 0u;
      }
#pragma unroll 1
      for (; q < b1; ++q) r += tmp[q] > v ? 1u : 0u;
      a[r] = v;
    }
    __syncthreads();
  } else if (n <= 4 * MT) {
    sort_lds_regs<4>(a, tmp, n);
  } else if (n <= 8 * MT) {
    sort_lds_regs<8>(a, tmp, n);
  } else {
    int N = 2;
    while (N < n) N <<= 1;
    for (int i = n + tid; i < N; i += MT) a[i] = 0ull;
    __syncthreads();
#pragma unroll 1
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll 1
      for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll 1
        for (int i = tid; i < N / 2; i += MT) {
          const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1)), hi = lo + j;
          const uint64_t x = a[lo], y = a[hi];
          if ((lo & k) == 0 ? x < y : x > y) {
            a[lo] = y;
            a[hi] = x;
          }
        }
        __syncthreads();
      }
    }
  }
}

// An all-ones mask word: what unmasked rows read in place of their mask words in load_full.
static __device__ const uint32_t ONES_WORD[1] = {0xFFFFFFFFu};

// A full chunk [cb, cb + CHK) of the row (every token inside the slice) into registers, with no bounds branches, so that
// the compiler can count the loads in flight: every call issues the same loads. valid false reads the row's first chunk
// instead (the row must hold CHK tokens) and the caller ignores it. Unmasked rows read ONES_WORD as their mask words.
template <int DT, bool AL>
__device__ __forceinline__ void load_full(const RowCtx &c, int cb, bool valid, float (&x)[EPL],
                                          uint32_t (&mw)[Lay<DT>::NV]) {
  using L = Lay<DT>;
  const int l = lane_id();
  const int b = valid ? cb : 0;
  const uint32_t *mp = c.mw ? c.mw : ONES_WORD;
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = b + v * L::STRIDE + l * L::VEC;
    mw[v] = mp[c.mw ? t0 >> 5 : 0];
    if constexpr (DT == GSE_F32) {
      if constexpr (AL) {
        const float4 f = *reinterpret_cast<const float4 *>((const float *)c.base + t0);
        x[4 * v] = f.x;
        x[4 * v + 1] = f.y;
        x[4 * v + 2] = f.z;
        x[4 * v + 3] = f.w;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[4 * v + k] = ((const float *)c.base)[t0 + k];
      }
    } else {
      if constexpr (AL) {
        const uint4 u = *reinterpret_cast<const uint4 *>((const uint16_t *)c.base + t0);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[8 * v + 2 * i] = __uint_as_float(w[i] << 16);
          x[8 * v + 2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[8 * v + k] = bf16_to_f32(((const uint16_t *)c.base)[t0 + k]);
      }
    }
  }
}

// Per-lane running state of a wave.
struct Lane {
  float m;         // running maximum of this lane's z
  double s;        // sum of this lane's unlisted exp(z - m) (fp32 terms)
  double b;        // its error bound
  uint32_t kap;    // the wave's listing threshold key in force (uniform in the wave; only rises)
  uint32_t woff;   // elements the wave has listed (uniform)
  float g;         // greedy rows: largest nan_to_num(x) so far, at token gid (the first one)
  uint32_t gid;
  uint32_t fid;    // first token of this lane with z not NaN (the lowest -inf when the row has no z > -inf)
  bool fnan, ffin;
};

// Phase 1 of a chunk: penalties, NaN test (before the mask), mask, z in place. Returns the lane's chunk maximum of z.
template <int DT>
__device__ __forceinline__ float chunk_phase1(const ScanArgs &a, const RowCtx &c, int row, int cb, int p0, int p1,
                                              float (&xr)[EPL], const uint32_t (&mw)[Lay<DT>::NV], Lane &ln,
                                              const HistTab &h) {
  using L = Lay<DT>;
  constexpr uint32_t VMASK = (1u << L::VEC) - 1u;
  const int l = lane_id();
  const bool divide = c.divide;
  const double Rd = c.Rd;
  float *proc = a.processed ? a.processed + (int64_t)row * a.processed_ld : nullptr;
  float cmax = -INFINITY;
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = cb + v * L::STRIDE + l * L::VEC;
    uint32_t bits = (mw[v] >> ((l * L::VEC) & 31)) & VMASK;
    if (t0 + L::VEC > p1) bits &= t0 >= p1 ? 0u : (1u << (p1 - t0)) - 1u;  // past the part end
    if (c.pen && t0 < p1) {
      const int o = t0 - p0;
      const uint32_t hw = h.bits[o >> 5];
      const uint32_t hb = (hw >> (o & 31)) & VMASK;
      if (hb) {
#pragma unroll
        for (int k = 0; k < L::VEC; ++k) {
          if ((hb >> k) & 1u) {
            const int ok = o + k;
            const uint32_t r = h.pre[ok >> 5] + __popc(h.bits[ok >> 5] & ((1u << (ok & 31)) - 1u));
            xr[v * L::VEC + k] = penalize(xr[v * L::VEC + k], h.cnt[min(r, (uint32_t)HMAX - 1u)], c.rp, c.fp,
                                          c.pp);
          }
        }
      }
    }
    if (bits == VMASK) {  // every token of the vector allowed
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        const float x = xr[i];
        ln.fnan |= (x != x);
        ln.ffin |= fabsf(x) < INFINITY;
        if (proc) proc[t0 + k] = x;
        const float z = divide ? div_exact(x, Rd) : x;
        xr[i] = z;
        cmax = fmaxf(cmax, z);
      }
    } else {
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        const float x = xr[i];
        ln.fnan |= (x != x);  // (a token past the part end loads 0)
        const bool al = (bits >> k) & 1u;
        const float xm = al ? x : -INFINITY;
        ln.ffin |= fabsf(xm) < INFINITY;
        if (proc && t0 + k < p1) proc[t0 + k] = xm;
        const float z = (divide && al) ? div_exact(x, Rd) : xm;
        xr[i] = z;
        cmax = fmaxf(cmax, z);
      }
    }
  }
  // the first token with z not NaN (only until this lane has one)
  if (ln.fid == 0xFFFFFFFFu) {
#pragma unroll
    for (int i = EPL - 1; i >= 0; --i) {
      const int t = cb + (i / L::VEC) * L::STRIDE + l * L::VEC + (i % L::VEC);
      if (t < p1 && xr[i] == xr[i]) ln.fid = (uint32_t)t;
    }
  }
  if (c.greedy) {  // first maximum of nan_to_num(x) (sampling.py:76), in token order
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const float g = fminf(fmaxf(xr[i], -FLTMAX), FLTMAX);
      const int t = cb + (i / L::VEC) * L::STRIDE + l * L::VEC + (i % L::VEC);
      if (t < p1 && xr[i] == xr[i] && (g > ln.g || ln.gid == 0xFFFFFFFFu)) {
        ln.g = g;
        ln.gid = (uint32_t)t;
      }
    }
  }
  return cmax;
}

}  // namespace strm
}  // namespace gse
