// Device helpers shared by the selection kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gse.h"
#include "gse_int.h"

namespace gse {

constexpr int WAVE = 64;

// Order-preserving 32-bit keys of fp32 values: larger value -> larger key; -0 and +0 share a key (numpy's stable
// argsort sees them as equal); NaN -> 0, below every other key (numpy sorts NaN of -z last).
constexpr uint32_t KEY_NEGINF = 0x007FFFFFu;
constexpr uint32_t KEY_POSINF = 0xFF800000u;
constexpr uint32_t KEY_ZERO = 0x80000000u;

__device__ __forceinline__ uint32_t fkey(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7FFFFFFFu) == 0u) return KEY_ZERO;
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float fkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Packed sort key: key desc, then token id asc, as one u64 compared descending.
__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - id);
}
__device__ __forceinline__ uint32_t pk_key(uint64_t p) { return (uint32_t)(p >> 32); }
__device__ __forceinline__ uint32_t pk_id(uint64_t p) { return 0xFFFFFFFFu - (uint32_t)p; }

// splitmix64 (goethe_engine/sampling.py:42-47) and uniform (sampling.py:50-51).
__device__ __forceinline__ uint64_t mix64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ double uniform64(uint64_t seed, uint64_t i) {
  return (double)(mix64(seed, i) >> 11) * (1.0 / 9007199254740992.0);
}

// Correctly rounded fp32 x / T. The fp64 quotient q1 (one Markstein correction step from R = RN(1/T)) is within
// about one fp64 ulp of x / T; an fp32 x / T that is not an fp32 midpoint lies at least 2^-49 (relative) away from
// every midpoint, so rounding q1 to fp32 gives RN(x / T) for every normal result. Zero, subnormal, infinite and NaN
// cases take the IEEE fp32 division.
__device__ __forceinline__ float div_rn(float x, float T, double Td, double Rd) {
  double xd = (double)x;
  double q0 = xd * Rd;
  double r = fma(-q0, Td, xd);
  double q1 = fma(r, Rd, q0);
  float z = (float)q1;
  if (!(fabs(q1) >= 0x1p-125) || !(fabs(q1) <= 0x1p+127)) z = x / T;
  return z;
}

// Penalties on one fp32 logit with history count c > 0: repetition, then frequency, then presence, each a separately
// rounded fp32 operation (the file is built with -ffp-contract=off).
__device__ __forceinline__ float penalize(float x, uint32_t c, float rp, float fp, float pp) {
  float y = (x < 0.0f) ? __fmul_rn(x, rp) : __fdiv_rn(x, rp);
  y = __fsub_rn(y, __fmul_rn(fp, (float)c));
  return __fsub_rn(y, pp);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Data one workgroup hands to another workgroup of the same launch goes through agent-scope relaxed atomic stores and
// loads (global_store / global_load with sc1 on gfx950: coherent across the XCDs' L2s), so no L2 writeback or
// invalidate (what __threadfence() emits) is needed. The writer waits for its stores to complete (store_wait) before
// the atomic ticket that publishes them; the reader issues its loads after it has seen the ticket.
template <typename T>
__device__ __forceinline__ T ld_ag(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_ag(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_wait() { __builtin_amdgcn_s_waitcnt(0); }
__device__ __forceinline__ uint32_t ticket_add(uint32_t *p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }

__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int m) { return (uint32_t)__shfl_xor((int)v, m, WAVE); }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = shfl_xor_u32((uint32_t)v, m), hi = shfl_xor_u32((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double shfl_up_f64(double v, int d) {
  int2 b = *reinterpret_cast<int2 *>(&v);
  b.x = __shfl_up(b.x, d, WAVE);
  b.y = __shfl_up(b.y, d, WAVE);
  return *reinterpret_cast<double *>(&b);
}
__device__ __forceinline__ double shfl_f64(double v, int src) {
  int2 b = *reinterpret_cast<int2 *>(&v);
  b.x = __shfl(b.x, src, WAVE);
  b.y = __shfl(b.y, src, WAVE);
  return *reinterpret_cast<double *>(&b);
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, WAVE), hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, WAVE);
  return ((uint64_t)hi << 32) | lo;
}

// Cross-lane moves through DPP (VALU, no LDS round trip): lane l receives v from the lane that CTRL names, or id where
// there is none or its row (16 lanes) is not in ROWM.
template <int CTRL, int ROWM>
__device__ __forceinline__ uint32_t dpp32(uint32_t id, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, ROWM, 0xF, false);
}
template <int CTRL, int ROWM, typename T>
__device__ __forceinline__ T dpp_mov(T id, T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, dpp32<CTRL, ROWM>(__builtin_bit_cast(uint32_t, id), __builtin_bit_cast(uint32_t, v)));
  } else {
    const uint64_t i = __builtin_bit_cast(uint64_t, id), x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp32<CTRL, ROWM>((uint32_t)i, (uint32_t)x);
    const uint32_t hi = dpp32<CTRL, ROWM>((uint32_t)(i >> 32), (uint32_t)(x >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}
// Inclusive scan over the 64 lanes (all active) with op and its identity id, in a fixed association: inside each row
// of 16 lanes by row shifts of 1, 2, 4 and 8, then across rows by the broadcasts of lanes 15 and 31.
template <typename T, typename Op>
__device__ __forceinline__ T wave_scan(T v, T id, Op op) {
  v = op(v, dpp_mov<0x111, 0xF>(id, v));  // row_shr:1
  v = op(v, dpp_mov<0x112, 0xF>(id, v));  // row_shr:2
  v = op(v, dpp_mov<0x114, 0xF>(id, v));  // row_shr:4
  v = op(v, dpp_mov<0x118, 0xF>(id, v));  // row_shr:8
  v = op(v, dpp_mov<0x142, 0xA>(id, v));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_mov<0x143, 0xC>(id, v));  // row_bcast:31 into rows 2 and 3
  return v;
}
// The value of lane 63 (wave-uniform).
template <typename T>
__device__ __forceinline__ T lane63(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  } else {
    const uint64_t x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 63);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

struct OpAdd {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct OpMin {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? a : b; }
};

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return lane63(wave_scan(v, (uint64_t)0, OpMax{})); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return lane63(wave_scan(v, 0u, OpMax{})); }
__device__ __forceinline__ double wave_sum_f64(double v) { return lane63(wave_scan(v, 0.0, OpAdd{})); }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { return lane63(wave_scan(v, (uint64_t)0, OpAdd{})); }
// Inclusive prefix sums over the 64 lanes (fixed association).
__device__ __forceinline__ double wave_incl_scan_f64(double v) { return wave_scan(v, 0.0, OpAdd{}); }
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) { return wave_scan(v, 0u, OpAdd{}); }
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) { return wave_scan(v, (uint64_t)0, OpAdd{}); }

// Bitonic sort of one u32 per lane across the wave, descending: lane i ends with the i-th largest value.
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v) {
  int l = lane_id();
#pragma unroll
  for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint32_t o = shfl_xor_u32(v, j);
      bool take_max = ((l & k) == 0) == ((l & j) == 0);
      uint32_t mx = max(v, o), mn = min(v, o);
      v = take_max ? mx : mn;
    }
  }
  return v;
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// The k-th largest (1-based) of the wave's 64 values: the largest r with at least k values >= r, bit by bit.
__device__ __forceinline__ uint32_t wave_kth_largest_u32(uint32_t v, int k) {
  uint32_t r = 0;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = r | (1u << b);
    if ((int)__popcll(ballot64(v >= c)) >= k) r = c;
  }
  return r;
}

// The same over 16-bit values (v < 2^16).
__device__ __forceinline__ uint32_t wave_kth_largest_u16(uint32_t v, int k) {
  uint32_t r = 0;
#pragma unroll
  for (int b = 15; b >= 0; --b) {
    const uint32_t c = r | (1u << b);
    if ((int)__popcll(ballot64(v >= c)) >= k) r = c;
  }
  return r;
}

__device__ __forceinline__ float wave_max_f32(float v) {
  return lane63(wave_scan(v, -INFINITY, [](float x, float y) { return fmaxf(x, y); }));
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return lane63(wave_scan(v, 0u, OpAdd{})); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return lane63(wave_scan(v, 0xFFFFFFFFu, OpMin{})); }
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Bitonic sort (descending) of n_pow2 u64 values in LDS by the whole workgroup; n_pow2 a power of two.
__device__ __forceinline__ void block_sort_desc_u64(uint64_t *a, int n_pow2) {
  for (int k = 2; k <= n_pow2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n_pow2; i += blockDim.x) {
        int p = i ^ j;
        if (p > i) {
          uint64_t x = a[i], y = a[p];
          bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            a[i] = y;
            a[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// 2^(j / 64), j = 0..63, correctly rounded.
static __constant__ double EXP2_64[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

// e^d in fp64 for d <= 0, within about 1.5 ulp: d = k ln2/64 + r with |r| <= ln2/128 (ln2/64 split in two, k * hi
// exact), e^r - 1 by its degree-5 Taylor polynomial (remainder < 4e-17), 2^(k/64) from the table tab (in LDS). 0 below
// -745 (and for -inf).
__device__ __forceinline__ double exp_nonpos(double d, const double *tab) {
  const double kd = rint(d * 92.33248261689366);  // 64 / ln 2
  double r = fma(-kd, 0x1.62e42ffp-7, d);
  r = fma(-kd, -6.563929801064195e-13, r);
  const double q = r * fma(r, fma(r, fma(r, fma(r, 1.0 / 120.0, 1.0 / 24.0), 1.0 / 6.0), 0.5), 1.0);
  const int k = (int)kd;
  const double t = tab[k & 63];
  const double e = ldexp(fma(t, q, t), k >> 6);
  return d >= -745.0 ? e : 0.0;
}

// Fixed-point masses (Fx, gse_int.h): an fp64 exp(z - M) in [0, 1] as hi * 2^-40 + lo * 2^-64 (both floors, so the
// value is within 2^-64 below the fp64 one).
// The conversions are exact and short: h = floor(s) < 2^52 is an integer, so h + 2^52 holds h in its 52 fraction
// bits; the remainder scaled by 2^24 is below 2^24, and the truncating conversion to u32 is its floor (it is >= 0).
__device__ __forceinline__ Fx fx_of(double e) {
  const double s = e * 1099511627776.0;  // 2^40
  const double h = floor(s);
  Fx f;
  f.hi = (uint64_t)__double_as_longlong(h + 4503599627370496.0) & 0x000FFFFFFFFFFFFFull;  // 2^52
  f.lo = (uint32_t)((s - h) * 16777216.0);                                                 // 2^24
  return f;
}
__device__ __forceinline__ Fx fx_add(Fx a, Fx b) { return Fx{a.hi + b.hi, a.lo + b.lo}; }
__device__ __forceinline__ double fx_val(Fx a) {
  return (double)a.hi * 9.094947017729282e-13 + (double)a.lo * 5.421010862427522e-20;  // 2^-40, 2^-64
}

__host__ __device__ constexpr int pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

}  // namespace gse
