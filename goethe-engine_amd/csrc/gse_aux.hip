// The rest of the selection call surface: dist (vocabulary-order fp64 probabilities), draw (vocabulary-order inverse
// CDF), mss (multi-step speculative sampling) and the bool -> packed mask conversion.
#include "gse_rowctx.h"

namespace gse {

namespace {

constexpr int AT = 256;  // threads of the elementwise kernels

// ---- dist: sampling.py:88-97 -------------------------------------------------------------------------------------------
// out[t] = q_t * keep_t / sum(q * keep) with q = exp(z - z_max) / S; keep_t = packed(key_t, t) >= packed key of the last
// kept rank. Rows whose z holds +inf / NaN or whose maximum is -inf give NaN everywhere, as numpy does.
__global__ __launch_bounds__(AT) void dist_kernel(ScanArgs a, double *probs, int64_t pld) {
  __shared__ uint32_t cnt[CH];
  const int row = blockIdx.y, chunk = blockIdx.x, c0 = chunk * CH;
  const gse_row P = a.params[row];
  const RowCtx c = make_ctx(a, row, P);
  const RowInfo ri = a.info[row];
  double *out = probs + (int64_t)row * pld;
  const bool nan_row = !(ri.flags & R_DONE) || (ri.flags & (R_SPECIAL | R_BAD));
  if (c.pen && !nan_row) build_counts(c, a.hist, c0, cnt);
  const double M = (double)fkey_inv(pk_key(ri.cmax));
  for (int i = threadIdx.x; i < CH; i += AT) {
    const int t = c0 + i;
    if (t >= c.V) break;
    if (nan_row) {
      out[t] = __builtin_nan("");
      continue;
    }
    bool fn = false, ff = false;
    float xm;
    const uint32_t k = elem_key(c, load_one(c, t), c.pen ? cnt[i] : 0u, mask_bit(c, t), fn, ff, xm);
    double v = 0.0;
    if (pack(k, (uint32_t)t) >= ri.kkeep && k > KEY_NEGINF) v = (exp((double)fkey_inv(k) - M) / ri.S) / ri.Z;
    out[t] = v;
  }
}

// ---- draw: sampling.py:100-104 -------------------------------------------------------------------------------------------
// One workgroup per row: thread-contiguous partial sums, a block scan, then the first index whose inclusive cumulative
// sum reaches u * total; clamped to the last index with q > 0.
constexpr int DT = 1024;

struct ScanTmp {
  double w[DT / WAVE];
  int found, last;
};

__device__ __forceinline__ double block_excl_scan_f64(double v, ScanTmp &st, double &total) {
  const double inc = wave_incl_scan_f64(v);
  __syncthreads();
  if (lane_id() == WAVE - 1) st.w[threadIdx.x >> 6] = inc;
  __syncthreads();
  double pre = 0.0, tot = 0.0;
  const int w = threadIdx.x >> 6;
  for (int k = 0; k < DT / WAVE; ++k) {
    if (k < w) pre += st.w[k];
    tot += st.w[k];
  }
  total = tot;
  __syncthreads();
  return pre + inc - v;
}

// Returns the drawn index for one row q[0, V) at u (every thread gets it). -1 when no q is positive.
__device__ int draw_row(const double *q, int V, double u, ScanTmp &st) {
  const int tid = threadIdx.x;
  const int per = (V + DT - 1) / DT;
  const int b = tid * per, e = min(V, b + per);
  double s = 0.0;
  int last = -1;
  for (int i = b; i < e; ++i) {
    const double v = q[i];
    s += v;
    if (v > 0.0) last = i;
  }
  if (tid == 0) {
    st.found = 0x7FFFFFFF;
    st.last = -1;
  }
  double total;
  const double pre = block_excl_scan_f64(s, st, total);
  atomicMax(&st.last, last);
  const double thr = u * total;
  double c = pre;
  for (int i = b; i < e; ++i) {
    c += q[i];
    if (c >= thr) {
      atomicMin(&st.found, i);
      break;
    }
  }
  __syncthreads();
  int j = st.found;
  const int lastpos = st.last;
  __syncthreads();
  if (j == 0x7FFFFFFF) j = (thr != thr) ? 0 : V;
  if (lastpos < 0) return -1;
  return j < lastpos ? j : lastpos;
}

__global__ __launch_bounds__(DT) void draw_kernel(const double *q, int64_t ld, int V, const double *u, int32_t *out) {
  __shared__ ScanTmp st;
  const int row = blockIdx.x;
  const int j = draw_row(q + (int64_t)row * ld, V, u[row], st);
  if (threadIdx.x == 0) out[row] = j;
}

// ---- mss: spec.py:88-103 --------------------------------------------------------------------------------------------------
constexpr uint64_t SALT_ACC = 1ull << 40, SALT_RES = 1ull << 41;

__global__ __launch_bounds__(DT) void mss_kernel(gse_mss_batch b) {
  __shared__ ScanTmp st;
  __shared__ double red[DT / WAVE];
  const int node = blockIdx.x, tid = threadIdx.x;
  const int V = (int)b.vocab;
  double *p = b.p + (int64_t)node * b.p_ld;
  const uint64_t seed = b.seed[node], i = b.idx[node];
  for (int r = 0; r < (int)b.max_kids; ++r) {
    const int x = b.kid_tok[(int64_t)node * b.max_kids + r];
    if (x < 0) break;
    if (x >= V) continue;  // not a token of this vocabulary (the Python layer raises before launching)
    const int qr = b.kid_q[(int64_t)node * b.max_kids + r];
    const double *q = qr >= 0 ? b.q + (int64_t)qr * b.q_ld : nullptr;
    const double qx = q ? q[x] : 1.0;
    const double px = p[x];
    if (qx > 0.0 && uniform64(mix64(seed, SALT_ACC + (uint64_t)r), i) * qx < px) {
      if (tid == 0) {
        b.out_token[node] = x;
        b.out_kid[node] = r;
      }
      return;
    }
    __syncthreads();  // every thread has read p[x] before it changes
    // residual: max(p - q, 0) (or p with p[x] = 0 for a one-hot kid), renormalised when its sum is positive
    const int per = (V + DT - 1) / DT;
    const int lo = tid * per, hi = min(V, lo + per);
    double s = 0.0;
    for (int k = lo; k < hi; ++k) {
      double v = p[k];
      if (q) {
        v = v - q[k];
        v = v > 0.0 ? v : 0.0;
      } else if (k == x) {
        v = 0.0;
      }
      p[k] = v;
      s += v;
    }
    s = wave_sum_f64(s);
    if (lane_id() == 0) red[tid >> 6] = s;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < DT / WAVE; ++w) tot += red[w];
    if (tot > 0.0)
      for (int k = lo; k < hi; ++k) p[k] = p[k] / tot;
    __syncthreads();
  }
  const int j = draw_row(p, V, uniform64(mix64(seed, SALT_RES), i), st);
  if (tid == 0) {
    b.out_token[node] = j;
    b.out_kid[node] = -1;
  }
}

// ---- q of a drafter row: spec.py:157 (q = softmax(float64(x) / t)) -------------------------------------------------------
// One workgroup per row: the maximum of x (z = x / t is monotone in x and rounds once, so max z = (max x) / t), the mass
// E = sum exp(z - M) in fixed point (the same sum in any order, exp_nonpos within 1.5 ulp), then q = exp(z - M) / E. A
// row holding NaN, +inf, or no value above -inf gives NaN everywhere, as torch.softmax does.
__global__ __launch_bounds__(DT) void qprob_kernel(gse_qrows q, int V, double *out, int64_t ld) {
  __shared__ double etab[64];
  __shared__ double redd[DT / WAVE];
  __shared__ uint64_t redh[DT / WAVE], redl[DT / WAVE];
  const int row = blockIdx.x, tid = threadIdx.x, w = tid >> 6;
  const bool bf = q.kind == GSE_Q_LOGITS_BF16;
  const char *base = (const char *)q.q + (size_t)row * (size_t)q.ld * (bf ? 2 : 4);
  const double t = q.temperature[row];
  double *o = out + (int64_t)row * ld;
  auto xat = [&](int i) -> double {
    return bf ? (double)bf16_to_f32(((const uint16_t *)base)[i]) : (double)((const float *)base)[i];
  };
  if (tid < 64) etab[tid] = EXP2_64[tid];
  double m = -INFINITY;
  bool nan = false;
  for (int i = tid; i < V; i += DT) {
    const double x = xat(i);
    nan |= x != x;
    m = fmax(m, x);
  }
  m = lane63(wave_scan(m, (double)-INFINITY, [](double a, double b) { return fmax(a, b); }));
  const bool wnan = ballot64(nan) != 0ull;
  if (lane_id() == 0) redd[w] = wnan ? __builtin_nan("") : m;
  __syncthreads();
  double M = -INFINITY;
  bool bad = false;
  for (int k = 0; k < DT / WAVE; ++k) {
    bad |= redd[k] != redd[k];
    M = fmax(M, redd[k]);
  }
  M = M / t;
  bad = bad || !(fabs(M) < INFINITY);
  if (bad) {
    for (int i = tid; i < V; i += DT) o[i] = __builtin_nan("");
    return;
  }
  Fx f = {0, 0};
  for (int i = tid; i < V; i += DT) f = fx_add(f, fx_of(exp_nonpos(xat(i) / t - M, etab)));
  f.hi = wave_sum_u64(f.hi);
  f.lo = wave_sum_u64(f.lo);
  if (lane_id() == 0) {
    redh[w] = f.hi;
    redl[w] = f.lo;
  }
  __syncthreads();
  Fx tot = {0, 0};
  for (int k = 0; k < DT / WAVE; ++k) tot = fx_add(tot, Fx{redh[k], redl[k]});
  const double E = fx_val(tot);
  for (int i = tid; i < V; i += DT) o[i] = exp_nonpos(xat(i) / t - M, etab) / E;
}

// ---- bool rows -> packed words (grammar.py:44-45 inverted) ---------------------------------------------------------------
__global__ __launch_bounds__(AT) void pack_kernel(const uint8_t *bools, int64_t bld, int V, int32_t *words, int64_t wld) {
  const int row = blockIdx.y;
  const int w = blockIdx.x * AT + threadIdx.x;
  const int nw = (V + 31) / 32;
  if (w >= nw) return;
  const uint8_t *src = bools + (int64_t)row * bld + (int64_t)w * 32;
  uint32_t v = 0;
  for (int k = 0; k < 32; ++k) {
    const int t = w * 32 + k;
    if (t < V && src[k]) v |= 1u << k;
  }
  words[(int64_t)row * wld + w] = (int32_t)v;
}

// ---- zero fill (a kernel, not hipMemsetAsync, so that a caller may capture it in a graph) ----------------------------
__global__ __launch_bounds__(AT) void zero_kernel(uint4 *p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * AT + threadIdx.x; i < n; i += (size_t)gridDim.x * AT) p[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

hipError_t launch_zero(void *p, size_t bytes, hipStream_t s) {
  const size_t n = bytes / sizeof(uint4);  // (bytes: a multiple of 256)
  const unsigned g = (unsigned)(n / AT < 4096 ? (n + AT - 1) / AT : 4096);
  if (n) hipLaunchKernelGGL(zero_kernel, dim3(g > 0 ? g : 1), dim3(AT), 0, s, (uint4 *)p, n);
  return hipGetLastError();
}

hipError_t launch_dist_write(const ScanArgs &a, double *probs, int64_t probs_ld, hipStream_t s) {
  hipLaunchKernelGGL(dist_kernel, dim3(a.nch, a.rows), dim3(AT), 0, s, a, probs, probs_ld);
  return hipGetLastError();
}

hipError_t launch_draw(const double *q, int64_t ld, int rows, int V, const double *u, int32_t *out, hipStream_t s) {
  hipLaunchKernelGGL(draw_kernel, dim3(rows), dim3(DT), 0, s, q, ld, V, u, out);
  return hipGetLastError();
}

hipError_t launch_mss(const gse_mss_batch &b, hipStream_t s) {
  hipLaunchKernelGGL(mss_kernel, dim3(b.nodes), dim3(DT), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_qprob(const gse_qrows &q, int V, double *out, int64_t ld, hipStream_t s) {
  hipLaunchKernelGGL(qprob_kernel, dim3(q.rows), dim3(DT), 0, s, q, V, out, ld);
  return hipGetLastError();
}

hipError_t launch_pack(const uint8_t *bools, int64_t bld, int rows, int V, int32_t *words, int64_t wld, hipStream_t s) {
  const int nw = (V + 31) / 32;
  hipLaunchKernelGGL(pack_kernel, dim3((nw + AT - 1) / AT, rows), dim3(AT), 0, s, bools, bld, V, words, wld);
  return hipGetLastError();
}

}  // namespace gse
