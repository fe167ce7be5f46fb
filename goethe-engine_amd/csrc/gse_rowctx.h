// Per-row element pipeline shared by the scan and the exact path: logit -> penalties -> NaN test -> mask -> key.
#pragma once
#include "gse_dev.h"
#include "gse_int.h"

namespace gse {

struct RowCtx {
  const char *base;  // row start
  int dtype, V;
  bool greedy, divide, pen;
  float T, rp, fp, pp;
  double Td, Rd;
  const uint32_t *mw;  // packed mask words of the row, or null
  int hb, he;          // history range
};

// Greedy rows: temperature 0 in sample mode (sampling.py:78 samples only t > 0). A positive t whose float32 is 0 is
// sampled and divides by 0, as sampling.py:61 does.
__device__ __forceinline__ bool is_greedy(int mode, const gse_row &P) {
  return mode == MODE_SAMPLE && P.temperature == 0.0f && !(P.flags & GSE_ROW_TEMP_UNDERFLOW);
}

__device__ __forceinline__ RowCtx make_ctx(const ScanArgs &a, int row, const gse_row &P) {
  RowCtx c;
  size_t es = a.dtype == GSE_BF16 ? 2 : 4;
  c.base = (const char *)a.logits + (size_t)row * (size_t)a.ld * es;
  c.dtype = a.dtype;
  c.V = a.V;
  c.greedy = is_greedy(a.mode, P);
  c.T = P.temperature;
  c.divide = !c.greedy && P.temperature != 1.0f;
  c.Td = (double)P.temperature;
  c.Rd = 1.0 / c.Td;
  c.rp = P.repetition_penalty;
  c.fp = P.frequency_penalty;
  c.pp = P.presence_penalty;
  c.hb = P.hist_begin;
  c.he = P.hist_end;
  c.pen = a.hist != nullptr && P.hist_end > P.hist_begin &&
          (P.repetition_penalty != 1.0f || P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f);
  c.mw = (a.mask != nullptr && P.mask_row >= 0) ? (const uint32_t *)(a.mask + (int64_t)P.mask_row * a.mask_ld) : nullptr;
  return c;
}

__device__ __forceinline__ float load_one(const RowCtx &c, int t) {
  if (c.dtype == GSE_BF16) return bf16_to_f32(((const uint16_t *)c.base)[t]);
  return ((const float *)c.base)[t];
}

// Rebuilds the LDS count table cnt[0, N) for tokens [c0, c0 + N) from the row's history. Ends with a barrier.
template <int N = CH>
__device__ __forceinline__ void build_counts(const RowCtx &c, const int32_t *hist, int c0, uint32_t *cnt) {
  static_assert(N % 4 == 0, "");
  for (int i = threadIdx.x; i < N / 4; i += blockDim.x) reinterpret_cast<uint4 *>(cnt)[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  for (int j = c.hb + (int)threadIdx.x; j < c.he; j += blockDim.x) {
    int t = hist[j];
    if (t >= c0 && t < c0 + N && t < c.V) atomicAdd(&cnt[t - c0], 1u);
  }
  __syncthreads();
}

// One element: x is the raw logit of token t (cnt_t its history count, 0 when no penalty applies).
// Returns the key (greedy: nan_to_num of the masked logit, sampling.py:76; otherwise z = x / float32(T), sampling.py:61),
// and updates the row flags. xm receives the processed logit (penalties and mask applied).
__device__ __forceinline__ uint32_t elem_key(const RowCtx &c, float x, uint32_t cnt_t, bool allowed, bool &fnan,
                                             bool &ffin, float &xm) {
  if (cnt_t) x = penalize(x, cnt_t, c.rp, c.fp, c.pp);
  fnan |= (x != x);
  xm = allowed ? x : -INFINITY;
  ffin |= (fabsf(xm) < INFINITY);
  if (c.greedy) {
    float y = (xm != xm) ? -INFINITY : fminf(fmaxf(xm, -3.402823466e+38f), 3.402823466e+38f);
    return fkey(y);
  }
  float z = c.divide ? div_rn(x, c.T, c.Td, c.Rd) : x;
  return allowed ? fkey(z) : KEY_NEGINF;
}

__device__ __forceinline__ bool mask_bit(const RowCtx &c, int t) {
  return c.mw == nullptr || ((c.mw[t >> 5] >> (t & 31)) & 1u);
}

}  // namespace gse
