/* Oracle (test infrastructure): an independent C restatement of the integer and byte parts of the reference's
 * token-selection path, used to pin the numpy oracle and the HIP path on the integer work.
 *
 *   ora_mix / ora_uniform   goethe_engine/sampling.py:42-51  splitmix64 of seed + (i + 1) * golden, (mix >> 11) / 2^53
 *   ora_greedy              goethe_engine/sampling.py:70-76,84  bad = NaN anywhere (before the mask) or no finite value
 *                           after the mask -> -1; else first index of the maximum of nan_to_num(x masked)
 *                           (NaN -> -inf, +inf -> FLT_MAX, -inf -> -FLT_MAX; masked tokens are -inf first)
 *   ora_unpack              goethe_engine/grammar.py:44-45   bit t % 32 of word t / 32, LSB first
 */
#include <float.h>
#include <math.h>
#include <stdint.h>

uint64_t ora_mix(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

double ora_uniform(uint64_t seed, uint64_t idx) { return (double)(ora_mix(seed, idx) >> 11) / 9007199254740992.0; }

static float nan_to_num(float v) {
  if (isnan(v)) return -INFINITY;
  if (isinf(v)) return v > 0 ? FLT_MAX : -FLT_MAX;
  return v;
}

/* rows x v fp32 logits (row stride ld); words: packed mask rows (wpr words per row) or NULL; out: token per row. */
void ora_greedy(const float *x, int64_t ld, int32_t rows, int32_t v, const int32_t *words, int32_t wpr, int32_t *out) {
  for (int32_t r = 0; r < rows; ++r) {
    const float *row = x + (int64_t)r * ld;
    const uint32_t *w = words ? (const uint32_t *)words + (int64_t)r * wpr : 0;
    int bad = 0, finite = 0, best = 0;
    float bv = 0;
    for (int32_t t = 0; t < v; ++t) {
      float a = row[t];
      if (isnan(a)) bad = 1;
      if (w && !((w[t >> 5] >> (t & 31)) & 1u)) a = -INFINITY;
      if (isfinite(a)) finite = 1;
      float k = nan_to_num(a);
      if (t == 0 || k > bv) { bv = k; best = t; }
    }
    out[r] = (bad || !finite) ? -1 : best;
  }
}

void ora_unpack(const int32_t *words, int32_t v, uint8_t *out) {
  const uint32_t *w = (const uint32_t *)words;
  for (int32_t t = 0; t < v; ++t) out[t] = (uint8_t)((w[t >> 5] >> (t & 31)) & 1u);
}
