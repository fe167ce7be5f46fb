// Internal structures of libgse: workspace records and kernel launch wrappers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gse.h"

namespace gse {

static_assert(sizeof(gse_row) == 72, "gse_row layout is part of the ABI");

enum : uint32_t {
  F_NAN = 1u,       // a NaN in the row after penalties (before the mask): the row is bad (sampling.py:71)
  F_FINITE = 2u,    // a finite value after the mask (sampling.py:75)
  F_OVERFLOW = 4u,  // a chunk's candidate list did not fit
};

enum : uint32_t {
  R_GREEDY = 1u,   // temperature 0 in sample mode
  R_BAD = 2u,      // token -1
  R_SPECIAL = 4u,  // processed z holds +inf, or its maximum is -inf / NaN: token = order[0], dist = NaN
  R_HARD = 8u,     // the exact radix-select path must finish the row
  R_DONE = 16u,
};

enum { MODE_SAMPLE = 0, MODE_DIST = 1 };

constexpr int CAPC = 256;  // candidates per chunk record
constexpr int CAPW = 128;  // candidates per wave during the scan
constexpr int KW = 16;     // lane maxima per wave that bound the certified threshold
constexpr int CERT_CAP = 4096;

struct ChunkHdr {   // 64 bytes, one per (row, chunk)
  uint64_t cmax;    // packed (key, id) maximum: greedy key in greedy rows, z key otherwise
  uint32_t tau;     // every element of the chunk with key >= tau is in its candidate list
  uint32_t ncand;
  uint32_t flags;
  uint32_t mkey;    // chunk maximum z key
  double sc;        // sum over the chunk of exp(z - z_max_chunk), v_exp_f32 based
  double mom;       // sum of exp(z - z_max_chunk) * |z - z_max_chunk| (error bound of sc)
  uint32_t pad[6];
};
static_assert(sizeof(ChunkHdr) == 64, "");

struct RowInfo {    // 64 bytes, one per row, written by the row resolve, read by the exact path and dist
  uint64_t cmax;    // packed maximum z (key, id)
  uint64_t kkeep;   // packed key of the last kept element (keep prefix boundary)
  double S;         // sum of exp(z - z_max)
  double Z;         // sum of the kept q (c[-1] of sampling.py:81)
  uint32_t flags;   // R_*
  uint32_t ncert;
  int32_t token;
  uint32_t pad[5];
};
static_assert(sizeof(RowInfo) == 64, "");

struct ScanArgs {
  const void *logits;
  int64_t ld;
  int dtype, V, rows, nch, nchmax, mode, force_exact, pad;
  const gse_row *params;
  const int32_t *mask;
  int64_t mask_ld;
  const int32_t *hist;
  const double *uni;
  float *processed;
  int64_t processed_ld;
  int32_t *tokens;
  int32_t *lp_ids;
  float *lps;
  int64_t lp_ld;
  ChunkHdr *hdr;
  uint64_t *cand;
  RowInfo *info;
  uint32_t *done;
};

hipError_t launch_scan(const ScanArgs &a, hipStream_t s);
hipError_t launch_exact(const ScanArgs &a, hipStream_t s);
hipError_t launch_dist_write(const ScanArgs &a, double *probs, int64_t probs_ld, hipStream_t s);
hipError_t launch_draw(const double *q, int64_t ld, int rows, int V, const double *u, int32_t *out, hipStream_t s);
hipError_t launch_mss(const gse_mss_batch &b, hipStream_t s);
hipError_t launch_pack(const uint8_t *bools, int64_t bld, int rows, int V, int32_t *words, int64_t wld, hipStream_t s);

}  // namespace gse
