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
  F_OVERFLOW = 4u,  // a slice's candidate list did not fit, or a history longer than the u16 counts allow
};

enum : uint32_t {
  R_GREEDY = 1u,   // temperature 0 in sample mode
  R_BAD = 2u,      // token -1
  R_SPECIAL = 4u,  // processed z holds +inf, or its maximum is -inf / NaN: token = order[0], dist = NaN
  R_HARD = 8u,     // the exact path must finish the row
  R_DONE = 16u,
  R_FULL = 32u,    // with R_HARD: the exact path also recomputes the flags and the greedy argmax
};

enum { MODE_SAMPLE = 0, MODE_DIST = 1 };

constexpr int CAPW = 512;   // candidates listed per wave per part
constexpr int PWAVES = 4;   // waves per part workgroup
constexpr int MAXP = 64;    // parts per row
constexpr int PTOK = 40960; // tokens per part, at most
constexpr int PCHUNK = 1024;  // part lengths are multiples of this (one wave chunk)

// One per (row, part), written by the part's workgroup with agent-scope stores, read by the row's resolve.
struct SliceRec {    // 64 bytes
  uint64_t top;      // packed (key, lowest id): of nan_to_num(x)'s maximum for greedy rows; of -inf for sampled rows
                     // (used when the row has no z > -inf)
  uint32_t kappa;    // certified key: every element of the part with key >= kappa is in its waves' lists
  uint32_t flags;    // F_*
  uint32_t mkey;     // key of the part maximum of z (z = x for greedy rows)
  uint32_t wcnt[PWAVES];  // elements listed by each wave (<= CAPW)
  uint32_t pad0;
  double s;          // sum over the part's unlisted elements of exp(z - z_part_max), fp32 exp2 terms
  double bnd;        // absolute error bound of s
  uint32_t pad[2];
};
static_assert(sizeof(SliceRec) == 64, "");

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
  int dtype, V, rows, nch, mode, force_exact, xcd_map;
  int nparts, plen;  // the main pass: parts per row, tokens per part (a multiple of 1024; the last part may be shorter)
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
  SliceRec *rec;    // [rows][nparts]: one record per part
  uint64_t *cand;   // [rows][nparts][PWAVES][CAPW]
  RowInfo *info;
  uint32_t *done;   // [rows] slice tickets, zero between calls
};

hipError_t launch_main(const ScanArgs &a, hipStream_t s);
hipError_t launch_exact(const ScanArgs &a, hipStream_t s);
hipError_t launch_dist_write(const ScanArgs &a, double *probs, int64_t probs_ld, hipStream_t s);
hipError_t launch_draw(const double *q, int64_t ld, int rows, int V, const double *u, int32_t *out, hipStream_t s);
hipError_t launch_mss(const gse_mss_batch &b, hipStream_t s);
hipError_t launch_pack(const uint8_t *bools, int64_t bld, int rows, int V, int32_t *words, int64_t wld, hipStream_t s);

}  // namespace gse
