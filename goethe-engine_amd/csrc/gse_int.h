// Internal structures of libgse: workspace records and kernel launch wrappers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gse.h"

namespace gse {

// Fixed-point masses: an fp64 value in [0, 1] as hi * 2^-40 + lo * 2^-64 (gse_dev.h fx_of). Sums of up to 2^24 of them
// add hi and lo separately with no carry, so a sum is the same whatever order its terms are added in.
struct Fx {
  uint64_t hi, lo;
};

static_assert(sizeof(gse_row) == 72, "gse_row layout is part of the ABI");

enum : uint32_t {
  F_NAN = 1u,       // a NaN in the row after penalties (before the mask): the row is bad (sampling.py:71)
  F_FINITE = 2u,    // a finite value after the mask (sampling.py:75)
  F_OVERFLOW = 4u,  // a wave's candidate list did not fit
  F_HOVER = 8u,     // a part with more distinct history ids than its count table holds
  F_PINF = 16u,     // +inf as the part maximum of z (x = +inf, or x / T overflowing): the exact path decides
};

enum : uint32_t {
  R_GREEDY = 1u,   // temperature 0 in sample mode
  R_BAD = 2u,      // token -1
  R_SPECIAL = 4u,  // processed z holds +inf, or its maximum is -inf / NaN: token = order[0], dist = NaN
  R_HARD = 8u,     // the exact path must finish the row
  R_DONE = 16u,
  R_FULL = 32u,    // with R_HARD: the exact path also recomputes the flags and the greedy argmax
  R_DEEP = 64u,    // with R_HARD: the split-row finish (gse_deep.hip) takes the row first
  R_BY_DEEP = 128u,   // finished by the split-row finish
  R_BY_EXACT = 256u,  // finished by the exact path
};

enum { MODE_SAMPLE = 0, MODE_DIST = 1 };

constexpr int CH = 8192;  // tokens per slice (the exact path, dist, and the verify and pick passes walk rows in these)
// gse_sample_noalloc's static workspace: batches of at most this many rows of at most this many tokens.
constexpr uint32_t NOALLOC_ROWS = 32;
constexpr uint32_t NOALLOC_VOCAB = 163840;
static_assert(NOALLOC_ROWS == GSE_NOALLOC_ROWS && NOALLOC_VOCAB == GSE_NOALLOC_VOCAB, "gse.h states the limits");

constexpr int CAPW = 512;   // candidates listed per wave per part
constexpr int PWAVES = 4;   // waves per part workgroup
constexpr int MAXP = 64;    // parts per row
constexpr int PTOK = 65536; // tokens per part, at most
constexpr int PTOK_PLAIN = 131072;  // tokens per part, at most, in a call with no histories and no masks (no part-sized
                                    // LDS tables: the parts are twice as long and the listing targets twice as high)
constexpr int KT = 200;       // tokens of a part of at most PTOK tokens its listing threshold aims to leave above it
constexpr int KT_HM = 150;    // the same in a call with histories or masks: its rows' heads certify with shorter lists,
                              // which the resolve gathers and sorts faster (much lower and some rows need the exact path)
constexpr int KT_VALVE = 222; // the listing target at which a part's first-chunk valve is CAPW / 4 (scaled with kt)
constexpr int PCHUNK = 1024;  // part lengths are multiples of this (one wave chunk)
constexpr int PMIN = 8192;    // tokens per part, at least, when a small batch is split to fill the device: every part
                              // lists its own candidates, so more parts make a longer row resolve

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

// Split-row finish of deep rows (gse_deep.hip).
constexpr int DEEP_MAX = 1024;  // split-row slots at most (a handle has min(max_rows, DEEP_MAX); more deep rows: the
                                // exact path takes them)
constexpr int DSMAX = 64;      // slices per deep row, at most
constexpr int DNB = 512;       // histogram bins of d = z_max - z, 1/32 wide (the last one open-ended)
constexpr int DCAP = 8192;     // window elements listed per deep row

enum : uint32_t { DS_PENDING = 0u, DS_PLANNED = 1u, DS_FAIL = 2u };

// DeepSlot::plan: the status in bits 0-7, then the windows w2lo, w2hi, w1lo, w1hi (inclusive bins, 12 bits each).
__host__ __device__ constexpr uint64_t plan_word(uint32_t st, uint32_t w2lo, uint32_t w2hi, uint32_t w1lo,
                                                 uint32_t w1hi) {
  return (uint64_t)st | (uint64_t)w2lo << 8 | (uint64_t)w2hi << 20 | (uint64_t)w1lo << 32 | (uint64_t)w1hi << 44;
}
__host__ __device__ constexpr uint32_t plan_status(uint64_t p) { return (uint32_t)(p & 0xFFu); }
__host__ __device__ constexpr uint32_t plan_win(uint64_t p, int i) {  // 0: w2lo, 1: w2hi, 2: w1lo, 3: w1hi
  return (uint32_t)(p >> (8 + 12 * i)) & 0xFFFu;
}

enum {  // DeepSlot.acc: exact fixed-point masses of the plan's regions (hi: 2^-40 units, lo: 2^-64 units) and counts
  DA_X0HI, DA_X0LO,  // bins before the draw window
  DA_X1HI, DA_X1LO,  // bins strictly between the two windows
  DA_RHI, DA_RLO,    // the other bins (the windows and after)
  DA_C0, DA_C1,      // element counts of the first two regions (from the count pass)
  DA_C2,             // elements after the cut window (from the count pass)
  DA_N
};

struct DeepSlot {    // 256 bytes, one per deep row of a call
  gse_row P;         // the row's parameters, copied by the row resolve of the main pass
  int32_t row;
  float M;           // maximum of z
  double u;          // the draw's uniform
  uint64_t plan;     // the planner's word (plan_word): DS_* status and the bin windows holding the draw and the last
                     // kept element, stored whole, so that a slice that sees the status also has the windows
  uint32_t lcnt;                    // listed window elements
  uint32_t cdone, pdone;            // slice tickets of the two passes (zero between calls)
  uint32_t pad0;
  uint64_t acc[DA_N];               // the plan's region sums and counts
  uint32_t spoil;                   // a slice gave up waiting for the plan: the exact path takes the row (zero between calls)
  uint32_t pad32;
  uint64_t pad[8];
};
static_assert(sizeof(DeepSlot) == 256, "");

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
  int kt, vfirst;    // tokens of a part its listing threshold aims to leave above it; list length that first opens the valve
  int pmajor;        // workgroup L streams part L / rows8 of row L % rows8 (else the parts of a row are consecutive)
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
  uint64_t *cand;   // [rows][nparts][PWAVES][CAPW]: listed elements, (bits of z) << 32 | token
  RowInfo *info;
  uint32_t *done;   // [rows] slice tickets, zero between calls
  // split-row finish
  uint32_t *dctl;    // [0..1]: the call's counts, one 64-bit word (low: deep rows; high: other hard rows); [2], [3]: tickets
  DeepSlot *dslot;   // [DEEP_MAX]
  uint64_t *dhist;   // [DEEP_MAX][3][DNB]: per bin, element count and exact mass (2^-40 and 2^-64 parts), atomic adds
  uint64_t *dlist;   // [DEEP_MAX][DCAP]: packed keys of the window elements
  int dslots;          // split-row slots of the workspace
  int dslices, dgrid;  // split-row finish enabled (slices per deep row, at most), workgroups per pass
  uint64_t plan_wait;  // wall-clock ticks (100 MHz) a split-row pick slice waits for its row's plan
  int fin_sorted;      // the split-row finish sorts short window lists whole (else every list takes the sub-bin walk)
  int tree;            // a verify round (gse_verify_tree): GSE_ROW_MSS rows need dist's keep boundary, not a token
  int32_t pstart[MAXP + 1];  // part p of every row is [pstart[p], pstart[p + 1]) (multiples of 1024; pstart[nparts] = V)
};

// Verify round state of one node (gse_tree.hip), in the handle's workspace.
struct TreeNode {
  uint32_t next;     // residual pass the next launch runs for this node (0: decided)
  uint32_t ticket;   // slice ticket of the current pass (zero between passes)
  int32_t token;     // the decision: the node's token and the accepted kid row (-1 none)
  int32_t kid;
  double clast;      // exact kept mass C = sum(keep exp(z - M)) of dist()
  double sig[GSE_MAX_KIDS + 1];  // totals of the residuals res_1.. (sig[0] = C)
};

struct QFin {        // a logits q row: max of z = x / t and the exact mass sum exp(z - M)
  double M, E;
  uint32_t ticket, pad;
};

struct TreeLaunch {
  ScanArgs s;
  const int32_t *parent, *token, *qrow, *anchor;
  gse_qrows q;
  int max_kids, requests;
  const int32_t *sampled;
  TreeNode *st;
  Fx *npart;
  int32_t *nlast;
  uint64_t *tseg;
  uint32_t *plist, *pcnt;  // [GSE_MAX_KIDS + 1][rows]: the nodes each residual pass r takes; [GSE_MAX_KIDS + 1]: counts
  int pgrid;               // workgroups of a residual pass
  double *qmax;
  Fx *qpart;
  QFin *qfin;
  gse_tree_out out;
};

struct PickLaunch {
  gse_pick_batch b;
  double *pmax;
  Fx *ppart;
  int32_t *plast;
  uint64_t *ptop;
  uint32_t *tick;
};

// Byte layout of a device workspace for max_rows x max_vocab; target: main-pass workgroups to aim for (4 per CU).
// Every buffer starts on a 256-byte boundary; the whole block starts zeroed (the kernels keep their tickets, slot
// counters and flags zero between calls). tree: with the buffers of verify rounds and drafter picks.
struct Layout {
  size_t rec, cand, info, done, dctl, dslot, dhist, dlist;
  size_t ttok, tstate, npart, nlast, tseg, qmax, qpart, qfin, pmax, ppart, plast, ptop, ptick, plist, pcnt;
  size_t total;
  uint32_t nrec, nsl, slots;
};

constexpr size_t al256(size_t x) { return (x + 255) / 256 * 256; }

constexpr Layout plan_layout(uint32_t R, uint32_t V, uint32_t target, bool tree) {
  Layout L = {};
  L.nrec = R * ((V + PTOK - 1) / PTOK + 1) + target;
  L.nsl = (V + CH - 1) / CH;
  L.slots = R < (uint32_t)DEEP_MAX ? R : (uint32_t)DEEP_MAX;
  size_t o = 0;
  auto put = [&o](size_t bytes) {
    const size_t at = o;
    o += al256(bytes);
    return at;
  };
  L.rec = put((size_t)L.nrec * sizeof(SliceRec));
  L.cand = put((size_t)L.nrec * PWAVES * CAPW * sizeof(uint64_t));
  L.info = put((size_t)R * sizeof(RowInfo));
  L.done = put((size_t)R * sizeof(uint32_t));
  L.dctl = put(64);
  L.dslot = put((size_t)L.slots * sizeof(DeepSlot));
  L.dhist = put((size_t)L.slots * 3 * DNB * sizeof(uint64_t));
  L.dlist = put((size_t)L.slots * DCAP * sizeof(uint64_t));
  if (tree) {
    const size_t K = GSE_MAX_KIDS + 1, S = L.nsl;
    L.ttok = put((size_t)R * sizeof(int32_t));
    L.tstate = put((size_t)R * sizeof(TreeNode));
    L.npart = put((size_t)R * K * S * sizeof(Fx));
    L.nlast = put((size_t)R * K * S * sizeof(int32_t));
    L.tseg = put((size_t)R * S * 2 * (CH / 64) * sizeof(uint64_t));  // the last residual's 64-token segment sums
    L.qmax = put((size_t)R * S * sizeof(double));
    L.qpart = put((size_t)R * S * sizeof(Fx));
    L.qfin = put((size_t)R * sizeof(QFin));
    L.pmax = put((size_t)R * S * sizeof(double));
    L.ppart = put((size_t)R * S * sizeof(Fx));
    L.plast = put((size_t)R * S * sizeof(int32_t));
    L.ptop = put((size_t)R * S * 4 * GSE_MAX_KIDS * sizeof(uint64_t));
    L.ptick = put((size_t)R * sizeof(uint32_t));
    L.plist = put((size_t)(GSE_MAX_KIDS + 1) * R * sizeof(uint32_t));  // the nodes of each residual pass
    L.pcnt = put((GSE_MAX_KIDS + 1) * sizeof(uint32_t));
  }
  L.total = o;
  return L;
}

hipError_t launch_main(const ScanArgs &a, hipStream_t s);
hipError_t launch_deep(const ScanArgs &a, hipStream_t s);
hipError_t launch_exact(const ScanArgs &a, hipStream_t s);
hipError_t launch_dist_write(const ScanArgs &a, double *probs, int64_t probs_ld, hipStream_t s);
hipError_t launch_draw(const double *q, int64_t ld, int rows, int V, const double *u, int32_t *out, hipStream_t s);
hipError_t launch_mss(const gse_mss_batch &b, hipStream_t s);
// The verify round after the selection pass (the statistics of the q rows given as drafter logits included).
hipError_t launch_tree(const TreeLaunch &L, hipStream_t s);
hipError_t launch_pick(const PickLaunch &L, hipStream_t s);
hipError_t launch_zero(void *p, size_t bytes, hipStream_t s);
hipError_t launch_qprob(const gse_qrows &q, int V, double *out, int64_t ld, hipStream_t s);
hipError_t launch_pack(const uint8_t *bools, int64_t bld, int rows, int V, int32_t *words, int64_t wld, hipStream_t s);

}  // namespace gse
