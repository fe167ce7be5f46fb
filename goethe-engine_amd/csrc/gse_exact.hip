// Exact radix-select path: one workgroup per row that the scan marked hard (1024 threads in the exact launch here, 256
// inside the split-row launch: the same body, gse_exact_body.h, in two shapes). It finds the keep prefix and the draw
// of goethe_engine/sampling.py:77-83 without sorting the row:
//
//   m   = min(top_k, #{q_i >= min_p * q_0}, first rank with cumsum(q)_i - q_i >= top_p)    (sampling.py:80)
//   j   = first rank with cumsum(q)_i >= u * c_last, c_last = cumsum(q)_{m-1}             (sampling.py:81-83)
//
// The head of the row (at most HEADN top elements, cut at a bin of the key histogram that the max pass counts) is
// collected into LDS and sorted once; a rank / mass query whose answer lies in it is a walk of that list. Any other
// query walks a histogram of the 32-bit key (4096 bins, 12 key bits per level; 1024 and 10 in the 256-thread shape;
// count and mass per bin), then collects the one bin that holds the answer into LDS and sorts it; a bin too large to
// collect is refined with a histogram of its own key range, and a single key with more elements than fit is ordered
// by token id (the stable order).
// Masses are exact sums of per-element fixed-point values (2^-64 resolution), so every prefix is deterministic and
// the same whichever order the atomics land in.
#include "gse_rowctx.h"

namespace gse {

namespace {

// The 1024-thread shape: the exact launch, for calls without the split-row launch (GSE_BATCH_NO_SPLIT, or a handle
// without split-row slots). Otherwise the split-row launch finishes the hard rows itself (gse_deep.hip, 256 threads).
namespace x1024 {
constexpr int XT = 1024;   // threads
constexpr int NB = 4096;   // histogram bins
constexpr int LB = 12;     // key bits per histogram level
constexpr int CAPS = 8192; // collected elements
constexpr int CHX = CH;    // tokens per chunk
#include "gse_exact_body.h"
__shared__ ExactShared xsh;
__device__ __forceinline__ ExactShared &xs() { return xsh; }
}  // namespace x1024
using namespace x1024;

constexpr int XGRID = 256;  // workgroups of the exact pass, at most (one per CU; every row when all are forced)

// The exact pass, launched when the split-row launch is not (GSE_BATCH_NO_SPLIT, GSE_BATCH_EXACT): with
// GSE_BATCH_EXACT one workgroup per row; otherwise a small grid, workgroup g owning the rows r = g (mod grid): it finds
// its hard ones (one scan of their flags, compacted in row order) and finishes them, so that a call with no hard row
// costs a launch and one round of loads.
__global__ __launch_bounds__(XT) void exact_kernel(ScanArgs a) {
  ExactShared &sh = xsh;
  __shared__ uint32_t wn[XT / WAVE];
  __shared__ int hrow[XT];
  // (the call's counts, deep rows and other hard rows, cleared for the next call)
  if (blockIdx.x == 0 && threadIdx.x == 0) *reinterpret_cast<uint64_t *>(a.dctl) = 0ull;
  const int G = (int)gridDim.x, w = threadIdx.x / WAVE;
  // A workgroup with no hard row ends here, before the set-up of the row code (its registers and spill slots).
  bool any = false;
  for (int r = (int)blockIdx.x + (int)threadIdx.x * G; r < a.rows; r += XT * G) any |= (a.info[r].flags & R_HARD) != 0;
  if (!__syncthreads_or(any)) return;
  for (int j0 = 0; (int)blockIdx.x + j0 * G < a.rows; j0 += XT) {
    const int r = (int)blockIdx.x + (j0 + (int)threadIdx.x) * G;
    const bool hard = r < a.rows && (a.info[r].flags & R_HARD);
    const uint64_t bl = ballot64(hard);
    if (lane_id() == 0) wn[w] = (uint32_t)__popcll(bl);
    __syncthreads();
    uint32_t base = 0, n = 0;
#pragma unroll
    for (int k = 0; k < XT / WAVE; ++k) {
      base += k < w ? wn[k] : 0u;
      n += wn[k];
    }
    if (hard) hrow[base + lanes_below(bl)] = r;
    __syncthreads();
    for (uint32_t i = 0; i < n; ++i) {
      exact_row(a, hrow[i], sh);
      __syncthreads();  // (LDS of the row)
    }
  }
}

}  // namespace

hipError_t launch_exact(const ScanArgs &a, hipStream_t s) {
  const int grid = a.force_exact ? a.rows : (a.rows < XGRID ? a.rows : XGRID);  // (forced: one row per workgroup)
  hipLaunchKernelGGL(exact_kernel, dim3(grid), dim3(XT), 0, s, a);
  return hipGetLastError();
}

}  // namespace gse
