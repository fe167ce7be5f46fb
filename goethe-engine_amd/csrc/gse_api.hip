// Host side of the C ABI in include/gse.h: handle, device workspace, argument checks, launches.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "gse_dev.h"
#include "gse_int.h"

struct gse_handle {
  int device = 0;
  uint32_t max_rows = 0, max_vocab = 0, nchmax = 0;
  uint32_t nrec = 0;     // part records (and wave lists) in the workspace
  uint32_t target = 0;   // main-pass workgroups to aim for (4 per CU: all resident at once)
  bool owned = false;    // the workspace block came from hipMalloc (gse_open), not the static array
  void *block = nullptr; // the workspace (gse::plan_layout)
  gse::SliceRec *rec = nullptr;
  uint64_t *cand = nullptr;
  gse::RowInfo *info = nullptr;
  uint32_t *done = nullptr;
  uint32_t *dctl = nullptr;           // split-row finish: control word, slots, histograms, parts, window lists
  gse::DeepSlot *dslot = nullptr;
  uint64_t *dhist = nullptr;
  uint64_t *dlist = nullptr;
  uint32_t dslots = 0;                // split-row slots
  // verify rounds and drafter picks (gse_tree.hip): per row slices of the vocabulary, nsl of them at most
  uint32_t nsl = 0;
  int32_t *ttok = nullptr;            // [max_rows] sampled tokens of the verify round's selection pass
  gse::TreeNode *tstate = nullptr;    // [max_rows]
  gse::Fx *npart = nullptr;           // [max_rows][GSE_MAX_KIDS + 1][nsl]
  uint64_t *tseg = nullptr;           // [max_rows][nsl][2 * 128]
  int32_t *nlast = nullptr;           // [max_rows][GSE_MAX_KIDS + 1][nsl]
  double *qmax = nullptr;             // [max_rows][nsl]
  gse::Fx *qpart = nullptr;           // [max_rows][nsl]
  gse::QFin *qfin = nullptr;          // [max_rows]
  double *pmax = nullptr;             // [max_rows][nsl]
  gse::Fx *ppart = nullptr;           // [max_rows][nsl]
  int32_t *plast = nullptr;           // [max_rows][nsl]
  uint64_t *ptop = nullptr;           // [max_rows][nsl][4 * GSE_MAX_KIDS]
  uint32_t *ptick = nullptr;
  uint32_t *plist = nullptr;          // [GSE_MAX_KIDS + 1][max_rows] nodes of each verify residual pass
  uint32_t *pcnt = nullptr;           // [GSE_MAX_KIDS + 1]          // [max_rows]
  hipEvent_t (*ring)[5] = nullptr;  // kernel boundaries of up to GSE_PROFILE_CALLS profiled calls
  int nring = 0;                    // calls recorded
  int nprof = 0;                    // kernels per recorded call
  bool is_static = false;           // gse_sample_noalloc's per-device handle: its errors go to the thread's fixed
                                    // buffer (no host allocation on that path)
  std::string err;
};

namespace {

thread_local char g_open_err[512];  // errors of calls without a handle (gse_open, gse_sample_noalloc)

int fail(gse_handle *h, int rc, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(gse_handle *h, int rc, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (h && !h->is_static) h->err = buf;
  else memcpy(g_open_err, buf, sizeof buf);
  return rc;
}

int hip_fail(gse_handle *h, hipError_t e, const char *what) {
  return fail(h, GSE_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

// Copies min(caller size, own size) bytes of a size-first struct; absent fields stay zero.
template <typename T>
bool take(const T *src, T &dst) {
  memset(&dst, 0, sizeof dst);
  if (!src) return false;
  uint32_t n = src->size;
  if (n < 8) return false;
  memcpy(&dst, src, n < sizeof(T) ? n : sizeof(T));
  return true;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// The event slot of the next profiled call (kernels per call must stay the same between two reads).
int prof_slot(gse_handle *h, int kernels, hipEvent_t **ev) {
  *ev = nullptr;
  if (!h->ring) {
    h->ring = new (std::nothrow) hipEvent_t[GSE_PROFILE_CALLS][5]();  // (null handles until created)
    if (!h->ring) return fail(h, GSE_E_DEVICE, "out of host memory");
    for (int c = 0; c < GSE_PROFILE_CALLS; ++c)
      for (int i = 0; i < 5; ++i) {
        hipError_t e = hipEventCreate(&h->ring[c][i]);
        if (e != hipSuccess) return hip_fail(h, e, "event create");
      }
  }
  if (h->nring > 0 && h->nprof != kernels) h->nring = 0;
  h->nprof = kernels;
  if (h->nring >= GSE_PROFILE_CALLS) return GSE_OK;  // record full: later calls run unprofiled until the next read
  *ev = h->ring[h->nring++];
  return GSE_OK;
}

int check_batch(gse_handle *h, const gse_batch &b) {
  if (!b.logits || !b.params) return fail(h, GSE_E_ARG, "logits and params are required");
  if (b.dtype != GSE_F32 && b.dtype != GSE_BF16) return fail(h, GSE_E_ARG, "dtype %u is neither f32 nor bf16", b.dtype);
  if (b.vocab == 0) return fail(h, GSE_E_ARG, "vocab is 0");
  if (b.ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "ld %lld < vocab %u", (long long)b.ld, b.vocab);
  if (b.rows > h->max_rows)
    return fail(h, GSE_E_CAPACITY, "%u rows, the handle was opened for %u", b.rows, h->max_rows);
  if (b.vocab > h->max_vocab)
    return fail(h, GSE_E_CAPACITY, "vocab %u, the handle was opened for %u", b.vocab, h->max_vocab);
  if (b.mask && b.mask_ld < (int64_t)((b.vocab + 31) / 32))
    return fail(h, GSE_E_ARG, "mask_ld %lld < ceil(vocab / 32)", (long long)b.mask_ld);
  return GSE_OK;
}

// Parts per row for the main pass: each at most ptok tokens (PTOK, or PTOK_PLAIN), a multiple of PCHUNK long, and
// enough of them over the batch to give every CU about four workgroups, as long as a part keeps at least PMIN tokens.
// rows * parts <= rows * (ceil(vocab / PTOK) + 1) + target.
void parts(const gse_handle *h, uint32_t rows, uint32_t vocab, uint32_t ptok, int *nparts, int *plen) {
  const uint32_t nck = (vocab + gse::PCHUNK - 1) / gse::PCHUNK;
  uint32_t np = (vocab + ptok - 1) / ptok;
  uint32_t want = (h->target + rows - 1) / rows;
  const uint32_t cap = vocab / gse::PMIN > 1u ? vocab / gse::PMIN : 1u;
  if (want > cap) want = cap;
  if (want > np) np = want;
  if (np > (uint32_t)gse::MAXP) np = gse::MAXP;
  if (np > nck) np = nck;
  const uint32_t len = ((vocab + np - 1) / np + gse::PCHUNK - 1) / gse::PCHUNK * gse::PCHUNK;
  *plen = (int)len;
  *nparts = (int)((vocab + len - 1) / len);
}

// Part boundaries of the main pass. By default the parts of a row are equal and its workgroups consecutive. When the
// batch is one resident round of three or four part workgroups per CU, the workgroups go part-major instead (L streams
// part L / rows8 of row L % rows8: every row has one part in each quarter of the dispatch order, and all parts of a row
// still share an XCD) and a part's length follows its quarter: the workgroups that reach a CU later stream slower, as
// the oldest wave wins issue and memory arbitration, at measured rates (C3, MI355X) of 1 : 0.89 : 0.73 : 0.63 by
// quarter, so parts in that proportion end a row's streams together instead of leaving the last quarter's rows behind.
void part_layout(const gse_handle *h, gse::ScanArgs &a) {
  const int np = a.nparts, V = a.V;
  for (int p = 0; p <= np; ++p) a.pstart[p] = p < np ? p * a.plen : V;
  a.pmajor = 0;
  const int rows8 = a.xcd_map ? (a.rows + 7) / 8 * 8 : a.rows;
  const int64_t wgs = (int64_t)rows8 * np;
  if (!a.xcd_map || np < 4 || np % 4 || wgs > (int64_t)h->target || 4 * wgs < 3 * (int64_t)h->target) return;
  static const double RATE[4] = {1.0, 0.89, 0.73, 0.63};
  double tot = 0.0;
  for (int p = 0; p < np; ++p) tot += RATE[(4 * p) / np];
  int32_t b[gse::MAXP + 1];
  double c = 0.0;
  b[0] = 0;
  for (int p = 1; p < np; ++p) {
    c += RATE[(4 * (p - 1)) / np];
    b[p] = (int32_t)((int64_t)(c / tot * V + gse::PCHUNK / 2) / gse::PCHUNK * gse::PCHUNK);
  }
  b[np] = V;
  for (int p = 0; p < np; ++p)  // (every part non-empty and within the part capacity, else the equal layout stays)
    if (b[p + 1] <= b[p] || b[p + 1] - b[p] > gse::PTOK) return;
  for (int p = 0; p <= np; ++p) a.pstart[p] = b[p];
  a.pmajor = 1;
}

void deep_grid(const gse_handle *h, uint32_t rows, int *nsl, int *grid) {
  const uint32_t slots = rows < h->dslots ? rows : h->dslots;
  const uint32_t items = slots * (uint32_t)gse::DSMAX;
  *nsl = gse::DSMAX;
  *grid = (int)(items < h->target ? items : h->target);
}

gse::ScanArgs make_args(gse_handle *h, const gse_batch &b, int mode) {
  gse::ScanArgs a = {};
  a.logits = b.logits;
  a.ld = b.ld;
  a.dtype = (int)b.dtype;
  a.V = (int)b.vocab;
  a.rows = (int)b.rows;
  a.nch = (int)((b.vocab + gse::CH - 1) / gse::CH);
  // A call with no histories and no masks keeps no part-sized tables in LDS: its parts may be twice as long (a large
  // batch then streams its rows in half the workgroups, each with one prologue and one first-chunk latency for twice
  // the tokens), and a part's listing target and valve grow with its length, so that a row lists as many candidates.
  const bool plain = !b.hist && !b.mask;
  parts(h, b.rows, b.vocab, plain ? (uint32_t)gse::PTOK_PLAIN : (uint32_t)gse::PTOK, &a.nparts, &a.plen);
  a.kt = a.plen > gse::PTOK ? (int)(((int64_t)gse::KT * a.plen + gse::PTOK - 1) / gse::PTOK)
                            : plain ? gse::KT : gse::KT_HM;
  a.vfirst = (int)((int64_t)gse::CAPW / 4 * a.kt / gse::KT_VALVE) + 1;
  a.mode = mode;
  a.xcd_map = 1;
  a.force_exact = (b.flags & GSE_BATCH_EXACT) ? 1 : 0;
  a.plan_wait = (b.flags & GSE_BATCH_NO_PLAN_WAIT) ? 0u : 400000u;  // 4 ms: only a grid the device cannot hold waits it out
  a.fin_sorted = (b.flags & GSE_BATCH_SUBBIN_FINISH) ? 0 : 1;
  a.params = b.params;
  a.mask = b.mask;
  a.mask_ld = b.mask_ld;
  a.hist = b.hist;
  a.uni = b.uniforms;
  a.rec = h->rec;
  a.cand = h->cand;
  a.info = h->info;
  a.done = h->done;
  a.dctl = h->dctl;
  a.dslot = h->dslot;
  a.dhist = h->dhist;
  a.dlist = h->dlist;
  a.dslots = (int)h->dslots;
  deep_grid(h, b.rows, &a.dslices, &a.dgrid);
  // Without the split-row launch the exact launch finishes the hard rows (the resolve sends them there: no slots);
  // with it, that launch finishes every hard row itself. A forced exact call takes the 1024-thread exact launch.
  if (b.flags & (GSE_BATCH_NO_SPLIT | GSE_BATCH_EXACT)) {
    a.dslices = 0;
    a.dgrid = 0;
  }
  part_layout(h, a);
  return a;
}

// Points the handle's buffers into a workspace block laid out by gse::plan_layout.
void carve(gse_handle *h, void *block, const gse::Layout &L, bool tree) {
  char *b = (char *)block;
  h->block = block;
  h->nrec = L.nrec;
  h->nsl = L.nsl;
  h->dslots = L.slots;
  h->rec = (gse::SliceRec *)(b + L.rec);
  h->cand = (uint64_t *)(b + L.cand);
  h->info = (gse::RowInfo *)(b + L.info);
  h->done = (uint32_t *)(b + L.done);
  h->dctl = (uint32_t *)(b + L.dctl);
  h->dslot = (gse::DeepSlot *)(b + L.dslot);
  h->dhist = (uint64_t *)(b + L.dhist);
  h->dlist = (uint64_t *)(b + L.dlist);
  if (!tree) return;
  h->ttok = (int32_t *)(b + L.ttok);
  h->tstate = (gse::TreeNode *)(b + L.tstate);
  h->npart = (gse::Fx *)(b + L.npart);
  h->tseg = (uint64_t *)(b + L.tseg);
  h->nlast = (int32_t *)(b + L.nlast);
  h->qmax = (double *)(b + L.qmax);
  h->qpart = (gse::Fx *)(b + L.qpart);
  h->qfin = (gse::QFin *)(b + L.qfin);
  h->pmax = (double *)(b + L.pmax);
  h->ppart = (gse::Fx *)(b + L.ppart);
  h->plast = (int32_t *)(b + L.plast);
  h->ptop = (uint64_t *)(b + L.ptop);
  h->ptick = (uint32_t *)(b + L.ptick);
  h->plist = (uint32_t *)(b + L.plist);
  h->pcnt = (uint32_t *)(b + L.pcnt);
}


// ---- the static workspace of gse_sample_noalloc --------------------------------------------------------------------
// One per GPU: a file-scope device array (each device holds its own copy from the library's load until the process
// ends), laid out like a handle's workspace for NOALLOC_ROWS x NOALLOC_VOCAB. Host code never uses the array's name as
// an address: hipGetSymbolAddress gives each device's address once, at that device's first call, and the handle of
// that device keeps it.
constexpr uint32_t NOALLOC_TARGET = 1024;  // main-pass workgroups aimed for (4 per CU of a 256-CU device, at most)
constexpr gse::Layout NOALLOC_LAYOUT = gse::plan_layout(gse::NOALLOC_ROWS, gse::NOALLOC_VOCAB, NOALLOC_TARGET, false);
static __device__ __align__(256) uint8_t scratch[NOALLOC_LAYOUT.total];

constexpr int NOALLOC_DEVICES = 64;
std::mutex g_static_mu;
gse_handle g_static[NOALLOC_DEVICES];
bool g_static_ready[NOALLOC_DEVICES];

// The handle of the current device over its static workspace; the first call on a device finds the array's address
// there, checks the device, and clears the workspace with a fill kernel on stream s (ordered before the call's own
// kernels).
int static_handle(gse_handle **out, hipStream_t s) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(nullptr, GSE_E_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_DEVICES) return fail(nullptr, GSE_E_DEVICE, "device %d: at most %d", dev, NOALLOC_DEVICES);
  std::lock_guard<std::mutex> lk(g_static_mu);
  gse_handle *h = &g_static[dev];
  if (!g_static_ready[dev]) {
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, dev)) != hipSuccess)
      return fail(nullptr, GSE_E_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      return fail(nullptr, GSE_E_DEVICE, "device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
    void *ptr = nullptr;
    if ((e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != hipSuccess || !ptr)
      return fail(nullptr, GSE_E_DEVICE, "static workspace address: %s", hipGetErrorString(e));
    if ((e = gse::launch_zero(ptr, NOALLOC_LAYOUT.total, s)) != hipSuccess)
      return fail(nullptr, GSE_E_DEVICE, "static workspace clear: %s", hipGetErrorString(e));
    h->device = dev;
    h->is_static = true;
    h->max_rows = gse::NOALLOC_ROWS;
    h->max_vocab = gse::NOALLOC_VOCAB;
    h->nchmax = (gse::NOALLOC_VOCAB + gse::CH - 1) / gse::CH;
    const uint32_t t = 4u * (uint32_t)(prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256);
    h->target = t < NOALLOC_TARGET ? t : NOALLOC_TARGET;
    carve(h, ptr, NOALLOC_LAYOUT, false);
    g_static_ready[dev] = true;
  }
  *out = h;
  return GSE_OK;
}

// gse_sample's checks and launches on a handle (its own workspace, or the static one of gse_sample_noalloc).
int sample_impl(gse_handle *h, const gse_batch &b, const gse_out &o) {
  int rc = check_batch(h, b);
  if (rc) return rc;
  if (!o.tokens) return fail(h, GSE_E_ARG, "tokens output is required");
  if ((o.logprob_ids == nullptr) != (o.logprobs == nullptr))
    return fail(h, GSE_E_ARG, "logprob_ids and logprobs go together");
  if (o.logprob_ids && o.logprobs_ld < GSE_MAX_LOGPROBS && o.logprobs_ld <= 0)
    return fail(h, GSE_E_ARG, "logprobs_ld must be > 0");
  if (o.processed && o.processed_ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "processed_ld < vocab");
  if (b.rows == 0) return GSE_OK;
  gse::ScanArgs a = make_args(h, b, gse::MODE_SAMPLE);
  a.processed = o.processed;
  a.processed_ld = o.processed_ld;
  a.tokens = o.tokens;
  a.lp_ids = o.logprob_ids;
  a.lps = o.logprobs;
  a.lp_ld = o.logprobs_ld;
  hipStream_t s = (hipStream_t)b.stream;
  hipEvent_t *ev = nullptr;
  if ((b.flags & GSE_BATCH_PROFILE) && (rc = prof_slot(h, 3, &ev)) != GSE_OK) return rc;
  hipError_t e;
  if (ev && (e = hipEventRecord(ev[0], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if ((e = gse::launch_main(a, s)) != hipSuccess) return hip_fail(h, e, "main launch");
  if (ev && (e = hipEventRecord(ev[1], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if (a.dgrid > 0 && (e = gse::launch_deep(a, s)) != hipSuccess) return hip_fail(h, e, "deep launch");
  if (ev && (e = hipEventRecord(ev[2], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if (a.dgrid == 0 && (e = gse::launch_exact(a, s)) != hipSuccess) return hip_fail(h, e, "exact launch");
  if (ev && (e = hipEventRecord(ev[3], s)) != hipSuccess) return hip_fail(h, e, "event record");
  return GSE_OK;
}

}  // namespace

extern "C" {

GSE_API uint32_t gse_abi_version(void) { return GSE_ABI_VERSION; }

GSE_API int gse_open(const gse_open_params *p, gse_handle **out) {
  gse_open_params o;
  if (!out || !take(p, o)) return fail(nullptr, GSE_E_ARG, "gse_open: null or short gse_open_params");
  *out = nullptr;
  if (o.max_rows == 0 || o.max_vocab == 0) return fail(nullptr, GSE_E_ARG, "max_rows and max_vocab must be > 0");
  if (o.max_vocab > (1u << 21)) return fail(nullptr, GSE_E_CAPACITY, "max_vocab %u > 2^21", o.max_vocab);
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess || ndev == 0) return fail(nullptr, GSE_E_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (o.device < 0 || o.device >= ndev) return fail(nullptr, GSE_E_DEVICE, "device %d of %d", o.device, ndev);
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, o.device)) != hipSuccess)
    return fail(nullptr, GSE_E_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, GSE_E_DEVICE, "device %d is %s; this library is built for gfx950", o.device, prop.gcnArchName);
  gse_handle *h = new (std::nothrow) gse_handle();
  if (!h) return fail(nullptr, GSE_E_DEVICE, "out of host memory");
  DeviceGuard g(o.device);
  h->device = o.device;
  h->max_rows = o.max_rows;
  h->max_vocab = o.max_vocab;
  h->nchmax = (o.max_vocab + gse::CH - 1) / gse::CH;
  h->target = 4u * (uint32_t)(prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256);
  const gse::Layout L = gse::plan_layout(h->max_rows, h->max_vocab, h->target, true);
  void *block = nullptr;
  if ((e = hipMalloc(&block, L.total)) != hipSuccess || (e = hipMemset(block, 0, L.total)) != hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess) {
    if (block) (void)hipFree(block);
    fail(nullptr, GSE_E_DEVICE, "workspace allocation (%zu bytes): %s", L.total, hipGetErrorString(e));
    delete h;
    return GSE_E_DEVICE;
  }
  h->owned = true;
  carve(h, block, L, true);
  *out = h;
  return GSE_OK;
}

GSE_API int gse_sample(gse_handle *h, const gse_batch *in, const gse_out *out) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_batch b;
  gse_out o;
  if (!take(in, b) || !take(out, o)) return fail(h, GSE_E_ARG, "null or short gse_batch / gse_out");
  DeviceGuard g(h->device);
  return sample_impl(h, b, o);
}

GSE_API int gse_sample_noalloc(const gse_batch *in, const gse_out *out) {
  gse_batch b;
  gse_out o;
  if (!take(in, b) || !take(out, o)) return fail(nullptr, GSE_E_ARG, "null or short gse_batch / gse_out");
  if (b.flags & GSE_BATCH_PROFILE)
    return fail(nullptr, GSE_E_UNSUPPORTED, "gse_sample_noalloc: GSE_BATCH_PROFILE allocates events; use gse_sample");
  if (b.rows > gse::NOALLOC_ROWS || b.vocab > gse::NOALLOC_VOCAB)
    return fail(nullptr, GSE_E_CAPACITY,
                "gse_sample_noalloc: %u rows of %u tokens; its static workspace holds at most %u rows of at most %u "
                "tokens (use gse_open / gse_sample for more)", b.rows, b.vocab, gse::NOALLOC_ROWS, gse::NOALLOC_VOCAB);
  gse_handle *h = nullptr;
  int rc = static_handle(&h, (hipStream_t)b.stream);
  if (rc) return rc;
  return sample_impl(h, b, o);  // (its errors land in the thread's fixed buffer: gse_last_error(NULL))
}

GSE_API int gse_dist(gse_handle *h, const gse_batch *in, double *probs, int64_t probs_ld) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_batch b;
  if (!take(in, b)) return fail(h, GSE_E_ARG, "null or short gse_batch");
  int rc = check_batch(h, b);
  if (rc) return rc;
  if (!probs || probs_ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "probs missing or probs_ld < vocab");
  if (b.rows == 0) return GSE_OK;
  DeviceGuard g(h->device);
  gse::ScanArgs a = make_args(h, b, gse::MODE_DIST);
  hipStream_t s = (hipStream_t)b.stream;
  hipEvent_t *ev = nullptr;
  if ((b.flags & GSE_BATCH_PROFILE) && (rc = prof_slot(h, 4, &ev)) != GSE_OK) return rc;
  hipError_t e;
  if (ev && (e = hipEventRecord(ev[0], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if ((e = gse::launch_main(a, s)) != hipSuccess) return hip_fail(h, e, "main launch");
  if (ev && (e = hipEventRecord(ev[1], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if (a.dgrid > 0 && (e = gse::launch_deep(a, s)) != hipSuccess) return hip_fail(h, e, "deep launch");
  if (ev && (e = hipEventRecord(ev[2], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if (a.dgrid == 0 && (e = gse::launch_exact(a, s)) != hipSuccess) return hip_fail(h, e, "exact launch");
  if (ev && (e = hipEventRecord(ev[3], s)) != hipSuccess) return hip_fail(h, e, "event record");
  if ((e = gse::launch_dist_write(a, probs, probs_ld, s)) != hipSuccess) return hip_fail(h, e, "dist launch");
  if (ev && (e = hipEventRecord(ev[4], s)) != hipSuccess) return hip_fail(h, e, "event record");
  return GSE_OK;
}

GSE_API int gse_verify_tree(gse_handle *h, const gse_batch *in, const gse_tree *tree, const gse_tree_out *out) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_batch b;
  gse_tree t;
  gse_tree_out o;
  if (!take(in, b) || !take(tree, t) || !take(out, o)) return fail(h, GSE_E_ARG, "null or short gse_batch / gse_tree / gse_tree_out");
  int rc = check_batch(h, b);
  if (rc) return rc;
  if (t.requests == 0 || b.rows == 0) return GSE_OK;
  if (!t.anchor || !t.parent || !t.token) return fail(h, GSE_E_ARG, "tree anchor, parent and token are required");
  if (t.requests > b.rows) return fail(h, GSE_E_ARG, "%u requests over %u node rows", t.requests, b.rows);
  if (t.max_kids > GSE_MAX_KIDS) return fail(h, GSE_E_UNSUPPORTED, "max_kids %u > %d", t.max_kids, GSE_MAX_KIDS);
  if (!o.emit_len || !o.emit_tokens || !o.emit_nodes || o.emit_ld <= 0)
    return fail(h, GSE_E_ARG, "emit_len, emit_tokens, emit_nodes and emit_ld > 0 are required");
  if (t.qrows.rows > 0) {
    const gse_qrows &q = t.qrows;
    if (q.size < 8) return fail(h, GSE_E_ARG, "short gse_qrows");
    if (q.kind > GSE_Q_LOGITS_BF16) return fail(h, GSE_E_ARG, "q kind %u", q.kind);
    if (!q.q || q.ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "q rows missing or q ld < vocab");
    if (q.kind != GSE_Q_PROB && !q.temperature) return fail(h, GSE_E_ARG, "q logits need temperatures");
    if (q.rows > h->max_rows)
      return fail(h, GSE_E_CAPACITY, "%u q rows, the handle was opened for %u rows", q.rows, h->max_rows);
  } else {
    t.qrows.rows = 0;
  }
  DeviceGuard g(h->device);
  gse::ScanArgs a = make_args(h, b, gse::MODE_SAMPLE);
  a.tree = 1;
  a.tokens = h->ttok;
  hipStream_t s = (hipStream_t)b.stream;
  hipError_t e;
  gse::TreeLaunch L = {};
  L.s = a;
  L.parent = t.parent;
  L.token = t.token;
  L.qrow = t.qrow;
  L.anchor = t.anchor;
  L.q = t.qrows;
  L.max_kids = (int)t.max_kids;
  L.requests = (int)t.requests;
  L.sampled = h->ttok;
  L.st = h->tstate;
  L.plist = h->plist;
  L.pcnt = h->pcnt;
  L.pgrid = (int)h->target;
  L.npart = h->npart;
  L.tseg = h->tseg;
  L.nlast = h->nlast;
  L.qmax = h->qmax;
  L.qpart = h->qpart;
  L.qfin = h->qfin;
  L.out = o;
  // (the drafter rows' statistics run in the verify launch's statistics kernel, after the selection pass: on a second
  // stream beside it they slowed the split-row pass by more than they saved, C4 315.4 -> 312.1 us per call without it)
  if ((e = gse::launch_main(a, s)) != hipSuccess) return hip_fail(h, e, "main launch");
  if (a.dgrid > 0 && (e = gse::launch_deep(a, s)) != hipSuccess) return hip_fail(h, e, "deep launch");
  if (a.dgrid == 0 && (e = gse::launch_exact(a, s)) != hipSuccess) return hip_fail(h, e, "exact launch");
  if ((e = gse::launch_tree(L, s)) != hipSuccess) return hip_fail(h, e, "verify launch");
  return GSE_OK;
}

GSE_API int gse_draft_pick(gse_handle *h, const gse_pick_batch *in) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_pick_batch b;
  if (!take(in, b)) return fail(h, GSE_E_ARG, "null or short gse_pick_batch");
  if (b.rows == 0) return GSE_OK;
  if (!b.x || !b.temperature || !b.n || !b.seed || !b.at || !b.out_tokens || !b.out_logq)
    return fail(h, GSE_E_ARG, "x, temperature, n, seed, at, out_tokens and out_logq are required");
  if (b.dtype != GSE_F32 && b.dtype != GSE_BF16) return fail(h, GSE_E_ARG, "dtype %u is neither f32 nor bf16", b.dtype);
  if (b.vocab == 0 || b.ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "vocab 0 or ld < vocab");
  if (b.out_ld <= 0) return fail(h, GSE_E_ARG, "out_ld must be > 0");
  if (b.rows > h->max_rows) return fail(h, GSE_E_CAPACITY, "%u rows, the handle was opened for %u", b.rows, h->max_rows);
  if (b.vocab > h->max_vocab)
    return fail(h, GSE_E_CAPACITY, "vocab %u, the handle was opened for %u", b.vocab, h->max_vocab);
  DeviceGuard g(h->device);
  gse::PickLaunch L = {};
  L.b = b;
  L.pmax = h->pmax;
  L.ppart = h->ppart;
  L.plast = h->plast;
  L.ptop = h->ptop;
  L.tick = h->ptick;
  hipError_t e = gse::launch_pick(L, (hipStream_t)b.stream);
  return e == hipSuccess ? GSE_OK : hip_fail(h, e, "pick launch");
}

GSE_API int gse_qprob(gse_handle *h, const gse_qrows *qrows, uint32_t vocab, double *out, int64_t out_ld,
                      void *stream) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_qrows q;
  if (!take(qrows, q)) return fail(h, GSE_E_ARG, "null or short gse_qrows");
  if (q.kind != GSE_Q_LOGITS_F32 && q.kind != GSE_Q_LOGITS_BF16)
    return fail(h, GSE_E_ARG, "q kind %u: gse_qprob takes drafter logits (GSE_Q_LOGITS_F32 / _BF16)", q.kind);
  if (q.rows == 0) return GSE_OK;
  if (!q.q || !q.temperature || !out) return fail(h, GSE_E_ARG, "q, temperature and out are required");
  if (vocab == 0 || q.ld < (int64_t)vocab || out_ld < (int64_t)vocab)
    return fail(h, GSE_E_ARG, "vocab 0, q ld < vocab or out_ld < vocab");
  DeviceGuard g(h->device);
  hipError_t e = gse::launch_qprob(q, (int)vocab, out, out_ld, (hipStream_t)stream);
  return e == hipSuccess ? GSE_OK : hip_fail(h, e, "qprob launch");
}

GSE_API int gse_draw(gse_handle *h, const double *q, int64_t q_ld, uint32_t rows, uint32_t vocab, const double *u,
                     int32_t *out, void *stream) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  if (!q || !u || !out) return fail(h, GSE_E_ARG, "q, u and out are required");
  if (vocab == 0 || q_ld < (int64_t)vocab) return fail(h, GSE_E_ARG, "vocab 0 or q_ld < vocab");
  if (rows == 0) return GSE_OK;
  DeviceGuard g(h->device);
  hipError_t e = gse::launch_draw(q, q_ld, (int)rows, (int)vocab, u, out, (hipStream_t)stream);
  return e == hipSuccess ? GSE_OK : hip_fail(h, e, "draw launch");
}

GSE_API int gse_mss(gse_handle *h, const gse_mss_batch *in) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  gse_mss_batch b;
  if (!take(in, b)) return fail(h, GSE_E_ARG, "null or short gse_mss_batch");
  if (!b.p || !b.kid_tok || !b.kid_q || !b.seed || !b.idx || !b.out_token || !b.out_kid)
    return fail(h, GSE_E_ARG, "p, kid_tok, kid_q, seed, idx, out_token, out_kid are required");
  if (b.vocab == 0 || b.p_ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "vocab 0 or p_ld < vocab");
  if (b.q && b.q_ld < (int64_t)b.vocab) return fail(h, GSE_E_ARG, "q_ld < vocab");
  if (b.nodes == 0) return GSE_OK;
  DeviceGuard g(h->device);
  hipError_t e = gse::launch_mss(b, (hipStream_t)b.stream);
  return e == hipSuccess ? GSE_OK : hip_fail(h, e, "mss launch");
}

GSE_API int gse_pack_mask(gse_handle *h, const uint8_t *bools, int64_t bool_ld, uint32_t rows, uint32_t vocab,
                          int32_t *words, int64_t words_ld, void *stream) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  if (!bools || !words) return fail(h, GSE_E_ARG, "bools and words are required");
  if (bool_ld < (int64_t)vocab || words_ld < (int64_t)((vocab + 31) / 32))
    return fail(h, GSE_E_ARG, "bool_ld < vocab or words_ld < ceil(vocab / 32)");
  if (rows == 0 || vocab == 0) return GSE_OK;
  DeviceGuard g(h->device);
  hipError_t e = gse::launch_pack(bools, bool_ld, (int)rows, (int)vocab, words, words_ld, (hipStream_t)stream);
  return e == hipSuccess ? GSE_OK : hip_fail(h, e, "pack launch");
}

GSE_API int gse_profile(gse_handle *h, float *ms, uint32_t n, uint32_t *calls) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  for (uint32_t i = 0; i < n && ms; ++i) ms[i] = 0.0f;
  if (calls) *calls = (uint32_t)h->nring;
  if (h->nring == 0) return 0;
  DeviceGuard g(h->device);
  hipError_t e = hipEventSynchronize(h->ring[h->nring - 1][h->nprof]);
  if (e != hipSuccess) return hip_fail(h, e, "event synchronize");
  for (int c = 0; c < h->nring; ++c) {
    for (int i = 0; i < h->nprof && (uint32_t)i < n; ++i) {
      float t = 0.0f;
      if ((e = hipEventElapsedTime(&t, h->ring[c][i], h->ring[c][i + 1])) != hipSuccess)
        return hip_fail(h, e, "event elapsed");
      if (ms) ms[i] += t;
    }
  }
  const int k = h->nprof;
  h->nring = 0;
  return k;
}

GSE_API int gse_row_paths(gse_handle *h, uint32_t rows, uint8_t *paths) {
  if (!h) return fail(nullptr, GSE_E_ARG, "null handle");
  if (!paths && rows) return fail(h, GSE_E_ARG, "paths is required");
  if (rows > h->max_rows) return fail(h, GSE_E_CAPACITY, "%u rows, the handle was opened for %u", rows, h->max_rows);
  if (rows == 0) return GSE_OK;
  DeviceGuard g(h->device);
  std::vector<gse::RowInfo> info(rows);
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(info.data(), h->info, rows * sizeof(gse::RowInfo), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(h, e, "row paths");
  for (uint32_t r = 0; r < rows; ++r)
    paths[r] = (info[r].flags & gse::R_BY_EXACT) ? GSE_PATH_EXACT : (info[r].flags & gse::R_BY_DEEP) ? GSE_PATH_DEEP
                                                                                                   : GSE_PATH_MAIN;
  return GSE_OK;
}

GSE_API const char *gse_last_error(gse_handle *h) { return h ? h->err.c_str() : g_open_err; }

GSE_API void gse_close(gse_handle *h) {
  if (!h) return;
  {
    DeviceGuard g(h->device);
    (void)hipDeviceSynchronize();
    if (h->owned && h->block) (void)hipFree(h->block);
    if (h->ring) {
      for (int c = 0; c < GSE_PROFILE_CALLS; ++c)
        for (int i = 0; i < 5; ++i)
          if (h->ring[c][i]) (void)hipEventDestroy(h->ring[c][i]);
      delete[] h->ring;
    }
  }
  delete h;
}

}  // extern "C"
