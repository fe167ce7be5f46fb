// The fused selection pass. One 256-thread workgroup per (row, part), a part being a contiguous run of at most 65536
// tokens of the row. Its four waves stream the part in 512-token chunks (64 lanes x 8 tokens), each wave on its own:
// wave w takes chunks w, w + 4, w + 8, ..., the next chunks' loads are in flight while the current one is processed,
// and no barrier separates two chunks. One HBM read of the logits, the packed mask words and the row's history ids; the
// last workgroup of each row to finish (atomic ticket, nothing waits) resolves the row.
//
// Reference semantics (goethe_engine/sampling.py:59-85):
//   bad   = NaN anywhere before the mask, or no finite value after it        -> token -1            (sampling.py:71-75,84)
//   T = 0 -> first argmax of nan_to_num(masked x)                            (sampling.py:76)
//   T > 0 -> z = x / float32(T); stable descending order; fp64 softmax q; keep = rank < top_k AND cumsum(q) - q < top_p
//            (AND q >= min_p * q_0); c = cumsum(q * keep); token = order[count(c < u * c[-1])]   (sampling.py:59-83)
//
// Per chunk, in registers: the NaN test, the mask and the history exclusion (one select), z = RN(x / T) computed as
// RN32(x * RN64(1 / T)) (exact, see div_exact), each lane's running maximum, and the softmax sum of the elements the
// wave does not list, from v_exp_f32 with a rigorous error bound (rescaled in fp64 when a lane's maximum rises). The
// row history's tokens of the part (penalties: counts from an LDS table indexed by rank) take a side pass with the same
// arithmetic. The part's listing threshold is the kp-th largest of the 256 lane maxima of its waves' first chunks (to
// 16 key bits; kp aims at a.kt tokens of the part above it (KT, KT_HM in a call with histories or masks, or more in
// proportion for a part longer than PTOK), scaled by the exact counts of allowed tokens in the sample and in the part);
// a wave whose list passes a.vfirst (a quarter of its capacity at KT_VALVE) raises its own to the KV-th largest of its
// running lane maxima. Every element at or above the threshold in force when it is processed is listed (z bits, id);
// thresholds only rise, so a wave's list certifies its top elements down to its final threshold.
//
// Row resolve: the union of the waves' lists cut at the largest certified key is the row's certified head: exactly its
// top elements, stable order included. The resolve sorts the whole head, takes exact fp64 masses of it (and of every
// listed element for S), and decides the keep prefix and the draw. Top-k, min-p and the draw do not depend on S (they compare masses with masses); top-p uses the S bounds.
// A decision inside the bound, a keep prefix that runs past the head, or an overflowing list marks the row hard: the
// split-row finish (gse_deep.hip) or, failing that, the exact path (gse_exact.hip) finishes it.
#include <utility>

#include "gse_stream.h"

namespace gse {

namespace {

using namespace strm;

constexpr int KV = 32;                 // rank, among a wave's running lane maxima, of its raised threshold (when its
                                       // list passes a.vfirst entries)
constexpr int NH = 2048;               // certified head capacity of the row resolve
constexpr int NBK = 512;               // key buckets of the head sort
constexpr int BKT = 64;                // largest bucket the head sort ranks by counting (else: bitonic)
constexpr int GPT = 8;                 // listed entries per thread per gather round
constexpr int NSL = MAXP * PWAVES;     // wave lists of a row, at most (one per resolve thread)
static_assert(NWV == PWAVES, "");
static_assert(NSL <= MT, "one wave list per resolve thread");

constexpr int KHP = 4;                // history tokens per thread whose logits are loaded ahead (ranks below KHP MT)

struct Shared {
  union {
    struct {
      HistTab h;               // history of the part's tokens
      float hx[KHP * MT];      // logits of its first KHP MT ranks, loaded ahead of the side pass
    };
    struct {
      uint64_t head[NH];       // listed elements at or above the certified key; then sorted (descending)
      uint64_t tmp[NH];        // the head grouped by bucket
      uint32_t bcnt[NBK];      // bucket counts, then their running ends
      uint32_t bofs[NBK];      // bucket starts
    } r;
  };
  uint32_t hover;              // more distinct history ids than HMAX
  uint32_t ticket;
  float wmax[NWV];
  uint32_t wflags[NWV], wkap[NWV], wcnt[NWV];
  uint32_t lmax[MT];           // first-chunk lane maxima (16 key bits)
  uint64_t wtop[NWV];
  double wred[NWV], wred2[NWV];
  // resolve
  uint32_t loff[NSL];           // wave list lengths
  uint64_t rtop, rtopL;
  uint32_t rflags, rkappa, rmkey, nh, mfail_sure, mfail_maybe, jcount, bmax, lpw;
  double rsc;
  double etab[64];             // 2^(j / 64) for exp_nonpos
};

// A listed element as the stream writes it: the bits of its x (the processed logit: penalties and mask applied) over the
// token. The resolve packs it into the sort key of z = RN(x / T) (x itself when the row does not divide).
__device__ __forceinline__ uint64_t raw_entry(float x, uint32_t tok) {
  return ((uint64_t)__float_as_uint(x) << 32) | tok;
}
__device__ __forceinline__ uint64_t key_of_raw(uint64_t r, bool divide, double Rd) {
  const float x = __uint_as_float((uint32_t)(r >> 32));
  return pack(fkey(divide ? div_exact(x, Rd) : x), (uint32_t)r);
}

__device__ __forceinline__ void lp_invalid(const ScanArgs &a, int row, int nlp) {
  for (int i = threadIdx.x; i < nlp; i += MT) {
    a.lp_ids[(int64_t)row * a.lp_ld + i] = -1;
    a.lps[(int64_t)row * a.lp_ld + i] = __builtin_nanf("");
  }
}

__device__ __forceinline__ void set_info(RowInfo *ri, uint64_t cmax, uint64_t kkeep, double S, double Z, uint32_t flags,
                                         int32_t token) {
  RowInfo r = {};
  r.cmax = cmax;
  r.kkeep = kkeep;
  r.S = S;
  r.Z = Z;
  r.flags = flags;
  r.token = token;
  *ri = r;
}

// A hard row's info; a row that the split-row finish does not take (no R_DEEP) is also counted, so that the split-row
// launch looks for such rows (its exact rows).
__device__ __forceinline__ void set_hard(const ScanArgs &a, RowInfo *ri, uint64_t cmax, double S, uint32_t flags,
                                         int32_t token) {
  set_info(ri, cmax, 0, S, 0.0, flags, token);
  if (!(flags & R_DEEP)) atomicAdd(reinterpret_cast<unsigned long long *>(a.dctl), 1ull << 32);
}

// ---------------------------------------------------------------------------------------------------------------------
// Row resolve, run by the last workgroup of the row.

enum { EV_DONE = 0, EV_MORE = 1, EV_HARD = 2 };

struct RowEval {
  const ScanArgs *a;
  int row, nlp, n;
  bool greedy, complete;
  double M;
  double S, B;    // the masses outside the head (unlisted, and listed below the certified key) and their error bound
  uint64_t gtop;  // greedy rows: packed argmax
  const gse_row *P;
};

// Sorts the head sh.r.head[0, n) descending in place (keys in [kappa, mk]): the counting sort of sort_desc_counting.
__device__ __forceinline__ void sort_head(Shared &sh, int n, uint32_t mk, uint32_t kappa) {
  sort_desc_counting<NBK, BKT>(sh.r.head, sh.r.tmp, sh.r.bcnt, sh.r.bofs, sh.wcnt, &sh.bmax, n, mk, kappa);
}

// Decides the keep prefix, the draw and the logprobs over the sorted head arr[0, n) (the whole certified head).
__device__ __forceinline__ int evaluate(const RowEval &ev, const uint64_t *arr, Shared &sh) {
  const ScanArgs &a = *ev.a;
  const gse_row &P = *ev.P;
  const int tid = threadIdx.x;
  const int n = ev.n;
  if (ev.nlp > n) return EV_HARD;  // logprobs past the finite elements: -inf ranks in id order
  if (tid == 0) {
    sh.mfail_sure = 0xFFFFFFFFu;
    sh.mfail_maybe = 0xFFFFFFFFu;
    sh.jcount = 0;
  }
  // Exact masses e_r of the sorted ranks, then their inclusive prefixes I_r in place (in LDS). Wave w takes ranks
  // [RPW w, RPW w + RPW), 64 consecutive ranks per step: conflict-free LDS accesses and wave scans (the additions are
  // the same, in the same order, for the same head). A_r = I_{r-1} is the exclusive prefix.
  double *ee = reinterpret_cast<double *>(sh.r.tmp);
  const double M = ev.M;
  const int lane = lane_id(), w = tid >> 6;
  // (two ranks a thread at a time: their exponentials' dependent chains overlap; an index past n reads rank 0 and its
  // result is dropped)
#pragma unroll 1
  for (int i = tid; i < n; i += 2 * MT) {
    const int i1 = i + MT < n ? i + MT : 0;
    const double e0 = exp_nonpos((double)fkey_inv(pk_key(arr[i])) - M, sh.etab);
    const double e1 = exp_nonpos((double)fkey_inv(pk_key(arr[i1])) - M, sh.etab);
    ee[i] = e0;
    if (i + MT < n) ee[i + MT] = e1;
  }
  __syncthreads();
  const int RPW = ((n + NWV - 1) / NWV + WAVE - 1) / WAVE * WAVE;  // ranks per wave (a multiple of 64, 4 RPW >= n)
  double carry = 0.0;
#pragma unroll 1
  for (int s = 0; s < RPW / WAVE; ++s) {
    const int r = w * RPW + s * WAVE + lane;
    double v = r < n ? ee[r] : 0.0;
    v = wave_incl_scan_f64(v) + carry;
    if (r < n) ee[r] = v;
    carry = shfl_f64(v, WAVE - 1);
  }
  if (lane == 0) sh.wred[w] = carry;
  __syncthreads();
  double base = 0.0, htot = 0.0;
  for (int q = 0; q < NWV; ++q) {
    if (q < w) base += sh.wred[q];
    htot += sh.wred[q];
  }
  const double Sm = ev.S + htot;  // S: the unlisted and listed masses outside the head, then the head's
  if (w > 0) {
#pragma unroll 1
    for (int s = 0; s < RPW / WAVE; ++s) {
      const int r = w * RPW + s * WAVE + lane;
      if (r < n) ee[r] += base;
    }
  }
  __syncthreads();
  if (ev.nlp > 0) {
    if (tid == 0) sh.lpw = 1;
    const double lS = log(Sm);
    for (int i = tid; i < ev.nlp; i += MT) {
      const uint64_t pk = arr[i];
      a.lp_ids[(int64_t)ev.row * a.lp_ld + i] = (int32_t)pk_id(pk);
      a.lps[(int64_t)ev.row * a.lp_ld + i] = (float)(((double)fkey_inv(pk_key(pk)) - M) - lS);
    }
  }
  RowInfo *ri = a.info + ev.row;
  if (ev.greedy) {
    if (tid == 0) set_info(ri, ev.gtop, 0, Sm, 0.0, R_DONE | R_GREEDY, (int32_t)pk_id(ev.gtop));
    return EV_DONE;
  }
  // keep_r = r < K AND A_r / S < top_p AND q_r >= min_p q_0 (sampling.py:80 plus min-p). A top-p decision is sure when
  // it holds for every S in [S - B, S + B] (A / S against top_p as A against top_p S: the margin B covers the
  // roundings); the first rank that surely fails and the first that may fail must agree. Min-p compares the rounded
  // quotients as the definition does, where e lies within 1e-12 of min_p (elsewhere e >= min_p decides it).
  const int64_t K = P.top_k > 0 ? (int64_t)P.top_k : (int64_t)0x7FFFFFFFFFFFll;
  const double topp = P.top_p, minp = P.min_p;
  const double B = ev.B + 2e-15 * Sm;
  const double q0 = 1.0 / Sm, tlo = topp * (Sm - B), thi = topp * (Sm + B);
  uint32_t fsure = 0xFFFFFFFFu, fmaybe = 0xFFFFFFFFu;
#pragma unroll 1
  for (int s = 0; s < RPW / WAVE; ++s) {
    const int r = w * RPW + s * WAVE + lane;
    if (r < n) {
      const double A = r > 0 ? ee[r - 1] : 0.0;
      const bool kk = (int64_t)r < K;
      bool km = true;
      if (minp > 0.0) {
        const double e = exp_nonpos((double)fkey_inv(pk_key(arr[r])) - M, sh.etab);
        km = e >= minp;
        if (fabs(e - minp) <= 1e-12 * minp) km = e / Sm >= minp * q0;
      }
      if ((!kk || !km || A >= thi) && fsure == 0xFFFFFFFFu) fsure = (uint32_t)r;
      if ((!kk || !km || !(A < tlo)) && fmaybe == 0xFFFFFFFFu) fmaybe = (uint32_t)r;
    }
  }
  fsure = wave_min_u32(fsure);
  fmaybe = wave_min_u32(fmaybe);
  if (lane == 0) {
    atomicMin(&sh.mfail_sure, fsure);
    atomicMin(&sh.mfail_maybe, fmaybe);
  }
  __syncthreads();
  uint32_t m = sh.mfail_sure;
  if (m != sh.mfail_maybe) return EV_HARD;
  if (m == 0xFFFFFFFFu) {  // every rank of the head is kept
    if (!ev.complete) return EV_HARD;  // the keep prefix runs past the certified head
    m = (uint32_t)n;
  }
  // c_last = I_{m-1}; j = #{r < m : I_r < u c_last}, clamped to [0, m - 1] (sampling.py:81-83)
  const double clast = ee[m - 1];
  int32_t tok = -1;
  if (a.mode == MODE_SAMPLE) {
    const double u = a.uni ? a.uni[ev.row] : uniform64(P.seed, P.idx);
    const double thr = u * clast;
    uint32_t cnt = 0;
#pragma unroll 1
    for (int s = 0; s < RPW / WAVE; ++s) {
      const int r = w * RPW + s * WAVE + lane;
      if ((uint32_t)r < m && ee[r] < thr) ++cnt;
    }
    cnt = wave_sum_u32(cnt);
    if (lane == 0 && cnt) atomicAdd(&sh.jcount, cnt);
    __syncthreads();
    tok = (int32_t)pk_id(arr[min(sh.jcount, m - 1u)]);
  }
  if (tid == 0) {
    set_info(ri, arr[0], arr[m - 1], Sm, clast / Sm, R_DONE, tok);
    if (a.mode == MODE_SAMPLE) a.tokens[ev.row] = tok;
  }
  return EV_DONE;
}

// A verify node that takes dist + mss and keeps every token (sampling.py:80 with top_k off and top_p 1, no min-p):
// dist needs only the maximum of z, and the verify round's statistics pass forms the exact kept mass itself, so its
// parts list nothing and sum nothing.
__device__ __forceinline__ bool keeps_all_mss(const ScanArgs &a, const gse_row &P) {
  return a.tree && (P.flags & GSE_ROW_MSS) && (P.top_k <= 0 || P.top_k >= a.V) && P.top_p >= 1.0 && !(P.min_p > 0.0);
}

__device__ __forceinline__ void resolve_row(const ScanArgs &a, int row, const gse_row &P, Shared &sh) {
  const int tid = threadIdx.x;
  const SliceRec *rb = a.rec + (size_t)row * a.nparts;
  const bool greedy = is_greedy(a.mode, P);
  RowInfo *ri = a.info + row;
  const int nlp = nlp_of(a, P);
  const int nsl = a.nparts * PWAVES;
  if (tid == 0) {
    sh.rtop = 0;
    sh.rtopL = 0;
    sh.rflags = 0;
    sh.rkappa = 0;
    sh.rmkey = 0;
    sh.nh = 0;
    sh.lpw = 0;
  }
  // One round of loads: the records (thread j holds wave list j (part j / 4), threads j % 4 == 0 the part's record) and,
  // before the list lengths are known, the first SPEC slots of every wave list (slot o of list j in thread
  // (j SPEC + o) % MT, round (j SPEC + o) / MT); slots past a list's length are dropped once it is known.
  const uint64_t *cl0 = a.cand + (size_t)row * nsl * CAPW;
  const int SPEC = max(1, (MT * GPT) / nsl);
  uint64_t pks[GPT];
#pragma unroll
  for (int g = 0; g < GPT; ++g) {  // (unconditional loads, clamped into the row's lists: the batch drops the extra)
    const int e = g * MT + tid, j = min(e / SPEC, nsl - 1);
    pks[g] = ld_ag(&cl0[(size_t)j * CAPW + min(e - j * SPEC, CAPW - 1)]);
  }
  const int prt = tid / PWAVES;
  uint32_t r_nc = 0, r_mkey = 0, r_kap = 0, r_fl = 0;
  uint64_t r_top = 0;
  double r_s = 0.0, r_b = 0.0;
  if (tid < nsl) {
    const SliceRec *r = rb + prt;
    r_nc = min(ld_ag(&r->wcnt[tid % PWAVES]), (uint32_t)CAPW);
    if (tid % PWAVES == 0) {
      r_top = ld_ag(&r->top);
      r_kap = ld_ag(&r->kappa);
      r_fl = ld_ag(&r->flags);
      r_mkey = ld_ag(&r->mkey);
      r_s = ld_ag(&r->s);
      r_b = ld_ag(&r->bnd);
    }
  }
  __syncthreads();
  if (tid < nsl && tid % PWAVES == 0) {
    atomicOr(&sh.rflags, r_fl);
    atomicMax((unsigned long long *)&sh.rtop, (unsigned long long)r_top);
    atomicMax(&sh.rkappa, r_kap);
    atomicMax(&sh.rmkey, r_mkey);
  }
  // the list lengths (sh.loff), and the exclusive prefix of the slots past SPEC of the longer lists (sh.lmax)
  {
    if (tid < nsl) sh.loff[tid] = r_nc;
    const uint32_t rem = r_nc > (uint32_t)SPEC ? r_nc - (uint32_t)SPEC : 0u;
    const uint32_t rinc = wave_incl_scan_u32(rem);
    if (lane_id() == WAVE - 1) sh.wcnt[tid >> 6] = rinc;
    __syncthreads();
    uint32_t rpre = 0, rtot = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      rpre += w < (tid >> 6) ? sh.wcnt[w] : 0u;
      rtot += sh.wcnt[w];
    }
    if (tid < nsl) sh.lmax[tid] = rpre + rinc - rem;
    if (tid == 0) sh.jcount = rtot;
  }
  __syncthreads();
  const uint32_t flags = sh.rflags;
  const uint32_t mk = sh.rmkey;
  const uint64_t gtop = sh.rtop;  // greedy argmax; or, for a row without z > -inf, the lowest id of its -inf
  const bool bad = (flags & F_NAN) || !(flags & F_FINITE);

  // z = x / T: no finite z over the allowed tokens may still hide a finite x whose quotient overflowed
  const bool divide = !greedy && P.temperature != 1.0f;
  const double Rd = 1.0 / (double)P.temperature;  // (the lists hold x; their keys are of z = RN(x / T))
  if (((flags & F_HOVER) && (greedy || bad)) ||
      (((flags & F_PINF) || (divide && !(flags & F_FINITE))) && !(flags & F_NAN))) {
    // more distinct history ids than a part can count, or a maximum of z that is not finite (the parts do not know
    // whether a finite x exists): the exact path redoes the whole row (flags, argmax, logprobs)
    if (tid == 0) set_hard(a, ri, gtop, 0.0, R_HARD | R_FULL | (greedy ? R_GREEDY : 0u), -1);
    return;
  }
  if (a.mode == MODE_SAMPLE && (greedy || bad)) {
    const int32_t tok = bad ? -1 : (int32_t)pk_id(gtop);
    if (tid == 0) a.tokens[row] = tok;
    const bool lp_head = greedy && !bad && nlp > 0 && mk > KEY_NEGINF && mk < KEY_POSINF;
    if (!lp_head) {
      if (tid == 0) set_info(ri, gtop, 0, 0.0, 0.0, (greedy ? R_GREEDY : 0u) | (bad ? R_BAD : 0u) | R_DONE, tok);
      lp_invalid(a, row, nlp);
      return;
    }
    // greedy row with logprobs: z = x, the head below gives them; the token stays the argmax
  } else if ((flags & F_NAN) || mk <= KEY_NEGINF) {
    // NaN in z (dist of a bad row) or no z > -inf: q is NaN, keep is empty and j clamps to 0 -> order[0]
    // (sampling.py:82); gtop is the lowest id holding -inf
    if (tid == 0) {
      set_info(ri, gtop, 0, 0.0, 0.0, R_DONE | R_SPECIAL, (int32_t)pk_id(gtop));
      if (a.mode == MODE_SAMPLE) a.tokens[row] = (int32_t)pk_id(gtop);
    }
    lp_invalid(a, row, nlp);
    return;
  }

  // Gather the listed elements: masses for S, the certified head, the packed maximum.
  const bool finite_max = mk < KEY_POSINF;
  const double M = finite_max ? (double)fkey_inv(mk) : 0.0;
  if (keeps_all_mss(a, P) && nlp == 0) {
    // its parts listed nothing: done with the maximum, or (more distinct history ids than a part can count, or a
    // maximum that is not finite) the exact path redoes the row
    if (tid == 0) {
      if (finite_max && !(flags & F_HOVER)) set_info(ri, pack(mk, 0u), 0ull, 0.0, 0.0, R_DONE, -1);
      else set_hard(a, ri, gtop, 0.0, R_HARD | R_FULL, -1);
    }
    return;
  }
  const uint32_t kappa = max(sh.rkappa, KEY_NEGINF + 1u);
  const bool complete = kappa <= KEY_NEGINF + 1u;
  double srest = 0.0, brest = 0.0;
  if (tid < nsl && tid % PWAVES == 0 && finite_max && r_mkey > KEY_NEGINF) {
    const double f = exp((double)fkey_inv(r_mkey) - M);
    srest = f * r_s;
    brest = f * r_b;
  }
  double scand = 0.0;
  uint64_t bestL = 0;
  // One batch of listed entries (raw, valid): the packed maximum, the masses of the entries below the certified key
  // (the head's masses are summed by the evaluation, which takes them anyway), head appends (one LDS atomic per wave).
  // Through LDS, so that the processing loop stays rolled: this code runs once per row, with a cold instruction cache,
  // and its length is its cost.
  auto batch = [&](const uint64_t(&pk)[GPT], const bool(&ok)[GPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < GPT; ++g) {  // (the key for every slot, then a select: no branch that waits for its load)
      const uint64_t kv = key_of_raw(pk[g], divide, Rd);
      sh.r.tmp[g * MT + tid] = ok[g] ? kv : 0ull;
    }
    // the masses of the entries below the certified key, two at a time (independent exponentials overlap), and the
    // head bits of the thread's GPT entries
    uint32_t hb = 0;
#pragma unroll 1
    for (int g = 0; g < GPT; g += 2) {
      const uint64_t v0 = sh.r.tmp[g * MT + tid], v1 = sh.r.tmp[(g + 1) * MT + tid];
      const uint32_t k0 = pk_key(v0), k1 = pk_key(v1);
      bestL = max(bestL, max(v0, v1));
      const bool m0 = v0 && finite_max && k0 > KEY_NEGINF && k0 < kappa;
      const bool m1 = v1 && finite_max && k1 > KEY_NEGINF && k1 < kappa;
      const double e0 = exp_nonpos(m0 ? (double)fkey_inv(k0) - M : 0.0, sh.etab);
      const double e1 = exp_nonpos(m1 ? (double)fkey_inv(k1) - M : 0.0, sh.etab);
      scand += (m0 ? e0 : 0.0);
      scand += (m1 ? e1 : 0.0);
      hb |= (v0 && k0 >= kappa ? 1u : 0u) << g;
      hb |= (v1 && k1 >= kappa ? 1u : 0u) << (g + 1);
    }
    // head appends: one LDS atomic per wave for all GPT rounds
    uint32_t cnt = 0;
    uint64_t bl[GPT];
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      bl[g] = ballot64((hb >> g) & 1u);
      cnt += (uint32_t)__popcll(bl[g]);
    }
    if (cnt) {
      uint32_t base = 0;
      if (lane_id() == 0) base = atomicAdd(&sh.nh, cnt);
      base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
      for (int g = 0; g < GPT; ++g) {
        const uint32_t pos = base + lanes_below(bl[g]);
        if (((hb >> g) & 1u) && pos < (uint32_t)NH) sh.r.head[pos] = sh.r.tmp[g * MT + tid];
        base += (uint32_t)__popcll(bl[g]);
      }
    }
  };
  // the slots past SPEC of the longer lists (flat index f over them; the list holding f: the last with prefix <= f),
  // a round of MT GPT at a time; the first such round is loaded before the speculative batch is processed, so that its
  // loads are in flight meanwhile
  const uint32_t rtot = sh.jcount;
  uint64_t pk[GPT];
  bool okr[GPT];
  // (the searches of the GPT slots advance together, one step of each per LDS round trip, over the log2(nsl) + 1 steps
  // the row's lists need: 16 lists at C3 take five round trips, where searches of NSL done one slot after the other
  // took up to 64)
  int top = 1;
  while (2 * top <= nsl) top *= 2;
  auto load_round = [&](uint32_t f0) __attribute__((always_inline)) {
    int lo[GPT];
#pragma unroll
    for (int g = 0; g < GPT; ++g) lo[g] = 0;
#pragma unroll 1
    for (int st = top; st > 0; st >>= 1) {
      uint32_t lv[GPT];  // (every read issued, in range, before any is used: one LDS round trip per step)
#pragma unroll
      for (int g = 0; g < GPT; ++g) lv[g] = sh.lmax[min(lo[g] + st, nsl - 1)];
#pragma unroll
      for (int g = 0; g < GPT; ++g) {
        const uint32_t f = f0 + g * MT + tid;
        const int m = lo[g] + st;
        lo[g] = (m < nsl && lv[g] <= f) ? m : lo[g];
      }
    }
    // (every load issued, into the row's lists: a load under a condition is waited for where the condition joins,
    // and the slots of one round then came in one after the other; the batch drops the slots past rtot)
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      const uint32_t f = f0 + g * MT + tid;
      okr[g] = f < rtot;
      pk[g] = ld_ag(&cl0[(size_t)lo[g] * CAPW + min((uint32_t)SPEC + f - sh.lmax[lo[g]], (uint32_t)CAPW - 1u)]);
    }
  };
  // (without a second round, as many loads of in-range slots: either way GPT loads follow the speculative batch's, so
  // that batch waits only for its own; with the round under a condition alone it waited for both)
  if (rtot > 0) {
    load_round(0);
  } else {
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      okr[g] = false;
      pk[g] = ld_ag(&cl0[g]);  // (distinct slots: loads of one address would merge)
    }
  }
  {
    bool ok[GPT];
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      const int e = g * MT + tid, j = e / SPEC;
      ok[g] = j < nsl && (uint32_t)(e - j * SPEC) < sh.loff[j];
    }
    batch(pks, ok);
  }
  for (uint32_t f0 = 0; f0 < rtot; f0 += MT * GPT) {
    if (f0 > 0) load_round(f0);
    batch(pk, okr);
  }
  bestL = wave_max_u64(bestL);
  if (lane_id() == 0) atomicMax((unsigned long long *)&sh.rtopL, (unsigned long long)bestL);
  if (!finite_max) {
    // z holds +inf: every +inf element is listed; token = the lowest id among them (sampling.py:82, order[0])
    __syncthreads();
    const uint64_t t = sh.rtopL;
    const bool hard = (flags & (F_OVERFLOW | F_HOVER)) || a.force_exact;
    if (tid == 0) {
      if (hard) {
        set_hard(a, ri, t, 0.0, R_HARD | (greedy ? R_GREEDY : 0u), -1);
      } else {
        set_info(ri, t, 0, 0.0, 0.0, R_DONE | R_SPECIAL | (greedy ? R_GREEDY : 0u), (int32_t)pk_id(t));
        if (a.mode == MODE_SAMPLE && !greedy) a.tokens[row] = (int32_t)pk_id(t);
      }
    }
    if (!hard) lp_invalid(a, row, nlp);
    return;
  }
  srest = block_sum_f64(srest, sh.wred);
  brest = block_sum_f64(brest, sh.wred);
  scand = block_sum_f64(scand, sh.wred);  // (its barriers order the head appends)
  RowEval ev;
  ev.a = &a;
  ev.row = row;
  ev.nlp = nlp;
  ev.greedy = greedy;
  ev.complete = complete;
  ev.M = M;
  ev.S = srest + scand;  // without the head's masses: the evaluation adds them
  ev.B = brest;
  ev.gtop = gtop;
  ev.P = &P;
  const uint32_t nh_all = sh.nh;
  ev.n = (int)min(nh_all, (uint32_t)NH);
  const int n = ev.n;
  int st = EV_HARD;
  if (!((flags & (F_OVERFLOW | F_HOVER)) || nh_all > (uint32_t)NH || a.force_exact)) {
    // A keep prefix that surely runs past the head goes on without the sort and the evaluation, whose answer it
    // already knows (EV_HARD): no logprobs, no top-k or min-p cut inside the head, an incomplete head, and the whole
    // head's mass h below top_p (S - B) even with margins far above the roundings of h and of the evaluation's own sums
    // (each within 2048 ulps). The rows of flat, hot nuclei that go to the split-row finish.
    bool past = false;
    if (!greedy && nlp == 0 && !complete && !(P.min_p > 0.0) && (P.top_k <= 0 || P.top_k > n)) {
      double h = 0.0;
      for (int i = tid; i < n; i += MT) h += exp_nonpos((double)fkey_inv(pk_key(sh.r.head[i])) - M, sh.etab);
      h = block_sum_f64(h, sh.wred);
      const double hhi = h * (1.0 + 1e-11), hlo = h * (1.0 - 1e-11);
      const double B = ev.B + 2e-15 * (ev.S + hhi);
      past = hhi < P.top_p * (ev.S + hlo - B);
    }
    if (!past) {
      sort_head(sh, n, mk, kappa);
      st = evaluate(ev, sh.r.head, sh);
    }
  }
  if (st != EV_DONE) {
    __syncthreads();  // (sh.lpw)
    if (tid == 0) {
      // The exact path finishes the row (for a greedy row: its logprobs; the token is already written). A sampled row
      // whose logprobs are written and whose part lists all fit goes to the split-row finish first.
      uint32_t fl = R_HARD | (greedy ? R_GREEDY : 0u);
      // (the split-row finish recomputes z and every mass itself: overflowing wave lists do not matter to it)
      const bool deep = a.dslices > 0 && !greedy && !(flags & F_HOVER) && !a.force_exact && (nlp == 0 || sh.lpw);
      if (deep) {
        const uint32_t slot = (uint32_t)atomicAdd(reinterpret_cast<unsigned long long *>(a.dctl), 1ull);
        if (slot < (uint32_t)a.dslots) {
          DeepSlot *ds = a.dslot + slot;
          ds->P = P;
          ds->row = row;
          ds->M = M;
          ds->u = a.mode == MODE_SAMPLE ? (a.uni ? a.uni[row] : uniform64(P.seed, P.idx)) : 0.0;
          ds->plan = plan_word(DS_PENDING, 0, 0, 0, 0);
          fl |= R_DEEP;
        }
      }
      // cmax: the greedy argmax, or the packed maximum of z (always listed) that the split-row finish reads
      const uint64_t zmax = pk_key(sh.rtopL) == mk ? sh.rtopL : pack(mk, 0u);  // (a list overflow may drop it)
      set_hard(a, ri, greedy ? gtop : zmax, ev.S, fl, greedy ? (int32_t)pk_id(gtop) : -1);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// Part streaming.
//
// The stream carries every token of the part below pv (the part end, rounded down to a whole vector for aligned rows)
// except the tokens of the row's history: those (at most a few hundred per part) and the ragged tokens [pv, p1) are
// penalized and masked by a side pass with exactly the same arithmetic, and enter the same running state out of order.
// Every chunk issues the same loads (a vector past pv loads the part's next tokens, or zeros past the part's end, and is
// ignored), so the compiler can count the loads in flight: each wave keeps three or five chunks loading while it works
// on one. The stream needs no per-element branch: the mask and the history exclusion are one bit select per element,
// the listing is skipped for a whole chunk when the lane maxima lie below the threshold, and the unlisted terms are
// summed in fp32 per chunk.

// The stream works on x, the processed logit (-inf where the mask or the history exclusion removes the token), never on
// z = RN(x / T): z is a monotone non-decreasing function of x (T > 0), so maxima and thresholds carry over (the maximum of
// z is z of the maximum of x; every z above z(x_t) belongs to an x above x_t), and each unlisted term exp(z - R) comes
// from one fma of x. Only the part maximum, a threshold and the listed elements are ever divided.
//
// Per-lane running state of a wave.
struct Run {
  float m;         // running maximum of this lane's x
  double s;        // sum of this lane's unlisted exp(z - R) (fp32 terms), R = z(xt) the wave's threshold in z
  double b;        // its error bound
  uint32_t xkey;   // the wave's listing threshold as a key of x (uniform in the wave; only rises)
  float xt;        // its value: every element with x >= xt is listed
  float R;         // z(xt): every unlisted element has z <= R
  float c1, c0;    // the exponent of an unlisted term: t = fma(x, c1, c0), (x / T - R) log2(e) rounded
  double bR;       // the part of a term's error bound that grows with |R| (the roundings of z, c1 and c0)
  float kb;        // a stream chunk's bound factor on its sum (EPL terms a lane): (2.4e-7 + 3 6e-8 + 5e-8 + bR), raised
                   // by 2^-20 relative to cover the fp32 rounding of the chunk's bound (uniform)
  uint32_t kcert;  // certified key of z: every element with key >= kcert is listed (fkey(R) + 1)
  bool ovf;        // c0 out of the fp32 range: the part's sums cannot be trusted
  uint32_t woff;   // elements the wave has listed (uniform)
  uint32_t vnext;  // list length at which the valve next recomputes the threshold (uniform)
  float g;         // greedy rows: largest nan_to_num(x) so far, at the lowest token gid holding it
  uint32_t gid;
  uint32_t fid;    // lowest token of this lane with x not NaN (found in the lane's first chunk)
  bool fid_all;    // every lane of the wave has found its fid (uniform): the stream's chunks skip the search
  uint64_t nanm;   // lanes that saw a NaN before the mask (wave-uniform)
};

constexpr int KH = HMAX / MT;  // history tokens a thread carries in the side pass

// Selects x where bit k of keep is set, -inf elsewhere: one bit-field insert (v_bfi_b32).
__device__ __forceinline__ float keep_or_ninf(float x, uint32_t keep, int k) {
  const uint32_t sel = (uint32_t)(((int32_t)(keep << (31 - k))) >> 31);  // all ones when bit k is set
  return __uint_as_float((__float_as_uint(x) & sel) | (0xFF800000u & ~sel));
}

// The wave's next chunk for the aligned loads: its first byte and the bytes left in the part, of the logits and of the
// mask words, stepped by one wave stride per chunk (scalar arithmetic). Each load goes through a buffer resource based
// at the chunk, so a lane's offsets are the same in every chunk (no per-chunk vector arithmetic), and a load at or past
// the part's end returns zeros without a memory access (a chunk past the part has an empty range).
struct Cursor {
  const char *x, *m;
  int xn, mn;
};
template <int DT>
__device__ __forceinline__ Cursor cursor(const RowCtx &c, int cb, int p1) {
  constexpr int ES = DT == GSE_F32 ? 4 : 2;
  Cursor r;
  r.x = c.base + (size_t)cb * ES;
  r.xn = (p1 - cb) * ES;
  r.m = c.mw ? (const char *)c.mw + (cb >> 5) * 4 : nullptr;  // (aligned rows: cb is a multiple of 32)
  r.mn = (((p1 + 31) >> 5) - (cb >> 5)) * 4;
  return r;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const char *base, int bytes) {
  constexpr int FMT = 0x00020000;  // raw 32-bit buffer (GFX9 resource word 3)
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, max(bytes, 0), FMT);
}

// One chunk's logits and mask words, the same loads for every chunk, as raw words: a lane's EPL logits of the chunk
// (fp32 bits, or bf16 pairs, token 2i in the low half of word i) stay packed until the chunk is processed, so that no
// arithmetic on a loaded value sits between the loads in flight and the loop's back edge (bf16 rows unpacked at load
// time made every iteration wait for all three chunks ahead). Aligned rows: one 16-byte buffer load per vector (a vector
// past the stream end pv loads the part's next tokens, or zeros past the part, and is ignored: its tokens are not in the
// chunk's in-range bits); unaligned rows load element by element, clamped to the part.
template <int DT>
constexpr int RAW = Lay<DT>::NV * 4;  // raw words of a lane's chunk
// Aligned rows read chunk cur and step cur to the wave's next chunk; unaligned rows read chunk cb.
template <int DT, bool AL, bool MASKED>
__device__ __forceinline__ void load_u(const RowCtx &c, Cursor &cur, int cb, int pv, int p1, uint32_t (&r)[RAW<DT>],
                                       uint32_t (&mw)[Lay<DT>::NV]) {
  using L = Lay<DT>;
  constexpr int ES = DT == GSE_F32 ? 4 : 2;
  constexpr int DX = NWV * CHK * ES, DM = NWV * CHK / 8;  // one wave stride, in logit and mask bytes
  const int l = lane_id();
  __amdgpu_buffer_rsrc_t rx, rm;
  if constexpr (AL) {
    rx = chunk_rsrc(cur.x, cur.xn);
    cur.x += DX;
    cur.xn -= DX;
    if constexpr (MASKED) {
      rm = chunk_rsrc(cur.m, cur.mn);
      cur.m += DM;
      cur.mn -= DM;
    }
  }
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = cb + v * L::STRIDE + l * L::VEC;
    const int o = v * L::STRIDE + l * L::VEC;  // t0 - cb
    if constexpr (MASKED) {
      if constexpr (AL) mw[v] = __builtin_amdgcn_raw_buffer_load_b32(rm, (o >> 5) * 4, 0, 0);
      else mw[v] = c.mw[min(t0, p1 - 1) >> 5];
    }
    if constexpr (AL) {
      const auto u = __builtin_amdgcn_raw_buffer_load_b128(rx, o * ES, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) r[4 * v + i] = u[i];
    } else if constexpr (DT == GSE_F32) {
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) r[v * L::VEC + k] = __float_as_uint(load_one(c, min(t0 + k, p1 - 1)));
    } else {
      const uint16_t *b = (const uint16_t *)c.base;
#pragma unroll
      for (int k = 0; k < L::VEC / 2; ++k)
        r[4 * v + k] = (uint32_t)b[min(t0 + 2 * k, p1 - 1)] | ((uint32_t)b[min(t0 + 2 * k + 1, p1 - 1)] << 16);
    }
  }
  (void)pv;
}

// The chunk's logits from its raw words (bf16: the value's bits in the high half of an fp32)
template <int DT>
__device__ __forceinline__ void unpack(const uint32_t (&r)[RAW<DT>], float (&x)[EPL]) {
  if constexpr (DT == GSE_F32) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) x[i] = __uint_as_float(r[i]);
  } else {
#pragma unroll
    for (int i = 0; i < RAW<DT>; ++i) {
      x[2 * i] = __uint_as_float(r[i] << 16);
      x[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
    }
  }
}

// The history words of a chunk's vectors (bit o of the part's history bitset = token p0 + o is in the row's history),
// read from LDS with the chunk's loads, so that the read is done by the time the chunk is processed. Raw words: token k
// of lane l's vector is bit (l VEC) % 32 + k (chunk starts lie 512 tokens apart from the part start, a multiple of 32).
template <int DT>
__device__ __forceinline__ void hist_words(const HistTab &h, int cb, int p0, int p1, uint32_t (&hw)[Lay<DT>::NV]) {
  using L = Lay<DT>;
  const int l = lane_id();
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int o = min(cb + v * L::STRIDE + l * L::VEC, p1 - 1) - p0;  // (a vector past the end reads a valid word)
    hw[v] = h.bits[o >> 5];
  }
}

// The processed logits of one vector's VEC tokens (-inf where al does not allow a token) into p[0, VEC), skipping the
// tokens whose bit in skip is set (history tokens: the side pass writes them). 16-byte stores when nothing is skipped
// and p is 16-byte aligned (a whole vector per 4 tokens), else one store per token.
template <int VEC>
__device__ __forceinline__ void put_proc(float *p, bool p16, const float *x, uint32_t al, uint32_t skip) {
  if (p16 && skip == 0u) {
#pragma unroll
    for (int q = 0; q < VEC; q += 4)
      *reinterpret_cast<float4 *>(p + q) = make_float4(keep_or_ninf(x[q], al, q), keep_or_ninf(x[q + 1], al, q + 1),
                                                       keep_or_ninf(x[q + 2], al, q + 2),
                                                       keep_or_ninf(x[q + 3], al, q + 3));
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      if (!((skip >> k) & 1u)) p[k] = keep_or_ninf(x[k], al, k);
  }
}

// x of a full chunk (every token below the stream end) of a sampled row in place: the keep bits of each vector, mask AND
// NOT history, from the raw words with one bit-field extract; the NaN flag; -inf where a token is not kept (no select
// when the whole wave's chunk keeps everything); the lane's chunk maximum. The same results as chunk_z for such a chunk,
// with the range tests and shifts of the general chunk left out. PLAIN: a row with no mask and no penalties, whose
// tokens the stream all keeps (no keep bits, no select).
template <int DT, bool MASKED, bool PLAIN>
__device__ __forceinline__ float chunk_x_full(const RowCtx &c, int cb, float (&xr)[EPL], const uint32_t (&mw)[Lay<DT>::NV],
                                              const uint32_t (&hw)[Lay<DT>::NV], Run &rn, float *proc) {
  using L = Lay<DT>;
  static_assert(!(PLAIN && MASKED), "");
  constexpr uint32_t VMASK = (1u << L::VEC) - 1u;
  const int l = lane_id();
  const uint32_t sh = (uint32_t)(l * L::VEC) & 31u;
  uint32_t keep[L::NV];
  bool full = true;
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    if constexpr (PLAIN) {
      keep[v] = VMASK;
    } else {
      uint32_t w = MASKED ? mw[v] : 0xFFFFFFFFu;
      if (c.pen) w &= ~hw[v];
      keep[v] = __builtin_amdgcn_ubfe(w, sh, (uint32_t)L::VEC);
      full = full && keep[v] == VMASK;
    }
  }
  if (proc) {  // processed logits (after penalties and mask, before T) of the streamed (non-history) tokens
    const bool p16 = ((uintptr_t)proc & 15u) == 0;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int t0 = cb + v * L::STRIDE + l * L::VEC;
      const uint32_t al = MASKED ? __builtin_amdgcn_ubfe(mw[v], sh, (uint32_t)L::VEC) : VMASK;
      const uint32_t hx = !PLAIN && c.pen ? __builtin_amdgcn_ubfe(hw[v], sh, (uint32_t)L::VEC) : 0u;
      put_proc<L::VEC>(proc + t0, p16, xr + v * L::VEC, al, hx);
    }
  }
#pragma unroll
  for (int i = 0; i < EPL; i += 2) rn.nanm |= ballot64(__builtin_isunordered(xr[i], xr[i + 1]));  // (a NaN in either)
  float cmax = -INFINITY;
  if (PLAIN || ballot64(!full) == 0ull) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) cmax = fmaxf(cmax, xr[i]);
  } else {
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        xr[i] = keep_or_ninf(xr[i], keep[v], k);
        cmax = fmaxf(cmax, xr[i]);
      }
    }
  }
  if (!rn.fid_all) {  // (only until every lane has seen a value that is not NaN)
    if (rn.fid == 0xFFFFFFFFu) {
#pragma unroll
      for (int i = EPL - 1; i >= 0; --i) {
        const int t = cb + (i / L::VEC) * L::STRIDE + l * L::VEC + (i % L::VEC);
        if (xr[i] == xr[i]) rn.fid = (uint32_t)t;
      }
    }
    rn.fid_all = ballot64(rn.fid == 0xFFFFFFFFu) == 0ull;
  }
  return cmax;
}

// x of one chunk in place: the mask and the history exclusion (-inf for tokens the stream does not carry; a select only
// in chunks where some lane has such a token), the NaN flag (every loaded value is one of the row's own, so any NaN seen
// is the row's), the lane's chunk maximum; greedy rows track the first maximum of nan_to_num(x). hw holds the raw
// history bitset words of the chunk's vectors (bit (l VEC) % 32 + k is token k of lane l's vector).
template <int DT, bool AL, bool MASKED, bool GREEDY>
__device__ __forceinline__ float chunk_z(const RowCtx &c, int cb, int p0, int pv, int p1, float (&xr)[EPL],
                                         const uint32_t (&mw)[Lay<DT>::NV], const uint32_t (&hw)[Lay<DT>::NV],
                                         Run &rn, float *proc) {
  using L = Lay<DT>;
  constexpr uint32_t VMASK = (1u << L::VEC) - 1u;
  const int l = lane_id();
  uint32_t inr[L::NV], keep[L::NV];
  bool full = true;
#pragma unroll
  for (int v = 0; v < L::NV; ++v) {
    const int t0 = cb + v * L::STRIDE + l * L::VEC;
    uint32_t in;
    if constexpr (AL) in = t0 + L::VEC <= pv ? VMASK : 0u;
    else in = t0 + L::VEC <= pv ? VMASK : (t0 >= pv ? 0u : (1u << (pv - t0)) - 1u);
    if (c.pen) in &= ~(hw[v] >> ((l * L::VEC) & 31));
    inr[v] = in & VMASK;
    keep[v] = (MASKED ? (mw[v] >> ((l * L::VEC) & 31)) : VMASK) & inr[v];
    full = full && keep[v] == VMASK;
  }
  if (proc) {  // processed logits (after penalties and mask, before T) of the streamed tokens
    const bool p16 = ((uintptr_t)proc & 15u) == 0;
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int t0 = cb + v * L::STRIDE + l * L::VEC;
      const uint32_t al = MASKED ? (mw[v] >> ((l * L::VEC) & 31)) & VMASK : VMASK;
      put_proc<L::VEC>(proc + t0, p16, xr + v * L::VEC, al, ~inr[v] & VMASK);
    }
  }
#pragma unroll
  for (int i = 0; i < EPL; i += 2) rn.nanm |= ballot64(__builtin_isunordered(xr[i], xr[i + 1]));  // (a NaN in either)
  float cmax = -INFINITY;
  if (!GREEDY && ballot64(!full) == 0ull) {  // every token of the chunk is carried and allowed: no select
#pragma unroll
    for (int i = 0; i < EPL; ++i) cmax = fmaxf(cmax, xr[i]);
  } else {
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int t0 = cb + v * L::STRIDE + l * L::VEC;
#pragma unroll
      for (int k = 0; k < L::VEC; ++k) {
        const int i = v * L::VEC + k;
        const float xm = keep_or_ninf(xr[i], keep[v], k);
        if constexpr (GREEDY) {  // masked tokens take part in the argmax as -FLT_MAX
          const float g = fminf(fmaxf(xm, -FLTMAX), FLTMAX);
          if (((inr[v] >> k) & 1u) && xm == xm && (g > rn.g || rn.gid == 0xFFFFFFFFu)) {
            rn.g = g;
            rn.gid = (uint32_t)(t0 + k);
          }
        }
        xr[i] = xm;
        cmax = fmaxf(cmax, xm);
      }
    }
  }
  if (!rn.fid_all) {  // the lane's first chunk: its lowest token whose value is not NaN
    if (rn.fid == 0xFFFFFFFFu) {
#pragma unroll
      for (int i = EPL - 1; i >= 0; --i) {
        const int t = cb + (i / L::VEC) * L::STRIDE + l * L::VEC + (i % L::VEC);
        if (t < p1 && xr[i] == xr[i]) rn.fid = (uint32_t)t;
      }
    }
    rn.fid_all = ballot64(rn.fid == 0xFFFFFFFFu) == 0ull;
  }
  return cmax;
}

// Fixed pairwise sum ((f(0) + f(1)) + (f(2) + f(3))) + ... of f over [LO, HI), evaluating f(LO), f(LO + 1), ... in
// order with log2(HI - LO) partial sums live.
template <int LO, int HI, typename F>
__device__ __forceinline__ float pairwise(F &f) {
  if constexpr (HI - LO == 1) {
    return f(std::integral_constant<int, LO>{});
  } else {
    constexpr int MID = (LO + HI) / 2;
    const float x = pairwise<LO, MID>(f);
    const float y = pairwise<MID, HI>(f);
    return x + y;
  }
}

// The bound factor of a stream chunk's sum (EPL = 8 terms a lane: three levels of pairwise additions), raised by 2^-20
// relative so that the fp32 arithmetic of the chunk's bound (two fmas of non-negative terms, 2^-23 relative at most)
// stays inside it.
__device__ __forceinline__ float chunk_bound_factor(double bR) {
  return (float)((2.4e-7 + 3.0 * 6.0e-8 + 5e-8 + bR) * (1.0 + 0x1p-20));
}

// max(a, b) of two values that are never signaling NaNs, one v_max_f32 (fmaxf first quiets both operands)
__device__ __forceinline__ float fmax_q(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Raises the wave's listing threshold to the x key k (uniform): xt = the value of k, R = z(xt), and the lanes' sums
// rescaled to the new reference (fp64). c0 = RN(-R log2(e)); an R whose c0 leaves the fp32 range (|R| > 2.3e38) marks
// the part (its row takes the split-row finish or the exact path). An R of -inf leaves only -inf elements unlisted, of
// mass 0: c0 = -inf gives them exp2(-256) = 0.
__device__ __forceinline__ void set_threshold(Run &rn, uint32_t k, bool divide, double Rd) {
  const float xt = fkey_inv(k);
  const float R = divide ? div_exact(xt, Rd) : xt;
  if (rn.R > -INFINITY && R > rn.R) {
    const double f = exp((double)rn.R - (double)R);
    rn.s *= f;
    rn.b *= f;
  }
  const double cr = -(double)R * 1.4426950408889634;
  const bool fin = fabsf(R) < INFINITY;
  rn.ovf = rn.ovf || (fin && !(fabs(cr) <= 3.4028234663852886e38));
  rn.c0 = fin && fabs(cr) <= 3.4028234663852886e38 ? (float)cr : -INFINITY;
  rn.bR = fin ? 1.8e-7 * fabs((double)R) : 0.0;
  rn.kb = chunk_bound_factor(rn.bR);
  rn.xkey = k;
  rn.xt = xt;
  rn.R = R;
  rn.kcert = fkey(R) + 1u;
}

// The lane maximum, the threshold valve, the unlisted terms exp2(t), t = fma(x, c1, c0) = (x / T - R) log2(e) rounded
// (fp32 per chunk, fp64 across chunks; x < xt for every unlisted element, so z <= R and t <= 0 up to rounding), the
// listing of the elements with x >= xt. tok(i) gives the token of slot i.
template <int N, typename Tok>
__device__ __forceinline__ void chunk_sum(const ScanArgs &a, int row, int wl, float cmax, const float (&xr)[N],
                                          Run &rn, Tok tok, bool divide, double Rd) {
  static_assert((N & (N - 1)) == 0 && N <= 256, "");
  rn.m = fmax_q(rn.m, cmax);
  if (rn.woff >= rn.vnext) {  // (again after every KV / 2 more listed elements)
    const uint32_t k = max(rn.xkey, wave_kth_largest_u16(fkey(rn.m) >> 16, KV) << 16);
    if (k > rn.xkey) set_threshold(rn, k, divide, Rd);
    rn.vnext = rn.woff + KV / 2;
  }
  const float xt = rn.xt, c1 = rn.c1, c0 = rn.c0;
  // -inf (masked, excluded) gives t = -256 and e = 0; a NaN x gives t = -256 too (the NaN flag is kept apart)
  float e[N], t[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    t[i] = fmaxf(fmaf(xr[i], c1, c0), -256.0f);
    e[i] = __builtin_amdgcn_exp2f(t[i]);
  }
  if (ballot64(cmax >= xt)) {  // some lane holds an element at or above the threshold: list them (they leave the sum)
    uint64_t *cl = a.cand + ((size_t)row * a.nparts * PWAVES + wl) * CAPW;
    uint32_t woff = rn.woff;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const bool p = xr[i] >= xt;
      const uint64_t bl = ballot64(p);
      if (bl) {
        if (p) {
          const uint32_t pos = woff + lanes_below(bl);
          if (pos < (uint32_t)CAPW) st_ag(&cl[pos], raw_entry(xr[i], tok(i)));
          e[i] = 0.0f;
          t[i] = 0.0f;
        }
        woff += (uint32_t)__popcll(bl);
      }
    }
    rn.woff = woff;
  }
  float mom = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) mom = fmaf(e[i], t[i], mom);
  auto term = [&](auto ic) __attribute__((always_inline)) { return e[decltype(ic)::value]; };
  const float s = pairwise<0, N>(term);
  // error bound, relative to the terms: v_exp_f32 (2 ulp), log2(N) fp32 pairwise additions, flushed subnormal results;
  // the exponent's roundings: z = RN(x / T) against x / T, c1 = RN(log2(e) / T) and c0 = RN(-R log2(e)) (each 2^-24
  // relative: 2^-24 log2(e) (2 |x / T| + |R|) <= 2^-24 (4.33 |R| + 2 |t|), since |x / T| <= |R| + |t| ln 2), the fma's
  // own rounding (2^-24 |t|): times ln 2, 1.8e-7 |R| (bR) + 1.25e-7 |t| (mom = -sum e |t|)
  constexpr double LV = N >= 16 ? 4.0 : N >= 8 ? 3.0 : N >= 4 ? 2.0 : 1.0;
  rn.s += (double)s;
  if constexpr (N == EPL) {  // a stream chunk: its bound in fp32 (kb: the factor above, raised to cover this rounding)
    static_assert(EPL == 8, "kb is the factor of three pairwise levels");
    rn.b += (double)fmaf(s, rn.kb, fmaf(-mom, 1.2500012e-7f, 1e-36f));
  } else {
    rn.b += (double)s * (2.4e-7 + LV * 6.0e-8 + 5e-8 + rn.bR) - (double)mom * 1.25e-7 + 1e-36;
  }
}

// Tokens outside the stream (history tokens with their counts, ragged tokens with count 0; tok < 0: empty slot), with
// their logits x0 and mask bits al: penalties, NaN test, mask, z, then the same running state as the stream (tokens out
// of order: ties go to the lower id). Every thread of the wave takes part, with empty slots where it has no token.
template <int N, bool GREEDY>
__device__ __forceinline__ void side_tokens(const ScanArgs &a, const RowCtx &c, int row, int wl,
                                            bool listing, const int (&tk)[N], const uint32_t (&cnt)[N],
                                            const float (&x0)[N], const bool (&al)[N], Run &rn, float *proc) {
  float xr[N];
  float cmax = -INFINITY;
  bool hnan = false;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    xr[k] = -INFINITY;
    if (tk[k] >= 0) {
      const uint32_t t = (uint32_t)tk[k];
      const float x = cnt[k] ? penalize(x0[k], cnt[k], c.rp, c.fp, c.pp) : x0[k];
      hnan |= x != x;
      const float xm = al[k] ? x : -INFINITY;
      if (proc) proc[t] = xm;
      if (x == x && t < rn.fid) rn.fid = t;
      if constexpr (GREEDY) {
        const float g = fminf(fmaxf(xm, -FLTMAX), FLTMAX);
        if (xm == xm && (g > rn.g || (g == rn.g && t < rn.gid) || rn.gid == 0xFFFFFFFFu)) {
          rn.g = g;
          rn.gid = t;
        }
      }
      xr[k] = xm;
      cmax = fmaxf(cmax, xm);
    }
  }
  rn.nanm |= ballot64(hnan);
  if (listing) chunk_sum<N>(a, row, wl, cmax, xr, rn, [&](int i) { return (uint32_t)tk[i]; }, c.divide, c.Rd);
  else rn.m = fmaxf(rn.m, cmax);
}

// One part [p0, p1) of the row. Returns true in the workgroup that finished the row last (it then resolves the row).
// PC: a call with no histories and no masks (its own kernel: every row takes the plain stream).
template <int DT, bool AL, bool MASKED, bool GREEDY, bool DIV, bool PC>
__device__ __forceinline__ bool part_body(const ScanArgs &a, const gse_row &P, const RowCtx &c, int row, int part,
                                          Shared &sh) {
  using L = Lay<DT>;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int p0 = a.pstart[part], p1 = a.pstart[part + 1];
  const int pv = AL ? max(p0, p1 & ~(L::VEC - 1)) : p1;  // the stream's end; [pv, p1) go to the side pass
  const int nck = (pv - p0 + CHK - 1) / CHK;
  // candidates and the softmax sum are needed (not for greedy rows without logprobs, nor for verify nodes that keep
  // every token)
  const bool listing = (!GREEDY || nlp_of(a, P) > 0) && !(keeps_all_mss(a, P) && nlp_of(a, P) == 0);
  const int wl = part * PWAVES + w;                  // this wave's list
  float *proc = a.processed ? a.processed + (int64_t)row * a.processed_ld : nullptr;

  // History ids first, then the wave's first two chunks: the history tables build while the logits stream in.
  int hid[HPT];
  if (c.pen) {
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int j = c.hb + k * MT + tid;
      hid[k] = j < c.he ? a.hist[j] : -1;
    }
  }
  Cursor cur = cursor<DT>(c, p0 + __builtin_amdgcn_readfirstlane(w) * CHK, p1);
  // A ring of NB chunk buffers: chunk j of the wave (token chunk wu + j NWV) in slot j % NB, NB - 1 chunks loading while
  // the wave works on one. bf16 rows of the plain kernel keep six (4 registers a chunk, 1 KB a wave: five in flight
  // carry 80 KB a CU, where three left the stream short of bytes in flight to cover the memory latency); the others four
  // (no registers to spare).
  constexpr int NB = (DT == GSE_BF16 && PC) ? 6 : 4;
  uint32_t xr[NB][RAW<DT>];
  uint32_t mk[NB][L::NV];
  uint32_t hk[NB][L::NV] = {};  // history words (penalized rows)
  const int wu = __builtin_amdgcn_readfirstlane(w);  // (the wave index as a scalar: the chunk loop stays uniform)
  const int c0 = wu;  // wave w takes chunks w, w + 4, w + 8, ...
  // First token of chunk ck (unaligned rows' loads, the history words). A chunk past the stream gets a start far past
  // the row (vocabularies are at most 2^21 tokens); the loads of unaligned rows clamp to the part, and aligned rows read
  // through the cursor, whose range ends at the part's end: the loads a wave issues ahead of its last chunk fetch
  // nothing.
  const auto cst = [&](int ck) -> int { return ck < nck ? p0 + ck * CHK : (1 << 28); };
  // allowed tokens of the part's stream range (masked rows: popcounts of its mask words, every load issued before the
  // first is used; the sum comes after the history build)
  constexpr int APW = (PTOK / 32 + MT - 1) / MT;  // mask words per thread
  const int nmw = (pv - p0 + 31) >> 5;
  uint32_t mwd[APW];
  // (only the listing threshold uses the count: a greedy row without logprobs skips it; for sampled rows listing is
  // true at compile time and the loads are unconditional)
  const bool count_allowed = MASKED && listing;
  if (count_allowed) {
#pragma unroll
    for (int k = 0; k < APW; ++k) mwd[k] = c.mw[(p0 >> 5) + max(min(tid + k * MT, nmw - 1), 0)];
  }
  // The first chunks' loads go out once the history ids are in: issued with them, they queued behind every workgroup's
  // first chunks (about 40 MB over the device at C3) and the ids, the history build and the first chunk's processing
  // waited for them (C3: ids in at 6-8 us, first chunk processed at 15-17 us); issued after them, they stream in while
  // the history tables are built.
  if (c.pen) asm volatile("" ::"v"(hid[0]), "v"(hid[1]), "v"(hid[2]), "v"(hid[3]), "v"(hid[4]), "v"(hid[5]),
                          "v"(hid[6]), "v"(hid[7]));
  static_assert(HPT == 8, "");
#pragma unroll
  for (int j = 0; j < 3; ++j) load_u<DT, AL, MASKED>(c, cur, cst(wu + j * NWV), pv, p1, xr[j], mk[j]);
  if (tid == 0) sh.hover = 0;
  if (c.pen) build_history(c, a.hist, hid, p0, p1, sh.h, sh.wcnt, sh.hover);
  else __syncthreads();
  uint32_t apc = 0;
  if constexpr (MASKED) {
#pragma unroll
    for (int k = 0; k < (count_allowed ? APW : 0); ++k) {
      const int i = tid + k * MT;
      if (i < nmw) {
        uint32_t word = mwd[k];
        const int below = pv - (p0 + 32 * i);  // tokens of this word below pv (>= 1)
        if (below < 32) word &= (1u << below) - 1u;
        apc += (uint32_t)__popc(word);
      }
    }
  } else {
    apc = tid == 0 ? (uint32_t)(pv - p0) : 0u;
  }
  // The logits and mask words of the part's first KHP MT history tokens (by rank), loaded now so that the loads overlap
  // the first chunks; they wait in LDS for the side pass (the logit in hx, the mask bit in bit 31 of the count). Every
  // slot loads (an empty one from the part's first token), so no branch waits for the loads.
  float hx0[KHP];
  uint32_t hmw[KHP];
  if (c.pen) {
    const uint32_t nd = sh.h.nd;
#pragma unroll
    for (int k = 0; k < KHP; ++k) {
      const uint32_t r = (uint32_t)(tid + k * MT);
      const int t = p0 + (r < nd ? (int)sh.h.off[r] : 0);
      hx0[k] = load_one(c, t);
      hmw[k] = c.mw ? c.mw[t >> 5] >> (t & 31) : 1u;
    }
  }

  if (c.pen) {  // (the first three chunks were loaded before the history tables existed)
#pragma unroll
    for (int j = 0; j < 3; ++j) hist_words<DT>(sh.h, cst(wu + j * NWV), p0, p1, hk[j]);
  }
  Run rn;
  rn.m = -INFINITY;
  rn.s = 0.0;
  rn.b = 0.0;
  rn.xkey = 0;
  rn.xt = -INFINITY;
  rn.R = -INFINITY;
  rn.c1 = DIV ? (float)(1.4426950408889634 * c.Rd) : LOG2E;  // RN(log2(e) / T)
  rn.c0 = -INFINITY;
  rn.bR = 0.0;
  rn.kb = chunk_bound_factor(0.0);
  rn.kcert = 0;
  rn.ovf = false;
  rn.woff = 0;
  rn.vnext = (uint32_t)a.vfirst;
  rn.g = -INFINITY;
  rn.gid = 0xFFFFFFFFu;
  rn.fid = 0xFFFFFFFFu;
  rn.fid_all = false;
  rn.nanm = 0;
  auto tok_of = [&](int cb) {
    return [=](int i) { return (uint32_t)(cb + (i / L::VEC) * L::STRIDE + lane * L::VEC + (i % L::VEC)); };
  };
  // First chunk of each wave; the part's listing threshold from the 256 lane maxima.
  float cmax = -INFINITY;
  float x0[EPL];
  unpack<DT>(xr[0], x0);
  if (c0 < nck) cmax = chunk_z<DT, AL, MASKED, GREEDY>(c, p0 + c0 * CHK, p0, pv, p1, x0, mk[0], hk[0], rn, proc);
  if (listing) {
    // The listing threshold: the rank-kp largest of the 256 lane maxima of the waves' first chunks (a 2048-token
    // sample). kp is scaled so that about T tokens of the part lie above it: kp = T * (allowed tokens in the sample) /
    // (allowed tokens in the part), counted exactly, so that a mask whose allowed tokens cluster in runs does not skew
    // it. T = a.kt (200 for a part of at most PTOK tokens, 150 in a call with histories or masks), or 2 top_k + 32 (at
    // most 2 a.kt) for rows that keep at most top_k elements.
    uint32_t as = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) as += x0[i] > -INFINITY ? 1u : 0u;
    if (c0 >= nck) as = 0;
    as = wave_sum_u32(as);
    apc = wave_sum_u32(apc);
    if (lane == 0) {
      sh.wkap[w] = as;
      sh.wflags[w] = apc;
    }
    sh.lmax[tid] = fkey(cmax) >> 16;
    __syncthreads();
    uint32_t act = 0, As = 0, Ap = 0;
#pragma unroll
    for (int q = 0; q < NWV; ++q) {
      act += (uint32_t)__popcll(ballot64(sh.lmax[q * WAVE + lane] > (KEY_NEGINF >> 16)));
      As += sh.wkap[q];
      Ap += sh.wflags[q];
    }
    const uint32_t kt = (uint32_t)a.kt;
    const uint32_t T = P.top_k > 0 ? min(2u * kt, (uint32_t)(2 * max(P.top_k, nlp_of(a, P)) + 32)) : kt;
    // (a sample with few allowed tokens estimates nothing: then the lowest lane maximum, and the valve bounds the lists)
    const uint32_t kp = As < 16u ? max(act, 1u) : max(1u, min(act, (T * As + Ap - 1) / max(Ap, 1u)));  // (T As < 2^22)
    uint32_t r = 0;
#pragma unroll
    for (int b = 15; b >= 0; --b) {
      const uint32_t cand = r | (1u << b);
      uint32_t cnt = 0;
#pragma unroll
      for (int q = 0; q < NWV; ++q) cnt += (uint32_t)__popcll(ballot64(sh.lmax[q * WAVE + lane] >= cand));
      if ((int)cnt >= (int)kp) r = cand;
    }
    set_threshold(rn, max(r << 16, KEY_NEGINF + 1u), DIV, c.Rd);
  }
#pragma unroll
  for (int j = 3; j < NB; ++j) {
    load_u<DT, AL, MASKED>(c, cur, cst(wu + j * NWV), pv, p1, xr[j], mk[j]);
    if (c.pen) hist_words<DT>(sh.h, cst(wu + j * NWV), p0, p1, hk[j]);
  }
  if (c.pen) {
    const uint32_t nd = sh.h.nd;
#pragma unroll
    for (int k = 0; k < KHP; ++k) {  // (rank r is this thread's in the side pass too: no barrier)
      const uint32_t r = (uint32_t)(tid + k * MT);
      if (r < nd) {
        sh.hx[r] = hx0[k];
        sh.h.cnt[r] |= (hmw[k] & 1u) << 31;
      }
    }
  }
  if (c0 < nck) {
    if (listing) chunk_sum<EPL>(a, row, wl, cmax, x0, rn, tok_of(p0 + c0 * CHK), DIV, c.Rd);
    else rn.m = fmax_q(rn.m, cmax);
  }
  // Steady state: chunk j of the wave is wu + j NWV (scalar arithmetic: no LDS round trip and no vector temporary
  // between a chunk's loads and its use); chunks 1 .. NB - 1 are loading and each step issues the load of the chunk
  // NB - 1 ahead into the slot the previous step freed. The loop runs whole rounds of NB steps (the loads past the wave's
  // last chunk fetch nothing, their steps are skipped) with one back edge and the loads issued in the same order before
  // it and in it: the wait before each step then leaves the newer loads in flight (a loop with an exit in every step,
  // or loads issued in another order before it, made the first step of every round wait for all of them). The kernel of a call with no masks and no histories streams with the keep bits compiled out.
  const int nw = wu < nck ? (nck - wu + NWV - 1) / NWV : 0;  // the wave's chunks (uniform)
  auto stream = [&](auto plain) __attribute__((always_inline)) {
    constexpr bool PLAIN = decltype(plain)::value;
    const bool pen = !PLAIN && c.pen;
    auto step = [&](int ck, const uint32_t(&raw)[RAW<DT>], const uint32_t(&mw)[L::NV], const uint32_t(&hw)[L::NV])
                    __attribute__((always_inline)) {
      float x[EPL];
      unpack<DT>(raw, x);
      const bool full = !GREEDY && AL && p0 + (ck + 1) * CHK <= pv;  // a full chunk (uniform): the lean path
      if constexpr (PLAIN) {  // (each path ends with its own sum: the two do not join with x in different registers)
        if (full) {
          const float cm = chunk_x_full<DT, MASKED, PLAIN>(c, p0 + ck * CHK, x, mw, hw, rn, proc);
          if (listing) chunk_sum<EPL>(a, row, wl, cm, x, rn, tok_of(p0 + ck * CHK), DIV, c.Rd);
          else rn.m = fmax_q(rn.m, cm);
        } else {
          const float cm = chunk_z<DT, AL, MASKED, GREEDY>(c, p0 + ck * CHK, p0, pv, p1, x, mw, hw, rn, proc);
          if (listing) chunk_sum<EPL>(a, row, wl, cm, x, rn, tok_of(p0 + ck * CHK), DIV, c.Rd);
          else rn.m = fmax_q(rn.m, cm);
        }
      } else {  // (one sum: the general kernel holds no registers to spare for a second copy)
        const float cm = full ? chunk_x_full<DT, MASKED, PLAIN>(c, p0 + ck * CHK, x, mw, hw, rn, proc)
                              : chunk_z<DT, AL, MASKED, GREEDY>(c, p0 + ck * CHK, p0, pv, p1, x, mw, hw, rn, proc);
        if (listing) chunk_sum<EPL>(a, row, wl, cm, x, rn, tok_of(p0 + ck * CHK), DIV, c.Rd);
        else rn.m = fmax_q(rn.m, cm);
      }
    };
    auto fetch = [&](int j, uint32_t(&raw)[RAW<DT>], uint32_t(&mw)[L::NV], uint32_t(&hw)[L::NV])
                     __attribute__((always_inline)) {
      const int ck = wu + j * NWV;
      load_u<DT, AL, MASKED>(c, cur, cst(ck), pv, p1, raw, mw);
      if (pen) hist_words<DT>(sh.h, cst(ck), p0, p1, hw);
    };
    for (int j = 1; j < nw; j += NB) {  // (j % NB == 1: step s works on slot (s + 1) % NB, and refills slot s)
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        fetch(j + q + NB - 1, xr[q], mk[q], hk[q]);
        if (q == 0 || j + q < nw) step(wu + (j + q) * NWV, xr[(q + 1) % NB], mk[(q + 1) % NB], hk[(q + 1) % NB]);
      }
    }
  };
  stream(std::integral_constant<bool, PC>{});
  // the history tokens of the part (the tables are still in LDS: the resolve has not started), then the ragged ones
  if (c.pen) {
    const uint32_t nd = sh.h.nd;
    int tk[KH];
    uint32_t cn[KH];
    float x0[KH];
    bool al[KH];
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const uint32_t r = (uint32_t)(tid + k * MT);
      tk[k] = r < nd ? p0 + (int)sh.h.off[r] : -1;
      const uint32_t cw = r < nd ? sh.h.cnt[r] : 0u;
      if (k < KHP) {  // loaded ahead
        cn[k] = cw & 0x7FFFFFFFu;
        x0[k] = r < nd ? sh.hx[r] : 0.0f;
        al[k] = r < nd && (cw >> 31) != 0u;
      } else {
        cn[k] = cw;
        x0[k] = tk[k] >= 0 ? load_one(c, tk[k]) : 0.0f;
        al[k] = tk[k] >= 0 && mask_bit(c, tk[k]);
      }
    }
    side_tokens<KH, GREEDY>(a, c, row, wl, listing, tk, cn, x0, al, rn, proc);
  }
  if (AL && pv < p1 && w == 0) {  // (uniform: at most VEC - 1 tokens, wave 0)
    const int t = pv + lane;
    int tk[1] = {-1};
    const uint32_t cn[1] = {0u};
    if (t < p1) {
      const int o = t - p0;
      if (!(c.pen && ((sh.h.bits[o >> 5] >> (o & 31)) & 1u))) tk[0] = t;
    }
    const float x0[1] = {tk[0] >= 0 ? load_one(c, tk[0]) : 0.0f};
    const bool al[1] = {tk[0] >= 0 && mask_bit(c, tk[0])};
    side_tokens<1, GREEDY>(a, c, row, wl, listing, tk, cn, x0, al, rn, proc);
  }

  // Part record: the part maximum of z (z of the maximum of x), then every lane's sum rescaled to it (fp64, fixed order).
  const float wm = wave_max_f32(rn.m);
  uint64_t top;
  if (GREEDY) {
    top = rn.gid != 0xFFFFFFFFu ? pack(fkey(rn.g), rn.gid) : 0ull;
  } else {
    top = rn.fid != 0xFFFFFFFFu ? pack(KEY_NEGINF, rn.fid) : 0ull;
  }
  top = wave_max_u64(top);
  if (lane == 0) {
    sh.wmax[w] = wm;
    sh.wflags[w] = (rn.nanm ? F_NAN : 0u) | (rn.ovf ? F_OVERFLOW : 0u);  // (rn.ovf is wave-uniform)
    sh.wtop[w] = top;
    sh.wkap[w] = rn.kcert;
    sh.wcnt[w] = rn.woff;
  }
  __syncthreads();
  float Mx = sh.wmax[0];
#pragma unroll
  for (int k = 1; k < NWV; ++k) Mx = fmaxf(Mx, sh.wmax[k]);
  const float M = DIV ? div_exact(Mx, c.Rd) : Mx;
  double s = 0.0, b = 0.0;
  if (rn.R > -INFINITY && fabsf(M) < INFINITY) {  // the lane's sum, relative to its wave's threshold R, to M
    const double f = exp((double)rn.R - (double)M);
    s = rn.s * f;
    b = rn.b * f;
  }
  if (listing) {  // (without a listing the sums are zero)
    s = block_sum_f64(s, sh.wred);
    b = block_sum_f64(b, sh.wred);
  }
  if (tid == 0) {
    // flags: a finite value exists if the maximum of z over the allowed tokens is finite; a maximum of +inf (x = +inf,
    // or x / T overflowing) leaves the row to the exact path
    uint32_t flags = (sh.hover ? F_HOVER : 0u) | (fabsf(M) < INFINITY ? F_FINITE : 0u) | (M == INFINITY ? F_PINF : 0u);
    uint32_t kap = 0;
    uint64_t t = 0;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      flags |= sh.wflags[k];
      t = sh.wtop[k] > t ? sh.wtop[k] : t;
      kap = max(kap, sh.wkap[k]);
      if (sh.wcnt[k] > (uint32_t)CAPW) flags |= F_OVERFLOW;
    }
    SliceRec *r = a.rec + (size_t)row * a.nparts + part;
    st_ag(&r->top, t);
    st_ag(&r->kappa, listing ? kap : 0u);
    st_ag(&r->flags, flags);
    st_ag(&r->mkey, fkey(M));
#pragma unroll
    for (int k = 0; k < NWV; ++k) st_ag(&r->wcnt[k], min(sh.wcnt[k], (uint32_t)CAPW));
    st_ag(&r->s, s);
    st_ag(&r->bnd, b);
  }
  // Ticket: the last workgroup of the row resolves it.
  store_wait();
  __syncthreads();
  if (tid == 0) sh.ticket = ticket_add(&a.done[row]);
  __syncthreads();
  return sh.ticket == (uint32_t)(a.nparts - 1);
}

// Four waves per SIMD: every workgroup of a 256-row batch is resident at once (4 per CU). PC: the kernel of a call with
// no histories and no masks.
template <int DT, bool PC>
__global__ __launch_bounds__(MT) __attribute__((amdgpu_waves_per_eu(4, 8))) void main_kernel(ScanArgs a) {
  __shared__ Shared sh;
  const int L = blockIdx.x;
  int row, part;
  const int rows8 = (a.rows + 7) / 8 * 8;
  if (a.pmajor) {  // part-major: row L % rows8 (rows8 a multiple of 8: still on XCD row % 8)
    row = L % rows8;
    part = L / rows8;
  } else if (a.xcd_map) {  // the parts of a row on one XCD (workgroups go round-robin over the 8 XCDs): shared L2
    const int x = L & 7, i = L >> 3;
    row = x + 8 * (i / a.nparts);
    part = i % a.nparts;
  } else {
    row = L / a.nparts;
    part = L % a.nparts;
  }
  if (row >= a.rows) return;
  if (threadIdx.x < 64) sh.etab[threadIdx.x] = EXP2_64[threadIdx.x];  // (published by the first barrier)
  const gse_row P = a.params[row];
  RowCtx c = make_ctx(a, row, P);
  if constexpr (PC) {
    c.mw = nullptr;
    c.pen = false;
  }
  // 16-byte vector loads: the row start is 16-byte aligned and the row holds a whole vector (a vector past the stream's
  // end loads the row's first one)
  const bool aligned = (((uintptr_t)c.base) & 15u) == 0 && a.V >= Lay<DT>::VEC;
  // variants: alignment (16-byte vector loads), mask, greedy (no division), division by T (T != 1)
  // (MASKED variants read the row's mask words unconditionally: only rows with a mask take them)
  auto run = [&](auto masked) __attribute__((always_inline)) -> bool {
    constexpr bool M = decltype(masked)::value;
    if (c.greedy) {
      return aligned ? part_body<DT, true, M, true, false, PC>(a, P, c, row, part, sh)
                     : part_body<DT, false, M, true, false, PC>(a, P, c, row, part, sh);
    } else if (c.divide) {
      return aligned ? part_body<DT, true, M, false, true, PC>(a, P, c, row, part, sh)
                     : part_body<DT, false, M, false, true, PC>(a, P, c, row, part, sh);
    } else {
      return aligned ? part_body<DT, true, M, false, false, PC>(a, P, c, row, part, sh)
                     : part_body<DT, false, M, false, false, PC>(a, P, c, row, part, sh);
    }
  };
  bool last;
  if constexpr (PC) last = run(std::false_type{});
  else last = c.mw ? run(std::true_type{}) : run(std::false_type{});
  if (!last) return;
  // the row resolve is a chain of short dependent steps: give its waves issue priority over the streaming waves of the
  // other workgroups on this CU
  __builtin_amdgcn_s_setprio(3);
  resolve_row(a, row, P, sh);
  if (threadIdx.x == 0) a.done[row] = 0u;
}

}  // namespace

hipError_t launch_main(const ScanArgs &a, hipStream_t s) {
  const int rows = a.xcd_map ? (a.rows + 7) / 8 * 8 : a.rows;
  dim3 grid((unsigned)(rows * a.nparts)), block(MT);
  const bool pc = a.hist == nullptr && a.mask == nullptr;
  if (a.dtype == GSE_BF16) {
    if (pc) hipLaunchKernelGGL((main_kernel<GSE_BF16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((main_kernel<GSE_BF16, false>), grid, block, 0, s, a);
  } else {
    if (pc) hipLaunchKernelGGL((main_kernel<GSE_F32, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((main_kernel<GSE_F32, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace gse
