// The fused selection pass: one workgroup per (row, 8192-token chunk), one HBM read of the logits, the mask words and
// the history ids; the last workgroup of each row to finish (atomic ticket, no waiting) resolves the row.
//
// Reference semantics (goethe_engine/sampling.py:68-85):
//   bad   = NaN anywhere before the mask, or no finite value after it        -> token -1
//   T = 0 -> first argmax of nan_to_num(masked x)                            (sampling.py:76)
//   T > 0 -> z = x / float32(T); stable descending order; fp64 softmax q; keep = rank < top_k AND cumsum(q) - q < top_p
//            (AND q >= min_p * q_0); c = cumsum(q * keep); token = order[count(c < u * c[-1])]   (sampling.py:59-83)
//
// The scan never sorts the row. Each wave keeps its 2048 keys in registers, sorts its 64 lane maxima and takes
// tau_w = the KW-th largest: every element >= tau_w is collected, so the union over a row's chunks, cut at
// tau* = max tau_c, is exactly the row's top elements in key order (the "certified head"). The resolve sorts only that
// head. A row whose keep prefix or draw lies past the head, or whose top-p decision is within the error bound of the
// cheap softmax sum, is marked hard and finished by the exact radix-select path (gse_exact.hip).
#include "gse_rowctx.h"

namespace gse {

namespace {

constexpr float LOG2E_F = 1.4426950408889634f;
constexpr int NWAVE = SCAN_THREADS / WAVE;

struct ScanShared {
  union {
    uint32_t cnt[CH];          // penalty counts of the chunk (sweep 1)
    uint64_t cert[CERT_CAP];   // certified head of the row (resolve)
  };
  uint64_t wc[NWAVE][CAPW];
  uint32_t wtau[NWAVE], wmax[NWAVE], wn[NWAVE];
  double ws[NWAVE], wm[NWAVE];
  uint64_t red64;
  uint32_t flags, ticket, ncand;
  // resolve scratch
  uint64_t rcmax;
  uint32_t rflags, rtau, ncert;
  double S, mom;
  int m, j, hard;
  double clast;
};

template <bool FULL, int VEC>
__device__ __forceinline__ void load_vec(const RowCtx &c, int tok0, float (&xv)[VEC]) {
  if (c.dtype == GSE_BF16) {
    const uint16_t *p = (const uint16_t *)c.base + tok0;
    if (FULL && VEC == 8) {
      const uint4 u = *reinterpret_cast<const uint4 *>(p);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) {
        xv[2 * i] = __uint_as_float(w[i] << 16);
        xv[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xv[v] = (tok0 + v < c.V) ? bf16_to_f32(p[v]) : 0.0f;
    }
  } else {
    const float *p = (const float *)c.base + tok0;
    if (FULL && VEC == 4) {
      const float4 u = *reinterpret_cast<const float4 *>(p);
      xv[0] = u.x;
      xv[1] = u.y;
      xv[2] = u.z;
      xv[3] = u.w;
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xv[v] = (tok0 + v < c.V) ? p[v] : 0.0f;
    }
  }
}

__device__ __forceinline__ int tok_of(int c0, int i, int vec) {
  return c0 + (i / vec) * (SCAN_THREADS * vec) + (int)threadIdx.x * vec + (i % vec);
}

// Sweep 1 over this thread's EPT tokens: keys into registers, the lane maximum, flags, processed logits.
// Token of register i: c0 + (i / VEC) * (SCAN_THREADS * VEC) + tid * VEC + i % VEC, increasing in i.
template <bool FULL, int VEC, bool GREEDY>
__device__ __forceinline__ void sweep1(const ScanArgs &a, const RowCtx &c, int row, int c0, const uint32_t *cnt,
                                       uint32_t (&key)[EPT], uint32_t &kmax, uint64_t &gmax, bool &fnan, bool &ffin) {
  constexpr int G = EPT / VEC;
  const int tid = threadIdx.x;
  float *proc = a.processed ? a.processed + (int64_t)row * a.processed_ld : nullptr;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int tok0 = c0 + g * (SCAN_THREADS * VEC) + tid * VEC;
    float xv[VEC];
    const bool any = FULL || tok0 < c.V;
    if (any) load_vec<FULL, VEC>(c, tok0, xv);
    const uint32_t mword = c.mw ? (any ? c.mw[tok0 >> 5] : 0u) : 0xFFFFFFFFu;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int t = tok0 + v;
      uint32_t k = 0;
      if (FULL || t < c.V) {
        const uint32_t ct = c.pen ? cnt[t - c0] : 0u;
        float xm;
        k = elem_key(c, xv[v], ct, (mword >> (t & 31)) & 1u, fnan, ffin, xm);
        if (proc) proc[t] = xm;
        if (GREEDY) {
          const uint64_t pk = pack(k, (uint32_t)t);
          gmax = pk > gmax ? pk : gmax;
        } else {
          kmax = max(kmax, k);
        }
      }
      key[g * VEC + v] = k;
    }
  }
}

// Sweep 2 (T > 0): the wave threshold, the cheap softmax sum of the wave, candidate collection into LDS.
template <bool FULL, int VEC>
__device__ __forceinline__ void sweep2(int c0, const uint32_t (&key)[EPT], uint32_t kmax, ScanShared &sh) {
  constexpr int G = EPT / VEC;
  const int tid = threadIdx.x, w = tid >> 6;
  const uint32_t srt = wave_sort_desc_u32(kmax);
  const uint32_t kw0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)srt);
  uint32_t tw = (uint32_t)__builtin_amdgcn_readfirstlane(__shfl((int)srt, KW - 1, WAVE));
  if (tw <= KEY_NEGINF) tw = KEY_NEGINF + 1u;
  double s = 0.0;
  float mom = 0.0f;
  if (kw0 > KEY_NEGINF && kw0 < KEY_POSINF) {
    const float mw = fkey_inv(kw0);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      if (FULL || key[i] > KEY_NEGINF) {
        const float d = fkey_inv(key[i]) - mw;  // <= 0; -inf for masked tokens (e = 0)
        const float e = __builtin_amdgcn_exp2f(d * LOG2E_F);
        s += (double)e;
        mom = fmaf(e, fminf(-d, 1.0e4f), mom);
      }
    }
  }
  uint32_t n = 0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const uint32_t k = key[g * VEC + v];
      const bool p = k >= tw;
      const uint64_t b = ballot64(p);
      if (b) {
        const uint32_t pos = n + lanes_below(b);
        if (p && pos < (uint32_t)CAPW)
          sh.wc[w][pos] = pack(k, (uint32_t)(c0 + g * (SCAN_THREADS * VEC) + tid * VEC + v));
        n += (uint32_t)__popcll(b);
      }
    }
  }
  s = wave_sum_f64(s);
  const double momd = wave_sum_f64((double)mom);
  if (lane_id() == 0) {
    sh.wtau[w] = tw;
    sh.wmax[w] = kw0;
    sh.wn[w] = n;
    sh.ws[w] = s;
    sh.wm[w] = momd;
  }
}

__device__ __forceinline__ void lp_invalid(const ScanArgs &a, int row, int nlp) {
  for (int i = threadIdx.x; i < nlp; i += blockDim.x) {
    a.lp_ids[(int64_t)row * a.lp_ld + i] = -1;
    a.lps[(int64_t)row * a.lp_ld + i] = __builtin_nanf("");
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// Row resolve, run by the last workgroup of the row.

__device__ void resolve_row(const ScanArgs &a, int row, const gse_row &P, ScanShared &sh) {
  const int tid = threadIdx.x;
  const ChunkHdr *hb = a.hdr + (size_t)row * a.nchmax;
  const bool greedy = is_greedy(a.mode, P);
  RowInfo *ri = a.info + row;
  const int nlp = a.lp_ids ? min(min(P.logprobs, GSE_MAX_LOGPROBS), (int)a.lp_ld) : 0;
  if (tid == 0) {
    sh.rcmax = 0;
    sh.rflags = 0;
    sh.rtau = 0;
    sh.ncert = 0;
    sh.hard = 0;
  }
  __syncthreads();
  for (int ch = tid; ch < a.nch; ch += blockDim.x) {
    const ChunkHdr *h = hb + ch;
    atomicOr(&sh.rflags, ld_acq(&h->flags));
    atomicMax((unsigned long long *)&sh.rcmax, (unsigned long long)ld_acq(&h->cmax));
    atomicMax(&sh.rtau, ld_acq(&h->tau));
  }
  __syncthreads();
  const uint32_t flags = sh.rflags;
  const uint64_t cmax = sh.rcmax;
  const uint32_t mk = pk_key(cmax);
  const bool bad = (flags & F_NAN) || !(flags & F_FINITE);

  if (a.mode == MODE_SAMPLE && (greedy || bad)) {
    const int32_t tok = bad ? -1 : (int32_t)pk_id(cmax);
    if (tid == 0) {
      a.tokens[row] = tok;
      RowInfo r = {};
      r.cmax = cmax;
      r.token = tok;
      // greedy rows' logprobs (z = x) come from the exact path, which leaves the token as is
      r.flags = (greedy ? R_GREEDY : 0u) | (bad ? R_BAD : 0u) | ((greedy && !bad && nlp) ? R_HARD : R_DONE);
      *ri = r;
    }
    if (bad || !nlp) lp_invalid(a, row, nlp);
    return;
  }
  const bool special = (flags & F_NAN) || P.temperature == 0.0f || mk >= KEY_POSINF || mk <= KEY_NEGINF;
  if (special) {
    // z holds +inf / NaN or its maximum is -inf: q is NaN, keep is empty and j clamps to 0 -> order[0] (sampling.py:82)
    if (tid == 0) {
      RowInfo r = {};
      r.cmax = cmax;
      r.flags = R_DONE | R_SPECIAL;
      r.token = (int32_t)pk_id(cmax);
      if (a.mode == MODE_SAMPLE) a.tokens[row] = r.token;
      *ri = r;
    }
    lp_invalid(a, row, nlp);
    return;
  }

  // Normal row: M finite; S from the chunk sums (fp64 exp of the chunk offsets, in chunk order).
  const double M = (double)fkey_inv(mk);
  if (tid == 0) {
    double S = 0.0, mom = 0.0;
    for (int ch = 0; ch < a.nch; ++ch) {
      const ChunkHdr *h = hb + ch;
      const uint32_t k = ld_acq(&h->mkey);
      if (k <= KEY_NEGINF || k >= KEY_POSINF) continue;
      const double mc = (double)fkey_inv(k);
      const double f = exp(mc - M);
      const double sc = ld_acq(&h->sc), mm = ld_acq(&h->mom);
      S += f * sc;
      mom += f * (mm + (M - mc) * sc);
    }
    sh.S = S;
    sh.mom = mom;
  }
  // Gather the certified head: every listed candidate with key >= tau*.
  const uint32_t tau = sh.rtau;
  for (int ch = 0; ch < a.nch; ++ch) {
    const uint32_t nc = ld_acq(&hb[ch].ncand);
    const uint64_t *cl = a.cand + ((size_t)row * a.nchmax + ch) * CAPC;
    for (uint32_t i = tid; i < nc; i += blockDim.x) {
      const uint64_t pk = ld_acq(&cl[i]);
      if (pk_key(pk) >= tau) {
        const uint32_t pos = atomicAdd(&sh.ncert, 1u);
        if (pos < (uint32_t)CERT_CAP) sh.cert[pos] = pk;
      }
    }
  }
  __syncthreads();
  const int ncert = (int)min(sh.ncert, (uint32_t)CERT_CAP);
  const bool overflow = (flags & F_OVERFLOW) || sh.ncert > (uint32_t)CERT_CAP;
  const bool complete = tau <= KEY_NEGINF + 1u;  // every element above -inf is in the head
  const int np2 = pow2_ceil(max(ncert, 2));
  for (int i = ncert + tid; i < np2; i += blockDim.x) sh.cert[i] = 0;
  __syncthreads();
  block_sort_desc_u64(sh.cert, np2);

  const double S = sh.S;
  const double epsS = 2.5e-7 * (sh.mom / S + 2.0);  // relative error bound of S (v_exp_f32 1 ulp, argument rounding)
  const double q0 = 1.0 / S;
  const int K = P.top_k > 0 ? P.top_k : 0x7FFFFFFF;
  const double topp = P.top_p, minp = P.min_p;
  const double u = a.uni ? a.uni[row] : uniform64(P.seed, P.idx);

  if (tid < WAVE) {
    // Walk the head in blocks of 64: q_i = exp(z_i - M) / S, C_i running inclusive sum; m = first rank failing keep.
    const int l = lane_id();
    double prefix = 0.0, prevC = 0.0, prevEx = 0.0;
    double cm1 = 0.0, exm1 = 0.0, exm = 0.0;
    int m = -1;
    bool hard = overflow || a.force_exact;
    bool topp_only_at_m = false;
    for (int b0 = 0; b0 < ncert && m < 0 && !hard; b0 += WAVE) {
      const int i = b0 + l;
      const bool valid = i < ncert;
      double q = 0.0;
      if (valid) q = exp((double)fkey_inv(pk_key(sh.cert[i])) - M) / S;
      const double C = prefix + wave_incl_scan_f64(q);
      const double ex = C - q;
      const bool kk = i < K, kp = ex < topp, km = q >= minp * q0;
      const uint64_t fail = ballot64(valid && !(kk && kp && km));
      if (fail) {
        const int fl = __builtin_ctzll(fail);
        m = b0 + fl;
        exm = shfl_f64(ex, fl);
        topp_only_at_m = __shfl((int)(kk && km && !kp), fl, WAVE) != 0;
        const double c1 = shfl_f64(C, (fl + WAVE - 1) & (WAVE - 1));
        const double e1 = shfl_f64(ex, (fl + WAVE - 1) & (WAVE - 1));
        cm1 = fl > 0 ? c1 : prevC;
        exm1 = fl > 0 ? e1 : prevEx;
      }
      prevC = shfl_f64(C, WAVE - 1);
      prevEx = shfl_f64(ex, WAVE - 1);
      prefix = prevC;
    }
    if (!hard && m < 0) {
      // every head element is kept: the boundary is past the head unless the head holds every element above -inf
      if (complete) {
        m = ncert;
        cm1 = prevC;
        exm1 = prevEx;
      } else {
        hard = true;
      }
    }
    if (!hard) {
      // top-p decisions must be robust to the relative error epsS of S (every q scales by 1 / S)
      const double delta = epsS * topp * 1.0001 + 1e-15;
      if (!(topp - exm1 > delta)) hard = true;
      if (m < ncert && topp_only_at_m && !(exm - topp > delta)) hard = true;
    }
    if (nlp > ncert) hard = true;
    int j = 0;
    if (!hard && a.mode == MODE_SAMPLE) {
      // j = number of kept ranks with C_i < u * c_last, recomputed with the same arithmetic (sampling.py:82)
      const double thr = u * cm1;
      double pre = 0.0;
      int cnt = 0;
      for (int b0 = 0; b0 < m; b0 += WAVE) {
        const int i = b0 + l;
        const bool valid = i < m;
        double q = 0.0;
        if (valid) q = exp((double)fkey_inv(pk_key(sh.cert[i])) - M) / S;
        const double C = pre + wave_incl_scan_f64(q);
        cnt += __popcll(ballot64(valid && C < thr));
        pre = shfl_f64(C, WAVE - 1);
      }
      j = min(cnt, m - 1);
      j = max(j, 0);
    }
    if (l == 0) {
      sh.m = m;
      sh.j = j;
      sh.hard = hard ? 1 : 0;
      sh.clast = cm1;
    }
  }
  __syncthreads();
  if (sh.hard) {
    if (tid == 0) {
      RowInfo r = {};
      r.cmax = cmax;
      r.flags = R_HARD;
      *ri = r;
    }
    return;
  }
  const int m = sh.m;
  if (tid == 0) {
    RowInfo r = {};
    r.cmax = cmax;
    r.kkeep = sh.cert[m - 1];
    r.S = S;
    r.Z = sh.clast;
    r.flags = R_DONE;
    r.ncert = (uint32_t)ncert;
    r.token = (int32_t)pk_id(sh.cert[sh.j]);
    if (a.mode == MODE_SAMPLE) a.tokens[row] = r.token;
    *ri = r;
  }
  if (nlp > 0) {
    const double lS = log(S);
    for (int i = tid; i < nlp; i += blockDim.x) {
      const uint64_t pk = sh.cert[i];
      a.lp_ids[(int64_t)row * a.lp_ld + i] = (int32_t)pk_id(pk);
      a.lps[(int64_t)row * a.lp_ld + i] = (float)(((double)fkey_inv(pk_key(pk)) - M) - lS);
    }
  }
}

template <bool FULL, int VEC, bool GREEDY>
__device__ void scan_body(const ScanArgs &a, const gse_row &P, const RowCtx &c, int row, int chunk, ScanShared &sh) {
  const int tid = threadIdx.x;
  const int c0 = chunk * CH;
  if (c.pen) build_counts(c, a.hist, c0, sh.cnt);
  uint32_t key[EPT];
  uint32_t kmax = 0;
  uint64_t gmax = 0;
  bool fnan = false, ffin = false;
  sweep1<FULL, VEC, GREEDY>(a, c, row, c0, sh.cnt, key, kmax, gmax, fnan, ffin);
  if (tid == 0) {
    sh.flags = 0;
    sh.red64 = 0;
    sh.ncand = 0;
  }
  __syncthreads();
  const uint32_t fl = (fnan ? F_NAN : 0u) | (ffin ? F_FINITE : 0u);
  if (fl) atomicOr(&sh.flags, fl);
  ChunkHdr *h = a.hdr + (size_t)row * a.nchmax + chunk;
  if (GREEDY) {
    const uint64_t wmx = wave_max_u64(gmax);
    if (lane_id() == 0) atomicMax((unsigned long long *)&sh.red64, (unsigned long long)wmx);
    __syncthreads();
    if (tid == 0) {
      st_rel(&h->cmax, sh.red64);
      st_rel(&h->flags, sh.flags);
      st_rel(&h->tau, 0u);
      st_rel(&h->ncand, 0u);
      st_rel(&h->mkey, pk_key(sh.red64));
    }
  } else {
    sweep2<FULL, VEC>(c0, key, kmax, sh);
    __syncthreads();
    uint32_t tau = 0, mkey = 0;
    bool over = false;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      tau = max(tau, sh.wtau[w]);
      mkey = max(mkey, sh.wmax[w]);
      over |= sh.wn[w] > (uint32_t)CAPW;
    }
    // lowest id holding the chunk maximum key (also when that maximum is -inf or NaN)
    uint64_t best = 0;
    if (kmax == mkey) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const int t = tok_of(c0, i, VEC);
        if ((FULL || t < c.V) && key[i] == mkey) {
          const uint64_t pk = pack(key[i], (uint32_t)t);
          best = pk > best ? pk : best;
        }
      }
    }
    best = wave_max_u64(best);
    if (lane_id() == 0) atomicMax((unsigned long long *)&sh.red64, (unsigned long long)best);
    // the chunk's certified list: wave candidates with key >= tau
    uint64_t *cl = a.cand + ((size_t)row * a.nchmax + chunk) * CAPC;
    for (int w = 0; w < NWAVE; ++w) {
      const uint32_t nw = min(sh.wn[w], (uint32_t)CAPW);
      for (uint32_t i = tid; i < nw; i += blockDim.x) {
        const uint64_t pk = sh.wc[w][i];
        if (pk_key(pk) >= tau) {
          const uint32_t pos = atomicAdd(&sh.ncand, 1u);
          if (pos < (uint32_t)CAPC) cl[pos] = pk;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      double sc = 0.0, mm = 0.0;
      if (mkey > KEY_NEGINF && mkey < KEY_POSINF) {
        const double mc = (double)fkey_inv(mkey);
        for (int w = 0; w < NWAVE; ++w) {
          if (sh.wmax[w] <= KEY_NEGINF || sh.wmax[w] >= KEY_POSINF) continue;
          const double mw = (double)fkey_inv(sh.wmax[w]);
          const double f = exp(mw - mc);
          sc += f * sh.ws[w];
          mm += f * (sh.wm[w] + (mc - mw) * sh.ws[w]);
        }
      }
      over |= sh.ncand > (uint32_t)CAPC;
      st_rel(&h->cmax, sh.red64);
      st_rel(&h->flags, sh.flags | (over ? F_OVERFLOW : 0u));
      st_rel(&h->tau, tau);
      st_rel(&h->ncand, min(sh.ncand, (uint32_t)CAPC));
      st_rel(&h->mkey, mkey);
      st_rel(&h->sc, sc);
      st_rel(&h->mom, mm);
    }
  }
  // Ticket: the last workgroup of the row resolves it (release our writes, acquire the others').
  __threadfence();
  __syncthreads();
  if (tid == 0) sh.ticket = atomicAdd(&a.done[row], 1u);
  __syncthreads();
  if (sh.ticket != (uint32_t)(a.nch - 1)) return;
  __threadfence();
  resolve_row(a, row, P, sh);
  if (tid == 0) a.done[row] = 0u;
}

template <int VEC>
__global__ __launch_bounds__(SCAN_THREADS, 4) void scan_kernel(ScanArgs a) {
  __shared__ ScanShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const gse_row P = a.params[row];
  const RowCtx c = make_ctx(a, row, P);
  const bool aligned = (((uintptr_t)c.base) & 15u) == 0;
  const bool full = aligned && (chunk + 1) * CH <= a.V;
  if (c.greedy) {
    if (full) scan_body<true, VEC, true>(a, P, c, row, chunk, sh);
    else scan_body<false, VEC, true>(a, P, c, row, chunk, sh);
  } else {
    if (full) scan_body<true, VEC, false>(a, P, c, row, chunk, sh);
    else scan_body<false, VEC, false>(a, P, c, row, chunk, sh);
  }
}

}  // namespace

hipError_t launch_scan(const ScanArgs &a, hipStream_t s) {
  dim3 grid(a.nch, a.rows), block(SCAN_THREADS);
  if (a.dtype == GSE_BF16) {
    hipLaunchKernelGGL(scan_kernel<8>, grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL(scan_kernel<4>, grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace gse
