/* gse.h: C ABI of libgse.so, the MI355X (gfx950) token-selection library.
 *
 * It replaces the host arithmetic under goethe-engine's sampling.py / spec.py / grammar.py call surface with HIP
 * kernels. Python binds it with ctypes (goethe-engine_amd/_lib.py), in the conventions of the reference's own C ABI
 * (abi/gc.h:1-22, bound by goethe_engine/gc_c.py:58-77):
 *
 *   Versioning  gse_abi_version() = MAJOR << 16 | MINOR. A minor only appends fields, flags and functions.
 *   Structs     every in/out struct starts with `size`, the caller's sizeof; the library reads only fields inside
 *               min(size, its own size) and treats absent fields as zero.
 *   Handles     gse_open returns an independent instance (own device workspace). One handle is not thread safe; each
 *               call takes the caller's HIP stream and is asynchronous on it.
 *   Errors      functions return GSE_OK (0) or a negative GSE_E_* code; gse_last_error(h) returns the text of the last
 *               error on that handle (gse_last_error(NULL): the last gse_open failure on this thread).
 *   Memory      every data pointer below is a device pointer unless marked host. Inputs are borrowed, never written;
 *               outputs are caller-owned buffers.
 */
#ifndef GSE_H
#define GSE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSE_ABI_MAJOR 1
#define GSE_ABI_MINOR 4
#define GSE_ABI_VERSION ((GSE_ABI_MAJOR << 16) | GSE_ABI_MINOR)

#if defined(__GNUC__)
#define GSE_API __attribute__((visibility("default")))
#else
#define GSE_API
#endif

typedef struct gse_handle gse_handle;

enum {
  GSE_OK = 0,
  GSE_E_ARG = -1,         /* bad argument or struct size */
  GSE_E_DEVICE = -4,      /* no such device, wrong architecture, out of device memory, HIP failure */
  GSE_E_UNSUPPORTED = -5, /* a request this library version cannot run */
  GSE_E_CAPACITY = -7     /* more rows / a larger vocabulary than the handle was opened for */
};

enum { GSE_F32 = 0, GSE_BF16 = 1 }; /* logits dtype */

typedef struct gse_open_params {
  uint32_t size;
  int32_t device;     /* HIP device ordinal */
  uint32_t max_rows;  /* rows per call */
  uint32_t max_vocab; /* vocabulary size per row, <= 2^21 */
} gse_open_params;

/* One row's selection parameters (device array of gse_row, 72 bytes each). The reference's SamplingParams
 * (goethe_engine/sampling.py:8-21) carries temperature, top_p, top_k; the other fields extend it with neutral
 * defaults (repetition 1, frequency 0, presence 0, min_p 0, logprobs 0). */
typedef struct gse_row {
  float temperature;        /* float32(t) as sampling.py:61 divides by; 0 = greedy (sampling.py:76-78) */
  int32_t top_k;            /* 0 = off (sampling.py:80 `top_k or V`) */
  double top_p;             /* (0, 1], compared in fp64 as sampling.py:80 does */
  double min_p;             /* [0, 1]; keep q_i >= min_p * q_0 */
  float repetition_penalty; /* > 0; 1 = off */
  float frequency_penalty;  /* finite; 0 = off */
  float presence_penalty;   /* finite; 0 = off */
  int32_t mask_row;         /* row of gse_batch.mask holding this row's packed bitmask, -1 = no mask */
  uint64_t seed;            /* uniform(seed, idx) (sampling.py:42-51) unless gse_batch.uniforms is given */
  uint64_t idx;
  int32_t hist_begin;       /* this row's token history: gse_batch.hist[hist_begin, hist_end) */
  int32_t hist_end;
  int32_t logprobs;         /* N of the top-N logprobs to return, 0..GSE_MAX_LOGPROBS */
  uint32_t flags;           /* GSE_ROW_* */
} gse_row;

/* gse_row.flags */
enum {
  GSE_ROW_TEMP_UNDERFLOW = 1u, /* temperature > 0 whose float32 is 0: sampled, dividing by 0 as sampling.py:61 does */
  GSE_ROW_MSS = 2u /* gse_verify_tree: this node's token comes from dist + mss over its kids (a strict request's node
                    * with kids, engine.py:278-283); without it the node samples and the walk follows the kid holding
                    * the sampled token (engine.py:270-276,284-285). Ignored by gse_sample / gse_dist. */
};

#define GSE_MAX_LOGPROBS 64

typedef struct gse_batch {
  uint32_t size;
  uint32_t dtype;          /* GSE_F32 or GSE_BF16 */
  uint32_t rows;
  uint32_t vocab;
  int64_t ld;              /* logits row stride in elements */
  const void *logits;      /* [rows][ld] (backend.py:37-42: one row per wanted token) */
  const gse_row *params;   /* [rows] */
  const int32_t *mask;     /* packed bitmask rows, token t = bit t % 32 of word t / 32 (grammar.py:42-45), or NULL */
  int64_t mask_ld;         /* words per mask row, >= ceil(vocab / 32) */
  const int32_t *hist;     /* token history ids for the penalties (ids outside [0, vocab) are ignored), or NULL */
  const double *uniforms;  /* [rows] shared per-row draws in [0, 1), or NULL: splitmix64(seed, idx) */
  void *stream;            /* hipStream_t; NULL = the null stream */
  uint32_t flags;          /* GSE_BATCH_* */
  uint32_t reserved;
} gse_batch;

/* gse_batch.flags */
enum {
  GSE_BATCH_EXACT = 1u,   /* finish every sampled row on the exact radix-select path (same results, slower) */
  GSE_BATCH_PROFILE = 2u, /* record HIP events around each kernel of this call on its stream (read with gse_profile) */
  GSE_BATCH_NO_PLAN_WAIT = 4u, /* testing: a split-row finish slice whose row's plan is not out when it first looks
                                * does not wait; the row takes the exact path (same results, slower) */
  GSE_BATCH_NO_SPLIT = 8u, /* the split-row finish is not launched: a row that would take it takes the exact path
                            * (same results). For batches that cannot use it, to save its launch: greedy rows of
                            * gse_sample never do (the Python layer sets it when every row is greedy). Since ABI 1.3. */
  GSE_BATCH_SUBBIN_FINISH = 16u /* testing: the split-row finish of every row takes its sub-bin walk, which it otherwise
                                 * keeps for window lists longer than 2048 entries (same results). Since ABI 1.4. */
};

typedef struct gse_out {
  uint32_t size;
  uint32_t reserved;
  int32_t *tokens;         /* [rows]: the sampled token, -1 for a row without a finite choice (sampling.py:84) */
  float *processed;        /* optional [rows][processed_ld]: logits after penalties and mask, before temperature */
  int64_t processed_ld;
  int32_t *logprob_ids;    /* optional [rows][logprobs_ld]: top-N token ids, descending, ties to the lowest id */
  float *logprobs;         /* optional [rows][logprobs_ld]: fp32 of fp64 log_softmax(z) at those ids */
  int64_t logprobs_ld;
} gse_out;

/* Node batch for multi-step speculative sampling (SpecInfer VerifyStochastic, goethe_engine/spec.py:88-103). */
typedef struct gse_mss_batch {
  uint32_t size;
  uint32_t nodes;          /* independent nodes */
  uint32_t vocab;
  uint32_t max_kids;
  double *p;               /* [nodes][p_ld] target distributions (vocabulary order); used as scratch, overwritten */
  int64_t p_ld;
  const double *q;         /* draft distribution rows [*][q_ld], or NULL when every kid is one-hot */
  int64_t q_ld;
  const int32_t *kid_tok;  /* [nodes][max_kids] kid tokens in draft order, -1 pads */
  const int32_t *kid_q;    /* [nodes][max_kids] row of q for the kid, -1 = one-hot (q None in spec.py:93) */
  const uint64_t *seed;    /* [nodes] request seed */
  const uint64_t *idx;     /* [nodes] uniform index (the engine's nout, engine.py:282) */
  int32_t *out_token;      /* [nodes] */
  int32_t *out_kid;        /* [nodes] index of the accepted kid, -1 when every kid was rejected */
  void *stream;
} gse_mss_batch;

/* Draft distributions of a speculative tree (the q of spec.py:26, Tree.q: the distribution each drafted token was drawn
 * from). Either fp64 probability rows in vocabulary order (GSE_Q_PROB, as the reference holds them), or drafter logits
 * / log-probabilities (GSE_Q_LOGITS_F32 / _BF16) with a per-row temperature t: q = softmax(float64(x) / t), as
 * spec.py:157 forms it, computed on the device and never materialised. */
enum { GSE_Q_PROB = 0, GSE_Q_LOGITS_F32 = 1, GSE_Q_LOGITS_BF16 = 2 };

typedef struct gse_qrows {
  uint32_t size;
  uint32_t kind;           /* GSE_Q_* */
  uint32_t rows;           /* q rows */
  uint32_t reserved;
  const void *q;           /* [rows][ld] */
  int64_t ld;
  const double *temperature; /* [rows] (GSE_Q_LOGITS_*): t > 0 */
} gse_qrows;

#define GSE_MAX_KIDS 16

/* One verify round of speculative decoding over many requests' draft trees (engine.py:262-298). Every tree node is one
 * row of the target batch: row u holds the target logits after node u, and its gse_row the request's parameters with
 * seed = the request's seed, idx = nout0 + depth(u) (the uniform index the walk gives the node, engine.py:272,282),
 * mask_row / history the grammar mask and penalty history that hold once the path to u is accepted, and GSE_ROW_MSS on
 * the nodes that take dist + mss. A request's nodes are consecutive rows starting at its anchor (parent -1), every
 * other node after its parent (spec.py:23-25). */
typedef struct gse_tree {
  uint32_t size;
  uint32_t requests;
  const int32_t *anchor;   /* [requests] row of each request's anchor, increasing */
  const int32_t *parent;   /* [rows] parent row (-1: an anchor) */
  const int32_t *token;    /* [rows] drafted token of the node (anchors: ignored) */
  const int32_t *qrow;     /* [rows] row of qrows holding the distribution the node's token was drawn from; -1 one-hot
                            * (a deterministic drafter, spec.py:93 q None); NULL: every kid one-hot */
  gse_qrows qrows;
  uint32_t max_kids;       /* >= the kids of any GSE_ROW_MSS node, <= GSE_MAX_KIDS */
  uint32_t reserved;
} gse_tree;

/* GSE_WALK_KIDS (since ABI 1.4): the walk reached a GSE_ROW_MSS node with more kids than gse_tree.max_kids (or
 * GSE_MAX_KIDS); its decision would have ignored the later kids, so the walk stops before it (emit_nodes[emit_len]
 * holds the node) instead of emitting a token the reference would not. */
enum { GSE_WALK_OK = 0, GSE_WALK_ERROR = 1, GSE_WALK_TRUNCATED = 2, GSE_WALK_KIDS = 3 };

typedef struct gse_tree_out {
  uint32_t size;
  uint32_t reserved;
  int32_t *emit_len;       /* [requests] tokens emitted by the walk */
  int32_t *emit_tokens;    /* [requests][emit_ld] the emitted tokens */
  int32_t *emit_nodes;     /* [requests][emit_ld] the node (row) each came from: the accepted path, anchor first; after
                            * an error, entry emit_len holds the node whose row had no valid token */
  int64_t emit_ld;         /* >= the deepest path + 1 (else GSE_WALK_TRUNCATED and the first emit_ld are written) */
  uint32_t *status;        /* [requests] GSE_WALK_*: ERROR when a node had no valid token (engine.py:286-288; the -1 is
                            * not emitted) */
  int32_t *node_token;     /* optional [rows]: the token each node emits if the walk reaches it */
  int32_t *node_kid;       /* optional [rows]: the kid row the node accepts, -1 none */
} gse_tree_out;

/* Drafter-side selection (spec.py:151-159 TreeDrafter._pick) for many nodes: row r of the drafter's logits /
 * log-probabilities picks n[r] children. temperature[r] == 0: the n best tokens in stable descending order; t > 0:
 * q = softmax(float64(x) / t) and n draws draw(q, uniform(mix(seed[r], SALT_DRAFT + k), at[r])), k = 0..n-1. */
typedef struct gse_pick_batch {
  uint32_t size;
  uint32_t dtype;          /* GSE_F32 or GSE_BF16 */
  uint32_t rows;
  uint32_t vocab;
  const void *x;           /* [rows][ld] */
  int64_t ld;
  const double *temperature; /* [rows] */
  const int32_t *n;        /* [rows] children to pick, <= out_ld */
  const uint64_t *seed;    /* [rows] */
  const uint64_t *at;      /* [rows] absolute index of the node's next token (spec.py:150 `at`) */
  int32_t *out_tokens;     /* [rows][out_ld] */
  double *out_logq;        /* [rows][out_ld] log q[x] (t > 0), or the input value x (t == 0), as spec.py:155,159 */
  int64_t out_ld;
  void *stream;
} gse_pick_batch;

/* Replaces: nothing (version handshake, as gc_abi_version, abi/gc.h:82). */
GSE_API uint32_t gse_abi_version(void);

/* Replaces: the host-side state of sampling.py (none); allocates the device workspace for max_rows x max_vocab. */
GSE_API int gse_open(const gse_open_params *p, gse_handle **out);

/* Replaces: goethe_engine/sampling.py:68-85 sample() with the mask application of grammar.py:42-45 / engine.py:272-273
 * fused in, plus penalties, min-p and top-N logprobs. One token per row; -1 for a NaN row or a row without a finite
 * choice. Greedy rows (temperature 0) take the first argmax of nan_to_num; the others the inverse CDF of
 * sampling.py:80-83 over the stable descending order. */
GSE_API int gse_sample(gse_handle *h, const gse_batch *in, const gse_out *out);

/* No counterpart in the reference. gse_sample for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no handle, and no hipMalloc / hipFree / allocating
 * library call. Its workspace is a static device array of about 21 MB that each GPU holds from the library's load until
 * the process ends, for batches of at most GSE_NOALLOC_ROWS rows of at most GSE_NOALLOC_VOCAB tokens (more:
 * GSE_E_CAPACITY). It runs on the current HIP device; the first call on a device sets that device's workspace up and
 * should not be captured. Every call on one GPU shares its workspace: calls that overlap on one GPU (two streams, two
 * threads) race. Errors: gse_last_error(NULL). Results are gse_sample's. GSE_BATCH_PROFILE is refused
 * (GSE_E_UNSUPPORTED): its events are host allocations, and without a handle nobody could read them. */
#define GSE_NOALLOC_ROWS 32
#define GSE_NOALLOC_VOCAB 163840
GSE_API int gse_sample_noalloc(const gse_batch *in, const gse_out *out);

/* Replaces: goethe_engine/sampling.py:88-97 dist(): fp64 probabilities over the vocabulary (vocabulary order) that
 * sample() draws a temperature > 0 row from, with top-k, top-p, min-p, penalties and mask; probs is [rows][probs_ld]. */
GSE_API int gse_dist(gse_handle *h, const gse_batch *in, double *probs, int64_t probs_ld);

/* Replaces: the acceptance walk of goethe_engine/engine.py:262-298 (one sample() call per tree level, dist + mss per
 * strict node, spec.py:88-103) with one call that runs every node of every request on the device and walks the trees
 * there: no host round trip per level. Stop rules (engine.py:218-229) stay with the caller, which ends each emitted
 * sequence at its first stop reason; the tokens before it do not depend on what follows. in->rows are the tree nodes.
 * With drafter logits, the q rows' statistics run on a stream of the handle, forked from in->stream at the call's start
 * and joined back before they are used: the call stays ordered on in->stream like every other. */
GSE_API int gse_verify_tree(gse_handle *h, const gse_batch *in, const gse_tree *tree, const gse_tree_out *out);

/* Replaces: goethe_engine/spec.py:151-159 TreeDrafter._pick (torch.sort / softmax / draw on the host) for a batch of
 * nodes. */
GSE_API int gse_draft_pick(gse_handle *h, const gse_pick_batch *in);

/* Replaces: the q of goethe_engine/spec.py:157 (TreeDrafter._pick: torch.softmax(lp.double() / t, 0), the distribution
 * a sampled child carries in Tree.q and that engine.py:282 hands to mss): fp64 rows q = softmax(float64(x) / t) of
 * drafter logits or log-probabilities (kind GSE_Q_LOGITS_F32 / _BF16, qrows->temperature[r] > 0), written to
 * out[r][0, vocab) (out_ld >= vocab). Since ABI 1.4. */
GSE_API int gse_qprob(gse_handle *h, const gse_qrows *qrows, uint32_t vocab, double *out, int64_t out_ld, void *stream);

/* Replaces: goethe_engine/sampling.py:100-104 draw(): inverse CDF in vocabulary order of each fp64 row q at u[r]:
 * min(count(cumsum(q) < u * sum(q)), last index with q > 0). */
GSE_API int gse_draw(gse_handle *h, const double *q, int64_t q_ld, uint32_t rows, uint32_t vocab, const double *u,
                     int32_t *out, void *stream);

/* Replaces: goethe_engine/spec.py:88-103 mss(), batched over independent nodes. */
GSE_API int gse_mss(gse_handle *h, const gse_mss_batch *in);

/* Replaces: the bool unpack of grammar.py:44-45 in reverse: bool rows [rows][bool_ld] (1 byte per token) -> packed
 * int32 words [rows][words_ld], so Matcher.mask() tensors can feed gse_batch.mask. */
GSE_API int gse_pack_mask(gse_handle *h, const uint8_t *bools, int64_t bool_ld, uint32_t rows, uint32_t vocab,
                          int32_t *words, int64_t words_ld, void *stream);

/* Replaces: nothing (measurement; the reference has no profiler). Calls made with GSE_BATCH_PROFILE record HIP events
 * around each of their kernels on their stream (no synchronisation), for up to GSE_PROFILE_CALLS calls. gse_profile
 * waits for the last recorded event, writes into ms[i] the total milliseconds of kernel slot i (launch order: main,
 * deep (the split-row finish), exact[, dist]) over the recorded calls and into *calls their number, then clears the
 * record. A call launches the split-row kernel, which then finishes every hard row itself, or, without it
 * (GSE_BATCH_NO_SPLIT, GSE_BATCH_EXACT), the exact kernel: the other one's slot holds only its two events. Returns the
 * number of kernel slots per call (<= n are written) or a negative GSE_E_* code. */
#define GSE_PROFILE_CALLS 512
GSE_API int gse_profile(gse_handle *h, float *ms, uint32_t n, uint32_t *calls);

/* Replaces: nothing (diagnostics; the reference has one path). Waits for the device, then writes into paths[r] which
 * path finished row r of the handle's last gse_sample / gse_dist call: GSE_PATH_MAIN (the fused pass), GSE_PATH_DEEP
 * (the split-row finish of a row whose keep prefix or top-p decision the pass could not settle), GSE_PATH_EXACT (the
 * exact radix-select path). rows must not exceed that call's rows. */
enum { GSE_PATH_MAIN = 0, GSE_PATH_DEEP = 1, GSE_PATH_EXACT = 2 };
GSE_API int gse_row_paths(gse_handle *h, uint32_t rows, uint8_t *paths);

/* Replaces: gc_last_error (abi/gc.h, goethe_engine/gc_c.py:222-227 turns it into RuntimeError). */
GSE_API const char *gse_last_error(gse_handle *h);

GSE_API void gse_close(gse_handle *h);

#ifdef __cplusplus
}
#endif

#endif /* GSE_H */
