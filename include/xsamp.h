/*
 * xsamp.h -- C ABI of the MI355X (gfx950) token sampler for xwen.
 *
 * One shared library (xwen_amd/libxsamp.so) exports these entry points.  Every
 * signature uses plain C types and pointers; no exceptions cross the ABI.  The
 * device buffers are HIP device pointers owned by the caller; the library only
 * borrows them for the duration of the (asynchronous) call on the context's
 * stream.
 *
 * Reference interface each entry point replaces (0rvar/xwen):
 *   xs_create / xs_destroy      Sampler::new                   src/sampler.rs:130-149
 *   xs_sample                   Sampler::sample_controlled     src/sampler.rs:190-232
 *                               + Sampler::draw                src/sampler.rs:235-243
 *                               (SampleControl, src/sampler.rs:85-121, and
 *                                apply_control src/sampler.rs:433-490)
 *                               + held_row / last_logprobs_for src/generate.rs:1871-1933
 *   xs_verify                   accept_drafts                  src/generate.rs:4020-4046
 *                               over the verify block          src/generate.rs:2410-2461
 *   xs_argmax_probs             argmax_probs_device /
 *                               draft_argmax_probs             src/generate.rs:4059-4087
 *   xs_keep_confident           keep_confident                 src/generate.rs:3898-3905
 *   xs_select_option            select_option                  src/batch.rs:1545-1588
 *
 * Randomness: the reference draws from a seeded StdRng inside the sampler.  Here
 * the caller supplies one uniform per sampled row, u = j * 2^-23 with j in
 * [0, 2^23) -- exactly the f32 rand 0.9's UniformFloat derives from 23 random
 * bits -- so the draw is a pure function of (logits, options, u).  Greedy rows
 * ignore their uniform, as the reference's greedy path never touches the RNG.
 *
 * Threading: a context is owned by one thread at a time and its calls are
 * serialised on its stream (the reference's Sampler is `&mut self`).  Two
 * contexts are independent.
 */
#ifndef XSAMP_H
#define XSAMP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes of the API calls (launch/argument errors, not data errors). */
#define XS_OK 0
#define XS_ERR_ARG (-1)      /* null pointer, bad size, misaligned row */
#define XS_ERR_HIP (-2)      /* a HIP runtime call failed */
#define XS_ERR_CAPACITY (-3) /* more rows / wider rows / larger k than the context holds */

/* Per-row data status, written to the `status` output.  The numbering matches
 * the reference's error conditions:
 *   XS_ROW_NAN         a NaN reached the draw (sampler.rs:268-286, :360-373)
 *   XS_ROW_NO_FINITE   nothing finite left after the controls (:483-488), or no
 *                      logit above -inf on the greedy path (:285)
 *   XS_ROW_MASK_SHORT  allow-mask narrower than the encodable ids (:437-442)
 *   XS_ROW_FORCE_OOR   forced id outside the vocabulary (:472-477)
 *   XS_ROW_ZERO_WEIGHT WeightedIndex saw no probability mass (:238-240)
 *   XS_ROW_NARROW      logit row narrower than the encodable bound (:196-200)
 *   XS_ROW_BAD_PARAM   min(top_k, enc) larger than the context's k_max, or a
 *                      control list past the context's ctl_max (XS_CTL_MAX by
 *                      default, xs_create_ex) entries (no reference
 *                      counterpart: the reference has no such limits)
 *   XS_ROW_INTERNAL    the row's workgroups did not all run on one XCD, as
 *                      the grid's placement expects (no reference
 *                      counterpart); the row was not sampled, its token is -1.
 *                      A context checks the placement when it is created and
 *                      otherwise hands sub-records off through memory, so
 *                      this is not seen in practice; xs_test_xcd forces it
 *   XS_ROW_ID_OOR      a scored id (score_ids) outside the encodable ids
 *                      (last_logprobs_for, generate.rs:1874-1879)           */
#define XS_ROW_OK 0
#define XS_ROW_NAN 1
#define XS_ROW_NO_FINITE 2
#define XS_ROW_MASK_SHORT 3
#define XS_ROW_FORCE_OOR 4
#define XS_ROW_ZERO_WEIGHT 5
#define XS_ROW_NARROW 6
#define XS_ROW_BAD_PARAM 7
#define XS_ROW_INTERNAL 8
#define XS_ROW_ID_OOR 9

/* Largest top_k the streaming selection serves (it keeps top_k + 1 entries).
 * A context created with k_max above it serves every top_k up to k_max --
 * top_k >= enc included, the reference's whole-row candidate set
 * (sampler.rs:322-338) -- through the whole-row path: every probability,
 * a (p desc, id asc) sort of the row and the serial f32 top-p and draw, in
 * kernels of their own after the row's finalizer. */
#define XS_K_MAX 127
/* Largest number of held_row log-probs per row. */
#define XS_TOP_MAX 128

typedef struct xs_context xs_context;

/* SamplerOptions (sampler.rs:36-41) minus the seed, one per row.
 * Sampler::new (sampler.rs:133-145): temperature <= 0 or top_k <= 1 is greedy;
 * otherwise top-k then top-p at this temperature.  top_p is the f32 the
 * reference stores (`top_p as f32`, sampler.rs:139). */
typedef struct {
  double temperature;
  int32_t top_k;
  float top_p;
} xs_row_params;

/* Sampler::new's allocation side: a context on `device` for up to `max_rows`
 * rows of up to `vocab` encodable ids (<= 1,048,576) and min(top_k, enc) <=
 * k_max (any k_max >= 0; the reference's top_k is an unbounded usize, and
 * INT32_MAX serves every top_k).  k_max above XS_K_MAX adds the whole-row
 * path's buffers, 16 bytes per row and id plus 1 KiB per row and 4,096 ids
 * (33 MB for 8 rows of 248,320), and every sampling call on such a context
 * then launches the whole-row kernels too (rows that do not take that path
 * return at once: about 33 us more per call when no row does), unless the
 * call bounds its own top_k at XS_K_MAX or less (xs_sample_args.k_max).
 * Allocates the device workspace once; calls allocate nothing afterwards. */
int xs_create(int device, int64_t max_rows, int64_t vocab, int32_t k_max, xs_context** out);

/* xs_create with room for control lists longer than XS_CTL_MAX: a row of a
 * call may then list up to ctl_max bans plus biases (SampleControl's lists are
 * unbounded slices, sampler.rs:85-121; a context is sized for the longest a
 * caller will pass, as for k_max).  ctl_max <= XS_CTL_MAX is xs_create;
 * above it the context holds 24 bytes per row and list entry (patch list and
 * sort buffers: 48 MB for 256 rows of 8,192).  Lists up to XS_CTL_MAX are
 * sorted in LDS, longer ones by a radix sort in those buffers. */
int xs_create_ex(int device, int64_t max_rows, int64_t vocab, int32_t k_max, int32_t ctl_max,
                 xs_context** out);
int xs_destroy(xs_context* ctx);
/* Bind the hipStream_t the context's kernels run on (NULL = the null stream). */
int xs_set_stream(xs_context* ctx, void* hip_stream);

/* The rest of one row's SampleControl (sampler.rs:85-121) past the allow-mask:
 * bans, additive biases, a pull and a force, applied after the mask in the
 * reference's order (apply_control, sampler.rs:433-490):
 *   banned  every listed id < enc goes to -inf (ids >= enc are skipped);
 *   bias    v[id] += delta for every listed (id, delta) with id < enc, in list
 *           order (a repeated id adds each delta in turn), f32 adds;
 *   pull    (id, alpha): if v[id] is finite, v[id] += alpha * max(0, M - v[id])
 *           with M the max over the row after the bans and biases (NaN
 *           ignored); a non-finite or out-of-range target is left alone;
 *   force   id: every other value goes to -inf and the target keeps its value
 *           if finite, else 0; id >= enc is XS_ROW_FORCE_OOR.
 * Without a force, a row left with no finite value is XS_ROW_NO_FINITE.  The
 * id lists live in two device pools shared by a call's rows: banned ids are
 * ctl_ids[ban_off .. ban_off + n_ban), bias entry i is (ctl_ids[bias_off + i],
 * ctl_delta[bias_off + i]).  A row may list at most XS_CTL_MAX bans and
 * biases together (the context's ctl_max for xs_create_ex); more (or a
 * negative count or offset) is XS_ROW_BAD_PARAM.  A row whose lists are empty and whose has_pull and
 * has_force are 0 is uncontrolled. */
#define XS_CTL_MAX 2048
typedef struct {
  int32_t ban_off, n_ban;
  int32_t bias_off, n_bias;
  int32_t has_pull;
  uint32_t pull_id;
  float pull_alpha;
  int32_t has_force;
  uint32_t force_id;
} xs_row_control;

/* One batched Sampler::sample_controlled + draw over `rows` independent rows.
 * All pointers are device pointers.  Required: logits, params, uniforms, token,
 * status.  Everything else may be NULL.
 *
 * The softmax denominator: a controlled row (an allow-mask or an active
 * xs_row_control) sums its terms serially in f32 in the reference
 * (softmax_in_place, sampler.rs:301-305), other rows through candle's softmax.
 * Where that sum reaches an output -- a stochastic controlled row at
 * top_p >= 1, whose weights are p = e / sum unrenormalized, in a call that
 * asks for cand_id, cand_w or soft_sum, and every controlled row of top_k >=
 * 128 -- it is reproduced bit for bit (a second kernel per call).  Elsewhere
 * the denominator is the exact sum of the same correctly rounded terms,
 * within 2e-6 of either reference sum, and on controlled rows the finalizer
 * proves that the serial sum would draw the same token (and candidate ids),
 * summing a row it cannot prove serially itself: the token of every
 * controlled row is the reference's on every call shape, xs_verify's too. */
typedef struct {
  const float* logits;   /* [rows, ld] row-major f32; 16-byte aligned, ld % 4 == 0 */
  int64_t rows;
  int64_t ld;            /* row stride in floats (>= width) */
  int64_t width;         /* logit row width; width < enc is XS_ROW_NARROW for every row */
  int64_t enc;           /* encodable ids: the draw is over ids [0, enc) (sampler.rs:191-201) */
  const xs_row_params* params; /* [rows] */
  const float* uniforms;       /* [rows], each j * 2^-23 */
  /* SampleControl::allowed: packed allow-mask, bit t%32 of word t/32 set means
   * id t may be drawn (sampler.rs:87-93).  NULL = no control (the reference's
   * no-op fast path).  allowed_words * 32 < enc is XS_ROW_MASK_SHORT. */
  const uint32_t* allowed; /* [rows, allowed_ld] */
  int64_t allowed_words;
  int64_t allowed_ld;
  /* outputs */
  int32_t* token;        /* [rows] sampled id (-1 on a row error) */
  int32_t* status;       /* [rows] XS_ROW_* */
  int32_t* cand_id;      /* [rows, cand_ld] the candidate set in draw order, or NULL */
  float* cand_w;         /* [rows, cand_ld] post-top-p weights (zeros included), or NULL */
  int32_t* n_cand;       /* [rows] candidates written (0 on greedy rows), or NULL;
                            entries past min(n_cand, cand_ld) are left as they were */
  int64_t cand_ld;       /* >= min(top_k, enc) of every row that writes candidates */
  float* soft_max;       /* [rows] max of the scaled, controlled row, or NULL */
  float* soft_sum;       /* [rows] softmax denominator used, or NULL */
  /* held_row statistics over the raw logits (generate.rs:1905-1933):
   * row_max, ln-sum-exp in f64, and the n_top highest logits (ties to the
   * lower id) as log-probs v - lse.  They ignore the allow-mask and the
   * controls, as held_row reads the raw row; a call with either makes a
   * second pass over its rows for them. */
  float* row_max;        /* [rows] or NULL */
  double* row_lse;       /* [rows] or NULL (NaN where held_row errors) */
  int32_t n_top;         /* 0..XS_TOP_MAX */
  int32_t* top_id;       /* [rows, top_ld] or NULL */
  float* top_logprob;    /* [rows, top_ld] or NULL */
  int64_t top_ld;
  /* SampleControl's bans, biases, pull and force (see xs_row_control), or
   * controls = NULL for none. */
  const xs_row_control* controls; /* [rows] */
  const uint32_t* ctl_ids;        /* banned and bias ids of every row */
  const float* ctl_delta;         /* bias deltas, indexed as ctl_ids */
  /* Scheduling hint, a HOST pointer (the one host pointer here), or NULL: a
   * permutation of 0..rows-1 giving the order in which rows are started.
   * Listing the rows with the costliest finalization first (top_k above 63,
   * held_row statistics, sparse controls) lets their long finalizers overlap
   * the other rows' streaming instead of ending the launch.  Outputs are the
   * same in any order.  Not a permutation is XS_ERR_ARG; the order of a call
   * of more than XS_ORDER_MAX rows is checked and not applied (its rows start
   * in their natural order), and neither is that of a call of fewer than 8
   * rows per XCD.  No counterpart in the reference, which samples one row at
   * a time. */
  const int32_t* row_order;
  /* A bound on min(top_k, enc) for this call, or 0 for the context's k_max:
   * rows above it report XS_ROW_BAD_PARAM, and a bound of XS_K_MAX or less
   * leaves out the whole-row kernels on a context sized for more, which
   * otherwise run on every call.  No counterpart in the reference, whose
   * options are per row: a caller batching rows of several top_k passes the
   * largest min(top_k, enc) among them. */
  int32_t k_max;
  /* Scoring reads of the held row (generate.rs:1871-1899, batch.rs:1504-1521,
   * :1628-1669), normalized by the same f64 lse as row_lse, over the raw row
   * as the held_row outputs are; each may be asked for alone (lse is then
   * computed without being written).  Not available
   * through xs_sample_noalloc (XS_ERR_ARG). */
  double* top_logprob64;          /* [rows, top_ld] the n_top log-probs in f64, or NULL */
  const int32_t* score_ids;       /* [rows, score_ld] ids to score, or NULL (last_logprobs_for) */
  int32_t n_score;                /* ids per row, 0..XS_SCORE_MAX */
  int64_t score_ld;
  double* score_logprob;          /* [rows, score_ld] f64(v[id]) - lse; an id outside
                                     [0, enc) makes the row XS_ROW_ID_OOR (token -1)
                                     and its entry NaN */
  /* Per-class probability masses: class c of row r holds id t when bit t%32
   * of word t/32 of class_masks[(r * n_class + c) * class_ld ..] is set (the
   * allow-mask layout); class_mass[r * n_class + c] = sum over those ids of
   * exp(f64(v) - lse), the sums escape_mass forms from last_probs. */
  const uint32_t* class_masks;    /* [rows, n_class, class_ld] or NULL */
  int32_t n_class;                /* 0..XS_CLASS_MAX */
  int64_t class_ld;               /* words per class mask, >= ceil(enc / 32) */
  double* class_mass;             /* [rows, n_class] */
  double* probs;                  /* [rows, probs_ld] exp(f64(v) - lse) of ids 0..enc-1
                                     (last_probs), or NULL */
  int64_t probs_ld;
} xs_sample_args;
#define XS_SCORE_MAX 4096
#define XS_CLASS_MAX 8
#define XS_ORDER_MAX 1024

int xs_sample(xs_context* ctx, const xs_sample_args* args);

/* xs_sample without a context, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is one
 * file-scope device array of XS_NOALLOC_BYTES (14.3 MiB) that each GPU the
 * library runs on holds until the process ends; the call runs on the current
 * device and on `hip_stream`, and allocates nothing.  Limits: rows <=
 * XS_NOALLOC_ROWS and enc <= XS_NOALLOC_VOCAB (else XS_ERR_CAPACITY);
 * min(top_k, enc) <= XS_K_MAX (else XS_ROW_BAD_PARAM for the row).  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two threads) race and must not be issued.  Each call clears the
 * arrival tickets it uses before its launch. */
#define XS_NOALLOC_ROWS 64
#define XS_NOALLOC_VOCAB 262144
#define XS_NOALLOC_BYTES 15030784
int xs_sample_noalloc(const xs_sample_args* args, void* hip_stream);

/* The speculative verify block: `seqs` sequences of `span` = D + 1 rows each
 * (D drafts plus the bonus position), laid out [seqs, span, ld].  Every row is
 * sampled as xs_sample would, with its own uniform; then each sequence runs
 * accept_drafts (generate.rs:4020-4046): walk i = 0..span-1, stop before a row
 * once `budget` tokens are committed, commit the sampled token, count it as
 * accepted while it equals drafts[i] (i < D), stop at the first mismatch or at
 * an end-of-generation id.  Because every row has its own uniform, sampling
 * all rows first and walking afterwards is the same walk. */
typedef struct {
  const float* logits;   /* [seqs * span, ld] */
  int64_t seqs;
  int64_t span;          /* D + 1, >= 1 */
  int64_t ld, width, enc;
  const xs_row_params* params;  /* [seqs * span] */
  const float* uniforms;        /* [seqs * span] */
  const uint32_t* allowed;      /* [seqs * span, allowed_ld] or NULL (per-position masks) */
  int64_t allowed_words, allowed_ld;
  const int32_t* drafts;        /* [seqs, span - 1] */
  const int32_t* budget;        /* [seqs] max committed tokens, or NULL = unbounded */
  /* end-of-generation ids (Sampler::is_eog, sampler.rs:245-247; the
   * reference's eog is a Vec<u32>, sampler.rs:130): n_eog >= 0 ids at the
   * device pointer eog (NULL when n_eog is 0) */
  int32_t n_eog;
  const int32_t* eog;           /* [n_eog] */
  /* outputs */
  int32_t* row_token;    /* [seqs * span] every row's sampled id */
  int32_t* row_status;   /* [seqs * span] */
  int32_t* accepted;     /* [seqs] m: matched drafts */
  int32_t* committed;    /* [seqs, span] committed ids (accepted drafts then the bonus) */
  int32_t* n_committed;  /* [seqs] */
  int32_t* seq_status;   /* [seqs] the first row error the walk reached, else XS_ROW_OK */
  /* per-position controls [seqs * span] as in xs_sample_args, or NULL: row i
   * of a sequence carries the bans and forces the caller derived for it
   * (generate.rs:2426-2461) */
  const xs_row_control* controls;
  const uint32_t* ctl_ids;
  const float* ctl_delta;
  /* [seqs * span] or NULL: nonzero at position i when committing drafts[i]
   * completes the grammar, which ends the walk like an EOG id
   * (generate.rs:2452-2459).  Row i+1 is reached only if draft i was
   * accepted, so the caller computes these, with the per-position masks,
   * by stepping a copy of its grammar state along the drafts. */
  const uint8_t* done_after;
  /* as xs_sample_args.k_max */
  int32_t k_max;
} xs_verify_args;

int xs_verify(xs_context* ctx, const xs_verify_args* args);

/* ---------------------------------------------------------------------------
 * Drafter confidence: argmax_probs_device / draft_argmax_probs
 * (generate.rs:4059-4087).  For each row of logits [rows, ld] (all `width`
 * columns: the reference reduces the raw lm_head row, with no encodable bound
 * and no temperature), the first maximal id (candle's argmax convention,
 * ties -> lower id) and p = 1 / sum_j exp(l_j - max), the sum taken in f64 and
 * rounded once to f32.  A row holding a NaN or +inf gets p = NaN (as candle's
 * exp(inf - inf) does), and a row holding a NaN or nothing above -inf gets
 * id -1; keep_confident truncates at a NaN p, so such ids are never drafted.
 * Outputs are device pointers [rows].  Rows are independent; the call runs on
 * the context's stream like xs_sample. */
typedef struct {
  const float* logits;   /* [rows, ld] row-major f32; 16-byte aligned, ld % 4 == 0 */
  int64_t rows;
  int64_t ld;            /* row stride in floats (>= width) */
  int64_t width;         /* columns reduced */
  int32_t* ids;          /* [rows] argmax id (-1: see above) */
  float* probs;          /* [rows] probability of the argmax */
} xs_argmax_args;

int xs_argmax_probs(xs_context* ctx, const xs_argmax_args* args);

/* Scored selection: select_option (batch.rs:1545-1588), host memory.  Over n
 * option scores (f64 sums of log-probs, e.g. from xs_sample's held_row
 * outputs): greedy (temperature <= 0 or top_k <= 1) returns the first maximal
 * score (argmax_index, batch.rs:1683-1693).  Otherwise the scores are
 * renormalized at the temperature (f64, batch.rs:1674-1680), ranked by
 * probability (desc, f64 total order) with ties to the lower index, cut to
 * top_k and then to the nucleus measured over the survivors' own mass (the
 * crossing option kept; none cut at top_p >= 1, truncate_nucleus,
 * batch.rs:1562-1588), and drawn with WeightedIndex<f64> from the uniform
 * u = j * 2^-52 (rand 0.9's f64 UniformFloat from 52 random bits).  Returns
 * XS_ROW_OK with *index set, XS_ROW_ZERO_WEIGHT when no option carries mass
 * (the reference's error), or XS_ERR_ARG. */
int32_t xs_select_option(const double* scores, int64_t n, double temperature, int64_t top_k,
                         double top_p, double u, int64_t* index);

/* keep_confident (generate.rs:3898-3905), host memory: the length of the
 * longest prefix whose probabilities are all >= p_min (a NaN ends it). */
int64_t xs_keep_confident(const float* probs, int64_t n, float p_min);

/* Library version string. */
const char* xs_version(void);

/* Test hook (no reference counterpart): y[i] = the kernels' correctly rounded
 * binary32 exp of x[i], device pointers, on `hip_stream`.  The parity tests use
 * it to compare the device exp with the CPU oracle's over millions of inputs. */
int xs_test_exp(const float* x, float* y, int64_t n, void* hip_stream);

/* Test hook (no reference counterpart): the finalizer's serial fallback.  A
 * controlled row (allow-mask or active controls) that no serial_kernel pass
 * finalizes is drawn with the exact softmax sum, and its finalizer checks
 * that the reference's serial f32 sum (sampler.rs:301-305) would draw the
 * same token; a row the check cannot settle is summed serially by its own
 * workgroup and drawn again.  *count (if not null) receives how many rows
 * took that fallback on this context so far (the call synchronizes the
 * context's stream); force != 0 sends every checked row of later calls
 * there, force == 0 restores the check. */
int xs_test_serial_fallback(xs_context* ctx, int32_t force, uint32_t* count);

/* Test hook (no reference counterpart): the XCD-local hand-off.  In a call
 * of at least 8 rows per XCD of the device, a row's workgroups run on
 * one XCD and hand their sub-records to the row's finalizer through that
 * XCD's L2; the row's arrival ticket proves the placement.  Smaller calls
 * spread each row over the XCDs and hand off through memory.  *xcd (if not
 * null) receives the context's XCD count (0: the placement was not confirmed
 * at creation, every call hands off through memory).  mode 0 is the normal
 * launch, 1 takes the split launch (the finalizers in a second kernel), 2
 * makes every XCD-local row of several chunks fail the placement check
 * (XS_ROW_INTERNAL). */
int xs_test_xcd(xs_context* ctx, int32_t mode, int32_t* xcd);

#ifdef __cplusplus
}
#endif
#endif
