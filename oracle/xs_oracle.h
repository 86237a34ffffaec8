/*
 * xs_oracle.h -- CPU restatement of xwen's sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP sampler is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; nothing in the product links or calls it.
 *
 * Every function restates one piece of the reference (0rvar/xwen) and cites
 * the file:line it follows.  Where the reference delegates arithmetic to a
 * third-party crate whose source is not in the reference tree (rand 0.9's
 * WeightedIndex/UniformFloat, the platform expf), the restatement follows the
 * crate's published algorithm and says so at the function.
 *
 * Pinning (what checks each function; details in the tests):
 *   xo_exp               exhaustive binary32 sweep against x87 expl, hard cases
 *                        adjudicated with 60-digit decimal; agrees with glibc expf
 *                        wherever glibc is correctly rounded.
 *   xo_argmax            reference known-answer tests (sampler.rs:544-576,
 *                        :606-621, :743-814, :1540-1614) + brute force.
 *   xo_softmax_in_place  closed form (f64 softmax) within 1e-6; reference KATs.
 *   xo_top_k_desc        sampler.rs:1491-1534 KATs + brute-force stable sort.
 *   xo_candidate_set /
 *   xo_truncate_top_p    sampler.rs:1102-1171 hand cases + an independent
 *                        full-sort llama.cpp restatement (sampler.rs:974-1006)
 *                        over the det_logits matrix of sampler.rs:1031-1060.
 *   xo_weighted_index    closed-form boundary cases (u=0, one nonzero weight,
 *                        exact cumulative boundaries) + 40k-draw frequencies
 *                        (sampler.rs:1177-1223).  The exact uniform->index map
 *                        is restated from rand 0.9's published WeightedIndex;
 *                        no reference test pins it bit-wise.
 *   xo_apply_control     sampler.rs:654-859 KATs.
 *   xo_accept_drafts     generate.rs:4119-4204 (the nine walks).
 *   xo_draft_argmax_probs generate.rs:5520-5552 (f64 scalar, 1e-5).
 *   xo_keep_confident    generate.rs:5560-5597.
 *   xo_held_row          f64 brute force (decimal) on small rows; the serial
 *                        f64 fold pinned by closed forms on dominant rows.
 *   xo_last_logprobs_for /
 *   xo_last_probs /
 *   xo_class_masses      60-digit decimal on small rows (each log-prob, each
 *                        probability, each class sum), the out-of-range error,
 *                        and the closed forms p = 1 / D of a dominant id and
 *                        sum of p = D_exact / D_fold.
 *   xo_select_option /
 *   xo_truncate_nucleus  batch.rs:2970-3016 (greedy on both conditions, a
 *                        top_k of 2 never reaching the third option, a tight
 *                        nucleus keeping the leader, an open draw reaching the
 *                        tail, the three nucleus cuts); the f64 uniform->index
 *                        map is restated from rand 0.9 as for f32.
 *   xo_det_logits        sampler.rs:903-914 generator, checked by the KATs
 *                        that consume it (top_p_of_zero, llama.cpp matrix).
 */
#ifndef XS_ORACLE_H
#define XS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Row status codes; the same numbering as the product's XS_ROW_* codes. */
enum {
  XO_OK = 0,
  XO_NAN = 1,          /* a NaN reached the draw (sampler.rs:268-286, :360-373) */
  XO_NO_FINITE = 2,    /* nothing finite left (sampler.rs:483-488, :285) */
  XO_MASK_SHORT = 3,   /* allow-mask narrower than the encodable ids (:437-442) */
  XO_FORCE_OOR = 4,    /* forced id outside the vocabulary (:472-477) */
  XO_ZERO_WEIGHT = 5,  /* WeightedIndex saw no mass (:238-240) */
  XO_NARROW = 6,       /* logit row narrower than the encodable bound (:196-200) */
  XO_ID_OOR = 9        /* a scored id outside the encodable ids (generate.rs:1874-1879) */
};

/* How softmax_in_place forms its denominator. */
enum {
  XO_SUM_SEQ_F32 = 0,  /* the reference's serial f32 sum (sampler.rs:301-305) */
  XO_SUM_F64 = 1,      /* the same f32 terms summed serially in f64, rounded once */
  XO_SUM_GIVEN = 2     /* use the caller's denominator (conditioning on a device sum) */
};

/* SampleControl (sampler.rs:85-121).  Null/zero members are "absent". */
typedef struct {
  const uint32_t* allowed;   /* packed allow-mask, bit t%32 of word t/32 */
  int64_t allowed_words;
  const uint32_t* banned;
  int64_t n_banned;
  const uint32_t* bias_id;
  const float* bias_delta;
  int64_t n_bias;
  int32_t has_pull;
  uint32_t pull_id;
  float pull_alpha;
  int32_t has_force;
  uint32_t force_id;
} xo_control;

/* The outcome of one sample_controlled call. */
typedef struct {
  int32_t status;
  uint32_t token;
  int64_t n_cand;     /* candidates written (0 on the greedy path) */
  float smax;         /* max of the scaled, controlled row */
  float ssum;         /* softmax denominator actually used */
  double margin_order;/* min relative gap between adjacent candidate numerators */
  double margin_cut;  /* |cumsum - top_p| / top_p at the cut (inf if no cut) */
  double margin_draw; /* min |x - cum_j| / total over the cumulative weights */
} xo_result;

float xo_exp(float x);
void xo_exp_array(const float* x, float* y, int64_t n); /* correctly rounded, always */
void xo_set_exp_mode(int32_t mode); /* 0 = correctly rounded (default), 1 = libm expf */
int32_t xo_argmax(const float* v, int64_t n, uint32_t* out);
void xo_softmax_in_place(float* v, int64_t n, double temperature, int32_t sum_mode,
                         float s_given, float* max_out, float* sum_out);
int32_t xo_top_k_desc(const float* p, int64_t n, int64_t k, float* w, uint32_t* id);
int32_t xo_candidate_set(const float* p, int64_t n, int64_t k, float top_p, float* w,
                         uint32_t* id, int64_t* n_out);
void xo_truncate_top_p(float* w, int64_t n, float top_p);
int32_t xo_weighted_index(const float* w, int64_t n, float u, int64_t* idx);
int32_t xo_apply_control(float* v, int64_t n, const xo_control* ctl);
int32_t xo_control_is_noop(const xo_control* ctl);

/* Sampler::sample_controlled (sampler.rs:190-232) + draw (:235-243).
 * work: scratch of at least `enc` floats.  cand_w/cand_id: at least min(k, enc). */
void xo_sample_controlled(const float* logits, int64_t width, int64_t enc, double temperature,
                          int64_t top_k, double top_p, const xo_control* ctl, float u,
                          int32_t sum_mode, float s_given, float* work, float* cand_w,
                          uint32_t* cand_id, int32_t want_margins, xo_result* out);

/* Row-parallel driver used by the CPU baseline: `rows` independent rows of
 * stride `ld`, each with its own options and uniform, no controls except an
 * optional per-row allow-mask (mask_ld words per row).  nthreads >= 1. */
void xo_sample_rows(const float* logits, int64_t rows, int64_t ld, int64_t enc,
                    const double* temperature, const int64_t* top_k, const double* top_p,
                    const float* u, const uint32_t* mask, int64_t mask_ld, int64_t k_out,
                    int32_t sum_mode, int32_t nthreads, uint32_t* token, int32_t* status,
                    float* cand_w, uint32_t* cand_id, float* smax, float* ssum);

int32_t xo_accept_drafts(const uint32_t* drafts, int64_t n_drafts, int64_t budget,
                         const uint32_t* row_token, const int32_t* row_status,
                         const uint8_t* row_eog, int64_t* m_out, uint32_t* committed,
                         int64_t* n_committed, int64_t* calls);
int32_t xo_draft_argmax_probs(const float* logits, int64_t n, int64_t vocab, uint32_t* ids,
                              float* probs);
int64_t xo_keep_confident(const uint32_t* ids, const float* probs, int64_t n, float p_min);
int32_t xo_held_row(const float* row, int64_t width, int64_t enc, float* max_out,
                    double* lse_out);
int32_t xo_last_logprobs_for(const float* row, int64_t width, int64_t enc, const int64_t* ids,
                             int64_t n, double* out);
int32_t xo_last_probs(const float* row, int64_t width, int64_t enc, double* out);
void xo_class_masses(const double* probs, int64_t enc, const uint32_t* masks, int64_t n_class,
                     int64_t mask_ld, double* out);
void xo_det_logits(int64_t n, uint64_t seed, float scale, float* out);
int64_t xo_truncate_nucleus(const double* prob, int64_t n, double top_p);
int32_t xo_select_option(const double* scores, int64_t n, double temperature, int64_t top_k,
                         double top_p, double u, int64_t* index);

#ifdef __cplusplus
}
#endif
#endif
