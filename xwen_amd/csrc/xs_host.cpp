// xs_host.cpp -- the host-only part of the C ABI: the argument checks of the
// device entry points, and the host entry points xs_select_option
// (select_option, batch.rs:1545-1588) and xs_keep_confident (keep_confident,
// generate.rs:3898-3905).  Plain C++: libxsamp.so links it, and oracle/Makefile
// builds it alone under AddressSanitizer and UBSan (target asan).
#include "xs_host.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <vector>

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The checks every device call shares: pointers, sizes, alignment, capacity.
int check_common(const xs_host_limits* lim, const float* logits, int64_t rows, int64_t ld,
                 int64_t width, int64_t enc, const void* params, const float* uniforms,
                 const uint32_t* allowed, int64_t allowed_words, int64_t allowed_ld) {
  if (!lim || !logits || !params || !uniforms) return XS_ERR_ARG;
  if (rows < 0 || enc < 1 || ld < 1) return XS_ERR_ARG;
  if (rows > lim->max_rows || enc > lim->vocab) return XS_ERR_CAPACITY;
  if (ld % 4 != 0 || !aligned16(logits)) return XS_ERR_ARG;
  if (width > ld) return XS_ERR_ARG;
  if (enc > ld && width >= enc) return XS_ERR_ARG;
  if (allowed && (allowed_ld < allowed_words || allowed_words < 0)) return XS_ERR_ARG;
  if (xs_host::chunks_for(enc) > lim->max_chunks) return XS_ERR_CAPACITY;
  return XS_OK;
}

}  // namespace

extern "C" {

bool xs_host_wants_lse(const xs_sample_args* in) {
  return in->row_max || in->row_lse || in->top_id || in->top_logprob || in->top_logprob64 ||
         in->score_ids || in->class_masks || in->probs;
}

bool xs_host_wants_scores(const xs_sample_args* in) {
  return in->score_ids || in->class_masks || in->probs;
}

int xs_host_check_sample(const xs_host_limits* lim, const xs_sample_args* in) {
  if (!lim || !in || !in->token || !in->status) return XS_ERR_ARG;
  const int rc = check_common(lim, in->logits, in->rows, in->ld, in->width, in->enc, in->params,
                              in->uniforms, in->allowed, in->allowed_words, in->allowed_ld);
  if (rc) return rc;
  if ((in->cand_id || in->cand_w) && in->cand_ld < 1) return XS_ERR_ARG;
  if (in->k_max < 0) return XS_ERR_ARG;
  if (in->n_top < 0 || in->n_top > XS_TOP_MAX) return XS_ERR_ARG;
  if ((in->top_id || in->top_logprob || in->top_logprob64) && in->top_ld < in->n_top) return XS_ERR_ARG;
  // the scoring reads (generate.rs:1871-1899)
  if (in->score_logprob && !in->score_ids) return XS_ERR_ARG;
  if (in->score_ids && (!in->score_logprob || in->n_score < 0 || in->n_score > XS_SCORE_MAX ||
                        in->score_ld < in->n_score))
    return XS_ERR_ARG;
  if ((in->class_masks != nullptr) != (in->class_mass != nullptr)) return XS_ERR_ARG;
  if (in->class_masks && (in->n_class < 0 || in->n_class > XS_CLASS_MAX || in->class_ld < (in->enc + 31) / 32))
    return XS_ERR_ARG;
  if (in->probs && in->probs_ld < in->enc) return XS_ERR_ARG;
  if (in->row_order) {  // a permutation of 0..rows-1 (a longer one is checked, then not applied)
    uint64_t small[XS_ORDER_MAX / 64] = {};
    std::vector<uint64_t> large;
    uint64_t* seen = small;
    if (in->rows > XS_ORDER_MAX) {
      large.assign((size_t)((in->rows + 63) / 64), 0ull);
      seen = large.data();
    }
    for (int64_t i = 0; i < in->rows; i++) {
      const int32_t r = in->row_order[i];
      if (r < 0 || r >= in->rows || ((seen[r >> 6] >> (r & 63)) & 1u)) return XS_ERR_ARG;
      seen[r >> 6] |= 1ull << (r & 63);
    }
  }
  return XS_OK;
}

int xs_host_check_verify(const xs_host_limits* lim, const xs_verify_args* in) {
  if (!lim || !in || !in->row_token || !in->row_status || !in->accepted || !in->committed ||
      !in->n_committed || !in->seq_status)
    return XS_ERR_ARG;
  if (in->seqs < 0 || in->span < 1 || in->n_eog < 0 || in->k_max < 0) return XS_ERR_ARG;
  if (in->n_eog > 0 && !in->eog) return XS_ERR_ARG;
  if (in->span > 1 && !in->drafts) return XS_ERR_ARG;
  if (in->seqs > INT64_MAX / in->span) return XS_ERR_CAPACITY;
  return check_common(lim, in->logits, in->seqs * in->span, in->ld, in->width, in->enc, in->params,
                      in->uniforms, in->allowed, in->allowed_words, in->allowed_ld);
}

int xs_host_check_argmax(const xs_host_limits* lim, const xs_argmax_args* in) {
  if (!lim || !in || !in->logits || !in->ids || !in->probs) return XS_ERR_ARG;
  if (in->rows < 0 || in->width < 1 || in->ld < in->width) return XS_ERR_ARG;
  if (in->rows > lim->max_rows || in->width > lim->vocab) return XS_ERR_CAPACITY;
  if (in->ld % 4 != 0 || !aligned16(in->logits)) return XS_ERR_ARG;
  if (xs_host::chunks_for(in->width) > lim->max_chunks) return XS_ERR_CAPACITY;
  return XS_OK;
}

int32_t xs_select_option(const double* scores, int64_t n, double temperature, int64_t top_k,
                         double top_p, double u, int64_t* index) {
  if (!scores || !index || n < 1) return XS_ERR_ARG;
  if (temperature <= 0.0 || top_k <= 1) {  // argmax_index: the first maximal score
    double best = -INFINITY;
    int64_t at = 0;
    for (int64_t i = 0; i < n; i++)
      if (scores[i] > best) {
        best = scores[i];
        at = i;
      }
    *index = at;
    return XS_ROW_OK;
  }
  // renormalize at the temperature: f64 softmax (the f64::max fold skips NaN)
  std::vector<double> p((size_t)n);
  double mx = -INFINITY;
  for (int64_t i = 0; i < n; i++) {
    p[i] = scores[i] / temperature;
    if (p[i] > mx) mx = p[i];
  }
  double total = -0.0;
  for (double& v : p) {
    v = std::exp(v - mx);
    total += v;
  }
  for (double& v : p) v = v / total;
  // rank by probability (f64::total_cmp, descending), ties to the lower index
  auto key = [](double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
  };
  std::vector<int64_t> order((size_t)n);
  for (int64_t i = 0; i < n; i++) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) { return key(p[x]) > key(p[y]); });
  const int64_t kept_k = std::min(top_k, n);
  // the nucleus over the survivors' own mass; the crossing option stays
  int64_t keep = kept_k;
  if (!(top_p >= 1.0)) {
    double mass = -0.0;
    for (int64_t i = 0; i < kept_k; i++) mass += p[order[i]];
    if (!(mass <= 0.0)) {
      double run = 0.0;
      for (int64_t i = 0; i < kept_k; i++) {
        run += p[order[i]] / mass;
        if (run >= top_p) {
          keep = i + 1;
          break;
        }
      }
    }
  }
  // WeightedIndex<f64> (rand 0.9): cumulative weights before each later
  // weight, the draw x = u * total, the count of cumulative weights <= x
  double acc = p[order[0]];
  if (!(acc >= 0.0)) return XS_ROW_ZERO_WEIGHT;
  std::vector<double> cum;
  for (int64_t i = 1; i < keep; i++) {
    const double w = p[order[i]];
    if (!(w >= 0.0)) return XS_ROW_ZERO_WEIGHT;
    cum.push_back(acc);
    acc += w;
  }
  if (acc == 0.0 || !std::isfinite(acc)) return XS_ROW_ZERO_WEIGHT;
  const double x = u * acc + 0.0;
  const int64_t c = std::upper_bound(cum.begin(), cum.end(), x) - cum.begin();
  *index = order[c];
  return XS_ROW_OK;
}

int64_t xs_keep_confident(const float* probs, int64_t n, float p_min) {
  int64_t kept = 0;
  while (kept < n && probs[kept] >= p_min) kept++;
  return kept;
}

}  // extern "C"
