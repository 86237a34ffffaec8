/*
 * xs_oracle.c -- CPU restatement of xwen's sampling path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, as the checker.  See xs_oracle.h for what pins each function.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: every float operation
 * here is one IEEE operation, exactly as the reference's Rust performs it).
 */
#include "xs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Correctly rounded binary32 exp.
 *
 * The reference computes every softmax term with f32::exp (sampler.rs:303),
 * i.e. the platform libm expf, which no reference test pins bit-wise.  The
 * oracle fixes it to the correctly rounded exp, which glibc's expf matches on
 * all but its rare 0.502-ulp cases.  Method: k = rint(32x/ln2), j = k mod 32,
 * r = x - k ln2/32 (Cody-Waite, 40-bit head so k*head is exact), exp(r) by its
 * Taylor series to r^7 (truncation < 2^-66), 2^(j/32) as a double-double, the
 * product carried as an unevaluated double-double, then one rounding to
 * binary32 that consults the tail only when the head sits exactly on a
 * binary32 midpoint.  Constants: 60-digit decimal evaluation, rounded once. */
static const double XO_INV_L = 0x1.71547652b82fep+5;
static const double XO_L_HI = 0x1.62e42fefa4000p-6;
static const double XO_L_LO = -0x1.8432a1b0e2634p-48;
static const double XO_T[32][2] = {
  {0x1.0000000000000p+0, 0x0.0p+0},
  {0x1.059b0d3158574p+0, 0x1.d73e2a475b465p-55},
  {0x1.0b5586cf9890fp+0, 0x1.8a62e4adc610bp-54},
  {0x1.11301d0125b51p+0, -0x1.6c51039449b3ap-54},
  {0x1.172b83c7d517bp+0, -0x1.19041b9d78a76p-55},
  {0x1.1d4873168b9aap+0, 0x1.e016e00a2643cp-54},
  {0x1.2387a6e756238p+0, 0x1.9b07eb6c70573p-54},
  {0x1.29e9df51fdee1p+0, 0x1.612e8afad1255p-55},
  {0x1.306fe0a31b715p+0, 0x1.6f46ad23182e4p-55},
  {0x1.371a7373aa9cbp+0, -0x1.63aeabf42eae2p-54},
  {0x1.3dea64c123422p+0, 0x1.ada0911f09ebcp-55},
  {0x1.44e086061892dp+0, 0x1.89b7a04ef80d0p-59},
  {0x1.4bfdad5362a27p+0, 0x1.d4397afec42e2p-56},
  {0x1.5342b569d4f82p+0, -0x1.07abe1db13cadp-55},
  {0x1.5ab07dd485429p+0, 0x1.6324c054647adp-54},
  {0x1.6247eb03a5585p+0, -0x1.383c17e40b497p-54},
  {0x1.6a09e667f3bcdp+0, -0x1.bdd3413b26456p-54},
  {0x1.71f75e8ec5f74p+0, -0x1.16e4786887a99p-55},
  {0x1.7a11473eb0187p+0, -0x1.41577ee04992fp-55},
  {0x1.82589994cce13p+0, -0x1.d4c1dd41532d8p-54},
  {0x1.8ace5422aa0dbp+0, 0x1.6e9f156864b27p-54},
  {0x1.93737b0cdc5e5p+0, -0x1.75fc781b57ebcp-57},
  {0x1.9c49182a3f090p+0, 0x1.c7c46b071f2bep-56},
  {0x1.a5503b23e255dp+0, -0x1.d2f6edb8d41e1p-54},
  {0x1.ae89f995ad3adp+0, 0x1.7a1cd345dcc81p-54},
  {0x1.b7f76f2fb5e47p+0, -0x1.5584f7e54ac3bp-56},
  {0x1.c199bdd85529cp+0, 0x1.11065895048ddp-55},
  {0x1.cb720dcef9069p+0, 0x1.503cbd1e949dbp-56},
  {0x1.d5818dcfba487p+0, 0x1.2ed02d75b3707p-55},
  {0x1.dfc97337b9b5fp+0, -0x1.1a5cd4f184b5cp-54},
  {0x1.ea4afa2a490dap+0, -0x1.e9c23179c2893p-54},
  {0x1.f50765b6e4540p+0, 0x1.9d3e12dd8a18bp-54},
};

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* The binary32 neighbour of f on the side of t (f != t, f finite or inf). */
static float xo_neighbour(float f, double t) {
  uint32_t u = f2u(f);
  if (f == 0.0f) return t > 0 ? u2f(1u) : u2f(0x80000001u);
  int up = (t > (double)f) ^ (f < 0.0f); /* move away from zero? */
  return u2f(up ? u + 1u : u - 1u);
}

static double xo_widen(float f) { /* inf counts as 2^128 when locating midpoints */
  return isinf(f) ? copysign(0x1p128, (double)f) : (double)f;
}

/* 0: correctly rounded exp (parity); 1: the platform libm expf, which is what
 * the reference's f32::exp calls (sampler.rs:303) -- used only to time the CPU
 * baseline at the reference's own speed. */
static int xo_exp_mode = 0;
void xo_set_exp_mode(int32_t mode) { xo_exp_mode = mode; }

static float xo_exp_cr(float xf);
float xo_exp(float xf) { return xo_exp_mode ? expf(xf) : xo_exp_cr(xf); }

void xo_exp_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = xo_exp_cr(x[i]);
}

static float xo_exp_cr(float xf) {
  if (xf != xf) return xf + xf;
  if (xf < -104.0f) return 0.0f;
  if (xf > 89.0f) return INFINITY;
  const double x = (double)xf;
  const double kd = rint(x * XO_INV_L);
  const int k = (int)kd;
  const double r1 = fma(-kd, XO_L_HI, x); /* exact */
  const double corr = -kd * XO_L_LO;
  const double r = r1 + corr;
  double h = 1.0 / 5040.0;
  h = fma(h, r, 1.0 / 720.0);
  h = fma(h, r, 1.0 / 120.0);
  h = fma(h, r, 1.0 / 24.0);
  h = fma(h, r, 1.0 / 6.0);
  h = fma(h, r, 0.5);
  const double q2 = (r * r) * h;
  const double w = corr + q2;
  const double uh = r1 + w; /* TwoSum(r1, w) */
  const double bb = uh - r1;
  const double ul = (r1 - (uh - bb)) + (w - bb);
  const int j = k & 31;
  const int e = (k - j) / 32;
  const double th = XO_T[j][0], tl = XO_T[j][1];
  const double p1 = th * uh;
  const double e1 = fma(th, uh, -p1);
  double s = th + p1; /* FastTwoSum: |th| >= 1 > |p1| */
  double err = (th - s) + p1;
  err = err + (e1 + (th * ul + tl * (1.0 + uh)));
  const double s2 = s + err;
  double err2 = (s - s2) + err;
  uint64_t scale_bits = (uint64_t)(e + 1023) << 52;
  double scale;
  memcpy(&scale, &scale_bits, 8);
  const double v = s2 * scale;
  err2 = err2 * scale;
  const float f = (float)v;
  if (xo_widen(f) == v) return f;
  const float g = xo_neighbour(f, v);
  const double mid = 0.5 * (xo_widen(f) + xo_widen(g));
  if (v == mid && err2 != 0.0) {
    const float lo = f < g ? f : g, hi = f < g ? g : f;
    return err2 > 0.0 ? hi : lo;
  }
  return f;
}

/* ------------------------------------------------------------------------ */
/* argmax -- sampler.rs:268-286.  First maximal index (strict >); any NaN is an
 * error; nothing above -inf is an error. */
int32_t xo_argmax(const float* v, int64_t n, uint32_t* out) {
  float best = -INFINITY;
  int64_t arg = -1, nans = 0;
  for (int64_t i = 0; i < n; i++) {
    if (isnan(v[i])) nans++;
    else if (v[i] > best) { best = v[i]; arg = i; }
  }
  if (nans) return XO_NAN;
  if (arg < 0) return XO_NO_FINITE;
  *out = (uint32_t)arg;
  return XO_OK;
}

/* softmax_in_place -- sampler.rs:289-310.  Scale by (float)(1/T) unless T==1,
 * max by the `b > a` fold, exp(v - max) with the serial f32 sum, divide. */
void xo_softmax_in_place(float* v, int64_t n, double temperature, int32_t sum_mode,
                         float s_given, float* max_out, float* sum_out) {
  if (temperature != 1.0) {
    const float inv = (float)(1.0 / temperature);
    for (int64_t i = 0; i < n; i++) v[i] *= inv;
  }
  float max = -INFINITY;
  for (int64_t i = 0; i < n; i++) if (v[i] > max) max = v[i];
  float sum;
  if (sum_mode == XO_SUM_SEQ_F32) {
    sum = 0.0f;
    for (int64_t i = 0; i < n; i++) { v[i] = xo_exp(v[i] - max); sum += v[i]; }
  } else if (sum_mode == XO_SUM_F64) {
    double sd = 0.0;
    for (int64_t i = 0; i < n; i++) { v[i] = xo_exp(v[i] - max); sd += (double)v[i]; }
    sum = (float)sd;
  } else {
    for (int64_t i = 0; i < n; i++) v[i] = xo_exp(v[i] - max);
    sum = s_given;
  }
  for (int64_t i = 0; i < n; i++) v[i] /= sum;
  if (max_out) *max_out = max;
  if (sum_out) *sum_out = sum;
}

/* Rust's f32::total_cmp as a signed key (core::f32::total_cmp). */
static int32_t total_key(float f) {
  int32_t b = (int32_t)f2u(f);
  b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
  return b;
}

typedef struct { float w; uint32_t id; } cand;

/* Stable descending sort by total_cmp: merge sort on (key desc, id asc). */
static int cand_before(const cand* a, const cand* b) {
  int32_t ka = total_key(a->w), kb = total_key(b->w);
  if (ka != kb) return ka > kb;
  return a->id < b->id;
}
static void merge_sort(cand* a, cand* tmp, int64_t n) {
  if (n < 2) return;
  int64_t h = n / 2;
  merge_sort(a, tmp, h);
  merge_sort(a + h, tmp, n - h);
  int64_t i = 0, j = h, o = 0;
  while (i < h && j < n) tmp[o++] = cand_before(&a[j], &a[i]) ? a[j++] : a[i++];
  while (i < h) tmp[o++] = a[i++];
  while (j < n) tmp[o++] = a[j++];
  memcpy(a, tmp, (size_t)n * sizeof(cand));
}

/* top_k_desc -- sampler.rs:356-384, literally: seed with the first k sorted
 * descending, then one `!(p <= floor)` test per entry and an insertion that
 * shifts while best[j-1] < p.  Requires 0 < k < n. */
int32_t xo_top_k_desc(const float* p, int64_t n, int64_t k, float* w, uint32_t* id) {
  for (int64_t i = 0; i < k; i++) if (isnan(p[i])) return XO_NAN;
  cand* best = (cand*)malloc((size_t)k * sizeof(cand) * 2);
  for (int64_t i = 0; i < k; i++) { best[i].w = p[i]; best[i].id = (uint32_t)i; }
  merge_sort(best, best + k, k);
  float floor_ = best[k - 1].w;
  for (int64_t i = k; i < n; i++) {
    const float q = p[i];
    if (!(q <= floor_)) {
      if (isnan(q)) { free(best); return XO_NAN; }
      int64_t j = k - 1;
      while (j > 0 && best[j - 1].w < q) { best[j] = best[j - 1]; j--; }
      best[j].w = q;
      best[j].id = (uint32_t)i;
      floor_ = best[k - 1].w;
    }
  }
  for (int64_t i = 0; i < k; i++) { w[i] = best[i].w; id[i] = best[i].id; }
  free(best);
  return XO_OK;
}

/* truncate_top_p -- sampler.rs:401-429.  No-op at top_p >= 1; else renormalise
 * by the serial f32 sum, keep the shortest prefix whose serial cumsum reaches
 * top_p (the crossing entry kept) and zero the rest.  The sum folds from -0.0
 * as Rust's f32 Sum does; for non-negative weights that equals folding from 0. */
void xo_truncate_top_p(float* w, int64_t n, float top_p) {
  if (top_p >= 1.0f) return;
  float sum = -0.0f;
  for (int64_t i = 0; i < n; i++) sum += w[i];
  if (sum <= 0.0f) return;
  for (int64_t i = 0; i < n; i++) w[i] /= sum;
  float cumsum = 0.0f;
  int64_t keep = n;
  for (int64_t i = 0; i < n; i++) {
    cumsum += w[i];
    if (cumsum >= top_p) { keep = i + 1; break; }
  }
  for (int64_t i = keep; i < n; i++) w[i] = 0.0f;
}

/* candidate_set -- sampler.rs:322-338.  k >= n: NaN check, then the whole row
 * stable-sorted descending; otherwise top_k_desc.  Then truncate_top_p. */
int32_t xo_candidate_set(const float* p, int64_t n, int64_t k, float top_p, float* w,
                         uint32_t* id, int64_t* n_out) {
  int64_t m;
  if (k >= n) {
    for (int64_t i = 0; i < n; i++) if (isnan(p[i])) return XO_NAN;
    cand* all = (cand*)malloc((size_t)(n > 0 ? n : 1) * sizeof(cand) * 2);
    for (int64_t i = 0; i < n; i++) { all[i].w = p[i]; all[i].id = (uint32_t)i; }
    merge_sort(all, all + n, n);
    for (int64_t i = 0; i < n; i++) { w[i] = all[i].w; id[i] = all[i].id; }
    free(all);
    m = n;
  } else {
    int32_t st = xo_top_k_desc(p, n, k, w, id);
    if (st) return st;
    m = k;
  }
  xo_truncate_top_p(w, m, top_p);
  *n_out = m;
  return XO_OK;
}

/* WeightedIndex<f32>::new + sample with a host uniform, restated from rand
 * 0.9's published algorithm (the crate is not in the reference tree; call site
 * sampler.rs:238-241).  new: total starts at w[0]; for each later weight the
 * running total is pushed before the weight is added (n-1 cumulative entries);
 * a negative/NaN weight or a zero total is an error.  sample: UniformFloat over
 * [0, total) maps its 23-bit uniform u to u*total + 0; the index is the
 * partition point of `cum <= x`, i.e. the count of cumulative entries <= x. */
int32_t xo_weighted_index(const float* w, int64_t n, float u, int64_t* idx) {
  if (n <= 0) return XO_ZERO_WEIGHT;
  float total = w[0];
  if (!(total >= 0.0f)) return XO_ZERO_WEIGHT;
  float* cum = (float*)malloc((size_t)(n > 1 ? n - 1 : 1) * sizeof(float));
  for (int64_t i = 1; i < n; i++) {
    if (!(w[i] >= 0.0f)) { free(cum); return XO_ZERO_WEIGHT; }
    cum[i - 1] = total;
    total += w[i];
  }
  if (total == 0.0f) { free(cum); return XO_ZERO_WEIGHT; }
  const float x = u * total + 0.0f;
  int64_t c = 0;
  while (c < n - 1 && cum[c] <= x) c++;
  free(cum);
  *idx = c;
  return XO_OK;
}

int32_t xo_control_is_noop(const xo_control* c) {
  /* SampleControl::is_noop -- sampler.rs:112-120 */
  return !c || (!c->allowed && c->n_banned == 0 && c->n_bias == 0 && !c->has_pull &&
                !c->has_force);
}

/* apply_control -- sampler.rs:433-490: allowed -> banned -> bias -> pull ->
 * force, with the short-mask, out-of-range-force and nothing-left errors. */
int32_t xo_apply_control(float* v, int64_t n, const xo_control* c) {
  if (c->allowed) {
    if (c->allowed_words * 32 < n) return XO_MASK_SHORT;
    for (int64_t i = 0; i < n; i++)
      if ((c->allowed[i / 32] & (1u << (i % 32))) == 0) v[i] = -INFINITY;
  }
  for (int64_t b = 0; b < c->n_banned; b++)
    if ((int64_t)c->banned[b] < n) v[c->banned[b]] = -INFINITY;
  for (int64_t b = 0; b < c->n_bias; b++)
    if ((int64_t)c->bias_id[b] < n) v[c->bias_id[b]] += c->bias_delta[b];
  if (c->has_pull) {
    const int64_t t = c->pull_id;
    if (t < n && isfinite(v[t])) {
      float max = -INFINITY;
      for (int64_t i = 0; i < n; i++) max = fmaxf(max, v[i]);
      v[t] += c->pull_alpha * fmaxf(max - v[t], 0.0f);
    }
  }
  if (c->has_force) {
    const int64_t t = c->force_id;
    if (t >= n) return XO_FORCE_OOR;
    const float target = v[t];
    for (int64_t i = 0; i < n; i++) v[i] = -INFINITY;
    v[t] = isfinite(target) ? target : 0.0f;
  } else {
    int64_t any = 0;
    for (int64_t i = 0; i < n && !any; i++) any = isfinite(v[i]);
    if (!any) return XO_NO_FINITE;
  }
  return XO_OK;
}

static double rel_gap(float a, float b) {
  if (a == b) return INFINITY;
  const double m = fmax(fabs((double)a), fabs((double)b));
  return fabs((double)a - (double)b) / m;
}

/* Sampler::sample_controlled -- sampler.rs:190-232, then draw -- :235-243.
 * The unadjusted stochastic draw in the reference softmaxes on the device
 * (candle, :216-224) in an association order no reference test pins; the
 * oracle runs the control-path softmax (:225-229) for every stochastic row
 * and exposes the denominator choice through sum_mode. */
void xo_sample_controlled(const float* logits, int64_t width, int64_t enc, double temperature,
                          int64_t top_k, double top_p, const xo_control* ctl, float u,
                          int32_t sum_mode, float s_given, float* work, float* cand_w,
                          uint32_t* cand_id, int32_t want_margins, xo_result* out) {
  memset(out, 0, sizeof(*out));
  out->margin_order = out->margin_cut = out->margin_draw = INFINITY;
  if (width < enc) { out->status = XO_NARROW; return; }
  memcpy(work, logits, (size_t)enc * sizeof(float));
  const int greedy = temperature <= 0.0 || top_k <= 1; /* Sampler::new, :133-145 */
  const int noop = xo_control_is_noop(ctl);
  if (!noop) {
    int32_t st = xo_apply_control(work, enc, ctl);
    if (st) { out->status = st; return; }
  }
  if (greedy) {
    out->status = xo_argmax(work, enc, &out->token);
    return;
  }
  const float p32 = (float)top_p; /* Strategy stores `top_p as f32` (:139) */
  float* ctl_vals = NULL;
  if (want_margins) {
    ctl_vals = (float*)malloc((size_t)enc * sizeof(float));
    memcpy(ctl_vals, work, (size_t)enc * sizeof(float));
  }
  xo_softmax_in_place(work, enc, temperature, sum_mode, s_given, &out->smax, &out->ssum);
  int64_t n = 0;
  int32_t st = xo_candidate_set(work, enc, top_k, p32, cand_w, cand_id, &n);
  if (!st) {
    out->n_cand = n;
    int64_t idx = 0;
    st = xo_weighted_index(cand_w, n, u, &idx);
    if (!st) out->token = cand_id[idx];
  }
  out->status = st;
  if (st || !want_margins) { free(ctl_vals); return; }
  /* Decision margins: how far each discrete decision sits from flipping when
   * the denominator moves.  order: adjacent numerators (the candidates and the
   * best excluded entry) that differ by a few ulps can collapse or separate
   * under another denominator; cut: the cumulative mass at the top-p crossing;
   * draw: the uniform's point against every cumulative boundary. */
  {
    const int64_t m = n < enc ? n + 1 : n;
    float* pw = (float*)malloc((size_t)m * sizeof(float));
    uint32_t* pid = (uint32_t*)malloc((size_t)m * sizeof(uint32_t));
    int64_t got = m;
    if (m < enc) xo_top_k_desc(work, enc, m, pw, pid);
    else xo_candidate_set(work, enc, enc, 1.0f, pw, pid, &got);
    const float inv = temperature != 1.0 ? (float)(1.0 / temperature) : 1.0f;
    double mo = INFINITY;
    for (int64_t i = 0; i + 1 < got; i++) {
      const float sa = temperature != 1.0 ? ctl_vals[pid[i]] * inv : ctl_vals[pid[i]];
      const float sb = temperature != 1.0 ? ctl_vals[pid[i + 1]] * inv : ctl_vals[pid[i + 1]];
      const double g = rel_gap(xo_exp(sa - out->smax), xo_exp(sb - out->smax));
      if (g < mo) mo = g;
    }
    out->margin_order = mo;
    free(pw);
    free(pid);
  }
  if (p32 < 1.0f) {
    float sum = -0.0f;
    float* w = (float*)malloc((size_t)n * sizeof(float));
    for (int64_t i = 0; i < n; i++) w[i] = work[cand_id[i]];
    for (int64_t i = 0; i < n; i++) sum += w[i];
    if (sum > 0.0f) {
      float cs = 0.0f;
      double mc = INFINITY;
      for (int64_t i = 0; i < n; i++) {
        cs += w[i] / sum;
        const double g = fabs((double)cs - (double)p32) / fmax((double)p32, 1e-30);
        if (g < mc) mc = g;
        if (cs >= p32) break;
      }
      out->margin_cut = mc;
    }
    free(w);
  }
  {
    float total = cand_w[0];
    double md = INFINITY;
    float cum[4096];
    int64_t nc = n - 1 < 4096 ? n - 1 : 4096;
    for (int64_t i = 1; i <= nc; i++) { cum[i - 1] = total; total += cand_w[i]; }
    const float x = u * total + 0.0f;
    for (int64_t i = 0; i < nc; i++) {
      if (cand_w[i + 1] == 0.0f && i + 1 < n) continue;
      const double g = fabs((double)x - (double)cum[i]) / (double)total;
      if (g < md) md = g;
    }
    out->margin_draw = md;
  }
  free(ctl_vals);
}

typedef struct {
  const float* logits; int64_t rows, ld, enc;
  const double* T; const int64_t* K; const double* P; const float* u;
  const uint32_t* mask; int64_t mask_ld; int64_t k_out; int32_t sum_mode;
  uint32_t* token; int32_t* status; float* cand_w; uint32_t* cand_id; float* smax; float* ssum;
  int64_t next; pthread_mutex_t mu;
} rows_job;

static void* rows_worker(void* arg) {
  rows_job* jb = (rows_job*)arg;
  float* work = (float*)malloc((size_t)jb->enc * sizeof(float));
  int64_t kcap = jb->k_out > 0 ? jb->k_out : 1;
  for (int64_t r = 0; r < jb->rows; r++) {
    const int64_t kk = jb->K[r] < jb->enc ? jb->K[r] : jb->enc;
    if (kk > kcap) kcap = kk;
  }
  float* cw = (float*)malloc((size_t)kcap * sizeof(float));
  uint32_t* ci = (uint32_t*)malloc((size_t)kcap * sizeof(uint32_t));
  for (;;) {
    pthread_mutex_lock(&jb->mu);
    const int64_t r = jb->next++;
    pthread_mutex_unlock(&jb->mu);
    if (r >= jb->rows) break;
    xo_control ctl;
    memset(&ctl, 0, sizeof(ctl));
    if (jb->mask) { ctl.allowed = jb->mask + r * jb->mask_ld; ctl.allowed_words = jb->mask_ld; }
    xo_result res;
    xo_sample_controlled(jb->logits + r * jb->ld, jb->ld, jb->enc, jb->T[r], jb->K[r], jb->P[r],
                         &ctl, jb->u[r], jb->sum_mode, 0.0f, work, cw, ci, 0, &res);
    jb->token[r] = res.token;
    jb->status[r] = res.status;
    if (jb->smax) jb->smax[r] = res.smax;
    if (jb->ssum) jb->ssum[r] = res.ssum;
    if (jb->cand_w) {
      for (int64_t i = 0; i < jb->k_out; i++) {
        const int in = i < res.n_cand;
        jb->cand_w[r * jb->k_out + i] = in ? cw[i] : 0.0f;
        jb->cand_id[r * jb->k_out + i] = in ? ci[i] : 0xFFFFFFFFu;
      }
    }
  }
  free(work);
  free(cw);
  free(ci);
  return NULL;
}

void xo_sample_rows(const float* logits, int64_t rows, int64_t ld, int64_t enc,
                    const double* temperature, const int64_t* top_k, const double* top_p,
                    const float* u, const uint32_t* mask, int64_t mask_ld, int64_t k_out,
                    int32_t sum_mode, int32_t nthreads, uint32_t* token, int32_t* status,
                    float* cand_w, uint32_t* cand_id, float* smax, float* ssum) {
  rows_job jb = {logits, rows, ld, enc, temperature, top_k, top_p, u, mask, mask_ld, k_out,
                 sum_mode, token, status, cand_w, cand_id, smax, ssum, 0,
                 PTHREAD_MUTEX_INITIALIZER};
  if (nthreads < 1) nthreads = 1;
  if (nthreads == 1) { rows_worker(&jb); return; }
  pthread_t* th = (pthread_t*)malloc((size_t)nthreads * sizeof(pthread_t));
  for (int i = 0; i < nthreads; i++) pthread_create(&th[i], NULL, rows_worker, &jb);
  for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
  free(th);
}

/* accept_drafts -- generate.rs:4020-4046.  The reference's sample_row closure
 * is replaced by precomputed per-row outcomes: with a host uniform per
 * position, row i's draw does not depend on whether rows < i were drawn, so
 * reading the precomputed outcome of row i only when the walk reaches it is
 * the same walk.  A row error propagates (the closure's `?`) only if reached. */
int32_t xo_accept_drafts(const uint32_t* drafts, int64_t n_drafts, int64_t budget,
                         const uint32_t* row_token, const int32_t* row_status,
                         const uint8_t* row_eog, int64_t* m_out, uint32_t* committed,
                         int64_t* n_committed, int64_t* calls) {
  const int64_t span = n_drafts + 1;
  int64_t m = 0, nc = 0, c = 0;
  for (int64_t i = 0; i < span; i++) {
    if (nc >= budget) break;
    c++;
    if (row_status && row_status[i]) {
      *m_out = m; *n_committed = nc; *calls = c;
      return row_status[i];
    }
    const uint32_t s = row_token[i];
    const int matched = i < n_drafts && s == drafts[i];
    committed[nc++] = s;
    if (matched) m++;
    if (!matched || row_eog[i]) break;
  }
  *m_out = m;
  *n_committed = nc;
  *calls = c;
  return XO_OK;
}

/* draft_argmax_probs / argmax_probs_device -- generate.rs:4059-4087: per row
 * the first maximal id and 1 / sum_j exp(l_j - max).  candle's reduction order
 * is not pinned by the reference; the oracle sums serially in f32. */
int32_t xo_draft_argmax_probs(const float* logits, int64_t n, int64_t vocab, uint32_t* ids,
                              float* probs) {
  for (int64_t r = 0; r < n; r++) {
    const float* row = logits + r * vocab;
    float max = -INFINITY;
    int64_t arg = 0;
    for (int64_t i = 0; i < vocab; i++) if (row[i] > max) { max = row[i]; arg = i; }
    float sum = 0.0f;
    for (int64_t i = 0; i < vocab; i++) sum += xo_exp(row[i] - max);
    ids[r] = (uint32_t)arg;
    probs[r] = 1.0f / sum;
  }
  return XO_OK;
}

/* keep_confident -- generate.rs:3898-3905: the longest prefix with p >= p_min
 * (a NaN fails the comparison and truncates). */
int64_t xo_keep_confident(const uint32_t* ids, const float* probs, int64_t n, float p_min) {
  (void)ids;
  int64_t kept = 0;
  while (kept < n && probs[kept] >= p_min) kept++;
  return kept;
}

/* held_row -- generate.rs:1905-1933: narrow to enc, NaN is an error, the
 * f32::max fold must be finite, denom = serial f64 sum of exp(f64(v - max)),
 * lse = f64(max) + ln(denom).  logprob(id) = f64(v[id]) - lse (:1871-1882). */
int32_t xo_held_row(const float* row, int64_t width, int64_t enc, float* max_out,
                    double* lse_out) {
  if (width < enc) return XO_NARROW;
  for (int64_t i = 0; i < enc; i++) if (isnan(row[i])) return XO_NAN;
  float max = -INFINITY;
  for (int64_t i = 0; i < enc; i++) max = fmaxf(max, row[i]);
  if (!isfinite(max)) return XO_NO_FINITE;
  double denom = 0.0;
  for (int64_t i = 0; i < enc; i++) denom += exp((double)(row[i] - max));
  *max_out = max;
  *lse_out = (double)max + log(denom);
  return XO_OK;
}

/* last_logprobs_for -- generate.rs:1871-1883: held_row's (values, lse), then
 * f64(v[id]) - lse for every id; an id outside [0, enc) fails the call. */
int32_t xo_last_logprobs_for(const float* row, int64_t width, int64_t enc, const int64_t* ids,
                             int64_t n, double* out) {
  float max;
  double lse;
  const int32_t st = xo_held_row(row, width, enc, &max, &lse);
  if (st != XO_OK) return st;
  for (int64_t i = 0; i < n; i++) {
    if (ids[i] < 0 || ids[i] >= enc) return XO_ID_OOR;
    out[i] = (double)row[ids[i]] - lse;
  }
  return XO_OK;
}

/* last_probs -- generate.rs:1893-1899: exp(f64(v) - lse) for every encodable
 * id, normalized as last_logprobs_for is. */
int32_t xo_last_probs(const float* row, int64_t width, int64_t enc, double* out) {
  float max;
  double lse;
  const int32_t st = xo_held_row(row, width, enc, &max, &lse);
  if (st != XO_OK) return st;
  for (int64_t i = 0; i < enc; i++) out[i] = exp((double)row[i] - lse);
  return XO_OK;
}

/* escape_mass's class sums -- batch.rs:1638-1662: the probabilities of the ids
 * a class holds, added one after another in id order (inside += p).  Class c
 * holds id t when bit t%32 of word t/32 of masks[c * mask_ld ..] is set. */
void xo_class_masses(const double* probs, int64_t enc, const uint32_t* masks, int64_t n_class,
                     int64_t mask_ld, double* out) {
  for (int64_t c = 0; c < n_class; c++) {
    const uint32_t* m = masks + c * mask_ld;
    double s = 0.0;
    for (int64_t t = 0; t < enc; t++)
      if ((m[t >> 5] >> (t & 31)) & 1u) s += probs[t];
    out[c] = s;
  }
}

/* det_logits -- sampler.rs:903-914 (the reference tests' input generator):
 * 64-bit LCG, u = (s >> 40) / 2^24, value (u - 0.5) * 2 * scale. */
void xo_det_logits(int64_t n, uint64_t seed, float scale, float* out) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i++) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    const float u = (float)(s >> 40) / (float)(1ull << 24);
    out[i] = (u - 0.5f) * 2.0f * scale;
  }
}

/* truncate_nucleus -- batch.rs:1562-1588: over probabilities already ranked
 * (desc), the number kept: all at top_p >= 1 or a total <= 0, else up to and
 * including the first whose running sum of p / total reaches top_p. */
int64_t xo_truncate_nucleus(const double* prob, int64_t n, double top_p) {
  if (top_p >= 1.0) return n;
  double total = -0.0;
  for (int64_t i = 0; i < n; i++) total += prob[i];
  if (total <= 0.0) return n;
  double cum = 0.0;
  for (int64_t i = 0; i < n; i++) {
    cum += prob[i] / total;
    if (cum >= top_p) return i + 1;
  }
  return n;
}

/* f64::total_cmp order as an unsigned key. */
static uint64_t total_key64(double d) {
  uint64_t b;
  memcpy(&b, &d, 8);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

/* select_option -- batch.rs:1545-1560, with renormalize (:1674-1680) and
 * argmax_index (:1683-1693): greedy on T <= 0 or top_k <= 1; else softmax at
 * T in f64 (libm exp), rank by (p desc by total_cmp, index asc), keep top_k,
 * cut the nucleus, and draw with WeightedIndex<f64> from u = j * 2^-52. */
int32_t xo_select_option(const double* scores, int64_t n, double temperature, int64_t top_k,
                         double top_p, double u, int64_t* index) {
  if (n < 1) return XO_ZERO_WEIGHT;
  if (temperature <= 0.0 || top_k <= 1) {
    double best = -INFINITY;
    int64_t at = 0;
    for (int64_t i = 0; i < n; i++)
      if (scores[i] > best) { best = scores[i]; at = i; }
    *index = at;
    return XO_OK;
  }
  double* p = (double*)malloc((size_t)n * sizeof(double));
  int64_t* rank = (int64_t*)malloc((size_t)n * sizeof(int64_t));
  double* w = (double*)malloc((size_t)n * sizeof(double));
  double mx = -INFINITY;
  for (int64_t i = 0; i < n; i++) {
    const double s = scores[i] / temperature;
    p[i] = s;
    if (s > mx) mx = s;  /* the f64::max fold from -inf: a NaN never replaces it */
  }
  double total = -0.0;
  for (int64_t i = 0; i < n; i++) {
    p[i] = exp(p[i] - mx);
    total += p[i];
  }
  for (int64_t i = 0; i < n; i++) p[i] = p[i] / total;
  /* insertion sort: stable, by total_cmp key desc */
  for (int64_t i = 0; i < n; i++) {
    int64_t j = i;
    while (j > 0 && total_key64(p[rank[j - 1]]) < total_key64(p[i])) { rank[j] = rank[j - 1]; j--; }
    rank[j] = i;
  }
  int64_t m = top_k < n ? top_k : n;
  for (int64_t i = 0; i < m; i++) w[i] = p[rank[i]];
  m = xo_truncate_nucleus(w, m, top_p);
  /* WeightedIndex<f64>::new + sample */
  int32_t st = XO_OK;
  double tw = w[0];
  if (!(tw >= 0.0)) st = XO_ZERO_WEIGHT;
  double* cum = (double*)malloc((size_t)(m > 1 ? m - 1 : 1) * sizeof(double));
  for (int64_t i = 1; i < m && st == XO_OK; i++) {
    if (!(w[i] >= 0.0)) { st = XO_ZERO_WEIGHT; break; }
    cum[i - 1] = tw;
    tw += w[i];
  }
  if (st == XO_OK && (tw == 0.0 || !isfinite(tw))) st = XO_ZERO_WEIGHT;
  if (st == XO_OK) {
    const double x = u * tw + 0.0;
    int64_t c = 0;
    while (c < m - 1 && cum[c] <= x) c++;
    *index = rank[c];
  }
  free(cum);
  free(w);
  free(rank);
  free(p);
  return st;
}
