/*
 * exp_sweep.c -- exhaustive check of xo_exp (TEST INFRASTRUCTURE).
 *
 * For every binary32 x in [-104, 89] (about 2.24e9 inputs) compare xo_exp(x)
 * with the binary32 rounding of x87 expl(x) (64-bit significand, error about
 * 2^-63).  Inputs whose expl value lies within 2^-58 (relative) of a binary32
 * rounding boundary cannot be decided by expl and are printed as HARD lines for
 * adjudication at 60 digits (tests/golden/make_exp_cases.py).  Also counts
 * disagreements with glibc expf, which is not correctly rounded everywhere.
 *
 * usage: exp_sweep [stride] [threads]    (stride 1 = exhaustive)
 * output: one summary line, then MISMATCH/HARD lines (capped).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "xs_oracle.h"

typedef struct {
  uint32_t lo, hi, stride;
  uint64_t n, mismatch, glibc_diff, hard;
  uint32_t mism[16], hardv[64];
} range_job;

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static void* run(void* arg) {
  range_job* j = (range_job*)arg;
  for (uint64_t b = j->lo; b <= j->hi; b += j->stride) {
    const float x = u2f((uint32_t)b);
    const float e = xo_exp(x);
    const long double L = expl((long double)x);
    const float f = (float)L;
    /* distance of L to the nearest rounding boundary of binary32 */
    const float up = nextafterf(f, INFINITY), dn = nextafterf(f, -INFINITY);
    const long double m1 = ((long double)f + (long double)up) / 2;
    const long double m2 = ((long double)f + (long double)dn) / 2;
    const long double d1 = fabsl(L - m1), d2 = fabsl(L - m2);
    const long double d = d1 < d2 ? d1 : d2;
    j->n++;
    if (L > 0 && d < L * 0x1p-58L) {
      if (j->hard < 64) j->hardv[j->hard] = (uint32_t)b;
      j->hard++;
      continue;
    }
    if (e != f) {
      if (j->mismatch < 16) j->mism[j->mismatch] = (uint32_t)b;
      j->mismatch++;
    }
    if (expf(x) != e) j->glibc_diff++;
  }
  return NULL;
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1;
  const int nt = argc > 2 ? atoi(argv[2]) : 8;
  /* positive part [0, 89] and negative part [-0, -104] as bit ranges */
  float a = 89.0f, b = -104.0f;
  uint32_t pos_hi, neg_hi;
  memcpy(&pos_hi, &a, 4);
  memcpy(&neg_hi, &b, 4);
  const uint64_t pos_n = (uint64_t)pos_hi + 1, neg_n = (uint64_t)(neg_hi - 0x80000000u) + 1;
  const uint64_t total = pos_n + neg_n;
  range_job* jobs = calloc((size_t)nt, sizeof(range_job));
  pthread_t* th = calloc((size_t)nt, sizeof(pthread_t));
  /* split each half into nt/2 pieces */
  int half = nt / 2 > 0 ? nt / 2 : 1;
  int idx = 0;
  for (int part = 0; part < 2; part++) {
    uint64_t base = part == 0 ? 0 : 0x80000000u, n = part == 0 ? pos_n : neg_n;
    for (int i = 0; i < half && idx < nt; i++, idx++) {
      uint64_t lo = base + n * (uint64_t)i / (uint64_t)half;
      uint64_t hi = base + n * (uint64_t)(i + 1) / (uint64_t)half - 1;
      jobs[idx].lo = (uint32_t)lo;
      jobs[idx].hi = (uint32_t)hi;
      jobs[idx].stride = stride;
    }
  }
  for (int i = 0; i < idx; i++) pthread_create(&th[i], NULL, run, &jobs[i]);
  uint64_t n = 0, mm = 0, gd = 0, hard = 0;
  for (int i = 0; i < idx; i++) {
    pthread_join(th[i], NULL);
    n += jobs[i].n;
    mm += jobs[i].mismatch;
    gd += jobs[i].glibc_diff;
    hard += jobs[i].hard;
  }
  printf("checked %llu of %llu inputs: mismatch %llu hard %llu glibc_expf_differs %llu\n",
         (unsigned long long)n, (unsigned long long)total, (unsigned long long)mm,
         (unsigned long long)hard, (unsigned long long)gd);
  for (int i = 0; i < idx; i++) {
    for (uint64_t k = 0; k < jobs[i].mismatch && k < 16; k++)
      printf("MISMATCH 0x%08x %a\n", jobs[i].mism[k], (double)u2f(jobs[i].mism[k]));
    for (uint64_t k = 0; k < jobs[i].hard && k < 64; k++)
      printf("HARD 0x%08x %a\n", jobs[i].hardv[k], (double)u2f(jobs[i].hardv[k]));
  }
  return mm ? 1 : 0;
}
