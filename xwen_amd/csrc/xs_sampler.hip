// xs_sampler.hip -- MI355X (gfx950) token sampler: one fused launch per batch.
//
// The reference (0rvar/xwen src/sampler.rs) reads each logit row back to the
// host and runs softmax -> streaming top-k -> top-p -> WeightedIndex on the CPU.
// Here one kernel does the whole draw on the device:
//
//   chunk pass   every workgroup streams one chunk of one row from HBM exactly
//                once (16-byte loads, one slot = 256 lanes x float4), applies
//                the allow-mask and the sparse controls, and each wave reduces
//                its share into a sub-record: max, NaN/finite flags, the
//                softmax partial sum, the held_row f64 partial sum, and a
//                candidate list that provably holds every element of the row's
//                K' best (logit desc, id asc) that lies in the chunk.  The
//                candidate bound is the K'-th largest maximum of the chunk's 64
//                four-lane groups, or of its 256 lanes for K' > 32 (distinct
//                elements, so at least K' elements of the chunk lie at or
//                above it); the sub-record also keeps the chunk's top 16 of
//                those maxima, for the row's survivor bound, and the filter's
//                floor.
//   finalize     the last workgroup of a row (atomic arrival ticket) merges the
//                sub-records: it keeps the entries at or above the K'-th
//                largest published maximum, recomputes the exact f32
//                probability of the K' = top_k + 1 survivors with a correctly
//                rounded exp, orders them by (p desc, id asc) -- the
//                reference's top_k_desc order -- proves the k-th boundary is
//                not a probability tie reaching past the survivors (or finds
//                the lowest tied ids of the row when it is: from the entries
//                wherever a filter floor lies below the tied band, else from
//                the logits), then runs the reference's serial f32 top-p cut
//                and WeightedIndex draw.
//   verify       for a speculative block, the last row finalizer of a
//                sequence runs accept_drafts over the sequence's rows.
//   controls     a call with sparse controls first runs control_kernel (one
//                workgroup per row), which turns the row's bans and biases into
//                a sorted list of final values, and keeps the pulled and the
//                forced values, for the chunk pass to apply.
//
// Exactness: every value that decides a token is computed with the reference's
// own f32 operations in the reference's order (scale by (float)(1/T), subtract
// the max, exp, divide by the denominator, serial sums).  The one quantity not
// reproduced bit-for-bit is the 248k-term softmax denominator, whose summation
// order the reference itself leaves to candle; it is summed here with f32
// per-lane partials combined in f64, written out (soft_sum), and everything
// downstream of it is exact given it.
//
// Compiled with -ffp-contract=off (no fused multiply-adds beyond the explicit
// __builtin_fma calls) and IEEE f32 denormals.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <cmath>
#include <mutex>
#include <cstring>
#include <vector>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/xsamp.h"
#include "xs_exp_table.h"
#include "xs_host.h"

#define XS_DEV __device__ __forceinline__

typedef float v4f __attribute__((ext_vector_type(4)));

namespace xs {

constexpr int BLOCK = 256;          // lanes per workgroup
constexpr int NWAVE = BLOCK / 64;   // wave64
constexpr int SLOT = BLOCK * 4;     // elements per slot: one float4 per lane
constexpr int SPC = 16;             // slots per chunk (16,384 logits, 64 KiB)
constexpr int KSEL = 128;           // largest selection size K'
constexpr int SURV = 256;           // survivor entries the finalizer sorts
constexpr float LOG2E = 1.44269504088896340736f;

__constant__ double kExpT[32][2] = XS_EXP_TABLE_INIT;

// ---------------------------------------------------------------------------
// Correctly rounded binary32 exp (the oracle's xo_exp, same operations in the
// same order, so both produce the same bits).  exp(x) = 2^e * 2^(j/32) * exp(r)
// with k = rint(32x/ln2), j = k mod 32; ln2/32 split Cody-Waite style (40-bit
// head, k*head exact); exp(r) by its Taylor series to r^7; 2^(j/32) as a
// double-double; the product carried as a double-double and rounded once to
// binary32, consulting the tail only on an exact binary32 midpoint.

XS_DEV double widen(float f) { return __builtin_isinf(f) ? __builtin_copysign(0x1p128, (double)f) : (double)f; }

XS_DEV float neighbour(float f, double t) {
  const uint32_t u = __float_as_uint(f);
  if (f == 0.0f) return t > 0.0 ? __uint_as_float(1u) : __uint_as_float(0x80000001u);
  const bool up = (t > (double)f) != (f < 0.0f);
  return __uint_as_float(up ? u + 1u : u - 1u);
}

template <typename TAB>
XS_DEV float cr_expf(float xf, TAB T) {
  if (xf != xf) return xf + xf;
  if (xf < -104.0f) return 0.0f;
  if (xf > 89.0f) return __builtin_huge_valf();
  const double x = (double)xf;
  const double kd = __builtin_rint(x * XS_EXP_INV_L);
  const int k = (int)kd;
  const double r1 = __builtin_fma(-kd, XS_EXP_L_HI, x);
  const double corr = -kd * XS_EXP_L_LO;
  const double r = r1 + corr;
  double h = 1.0 / 5040.0;
  h = __builtin_fma(h, r, 1.0 / 720.0);
  h = __builtin_fma(h, r, 1.0 / 120.0);
  h = __builtin_fma(h, r, 1.0 / 24.0);
  h = __builtin_fma(h, r, 1.0 / 6.0);
  h = __builtin_fma(h, r, 0.5);
  const double q2 = (r * r) * h;
  const double w = corr + q2;
  const double uh = r1 + w;
  const double bb = uh - r1;
  const double ul = (r1 - (uh - bb)) + (w - bb);
  const int j = k & 31;
  const int e = (k - j) / 32;
  const double th = T[2 * j], tl = T[2 * j + 1];
  const double p1 = th * uh;
  const double e1 = __builtin_fma(th, uh, -p1);
  const double s = th + p1;
  double err = (th - s) + p1;
  err = err + (e1 + (th * ul + tl * (1.0 + uh)));
  const double s2 = s + err;
  double err2 = (s - s2) + err;
  const double scale = __longlong_as_double((long long)((uint64_t)(e + 1023) << 52));
  const double v = s2 * scale;
  err2 = err2 * scale;
  const float f = (float)v;
  if (widen(f) == v) return f;
  const float g = neighbour(f, v);
  const double mid = 0.5 * (widen(f) + widen(g));
  if (v == mid && err2 != 0.0) {
    const float lo = f < g ? f : g, hi = f < g ? g : f;
    return err2 > 0.0 ? hi : lo;
  }
  return f;
}

// ---------------------------------------------------------------------------
// Keys.  fkey maps a non-NaN float to a u32 whose unsigned order is the float
// order (-0 canonicalised to +0).  A candidate packs (fkey, id) so that a larger
// u64 is the better candidate: higher logit, then lower id.

XS_DEV uint32_t fkey(float f) {
  const uint32_t b = __float_as_uint(f + 0.0f);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
XS_DEV float keyf(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
XS_DEV uint64_t pack(uint32_t key, uint32_t id) { return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - id); }
XS_DEV uint32_t pk_key(uint64_t p) { return (uint32_t)(p >> 32); }
XS_DEV uint32_t pk_id(uint64_t p) { return 0xFFFFFFFFu - (uint32_t)p; }

// ---------------------------------------------------------------------------
// Wave / block primitives (wave64, 4 waves per block).

XS_DEV int lane_id() { return threadIdx.x & 63; }
XS_DEV int wave_id() { return threadIdx.x >> 6; }

// Lane exchange with lane ^ d (d a power of two below 64, constant after
// unrolling).  d = 1, 2: DPP quad permutes; d = 4: two DPP row rotates and a
// select; d = 8: DPP row rotate; d = 16: ds_swizzle (bitmask mode); d = 32:
// v_permlane32_swap.  All are register-to-register exchanges with no LDS
// traffic, much shorter latency than ds_bpermute.
XS_DEV int xor_lane(int v, int d) {
  if (d == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  if (d == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  if (d == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x12C, 0xF, 0xF, false);   // row_ror:12 -> lane+4
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);   // row_ror:4  -> lane-4
    return (threadIdx.x & 4) ? dn : up;
  }
  if (d == 8) return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  if (d == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);                     // lane ^ 16
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);          // lane ^ 32
  return (threadIdx.x & 32) ? (int)r[0] : (int)r[1];
}
XS_DEV uint32_t xor_u32(uint32_t v, int d) { return (uint32_t)xor_lane((int)v, d); }
XS_DEV float xor_f32(float v, int d) { return __int_as_float(xor_lane(__float_as_int(v), d)); }
XS_DEV double xor_f64(double v, int d) {
  const long long b = __double_as_longlong(v);
  const uint32_t lo = (uint32_t)xor_lane((int)(uint32_t)b, d);
  const uint32_t hi = (uint32_t)xor_lane((int)(uint32_t)((unsigned long long)b >> 32), d);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

XS_DEV float wave_maxf(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, xor_f32(v, o));
  return v;
}
XS_DEV double wave_sumd(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += xor_f64(v, o);
  return v;
}
// (written out: the unroller leaves a loop over these exchanges rolled, and a
// rolled one selects its DPP pattern by comparisons at run time)
XS_DEV uint32_t wave_sum_u32(uint32_t v) {
  v += xor_u32(v, 32);
  v += xor_u32(v, 16);
  v += xor_u32(v, 8);
  v += xor_u32(v, 4);
  v += xor_u32(v, 2);
  v += xor_u32(v, 1);
  return v;
}
XS_DEV uint32_t wave_or(uint32_t v) {
  v |= xor_u32(v, 32);
  v |= xor_u32(v, 16);
  v |= xor_u32(v, 8);
  v |= xor_u32(v, 4);
  v |= xor_u32(v, 2);
  v |= xor_u32(v, 1);
  return v;
}

// Lane exchange for throughput-bound code (many waves per SIMD): ds_bpermute
// runs in the LDS pipe and leaves the VALU to the streaming arithmetic.
// Latency-bound single-wave code uses the DPP forms instead.
template <bool DPP>
XS_DEV uint32_t xshfl(uint32_t v, int d) {
  return DPP ? (uint32_t)xor_lane((int)v, d) : (uint32_t)__shfl_xor((int)v, d);
}

// Bitonic sort, descending, of 64*R u32 keys held R per lane (element r*64+lane).
template <int R, bool DPP = true>
XS_DEV void wave_sort_desc(uint32_t (&x)[R]) {
  const int lane = lane_id();
  constexpr int N = 64 * R;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int d = size >> 1; d > 0; d >>= 1) {
      if (d >= 64) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const int p = r ^ (d >> 6);
          if (p > r) {
            const bool desc = ((r * 64 + lane) & size) == 0;
            const uint32_t a = x[r], b = x[p];
            const uint32_t hi = max(a, b), lo = min(a, b);
            x[r] = desc ? hi : lo;
            x[p] = desc ? lo : hi;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t b = xshfl<DPP>(x[r], d);
          const bool desc = ((r * 64 + lane) & size) == 0;
          const bool lower = (lane & d) == 0;
          const uint32_t hi = max(x[r], b), lo = min(x[r], b);
          x[r] = (lower == desc) ? hi : lo;
        }
      }
    }
  }
}

XS_DEV int wave_incl_scan(int v);

// Exclusive prefix sum over the block in thread order; *total gets the sum.
// Contains barriers: call from block-uniform control flow only.
XS_DEV int block_excl_scan(int v, int* s4, int* total) {
  const int lane = lane_id(), wave = wave_id();
  const int inc = wave_incl_scan(v);
  if (lane == 63) s4[wave] = inc;
  __syncthreads();
  int pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; w++) {
    const int t = s4[w];
    pre += (w < wave) ? t : 0;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return pre + inc - v;
}

// ---------------------------------------------------------------------------
// Per-row configuration: Sampler::new (sampler.rs:133-145) plus the selection
// size.  Greedy when temperature <= 0 or top_k <= 1; otherwise the candidate
// set is the top min(top_k, enc) by (p desc, id asc) and the selection keeps
// one entry past it (K' = k + 1) to prove the boundary, or the whole row when
// top_k >= enc (candidate_set's sort-everything branch, sampler.rs:323-332).

// A whole-row row as its finalizer leaves it for the whole-row kernels.
struct BigRow {
  int32_t state;  // 1: the whole-row kernels draw the row in this call; 0: not
  float m_s, S;   // scaled max and softmax denominator
  int32_t kk;     // candidates: min(top_k, enc)
  float sum;      // the candidate weights' serial sum (big_sum_kernel; top_p < 1)
};

struct Cfg {
  float inv;     // (float)(1/T)  (softmax_in_place, sampler.rs:291)
  float top_p;
  int k;         // candidates drawn from (0 on greedy rows)
  int kp;        // selection size K' the streaming pass keeps per chunk
  bool greedy, scale, full, bad;
  bool big;      // more candidates than the streaming selection holds: the
                 // whole-row kernels draw the row
  bool force;    // a controlled row's check always sends it to the serial fallback (test hook)
  float dthr;    // 2^-148 / S times every denominator the serial sum of enc terms can take
};

XS_DEV Cfg make_cfg(const xs_row_params& p, int64_t enc, int n_top, int k_max, int force = 0) {
  Cfg c;
  c.force = force != 0;
  c.dthr = (1.01f + (float)enc * 0x1p-24f * 1.02f) * 0x1p-148f;
  c.greedy = (p.temperature <= 0.0) || (p.top_k <= 1);
  c.scale = p.temperature != 1.0;
  c.inv = (float)(1.0 / p.temperature);
  c.top_p = p.top_p;
  if (c.greedy) {
    c.k = 0;
    c.kp = 1;
    c.full = false;
  } else if ((int64_t)p.top_k >= enc) {
    c.k = (int)enc;
    c.kp = (int)min(enc, (int64_t)(KSEL + 1));
    c.full = true;
  } else {
    c.k = p.top_k;
    c.kp = p.top_k + 1;
    c.full = false;
  }
  // K' past KSEL (top_k >= 128, or a whole row wider than KSEL): the streaming
  // pass keeps only what the argmax and held_row need, and the whole-row kernels sort
  // the whole row
  c.big = !c.greedy && (c.kp > KSEL || (c.full && enc > KSEL));
  if (c.big) c.kp = 1;
  if (n_top > 0) c.kp = max(c.kp, (int)min((int64_t)n_top, enc));
  c.bad = !c.greedy && c.k > k_max;
  return c;
}

// Every row greedy at T 1 (argmax_probs, and the held_row launch of a call
// that also masks or controls its rows): the streaming selection keeps the
// argmax and, when asked, the n_top highest logits.
XS_DEV Cfg greedy_cfg(int n_top, int64_t enc) {
  Cfg c;
  c.inv = 1.0f;
  c.top_p = 1.0f;
  c.k = 0;
  c.kp = n_top > 0 ? (int)min((int64_t)n_top, enc) : 1;
  c.greedy = true;
  c.scale = c.full = c.bad = c.big = c.force = false;
  c.dthr = 0.0f;
  return c;
}

// ---------------------------------------------------------------------------
// Workspace and launch arguments.
//
// sample_kernel writes one sub-record per wave into the workspace with
// agent-scope stores; the row's last workgroup (arrival ticket) reads them
// back with agent-scope loads and finalizes the row in the same launch.

// What control_kernel leaves for the other kernels about one row's sparse
// controls (the bans and biases themselves become the row's patch list).
struct CtlRow {
  int32_t active;     // the row has a ban, bias, pull or force
  int32_t status;     // XS_ROW_OK, XS_ROW_FORCE_OOR or XS_ROW_BAD_PARAM
  int32_t n_patch;    // entries of the row's patch list
  int32_t pull_id;    // the pulled id with its new value, or -1
  float pull_val;
  int32_t force_id;   // the forced id with its final value, or -1
  float force_val;
  int32_t pad;
};
constexpr int CTL_MAX = XS_CTL_MAX;
constexpr int TSTRIDE = 32;  // one arrival ticket per 128-byte line: tickets of different rows never share one
constexpr int TS_N = 1;  // whole-row path, big_ticket line: the row's sorted entries (KCUT below)

struct Args {
  const float* logits;
  int64_t ld, enc;
  const xs_row_params* params;
  const float* uniforms;
  const uint32_t* allowed;
  int64_t allowed_ld;
  int32_t* token;
  int32_t* status;
  int32_t* cand_id;
  float* cand_w;
  int32_t* n_cand;
  int64_t cand_ld;
  float* soft_max;
  float* soft_sum;
  float* row_max;
  double* row_lse;
  int32_t n_top;
  int32_t* top_id;
  float* top_logprob;
  double* top_logprob64;
  int64_t top_ld;
  // scoring reads (score_kernel), normalized by row_lse (the context's
  // lse workspace when the caller takes no row_lse)
  const int32_t* score_ids;
  int32_t n_score;
  int64_t score_ld;
  double* score_logprob;
  const uint32_t* class_masks;
  int32_t n_class;
  int64_t class_ld;
  double* class_mass;
  double* probs;
  int64_t probs_ld;
  uint64_t* score_part;  // [rows, n_chunks, XS_CLASS_MAX] the chunks' class sums (f64 bits)
  // verify walk (span == 0: plain batch)
  int32_t span;
  const int32_t* drafts;
  const int32_t* budget;
  const uint8_t* done_after;  // [seqs * span] or null: committing this draft completes the grammar
  int32_t n_eog;
  const int32_t* eog;  // [n_eog] device ids
  int32_t* accepted;
  int32_t* committed;
  int32_t* n_committed;
  int32_t* seq_status;
  // argmax_probs: every row greedy (params and uniforms unused), p_max[row] =
  // 1 / sum exp(v - max) over the raw row
  int32_t greedy_all;
  float* p_max;
  // sparse controls (controls == nullptr: none) and what control_kernel makes
  // of them: per row a patch list of (id << 32 | final value bits) sorted by id,
  // CTL_MAX entries apart, and the first patch of every chunk (n_chunks + 1
  // offsets per row)
  const xs_row_control* controls;
  const uint32_t* ctl_ids;
  const float* ctl_delta;
  uint64_t* patch;      // [rows, ctl_cap]
  uint64_t* ctl_keys;   // [rows, 2, ctl_cap]: control_kernel's sort buffers for lists past CTL_MAX, or null
  int32_t ctl_cap;      // the context's largest control list (bans plus biases of one row)
  CtlRow* ctl_row;
  int32_t* ctl_chunk;
  // geometry + workspace
  int32_t* row_ticket;  // [rows * TSTRIDE] workgroups of the row that have published (0 between calls)
  int32_t* seq_ticket;  // [seqs * TSTRIDE] rows of the sequence that are finalized (0 between calls)
  int32_t n_chunks, nslots;
  int32_t k_max;     // the context's largest top_k (of min(top_k, enc)); larger is XS_ROW_BAD_PARAM
  uint64_t* big;     // [rows, 2, big_ld]: the whole-row sort's buffers (contexts with k_max > XS_K_MAX)
  int64_t big_ld;
  struct BigRow* big_state;  // [rows]: what the finalizer leaves for the whole-row kernels
  uint32_t* big_hist;        // [rows, big_hld]: per-tile digit counts (then first positions) of a sort pass
  int64_t big_hld;
  int32_t* big_ticket;       // [rows * TSTRIDE]: the sort passes' arrival tickets, zero between kernels
  int32_t big_tiles;         // tiles of BTILE ids per row
  int32_t big_nblk;          // chain blocks per row past the first CHEAD terms
  int32_t big_cut;           // tokens only, enc <= 2^20: rows at top_k >= enc sort only p >= 2^-26
  // the serial denominator (serial_kernel), on calls with a mask or controls:
  // bit 0, the call observes it (candidates or soft_sum), and serial_kernel
  // finalizes its controlled rows at top_p >= 1; bit 1, the call may hold
  // rows of top_k >= 128, and serial_kernel finalizes its controlled ones
  int32_t serial;
  // the finalizer's fallback to the serial sum (ser_local) for the other
  // controlled rows: rows sent there are counted (null: not counted), and
  // ser_force sends every checked row there (a test hook)
  uint32_t* ser_count;
  int32_t ser_force;
  // split launch: sample_kernel's workgroups publish and exit; finalize_kernel
  // (one workgroup per row) finalizes every row afterwards
  int32_t split;
  // sample_kernel's grid: rows in groups of 2^xcd_log2 (the device's XCD
  // count, or 1), nrows of them; xcd_test 2 makes the rows of several chunks
  // fail their placement check (a test hook)
  int32_t xcd_log2, nrows, xcd_test;
  // held_fold's re-reads are shared by the finalizing workgroup's four waves
  // (1) or left to its first wave (0): shared when the launch's workgroups
  // fit on the device at once, so that the waves that wait for the first
  // wave's finalization hold no slot another workgroup needs
  int32_t fold_shared;
  uint64_t* ser_sum;  // [rows, ser_ld, 2]: segment summaries
  uint64_t* ser_e;    // [rows, SER_NB, SEG / 2]: kept segments' terms, two f32 per word
  int64_t ser_ld;     // segments per row of ser_sum
  uint64_t* rec;     // [rows, SRECW, nsp]: word i of sub-record s of a row at i * nsp + s
};

// The row the r-th group of n_chunks workgroups takes, for launches given a
// row order; other launches pass the empty struct, so their kernel arguments
// stay small (a 2 KiB table in every launch's arguments cost 0.2-0.5 us).
template <bool ORD> struct RowOrder { uint16_t v[XS_ORDER_MAX]; };
template <> struct RowOrder<false> {};



// Agent-scope (sc1) stores and loads: coherent across the XCDs' L2 caches
// without the whole-L2 writeback / invalidate a __threadfence() costs.  A
// workgroup hands its sub-records to the row's finalizing wave through them:
// it waits for its stores to be acknowledged (drain) before it takes the
// row's arrival ticket, and the wave that takes the last ticket reads the
// sub-records back with agent-scope loads.
XS_DEV void st_agent(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
XS_DEV void st_agent(int32_t* p, int32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
XS_DEV uint64_t ld_agent(const uint64_t* p) { return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
XS_DEV int32_t ld_agent(const int32_t* p) { return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Sub-record stores and loads: sc0, which misses the CU's L1 and is served by
// the XCD's L2.  sample_kernel places all workgroups of a row on one XCD (the
// grid mapping in sample_kernel), so a row's sub-records go from its chunk
// workgroups to its finalizer through that L2 alone, without the write-through
// to memory and the memory round trips of sc1.  The row's arrival ticket
// proves the placement (row_ticket_add); a row whose workgroups did not share
// the finalizer's XCD is failed, never read.  Kernels launched later read the
// sub-records after the launch boundary has written the L2 back.
//
// A launch of fewer than 8 rows per XCD spreads each row over the XCDs
// instead (a lone row streamed through one XCD gets that XCD's share of the
// bandwidth: C1 greedy took 9.3 us instead of 8.8) and instantiates the
// kernel with LOC false: the hand-off then takes agent-scope sc1 stores and
// loads, performed beyond the L2s.
template <bool LOC>
XS_DEV void st_sub(uint64_t* p, uint64_t v) {
  if constexpr (LOC) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool LOC>
XS_DEV uint64_t ld_sub(const uint64_t* p) {
  if constexpr (LOC) return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The XCD (XCC_ID hardware register, bits 3:0) the calling wave runs on.
XS_DEV uint32_t xcc_id() { return (uint32_t)__builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15u; }

// Wait until every memory operation this wave issued has completed.
XS_DEV void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Order this wave's LDS writes before its later LDS reads by other lanes.
XS_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
}

// Sorts n <= 256 distinct u64 keys from src into dst, descending: a key's
// position is the number of keys above it, counted by every lane over all n
// keys (LDS broadcast reads).  One wave; both arrays in LDS.
XS_DEV void rank_sort_lds(const uint64_t* src, uint64_t* dst, int n) {
  const int lane = threadIdx.x & 63;
  uint64_t x[4];
  int rk[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    x[r] = (r * 64 + lane < n) ? src[r * 64 + lane] : 0ull;
    rk[r] = 0;
  }
#pragma unroll 8
  for (int j = 0; j < n; j++) {
    const uint64_t y = src[j];
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (r * 64 < n) rk[r] += (y > x[r]) ? 1 : 0;
  }
#pragma unroll
  for (int r = 0; r < 4; r++)
    if (r * 64 + lane < n) dst[rk[r]] = x[r];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);
}

XS_DEV uint32_t rdl(uint32_t x, int i) { return (uint32_t)__builtin_amdgcn_readlane((int)x, i); }
// The k-th largest of 64*R u32 keys held R per lane, by a bitwise search:
// the largest value with at least k keys at or above it (ballot counts; no
// sort).  k >= 1.
template <int R>
XS_DEV uint32_t kth_largest(const uint32_t (&x)[R], int k) {
  uint32_t t = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; bit--) {
    const uint32_t c = t | (1u << bit);
    int n = 0;
#pragma unroll
    for (int r = 0; r < R; r++) n += (int)__popcll(__ballot(x[r] >= c));
    if (n >= k) t = c;
  }
  return t;
}
XS_DEV float rdlf(float x, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), i)); }
XS_DEV uint64_t rdl64(uint64_t x, int i) {
  return ((uint64_t)rdl((uint32_t)(x >> 32), i) << 32) | rdl((uint32_t)x, i);
}
XS_DEV uint64_t shfl64(uint64_t x, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)x, src);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(x >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}
XS_DEV uint64_t shfl_xor64(uint64_t x, int m) {
  const uint32_t lo = xor_u32((uint32_t)x, m);
  const uint32_t hi = xor_u32((uint32_t)(x >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}
// Lanes below this one whose bit is set in `mask`.
XS_DEV int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
// Inclusive prefix sum over the wave: DPP row shifts within each row of 16,
// then the row totals carried across rows with row broadcasts.
XS_DEV int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false); // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false); // row_bcast:31 -> rows 2, 3
  return v;
}
XS_DEV int wave_sumi(int v) {
  v += xor_lane(v, 32);
  v += xor_lane(v, 16);
  v += xor_lane(v, 8);
  v += xor_lane(v, 4);
  v += xor_lane(v, 2);
  v += xor_lane(v, 1);
  return v;
}

// Bitonic sort, descending, of 64*R u64 keys held R per lane (element r*64+lane).
template <int R>
XS_DEV void wave_sort_desc64(uint64_t (&x)[R]) {
  const int lane = lane_id();
  constexpr int N = 64 * R;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int d = size >> 1; d > 0; d >>= 1) {
      if (d >= 64) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const int p = r ^ (d >> 6);
          if (p > r) {
            const bool desc = ((r * 64 + lane) & size) == 0;
            const uint64_t a = x[r], b = x[p];
            const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
            x[r] = desc ? hi : lo;
            x[p] = desc ? lo : hi;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint64_t b = shfl_xor64(x[r], d);
          const bool desc = ((r * 64 + lane) & size) == 0;
          const bool lower = (lane & d) == 0;
          const uint64_t hi = x[r] > b ? x[r] : b, lo = x[r] > b ? b : x[r];
          x[r] = (lower == desc) ? hi : lo;
        }
      }
    }
  }
}

// Element `i` of a list held R per lane (i uniform).
template <int R>
XS_DEV uint64_t pick64(const uint64_t (&x)[R], int i) {
  uint64_t out = 0;
#pragma unroll
  for (int r = 0; r < R; r++)
    if ((i >> 6) == r) out = rdl64(x[r], i & 63);
  return out;
}

// Sub-record of one wave of one chunk in the workspace, SRECW u64 words:
//   w0  P (f64 bits): sum over the wave's elements of e^(s - c_s), s the
//       scaled, controlled logit (the softmax partial)
//   w1  c_s (f32 bits) | c_r (f32 bits) << 32: the partials' offsets
//   w2  R (f64 bits): sum of e^(v - c_r) over the raw logits (held_row)
//   w3  wave max (f32 bits) | flags << 32 (1 NaN seen, 2 a finite value
//       seen, 4 entries in descending order, 8 w8/w9 hold fold data)
//   w4  entry count
//   w5  bound keys 0 | 1 << 32;  w6  bound keys 2 | 3 << 32
//   w7  the filter's floor (f32 bits): the entries are every element of the
//       wave at or above it; +inf when they are not (an overflow)
//   w8  held_row fold data (flag 8; see held_fold): in a chunk whose own max
//       m_c dominates it, the f64 sum of this wave's terms exp(f64(v - m_c))
//       before the chunk's first maximal id
//   w9  and the sum (f64) of rint(2^52 * term) over its terms after that id
//   w10.. entries: pack(key, id) of the wave's candidates
// A row has n_chunks * NWAVE sub-records, chunk-major, stored transposed:
// word i of sub-record s sits at i * nsp + s of the row's block (nsp = the
// sub-record count rounded up to 64), so the finalizer's lanes read one word
// of 64 sub-records with one coalesced load.
constexpr int SHDR = 10;
constexpr int CAPW = 256;           // entries per sub-record
constexpr int SRECW = SHDR + CAPW;
constexpr int NHW = 7;              // header words the finalizer reads
constexpr int EPRE = 16;            // entries per sub-record read with the headers
constexpr int GMAX = 4;             // sub-record groups of 64 a finalizer handles
constexpr int KGRP = 32;            // largest K' whose chunk bound comes from group maxima
constexpr uint32_t KEY_NEG_INF = 0x007FFFFFu;  // fkey(-inf)

// The k-th largest of the 64R keys x, as kth_largest returns it, where the
// keys above KEY_NEG_INF (finite values) number at most 128: those are
// compacted into scr (this wave's, 128 words of LDS) and sorted, which takes
// a fraction of the 32 ballot rounds of the bitwise search.  When fewer than
// k keys are finite the result is 0: at or below KEY_NEG_INF, a bound that
// admits every finite value, as any such result does for the callers.
// More than 128 finite keys take kth_largest (so does any k above 128 that
// has k of them).
template <int R>
XS_DEV uint32_t kth_largest_few(const uint32_t (&x)[R], int k, uint32_t* scr) {
  uint64_t b[R];
  int n = 0;
#pragma unroll
  for (int r = 0; r < R; r++) {
    b[r] = __ballot(x[r] > KEY_NEG_INF);
    n += (int)__popcll(b[r]);
  }
  if (n < k) return 0u;
  if (n > 128) return kth_largest<R>(x, k);
  int base = 0;
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (x[r] > KEY_NEG_INF) scr[base + lanes_below(b[r])] = x[r];
    base += (int)__popcll(b[r]);
  }
  wave_lds_sync();
  const int lane = lane_id();
  uint32_t v[2] = {lane < n ? scr[lane] : 0u, lane + 64 < n ? scr[lane + 64] : 0u};
  wave_sort_desc<2, true>(v);
  return k <= 64 ? rdl(v[0], k - 1) : rdl(v[1], k - 65);
}

struct ChunkLds {
  uint32_t groupmax[BLOCK / 4];     // maxima of 4-lane groups
  uint32_t lanemax[BLOCK];          // lane maxima
  int32_t last;                     // this workgroup took the row's last ticket
  // held_row launches: each wave's max, f64 partial (offset: that max) and
  // first maximal id, for the chunk's own fold data
  float wmax[NWAVE];
  uint32_t wtop[NWAVE];
  uint32_t wprev[NWAVE];            // the row's running max key before each wave's update
  double wr[NWAVE];
};
// What the finalizing wave leaves for held_row's fold (held_fold), which the
// whole workgroup runs after it: the row statistics and the top-n logits.
struct HeldLds {
  double R_d;                       // exactly summed denominator
  double pre[4];                    // per wave: terms before the argmax
  long long post[4];                // per wave: 2^-52 units of the terms after it
  float m_v;                        // row max
  uint32_t top;                     // first maximal id
  int32_t ok;                       // statistics defined (no NaN, finite max)
  int32_t can_fold;                 // the argmax is known (not a row refused for its top_k)
  int32_t n_have;                   // top-n entries below
  float vals[XS_TOP_MAX];           // top-n logits, (logit desc, id asc)
};
// What the finalizing wave leaves for the whole-row kernels.
struct BigStash {
  float m_s, S;                     // scaled max and softmax denominator of the row
  int32_t defer;                    // the row is drawn by the whole-row kernels
  int32_t pad;
};
struct FinLds {
  uint64_t list[SURV];              // gathered survivors
  uint64_t srt[SURV];               // survivors in (logit desc, id asc) order
  uint64_t psel[KSEL];              // the candidate set in draw order: (p bits << 32) | ~id
  double expt[64];                  // kExpT, flattened
  uint32_t keys[GMAX * 64 * 4];     // published bound keys (more than 64 sub-records)
  uint32_t zmap[KSEL / 32];         // a whole short row: the ids with p > 0
  HeldLds held;
  BigStash big;
  int32_t need_ser;                 // the exact denominator did not settle this controlled row's token
  float ser_ms;                     // and its scaled max, for the serial sum
};
// The serial denominator's segments (serial_kernel, ser_local): SEG ids each,
// one wave's float4s of one slot.
constexpr int SEG = 256;               // ids per segment
constexpr int SER_QCAP = 128;          // per wave: terms queued for the correctly rounded exp
// What one workgroup needs to sum one row's serial denominator by itself
// (ser_local): one chunk's segment sums, prefixes, grid units and flags, the
// queue of terms for the correctly rounded exp, the chunk's summaries for the
// walk, a segment of recounted terms, and the running sums.
struct SerLocal {
  double expt[64];
  double segsum[SPC * NWAVE];
  double segpre[SPC * NWAVE];
  uint32_t R[SPC * NWAVE][2];
  uint32_t meta[SPC * NWAVE];
  float qd[NWAVE][SER_QCAP];
  uint8_t qt[NWAVE][SER_QCAP];
  uint64_t sum[SPC * NWAVE][2];
  float scr[SEG];
  double X;                         // exact sum of the chunks walked so far
  uint32_t sb;                      // the serial sum's bits after them
};
// The chunk pass stages each wave's entries here before it publishes them;
// after the hand-off only the row's last workgroup uses the memory again, as
// its finalizer's (and, for a row the finalizer sends back, its serial sum's).
union TailLds {
  uint64_t stage[NWAVE][CAPW];
  FinLds fin;
  SerLocal ser;
};
// p = rn(e / S) of one controlled logit v (the reference's softmax_in_place:
// v *= inv unless T == 1, then exp(v - max), then / sum; sampler.rs:289-310).
// T: the 2^(j/32) table (kExpT flattened), here the finalizer's LDS copy.
template <typename TAB>
XS_DEV float exact_p(float v, const Cfg& cfg, float m_s, float S, TAB T) {
  const float s = cfg.scale ? v * cfg.inv : v;
  const float e = cr_expf(s - m_s, T);
  return __fdiv_rn(e, S);
}
// The softmax numerator e = exp(v * inv - max) of the same logit (p = e / S).
template <typename TAB>
XS_DEV float exact_e(float v, const Cfg& cfg, float m_s, TAB T) {
  const float s = cfg.scale ? v * cfg.inv : v;
  return cr_expf(s - m_s, T);
}

// The largest float below f (f > -inf, not NaN).
XS_DEV float next_below(float f) {
  if (f == 0.0f) return -__uint_as_float(1u);
  const uint32_t b = __float_as_uint(f);
  return __uint_as_float(f > 0.0f ? b - 1u : b + 1u);
}

XS_DEV float xexp2(float x) { return __builtin_amdgcn_exp2f(x); }
// max without the sNaN-quieting canonicalisation fmaxf brings: a NaN operand
// may or may not survive, which is fine wherever a NaN already fails the row
XS_DEV float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
XS_DEV float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
XS_DEV float q4(const v4f& q, int e) { return e == 0 ? q.x : e == 1 ? q.y : e == 2 ? q.z : q.w; }

// ---------------------------------------------------------------------------
// Rare path of the chunk pass: more than CAPW of this wave's elements lie at
// or above the chunk bound (ties at the bound, or a bound far below the
// wave's values).  Writes the wave's exact K' best (logit desc, id asc)
// elements: every key above a threshold key, then the lowest ids equal to it.
// The threshold is the bound when fewer than K' keys lie strictly above it,
// else the wave's K'-th largest key (bisection).  Elements that are -inf or
// NaN never become candidates.  Re-reads the wave's elements from memory (the
// streaming pass's registers are free by then) and masks and controls them as
// that pass did, so a controlled row's bans and biases count here as they do
// in the filter.  Returns the count.
// The chunk's sparse controls as the streaming pass applies them.
struct ChunkCtl {
  const uint64_t* pl;  // the row's patch list, (id << 32) | final value bits, by id
  int p0, p1;          // this chunk's patches
  int pull, force;     // ids, or -1
  float pull_val, force_val;
};

template <bool HAS_MASK, bool HAS_CTL, bool LOC>
XS_DEV int wave_overflow(const float* rowp, const uint32_t* mrow, int s0, int ns, int enc,
                         uint64_t* sub, int nsp, int kp, uint32_t tk, const ChunkCtl& cc) {
  constexpr int H = SPC / 2;  // slots per round of loads
  const int tid = threadIdx.x;
  // Slots h*H .. h*H+H-1 of the wave's elements as the streaming pass saw
  // them (masked, controlled, -inf where absent), re-read with one round of
  // loads; pc is the patch cursor, consumed in slot order.
  auto load = [&](int h, v4f (&xv)[H], int& pc) __attribute__((always_inline)) {
    uint32_t mw[H];
#pragma unroll
    for (int u = 0; u < H; u++) {
      const int j = h * H + u;
      const int id0 = (s0 + j) * SLOT + 4 * tid;
      const bool in = j < ns && id0 < enc;
      xv[u] = v4f{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (in) xv[u] = *reinterpret_cast<const v4f*>(rowp + id0);
      mw[u] = (HAS_MASK && in) ? mrow[id0 >> 5] >> (id0 & 31) : 0xFu;
    }
#pragma unroll
    for (int u = 0; u < H; u++) {
      const int j = h * H + u;
      const int id0 = (s0 + j) * SLOT + 4 * tid;
      float x[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (j >= ns || id0 + e >= enc || (HAS_MASK && !((mw[u] >> e) & 1u))) x[e] = -INFINITY;
      if (HAS_CTL && j < ns) {
        const int sb = (s0 + j) * SLOT;
        if (cc.force >= 0) {
#pragma unroll
          for (int e = 0; e < 4; e++) x[e] = (id0 + e == cc.force) ? cc.force_val : -INFINITY;
        } else {
          while (pc < cc.p1) {
            const uint64_t pe = cc.pl[pc];
            const int off = (int)(uint32_t)(pe >> 32) - sb;
            if (off >= SLOT) break;
            if ((off >> 2) == tid) {
              const float pv = __uint_as_float((uint32_t)pe);
#pragma unroll
              for (int e = 0; e < 4; e++) x[e] = ((off & 3) == e) ? pv : x[e];
            }
            pc++;
          }
          const int pt = cc.pull - sb;
          if (pt >= 0 && pt < SLOT && (pt >> 2) == tid) {
#pragma unroll
            for (int e = 0; e < 4; e++) x[e] = ((pt & 3) == e) ? cc.pull_val : x[e];
          }
        }
      }
      xv[u] = v4f{x[0], x[1], x[2], x[3]};
    }
  };
  auto valid = [](float x) __attribute__((always_inline)) { return x == x && x > -INFINITY; };
  auto count = [&](uint32_t key, bool strict) __attribute__((always_inline)) -> int {
    int c = 0, pc = cc.p0;
#pragma unroll 1
    for (int h = 0; h < 2; h++) {
      v4f xv[H];
      load(h, xv, pc);
#pragma unroll
      for (int u = 0; u < H; u++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float x = q4(xv[u], e);
          const uint32_t k = fkey(x);
          c += (valid(x) && (strict ? k > key : k >= key)) ? 1 : 0;
        }
    }
    return wave_sumi(c);
  };
  uint32_t eq = max(tk, fkey(-__FLT_MAX__));
  if (count(eq, true) >= kp) {
    uint32_t ans = 0;
#pragma unroll 1
    for (int bit = 31; bit >= 0; bit--) {
      const uint32_t cand = ans | (1u << bit);
      if (count(cand, false) >= kp) ans = cand;
    }
    eq = ans;
  }
  // everything above eq, in slot order
  int n = 0;
  {
    int pc = cc.p0;
#pragma unroll 1
    for (int h = 0; h < 2; h++) {
      v4f xv[H];
      load(h, xv, pc);
#pragma unroll
      for (int u = 0; u < H; u++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float x = q4(xv[u], e);
          const bool hit = valid(x) && fkey(x) > eq;
          const uint64_t b = __ballot(hit);
          if (b) {
            const int pos = n + lanes_below(b);
            if (hit && pos < CAPW) st_sub<LOC>(&sub[(int64_t)(SHDR + pos) * nsp], pack(fkey(x), (uint32_t)((s0 + h * H + u) * SLOT + 4 * tid + e)));
            n += __popcll(b);
          }
        }
    }
  }
  n = min(n, CAPW);
  // ties at eq, lowest ids first: slot j covers ids (s0 + j) * SLOT in lane order
  int need = kp - n;
  {
    int pc = cc.p0;
#pragma unroll 1
    for (int h = 0; h < 2 && need > 0; h++) {
      v4f xv[H];
      load(h, xv, pc);
#pragma unroll
      for (int u = 0; u < H; u++) {
        if (need > 0) {
          bool t[4];
          int c = 0;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float x = q4(xv[u], e);
            t[e] = valid(x) && fkey(x) == eq;
            c += t[e] ? 1 : 0;
          }
          const int incl = wave_incl_scan(c);
          int pos = incl - c;
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (t[e]) {
              if (pos < need && n + pos < CAPW)
                st_sub<LOC>(&sub[(int64_t)(SHDR + n + pos) * nsp], pack(eq, (uint32_t)((s0 + h * H + u) * SLOT + 4 * tid + e)));
              pos++;
            }
          const int tot = (int)rdl((uint32_t)incl, 63);
          n += min(tot, need);
          need -= tot;
        }
      }
    }
  }
  return min(n, CAPW);
}

// ---------------------------------------------------------------------------
// Wave reductions to a uniform value: an inclusive pass within each row of 16
// lanes (DPP row_shr 1, 2, 4, 8), then the row totals carried with row_bcast
// 15 and 31, so lane 63 holds the result; all VALU, no LDS traffic.
template <int CTRL, int RM>
XS_DEV int dppi(int old, int v) { return __builtin_amdgcn_update_dpp(old, v, CTRL, RM, 0xF, false); }
template <int CTRL, int RM>
XS_DEV float dppf(float old, float v) { return __int_as_float(dppi<CTRL, RM>(__float_as_int(old), __float_as_int(v))); }
template <int CTRL, int RM>
XS_DEV double dppd(double v) {  // identity 0.0 (the f64 sum)
  const long long b = __double_as_longlong(v);
  const int lo = dppi<CTRL, RM>(0, (int)(uint32_t)b);
  const int hi = dppi<CTRL, RM>(0, (int)(uint32_t)((unsigned long long)b >> 32));
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
#define XS_ROWRED(STEP)                                                        \
  STEP(0x111, 0xF) STEP(0x112, 0xF) STEP(0x114, 0xF) STEP(0x118, 0xF)          \
  STEP(0x142, 0xA) STEP(0x143, 0xC)
XS_DEV float red_maxf(float v) {
#define XS_S(C, R) v = fmaxf(v, dppf<C, R>(-INFINITY, v));
  XS_ROWRED(XS_S)
#undef XS_S
  return rdlf(v, 63);
}
XS_DEV int red_maxi(int v) {
#define XS_S(C, R) v = max(v, dppi<C, R>(INT32_MIN, v));
  XS_ROWRED(XS_S)
#undef XS_S
  return (int)rdl((uint32_t)v, 63);
}
XS_DEV uint32_t red_or(uint32_t v) {
#define XS_S(C, R) v |= (uint32_t)dppi<C, R>(0, (int)v);
  XS_ROWRED(XS_S)
#undef XS_S
  return rdl(v, 63);
}
XS_DEV double red_sumd(double v) {
#define XS_S(C, R) v += dppd<C, R>(v);
  XS_ROWRED(XS_S)
#undef XS_S
  const long long b = __double_as_longlong(v);
  const uint32_t lo = rdl((uint32_t)b, 63), hi = rdl((uint32_t)((unsigned long long)b >> 32), 63);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
#undef XS_ROWRED

// ---------------------------------------------------------------------------
// held_row's denominator as the reference folds it (generate.rs:1931-1932):
// the f64 terms exp(f64(v - max)) summed one after another in id order.
//
// Once the max's own term (exactly 1.0) is in, a running sum in [1, 2) rounds
// every later term to its grid of 2^-52: a term below 2^-53 is absorbed, a
// larger one lands on a multiple of 2^-52.  So while the sum stays below 2,
// the fold equals rn(1 + pre) + 2^-52 * sum_i rint(t_i * 2^52) over the terms
// t_i after the argmax, where pre is the sum of the terms before it -- an
// integer sum, in any order.  On rows like that (a dominant token) the exact
// sum of the same terms differs from the fold by up to the whole of
// (denominator - 1), that is up to 100 % of the top log-prob; from 2 up the
// fold's rounding moves lse by less than V * 2^-53 while |log-prob| >= ln 2,
// and the exactly summed R_d stands.
//
// Every sub-record wholly before the argmax adds its f64 partial to pre.  The
// argmax's own chunk, whose waves interleave ids before and after it, adds the
// fold data its streaming pass published (taken at the chunk's max, which is
// the row max there).  A sub-record after it whose max lies within 36.74 of
// the row max may hold terms of 2^-53 or more: they come from its candidate
// entries when its filter floor lies below them all; every other term there
// is absorbed.  Only what none of this covers is read from the logits again.

// Below this f32 difference v - max, exp(f64(v - max)) < 2^-53: a term that a
// running sum in [1, 2) absorbs (ln 2^-53 = -36.7368).
constexpr float LN_HALF_ULP1 = -36.74f;

// exp(x) in f64 for x <= 0 (x >= -700; below, 0), to about 1e-16 relative:
// the correctly rounded exp's reduction and table, without its final rounding.
template <typename TAB>
XS_DEV double exp_f64(double x, TAB T) {
  if (!(x >= -700.0)) return 0.0;
  const double kd = __builtin_rint(x * XS_EXP_INV_L);
  const int k = (int)kd;
  const double r1 = __builtin_fma(-kd, XS_EXP_L_HI, x);
  const double r = r1 - kd * XS_EXP_L_LO;
  double h = 1.0 / 5040.0;
  h = __builtin_fma(h, r, 1.0 / 720.0);
  h = __builtin_fma(h, r, 1.0 / 120.0);
  h = __builtin_fma(h, r, 1.0 / 24.0);
  h = __builtin_fma(h, r, 1.0 / 6.0);
  h = __builtin_fma(h, r, 0.5);
  const double em1 = __builtin_fma(r * r, h, r);  // exp(r) - 1
  const int j = k & 31;
  const int e = (k - j) / 32;
  const double th = T[2 * j], tl = T[2 * j + 1];
  const double v = th + __builtin_fma(th, em1, tl * (1.0 + em1));
  return v * __longlong_as_double((long long)((uint64_t)(e + 1023) << 52));
}

// The workgroup's first nw waves (1, or all four) share the re-reads (one
// sub-record each at a time, all 16 slots' loads in flight); wave 0 adds the
// partials of the sub-records wholly before the argmax.  Then wave 0 writes
// row_lse and the top-n log-probs.  With nw > 1 it contains a barrier: all
// waves of the workgroup call it.
template <bool LOC>
XS_DEV void held_fold(const Args& a, int row, const float* rowp, const uint64_t* rowrec, int nsp,
                      int nsub, FinLds& F, int nw) {
  HeldLds& H = F.held;
  const int lane = lane_id(), wave = wave_id();
  const int enc = (int)a.enc;
  const float m_v = H.m_v;
  const double R_d = H.R_d;
  const uint32_t top = H.top;
  const bool fold = H.ok && H.can_fold && R_d < 2.0;
  const double* T = F.expt;
  double pre = 0.0;
  long long post = 0;
  if (fold) {
    const int jc = (int)(top / (uint32_t)(SPC * SLOT));  // the argmax's chunk
    int nth = 0;  // re-read sub-records met so far, dealt to the waves in turn
    for (int g = 0; g * 64 < nsub; g++) {
      const int s = g * 64 + lane;
      const bool has = s < nsub;
      // (s < nsp: the words lie inside the row's record; loaded unguarded,
      // so that all go out at once, and dropped where !has)
      const uint64_t h1 = ld_sub<LOC>(&rowrec[1 * nsp + s]), h2 = ld_sub<LOC>(&rowrec[2 * nsp + s]);
      const uint64_t h3 = ld_sub<LOC>(&rowrec[3 * nsp + s]), h4 = ld_sub<LOC>(&rowrec[4 * nsp + s]);
      const uint64_t h7 = ld_sub<LOC>(&rowrec[7 * nsp + s]), h8 = ld_sub<LOC>(&rowrec[8 * nsp + s]);
      const uint64_t h9 = ld_sub<LOC>(&rowrec[9 * nsp + s]);
      const int c = s / NWAVE;
      const float mw = __uint_as_float((uint32_t)h3);
      const bool fold_data = ((h3 >> 32) & 8u) != 0;
      // Wholly before the argmax: the wave's f64 partial joins pre (its terms
      // carry ~2e-6 relative error, so pre does, and so does denominator - 1).
      // The argmax's chunk: its own fold data, taken at its max, the row max.
      // After it: absorbed when every term is below 2^-53; else the terms of
      // 2^-53 or more come from the entries when the filter's floor lies below
      // them all (e^-36.75 < 2^-53 with room for the f32 difference).
      const bool after_big = has && c > jc && (mw - m_v) >= LN_HALF_ULP1;
      const float fl = __uint_as_float((uint32_t)h7);
      const bool from_entries = after_big && (fl - m_v) <= -36.75f;
      const bool reread = has && ((c == jc && !fold_data) || (after_big && !from_entries));
      if (wave == 0 && has && c < jc) {
        const double r = __longlong_as_double((long long)h2);
        if (r != 0.0) pre += r * (double)xexp2((__uint_as_float((uint32_t)(h1 >> 32)) - m_v) * LOG2E);
      }
      if (wave == 0 && has && c == jc && fold_data) {
        pre += __longlong_as_double((long long)h8);
        post += (long long)__longlong_as_double((long long)h9);
      }
      if (wave == 0 && from_entries) {
        const int cnt = (int)min((uint32_t)h4, (uint32_t)CAPW);
        for (int j0 = 0; j0 < cnt; j0 += 8) {
          uint64_t e[8];  // (clamped inside the sub-record, not guarded: eight loads in flight)
#pragma unroll
          for (int u = 0; u < 8; u++) e[u] = ld_sub<LOC>(&rowrec[(int64_t)(SHDR + min(j0 + u, CAPW - 1)) * nsp + s]);
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const float x = keyf(pk_key(e[u])) - m_v;
            if (j0 + u < cnt && x >= LN_HALF_ULP1) post += (long long)__builtin_rint(exp_f64((double)x, T) * 0x1p52);
          }
        }
      }
      uint64_t m = __ballot(reread);
      while (m) {  // one sub-record's elements: wave w of chunk cc
        const int sr = g * 64 + (int)__builtin_ctzll(m);
        m &= m - 1ull;
        if ((nth++ % nw) != wave) continue;
        const int cc = sr / NWAVE, w = sr % NWAVE;
        float4 v[SPC];
#pragma unroll
        for (int jj = 0; jj < SPC; jj++) {
          const int id0 = ((cc * SPC + jj) * SLOT) + 4 * (w * 64 + lane);
          v[jj] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
          if (id0 < enc) v[jj] = reinterpret_cast<const float4*>(rowp)[id0 >> 2];
        }
#pragma unroll
        for (int jj = 0; jj < SPC; jj++) {
          const int id0 = ((cc * SPC + jj) * SLOT) + 4 * (w * 64 + lane);
          const float xv[4] = {v[jj].x, v[jj].y, v[jj].z, v[jj].w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int id = id0 + e;
            const float x = xv[e] - m_v;  // f32, as the reference's v - max
            if (id < enc && (uint32_t)id != top) {
              if (x >= LN_HALF_ULP1) {  // a term of 2^-53 or more: exactly
                const double t = exp_f64((double)x, T);
                if ((uint32_t)id < top) pre += t;
                else post += (long long)__builtin_rint(t * 0x1p52);
              } else if ((uint32_t)id < top) {  // below it: only pre holds it, to ~2e-6
                pre += (double)xexp2(x * LOG2E);
              }
            }
          }
        }
      }
    }
    pre = wave_sumd(pre);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const long long lo = (long long)(uint32_t)xor_lane((int)(uint32_t)post, o);
      const long long hi = (long long)xor_lane((int)(post >> 32), o);
      post += (hi << 32) | lo;
    }
  }
  if (lane == 0) {
    H.pre[wave] = pre;
    H.post[wave] = post;
  }
  if (nw > 1) __syncthreads();
  if (wave != 0) return;
  double D = R_d;
  if (fold) {
    double p4 = 0.0;
    long long q4 = 0;
    for (int w = 0; w < nw; w++) {
      p4 += H.pre[w];
      q4 += H.post[w];
    }
    const double Dn = (1.0 + p4) + (double)q4 * 0x1p-52;
    if (Dn < 2.0) D = Dn;
  }
  const double lse = H.ok ? (double)m_v + log(D) : __builtin_nan("");
  if (lane == 0 && a.row_lse) a.row_lse[row] = lse;
  if (a.top_logprob || a.top_logprob64) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int i = r * 64 + lane;
      if (i < a.n_top) {
        const double lp = i < H.n_have ? (double)H.vals[i] - lse : __builtin_nan("");
        if (a.top_logprob) a.top_logprob[(int64_t)row * a.top_ld + i] = (float)lp;
        if (a.top_logprob64) a.top_logprob64[(int64_t)row * a.top_ld + i] = lp;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Whether the exact denominator settles a controlled row's token.
//
// On a controlled row the reference divides by its serial f32 sum S' of the
// softmax terms (sampler.rs:301-305); the finalizer divided by S, the exact
// sum rounded to f32.  A serial sum of n terms >= 0 lies within a factor
// 1 +- n 2^-24 of the exact one, and every weight rn(e / D) of a denominator
// D is e / D up to one rounding: the scale 1 / D is common to the weights,
// the serial sums of weights, their renormalisation and u times their total,
// so it cancels from every decision of the draw, and only roundings remain.
// The token drawn with S is therefore the one drawn with S' when:
//  - consecutive entries of the selection (logit order: e non-increasing)
//    have equal e (equal p for every D, ordered by id), or e so far apart
//    that no D rounds them to one p: e_a - e_b > 2^-22 e_a (more than an ulp
//    of the larger p) and e_a - e_b > 2^-148 D (more than a subnormal ulp).
//    Every D then yields the same candidates in the same order.  A call that
//    takes tokens only passes over entries with e < 2^-65: their weights are
//    under 2^-64 of the largest, never drawn, and move a sum by less than the
//    2^-50 slack below;
//  - a run of equal e that crosses the top-k boundary and reaches the last
//    selected entry lies far above everything outside the selection (at most
//    e(next_below(vL)), or +0 when every finite value is selected);
//  - the top-p cut and the draw hold with a margin over the roundings of both
//    computations: a serial prefix c_j of renormalised weights is C_j (1 + r)
//    with |r| <= (k + j + 2) 2^-24 (each p, the k-term sum, the division, j
//    additions); x = rn(u T_w) is within (k + keep + 3) 2^-24 of u times its
//    exact total; twice each (S and S'), plus the p's subnormal ulps.
// A row that fails is summed serially by its finalizing wave (ser_local)
// and finalized again with S'.  The order part (order_settled) runs as soon
// as the selection's e are known, the margins (draw_settled) after the draw.
template <int R>
XS_DEV float at_lane(const float (&v)[R], int i) {  // element i of a list held R per lane (i uniform)
  float out = 0.0f;
#pragma unroll
  for (int r = 0; r < R; r++)
    if ((i >> 6) == r) out = rdlf(v[r], i & 63);
  return out;
}
// The largest logit of the row below vL, the selection's last, or a bound
// above it: each sub-record's entries are every element of its wave at or
// above its filter floor (header word 7), and every floor lies at or below vL
// (a wave with K' elements above vL would have put them in the selection), so
// what lies below vL is an entry below vL or lies below some floor.  A
// sub-record whose entries past the preloaded EPRE may hold the answer, or
// whose floor is unknown (+inf after an overflow), gives next_below(vL).  One
// wave; E: sub-records 0..63's first EPRE entries, as load_heads read them.
template <bool LOC>
XS_DEV float below_selection(const uint64_t* rowrec, int nsp, int nsub, const uint64_t (&E)[EPRE], float vL) {
  const int lane = lane_id();
  float best = -INFINITY;
  for (int g = 0; g * 64 < nsub; g++) {
    const int s = g * 64 + lane;
    const bool live = s < nsub;
    const int sc = min(s, nsp - 1);  // (clamped, not guarded: the loads go out together)
    const uint64_t h3 = ld_sub<LOC>(&rowrec[3 * nsp + sc]), h4 = ld_sub<LOC>(&rowrec[4 * nsp + sc]);
    const uint64_t h7 = ld_sub<LOC>(&rowrec[7 * nsp + sc]);
    uint64_t e[EPRE];
#pragma unroll
    for (int j = 0; j < EPRE; j++) e[j] = g == 0 ? E[j] : ld_sub<LOC>(&rowrec[(SHDR + j) * nsp + sc]);
    const int cnt = live ? (int)min((uint32_t)h4, (uint32_t)CAPW) : 0;
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPRE; j++) {
      const float x = keyf(pk_key(e[j]));
      if (j < cnt && x < vL) mb = fmaxf(mb, x);
    }
    const bool srt = ((h3 >> 32) & 4u) != 0;
    const bool complete = cnt <= EPRE || (srt && keyf(pk_key(e[EPRE - 1])) < vL);
    const float fl = __uint_as_float((uint32_t)h7);
    float b = -INFINITY;
    if (live) b = (complete && fl <= vL) ? fmaxf(mb, next_below(fl)) : next_below(vL);
    best = fmaxf(best, b);
  }
  return wave_maxf(best);
}

template <int R>
XS_DEV bool order_settled(const float (&ee)[R], int nsel, int kp, int k, bool full, float e_below, float S,
                          float dthr, bool cands) {
  const int lane = lane_id();
  const float thr = S * dthr;  // 2^-148 D for every D the serial sum can take (f32: the constants carry 1 %)
  const float NEG = 0x1p-65f;
  auto robust = [&](float ea, float eb) __attribute__((always_inline)) {
    const float g = ea - eb;  // (ea >= eb >= 0: exact when eb >= ea / 2, far above the bounds otherwise)
    return ea == eb || (g > ea * 0x1p-21f && g > thr);
  };
  bool bad = false;
#pragma unroll
  for (int r = 0; r < R; r++) {  // consecutive selected entries i, i + 1
    const float first_next = (r + 1 < R) ? rdlf(ee[r + 1 < R ? r + 1 : r], 0) : 0.0f;
    const float en = lane == 63 ? first_next : __shfl(ee[r], (lane + 1) & 63);
    const int i = r * 64 + lane;
    if (i + 1 < nsel && (cands || ee[r] >= NEG) && !robust(ee[r], en)) bad = true;
  }
  bool ubad = false;  // (uniform)
  const bool all_sel = nsel < kp;  // every finite value is selected; the rest are +0
  if (nsel >= 1 && all_sel) {
    const float el = at_lane(ee, nsel - 1);
    if ((cands || el >= NEG) && !robust(el, 0.0f)) ubad = true;
  }
  if (!full && nsel > k && nsel >= 1) {
    const float e1 = at_lane(ee, k - 1), eL = at_lane(ee, nsel - 1);
    const float below = all_sel ? 0.0f : e_below;
    if (e1 == eL && (cands || e1 >= NEG) && !(below < eL && robust(eL, below))) ubad = true;
  }
  return __ballot(bad) == 0 && !ubad;
}
template <int R>
XS_DEV bool draw_settled(const float (&c)[R], float tot, float x, int idx, int keep, int k, bool cut_found,
                         bool renorm, float S, float top_p) {
  // Lane-parallel: lane j tests its own prefix c_j where a decision uses it,
  // against uu (k + j + 4) c_j plus the slack; one ballot.  (f32 without
  // divisions: a difference of close values is exact, the margins carry
  // 2 %, and the p's subnormal ulps, 2^-150 / sum in renormalised units, are
  // bounded with 1 / sum <= S.)
  const int lane = lane_id();
  const float uu = 0x1p-23f * 1.02f;
  const float sl = (float)(2 * k + 8) * 0x1p-148f * S + 0x1p-50f;
  const float mt = uu * (float)(k + keep + 4) * tot + sl;  // x's own share
  const int jc = cut_found ? keep - 1 : k - 1;               // the top-p decision's prefix
  bool bad = false;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int j = r * 64 + lane;
    const float cj = c[r];
    const float m = uu * (float)(k + j + 4) * cj;
    if (renorm && j == jc && !(cut_found ? cj - top_p > m + sl : top_p - cj > m + sl)) bad = true;
    if (renorm && cut_found && j == keep - 2 && !(top_p - cj > m + sl)) bad = true;
    if (j == idx - 1 && !(x - cj > m + mt)) bad = true;            // cum_(idx-1) <= x
    if (j == idx && j < keep - 1 && !(cj - x > m + mt)) bad = true;  // x < cum_idx (at keep - 1: the total)
  }
  return __ballot(bad) == 0;
}

// ---------------------------------------------------------------------------
// Row finalize, common case: at most 64 sub-records (one per lane), K' <= 64,
// at most SURV survivors, and no boundary
// tie that needs the id-ordered row scan.  Returns false (having written
// nothing) when the row is outside that case; the general finalizer then
// does the row.  Same arithmetic, in the same order, as the general path.
template <bool HAS_MASK, bool WANT_LSE, bool LOC>
XS_DEV bool fin_fast(const Args& a, const Cfg& cfg, int row, int nsub, const uint64_t (&h)[NHW],
                     const uint64_t (&E)[EPRE], const uint64_t* rowrec, int nsp, const float* rowp,
                     FinLds& F, float S_ser) {
  const int lane = lane_id();
  const bool live = lane < nsub;
  const bool stoch = !cfg.greedy;
  const int kp = cfg.kp, k = cfg.k;
  const float u_row = a.greedy_all ? 0.0f : a.uniforms[row];
  const double et = (&kExpT[0][0])[lane];

  const int cnt = live ? (int)min((uint32_t)h[4], (uint32_t)CAPW) : 0;  // clamped: never read past a sub-record
  const float m_v = red_maxf(live ? __uint_as_float((uint32_t)h[3]) : -INFINITY);
  const uint32_t hf = live ? (uint32_t)(h[3] >> 32) : 0u;
  const bool nan_seen = __ballot(hf & 1u) != 0;
  const bool finite_seen = __ballot(hf & 2u) != 0;
  const float m_s = cfg.scale ? m_v * cfg.inv : m_v;
  double part = 0.0, rpart = 0.0;
  if (live) {
    const double p = __longlong_as_double((long long)h[0]);
    if (p != 0.0) part = p * (double)xexp2((__uint_as_float((uint32_t)h[1]) - m_s) * LOG2E);
    if (WANT_LSE) {
      const double r = __longlong_as_double((long long)h[2]);
      if (r != 0.0) rpart = r * (double)xexp2((__uint_as_float((uint32_t)(h[1] >> 32)) - m_v) * LOG2E);
    }
  }
  const double S_d = red_sumd(part);
  const double R_d = WANT_LSE ? red_sumd(rpart) : 0.0;
  const float S = S_ser >= 0.0f ? S_ser : (float)S_d;  // a controlled row's serial sum, when given
  int st = XS_ROW_OK;
  if (HAS_MASK && !finite_seen) st = XS_ROW_NO_FINITE;
  else if (cfg.greedy) st = nan_seen ? XS_ROW_NAN : (m_v == -INFINITY ? XS_ROW_NO_FINITE : XS_ROW_OK);
  else if (nan_seen || __builtin_isinf(m_s)) st = XS_ROW_NAN;

  // Survivor bound: the K'-th largest of the sub-records' first published
  // keys; of all four when fewer than 2K' of the first are finite (a sparse
  // mask), which would leave the first bound weak or absent.
  uint32_t tau = 0;
  const int nfin = __popcll(__ballot(live && (uint32_t)h[5] > KEY_NEG_INF));
  if (nfin >= 2 * kp) {
    uint32_t x[1] = {live ? (uint32_t)h[5] : 0u};
    wave_sort_desc<1>(x);
    tau = rdl(x[0], kp - 1);
  } else if (4 * nsub >= kp) {
    const uint32_t x[4] = {live ? (uint32_t)h[5] : 0u, live ? (uint32_t)(h[5] >> 32) : 0u,
                           live ? (uint32_t)h[6] : 0u, live ? (uint32_t)(h[6] >> 32) : 0u};
    tau = kth_largest_few<4>(x, kp, reinterpret_cast<uint32_t*>(F.srt));
  }
  // Gather the survivors into LDS, then order them by rank: a survivor's
  // position is the number of survivors above it ((key, ~id) are distinct).
  const uint64_t floor_e = (uint64_t)tau << 32;
  int M = 0;
  auto put = [&](uint64_t e, bool ok) __attribute__((always_inline)) {
    const uint64_t b = __ballot(ok);
    if (b) {
      const int pos = M + lanes_below(b);
      if (ok && pos < SURV) F.list[pos] = e;
      M += __popcll(b);
    }
  };
  {
    // the preloaded entries: each lane's survivors go after those of the
    // lanes below it (an exclusive scan of the per-lane counts)
    bool ok[EPRE];
    int c = 0;
#pragma unroll
    for (int j = 0; j < EPRE; j++) {
      ok[j] = j < cnt && E[j] >= floor_e;
      c += ok[j] ? 1 : 0;
    }
    const int incl = wave_incl_scan(c);
    int pos = incl - c;
    uint64_t* const spare = &F.srt[lane];  // non-survivors write here: no exec-mask branches
#pragma unroll
    for (int j = 0; j < EPRE; j++) {
      uint64_t* const dst = (ok[j] && pos < SURV) ? &F.list[pos] : spare;
      *dst = E[j];
      pos += ok[j] ? 1 : 0;
    }
    M = (int)rdl((uint32_t)incl, 63);
  }
  // entries past the preloaded ones (a sub-record holding more than EPRE); in
  // a sorted sub-record (flag 4) they end at the first one below the floor
  const bool srt = (hf & 4u) != 0;
  int lim = (srt && E[EPRE - 1] < floor_e) ? EPRE : cnt;
#pragma unroll 1
  for (int j0 = EPRE; __ballot(j0 < lim); j0 += 4) {
    uint64_t e[4];
#pragma unroll
    for (int u = 0; u < 4; u++)  // (clamped inside the sub-record, not guarded: all four in flight)
      e[u] = ld_sub<LOC>(rowrec + (int64_t)(SHDR + min(j0 + u, CAPW - 1)) * nsp + lane);
#pragma unroll
    for (int u = 0; u < 4; u++) put(e[u], j0 + u < lim && e[u] >= floor_e);
    if (srt && j0 + 3 < lim && e[3] < floor_e) lim = j0;
  }
  if (M > SURV) return false;
  F.expt[lane] = et;
  wave_lds_sync();
  // rank by counting the survivors above, LDS broadcast reads
  uint64_t sel;
  if (M <= 64) {
    const uint64_t xv = lane < M ? F.list[lane] : 0ull;
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < M; j++) rank += (F.list[j] > xv) ? 1 : 0;
    if (lane < M) F.srt[rank] = xv;
    wave_lds_sync();
    sel = lane < M ? F.srt[lane] : 0ull;
  } else {
    rank_sort_lds(F.list, F.srt, M);
    sel = F.srt[lane];
  }
  const int nsel = min(M, kp);
  const bool want_cands = a.cand_id != nullptr || a.cand_w != nullptr;
  // a whole short row with ids the selection never holds (-inf): the
  // general path lists them
  if (cfg.full && stoch && nsel < k && want_cands) return false;

  // Probabilities of the selection (lanes < nsel) and, on lane nsel, of the
  // largest value below the last selected logit (the boundary proof).
  const double* T = F.expt;
  float pw = 0.0f;
  uint64_t pk = 0ull;
  float w = 0.0f;
  int tok = -1;
  // a masked row not given the serial sum: its token is checked against the
  // roundings that sum could change (order_settled, draw_settled); with one
  // finite value the token is that id for every denominator
  const bool check = HAS_MASK && S_ser < 0.0f && nsel > 1;
  bool unsettled = false;
  if (stoch && st == XS_ROW_OK) {
    const float vL = nsel > 0 ? keyf(pk_key(rdl64(sel, nsel - 1))) : -INFINITY;
    const bool need_below = !cfg.full && vL != -INFINITY;
    const bool in = lane < nsel;
    float pe = 0.0f, ee = 0.0f;
    if (in || (lane == nsel && need_below)) {
      ee = exact_e(in ? keyf(pk_key(sel)) : next_below(vL), cfg, m_s, T);
      pe = __fdiv_rn(ee, S);  // exact_p
    }
    if (in) {
      pw = pe;
      pk = ((uint64_t)__float_as_uint(pe + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - pk_id(sel));
    }
    float pbelow = 0.0f, ebelow = 0.0f;
    if (need_below) {
      if (nsel < 64) {
        pbelow = rdlf(pe, nsel);
        ebelow = rdlf(ee, nsel);
      } else {
        ebelow = exact_e(next_below(vL), cfg, m_s, T);
        pbelow = __fdiv_rn(ebelow, S);
      }
    }
    if (!in) ee = 0.0f;
    if (check) {
      const float ea[1] = {ee};
      // a run of equal e across the top-k boundary: bounded below by the
      // row's actual next logit rather than next_below(vL)
      if (!cfg.full && nsel == kp && nsel > k && rdlf(ee, k - 1) == rdlf(ee, nsel - 1))
        ebelow = exact_e(below_selection<LOC>(rowrec, nsp, nsub, E, vL), cfg, m_s, T);
      unsettled = !order_settled<1>(ea, nsel, kp, k, cfg.full, ebelow, S, cfg.dthr, want_cands);
    }
    // (p desc, id asc): p is non-increasing along the logit order, so only
    // runs of equal p can be out of order
    const uint64_t nxt = shfl64(pk, (lane + 1) & 63);
    if (__ballot(lane + 1 < nsel && pk < nxt)) {
      uint64_t x[1] = {pk};
      wave_sort_desc64<1>(x);
      pk = x[0];
    }
    if (!cfg.full) {
      const float Pk = __uint_as_float((uint32_t)(rdl64(pk, k - 1) >> 32));
      const float pL = rdlf(pw, nsel - 1);
      bool slow = nsel < kp;
      if (!slow && pL == Pk) {
        const bool other = __ballot(in && pw == Pk && keyf(pk_key(sel)) != vL) != 0;
        slow = other || pbelow == Pk;
      }
      if (slow && Pk == 0.0f && !want_cands) slow = false;
      if (slow) return false;  // ties at P_k: the general path resolves them
    }

    // The draw (truncate_top_p, then WeightedIndex), serial f32: lane i
    // ends each chain with the serial prefix sum through weight i.
    w = lane < k ? __uint_as_float((uint32_t)(pk >> 32)) : 0.0f;
    // Every lane adds the same weights (uniform, from scalar registers) in
    // order; lane j keeps the running value after weight j.  The weights past
    // k are +0.0 and leave the sums unchanged.
    auto chain = [&](float init, float& at_lane) __attribute__((always_inline)) -> float {
      float acc = init, mine = 0.0f;
#pragma unroll
      for (int b0 = 0; b0 < 64; b0 += 8) {
        if (b0 < k) {
          float q[8];
#pragma unroll
          for (int u = 0; u < 8; u++) q[u] = rdlf(w, b0 + u);
#pragma unroll
          for (int u = 0; u < 8; u++) {
            acc = acc + q[u];
            mine = (lane == b0 + u) ? acc : mine;
          }
        }
      }
      at_lane = mine;
      return acc;
    };
    bool zero = false;
    const bool renorm = !(cfg.top_p >= 1.0f);
    float sumc = 1.0f;
    if (renorm) {
      float unused;
      sumc = chain(-0.0f, unused);  // folds from -0.0 as Rust's f32 Sum does
      if (!(sumc > 0.0f)) zero = true;  // all weights zero: returned unchanged
      else w = __fdiv_rn(w, sumc);
    }
    if (zero) {
      st = XS_ROW_ZERO_WEIGHT;
    } else {
      float c;
      (void)chain(0.0f, c);
      int keep = k;
      bool found = false;
      if (renorm) {
        const uint64_t bm = __ballot(lane < k && c >= cfg.top_p);
        found = bm != 0ull;
        if (bm) keep = (int)__builtin_ctzll(bm) + 1;
        if (lane >= keep) w = 0.0f;
      }
      const float tot = rdlf(c, keep - 1);
      if (__ballot(lane < k && !(w >= 0.0f)) || tot == 0.0f) {
        st = XS_ROW_ZERO_WEIGHT;
      } else {
        const float x_draw = u_row * tot + 0.0f;
        const float cum = lane < keep - 1 ? c : tot;
        const int idx = (int)__popcll(__ballot(lane < k - 1 && cum <= x_draw));
        tok = (int)pk_id(rdl64(pk, idx));
        if (check) {
          const float ca[1] = {c};
          unsettled = unsettled || cfg.force ||
                      !draw_settled<1>(ca, tot, x_draw, idx, keep, k, found, renorm, S, cfg.top_p);
        }
      }
    }
  } else if (st == XS_ROW_OK) {
    tok = (int)pk_id(rdl64(sel, 0));
  }

  if (unsettled) {  // (nothing written) the workgroup sums the serial denominator
    if (lane == 0) {
      F.need_ser = 1;
      F.ser_ms = m_s;
    }
    return true;
  }

  // held_row: the statistics for held_fold, which writes row_lse and the
  // top-n log-probs once the workgroup has folded the denominator
  const bool lse_ok = !nan_seen && !__builtin_isinf(m_v);
  if (WANT_LSE && (a.row_lse || a.n_top > 0)) {
    const int nh = min(min(a.n_top, (int)a.enc), nsel);
    if (lane == 0) {
      F.held.R_d = R_d;
      F.held.m_v = m_v;
      F.held.top = pk_id(rdl64(sel, 0));
      F.held.ok = lse_ok ? 1 : 0;
      F.held.can_fold = 1;
      F.held.n_have = nh;
    }
    if (lane < nh) F.held.vals[lane] = keyf(pk_key(sel));
  }

  // Outputs.
  if (lane == 0) {
    st_agent(&a.token[row], st == XS_ROW_OK ? tok : -1);
    st_agent(&a.status[row], st);
    if (a.n_cand) a.n_cand[row] = (stoch && st == XS_ROW_OK) ? k : 0;
    if (a.soft_max) a.soft_max[row] = m_s;
    if (a.soft_sum) a.soft_sum[row] = S;
    if (WANT_LSE) {
      if (a.row_max) a.row_max[row] = m_v;
      if (a.p_max) a.p_max[row] = lse_ok ? (float)(1.0 / R_d) : __builtin_nanf("");
    }
  }
  if (want_cands && stoch && st == XS_ROW_OK) {
    const int kw = (int)min((int64_t)k, a.cand_ld);
    if (lane < kw) {
      if (a.cand_id) a.cand_id[(int64_t)row * a.cand_ld + lane] = (int32_t)(0xFFFFFFFFu - (uint32_t)pk);
      if (a.cand_w) a.cand_w[(int64_t)row * a.cand_ld + lane] = w;
    }
  }
  if (WANT_LSE && a.n_top > 0 && a.top_id) {
    const int nt = min(a.n_top, (int)a.enc);
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int i = r * 64 + lane;
      if (i < a.n_top) a.top_id[(int64_t)row * a.top_ld + i] = (r == 0 && i < nt && i < nsel) ? (int32_t)pk_id(sel) : -1;
    }
  }
  return true;
}

// ---------------------------------------------------------------------------
// Row finalize, general case (the rows fin_fast leaves): any number of
// sub-records up to GMAX * 64, K' up to KSEL, survivors past SURV, sparse
// controls, and probability ties at the top-k boundary.  Lane l handles
// sub-records l + 64g; group 0's header words and first EPRE entries are the
// ones finalize_row preloaded, the rest are read where they are used.
template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL, bool LOC>
XS_DEV void fin_general(const Args& a, const Cfg cfg, int row, const uint64_t* rowrec,
                        int nsp, int nsub, const float* rowp, const uint32_t* mrow, const CtlRow& cr,
                        const uint64_t (&h)[NHW], const uint64_t (&E)[EPRE], FinLds& F, float S_ser) {
  const int lane = lane_id();
  const int kp = cfg.kp, enc = (int)a.enc;
  const bool stoch = !cfg.greedy && !cfg.bad;
  const uint64_t* rr = rowrec;
  const int G = (nsub + 63) >> 6;
  const float u_row = a.greedy_all ? 0.0f : a.uniforms[row];  // prefetched for the draw
  const double et = (&kExpT[0][0])[lane];  // the exp table, staged into LDS below
  auto has = [&](int g) __attribute__((always_inline)) { return g < G && g * 64 + lane < nsub; };
  auto hdr = [&](int g, int i) __attribute__((always_inline)) -> uint64_t {
    if (g == 0 && i < NHW) {  // sub-records 0..63: the words finalize_row preloaded
      uint64_t v = h[0];
#pragma unroll
      for (int t = 1; t < NHW; t++) v = i == t ? h[t] : v;
      return has(0) ? v : 0ull;
    }
    const uint64_t v = ld_sub<LOC>(&rr[i * nsp + min(g * 64 + lane, nsp - 1)]);  // (clamped, not guarded)
    return has(g) ? v : 0ull;
  };

  float mv = -INFINITY;
  uint32_t fw = 0;
#pragma unroll
  for (int g = 0; g < GMAX; g++) {
    if (has(g)) {
      const uint64_t h3 = hdr(g, 3);
      mv = fmaxf(mv, __uint_as_float((uint32_t)h3));
      fw |= (uint32_t)(h3 >> 32);
    }
  }
  const float m_v = wave_maxf(mv);
  const uint32_t fl = wave_or(fw);
  const float m_s = cfg.scale ? m_v * cfg.inv : m_v;
  double S_d = 0.0, R_d = 0.0;
#pragma unroll
  for (int g = 0; g < GMAX; g++) {
    if (has(g)) {
      const uint64_t h1 = hdr(g, 1);
      const double p = __longlong_as_double((long long)hdr(g, 0));
      if (p != 0.0) S_d += p * (double)xexp2((__uint_as_float((uint32_t)h1) - m_s) * LOG2E);
      if (WANT_LSE) {
        const double r = __longlong_as_double((long long)hdr(g, 2));
        if (r != 0.0) R_d += r * (double)xexp2((__uint_as_float((uint32_t)(h1 >> 32)) - m_v) * LOG2E);
      }
    }
  }
  S_d = wave_sumd(S_d);
  if (WANT_LSE) R_d = wave_sumd(R_d);
  const float S = S_ser >= 0.0f ? S_ser : (float)S_d;  // a controlled row's serial sum, when given
  const bool nan_seen = fl & 1u;
  const bool finite_seen = fl & 2u;

  // A controlled row (mask or sparse controls) errors when nothing finite is
  // left (sampler.rs:483-488); a forced row always keeps its target.
  const bool ctl_on = HAS_CTL && cr.active;
  int st = XS_ROW_OK;
  if (ctl_on && cr.status != XS_ROW_OK) st = cr.status;
  else if (cfg.bad) st = XS_ROW_BAD_PARAM;
  else if ((HAS_MASK || ctl_on) && !finite_seen) st = XS_ROW_NO_FINITE;
  else if (cfg.greedy) st = nan_seen ? XS_ROW_NAN : (m_v == -INFINITY ? XS_ROW_NO_FINITE : XS_ROW_OK);
  else if (nan_seen || __builtin_isinf(m_s)) st = XS_ROW_NAN;

  // Survivor bound: the K'-th largest of the published keys (distinct
  // elements: each chunk's top group or lane maxima), as many per sub-record
  // as one four-register sort holds.
  uint32_t tau_row = 0;
  {
    const int qk = (G == 1) ? 4 : (G == 2 ? 2 : 1);  // keys used per sub-record
    const int nv = qk * nsub;
    if (nv >= kp && !cfg.bad) {
      uint32_t x[4] = {0u, 0u, 0u, 0u};
      if (G == 1) {
        if (lane < nsub) {
          const uint64_t h5 = hdr(0, 5), h6 = hdr(0, 6);
          x[0] = (uint32_t)h5;
          if (qk == 4) {
            x[1] = (uint32_t)(h5 >> 32);
            x[2] = (uint32_t)h6;
            x[3] = (uint32_t)(h6 >> 32);
          }
        }
      } else {
#pragma unroll
        for (int g = 0; g < GMAX; g++) {
          const int s = g * 64 + lane;
          if (has(g)) {
            const uint64_t h5 = hdr(g, 5);
            F.keys[s * qk] = (uint32_t)h5;
            if (qk == 2) F.keys[s * qk + 1] = (uint32_t)(h5 >> 32);
          }
        }
        wave_lds_sync();
#pragma unroll
        for (int r = 0; r < 4; r++) x[r] = (r * 64 + lane < nv) ? F.keys[r * 64 + lane] : 0u;
        wave_lds_sync();
      }
      tau_row = kth_largest<4>(x, kp);
    }
  }

  // Gather the survivors (entries at or above the bound) into LDS.
  uint64_t floor_e = (uint64_t)tau_row << 32;
  int M = 0;
  auto put = [&](uint64_t e, bool ok) __attribute__((always_inline)) {
    const uint64_t b = __ballot(ok);
    if (b) {
      const int pos = M + lanes_below(b);
      if (ok && pos < SURV) F.list[pos] = e;
      M += __popcll(b);
    }
  };
  auto gather_global = [&](int g, int s, int c, bool srt, uint64_t fl_e) __attribute__((always_inline)) {
    // the c entries of sub-record s (the first EPRE of group 0 preloaded, the
    // rest read from the workspace); in a sorted sub-record (flag 4) they end
    // at the first one below the floor
    int lim = c, j = 0;
    if (g == 0) {
#pragma unroll
      for (int u = 0; u < EPRE; u++) put(E[u], u < lim && E[u] >= fl_e);
      if (srt && EPRE - 1 < lim && E[EPRE - 1] < fl_e) lim = EPRE;
      j = EPRE;
    }
    for (; __ballot(j < lim); j += 4) {
      uint64_t e[4];
#pragma unroll
      for (int u = 0; u < 4; u++)  // (clamped inside the sub-record, not guarded: all four in flight)
        e[u] = ld_sub<LOC>(rr + (int64_t)(SHDR + min(j + u, CAPW - 1)) * nsp + s);
#pragma unroll
      for (int u = 0; u < 4; u++) put(e[u], j + u < lim && e[u] >= fl_e);
      if (srt && j + 3 < lim && e[3] < fl_e) lim = j;
    }
  };
  auto gather = [&](uint64_t fl_e) __attribute__((always_inline)) {
    M = 0;
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
      const int s = g * 64 + lane;
      if (g < G) {
        const uint64_t h3 = hdr(g, 3), h4 = hdr(g, 4);
        gather_global(g, s, has(g) ? (int)min((uint32_t)h4, (uint32_t)CAPW) : 0, ((h3 >> 32) & 4u) != 0, fl_e);
      }
    }
  };
  if (!cfg.bad) gather(floor_e);
  if (M > SURV) {
    // More survivors than one wave sorts (ties at the bound across many
    // waves): move the floor to the exact K'-th largest entry by bisection
    // over every entry, then gather again.
    uint64_t ans = 0;
    for (int bit = 63; bit >= 0; bit--) {
      const uint64_t cnd = ans | (1ull << bit);
      int c = 0;
#pragma unroll
      for (int g = 0; g < GMAX; g++) {
        const int s = g * 64 + lane;
        const int n = has(g) ? (int)min((uint32_t)hdr(g, 4), (uint32_t)CAPW) : 0;
        for (int j = 0; j < n; j++) c += ld_sub<LOC>(rr + (int64_t)(SHDR + j) * nsp + s) >= cnd ? 1 : 0;
      }
      if (wave_sumi(c) >= kp) ans = cnd;
    }
    floor_e = ans;
    gather(floor_e);
  }
  F.expt[lane] = et;
  wave_lds_sync();

  // Sort the survivors (logit desc, id asc); the first K' are the selection:
  // up to 128 by a bitonic sort in registers, more by rank in LDS.
  const int nsel = min(M, kp);  // == kp unless the row holds fewer finite values
  uint64_t sel[2];
  uint64_t last_sel;  // the K'-th survivor
  if (M <= 128) {
    uint64_t x[2];
#pragma unroll
    for (int r = 0; r < 2; r++) x[r] = (r * 64 + lane < M) ? F.list[r * 64 + lane] : 0ull;  // entries are > 0
    wave_sort_desc64<2>(x);
#pragma unroll
    for (int r = 0; r < 2; r++) sel[r] = (r * 64 + lane < nsel) ? x[r] : 0ull;
    last_sel = nsel > 0 ? pick64(x, nsel - 1) : 0ull;
  } else {
    rank_sort_lds(F.list, F.srt, min(M, SURV));
#pragma unroll
    for (int r = 0; r < 2; r++) sel[r] = (r * 64 + lane < nsel) ? F.srt[r * 64 + lane] : 0ull;
    last_sel = nsel > 0 ? F.srt[nsel - 1] : 0ull;
  }

  // Probabilities of the selection and the (p desc, id asc) order; p is
  // non-increasing along the logit order, so only runs of equal p move.
  const int k = cfg.k;
  const bool want_cands = a.cand_id != nullptr || a.cand_w != nullptr;
  float pw[2] = {0.0f, 0.0f};    // p of selection entry r*64+lane (K' <= 128)
  uint64_t pk[2] = {0ull, 0ull};  // (p bits << 32) | ~id
  const double* T = F.expt;
  // the value the boundary proof needs, p(next_below(vL)), is computed in the
  // same pass, by the lane just past the selection
  const float vL = nsel > 0 ? keyf(pk_key(last_sel)) : -INFINITY;
  float pbelow = 0.0f;
  float ee[2] = {0.0f, 0.0f};  // e of selection entry r*64+lane (the numerators of pw)
  float ebelow = 0.0f;
  // a controlled row not given the serial sum: its token is checked against
  // the roundings that sum could change (order_settled, draw_settled); with
  // one finite value the token is that id for every denominator
  const bool check = (HAS_MASK || ctl_on) && S_ser < 0.0f && nsel > 1;
  bool unsettled = false;
  bool lazy_order = false;  // the (p desc, id asc) repair left to the draw
  if (stoch && st == XS_ROW_OK && !cfg.big) {
    const bool need_below = !cfg.full && vL != -INFINITY;
#pragma unroll
    for (int r = 0; r < 2; r++) {
      if (r * 64 <= nsel) {
        const int i = r * 64 + lane;
        const bool in = i < nsel;
        if (in || (i == nsel && need_below)) {
          const float e = exact_e(in ? keyf(pk_key(sel[r])) : next_below(vL), cfg, m_s, T);
          const float pe = __fdiv_rn(e, S);  // exact_p
          pw[r] = pe;  // (lane nsel: the boundary value, read below and then cleared)
          ee[r] = e;
          if (in) pk[r] = ((uint64_t)__float_as_uint(pe + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - pk_id(sel[r]));
        }
      }
    }
    if (need_below) {
      if (nsel < 128) {
        pbelow = rdlf(nsel < 64 ? pw[0] : pw[1], nsel & 63);
        ebelow = rdlf(nsel < 64 ? ee[0] : ee[1], nsel & 63);
      } else {
        ebelow = exact_e(next_below(vL), cfg, m_s, T);
        pbelow = __fdiv_rn(ebelow, S);
      }
    }
    if (lane == (nsel & 63)) {
      if (nsel < 64) pw[0] = ee[0] = 0.0f;
      else if (nsel < 128) pw[1] = ee[1] = 0.0f;
    }
    if (check) {
      // a run of equal e across the top-k boundary: bounded below by the
      // row's actual next logit rather than next_below(vL)
      if (!cfg.full && nsel == kp && nsel > k && at_lane(ee, k - 1) == at_lane(ee, nsel - 1))
        ebelow = exact_e(below_selection<LOC>(rr, nsp, nsub, E, vL), cfg, m_s, T);
      unsettled = !order_settled<2>(ee, nsel, kp, k, cfg.full, ebelow, S, cfg.dthr, want_cands);
    }
    bool bad = false;
    const uint64_t n0 = shfl64(pk[0], (lane + 1) & 63);
    const uint64_t n1 = shfl64(pk[1], (lane + 1) & 63);
    const uint64_t first1 = shfl64(pk[1], 0);
    if (lane + 1 < nsel && pk[0] < (lane < 63 ? n0 : first1)) bad = true;
    if (64 + lane + 1 < nsel && pk[1] < n1) bad = true;
    // Without a candidate list only the drawn entry's id needs the repaired
    // order: permuting a run of equal p leaves the weight sequence, and so
    // top-p and the draw's index, unchanged.  The draw then picks the id at
    // its index within the run (run_pick below) instead of sorting here.
    lazy_order = __ballot(bad) != 0 && !want_cands;
    if (__ballot(bad) && !lazy_order) {
      F.psel[lane] = pk[0];
      F.psel[64 + lane] = pk[1];
      wave_lds_sync();
      rank_sort_lds(F.psel, F.list, nsel);
      pk[0] = lane < nsel ? F.list[lane] : 0ull;
      pk[1] = 64 + lane < nsel ? F.list[64 + lane] : 0ull;
    }

    // Boundary proof (top_k < enc): the k-th probability P_k must not be shared
    // by an entry outside the selection.  Safe when the last selected entry is
    // strictly less probable, or when the tie is an exact logit tie (every
    // selected entry at P_k has the last logit vL and nothing below vL reaches
    // P_k), whose lowest ids the (logit desc, id asc) selection already kept.
    if (!cfg.full) {
      const float Pk = __uint_as_float((uint32_t)(pick64(pk, k - 1) >> 32));
      const float pL = rdlf(nsel - 1 < 64 ? pw[0] : pw[1], (nsel - 1) & 63);
      bool slow = nsel < kp;
      if (!slow && pL == Pk) {
        bool other = false;
#pragma unroll
        for (int r = 0; r < 2; r++)
          if (r * 64 + lane < nsel && pw[r] == Pk && keyf(pk_key(sel[r])) != vL) other = true;
        const bool below = vL != -INFINITY && pbelow == Pk;
        slow = __ballot(other) != 0 || below;
      }
      // Entries tied at P_k = 0 carry no weight: the draw does not depend on
      // which ids fill them, only the returned candidate list does.
      if (slow && Pk == 0.0f && !want_cands) slow = false;
      if (slow) {
        // the candidates are every selected entry with p > P_k, then the lowest
        // ids of the whole row with p == P_k
        F.psel[lane] = pk[0];
        F.psel[64 + lane] = pk[1];
        int g = 0;
        while (g < k && __uint_as_float((uint32_t)(pick64(pk, g) >> 32)) > Pk) g++;
        // exp arguments d = s - max whose exp can round to P_k * S: the rounding
        // interval of P_k widened generously; inside it every element gets the
        // exact test, outside it every element provably misses
        const double lo_p = Pk == 0.0f ? 0.0 : 0.5 * ((double)Pk + (double)__uint_as_float(__float_as_uint(Pk) - 1u));
        const double hi_p = 0.5 * ((double)Pk + (double)__uint_as_float(__float_as_uint(Pk) + 1u));
        // (e = rn(exp(d)) is within 2^-24 e, or 2^-150 where subnormal, of
        // exp(d); rn(e / S) == P_k needs lo_p <= e / S <= hi_p, and P_k > 0
        // needs e > 0, so exp(d) > 2^-150)
        const double elo = Pk == 0.0f ? 0.0 : fmax(lo_p * (double)S * (1.0 - 0x1p-10) - 0x1p-148, 0x1p-150);
        const double ehi = hi_p * (double)S * (1.0 + 0x1p-10) + 0x1p-148;
        const float x_lo = elo > 0.0 ? (float)(log(elo) - 0x1p-8) : -INFINITY;
        const float x_hi = (float)(log(ehi) + 0x1p-8);
        int need = k - g, have = g;
        auto dv = [&](float x) __attribute__((always_inline)) { return (cfg.scale ? x * cfg.inv : x) - m_s; };
        if (Pk > 0.0f) {
          // From the workspace first: a sub-record's entries are all of its
          // elements at or above its filter floor (header word 7), so all of
          // its band elements when the floor lies below the band; the other
          // sub-records' logits are read, in id order, until the ties found
          // below the next chunk's first id number `need` (not for a
          // controlled row: only the row scan below rebuilds controlled
          // values).  The list keeps ~id, so its descending order is id order;
          // when it fills, only its `need` lowest ids are kept.
          int nt = 0;
          auto compact = [&]() __attribute__((always_inline)) {
            wave_lds_sync();
            rank_sort_lds(F.list, F.srt, nt);
#pragma unroll
            for (int r = 0; r < 2; r++)
              if (r * 64 + lane < need) F.list[r * 64 + lane] = F.srt[r * 64 + lane];
            wave_lds_sync();
            nt = min(nt, need);
          };
          auto push = [&](bool hit, uint32_t id) __attribute__((always_inline)) {
            const uint64_t b = __ballot(hit);
            if (b) {
              if (nt + __popcll(b) > SURV) compact();
              const int pos = nt + lanes_below(b);
              if (hit) F.list[pos] = (uint64_t)(0xFFFFFFFFu - id);
              nt += __popcll(b);
            }
          };
          uint64_t inc[GMAX];  // sub-records whose entries may miss band elements
#pragma unroll
          for (int g2 = 0; g2 < GMAX; g2++) {
            inc[g2] = 0ull;
            if (g2 < G) {
              const int s = g2 * 64 + lane;
              const uint64_t h3 = hdr(g2, 3), h4 = hdr(g2, 4), h7 = hdr(g2, 7);
              const float fx = __uint_as_float((uint32_t)h7);
              const bool complete = !has(g2) || fx == -__FLT_MAX__ || dv(fx) < x_lo;
              inc[g2] = __ballot(!complete);
              const bool srt = ((h3 >> 32) & 4u) != 0;
              int lim = (complete && has(g2)) ? (int)min((uint32_t)h4, (uint32_t)CAPW) : 0;
              for (int j = 0; __ballot(j < lim); j += 4) {
                uint64_t e[4];
#pragma unroll
                for (int u = 0; u < 4; u++)  // (clamped inside the sub-record, not guarded)
                  e[u] = ld_sub<LOC>(rr + (int64_t)(SHDR + min(j + u, CAPW - 1)) * nsp + s);
                uint32_t hb = 0;  // bit u: entry j + u ties
#pragma unroll
                for (int u = 0; u < 4; u++) {
                  const float x = keyf(pk_key(e[u]));
                  const float d = dv(x);
                  if (j + u < lim && d >= x_lo && d <= x_hi && exact_p(x, cfg, m_s, S, T) == Pk) hb |= 1u << u;
                }
                if (srt && j + 3 < lim && dv(keyf(pk_key(e[3]))) < x_lo) lim = j;  // the rest lie below
                while (__ballot(hb != 0u)) {
                  const int u = hb ? (int)__builtin_ctz(hb) : 0;
                  const uint64_t eu = u == 0 ? e[0] : u == 1 ? e[1] : u == 2 ? e[2] : e[3];
                  push(hb != 0u, pk_id(eu));
                  hb &= hb - 1u;
                }
              }
            }
          }
          const bool ok = !(ctl_on && ((inc[0] | inc[1] | inc[2] | inc[3]) != 0ull));
          int cur = -1;  // chunk of the last sub-record read
          bool enough = !ok;
#pragma unroll
          for (int g2 = 0; g2 < GMAX; g2++) {
            uint64_t m = inc[g2];
            while (m && !enough) {  // one sub-record's logits: wave w of chunk c, as the chunk pass read them
              const int s = g2 * 64 + (int)__builtin_ctzll(m);
              m &= m - 1ull;
              const int c = s / NWAVE, w = s % NWAVE, s0 = c * SPC;
              if (c != cur) {  // every tie below chunk c's first id is known: enough of them?
                cur = c;
                const uint32_t lim_id = (uint32_t)s0 * SLOT;
                wave_lds_sync();
                int below = 0;
#pragma unroll
                for (int r = 0; r < 4; r++)
                  if (r * 64 + lane < nt) below += (0xFFFFFFFFu - (uint32_t)F.list[r * 64 + lane]) < lim_id ? 1 : 0;
                enough = wave_sumi(below) >= need;
                if (enough) break;
              }
#pragma unroll 1
              for (int j0 = 0; j0 < SPC; j0 += 4) {  // four slots at a time
                float4 v[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                  const int id0 = (s0 + j0 + j) * SLOT + 4 * (w * 64 + lane);
                  v[j] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
                  if (id0 < enc) v[j] = reinterpret_cast<const float4*>(rowp)[id0 >> 2];
                }
                uint32_t hb = 0u;  // bit 4j + e: element e of slot j0 + j ties
#pragma unroll
                for (int j = 0; j < 4; j++) {
                  const int id0 = (s0 + j0 + j) * SLOT + 4 * (w * 64 + lane);
                  const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                  for (int e = 0; e < 4; e++) {
                    const int id = id0 + e;
                    bool hit = id < enc;
                    if (HAS_MASK && hit && !((mrow[id >> 5] >> (id & 31)) & 1u)) hit = false;
                    const float d = dv(xv[e]);
                    if (hit && d >= x_lo && d <= x_hi && exact_p(xv[e], cfg, m_s, S, T) == Pk) hb |= 1u << (4 * j + e);
                  }
                }
                while (__ballot(hb != 0u)) {
                  const int t = hb ? (int)__builtin_ctz(hb) : 0;
                  push(hb != 0u, (uint32_t)((s0 + j0 + (t >> 2)) * SLOT + 4 * (w * 64 + lane) + (t & 3)));
                  hb &= hb - 1u;
                }
              }
            }
          }
          if (ok && nt >= need) {
            wave_lds_sync();
            rank_sort_lds(F.list, F.srt, nt);
            const uint64_t pkb = (uint64_t)__float_as_uint(Pk + 0.0f) << 32;
#pragma unroll
            for (int r = 0; r < 2; r++)
              if (r * 64 + lane < need) F.psel[have + r * 64 + lane] = pkb | (uint32_t)F.srt[r * 64 + lane];
            need = 0;  // done: the row scan below does not run
          }
        }
        int sc = 0;  // next patch (the list is sorted by id, as the scan runs)
        const uint64_t* pl = HAS_CTL ? a.patch + (int64_t)row * a.ctl_cap : nullptr;
        for (int base = 0; base < enc && need > 0; base += 256) {
          const int f = base / 4 + lane;
          float4 qv = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
          if (4 * f < enc) qv = reinterpret_cast<const float4*>(rowp)[f];
          float xv[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int id = 4 * f + e;
            if (HAS_MASK && id < enc && !((mrow[id >> 5] >> (id & 31)) & 1u)) xv[e] = -INFINITY;
          }
          if (ctl_on) {  // the controlled values, as sample_kernel saw them
            if (cr.force_id >= 0) {
#pragma unroll
              for (int e = 0; e < 4; e++) xv[e] = (4 * f + e == cr.force_id) ? cr.force_val : -INFINITY;
            } else {
              while (sc < cr.n_patch) {
                const uint64_t pe = pl[sc];
                const int off = (int)(uint32_t)(pe >> 32) - base;
                if (off >= 256) break;
                if ((off >> 2) == lane) {
                  const float pv = __uint_as_float((uint32_t)pe);
#pragma unroll
                  for (int e = 0; e < 4; e++) xv[e] = ((off & 3) == e) ? pv : xv[e];
                }
                sc++;
              }
              const int pt = cr.pull_id - base;
              if (pt >= 0 && pt < 256 && (pt >> 2) == lane) {
#pragma unroll
                for (int e = 0; e < 4; e++) xv[e] = ((pt & 3) == e) ? cr.pull_val : xv[e];
              }
            }
          }
          bool hit[4];
          int c = 0;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int id = 4 * f + e;
            const float x = xv[e];
            hit[e] = false;
            if (id < enc) {
              const float sx = cfg.scale ? x * cfg.inv : x;
              const float d = sx - m_s;
              if (d >= x_lo && d <= x_hi) hit[e] = exact_p(x, cfg, m_s, S, T) == Pk;
            }
            c += hit[e];
          }
          const int incl = wave_incl_scan(c);
          int pos = incl - c;
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (hit[e]) {
              if (pos < need) F.psel[have + pos] = ((uint64_t)__float_as_uint(Pk + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(4 * f + e));
              pos++;
            }
          const int tot = (int)rdl((uint32_t)incl, 63);
          have += min(tot, need);
          need -= tot;
        }
        wave_lds_sync();
        pk[0] = F.psel[lane];
        pk[1] = F.psel[64 + lane];
      }
    }
  }

  // The draw: truncate_top_p (sampler.rs:401-429) and WeightedIndex
  // (sampler.rs:235-243, rand 0.9), serial f32.  Weight i lives in lane i % 64
  // of w[i / 64].  Every lane runs the serial chain over weights 0..i of its
  // own index (adding 0.0 for the later ones, which changes nothing), so lane
  // i ends with the serial prefix sum through i: the top-p cumsum, the
  // WeightedIndex cumulative weights and its total all come from one chain.
  float w[2];
  w[0] = __uint_as_float((uint32_t)(pk[0] >> 32));
  w[1] = __uint_as_float((uint32_t)(pk[1] >> 32));
  int tok = -1;
  // a row with more candidates than the selection holds is drawn by the
  // whole-row kernels afterwards; here only its statistics
  const bool defer = cfg.big && stoch && st == XS_ROW_OK;
  if (st == XS_ROW_OK && !defer) {
    if (!stoch) {
      tok = (int)rdl(pk_id(sel[0]), 0);
    } else {
      if (lane >= k) w[0] = 0.0f;
      if (64 + lane >= k) w[1] = 0.0f;
      // prefix[r] = init + w_0 + ... + w_(r*64+lane), left to right in f32
      // A chain given a finite `stop` ends after the batch of 8 in which some
      // prefix reaches it: the top-p cut uses the prefixes only up to the
      // first that reaches top_p, and the draw only the total there.
      auto prefix = [&](float init, float (&pre)[2], float stop) __attribute__((always_inline)) {
        float acc = init;
        const int k0 = min(k, 64);
        bool cut = false;
        for (int b0 = 0; b0 < k0; b0 += 8) {
          float qv[8];
#pragma unroll
          for (int u = 0; u < 8; u++) qv[u] = rdlf(w[0], (b0 + u) & 63);
#pragma unroll
          for (int u = 0; u < 8; u++) acc = acc + ((lane >= b0 + u) ? qv[u] : 0.0f);
          if (__ballot(lane < b0 + 8 && lane < k && acc >= stop)) {
            cut = true;
            break;
          }
        }
        pre[0] = acc;
        pre[1] = acc;
        if (k > 64 && !cut) {
          float acc1 = rdlf(acc, 63);
          for (int b0 = 0; b0 < k - 64; b0 += 8) {
            float qv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) qv[u] = rdlf(w[1], (b0 + u) & 63);
#pragma unroll
            for (int u = 0; u < 8; u++) acc1 = acc1 + ((lane >= b0 + u) ? qv[u] : 0.0f);
          }
          pre[1] = acc1;
        }
      };
      auto at = [&](const float (&pre)[2], int i) __attribute__((always_inline)) -> float {
        return rdlf(i < 64 ? pre[0] : pre[1], i & 63);
      };
      bool zero = false;
      const bool renorm = !(cfg.top_p >= 1.0f);
      float sumc = 1.0f;
      if (renorm) {
        float pre[2];
        prefix(-0.0f, pre, INFINITY);  // the serial sum folds from -0.0 as Rust's f32 Sum does
        sumc = at(pre, k - 1);
        if (!(sumc > 0.0f)) {
          zero = true;  // all weights zero: truncate_top_p returns them unchanged
        } else {
          w[0] = __fdiv_rn(w[0], sumc);
          w[1] = __fdiv_rn(w[1], sumc);
        }
      }
      if (zero) {
        st = XS_ROW_ZERO_WEIGHT;
      } else {
        float c[2];
        prefix(0.0f, c, cfg.top_p >= 1.0f ? INFINITY : cfg.top_p);
        int keep = k;
        bool found = false;
        if (renorm) {
          const uint64_t b0m = __ballot(lane < k && c[0] >= cfg.top_p);
          const uint64_t b1m = __ballot(64 + lane < k && c[1] >= cfg.top_p);
          found = (b0m | b1m) != 0ull;
          keep = b0m ? (int)__builtin_ctzll(b0m) + 1 : (b1m ? 64 + (int)__builtin_ctzll(b1m) + 1 : k);
          if (lane >= keep) w[0] = 0.0f;
          if (64 + lane >= keep) w[1] = 0.0f;
        }
        const float tot = at(c, keep - 1);
        bool okw = !(lane < k && !(w[0] >= 0.0f)) && !(64 + lane < k && !(w[1] >= 0.0f));
        okw = __ballot(!okw) == 0;
        if (!okw || tot == 0.0f) {
          st = XS_ROW_ZERO_WEIGHT;
        } else {
          // cumulative weights cum[i] = prefix through i (i < keep - 1), the
          // total after it; the index is the number of them <= x
          const float x_draw = u_row * tot + 0.0f;
          const float cum0 = (lane < keep - 1) ? c[0] : tot;
          const float cum1 = (64 + lane < keep - 1) ? c[1] : tot;
          const int idx = (int)__popcll(__ballot(lane < k - 1 && cum0 <= x_draw)) +
                          (int)__popcll(__ballot(64 + lane < k - 1 && cum1 <= x_draw));
          tok = (int)pk_id(pick64(pk, idx));
          if (lazy_order) {
            // entries < k with the drawn entry's p: a contiguous run [lo, hi);
            // the id at position idx of its (id asc) order is the (idx - lo)-th
            // smallest id of the run, found by bisection over id bits
            const uint32_t pi = (uint32_t)(pick64(pk, idx) >> 32);
            const uint32_t ph0 = (uint32_t)(pk[0] >> 32), ph1 = (uint32_t)(pk[1] >> 32);
            const bool in0 = lane < k, in1 = 64 + lane < k;
            const int lo = (int)__popcll(__ballot(in0 && ph0 > pi)) + (int)__popcll(__ballot(in1 && ph1 > pi));
            const int hi = (int)__popcll(__ballot(in0 && ph0 >= pi)) + (int)__popcll(__ballot(in1 && ph1 >= pi));
            if (hi - lo > 1) {
              const bool r0 = in0 && ph0 == pi, r1 = in1 && ph1 == pi;
              const uint32_t i0 = pk_id(pk[0]), i1 = pk_id(pk[1]);
              const int t = idx - lo;
              uint32_t y = 0;  // the largest y with at most t run ids below it
              for (int bit = 30; bit >= 0; bit--) {
                const uint32_t c = y | (1u << bit);
                const int n = (int)__popcll(__ballot(r0 && i0 < c)) + (int)__popcll(__ballot(r1 && i1 < c));
                if (n <= t) y = c;
              }
              tok = (int)y;
            }
          }
          if (check)
            unsettled = unsettled || cfg.force ||
                        !draw_settled<2>(c, tot, x_draw, idx, keep, k, found, renorm, S, cfg.top_p);
        }
      }
    }
  }
  if (unsettled) {  // (nothing written) the workgroup sums the serial denominator
    if (lane == 0) {
      F.need_ser = 1;
      F.ser_ms = m_s;
    }
    return;
  }

  // held_row: the statistics for held_fold, which writes row_lse and the
  // top-n log-probs once the workgroup has folded the denominator; a row
  // refused for its top_k (no selection gathered) keeps the exact sum
  const bool lse_ok = !nan_seen && !__builtin_isinf(m_v);
  if (WANT_LSE && (a.row_lse || a.n_top > 0)) {
    const int nh = cfg.bad ? 0 : min(min(a.n_top, enc), nsel);
    if (lane == 0) {
      F.held.R_d = R_d;
      F.held.m_v = m_v;
      F.held.top = cfg.bad ? 0u : rdl(pk_id(sel[0]), 0);
      F.held.ok = lse_ok ? 1 : 0;
      F.held.can_fold = cfg.bad ? 0 : 1;
      F.held.n_have = nh;
    }
#pragma unroll
    for (int r = 0; r < 2; r++)
      if (r * 64 + lane < nh) F.held.vals[r * 64 + lane] = keyf(pk_key(sel[r]));
  }

  // Outputs.
  if (lane == 0) {
    if (!defer) {
      st_agent(&a.token[row], st == XS_ROW_OK ? tok : -1);
      st_agent(&a.status[row], st);
      if (a.n_cand) a.n_cand[row] = (stoch && st == XS_ROW_OK) ? k : 0;
    }
    if (a.soft_max) a.soft_max[row] = m_s;
    if (a.soft_sum) a.soft_sum[row] = S;
    if (WANT_LSE) {
      if (a.row_max) a.row_max[row] = m_v;
      if (a.p_max) a.p_max[row] = lse_ok ? (float)(1.0 / R_d) : __builtin_nanf("");
    }
    F.big.defer = defer ? 1 : 0;
    F.big.m_s = m_s;
    F.big.S = S;
    if (cfg.big && a.big_state) a.big_state[row] = BigRow{defer ? 1 : 0, m_s, S, k, 1.0f};
  }
  if (want_cands && stoch && st == XS_ROW_OK && !defer) {
    const int kw = (int)min((int64_t)k, a.cand_ld);  // a short cand_ld truncates the list
    // k >= enc on a row of at most KSEL ids, some of which the selection never
    // holds (-inf: masked or banned): the sort-everything branch lists every
    // id (candidate_set, sampler.rs:322-332), those at p = 0 in id order
    // after the g entries with p > 0
    const bool fill = cfg.full && nsel < k;
    int g = kw;
    if (fill) {
      if (lane < KSEL / 32) F.zmap[lane] = 0u;
      wave_lds_sync();
      int npos = 0;
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const bool pos = r * 64 + lane < nsel && (uint32_t)(pk[r] >> 32) != 0u;
        if (pos) {
          const uint32_t id = 0xFFFFFFFFu - (uint32_t)pk[r];
          atomicOr(&F.zmap[id >> 5], 1u << (id & 31));
        }
        npos += __popcll(__ballot(pos));
      }
      wave_lds_sync();
      g = min(npos, kw);
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int i = r * 64 + lane;
      if (i < g) {
        if (a.cand_id) a.cand_id[(int64_t)row * a.cand_ld + i] = (int32_t)(0xFFFFFFFFu - (uint32_t)pk[r]);
        if (a.cand_w) a.cand_w[(int64_t)row * a.cand_ld + i] = w[r];
      }
    }
    if (fill) {
      int below = 0;  // p = 0 ids of the earlier rounds
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const int i = r * 64 + lane;
        const bool zero = i < enc && !((F.zmap[i >> 5] >> (i & 31)) & 1u);
        const uint64_t zb = __ballot(zero);
        const int at = g + below + lanes_below(zb);
        if (zero && at < kw) {
          if (a.cand_id) a.cand_id[(int64_t)row * a.cand_ld + at] = i;
          if (a.cand_w) a.cand_w[(int64_t)row * a.cand_ld + at] = 0.0f;
        }
        below += __popcll(zb);
      }
    }
  }
  if (WANT_LSE && a.n_top > 0 && a.top_id) {
    const int nt = min(a.n_top, enc);
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int i = r * 64 + lane;
      if (i < a.n_top)
        a.top_id[(int64_t)row * a.top_ld + i] = (i < nt && i < nsel && !cfg.bad) ? (int32_t)pk_id(sel[r]) : -1;
    }
  }

}

// ---------------------------------------------------------------------------
// Row finalize, run by the first wave of the row's last workgroup (or of
// finalize_kernel's workgroup for the row).  First one round of coalesced
// agent-scope loads: the row's sub-record headers and first EPRE entries,
// sub-record `lane` per lane.  Every lane loads (its word lies inside the row's record: nsp >= 64),
// and the lanes past nsub drop what they read: unguarded loads all go out at
// once, where guarded ones were waited for in turn.
template <bool WANT_LSE, bool LOC>
XS_DEV void load_heads(const uint64_t* rowrec, int nsp, int nsub, uint64_t (&h)[NHW], uint64_t (&E)[EPRE]) {
  const int lane = lane_id();
  const bool live = lane < nsub;
#pragma unroll
  for (int i = 0; i < NHW; i++)  // (word 2, the held_row partial, only when it is read)
    h[i] = (i == 2 && !WANT_LSE) ? 0ull : ld_sub<LOC>(&rowrec[(uint32_t)(i * nsp + lane)]);
#pragma unroll
  for (int j = 0; j < EPRE; j++) E[j] = ld_sub<LOC>(&rowrec[(uint32_t)((SHDR + j) * nsp + lane)]);
#pragma unroll
  for (int i = 0; i < NHW; i++) h[i] = live ? h[i] : 0ull;
#pragma unroll
  for (int j = 0; j < EPRE; j++) E[j] = live ? E[j] : 0ull;
}

// Then fin_fast, or fin_general when the row falls outside the common case,
// from the headers load_heads read.  For a speculative block the
// row then takes its sequence's ticket, and the sequence's last finalized row
// walks it (accept_drafts).
template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL, bool LOC>
XS_DEV void finalize_heads(const Args& a, const Cfg& cfg, int row, const uint64_t* rowrec, int nsp,
                           int nsub, const float* rowp, const uint32_t* mrow, FinLds& F,
                           const uint64_t (&h)[NHW], const uint64_t (&E)[EPRE], float S_ser = -1.0f) {
  CtlRow cr{};
  if (HAS_CTL) cr = a.ctl_row[row];
  if (lane_id() == 0) F.need_ser = 0;
  const bool done = !(HAS_CTL && cr.active) && nsub <= 64 && cfg.kp <= 64 && !cfg.bad && !cfg.big &&
                    fin_fast<HAS_MASK, WANT_LSE, LOC>(a, cfg, row, nsub, h, E, rowrec, nsp, rowp, F, S_ser);
  if (!done) fin_general<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nsub, rowp, mrow, cr, h, E, F, S_ser);
}

template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL, bool LOC>
XS_DEV void finalize_row(const Args& a, const Cfg& cfg, int row, const uint64_t* rowrec, int nsp,
                         int nsub, const float* rowp, const uint32_t* mrow, FinLds& F,
                         float S_ser = -1.0f) {
  uint64_t h[NHW], E[EPRE];
  load_heads<WANT_LSE, LOC>(rowrec, nsp, nsub, h, E);
  finalize_heads<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nsub, rowp, mrow, F, h, E, S_ser);
}

// The speculative walk: a finalized row of a verify block takes its sequence's
// ticket, and the sequence's last finalized row walks accept_drafts
// (generate.rs:4020-4046) over the sequence's rows.  One wave, after the row's
// token and status are written.  The walk stops before row i when the budget
// is spent (i >= budget) or the row failed (its status then becomes the
// sequence's), and after committing row i when it is the bonus position, did
// not match its draft, is end-of-generation, or completes the grammar.  Lane l
// holds row b + l of each group of 64 (every load of a group in flight at
// once), and the first stop is the lowest lane of a ballot: every row before
// it matched its draft and was committed.
XS_DEV void verify_walk(const Args& a, int row) {
  const int lane = lane_id();
  drain();  // this row's token and status are acknowledged
  const int seq = row / a.span;
  int t = 0;
  if (lane == 0) t = __hip_atomic_fetch_add(&a.seq_ticket[seq * TSTRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  t = __builtin_amdgcn_readfirstlane(t);
  if (t != a.span - 1) return;
  if (lane == 0) st_agent(&a.seq_ticket[seq * TSTRIDE], 0);
  const int span = a.span, D = span - 1;
  const int64_t r0 = (int64_t)seq * span;
  const int bud = a.budget ? a.budget[seq] : 0x7FFFFFFF;
  int ncom = -1, mcount = 0, sst = XS_ROW_OK;
  int b = 0;
  for (; b < span && ncom < 0; b += 64) {
    const int i = b + lane;
    const int ic = min(i, span - 1);  // (clamped, not guarded: the loads go out together)
    const int rs = ld_agent(&a.status[r0 + ic]);
    const int s = ld_agent(&a.token[r0 + ic]);
    const int dr = D > 0 ? a.drafts[(int64_t)seq * D + min(ic, D - 1)] : 0;
    const bool fin = a.done_after != nullptr && a.done_after[r0 + ic] != 0;
    bool eog = false;
    for (int e = 0; e < a.n_eog; e++) eog |= (s == a.eog[e]);
    const bool in = i < span;
    const bool matched = i < D && s == dr;
    const bool before = in && (i >= bud || rs != XS_ROW_OK);
    const bool after = in && !before && (!matched || eog || fin);
    const uint64_t bb = __ballot(before), stop = bb | __ballot(after);
    int lim = 0x7FFFFFFF;  // rows of this group below lim are committed
    if (stop) {
      const int f = (int)__builtin_ctzll(stop);
      if ((bb >> f) & 1ull) {
        ncom = b + f;
        mcount = b + f;
        const int rsf = __builtin_amdgcn_readlane(rs, f);
        if (b + f < bud) sst = rsf;
      } else {
        ncom = b + f + 1;
        mcount = b + f + ((__ballot(matched) >> f) & 1ull ? 1 : 0);
      }
      lim = ncom;
    }
    if (in) a.committed[r0 + i] = i < lim ? s : -1;
  }
  for (; b < span; b += 64)
    if (b + lane < span) a.committed[r0 + b + lane] = -1;
  if (lane == 0) {
    a.accepted[seq] = mcount;
    a.n_committed[seq] = ncom;
    a.seq_status[seq] = sst;
  }
}

// radix_sort_desc's counters.
struct SortLds {
  uint32_t cnt[16][BLOCK];          // per digit, per thread: count, then write position
  int32_t s4[NWAVE];
};

// Stable LSD radix sort of n u64 entries by their high 32 bits, descending;
// src holds the result afterwards (an even number of passes).  All waves.
XS_DEV void radix_sort_desc(uint64_t* src, uint64_t* dst, int n, SortLds& B) {
  const int t = threadIdx.x;
  const int L = (n + BLOCK - 1) / BLOCK;
  const int i0 = min(n, t * L), i1 = min(n, i0 + L);
#pragma unroll 1
  for (int pass = 0; pass < 8; pass++) {
    const int sh = 4 * pass;
#pragma unroll
    for (int d = 0; d < 16; d++) B.cnt[d][t] = 0u;
#pragma unroll 4
    for (int i = i0; i < i1; i++) B.cnt[((~(uint32_t)(src[i] >> 32)) >> sh) & 15u][t]++;
    __syncthreads();
    // exclusive scan in (digit, thread) order: thread t owns flat entries 16t..16t+15
    uint32_t* flat = &B.cnt[0][0];
    uint32_t loc[16], sum = 0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      loc[j] = flat[16 * t + j];
      sum += loc[j];
    }
    int total;
    uint32_t run = (uint32_t)block_excl_scan((int)sum, B.s4, &total);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      flat[16 * t + j] = run;
      run += loc[j];
    }
    __syncthreads();
#pragma unroll 4
    for (int i = i0; i < i1; i++) {
      const uint64_t e = src[i];
      const uint32_t d = ((~(uint32_t)(e >> 32)) >> sh) & 15u;
      dst[B.cnt[d][t]++] = e;
    }
    __syncthreads();
    uint64_t* const tmp = src;
    src = dst;
    dst = tmp;
  }
}

// The finalizing wave left the row to the whole-row kernels (which then walk
// its verify block once they have drawn it).
XS_DEV bool deferred(const Cfg& cfg, const FinLds& F) {
  wave_lds_sync();  // lane 0 wrote the stash
  return cfg.big && !cfg.bad && F.big.defer != 0;
}

// ---------------------------------------------------------------------------
// The serial denominator.  On a controlled row (an allow-mask or active sparse
// controls) the reference adds the softmax terms one at a time in f32, in id
// order, from +0 (softmax_in_place, sampler.rs:301-305), and at top_p >= 1
// the candidate weights p = e / sum reach the caller unrenormalized: that sum
// is reproduced bit for bit.
//
// The terms are >= 0, so the running sum s never falls, and while s stays in
// one binade [2^b, 2^(b+1)) every addition rounds its term to that binade's
// grid 2^(b-23): fl(s + e) = s + rn(e / grid) * grid, which adds an integer to
// s's bit pattern (subnormal s: the grid 2^-149).  serial_kernel cuts the row
// into segments of SEG ids (one wave's float4s of one slot) and sums, per
// segment, its terms in grid units of the binade the exact sum before the
// segment lies in -- and of the binade below too when that sum lies within
// SER_DELTA above a power of two: the serial sum stays within a fraction of a
// percent of the exact one -- noting any term exactly half-way between two
// grid points, whose rounding (half to even) depends on s itself.  A term's
// units come from a short f32 exp whose error bound settles almost all of
// them; a term the bound leaves open, or a subnormal one, is recomputed
// correctly rounded.  The row's last workgroup walks the segments in order: a
// segment whose summary holds s's binade, with no half-way term, and whose
// units keep s below the next binade adds them to s's bits; any other
// segment adds units up to its first term that carries or ties, and from
// there its terms one at a time in f32, as the reference does.  Segments
// where the exact sum may pass a power of two, or that hold a half-way term,
// keep their correctly rounded terms in a side buffer for that.
constexpr uint32_t GSAT = 1u << 23;    // grid units that always carry into the next binade
constexpr int SER_NB = 64;             // segments per row whose terms are kept
constexpr int SER_WIN = 1024;          // segment summaries the walk stages at a time
constexpr int SER_LDS = 32;            // kept segments staged in LDS
constexpr double SER_DELTA = 1.0 / 512;  // margin on the exact prefix for a binade change
constexpr float LOG2E_LO = 1.925963033500011e-08f;  // log2(e) - LOG2E
constexpr float LN2F = 0.6931471805599453f;
// summary word 1, high half: the lower binade's exponent field, a half-way
// term at it (bit 8) or at the next binade (9), units of that next binade
// present (10), every term +0 (11), and 1 + the kept-terms slot (16..)
constexpr uint32_t SM_TIE0 = 1u << 8, SM_TIE1 = 1u << 9, SM_TWO = 1u << 10, SM_ZERO = 1u << 11;

// A row that serial_kernel finalizes: stochastic and controlled, and either
// at top_p >= 1 in a call that observes the denominator (the weights reach
// the caller unrenormalized), or drawn by the whole-row kernels (whose
// order of every p follows the denominator).  The other controlled rows are
// finalized with the exact sum and checked (draw_settled).
template <bool HAS_MASK, bool HAS_CTL>
XS_DEV bool serial_row(const Args& a, const Cfg& cfg, int row) {
  if (cfg.greedy || cfg.bad) return false;
  if (!(((a.serial & 1) && cfg.top_p >= 1.0f) || ((a.serial & 2) && cfg.big))) return false;
  if (HAS_MASK) return true;
  return HAS_CTL && a.ctl_row[row].active != 0;
}

// rn(e / grid) of a term e >= 0 (bits eb) at the grid of binade field F
// (the f32 exponent field, 0 for subnormals), saturated at GSAT; *tie when e
// lies exactly half-way between two grid points.  Branch-free.
XS_DEV uint32_t grid_units(uint32_t eb, int F, bool& tie) {
  const int c = (int)(eb >> 23);
  const uint32_t M = (eb & 0x7FFFFFu) | (c ? 0x800000u : 0u);
  const int k = max(F, 1) - max(c, 1);     // bits of e below the grid
  const int ks = min(max(k, 1), 31);
  const uint32_t half = 1u << (ks - 1);
  const uint32_t rem = M & ((half << 1) - 1u);
  const uint32_t rq = (M >> ks) + (rem > half ? 1u : 0u);  // 0 once k > 24
  tie = k >= 1 && rem == half;
  return min(k < 0 ? GSAT : (k == 0 ? M : rq), GSAT);
}

XS_DEV int f32_field(float f) { return (int)(__float_as_uint(f) >> 23); }

// grid_units of a term w >= 0 in float operations, the same value and tie
// flag: w scaled onto the grid (by 2^(150 - F), exact: a multiple of the grid
// below 2^24 stays normal), its floor and fraction, both exact.  A term the
// scaling makes subnormal rounds to 0 units either way.
XS_DEV uint32_t grid_units_f(float w, int F, bool& tie) {
  const float v = __builtin_ldexpf(w, 150 - max(F, 1));
  const float fl = __builtin_floorf(v);
  const float fr = v - fl;
  tie = fr == 0.5f;
  return min((uint32_t)fminf(fl, (float)GSAT) + (fr > 0.5f ? 1u : 0u), GSAT);
}

// exp(d), d <= 0: within 2^-21 of the correctly rounded f32 value for
// d >= -87 (d * log2e split in two, v_exp_f32 on the high part, a first-order
// correction for the low one)
XS_DEV float fast_expf(float d) {
  const float dc = fmaxf(d, -200.0f);  // -inf: 0, not a NaN
  const float hi = dc * LOG2E;
  const float lo = __builtin_fmaf(dc, LOG2E, -hi) + dc * LOG2E_LO;
  const float e2 = xexp2(hi);
  return e2 + e2 * (lo * LN2F);
}

// rn(e / grid) at binade field F from an estimate ef within 2^-21 of e; false
// when that bound cannot settle it (a value near a grid midpoint, or 2^20
// units and more)
XS_DEV bool fast_units(float ef, int F, uint32_t& r) {
  const float u = __builtin_ldexpf(ef, 150 - max(F, 1));
  const float fl = __builtin_floorf(u);
  const float fr = u - fl;
  r = (uint32_t)fminf(fl, (float)GSAT) + (fr > 0.5f ? 1u : 0u);
  return u < 0x1p20f && __builtin_fabsf(fr - 0.5f) > u * 0x1p-19f + 0x1p-60f;
}

// The sparse controls of one slot (first id sb) on the thread whose float4
// is pos: the forced id alone, or the slot's patches (final values, sorted by
// id, read from pc on; patches of earlier slots are passed over) and then the
// pulled id.
XS_DEV void ctl_slot(float (&x)[4], int sb, int pos, const uint64_t* pl, int& pc, int phi, int pull,
                     float pval, int force, float fval) {
  if (force >= 0) {
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = (sb + 4 * pos + e == force) ? fval : -INFINITY;
    return;
  }
  while (pc < phi) {
    const uint64_t pe = pl[pc];
    const int off = (int)(uint32_t)(pe >> 32) - sb;
    if (off >= SLOT) break;
    if (off >= 0 && (off >> 2) == pos) {
      const float pv = __uint_as_float((uint32_t)pe);
#pragma unroll
      for (int e = 0; e < 4; e++) x[e] = ((off & 3) == e) ? pv : x[e];
    }
    pc++;
  }
  const int pt = pull - sb;
  if (pt >= 0 && pt < SLOT && (pt >> 2) == pos) {
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = ((pt & 3) == e) ? pval : x[e];
  }
}

// The softmax terms of segment g, this lane's four: exp(v * inv - max) of the
// masked and controlled values, correctly rounded (the walk's rare recount of
// a segment whose terms were not kept).
template <bool HAS_MASK, bool HAS_CTL>
XS_DEV void seg_terms(const Args& a, const Cfg& cfg, int row, int g, float m_s, const double* T,
                      float (&ev)[4]) {
  const int lane = lane_id();
  const int enc = (int)a.enc;
  const int slot = g >> 2, w = g & 3;
  const int sb = slot * SLOT, pos = 64 * w + lane, id0 = sb + 4 * pos;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int f = min(id0 >> 2, (enc - 1) >> 2);
  const float4 q = reinterpret_cast<const float4*>(rowp)[f];
  float x[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int id = id0 + e;
    if (id >= enc) x[e] = -INFINITY;
    else if (HAS_MASK && !((a.allowed[(int64_t)row * a.allowed_ld + (id >> 5)] >> (id & 31)) & 1u)) x[e] = -INFINITY;
  }
  if (HAS_CTL) {
    const CtlRow cr = a.ctl_row[row];
    if (cr.active) {
      const int chunk = slot / SPC;
      int pc = a.ctl_chunk[(int64_t)row * (a.n_chunks + 1) + chunk];
      const int phi = a.ctl_chunk[(int64_t)row * (a.n_chunks + 1) + chunk + 1];
      ctl_slot(x, sb, pos, a.patch + (int64_t)row * a.ctl_cap, pc, phi, cr.pull_id, cr.pull_val, cr.force_id,
               cr.force_val);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) ev[e] = cr_expf((cfg.scale ? x[e] * cfg.inv : x[e]) - m_s, T);
}

// The queued terms of one wave (qd, qt of the LDS struct L): each correctly
// rounded, its units and half-way flags added to its segment's summary (LDS
// atomics).
template <typename L_T>
XS_DEV void ser_flush_t(L_T& L, int wave, int n, const double* T) {
  const int lane = lane_id();
  wave_lds_sync();  // the queue and the segments' binades are written
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    if (i < n) {
      const int t = L.qt[wave][i];
      const float e = cr_expf(L.qd[wave][i], T);
      const uint32_t mt = L.meta[t];
      const int FB = (int)(mt & 0xFFu);
      bool t0, t1 = false;
      atomicAdd(&L.R[t][0], grid_units(__float_as_uint(e), FB, t0));
      if (mt & SM_TWO) atomicAdd(&L.R[t][1], grid_units(__float_as_uint(e), FB + 1, t1));
      if (t0 || t1) atomicOr(&L.meta[t], (t0 ? SM_TIE0 : 0u) | (t1 ? SM_TIE1 : 0u));
    }
  }
  wave_lds_sync();
}

// One segment added to the running sum's bits sb, its SEG terms at evp (LDS,
// in id order): grid units up to the first term that carries into the next
// binade or lies half-way, that term by the f32 add (the reference's own
// operation), then grid units again at the sum's new binade; after a few
// such terms, the rest one at a time by f32 adds.  One wave.
XS_DEV uint32_t ser_segment(uint32_t sb, const float* evp) {
  const int lane = lane_id();
  const float4 e4 = reinterpret_cast<const float4*>(evp)[lane];
  const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
  int from = 0;  // the first term not yet added (uniform)
#pragma unroll 1
  for (int round = 0; round < 4; round++) {
    const uint32_t F = sb >> 23, m = F ? (sb & 0x7FFFFFu) : sb;
    uint32_t p[4], P = 0;
    bool tie[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      bool t;
      const uint32_t u = grid_units(__float_as_uint(ev[k]), (int)F, t);
      const bool live = 4 * lane + k >= from;  // (terms before `from` are added)
      P += live ? u : 0u;
      p[k] = P;
      tie[k] = live && t;
    }
    const uint32_t Pc = min(P, GSAT);
    const uint32_t incl = (uint32_t)wave_incl_scan((int)Pc);
    const uint32_t excl = incl - Pc;
    int kf = 4;  // this lane's first term that carries or ties
#pragma unroll
    for (int k = 3; k >= 0; k--)
      if (tie[k] || m + excl + p[k] >= GSAT) kf = k;
    const uint64_t bm = __ballot(kf < 4);
    if (!bm) return sb + rdl(incl, 63);
    const int L = (int)__builtin_ctzll(bm);
    uint32_t before = excl;  // units before that term
#pragma unroll
    for (int k = 1; k < 4; k++) before = (kf == k) ? excl + p[k - 1] : before;
    sb += rdl(before, L);
    const int t = 4 * L + (int)rdl((uint32_t)kf, L);
    sb = __float_as_uint(__uint_as_float(sb) + evp[t]);
    from = t + 1;
    if (from >= SEG) return sb;
  }
  float s = __uint_as_float(sb);
  if (lane == 0) {
#pragma unroll 8
    for (int i = from; i < SEG; i++) s = s + evp[i];
  }
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(s));
}

// The walk over segments w0 .. w0 + wn - 1 of a row (their summaries staged
// in sum), from the running sum's bits sb.  One wave; lane i holds the
// summary of the i-th segment of each group of 64.  A segment added term by
// term has its terms in LDS (evl[0 .. nbl)), or copied from the side buffer,
// or recounted from the logits, into scr (one segment of LDS).
template <bool HAS_MASK, bool HAS_CTL>
XS_DEV uint32_t ser_walk(const Args& a, const Cfg& cfg, int row, uint32_t sb, const uint64_t (*sum)[2], int w0,
                         int wn, float (*evl)[SEG], int nbl, const uint64_t* skeep, float m_s, const double* T,
                         float* scr) {
  const int lane = lane_id();
#pragma unroll 1
  for (int b0 = 0; b0 < wn; b0 += 64) {
    const int i = b0 + lane;
    const bool v = i < wn;
    const uint64_t u01 = v ? sum[i][0] : 0ull, u1m = v ? sum[i][1] : 0ull;
    const uint32_t meta = (uint32_t)(u1m >> 32);
    const bool zero = (meta & SM_ZERO) != 0;  // a segment of +0 terms adds nothing at any grid
    const int nl = min(64, wn - b0);
    int cur = 0;  // the first segment of the group not yet added
#pragma unroll 1
    while (cur < nl) {
      const uint32_t F = sb >> 23, m = F ? (sb & 0x7FFFFFu) : sb;
      const int d = (int)F - (int)(meta & 0xFFu);
      const bool okd = zero || (d == 0 && !(meta & SM_TIE0)) ||
                       (d == 1 && (meta & SM_TWO) && !(meta & SM_TIE1));
      uint32_t r = d == 0 ? (uint32_t)u01 : (uint32_t)(u01 >> 32);
      r = zero ? 0u : (okd ? min(r, GSAT) : GSAT);
      if (lane < cur || !v) r = 0;
      const uint32_t inc = (uint32_t)wave_incl_scan((int)r);
      const uint64_t bm = __ballot(v && lane >= cur && (!okd || m + inc >= GSAT));
      if (!bm) {
        sb += rdl(inc, 63);
        break;
      }
      const int f = (int)__builtin_ctzll(bm);
      if (f > 0) sb += rdl(inc, f - 1);
      const int kept = (int)(rdl(meta, f) >> 16);
      const float* evp;
      if (kept > 0 && kept <= nbl) {
        evp = evl[kept - 1];
      } else {
        float ev[4];
        if (kept > 0) {
          const uint64_t* src = skeep + (int64_t)(kept - 1) * (SEG / 2) + 2 * lane;
          const uint64_t e01 = ld_agent(src), e23 = ld_agent(src + 1);
          ev[0] = __uint_as_float((uint32_t)e01);
          ev[1] = __uint_as_float((uint32_t)(e01 >> 32));
          ev[2] = __uint_as_float((uint32_t)e23);
          ev[3] = __uint_as_float((uint32_t)(e23 >> 32));
        } else {
          seg_terms<HAS_MASK, HAS_CTL>(a, cfg, row, w0 + b0 + f, m_s, T, ev);
        }
        reinterpret_cast<float4*>(scr)[lane] = make_float4(ev[0], ev[1], ev[2], ev[3]);
        wave_lds_sync();
        evp = scr;
      }
      sb = ser_segment(sb, evp);
      wave_lds_sync();  // (the scratch row is rewritten by the next recount)
      cur = f + 1;
    }
  }
  return sb;
}


// ---------------------------------------------------------------------------
// The serial denominator of one row, summed by the wave that finalizes it:
// the fallback for a controlled row whose token the exact sum does not settle
// (order_settled, draw_settled), rare by construction.  Chunk after chunk it
// does serial_kernel's per-chunk work -- each term's exp argument, the exact
// sums and prefixes of the chunk's 64 segments, their grid units at the
// binades those prefixes lie in, the half-way flags -- then walks the
// chunk's segments onto the running serial sum (ser_walk; a segment its
// summary does not settle is recounted from the logits).  One wave does it
// all, so the workgroup's other waves need not stay for the finalizer's
// verdict; the logits are read once per phase, four segments at a time.
template <bool HAS_MASK, bool HAS_CTL>
XS_DEV float ser_local(const Args& a, const Cfg& cfg, int row, float m_s, SerLocal& L) {
  constexpr int NB = 4;  // segments loaded at a time
  constexpr int NSEG = SPC * NWAVE;  // segments per chunk
  const int lane = lane_id();
  const int enc = (int)a.enc, nc = a.n_chunks;
  const v4f* rp4 = reinterpret_cast<const v4f*>(a.logits + (int64_t)row * a.ld);
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  const int fmax = (enc - 1) >> 2;
  CtlRow cr{};
  if (HAS_CTL) cr = a.ctl_row[row];
  const bool ctl_on = HAS_CTL && cr.active;
  const uint64_t* pl = ctl_on ? a.patch + (int64_t)row * a.ctl_cap : nullptr;
  L.expt[lane] = (&kExpT[0][0])[lane];
  double X = 0.0;   // exact sum of the chunks walked so far
  uint32_t sb = 0;  // the serial sum's bits after them, from +0
  wave_lds_sync();
#pragma unroll 1
  for (int chunk = 0; chunk < nc; chunk++) {
    const int s0 = chunk * SPC;
    const int nseg = min(SPC, a.nslots - s0) * NWAVE;  // segment t: slot t / NWAVE, quarter t % NWAVE
    const int pc0 = ctl_on ? a.ctl_chunk[(int64_t)row * (nc + 1) + chunk] : 0;
    const int phi = ctl_on ? a.ctl_chunk[(int64_t)row * (nc + 1) + chunk + 1] : 0;
    v4f q[NB];
    uint32_t mw[NB];
    auto load = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < NB; u++) {
        const int t = tb + u;  // (clamped: segments past nseg are not used)
        const int f = min((s0 + t / NWAVE) * BLOCK + (t % NWAVE) * 64 + lane, fmax);
        q[u] = rp4[f];
        if (HAS_MASK) mw[u] = mrow[f >> 3];
      }
    };
    // the exp arguments d = v * inv - max of segment t's float4 on this lane,
    // the values masked and controlled as the streaming pass saw them (each
    // slot's patches scanned from the slot's first, once per quarter)
    int pc = pc0, pc_slot = pc0;
    auto args = [&](int t, int u, float (&dv)[4]) __attribute__((always_inline)) {
      const int j = t / NWAVE, pos = (t % NWAVE) * 64 + lane;
      float x[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
      if (HAS_MASK) {
        const uint32_t bits = mw[u] >> ((((s0 + j) * BLOCK + pos) & 7) * 4);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (!((bits >> e) & 1u)) x[e] = -INFINITY;
      }
      if ((s0 + j + 1) * SLOT > enc) {
        const int id0 = (s0 + j) * SLOT + 4 * pos;
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (id0 + e >= enc) x[e] = -INFINITY;
      }
      if (ctl_on) {
        if (t % NWAVE == 0) pc_slot = pc;
        pc = pc_slot;
        ctl_slot(x, (s0 + j) * SLOT, pos, pl, pc, phi, cr.pull_id, cr.pull_val, cr.force_id, cr.force_val);
      }
#pragma unroll
      for (int e = 0; e < 4; e++) dv[e] = (cfg.scale ? x[e] * cfg.inv : x[e]) - m_s;
    };
    // 1. each segment's exact sum (short exp); a segment whose terms all lie
    //    below -104 adds +0 at any grid
#pragma unroll 1
    for (int tb = 0; tb < NSEG; tb += NB) {
      if (tb < nseg) load(tb);
#pragma unroll
      for (int u = 0; u < NB; u++) {
        const int t = tb + u;
        double ssum = 0.0;
        bool any = false;
        if (t < nseg) {
          float dv[4], tt = 0.0f;
          args(t, u, dv);
#pragma unroll
          for (int e = 0; e < 4; e++) tt += fast_expf(dv[e]);
          ssum = wave_sumd((double)tt);
          any = __ballot(dv[0] >= -104.0f || dv[1] >= -104.0f || dv[2] >= -104.0f || dv[3] >= -104.0f) != 0;
        }
        if (lane == 0) {
          L.segsum[t] = ssum;
          L.meta[t] = any ? 0u : SM_ZERO;
          L.R[t][0] = 0u;
          L.R[t][1] = 0u;
        }
      }
    }
    wave_lds_sync();
    // 2. the exact sum before each segment (lane t), in row order
    double ctot;
    {
      double inc = L.segsum[lane];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const double t = __shfl_up(inc, d);
        if (lane >= d) inc += t;
      }
      const double ex = __shfl_up(inc, 1);
      L.segpre[lane] = X + (lane == 0 ? 0.0 : ex);
      ctot = __shfl(inc, 63);
    }
    wave_lds_sync();
    // 3. each segment's grid units at the binade its prefix lies in (and the
    //    next, near a power of two), from the short exp where its error bound
    //    settles them, else queued for the correctly rounded one
    pc = pc_slot = pc0;
    int qn = 0;
#pragma unroll 1
    for (int tb = 0; tb < NSEG; tb += NB) {
      if (tb < nseg) load(tb);
#pragma unroll
      for (int u = 0; u < NB; u++) {
        const int t = tb + u;
        if (t < nseg) {
          const double X0 = L.segpre[t];
          const int FB = f32_field((float)(X0 * (1.0 - SER_DELTA)));
          const bool two = f32_field((float)(X0 * (1.0 + SER_DELTA))) != FB;
          if (lane == 0) L.meta[t] |= (uint32_t)FB | (two ? SM_TWO : 0u);
          float dv[4];
          args(t, u, dv);
          uint32_t r0 = 0, r1 = 0;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float ef = fast_expf(dv[e]);
            uint32_t u0, u1 = 0;
            bool settled = fast_units(ef, FB, u0);
            if (two) settled = fast_units(ef, FB + 1, u1) && settled;
            const bool amb = !(dv[e] < -104.0f) && (!settled || dv[e] < -87.0f);
            if (!amb) {
              r0 += u0;
              r1 += u1;
            }
            const uint64_t b = __ballot(amb);
            if (b) {
              if (qn + 64 > SER_QCAP) {
                ser_flush_t(L, 0, qn, L.expt);
                qn = 0;
              }
              const int pos = qn + lanes_below(b);
              if (amb) {
                L.qd[0][pos] = dv[e];
                L.qt[0][pos] = (uint8_t)t;
              }
              qn += __popcll(b);
            }
          }
          const uint32_t s0u = wave_sum_u32(r0), s1u = wave_sum_u32(r1);
          if (lane == 0) {
            atomicAdd(&L.R[t][0], s0u);
            atomicAdd(&L.R[t][1], s1u);
          }
        }
      }
    }
    ser_flush_t(L, 0, qn, L.expt);
    // 4. the chunk's segments onto the running sum, in order
    L.sum[lane][0] = (uint64_t)L.R[lane][0] | ((uint64_t)L.R[lane][1] << 32);
    L.sum[lane][1] = (uint64_t)L.meta[lane] << 32;
    wave_lds_sync();
    sb = ser_walk<HAS_MASK, HAS_CTL>(a, cfg, row, sb, L.sum, s0 * NWAVE, nseg, nullptr, 0, nullptr, m_s, L.expt,
                                     L.scr);
    X += ctot;
    wave_lds_sync();
  }
  return __uint_as_float(sb);
}

// After the finalizing wave's finalize_row: when it left a controlled row
// unsettled (F.need_ser), the wave sums the row's serial denominator
// (ser_local) and finalizes the row again with it, which settles it by
// construction.  Rows sent here are counted.
template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL, bool LOC>
XS_DEV void ser_fallback(const Args& a, const Cfg& cfg, int row, const uint64_t* rowrec, int nsp, int nsub,
                         const float* rowp, const uint32_t* mrow, TailLds& Tl) {
  wave_lds_sync();  // lane 0 wrote the verdict
  if (!Tl.fin.need_ser) return;
  const float m_s = Tl.fin.ser_ms;
  wave_lds_sync();  // read before ser_local reuses the memory
  const float S_ser = ser_local<HAS_MASK, HAS_CTL>(a, cfg, row, m_s, Tl.ser);
  if (lane_id() == 0 && a.ser_count) atomicAdd(a.ser_count, 1u);
  // The record's address and stride pass through an empty asm statement, so
  // the compiler forms this finalize_row's addresses afresh instead of
  // keeping the first one's live across it (18 such registers spilled to
  // scratch in the masked and controlled kernels).
  // (both made uniform first, so the scalar-register constraint always holds)
  const uint64_t ra = reinterpret_cast<uint64_t>(rowrec);
  const uint64_t* rr = reinterpret_cast<const uint64_t*>(
      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(ra >> 32)) << 32) |
      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ra));
  int np = __builtin_amdgcn_readfirstlane(nsp);
  asm volatile("" : "+s"(rr), "+s"(np));
  finalize_row<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rr, np, nsub, rowp, mrow, Tl.fin, S_ser);
}

// The row's arrival ticket counts its workgroups (bits 0-7; a row has at most
// GMAX * 64 / NWAVE = 64 chunks) and sums their XCDs x (bits 8-17, at most
// 64 * 15) and x^2 (bits 18-31, at most 64 * 225): the fields never carry
// into each other.  The last workgroup, on XCD y, holds the totals of all nc
// workgroups; sum x = nc y and sum x^2 = nc y^2 make sum (x - y)^2 = 0, so
// every workgroup of the row ran on XCD y and its sub-records are in y's L2.
XS_DEV uint32_t row_ticket_add(uint32_t x) { return 1u | (x << 8) | ((x * x) << 18); }
XS_DEV bool row_on_one_xcd(uint32_t total, int nc, uint32_t y) {
  return ((total >> 8) & 0x3FFu) == (uint32_t)nc * y && (total >> 18) == (uint32_t)nc * y * y;
}

// ---------------------------------------------------------------------------
// The kernel.  Grid (LOC, the XCD-local hand-off): groups of n = 2^xcd_log2
// rows x n_chunks workgroups of BLOCK lanes (the row count rounded up to whole
// groups; workgroups past the last row return at once); chunk c of a row
// covers slots [c*SPC, c*SPC + SPC).  The hardware hands workgroup b of a
// launch to XCD b mod n (round robin over the device's n XCDs, measured on
// every launch shape), so workgroup (g*nc + c)*n + r takes chunk c of row
// g*n + r: all of a row's workgroups run on one XCD.  Without LOC the grid is
// row-major, rows x n_chunks, and a row's workgroups spread over the XCDs.
// Every wave reduces its own share of the chunk and publishes it as one
// sub-record; the row's last workgroup to arrive (an atomic ticket per row)
// finalizes the row with its first wave.

template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL, bool ORD, bool LOC>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(4, 8))) void sample_kernel(Args a, RowOrder<ORD> ro) {
  __shared__ ChunkLds Lc;
  __shared__ TailLds Tl;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int nc = a.n_chunks;
  int rb, chunk;
  if constexpr (LOC) {
    const int gc = (int)(blockIdx.x >> a.xcd_log2);  // (group, chunk) of the workgroup
    const int grp = gc / nc;
    chunk = gc - grp * nc;
    rb = (grp << a.xcd_log2) | (int)(blockIdx.x & ((1u << a.xcd_log2) - 1u));
    if (rb >= a.nrows) return;  // the last group's padding
  } else {  // row-major, no padding
    rb = blockIdx.x / nc;
    chunk = blockIdx.x - rb * nc;
  }
  int row = rb;
  if constexpr (ORD) row = ro.v[rb];
  const int enc = (int)a.enc;

  // ---------------- chunk pass ----------------
  const int s0 = chunk * SPC;
  const int ns = min(SPC, a.nslots - s0);
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const v4f* rp4 = reinterpret_cast<const v4f*>(rowp);
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  const int fmax = (enc - 1) >> 2;  // last float4 holding an encodable id

  // Every load is unconditional (clamped to the row's last float4), so the
  // compiler can wait for them one at a time, in order, while the arithmetic
  // below runs on the ones that have arrived.
  v4f q[SPC];
  uint32_t mw[SPC];
#pragma unroll
  for (int j = 0; j < SPC; j++) {
    const int f = min((s0 + j) * BLOCK + tid, fmax);
    q[j] = __builtin_nontemporal_load(rp4 + f);
    if (HAS_MASK) mw[j] = mrow[f >> 3];
  }
  // The row's parameters are read only now, so that round trip overlaps the
  // loads instead of delaying them.
  const Cfg cfg = a.greedy_all ? greedy_cfg(a.n_top, a.enc) : make_cfg(a.params[row], a.enc, a.n_top, a.k_max, a.ser_force);
  const bool stoch = !cfg.greedy && !cfg.bad;
  const int kp = cfg.kp;
  // Sparse controls: the chunk's patches (final values written by
  // control_kernel), the pulled id, or the forced id.
  int pc = 0, phi = 0, ctl_pull = -1, ctl_force = -1;
  float ctl_pval = 0.0f, ctl_fval = 0.0f;
  const uint64_t* pl = nullptr;
  if (HAS_CTL) {
    const CtlRow cr = a.ctl_row[row];
    pc = a.ctl_chunk[(int64_t)row * (nc + 1) + chunk];
    phi = a.ctl_chunk[(int64_t)row * (nc + 1) + chunk + 1];
    pl = a.patch + (int64_t)row * a.ctl_cap;
    ctl_pull = cr.pull_id;
    ctl_pval = cr.pull_val;
    ctl_force = cr.force_id;
    ctl_fval = cr.force_val;
  }
  const int pc0 = pc;  // the chunk's first patch

  // Online reduction, one float4 at a time, branch-free.  The softmax partial
  // is summed in the reference's scaled domain, s = v * inv rounded to f32 as
  // softmax_in_place does (inv_e = 1 on rows with T = 1, where s = v: a
  // uniform multiplier instead of a branch per float4), as sum
  // exp2(s*log2e - cL) with a per-lane offset cL = rn(c*log2e), c the lane's
  // first scaled float4 max (0 if that is not finite).  A lane whose max
  // sits more than 40 above c is summed again after the loop against its max:
  // that keeps the f32 exponent of a lane's largest term below 64, where half
  // an ulp is 1.3e-6 relative (at 60, an LLM-like row whose top token stands
  // far above the bulk reached 5e-6), and no term can overflow.  The lanes are
  // combined at the wave max with the factor 2^(cL - c_w*log2e), its exponent
  // formed in f64 (exact for the product of two floats) and applied as
  // 2^n * 2^f, |f| <= 1/2, so it adds no rounding of its own.  A NaN, or a
  // +inf value (inf - inf at the recount), makes the sum NaN: the stochastic
  // NaN test.  The four terms of a float4 are added pairwise.
  //
  // The held_row partial (raw logits, f64 like the reference's denominator)
  // is summed after the loop against the lane's max instead, so the largest
  // term is exactly exp2(0) = 1 and the others, far smaller, accumulate in
  // f64 without being absorbed: ln of a near-1 sum stays accurate to ~1e-15.
  // (A running max rescaled at every float4 cost C5 1.8 us more.)
  const float inv = cfg.inv;
  const float inv_e = cfg.scale ? inv : 1.0f;
  float mr = -INFINITY;
  float gm[SPC];
  float sum = 0.0f, cL = 0.0f, c_s = 0.0f;
  double racc = 0.0;
  float rc = -__FLT_MAX__;
  uint32_t nanl = 0;
  // The loop comes in four copies, so that the uniform tests leave the
  // per-float4 path where they can: EDGE for a chunk with absent or partial
  // slots (the row's last), STOCH for a stochastic row of a chunk without
  // them, and UNIT for such a row at T = 1, whose s = v * 1 is v itself (for
  // every float, NaN and -0 included) and needs no multiply.  Masked and
  // controlled rows keep one copy (a second one spills).
  auto stream = [&](auto edge_c, auto stoch_c, auto unit_c) __attribute__((always_inline)) {
    constexpr bool EDGE = decltype(edge_c)::value, STOCH = decltype(stoch_c)::value;
    constexpr bool UNIT = decltype(unit_c)::value;
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      float x[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
      if (HAS_MASK) {
        const uint32_t bits = mw[j] >> ((((s0 + j) * BLOCK + tid) & 7) * 4);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (!((bits >> e) & 1u)) x[e] = -INFINITY;
      }
      if (EDGE && (j >= ns || (s0 + j + 1) * SLOT > enc)) {  // absent or partial slot
        const int id0 = (s0 + j) * SLOT + 4 * tid;
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (j >= ns || id0 + e >= enc) x[e] = -INFINITY;
      }
      if (HAS_CTL) {
        const int sb = (s0 + j) * SLOT;
        if (ctl_force >= 0) {
#pragma unroll
          for (int e = 0; e < 4; e++) x[e] = (sb + 4 * tid + e == ctl_force) ? ctl_fval : -INFINITY;
        } else {
          // this slot's patches: the next ones in the sorted list
          while (pc < phi) {
            const uint64_t pe = pl[pc];
            const int off = (int)(uint32_t)(pe >> 32) - sb;
            if (off >= SLOT) break;
            if ((off >> 2) == tid) {
              const float pv = __uint_as_float((uint32_t)pe);
#pragma unroll
              for (int e = 0; e < 4; e++) x[e] = ((off & 3) == e) ? pv : x[e];
            }
            pc++;
          }
          const int pt = ctl_pull - sb;
          if (pt >= 0 && pt < SLOT && (pt >> 2) == tid) {
#pragma unroll
            for (int e = 0; e < 4; e++) x[e] = ((pt & 3) == e) ? ctl_pval : x[e];
          }
        }
      }
      q[j] = v4f{x[0], x[1], x[2], x[3]};
      gm[j] = vmax(vmax3(x[0], x[1], x[2]), x[3]);
      mr = vmax(mr, gm[j]);
      if (STOCH || stoch) {
        if (j == 0) {
          const float c = gm[0] * inv_e;
          c_s = (c > -INFINITY && c < INFINITY) ? c : 0.0f;
          cL = c_s * LOG2E;
        }
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = xexp2(__builtin_fmaf(UNIT ? x[e] : x[e] * inv_e, LOG2E, -cL));
        sum += (t[0] + t[1]) + (t[2] + t[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) nanl |= (x[e] != x[e]) ? 1u : 0u;
      }
    }
  };
  using Yes = std::true_type;
  using No = std::false_type;
  if (HAS_MASK || HAS_CTL || ns < SPC || (s0 + SPC) * SLOT > enc) {
    stream(Yes{}, No{}, No{});
  } else if constexpr (!HAS_MASK && !HAS_CTL) {
    if (stoch && cfg.scale) stream(No{}, Yes{}, No{});
    else if (stoch) stream(No{}, Yes{}, Yes{});
    else stream(No{}, No{}, No{});
  }
  if (WANT_LSE) {  // the held_row partial, against the lane max (every value is in registers)
    rc = (mr > -__FLT_MAX__) ? mr : -__FLT_MAX__;
#pragma unroll
    for (int j = 0; j < SPC; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) racc += (double)xexp2((q4(q[j], e) - rc) * LOG2E);
  }
  const float m_w = red_maxf(mr);
  double P = 0.0, R = 0.0;
  float c_w = 0.0f;  // offset of the published softmax partial
  uint32_t flags = 0;
  if (stoch) {
    // lanes whose max sits more than 40 above their offset, or whose offset
    // is so large (|c_s| >= 2^20, e.g. -1e30 standing for a masked id) that
    // rn(c_s * log2e) misses c_s * log2e by units and the terms above are
    // garbage: recount against the lane max as exp2((s - max) * log2e), the
    // difference taken first (rare; makes +inf a NaN)
    const float ms = mr * inv_e;
    const bool redo = ms > c_s + 40.0f || !(__builtin_fabsf(c_s) < 0x1p20f);
    bool exact_off = false;
    if (__ballot(redo)) {
      const float cn = redo ? ms : c_s;
      float s2 = 0.0f;
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float xv = q4(q[j], e);
          t[e] = xexp2((xv * inv_e - cn) * LOG2E);
        }
        s2 += (t[0] + t[1]) + (t[2] + t[3]);
      }
      if (redo) {
        sum = s2;
        c_s = cn;
        exact_off = true;
      }
    }
    // lanes to the wave's scaled max c_w: factor e^(c_s - c_w), as
    // 2^(cL - c_w*log2e) with cL's own rounding taken out on lanes summed
    // against cL, as 2^((c_s - c_w)*log2e) on recounted ones (0 for a NaN or
    // -inf exponent, which keeps a NaN sum NaN)
    c_w = m_w * inv_e;
    const double dd = exact_off ? ((double)c_s - (double)c_w) * (double)LOG2E
                                : (double)cL - (double)c_w * (double)LOG2E;
    const double dn = ::fmin(::fmax(::rint(dd), -2100.0), 2100.0);
    const double fac = (dd > -2100.0) ? ldexp((double)xexp2((float)(dd - dn)), (int)dn) : 0.0;
    const double part = (sum != 0.0f) ? (double)sum * fac : (double)sum;
    P = red_sumd(part);
    if (P != P) flags |= 1u;
  } else if (red_or(nanl)) {
    flags |= 1u;
  }
  if (WANT_LSE) {
    // lanes to the wave max (the max's own lane by exactly exp2(0) = 1)
    // (a NaN R needs no flag of its own: a NaN logit already sets bit 0, and
    // a +inf one leaves the row max infinite, which voids the statistics but
    // not a greedy draw: argmax returns the first +inf, sampler.rs:268-286)
    R = red_sumd((racc != 0.0) ? racc * (double)xexp2((rc - m_w) * LOG2E) : racc);
  }
  const float c_r = m_w;
  if (HAS_MASK || HAS_CTL) {
    if (__builtin_isfinite(m_w)) {
      flags |= 2u;
    } else if (m_w == INFINITY) {
      bool fin = false;
#pragma unroll
      for (int j = 0; j < SPC; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) fin |= __builtin_isfinite(q4(q[j], e));
      if (__ballot(fin)) flags |= 2u;
    }
  }

  // Candidate bound: the K'-th largest of a set of distinct chunk elements, so
  // at least K' elements of the chunk lie at or above it.  For K' <= KGRP the
  // set is the 64 maxima of 4-lane groups (each group holds 4 x 64 logits);
  // for larger K' it is the 256 lane maxima, whose K'-th passes fewer
  // elements than the group maxima's would.  Every wave finds it for itself
  // (no second barrier) with a DPP bitonic sort; when fewer than K' groups
  // hold a finite value, as the K'-th largest lane max (the finite ones,
  // compacted and sorted).
  const uint32_t km = fkey(mr);
  {
    uint32_t g = max(km, xor_u32(km, 1));
    g = max(g, xor_u32(g, 2));
    if ((lane & 3) == 0) Lc.groupmax[wave * 16 + (lane >> 2)] = g;
    Lc.lanemax[tid] = km;
  }
  // held_row launches: the wave's max and f64 partial, and the row's running
  // max key (a relaxed atomic max, slot 1 of the row's ticket line) as it was
  // before this wave's update: a chunk that sees a larger max already
  // published cannot hold the row's argmax, and skips its fold data
  const bool held = WANT_LSE && (a.row_lse != nullptr || a.n_top > 0);
  if (held && lane == 0) {
    uint32_t* const rmax = reinterpret_cast<uint32_t*>(&a.row_ticket[row * TSTRIDE + 1]);
    Lc.wprev[wave] = __hip_atomic_fetch_max(rmax, fkey(m_w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Lc.wmax[wave] = m_w;
    Lc.wr[wave] = R;
  }
  __syncthreads();
  uint32_t tk = 0;
  // Keys this sub-record publishes for the row's survivor bound, keys of
  // distinct elements of the chunk: its group maxima (K' <= KGRP) or lane
  // maxima (K' > KGRP) of rank wave + 4r, so the chunk's four sub-records
  // hold its top 16.
  uint32_t pub[4] = {fkey(m_w), 0u, 0u, 0u};
  if (!cfg.bad) {
    bool none = false;  // every element of the chunk is -inf: no entries at all
    if (kp <= KGRP) {  // the kp-th largest group max: a DPP bitonic sort of the 64
      uint32_t gv[1] = {Lc.groupmax[lane]};
      wave_sort_desc<1, true>(gv);
      tk = rdl(gv[0], kp - 1);
      none = rdl(gv[0], 0) <= KEY_NEG_INF;
#pragma unroll
      for (int r = 0; r < 4; r++) pub[r] = rdl(gv[0], wave + 4 * r);
    }
    if (kp > KGRP) {  // the kp-th largest lane max: a sort of the 256
      uint32_t all[4];
#pragma unroll
      for (int r = 0; r < 4; r++) all[r] = Lc.lanemax[r * 64 + lane];
      wave_sort_desc<4, true>(all);
      const int i = kp - 1;
#pragma unroll
      for (int r = 0; r < 4; r++)
        if ((i >> 6) == r) tk = rdl(all[r], i & 63);
#pragma unroll
      for (int r = 0; r < 4; r++) pub[r] = rdl(all[0], wave + 4 * r);
    } else if (tk <= KEY_NEG_INF && !none) {
      // fewer than K' group maxima are finite, so at most 4(K' - 1) < 128 lane
      // maxima are (the staging area is free until the filter)
      uint32_t all[4];
#pragma unroll
      for (int r = 0; r < 4; r++) all[r] = Lc.lanemax[r * 64 + lane];
      tk = kth_largest_few<4>(all, kp, reinterpret_cast<uint32_t*>(Tl.stage[wave]));
    }
  }

  // held_row fold data (held_fold reads it for the row's argmax chunk): when
  // the chunk's own terms relative to its max m_c sum below 2 -- every chunk
  // that can hold the argmax of a row whose fold applies -- and no larger max
  // was published before it, this wave's terms before the chunk's first
  // maximal id top_c go to an f64 sum and its terms of 2^-53 or more after
  // top_c to integer units of 2^-52 (an f64 sum of integers, exact below
  // 2^53).  The terms are f32 exps with the argument split in two, about
  // 2e-7 relative: within that of the reference's f64 terms, and for a term
  // after top_c rint(2^52 t) moves by at most 2e-7 of its own size plus a
  // rare flip of one unit at a half, so both sums, and denominator - 1, stay
  // within ~1e-6 of the reference's.
  uint64_t hw8 = 0, hw9 = 0;
  if (held) {
    float m_c = Lc.wmax[0];
    uint32_t prev = Lc.wprev[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) {
      m_c = fmaxf(m_c, Lc.wmax[w]);
      prev = max(prev, Lc.wprev[w]);
    }
    double D_c = 0.0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) {
      const double r = Lc.wr[w];
      if (r != 0.0) D_c += r * (double)xexp2((Lc.wmax[w] - m_c) * LOG2E);
    }
    if (__builtin_isfinite(m_c) && D_c < 2.0 && prev <= fkey(m_c)) {  // uniform in the workgroup
      // the chunk's first maximal id: the wave's first (ids rise with the
      // slot, then the lane, then the element), then the least of the waves'
      uint32_t fid = 0xFFFFFFFFu;
      if (m_w == m_c) {
        if (mr == m_c) {
#pragma unroll
          for (int j = SPC - 1; j >= 0; j--)
#pragma unroll
            for (int e = 3; e >= 0; e--)
              fid = (q4(q[j], e) == m_c) ? (uint32_t)((s0 + j) * SLOT + 4 * tid + e) : fid;
        }
        fid = ~((uint32_t)red_maxi((int)(~fid ^ 0x80000000u)) ^ 0x80000000u);
      }
      if (lane == 0) Lc.wtop[wave] = fid;
      __syncthreads();
      uint32_t top_c = Lc.wtop[0];
#pragma unroll
      for (int w = 1; w < NWAVE; w++) top_c = min(top_c, Lc.wtop[w]);
      const int jt = (int)(top_c / (uint32_t)SLOT) - s0;  // top_c's slot in the chunk
      const int rt = (int)(top_c % (uint32_t)SLOT);       // and its place in that slot
      // exp(d), d <= 0, as exp2 of d*log2e carried in two parts
      auto ex = [&](float d0) __attribute__((always_inline)) -> float {
        const float d = fmaxf(d0, -200.0f);  // -inf (an absent id) gives 0, not a NaN
        const float hi = d * LOG2E;
        const float lo = __builtin_fmaf(d, LOG2E, -hi) + d * 1.925963033500011e-08f;
        const float e2 = xexp2(hi);
        return e2 + e2 * (lo * 0.6931471805599453f);
      };
      double pre = 0.0, post = 0.0;
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        const float x4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
        if (j < jt) {  // before top_c
          pre += (double)((ex(x4[0] - m_c) + ex(x4[1] - m_c)) + (ex(x4[2] - m_c) + ex(x4[3] - m_c)));
        } else if (j == jt) {  // the slot of top_c: before it, then after it
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int o = 4 * tid + e;
            const float d = x4[e] - m_c;
            if (o < rt) pre += (double)ex(d);
            else if (o > rt && d >= LN_HALF_ULP1) post += (double)__builtin_rintf(ex(d) * 0x1p52f);
          }
        } else if (__ballot((gm[j] - m_c) >= LN_HALF_ULP1)) {  // after top_c: terms of 2^-53 or more
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float d = x4[e] - m_c;
            if (d >= LN_HALF_ULP1) post += (double)__builtin_rintf(ex(d) * 0x1p52f);
          }
        }
      }
      hw8 = (uint64_t)__double_as_longlong(red_sumd(pre));
      hw9 = (uint64_t)__double_as_longlong(red_sumd(post));
      flags |= 8u;
    }
  }

  // Filter: this wave's elements at or above the bound (never -inf, never
  // NaN), written straight into the wave's sub-record, in slot order, at
  // positions a ballot prefix hands out.
  const int nsp = ((nc * NWAVE + 63) >> 6) << 6;
  uint64_t* const rowrec = a.rec + (int64_t)row * SRECW * nsp;
  uint64_t* sub = rowrec + chunk * NWAVE + wave;
  const int base_id = s0 * SLOT + 4 * tid;
  int cnt = 0;
  bool ovf = false;
  uint64_t* const stg = Tl.stage[wave];
  const float tf = (tk <= KEY_NEG_INF) ? -__FLT_MAX__ : keyf(tk);  // the filter's floor
  if (!cfg.bad) {
    // every slot's ballot first, so the branches below test values already in
    // scalar registers instead of waiting on each compare
    uint64_t sb[SPC];
#pragma unroll
    for (int j = 0; j < SPC; j++) sb[j] = __ballot(gm[j] >= tf);
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      if (sb[j]) {
        uint64_t eb[4];
#pragma unroll
        for (int e = 0; e < 4; e++) eb[e] = __ballot(q4(q[j], e) >= tf);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          if (eb[e]) {
            const float x = q4(q[j], e);
            const uint32_t pos = (uint32_t)cnt + (uint32_t)lanes_below(eb[e]);
            if (x >= tf && pos < (uint32_t)CAPW) stg[pos] = pack(fkey(x), (uint32_t)(base_id + j * SLOT + e));
            cnt += __popcll(eb[e]);
          }
        }
      }
    }
    if (cnt > CAPW) {  // the exact re-scan writes its entries straight to the sub-record
      const ChunkCtl cc{pl, pc0, phi, ctl_pull, ctl_force, ctl_pval, ctl_fval};
      cnt = wave_overflow<HAS_MASK, HAS_CTL, LOC>(rowp, mrow, s0, ns, enc, sub, nsp, kp, tk, cc);
      ovf = true;
    }
  }
  // More entries than the finalizer preloads (EPRE), at most 64: stored in
  // descending order (flag 4), so the finalizer reads past the preloaded ones
  // only while they reach its bound.
  if (!ovf && cnt > EPRE && cnt <= 64) {
    wave_lds_sync();
    uint64_t v[1] = {lane < cnt ? stg[lane] : 0ull};
    wave_sort_desc64<1>(v);
    if (lane < cnt) stg[lane] = v[0];
    flags |= 4u;
  }

  // Publish the sub-record: header word i and staged entry p go to words i
  // and SHDR + p, one word per lane (an overflow wrote its entries itself).
  {
    const uint64_t w0 = (uint64_t)__double_as_longlong(P);
    const uint64_t w1 = ((uint64_t)__float_as_uint(c_r) << 32) | __float_as_uint(c_w);
    const uint64_t w2 = (uint64_t)__double_as_longlong(R);
    const uint64_t w3 = ((uint64_t)flags << 32) | __float_as_uint(m_w);
    const uint64_t w4 = (uint64_t)(uint32_t)cnt;
    const uint64_t w5 = ((uint64_t)pub[1] << 32) | pub[0];
    const uint64_t w6 = ((uint64_t)pub[3] << 32) | pub[2];
    const uint64_t w7 = __float_as_uint(ovf || cfg.bad ? INFINITY : tf);
    const int staged = ovf ? 0 : cnt;
    wave_lds_sync();
    for (int i = lane; i < SHDR + staged; i += 64) {
      uint64_t v = w0;
      v = i == 1 ? w1 : v;
      v = i == 2 ? w2 : v;
      v = i == 3 ? w3 : v;
      v = i == 4 ? w4 : v;
      v = i == 5 ? w5 : v;
      v = i == 6 ? w6 : v;
      v = i == 7 ? w7 : v;
      v = i == 8 ? hw8 : v;
      v = i == 9 ? hw9 : v;
      if (i >= SHDR) v = stg[i - SHDR];
      st_sub<LOC>(sub + (uint32_t)i * (uint32_t)nsp, v);
    }
  }

  // Hand-off: every wave's stores acknowledged, the workgroup takes the row's
  // arrival ticket; the last of the row's workgroups resets it for the next
  // call and its first wave finalizes the row.  A split launch leaves all of
  // that to finalize_kernel: the workgroup's slot goes to the next chunk at
  // once, its stores completing on their own.
  if (a.split) return;
  drain();
  __syncthreads();
  if (tid == 0) {
    // (xcd_test 2 flips the low bit of the XCD the odd chunks report: a row
    // of several chunks then fails the placement check, a test hook)
    const uint32_t x = LOC ? xcc_id() ^ ((a.xcd_test == 2) ? (uint32_t)(chunk & 1) : 0u) : 0u;
    const uint32_t add = LOC ? row_ticket_add(x) : 1u;
    const uint32_t t = (uint32_t)__hip_atomic_fetch_add(&a.row_ticket[row * TSTRIDE], (int32_t)add, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
    const bool lastw = (int)(t & 0xFFu) == nc - 1;
    Lc.last = lastw ? ((!LOC || row_on_one_xcd(t + add, nc, x)) ? 1 : 2) : 0;
    if (lastw) {
      st_agent(&a.row_ticket[row * TSTRIDE], 0);
      st_agent(&a.row_ticket[row * TSTRIDE + 1], 0);  // held_row's running max key
    }
  }
  __syncthreads();
  if (!Lc.last) return;
  if (a.serial && serial_row<HAS_MASK, HAS_CTL>(a, cfg, row)) return;  // serial_kernel finalizes it

  // The first wave finalizes the row; held_row outputs then get the reference's
  // serial fold (held_fold); a verify block's rows then walk accept_drafts
  // (verify_walk), except a row with more candidates than the selection
  // holds: the whole-row kernels draw it and walk its block.  On a masked or
  // controlled launch a row whose token the exact sum does not settle is
  // summed serially by the same wave and finalized again (ser_fallback).
  // A row whose workgroups did not all run on this XCD (Lc.last 2) has
  // sub-records outside this L2: it is failed, not read, and its sequence's
  // walk stops at it.  In a launch whose workgroups fit on the device at
  // once, held_fold's re-reads (a whole row, on a row whose fold leaves every
  // term above 2^-53) are shared by the four waves: the other three wait at
  // one barrier for the first wave's finalization (whose code holds no
  // barrier) and leave after the fold.
  if constexpr (!WANT_LSE) {  // (the first wave alone)
    if (wave != 0) return;
    const bool placed = !LOC || Lc.last == 1;
    if (placed) {
      finalize_row<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl.fin);
      if (HAS_MASK || HAS_CTL) ser_fallback<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl);
    } else if (lane == 0) {
      st_agent(&a.token[row], -1);
      st_agent(&a.status[row], XS_ROW_INTERNAL);
      if (a.n_cand) a.n_cand[row] = 0;
      if (cfg.big && a.big_state) a.big_state[row].state = 0;  // the whole-row kernels pass it by
    }
    if (a.span > 0 && (!placed || !deferred(cfg, Tl.fin))) verify_walk(a, row);
    return;
  }
  const bool placed = !LOC || Lc.last == 1;
  const bool shared = held && placed && a.fold_shared;  // (uniform)
  if (wave != 0 && !shared) return;
  if (wave == 0) {
    if (placed) {
      finalize_row<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl.fin);
      if (HAS_MASK || HAS_CTL) ser_fallback<HAS_MASK, WANT_LSE, HAS_CTL, LOC>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl);
    } else if (lane == 0) {
      st_agent(&a.token[row], -1);
      st_agent(&a.status[row], XS_ROW_INTERNAL);
      if (a.n_cand) a.n_cand[row] = 0;
      if (cfg.big && a.big_state) a.big_state[row].state = 0;  // the whole-row kernels pass it by
    }
  }
  if constexpr (WANT_LSE) {
    if (held && placed) {
      if (shared) __syncthreads();  // the first wave's finalization is in LDS
      held_fold<LOC>(a, row, rowp, rowrec, nsp, nc * NWAVE, Tl.fin, shared ? NWAVE : 1);
      if (wave != 0) return;
    }
  }
  if (a.span > 0 && (!placed || !deferred(cfg, Tl.fin))) verify_walk(a, row);
}

// ---------------------------------------------------------------------------
// finalize_kernel: the rows of a split launch, one workgroup per row, after
// sample_kernel published every chunk (the launch boundary orders the
// sub-records before these loads).  The same finalization as sample_kernel's
// last workgroup; it also clears held_row's running max key for the next
// call.  Batches larger than the workgroups the GPU holds at once take this
// path: their streaming workgroups then free their slots as soon as they
// have published, instead of waiting for the hand-off or a finalizer.
template <bool HAS_MASK, bool WANT_LSE, bool HAS_CTL>
__global__ __launch_bounds__(BLOCK) void finalize_kernel(Args a) {
  __shared__ TailLds Tl;
  const int row = blockIdx.x;
  const int nc = a.n_chunks;
  const int nsp = ((nc * NWAVE + 63) >> 6) << 6;
  const uint64_t* const rowrec = a.rec + (int64_t)row * SRECW * nsp;
  const bool held = WANT_LSE && (a.row_lse != nullptr || a.n_top > 0);
  const bool shared = held && a.fold_shared;  // as sample_kernel's finalizer
  const int wave = wave_id();
  if (wave != 0 && !shared) return;  // one wave finalizes the row; all four may share held_fold
  // the row's headers first: their round trip overlaps the row's parameters
  uint64_t h[NHW], E[EPRE];
  if (wave == 0) load_heads<WANT_LSE, true>(rowrec, nsp, nc * NWAVE, h, E);
  const Cfg cfg = a.greedy_all ? greedy_cfg(a.n_top, a.enc) : make_cfg(a.params[row], a.enc, a.n_top, a.k_max, a.ser_force);
  if (threadIdx.x == 0) st_agent(&a.row_ticket[row * TSTRIDE + 1], 0);  // held_row's running max key
  if (a.serial && serial_row<HAS_MASK, HAS_CTL>(a, cfg, row)) return;  // serial_kernel finalizes it
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  if (wave == 0) {
    finalize_heads<HAS_MASK, WANT_LSE, HAS_CTL, true>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl.fin, h, E);
    if (HAS_MASK || HAS_CTL) ser_fallback<HAS_MASK, WANT_LSE, HAS_CTL, true>(a, cfg, row, rowrec, nsp, nc * NWAVE, rowp, mrow, Tl);
  }
  if (held) {
    if (shared) __syncthreads();  // the first wave's finalization is in LDS
    held_fold<true>(a, row, rowp, rowrec, nsp, nc * NWAVE, Tl.fin, shared ? NWAVE : 1);
    if (wave != 0) return;
  }
  if (a.span > 0 && !deferred(cfg, Tl.fin)) verify_walk(a, row);
}

// ---------------------------------------------------------------------------
// score_kernel: the scoring reads of held rows, launched after sample_kernel
// has written each row's lse (held_row, generate.rs:1905-1933).  Grid: rows x
// n_chunks, the chunks of sample_kernel.  Each workgroup forms, for the ids of
// its chunk, p = exp(f64(v) - lse) -- the reference's last_probs term
// (generate.rs:1893-1899), written out when `probs` is asked for -- and adds
// the p of each class's ids, as escape_mass sums last_probs over its classes
// (batch.rs:1638-1662).  The row's last workgroup to arrive (an arrival
// ticket, slot 3 of the row's ticket line) adds the chunks' class sums in
// chunk order.  Chunk 0's workgroup also reads the scored ids:
// f64(v[id]) - lse, and an id outside [0, enc) fails the row as
// last_logprobs_for does (generate.rs:1871-1883).  A row whose held_row
// failed (NaN lse) keeps its status; its scores are NaN.
__global__ __launch_bounds__(BLOCK) void score_kernel(Args a) {
  __shared__ double expt[64];
  __shared__ double part[NWAVE][XS_CLASS_MAX];
  __shared__ int32_t last;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int nc = a.n_chunks;
  const int row = blockIdx.x / nc, chunk = blockIdx.x - row * nc;
  const int enc = (int)a.enc;
  const int ncl = a.class_masks ? a.n_class : 0;
  if (tid < 64) expt[tid] = (&kExpT[0][0])[tid];
  const double lse = a.row_lse[row];
  const bool ok = !__builtin_isnan(lse);
  const float* rowp = a.logits + (int64_t)row * a.ld;
  __syncthreads();
  double acc[XS_CLASS_MAX];
#pragma unroll
  for (int c = 0; c < XS_CLASS_MAX; c++) acc[c] = 0.0;
  const int s0 = chunk * SPC;
  const int ns = min(SPC, a.nslots - s0);
  for (int j = 0; j < ns; j++) {
    const int id0 = ((s0 + j) * BLOCK + tid) * 4;
    if (id0 < enc) {  // (the float4 lies inside the row: ld % 4 == 0 and id0 < enc <= ld)
      const float4 v = reinterpret_cast<const float4*>(rowp)[id0 >> 2];
      const float xv[4] = {v.x, v.y, v.z, v.w};
      uint32_t w[XS_CLASS_MAX];
#pragma unroll
      for (int c = 0; c < XS_CLASS_MAX; c++)
        w[c] = c < ncl ? a.class_masks[((int64_t)row * a.n_class + c) * a.class_ld + (id0 >> 5)] : 0u;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int id = id0 + e;
        if (id < enc) {
          const double p = ok ? exp_f64((double)xv[e] - lse, expt) : __builtin_nan("");
          if (a.probs) a.probs[(int64_t)row * a.probs_ld + id] = p;
#pragma unroll
          for (int c = 0; c < XS_CLASS_MAX; c++)
            if (c < ncl && ((w[c] >> (id & 31)) & 1u)) acc[c] += p;
        }
      }
    }
  }
  if (chunk == 0 && a.score_ids) {
    bool oor = false;
    for (int i = tid; i < a.n_score; i += BLOCK) {
      const int id = a.score_ids[(int64_t)row * a.score_ld + i];
      const bool out = id < 0 || id >= enc;
      oor |= out;
      a.score_logprob[(int64_t)row * a.score_ld + i] = (out || !ok) ? __builtin_nan("") : (double)rowp[id] - lse;
    }
    if (__syncthreads_or(oor) && ok && tid == 0) {
      a.status[row] = XS_ROW_ID_OOR;
      a.token[row] = -1;
    }
  }
  if (ncl == 0) return;
  // the chunk's class sums: waves in order, then the row's chunks in order
#pragma unroll
  for (int c = 0; c < XS_CLASS_MAX; c++) {
    if (c < ncl) {
      const double t = wave_sumd(acc[c]);
      if (lane == 0) part[wave][c] = t;
    }
  }
  __syncthreads();
  uint64_t* const prow = a.score_part + (int64_t)row * nc * XS_CLASS_MAX;
  if (tid < ncl) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) t += part[w][tid];
    st_agent(&prow[chunk * XS_CLASS_MAX + tid], (uint64_t)__double_as_longlong(t));
  }
  drain();
  __syncthreads();
  if (tid == 0) {
    const int t = __hip_atomic_fetch_add(&a.row_ticket[row * TSTRIDE + 3], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = (t == nc - 1) ? 1 : 0;
    if (t == nc - 1) st_agent(&a.row_ticket[row * TSTRIDE + 3], 0);
  }
  __syncthreads();
  if (!last || tid >= ncl) return;
  double m = 0.0;
  for (int k = 0; k < nc; k++) m += __longlong_as_double((long long)ld_agent(&prow[k * XS_CLASS_MAX + tid]));
  a.class_mass[(int64_t)row * a.n_class + tid] = m;
}

// ---------------------------------------------------------------------------
// serial_kernel: the serial denominator of a call's controlled rows at
// top_p >= 1, launched after sample_kernel on calls with a mask or controls
// that can observe it (sample_kernel's last workgroup leaves those rows
// unfinalized).  Grid: rows x n_chunks workgroups, the chunks of
// sample_kernel; other rows' return at once.  Each workgroup reads the row's
// max and the exact sum before its chunk from the row's sub-record headers,
// recomputes its chunk's terms, and writes one summary per segment (the grid
// units, the half-way flags, and the kept terms where the exact prefix may
// pass a power of two or a flag is set).  The row's last workgroup (the
// arrival ticket, as in sample_kernel) walks the summaries and finalizes the
// row with the serial sum as its denominator.
struct SerLds {
  double expt[64];
  double segsum[SPC * NWAVE];  // exact sums of the chunk's segments, row order (short exp)
  double segpre[SPC * NWAVE];  // the exact sum before each
  double xc;                   // the exact sum before the chunk
  uint32_t R[SPC * NWAVE][2];  // units at the segment's lower binade and the next
  uint32_t meta[SPC * NWAVE];  // summary word 1's high half, without the kept slot
  uint64_t kmask;              // segments of the chunk that keep their terms
  float qd[NWAVE][SER_QCAP];   // per wave: exp arguments queued for the correctly rounded exp
  uint8_t qt[NWAVE][SER_QCAP]; // and their segments
  float m_s;
  int32_t ok, last, nb, kbase;
};
union SerTail {
  struct {
    uint64_t sum[SER_WIN][2];    // staged summaries
    float ev[SER_LDS + 1][SEG];  // staged kept terms, and a scratch segment
  } w;
  TailLds tl;
};

// The queued terms of one wave: each correctly rounded, its units and
// half-way flags added to its segment's summary (LDS atomics: a segment's
// fast units are added the same way).  Out of line: the pass calls it from
// many places, and seldom.
__device__ __attribute__((noinline)) void ser_flush(SerLds& L, int wave, int n, const double* T) {
  ser_flush_t(L, wave, n, T);
}

// Four terms correctly rounded, out of line (only kept segments need them).
__device__ __attribute__((noinline)) float4 cr_exp4(float4 d, const double* T) {
  return make_float4(cr_expf(d.x, T), cr_expf(d.y, T), cr_expf(d.z, T), cr_expf(d.w, T));
}

template <bool HAS_MASK, bool HAS_CTL>
__global__ __launch_bounds__(BLOCK) void serial_kernel(Args a) {
  __shared__ SerLds Ls;
  __shared__ SerTail St;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int nc = a.n_chunks;
  const int row = blockIdx.x / nc;
  const int chunk = blockIdx.x - row * nc;
  const Cfg cfg = make_cfg(a.params[row], a.enc, a.n_top, a.k_max, a.ser_force);
  if (!serial_row<HAS_MASK, HAS_CTL>(a, cfg, row)) return;
  const int enc = (int)a.enc;
  const int s0 = chunk * SPC;
  const int ns = min(SPC, a.nslots - s0);
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const v4f* rp4 = reinterpret_cast<const v4f*>(rowp);
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  const int fmax = (enc - 1) >> 2;
  const int nsp = ((nc * NWAVE + 63) >> 6) << 6;
  const uint64_t* const rowrec = a.rec + (int64_t)row * SRECW * nsp;
  const int nsub = nc * NWAVE;
  // the row max (sample_kernel's headers) and the exact sum before this
  // chunk: their loads go out first, the chunk's after them
  uint64_t h0[GMAX], h1[GMAX], h3[GMAX];
  if (wave == 0) {
#pragma unroll
    for (int gi = 0; gi < GMAX; gi++) {
      const int sub = gi * 64 + lane;
      const bool before = sub < chunk * NWAVE;
      const int sc = min(sub, nsp - 1);  // (clamped, not guarded: all in flight)
      h3[gi] = ld_agent(&rowrec[3 * nsp + sc]);
      h0[gi] = ld_agent(&rowrec[sc]);
      h1[gi] = ld_agent(&rowrec[nsp + sc]);
      h3[gi] = sub < nsub ? h3[gi] : 0ull;
      h0[gi] = before ? h0[gi] : 0ull;
      h1[gi] = before ? h1[gi] : 0ull;
    }
  }
  v4f q[SPC];
  uint32_t mw[SPC];
#pragma unroll
  for (int j = 0; j < SPC; j++) {
    const int f = min((s0 + j) * BLOCK + tid, fmax);
    q[j] = rp4[f];
    if (HAS_MASK) mw[j] = mrow[f >> 3];
  }
  CtlRow cr{};
  if (HAS_CTL) cr = a.ctl_row[row];
  if (tid < 64) Ls.expt[tid] = (&kExpT[0][0])[tid];
  if (wave == 0) {
    float mv = -INFINITY;
    uint32_t fw = 0;
#pragma unroll
    for (int gi = 0; gi < GMAX; gi++) {
      if (gi * 64 + lane < nsub) {
        mv = fmaxf(mv, __uint_as_float((uint32_t)h3[gi]));
        fw |= (uint32_t)(h3[gi] >> 32);
      }
    }
    const float m_v = wave_maxf(mv);
    const uint32_t fl = wave_or(fw);
    const float m_s = cfg.scale ? m_v * cfg.inv : m_v;
    double xc = 0.0;
#pragma unroll
    for (int gi = 0; gi < GMAX; gi++) {
      const double p = __longlong_as_double((long long)h0[gi]);
      if (p != 0.0) xc += p * (double)xexp2((__uint_as_float((uint32_t)h1[gi]) - m_s) * LOG2E);
    }
    xc = wave_sumd(xc);
    if (lane == 0) {
      Ls.m_s = m_s;
      Ls.xc = xc;
      // the row draws (else the finalizer reports its status, and no sum is needed)
      Ls.ok = ((fl & 2u) && !(fl & 1u) && !__builtin_isinf(m_s) &&
               (!(HAS_CTL && cr.active) || cr.status == XS_ROW_OK)) ? 1 : 0;
    }
  }
  __syncthreads();
  const bool ok = Ls.ok != 0;  // uniform
  const float m_s = Ls.m_s;
  if (ok) {
    // each term's exp argument d = s - max, the values masked and controlled
    // as sample_kernel's pass does, and the segments' exact sums (short exp)
    const bool ctl_on = HAS_CTL && cr.active;
    int pc = 0, phi = 0;
    const uint64_t* pl = nullptr;
    if (ctl_on) {
      pc = a.ctl_chunk[(int64_t)row * (nc + 1) + chunk];
      phi = a.ctl_chunk[(int64_t)row * (nc + 1) + chunk + 1];
      pl = a.patch + (int64_t)row * a.ctl_cap;
    }
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      float x[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
      if (HAS_MASK) {
        const uint32_t bits = mw[j] >> ((((s0 + j) * BLOCK + tid) & 7) * 4);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (!((bits >> e) & 1u)) x[e] = -INFINITY;
      }
      if (j >= ns || (s0 + j + 1) * SLOT > enc) {
        const int id0 = (s0 + j) * SLOT + 4 * tid;
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (j >= ns || id0 + e >= enc) x[e] = -INFINITY;
      }
      if (ctl_on) ctl_slot(x, (s0 + j) * SLOT, tid, pl, pc, phi, cr.pull_id, cr.pull_val, cr.force_id, cr.force_val);
      float dv[4], t = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        dv[e] = (cfg.scale ? x[e] * cfg.inv : x[e]) - m_s;
        t += fast_expf(dv[e]);
      }
      q[j] = v4f{dv[0], dv[1], dv[2], dv[3]};
      const double ssum = wave_sumd((double)t);
      const bool any = __ballot(dv[0] >= -104.0f || dv[1] >= -104.0f || dv[2] >= -104.0f || dv[3] >= -104.0f) != 0;
      if (lane == 0) {
        Ls.segsum[j * NWAVE + wave] = ssum;
        Ls.meta[j * NWAVE + wave] = any ? 0u : SM_ZERO;  // below -104 every term is +0
      }
    }
  }
  __syncthreads();
  if (ok && wave == 0) {  // exact prefixes, in row order
    const double v = Ls.segsum[lane];
    double inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const double t = __shfl_up(inc, d);
      if (lane >= d) inc += t;
    }
    const double ex = __shfl_up(inc, 1);
    Ls.segpre[lane] = Ls.xc + (lane == 0 ? 0.0 : ex);
  }
  __syncthreads();
  uint64_t* const ssum = a.ser_sum + (int64_t)row * a.ser_ld * 2;
  uint64_t* const skeep = a.ser_e + (int64_t)row * SER_NB * (SEG / 2);
  if (ok) {
    // units per segment: each term's from the short exp where its error bound
    // settles them, else queued for the correctly rounded exp (subnormal
    // terms too: d in [-104, -87)); the settled units stay in registers until
    // the queue is empty
    int qn = 0;
    uint32_t fr0[SPC], fr1[SPC];
    if (lane < SPC) {
      const int t = lane * NWAVE + wave;
      Ls.R[t][0] = 0u;
      Ls.R[t][1] = 0u;
    }
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      fr0[j] = fr1[j] = 0u;
      if (j < ns) {
        const int t = j * NWAVE + wave;
        const double X0 = Ls.segpre[t];
        const int FB = f32_field((float)(X0 * (1.0 - SER_DELTA)));
        const bool two = f32_field((float)(X0 * (1.0 + SER_DELTA))) != FB;
        if (lane == 0) Ls.meta[t] |= (uint32_t)FB | (two ? SM_TWO : 0u);
        const float dv[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
        uint32_t r0 = 0, r1 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float ef = fast_expf(dv[k]);
          uint32_t u0, u1 = 0;
          bool settled = fast_units(ef, FB, u0);
          if (two) settled = fast_units(ef, FB + 1, u1) && settled;
          const bool amb = !(dv[k] < -104.0f) && (!settled || dv[k] < -87.0f);
          if (!amb) {
            r0 += u0;
            r1 += u1;
          }
          const uint64_t b = __ballot(amb);
          if (b) {
            if (qn + 64 > SER_QCAP) {
              ser_flush(Ls, wave, qn, Ls.expt);
              qn = 0;
            }
            const int pos = qn + lanes_below(b);
            if (amb) {
              Ls.qd[wave][pos] = dv[k];
              Ls.qt[wave][pos] = (uint8_t)t;
            }
            qn += __popcll(b);
          }
        }
        fr0[j] = wave_sum_u32(r0);
        fr1[j] = wave_sum_u32(r1);
      }
    }
    ser_flush(Ls, wave, qn, Ls.expt);
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        Ls.R[j * NWAVE + wave][0] += fr0[j];
        Ls.R[j * NWAVE + wave][1] += fr1[j];
      }
    }
  }
  __syncthreads();
  if (ok && wave == 0) {
    // segments that keep their terms: nonzero ones where the exact sum may
    // pass a power of two, or with a half-way term (lane t: segment t); one
    // reservation of side-buffer slots for the workgroup
    static_assert(SPC * NWAVE == 64, "one segment per lane");
    const int t = lane;
    bool keep = false;
    if (t / NWAVE < ns) {
      const uint32_t mt = Ls.meta[t];
      const double X1 = Ls.segpre[t] + Ls.segsum[t];
      const bool pass2 = f32_field((float)(X1 * (1.0 + SER_DELTA))) != (int)(mt & 0xFFu);
      keep = !(mt & SM_ZERO) && (pass2 || (mt & (SM_TIE0 | SM_TIE1)));
    }
    const uint64_t km = __ballot(keep);
    if (lane == 0) {
      Ls.kmask = km;
      Ls.kbase = km ? __hip_atomic_fetch_add(&a.row_ticket[row * TSTRIDE + 2], __popcll(km), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)
                    : 0;
    }
  }
  __syncthreads();
  if (ok) {
    const uint64_t km = Ls.kmask;
    const int kbase = Ls.kbase;
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      const int t = j * NWAVE + wave;
      const int idx = kbase + __popcll(km & ((1ull << t) - 1ull));
      if (j < ns && ((km >> t) & 1ull) && idx < SER_NB) {  // a kept segment: its terms correctly rounded
        const float4 e = cr_exp4(make_float4(q[j].x, q[j].y, q[j].z, q[j].w), Ls.expt);
        uint64_t* const dst = skeep + (int64_t)idx * (SEG / 2) + 2 * lane;
        st_agent(dst, (uint64_t)__float_as_uint(e.x) | ((uint64_t)__float_as_uint(e.y) << 32));
        st_agent(dst + 1, (uint64_t)__float_as_uint(e.z) | ((uint64_t)__float_as_uint(e.w) << 32));
      }
      if (j < ns && lane == 0) {
        const int g = (s0 + j) * NWAVE + wave;  // the segment's place in the row
        const int idx = kbase + __popcll(km & ((1ull << t) - 1ull));
        const uint32_t kept = ((km >> t) & 1ull) && idx < SER_NB ? (uint32_t)idx + 1 : 0u;
        st_agent(&ssum[2 * g], (uint64_t)Ls.R[t][0] | ((uint64_t)Ls.R[t][1] << 32));
        st_agent(&ssum[2 * g + 1], (uint64_t)(Ls.meta[t] | (kept << 16)) << 32);
      }
    }
  }
  // hand-off, as in sample_kernel; slot 2 of the row's ticket line counts kept segments
  drain();
  __syncthreads();
  if (tid == 0) {
    const int t = __hip_atomic_fetch_add(&a.row_ticket[row * TSTRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Ls.last = (t == nc - 1) ? 1 : 0;
    if (t == nc - 1) {
      Ls.nb = ld_agent(&a.row_ticket[row * TSTRIDE + 2]);
      st_agent(&a.row_ticket[row * TSTRIDE], 0);
      st_agent(&a.row_ticket[row * TSTRIDE + 2], 0);
    }
  }
  __syncthreads();
  if (!Ls.last) return;

  float S_ser = -1.0f;
  if (ok) {
    const int nseg = a.nslots * NWAVE;
    const int nbl = min(min(Ls.nb, SER_NB), SER_LDS);
    for (int i = tid; i < nbl * (SEG / 2); i += BLOCK)
      reinterpret_cast<uint64_t*>(&St.w.ev[0][0])[i] = ld_agent(&skeep[i]);
    uint32_t sb = 0;  // the running sum's bits, from +0
#pragma unroll 1
    for (int w0 = 0; w0 < nseg; w0 += SER_WIN) {
      const int wn = min(SER_WIN, nseg - w0);
      for (int i = tid; i < 2 * wn; i += BLOCK) (&St.w.sum[0][0])[i] = ld_agent(&ssum[2 * (int64_t)w0 + i]);
      __syncthreads();
      if (wave == 0)
        sb = ser_walk<HAS_MASK, HAS_CTL>(a, cfg, row, sb, St.w.sum, w0, wn, St.w.ev, nbl, skeep, m_s, Ls.expt,
                                         St.w.ev[SER_LDS]);
      __syncthreads();
    }
    S_ser = __uint_as_float(sb);
  }
  if (wave != 0) return;
  finalize_row<HAS_MASK, false, HAS_CTL, true>(a, cfg, row, rowrec, nsp, nsub, rowp, mrow, St.tl.fin, S_ser);
  if (a.span > 0 && !deferred(cfg, St.tl.fin)) verify_walk(a, row);
}

// ---------------------------------------------------------------------------
// Sparse controls (apply_control, sampler.rs:433-490): one workgroup per row,
// launched before sample_kernel when a call carries controls.  The row's bans
// and biases become its patch list: every distinct listed id < enc with its
// value after the mask, the bans (sampler.rs:450-454) and then the biases in
// list order (:455-459).  A pull needs the row max after those (:460-470): the
// workgroup reads the row once for it, and only for a finite target, and keeps
// the target's new value.  A force keeps the target's final value (:471-482).
// sample_kernel overwrites exactly these elements before anything reads them.
template <bool HAS_MASK>
__global__ __launch_bounds__(BLOCK) void control_kernel(Args a) {
  __shared__ uint64_t lkeys[CTL_MAX];  // (id << 32 | list position), sorted (lists of CTL_MAX or fewer)
  __shared__ uint64_t lpl[CTL_MAX];    // the patch list (idem)
  __shared__ SortLds B;                // the radix sort's counters (longer lists)
  __shared__ int s4[NWAVE];
  __shared__ float wmax[NWAVE];
  const int row = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const xs_row_control c = a.controls[row];
  const int enc = (int)a.enc, nc = a.n_chunks;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  int32_t* cb = a.ctl_chunk + (int64_t)row * (nc + 1);
  uint64_t* patch = a.patch + (int64_t)row * a.ctl_cap;
  auto allowed = [&](int id) __attribute__((always_inline)) {
    return !HAS_MASK || ((mrow[id >> 5] >> (id & 31)) & 1u);
  };
  const bool active = c.n_ban != 0 || c.n_bias != 0 || c.has_pull != 0 || c.has_force != 0;
  const int64_t n64 = (int64_t)c.n_ban + (int64_t)c.n_bias;
  int status = XS_ROW_OK;
  if (c.n_ban < 0 || c.n_bias < 0 || c.ban_off < 0 || c.bias_off < 0 || n64 > a.ctl_cap ||
      (n64 > 0 && !a.ctl_ids) || (c.n_bias > 0 && !a.ctl_delta))
    status = XS_ROW_BAD_PARAM;
  if (!active || status != XS_ROW_OK) {
    for (int i = tid; i <= nc; i += BLOCK) cb[i] = 0;
    if (tid == 0) a.ctl_row[row] = CtlRow{active ? 1 : 0, status, 0, -1, 0.0f, -1, 0.0f, 0};
    return;
  }

  // Sort the listed ids, each tagged with its list position (bans first):
  // a list of CTL_MAX or fewer in LDS (bitonic), a longer one in the
  // context's sort buffers (the stable LSD radix sort of the whole-row path,
  // by ~id descending, which keeps equal ids in list order); the patch list
  // then goes straight to the row's patch array.
  const int n = (int)n64;
  const bool lds = n <= CTL_MAX;
  uint64_t* const gk = lds ? nullptr : a.ctl_keys + (int64_t)row * 2 * a.ctl_cap;
  uint64_t* const pl = lds ? lpl : patch;
  if (lds) {
    int np2 = 1;
    while (np2 < n) np2 <<= 1;
    for (int i = tid; i < np2; i += BLOCK) {
      uint64_t k = ~0ull;
      if (i < n) {
        const uint32_t id = i < c.n_ban ? a.ctl_ids[c.ban_off + i] : a.ctl_ids[c.bias_off + (i - c.n_ban)];
        k = ((uint64_t)id << 32) | (uint32_t)i;
      }
      lkeys[i] = k;
    }
    __syncthreads();
    for (int size = 2; size <= np2; size <<= 1) {  // bitonic, ascending
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < np2 / 2; i += BLOCK) {
          const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
          const bool asc = (lo & size) == 0;
          const uint64_t x = lkeys[lo], y = lkeys[hi];
          if ((x > y) == asc) {
            lkeys[lo] = y;
            lkeys[hi] = x;
          }
        }
        __syncthreads();
      }
    }
  } else {
    for (int i = tid; i < n; i += BLOCK) {
      const uint32_t id = i < c.n_ban ? a.ctl_ids[c.ban_off + i] : a.ctl_ids[c.bias_off + (i - c.n_ban)];
      gk[i] = ((uint64_t)(0xFFFFFFFFu - id) << 32) | (uint32_t)i;
    }
    __syncthreads();
    radix_sort_desc(gk, gk + a.ctl_cap, n, B);  // (every pass ends in a barrier)
  }
  auto keys = [&](int i) __attribute__((always_inline)) -> uint64_t {  // (id << 32 | list position)
    if (lds) return lkeys[i];
    const uint64_t k = gk[i];
    return ((uint64_t)(0xFFFFFFFFu - (uint32_t)(k >> 32)) << 32) | (uint32_t)k;
  };

  // One patch per distinct id < enc: the run of its entries holds its bans
  // (lower positions) and then its biases in list order.
  const int seg = (n + BLOCK - 1) / BLOCK;
  const int b0 = min(n, tid * seg), b1 = min(n, b0 + seg);
  auto starts = [&](int i) __attribute__((always_inline)) {
    const uint32_t id = (uint32_t)(keys(i) >> 32);
    return id < (uint32_t)enc && (i == 0 || (uint32_t)(keys(i - 1) >> 32) != id);
  };
  int cnt = 0;
  for (int i = b0; i < b1; i++) cnt += starts(i) ? 1 : 0;
  int total;
  int p = block_excl_scan(cnt, s4, &total);
  for (int i = b0; i < b1; i++) {
    if (!starts(i)) continue;
    const uint32_t id = (uint32_t)(keys(i) >> 32);
    float x = allowed((int)id) ? rowp[id] : -INFINITY;
    for (int j = i; j < n && (uint32_t)(keys(j) >> 32) == id; j++) {
      const int o = (int)(uint32_t)keys(j);
      if (o < c.n_ban) x = -INFINITY;
      else x = x + a.ctl_delta[c.bias_off + (o - c.n_ban)];
    }
    pl[p++] = ((uint64_t)id << 32) | __float_as_uint(x);
  }
  __syncthreads();
  auto lower = [&](uint32_t v) __attribute__((always_inline)) {  // first patch with id >= v
    int lo = 0, hi = total;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((uint32_t)(pl[mid] >> 32) < v) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  auto patched = [&](int id) __attribute__((always_inline)) {
    const int q = lower((uint32_t)id);
    return q < total && (uint32_t)(pl[q] >> 32) == (uint32_t)id;
  };
  if (lds)
    for (int i = tid; i < total; i += BLOCK) patch[i] = pl[i];
  for (int i = tid; i <= nc; i += BLOCK) cb[i] = (i == nc) ? total : lower((uint32_t)(i * SPC * SLOT));

  // pull: the max M over the row after the bans and biases (f32::max folds
  // skip NaN; so does every `>` test here), then v += alpha * max(0, M - v)
  int pull_id = -1;
  float pull_val = 0.0f;
  if (c.has_pull && c.pull_id < (uint32_t)enc) {
    const int t = (int)c.pull_id;
    const float vt = patched(t) ? __uint_as_float((uint32_t)pl[lower((uint32_t)t)])
                                : (allowed(t) ? rowp[t] : -INFINITY);
    if (__builtin_isfinite(vt)) {
      float best = -INFINITY;
      const v4f* r4 = reinterpret_cast<const v4f*>(rowp);
      for (int f = tid; 4 * f < enc; f += BLOCK) {
        const v4f q = r4[f];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int id = 4 * f + e;
          const float x = q4(q, e);
          if (id < enc && x > best && allowed(id) && !patched(id)) best = x;
        }
      }
      for (int i = tid; i < total; i += BLOCK) {
        const float v = __uint_as_float((uint32_t)pl[i]);
        if (v > best) best = v;
      }
      best = wave_maxf(best);
      if (lane == 0) wmax[wave] = best;
      __syncthreads();
      float M = wmax[0];
      for (int w = 1; w < NWAVE; w++) M = wmax[w] > M ? wmax[w] : M;
      pull_val = vt + c.pull_alpha * fmaxf(M - vt, 0.0f);
      pull_id = t;
    }
  }
  // force: the target keeps its final value if finite, else 0
  int force_id = -1;
  float force_val = 0.0f;
  if (c.has_force) {
    if (c.force_id >= (uint32_t)enc) {
      status = XS_ROW_FORCE_OOR;
    } else {
      const int t = (int)c.force_id;
      const float v = t == pull_id ? pull_val
                                   : (patched(t) ? __uint_as_float((uint32_t)pl[lower((uint32_t)t)])
                                                 : (allowed(t) ? rowp[t] : -INFINITY));
      force_val = __builtin_isfinite(v) ? v : 0.0f;
      force_id = t;
    }
  }
  if (tid == 0) a.ctl_row[row] = CtlRow{1, status, total, pull_id, pull_val, force_id, force_val, 0};
}

// Fills every row's status with one data error (a call-level condition such as
// a narrow row or a short mask) and clears the outputs the caller asked for.
__global__ void fill_status_kernel(int32_t* token, int32_t* status, int32_t* n_cand, int64_t rows, int32_t st) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows) {
    token[i] = -1;
    status[i] = st;
    if (n_cand) n_cand[i] = 0;
  }
}

__global__ void fill_verify_kernel(const xs_verify_args a, int32_t st) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.seqs * a.span) { a.row_token[i] = -1; a.row_status[i] = st; a.committed[i] = -1; }
  if (i < a.seqs) {
    // accept_drafts propagates the first row's error unless the budget stops
    // the walk before any row is sampled.
    const int bud = a.budget ? a.budget[i] : 0x7FFFFFFF;
    a.accepted[i] = 0;
    a.n_committed[i] = 0;
    a.seq_status[i] = bud <= 0 ? XS_ROW_OK : st;
  }
}

// Zeroes n ints (the arrival tickets of the no-allocation entry point; a
// kernel rather than hipMemsetAsync, so a captured call records no memset node).
// Each workgroup's XCD (xcd_placement).
__global__ void xcc_probe_kernel(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

__global__ void zero_kernel(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ void exp_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = cr_expf(x[i], &xs::kExpT[0][0]);
}

// Layout of the no-allocation entry point's workspace (xs_sample_noalloc): a
// context of NA_ROWS rows of up to NA_VOCAB ids with k_max = XS_K_MAX, carved
// out of one file-scope device array in u64 words, each part 256-byte aligned.
constexpr int64_t NA_ROWS = XS_NOALLOC_ROWS;
constexpr int64_t NA_VOCAB = XS_NOALLOC_VOCAB;
constexpr int64_t NA_CHUNKS = ((NA_VOCAB + SLOT - 1) / SLOT + SPC - 1) / SPC;
constexpr int64_t NA_NSP = (NA_CHUNKS * NWAVE + 63) / 64 * 64;
constexpr int64_t na_up(int64_t w) { return (w + 31) / 32 * 32; }
constexpr int64_t NA_OFF_REC = 0;
constexpr int64_t NA_OFF_PATCH = na_up(NA_OFF_REC + NA_ROWS * NA_NSP * SRECW);
constexpr int64_t NA_OFF_CTLROW = na_up(NA_OFF_PATCH + NA_ROWS * CTL_MAX);
constexpr int64_t NA_OFF_CTLCHUNK = na_up(NA_OFF_CTLROW + NA_ROWS * (int64_t)sizeof(CtlRow) / 8);
constexpr int64_t NA_OFF_TICKET = na_up(NA_OFF_CTLCHUNK + (NA_ROWS * (NA_CHUNKS + 1) + 1) / 2);
constexpr int64_t NA_TICKETS = NA_ROWS * TSTRIDE;  // ints
constexpr int64_t NA_OFF_SEQ = na_up(NA_OFF_TICKET + NA_TICKETS / 2);
constexpr int64_t NA_OFF_STATUS = na_up(NA_OFF_SEQ + NA_TICKETS / 2);
constexpr int64_t NA_OFF_SERSUM = na_up(NA_OFF_STATUS + NA_ROWS / 2);
constexpr int64_t NA_OFF_SERE = na_up(NA_OFF_SERSUM + NA_ROWS * NA_CHUNKS * SPC * NWAVE * 2);
constexpr int64_t NA_WORDS = na_up(NA_OFF_SERE + NA_ROWS * SER_NB * (SEG / 2));
static_assert(sizeof(CtlRow) % 8 == 0, "CtlRow packs into u64 words");
static_assert(NA_WORDS * 8 == XS_NOALLOC_BYTES, "XS_NOALLOC_BYTES states the array's size");

// ---------------------------------------------------------------------------
// The whole-row path: rows whose candidate set is larger than the streaming
// selection holds -- top_k of 128 or more, and top_k >= enc, the reference's
// candidate_set branch that sorts the whole row (sampler.rs:322-338), which is
// xwen's only top-p-only mode because top_k <= 1 means greedy.  The row's
// finalizer leaves its max and softmax denominator in big_state; then, on the
// row's tiles of BTILE ids (one workgroup each):
//   big_key_kernel      p = rn(exp(s - max) / S) of every id (the selection
//                       path's correctly rounded f32 arithmetic) as a sort key
//                       that ascends as p descends, with the id, in id order;
//                       the tile's counts of the first digit, which the row's
//                       last tile turns into every tile's first positions;
//   big_scatter_kernel  one pass of a stable LSD radix sort (RB-bit digits,
//                       RPASS passes): each tile places its entries at those
//                       positions, in order within the tile, so equal p keep
//                       ascending ids -- the (p desc, id asc) order of
//                       top_k_desc and of the stable whole-row sort;
//   big_hist_kernel     the next pass's counts of the reordered tiles, and
//                       their positions;
// then the first min(top_k, enc) sorted entries are the candidates, and
// truncate_top_p (sampler.rs:401-429) and WeightedIndex (:235-243, rand 0.9)
// run as the reference's serial f32 chains, each evaluated by big_chain:
//   big_units_kernel    per block of chain terms, their grid units at the
//                       binades where sums of probabilities end (one
//                       workgroup per block), for the chains to cross blocks
//                       in one step;
//   big_sum_kernel      one workgroup per row: the weights' sum (rows that
//                       top_p renormalises);
//   big_draw_kernel     one workgroup per row: the cut, the draw, the
//                       candidate list.

constexpr int RB = 8;               // radix bits per pass
constexpr int RBINS = 1 << RB;      // digits per pass: one per thread
constexpr int RPASS = 4;            // the sort keys have 31 bits
constexpr int SPT = 4;              // slots per tile
constexpr int BTILE = SPT * SLOT;   // ids per tile
constexpr int EPL = BTILE / BLOCK;  // a lane's entries of a tile
constexpr int QW = BTILE / NWAVE;   // a wave's quarter of a tile
constexpr int CPT = 16;             // chain terms per thread and block
constexpr int CBLK = CPT * BLOCK;   // chain terms per block
constexpr int CHEAD = 128;          // chain terms added one at a time first
// A tokens-only call's rows at top_k >= enc leave p < 1.75 * 2^-26 out of the
// sort and the chains (their pkey above KCUT; KSENT marks them in the first
// pass's source).  Such a row's p sum to about 1 and it holds at most 2^20
// ids, so those terms sum to under 0.03, and the serial f32 sum of the others
// (at most 2^20 additions, each off by at most 2^-24 relative) is at least
// 0.9.  So each left-out term, raw (p) or renormalised (p / sum < 1.95 *
// 2^-26), is below 2^-25, half an ulp of any sum of 0.5 or more, and every
// addition of one rounds back to the sum.  No chain depends on them or their
// order.  (The draw's index never passes every cumulative weight: any u <=
// 1 - 2^-24, the largest float below 1, keeps x = rn(u * total) below a
// normal total such as this one (at least 0.9): u * total <= total - total *
// 2^-24, which is more than half an ulp of total below it, or exactly the
// float below it when total is a power of two.  A uniform of 1 or more takes
// the last kept entry.)  big_key_kernel
// decides most ids with a plain f32 exp and a margin (PLO), and computes the
// correctly rounded p only for the rest.
constexpr uint32_t KCUT = 0x7FFFFFFFu - 0x32E00000u;  // pkey(1.75 * 2^-26)
constexpr uint32_t KSENT = 0xFFFFFFFFu;
// 1.75 * 2^-26 * (1 - 2^-10): an f32 estimate exp2(d * log2e) / S below it
// (off by under 1e-5 relative for the d that reach it) is a p below the cut
constexpr float PLO = 0x1.bf9p-26f;
constexpr int NG = 4;               // binades whose grid units big_units_kernel sums per block
constexpr int FTOP = 127;           // the highest of them: sums of probabilities stay below 2
constexpr int NBU = 256;            // blocks whose units a chain holds in LDS
constexpr int UW = NG + 1;          // words per block: NG sums, then the tie and absorb bits
static_assert(RBINS == BLOCK && EPL * 64 == QW, "one digit per thread; a wave's quarter in EPL steps");
static_assert(SPC % SPT == 0, "tiles inside chunks");

// The sort key of p >= +0: ascending as p descends.
XS_DEV uint32_t pkey(float p) { return 0x7FFFFFFFu - __float_as_uint(p + 0.0f); }
XS_DEV float pkey_p(uint32_t k) { return __uint_as_float(0x7FFFFFFFu - k); }
XS_DEV uint32_t rdigit(uint32_t k, int pass) { return (k >> (RB * pass)) & (uint32_t)(RBINS - 1); }

// The lanes whose digit d equals this lane's, among the lanes with `valid`
// (meaningless on the others).  Wave-uniform control flow only.
XS_DEV uint64_t digit_peers(uint32_t d, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < RB; b++) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bb = __ballot(valid && bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}
XS_DEV uint64_t lanes_below() { return (1ull << lane_id()) - 1ull; }
// Count this lane's digit once per group of equal digits (the group's lowest lane).
XS_DEV void count_digit(uint32_t* cnt, uint32_t d, bool valid) {
  const uint64_t pe = digit_peers(d, valid);
  if (valid && (pe & lanes_below()) == 0) atomicAdd(&cnt[d], (uint32_t)__popcll(pe));
}

// The row's whole-row state for the kernels below: null when the call does not
// draw the row on this path.
XS_DEV const BigRow* big_live(const Args& a, int row, Cfg& cfg) {
  cfg = a.greedy_all ? greedy_cfg(a.n_top, a.enc) : make_cfg(a.params[row], a.enc, a.n_top, a.k_max, a.ser_force);
  if (!cfg.big || cfg.bad) return nullptr;  // (then big_state[row] is not this call's)
  const BigRow* br = a.big_state + row;
  return br->state ? br : nullptr;
}

// A tile's digit counts `c` (thread t: digit t) go out; the row's last of its
// nt tiles to arrive (an arrival ticket, as in sample_kernel's hand-off) turns
// every tile's counts into the tile's first position of each digit, in place:
// digits ascending, and within a digit the tiles in order.
XS_DEV void big_counts(const Args& a, int row, int tile, uint32_t c, int32_t* s4, int32_t& last, int nt) {
  int32_t* const H = reinterpret_cast<int32_t*>(a.big_hist) + (int64_t)row * a.big_hld;
  const int tid = threadIdx.x;
  st_agent(&H[(int64_t)tile * RBINS + tid], (int32_t)c);
  drain();
  __syncthreads();
  if (tid == 0) {
    const int t = __hip_atomic_fetch_add(&a.big_ticket[row * TSTRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = (t == nt - 1) ? 1 : 0;
    if (t == nt - 1) st_agent(&a.big_ticket[row * TSTRIDE], 0);
  }
  __syncthreads();
  if (!last) return;
  constexpr int U = 64;  // (one round for rows of up to 262,144 ids)
  uint32_t tot = 0;
#pragma unroll 1
  for (int t0 = 0; t0 < nt; t0 += U) {
    int32_t v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = ld_agent(&H[(int64_t)min(t0 + u, nt - 1) * RBINS + tid]);  // (clamped)
#pragma unroll
    for (int u = 0; u < U; u++) tot += t0 + u < nt ? (uint32_t)v[u] : 0u;
  }
  int total;
  uint32_t pos = (uint32_t)block_excl_scan((int)tot, s4, &total);
  if (tid == 0) a.big_ticket[row * TSTRIDE + TS_N] = total;  // the entries every pass sorts
#pragma unroll 1
  for (int t0 = 0; t0 < nt; t0 += U) {
    int32_t v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = ld_agent(&H[(int64_t)min(t0 + u, nt - 1) * RBINS + tid]);  // (clamped)
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (t0 + u < nt) H[(int64_t)(t0 + u) * RBINS + tid] = (int32_t)pos;
      pos += t0 + u < nt ? (uint32_t)v[u] : 0u;
    }
  }
}

// Grid: rows x big_tiles.  The sort keys of the tile's ids and the first
// pass's digit counts.
template <bool HAS_MASK, bool HAS_CTL>
__global__ __launch_bounds__(BLOCK) void big_key_kernel(Args a) {
  __shared__ struct { uint2 ent[NWAVE][SPT * 256]; } Kl;  // per wave: (value bits, id) for the exact p
  __shared__ double expt[64];
  __shared__ uint32_t hist[RBINS];
  __shared__ int32_t s4[NWAVE];
  __shared__ int32_t last;
  const int row = blockIdx.x / a.big_tiles, tile = blockIdx.x % a.big_tiles;
  Cfg cfg;
  const BigRow* br = big_live(a, row, cfg);
  if (!br) return;
  const float m_s = br->m_s, S = br->S;
  const int tid = threadIdx.x;
  const int enc = (int)a.enc;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;
  const int fmax = (enc - 1) >> 2;
  const int s0 = tile * SPT;
  const int ns = min(SPT, a.nslots - s0);
  float4 q[SPT];
  uint32_t mw[SPT];
#pragma unroll
  for (int j = 0; j < SPT; j++) {
    const int f = min((s0 + j) * BLOCK + tid, fmax);
    q[j] = reinterpret_cast<const float4*>(rowp)[f];
    mw[j] = HAS_MASK ? mrow[f >> 3] : 0xFFFFFFFFu;
  }
  CtlRow cr{};
  const uint64_t* pl = nullptr;
  int pc = 0, phi = 0;
  if (HAS_CTL) {
    // the chunk's patches from its first (ctl_slot passes over earlier slots')
    const int chunk = s0 / SPC;
    cr = a.ctl_row[row];
    pl = a.patch + (int64_t)row * a.ctl_cap;
    pc = a.ctl_chunk[(int64_t)row * (a.n_chunks + 1) + chunk];
    phi = a.ctl_chunk[(int64_t)row * (a.n_chunks + 1) + chunk + 1];
  }
  const bool ctl_on = HAS_CTL && cr.active;
  const bool cut = a.big_cut && br->kk == enc;  // p < 1.75 * 2^-26 stays out of the sort (KCUT)
  if (tid < 64) expt[tid] = (&kExpT[0][0])[tid];
  hist[tid] = 0u;
  __syncthreads();
  uint64_t* const A = a.big + (int64_t)row * 2 * a.big_ld;
  const int lane = lane_id(), wave = wave_id();
  int nl = 0;  // this wave's ids left for the exact p (a cut row)
  const float invS = 1.0f / S;
#pragma unroll
  for (int j = 0; j < SPT; j++) {
    if (j >= ns) break;  // (uniform)
    const int sb = (s0 + j) * SLOT;
    const int id0 = sb + 4 * tid;
    float x[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if (id0 + e >= enc) x[e] = -INFINITY;
      else if (HAS_MASK && !((mw[j] >> ((id0 + e) & 31)) & 1u)) x[e] = -INFINITY;
    }
    if (ctl_on) ctl_slot(x, sb, tid, pl, pc, phi, cr.pull_id, cr.pull_val, cr.force_id, cr.force_val);
    if (cut) {
      // the plain estimate decides the ids well below the cut; the others go
      // to the wave's list, for the exact p below with every lane busy
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int id = id0 + e;
        const bool in = id < enc;
        const float sv = cfg.scale ? x[e] * cfg.inv : x[e];
        const float pa = xexp2((sv - m_s) * LOG2E) * invS;
        const bool need = in && !(pa < PLO);
        const uint64_t b = __ballot(need);
        if (need) Kl.ent[wave][nl + lanes_below(b)] = make_uint2(__float_as_uint(x[e]), (uint32_t)id);
        nl += (int)__popcll(b);
        if (in && !need) A[id] = ((uint64_t)KSENT << 32) | (uint32_t)id;
      }
      continue;
    }
    uint32_t k[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      k[e] = pkey(exact_p(x[e], cfg, m_s, S, expt));
      count_digit(hist, rdigit(k[e], 0), id0 + e < enc);
    }
    if (id0 + 3 < enc) {
#pragma unroll
      for (int e = 0; e < 4; e++) A[id0 + e] = ((uint64_t)k[e] << 32) | (uint32_t)(id0 + e);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (id0 + e < enc) A[id0 + e] = ((uint64_t)k[e] << 32) | (uint32_t)(id0 + e);
    }
  }
  if (cut) {
    wave_lds_sync();
#pragma unroll 1
    for (int b0 = 0; b0 < nl; b0 += 64) {
      const int i = b0 + lane;
      const bool v = i < nl;
      const uint2 it = Kl.ent[wave][v ? i : 0];
      uint32_t k = pkey(exact_p(__uint_as_float(it.x), cfg, m_s, S, expt));
      if (k > KCUT) k = KSENT;  // (below the cut after all)
      count_digit(hist, rdigit(k, 0), v && k != KSENT);
      if (v) A[it.y] = ((uint64_t)k << 32) | it.y;
    }
  }
  __syncthreads();
  big_counts(a, row, tile, hist[tid], s4, last, a.big_tiles);
}

// The entries a row's passes after the first sort: all of them, or those at
// p >= 2^-26 (KCUT), as the first pass's counts found.
XS_DEV int big_sorted(const Args& a, int row) { return a.big_ticket[row * TSTRIDE + TS_N]; }
XS_DEV int big_sorted_tiles(const Args& a, int row) { return (big_sorted(a, row) + BTILE - 1) / BTILE; }
// The sorted entries a row's chains add: its kk candidates, or those the cut
// kept (every term past them is absorbed).
XS_DEV int big_chain_len(const Args& a, int row, const BigRow* br) {
  return (a.big_cut && br->kk == (int)a.enc) ? big_sorted(a, row) : br->kk;
}

// Grid: rows x big_tiles.  Pass `pass`'s digit counts of the reordered tiles.
__global__ __launch_bounds__(BLOCK) void big_hist_kernel(Args a, int pass) {
  __shared__ uint32_t hist[RBINS];
  __shared__ int32_t s4[NWAVE];
  __shared__ int32_t last;
  const int row = blockIdx.x / a.big_tiles, tile = blockIdx.x % a.big_tiles;
  Cfg cfg;
  if (!big_live(a, row, cfg)) return;
  const int ntl = big_sorted_tiles(a, row);  // the tiles the first pass filled
  if (tile >= ntl) return;
  const int tid = threadIdx.x;
  const int t0 = tile * BTILE, nt = min(BTILE, big_sorted(a, row) - t0);
  // the keys: the high words of the entries
  const uint32_t* src = reinterpret_cast<const uint32_t*>(a.big + (int64_t)row * 2 * a.big_ld +
                                                         ((pass & 1) ? a.big_ld : 0) + t0);
  uint32_t k[EPL];
#pragma unroll
  for (int s = 0; s < EPL; s++) {
    const int i = s * BLOCK + tid;
    k[s] = i < nt ? src[2 * i + 1] : 0u;
  }
  hist[tid] = 0u;
  __syncthreads();
#pragma unroll
  for (int s = 0; s < EPL; s++) count_digit(hist, rdigit(k[s], pass), s * BLOCK + tid < nt);
  __syncthreads();
  big_counts(a, row, tile, hist[tid], s4, last, ntl);
}

// One stable pass: the tile's entries go to their digit's place among all
// tiles' (big_counts' first positions).  Each wave places a quarter of the
// tile, in order, after the earlier quarters' entries of the same digit.
// Grid: rows x big_tiles.
__global__ __launch_bounds__(BLOCK) void big_scatter_kernel(Args a, int pass) {
  __shared__ uint32_t cnt[NWAVE][RBINS];  // per wave: count, then next position
  __shared__ uint64_t ent[NWAVE][QW];     // per wave: its quarter of the tile
  const int row = blockIdx.x / a.big_tiles, tile = blockIdx.x % a.big_tiles;
  Cfg cfg;
  if (!big_live(a, row, cfg)) return;
  // the first pass reads every id (in id order, KSENT on those left out),
  // the others the entries it sorted
  if (pass > 0 && tile >= big_sorted_tiles(a, row)) return;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int t0 = tile * BTILE, nt = min(BTILE, (pass == 0 ? (int)a.enc : big_sorted(a, row)) - t0);
  uint64_t* const A = a.big + (int64_t)row * 2 * a.big_ld;
  const uint64_t* src = A + ((pass & 1) ? a.big_ld : 0) + t0;
  uint64_t* dst = A + ((pass & 1) ? 0 : a.big_ld);
  const uint32_t first = a.big_hist[(int64_t)row * a.big_hld + (int64_t)tile * RBINS + tid];
  const int q0 = wave * QW;
  {
    uint64_t e[EPL];  // all of the quarter's loads in flight at once
#pragma unroll
    for (int s = 0; s < EPL; s++) {
      const int i = q0 + s * 64 + lane;
      e[s] = i < nt ? src[i] : 0ull;
    }
#pragma unroll
    for (int s = 0; s < EPL; s++) ent[wave][s * 64 + lane] = e[s];
  }
  // each wave's count of every digit in its quarter
#pragma unroll
  for (int i = lane; i < RBINS; i += 64) cnt[wave][i] = 0u;
  wave_lds_sync();
#pragma unroll 1
  for (int s = 0; s < EPL; s++) {
    const uint32_t key = (uint32_t)(ent[wave][s * 64 + lane] >> 32);
    count_digit(cnt[wave], rdigit(key, pass), q0 + s * 64 + lane < nt && key != KSENT);
    wave_lds_sync();
  }
  __syncthreads();
  // each wave's first position of every digit (thread t: digit t)
  uint32_t pos = first;
#pragma unroll
  for (int w = 0; w < NWAVE; w++) {
    const uint32_t c = cnt[w][tid];
    cnt[w][tid] = pos;
    pos += c;
  }
  __syncthreads();
  // the entries, in order
#pragma unroll 1
  for (int s = 0; s < EPL; s++) {
    const uint64_t e = ent[wave][s * 64 + lane];
    const bool valid = q0 + s * 64 + lane < nt && (uint32_t)(e >> 32) != KSENT;
    const uint32_t d = rdigit((uint32_t)(e >> 32), pass);
    const uint64_t pe = digit_peers(d, valid);
    const uint32_t at = valid ? cnt[wave][d] : 0u;
    const uint32_t p = at + (uint32_t)__popcll(pe & lanes_below());
    if (valid && p < (uint32_t)a.enc) dst[p] = e;  // (always below enc when the counts are the tiles')
    wave_lds_sync();
    if (valid && (pe & lanes_below()) == 0) cnt[wave][d] = at + (uint32_t)__popcll(pe);
    wave_lds_sync();
  }
}

// A workgroup barrier for LDS traffic only: this wave's LDS operations done,
// then s_barrier.  Unlike __syncthreads (a workgroup release fence, which on
// this target waits for every outstanding vector memory operation) it leaves
// global loads in flight, so a block's prefetched terms keep coming.
XS_DEV void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// 64-bit prefix sums over the block (in thread order); *total gets the sum.
XS_DEV uint64_t wave_incl_scan64(uint64_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t t = __shfl_up(v, (unsigned)o, 64);
    if (lane >= o) v += t;
  }
  return v;
}
XS_DEV uint64_t block_excl_scan64(uint64_t v, uint64_t* s4, uint64_t* total) {
  const int lane = lane_id(), wave = wave_id();
  const uint64_t inc = wave_incl_scan64(v);
  if (lane == 63) s4[wave] = inc;
  lds_barrier();
  uint64_t pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; w++) {
    const uint64_t t = s4[w];
    pre += (w < wave) ? t : 0ull;
    tot += t;
  }
  lds_barrier();
  *total = tot;
  return pre + inc - v;
}

struct ChainLds {
  uint64_t bu[NBU * UW];  // per block: its units at the NG binades, tie and absorb bits
  uint64_t s4[NWAVE];
  int32_t stop;    // the block's first index that ends grid stepping
  int32_t absorb;  // the block's last term rounds away at the block's grid
  int32_t hit;
  float acc;
  float w1;
};
struct ChainOut {
  float acc;  // the prefix sum through idx, or the whole sum when idx == n
  int idx;    // the first index whose prefix sum reaches the target, or n
};

// The serial f32 sum acc_{i+1} = fl(acc_i + w_i) from acc_0 = acc0 over
// terms w_0 >= w_1 >= ... >= 0 (term(i), i < n), as the reference's f32 loops
// add them one at a time, and (mode 1) the first i whose prefix is >= thr, or
// (mode 2) > thr.  The first CHEAD terms (the largest: the sum climbs through
// most of its binades there) go one at a time, by one wave.  After them, while
// the sum stays in one binade every addition lands on that binade's grid, so
// it adds rn(w_i / grid) grid units (grid_units), independent of the others:
// a block of CBLK terms then advances by an exact integer prefix sum.  Term
// by term (the hardware f32 addition) go only a term that carries the sum
// into the next binade and a term exactly half-way between grid points
// (rounded to even, which depends on the sum before it).  The terms are
// non-increasing, so once one rounds to no units, every later one does: the
// sum is final.  Every thread of the block, uniform arguments.
// The terms: conv(srt[i]), from the sorted entries.  With nbu > 0, L.bu holds
// big_units_kernel's sums for the first nbu blocks of the nu-term chain these
// terms begin (nu >= n): a block wholly inside both, whose units at the sum's
// binade keep the sum in it with no half-way term and do not reach the
// target, is crossed in one step.
template <typename CONV>
XS_DEV ChainOut big_chain(const uint64_t* srt, int n, float acc, int mode, float thr, CONV conv, ChainLds& L,
                          int nbu, int nu) {
  const int tid = threadIdx.x, lane = lane_id();
  auto reached = [&](double c) __attribute__((always_inline)) { return mode == 1 ? c >= (double)thr : c > (double)thr; };
  // 1. the head
  const int nh = min(n, CHEAD);
  if (wave_id() == 0) {
    float s = acc;
    int found = -1;
#pragma unroll 1
    for (int b = 0; b < nh && found < 0; b += 64) {
      const uint64_t rl = srt[min(b + lane, nh - 1)];
      const float wl = b + lane < nh ? conv(rl) : 0.0f;
      const int m = min(64, nh - b);
#pragma unroll 1
      for (int u = 0; u < m; u++) {
        s = s + rdlf(wl, u);
        if (mode && reached((double)s)) {
          found = b + u;
          break;
        }
      }
    }
    if (lane == 0) {
      L.acc = s;
      L.hit = found;
    }
  }
  lds_barrier();
  acc = L.acc;
  const int f = L.hit;
  lds_barrier();
  if (f >= 0) return ChainOut{acc, f};
  // 2. blocks of CBLK terms: in one step where the block's units allow, else
  // term by term as below
  float w[CPT];
#pragma unroll 1
  for (int b0 = nh, bi = 0; b0 < n; b0 += CBLK, bi++) {
    const int j0 = b0 + CPT * tid;
    const int bend = min(n, b0 + CBLK);
    if (bi < nbu && bend == min(nu, b0 + CBLK) && acc > 0.0f) {
      const int fa = f32_field(acc), g = max(fa, 1) - (FTOP - NG + 1);
      if (g >= 0 && g < NG) {
        const uint64_t* B = &L.bu[bi * UW];
        const uint64_t Ma = (__float_as_uint(acc) & 0x7FFFFFu) | (fa ? 0x800000u : 0u);
        const uint64_t end = Ma + B[g];
        const double gridv = __builtin_ldexp(1.0, max(fa, 1) - 150);
        if (!((B[NG] >> g) & 1u) && end < (1ull << 24) && !(mode && reached((double)end * gridv))) {
          acc = (float)((double)end * gridv);  // exact: below the binade's end
          if ((B[NG] >> (NG + g)) & 1u) return ChainOut{acc, n};  // every later term rounds away
          continue;
        }
      }
    }
    uint64_t r[CPT];  // clamped indices, not guarded loads: all of them in flight at once
#pragma unroll
    for (int g = 0; g < CPT; g++) r[g] = srt[min(j0 + g, n - 1)];
#pragma unroll
    for (int g = 0; g < CPT; g++) w[g] = j0 + g < n ? conv(r[g]) : 0.0f;
    int start = b0;
#pragma unroll 1
    while (start < bend) {  // (uniform)
      if (!(acc > 0.0f)) {
        // a zero sum (from -0 or +0): the next term alone
        if (j0 <= start && start < j0 + CPT) {
#pragma unroll
          for (int g = 0; g < CPT; g++)
            if (j0 + g == start) L.w1 = w[g];
        }
        lds_barrier();
        acc = acc + L.w1;
        lds_barrier();
        if (mode && reached((double)acc)) return ChainOut{acc, start};
        if (!(acc > 0.0f)) return ChainOut{acc, n};  // every later term is 0 too
        start++;
        continue;
      }
      const int fa = f32_field(acc), F = max(fa, 1);
      const uint64_t Ma = (__float_as_uint(acc) & 0x7FFFFFu) | (fa ? 0x800000u : 0u);
      const double grid = __builtin_ldexp(1.0, F - 150);
      uint32_t u[CPT];
      uint32_t ties = 0;
      uint64_t mysum = 0;
#pragma unroll
      for (int g = 0; g < CPT; g++) {
        bool t;
        const uint32_t v = grid_units_f(w[g], F, t);
        const bool live = j0 + g >= start && j0 + g < n;
        u[g] = live ? v : 0u;
        ties |= (live && t) ? (1u << g) : 0u;
        mysum += u[g];
      }
      if (tid == 0) L.stop = 0x7FFFFFFF;
      if (j0 <= bend - 1 && bend - 1 < j0 + CPT) {
#pragma unroll
        for (int g = 0; g < CPT; g++)
          if (j0 + g == bend - 1) L.absorb = (u[g] == 0u && !((ties >> g) & 1u)) ? 1 : 0;
      }
      uint64_t tot;
      const uint64_t ex = block_excl_scan64(mysum, L.s4, &tot);  // (its barriers order the stores above)
      // this thread's first stop: a tie, a carry into the next binade, or the
      // target (none when its terms hold no tie and its end stays below both:
      // the prefix only grows)
      uint64_t run = Ma + ex;
      int stop = 0x7FFFFFFF, sg = 0;
      bool hit = false;
      const bool calm = ties == 0u && run + mysum < (1ull << 24) &&
                        !(mode && reached((double)(run + mysum) * grid));
#pragma unroll
      for (int g = 0; g < CPT; g++) {
        if (!calm && stop == 0x7FFFFFFF && j0 + g >= start && j0 + g < n) {
          if (((ties >> g) & 1u) || run + u[g] >= (1ull << 24)) {
            stop = j0 + g;
            sg = g;
          } else {
            run += u[g];
            if (mode && reached((double)run * grid)) {
              stop = j0 + g;
              sg = g;
              hit = true;
            }
          }
        }
      }
      if (stop != 0x7FFFFFFF) atomicMin(&L.stop, stop);
      lds_barrier();
      const int first = L.stop;
      if (first == 0x7FFFFFFF) {
        acc = (float)((double)(Ma + tot) * grid);  // exact: below the binade's end
        const bool absorbed = L.absorb != 0;
        lds_barrier();
        if (absorbed) return ChainOut{acc, n};
        break;
      }
      if (stop == first) {
        // run: the units through the term before `first` (or through it, on a hit)
        float nv;
        bool h = hit;
        if (hit) {
          nv = (float)((double)run * grid);
        } else {
          float wv = 0.0f;
#pragma unroll
          for (int g = 0; g < CPT; g++) wv = g == sg ? w[g] : wv;
          nv = (float)((double)run * grid) + wv;  // the reference's own addition
          h = mode && reached((double)nv);
        }
        L.acc = nv;
        L.hit = h ? 1 : 0;
      }
      lds_barrier();
      acc = L.acc;
      const bool h = L.hit != 0;
      lds_barrier();
      if (h) return ChainOut{acc, first};
      start = first + 1;
    }
  }
  return ChainOut{acc, n};
}

// Grid: rows x big_nblk.  Per block of CBLK chain terms past the first CHEAD
// (the sorted entries' weights: `which` 0 the probabilities, for the sum of
// a row that top_p renormalises; 1 the weights its cut and draw add, p / sum
// or p), the block's grid units at each of the NG binades below 2^(FTOP-126),
// whether a term lies half-way between grid points there, and whether the
// block's last term rounds to no units there.  Units saturate at 2^24: a
// block with that many carries the sum out of any of these binades.
__global__ __launch_bounds__(BLOCK) void big_units_kernel(Args a, int which) {
  __shared__ uint32_t red[NWAVE][NG + 1];
  const int nb = a.big_nblk;
  const int row = blockIdx.x / nb, blk = blockIdx.x % nb;
  Cfg cfg;
  const BigRow* br = big_live(a, row, cfg);
  if (!br) return;
  const bool renorm = !(cfg.top_p >= 1.0f);
  if (which == 0 && !renorm) return;
  const float sum = br->sum;
  if (which == 1 && renorm && !(sum > 0.0f)) return;  // no chain follows
  const int kk = big_chain_len(a, row, br);
  const int b0 = CHEAD + blk * CBLK;
  if (b0 >= kk) return;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int bend = min(kk, b0 + CBLK);
  const uint64_t* srt = a.big + (int64_t)row * 2 * a.big_ld + ((RPASS & 1) ? a.big_ld : 0);
  // (the sums take the block's terms in any order: strided, so that each load
  // is one contiguous run across the block)
  uint64_t e[CPT];
#pragma unroll
  for (int g = 0; g < CPT; g++) e[g] = srt[min(b0 + g * BLOCK + tid, bend - 1)];  // (clamped, not guarded: all in flight)
  float v[CPT];
#pragma unroll
  for (int g = 0; g < CPT; g++) {
    v[g] = pkey_p((uint32_t)(e[g] >> 32));
    if (which == 1 && renorm) v[g] = __fdiv_rn(v[g], sum);
  }
  uint32_t ties = 0u, absorb = 0u;
#pragma unroll 1
  for (int f = 0; f < NG; f++) {
    uint32_t su = 0u;
#pragma unroll
    for (int g = 0; g < CPT; g++) {
      bool t;
      const int j = b0 + g * BLOCK + tid;
      const bool live = j < bend;
      const uint32_t u = grid_units_f(v[g], FTOP - NG + 1 + f, t);
      su = min(su + (live ? u : 0u), 1u << 24);
      ties |= (live && t) ? (1u << f) : 0u;
      absorb |= (j == bend - 1 && u == 0u && !t) ? (1u << f) : 0u;
    }
    const uint32_t ws = (uint32_t)wave_sumi((int)su);  // (64 x 2^24 fits)
    if (lane == 0) red[wave][f] = min(ws, 1u << 24);
  }
  const uint32_t fl = wave_or(ties | (absorb << NG));
  if (lane == 0) red[wave][NG] = fl;
  __syncthreads();
  if (tid <= NG) {
    uint64_t* U = a.big + (int64_t)row * 2 * a.big_ld + ((RPASS & 1) ? 0 : a.big_ld) +
                  (int64_t)(which * nb + blk) * UW;
    uint64_t v = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) v = tid < NG ? v + red[w][tid] : (v | red[w][tid]);
    U[tid] = tid < NG ? min(v, (uint64_t)1 << 24) : v;
  }
}

// A chain's block units into LDS (the first NBU blocks); returns how many.
XS_DEV int load_units(const Args& a, int row, int which, ChainLds& L) {
  const int nb = min(a.big_nblk, NBU);
  const uint64_t* U = a.big + (int64_t)row * 2 * a.big_ld + ((RPASS & 1) ? 0 : a.big_ld) +
                      (int64_t)which * a.big_nblk * UW;
  for (int i = threadIdx.x; i < nb * UW; i += BLOCK) L.bu[i] = U[i];
  __syncthreads();
  return nb;
}

// Grid: rows.  A row that top_p renormalises: the serial sum of its candidate
// weights (truncate_top_p's total, folded from -0.0 as Rust's f32 Sum does).
__global__ __launch_bounds__(BLOCK) void big_sum_kernel(Args a) {
  __shared__ ChainLds L;
  const int row = blockIdx.x;
  Cfg cfg;
  const BigRow* br = big_live(a, row, cfg);
  if (!br || cfg.top_p >= 1.0f) return;
  const int kk = big_chain_len(a, row, br);
  const uint64_t* srt = a.big + (int64_t)row * 2 * a.big_ld + ((RPASS & 1) ? a.big_ld : 0);
  auto pw = [&](uint64_t e) __attribute__((always_inline)) { return pkey_p((uint32_t)(e >> 32)); };
  const int nbu = load_units(a, row, 0, L);
  const float sum = big_chain(srt, kk, -0.0f, 0, 0.0f, pw, L, nbu, kk).acc;
  if (threadIdx.x == 0) a.big_state[row].sum = sum;
}

// Grid: rows.  The cut and the draw over the sorted row, the outputs.
__global__ __launch_bounds__(BLOCK) void big_draw_kernel(Args a) {
  __shared__ ChainLds L;
  const int row = blockIdx.x;
  Cfg cfg;
  const BigRow* br = big_live(a, row, cfg);
  if (!br) return;
  const int tid = threadIdx.x;
  const int kk = br->kk;
  const int n = big_chain_len(a, row, br);  // kk, or the entries the cut kept
  const uint64_t* srt = a.big + (int64_t)row * 2 * a.big_ld + ((RPASS & 1) ? a.big_ld : 0);
  auto pw = [&](uint64_t e) __attribute__((always_inline)) { return pkey_p((uint32_t)(e >> 32)); };
  const bool renorm = !(cfg.top_p >= 1.0f);
  int st = XS_ROW_OK;
  const float sum = renorm ? br->sum : 1.0f;
  int keep = kk, tok = -1;
  if (renorm && !(sum > 0.0f)) st = XS_ROW_ZERO_WEIGHT;  // weights left unchanged: no mass to draw
  if (st == XS_ROW_OK) {
    // renormalised weights (or the raw ones at top_p >= 1), their serial prefix
    // from 0 (truncate_top_p's cumsum, the same sums as WeightedIndex's
    // cumulative weights) until the cut
    auto ww = [&](uint64_t e) __attribute__((always_inline)) {
      const float v = pw(e);
      return renorm ? __fdiv_rn(v, sum) : v;
    };
    const int nbu = load_units(a, row, 1, L);
    const ChainOut c = big_chain(srt, n, 0.0f, renorm ? 1 : 0, cfg.top_p, ww, L, nbu, n);
    if (c.idx < n) keep = c.idx + 1;  // (not reached by the kept entries: not by any)
    const float tot = c.acc;  // the prefix through keep - 1
    if (!(tot > 0.0f)) {
      st = XS_ROW_ZERO_WEIGHT;
    } else {
      // the index: the cumulative weights (prefix through i, i < keep - 1; the
      // total from keep - 1 on) at or below x
      const float x = a.uniforms[row] * tot + 0.0f;
      const int m = min(keep - 1, n);
      const ChainOut d = big_chain(srt, m, 0.0f, 2, x, ww, L, nbu, n);
      const int idx = d.idx < m ? d.idx : keep - 1;
      tok = (int)(uint32_t)srt[min(idx, n - 1)];  // (past n only for a uniform of 1 or more)
    }
  }
  if (tid == 0) {
    st_agent(&a.token[row], st == XS_ROW_OK ? tok : -1);
    st_agent(&a.status[row], st);
    if (a.n_cand) a.n_cand[row] = st == XS_ROW_OK ? kk : 0;
  }
  if (st == XS_ROW_OK && (a.cand_id || a.cand_w)) {
    const int kw = (int)min((int64_t)kk, a.cand_ld);
    for (int i = tid; i < kw; i += BLOCK) {
      const uint64_t e = srt[i];
      float v = pkey_p((uint32_t)(e >> 32));
      if (renorm) v = i < keep ? __fdiv_rn(v, sum) : 0.0f;
      if (a.cand_id) a.cand_id[(int64_t)row * a.cand_ld + i] = (int32_t)(uint32_t)e;
      if (a.cand_w) a.cand_w[(int64_t)row * a.cand_ld + i] = v;
    }
  }
  if (a.span > 0 && wave_id() == 0) verify_walk(a, row);
}

}  // namespace xs

// The no-allocation entry point's workspace.  Each GPU holds its own copy at
// its own address until the process ends; host code never passes this name
// to a kernel, only the address hipGetSymbolAddress returns for the device.
static __device__ __align__(256) uint64_t scratch[xs::NA_WORDS];

// ---------------------------------------------------------------------------
// Host side: the context and the C ABI.

struct xs_context {
  int device;
  hipStream_t stream;
  int64_t max_rows, vocab;
  int32_t k_max;
  int32_t max_chunks;
  int32_t n_cu;         // compute units of the device
  int32_t xcd;          // the device's XCDs, whose round-robin placement sample_kernel's grid
                        // follows; 0: the placement was not confirmed, no call hands off XCD-locally
  int32_t xcd_test;     // test hook: 1 the split launch, 2 the placement check fails (odd chunks report another XCD)
  uint64_t* rec;
  int32_t* row_status;  // [max_rows] statuses of calls whose caller takes none (xs_argmax_probs)
  uint64_t* ctl_patch;  // [max_rows, ctl_cap] patch lists of controlled calls
  uint64_t* ctl_keys;   // [max_rows, 2, ctl_cap] sort buffers for lists past CTL_MAX (ctl_cap > CTL_MAX), or null
  int32_t ctl_cap;      // the largest control list (bans plus biases) of one row
  xs::CtlRow* ctl_row;  // [max_rows]
  int32_t* ctl_chunk;   // [max_rows, max_chunks + 1]
  int32_t* row_ticket;  // [max_rows * TSTRIDE] arrival tickets, zero between calls
  int32_t* seq_ticket;  // [max_rows * TSTRIDE]
  uint64_t* big;        // [max_rows, 2, vocab] whole-row sort buffers (k_max > XS_K_MAX), or null
  xs::BigRow* big_state;  // [max_rows] (with big)
  uint32_t* big_hist;   // [max_rows, big_tiles_max, RBINS] (with big)
  int32_t* big_ticket;  // [max_rows * TSTRIDE] (with big)
  int32_t big_tiles_max;
  uint64_t* ser_sum;    // [max_rows, max_chunks * SPC * NWAVE, 2] serial_kernel's segment summaries
  uint64_t* ser_e;      // [max_rows, SER_NB, SEG / 2] its kept terms
  uint32_t* ser_count;  // [1] rows the finalizers summed serially themselves (ser_local), or null
  int32_t ser_force;    // test hook: every checked row takes that fallback
  double* lse_ws;       // [max_rows] held_row lse of calls that score without taking row_lse
  uint64_t* score_part; // [max_rows, max_chunks, XS_CLASS_MAX] score_kernel's chunk class sums
};

namespace {

using xs_host::chunks_for;
using xs_host::slots_for;
static_assert(xs_host::SLOT == xs::SLOT && xs_host::SPC == xs::SPC, "the host checks' chunk geometry");

xs_host_limits limits_of(const xs_context* ctx) { return xs_host_limits{ctx->max_rows, ctx->vocab, ctx->max_chunks}; }

// The device's XCD count n when its placement is confirmed, else 0: a probe
// launch of 64 n workgroups records each one's XCD, and n is kept when every
// workgroup b ran on the XCD of workgroup b mod n (sample_kernel's grid puts
// a row's workgroups n apart).  Kernels still check each row's placement.
int xcd_placement(int device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, device) != hipSuccess || n < 1 || n > 16 ||
      (n & (n - 1)) != 0)
    return 0;
  const int nb = 64 * n;
  uint32_t* d = nullptr;
  if (hipMalloc((void**)&d, nb * sizeof(uint32_t)) != hipSuccess) return 0;
  hipLaunchKernelGGL(xs::xcc_probe_kernel, dim3((unsigned)nb), dim3(64), 0, nullptr, d);
  std::vector<uint32_t> h((size_t)nb);
  const bool ok = hipGetLastError() == hipSuccess &&
                  hipMemcpy(h.data(), d, nb * sizeof(uint32_t), hipMemcpyDeviceToHost) == hipSuccess;
  (void)hipFree(d);
  if (!ok) return 0;
  for (int b = 0; b < nb; b++)
    if (h[(size_t)b] != h[(size_t)(b % n)]) return 0;
  return n;
}

// One sample_kernel launch over rows x n_chunks workgroups (it finalizes the
// rows itself), or, for a large batch, sample_kernel then finalize_kernel; a
// call with sparse controls runs control_kernel (one workgroup per row) first,
// one that can observe the serial denominator serial_kernel after them, and a
// context sized for top_k >= 128 the whole-row kernels last.
template <bool M, bool S, bool C>
void launch2(xs_context* ctx, xs::Args& a, int64_t rows, dim3 g1, dim3 gs, const int32_t* order, bool loc) {
  // More workgroups than the GPU holds at once (4 per CU): the split launch,
  // unless the rows carry held_row statistics or a cost order -- their long
  // finalizers then overlap the later rows' streaming inside one launch (C5:
  // 75 us in one launch, 91 us split; C4: 57.2 us in one, 55.4 us split).
  a.split = ((g1.x > (unsigned)(4 * ctx->n_cu) && !S && !order) || ctx->xcd_test == 1) ? 1 : 0;
  if (C) hipLaunchKernelGGL((xs::control_kernel<M>), dim3((unsigned)rows), dim3(xs::BLOCK), 0, ctx->stream, a);
  // (a call of fewer rows than XCDs drops its row order: its rows all start
  // at once, and outputs do not depend on the order)
  if (order && loc) {
    xs::RowOrder<true> ro;
    for (int64_t i = 0; i < rows; i++) ro.v[i] = (uint16_t)order[i];
    hipLaunchKernelGGL((xs::sample_kernel<M, S, C, true, true>), gs, dim3(xs::BLOCK), 0, ctx->stream, a, ro);
  } else if (loc) {
    hipLaunchKernelGGL((xs::sample_kernel<M, S, C, false, true>), gs, dim3(xs::BLOCK), 0, ctx->stream, a,
                       xs::RowOrder<false>{});
  } else {
    hipLaunchKernelGGL((xs::sample_kernel<M, S, C, false, false>), gs, dim3(xs::BLOCK), 0, ctx->stream, a,
                       xs::RowOrder<false>{});
  }
  if (a.split) hipLaunchKernelGGL((xs::finalize_kernel<M, S, C>), dim3((unsigned)rows), dim3(xs::BLOCK), 0, ctx->stream, a);
  if ((M || C) && a.serial) hipLaunchKernelGGL((xs::serial_kernel<M, C>), g1, dim3(xs::BLOCK), 0, ctx->stream, a);
  // a call that may hold top_k >= 128 on a context sized for it: the
  // whole-row kernels (rows not drawn there return at once)
  if (a.big && !a.greedy_all && a.k_max > XS_K_MAX) {
    const dim3 gt((unsigned)(rows * a.big_tiles));
    hipLaunchKernelGGL((xs::big_key_kernel<M, C>), gt, dim3(xs::BLOCK), 0, ctx->stream, a);
    for (int pass = 0; pass < xs::RPASS; pass++) {
      if (pass > 0) hipLaunchKernelGGL(xs::big_hist_kernel, gt, dim3(xs::BLOCK), 0, ctx->stream, a, pass);
      hipLaunchKernelGGL(xs::big_scatter_kernel, gt, dim3(xs::BLOCK), 0, ctx->stream, a, pass);
    }
    const dim3 gb((unsigned)(rows * a.big_nblk));
    if (a.big_nblk > 0) hipLaunchKernelGGL(xs::big_units_kernel, gb, dim3(xs::BLOCK), 0, ctx->stream, a, 0);
    hipLaunchKernelGGL(xs::big_sum_kernel, dim3((unsigned)rows), dim3(xs::BLOCK), 0, ctx->stream, a);
    if (a.big_nblk > 0) hipLaunchKernelGGL(xs::big_units_kernel, gb, dim3(xs::BLOCK), 0, ctx->stream, a, 1);
    hipLaunchKernelGGL(xs::big_draw_kernel, dim3((unsigned)rows), dim3(xs::BLOCK), 0, ctx->stream, a);
  }
}

// order: null, or a host permutation of the rows (checked by the caller,
// rows <= XS_ORDER_MAX).  serial: the call can observe the serial denominator
// of its controlled rows at top_p >= 1 (serial_kernel then finalizes them);
// the controlled rows of top_k >= 128 always take it.
int launch(xs_context* ctx, xs::Args& a, int64_t rows, int span, bool mask, bool lse, bool serial,
           const int32_t* order = nullptr) {
  const bool ctl = a.controls != nullptr;
  const int64_t grid = rows * (int64_t)a.n_chunks;
  if (grid == 0) return XS_OK;
  // sample_kernel's grid: whole groups of xcd rows, all workgroups of a row on
  // one XCD (the XCD-local hand-off), when the context confirmed the placement
  // and the call has at least 8 rows per XCD; otherwise row-major, each row
  // spread over every XCD, handing off through memory.  (Measured: C2's 64
  // rows 19.58 -> 19.12 us, C4 54.2 -> 49.2, C5 71.8 -> 67.4 with it; C3's 32
  // masked rows 16.94 -> 17.45 and a lone row, through one XCD's share of
  // the bandwidth, 8.86 -> 9.28 us greedy.)
  const bool loc = ctx->xcd > 0 && rows >= 8 * (int64_t)ctx->xcd;
  const int nx = loc ? ctx->xcd : 1;
  a.xcd_log2 = __builtin_ctz((unsigned)nx);
  a.nrows = (int32_t)rows;
  a.xcd_test = ctx->xcd_test;
  const int64_t gpad = (rows + nx - 1) / nx * nx * (int64_t)a.n_chunks;
  a.fold_shared = gpad <= 4 * (int64_t)ctx->n_cu ? 1 : 0;  // (alike for a split launch of the same call)
  if (gpad > 0x7FFFFFFF || span < 1) return XS_ERR_CAPACITY;
  // (no instantiation streams a masked or controlled row with held_row's
  // statistics: sample_impl splits such a call into two launches)
  if ((mask || ctl) && lse) return XS_ERR_ARG;
  a.patch = ctx->ctl_patch;
  a.ctl_keys = ctx->ctl_keys;
  a.ctl_cap = ctx->ctl_cap;
  a.ctl_row = ctx->ctl_row;
  a.ctl_chunk = ctx->ctl_chunk;
  a.row_ticket = ctx->row_ticket;
  a.seq_ticket = ctx->seq_ticket;
  a.k_max = (a.k_max > 0 && a.k_max < ctx->k_max) ? a.k_max : ctx->k_max;  // the call's bound, if tighter
  a.big = ctx->big;
  a.big_ld = ctx->vocab;
  a.big_state = ctx->big_state;
  a.big_hist = ctx->big_hist;
  a.big_hld = (int64_t)ctx->big_tiles_max * xs::RBINS;
  a.big_ticket = ctx->big_ticket;
  a.big_tiles = (int32_t)((a.enc + xs::BTILE - 1) / xs::BTILE);
  a.big_nblk = (int32_t)(a.enc > xs::CHEAD ? (a.enc - xs::CHEAD + xs::CBLK - 1) / xs::CBLK : 0);
  a.big_cut = (a.big && !a.cand_id && !a.cand_w && a.enc <= (1 << 20)) ? 1 : 0;
  if (a.big && rows * (int64_t)a.big_tiles > 0x7FFFFFFF) return XS_ERR_CAPACITY;  // the whole-row grids
  const bool big_rows = a.big && !a.greedy_all && a.k_max > XS_K_MAX;
  a.serial = (mask || ctl) ? ((serial ? 1 : 0) | (big_rows ? 2 : 0)) : 0;
  a.ser_count = ctx->ser_count;
  a.ser_force = ctx->ser_force;
  a.ser_sum = ctx->ser_sum;
  a.ser_e = ctx->ser_e;
  a.ser_ld = (int64_t)ctx->max_chunks * xs::SPC * xs::NWAVE;
  const dim3 g1((unsigned)grid), gs((unsigned)gpad);
  if (ctl && mask) launch2<true, false, true>(ctx, a, rows, g1, gs, order, loc);
  else if (ctl) launch2<false, false, true>(ctx, a, rows, g1, gs, order, loc);
  else if (mask) launch2<true, false, false>(ctx, a, rows, g1, gs, order, loc);
  else if (lse) launch2<false, true, false>(ctx, a, rows, g1, gs, order, loc);
  else launch2<false, false, false>(ctx, a, rows, g1, gs, order, loc);
  return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
}

}  // namespace

extern "C" {

const char* xs_version(void) { return "xsamp 0.1 gfx950"; }

int xs_create(int device, int64_t max_rows, int64_t vocab, int32_t k_max, xs_context** out) {
  return xs_create_ex(device, max_rows, vocab, k_max, XS_CTL_MAX, out);
}

int xs_create_ex(int device, int64_t max_rows, int64_t vocab, int32_t k_max, int32_t ctl_max,
                 xs_context** out) {
  if (!out || max_rows < 1 || vocab < 1 || k_max < 0 || ctl_max < 0) return XS_ERR_ARG;
  *out = nullptr;
  if (hipSetDevice(device) != hipSuccess) return XS_ERR_HIP;
  const int32_t mc = chunks_for(vocab);
  if (mc * xs::NWAVE > xs::GMAX * 64) return XS_ERR_CAPACITY;  // sub-records a finalizing wave reads
  xs_context* c = (xs_context*)calloc(1, sizeof(xs_context));
  if (!c) return XS_ERR_HIP;
  c->device = device;
  c->stream = nullptr;
  c->max_rows = max_rows;
  c->vocab = vocab;
  c->k_max = k_max;
  c->max_chunks = mc;
  if (hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || c->n_cu < 1)
    c->n_cu = 256;
  c->xcd = xcd_placement(device);
  c->ctl_cap = ctl_max > xs::CTL_MAX ? ctl_max : xs::CTL_MAX;
  const int64_t nsp = ((int64_t)mc * xs::NWAVE + 63) / 64 * 64;  // sub-records per row, padded
  const int64_t units = max_rows * nsp;
  bool ok = hipMalloc((void**)&c->rec, units * xs::SRECW * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMemset(c->rec, 0, units * xs::SRECW * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->row_status, max_rows * sizeof(int32_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->ctl_patch, max_rows * c->ctl_cap * sizeof(uint64_t)) == hipSuccess;
  if (c->ctl_cap > xs::CTL_MAX)  // lists past CTL_MAX: control_kernel sorts them in memory
    ok = ok && hipMalloc((void**)&c->ctl_keys, (size_t)max_rows * 2 * c->ctl_cap * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->ctl_row, max_rows * sizeof(xs::CtlRow)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->ctl_chunk, max_rows * (mc + 1) * sizeof(int32_t)) == hipSuccess;
  const size_t tbytes = (size_t)max_rows * xs::TSTRIDE * sizeof(int32_t);
  ok = ok && hipMalloc((void**)&c->row_ticket, tbytes) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->seq_ticket, tbytes) == hipSuccess;
  ok = ok && hipMemset(c->row_ticket, 0, tbytes) == hipSuccess;
  ok = ok && hipMemset(c->seq_ticket, 0, tbytes) == hipSuccess;
  const int64_t nseg = (int64_t)mc * xs::SPC * xs::NWAVE;
  ok = ok && hipMalloc((void**)&c->ser_sum, max_rows * nseg * 2 * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->ser_e, max_rows * xs::SER_NB * (xs::SEG / 2) * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->ser_count, sizeof(uint32_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->lse_ws, max_rows * sizeof(double)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->score_part, (size_t)max_rows * mc * XS_CLASS_MAX * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMemset(c->ser_count, 0, sizeof(uint32_t)) == hipSuccess;
  if (k_max > XS_K_MAX) {  // top_k past the streaming selection: the whole-row path's buffers
    ok = ok && hipMalloc((void**)&c->big, (size_t)max_rows * 2 * vocab * sizeof(uint64_t)) == hipSuccess;
    ok = ok && hipMalloc((void**)&c->big_state, (size_t)max_rows * sizeof(xs::BigRow)) == hipSuccess;
    c->big_tiles_max = (int32_t)((vocab + xs::BTILE - 1) / xs::BTILE);
    ok = ok && hipMalloc((void**)&c->big_hist, (size_t)max_rows * c->big_tiles_max * xs::RBINS * sizeof(uint32_t)) == hipSuccess;
    ok = ok && hipMalloc((void**)&c->big_ticket, tbytes) == hipSuccess;
    ok = ok && hipMemset(c->big_ticket, 0, tbytes) == hipSuccess;
  }
  ok = ok && hipDeviceSynchronize() == hipSuccess;
  if (!ok) {
    xs_destroy(c);
    return XS_ERR_HIP;
  }
  *out = c;
  return XS_OK;
}

int xs_destroy(xs_context* c) {
  if (!c) return XS_OK;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream); else (void)hipDeviceSynchronize();
  (void)hipFree(c->rec);
  (void)hipFree(c->row_status);
  (void)hipFree(c->ctl_patch);
  if (c->ctl_keys) (void)hipFree(c->ctl_keys);
  (void)hipFree(c->ctl_row);
  (void)hipFree(c->ctl_chunk);
  (void)hipFree(c->row_ticket);
  (void)hipFree(c->seq_ticket);
  if (c->big) (void)hipFree(c->big);
  if (c->big_state) (void)hipFree(c->big_state);
  if (c->big_hist) (void)hipFree(c->big_hist);
  if (c->big_ticket) (void)hipFree(c->big_ticket);
  (void)hipFree(c->ser_sum);
  (void)hipFree(c->ser_e);
  if (c->ser_count) (void)hipFree(c->ser_count);
  if (c->lse_ws) (void)hipFree(c->lse_ws);
  if (c->score_part) (void)hipFree(c->score_part);
  free(c);
  return XS_OK;
}

int xs_set_stream(xs_context* c, void* s) {
  if (!c) return XS_ERR_ARG;
  c->stream = (hipStream_t)s;
  return XS_OK;
}

namespace {
int sample_impl(xs_context* ctx, const xs_sample_args* in, bool clear_tickets);
}

int xs_sample(xs_context* ctx, const xs_sample_args* in) { return sample_impl(ctx, in, false); }

namespace {
int sample_impl(xs_context* ctx, const xs_sample_args* in, bool clear_tickets) {
  if (!ctx) return XS_ERR_ARG;
  const xs_host_limits lim = limits_of(ctx);
  const int rc = xs_host_check_sample(&lim, in);
  if (rc) return rc;
  const bool lse = xs_host_wants_lse(in);
  const bool scores = xs_host_wants_scores(in);
  if (scores && !ctx->lse_ws) return XS_ERR_ARG;  // (the static workspace of xs_sample_noalloc holds none)
  if (hipSetDevice(ctx->device) != hipSuccess) return XS_ERR_HIP;
  int32_t data_err = XS_ROW_OK;
  if (in->width < in->enc) data_err = XS_ROW_NARROW;
  else if (in->allowed && in->allowed_words * 32 < in->enc) data_err = XS_ROW_MASK_SHORT;
  if (data_err != XS_ROW_OK) {
    if (in->rows == 0) return XS_OK;
    const unsigned blocks = (unsigned)((in->rows + 255) / 256);
    hipLaunchKernelGGL(xs::fill_status_kernel, dim3(blocks), dim3(256), 0, ctx->stream, in->token,
                       in->status, in->n_cand, in->rows, data_err);
    return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
  }
  xs::Args a;
  memset(&a, 0, sizeof(a));
  a.logits = in->logits;
  a.ld = in->ld;
  a.enc = in->enc;
  a.params = in->params;
  a.uniforms = in->uniforms;
  a.allowed = in->allowed;
  a.allowed_ld = in->allowed_ld;
  a.token = in->token;
  a.status = in->status;
  a.cand_id = in->cand_id;
  a.cand_w = in->cand_w;
  a.n_cand = in->n_cand;
  a.cand_ld = in->cand_ld;
  a.soft_max = in->soft_max;
  a.soft_sum = in->soft_sum;
  a.row_max = in->row_max;
  a.row_lse = in->row_lse ? in->row_lse : (scores ? ctx->lse_ws : nullptr);
  a.n_top = (in->top_id || in->top_logprob || in->top_logprob64) ? in->n_top : 0;
  a.top_id = in->top_id;
  a.top_logprob = in->top_logprob;
  a.top_logprob64 = in->top_logprob64;
  a.score_ids = in->score_ids;
  a.n_score = in->score_ids ? in->n_score : 0;
  a.score_ld = in->score_ld;
  a.score_logprob = in->score_logprob;
  a.class_masks = in->class_masks;
  a.n_class = in->class_masks ? in->n_class : 0;
  a.class_ld = in->class_ld;
  a.class_mass = in->class_mass;
  a.probs = in->probs;
  a.probs_ld = in->probs_ld;
  a.score_part = ctx->score_part;
  a.top_ld = in->top_ld;
  a.controls = in->controls;
  a.ctl_ids = in->ctl_ids;
  a.ctl_delta = in->ctl_delta;
  a.k_max = in->k_max;  // (0: the context's)
  a.span = 0;
  a.n_chunks = chunks_for(in->enc);
  a.nslots = (int32_t)slots_for(in->enc);
  a.rec = ctx->rec;
  if (clear_tickets && in->rows > 0) {
    const int64_t n = in->rows * xs::TSTRIDE;
    hipLaunchKernelGGL(xs::zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream,
                       ctx->row_ticket, n);
  }
  // the serial denominator shows in the candidate weights and in soft_sum of
  // rows at top_p >= 1; every other controlled row draws with the exact sum,
  // and a row whose token that sum does not settle is summed serially by its
  // finalizer (draw_settled, ser_local)
  bool serial = in->cand_id || in->cand_w || in->soft_sum;
  // (the launch's arguments carry an order of at most XS_ORDER_MAX rows)
  const int32_t* order = in->rows <= XS_ORDER_MAX ? in->row_order : nullptr;
  const bool masked = in->allowed != nullptr || in->controls != nullptr;
  if (lse && masked) {
    // held_row reads the raw row (generate.rs:1905-1933), whatever mask or
    // controls the draw takes: the masked draw runs without the held_row
    // outputs, then a second pass over the raw rows, every row greedy at T 1,
    // writes them (its tokens and statuses land in row_status, unread)
    xs::Args d = a;
    d.row_max = nullptr;
    d.row_lse = nullptr;
    d.n_top = 0;
    d.top_id = nullptr;
    d.top_logprob = nullptr;
    d.top_logprob64 = nullptr;
    d.n_score = 0;
    d.score_ids = nullptr;
    d.n_class = 0;
    d.class_masks = nullptr;
    d.probs = nullptr;
    const int drc = launch(ctx, d, in->rows, 1, in->allowed != nullptr, false, serial, order);
    if (drc != XS_OK) return drc;
    a.params = nullptr;
    a.uniforms = nullptr;
    a.allowed = nullptr;
    a.controls = nullptr;
    a.ctl_ids = nullptr;
    a.ctl_delta = nullptr;
    a.token = ctx->row_status;
    a.status = ctx->row_status;
    a.cand_id = nullptr;
    a.cand_w = nullptr;
    a.n_cand = nullptr;
    a.soft_max = nullptr;
    a.soft_sum = nullptr;
    a.greedy_all = 1;
    order = nullptr;
    serial = false;
  }
  const int lrc = launch(ctx, a, in->rows, 1, a.allowed != nullptr, lse, serial, order);
  if (lrc != XS_OK || !scores || in->rows == 0) return lrc;
  // the scoring reads, once every row's lse is written (an id out of range
  // fails the caller's row)
  a.token = in->token;
  a.status = in->status;
  hipLaunchKernelGGL(xs::score_kernel, dim3((unsigned)(in->rows * a.n_chunks)), dim3(xs::BLOCK), 0, ctx->stream, a);
  return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
}
}  // namespace

// The device address of `scratch` on each device, looked up once per device
// (with that device current) and kept for the process.
namespace {
constexpr int NA_MAX_DEVICES = 64;
std::mutex na_mu;
uint64_t* na_ptr[NA_MAX_DEVICES];

int na_cu[NA_MAX_DEVICES];

int na_cus(int dev) {  // the device's compute units, asked once
  std::lock_guard<std::mutex> g(na_mu);
  if (na_cu[dev] < 1 && (hipDeviceGetAttribute(&na_cu[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                         na_cu[dev] < 1))
    na_cu[dev] = 256;
  return na_cu[dev];
}

// The device's XCD count, asked once (no probe launch: this entry point may
// run under graph capture; sample_kernel checks each row's placement), or 0
// when the device does not report one: no call then hands off XCD-locally.
int na_xcd[NA_MAX_DEVICES];
bool na_xcd_known[NA_MAX_DEVICES];
int na_xcds(int dev) {
  std::lock_guard<std::mutex> g(na_mu);
  if (!na_xcd_known[dev]) {
    int n = 0;
    na_xcd[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && n >= 1 && n <= 16 &&
                   (n & (n - 1)) == 0) ? n : 0;
    na_xcd_known[dev] = true;
  }
  return na_xcd[dev];
}

uint64_t* noalloc_scratch(int dev) {
  std::lock_guard<std::mutex> g(na_mu);
  if (!na_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    na_ptr[dev] = (uint64_t*)p;
  }
  return na_ptr[dev];
}
}  // namespace

int xs_sample_noalloc(const xs_sample_args* in, void* hip_stream) {
  if (!in) return XS_ERR_ARG;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return XS_ERR_HIP;
  if (dev < 0 || dev >= NA_MAX_DEVICES) return XS_ERR_CAPACITY;
  uint64_t* base = noalloc_scratch(dev);
  if (!base) return XS_ERR_HIP;
  // a context on the host stack that describes the static workspace
  xs_context c;
  memset(&c, 0, sizeof(c));
  c.device = dev;
  c.stream = (hipStream_t)hip_stream;
  c.max_rows = xs::NA_ROWS;
  c.vocab = xs::NA_VOCAB;
  c.k_max = XS_K_MAX;
  c.max_chunks = (int32_t)xs::NA_CHUNKS;
  c.n_cu = na_cus(dev);
  c.xcd = na_xcds(dev);
  c.rec = base + xs::NA_OFF_REC;
  c.ctl_patch = base + xs::NA_OFF_PATCH;
  c.ctl_cap = xs::CTL_MAX;
  c.ctl_row = reinterpret_cast<xs::CtlRow*>(base + xs::NA_OFF_CTLROW);
  c.ctl_chunk = reinterpret_cast<int32_t*>(base + xs::NA_OFF_CTLCHUNK);
  c.row_ticket = reinterpret_cast<int32_t*>(base + xs::NA_OFF_TICKET);
  c.seq_ticket = reinterpret_cast<int32_t*>(base + xs::NA_OFF_SEQ);
  c.row_status = reinterpret_cast<int32_t*>(base + xs::NA_OFF_STATUS);
  c.ser_sum = base + xs::NA_OFF_SERSUM;
  c.ser_e = base + xs::NA_OFF_SERE;
  return sample_impl(&c, in, true);
}

int xs_verify(xs_context* ctx, const xs_verify_args* in) {
  if (!ctx) return XS_ERR_ARG;
  const xs_host_limits lim = limits_of(ctx);
  const int rc = xs_host_check_verify(&lim, in);
  if (rc) return rc;
  const int64_t rows = in->seqs * in->span;
  if (hipSetDevice(ctx->device) != hipSuccess) return XS_ERR_HIP;
  int32_t data_err = XS_ROW_OK;
  if (in->width < in->enc) data_err = XS_ROW_NARROW;
  else if (in->allowed && in->allowed_words * 32 < in->enc) data_err = XS_ROW_MASK_SHORT;
  if (data_err != XS_ROW_OK) {
    if (rows == 0) return XS_OK;
    const unsigned blocks = (unsigned)((rows + 255) / 256);
    hipLaunchKernelGGL(xs::fill_verify_kernel, dim3(blocks), dim3(256), 0, ctx->stream, *in, data_err);
    return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
  }
  xs::Args a;
  memset(&a, 0, sizeof(a));
  a.logits = in->logits;
  a.ld = in->ld;
  a.enc = in->enc;
  a.params = in->params;
  a.uniforms = in->uniforms;
  a.allowed = in->allowed;
  a.allowed_ld = in->allowed_ld;
  a.token = in->row_token;
  a.status = in->row_status;
  a.span = (int32_t)in->span;
  a.drafts = in->drafts;
  a.budget = in->budget;
  a.n_eog = in->n_eog;
  a.eog = in->eog;
  a.accepted = in->accepted;
  a.committed = in->committed;
  a.n_committed = in->n_committed;
  a.seq_status = in->seq_status;
  a.done_after = in->done_after;
  a.controls = in->controls;
  a.ctl_ids = in->ctl_ids;
  a.ctl_delta = in->ctl_delta;
  a.k_max = in->k_max;  // (0: the context's)
  a.n_chunks = chunks_for(in->enc);
  a.nslots = (int32_t)slots_for(in->enc);
  a.rec = ctx->rec;
  // tokens are all it returns: the exact sum, checked (draw_settled)
  return launch(ctx, a, rows, (int)in->span, in->allowed != nullptr, false, false);
}

int xs_argmax_probs(xs_context* ctx, const xs_argmax_args* in) {
  if (!ctx) return XS_ERR_ARG;
  const xs_host_limits lim = limits_of(ctx);
  const int rc = xs_host_check_argmax(&lim, in);
  if (rc) return rc;
  if (hipSetDevice(ctx->device) != hipSuccess) return XS_ERR_HIP;
  xs::Args a;
  memset(&a, 0, sizeof(a));
  a.logits = in->logits;
  a.ld = in->ld;
  a.enc = in->width;  // the whole row: the reference reduces the raw lm_head output
  a.token = in->ids;
  a.status = ctx->row_status;
  a.greedy_all = 1;
  a.p_max = in->probs;
  a.n_chunks = chunks_for(in->width);
  a.nslots = (int32_t)slots_for(in->width);
  a.rec = ctx->rec;
  return launch(ctx, a, in->rows, 1, false, true, false);
}

int xs_test_serial_fallback(xs_context* c, int32_t force, uint32_t* count) {
  if (!c) return XS_ERR_ARG;
  if (hipSetDevice(c->device) != hipSuccess) return XS_ERR_HIP;
  if (count) {
    if ((c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize()) != hipSuccess) return XS_ERR_HIP;
    if (hipMemcpy(count, c->ser_count, sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) return XS_ERR_HIP;
  }
  c->ser_force = force != 0 ? 1 : 0;
  return XS_OK;
}

int xs_test_xcd(xs_context* c, int32_t mode, int32_t* xcd) {
  if (!c || mode < 0 || mode > 2) return XS_ERR_ARG;
  if (xcd) *xcd = c->xcd;
  c->xcd_test = mode;
  return XS_OK;
}

int xs_test_exp(const float* x, float* y, int64_t n, void* s) {
  if (n < 0 || (n > 0 && (!x || !y))) return XS_ERR_ARG;
  if (n == 0) return XS_OK;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(xs::exp_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)s, x, y, n);
  return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
}

}  // extern "C"
