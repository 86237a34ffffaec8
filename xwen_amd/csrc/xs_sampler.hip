// xs_sampler.hip -- MI355X (gfx950) token sampler: one fused launch per batch.
//
// The reference (0rvar/xwen src/sampler.rs) reads each logit row back to the
// host and runs softmax -> streaming top-k -> top-p -> WeightedIndex on the CPU.
// Here one kernel does the whole draw on the device:
//
//   chunk pass   every workgroup streams one chunk of one row from HBM exactly
//                once (16-byte loads, one slot = 256 lanes x float4), applies
//                the allow-mask, and reduces the chunk: max, NaN/finite flags,
//                the softmax partial sum, the held_row f64 partial sum, and a
//                candidate list that provably holds the chunk's K' best
//                (logit desc, id asc) entries.  The candidate bound is the K'-th
//                largest lane maximum of the block (lane maxima are distinct
//                elements, so at least K' elements lie at or above it).
//   finalize     the last workgroup of a row (atomic ticket) merges the chunk
//                summaries and candidate lists, recomputes the exact f32
//                probability of the K' = top_k + 1 survivors with a correctly
//                rounded exp, orders them by (p desc, id asc) -- the
//                reference's top_k_desc order -- proves the k-th boundary is
//                not a probability tie reaching past the survivors (or scans
//                the row for the lowest tied ids when it is), then runs the
//                reference's serial f32 top-p cut and WeightedIndex draw.
//   verify       for a speculative block, the last row finalizer of a
//                sequence runs accept_drafts over the sequence's rows.
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
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/xsamp.h"
#include "xs_exp_table.h"

#define XS_DEV __device__ __forceinline__

typedef float v4f __attribute__((ext_vector_type(4)));

namespace xs {

constexpr int BLOCK = 256;          // lanes per workgroup
constexpr int NWAVE = BLOCK / 64;   // wave64
constexpr int SLOT = BLOCK * 4;     // elements per slot: one float4 per lane
constexpr int SPC = 16;             // slots per chunk (16,384 logits, 64 KiB)
constexpr int KSEL = 128;           // largest selection size K'
constexpr int CAP = 1024;           // candidate entries per chunk
constexpr int QPUB = 32;            // sorted lane maxima a chunk publishes
constexpr int SURV = 2048;          // survivor entries the finalizer ranks
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

XS_DEV float cr_expf(float xf) {
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
  const double th = kExpT[j][0], tl = kExpT[j][1];
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

XS_DEV float wave_maxf(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
XS_DEV double wave_sumd(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
XS_DEV uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= (uint32_t)__shfl_xor((int)v, o);
  return v;
}
XS_DEV uint32_t wave_minu(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

// Bitonic sort, descending, of 64*R u32 keys held R per lane (element r*64+lane).
template <int R>
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
          const uint32_t b = (uint32_t)__shfl_xor((int)x[r], d);
          const bool desc = ((r * 64 + lane) & size) == 0;
          const bool lower = (lane & d) == 0;
          const uint32_t hi = max(x[r], b), lo = min(x[r], b);
          x[r] = (lower == desc) ? hi : lo;
        }
      }
    }
  }
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
// Contains barriers: call from block-uniform control flow only.
XS_DEV int block_excl_scan(int v, int* s4, int* total) {
  const int lane = lane_id(), wave = wave_id();
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
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

struct Cfg {
  float inv;     // (float)(1/T)  (softmax_in_place, sampler.rs:291)
  float top_p;
  int k;         // candidates drawn from (0 on greedy rows)
  int kp;        // selection size K'
  bool greedy, scale, full, bad;
};

XS_DEV Cfg make_cfg(const xs_row_params& p, int64_t enc, int n_top) {
  Cfg c;
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
  if (n_top > 0) c.kp = max(c.kp, (int)min((int64_t)n_top, enc));
  c.bad = c.kp > KSEL || (c.full && enc > KSEL);
  return c;
}

// ---------------------------------------------------------------------------
// Workspace and launch arguments.

struct Summary {  // one per (row, chunk)
  float vmax;     // max of the controlled logits (NaN ignored)
  float ssum;     // sum over the chunk of exp((v - vmax) * inv)   (stochastic rows)
  double rsum;    // sum over the chunk of exp(v - vmax) in f64    (held_row)
  uint32_t flags; // bit 0: a NaN was seen; bit 1: a finite value was seen
  int32_t count;  // candidate entries written
  int32_t pad0, pad1;
};

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
  int64_t top_ld;
  // verify walk (span == 0: plain batch)
  int32_t span;
  const int32_t* drafts;
  const int32_t* budget;
  int32_t n_eog;
  int32_t eog[8];
  int32_t* accepted;
  int32_t* committed;
  int32_t* n_committed;
  int32_t* seq_status;
  // geometry + workspace
  int32_t n_chunks, nslots;
  Summary* summ;
  uint32_t* pub;     // [rows, n_chunks, QPUB]
  uint64_t* cand;    // [rows, n_chunks, CAP]
  int32_t* row_ticket;
  int32_t* seq_ticket;
};

struct Lds {
  uint64_t list[SURV];     // chunk candidates / finalizer survivors
  uint64_t sel[KSEL];      // survivors in (logit desc, id asc) order
  uint64_t psel[KSEL];     // the same in (p desc, id asc) order
  float w[KSEL];           // probabilities / weights in draw order
  int32_t prefix[257];     // chunk candidate offsets
  int32_t s4[NWAVE];
  float f4[NWAVE];
  double d4[NWAVE];
  uint32_t u4[NWAVE];
  int32_t count;
  int32_t flag;
  int32_t misc[8];
};

// p = rn(e / S) of one controlled logit v (the reference's softmax_in_place:
// v *= inv unless T == 1, then exp(v - max), then / sum; sampler.rs:289-310).
XS_DEV float exact_p(float v, const Cfg& cfg, float m_s, float S) {
  const float s = cfg.scale ? v * cfg.inv : v;
  const float e = cr_expf(s - m_s);
  return __fdiv_rn(e, S);
}

// The largest float below f (f > -inf, not NaN).
XS_DEV float next_below(float f) {
  if (f == 0.0f) return -__uint_as_float(1u);
  const uint32_t b = __float_as_uint(f);
  return __uint_as_float(f > 0.0f ? b - 1u : b + 1u);
}

// Rare path of the chunk pass: more than CAP elements at or above the bound
// (ties at the bound: constant or masked stretches).  Keeps the elements
// strictly above the bound, then the lowest ids equal to it; if even the
// strict set overflows, finds the exact K'-th largest key by bisection first.
// Re-reads the chunk from memory so the streaming path keeps no registers for
// it.  Every lane of the block calls it (it contains barriers).
template <bool HAS_MASK>
__device__ __noinline__ int chunk_overflow(const float* rowp, const uint32_t* mrow, int s0, int ns,
                                           int enc, uint32_t tau_key, int kp, Lds& L) {
  const int tid = threadIdx.x;
  // Element e of lane tid in slot j; NaN marks an absent element (no compare holds).
  auto load = [&](int j, int e, int* idp) -> float {
    const int id = (s0 + j) * SLOT + 4 * tid + e;
    *idp = id;
    if (j >= ns || id >= enc) return __builtin_nanf("");
    float x = rowp[id];
    if (HAS_MASK && !((mrow[id >> 5] >> (id & 31)) & 1u)) x = -INFINITY;
    return x;
  };
  uint32_t eq_key = tau_key;
  if (tid == 0) L.count = 0;
  __syncthreads();
  for (int j = 0; j < ns; j++)
    for (int e = 0; e < 4; e++) {
      int id;
      const float x = load(j, e, &id);
      if (x == x && fkey(x) > tau_key) {
        const int pos = atomicAdd(&L.count, 1);
        if (pos < CAP) L.list[pos] = pack(fkey(x), (uint32_t)id);
      }
    }
  __syncthreads();
  int gt = L.count;
  __syncthreads();
  if (gt > CAP - KSEL) {
    uint32_t ans = 0;
    for (int bit = 31; bit >= 0; bit--) {
      const uint32_t cnd = ans | (1u << bit);
      int c = 0;
      for (int j = 0; j < ns; j++)
        for (int e = 0; e < 4; e++) {
          int id;
          const float x = load(j, e, &id);
          c += (x == x && fkey(x) >= cnd) ? 1 : 0;
        }
      int tot;
      block_excl_scan(c, L.s4, &tot);
      if (tot >= kp) ans = cnd;
    }
    eq_key = ans;
    if (tid == 0) L.count = 0;
    __syncthreads();
    for (int j = 0; j < ns; j++)
      for (int e = 0; e < 4; e++) {
        int id;
        const float x = load(j, e, &id);
        if (x == x && fkey(x) > eq_key) {
          const int pos = atomicAdd(&L.count, 1);
          if (pos < CAP) L.list[pos] = pack(fkey(x), (uint32_t)id);
        }
      }
    __syncthreads();
    gt = L.count;
    __syncthreads();
  }
  // Ties at eq_key, lowest ids first: slot j covers ids s0*SLOT + j*SLOT +
  // [0, SLOT) in lane order, so a block prefix count per slot is id order.
  int need = kp - gt, have = gt;
  for (int j = 0; j < ns && need > 0; j++) {
    int c = 0;
    float xs[4];
    int ids[4];
    for (int e = 0; e < 4; e++) {
      xs[e] = load(j, e, &ids[e]);
      c += (xs[e] == xs[e] && fkey(xs[e]) == eq_key) ? 1 : 0;
    }
    int tot;
    int pre = block_excl_scan(c, L.s4, &tot);
    for (int e = 0; e < 4; e++) {
      if (xs[e] == xs[e] && fkey(xs[e]) == eq_key) {
        if (pre < need) L.list[have + pre] = pack(eq_key, (uint32_t)ids[e]);
        pre++;
      }
    }
    have += min(tot, need);
    need -= tot;
    __syncthreads();
  }
  return have;
}

// ---------------------------------------------------------------------------
// The kernel.

template <bool HAS_MASK, bool WANT_LSE>
__global__ __launch_bounds__(BLOCK) void sample_kernel(Args a) {
  __shared__ Lds L;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int row = blockIdx.x / a.n_chunks;
  const int chunk = blockIdx.x - row * a.n_chunks;
  const int64_t enc = a.enc;
  const Cfg cfg = make_cfg(a.params[row], enc, a.n_top);
  const bool stoch = !cfg.greedy && !cfg.bad;
  const int kp = cfg.kp;

  // ---------------- chunk pass ----------------
  const int s0 = (int)((int64_t)chunk * a.nslots / a.n_chunks);
  const int s1 = (int)((int64_t)(chunk + 1) * a.nslots / a.n_chunks);
  const int ns = s1 - s0;  // <= SPC by construction of n_chunks
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const float4* rp4 = reinterpret_cast<const float4*>(rowp);
  const uint32_t* mrow = HAS_MASK ? a.allowed + (int64_t)row * a.allowed_ld : nullptr;

  float v[SPC * 4];
#pragma unroll
  for (int j = 0; j < SPC; j++) {
    const int64_t f = (int64_t)(s0 + j) * BLOCK + tid;  // float4 index in the row
    float4 q = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (j < ns && 4 * f < enc) {
      const v4f t = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(rp4 + f));
      q = make_float4(t.x, t.y, t.z, t.w);
      if (4 * f + 3 >= enc) {  // ids past the encodable bound take no part
        if (4 * f + 1 >= enc) q.y = -INFINITY;
        if (4 * f + 2 >= enc) q.z = -INFINITY;
        q.w = -INFINITY;
      }
    }
    v[4 * j + 0] = q.x;
    v[4 * j + 1] = q.y;
    v[4 * j + 2] = q.z;
    v[4 * j + 3] = q.w;
  }

  // held_row partial sum over the raw logits (no mask with WANT_LSE).
  float m_raw = -INFINITY;
  double rsum = 0.0;
  if (WANT_LSE) {
#pragma unroll
    for (int i = 0; i < SPC * 4; i++) m_raw = fmaxf(m_raw, v[i]);
    const float off = __builtin_isinf(m_raw) ? 0.0f : m_raw;
#pragma unroll
    for (int i = 0; i < SPC * 4; i++) rsum += (double)expf(v[i] - off);
  }

  uint32_t flags = 0;
  if (HAS_MASK) {
#pragma unroll
    for (int j = 0; j < SPC; j++) {
      const int64_t f = (int64_t)(s0 + j) * BLOCK + tid;
      if (j < ns && 4 * f < enc) {
        const uint32_t bits = mrow[f >> 3] >> ((f & 7) * 4);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (!((bits >> e) & 1u)) v[4 * j + e] = -INFINITY;
      }
    }
#pragma unroll
    for (int i = 0; i < SPC * 4; i++) flags |= (__builtin_fabsf(v[i]) < INFINITY) ? 2u : 0u;
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < SPC * 4; i++) {
    m = fmaxf(m, v[i]);
    flags |= (v[i] != v[i]) ? 1u : 0u;
  }
  // Softmax partial sum in the reference's scaled domain: s = v * inv rounded to
  // f32 exactly as softmax_in_place does, then exp(s - off_s) with off_s the
  // lane's scaled max, so each term carries the reference's own roundings.
  float ssum = 0.0f;
  const float off = (m == -INFINITY) ? 0.0f : m;
  const float off_s = cfg.scale ? off * cfg.inv : off;
  if (stoch) {
    if (cfg.scale) {
#pragma unroll
      for (int i = 0; i < SPC * 4; i++) ssum += __builtin_amdgcn_exp2f((v[i] * cfg.inv - off_s) * LOG2E);
    } else {
#pragma unroll
      for (int i = 0; i < SPC * 4; i++) ssum += __builtin_amdgcn_exp2f((v[i] - off_s) * LOG2E);
    }
  }

  // Block reductions: chunk max, flags, then the partial sums rescaled to it.
  {
    const float wm = wave_maxf(m);
    const uint32_t wf = wave_or(flags);
    if (lane == 0) { L.f4[wave] = wm; L.u4[wave] = wf; }
  }
  __syncthreads();
  float m_c = L.f4[0];
  uint32_t f_c = L.u4[0];
#pragma unroll
  for (int w = 1; w < NWAVE; w++) { m_c = fmaxf(m_c, L.f4[w]); f_c |= L.u4[w]; }
  const float off_c = (m_c == -INFINITY) ? 0.0f : m_c;
  const float off_cs = cfg.scale ? off_c * cfg.inv : off_c;
  __syncthreads();
  if (stoch) {
    double t = 0.0;
    if (ssum != 0.0f) t = (double)ssum * exp((double)off_s - (double)off_cs);
    t = wave_sumd(t);
    if (lane == 0) L.d4[wave] = t;
  }
  __syncthreads();
  double ssum_c = 0.0;
  if (stoch) {
#pragma unroll
    for (int w = 0; w < NWAVE; w++) ssum_c += L.d4[w];
  }
  __syncthreads();
  double rsum_c = 0.0;
  if (WANT_LSE) {
    const float moff = __builtin_isinf(m_raw) ? 0.0f : m_raw;
    double t = 0.0;
    if (rsum != 0.0) t = rsum * exp((double)moff - (double)off_c);
    t = wave_sumd(t);
    if (lane == 0) L.d4[wave] = t;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NWAVE; w++) rsum_c += L.d4[w];
    __syncthreads();
  }

  // Candidate bound: the K'-th largest of the block's 256 lane maxima (distinct
  // elements, so at least K' elements of the chunk lie at or above it).  Each
  // wave sorts its 64 lane maxima; wave 0 merges the four sorted lists with two
  // bitonic top-64 merges (max(A[i], B[63-i]) is bitonic and holds the top 64
  // of A u B), or sorts all 256 when K' > 64.  The chunk publishes its 32
  // largest lane maxima for the row-level bound.
  uint32_t* lu = reinterpret_cast<uint32_t*>(L.list);
  {
    uint32_t srt[1] = {fkey(m)};
    wave_sort_desc<1>(srt);
    lu[wave * 64 + lane] = srt[0];
  }
  __syncthreads();
  if (wave == 0) {
    uint32_t top;  // element `lane` of the block's sorted lane maxima
    uint32_t tk = 0;
    if (kp <= 64) {
      uint32_t c1 = max(lu[lane], lu[64 + 63 - lane]);
      uint32_t c2 = max(lu[128 + lane], lu[192 + 63 - lane]);
#pragma unroll
      for (int d = 32; d > 0; d >>= 1) {
        const uint32_t b1 = (uint32_t)__shfl_xor((int)c1, d);
        const uint32_t b2 = (uint32_t)__shfl_xor((int)c2, d);
        const bool lower = (lane & d) == 0;
        c1 = lower ? max(c1, b1) : min(c1, b1);
        c2 = lower ? max(c2, b2) : min(c2, b2);
      }
      uint32_t c = max(c1, (uint32_t)__shfl((int)c2, 63 - lane));
#pragma unroll
      for (int d = 32; d > 0; d >>= 1) {
        const uint32_t b = (uint32_t)__shfl_xor((int)c, d);
        c = ((lane & d) == 0) ? max(c, b) : min(c, b);
      }
      top = c;
      tk = (uint32_t)__shfl((int)c, kp - 1);
    } else {
      uint32_t all[4];
#pragma unroll
      for (int r = 0; r < 4; r++) all[r] = lu[r * 64 + lane];
      wave_sort_desc<4>(all);
      top = all[0];
      const int i = kp - 1;  // < 256
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t t = (uint32_t)__shfl((int)all[r], i & 63);
        if ((i >> 6) == r) tk = t;
      }
    }
    if (lane < QPUB) a.pub[((int64_t)row * a.n_chunks + chunk) * QPUB + lane] = top;
    if (lane == 0) L.misc[0] = (int32_t)tk;
  }
  if (tid == 0) L.count = 0;
  __syncthreads();
  const uint32_t tau_key = (uint32_t)L.misc[0];
  const float tau = keyf(tau_key);

  // Filter: every element at or above the bound (ids < enc).  One compare per
  // element; the append branch is taken by ~K' lanes of the whole block.
  const int base_id = s0 * SLOT + 4 * tid;
#pragma unroll
  for (int j = 0; j < SPC; j++) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float x = v[4 * j + e];
      if (x >= tau && j < ns) {
        const int id = base_id + j * SLOT + e;
        if (id < enc) {
          const int pos = atomicAdd(&L.count, 1);
          if (pos < CAP) L.list[pos] = pack(fkey(x), (uint32_t)id);
        }
      }
    }
  }
  __syncthreads();
  int count = L.count;
  __syncthreads();
  if (count > CAP) count = chunk_overflow<HAS_MASK>(rowp, mrow, s0, ns, (int)enc, tau_key, kp, L);
  // Publish the chunk: candidates, then the summary.
  {
    uint64_t* gl = a.cand + ((int64_t)row * a.n_chunks + chunk) * CAP;
    for (int i = tid; i < count; i += BLOCK) gl[i] = L.list[i];
    if (tid == 0) {
      Summary s;
      s.vmax = m_c;
      s.ssum = (float)ssum_c;
      s.rsum = rsum_c;
      s.flags = f_c;
      s.count = count;
      s.pad0 = s.pad1 = 0;
      a.summ[(int64_t)row * a.n_chunks + chunk] = s;
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int t = atomicAdd(&a.row_ticket[row], 1);
    L.flag = (t == a.n_chunks - 1);
    if (L.flag) a.row_ticket[row] = 0;
  }
  __syncthreads();
  if (!L.flag) return;
  __threadfence();

  // ---------------- row finalize (last workgroup of the row) ----------------
  const int nc = a.n_chunks;
  const Summary* sm = a.summ + (int64_t)row * nc;
  float vmax = -INFINITY;
  uint32_t fl = 0;
  int cnt = 0;
  for (int c = tid; c < nc; c += BLOCK) {
    const Summary s = sm[c];
    vmax = fmaxf(vmax, s.vmax);
    fl |= s.flags;
  }
  {
    const float wm = wave_maxf(vmax);
    const uint32_t wf = wave_or(fl);
    if (lane == 0) { L.f4[wave] = wm; L.u4[wave] = wf; }
  }
  __syncthreads();
  float m_v = L.f4[0];
  fl = L.u4[0];
#pragma unroll
  for (int w = 1; w < NWAVE; w++) { m_v = fmaxf(m_v, L.f4[w]); fl |= L.u4[w]; }
  __syncthreads();
  const float moff = (m_v == -INFINITY) ? 0.0f : m_v;
  const float moff_s = cfg.scale ? moff * cfg.inv : moff;
  // Denominator: chunk partials rescaled to the row max, summed in f64.
  double S_d = 0.0, R_d = 0.0;
  for (int c = tid; c < nc; c += BLOCK) {
    const Summary s = sm[c];
    const float co = (s.vmax == -INFINITY) ? 0.0f : s.vmax;
    const float co_s = cfg.scale ? co * cfg.inv : co;
    if (s.ssum != 0.0f) S_d += (double)s.ssum * exp((double)co_s - (double)moff_s);
    if (WANT_LSE && s.rsum != 0.0) R_d += s.rsum * exp((double)co - (double)moff);
  }
  S_d = wave_sumd(S_d);
  if (lane == 0) L.d4[wave] = S_d;
  __syncthreads();
  S_d = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; w++) S_d += L.d4[w];
  __syncthreads();
  if (WANT_LSE) {
    R_d = wave_sumd(R_d);
    if (lane == 0) L.d4[wave] = R_d;
    __syncthreads();
    R_d = 0.0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) R_d += L.d4[w];
    __syncthreads();
  }
  const float S = (float)S_d;
  const float m_s = cfg.scale ? m_v * cfg.inv : m_v;
  const bool nan_seen = fl & 1u;
  const bool finite_seen = fl & 2u;

  int st = XS_ROW_OK;
  if (cfg.bad) st = XS_ROW_BAD_PARAM;
  else if (HAS_MASK && !finite_seen) st = XS_ROW_NO_FINITE;
  else if (cfg.greedy) st = nan_seen ? XS_ROW_NAN : (m_v == -INFINITY ? XS_ROW_NO_FINITE : XS_ROW_OK);
  else if (nan_seen || __builtin_isinf(m_s)) st = XS_ROW_NAN;

  // Survivor bound: the K'-th largest of the chunks' published lane maxima
  // (distinct elements), using the top q of every chunk's list, <= 256 values.
  int q = (kp + nc - 1) / nc + 1;
  q = min(q, QPUB);
  while (q > 1 && nc * q > 256) q--;
  const int nv = min(nc * q, 256);
  if (wave == 0) {
    uint32_t x[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = r * 64 + lane;
      x[r] = 0u;
      if (i < nv) {
        const int c = i / q, qi = i - c * q;
        x[r] = a.pub[((int64_t)row * nc + c) * QPUB + qi];
      }
    }
    wave_sort_desc<4>(x);
    uint32_t tk = 0;
    if (nv >= kp) {
      const int i = kp - 1;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t t = (uint32_t)__shfl((int)x[r], i & 63);
        if ((i >> 6) == r) tk = t;
      }
    }
    if (lane == 0) L.misc[2] = (int32_t)tk;
  }
  // chunk candidate offsets (nc <= BLOCK is enforced by the host)
  {
    const int c0 = tid < nc ? sm[tid].count : 0;
    int tot;
    const int pre = block_excl_scan(c0, L.s4, &tot);
    if (tid < nc) L.prefix[tid] = pre;
    if (tid == 0) { L.prefix[nc] = tot; L.count = 0; }
  }
  __syncthreads();
  uint64_t floor_e = (uint64_t)(uint32_t)L.misc[2] << 32;  // survivors: entries >= floor_e
  const int total = L.prefix[nc];
  for (int pass = 0; pass < 2; pass++) {
    for (int i = tid; i < total; i += BLOCK) {
      int lo = 0, hi = nc - 1;  // chunk c with prefix[c] <= i < prefix[c+1]
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (L.prefix[mid] <= i) lo = mid; else hi = mid - 1;
      }
      const uint64_t e = a.cand[((int64_t)row * nc + lo) * CAP + (i - L.prefix[lo])];
      if (e >= floor_e) {
        const int pos = atomicAdd(&L.count, 1);
        if (pos < SURV) L.list[pos] = e;
      }
    }
    __syncthreads();
    if (L.count <= SURV) break;  // block-uniform
    // Too many survivors (ties at the bound across many chunks): find the exact
    // K'-th largest entry by bisection over the unique u64 entries, then refilter.
    uint64_t ans = 0;
    for (int bit = 63; bit >= 0; bit--) {
      const uint64_t cnd = ans | (1ull << bit);
      int c = 0;
      for (int i = tid; i < total; i += BLOCK) {
        int lo = 0, hi = nc - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (L.prefix[mid] <= i) lo = mid; else hi = mid - 1;
        }
        c += a.cand[((int64_t)row * nc + lo) * CAP + (i - L.prefix[lo])] >= cnd ? 1 : 0;
      }
      int tot;
      block_excl_scan(c, L.s4, &tot);
      if (tot >= kp) ans = cnd;
    }
    floor_e = ans;
    if (tid == 0) L.count = 0;
    __syncthreads();
  }
  const int M = min(L.count, SURV);
  // Exact selection: rank every survivor against all others (keys are unique).
  for (int i = tid; i < M; i += BLOCK) {
    const uint64_t me = L.list[i];
    int rank = 0;
    for (int j2 = 0; j2 < M; j2++) rank += (L.list[j2] > me) ? 1 : 0;
    if (rank < kp) L.sel[rank] = me;
  }
  __syncthreads();
  const int nsel = min(M, kp);

  // Probabilities of the survivors and the (p desc, id asc) order.
  if (stoch && st == XS_ROW_OK) {
    if (tid < nsel) {
      const uint64_t e = L.sel[tid];
      const float p = exact_p(keyf(pk_key(e)), cfg, m_s, S);
      L.w[tid] = p;
    }
    __syncthreads();
    if (tid < nsel) {
      const uint64_t me = ((uint64_t)__float_as_uint(L.w[tid] + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - pk_id(L.sel[tid]));
      int rank = 0;
      for (int j2 = 0; j2 < nsel; j2++) {
        const uint64_t o = ((uint64_t)__float_as_uint(L.w[j2] + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - pk_id(L.sel[j2]));
        rank += (o > me) ? 1 : 0;
      }
      L.psel[rank] = me;
    }
    __syncthreads();
  }

  // Boundary proof (stochastic, top_k < enc): the k-th probability P_k must
  // not be shared by an entry outside the survivors.
  int k = cfg.k;
  const bool want_cands = a.cand_id != nullptr || a.cand_w != nullptr;
  if (stoch && st == XS_ROW_OK && !cfg.full) {
    if (tid == 0) {
      // L.w[i] holds p of L.sel[i] (logit order).
      const float Pk = __uint_as_float((uint32_t)(L.psel[k - 1] >> 32));
      const float vL = keyf(pk_key(L.sel[nsel - 1]));
      const float pL = L.w[nsel - 1];
      int slow = 0;
      if (nsel < kp) slow = 1;  // cannot happen (k < enc); scan to be safe
      else if (pL == Pk) {
        // Safe only if every survivor tied at P_k has logit vL and nothing
        // below vL reaches P_k: then the tie is an exact logit tie, whose lowest
        // ids the (logit desc, id asc) selection already kept.
        bool only_vl = true;
        for (int i = 0; i < nsel; i++)
          if (L.w[i] == Pk && keyf(pk_key(L.sel[i])) != vL) only_vl = false;
        bool below = false;
        if (vL != -INFINITY) below = exact_p(next_below(vL), cfg, m_s, S) == Pk;
        slow = (!only_vl || below) ? 1 : 0;
      }
      // Entries tied at P_k = 0 carry no weight: the draw does not depend on
      // which ids fill them, only the returned candidate list does.
      if (slow && Pk == 0.0f && !want_cands) slow = 0;
      L.misc[3] = slow;
      L.misc[4] = (int32_t)__float_as_uint(Pk);
    }
    __syncthreads();
    if (L.misc[3]) {
      // Slow path: the candidates are every survivor with p > P_k, then the
      // lowest ids of the whole row with p == P_k, found by an id-ordered scan.
      const float Pk = __uint_as_float((uint32_t)L.misc[4]);
      int g = 0;
      while (g < k && __uint_as_float((uint32_t)(L.psel[g] >> 32)) > Pk) g++;
      // Band of exp arguments d = s - max whose exp can round to P_k * S: the
      // rounding interval of P_k, widened generously; every element inside it
      // gets the exact test, every element outside it provably misses.
      const double lo_p = Pk == 0.0f ? 0.0 : 0.5 * ((double)Pk + (double)__uint_as_float(__float_as_uint(Pk) - 1u));
      const double hi_p = 0.5 * ((double)Pk + (double)__uint_as_float(__float_as_uint(Pk) + 1u));
      const double elo = lo_p * (double)S * (1.0 - 0x1p-10), ehi = hi_p * (double)S * (1.0 + 0x1p-10) + 0x1p-148;
      const float x_lo = elo > 0x1p-100 ? (float)(log(elo) - 0x1p-8) : -INFINITY;
      const float x_hi = (float)(log(ehi) + 0x1p-8);
      __syncthreads();
      int need = k - g, have = g;
      for (int64_t base = 0; base < enc && need > 0; base += SLOT) {
        const int64_t f = base / 4 + tid;
        float4 qv = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (4 * f < enc) qv = rp4[f];
        float xv[4] = {qv.x, qv.y, qv.z, qv.w};
        int hit[4];
        int c = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int64_t id = 4 * f + e;
          float x = xv[e];
          if (HAS_MASK && id < enc && !((mrow[id >> 5] >> (id & 31)) & 1u)) x = -INFINITY;
          hit[e] = 0;
          if (id < enc) {
            const float sx = cfg.scale ? x * cfg.inv : x;
            const float d = sx - m_s;
            if (d >= x_lo && d <= x_hi) hit[e] = exact_p(x, cfg, m_s, S) == Pk;
          }
          c += hit[e];
        }
        int tot;
        int pre = block_excl_scan(c, L.s4, &tot);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          if (hit[e]) {
            if (pre < need) L.psel[have + pre] = ((uint64_t)__float_as_uint(Pk + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(4 * f + e));
            pre++;
          }
        }
        have += min(tot, need);
        need -= tot;
        __syncthreads();
      }
    }
  }

  // The draw: truncate_top_p (sampler.rs:401-429) and WeightedIndex
  // (sampler.rs:235-243, rand 0.9), serial f32 in one lane.
  if (tid == 0) {
    int tok = -1;
    if (st == XS_ROW_OK) {
      if (!stoch) {
        tok = (int)pk_id(L.sel[0]);
      } else {
        for (int i = 0; i < k; i++) L.w[i] = __uint_as_float((uint32_t)(L.psel[i] >> 32));
        if (!(cfg.top_p >= 1.0f)) {
          float sum = -0.0f;
          for (int i = 0; i < k; i++) sum += L.w[i];
          if (sum > 0.0f) {
            for (int i = 0; i < k; i++) L.w[i] = L.w[i] / sum;
            float cs = 0.0f;
            int keep = k;
            for (int i = 0; i < k; i++) {
              cs += L.w[i];
              if (cs >= cfg.top_p) { keep = i + 1; break; }
            }
            for (int i = keep; i < k; i++) L.w[i] = 0.0f;
          }
        }
        float tw = L.w[0];
        bool okw = tw >= 0.0f;
        // cumulative weights: cum[i-1] = total before adding w[i]
        float x_draw = 0.0f;
        int idx = 0;
        {
          float tot = tw;
          for (int i = 1; i < k; i++) {
            if (!(L.w[i] >= 0.0f)) okw = false;
            tot += L.w[i];
          }
          if (!okw || tot == 0.0f) {
            st = XS_ROW_ZERO_WEIGHT;
          } else {
            x_draw = a.uniforms[row] * tot + 0.0f;
            float run = tw;
            for (int i = 1; i < k; i++) {
              if (run <= x_draw) idx = i; else break;
              run += L.w[i];
            }
            tok = (int)pk_id(L.psel[idx]);
          }
        }
      }
    }
    L.misc[5] = st;
    L.misc[6] = tok;
  }
  __syncthreads();
  st = L.misc[5];
  const int tok = L.misc[6];

  // Outputs.
  if (tid == 0) {
    a.token[row] = st == XS_ROW_OK ? tok : -1;
    a.status[row] = st;
    if (a.n_cand) a.n_cand[row] = (stoch && st == XS_ROW_OK) ? k : 0;
    if (a.soft_max) a.soft_max[row] = m_s;
    if (a.soft_sum) a.soft_sum[row] = S;
    if (WANT_LSE) {
      if (a.row_max) a.row_max[row] = m_v;
      if (a.row_lse) {
        const bool ok = !nan_seen && !__builtin_isinf(m_v);
        a.row_lse[row] = ok ? (double)m_v + log(R_d) : __builtin_nan("");
      }
    }
  }
  if (want_cands && stoch && st == XS_ROW_OK) {
    const int kw = (int)min((int64_t)k, a.cand_ld);  // a short cand_ld truncates the list
    for (int i = tid; i < kw; i += BLOCK) {
      if (a.cand_id) a.cand_id[(int64_t)row * a.cand_ld + i] = (int32_t)(0xFFFFFFFFu - (uint32_t)L.psel[i]);
      if (a.cand_w) a.cand_w[(int64_t)row * a.cand_ld + i] = L.w[i];
    }
  }
  if (WANT_LSE && a.n_top > 0) {
    const bool ok = !nan_seen && !__builtin_isinf(m_v);
    const double lse = ok ? (double)m_v + log(R_d) : __builtin_nan("");
    const int nt = (int)min((int64_t)a.n_top, enc);
    for (int i = tid; i < a.n_top; i += BLOCK) {
      const bool have = i < nt && i < nsel && !cfg.bad;
      if (a.top_id) a.top_id[(int64_t)row * a.top_ld + i] = have ? (int32_t)pk_id(L.sel[i]) : -1;
      if (a.top_logprob)
        a.top_logprob[(int64_t)row * a.top_ld + i] = have ? (float)((double)keyf(pk_key(L.sel[i])) - lse) : __builtin_nanf("");
    }
  }

  // Speculative verify: the last finalizer of a sequence walks its rows.
  if (a.span > 0) {
    __threadfence();
    __syncthreads();
    const int seq = row / a.span;
    if (tid == 0) {
      const int t = atomicAdd(&a.seq_ticket[seq], 1);
      L.flag = (t == a.span - 1);
      if (L.flag) a.seq_ticket[seq] = 0;
    }
    __syncthreads();
    if (L.flag && tid == 0) {
      __threadfence();
      const int span = a.span, D = span - 1;
      const int64_t r0 = (int64_t)seq * span;
      const int bud = a.budget ? a.budget[seq] : 0x7FFFFFFF;
      int mcount = 0, ncom = 0, sst = XS_ROW_OK;
      for (int i = 0; i < span; i++) {
        if (ncom >= bud) break;
        const int rs = __atomic_load_n(&a.status[r0 + i], __ATOMIC_RELAXED);
        if (rs != XS_ROW_OK) { sst = rs; break; }
        const int s = __atomic_load_n(&a.token[r0 + i], __ATOMIC_RELAXED);
        const bool matched = i < D && s == a.drafts[(int64_t)seq * D + i];
        a.committed[(int64_t)seq * span + ncom] = s;
        ncom++;
        if (matched) mcount++;
        bool eog = false;
        for (int e = 0; e < a.n_eog; e++) eog |= (s == a.eog[e]);
        if (!matched || eog) break;
      }
      for (int i = ncom; i < span; i++) a.committed[(int64_t)seq * span + i] = -1;
      a.accepted[seq] = mcount;
      a.n_committed[seq] = ncom;
      a.seq_status[seq] = sst;
    }
  }
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

__global__ void exp_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = cr_expf(x[i]);
}

}  // namespace xs

// ---------------------------------------------------------------------------
// Host side: the context and the C ABI.

struct xs_context {
  int device;
  hipStream_t stream;
  int64_t max_rows, vocab;
  int32_t k_max;
  int32_t max_chunks;
  xs::Summary* summ;
  uint32_t* pub;
  uint64_t* cand;
  int32_t* row_ticket;
  int32_t* seq_ticket;
};

namespace {

int64_t slots_for(int64_t enc) { return (enc + xs::SLOT - 1) / xs::SLOT; }
int32_t chunks_for(int64_t enc) {
  const int64_t ns = slots_for(enc);
  return (int32_t)((ns + xs::SPC - 1) / xs::SPC);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

struct Call {
  const float* logits;
  int64_t rows, ld, width, enc;
  const xs_row_params* params;
  const float* uniforms;
  const uint32_t* allowed;
  int64_t allowed_words, allowed_ld;
};

int check_common(xs_context* ctx, const Call& c) {
  if (!ctx || !c.logits || !c.params || !c.uniforms) return XS_ERR_ARG;
  if (c.rows < 0 || c.enc < 1 || c.ld < 1) return XS_ERR_ARG;
  if (c.rows > ctx->max_rows || c.enc > ctx->vocab) return XS_ERR_CAPACITY;
  if (c.ld % 4 != 0 || !aligned16(c.logits)) return XS_ERR_ARG;
  if (c.width > c.ld) return XS_ERR_ARG;
  if (c.enc > c.ld && c.width >= c.enc) return XS_ERR_ARG;
  if (c.allowed && (c.allowed_ld < c.allowed_words || c.allowed_words < 0)) return XS_ERR_ARG;
  if (chunks_for(c.enc) > ctx->max_chunks || chunks_for(c.enc) > xs::BLOCK) return XS_ERR_CAPACITY;
  return XS_OK;
}

int launch(xs_context* ctx, xs::Args& a, int64_t rows, bool mask, bool lse) {
  const int64_t grid = rows * (int64_t)a.n_chunks;
  if (grid == 0) return XS_OK;
  if (grid > 0x7FFFFFFF) return XS_ERR_CAPACITY;
  dim3 g((unsigned)grid), b(xs::BLOCK);
  if (mask && lse) return XS_ERR_ARG;
  if (mask) hipLaunchKernelGGL((xs::sample_kernel<true, false>), g, b, 0, ctx->stream, a);
  else if (lse) hipLaunchKernelGGL((xs::sample_kernel<false, true>), g, b, 0, ctx->stream, a);
  else hipLaunchKernelGGL((xs::sample_kernel<false, false>), g, b, 0, ctx->stream, a);
  return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
}

}  // namespace

extern "C" {

const char* xs_version(void) { return "xsamp 0.1 gfx950"; }

int xs_create(int device, int64_t max_rows, int64_t vocab, int32_t k_max, xs_context** out) {
  if (!out || max_rows < 1 || vocab < 1 || k_max < 0 || k_max > XS_K_MAX) return XS_ERR_ARG;
  *out = nullptr;
  if (hipSetDevice(device) != hipSuccess) return XS_ERR_HIP;
  const int32_t mc = chunks_for(vocab);
  if (mc > xs::BLOCK) return XS_ERR_CAPACITY;
  xs_context* c = (xs_context*)calloc(1, sizeof(xs_context));
  if (!c) return XS_ERR_HIP;
  c->device = device;
  c->stream = nullptr;
  c->max_rows = max_rows;
  c->vocab = vocab;
  c->k_max = k_max;
  c->max_chunks = mc;
  const int64_t units = max_rows * (int64_t)mc;
  bool ok = hipMalloc((void**)&c->summ, units * sizeof(xs::Summary)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->pub, units * xs::NWAVE * xs::QPUB * sizeof(uint32_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->cand, units * xs::CAP * sizeof(uint64_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->row_ticket, max_rows * sizeof(int32_t)) == hipSuccess;
  ok = ok && hipMalloc((void**)&c->seq_ticket, max_rows * sizeof(int32_t)) == hipSuccess;
  ok = ok && hipMemset(c->row_ticket, 0, max_rows * sizeof(int32_t)) == hipSuccess;
  ok = ok && hipMemset(c->seq_ticket, 0, max_rows * sizeof(int32_t)) == hipSuccess;
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
  (void)hipFree(c->summ);
  (void)hipFree(c->pub);
  (void)hipFree(c->cand);
  (void)hipFree(c->row_ticket);
  (void)hipFree(c->seq_ticket);
  free(c);
  return XS_OK;
}

int xs_set_stream(xs_context* c, void* s) {
  if (!c) return XS_ERR_ARG;
  c->stream = (hipStream_t)s;
  return XS_OK;
}

int xs_sample(xs_context* ctx, const xs_sample_args* in) {
  if (!ctx || !in || !in->token || !in->status) return XS_ERR_ARG;
  const Call c{in->logits, in->rows, in->ld, in->width, in->enc, in->params, in->uniforms,
               in->allowed, in->allowed_words, in->allowed_ld};
  int rc = check_common(ctx, c);
  if (rc) return rc;
  if ((in->cand_id || in->cand_w) && in->cand_ld < 1) return XS_ERR_ARG;
  if (in->n_top < 0 || in->n_top > XS_TOP_MAX) return XS_ERR_ARG;
  if ((in->top_id || in->top_logprob) && in->top_ld < in->n_top) return XS_ERR_ARG;
  const bool lse = in->row_max || in->row_lse || in->top_id || in->top_logprob;
  if (lse && in->allowed) return XS_ERR_ARG;
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
  a.row_lse = in->row_lse;
  a.n_top = (in->top_id || in->top_logprob) ? in->n_top : 0;
  a.top_id = in->top_id;
  a.top_logprob = in->top_logprob;
  a.top_ld = in->top_ld;
  a.span = 0;
  a.n_chunks = chunks_for(in->enc);
  a.nslots = (int32_t)slots_for(in->enc);
  a.summ = ctx->summ;
  a.pub = ctx->pub;
  a.cand = ctx->cand;
  a.row_ticket = ctx->row_ticket;
  a.seq_ticket = ctx->seq_ticket;
  return launch(ctx, a, in->rows, in->allowed != nullptr, lse);
}

int xs_verify(xs_context* ctx, const xs_verify_args* in) {
  if (!ctx || !in || !in->row_token || !in->row_status || !in->accepted || !in->committed ||
      !in->n_committed || !in->seq_status)
    return XS_ERR_ARG;
  if (in->seqs < 0 || in->span < 1 || in->n_eog < 0 || in->n_eog > 8) return XS_ERR_ARG;
  if (in->span > 1 && !in->drafts) return XS_ERR_ARG;
  const int64_t rows = in->seqs * in->span;
  const Call c{in->logits, rows, in->ld, in->width, in->enc, in->params, in->uniforms,
               in->allowed, in->allowed_words, in->allowed_ld};
  int rc = check_common(ctx, c);
  if (rc) return rc;
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
  for (int i = 0; i < 8; i++) a.eog[i] = i < in->n_eog ? in->eog[i] : -1;
  a.accepted = in->accepted;
  a.committed = in->committed;
  a.n_committed = in->n_committed;
  a.seq_status = in->seq_status;
  a.n_chunks = chunks_for(in->enc);
  a.nslots = (int32_t)slots_for(in->enc);
  a.summ = ctx->summ;
  a.pub = ctx->pub;
  a.cand = ctx->cand;
  a.row_ticket = ctx->row_ticket;
  a.seq_ticket = ctx->seq_ticket;
  return launch(ctx, a, rows, in->allowed != nullptr, false);
}

int64_t xs_keep_confident(const float* probs, int64_t n, float p_min) {
  int64_t kept = 0;
  while (kept < n && probs[kept] >= p_min) kept++;
  return kept;
}

int xs_test_exp(const float* x, float* y, int64_t n, void* s) {
  if (n < 0 || (n > 0 && (!x || !y))) return XS_ERR_ARG;
  if (n == 0) return XS_OK;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(xs::exp_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)s, x, y, n);
  return hipGetLastError() == hipSuccess ? XS_OK : XS_ERR_HIP;
}

}  // extern "C"
