// xs_host.h -- the host-only part of the C ABI (argument checks, and the
// host entry points select_option and keep_confident), in plain C++ so that
// it also builds with g++ alone, under AddressSanitizer and UBSan
// (oracle/Makefile, target asan).  Private to the library.
#pragma once
#include <stdint.h>

#include "../../include/xsamp.h"

namespace xs_host {
constexpr int64_t SLOT = 1024;  // logits per slot: one float4 per lane of a 256-lane workgroup
constexpr int64_t SPC = 16;     // slots per chunk
inline int64_t slots_for(int64_t enc) { return (enc + SLOT - 1) / SLOT; }
inline int32_t chunks_for(int64_t enc) { return (int32_t)((slots_for(enc) + SPC - 1) / SPC); }
}  // namespace xs_host

extern "C" {
// What a context holds, for the capacity checks.
typedef struct {
  int64_t max_rows, vocab;
  int32_t max_chunks;
} xs_host_limits;

// The checks xs_sample, xs_verify and xs_argmax_probs make before touching the
// device: XS_OK, XS_ERR_ARG or XS_ERR_CAPACITY, exactly as those calls return.
int xs_host_check_sample(const xs_host_limits* lim, const xs_sample_args* in);
int xs_host_check_verify(const xs_host_limits* lim, const xs_verify_args* in);
int xs_host_check_argmax(const xs_host_limits* lim, const xs_argmax_args* in);
// Whether a sample call needs the rows' held_row lse (any held_row or scoring
// output), and whether it asks for the scoring reads that score_kernel writes.
bool xs_host_wants_lse(const xs_sample_args* in);
bool xs_host_wants_scores(const xs_sample_args* in);
}
