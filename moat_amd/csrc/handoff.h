// Word encoding and per-batch decisions of the record-stream GEMM's in-kernel
// hand-off, shared by the device code and by host-side tests (plain C++, no
// HIP types, so that g++ compiles it too).
//
// A workgroup that shares a tile group with others stores its fp32 partial
// sums in workspace slots, one 16-byte chunk (four words) per store; the
// group's owner reads them back with device-coherent loads, polling while a
// chunk still reads "not written".
//  * A word travels as the bitwise complement of the value, NaN first made
//    the canonical 0x7FC00000, so no value encodes to 0: a zero word means
//    "not written yet", and every slot starts (and is left) at zero.
//  * After adding a batch the owner clears all of its chunks.  If its poll
//    budget runs out, it adds what it has (a missing word decodes to NaN)
//    and sets the workspace's sticky status word; a contributor whose store
//    lands after the owner's clear then leaves a non-zero chunk behind, which
//    a later call could take for its own partial.  So every later call on a
//    workspace whose status word is set writes NaN instead of results, until
//    the caller clears the workspace.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define MOAT_HD __host__ __device__ __forceinline__
#else
#define MOAT_HD inline
#endif

namespace moat {

// Status word at the start of the GEMM workspace (bit flags).
constexpr uint32_t kWsStatusHandoffTimeout = 1u;  // an owner stopped waiting for a partial
// Bytes at the start of the workspace reserved for the status word (the
// general kernel's per-tile counters follow them).
constexpr int kWsStatusBytes = 256;

MOAT_HD bool handoff_is_nan(uint32_t b) { return (b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0u; }

MOAT_HD uint32_t handoff_encode(uint32_t b) { return ~(handoff_is_nan(b) ? 0x7FC00000u : b); }

MOAT_HD uint32_t handoff_decode(uint32_t w) { return ~w; }

// A chunk is written when all four of its words are.
MOAT_HD bool handoff_chunk_written(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  return w0 != 0u && w1 != 0u && w2 != 0u && w3 != 0u;
}

// After loading a batch: stop polling (and consume) when every chunk the
// owner needs is written, or when no polls are left -- the latter is a
// give-up, reported through the status word.
MOAT_HD bool handoff_stop(bool all_written, int polls_left) { return all_written || polls_left <= 0; }
MOAT_HD bool handoff_gave_up(bool all_written, int polls_left) { return !all_written && polls_left <= 0; }

}  // namespace moat
