// Single-pass chunked scan support: dynamic tile tickets and a decoupled
// look-back over per-channel carries.
//
// Every carry value is published as one 64-bit word {float bits, tag}, stored
// and loaded with relaxed device-scope atomics (global_store/load_dwordx2
// sc1).  Because the tag travels in the same word as the value, a reader that
// sees the current tag also sees the value: no release/acquire fences (and so
// no L2 write-back or invalidate) are needed between the per-XCD L2 caches.
//
// Workspace layout (caller-owned, zero-filled once when allocated):
//   WsHeader (256 B) | uint64 words ...
// The header holds the ticket counter, the retire counter, the launch epoch
// and a sticky error word.  The last workgroup of a launch to retire resets
// both counters and advances the epoch, so no per-launch clearing is needed
// and stale words from earlier launches never match the current tag.
// One workspace serves one stream at a time: launches that overlap on the
// same workspace race.
#pragma once

#include "common.h"

namespace tssm {

struct WsHeader {
  uint32_t ticket;
  uint32_t done;
  uint32_t epoch;
  uint32_t error;   // sticky: set to 1 when a bounded look-back wait expired
  uint32_t pad[60];
};
static_assert(sizeof(WsHeader) == 256, "header is 256 bytes");

constexpr uint32_t kDefaultSpinLimit = 1u << 20;  // ~1 s of polling

__device__ inline uint32_t ld_relaxed_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ld_word(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_word(uint64_t* p, float v, uint32_t tag) {
  uint64_t w = ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t word_tag(uint64_t w) { return (uint32_t)(w >> 32); }
__device__ inline float word_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Thread 0 of a workgroup: take the next tile ticket and read the epoch.
__device__ inline void take_ticket(WsHeader* hdr, uint32_t* ticket, uint32_t* tag) {
  *ticket = __hip_atomic_fetch_add(&hdr->ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *tag = ld_relaxed_u32(&hdr->epoch) + 1u;   // never 0: a zeroed word is "not ready"
}

// Thread 0 of a workgroup, after its last use of the ticket/epoch.  The last
// of ``total`` workgroups resets the counters and advances the epoch.
__device__ inline void retire(WsHeader* hdr, uint32_t total) {
  uint32_t d = __hip_atomic_fetch_add(&hdr->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (d == total - 1) {
    uint32_t e = ld_relaxed_u32(&hdr->epoch);
    __hip_atomic_store(&hdr->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&hdr->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&hdr->epoch, e + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ inline void flag_error(WsHeader* hdr) {
  __hip_atomic_store(&hdr->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Carry words of one tile for one channel: aggregate (a, x) of the tile alone
// and the inclusive state after the tile.  ``stride`` is the distance between
// the three word arrays of a tile (= channels per tile).
struct CarrySlot {
  uint64_t* base;      // words of tile 0 of this row
  int64_t tile_words;  // 3 * channels
  int64_t stride;      // channels
  __device__ inline uint64_t* agg_a(int64_t c, int ch) const { return base + c * tile_words + ch; }
  __device__ inline uint64_t* agg_x(int64_t c, int ch) const { return base + c * tile_words + stride + ch; }
  __device__ inline uint64_t* inc(int64_t c, int ch) const { return base + c * tile_words + 2 * stride + ch; }
};

// Resolve the state entering chunk ``c`` for one channel by walking back over
// predecessors: an inclusive word ends the walk, an aggregate pair is folded
// in and the walk continues, a missing word is re-polled (bounded).
// ``h0`` is the state before chunk 0.
__device__ inline float lookback_channel(const CarrySlot& s, int64_t c, int ch, uint32_t tag,
                                         float h0, uint32_t spin_limit, WsHeader* hdr) {
  float A_acc = 1.0f, X_acc = 0.0f;
  int64_t j = c - 1;
  uint32_t spins = 0;
  while (j >= 0) {
    uint64_t wi = ld_word(s.inc(j, ch));
    uint64_t wa = ld_word(s.agg_a(j, ch));
    uint64_t wx = ld_word(s.agg_x(j, ch));
    if (word_tag(wi) == tag) {
      return __builtin_fmaf(A_acc, word_val(wi), X_acc);
    }
    if (word_tag(wa) == tag && word_tag(wx) == tag) {
      X_acc = __builtin_fmaf(A_acc, word_val(wx), X_acc);
      A_acc = A_acc * word_val(wa);
      --j;
      continue;
    }
    if (++spins > spin_limit) {   // predecessor never published: give up loudly
      flag_error(hdr);
      return X_acc;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return __builtin_fmaf(A_acc, h0, X_acc);
}

}  // namespace tssm
