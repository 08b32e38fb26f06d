// Single-pass chunked scan support: decoupled look-back over per-channel
// carries between the chunks (tiles) of one sequence row.
//
// Every carry value is published as one 64-bit word {float bits, tag}, stored
// and loaded with relaxed device-scope atomics (global_store/load_dwordx2
// sc1).  Because the tag travels in the same word as the value, a reader that
// sees the current tag also sees the value: no release/acquire fences (and so
// no L2 write-back or invalidate) are needed between the per-XCD L2 caches.
//
// Tiles are numbered by blockIdx so that a tile only waits on tiles with a
// smaller index (earlier chunks of its row).  No device-scope atomics are used:
// one shared counter serialises at ~27 ns per operation, which at thousands
// of tiles costs more than the scan itself.  Progress relies on each XCD
// starting its workgroups in increasing index order; every wait is bounded
// regardless (a timeout sets the sticky error word and the kernel finishes).
//
// Workspace layout (caller-owned, zero-filled ONCE when allocated):
//   WsHeader (256 B: sticky error word, device epoch, host flag address)
//   | uint64 carry words ...
// The tag of a launch is an epoch that advances on every launch that uses
// the workspace, so stale words never match and no per-launch clearing is
// needed.  Workspace launches take it from a host counter (``next_epoch``)
// as a kernel argument; the no-allocation scratch advances it on the device
// (a one-thread kernel enqueued before the scan, which reads it from the
// header), so a launch captured in a HIP graph gets a fresh tag on every
// replay.  One workspace serves one stream at a time: launches that overlap
// on the same workspace race.
#pragma once

#include "common.h"

namespace tssm {

struct WsHeader {
  uint32_t error;      // sticky: set to 1 when a bounded look-back wait expired
  uint32_t epoch;      // device-advanced tag (no-allocation scratch only)
  uint64_t host_flag;  // 0, or the device address of a host-visible int that
                       // is set to 1 together with `error`
  uint32_t pad[60];
};
static_assert(sizeof(WsHeader) == 256, "header is 256 bytes");

constexpr uint32_t kDefaultSpinLimit = 1u << 20;  // ~1 s of polling

// Host: the tag of the next launch on ``workspace`` (never 0; a zero-filled
// word is "not ready").  Thread-safe; defined in abi.hip.
uint32_t next_epoch(const void* workspace);

// Host: the sticky error word of the current device's no-allocation scratch
// (0 when no no-allocation launch ran there yet); defined in multihead.hip.
int noalloc_scratch_error(int clear, int* error_out);

// Host: device address of the current device's no-allocation scratch (its
// WsHeader), resolved on first use; defined in multihead.hip.
int noalloc_scratch_header(void** ptr);

__device__ inline uint64_t ld_word(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_word(uint64_t* p, float v, uint32_t tag) {
  uint64_t w = ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t word_tag(uint64_t w) { return (uint32_t)(w >> 32); }
__device__ inline float word_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Expired wait: the sticky word, and the host's flag when one is attached
// (a system-scope store, visible to the host without a synchronisation once
// it lands; only this error path writes host memory).
__device__ inline void flag_error(WsHeader* hdr) {
  __hip_atomic_store(&hdr->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hf =
      __hip_atomic_load(&hdr->host_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (hf != 0)
    __hip_atomic_store(reinterpret_cast<uint32_t*>(hf), 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

// Tag of the current launch on a workspace whose epoch the device advances.
__device__ inline uint32_t load_epoch(const WsHeader* hdr) {
  return __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// predecessors, WIN of them per round trip: the words of chunks j, j-1, ...,
// j-WIN+1 are loaded together, then folded newest first -- an inclusive word
// ends the walk, an aggregate pair is folded in, a missing word stops the
// batch and is re-polled (bounded).  ``h0`` is the state before chunk 0.
// ``cha`` is the channel whose word holds the decay aggregate: ``ch`` itself,
// or the first channel of the head when the channels of a head share one
// decay (one word per head is then published and read).  A tile whose decay
// product is exactly zero may publish its inclusive word only.
template <int WIN>
__device__ inline float lookback_channel(const CarrySlot& s, int64_t c, int ch, int cha,
                                         uint32_t tag, float h0, uint32_t spin_limit,
                                         WsHeader* hdr) {
  float A_acc = 1.0f, X_acc = 0.0f;
  int64_t j = c - 1;
  uint32_t spins = 0;
  while (j >= 0) {
    uint64_t wi[WIN], wa[WIN], wx[WIN];
#pragma unroll
    for (int k = 0; k < WIN; ++k) {
      if (j - k >= 0) {
        wi[k] = ld_word(s.inc(j - k, ch));
        wa[k] = ld_word(s.agg_a(j - k, cha));
        wx[k] = ld_word(s.agg_x(j - k, ch));
      } else {
        wi[k] = wa[k] = wx[k] = 0;
      }
    }
    bool stalled = false;
#pragma unroll
    for (int k = 0; k < WIN; ++k) {
      if (stalled || j < 0) continue;
      if (word_tag(wi[k]) == tag) return __builtin_fmaf(A_acc, word_val(wi[k]), X_acc);
      if (word_tag(wa[k]) == tag && word_tag(wx[k]) == tag) {
        X_acc = __builtin_fmaf(A_acc, word_val(wx[k]), X_acc);
        A_acc = A_acc * word_val(wa[k]);
        --j;
      } else {
        stalled = true;
      }
    }
    if (stalled) {
      if (++spins > spin_limit) {   // predecessor never published: give up loudly
        flag_error(hdr);
        return X_acc;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return __builtin_fmaf(A_acc, h0, X_acc);
}

// Per-tile status of one row: a word pair per chunk {aggregate out, inclusive
// out} carrying only the tag, stored by the lane of channel 0 after its own
// carry words.  A status word says that the tile's carry words are (about to
// be) visible; every carry word is still checked by its own tag.  Polling the
// status instead of the carry words costs one 128-byte line per round trip
// per tile instead of 3 words x channels: under a full HBM stream, polling
// traffic competes with the data.
struct TileStatus {
  uint64_t* base;  // status of chunk 0 of this row
  __device__ inline uint64_t* agg(int64_t c) const { return base + 2 * c; }
  __device__ inline uint64_t* inc(int64_t c) const { return base + 2 * c + 1; }
};

// Bounded wait for one carry word whose status was already seen.
__device__ inline uint64_t settle_word(const uint64_t* p, uint64_t w, uint32_t tag,
                                       uint32_t& spins, uint32_t spin_limit, WsHeader* hdr) {
  while (word_tag(w) != tag && spins <= spin_limit) {
    if (++spins > spin_limit) {
      flag_error(hdr);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    w = ld_word(p);
  }
  return w;
}

// Look-back of whole waves (all 64 lanes active, lane = channel ch): the walk
// is decided per wave from the status of SW predecessors read at once (lane k
// reads chunk j-k), then exactly the carry words it needs are loaded, FB
// predecessors per round trip.  Resolves like lookback_channel: fold
// aggregates newest first until an inclusive state (or the row start, h0).
template <int SW, int FB>
__device__ inline float lookback_wave(const CarrySlot& s, const TileStatus& st, int64_t c, int ch,
                                      uint32_t tag, float h0, uint32_t spin_limit,
                                      WsHeader* hdr) {
  static_assert(SW >= 1 && SW <= 64 && FB >= 1, "status window within a wave");
  const int lane = threadIdx.x & 63;
  float A = 1.0f, X = 0.0f;
  int64_t j = c - 1;  // newest predecessor not folded yet
  uint32_t spins = 0;
  while (true) {
    // lanes k < SW: predecessor j-k; before chunk 0 stands the row's initial
    // state, an inclusive value
    bool inc_k = false, rdy_k = false;
    if (lane < SW) {
      if (j - lane < 0) {
        inc_k = rdy_k = true;
      } else {
        const uint64_t wi = ld_word(st.inc(j - lane));
        const uint64_t wa = ld_word(st.agg(j - lane));
        inc_k = word_tag(wi) == tag;
        rdy_k = inc_k || word_tag(wa) == tag;
      }
    }
    const uint64_t m_inc = __ballot(inc_k);
    const uint64_t m_rdy = __ballot(rdy_k);
    const int k_inc = m_inc ? __builtin_ctzll(m_inc) : 64;   // nearest inclusive
    const int k_gap = ~m_rdy ? __builtin_ctzll(~m_rdy) : 64;  // nearest with nothing out
    const bool resolve = k_inc < k_gap;
    const int n = resolve ? k_inc : k_gap;  // aggregates to fold this round
    // inclusive word in flight together with the aggregates
    const int64_t ji = j - k_inc;
    uint64_t wi = 0;
    if (resolve && ji >= 0) wi = ld_word(s.inc(ji, ch));
    for (int k0 = 0; k0 < n; k0 += FB) {
      uint64_t wa[FB], wx[FB];
#pragma unroll
      for (int k = 0; k < FB; ++k) {
        if (k0 + k < n) {
          wa[k] = ld_word(s.agg_a(j - k0 - k, ch));
          wx[k] = ld_word(s.agg_x(j - k0 - k, ch));
        }
      }
#pragma unroll
      for (int k = 0; k < FB; ++k) {
        if (k0 + k < n) {
          wa[k] = settle_word(s.agg_a(j - k0 - k, ch), wa[k], tag, spins, spin_limit, hdr);
          wx[k] = settle_word(s.agg_x(j - k0 - k, ch), wx[k], tag, spins, spin_limit, hdr);
          X = __builtin_fmaf(A, word_val(wx[k]), X);
          A = A * word_val(wa[k]);
        }
      }
    }
    if (resolve) {
      if (ji < 0) return __builtin_fmaf(A, h0, X);
      wi = settle_word(s.inc(ji, ch), wi, tag, spins, spin_limit, hdr);
      return __builtin_fmaf(A, word_val(wi), X);
    }
    j -= n;
    // every channel's decay product is exactly zero: earlier tiles cannot matter
    if (__ballot(A != 0.0f) == 0) return X;
    if (n == 0) {
      if (++spins > spin_limit) {  // predecessor never published: give up loudly
        flag_error(hdr);
        return X;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (spins > spin_limit) return X;
  }
}

}  // namespace tssm
