// Shapes and matrix-core helpers shared by the SSD translation units
// (ssd.hip: generic passes, N = 16 tile passes, one-launch kernel, streaming
// step; ssd_n64.hip: the bf16 N = 64 one-pass kernel and its time segments).
#pragma once

#include "common.h"
#include "lookback.h"

namespace tssm {

struct SsdArgs {
  const void* x;
  const float* dt;
  const float* A_log;
  const void* B;
  const void* C;
  const float* D;
  const float* h0;
  void* y;
  float* h_last;
  int64_t L;
  int64_t sx_b, sx_l, sx_h, sdt_b, sdt_l, sdt_h, sB_b, sB_l, sB_h, sC_b, sC_l, sC_h;
  int64_t sy_b, sy_l, sy_h;
  float* chunkA;   // [rows][nchunks] decay product of each chunk
  float* chunkX;   // [rows][nchunks][P*N] local end state of each chunk (from zero)
  float* entry;    // [rows][nchunks][P*N] state entering each chunk
  uint32_t H, P, rows, nchunks, tc;
};

// ---------------------------------------------------------------- MFMA passes
// bf16 inputs on the matrix cores: shared types, sizes and conversions.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kMq = 256;           // steps per tile (the chunk the caller names)
constexpr int kMp = 64, kMn = 16;  // head dim, state size of the tile passes

__device__ inline bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// hi/lo bf16 parts of 8 floats (v = hi + lo to ~2^-16 relative).
__device__ inline void split_bf16(const float* v, bf16x8_t& hi, bf16x8_t& lo) {
  u32x4 h, l;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t hp = pk_bf16(v[2 * k], v[2 * k + 1]);
    const float r0 = v[2 * k] - __uint_as_float(hp << 16);
    const float r1 = v[2 * k + 1] - __uint_as_float(hp & 0xffff0000u);
    h[k] = hp;
    l[k] = pk_bf16(r0, r1);
  }
  hi = as_bf16x8(h);
  lo = as_bf16x8(l);
}

__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Low (sel 0x05040100) or high (0x07060302) 16-bit halves of two words,
// packed (first word's half in the low half): one v_perm_b32.
__device__ inline uint32_t perm_lo(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x05040100u);
}
__device__ inline uint32_t perm_hi(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x07060302u);
}

// Per-step decay exponent (log2 units) and input coefficient of step t0+tid;
// steps at or past L get dt = 0 (decay 1, coefficient 0).
template <int DISC>
__device__ inline void mfma_step_scalars(const SsdArgs& a, uint32_t h, int64_t t0, int tid,
                                         float dl, float* l2, float* coef) {
  const float d = t0 + tid < a.L ? dl : 0.0f;
  const float a2 = -expf(a.A_log[h]) * kLog2e;
  const float x = d * a2;
  *l2 = x;
  *coef = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(x * 0.6931471805599453f, exp2_fast(x)) * d : d;
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 N = 64 on the matrix cores (ssd_n64.hip)
constexpr int kSqQ = 128;  // steps per block
constexpr int kSqN = 64;   // state size
constexpr int kSqP = 16;   // channels per product tile (a workgroup takes 1 or 2)

// The bf16 N = 64 one-pass path (ssd_n64.hip) for `rows` rows of P channels:
// time segments when the rows leave workgroups idle, then the one-pass kernel.
int launch_ssd_seq_any(int disc, bool has_d, int64_t rows, int64_t P, hipStream_t s,
                       const SsdArgs& a);

}  // namespace tssm
