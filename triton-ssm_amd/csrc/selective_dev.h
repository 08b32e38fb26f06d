// Device helpers and shapes shared by the translation units of the three-pass
// Mamba-1 selective scan (selective.hip, selective_interp.hip).
#pragma once

#include <stdint.h>

#include "common.h"
#include "selective.h"

namespace tssm {

constexpr int kSelWaves = 4;                  // waves per workgroup
constexpr int kSelThreads = 64 * kSelWaves;   // consecutive channels per workgroup
constexpr int kSelCarryWaves = 4;             // pass 2: waves sharing a lane's chunks
constexpr int kSelCarryBatch = 16;            // chunks a pass-2 wave loads at once
constexpr int kSelPf = 4;                     // steps of x and dt fetched ahead

struct SelDims {
  int64_t L, Dc, Rs, nch;
  int64_t sx_b, sx_l, sdt_b, sdt_l, sdt_d, sB_b, sB_l, sC_b, sC_l, sy_b, sy_l;
  int64_t nbatch;
  // dt produced from raw rows (DTP instances): W [rank][Dc] row stride sw_r
  const float* W;
  const float* bias;
  int64_t sw_r;
  int rank;
  float dt_min, dt_max;
  float* dtw;  // NULL, or [nbatch][L][Dc]: pass 1 stores the produced dt there
};

// Row stride of the produced-dt table s_dt[step][channel] in LDS: 260 = 4
// mod 32 floats, so the 16-byte writes of the transpose (8 lanes per pass,
// 8 consecutive steps) land on distinct banks; reads are one row of
// consecutive channels.
constexpr int kSelDtStride = kSelThreads + 4;

// dt of the chunk's steps for the wave's 64 channels (first channel dw0),
// into s_dt[r * kSelDtStride + column] (column = channel - the workgroup's
// first channel).  The product raw[t0 + r, :] W[:, d] + bias[d] runs on the
// matrix cores in the operand order of the standalone projection kernel
// (dt_project_mfma_kernel: A = W columns, B = raw rows, 16x16x4 f32, the
// rank in blocks of 16 with lane group lj holding ranks q0 + 4 lj + s), so
// the values are those that kernel stores; then softplus and the clamp.
// Lane (li, lj) holds D[h][t] for channels 16 ct + 4 lj + i and steps
// 16 rt + li, written as one 16-byte row piece per (rt, ct).  Steps past the
// chunk's n repeat step n-1 (the readers give padded steps dt = 0); columns
// of channels past Dc hold values of no channel (clamped weights and bias)
// and are never read: a lane past Dc computes channel Dc-1 and reads that
// channel's column.  Every load is in bounds: Dc, rank and the row strides
// are multiples of 4 (sel_proj_ok).
__device__ inline void sel_proj_table(const float* __restrict__ raw_b, int64_t sr_l,
                                      int64_t t0, int n, const SelDims& m, int64_t dw0,
                                      int col0, float* s_dt) {
  const int lane = threadIdx.x & 63, li = lane & 15, lj = lane >> 4;
  f32x4 acc[2][4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int64_t h = dw0 + 16 * ct + 4 * lj;  // 4 channels, all in range or all out
    const float4 bq = *reinterpret_cast<const float4*>(m.bias + (h < m.Dc ? h : 0));
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) acc[rt][ct] = f32x4{bq.x, bq.y, bq.z, bq.w};
  }
  for (int q0 = 0; q0 < m.rank; q0 += 16) {
    const bool qok = q0 + 4 * lj < m.rank;  // rank % 4 == 0: a group is all in or all out
    const int64_t qa = qok ? q0 + 4 * lj : 0;
    float wa[4][4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int64_t h = dw0 + 16 * ct + li;
      const float* wp = m.W + (h < m.Dc ? h : m.Dc - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float v = wp[(qa + s) * m.sw_r];
        wa[ct][s] = qok ? v : 0.0f;
      }
    }
    f32x4 rv[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int r = 16 * rt + li;
      const f32x4 v =
          *reinterpret_cast<const f32x4*>(raw_b + (t0 + (r < n ? r : n - 1)) * sr_l + qa);
      rv[rt] = qok ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[ct][s], rv[rt][s], acc[rt][ct],
                                                              0, 0, 0);
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      float4 v;
      v.x = clamp_med3(softplus_fast(acc[rt][ct][0]), m.dt_min, m.dt_max);
      v.y = clamp_med3(softplus_fast(acc[rt][ct][1]), m.dt_min, m.dt_max);
      v.z = clamp_med3(softplus_fast(acc[rt][ct][2]), m.dt_min, m.dt_max);
      v.w = clamp_med3(softplus_fast(acc[rt][ct][3]), m.dt_min, m.dt_max);
      *reinterpret_cast<float4*>(s_dt + (16 * rt + li) * kSelDtStride + col0 + 16 * ct +
                                 4 * lj) = v;
    }
  }
}

// ab = exp2(dt a log2e) for each state; ZOH input term (ab - 1) B x / a
// (h' = ab h + (ab - 1) B x / a); Euler B dt x.
template <int DISC, int NST>
__device__ inline void sel_update(float (&h)[NST], const float (&a2)[NST], const float (&nia)[NST],
                                  const float (&Bv)[NST], float u, float dtv) {
  if constexpr (DISC == TSSM_DISC_ZOH) {
#pragma unroll
    for (int k = 0; k < NST; ++k) {
      // h' = ab (h + B x / a) - B x / a = h + (ab - 1)(h + B x / a): the
      // accumulating form adds onto h itself (no register copy per state),
      // and ab - 1 is exact for ab in [0.5, 1] (Sterbenz)
      const float abm1 = __builtin_amdgcn_exp2f(dtv * a2[k]) - 1.0f;
      const float hb = __builtin_fmaf(-nia[k], Bv[k] * u, h[k]);
      h[k] = __builtin_fmaf(abm1, hb, h[k]);
    }
  } else {
    const float du = dtv * u;
#pragma unroll
    for (int k = 0; k < NST; ++k) {
      const float ab = __builtin_amdgcn_exp2f(dtv * a2[k]);
      h[k] = __builtin_fmaf(ab, h[k], Bv[k] * du);
    }
  }
}

// Lane parameters: a log2(e) and -1/a with a = -exp(A_log[d, k]).
// Lane parameters from the raw A_log values: a log2(e) and -1/a with
// a = -exp(A_log[d, k]).
template <int NST>
__device__ inline void sel_params(const float (&al)[NST], float (&a2)[NST], float (&nia)[NST]) {
#pragma unroll
  for (int k = 0; k < NST; ++k) {
    const float x = al[k] * kLog2e;
    a2[k] = -__builtin_amdgcn_exp2f(x) * kLog2e;
    nia[k] = __builtin_amdgcn_exp2f(-x);
  }
}

template <int NST>
__device__ inline void load_alog(const float* __restrict__ A_log, int64_t d, float (&al)[NST]) {
  const float4* ap = reinterpret_cast<const float4*>(A_log + d * NST);
#pragma unroll
  for (int q = 0; q < NST / 4; ++q) {
    const float4 v = ap[q];
    al[4 * q] = v.x; al[4 * q + 1] = v.y; al[4 * q + 2] = v.z; al[4 * q + 3] = v.w;
  }
}

// The chunk's rows [n4][NST] of B (or C) of this batch, staged once per
// workgroup in LDS as fp32: thread i holds elements 4i .. 4i+3 (one pass:
// kSelChunkSteps * NST <= 4 kSelThreads); rows n .. n4-1 (the padding to
// whole groups of kSelPf steps) repeat row n-1.  Every wave then reads a
// step's row with broadcast LDS reads.  Loaded in the prologue with every
// other prologue load, stored to LDS after their one wait.
template <typename T, int NST>
__device__ inline float4 stage_row_load(const T* __restrict__ base, int64_t sl, int n, int n4) {
  static_assert(kSelChunkSteps * NST <= 4 * kSelThreads, "one staging pass");
  const int i0 = (int)threadIdx.x * 4;
  const int i = i0 < n4 * NST ? i0 : 0;  // threads past the rows load row 0 and store nothing
  const int row = i / NST, col = i - row * NST;
  const T* p = base + (int64_t)(row < n ? row : n - 1) * sl + col;
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
  }
}
template <int NST>
__device__ inline void stage_row_store(float* s, float4 v, int n4) {
  const int i = (int)threadIdx.x * 4;
  if (i < n4 * NST) *reinterpret_cast<float4*>(s + i) = v;
}

// dt shared by the channels: the chunk's values [n4] (n4 <= kSelThreads), one
// per thread (with timestamps the differences, dt_0 = tau_0); padded steps 0.
template <bool TAU>
__device__ inline float stage_dt_load(const float* __restrict__ row, int64_t sl, int64_t t0,
                                      int n) {
  const int i = (int)threadIdx.x;
  const int64_t tt = t0 + (i < n ? i : n - 1);
  float v = row[tt * sl];
  if constexpr (TAU) v -= (tt > 0) ? row[(tt - 1) * sl] : 0.0f;
  return i < n ? v : 0.0f;
}

template <int NST>
__device__ inline void lds_row(const float* s, float (&v)[NST]) {
  const float4* q = reinterpret_cast<const float4*>(s);
#pragma unroll
  for (int i = 0; i < NST / 4; ++i) {
    const float4 w = q[i];
    v[4 * i] = w.x; v[4 * i + 1] = w.y; v[4 * i + 2] = w.z; v[4 * i + 3] = w.w;
  }
}

// x (and a per-channel dt) of the chunk's first kSelPf steps, issued in the
// prologue with its other loads.
template <typename T, bool DTS>
__device__ inline void chunk_prefetch(const T* __restrict__ xp, int64_t sx_l,
                                      const float* __restrict__ dtp, int64_t sdt_l, int64_t t0,
                                      int n, float (&u)[kSelPf], float (&dr)[kSelPf]) {
#pragma unroll
  for (int j = 0; j < kSelPf; ++j) {
    const int64_t tt = t0 + (j < n ? j : n - 1);
    u[j] = ldf(xp + tt * sx_l);
    dr[j] = DTS ? 0.0f : dtp[tt * sdt_l];
  }
}

// One chunk of the recurrence for a lane (channel dc of batch b), in groups
// of kSelPf steps: x (and a per-channel dt) of step r + kSelPf is fetched
// right after step r, into the register step r just freed, so no value is
// copied and each fetch has kSelPf - 1 steps to arrive.  u/dr hold the
// prologue's fetches (chunk_prefetch), already waited on: they pass through
// opaque copies once, with every other prologue load, so the compiler neither
// merges them with the loop's fetches nor waits on them one by one.  Padded
// steps (r >= n) have dt = 0 -- an identity step -- and repeat step n-1's x
// and B/C rows, so they reproduce step n-1's output.  `step(r, u, dtv)` gets
// every step.
// DTP: dt produced in the pass, read from the lane's column of the LDS table
// (s_dt then points at that column, row stride kSelDtStride).
template <typename T, bool DTS, bool DTP = false, typename F>
__device__ inline void chunk_steps(const T* __restrict__ xp, int64_t sx_l,
                                   const float* __restrict__ dtp, int64_t sdt_l,
                                   const float* s_dt, int64_t t0, int n, int n4,
                                   float (&u)[kSelPf], float (&dr)[kSelPf], F&& step) {
  for (int r = 0; r < n4; r += kSelPf) {
#pragma unroll
    for (int j = 0; j < kSelPf; ++j) {
      const int rr = r + j;
      float dtv;
      if constexpr (DTS) dtv = s_dt[rr];
      else if constexpr (DTP) dtv = rr < n ? s_dt[rr * kSelDtStride] : 0.0f;
      else dtv = rr < n ? dr[j] : 0.0f;
      step(rr, u[j], dtv);
      // refill the registers step rr just used (no copies across the loop)
      __builtin_amdgcn_sched_barrier(0);
      const int64_t tn = t0 + min(rr + kSelPf, n - 1);
      u[j] = ldf(xp + tn * sx_l);
      if constexpr (!DTS && !DTP) dr[j] = dtp[tn * sdt_l];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// ---------------------------------------------------------------- interpolation in pass 1
// Time-aware interpolation (fused_interp_kernel.py:29-100, reference
// semantics as in interp.hip: "observed" is the FTILE-wide tile's mask sum
// > 0.5, prev/next the nearest observed step within K on each side,
// w = clip((tau_t - tau_prev)/(tau_next - tau_prev), 0, 1) or 0.5 when the
// denominator <= 1e-9, vhat = interpolation / v_prev / v_next / v_cur)
// formed inside pass 1 of the three-pass scan, which consumes it as x
// (fused_ssm_interp.py:12-101 does the interpolation and the SSM update in
// one kernel too, one step per launch).  Vhat is written once and never read
// back; pass 3 reads y, C and tau only.
//
// A workgroup (256 channels of one batch, one chunk of n <= 32 steps):
//  1. the tile flags of rows t0-K .. t0+n+K-1: wave w sums rows w, w+4, ...,
//     lane l the 16-byte mask vector of channels 4l..4l+3, then an xor
//     butterfly over the tile's FTILE/4 lanes -- the per-lane sums and the
//     reduction order of interp_fused_kernel, so the same flags -- and the
//     rows' timestamps, staged in LDS with the chunk's B/C rows and dt;
//  2. per (step, tile): the neighbours and the weight, into LDS tables
//     (padded steps repeat step n-1);
//  3. the recurrence of pass 1, x_t of each lane interpolated in registers
//     from V[prev] and V[next] (fetched four steps ahead), rounded to the
//     I/O dtype as Vhat is, and stored to Vhat.
constexpr int kSiMaxK = 64;       // search window the LDS tables hold
constexpr int kSiMaxTiles = 16;   // FTILE >= 16: at most 16 tiles per 256 channels
constexpr int kSiRows = kSelChunkSteps + 2 * kSiMaxK;

struct SiDims {
  int64_t svb, svt, smb, smt, sob, sot;  // V, M, Vhat strides (unit over features)
  int K, lf, lvpt;                       // lf = log2 FTILE, lvpt = log2(FTILE / 4)
};

template <typename T>
__device__ inline float round_io(float v) {
  if constexpr (sizeof(T) == 4) return v;
  else return bf16_bits_to_f32((uint16_t)f32_to_bf16_bits(v));
}

constexpr int kSiMaskU = 13;  // mask rows per wave in flight (one batch at K = 10)

// Pass 1 with the interpolation formed inside it (selective_interp.hip): the
// sel_interp_state_kernel instance for bf16 or f32 I/O, the discretization,
// N = 8 or 16 and the skip term.
int sel_interp_pass1(bool bf16, int disc, int nst, bool has_d, const void* V, const float* M,
                     const float* tau, void* Vhat, const SelPtrs& p, const SelDims& m,
                     const SiDims& q, hipStream_t s);

}  // namespace tssm
