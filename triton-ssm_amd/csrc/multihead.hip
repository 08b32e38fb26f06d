// Multihead DIAG selective scan (multihead_ssm_kernel.py).
//
// mh_scan_fused_kernel -- single pass over HBM:
//   tile = (batch b, row h, chunk c) of TC time steps x P channels, numbered
//   row-major (blockIdx = (b*rows_per_batch + h) * nchunks + c): the chunks of
//   one row are neighbours in launch order, which measured ~20% faster on
//   MI355X HBM than chunk-major numbering.  A row is one head, or 2 (4) heads
//   of 64 (32) channels when the head count allows: then a load instruction
//   reads 256 contiguous bytes per bf16 step instead of 128, which copies at
//   75% of HBM peak in this tile shape against 71-72% for one head.
//   Thread layout: a wave covers ROWS = 64/G "runs" of R consecutive steps;
//   each thread owns 8 consecutive channels (one 16-byte bf16 vector) of one
//   run, so every load instruction reads ROWS whole 128-byte channel rows.
//   1. load u, B, C (bf16/fp16/fp32) and dt for the thread's R steps;
//   2. sweep 1: discretize in registers (Abar = exp(dt a), Euler or ZOH input
//      term), run-local scan from (1, 0), keep w_t = C_t * a_loc_t and
//      y1_t = sum C_t x_loc_t + D u_t;
//   3. run aggregates -> LDS; a parallel scan over runs (each thread owns one
//      channel of 8 runs) gives every run's exclusive prefix within the tile;
//      the threads of the last segment publish the tile aggregate, look back
//      for the carry-in and publish the inclusive state (at once, before the
//      look-back, when the tile's decay product is exactly zero: such a tile
//      forgets its entry state, so its successors never wait on it);
//   4. sweep 2: y_t = y1_t + sum_j w_t[j] S[j] (with one decay per head,
//      w_t[j] = C_t[j] a_loc_t is rebuilt from C), reduced over the G threads of
//      the run with DPP and stored broadcast over the head's channels.
//   HBM traffic = inputs once + y once + ~1.5 KB of carry words per tile.
//
// mh_fwd_local_kernel / mh_output_kernel -- the reference's phase-exact
// kernels with its intermediate layouts (loc_a, loc_x, carry).
#include <mutex>

#include "common.h"
#include "lookback.h"
#include "selective.h"

namespace tssm {


// k * s for a small non-negative per-lane k and a (uniform) 64-bit stride:
// one 32 x 64-bit product (two's complement, so negative strides work too).
__device__ inline int64_t lane_mul(uint32_t k, int64_t s) {
  return (int64_t)((uint64_t)k * (uint64_t)s);
}

struct MhArgs {
  const void* u;
  const float* A_log;
  const void* B;
  const void* C;
  const float* dt;
  const float* D;
  const float* h0;
  void* y;
  float* h_last;
  int64_t L;
  int64_t su_b, su_l, sB_b, sB_l, sB_h, sC_b, sC_l, sC_h, sdt_b, sdt_l, sdt_h, sy_b, sy_l;
  WsHeader* hdr;
  uint64_t* words;
  uint32_t n_heads, nchunks, nrows;
  uint32_t tag;
  // nonzero: the launch's tag is the header's device-advanced epoch
  // (no-allocation scratch), not `tag`
  uint32_t tag_in_ws = 0;
  uint32_t spin_limit;
  uint32_t dt_is_tau;    // dt holds timestamps: dt_t = tau_t - tau_{t-1}, dt_0 = tau_0
  // Every operand's per-lane offset within a tile (steps x row stride +
  // column, in bytes) fits in 31 bits: full tiles take the scalar-base loads.
  uint32_t off32 = 0;
  // MODE_MAMBA1 only: dt projected in the load stage,
  // dt[b,t,d] = clamp(softplus(sum_k dt[b,t,k] W[k,d] + bias[d]), dt_min, dt_max)
  // with `dt` then holding the raw rows [B, L, dt_rank] (strides sdt_b, sdt_l, 1).
  const float* dtW = nullptr;     // [dt_rank, channels], row stride sw_r; NULL: dt given
  const float* dtbias = nullptr;  // [channels]
  int64_t sw_r = 0;
  uint32_t dt_rank = 0;
  float dt_min = 0.0f, dt_max = 0.0f;
};

// MODE_DIAG:   reference multihead layout -- u [B,L,nh*hd] per channel, y
//              broadcast over the head's channels, D per channel.  A row holds
//              G / NS consecutive heads of 8 NS channels (1 for head_dim >= 128;
//              several when they fit, so a load covers more contiguous bytes).
// MODE_MAMBA1: selective scan with lanes (channel d, state n): "head" = d,
//              channels = states; x [B,L,Dc] broadcast over the states, B/C
//              shared by all channels (head stride 0), y [B,L,Dc] one value per
//              channel, D per channel (y += D[d] x[d]).
constexpr int MODE_DIAG = 0;
constexpr int MODE_MAMBA1 = 1;

constexpr int kMhR = 4;    // consecutive steps per thread
constexpr int kMhWin = 1;  // predecessors read per look-back round trip (measured best)

// DTP (MODE_MAMBA1 only): dt produced in the load stage by the projection
// (MhArgs::dtW); a template flag so that the other instances carry none of
// its code and registers.
template <typename T, int DISC, bool APH, bool HAS_D, int G, int MODE, int NS, bool DTP = false,
          int R = kMhR, int WIN = kMhWin>
__global__ __launch_bounds__(512) void mh_scan_fused_kernel(MhArgs a) {
  // NS = threads summed into one output value: one head's head_dim/8 threads
  // for MODE_DIAG, one channel's N/8 threads for MODE_MAMBA1.
  constexpr int P = G * 8;
  constexpr int ROWS = 64 / G;
  extern __shared__ float s_mem[];
  const int W = blockDim.x >> 6;
  const int NRUN = W * ROWS;   // runs of R steps per tile
  const int NSEG = NRUN / 8;   // run-scan segments of 8 runs (NSEG * P == blockDim.x)
  const int TC = NRUN * R;     // steps per tile
  float* s_a = s_mem;                  // [NRUN][P] run aggregates -> exclusive prefixes
  float* s_x = s_a + NRUN * P;
  float* s_sa = s_x + NRUN * P;        // [NSEG][P] segment totals
  float* s_sx = s_sa + NSEG * P;
  float* s_carry = s_sx + NSEG * P;    // [P] state entering the tile
  float* s_par = s_carry + P;          // [2][P] per-lane a log2(e) and 1/a (decay per lane)
  // dt projection (MODE_MAMBA1): [TC][CPR] dt values, [TC][rank] raw rows,
  // [rank][CPR] weights of the row's channels
  float* s_dt = s_par + 2 * P;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane % G;
  const int run = wave * ROWS + lane / G;
  const int ch0 = g * 8;

  // ---- tile = blockIdx, row-major (row, chunk c): (row, c) waits only on
  // (row, c-1), a smaller index.  Numbering the chunks of all rows in groups
  // (chunk-major, or groups of 4-16 chunks) measured 7-25% slower: the
  // resident tiles then cover a scattered address range.
  const uint32_t tag = a.tag_in_ws ? load_epoch(a.hdr) : a.tag;
  const uint32_t row = blockIdx.x / a.nchunks;
  const uint32_t c = blockIdx.x - row * a.nchunks;
  const uint32_t b = row / a.n_heads;
  const uint32_t h = row - b * a.n_heads;
  // step t0 = tw + tr: tw uniform over the workgroup, tr a small per-lane
  // count, so address arithmetic splits into scalar 64-bit products and
  // per-lane 32 x 64-bit ones (lane_mul)
  const int64_t tw = (int64_t)c * TC;
  const uint32_t tr = (uint32_t)(run * R);
  const int64_t t0 = tw + tr;
  // A row packs CPR = G / NS groups of NS threads: heads of 8 NS channels
  // (MODE_DIAG) or channels of N = 8 NS states (MODE_MAMBA1).
  constexpr int CPR = G / NS;
  const uint32_t cl = CPR == 1 ? 0u : (uint32_t)(g / NS);  // head / channel within the row
  const int64_t chan = (int64_t)h * CPR + cl;

  // ---- per-channel parameters: raw values loaded first (small, cached), then
  // the step inputs; transformed after the scheduling barrier below
  float a2[8];  // a * log2(e) per channel (or per head)
  float ia[(APH || DISC != TSSM_DISC_ZOH) ? 1 : 8];  // 1 / a per channel (ZOH)
  // MODE_DIAG with a decay per channel: the row's P lanes share their
  // parameters over the workgroup's runs, so thread tid < P forms lane tid's
  // a log2(e) (and 1/a) once, into LDS, read back after the step loads are
  // issued (measured 4% faster at the headline shape).  For MODE_MAMBA1 the
  // extra barrier measured as costly as the exp2s it saves.
  constexpr bool PAR_LDS = !APH && MODE == MODE_DIAG;
  // MODE_MAMBA1 with at least 8 runs per wave: the wave's runs share the
  // parameters of each lane group g, so lane (run k, g) forms those of state
  // k % 8 only and the group's 8 values are gathered by ds_bpermute (no
  // barrier, 2 exp2 per thread instead of 16; measured ~1% faster at
  // B=16 L=2048 Dc=256 N=16).
  constexpr bool PAR_SHFL = !APH && MODE == MODE_MAMBA1 && ROWS >= 8;
  float alog = 0.0f;
  if constexpr (APH) {
    a2[0] = a.A_log[chan];
  } else if constexpr (PAR_LDS) {
    if (tid < P) alog = a.A_log[h * P + tid];
    __builtin_amdgcn_sched_barrier(0);  // issued before the step loads
  } else if constexpr (PAR_SHFL) {
    alog = a.A_log[h * P + ch0 + (lane / G) % 8];
  } else {
    const float4* ap = reinterpret_cast<const float4*>(a.A_log + h * P + ch0);
    const float4 l0 = ap[0], l1 = ap[1];
    a2[0] = l0.x; a2[1] = l0.y; a2[2] = l0.z; a2[3] = l0.w;
    a2[4] = l1.x; a2[5] = l1.y; a2[6] = l1.z; a2[7] = l1.w;
  }
  float Dv[8];
  if constexpr (HAS_D && MODE == MODE_MAMBA1) {
    Dv[0] = a.D[chan];
  } else if constexpr (HAS_D) {
    const float4* dp4 = reinterpret_cast<const float4*>(a.D + h * P + ch0);
    const float4 d0 = dp4[0], d1 = dp4[1];
    Dv[0] = d0.x; Dv[1] = d0.y; Dv[2] = d0.z; Dv[3] = d0.w;
    Dv[4] = d1.x; Dv[5] = d1.y; Dv[6] = d1.z; Dv[7] = d1.w;
  }

  // dt from the projection (computed below, once per (step, channel) of the tile)
  constexpr bool dtp = MODE == MODE_MAMBA1 && DTP;

  // ---- loads (all issued before any use)
  Vec8<T> vu[R], vB[R], vC[R];
  float us[R];  // MODE_MAMBA1: the channel's input, shared by its 8 state lanes
  float dtv[R];
  // A full tile (every tile of a row but the last) with 32-bit lane offsets:
  // each load is a uniform per-step base plus one per-lane byte offset
  // (global_load with a scalar base), so addresses take no per-step vector
  // arithmetic and no clamps.  Otherwise steps past the end read row L-1
  // instead (no branch around the loads, so no wait between them) and become
  // identity steps through dt = 0: Abar = 1 and a zero input term whatever u,
  // B and C hold.
  const bool fast = a.off32 && tw + TC <= a.L;
  // With one dt row per tile row (CPR == 1) and the wave's steps fitting in
  // its lanes, lane k loads the dt of the wave's k-th step and the threads
  // take theirs by lane shuffles: one load instruction per wave instead of
  // R (measured +2% of HBM peak on this tile's traffic).
  constexpr int WSTEPS = ROWS * R;  // steps covered by one wave
  constexpr bool DT_SHFL = CPR == 1 && WSTEPS <= 64;
  {
    const int bc = (g % NS) * 8;  // offset within the group's B/C row
    // uniform row bases (B/C head stride is 0 in MODE_MAMBA1: shared by all
    // channels) and the lane's column within the row
    const T* ur = reinterpret_cast<const T*>(a.u) + b * a.su_b +
                  (MODE == MODE_DIAG ? (int64_t)h * P : (int64_t)h * CPR);
    const T* Br = reinterpret_cast<const T*>(a.B) + b * a.sB_b + (int64_t)h * CPR * a.sB_h;
    const T* Cr = reinterpret_cast<const T*>(a.C) + b * a.sC_b + (int64_t)h * CPR * a.sC_h;
    const float* dr = a.dt + b * a.sdt_b + (int64_t)h * CPR * a.sdt_h;
    const int64_t ucol = MODE == MODE_DIAG ? ch0 : cl;
    const int64_t Bcol = lane_mul(cl, a.sB_h) + bc;
    const int64_t Ccol = lane_mul(cl, a.sC_h) + bc;
    const int64_t dcol = lane_mul(cl, a.sdt_h);
    float draw[DT_SHFL ? 1 : R];
    float dlane = 0.0f, tprev_lane = 0.0f, tprev = 0.0f;
    const int64_t tk = tw + (int64_t)wave * WSTEPS + lane;  // DT_SHFL: this lane's step
    if (fast) {
      // one descriptor per operand at the tile's first step, the lane's byte
      // offset in a VGPR, each step's in a scalar register
      const __amdgpu_buffer_rsrc_t ru = buf_rsrc(ur + tw * a.su_l);
      const __amdgpu_buffer_rsrc_t rB = buf_rsrc(Br + tw * a.sB_l);
      const __amdgpu_buffer_rsrc_t rC = buf_rsrc(Cr + tw * a.sC_l);
      const __amdgpu_buffer_rsrc_t rd = buf_rsrc(dr + tw * a.sdt_l);
      const uint32_t uo = (uint32_t)((lane_mul(tr, a.su_l) + ucol) * (int64_t)sizeof(T));
      const uint32_t Bo = (uint32_t)((lane_mul(tr, a.sB_l) + Bcol) * (int64_t)sizeof(T));
      const uint32_t Co = (uint32_t)((lane_mul(tr, a.sC_l) + Ccol) * (int64_t)sizeof(T));
      if constexpr (DT_SHFL) {
        if (lane < WSTEPS && !dtp) {
          const uint32_t ko = (uint32_t)(lane_mul((uint32_t)(wave * WSTEPS + lane), a.sdt_l) * 4);
          dlane = buf_ldf<float>(rd, ko, 0);
          // timestamp of step tk - 1 (0 before the first step)
          if (a.dt_is_tau && tk > 0) tprev_lane = buf_ldf<float>(rd, ko - (uint32_t)(a.sdt_l * 4), 0);
        }
      }
      const uint32_t dof = (uint32_t)((lane_mul(tr, a.sdt_l) + dcol) * 4);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int32_t su = (int32_t)(r * a.su_l * (int64_t)sizeof(T));
        const int32_t sb = (int32_t)(r * a.sB_l * (int64_t)sizeof(T));
        const int32_t sc = (int32_t)(r * a.sC_l * (int64_t)sizeof(T));
        if constexpr (MODE == MODE_DIAG) vu[r].load_nt(ru, uo, su);
        else us[r] = buf_ldf<T>(ru, uo, su);
        vB[r].load_nt(rB, Bo, sb);
        vC[r].load_nt(rC, Co, sc);
        if constexpr (!DT_SHFL)
          draw[r] = dtp ? 0.0f : buf_ldf<float>(rd, dof, (int32_t)(r * a.sdt_l * 4));
      }
      // timestamp of step t0 - 1 when dt holds timestamps (row 0 for t0 = 0)
      if (!DT_SHFL && a.dt_is_tau) tprev = *(dr + dcol + (t0 > 0 ? t0 - 1 : 0) * a.sdt_l);
    } else {
      const T* up = ur + ucol + tw * a.su_l + lane_mul(tr, a.su_l);
      const T* Bp = Br + Bcol + tw * a.sB_l + lane_mul(tr, a.sB_l);
      const T* Cp = Cr + Ccol + tw * a.sC_l + lane_mul(tr, a.sC_l);
      const float* db = dr + dcol;
      const float* dp = db + tw * a.sdt_l + lane_mul(tr, a.sdt_l);
      const int64_t tl = a.L - 1;
      const T* up_l = ur + ucol + tl * a.su_l;
      const T* Bp_l = Br + Bcol + tl * a.sB_l;
      const T* Cp_l = Cr + Ccol + tl * a.sC_l;
      const float* dp_l = db + tl * a.sdt_l;
      if constexpr (DT_SHFL) {
        if (lane < WSTEPS && !dtp) {
          dlane = *(tk < a.L ? db + tk * a.sdt_l : dp_l);
          if (a.dt_is_tau && tk > 0) tprev_lane = *(tk <= a.L ? db + (tk - 1) * a.sdt_l : dp_l);
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool in = t0 + r < a.L;
        if constexpr (MODE == MODE_DIAG) vu[r].load_nt(in ? up + r * a.su_l : up_l);
        else us[r] = ldf(in ? up + r * a.su_l : up_l);
        vB[r].load_nt(in ? Bp + r * a.sB_l : Bp_l);
        vC[r].load_nt(in ? Cp + r * a.sC_l : Cp_l);
        if constexpr (!DT_SHFL) draw[r] = dtp ? 0.0f : *(in ? dp + r * a.sdt_l : dp_l);
      }
      if (!DT_SHFL && a.dt_is_tau) tprev = *(t0 == 0 ? dp : (t0 <= a.L ? dp - a.sdt_l : dp_l));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
    if constexpr (PAR_LDS) {
      // lane parameters while the step loads are in flight: every wave
      // reaches this barrier right after issuing its loads.  Hardware exp2 of
      // the base-2 argument: within ~4e-7 relative of -exp(A_log), at 4
      // operations per lane instead of a library expf.
      if (tid < P) {
        const float x = alog * kLog2e;
        s_par[tid] = -exp2_fast(x) * kLog2e;
        if constexpr (DISC == TSSM_DISC_ZOH) s_par[P + tid] = -exp2_fast(-x);
      }
      // nothing that waits on the step loads may move above the barrier
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      const float4* pa = reinterpret_cast<const float4*>(s_par + ch0);
      const float4 a0 = pa[0], a1 = pa[1];
      a2[0] = a0.x; a2[1] = a0.y; a2[2] = a0.z; a2[3] = a0.w;
      a2[4] = a1.x; a2[5] = a1.y; a2[6] = a1.z; a2[7] = a1.w;
      if constexpr (DISC == TSSM_DISC_ZOH) {
        const float4* pi = reinterpret_cast<const float4*>(s_par + P + ch0);
        const float4 i0 = pi[0], i1 = pi[1];
        ia[0] = i0.x; ia[1] = i0.y; ia[2] = i0.z; ia[3] = i0.w;
        ia[4] = i1.x; ia[5] = i1.y; ia[6] = i1.z; ia[7] = i1.w;
      }
    }
    if constexpr (DT_SHFL) {
      float d = a.dt_is_tau ? dlane - tprev_lane : dlane;
      d = tk < a.L ? d : 0.0f;  // steps past the end are identity steps
      const int src0 = (lane / G) * R;  // lane of the thread's first step
#pragma unroll
      for (int r = 0; r < R; ++r) dtv[r] = __shfl(d, src0 + r);
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = draw[r];
        if (a.dt_is_tau) d -= (t0 + r > 0) ? (r > 0 ? draw[r - 1] : tprev) : 0.0f;
        dtv[r] = (t0 + r < a.L) ? d : 0.0f;
      }
    }
  }
  if constexpr (dtp) {
    {
      // stage the tile's raw rows [TC][RS] and the row's weights, transposed
      // to [CPR][RP] (a channel's column contiguous), in LDS; then one thread
      // per (step, channel) pair: rank FMAs from 16-byte LDS reads, softplus,
      // clamp -> s_dt.  Rows are padded to whole float4s (RP) and spaced RS =
      // RP + 4 floats apart, so the 16-byte reads of different steps fall in
      // different bank groups.
      const int rank = (int)a.dt_rank;
      const int RP = (rank + 3) & ~3;
      const int RS = RP + 4;
      float* s_raw = s_dt + TC * CPR;
      float* s_w = s_raw + TC * RS;
      const float* rawb = a.dt + b * a.sdt_b;
      for (int i = tid; i < TC * RP; i += blockDim.x) {
        const int st = i / RP, k = i - st * RP;
        const int64_t t = tw + st;
        s_raw[st * RS + k] = (t < a.L && k < rank) ? rawb[t * a.sdt_l + k] : 0.0f;
      }
      for (int i = tid; i < CPR * RP; i += blockDim.x) {
        const int cw = i / RP, k = i - cw * RP;
        s_w[i] = k < rank ? a.dtW[k * a.sw_r + (int64_t)h * CPR + cw] : 0.0f;
      }
      __syncthreads();
      const int cl_t = tid % CPR;  // the same channel for every pair of this thread
      const float bias = a.dtbias[(int64_t)h * CPR + cl_t];
      const float4* wv = reinterpret_cast<const float4*>(s_w + cl_t * RP);
      for (int pr = tid; pr < TC * CPR; pr += blockDim.x) {
        const int st = pr / CPR;
        const float4* rv = reinterpret_cast<const float4*>(s_raw + st * RS);
        float acc0 = bias, acc1 = 0.0f;
#pragma unroll 4
        for (int k = 0; k < RP / 4; ++k) {
          const float4 r4 = rv[k], w4 = wv[k];
          acc0 = __builtin_fmaf(r4.x, w4.x, acc0);
          acc1 = __builtin_fmaf(r4.y, w4.y, acc1);
          acc0 = __builtin_fmaf(r4.z, w4.z, acc0);
          acc1 = __builtin_fmaf(r4.w, w4.w, acc1);
        }
        // steps past the end are identity steps (dt = 0)
        s_dt[pr] = tw + st < a.L ? clamp_med3(softplus_fast(acc0 + acc1), a.dt_min, a.dt_max)
                                 : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r) dtv[r] = s_dt[(tr + r) * CPR + cl];
    }
  }
  // ZOH with a decay per lane updates h' = ab h + (ab - 1) B u / a, which must
  // stay h at the identity steps past the end: their input is zeroed.
  if (!APH && DISC == TSSM_DISC_ZOH && !fast) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (MODE == MODE_MAMBA1) {
        us[r] = t0 + r < a.L ? us[r] : 0.0f;
      } else {
        if (!(t0 + r < a.L)) vB[r].zero();
      }
    }
  }
  if constexpr (APH) {
    const float v = -expf(a2[0]) * kLog2e;
#pragma unroll
    for (int j = 0; j < 8; ++j) a2[j] = v;
  } else if constexpr (PAR_SHFL) {
    const float x = alog * kLog2e;
    const float pa = -exp2_fast(x) * kLog2e;
    const float pi = DISC == TSSM_DISC_ZOH ? -exp2_fast(-x) : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // state j of group g: lane (run j, g)
      const int src = (j * G + g) << 2;
      a2[j] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(pa)));
      if constexpr (DISC == TSSM_DISC_ZOH)
        ia[j] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(pi)));
    }
  } else if constexpr (!PAR_LDS) {
    // hardware exp2 of the base-2 argument: within ~4e-7 relative of
    // -exp(A_log), at 4 operations per channel instead of a library expf
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = a2[j] * kLog2e;
      if constexpr (DISC == TSSM_DISC_ZOH) ia[j] = -exp2_fast(-x);
      a2[j] = -exp2_fast(x) * kLog2e;
    }
  }

  // ---- sweep 1: discretize + run-local scan from (1, 0)
  // With one decay per head (APH) the run-local decay product is the same for
  // the thread's 8 channels, so sweep 2 rebuilds w_t = C_t * a_loc_t from the
  // C vector still held in registers instead of keeping 8 w values per step.
  float al[8], xl[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    al[j] = 1.0f;
    xl[j] = 0.0f;
  }
  float w[APH ? 1 : R][8];
  float alr[R];
  float y1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.0f;
    float ab_h = 0.0f, coef_h = 0.0f;
    if constexpr (APH) {
      const float arg = dtv[r] * a2[0];
      ab_h = exp2_fast(arg);
      coef_h = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(arg * 0.6931471805599453f, ab_h) * dtv[r]
                                       : dtv[r];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float ab, coef;
      if constexpr (APH) {
        ab = ab_h;
        coef = coef_h;
      } else {
        ab = exp2_fast(dtv[r] * a2[j]);
        coef = dtv[r];  // Euler input term
      }
      const float uj = (MODE == MODE_DIAG) ? vu[r].get(j) : us[r];
      if constexpr (!APH && DISC == TSSM_DISC_ZOH) {
        // ZOH with a decay per lane: the input term expm1(dt a) / a B u equals
        // (ab - 1) ibx with ibx = B u / a, so h' = ab h + (ab - 1) ibx =
        // fma(ab, h + ibx, -ibx): two operations instead of a coefficient
        // series, a select and two products.  Exact in real arithmetic; the
        // rounding of h + ibx adds one half-ulp of max(|h|, |ibx|) per step.
        const float ibx = ia[j] * (vB[r].get(j) * uj);
        xl[j] = __builtin_fmaf(ab, xl[j] + ibx, -ibx);
      } else {
        xl[j] = __builtin_fmaf(ab, xl[j], coef * vB[r].get(j) * uj);
      }
      al[j] = al[j] * ab;
      const float cj = vC[r].get(j);
      if constexpr (!APH) w[r][j] = cj * al[j];
      acc = __builtin_fmaf(cj, xl[j], acc);
      if constexpr (HAS_D && MODE == MODE_DIAG) acc = __builtin_fmaf(Dv[j], uj, acc);
    }
    alr[r] = al[0];
    // MODE_MAMBA1: D[d] x[d] once per channel (the group's first thread)
    if constexpr (HAS_D && MODE == MODE_MAMBA1)
      acc = (g % NS) == 0 ? __builtin_fmaf(Dv[0], us[r], acc) : acc;
    y1[r] = acc;
  }
  {
    float4* pa = reinterpret_cast<float4*>(s_a + run * P + ch0);
    float4* px = reinterpret_cast<float4*>(s_x + run * P + ch0);
    pa[0] = make_float4(al[0], al[1], al[2], al[3]);
    pa[1] = make_float4(al[4], al[5], al[6], al[7]);
    px[0] = make_float4(xl[0], xl[1], xl[2], xl[3]);
    px[1] = make_float4(xl[4], xl[5], xl[6], xl[7]);
  }
  __syncthreads();

  // ---- run scan: thread (channel ch, segment sg) owns runs sg*8 .. sg*8+7
  {
    const int ch = tid % P;
    const int sg = tid / P;
    const int q0 = sg * 8;
    float ea[8], ex[8];
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float ra = s_a[(q0 + q) * P + ch];
      const float rx = s_x[(q0 + q) * P + ch];
      ea[q] = A;
      ex[q] = X;
      X = __builtin_fmaf(ra, X, rx);
      A = A * ra;
    }
    s_sa[sg * P + ch] = A;
    s_sx[sg * P + ch] = X;
    __syncthreads();
    // segments 0 .. sg-1 combined (sg is uniform per wave): their totals are
    // read 4 at a time, all reads of a batch issued before the first is used
    float SA = 1.0f, SX = 0.0f;
    for (int k0 = 0; k0 < sg; k0 += 4) {
      float ka[4], kx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = k0 + i < sg ? k0 + i : sg - 1;
        ka[i] = s_sa[k * P + ch];
        kx[i] = s_sx[k * P + ch];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (k0 + i < sg) {
          SX = __builtin_fmaf(ka[i], SX, kx[i]);
          SA = SA * ka[i];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {  // exclusive prefix of run q0+q within the tile
      s_a[(q0 + q) * P + ch] = ea[q] * SA;
      s_x[(q0 + q) * P + ch] = __builtin_fmaf(ea[q], SX, ex[q]);
    }
    if (sg == NSEG - 1) {  // tile aggregate, look-back, inclusive state
      const float TA = A * SA;
      const float TX = __builtin_fmaf(A, SX, X);
      CarrySlot slot{a.words + (int64_t)row * a.nchunks * 3 * P, 3 * P, P};
      // With one decay per head its channels' tile decays are bit-identical
      // (the same products in the same order): the head's first channel
      // carries it in one word, written once and read by every channel.
      const int cha = APH ? ch - ch % (8 * NS) : ch;
      // A tile whose decay product underflowed to exactly zero forgets its
      // entry state: its inclusive state is TX whatever the carry, so it is
      // published before the look-back, alone (no walker needs its aggregate),
      // and later tiles need not wait on it.
      const bool forgets = TA == 0.0f;
      if (forgets) {
        st_word(slot.inc(c, ch), TX, tag);
      } else if (c > 0) {
        if (ch == cha) st_word(slot.agg_a(c, ch), TA, tag);
        st_word(slot.agg_x(c, ch), TX, tag);
      }
      const float hin = a.h0 ? a.h0[row * P + ch] : 0.0f;
      // per-channel walk: measured faster here than the status-word walk
      // (lookback_wave), which costs a second round trip per step
      const float carry =
          (c > 0) ? lookback_channel<WIN>(slot, c, ch, cha, tag, hin, a.spin_limit, a.hdr) : hin;
      const float incl = __builtin_fmaf(TA, carry, TX);
      if (!forgets) st_word(slot.inc(c, ch), incl, tag);
      if (a.h_last && c == a.nchunks - 1) a.h_last[row * P + ch] = incl;
      s_carry[ch] = carry;
    }
  }
  __syncthreads();

  // ---- sweep 2: entry state of the run, reduce over channels, store
  float S[8];
  {
    const float4* pa = reinterpret_cast<const float4*>(s_a + run * P + ch0);
    const float4* px = reinterpret_cast<const float4*>(s_x + run * P + ch0);
    const float4* pc = reinterpret_cast<const float4*>(s_carry + ch0);
    const float4 a0 = pa[0], a1 = pa[1], x0 = px[0], x1 = px[1], c0 = pc[0], c1 = pc[1];
    S[0] = __builtin_fmaf(a0.x, c0.x, x0.x); S[1] = __builtin_fmaf(a0.y, c0.y, x0.y);
    S[2] = __builtin_fmaf(a0.z, c0.z, x0.z); S[3] = __builtin_fmaf(a0.w, c0.w, x0.w);
    S[4] = __builtin_fmaf(a1.x, c1.x, x1.x); S[5] = __builtin_fmaf(a1.y, c1.y, x1.y);
    S[6] = __builtin_fmaf(a1.z, c1.z, x1.z); S[7] = __builtin_fmaf(a1.w, c1.w, x1.w);
  }
  T* yp = reinterpret_cast<T*>(a.y) + b * a.sy_b + tw * a.sy_l + lane_mul(tr, a.sy_l) +
          (MODE == MODE_DIAG ? (int64_t)h * P + ch0 : (int64_t)h * CPR + cl);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float v = y1[r];
    if constexpr (APH) {
      float cs = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) cs = __builtin_fmaf(vC[r].get(j), S[j], cs);
      v = __builtin_fmaf(alr[r], cs, v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v = __builtin_fmaf(w[r][j], S[j], v);
    }
    v = group_sum<NS>(v);
    if (t0 + r < a.L) {
      if constexpr (MODE == MODE_DIAG) store_bcast8<T>(yp + r * a.sy_l, v);
      else if ((g % NS) == 0) stf(yp + r * a.sy_l, v);
    }
  }
}

// ---------------------------------------------------------------- phase-exact kernels
// multihead_ssm_fwd_local_kernel (multihead_ssm_kernel.py:20-102): one
// workgroup per Triton program (row = b*nh + h, blk); thread per channel p,
// sequential over the chunk.
template <typename T>
__global__ void mh_fwd_local_kernel(const T* __restrict__ u, const float* __restrict__ A_log,
                                    const T* __restrict__ Bm, const float* __restrict__ dt,
                                    float* __restrict__ loc_a, float* __restrict__ loc_x,
                                    float* __restrict__ carry, int64_t nbatch, int64_t L,
                                    int64_t H, int64_t nh, int64_t hd, int64_t su_b, int64_t su_l,
                                    int64_t sal_h, int64_t sB_b, int64_t sB_l, int64_t sB_h,
                                    int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t blk_l,
                                    int64_t nblk) {
  const int64_t rowi = blockIdx.y;
  const int64_t blk = blockIdx.x;
  const int64_t bi = rowi / nh;
  const int64_t hi = rowi - bi * nh;
  const int64_t ts = blk * blk_l;
  const int64_t te = ts + blk_l > L ? L : ts + blk_l;
  const int64_t rows_tot = nbatch * nh * hd;
  // The loads of a step are issued kB steps before it is computed: after each
  // step its registers are refilled with step t + kB (clamped to the block's
  // last step, whose duplicates are never used), so the wave streams instead
  // of alternating a load round trip with kB steps of compute.  exp(d a) as
  // hardware exp2 of d a log2e.
  constexpr int kB = 8;
  for (int64_t p = threadIdx.x; p < hd; p += blockDim.x) {
    const float a2 = -expf(A_log[hi * sal_h + p]) * kLog2e;
    const int64_t uo = hi * hd + p;
    const bool u_ok = uo < H;
    const float* dtp = dt + bi * sdt_b + hi * sdt_h;
    const T* bp = Bm + bi * sB_b + hi * sB_h + p;
    const T* up = u + bi * su_b + (u_ok ? uo : 0);
    float* lap = loc_a + bi * (L * nh * hd) + hi * hd + p;
    float* lxp = loc_x + bi * (L * nh * hd) + hi * hd + p;
    float ar = 1.0f, xr = 0.0f;
    float dv[kB], bv[kB], uv[kB];
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int64_t t = ts + k < te ? ts + k : te - 1;
      dv[k] = dtp[t * sdt_l];
      bv[k] = ldf(bp + t * sB_l);
      uv[k] = ldf(up + t * su_l);
    }
    for (int64_t t0 = ts; t0 < te; t0 += kB) {
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int64_t t = t0 + k;
        if (t < te) {  // uniform
          const float ab = exp2_fast(dv[k] * a2);
          xr = ab * xr + dv[k] * bv[k] * (u_ok ? uv[k] : 0.0f);
          ar = ab * ar;
          const int64_t off = t * (nh * hd);
          lap[off] = ar;
          lxp[off] = xr;
        }
        __builtin_amdgcn_sched_barrier(0);
        const int64_t tn = t + kB < te ? t + kB : te - 1;
        dv[k] = dtp[tn * sdt_l];
        bv[k] = ldf(bp + tn * sB_l);
        uv[k] = ldf(up + tn * su_l);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const int64_t rf = bi * (nh * hd) + hi * hd + p;
    carry[rf * nblk + blk] = ar;
    carry[rows_tot * nblk + rf * nblk + blk] = xr;
  }
}

// Block-wide sum (blockDim multiple of 64, <= 1024) returned to every thread.
__device__ inline float block_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int nw = blockDim.x >> 6;
  if (nw == 1) return v;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}

// multihead_ssm_output_kernel (multihead_ssm_kernel.py:121-187).
template <typename T>
__global__ void mh_output_kernel(const float* __restrict__ loc_a, const float* __restrict__ loc_x,
                                 const float* __restrict__ carry, const T* __restrict__ Cm,
                                 const float* __restrict__ D, const T* __restrict__ u,
                                 T* __restrict__ y, int64_t nbatch, int64_t L, int64_t H,
                                 int64_t nh, int64_t hd, int64_t su_b, int64_t su_l, int64_t sC_b,
                                 int64_t sC_l, int64_t sC_h, int64_t blk_l, int64_t nblk) {
  __shared__ float red[16];
  const int64_t rowi = blockIdx.y;
  const int64_t blk = blockIdx.x;
  const int64_t bi = rowi / nh;
  const int64_t hi = rowi - bi * nh;
  const int64_t ts = blk * blk_l;
  const int64_t te = ts + blk_l > L ? L : ts + blk_l;
  const int64_t rows_tot = nbatch * nh * hd;
  const int64_t p = threadIdx.x;
  const bool active = p < hd;
  const int64_t uo = hi * hd + p;
  const bool u_ok = active && uo < H;
  float x_pref = 0.0f;
  if (active && blk > 0) {
    const int64_t rf = bi * (nh * hd) + hi * hd + p;
    x_pref = carry[rows_tot * nblk + rf * nblk + blk - 1];
  }
  const float dv = u_ok ? D[uo] : 0.0f;
  // kU steps at a time: every load of the batch is issued before the first
  // reduction (steps past the block re-read its last step and store nothing)
  constexpr int kU = 8;
  const bool one_wave = blockDim.x == 64;
  for (int64_t t = ts; t < te; t += kU) {
    float c[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
      const int64_t tt = t + k < te ? t + k : te - 1;
      float contrib = 0.0f;
      if (active) {
        const int64_t off = bi * (L * nh * hd) + tt * (nh * hd) + hi * hd + p;
        const float hv = loc_a[off] * x_pref + loc_x[off];
        contrib = ldf(Cm + bi * sC_b + tt * sC_l + hi * sC_h + p) * hv;
        if (u_ok) contrib += dv * ldf(u + bi * su_b + tt * su_l + uo);
      }
      c[k] = contrib;
    }
    if (one_wave) {  // uniform: the kU wave sums interleaved
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int k = 0; k < kU; ++k) c[k] += __shfl_xor(c[k], o);
    } else {
#pragma unroll
      for (int k = 0; k < kU; ++k) c[k] = block_sum(c[k], red);
    }
#pragma unroll
    for (int k = 0; k < kU; ++k)
      if (u_ok && t + k < te) stf(y + bi * (L * H) + (t + k) * H + uo, c[k]);
  }
}

// Vector form for 4-aligned operands (head_dim = 4 LPS, LPS in 4..32): a
// thread owns 4 channels (16-byte fp32 / 8-byte 16-bit accesses), LPS lanes
// cover one step, so one wave instruction covers 64 / LPS steps.  Per step:
// the 4-channel partial sum, then an LPS-lane sum (DPP up to 16 lanes), the
// head value stored broadcast over the thread's 4 channels.  kOutR steps per
// thread are loaded before any is reduced.  Same grid and results as
// mh_output_kernel (the sums reassociate).
constexpr int kOutR = 8;

template <int LPS>
__device__ inline float lanes_sum(float v) {
  if constexpr (LPS <= 16) {
    return group_sum<LPS>(v);
  } else {
#pragma unroll
    for (int o = LPS / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
  }
}

template <typename T, int LPS>
__global__ __launch_bounds__(256) void mh_output_vec_kernel(
    const float* __restrict__ loc_a, const float* __restrict__ loc_x,
    const float* __restrict__ carry, const T* __restrict__ Cm, const float* __restrict__ D,
    const T* __restrict__ u, T* __restrict__ y, int64_t nbatch, int64_t L, int64_t H, int64_t nh,
    int64_t hd, int64_t su_b, int64_t su_l, int64_t sC_b, int64_t sC_l, int64_t sC_h,
    int64_t blk_l, int64_t nblk) {
  constexpr int SPW = 64 / LPS;  // steps per wave instruction
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane % LPS, sl = lane / LPS;
  const int64_t rowi = blockIdx.y, blk = blockIdx.x;
  const int64_t bi = rowi / nh, hi = rowi - bi * nh;
  const int64_t ts = blk * blk_l;
  const int64_t te = ts + blk_l > L ? L : ts + blk_l;
  const int64_t p = 4 * q;
  const int64_t uo = hi * hd + p;
  const bool u_ok = uo < H;  // H % 4 == 0: all 4 channels or none
  float xp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (blk > 0) {
    const int64_t rows_tot = nbatch * nh * hd;
    const int64_t rf = bi * (nh * hd) + hi * hd + p;
#pragma unroll
    for (int j = 0; j < 4; ++j) xp[j] = carry[rows_tot * nblk + (rf + j) * nblk + blk - 1];
  }
  float dv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (u_ok) ld_lanes<float, 4>(D + uo, dv);
  const float* la = loc_a + bi * (L * nh * hd) + hi * hd + p;
  const float* lx = loc_x + bi * (L * nh * hd) + hi * hd + p;
  const T* cb = Cm + bi * sC_b + hi * sC_h + p;
  const T* ub = u + bi * su_b + (u_ok ? uo : 0);
  T* yb = y + bi * (L * H) + uo;
  const int64_t row = nh * hd;  // loc_a / loc_x step stride
  constexpr int PASS = 4 * SPW * kOutR;  // steps per workgroup pass (4 waves)
  for (int64_t t0 = ts; t0 < te; t0 += PASS) {
    float a4[kOutR][4], x4[kOutR][4], c4[kOutR][4], u4[kOutR][4];
#pragma unroll
    for (int k = 0; k < kOutR; ++k) {
      const int64_t t = t0 + (k * 4 + wave) * SPW + sl;
      const int64_t tt = t < te ? t : te - 1;  // steps past the block re-read its last step
      // loc_a / loc_x are read exactly once: streaming (nontemporal) loads
      const f32x4 va = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(la + tt * row));
      const f32x4 vx = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(lx + tt * row));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a4[k][j] = va[j];
        x4[k][j] = vx[j];
      }
      ld_lanes<T, 4>(cb + tt * sC_l, c4[k]);
      ld_lanes<T, 4>(ub + tt * su_l, u4[k]);
    }
    float c[kOutR];
#pragma unroll
    for (int k = 0; k < kOutR; ++k) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = __builtin_fmaf(c4[k][j], __builtin_fmaf(a4[k][j], xp[j], x4[k][j]), acc);
        if (u_ok) acc = __builtin_fmaf(dv[j], u4[k][j], acc);
      }
      c[k] = acc;
    }
#pragma unroll
    for (int k = 0; k < kOutR; ++k) c[k] = lanes_sum<LPS>(c[k]);
#pragma unroll
    for (int k = 0; k < kOutR; ++k) {
      const int64_t t = t0 + (k * 4 + wave) * SPW + sl;
      if (u_ok && t < te) {
        const float v[4] = {c[k], c[k], c[k], c[k]};
        st_lanes<T, 4>(yb + t * H, v);
      }
    }
  }
}

// ---------------------------------------------------------------- host side
namespace {

struct TileCfg {
  int G, NS, W, TC;
  int64_t hpr;  // heads per row (MODE_DIAG)
};

inline bool mh_tile_cfg(int64_t head_dim, int64_t chunk, TileCfg* cfg) {
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 128) return false;
  const int G = (int)(head_dim / 8);
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) return false;
  const int rows = 64 / G;
  int W = (int)(chunk / (rows * kMhR));
  if (W < 1) W = 1;
  if (W > 8) W = 8;
  cfg->G = G;
  cfg->NS = G;
  cfg->W = W;
  cfg->TC = W * rows * kMhR;
  cfg->hpr = 1;
  return true;
}

// MODE_DIAG rows: heads narrower than 64 channels (64-, 32- or 16-byte bf16
// rows, 8-32 rows per wave instruction) are packed 128 / head_dim to a
// 128-lane row when n_heads allows, with tiles of the same chunk of steps.
// 64-channel heads stay one per row: packed in pairs they measured slower.
inline bool mh_diag_cfg(int64_t head_dim, int64_t n_heads, int64_t chunk, TileCfg* cfg) {
  if (!mh_tile_cfg(head_dim, chunk, cfg)) return false;
  if (head_dim < 64) {
    const int64_t hpr = 128 / head_dim;
    TileCfg p;
    if (n_heads % hpr == 0 && mh_tile_cfg(128, chunk, &p)) {
      p.NS = (int)(head_dim / 8);
      p.hpr = hpr;
      *cfg = p;
    }
  }
  return true;
}

// True when every per-lane byte offset of a tile -- up to TC steps of the
// largest row stride plus the row's columns, for the I/O operands (element
// size esize) and for dt (fp32) -- stays below 2^31: full tiles then load
// through a uniform base plus a 32-bit lane offset.  Strides are >= 0.
inline bool tile_offsets_fit(int64_t TC, int64_t cpr, int64_t cols, int64_t esize, int64_t su_l,
                             int64_t sB_l, int64_t sC_l, int64_t sB_h, int64_t sC_h,
                             int64_t sdt_l, int64_t sdt_h) {
  const int64_t lim = int64_t(1) << 31;
  const int64_t sl = su_l > sB_l ? (su_l > sC_l ? su_l : sC_l) : (sB_l > sC_l ? sB_l : sC_l);
  const int64_t sh = sB_h > sC_h ? sB_h : sC_h;
  if (sl >= lim || sh >= lim || sdt_l >= lim || sdt_h >= lim) return false;
  const int64_t io = (TC * sl + cpr * sh + cols + 8) * esize;
  const int64_t dt = (TC * sdt_l + cpr * sdt_h) * 4;
  return io < lim && dt < lim;
}

inline int64_t mh_ws_bytes(int64_t nrows, int64_t L, int64_t P, int TC) {
  return (int64_t)sizeof(WsHeader) + nrows * ((L + TC - 1) / TC) * 3 * P * 8;
}

template <typename T, int DISC, bool APH, bool HAS_D, int MODE>
int launch_mh_fused_g(int G, int NS, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                      const MhArgs& a) {
#define TSSM_MH(GV, NV)                                                                         \
  if (G == GV && NS == NV) {                                                                   \
    hipLaunchKernelGGL((mh_scan_fused_kernel<T, DISC, APH, HAS_D, GV, MODE, NV>), grid, block, \
                       lds, s, a);                                                             \
    return launch_status();                                                                    \
  }
  TSSM_MH(1, 1) TSSM_MH(2, 2) TSSM_MH(4, 4) TSSM_MH(8, 8) TSSM_MH(16, 16)
  TSSM_MH(16, 4) TSSM_MH(16, 2) TSSM_MH(16, 1)
#undef TSSM_MH
  return TSSM_ERR_UNSUPPORTED;
}

// MODE_MAMBA1 rows of P = 8 G lanes holding channels of N = 8 NS states.
template <typename T, int DISC, bool HAS_D>
int launch_sel_gn(int G, int NS, dim3 grid, dim3 block, size_t lds, hipStream_t s, const MhArgs& a) {
  const bool dtp = a.dtW != nullptr;
#define TSSM_SEL(GV, NV)                                                                          \
  if (G == GV && NS == NV) {                                                                    \
    if (dtp)                                                                                    \
      hipLaunchKernelGGL((mh_scan_fused_kernel<T, DISC, false, HAS_D, GV, MODE_MAMBA1, NV, true>), \
                         grid, block, lds, s, a);                                               \
    else                                                                                        \
      hipLaunchKernelGGL((mh_scan_fused_kernel<T, DISC, false, HAS_D, GV, MODE_MAMBA1, NV>), grid, \
                         block, lds, s, a);                                                     \
    return launch_status();                                                                     \
  }
  TSSM_SEL(8, 1) TSSM_SEL(8, 2) TSSM_SEL(8, 4) TSSM_SEL(8, 8) TSSM_SEL(16, 16)
  TSSM_SEL(1, 1) TSSM_SEL(2, 1) TSSM_SEL(2, 2) TSSM_SEL(4, 1) TSSM_SEL(4, 2) TSSM_SEL(4, 4)
#undef TSSM_SEL
  return TSSM_ERR_UNSUPPORTED;
}

template <typename T, int DISC>
int launch_mh_fused_d(bool aph, bool has_d, int G, int NS, dim3 grid, dim3 block, size_t lds,
                      hipStream_t s, const MhArgs& a) {
  if (aph)
    return has_d ? launch_mh_fused_g<T, DISC, true, true, MODE_DIAG>(G, NS, grid, block, lds, s, a)
                 : launch_mh_fused_g<T, DISC, true, false, MODE_DIAG>(G, NS, grid, block, lds, s, a);
  return has_d ? launch_mh_fused_g<T, DISC, false, true, MODE_DIAG>(G, NS, grid, block, lds, s, a)
               : launch_mh_fused_g<T, DISC, false, false, MODE_DIAG>(G, NS, grid, block, lds, s, a);
}

template <typename T>
int launch_mh_fused_t(int disc, bool aph, bool has_d, int G, int NS, dim3 grid, dim3 block,
                      size_t lds, hipStream_t s, const MhArgs& a) {
  if (disc == TSSM_DISC_ZOH)
    return launch_mh_fused_d<T, TSSM_DISC_ZOH>(aph, has_d, G, NS, grid, block, lds, s, a);
  return launch_mh_fused_d<T, TSSM_DISC_EULER>(aph, has_d, G, NS, grid, block, lds, s, a);
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace tssm

using namespace tssm;

extern "C" int64_t tssm_mh_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t n_heads,
                                                int64_t head_dim, int64_t chunk) {
  TileCfg cfg;
  if (nbatch <= 0 || L <= 0 || n_heads <= 0 || !mh_diag_cfg(head_dim, n_heads, chunk, &cfg))
    return -1;
  return mh_ws_bytes(nbatch * n_heads / cfg.hpr, L, head_dim * cfg.hpr, cfg.TC);
}

namespace tssm {
namespace {

// Scratch of the no-allocation entry point (tssm_mh_scan_fused_noalloc): the
// look-back workspace as one fixed array per device, zero when the module is
// loaded.  Host code never passes `scratch` itself to a kernel (on the host
// the name is a stand-in, not a device address): each device's address is
// resolved once with hipGetSymbolAddress, with that device current, and kept
// in g_scratch.  The epoch scheme needs no clearing between calls; calls that
// overlap on one device race on the array.
constexpr int64_t kScratchBytes = TSSM_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// Device address of the current device's scratch.  `device` is the current
// device.
int scratch_for(int device, void** ptr) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    g_scratch[device] = p;
  }
  *ptr = g_scratch[device];
  return TSSM_OK;
}

// The scratch's launch tag lives in its header and is advanced on the
// device, by this one-thread kernel enqueued right before each scan on the
// same stream: a launch captured in a HIP graph then takes a fresh tag on
// every replay (a tag fixed at capture time would let a replay read the
// previous replay's words as its own).  Vector stores only.
__global__ void advance_epoch_kernel(WsHeader* hdr) {
  if (threadIdx.x == 0) {
    uint32_t e = load_epoch(hdr) + 1u;
    if (e == 0) e = 1;  // 0 is the tag of a zero-filled word
    __hip_atomic_store(&hdr->epoch, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Argument checks and launch shared by tssm_mh_scan_fused and its
// no-allocation variant; `tag` is the epoch of this launch on `workspace`,
// or 0 when the kernel takes the header's device-advanced epoch.
int mh_scan_fused_launch(int dtype, int disc, const void* u, const float* A_log, const void* B,
                         const void* C, const float* dt, const float* D, const float* h0,
                         void* y, float* h_last, int64_t nbatch, int64_t L, int64_t n_heads,
                         int64_t head_dim, int a_per_head, int64_t su_b, int64_t su_l,
                         int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sC_b, int64_t sC_l,
                         int64_t sC_h, int64_t sdt_b, int64_t sdt_l, int64_t sdt_h,
                         int64_t sy_b, int64_t sy_l, const TileCfg& cfg, void* workspace,
                         uint32_t tag, void* stream) {
  // 8-channel vectors must be 16-byte aligned: base pointers and every stride.
  const int64_t vec = dtype == TSSM_F32 ? 4 : 8;
  const int64_t strides[] = {su_b, su_l, sB_b, sB_l, sB_h, sC_b, sC_l, sC_h, sy_b, sy_l};
  for (int64_t s : strides) TSSM_CHECK(s >= 0 && s % vec == 0, TSSM_ERR_ALIGN);
  TSSM_CHECK(aligned(u, 16) && aligned(B, 16) && aligned(C, 16) && aligned(y, 16),
             TSSM_ERR_ALIGN);
  TSSM_CHECK((a_per_head || aligned(A_log, 16)) && (!D || aligned(D, 16)), TSSM_ERR_ALIGN);
  TSSM_CHECK(sdt_b >= 0 && sdt_l >= 0 && sdt_h >= 0, TSSM_ERR_STRIDE);

  const int64_t nchunks = cdiv(L, cfg.TC);
  const int64_t nrows = nbatch * (n_heads / cfg.hpr);
  const int64_t P = head_dim * cfg.hpr;  // lanes per row
  TSSM_CHECK(nchunks * nrows < (int64_t)INT32_MAX, TSSM_ERR_UNSUPPORTED);
  MhArgs a;
  a.u = u; a.A_log = A_log; a.B = B; a.C = C; a.dt = dt; a.D = D; a.h0 = h0; a.y = y;
  a.h_last = h_last;
  a.L = L;
  a.su_b = su_b; a.su_l = su_l; a.sB_b = sB_b; a.sB_l = sB_l; a.sB_h = sB_h;
  a.sC_b = sC_b; a.sC_l = sC_l; a.sC_h = sC_h;
  a.sdt_b = sdt_b; a.sdt_l = sdt_l; a.sdt_h = sdt_h; a.sy_b = sy_b; a.sy_l = sy_l;
  a.hdr = reinterpret_cast<WsHeader*>(workspace);
  a.words = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + sizeof(WsHeader));
  a.n_heads = (uint32_t)(n_heads / cfg.hpr);  // rows per batch
  a.nchunks = (uint32_t)nchunks;
  a.nrows = (uint32_t)nrows;
  a.tag = tag;
  a.tag_in_ws = tag == 0 ? 1u : 0u;
  a.spin_limit = kDefaultSpinLimit;
  a.dt_is_tau = 0;
  a.off32 = tile_offsets_fit(cfg.TC, cfg.hpr, P, dtype == TSSM_F32 ? 4 : 2, su_l, sB_l, sC_l,
                             sB_h, sC_h, sdt_l, sdt_h) ? 1u : 0u;

  const dim3 grid((unsigned)(nchunks * nrows)), block((unsigned)(cfg.W * 64));
  const int nrun = cfg.W * (64 / cfg.G);
  const size_t lds = ((size_t)2 * nrun * P + 2 * (nrun / 8) * P + 3 * P) * sizeof(float);
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
  const bool aph = a_per_head != 0;
  if (a.tag_in_ws) {
    hipLaunchKernelGGL(advance_epoch_kernel, dim3(1), dim3(64), 0, s, a.hdr);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  switch (dtype) {
    case TSSM_BF16: return launch_mh_fused_t<bf16_t>(disc, aph, has_d, cfg.G, cfg.NS, grid, block, lds, s, a);
    case TSSM_F16: return launch_mh_fused_t<f16_t>(disc, aph, has_d, cfg.G, cfg.NS, grid, block, lds, s, a);
    default: return launch_mh_fused_t<float>(disc, aph, has_d, cfg.G, cfg.NS, grid, block, lds, s, a);
  }
}

}  // namespace

int noalloc_scratch_header(void** ptr) {
  int device = 0;
  const hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return (int)st;
  TSSM_CHECK(device >= 0 && device < kMaxDevices, TSSM_ERR_UNSUPPORTED);
  return scratch_for(device, ptr);
}

int noalloc_scratch_error(int clear, int* error_out) {
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return (int)st;
  TSSM_CHECK(device >= 0 && device < kMaxDevices, TSSM_ERR_UNSUPPORTED);
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[device];
  }
  *error_out = 0;
  if (p == nullptr) return TSSM_OK;  // no no-allocation launch on this device yet
  const auto* hdr = reinterpret_cast<const WsHeader*>(p);
  uint32_t e = 0;
  st = hipMemcpy(&e, &hdr->error, sizeof(e), hipMemcpyDeviceToHost);
  if (st != hipSuccess) return (int)st;
  *error_out = (int)e;
  if (clear && e) {
    const uint32_t z = 0;
    st = hipMemcpy(const_cast<uint32_t*>(&hdr->error), &z, sizeof(z), hipMemcpyHostToDevice);
    if (st != hipSuccess) return (int)st;
  }
  return TSSM_OK;
}

}  // namespace tssm

extern "C" int tssm_mh_scan_fused(int dtype, int disc, const void* u, const float* A_log,
                                  const void* B, const void* C, const float* dt, const float* D,
                                  const float* h0, void* y, float* h_last, int64_t nbatch,
                                  int64_t L, int64_t n_heads, int64_t head_dim, int a_per_head,
                                  int64_t su_b, int64_t su_l, int64_t sB_b, int64_t sB_l,
                                  int64_t sB_h, int64_t sC_b, int64_t sC_l, int64_t sC_h,
                                  int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t sy_b,
                                  int64_t sy_l, int64_t chunk, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(u && A_log && B && C && dt && y, TSSM_ERR_NULL);
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16 || dtype == TSSM_F16, TSSM_ERR_DTYPE);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && n_heads > 0, TSSM_ERR_SHAPE);
  TileCfg cfg;
  TSSM_CHECK(mh_diag_cfg(head_dim, n_heads, chunk, &cfg), TSSM_ERR_UNSUPPORTED);
  const int64_t need = tssm_mh_scan_workspace_bytes(nbatch, L, n_heads, head_dim, chunk);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 256), TSSM_ERR_ALIGN);
  return mh_scan_fused_launch(dtype, disc, u, A_log, B, C, dt, D, h0, y, h_last, nbatch, L,
                              n_heads, head_dim, a_per_head, su_b, su_l, sB_b, sB_l, sB_h, sC_b,
                              sC_l, sC_h, sdt_b, sdt_l, sdt_h, sy_b, sy_l, cfg, workspace,
                              next_epoch(workspace), stream);
}

extern "C" int tssm_mh_scan_fused_noalloc(int dtype, int disc, const void* u, const float* A_log,
                                          const void* B, const void* C, const float* dt,
                                          const float* D, const float* h0, void* y,
                                          float* h_last, int64_t nbatch, int64_t L,
                                          int64_t n_heads, int64_t head_dim, int a_per_head,
                                          int64_t su_b, int64_t su_l, int64_t sB_b, int64_t sB_l,
                                          int64_t sB_h, int64_t sC_b, int64_t sC_l, int64_t sC_h,
                                          int64_t sdt_b, int64_t sdt_l, int64_t sdt_h,
                                          int64_t sy_b, int64_t sy_l, int64_t chunk,
                                          void* stream) {
  TSSM_CHECK(u && A_log && B && C && dt && y, TSSM_ERR_NULL);
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16 || dtype == TSSM_F16, TSSM_ERR_DTYPE);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && n_heads > 0, TSSM_ERR_SHAPE);
  TileCfg cfg;
  TSSM_CHECK(mh_diag_cfg(head_dim, n_heads, chunk, &cfg), TSSM_ERR_UNSUPPORTED);
  const int64_t need = tssm_mh_scan_workspace_bytes(nbatch, L, n_heads, head_dim, chunk);
  TSSM_CHECK(need > 0 && need <= kScratchBytes, TSSM_ERR_SCRATCH);
  // the scratch is resolved for the current device: the stream must be on it
  int device = 0, stream_device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return (int)st;
  st = hipStreamGetDevice(as_stream(stream), &stream_device);
  if (st != hipSuccess) return (int)st;
  TSSM_CHECK(device == stream_device && device >= 0 && device < kMaxDevices,
             TSSM_ERR_UNSUPPORTED);
  void* ws = nullptr;
  const int rc = scratch_for(device, &ws);
  if (rc != TSSM_OK) return rc;
  // tag 0: the scan takes the epoch that advance_epoch_kernel sets
  return mh_scan_fused_launch(dtype, disc, u, A_log, B, C, dt, D, h0, y, h_last, nbatch, L,
                              n_heads, head_dim, a_per_head, su_b, su_l, sB_b, sB_l, sB_h, sC_b,
                              sC_l, sC_h, sdt_b, sdt_l, sdt_h, sy_b, sy_l, cfg, ws, 0, stream);
}

extern "C" int tssm_mh_fwd_local(int dtype, const void* u, const float* A_log, const void* B,
                                 const float* dt, float* loc_a, float* loc_x, float* carry,
                                 int64_t nbatch, int64_t L, int64_t H, int64_t n_heads,
                                 int64_t head_dim, int64_t su_b, int64_t su_l, int64_t sal_h,
                                 int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sdt_b,
                                 int64_t sdt_l, int64_t sdt_h, int64_t blk_l, int64_t nblk,
                                 int64_t grid_rows, int64_t grid_blks, void* stream) {
  TSSM_CHECK(u && A_log && B && dt && loc_a && loc_x && carry, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch > 0 && L > 0 && H > 0 && n_heads > 0 && head_dim > 0 && blk_l > 0 &&
                 nblk > 0 && grid_rows >= 0 && grid_blks >= 0,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_rows <= nbatch * n_heads && grid_blks <= nblk, TSSM_ERR_SHAPE);
  if (grid_rows == 0 || grid_blks == 0) return TSSM_OK;
  TSSM_CHECK(grid_rows <= 65535, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)grid_blks, (unsigned)grid_rows);
  const dim3 block(head_dim >= 256 ? 256 : (unsigned)(cdiv(head_dim, 64) * 64));
  const hipStream_t s = as_stream(stream);
#define TSSM_MH_LOCAL(T)                                                                        \
  hipLaunchKernelGGL(mh_fwd_local_kernel<T>, grid, block, 0, s, (const T*)u, A_log,          \
                     (const T*)B, dt, loc_a, loc_x, carry, nbatch, L, H, n_heads, head_dim,   \
                     su_b, su_l, sal_h, sB_b, sB_l, sB_h, sdt_b, sdt_l, sdt_h, blk_l, nblk)
  switch (dtype) {
    case TSSM_F32: TSSM_MH_LOCAL(float); break;
    case TSSM_BF16: TSSM_MH_LOCAL(bf16_t); break;
    case TSSM_F16: TSSM_MH_LOCAL(f16_t); break;
    default: return TSSM_ERR_DTYPE;
  }
#undef TSSM_MH_LOCAL
  return launch_status();
}

extern "C" int tssm_mh_output(int dtype, const float* loc_a, const float* loc_x,
                              const float* carry, const void* C, const float* D, const void* u,
                              void* y, int64_t nbatch, int64_t L, int64_t H, int64_t n_heads,
                              int64_t head_dim, int64_t su_b, int64_t su_l, int64_t sC_b,
                              int64_t sC_l, int64_t sC_h, int64_t blk_l, int64_t nblk,
                              int64_t grid_rows, int64_t grid_blks, void* stream) {
  TSSM_CHECK(loc_a && loc_x && carry && C && D && u && y, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch > 0 && L > 0 && H > 0 && n_heads > 0 && head_dim > 0 && blk_l > 0 &&
                 nblk > 0 && grid_rows >= 0 && grid_blks >= 0,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_rows <= nbatch * n_heads && grid_blks <= nblk, TSSM_ERR_SHAPE);
  TSSM_CHECK(head_dim <= 1024, TSSM_ERR_UNSUPPORTED);
  if (grid_rows == 0 || grid_blks == 0) return TSSM_OK;
  TSSM_CHECK(grid_rows <= 65535, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)grid_blks, (unsigned)grid_rows);
  const hipStream_t s = as_stream(stream);
  {
    // 4 channels per thread when every row start is a 4-element vector
    const int64_t ve = dtype == TSSM_F32 ? 16 : 8;  // bytes of 4 elements
    const int lps = (int)(head_dim / 4);
    const bool vec = head_dim % 4 == 0 && (lps == 4 || lps == 8 || lps == 16 || lps == 32) &&
                     H % 4 == 0 && su_b % 4 == 0 && su_l % 4 == 0 && sC_b % 4 == 0 &&
                     sC_l % 4 == 0 && sC_h % 4 == 0 && aligned(loc_a, 16) && aligned(loc_x, 16) &&
                     aligned(D, 16) && aligned(C, ve) && aligned(u, ve) && aligned(y, ve);
    if (vec) {
#define TSSM_MH_OV(T, LP)                                                                      \
  hipLaunchKernelGGL((mh_output_vec_kernel<T, LP>), grid, dim3(256), 0, s, loc_a, loc_x, carry, \
                     (const T*)C, D, (const T*)u, (T*)y, nbatch, L, H, n_heads, head_dim, su_b, \
                     su_l, sC_b, sC_l, sC_h, blk_l, nblk)
#define TSSM_MH_OVL(T)                       \
  switch (lps) {                             \
    case 4: TSSM_MH_OV(T, 4); break;         \
    case 8: TSSM_MH_OV(T, 8); break;         \
    case 16: TSSM_MH_OV(T, 16); break;       \
    default: TSSM_MH_OV(T, 32); break;       \
  }
      switch (dtype) {
        case TSSM_F32: TSSM_MH_OVL(float); break;
        case TSSM_BF16: TSSM_MH_OVL(bf16_t); break;
        case TSSM_F16: TSSM_MH_OVL(f16_t); break;
        default: return TSSM_ERR_DTYPE;
      }
#undef TSSM_MH_OVL
#undef TSSM_MH_OV
      return launch_status();
    }
  }
  const dim3 block((unsigned)(cdiv(head_dim, 64) * 64));
#define TSSM_MH_OUT(T)                                                                         \
  hipLaunchKernelGGL(mh_output_kernel<T>, grid, block, 0, s, loc_a, loc_x, carry, (const T*)C, \
                     D, (const T*)u, (T*)y, nbatch, L, H, n_heads, head_dim, su_b, su_l, sC_b, \
                     sC_l, sC_h, blk_l, nblk)
  switch (dtype) {
    case TSSM_F32: TSSM_MH_OUT(float); break;
    case TSSM_BF16: TSSM_MH_OUT(bf16_t); break;
    case TSSM_F16: TSSM_MH_OUT(f16_t); break;
    default: return TSSM_ERR_DTYPE;
  }
#undef TSSM_MH_OUT
  return launch_status();
}

// ---------------------------------------------------------------- selective scan (Mamba-1 lanes)
namespace tssm {
namespace {
template <typename T, int DISC>
int launch_sel_d(bool has_d, int G, int NS, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                 const MhArgs& a) {
  return has_d ? launch_sel_gn<T, DISC, true>(G, NS, grid, block, lds, s, a)
               : launch_sel_gn<T, DISC, false>(G, NS, grid, block, lds, s, a);
}
template <typename T>
int launch_sel_t(int disc, bool has_d, int G, int NS, dim3 grid, dim3 block, size_t lds,
                 hipStream_t s, const MhArgs& a) {
  if (disc == TSSM_DISC_ZOH) return launch_sel_d<T, TSSM_DISC_ZOH>(has_d, G, NS, grid, block, lds, s, a);
  return launch_sel_d<T, TSSM_DISC_EULER>(has_d, G, NS, grid, block, lds, s, a);
}
// Channels packed per row: rows of 64 lanes (128 when N = 128), so tiles are
// as large as the multihead ones; must divide Dc.
inline int64_t sel_channels_per_row(int64_t Dc, int64_t N) {
  int64_t cpr = N >= 64 ? 1 : 64 / N;
  while (cpr > 1 && Dc % cpr != 0) cpr /= 2;
  return cpr;
}
}  // namespace
}  // namespace tssm

namespace tssm {
namespace {
// Look-back words of the single-pass scan (tagged, epoch-checked), then the
// three-pass scan's chunk states in a separate region, so neither ever reads
// the other's data as its own.
int64_t sel_lookback_bytes(int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t chunk) {
  if (Dc <= 0 || N <= 0 || N % 8 != 0) return -1;
  const int64_t cpr = sel_channels_per_row(Dc, N);
  TileCfg cfg;
  if (nbatch <= 0 || L <= 0 || !mh_tile_cfg(cpr * N, chunk, &cfg)) return -1;
  return mh_ws_bytes(nbatch * (Dc / cpr), L, cpr * N, cfg.TC);
}
int64_t sel_chunked_offset(int64_t lookback_bytes) { return (lookback_bytes + 255) / 256 * 256; }
}  // namespace
}  // namespace tssm

extern "C" int64_t tssm_selective_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t Dc,
                                                       int64_t N, int64_t chunk) {
  const int64_t lb = sel_lookback_bytes(nbatch, L, Dc, N, chunk);
  if (lb < 0) return -1;
  const int64_t cb = sel_chunked_bytes(nbatch, L, Dc, N);
  return cb > 0 ? sel_chunked_offset(lb) + cb : lb;
}

extern "C" int64_t tssm_selective_scan_dtproj_workspace_bytes(int64_t nbatch, int64_t L,
                                                              int64_t Dc, int64_t N,
                                                              int64_t chunk) {
  const int64_t base = tssm_selective_scan_workspace_bytes(nbatch, L, Dc, N, chunk);
  if (base < 0) return -1;
  if (sel_chunked_bytes(nbatch, L, Dc, N) == 0) return base;
  return sel_chunked_offset(base) + sel_dt_table_bytes(nbatch, L, Dc);
}

namespace tssm {
namespace {

// Largest rank of the fused dt projection: raw rows, weights and dt values of
// a tile are staged in LDS.
constexpr int64_t kMaxDtRank = 64;

struct DtProj {
  const float* W = nullptr;
  const float* bias = nullptr;
  int64_t sw_r = 0, rank = 0;
  float dt_min = 0.0f, dt_max = 0.0f;
};

// Whether a selective scan takes the three-pass path: large problems with 8
// or 16 states, fp32 or bf16 I/O; dt given (timestamps only when shared by
// the channels) or projected from raw rows of 16-byte vectors.
bool sel_takes_passes(int dtype, int64_t nbatch, int64_t L, int64_t Dc, int64_t N,
                      bool dt_shared, bool dt_is_tau, bool proj, bool proj_ok) {
  const int64_t rs = sel_chunk_steps(nbatch, L, Dc);
  const int64_t cb = sel_chunked_bytes(nbatch, L, Dc, N);
  return (!proj || proj_ok) && cb > 0 && (dtype == TSSM_F32 || dtype == TSSM_BF16) &&
         (dt_shared || !dt_is_tau) && nbatch <= 65535 &&
         nbatch * ((Dc + 63) / 64) * ((L + rs - 1) / rs) >= kSelMinWaves;
}

int selective_scan_launch(int dtype, int disc, const void* x, const float* dt, int dt_is_tau,
                          const DtProj& proj, const float* A_log, const void* B, const void* C,
                          const float* D, const float* h0, void* y, float* h_last,
                          int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t sx_b,
                          int64_t sx_l, int64_t sdt_b, int64_t sdt_l, int64_t sdt_d,
                          int64_t sB_b, int64_t sB_l, int64_t sC_b, int64_t sC_l, int64_t sy_b,
                          int64_t sy_l, int64_t chunk, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  TSSM_CHECK(x && dt && A_log && B && C && y, TSSM_ERR_NULL);
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16 || dtype == TSSM_F16, TSSM_ERR_DTYPE);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && Dc > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(N > 0 && N % 8 == 0 && N <= 128, TSSM_ERR_UNSUPPORTED);
  const int64_t cpr = sel_channels_per_row(Dc, N);
  const int64_t P = cpr * N;  // lanes per row
  TileCfg cfg;
  TSSM_CHECK(mh_tile_cfg(P, chunk, &cfg), TSSM_ERR_UNSUPPORTED);
  const int64_t need = tssm_selective_scan_workspace_bytes(nbatch, L, Dc, N, chunk);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 256), TSSM_ERR_ALIGN);
  const int64_t vec = dtype == TSSM_F32 ? 4 : 8;
  TSSM_CHECK(sB_b % vec == 0 && sB_l % vec == 0 && sC_b % vec == 0 && sC_l % vec == 0,
             TSSM_ERR_ALIGN);
  TSSM_CHECK(aligned(B, 16) && aligned(C, 16) && aligned(A_log, 16), TSSM_ERR_ALIGN);
  const int64_t strides[] = {sx_b, sx_l, sdt_b, sdt_l, sdt_d, sB_b, sB_l, sC_b, sC_l, sy_b, sy_l};
  for (int64_t s : strides) TSSM_CHECK(s >= 0, TSSM_ERR_STRIDE);
  if (proj.W) {
    TSSM_CHECK(proj.bias, TSSM_ERR_NULL);
    TSSM_CHECK(!dt_is_tau, TSSM_ERR_UNSUPPORTED);
    TSSM_CHECK(proj.rank > 0 && proj.rank <= kMaxDtRank, TSSM_ERR_UNSUPPORTED);
    TSSM_CHECK(proj.sw_r >= 0 && proj.dt_min <= proj.dt_max, TSSM_ERR_SHAPE);
  }
  // Large problems with 8 or 16 states take the three-pass scan (lanes =
  // channels, B/C staged in LDS): fp32 or bf16 I/O; dt given (timestamps
  // only when shared by the channels) or projected from raw rows of 16-byte
  // vectors (produced on the matrix cores in passes 1 and 3).
  {
    const int64_t rs = sel_chunk_steps(nbatch, L, Dc);
    const int64_t cb = sel_chunked_bytes(nbatch, L, Dc, N);
    const bool dt_shared = !proj.W && sdt_d == 0;
    const bool proj_ok = proj.W && sel_proj_ok(dt, proj.W, proj.bias, Dc, proj.rank, sdt_b,
                                               sdt_l, proj.sw_r);
    if (sel_takes_passes(dtype, nbatch, L, Dc, N, dt_shared, dt_is_tau != 0, proj.W != nullptr,
                         proj_ok)) {
      SelPtrs p;
      p.x = x; p.dt = dt; p.A_log = A_log; p.B = B; p.C = C; p.D = D; p.h0 = h0; p.y = y;
      p.h_last = h_last;
      p.W = proj.W; p.bias = proj.bias; p.sw_r = proj.sw_r; p.rank = proj.rank;
      p.dt_min = proj.dt_min; p.dt_max = proj.dt_max;
      const int64_t off = sel_chunked_offset(sel_lookback_bytes(nbatch, L, Dc, N, chunk));
      p.S = reinterpret_cast<float*>(static_cast<char*>(workspace) + off);
      p.T = p.S + nbatch * ((L + rs - 1) / rs) * Dc * N;
      if (proj.W) {
        // room for the produced-dt table: pass 1 stores it, pass 3 reads it
        const int64_t toff = sel_chunked_offset(off + cb);
        if (workspace_bytes >= toff + sel_dt_table_bytes(nbatch, L, Dc))
          p.dtw = reinterpret_cast<float*>(static_cast<char*>(workspace) + toff);
      }
      return sel_chunked_launch(dtype, disc, dt_shared, dt_is_tau != 0, p, nbatch, L, Dc, N,
                                sx_b, sx_l, sdt_b, sdt_l, sdt_d, sB_b, sB_l, sC_b, sC_l, sy_b,
                                sy_l, as_stream(stream));
    }
  }
  const int64_t nchunks = cdiv(L, cfg.TC);
  const int64_t nrows = nbatch * (Dc / cpr);
  TSSM_CHECK(nchunks * nrows < (int64_t)INT32_MAX, TSSM_ERR_UNSUPPORTED);
  const int nrun = cfg.W * (64 / cfg.G);
  size_t lds = ((size_t)2 * nrun * P + 2 * (nrun / 8) * P + 3 * P) * sizeof(float);
  if (proj.W) {
    const int64_t rp = (proj.rank + 3) & ~3ll;  // rank padded to whole float4s
    lds += (size_t)(cfg.TC * cpr + cfg.TC * (rp + 4) + rp * cpr) * sizeof(float);
    TSSM_CHECK(lds <= 64 * 1024, TSSM_ERR_UNSUPPORTED);
  }
  MhArgs a;
  a.u = x; a.A_log = A_log; a.B = B; a.C = C; a.dt = dt; a.D = D; a.h0 = h0; a.y = y;
  a.h_last = h_last;
  a.L = L;
  a.su_b = sx_b; a.su_l = sx_l;
  a.sB_b = sB_b; a.sB_l = sB_l; a.sB_h = 0;
  a.sC_b = sC_b; a.sC_l = sC_l; a.sC_h = 0;
  a.sdt_b = sdt_b; a.sdt_l = sdt_l; a.sdt_h = proj.W ? 0 : sdt_d;
  a.sy_b = sy_b; a.sy_l = sy_l;
  a.hdr = reinterpret_cast<WsHeader*>(workspace);
  a.words = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + sizeof(WsHeader));
  a.n_heads = (uint32_t)(Dc / cpr);
  a.nchunks = (uint32_t)nchunks;
  a.nrows = (uint32_t)nrows;
  a.tag = next_epoch(workspace);
  a.spin_limit = kDefaultSpinLimit;
  a.dt_is_tau = dt_is_tau ? 1u : 0u;
  a.off32 = tile_offsets_fit(cfg.TC, cpr, P, dtype == TSSM_F32 ? 4 : 2, sx_l, sB_l, sC_l, 0, 0,
                             sdt_l, proj.W ? 0 : sdt_d) ? 1u : 0u;
  a.dtW = proj.W; a.dtbias = proj.bias; a.sw_r = proj.sw_r; a.dt_rank = (uint32_t)proj.rank;
  a.dt_min = proj.dt_min; a.dt_max = proj.dt_max;
  const dim3 grid((unsigned)(nchunks * nrows)), block((unsigned)(cfg.W * 64));
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
  const int NS = (int)(N / 8);
  switch (dtype) {
    case TSSM_BF16: return launch_sel_t<bf16_t>(disc, has_d, cfg.G, NS, grid, block, lds, s, a);
    case TSSM_F16: return launch_sel_t<f16_t>(disc, has_d, cfg.G, NS, grid, block, lds, s, a);
    default: return launch_sel_t<float>(disc, has_d, cfg.G, NS, grid, block, lds, s, a);
  }
}

}  // namespace
}  // namespace tssm

extern "C" int tssm_selective_scan_takes_passes(int dtype, int64_t nbatch, int64_t L, int64_t Dc,
                                                int64_t N, int64_t sdt_d, int dt_is_tau,
                                                const float* dt_raw, const float* W,
                                                const float* bias, int64_t rank, int64_t sr_b,
                                                int64_t sr_l, int64_t sw_r) {
  const bool proj = W != nullptr;
  const bool proj_ok = proj && sel_proj_ok(dt_raw, W, bias, Dc, rank, sr_b, sr_l, sw_r);
  return sel_takes_passes(dtype, nbatch, L, Dc, N, !proj && sdt_d == 0, dt_is_tau != 0, proj,
                          proj_ok) ? 1 : 0;
}

extern "C" int tssm_selective_scan(int dtype, int disc, const void* x, const float* dt,
                                   int dt_is_tau, const float* A_log, const void* B,
                                   const void* C, const float* D, const float* h0, void* y,
                                   float* h_last, int64_t nbatch, int64_t L, int64_t Dc,
                                   int64_t N, int64_t sx_b, int64_t sx_l, int64_t sdt_b,
                                   int64_t sdt_l, int64_t sdt_d, int64_t sB_b, int64_t sB_l,
                                   int64_t sC_b, int64_t sC_l, int64_t sy_b, int64_t sy_l,
                                   int64_t chunk, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  return selective_scan_launch(dtype, disc, x, dt, dt_is_tau, DtProj{}, A_log, B, C, D, h0, y,
                               h_last, nbatch, L, Dc, N, sx_b, sx_l, sdt_b, sdt_l, sdt_d, sB_b,
                               sB_l, sC_b, sC_l, sy_b, sy_l, chunk, workspace, workspace_bytes,
                               stream);
}

extern "C" int tssm_selective_scan_dtproj(int dtype, int disc, const void* x,
                                          const float* dt_raw, const float* W, const float* bias,
                                          float dt_min, float dt_max, const float* A_log,
                                          const void* B, const void* C, const float* D,
                                          const float* h0, void* y, float* h_last,
                                          int64_t nbatch, int64_t L, int64_t Dc, int64_t N,
                                          int64_t rank, int64_t sx_b, int64_t sx_l, int64_t sr_b,
                                          int64_t sr_l, int64_t sw_r, int64_t sB_b, int64_t sB_l,
                                          int64_t sC_b, int64_t sC_l, int64_t sy_b, int64_t sy_l,
                                          int64_t chunk, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(W && bias, TSSM_ERR_NULL);
  DtProj proj;
  proj.W = W; proj.bias = bias; proj.sw_r = sw_r; proj.rank = rank;
  proj.dt_min = dt_min; proj.dt_max = dt_max;
  return selective_scan_launch(dtype, disc, x, dt_raw, 0, proj, A_log, B, C, D, h0, y, h_last,
                               nbatch, L, Dc, N, sx_b, sx_l, sr_b, sr_l, 0, sB_b, sB_l, sC_b,
                               sC_l, sy_b, sy_l, chunk, workspace, workspace_bytes, stream);
}
