// Mamba-1 selective scan in three passes over lanes = channels (N = 8 or 16
// states per lane, fp32 or bf16 I/O), the path tssm_selective_scan takes for
// large problems.  The recurrence is the one of discretize_kernel.py:16-57
// followed by ssm_scan.py:239-264 and a sum over n (y[b,t,d] = sum_n
// C[b,t,n] h[b,t,d,n] + D[d] x[b,t,d]), as in the single-pass kernel of
// multihead.hip; only the blocking differs.
//
//   pass 1 (sel_chunk_state_kernel): a workgroup takes 256 consecutive
//     channels of one batch over one chunk of Rs steps and runs the
//     recurrence from a zero state, each lane keeping the N states of its
//     channel in registers.  It stores y for that zero entry state, the
//     chunk's end state X[b,c,d,:] and the chunk's dt sum.
//   pass 2 (sel_carry_kernel): S_0 = h0, S_{c+1} = exp2(a log2e sum_c dt)
//     S_c + X_c per (b, d, n), overwriting X_c with the entry state S_c and
//     writing h_last = S_nch.  Four waves split a lane's chunks in quarters:
//     each folds its quarter from zero, the quarters' (decay, state) pairs
//     meet in LDS, and each wave walks its quarter again from its entry.
//   pass 3 (sel_output_kernel): adds the entry state's share of the output,
//     y[t] += sum_n C_t[n] exp2(a[n] log2e cum_t) S_c[n].
//
// B and C rows are the same for every channel of a batch, so a workgroup
// stages the chunk's rows (and a dt shared by the channels) in LDS once and
// every wave reads a step's row with broadcast LDS reads; x (y in pass 3,
// and a per-channel dt) is fetched four steps ahead into registers.  No pass
// has a look-back; passes 1 and 3 have one barrier each.  Vector
// instructions per step of 16 states: ~116.5 in pass 1 (6 per state update
// -- mul, exp2, add, mul, fma, fma -- and 1 per state of readout) and ~68.5
// in pass 3 (mul, exp2, mul, fma per state), against ~300 (19 per lane
// update) for the single-pass kernel with its run scan and second sweep.
#include <stdint.h>

#include "common.h"
#include "selective.h"
#include "selective_dev.h"

namespace tssm {

template <typename T, int DISC, int NST, bool DTS, bool TAU, bool HAS_D, bool DTP = false>
__global__ __launch_bounds__(kSelThreads) void sel_chunk_state_kernel(
    const T* __restrict__ x, const float* __restrict__ dt, const float* __restrict__ A_log,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ D,
    T* __restrict__ y, float* __restrict__ S, float* __restrict__ Tsum, SelDims m) {
  static_assert(!TAU || DTS, "timestamps only when shared by the channels");
  static_assert(!DTP || (!DTS && !TAU), "produced dt is per channel");
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int64_t d = (int64_t)blockIdx.y * kSelThreads + threadIdx.x;
  const bool ok = d < m.Dc;
  const int64_t dc = ok ? d : m.Dc - 1;  // lanes past Dc compute channel Dc-1
  const int64_t t0 = c * m.Rs;
  const int n = (int)(m.L - t0 < m.Rs ? m.L - t0 : m.Rs);
  const int n4 = (n + kSelPf - 1) / kSelPf * kSelPf;

  __shared__ float sB[kSelChunkSteps * NST], sC[kSelChunkSteps * NST];
  __shared__ float sD[DTS ? kSelChunkSteps : 1];
  __shared__ float sP[DTP ? kSelChunkSteps * kSelDtStride : 1];  // produced dt [step][column]
  // every prologue load first (rows to stage, lane parameters, the first x
  // fetches), then one wait: each load would otherwise be a round trip of its own
  const float* dtb = dt + b * m.sdt_b + (DTS || DTP ? 0 : dc * m.sdt_d);
  const float4 vB = stage_row_load<T, NST>(Bm + b * m.sB_b + t0 * m.sB_l, m.sB_l, n, n4);
  const float4 vC = stage_row_load<T, NST>(Cm + b * m.sC_b + t0 * m.sC_l, m.sC_l, n, n4);
  float vdt = 0.0f;
  if constexpr (DTS) vdt = stage_dt_load<TAU>(dt + b * m.sdt_b, m.sdt_l, t0, n);
  float al[NST];
  load_alog<NST>(A_log, dc, al);
  float Dd = HAS_D ? D[dc] : 0.0f;
  float u[kSelPf], dr[kSelPf];
  chunk_prefetch<T, DTS || DTP>(x + b * m.sx_b + dc, m.sx_l, dtb, m.sdt_l, t0, n, u, dr);
#pragma unroll
  for (int j = 0; j < kSelPf; ++j) asm volatile("" : "+v"(u[j]), "+v"(dr[j]));
  stage_row_store<NST>(sB, vB, n4);
  stage_row_store<NST>(sC, vC, n4);
  if constexpr (DTS) {
    if ((int)threadIdx.x < n4) sD[threadIdx.x] = vdt;
  }
  if constexpr (DTP)
    sel_proj_table(dtb, m.sdt_l, t0, n, m,
                   (int64_t)blockIdx.y * kSelThreads + (threadIdx.x & ~63u),
                   (int)(threadIdx.x & ~63u), sP);
  float a2[NST], nia[NST], h[NST];
  sel_params<NST>(al, a2, nia);
#pragma unroll
  for (int k = 0; k < NST; ++k) {
    h[k] = 0.0f;
    asm volatile("" : "+v"(a2[k]), "+v"(nia[k]));  // complete before the loop
  }
  asm volatile("" : "+v"(Dd));
  T* yp = y + b * m.sy_b + dc;
  __syncthreads();  // rows (and shared dt) staged
  // Waves whose lanes are all past Dc have staged their share and are done
  // (no barrier follows).
  if ((int64_t)blockIdx.y * kSelThreads + (threadIdx.x & ~63u) >= m.Dc) return;

  float sdt = 0.0f;
  // lanes past Dc read channel Dc-1's column: they store its outputs
  chunk_steps<T, DTS, DTP>(x + b * m.sx_b + dc, m.sx_l, dtb, m.sdt_l,
                           DTP ? sP + (dc - (int64_t)blockIdx.y * kSelThreads) : sD, t0, n, n4,
                           u, dr,
                      [&](int rr, float u, float dtv) {
                        float Bv[NST], Cv[NST];
                        lds_row<NST>(sB + rr * NST, Bv);
                        lds_row<NST>(sC + rr * NST, Cv);
                        sel_update<DISC, NST>(h, a2, nia, Bv, u, dtv);
                        sdt += dtv;
                        // output for a zero entry state, in two interleaved
                        // partial sums; pass 3 adds the entry state's part
                        float acc0 = HAS_D ? Dd * u : 0.0f, acc1 = 0.0f;
#pragma unroll
                        for (int k = 0; k < NST; k += 2) {
                          acc0 = __builtin_fmaf(Cv[k], h[k], acc0);
                          acc1 = __builtin_fmaf(Cv[k + 1], h[k + 1], acc1);
                        }
                        // Unconditional store: lanes past Dc (in the wave of
                        // channel Dc-1) computed channel Dc-1 and padded steps
                        // step n-1, identical values to what those write
                        // there, so no branch holds up the waits for later
                        // fetches.
                        const int64_t tw = t0 + (rr < n ? rr : n - 1);
                        stf(yp + tw * m.sy_l, acc0 + acc1);
                        if constexpr (DTP) {
                          // the table's row rr (a padded row repeats row n-1,
                          // whose value it then stores again), for pass 3
                          if (m.dtw)
                            m.dtw[(b * m.L + tw) * m.Dc + dc] =
                                sP[rr * kSelDtStride + (dc - (int64_t)blockIdx.y * kSelThreads)];
                        }
                      });
  if (ok) {
    float4* sp = reinterpret_cast<float4*>(S + ((b * m.nch + c) * m.Dc + d) * NST);
#pragma unroll
    for (int q = 0; q < NST / 4; ++q)
      sp[q] = make_float4(h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]);
    if constexpr (DTS) {
      if (d == 0) Tsum[b * m.nch + c] = sdt;
    } else {
      Tsum[(b * m.nch + c) * m.Dc + d] = sdt;
    }
  }
}

// Pass 2.  Workgroup = 64 consecutive (d, n) entries of one batch (blockIdx.y)
// x kSelCarryWaves waves; wave w takes chunks [w cpw, (w + 1) cpw) of the
// entries, cpw = ceil(nch / kSelCarryWaves).  Walk 1 folds the wave's chunks
// from zero into (decay product, state); after one barrier a wave's entry is
// h0 folded through the pairs of the waves before it, and walk 2 stores each
// chunk's entry state over its end state.  A quarter of up to kSelCarryBatch
// chunks stays in registers between the walks; longer quarters are loaded
// again (the chunks of one batch are all read before any is overwritten, and
// the waves' chunk ranges are disjoint).  Lanes past the row read its last
// entry and store nothing.  The last wave ends with h_last.
template <int NST, bool DTS>
__global__ __launch_bounds__(64 * kSelCarryWaves) void sel_carry_kernel(
    const float* __restrict__ A_log, const float* __restrict__ h0, float* __restrict__ S,
    const float* __restrict__ Tsum, float* __restrict__ h_last, SelDims m) {
  constexpr int kB = kSelCarryBatch;
  __shared__ float s_dec[kSelCarryWaves][64], s_agg[kSelCarryWaves][64];
  const int64_t b = blockIdx.y;
  const int64_t per_b = m.Dc * NST;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t rem0 = (int64_t)blockIdx.x * 64 + lane;
  const bool live = rem0 < per_b;
  const int64_t rem = live ? rem0 : per_b - 1;
  const int64_t d = rem / NST;
  const int64_t idx = b * per_b + rem;
  float* sp = S + b * m.nch * per_b + rem;
  const int64_t ts = DTS ? 1 : m.Dc;
  const float* tp = Tsum + b * m.nch * ts + (DTS ? 0 : d);
  const float a2 = -__builtin_amdgcn_exp2f(A_log[rem] * kLog2e) * kLog2e;
  const int64_t cpw = (m.nch + kSelCarryWaves - 1) / kSelCarryWaves;
  const int64_t cb = wv * cpw < m.nch ? wv * cpw : m.nch;
  const int64_t ce = cb + cpw < m.nch ? cb + cpw : m.nch;

  // chunk end states and per-chunk decays of chunks c0 .. c0 + kB - 1; slots
  // past the quarter get decay 1 and state 0 (they change nothing)
  float X[kB], E[kB];
#pragma unroll
  for (int i = 0; i < kB; ++i) X[i] = 0.0f, E[i] = 1.0f;
  auto load = [&](int64_t c0) {
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int64_t c = c0 + i < ce ? c0 + i : ce - 1;
      X[i] = sp[c * per_b];
      E[i] = tp[c * ts];
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const bool ok = c0 + i < ce;
      E[i] = ok ? __builtin_amdgcn_exp2f(a2 * E[i]) : 1.0f;
      X[i] = ok ? X[i] : 0.0f;
    }
  };

  // walk 1: the quarter from a zero state
  float agg = 0.0f, dec = 1.0f;
  for (int64_t c0 = cb; c0 < ce; c0 += kB) {
    load(c0);
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      agg = __builtin_fmaf(E[i], agg, X[i]);
      dec *= E[i];
    }
  }
  s_dec[wv][lane] = dec;
  s_agg[wv][lane] = agg;
  __syncthreads();
  float st = h0 ? h0[idx] : 0.0f;
  for (int v = 0; v < wv; ++v) st = __builtin_fmaf(s_dec[v][lane], st, s_agg[v][lane]);

  // walk 2: entry states from the quarter's entry
  auto walk = [&](int64_t c0) {
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      if (live && c0 + i < ce) sp[(c0 + i) * per_b] = st;
      st = __builtin_fmaf(E[i], st, X[i]);
    }
  };
  if (ce - cb <= kB) {
    walk(cb);
  } else {
    for (int64_t c0 = cb; c0 < ce; c0 += kB) {
      load(c0);
      walk(c0);
    }
  }
  if (wv == kSelCarryWaves - 1 && h_last && live) h_last[idx] = st;
}

// Pass 2 over segments, for long sequences with few lanes: one wave per
// (64 lanes, segment of kSelSegChunks chunks, batch).  FOLD: the segment's
// chunks from a zero state into Sg[b][seg][Dc N] and their dt sums into
// Tg[b][seg] (Tg[b][seg][Dc] for per-channel dt).  Then sel_carry_kernel runs
// over the segments (decay exp2(a log2e sum dt)) and leaves each segment's
// entry state in Sg; !FOLD walks the segment's chunks again from that entry
// and stores each chunk's entry state over its end state.
template <int NST, bool DTS, bool FOLD>
__global__ __launch_bounds__(256) void sel_carry_seg_kernel(
    const float* __restrict__ A_log, float* __restrict__ S, const float* __restrict__ Tsum,
    float* __restrict__ Sg, float* __restrict__ Tg, SelDims m, int64_t nseg) {
  constexpr int kB = kSelCarryBatch;
  const int64_t b = blockIdx.z;
  const int64_t per_b = m.Dc * NST;
  const int lane = threadIdx.x & 63;
  const int64_t sg = (int64_t)blockIdx.y * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (sg >= nseg) return;  // whole waves; no barrier in this kernel
  const int64_t rem0 = (int64_t)blockIdx.x * 64 + lane;
  const bool live = rem0 < per_b;
  const int64_t rem = live ? rem0 : per_b - 1;
  const int64_t d = rem / NST;
  float* sp = S + b * m.nch * per_b + rem;
  const int64_t ts = DTS ? 1 : m.Dc;
  const float* tp = Tsum + b * m.nch * ts + (DTS ? 0 : d);
  const float a2 = -__builtin_amdgcn_exp2f(A_log[rem] * kLog2e) * kLog2e;
  const int64_t cb = sg * kSelSegChunks;
  const int64_t ce = cb + kSelSegChunks < m.nch ? cb + kSelSegChunks : m.nch;
  float* gp = Sg + (b * nseg + sg) * per_b + rem;
  float st = FOLD ? 0.0f : *gp, tsum = 0.0f;
  for (int64_t c0 = cb; c0 < ce; c0 += kB) {
    float X[kB], Tv[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int64_t c = c0 + i < ce ? c0 + i : ce - 1;
      X[i] = sp[c * per_b];
      Tv[i] = tp[c * ts];
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const bool ok = c0 + i < ce;
      if (!FOLD && live && ok) sp[(c0 + i) * per_b] = st;
      const float e = ok ? __builtin_amdgcn_exp2f(a2 * Tv[i]) : 1.0f;
      st = __builtin_fmaf(e, st, ok ? X[i] : 0.0f);
      tsum += ok ? Tv[i] : 0.0f;
    }
  }
  if (FOLD) {
    if (live) *gp = st;
    const bool writer = DTS ? (blockIdx.x == 0 && lane == 0) : (live && rem % NST == 0);
    if (writer) Tg[(b * nseg + sg) * ts + (DTS ? 0 : d)] = tsum;
  }
}

// Host side of pass 2.  Enough lanes: sel_carry_kernel on the chunks, grid
// (ceil(Dc N / 64), batches) of kSelCarryWaves waves.  Few lanes and at least
// four segments of chunks: fold the segments, carry over them, walk them
// again (three launches, each with a wave per segment and 64 lanes).
template <int NST, bool DTS>
int launch_sel_carry(hipStream_t s, const SelPtrs& p, const SelDims& m) {
  const int64_t lanes = m.Dc * NST;  // per batch
  const int64_t groups = (lanes + 63) / 64;
  const int64_t nseg = (m.nch + kSelSegChunks - 1) / kSelSegChunks;
  if (m.nbatch * groups >= 512 || nseg < 4 || (nseg + 3) / 4 > 65535) {
    hipLaunchKernelGGL((sel_carry_kernel<NST, DTS>), dim3((unsigned)groups, (unsigned)m.nbatch),
                       dim3(64 * kSelCarryWaves), 0, s, p.A_log, p.h0, p.S, p.T, p.h_last, m);
    return (int)hipGetLastError();
  }
  float* Sg = p.T + m.nbatch * m.nch * m.Dc;
  float* Tg = Sg + m.nbatch * nseg * lanes;
  const dim3 grid((unsigned)groups, (unsigned)((nseg + 3) / 4), (unsigned)m.nbatch);
  hipLaunchKernelGGL((sel_carry_seg_kernel<NST, DTS, true>), grid, dim3(256), 0, s, p.A_log, p.S,
                     p.T, Sg, Tg, m, nseg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  SelDims mg = m;
  mg.nch = nseg;
  hipLaunchKernelGGL((sel_carry_kernel<NST, DTS>), dim3((unsigned)groups, (unsigned)m.nbatch),
                     dim3(64 * kSelCarryWaves), 0, s, p.A_log, p.h0, Sg, Tg, p.h_last, mg);
  e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((sel_carry_seg_kernel<NST, DTS, false>), grid, dim3(256), 0, s, p.A_log,
                     p.S, p.T, Sg, Tg, m, nseg);
  return (int)hipGetLastError();
}

// Pass 3: y[t] += sum_n C_t[n] 2^(a[n] log2e cum_t) S_c[n], the part of the
// output carried in by the chunk's entry state (cum_t: dt summed over the
// chunk up to and including t); pass 1 stored the rest.  The decay factor is
// the product of the per-step factors of the recurrence written as one
// exponential; it does not depend on the discretization.  y is read (four
// steps ahead) and written in place, so it is not declared restrict.
template <typename T, int NST, bool DTS, bool TAU, bool DTP = false>
__global__ __launch_bounds__(kSelThreads) void sel_output_kernel(
    const float* __restrict__ dt, const float* __restrict__ A_log, const T* __restrict__ Cm,
    const float* __restrict__ S, T* y, SelDims m) {
  static_assert(!TAU || DTS, "timestamps only when shared by the channels");
  static_assert(!DTP || (!DTS && !TAU), "produced dt is per channel");
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int64_t d = (int64_t)blockIdx.y * kSelThreads + threadIdx.x;
  const int64_t dc = d < m.Dc ? d : m.Dc - 1;
  const int64_t t0 = c * m.Rs;
  const int n = (int)(m.L - t0 < m.Rs ? m.L - t0 : m.Rs);
  const int n4 = (n + kSelPf - 1) / kSelPf * kSelPf;

  __shared__ float sC[kSelChunkSteps * NST];
  __shared__ float sD[DTS ? kSelChunkSteps : 1];
  __shared__ float sP[DTP ? kSelChunkSteps * kSelDtStride : 1];  // produced dt [step][column]
  // every prologue load first, then one wait (as in pass 1)
  const float* dtb = dt + b * m.sdt_b + (DTS || DTP ? 0 : dc * m.sdt_d);
  T* yp = y + b * m.sy_b + dc;
  const float4 vC = stage_row_load<T, NST>(Cm + b * m.sC_b + t0 * m.sC_l, m.sC_l, n, n4);
  float vdt = 0.0f;
  if constexpr (DTS) vdt = stage_dt_load<TAU>(dt + b * m.sdt_b, m.sdt_l, t0, n);
  float al[NST], h[NST];
  load_alog<NST>(A_log, dc, al);
  {
    const float4* sp = reinterpret_cast<const float4*>(S + ((b * m.nch + c) * m.Dc + dc) * NST);
#pragma unroll
    for (int q = 0; q < NST / 4; ++q) {
      const float4 v = sp[q];
      h[4 * q] = v.x; h[4 * q + 1] = v.y; h[4 * q + 2] = v.z; h[4 * q + 3] = v.w;
    }
  }
  float u[kSelPf], dr[kSelPf];
  chunk_prefetch<T, DTS || DTP>(yp, m.sy_l, dtb, m.sdt_l, t0, n, u, dr);
#pragma unroll
  for (int j = 0; j < kSelPf; ++j) asm volatile("" : "+v"(u[j]), "+v"(dr[j]));
  stage_row_store<NST>(sC, vC, n4);
  if constexpr (DTS) {
    if ((int)threadIdx.x < n4) sD[threadIdx.x] = vdt;
  }
  if constexpr (DTP)
    sel_proj_table(dtb, m.sdt_l, t0, n, m,
                   (int64_t)blockIdx.y * kSelThreads + (threadIdx.x & ~63u),
                   (int)(threadIdx.x & ~63u), sP);
  float a2[NST], nia[NST];
  sel_params<NST>(al, a2, nia);
#pragma unroll
  for (int k = 0; k < NST; ++k) asm volatile("" : "+v"(h[k]), "+v"(a2[k]));  // before the loop
  __syncthreads();  // rows (and shared dt) staged
  // y is updated in place (y += carried share), which is not idempotent: a
  // wave whose lanes are all past Dc would read y[., Dc-1] at a time of its
  // own and could add the carried share a second time.  Such waves have
  // staged their share and leave here (no barrier follows).  Lanes past Dc
  // in the wave of channel Dc-1 load and store in lockstep with that lane,
  // so they write exactly its values.
  if ((int64_t)blockIdx.y * kSelThreads + (threadIdx.x & ~63u) >= m.Dc) return;

  float cum = 0.0f;
  // lanes past Dc read channel Dc-1's column: they store its outputs
  chunk_steps<T, DTS, DTP>(yp, m.sy_l, dtb, m.sdt_l,
                           DTP ? sP + (dc - (int64_t)blockIdx.y * kSelThreads) : sD, t0, n, n4,
                           u, dr,
                      [&](int rr, float y1, float dtv) {
                        float Cv[NST];
                        lds_row<NST>(sC + rr * NST, Cv);
                        cum += dtv;
                        float acc0 = y1, acc1 = 0.0f;
#pragma unroll
                        for (int k = 0; k < NST; k += 2) {
                          acc0 = __builtin_fmaf(Cv[k] * h[k],
                                                __builtin_amdgcn_exp2f(a2[k] * cum), acc0);
                          acc1 = __builtin_fmaf(Cv[k + 1] * h[k + 1],
                                                __builtin_amdgcn_exp2f(a2[k + 1] * cum), acc1);
                        }
                        // Unconditional: the lanes past Dc that get here
                        // share the wave of channel Dc-1 and store its value.
                        const int64_t tw = t0 + (rr < n ? rr : n - 1);
                        stf(yp + tw * m.sy_l, acc0 + acc1);
                      });
}

// ---------------------------------------------------------------- x -> (B, C) in pass 1
// The selective input projection producing B and C from x (B_t = x_t W_B,
// C_t = x_t W_C: Mamba-1's x_proj columns for B and C) formed inside pass 1,
// so B and C [B, L, N] are never read from a caller's tensor and no
// projection launch runs.  fp32 I/O, Dc <= 256 (one workgroup holds every
// channel of a step).  A workgroup stages its chunk's x tile [32][Dc] in LDS
// (every step's row, padded steps repeating step n-1), wave w forms the
// 16 x 16 output tile (steps 16 (w & 1).., columns 16 (w >> 1)..) of
// [32][2N] = x W_BC on the fp32 matrix cores (16x16x4, the channels in steps
// of 4), the rows are staged as pass 1's B/C rows, C's rows are also stored
// for pass 3, and the recurrence reads x from the LDS tile instead of HBM.
//
// XR > 0 (the whole input projection, x -> (dt, B, C), Mamba-1's x_proj and
// dt_proj): W_bc's first XR columns give the rank-XR rows dt_raw_t = x_t W_x,
// staged in LDS; each wave then forms dt = clamp(softplus(dt_raw W_dt +
// bias)) for its 64 channels on the matrix cores, in the operand order of
// dt_project_mfma_kernel (so the dt it stores is what that kernel stores for
// the same dt_raw), into the dt table that pass 3 reads; after a workgroup
// fence the recurrence reads it back per channel (L2-resident) as a
// per-channel dt.
constexpr int kBcRow = kSelThreads + 4;  // x tile row stride (floats): 16-byte rows, banks spread
constexpr int kBcKb = 16;                // W values per lane in flight in the B/C product

template <int DISC, int NST, bool DTS, bool TAU, bool HAS_D, int XR>
__device__ __forceinline__ void sel_bcproj_state_body(
    const float* __restrict__ x, const float* __restrict__ dt, const float* __restrict__ A_log,
    const float* __restrict__ Wbc, int64_t sw_d, const float* __restrict__ D,
    float* __restrict__ y, float* __restrict__ S, float* __restrict__ Tsum,
    float* __restrict__ Cws, SelDims m) {
  static_assert(!TAU || DTS, "timestamps only when shared by the channels");
  static_assert(NST == 8 || NST == 16, "8 or 16 states");
  static_assert(XR == 0 || (!DTS && XR % 16 == 0 && XR <= kSelMaxRank), "dt produced per channel");
  constexpr int kXrRow = XR + 4;  // dt_raw row stride in LDS (floats)
  const int64_t c = blockIdx.x, b = blockIdx.z;  // one channel block (blockIdx.y == 0)
  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t d = tid;
  const bool ok = d < m.Dc;
  const int64_t dc = ok ? d : m.Dc - 1;  // lanes past Dc compute channel Dc-1
  const int64_t t0 = c * m.Rs;
  const int n = (int)(m.L - t0 < m.Rs ? m.L - t0 : m.Rs);
  const int n4 = (n + kSelPf - 1) / kSelPf * kSelPf;

  __shared__ __align__(16) float sX[kSelChunkSteps * kBcRow];
  __shared__ float sB[kSelChunkSteps * NST], sC[kSelChunkSteps * NST];
  __shared__ float sD[DTS ? kSelChunkSteps : 1];
  __shared__ __align__(16) float sR[XR ? kSelChunkSteps * kXrRow : 1];  // dt_raw rows
  // ---- prologue loads: the x tile (thread: columns 4 (tid & 63).. of rows
  // (tid >> 6) + 4 k; columns past Dc read as zero), shared dt, lane
  // parameters, a per-channel dt's first fetches; then one wait
  const float* xb = x + b * m.sx_b;
  const int col = 4 * lane;
  const bool cok = col < m.Dc;  // Dc a multiple of 4
  float4 xv[kSelChunkSteps / 4];
#pragma unroll
  for (int k = 0; k < kSelChunkSteps / 4; ++k) {
    const int r = wv + 4 * k;
    const int rr = r < n ? r : n - 1;
    const float4 v = *reinterpret_cast<const float4*>(xb + (t0 + rr) * m.sx_l + (cok ? col : 0));
    xv[k] = cok ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float vdt = 0.0f;
  if constexpr (DTS) vdt = stage_dt_load<TAU>(dt + b * m.sdt_b, m.sdt_l, t0, n);
  // XR: dt is the table this pass writes below (m.dtw, [nbatch][L][Dc])
  const float* dtb = XR ? m.dtw + (b * m.L) * m.Dc + dc : dt + b * m.sdt_b + (DTS ? 0 : dc * m.sdt_d);
  const int64_t sdt_l = XR ? m.Dc : m.sdt_l;
  float dr[kSelPf];
#pragma unroll
  for (int j = 0; j < kSelPf; ++j)
    dr[j] = (DTS || XR) ? 0.0f : dtb[(t0 + (j < n ? j : n - 1)) * sdt_l];
  float al[NST];
  load_alog<NST>(A_log, dc, al);
  float Dd = HAS_D ? D[dc] : 0.0f;
  // XR: the recurrence reads x from memory (the tile's LDS becomes the dt
  // table); its first steps load with the prologue
  float u[kSelPf];
  if constexpr (XR > 0) {
    chunk_prefetch<float, true>(xb + dc, m.sx_l, nullptr, 0, t0, n, u, dr);
#pragma unroll
    for (int j = 0; j < kSelPf; ++j) asm volatile("" : "+v"(u[j]));
  }
#pragma unroll
  for (int k = 0; k < kSelChunkSteps / 4; ++k)
    *reinterpret_cast<float4*>(sX + (wv + 4 * k) * kBcRow + col) = xv[k];
  if constexpr (DTS) {
    if (tid < n4) sD[tid] = vdt;
  }
  __syncthreads();  // x tile staged

  // ---- (dt_raw,) B and C rows of the chunk on the matrix cores: (XR + 2N) / 16
  // column tiles x 2 step tiles, tile tt = rt + 2 ct taken by wave tt mod 4
  constexpr int kNt = 2 * ((XR + 2 * NST) / 16);
  for (int tt = wv; tt < kNt; tt += kSelWaves) {
    const int rt = tt & 1, ct = tt >> 1;
    const int li = lane & 15, lj = lane >> 4;
    f32x4 acc0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    const float* xa = sX + (16 * rt + li) * kBcRow + lj;
    const float* wb = Wbc + (int64_t)lj * sw_d + 16 * ct + li;
    // W values (k-step j: W[4 j + lj][16 ct + li]) in blocks of kBcKb, the
    // next block's loads in flight while the current block's products run
    // (each product would otherwise wait on its own L2 round trip)
    const int nk = (int)(m.Dc / 4);  // k-steps of 4 channels
    float wcur[kBcKb], wnxt[kBcKb];
    auto load_w = [&](int kb, float (&w)[kBcKb]) {
#pragma unroll
      for (int j = 0; j < kBcKb; ++j) {
        const int kk = kb + j < nk ? kb + j : nk - 1;  // past the last k-step: any row, unused
        w[j] = wb[(int64_t)(4 * kk) * sw_d];
      }
    };
    load_w(0, wcur);
    for (int kb = 0; kb < nk; kb += kBcKb) {
      if (kb + kBcKb < nk) load_w(kb + kBcKb, wnxt);
#pragma unroll
      for (int j = 0; j < kBcKb; j += 2) {
        if (kb + j < nk)
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[4 * (kb + j)], wcur[j], acc0, 0, 0, 0);
        if (kb + j + 1 < nk)
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[4 * (kb + j + 1)], wcur[j + 1], acc1, 0,
                                                      0, 0);
      }
#pragma unroll
      for (int j = 0; j < kBcKb; ++j) wcur[j] = wnxt[j];
    }
    // lane (li, lj): steps 16 rt + 4 lj + i, column 16 ct + li of [dt_raw | B | C]
    const int cc = 16 * ct + li - XR;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rt + 4 * lj + i;
      const float v = acc0[i] + acc1[i];
      if (XR && cc < 0) {
        sR[r * kXrRow + cc + XR] = v;
      } else if (cc < NST) {
        sB[r * NST + cc] = v;
      } else {
        sC[r * NST + cc - NST] = v;
        if (r < n) Cws[(b * m.L + t0 + r) * NST + cc - NST] = v;  // for pass 3
      }
    }
  }
  if constexpr (XR > 0) {
    __syncthreads();  // dt_raw rows staged; every wave is done with the x tile
    // ---- dt of the wave's 64 channels for the chunk's steps: into the table
    // (in the x tile's LDS, row stride kSelDtStride) for the recurrence, and
    // into m.dtw for pass 3
    float* sP = sX;
    const int dw0 = 64 * wv;
    if (dw0 < m.Dc) {
      const int li = lane & 15, lj = lane >> 4;
      f32x4 acc[2][4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int h = dw0 + 16 * ct + 4 * lj;  // 4 channels, all in range or all out
        const float4 bq = *reinterpret_cast<const float4*>(m.bias + (h < m.Dc ? h : 0));
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) acc[rt][ct] = f32x4{bq.x, bq.y, bq.z, bq.w};
      }
#pragma unroll
      for (int q0 = 0; q0 < XR; q0 += 16) {
        const int qa = q0 + 4 * lj;
        float wa[4][4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const int h = dw0 + 16 * ct + li;
          const float* wp = m.W + (h < m.Dc ? h : m.Dc - 1);
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) wa[ct][s2] = wp[(int64_t)(qa + s2) * m.sw_r];
        }
        f32x4 rv[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          rv[rt] = *reinterpret_cast<const f32x4*>(sR + (16 * rt + li) * kXrRow + qa);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
              acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[ct][s2], rv[rt][s2],
                                                                  acc[rt][ct], 0, 0, 0);
      }
      // lane (li, lj): step 16 rt + li, channels 16 ct + 4 lj .. + 3
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int r = 16 * rt + li;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const int h = dw0 + 16 * ct + 4 * lj;
          float4 v;
          v.x = clamp_med3(softplus_fast(acc[rt][ct][0]), m.dt_min, m.dt_max);
          v.y = clamp_med3(softplus_fast(acc[rt][ct][1]), m.dt_min, m.dt_max);
          v.z = clamp_med3(softplus_fast(acc[rt][ct][2]), m.dt_min, m.dt_max);
          v.w = clamp_med3(softplus_fast(acc[rt][ct][3]), m.dt_min, m.dt_max);
          *reinterpret_cast<float4*>(sP + r * kSelDtStride + h) = v;
          if (r < n && h < m.Dc)
            *reinterpret_cast<float4*>(m.dtw + (b * m.L + t0 + r) * m.Dc + h) = v;
        }
      }
    }
  }
  float a2[NST], nia[NST], h[NST];
  sel_params<NST>(al, a2, nia);
#pragma unroll
  for (int k = 0; k < NST; ++k) {
    h[k] = 0.0f;
    asm volatile("" : "+v"(a2[k]), "+v"(nia[k]));  // complete before the loop
  }
  asm volatile("" : "+v"(Dd));
  __syncthreads();  // B/C rows (and the dt table) staged
  // Waves whose lanes are all past Dc are done (no barrier follows).
  if ((tid & ~63) >= m.Dc) return;

  float* yp = y + b * m.sy_b + dc;
  float sdt = 0.0f;
  if constexpr (XR > 0) {
    // x from memory (fetched kSelPf steps ahead), dt from the lane's column
    // of the table, B/C rows from LDS
    chunk_steps<float, false, true>(xb + dc, m.sx_l, nullptr, 0, sX + dc, t0, n, n4, u, dr,
                                    [&](int rr, float uv, float dtv) {
                                      float Bv[NST], Cv[NST];
                                      lds_row<NST>(sB + rr * NST, Bv);
                                      lds_row<NST>(sC + rr * NST, Cv);
                                      sel_update<DISC, NST>(h, a2, nia, Bv, uv, dtv);
                                      sdt += dtv;
                                      float acc0 = HAS_D ? Dd * uv : 0.0f, acc1 = 0.0f;
#pragma unroll
                                      for (int kk = 0; kk < NST; kk += 2) {
                                        acc0 = __builtin_fmaf(Cv[kk], h[kk], acc0);
                                        acc1 = __builtin_fmaf(Cv[kk + 1], h[kk + 1], acc1);
                                      }
                                      // unconditional (as below)
                                      const int64_t tw = t0 + (rr < n ? rr : n - 1);
                                      yp[tw * m.sy_l] = acc0 + acc1;
                                    });
  } else {
    const float* xcol = sX + dc;
    for (int r = 0; r < n4; r += kSelPf) {
#pragma unroll
      for (int j = 0; j < kSelPf; ++j) {
        const int rr = r + j;
        const float u = xcol[rr * kBcRow];
        const float dtv = DTS ? sD[rr] : (rr < n ? dr[j] : 0.0f);
        float Bv[NST], Cv[NST];
        lds_row<NST>(sB + rr * NST, Bv);
        lds_row<NST>(sC + rr * NST, Cv);
        sel_update<DISC, NST>(h, a2, nia, Bv, u, dtv);
        sdt += dtv;
        float acc0 = HAS_D ? Dd * u : 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int k = 0; k < NST; k += 2) {
          acc0 = __builtin_fmaf(Cv[k], h[k], acc0);
          acc1 = __builtin_fmaf(Cv[k + 1], h[k + 1], acc1);
        }
        // unconditional store: lanes past Dc (in the wave of channel Dc-1) and
        // padded steps store the values of channel Dc-1 / step n-1
        const int64_t tw = t0 + (rr < n ? rr : n - 1);
        yp[tw * m.sy_l] = acc0 + acc1;
        if constexpr (!DTS) {
          __builtin_amdgcn_sched_barrier(0);
          dr[j] = dtb[(t0 + min(rr + kSelPf, n - 1)) * sdt_l];
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  if (ok) {
    float4* sp = reinterpret_cast<float4*>(S + ((b * m.nch + c) * m.Dc + d) * NST);
#pragma unroll
    for (int q = 0; q < NST / 4; ++q)
      sp[q] = make_float4(h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]);
    if constexpr (DTS) {
      if (d == 0) Tsum[b * m.nch + c] = sdt;
    } else {
      Tsum[(b * m.nch + c) * m.Dc + d] = sdt;
    }
  }
}

template <int DISC, int NST, bool DTS, bool TAU, bool HAS_D>
__global__ __launch_bounds__(kSelThreads) void sel_bcproj_state_kernel(
    const float* __restrict__ x, const float* __restrict__ dt, const float* __restrict__ A_log,
    const float* __restrict__ Wbc, int64_t sw_d, const float* __restrict__ D,
    float* __restrict__ y, float* __restrict__ S, float* __restrict__ Tsum,
    float* __restrict__ Cws, SelDims m) {
  sel_bcproj_state_body<DISC, NST, DTS, TAU, HAS_D, 0>(x, dt, A_log, Wbc, sw_d, D, y, S, Tsum,
                                                      Cws, m);
}

// The XR > 0 instances, held to 4 waves per SIMD up to rank 16 (left alone
// the compiler gives them 144 registers, 3 waves per SIMD, and the pass runs
// ~9% slower); rank 32 does not fit 4 and is held to 3.
template <int DISC, int NST, bool HAS_D, int XR>
__global__ __launch_bounds__(kSelThreads) __attribute__((amdgpu_waves_per_eu(XR <= 16 ? 4 : 3))) void
sel_xproj_state_kernel(const float* __restrict__ x, const float* __restrict__ A_log,
                       const float* __restrict__ Wx, int64_t swx_d, const float* __restrict__ D,
                       float* __restrict__ y, float* __restrict__ S, float* __restrict__ Tsum,
                       float* __restrict__ Cws, SelDims m) {
  sel_bcproj_state_body<DISC, NST, false, false, HAS_D, XR>(x, nullptr, A_log, Wx, swx_d, D, y,
                                                            S, Tsum, Cws, m);
}

// ---------------------------------------------------------------- host
namespace {

template <typename T, int DISC, int NST, bool DTS, bool TAU, bool DTP = false>
int sel_chunked_t(bool has_d, const SelPtrs& p, const SelDims& m, hipStream_t s) {
  const dim3 grid((unsigned)m.nch, (unsigned)((m.Dc + kSelThreads - 1) / kSelThreads),
                  (unsigned)m.nbatch);
  const T* x = static_cast<const T*>(p.x);
  const T* Bm = static_cast<const T*>(p.B);
  const T* Cm = static_cast<const T*>(p.C);
  T* y = static_cast<T*>(p.y);
  if (has_d)
    hipLaunchKernelGGL((sel_chunk_state_kernel<T, DISC, NST, DTS, TAU, true, DTP>), grid,
                       dim3(kSelThreads), 0, s, x, p.dt, p.A_log, Bm, Cm, p.D, y, p.S, p.T, m);
  else
    hipLaunchKernelGGL((sel_chunk_state_kernel<T, DISC, NST, DTS, TAU, false, DTP>), grid,
                       dim3(kSelThreads), 0, s, x, p.dt, p.A_log, Bm, Cm, p.D, y, p.S, p.T, m);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int rc = launch_sel_carry<NST, DTS>(s, p, m);
  if (rc != 0) return rc;
  if (DTP && p.dtw) {
    // pass 3 reads the dt table pass 1 stored: the per-channel dt instance
    SelDims m3 = m;
    m3.sdt_b = m.L * m.Dc; m3.sdt_l = m.Dc; m3.sdt_d = 1;
    hipLaunchKernelGGL((sel_output_kernel<T, NST, false, false, false>), grid, dim3(kSelThreads),
                       0, s, p.dtw, p.A_log, Cm, p.S, y, m3);
  } else {
    hipLaunchKernelGGL((sel_output_kernel<T, NST, DTS, TAU, DTP>), grid, dim3(kSelThreads), 0, s,
                       p.dt, p.A_log, Cm, p.S, y, m);
  }
  return (int)hipGetLastError();
}

template <typename T, int DISC, int NST>
int sel_chunked_dt(bool has_d, bool dts, bool tau, const SelPtrs& p, const SelDims& m,
                   hipStream_t s) {
  if (p.W) return sel_chunked_t<T, DISC, NST, false, false, true>(has_d, p, m, s);
  if (dts) {
    return tau ? sel_chunked_t<T, DISC, NST, true, true>(has_d, p, m, s)
               : sel_chunked_t<T, DISC, NST, true, false>(has_d, p, m, s);
  }
  return sel_chunked_t<T, DISC, NST, false, false>(has_d, p, m, s);  // per-channel dt, no tau
}

template <typename T, int DISC>
int sel_chunked_n(int64_t N, bool has_d, bool dts, bool tau, const SelPtrs& p, const SelDims& m,
                  hipStream_t s) {
  return N == 16 ? sel_chunked_dt<T, DISC, 16>(has_d, dts, tau, p, m, s)
                 : sel_chunked_dt<T, DISC, 8>(has_d, dts, tau, p, m, s);
}

template <typename T, int DISC, int NST>
int sel_interp_t(bool has_d, const void* V, const float* M, const float* tau, void* Vhat,
                 const SelPtrs& p, const SelDims& m, const SiDims& q, hipStream_t s) {
  const dim3 grid((unsigned)m.nch, (unsigned)((m.Dc + kSelThreads - 1) / kSelThreads),
                  (unsigned)m.nbatch);
  const T* Cm = static_cast<const T*>(p.C);
  T* y = static_cast<T*>(p.y);
  const int e = sel_interp_pass1(sizeof(T) == 2, DISC, NST, has_d, V, M, tau, Vhat, p, m, q, s);
  if (e != hipSuccess) return e;
  const int rc = launch_sel_carry<NST, true>(s, p, m);
  if (rc != 0) return rc;
  hipLaunchKernelGGL((sel_output_kernel<T, NST, true, true>), grid, dim3(kSelThreads), 0, s, tau,
                     p.A_log, Cm, p.S, y, m);
  return (int)hipGetLastError();
}

template <typename T, int DISC>
int sel_interp_n(int64_t N, bool has_d, const void* V, const float* M, const float* tau,
                 void* Vhat, const SelPtrs& p, const SelDims& m, const SiDims& q, hipStream_t s) {
  return N == 16 ? sel_interp_t<T, DISC, 16>(has_d, V, M, tau, Vhat, p, m, q, s)
                 : sel_interp_t<T, DISC, 8>(has_d, V, M, tau, Vhat, p, m, q, s);
}

int ilog2(int64_t v) {
  int l = 0;
  while ((int64_t)1 << (l + 1) <= v) ++l;
  return l;
}

}  // namespace

template <int DISC, int NST, bool DTS, bool TAU>
int sel_bcproj_t(bool has_d, const float* x, const float* dt, const float* Wbc, int64_t sw_d,
                 float* Cws, const SelPtrs& p, const SelDims& m, hipStream_t s) {
  const dim3 grid((unsigned)m.nch, 1u, (unsigned)m.nbatch);
  float* y = static_cast<float*>(p.y);
  if (has_d)
    hipLaunchKernelGGL((sel_bcproj_state_kernel<DISC, NST, DTS, TAU, true>), grid,
                       dim3(kSelThreads), 0, s, x, dt, p.A_log, Wbc, sw_d, p.D, y, p.S, p.T, Cws,
                       m);
  else
    hipLaunchKernelGGL((sel_bcproj_state_kernel<DISC, NST, DTS, TAU, false>), grid,
                       dim3(kSelThreads), 0, s, x, dt, p.A_log, Wbc, sw_d, p.D, y, p.S, p.T, Cws,
                       m);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int rc = launch_sel_carry<NST, DTS>(s, p, m);
  if (rc != 0) return rc;
  // pass 3 reads the C rows pass 1 stored
  SelDims m3 = m;
  m3.sC_b = m.L * NST; m3.sC_l = NST;
  hipLaunchKernelGGL((sel_output_kernel<float, NST, DTS, TAU>), grid, dim3(kSelThreads), 0, s,
                     dt, p.A_log, Cws, p.S, y, m3);
  return (int)hipGetLastError();
}

// The whole input projection in the pass: dt from the dt_raw columns of W_x
// (into the dt table p.dtw), B and C from the next 2N columns.
template <int DISC, int NST, int XR>
int sel_xproj_t(bool has_d, const float* x, const float* Wx, int64_t swx_d, float* Cws,
                const SelPtrs& p, const SelDims& m, hipStream_t s) {
  const dim3 grid((unsigned)m.nch, 1u, (unsigned)m.nbatch);
  float* y = static_cast<float*>(p.y);
  if (has_d)
    hipLaunchKernelGGL((sel_xproj_state_kernel<DISC, NST, true, XR>), grid, dim3(kSelThreads), 0,
                       s, x, p.A_log, Wx, swx_d, p.D, y, p.S, p.T, Cws, m);
  else
    hipLaunchKernelGGL((sel_xproj_state_kernel<DISC, NST, false, XR>), grid, dim3(kSelThreads),
                       0, s, x, p.A_log, Wx, swx_d, p.D, y, p.S, p.T, Cws, m);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int rc = launch_sel_carry<NST, false>(s, p, m);
  if (rc != 0) return rc;
  // pass 3 reads the dt table and the C rows pass 1 stored
  SelDims m3 = m;
  m3.sdt_b = m.L * m.Dc; m3.sdt_l = m.Dc; m3.sdt_d = 1;
  m3.sC_b = m.L * NST; m3.sC_l = NST;
  hipLaunchKernelGGL((sel_output_kernel<float, NST, false, false>), grid, dim3(kSelThreads), 0,
                     s, m.dtw, p.A_log, Cws, p.S, y, m3);
  return (int)hipGetLastError();
}

template <int DISC, int NST>
int sel_xproj_r(int64_t R, bool has_d, const float* x, const float* Wx, int64_t swx_d, float* Cws,
                const SelPtrs& p, const SelDims& m, hipStream_t s) {
  switch (R) {
    case 16: return sel_xproj_t<DISC, NST, 16>(has_d, x, Wx, swx_d, Cws, p, m, s);
    case 32: return sel_xproj_t<DISC, NST, 32>(has_d, x, Wx, swx_d, Cws, p, m, s);
    case 48: return sel_xproj_t<DISC, NST, 48>(has_d, x, Wx, swx_d, Cws, p, m, s);
    default: return sel_xproj_t<DISC, NST, 64>(has_d, x, Wx, swx_d, Cws, p, m, s);
  }
}

template <int DISC, int NST>
int sel_bcproj_dt(bool has_d, bool dts, bool tau, const float* x, const float* dt,
                  const float* Wbc, int64_t sw_d, float* Cws, const SelPtrs& p, const SelDims& m,
                  hipStream_t s) {
  if (dts) {
    return tau ? sel_bcproj_t<DISC, NST, true, true>(has_d, x, dt, Wbc, sw_d, Cws, p, m, s)
               : sel_bcproj_t<DISC, NST, true, false>(has_d, x, dt, Wbc, sw_d, Cws, p, m, s);
  }
  return sel_bcproj_t<DISC, NST, false, false>(has_d, x, dt, Wbc, sw_d, Cws, p, m, s);
}

bool sel_interp_ok(int dtype, int64_t nbatch, int64_t T, int64_t F, int64_t N, int64_t K,
                   int64_t FTILE, const void* M, int64_t sm_b, int64_t sm_t, int64_t sv_t) {
  const bool pow2 = FTILE > 0 && (FTILE & (FTILE - 1)) == 0;
  const int64_t rs = sel_chunk_steps(nbatch, T, F);
  return (dtype == TSSM_F32 || dtype == TSSM_BF16) && (N == 8 || N == 16) && rs > 0 &&
         pow2 && FTILE >= 16 && FTILE <= kSelThreads && K >= 1 && K <= kSiMaxK && F > 0 &&
         sv_t >= 0 && (kSelChunkSteps + 2 * K) * sv_t * (dtype == TSSM_F32 ? 4 : 2) < INT32_MAX &&
         F % 4 == 0 && sm_b % 4 == 0 && sm_t % 4 == 0 && sm_b >= 0 && sm_t >= 0 &&
         aligned(M, 16) && nbatch > 0 && nbatch <= 65535 &&
         nbatch * ((F + 63) / 64) * ((T + rs - 1) / rs) >= kSelMinWaves;
}

int sel_interp_launch(int dtype, int disc, const void* V, const float* M, const float* tau,
                      void* Vhat, const SelPtrs& p, int64_t nbatch, int64_t T, int64_t F,
                      int64_t N, int64_t sv_b, int64_t sv_t, int64_t sm_b, int64_t sm_t,
                      int64_t stau_b, int64_t stau_t, int64_t sB_b, int64_t sB_l, int64_t sC_b,
                      int64_t sC_l, int64_t so_b, int64_t so_t, int64_t sy_b, int64_t sy_t,
                      int64_t K, int64_t FTILE, hipStream_t s) {
  SelDims m{};
  m.L = T; m.Dc = F; m.nbatch = nbatch;
  m.Rs = sel_chunk_steps(nbatch, T, F);
  m.nch = (T + m.Rs - 1) / m.Rs;
  m.sdt_b = stau_b; m.sdt_l = stau_t; m.sdt_d = 0;
  m.sB_b = sB_b; m.sB_l = sB_l; m.sC_b = sC_b; m.sC_l = sC_l; m.sy_b = sy_b; m.sy_l = sy_t;
  SiDims q;
  q.svb = sv_b; q.svt = sv_t; q.smb = sm_b; q.smt = sm_t; q.sob = so_b; q.sot = so_t;
  q.K = (int)K;
  q.lf = ilog2(FTILE);
  q.lvpt = q.lf - 2;
  const bool has_d = p.D != nullptr;
  if (dtype == TSSM_BF16) {
    return disc == TSSM_DISC_ZOH
               ? sel_interp_n<bf16_t, TSSM_DISC_ZOH>(N, has_d, V, M, tau, Vhat, p, m, q, s)
               : sel_interp_n<bf16_t, TSSM_DISC_EULER>(N, has_d, V, M, tau, Vhat, p, m, q, s);
  }
  return disc == TSSM_DISC_ZOH
             ? sel_interp_n<float, TSSM_DISC_ZOH>(N, has_d, V, M, tau, Vhat, p, m, q, s)
             : sel_interp_n<float, TSSM_DISC_EULER>(N, has_d, V, M, tau, Vhat, p, m, q, s);
}

int64_t sel_chunk_steps(int64_t nbatch, int64_t L, int64_t Dc) {
  (void)nbatch;
  (void)Dc;
  return L >= 64 ? kSelChunkSteps : 0;
}

bool sel_proj_ok(const float* raw, const float* W, const float* bias, int64_t Dc, int64_t rank,
                 int64_t sr_b, int64_t sr_l, int64_t sw_r) {
  return rank > 0 && rank <= kSelMaxRank && rank % 4 == 0 && Dc % 4 == 0 && sr_b % 4 == 0 &&
         sr_l % 4 == 0 && sw_r % 4 == 0 && sr_b >= 0 && sr_l >= 0 && sw_r >= 0 &&
         aligned(raw, 16) && aligned(W, 16) && aligned(bias, 16);
}

int64_t sel_dt_table_bytes(int64_t nbatch, int64_t L, int64_t Dc) {
  return nbatch * L * Dc * (int64_t)sizeof(float);
}

int64_t sel_state_floats(int64_t nbatch, int64_t nch, int64_t Dc, int64_t N) {
  const int64_t nseg = (nch + kSelSegChunks - 1) / kSelSegChunks;
  return nbatch * (nch + nseg) * Dc * (N + 1);
}

int64_t sel_chunked_bytes(int64_t nbatch, int64_t L, int64_t Dc, int64_t N) {
  if (!(N == 8 || N == 16) || nbatch <= 0 || L <= 0 || Dc <= 0) return 0;
  const int64_t rs = sel_chunk_steps(nbatch, L, Dc);
  if (rs == 0) return 0;
  const int64_t nch = (L + rs - 1) / rs;
  return sel_state_floats(nbatch, nch, Dc, N) * (int64_t)sizeof(float);
}

int sel_chunked_launch(int dtype, int disc, bool dt_shared, bool tau, const SelPtrs& p,
                       int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t sx_b,
                       int64_t sx_l, int64_t sdt_b, int64_t sdt_l, int64_t sdt_d, int64_t sB_b,
                       int64_t sB_l, int64_t sC_b, int64_t sC_l, int64_t sy_b, int64_t sy_l,
                       hipStream_t s) {
  SelDims m;
  m.L = L; m.Dc = Dc; m.nbatch = nbatch;
  m.Rs = sel_chunk_steps(nbatch, L, Dc);
  m.nch = (L + m.Rs - 1) / m.Rs;
  m.sx_b = sx_b; m.sx_l = sx_l; m.sdt_b = sdt_b; m.sdt_l = sdt_l; m.sdt_d = sdt_d;
  m.sB_b = sB_b; m.sB_l = sB_l; m.sC_b = sC_b; m.sC_l = sC_l; m.sy_b = sy_b; m.sy_l = sy_l;
  m.W = p.W; m.bias = p.bias; m.sw_r = p.sw_r; m.rank = (int)p.rank;
  m.dt_min = p.dt_min; m.dt_max = p.dt_max; m.dtw = p.W ? p.dtw : nullptr;
  if (p.W && (dt_shared || tau)) return TSSM_ERR_UNSUPPORTED;
  const bool has_d = p.D != nullptr;
  if (dtype == TSSM_BF16) {
    return disc == TSSM_DISC_ZOH
               ? sel_chunked_n<bf16_t, TSSM_DISC_ZOH>(N, has_d, dt_shared, tau, p, m, s)
               : sel_chunked_n<bf16_t, TSSM_DISC_EULER>(N, has_d, dt_shared, tau, p, m, s);
  }
  return disc == TSSM_DISC_ZOH
             ? sel_chunked_n<float, TSSM_DISC_ZOH>(N, has_d, dt_shared, tau, p, m, s)
             : sel_chunked_n<float, TSSM_DISC_EULER>(N, has_d, dt_shared, tau, p, m, s);
}

}  // namespace tssm

using namespace tssm;

extern "C" int64_t tssm_interp_selective_scan_workspace_bytes(int64_t nbatch, int64_t T,
                                                              int64_t F, int64_t N) {
  const int64_t cb = sel_chunked_bytes(nbatch, T, F, N);
  return cb > 0 ? cb : -1;
}

extern "C" int tssm_interp_selective_scan_supported(int dtype, int m_dtype, int tau_dtype,
                                                    int64_t nbatch, int64_t T, int64_t F,
                                                    int64_t N, int64_t K, int64_t FTILE,
                                                    const void* M, int64_t sm_b, int64_t sm_t,
                                                    int64_t sv_t) {
  return m_dtype == TSSM_F32 && tau_dtype == TSSM_F32 &&
                 sel_interp_ok(dtype, nbatch, T, F, N, K, FTILE, M, sm_b, sm_t, sv_t)
             ? 1
             : 0;
}

extern "C" int tssm_interp_selective_scan(int dtype, int disc, const void* V, const float* M,
                                          const float* tau, const float* A_log, const void* B,
                                          const void* C, const float* D, const float* h0,
                                          void* Vhat, void* y, float* h_last, int64_t nbatch,
                                          int64_t T, int64_t F, int64_t N, int64_t sv_b,
                                          int64_t sv_t, int64_t sm_b, int64_t sm_t,
                                          int64_t stau_b, int64_t stau_t, int64_t sB_b,
                                          int64_t sB_l, int64_t sC_b, int64_t sC_l, int64_t so_b,
                                          int64_t so_t, int64_t sy_b, int64_t sy_t, int64_t K,
                                          int64_t FTILE, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(V && M && tau && A_log && B && C && Vhat && y, TSSM_ERR_NULL);
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16, TSSM_ERR_DTYPE);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && T > 0 && F > 0, TSSM_ERR_SHAPE);
  const int64_t strides[] = {sv_b, sv_t, sm_b, sm_t, stau_b, stau_t, sB_b,
                             sB_l, sC_b, sC_l, so_b, so_t, sy_b, sy_t};
  for (int64_t st : strides) TSSM_CHECK(st >= 0, TSSM_ERR_STRIDE);
  TSSM_CHECK(sel_interp_ok(dtype, nbatch, T, F, N, K, FTILE, M, sm_b, sm_t, sv_t),
             TSSM_ERR_UNSUPPORTED);
  const int64_t vec = dtype == TSSM_F32 ? 4 : 8;
  TSSM_CHECK(sB_b % vec == 0 && sB_l % vec == 0 && sC_b % vec == 0 && sC_l % vec == 0,
             TSSM_ERR_ALIGN);
  TSSM_CHECK(aligned(B, 16) && aligned(C, 16) && aligned(A_log, 16), TSSM_ERR_ALIGN);
  const int64_t need = tssm_interp_selective_scan_workspace_bytes(nbatch, T, F, N);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 16), TSSM_ERR_ALIGN);
  SelPtrs p;
  p.A_log = A_log; p.B = B; p.C = C; p.D = D; p.h0 = h0; p.y = y; p.h_last = h_last;
  p.S = static_cast<float*>(workspace);
  const int64_t nch = (T + sel_chunk_steps(nbatch, T, F) - 1) / sel_chunk_steps(nbatch, T, F);
  p.T = p.S + nbatch * nch * F * N;
  return sel_interp_launch(dtype, disc, V, M, tau, Vhat, p, nbatch, T, F, N, sv_b, sv_t, sm_b,
                           sm_t, stau_b, stau_t, sB_b, sB_l, sC_b, sC_l, so_b, so_t, sy_b, sy_t,
                           K, FTILE, as_stream(stream));
}

extern "C" int64_t tssm_selective_scan_xproj_workspace_bytes(int64_t nbatch, int64_t L,
                                                             int64_t Dc, int64_t N) {
  if (nbatch <= 0 || L <= 0 || Dc <= 0 || !(N == 8 || N == 16)) return -1;
  const int64_t nch = (L + kSelChunkSteps - 1) / kSelChunkSteps;
  // chunk-state block, the C rows and the dt table for pass 3
  return sel_state_floats(nbatch, nch, Dc, N) * 4 + nbatch * L * N * 4 +
         sel_dt_table_bytes(nbatch, L, Dc) + 512;
}

extern "C" int tssm_selective_scan_xproj(int disc, const float* x, const float* A_log,
                                         const float* W_x, int64_t swx_d, int64_t rank,
                                         const float* W_dt, int64_t sw_r, const float* bias,
                                         float dt_min, float dt_max, const float* D,
                                         const float* h0, float* y, float* h_last,
                                         int64_t nbatch, int64_t L, int64_t Dc, int64_t N,
                                         int64_t sx_b, int64_t sx_l, int64_t sy_b, int64_t sy_l,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(x && A_log && W_x && W_dt && bias && y, TSSM_ERR_NULL);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && Dc > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK((N == 8 || N == 16) && Dc <= kSelThreads && Dc % 4 == 0 && nbatch <= 65535 &&
                 (rank == 16 || rank == 32 || rank == 48 || rank == 64),
             TSSM_ERR_UNSUPPORTED);
  const int64_t strides[] = {sx_b, sx_l, sy_b, sy_l, sw_r};
  for (int64_t st : strides) TSSM_CHECK(st >= 0, TSSM_ERR_STRIDE);
  TSSM_CHECK(swx_d >= rank + 2 * N && sw_r >= Dc && sw_r % 4 == 0, TSSM_ERR_STRIDE);
  TSSM_CHECK(aligned(x, 16) && sx_b % 4 == 0 && sx_l % 4 == 0 && aligned(A_log, 16) &&
                 aligned(W_dt, 16) && aligned(bias, 16),
             TSSM_ERR_ALIGN);
  TSSM_CHECK(dt_min <= dt_max, TSSM_ERR_SHAPE);
  const int64_t need = tssm_selective_scan_xproj_workspace_bytes(nbatch, L, Dc, N);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 16), TSSM_ERR_ALIGN);
  SelDims m{};
  m.L = L; m.Dc = Dc; m.nbatch = nbatch;
  m.Rs = kSelChunkSteps;
  m.nch = (L + m.Rs - 1) / m.Rs;
  m.sx_b = sx_b; m.sx_l = sx_l;
  m.sy_b = sy_b; m.sy_l = sy_l;
  m.W = W_dt; m.bias = bias; m.sw_r = sw_r; m.rank = (int)rank;
  m.dt_min = dt_min; m.dt_max = dt_max;
  SelPtrs p;
  p.x = x; p.A_log = A_log; p.D = D; p.h0 = h0; p.y = y; p.h_last = h_last;
  p.S = static_cast<float*>(workspace);
  p.T = p.S + nbatch * m.nch * Dc * N;
  float* Cws = p.S + sel_state_floats(nbatch, m.nch, Dc, N);
  // the dt table after the C rows, 16-byte aligned
  const int64_t cws_end = (int64_t)(reinterpret_cast<uintptr_t>(Cws + nbatch * L * N));
  m.dtw = reinterpret_cast<float*>((cws_end + 15) & ~int64_t(15));
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
  if (N == 16)
    return disc == TSSM_DISC_ZOH
               ? sel_xproj_r<TSSM_DISC_ZOH, 16>(rank, has_d, x, W_x, swx_d, Cws, p, m, s)
               : sel_xproj_r<TSSM_DISC_EULER, 16>(rank, has_d, x, W_x, swx_d, Cws, p, m, s);
  return disc == TSSM_DISC_ZOH
             ? sel_xproj_r<TSSM_DISC_ZOH, 8>(rank, has_d, x, W_x, swx_d, Cws, p, m, s)
             : sel_xproj_r<TSSM_DISC_EULER, 8>(rank, has_d, x, W_x, swx_d, Cws, p, m, s);
}

extern "C" int64_t tssm_selective_scan_bcproj_workspace_bytes(int64_t nbatch, int64_t L,
                                                              int64_t Dc, int64_t N) {
  if (nbatch <= 0 || L <= 0 || Dc <= 0 || !(N == 8 || N == 16)) return -1;
  const int64_t nch = (L + kSelChunkSteps - 1) / kSelChunkSteps;
  // chunk-state block, then the C rows for pass 3
  return sel_state_floats(nbatch, nch, Dc, N) * 4 + nbatch * L * N * 4 + 256;
}

extern "C" int tssm_selective_scan_bcproj(int disc, const float* x, const float* dt,
                                          int dt_is_tau, const float* A_log, const float* W_bc,
                                          int64_t sw_d, const float* D, const float* h0,
                                          float* y, float* h_last, int64_t nbatch, int64_t L,
                                          int64_t Dc, int64_t N, int64_t sx_b, int64_t sx_l,
                                          int64_t sdt_b, int64_t sdt_l, int64_t sdt_d,
                                          int64_t sy_b, int64_t sy_l, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(x && dt && A_log && W_bc && y, TSSM_ERR_NULL);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && Dc > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK((N == 8 || N == 16) && Dc <= kSelThreads && Dc % 4 == 0 && nbatch <= 65535,
             TSSM_ERR_UNSUPPORTED);
  const bool dt_shared = sdt_d == 0;
  TSSM_CHECK(dt_shared || !dt_is_tau, TSSM_ERR_UNSUPPORTED);
  const int64_t strides[] = {sx_b, sx_l, sdt_b, sdt_l, sdt_d, sy_b, sy_l};
  for (int64_t st : strides) TSSM_CHECK(st >= 0, TSSM_ERR_STRIDE);
  TSSM_CHECK(sw_d >= 2 * N, TSSM_ERR_STRIDE);
  TSSM_CHECK(aligned(x, 16) && sx_b % 4 == 0 && sx_l % 4 == 0 && aligned(A_log, 16),
             TSSM_ERR_ALIGN);
  const int64_t need = tssm_selective_scan_bcproj_workspace_bytes(nbatch, L, Dc, N);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 16), TSSM_ERR_ALIGN);
  SelDims m{};
  m.L = L; m.Dc = Dc; m.nbatch = nbatch;
  m.Rs = kSelChunkSteps;
  m.nch = (L + m.Rs - 1) / m.Rs;
  m.sx_b = sx_b; m.sx_l = sx_l; m.sdt_b = sdt_b; m.sdt_l = sdt_l; m.sdt_d = sdt_d;
  m.sy_b = sy_b; m.sy_l = sy_l;
  SelPtrs p;
  p.x = x; p.dt = dt; p.A_log = A_log; p.D = D; p.h0 = h0; p.y = y; p.h_last = h_last;
  p.S = static_cast<float*>(workspace);
  p.T = p.S + nbatch * m.nch * Dc * N;
  float* Cws = p.S + sel_state_floats(nbatch, m.nch, Dc, N);
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr, tau = dt_is_tau != 0;
  if (N == 16)
    return disc == TSSM_DISC_ZOH
               ? sel_bcproj_dt<TSSM_DISC_ZOH, 16>(has_d, dt_shared, tau, x, dt, W_bc, sw_d, Cws, p, m, s)
               : sel_bcproj_dt<TSSM_DISC_EULER, 16>(has_d, dt_shared, tau, x, dt, W_bc, sw_d, Cws, p, m, s);
  return disc == TSSM_DISC_ZOH
             ? sel_bcproj_dt<TSSM_DISC_ZOH, 8>(has_d, dt_shared, tau, x, dt, W_bc, sw_d, Cws, p, m, s)
             : sel_bcproj_dt<TSSM_DISC_EULER, 8>(has_d, dt_shared, tau, x, dt, W_bc, sw_d, Cws, p, m, s);
}

