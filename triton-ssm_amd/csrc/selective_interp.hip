// The interpolating pass 1 of the three-pass Mamba-1 selective scan
// (tssm_interp_selective_scan), in a translation unit of its own so that it
// is built with its own instruction-scheduling strategy (the build adds
// -mllvm -amdgpu-sched-strategy=max-ilp for this file: 91.6 -> 87.6 us per
// step at B=16 T=2048 F=256 N=16; the other passes keep the default, which
// measured faster for them).
#include <stdint.h>

#include "common.h"
#include "selective.h"
#include "selective_dev.h"

namespace tssm {

template <typename T, int DISC, int NST, bool HAS_D>
__global__ __launch_bounds__(kSelThreads) void sel_interp_state_kernel(
    const T* __restrict__ V, const float* __restrict__ M, const float* __restrict__ tau,
    const float* __restrict__ A_log, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const float* __restrict__ D, T* __restrict__ Vhat, T* __restrict__ y,
    float* __restrict__ S, float* __restrict__ Tsum, SelDims m, SiDims q) {
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int64_t cb0 = (int64_t)blockIdx.y * kSelThreads;  // first channel of the workgroup
  const int64_t d = cb0 + tid;
  const bool ok = d < m.Dc;
  const int64_t dc = ok ? d : m.Dc - 1;  // lanes past Dc compute channel Dc-1
  const int64_t t0 = c * m.Rs;
  const int n = (int)(m.L - t0 < m.Rs ? m.L - t0 : m.Rs);
  const int n4 = (n + kSelPf - 1) / kSelPf * kSelPf;
  const int K = q.K;
  const int R = n + 2 * K;  // flag rows t0-K .. t0+n+K-1

  __shared__ float sB[kSelChunkSteps * NST], sC[kSelChunkSteps * NST];
  __shared__ float sD[kSelChunkSteps];
  __shared__ float sTau[kSiRows];
  // per flag row: the ballot of the row's tile sums > 0.5 over the lanes
  // (lanes of one tile hold the same sum; bit lt << lvpt is tile lt's flag)
  __shared__ uint64_t sRowB[kSiRows];
  // per (step, tile): byte offsets of the rows read as "prev" and "next" from
  // the row t0-K of the lane's column, and the weight (-1: no pair, vhat is
  // the "prev" row's value)
  __shared__ int4 sNb[kSelChunkSteps * kSiMaxTiles];

  // ---- 1. prologue loads: rows to stage, timestamps, lane parameters, and
  // the first batch of mask rows, before one wait
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float4 vB = stage_row_load<T, NST>(Bm + b * m.sB_b + t0 * m.sB_l, m.sB_l, n, n4);
  const float4 vC = stage_row_load<T, NST>(Cm + b * m.sC_b + t0 * m.sC_l, m.sC_l, n, n4);
  const float* taub = tau + b * m.sdt_b;
  float vtau = 0.0f;
  if (tid < R) {
    const int64_t t = t0 - K + tid;
    vtau = taub[(t < 0 ? 0 : (t >= m.L ? m.L - 1 : t)) * m.sdt_l];
  }
  float al[NST];
  load_alog<NST>(A_log, dc, al);
  float Dd = HAS_D ? D[dc] : 0.0f;
  // wave wv sums rows wv, wv+4, ...: a uniform row pointer, lane l the
  // 16-byte vector of channels cb0+4l .. cb0+4l+3 (rows outside [0, L) and
  // vectors past F read a valid vector and count 0)
  const bool vec_ok = cb0 + 4 * lane < m.Dc;  // F = Dc, a multiple of 4
  const int vpt = 1 << q.lvpt;
  for (int i0 = wv; i0 < R; i0 += 4 * kSiMaskU) {
    float sv[kSiMaskU];
#pragma unroll
    for (int u = 0; u < kSiMaskU; ++u) {
      const int i = i0 + 4 * u;
      const int64_t t = t0 - K + i;
      const bool rok = i < R && t >= 0 && t < m.L;
      const float* rowp = M + b * q.smb + (rok ? t : 0) * q.smt + cb0;
      const float4 v = *reinterpret_cast<const float4*>(rowp + (vec_ok ? 4 * lane : 0));
      float sum = 0.0f;
      sum += v.x; sum += v.y; sum += v.z; sum += v.w;
      sv[u] = rok && vec_ok ? sum : 0.0f;
    }
    // The tile sum over its vpt lanes, level by level across the rows (the
    // rows' exchanges overlap).  Each level adds the partner group's sum, the
    // value the xor butterfly of interp_fused_kernel adds (after a level all
    // lanes of a group hold the same sum), so the flags are that kernel's.
#pragma unroll
    for (int u = 0; u < kSiMaskU; ++u) sv[u] += dpp_mov<0xB1>(sv[u]);   // xor 1
#pragma unroll
    for (int u = 0; u < kSiMaskU; ++u) sv[u] += dpp_mov<0x4E>(sv[u]);   // xor 2
    if (vpt >= 8) {
#pragma unroll
      for (int u = 0; u < kSiMaskU; ++u) sv[u] += dpp_mov<0x141>(sv[u]);  // the other quad
    }
    if (vpt >= 16) {
#pragma unroll
      for (int u = 0; u < kSiMaskU; ++u) sv[u] += dpp_mov<0x140>(sv[u]);  // the other 8
    }
    if (vpt >= 32) {
#pragma unroll
      for (int u = 0; u < kSiMaskU; ++u) sv[u] += swizzle_xor16(sv[u]);
    }
    if (vpt >= 64) {
#pragma unroll
      for (int u = 0; u < kSiMaskU; ++u) sv[u] += __shfl_xor(sv[u], 32);
    }
#pragma unroll
    for (int u = 0; u < kSiMaskU; ++u) {
      const int i = i0 + 4 * u;  // uniform per wave
      const uint64_t bb = __ballot(sv[u] > 0.5f);
      if (i < R && lane == 0) sRowB[i] = bb;
    }
  }
  stage_row_store<NST>(sB, vB, n4);
  stage_row_store<NST>(sC, vC, n4);
  if (tid < R) sTau[tid] = vtau;
  float a2[NST], nia[NST], h[NST];
  sel_params<NST>(al, a2, nia);
#pragma unroll
  for (int k = 0; k < NST; ++k) {
    h[k] = 0.0f;
    asm volatile("" : "+v"(a2[k]), "+v"(nia[k]));  // complete before the loop
  }
  asm volatile("" : "+v"(Dd));
  __syncthreads();  // flags, timestamps, rows staged

  // ---- 2. dt of the chunk's steps (timestamps differenced, padded steps 0)
  // and the neighbour tables (padded steps repeat step n-1)
  if (tid < n4) {
    const int64_t t = t0 + tid;
    sD[tid] = tid < n ? sTau[tid + K] - (t > 0 ? sTau[tid + K - 1] : 0.0f) : 0.0f;
  }
  // Wave wv takes tiles wv, wv+4, ...: three ballots give the tile's flags of
  // rows 0..191 (bit i: row t0-K+i) as uniform words, then lane r < n4 finds
  // step r's neighbours with bit scans: the highest flagged row of
  // [r, r+K-1] (prev) and the lowest of [r+K+1, r+2K] (next), row r+K being
  // the step itself.
  const int ntl = kSelThreads >> q.lf;
  const uint64_t kmask = K >= 64 ? ~0ull : ((1ull << K) - 1);
  for (int lt = wv; lt < ntl; lt += 4) {
    const int bit = lt << q.lvpt;
    uint64_t mw[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const int i = g * 64 + lane;
      mw[g] = __ballot(i < R && ((sRowB[i < R ? i : 0] >> bit) & 1ull));
    }
    if (lane < n4) {
      const int rr = lane < n ? lane : n - 1;
      const int64_t t = t0 + rr;
      // 64 flag bits starting at row s (rows past 191 read 0)
      auto bits64 = [&](int s) -> uint64_t {
        const int g = s >> 6, sh = s & 63;
        const uint64_t lo = g == 0 ? mw[0] : (g == 1 ? mw[1] : (g == 2 ? mw[2] : 0ull));
        const uint64_t hi = g == 0 ? mw[1] : (g == 1 ? mw[2] : 0ull);
        return sh == 0 ? lo : ((lo >> sh) | (hi << (64 - sh)));
      };
      const uint64_t wp = bits64(rr) & kmask;
      const uint64_t wn = bits64(rr + K + 1) & kmask;
      const int prev = wp ? (int)(t - K + (63 - __builtin_clzll(wp))) : -1;
      const int next = wn ? (int)(t + 1 + __builtin_ctzll(wn)) : -1;
      const float tau_t = sTau[rr + K];
      const float tp = prev >= 0 ? sTau[rr + K - (int)(t - prev)] : 0.0f;
      const float tn = next >= 0 ? sTau[rr + K + (int)(next - t)] : 0.0f;
      const float den = tn - tp;
      float w = den > 1e-9f ? (tau_t - tp) / den : 0.5f;
      w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
      // rows read as "prev" and "next" (as interp_kernel: v_prev, else
      // v_next, else v_cur; next falls back to the prev row), as byte offsets
      // from row t0-K (both rows lie in [t0-K, t0+n+K): the host bounds
      // (n+2K) row strides below 2^31 bytes)
      const int64_t rp = prev >= 0 ? prev : (next >= 0 ? next : t);
      const int64_t rn = next >= 0 ? next : rp;
      const int64_t rs = q.svt * (int64_t)sizeof(T);
      sNb[lane * kSiMaxTiles + lt] =
          make_int4((int)((rp - (t0 - K)) * rs), (int)((rn - (t0 - K)) * rs),
                    __float_as_int(prev >= 0 && next >= 0 ? w : -1.0f), 0);
    }
  }
  __syncthreads();
  // Waves whose lanes are all past Dc are done (no barrier follows).
  if (cb0 + (tid & ~63) >= m.Dc) return;

  // ---- 3. the recurrence over interpolated inputs
  const int lt = (int)((dc - cb0) >> q.lf);  // the lane's tile (of channel dc)
  // row t0-K of the workgroup's first channel (uniform; for the first chunk
  // it lies before V's row 0, and only rows >= 0 are read from it)
  const char* vbase =
      reinterpret_cast<const char*>(V + b * q.svb + (t0 - K) * q.svt + cb0);
  const uint32_t lboff = (uint32_t)((dc - cb0) * (int64_t)sizeof(T));
  T* ocol = Vhat + b * q.sob + dc;
  T* yp = y + b * m.sy_b + dc;
  // the pair of a table entry, and its weight
  auto fetch = [&](const int4& e, float& vp, float& vn, float& w) {
    vp = ldf(reinterpret_cast<const T*>(vbase + ((uint32_t)e.x + lboff)));
    vn = ldf(reinterpret_cast<const T*>(vbase + ((uint32_t)e.y + lboff)));
    w = __int_as_float(e.z);
  };
  float vp[kSelPf], vn[kSelPf], wq[kSelPf];
#pragma unroll
  for (int j = 0; j < kSelPf; ++j) fetch(sNb[(j < n4 ? j : n4 - 1) * kSiMaxTiles + lt], vp[j], vn[j], wq[j]);
  // dt one step ahead (the step's exp2s need only dt, so the B and C rows,
  // read at the top of the step, arrive while they issue); the neighbour
  // entry for step rr + 4 is read at the top too, used at the end
  float dtc = sD[0];
  float sdt = 0.0f;
  for (int r = 0; r < n4; r += kSelPf) {
#pragma unroll
    for (int j = 0; j < kSelPf; ++j) {
      const int rr = r + j;
      const int r1 = rr + 1 < n4 ? rr + 1 : n4 - 1;
      const int r4 = rr + kSelPf < n4 ? rr + kSelPf : n4 - 1;
      float Bv[NST], Cv[NST];
      lds_row<NST>(sB + rr * NST, Bv);
      lds_row<NST>(sC + rr * NST, Cv);
      const float dtn = sD[r1];
      const int4 e4 = sNb[r4 * kSiMaxTiles + lt];
      __builtin_amdgcn_sched_barrier(0);  // the step's LDS reads issue first
      // both forms computed, then a select (no branch around the loads' waits)
      const float li = lerp_pair(vp[j], vn[j], wq[j]);
      const float vh = wq[j] >= 0.0f ? li : vp[j];
      const float u = round_io<T>(vh);  // the scan consumes Vhat as stored
      const int64_t tw = t0 + (rr < n ? rr : n - 1);
      sel_update<DISC, NST>(h, a2, nia, Bv, u, dtc);
      sdt += dtc;
      float acc0 = HAS_D ? Dd * u : 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int k = 0; k < NST; k += 2) {
        acc0 = __builtin_fmaf(Cv[k], h[k], acc0);
        acc1 = __builtin_fmaf(Cv[k + 1], h[k + 1], acc1);
      }
      // unconditional stores: padded steps and lanes past Dc (in the wave of
      // channel Dc-1) store exactly the values of step n-1 / channel Dc-1
      stf(ocol + tw * q.sot, vh);
      stf(yp + tw * m.sy_l, acc0 + acc1);
      dtc = dtn;
      // refill the registers this step used, for step rr + 4
      __builtin_amdgcn_sched_barrier(0);
      fetch(e4, vp[j], vn[j], wq[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (ok) {
    float4* sp = reinterpret_cast<float4*>(S + ((b * m.nch + c) * m.Dc + d) * NST);
#pragma unroll
    for (int qq = 0; qq < NST / 4; ++qq)
      sp[qq] = make_float4(h[4 * qq], h[4 * qq + 1], h[4 * qq + 2], h[4 * qq + 3]);
    if (d == 0) Tsum[b * m.nch + c] = sdt;
  }
}

// Host side: pass 1 with interpolation, for the caller's dtype,
// discretization, state count and skip term.
template <typename T, int DISC, int NST>
int sel_interp_pass1_t(bool has_d, const void* V, const float* M, const float* tau, void* Vhat,
                       const SelPtrs& p, const SelDims& m, const SiDims& q, hipStream_t s) {
  const dim3 grid((unsigned)m.nch, (unsigned)((m.Dc + kSelThreads - 1) / kSelThreads),
                  (unsigned)m.nbatch);
  const T* Bm = static_cast<const T*>(p.B);
  const T* Cm = static_cast<const T*>(p.C);
  T* y = static_cast<T*>(p.y);
  const T* Vt = static_cast<const T*>(V);
  T* Ot = static_cast<T*>(Vhat);
  if (has_d)
    hipLaunchKernelGGL((sel_interp_state_kernel<T, DISC, NST, true>), grid, dim3(kSelThreads), 0,
                       s, Vt, M, tau, p.A_log, Bm, Cm, p.D, Ot, y, p.S, p.T, m, q);
  else
    hipLaunchKernelGGL((sel_interp_state_kernel<T, DISC, NST, false>), grid, dim3(kSelThreads),
                       0, s, Vt, M, tau, p.A_log, Bm, Cm, p.D, Ot, y, p.S, p.T, m, q);
  return (int)hipGetLastError();
}

int sel_interp_pass1(bool bf16, int disc, int nst, bool has_d, const void* V, const float* M,
                     const float* tau, void* Vhat, const SelPtrs& p, const SelDims& m,
                     const SiDims& q, hipStream_t s) {
#define TSSM_SIP(T, DI)                                                                     \
  (nst == 16 ? sel_interp_pass1_t<T, DI, 16>(has_d, V, M, tau, Vhat, p, m, q, s)          \
             : sel_interp_pass1_t<T, DI, 8>(has_d, V, M, tau, Vhat, p, m, q, s))
  if (bf16)
    return disc == TSSM_DISC_ZOH ? TSSM_SIP(bf16_t, TSSM_DISC_ZOH) : TSSM_SIP(bf16_t, TSSM_DISC_EULER);
  return disc == TSSM_DISC_ZOH ? TSSM_SIP(float, TSSM_DISC_ZOH) : TSSM_SIP(float, TSSM_DISC_EULER);
#undef TSSM_SIP
}

}  // namespace tssm
