// SSD selective scan (scalar decay per head, state P x N per (batch, head)).
//
//   h_t[p, n] = exp(dt_t a) h_{t-1}[p, n] + Bbar_t x_t[p] B_t[n]
//   y_t[p]    = sum_n C_t[n] h_t[p, n] + D[p] x_t[p]
// with Bbar_t = dt_t (Euler) or expm1(dt_t a)/a (ZOH) -- the recurrence of
// ssm_scan.py:5-10 with the discretization of discretize_kernel.py:44-54 and
// one decay per head.
//
// ssd_scan: three passes (chunk states, state passing, chunk outputs).  With
// few (batch, head) rows and very long sequences a single pass would keep
// hundreds of chunks of one row in flight, each look-back hop moving a whole
// P x N state; the passes instead re-read x, B and dt once.
//   pass 1 ssd_state_kernel: one wave per (row, chunk of TC steps), lane = p
//     with its N states in registers; writes the chunk's decay product and
//     local end state (from zero).
//   pass 2 ssd_pass_kernel: per state entry, a segmented scan over chunks
//     gives every chunk's entry state (and the final state).
//   pass 3 ssd_out_kernel: one wave per chunk rescans from its entry state and
//     writes y.
//   Both scans use the rescaled state h_t = P_t g_t (P_t = decay product since
//   the chunk start), so a step costs one FMA per state for the update; g is
//   folded back into h whenever P_t would drop below 2^-64.
// ssd_stream_step_kernel: one streaming step with the state [S,H,P,N] fp32
//   resident in HBM, updated in place; one workgroup per (stream, head).
#include "common.h"
#include "lookback.h"

#include "ssd_dev.h"

namespace tssm {

constexpr float kRescaleFloor = 5.421010862427522e-20f;  // 2^-64
constexpr int kSsdSub = 16;  // steps staged per sub-block

// One step of the rescaled recurrence h = Pt g:  h_t = ab h_{t-1} + xs B_t.
// When Pt ab would fall below 2^-64 the factor is folded into g (the branch is
// uniform: Pt and ab are the same on every lane of the wave).
template <int N>
__device__ inline void rescaled_step(float* g, float& Pt, float ab, float xs, const float* bv) {
  // Pt and ab hold the same value on every lane; reading the product through
  // lane 0 makes the fold decision a scalar branch.
  const float Pn = __builtin_bit_cast(
      float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, Pt * ab)));
  if (Pn < kRescaleFloor) {
#pragma unroll
    for (int n = 0; n < N; ++n) g[n] = __builtin_fmaf(xs, bv[n], g[n] * Pn);
    Pt = 1.0f;
  } else {
    const float xr = xs * __builtin_amdgcn_rcpf(Pn);
#pragma unroll
    for (int n = 0; n < N; ++n) g[n] = __builtin_fmaf(xr, bv[n], g[n]);
    Pt = Pn;
  }
}

// Registers of one sub-block of kSsdSub steps: x of the lane's channel and
// the B (and, for the outputs, C) rows, spread over the wave.  Every load of
// a sub-block is issued before the first is used: clamped addresses (steps
// past L re-read step L-1) and selects at the LDS store, no branch around a
// load (the compiler would wait for a load inside a branch on its own).
//
// With kSsdPipe<N> the loads of sub-block k+1 (and the dt of the next 64-step
// group) are issued before sub-block k is computed from LDS, so they are in
// flight during its steps.  That holds one more sub-block in registers:
// fp32 at L=65536 H=8 P=64: N=16 195.98 -> 178.13 us (state 76 -> 109,
// output 87 -> 127 VGPRs), N=32 267.1 -> 253.2 us; at N=64 the output pass
// drops to one wave per SIMD and the passes slow 432.4 -> 585.7 us, so N=64
// loads each sub-block just before it is used.
template <int N>
constexpr bool kSsdPipe = N <= 32;

template <int N, bool WITH_C>
struct SsdSub {
  static constexpr int K = (kSsdSub * N + 63) / 64;
  float x[kSsdSub], b[K], c[WITH_C ? K : 1];
};

template <typename T, int N, bool WITH_C>
__device__ inline void sub_load(SsdSub<N, WITH_C>& r, const T* __restrict__ xp, int64_t sx_l,
                                const T* __restrict__ Bp, int64_t sB_l, const T* __restrict__ Cp,
                                int64_t sC_l, int64_t ts, int64_t L, int lane) {
#pragma unroll
  for (int i = 0; i < kSsdSub; ++i) {
    const int64_t t = ts + i;
    r.x[i] = ldf(xp + (t < L ? t : L - 1) * sx_l);
  }
#pragma unroll
  for (int q = 0; q < SsdSub<N, WITH_C>::K; ++q) {
    const int k = lane + 64 * q;
    const int kc = k < kSsdSub * N ? k : 0;
    const int i = kc / N, n = kc - (kc / N) * N;
    const int64_t t = ts + i < L ? ts + i : L - 1;
    r.b[q] = ldf(Bp + t * sB_l + n);
    if constexpr (WITH_C) r.c[q] = ldf(Cp + t * sC_l + n);
  }
}

template <int N, bool WITH_C>
__device__ inline void sub_store(const SsdSub<N, WITH_C>& r, int64_t ts, int64_t L, bool act,
                                 float* s_x, float* s_B, float* s_C, int lane) {
#pragma unroll
  for (int i = 0; i < kSsdSub; ++i) s_x[i * 64 + lane] = (act && ts + i < L) ? r.x[i] : 0.0f;
#pragma unroll
  for (int q = 0; q < SsdSub<N, WITH_C>::K; ++q) {
    const int k = lane + 64 * q;
    if (k < kSsdSub * N) {
      const bool in = ts + k / N < L;
      s_B[k] = in ? r.b[q] : 0.0f;
      if constexpr (WITH_C) s_C[k] = in ? r.c[q] : 0.0f;
    }
  }
}

// dt of step t0 + lane (clamped address; steps at or past L are zeroed by
// step_scalars_of).
__device__ inline float dt_ahead(const float* dtp, int64_t sdt_l, int64_t t0, int64_t L,
                                 int lane) {
  const int64_t t = t0 + lane;
  return dtp[(t < L ? t : L - 1) * sdt_l];
}

// Per-step decay and input coefficient for steps [t0, t0+64) of one head,
// computed by lane i for step t0+i from its dt and shared through LDS.  Steps
// at or past L get dt = 0, i.e. decay 1 and coefficient 0, so they leave the
// state alone.
template <int DISC>
__device__ inline void step_scalars_of(float dl, int64_t t0, int64_t L, float a2, float* s_ab,
                                       float* s_cf, int lane) {
  const float d = t0 + lane < L ? dl : 0.0f;
  const float arg = d * a2;
  const float ab = exp2_fast(arg);
  s_ab[lane] = ab;
  s_cf[lane] = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(arg * 0.6931471805599453f, ab) * d : d;
}

// Pass 1 of the generic passes: the chunk's end state from a zero state,
// walked last step first, X += R_s coef_s x_s B_s with R_s the decay from
// step s+1 to the chunk end (a running product of the per-step decays), and
// the chunk's decay product R.  Once R has underflowed to exactly zero every
// earlier step adds an exact zero: the walk stops there (uniform: R depends
// only on the head's dt), and the decay product is zero.
template <typename T, int DISC, int N>
__global__ __launch_bounds__(64) void ssd_state_kernel(SsdArgs a) {
  __shared__ float s_ab[64], s_cf[64];
  __shared__ __align__(16) float s_B[kSsdSub * N];
  __shared__ float s_x[kSsdSub * 64];
  const int lane = threadIdx.x;
  const int P = (int)a.P;
  const bool act = lane < P;
  const uint32_t row = blockIdx.x / a.nchunks;
  const uint32_t c = blockIdx.x - row * a.nchunks;
  const uint32_t b = row / a.H, h = row - (row / a.H) * a.H;
  const float a2 = -expf(a.A_log[h]) * kLog2e;
  const int64_t tbeg = (int64_t)c * a.tc;
  const int64_t tend = tbeg + a.tc < a.L ? tbeg + a.tc : a.L;
  const float* dtp = a.dt + b * a.sdt_b + h * a.sdt_h;
  const T* xp = reinterpret_cast<const T*>(a.x) + b * a.sx_b + h * a.sx_h + (act ? lane : 0);
  const T* Bp = reinterpret_cast<const T*>(a.B) + b * a.sB_b + h * a.sB_h;
  float g[N];
#pragma unroll
  for (int n = 0; n < N; ++n) g[n] = 0.0f;
  float R = 1.0f;
  constexpr bool PIPE = kSsdPipe<N>;
  // sub-blocks of kSsdSub steps (a.tc is a multiple of 64), walked from the
  // last; each 64-step group's step scalars are formed on entering it
  const int64_t nsb = (tend - tbeg + kSsdSub - 1) / kSsdSub;
  auto group_t0 = [&](int64_t k) { return tbeg + (k * kSsdSub) / 64 * 64; };
  SsdSub<N, false> nxt;
  float dnext = 0.0f;
  if constexpr (PIPE) {
    sub_load<T, N, false>(nxt, xp, a.sx_l, Bp, a.sB_l, Bp, 0, tbeg + (nsb - 1) * kSsdSub, a.L,
                          lane);
    dnext = dt_ahead(dtp, a.sdt_l, group_t0(nsb - 1), a.L, lane);
  }
  for (int64_t k = nsb - 1; k >= 0; --k) {
    const int64_t ts = tbeg + k * kSsdSub;
    const int64_t t0 = group_t0(k);
    const int j = (int)(ts - t0);
    if (k == nsb - 1 || j + kSsdSub == 64) {  // entering a group from its end
      if constexpr (PIPE) {
        step_scalars_of<DISC>(dnext, t0, a.L, a2, s_ab, s_cf, lane);
        dnext = dt_ahead(dtp, a.sdt_l, t0 > tbeg ? t0 - 64 : tbeg, a.L, lane);
      } else {
        step_scalars_of<DISC>(dt_ahead(dtp, a.sdt_l, t0, a.L, lane), t0, a.L, a2, s_ab, s_cf,
                              lane);
      }
    }
    if constexpr (!PIPE) sub_load<T, N, false>(nxt, xp, a.sx_l, Bp, a.sB_l, Bp, 0, ts, a.L, lane);
    sub_store<N, false>(nxt, ts, a.L, act, s_x, s_B, s_B, lane);
    __syncthreads();
    if constexpr (PIPE)
      sub_load<T, N, false>(nxt, xp, a.sx_l, Bp, a.sB_l, Bp, 0, k > 0 ? ts - kSsdSub : ts, a.L,
                            lane);
#pragma unroll 2
    for (int i = kSsdSub - 1; i >= 0; --i) {
      const float w = R * (s_cf[j + i] * s_x[i * 64 + lane]);
#pragma unroll
      for (int n = 0; n < N; ++n) g[n] = __builtin_fmaf(w, s_B[i * N + n], g[n]);
      R *= s_ab[j + i];
    }
    __syncthreads();
    if (R == 0.0f) break;  // uniform: the earlier steps add exact zeros
  }
  const int64_t PN = (int64_t)P * N;
  if (act) {
    float* out = a.chunkX + ((int64_t)row * a.nchunks + c) * PN + (int64_t)lane * N;
#pragma unroll
    for (int n = 0; n < N; ++n) out[n] = g[n];
  }
  if (lane == 0) a.chunkA[(int64_t)row * a.nchunks + c] = R;
}

// Pass 2: thread (entry e, segment sg) of a 1024-thread workgroup covering 32
// consecutive state entries of one row and 32 segments of its chunks.  A
// segment's first kPassBatch chunks are loaded at once and stay in registers
// for the second sweep, so with up to 32 x kPassBatch chunks per row each
// sweep is one round trip to memory; longer segments continue kPassTail
// chunks at a time (indices clamped into the segment, so every load is in
// bounds and none waits behind a branch).
constexpr int kPassEntries = 32, kPassSegs = 32, kPassBatch = 32, kPassTail = 8;
__global__ __launch_bounds__(1024) void ssd_pass_kernel(SsdArgs a, int64_t PN) {
  __shared__ float s_a[kPassSegs][kPassEntries], s_x[kPassSegs][kPassEntries];
  __shared__ __align__(16) float s_ca[kPassSegs][kPassBatch];
  const int el = threadIdx.x % kPassEntries;
  const int sg = threadIdx.x / kPassEntries;
  const int64_t nblk = (PN + kPassEntries - 1) / kPassEntries;
  const int64_t row = blockIdx.x / nblk;
  const int64_t e = (blockIdx.x - row * nblk) * kPassEntries + el;
  const bool act = e < PN;
  const int64_t nc = a.nchunks;
  const int64_t seg = (nc + kPassSegs - 1) / kPassSegs;
  const int64_t c0 = sg * seg < nc ? sg * seg : nc, c1 = c0 + seg < nc ? c0 + seg : nc;
  // row bases are uniform; a row's chunk states are indexed with 32 bits
  // (the host keeps nchunks * P * N below 2^31)
  const char* cA = reinterpret_cast<const char*>(a.chunkA + row * nc);
  const char* cX = reinterpret_cast<const char*>(a.chunkX + row * nc * PN);
  const uint32_t e0 = act ? (uint32_t)e : 0u, pn = (uint32_t)PN;
  const uint32_t cmax = (uint32_t)(c1 > c0 ? c1 - 1 : 0);  // last chunk of the segment
  // byte offsets as 32-bit lane registers on a uniform base
  auto ldx = [&](uint32_t cc) {
    return *reinterpret_cast<const float*>(cX + (uint32_t)((cc * pn + e0) * 4u));
  };
  auto lda = [&](uint32_t cc) { return *reinterpret_cast<const float*>(cA + (uint32_t)(cc * 4u)); };
  // the segment's first batch: chunk states in registers, chunk decays (the
  // same for every entry) loaded once per segment into LDS, thread el taking
  // chunk c0 + el
  static_assert(kPassBatch == kPassEntries, "one decay per thread of a segment");
  s_ca[sg][el] = lda(min((uint32_t)c0 + (uint32_t)el, cmax));
  float x0[kPassBatch];
#pragma unroll
  for (int k = 0; k < kPassBatch; ++k) x0[k] = ldx(min((uint32_t)c0 + (uint32_t)k, cmax));
  __syncthreads();
  const float* a0 = s_ca[sg];
  float A = 1.0f, X = 0.0f;
#pragma unroll
  for (int k = 0; k < kPassBatch; ++k) {
    if (c0 + k < c1) {
      X = __builtin_fmaf(a0[k], X, x0[k]);
      A *= a0[k];
    }
  }
  for (int64_t c = c0 + kPassBatch; c < c1; c += kPassTail) {
    float xa[kPassTail], aa[kPassTail];
#pragma unroll
    for (int k = 0; k < kPassTail; ++k) {
      const uint32_t cc = min((uint32_t)(c + k), cmax);
      xa[k] = ldx(cc);
      aa[k] = lda(cc);
    }
#pragma unroll
    for (int k = 0; k < kPassTail; ++k) {
      if (c + k < c1) {
        X = __builtin_fmaf(aa[k], X, xa[k]);
        A *= aa[k];
      }
    }
  }
  s_a[sg][el] = A;
  s_x[sg][el] = X;
  __syncthreads();
  float S = (act && a.h0) ? a.h0[row * PN + e] : 0.0f;
  for (int k = 0; k < sg; ++k) S = __builtin_fmaf(s_a[k][el], S, s_x[k][el]);
  float* en = a.entry + row * nc * PN;
#pragma unroll
  for (int k = 0; k < kPassBatch; ++k) {
    if (c0 + k < c1) {
      if (act) en[(uint32_t)(c0 + k) * pn + e0] = S;
      S = __builtin_fmaf(a0[k], S, x0[k]);
    }
  }
  for (int64_t c = c0 + kPassBatch; c < c1; c += kPassTail) {
    float xa[kPassTail], aa[kPassTail];
#pragma unroll
    for (int k = 0; k < kPassTail; ++k) {
      const uint32_t cc = min((uint32_t)(c + k), cmax);
      xa[k] = ldx(cc);
      aa[k] = lda(cc);
    }
#pragma unroll
    for (int k = 0; k < kPassTail; ++k) {
      if (c + k < c1) {
        if (act) en[(uint32_t)(c + k) * pn + e0] = S;
        S = __builtin_fmaf(aa[k], S, xa[k]);
      }
    }
  }
  if (act && a.h_last && sg == kPassSegs - 1) a.h_last[row * PN + e] = S;
}

template <typename T, int DISC, int N, bool HAS_D>
__global__ __launch_bounds__(64) void ssd_out_kernel(SsdArgs a) {
  __shared__ float s_ab[64], s_cf[64];
  __shared__ __align__(16) float s_B[kSsdSub * N];
  __shared__ __align__(16) float s_C[kSsdSub * N];
  __shared__ float s_x[kSsdSub * 64];
  const int lane = threadIdx.x;
  const int P = (int)a.P;
  const bool act = lane < P;
  const uint32_t row = blockIdx.x / a.nchunks;
  const uint32_t c = blockIdx.x - row * a.nchunks;
  const uint32_t b = row / a.H, h = row - (row / a.H) * a.H;
  const float a2 = -expf(a.A_log[h]) * kLog2e;
  const int64_t tbeg = (int64_t)c * a.tc;
  const int64_t tend = tbeg + a.tc < a.L ? tbeg + a.tc : a.L;
  const float* dtp = a.dt + b * a.sdt_b + h * a.sdt_h;
  const T* xp = reinterpret_cast<const T*>(a.x) + b * a.sx_b + h * a.sx_h + (act ? lane : 0);
  const T* Bp = reinterpret_cast<const T*>(a.B) + b * a.sB_b + h * a.sB_h;
  const T* Cp = reinterpret_cast<const T*>(a.C) + b * a.sC_b + h * a.sC_h;
  T* yp = reinterpret_cast<T*>(a.y) + b * a.sy_b + h * a.sy_h + (act ? lane : 0);
  const int64_t PN = (int64_t)P * N;
  float g[N];
  {
    const float* en = a.entry + ((int64_t)row * a.nchunks + c) * PN + (int64_t)(act ? lane : 0) * N;
#pragma unroll
    for (int n = 0; n < N; ++n) g[n] = act ? en[n] : 0.0f;
  }
  const float dv = (HAS_D && act) ? a.D[h * P + lane] : 0.0f;
  float Pt = 1.0f;
  constexpr bool PIPE = kSsdPipe<N>;
  SsdSub<N, true> nxt;
  float dnext = 0.0f;
  if constexpr (PIPE) {
    sub_load<T, N, true>(nxt, xp, a.sx_l, Bp, a.sB_l, Cp, a.sC_l, tbeg, a.L, lane);
    dnext = dt_ahead(dtp, a.sdt_l, tbeg, a.L, lane);
  }
  for (int64_t t0 = tbeg; t0 < tend; t0 += 64) {
    if constexpr (PIPE) {
      step_scalars_of<DISC>(dnext, t0, a.L, a2, s_ab, s_cf, lane);
      dnext = dt_ahead(dtp, a.sdt_l, t0 + 64, a.L, lane);
    } else {
      step_scalars_of<DISC>(dt_ahead(dtp, a.sdt_l, t0, a.L, lane), t0, a.L, a2, s_ab, s_cf, lane);
    }
    for (int j = 0; j < 64 && t0 + j < tend; j += kSsdSub) {
      const int64_t ts = t0 + j;
      if constexpr (!PIPE)
        sub_load<T, N, true>(nxt, xp, a.sx_l, Bp, a.sB_l, Cp, a.sC_l, ts, a.L, lane);
      sub_store<N, true>(nxt, ts, a.L, act, s_x, s_B, s_C, lane);
      __syncthreads();
      if constexpr (PIPE)
        sub_load<T, N, true>(nxt, xp, a.sx_l, Bp, a.sB_l, Cp, a.sC_l, ts + kSsdSub, a.L, lane);
      const int m = a.L - ts < kSsdSub ? (int)(a.L - ts) : kSsdSub;
#pragma unroll 2
      for (int i = 0; i < kSsdSub; ++i) {
        const float xv = s_x[i * 64 + lane];
        float bv[N];
#pragma unroll
        for (int n = 0; n < N; ++n) bv[n] = s_B[i * N + n];
        rescaled_step<N>(g, Pt, s_ab[j + i], s_cf[j + i] * xv, bv);
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < N; ++n) acc = __builtin_fmaf(s_C[i * N + n], g[n], acc);
        acc *= Pt;
        if (HAS_D) acc = __builtin_fmaf(dv, xv, acc);
        if (act && i < m) stf(yp + (ts + i) * a.sy_l, acc);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- streaming step
// One (stream s, head h) per workgroup of 256 threads: thread = (p row within
// a pass of 8 rows, group of 4 state columns); 32 threads cover a row's 128
// columns (N = 128), reduced with cross-lane sums for y.
struct StreamArgs {
  const float* x;
  const float* dt;
  const float* A_log;
  const float* B;
  const float* C;
  const float* D;
  float* state;
  float* y;
  int64_t H, P, N, sdt_s, sdt_h;
  int64_t sx_s, sx_h, sB_s, sB_h, sC_s, sC_h, sy_s, sy_h;
};

constexpr int kStreamPB = 8;  // passes whose loads are in flight together

template <int DISC, bool HAS_D, int NG>
__global__ __launch_bounds__(256) void ssd_stream_step_kernel(StreamArgs a) {
  // NG = threads per state row (N / 4); rows per pass = 256 / NG
  constexpr int RPP = 256 / NG;
  const int64_t s = blockIdx.x / a.H;
  const int64_t h = blockIdx.x - s * a.H;
  const int tid = threadIdx.x;
  const int ng = tid % NG;
  const int rp = tid / NG;
  const float d = a.dt[s * a.sdt_s + h * a.sdt_h];
  const float arg = d * (-expf(a.A_log[h]) * kLog2e);
  const float ab = exp2_fast(arg);
  const float cf = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(arg * 0.6931471805599453f, ab) * d : d;
  const float4 bq = *reinterpret_cast<const float4*>(a.B + s * a.sB_s + h * a.sB_h + ng * 4);
  const float4 cq = *reinterpret_cast<const float4*>(a.C + s * a.sC_s + h * a.sC_h + ng * 4);
  float* st = a.state + ((s * a.H + h) * a.P) * a.N;
  // kStreamPB passes of RPP rows per batch: every load of a batch (x and the
  // state rows) is issued before the first update, so a workgroup makes one
  // round trip per batch instead of one per pass.  Rows past P re-read row
  // P-1 and store nothing.
  const float* xr = a.x + s * a.sx_s + h * a.sx_h;
  for (int64_t p0 = 0; p0 < a.P; p0 += RPP * kStreamPB) {
    f32x4 v[kStreamPB];
    float xv[kStreamPB], dv[kStreamPB];
#pragma unroll
    for (int u = 0; u < kStreamPB; ++u) {
      const int64_t p = p0 + u * RPP + rp;
      const int64_t pc = p < a.P ? p : a.P - 1;
      xv[u] = xr[pc];
      dv[u] = HAS_D ? a.D[h * a.P + pc] : 0.0f;  // with the batch, not behind the store's branch
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(st + pc * a.N + ng * 4));
    }
#pragma unroll
    for (int u = 0; u < kStreamPB; ++u) {
      const int64_t p = p0 + u * RPP + rp;
      const float xs = cf * xv[u];
      f32x4 w = v[u];
      w.x = __builtin_fmaf(ab, w.x, xs * bq.x);
      w.y = __builtin_fmaf(ab, w.y, xs * bq.y);
      w.z = __builtin_fmaf(ab, w.z, xs * bq.z);
      w.w = __builtin_fmaf(ab, w.w, xs * bq.w);
      if (p < a.P) __builtin_nontemporal_store(w, reinterpret_cast<f32x4*>(st + p * a.N + ng * 4));
      float acc = cq.x * w.x + cq.y * w.y + cq.z * w.z + cq.w * w.w;
      // sum over the NG threads of the row (aligned lane groups)
      for (int o = NG / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
      if (ng == 0 && p < a.P) {
        if (HAS_D) acc = __builtin_fmaf(dv[u], xv[u], acc);
        a.y[s * a.sy_s + h * a.sy_h + p] = acc;
      }
    }
  }
}


// Tile passes on the matrix cores, one wave per tile: wave w of a workgroup
// takes one (row, chunk) tile and walks its 32-step sub-chunks in order, the
// P x N state held in registers (16 per lane).  The waves of a workgroup (4
// rows of one chunk, sharing the 128-byte lines of B, C and dt) never wait
// for each other.  Every product is a 16x16x16 bf16 MFMA.  Its result layout
// (lane: column l%16, rows 4(l/16)+r) is its B operand layout (column l%16,
// k = 4(l/16)+j), and its A operand layout (row l%16, k = 4(l/16)+j) is that
// of the state as the state update leaves it, so Gram block, x product,
// carried-state product and state update chain without moving data between
// lanes.  With cum the inclusive prefix of log2 decay over a sub-chunk and
// cumE its total:
//   G[s][t]    = B_s . C_t                                (A = B rows, B = C rows)
//   M[s][t]    = G[s][t] 2^(cum_t - cum_s) coef_s,  s <= t
//   Y^T[p][t]  = 2^cum_t sum_n H[p][n] C_t[n] + sum_s x_s[p] M[s][t]
//   H^T[n][p] <- 2^cumE H^T[n][p] + sum_s w_s B_s[n] x_s[p],  w_s = 2^(cumE - cum_s) coef_s
// Pass 1 (ssd_state_wave_kernel) runs the state update from zero and writes
// each tile's end state and decay product; pass 3 (ssd_out_wave_kernel)
// starts from the tile's entry state and forms the outputs.  x, B and C
// enter the products exactly; operands formed in fp32 (weighted Gram blocks,
// weighted B, the state) enter as bf16 hi + lo parts (two products, ~16
// mantissa bits), and every product and the state accumulate in fp32.
constexpr int kWsub = 32;      // steps per sub-chunk
constexpr int kWaveRows = 4;   // tiles (one per wave) per workgroup


// Wave-private LDS tiles, rows padded so that every access of a lane is one
// base register plus a constant offset and the 16-row operand reads spread
// over the banks (units of 8 bytes: bank pair 9 p + unit for x^T, 18 t + unit
// for y, 10-dword rows for B):
//   x^T [p][s]  64 rows x 32 steps bf16, 72-byte rows
//   y   [t][p]  32 rows x 64 channels bf16, 144-byte rows (in the x^T space)
//   B   [s][n]  32 rows x 16 states bf16, 40-byte rows
constexpr int kWxRow = 36;   // bf16 elements per x^T row
constexpr int kWyRow = 72;   // per y row (16-byte aligned rows)
constexpr int kWbRow = 20;   // per B row
constexpr int kWxElems = kMp * kWxRow;  // 2304 (= 32 * kWyRow)

__device__ inline s16x4_t pk_s16x4(f32x4 v) {
  return __builtin_bit_cast(s16x4_t, make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])));
}
__device__ inline f32x4 unpk_s16x4(s16x4_t v) {
  const uint2 w = __builtin_bit_cast(uint2, v);
  return f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
}
__device__ inline f32x4 mfma16(s16x4_t a, s16x4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// Buffer descriptor over [base, base + bytes): loads past the end read zero,
// stores past it are dropped.
__device__ inline __amdgpu_buffer_rsrc_t wave_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

// One wave's tile.  blockIdx -> (chunk, group of rows): XCD x (blockIdx % 8)
// takes the chunks c = x (mod 8), all row groups of a chunk in consecutive
// slots, so every line shared by the heads of a step is fetched into one L2.
// Global memory goes through buffer descriptors based at the tile's first row
// and ending at the sequence's last row, so rows past L read as zero and
// their stores are dropped (every row stride covers a row, which the host
// checks); lane offsets are 32-bit registers, sub-chunk offsets scalars.
// x is read as (step quad sq, channel group g8) 16-byte pieces, B and C as
// (step 16 sg + c16, states 4q..4q+3) 8-byte pieces, dt at step lane % 32.
struct WaveTile {
  uint32_t row, c, b, h;
  int64_t tbeg;
  int nsub;
  __amdgpu_buffer_rsrc_t rx, rB, rd;
  int32_t bx, bB, bd;
  uint32_t ox, oB, od;
  // wave index as a scalar: every base below is uniform per wave
  __device__ bool init(const SsdArgs& a, uint32_t ngroups, int wv, int lane) {
    const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    c = xcd + 8u * (slot / ngroups);
    row = (slot % ngroups) * kWaveRows + (uint32_t)wv;
    if (c >= a.nchunks || row >= a.rows) return false;
    b = row / a.H;
    h = row - b * a.H;
    tbeg = (int64_t)c * a.tc;
    const int64_t nrow = (tbeg + a.tc < a.L ? tbeg + a.tc : a.L) - tbeg;
    nsub = (int)((nrow + kWsub - 1) / kWsub);
    const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x) + b * a.sx_b + h * a.sx_h;
    const uint16_t* Bb = reinterpret_cast<const uint16_t*>(a.B) + b * a.sB_b + h * a.sB_h;
    const float* dtb = a.dt + b * a.sdt_b + h * a.sdt_h;
    rx = wave_rsrc(xb + tbeg * a.sx_l, ((nrow - 1) * a.sx_l + kMp) * 2);
    rB = wave_rsrc(Bb + tbeg * a.sB_l, ((nrow - 1) * a.sB_l + kMn) * 2);
    rd = wave_rsrc(dtb + tbeg * a.sdt_l, ((nrow - 1) * a.sdt_l + 1) * 4);
    bx = (int32_t)(a.sx_l * 2);
    bB = (int32_t)(a.sB_l * 2);
    bd = (int32_t)(a.sdt_l * 4);
    const int c16 = lane & 15, q = lane >> 4, g8 = lane & 7, sq = lane >> 3;
    ox = (uint32_t)(4 * sq * bx + 16 * g8);
    oB = (uint32_t)(c16 * bB + 8 * q);
    od = (uint32_t)((lane & 31) * bd);
    return true;
  }
  // XPOL: cache policy of the x loads (non-temporal by default: a pass that
  // reads x once; the fused kernel's first sweep reads it through the caches
  // for its second sweep)
  template <int XPOL = kBufNt>
  __device__ void load(int r0, u32x4* xr, u32x2* bq, float& dtv) const {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      xr[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)ox, (r0 + k) * bx, XPOL);
#pragma unroll
    for (int sg = 0; sg < 2; ++sg)
      bq[sg] = __builtin_amdgcn_raw_buffer_load_b64(rB, (int)oB, (r0 + 16 * sg) * bB, 0);
    dtv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, (int)od, r0 * bd, 0));
  }
};

// x^T of a sub-chunk into LDS: the lane holds rows 4sq..4sq+3, channels
// 8g8..8g8+7, and writes 4 steps of each of its 8 channels.
__device__ inline void wave_put_xt(uint16_t* xt, const u32x4* w, int g8, int sq) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const int m = e >> 1;
    *reinterpret_cast<uint2*>(xt + (8 * g8 + e) * kWxRow + 4 * sq) =
        make_uint2(perm_lo(w[0][m], w[1][m]), perm_lo(w[2][m], w[3][m]));
    *reinterpret_cast<uint2*>(xt + (8 * g8 + e + 1) * kWxRow + 4 * sq) =
        make_uint2(perm_hi(w[0][m], w[1][m]), perm_hi(w[2][m], w[3][m]));
  }
}

// Per-step scalars of a sub-chunk (lanes i and i + 32: step i): inclusive
// prefix of the log2 decay, input coefficient and the sub-chunk total.
// Steps at or past L get dt = 0 (decay 1, coefficient 0).
template <int DISC>
__device__ inline void wave_scalars(float dtv, bool live, float a2, float& pre, float& cf,
                                    float& cumE) {
  const float d = live ? dtv : 0.0f;
  const float l2 = d * a2;
  cf = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(l2 * 0.6931471805599453f, exp2_fast(l2)) * d : d;
  pre = scan_incl<32>(l2);
  cumE = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pre), 31));
}

// x^T pieces: x_s[p] for p = 16 pi + c16, s = 16 sg + 4q .. +3.
__device__ inline void wave_get_xa(const uint16_t* xt, int c16, int q, s16x4_t (*xa)[2]) {
#pragma unroll
  for (int pi = 0; pi < 4; ++pi)
#pragma unroll
    for (int sg = 0; sg < 2; ++sg)
      xa[pi][sg] = __builtin_bit_cast(
          s16x4_t, *reinterpret_cast<const uint2*>(xt + (16 * pi + c16) * kWxRow + 16 * sg + 4 * q));
}

// State update to the end of a sub-chunk: H^T <- At H^T + (w B)^T x, with the
// A operand (w B)^T (row n = c16, k = steps 16 sg + 4q .. +3) read transposed
// from the B rows in LDS and split hi/lo.
__device__ inline void wave_state_update(f32x4* st, const s16x4_t (*xa)[2], const uint16_t* bs,
                                         const float* sw, int c16, int q, float At) {
  s16x4_t wb[2], wl[2];
#pragma unroll
  for (int sg = 0; sg < 2; ++sg) {
    const f32x4 ws = *reinterpret_cast<const f32x4*>(sw + 16 * sg + 4 * q);
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = bf16_bits_to_f32(bs[(16 * sg + 4 * q + j) * kWbRow + c16]) * ws[j];
    wb[sg] = pk_s16x4(v);
    wl[sg] = pk_s16x4(v - unpk_s16x4(wb[sg]));
  }
#pragma unroll
  for (int pi = 0; pi < 4; ++pi) {
    f32x4 v = st[pi];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] *= At;
    v = mfma16(wb[0], xa[pi][0], v);
    v = mfma16(wl[0], xa[pi][0], v);
    v = mfma16(wb[1], xa[pi][1], v);
    v = mfma16(wl[1], xa[pi][1], v);
    st[pi] = v;
  }
}

// Pass 1: end state of each tile from zero ([p][n] in chunkX) and its decay
// product (chunkA).  The tile is walked last sub-chunk first, each weight
// carrying the log2 decay of the later sub-chunks (lsum), and the walk stops
// where the decay from the tile end has underflowed to exactly zero: every
// earlier step's weight is then exactly zero, and so is the decay product.
template <int DISC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void ssd_state_wave_kernel(SsdArgs a, uint32_t ngroups) {
  __shared__ __align__(16) uint16_t s_xt[kWaveRows][kMp * kWxRow];
  __shared__ __align__(16) uint16_t s_b[kWaveRows][kWsub * kWbRow];
  __shared__ __align__(16) float s_w[kWaveRows][kWsub];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, q = lane >> 4, g8 = lane & 7, sq = lane >> 3;
  WaveTile wt;
  if (!wt.init(a, ngroups, wv, lane)) return;  // whole waves; no barriers below
  uint16_t* xt = s_xt[wv];
  uint16_t* bs = s_b[wv];
  float* sw = s_w[wv];
  const float a2 = -expf(a.A_log[wt.h]) * kLog2e;
  u32x4 xr[4];
  u32x2 bq[2];
  float dtv;
  wt.load((wt.nsub - 1) * kWsub, xr, bq, dtv);
  f32x4 st[4];
#pragma unroll
  for (int pi = 0; pi < 4; ++pi) st[pi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float lsum = 0.0f;  // log2 decay from the end of the current sub-chunk to the tile end
#pragma unroll 1
  for (int k = wt.nsub - 1; k >= 0; --k) {
    const int r0 = k * kWsub;
    wave_put_xt(xt, xr, g8, sq);
#pragma unroll
    for (int sg = 0; sg < 2; ++sg)
      *reinterpret_cast<u32x2*>(bs + (16 * sg + c16) * kWbRow + 4 * q) = bq[sg];
    float pre, cf, cumE;
    wave_scalars<DISC>(dtv, wt.tbeg + r0 + (lane & 31) < a.L, a2, pre, cf, cumE);
    if (lane < 32) sw[lane] = exp2_fast(lsum + cumE - pre) * cf;
    lsum += cumE;
    // uniform: the earlier sub-chunks would add exact zeros
    const bool done = k == 0 || exp2_fast(lsum) == 0.0f;
    // the previous sub-chunk's loads overlap everything below
    if (!done) wt.load(r0 - kWsub, xr, bq, dtv);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    s16x4_t xa[4][2];
    wave_get_xa(xt, c16, q, xa);
    wave_state_update(st, xa, bs, sw, c16, q, 1.0f);
    if (done) break;
  }
  float* out = a.chunkX + ((int64_t)wt.row * a.nchunks + wt.c) * (kMp * kMn);
#pragma unroll
  for (int pi = 0; pi < 4; ++pi)
    *reinterpret_cast<f32x4*>(out + (16 * pi + c16) * kMn + 4 * q) = st[pi];
  if (lane == 0) a.chunkA[(int64_t)wt.row * a.nchunks + wt.c] = exp2_fast(lsum);
}

// LDS of one wave in the output sweep.
struct WaveOutLds {
  uint16_t* xt;   // x^T, then the staged y rows
  uint16_t* bs;   // B rows
  float* scum;    // per-step scalars: inclusive log2 decay, coefficient, weight
  float* scoef;
  float* sw;
  uint16_t* xrow; // row-major x (skip term)
};

// Outputs of one wave's segment from its entry state `st` (the state
// advances through the segment; the lane holds H[16 pi + c16][4q..4q+3]).
// XPOL: cache policy of the x loads.
template <int DISC, bool HAS_D, int XPOL = kBufNt>
__device__ inline void wave_out_sweep(const SsdArgs& a, const WaveTile& wt, f32x4* st,
                                      const WaveOutLds& ld, float a2, int lane) {
  const int c16 = lane & 15, q = lane >> 4, g8 = lane & 7, sq = lane >> 3;
  uint16_t* xt = ld.xt;
  uint16_t* bs = ld.bs;
  float* scum = ld.scum;
  float* scoef = ld.scoef;
  float* sw = ld.sw;
  uint16_t* xrow = ld.xrow;
  const int64_t nrow = (wt.tbeg + a.tc < a.L ? wt.tbeg + a.tc : a.L) - wt.tbeg;
  const uint16_t* Cb =
      reinterpret_cast<const uint16_t*>(a.C) + wt.b * a.sC_b + wt.h * a.sC_h + wt.tbeg * a.sC_l;
  uint16_t* yb = reinterpret_cast<uint16_t*>(a.y) + wt.b * a.sy_b + wt.h * a.sy_h + wt.tbeg * a.sy_l;
  const __amdgpu_buffer_rsrc_t rC = wave_rsrc(Cb, ((nrow - 1) * a.sC_l + kMn) * 2);
  const __amdgpu_buffer_rsrc_t ry = wave_rsrc(yb, ((nrow - 1) * a.sy_l + kMp) * 2);
  const int32_t bC = (int32_t)(a.sC_l * 2), by = (int32_t)(a.sy_l * 2);
  const uint32_t oC = (uint32_t)(c16 * bC + 8 * q);
  const uint32_t oy = (uint32_t)((lane >> 3) * by + 16 * (lane & 7));
  // C through the caches: the 4 waves of a workgroup share its 128-byte lines
  // (a streaming hint let them be evicted between the waves' reads: 20% more
  // bytes fetched).  Two sub-chunks of loads are in flight: sub-chunk k + 2
  // is loaded into k's registers once k is staged (rows clamped to the last
  // sub-chunk, which is then re-read from the caches instead of branching).
  auto load_sub = [&](int r0, u32x4* xr, u32x2* bq, u32x2* cq, float& dtv) {
    wt.template load<XPOL>(r0, xr, bq, dtv);
#pragma unroll
    for (int sg = 0; sg < 2; ++sg)
      cq[sg] = __builtin_amdgcn_raw_buffer_load_b64(rC, (int)oC, (r0 + 16 * sg) * bC, 0);
  };
  const int last_r0 = (wt.nsub - 1) * kWsub;
  u32x4 xrA[4], xrB[4];
  u32x2 bqA[2], cqA[2], bqB[2], cqB[2];
  float dtA, dtB;
  load_sub(0, xrA, bqA, cqA, dtA);
  __builtin_amdgcn_sched_barrier(0);
  load_sub(kWsub < last_r0 ? kWsub : last_r0, xrB, bqB, cqB, dtB);
  float dsk[4][4];
  if constexpr (HAS_D) {
#pragma unroll
    for (int pi = 0; pi < 4; ++pi)
#pragma unroll
      for (int r = 0; r < 4; ++r) dsk[pi][r] = a.D[wt.h * kMp + 16 * pi + 4 * q + r];
  }

  auto body = [&](int k, u32x4* xr, u32x2* bq, u32x2* cq, float& dtv) {
    const int r0 = k * kWsub;
    // x^T, B rows (and the row-major x for the skip term) into LDS
    const u32x2 bz[2] = {bq[0], bq[1]}, cz[2] = {cq[0], cq[1]};
    wave_put_xt(xt, xr, g8, sq);
    if constexpr (HAS_D) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        *reinterpret_cast<u32x4*>(xrow + (4 * sq + kk) * kMp + 8 * g8) = xr[kk];
    }
#pragma unroll
    for (int sg = 0; sg < 2; ++sg)
      *reinterpret_cast<u32x2*>(bs + (16 * sg + c16) * kWbRow + 4 * q) = bz[sg];
    float pre, cf, cumE;
    wave_scalars<DISC>(dtv, wt.tbeg + r0 + (lane & 31) < a.L, a2, pre, cf, cumE);
    if (lane < 32) {
      scum[lane] = pre;
      scoef[lane] = cf;
      sw[lane] = exp2_fast(cumE - pre) * cf;
    }
    // sub-chunk k + 2's loads overlap everything below and the next sub-chunk
    load_sub(r0 + 2 * kWsub < last_r0 ? r0 + 2 * kWsub : last_r0, xr, bq, cq, dtv);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");

    // decay-weighted Gram blocks (s-block sg <= t-block tb) as the B operands
    // of the x products, split hi/lo
    s16x4_t mb[3], ml[3];  // (tb, sg) = (0, 0), (1, 0), (1, 1)
    {
      const f32x4 cs[2] = {*reinterpret_cast<const f32x4*>(scum + 4 * q),
                           *reinterpret_cast<const f32x4*>(scum + 16 + 4 * q)};
      const f32x4 cfv[2] = {*reinterpret_cast<const f32x4*>(scoef + 4 * q),
                            *reinterpret_cast<const f32x4*>(scoef + 16 + 4 * q)};
      const float cumt[2] = {scum[c16], scum[16 + c16]};
#pragma unroll
      for (int blk = 0; blk < 3; ++blk) {
        const int tb = blk == 0 ? 0 : 1, sg = blk == 2 ? 1 : 0;
        const f32x4 g = mfma16(__builtin_bit_cast(s16x4_t, bz[sg]),
                               __builtin_bit_cast(s16x4_t, cz[tb]), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        f32x4 m;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          m[r] = g[r] * exp2_fast(cumt[tb] - cs[sg][r]) * cfv[sg][r];
          if (sg == tb) m[r] = 4 * q + r <= c16 ? m[r] : 0.0f;
        }
        mb[blk] = pk_s16x4(m);
        ml[blk] = pk_s16x4(m - unpk_s16x4(mb[blk]));
      }
    }
    s16x4_t xa[4][2];
    wave_get_xa(xt, c16, q, xa);

    // outputs, 16 steps t at a time; the staged rows replace x^T (all of
    // whose reads are above)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const s16x4_t cb = __builtin_bit_cast(s16x4_t, cz[tb]);
      const int t = 16 * tb + c16;
      const float ut = exp2_fast(scum[t]);
#pragma unroll
      for (int pi = 0; pi < 4; ++pi) {
        const s16x4_t sh = pk_s16x4(st[pi]);
        f32x4 acc = mfma16(sh, cb, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        acc = mfma16(pk_s16x4(st[pi] - unpk_s16x4(sh)), cb, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= ut;
        acc = mfma16(xa[pi][0], mb[tb], acc);
        acc = mfma16(xa[pi][0], ml[tb], acc);
        if (tb == 1) {
          acc = mfma16(xa[pi][1], mb[2], acc);
          acc = mfma16(xa[pi][1], ml[2], acc);
        }
        if constexpr (HAS_D) {
          const uint2 xv = *reinterpret_cast<const uint2*>(xrow + t * kMp + 16 * pi + 4 * q);
          acc[0] = __builtin_fmaf(dsk[pi][0], bf16_lo(xv.x), acc[0]);
          acc[1] = __builtin_fmaf(dsk[pi][1], bf16_hi(xv.x), acc[1]);
          acc[2] = __builtin_fmaf(dsk[pi][2], bf16_lo(xv.y), acc[2]);
          acc[3] = __builtin_fmaf(dsk[pi][3], bf16_hi(xv.y), acc[3]);
        }
        *reinterpret_cast<uint2*>(xt + t * kWyRow + 16 * pi + 4 * q) =
            make_uint2(pk_bf16(acc[0], acc[1]), pk_bf16(acc[2], acc[3]));
      }
    }
    wave_state_update(st, xa, bs, sw, c16, q, exp2_fast(cumE));

    // the staged 32 x 64 outputs leave as whole 128-byte rows (8 lanes a row)
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = (lane >> 3) + 8 * i;
      const u32x4 v = *reinterpret_cast<const u32x4*>(xt + tr * kWyRow + 8 * (lane & 7));
      __builtin_amdgcn_raw_buffer_store_b128(v, ry, (int)oy, (r0 + 8 * i) * by, kBufNt);
    }
  };
#pragma unroll 1
  for (int k = 0; k < wt.nsub; k += 2) {
    body(k, xrA, bqA, cqA, dtA);
    if (k + 1 < wt.nsub) body(k + 1, xrB, bqB, cqB, dtB);
  }
}


// Pass 3: outputs of each tile from its entry state.
template <int DISC, bool HAS_D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HAS_D ? 2 : 3))) void ssd_out_wave_kernel(SsdArgs a, uint32_t ngroups) {
  __shared__ __align__(16) uint16_t s_xt[kWaveRows][kWxElems];
  __shared__ __align__(16) uint16_t s_b[kWaveRows][kWsub * kWbRow];
  __shared__ __align__(16) float s_sc[kWaveRows][3][kWsub];  // cum, coef, w
  __shared__ __align__(16) uint16_t s_xr[HAS_D ? kWaveRows : 1][HAS_D ? kWsub * kMp : 4];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  WaveTile wt;
  if (!wt.init(a, ngroups, wv, lane)) return;  // whole waves; no barriers below
  const WaveOutLds ld{s_xt[wv], s_b[wv], s_sc[wv][0], s_sc[wv][1], s_sc[wv][2],
                      s_xr[HAS_D ? wv : 0]};
  const float a2 = -expf(a.A_log[wt.h]) * kLog2e;
  // state entering the tile: lane holds H[16 pi + c16][4q..4q+3]
  f32x4 st[4];
  {
    const float* en = a.entry + ((int64_t)wt.row * a.nchunks + wt.c) * (kMp * kMn);
#pragma unroll
    for (int pi = 0; pi < 4; ++pi)
      st[pi] = *reinterpret_cast<const f32x4*>(en + (16 * pi + c16) * kMn + 4 * q);
  }
  wave_out_sweep<DISC, HAS_D>(a, wt, st, ld, a2, lane);
}

// ---------------------------------------------------------------- fused tile kernel
// One launch in place of the three tile passes (chunk states, state passing,
// outputs): a wave takes one (row, segment) and
//  1. sweeps the segment's 32-step sub-chunks LAST TO FIRST, accumulating the
//     segment's end state from zero with each sub-chunk's weights taken to
//     the segment end, H^T += sum_s 2^(lsum + cumE - cum_s) coef_s B_s x_s
//     (lsum: the log2 decay of the later sub-chunks) -- the products of pass
//     1, in reverse order -- and stops where the decay from the segment end
//     has underflowed to exactly zero (the earlier steps add exact zeros);
//  2. publishes the segment's carry as tagged look-back words (its end state
//     from zero and decay product, or, when the decay product is exactly
//     zero, its inclusive state -- the end state itself -- at once);
//  3. resolves its entry state by a decoupled look-back over the segments of
//     its row (ssd_lookback), publishes its inclusive state;
//  4. sweeps the segment forward from the entry state, forming the outputs
//     (wave_out_sweep, the products of pass 3).
// Waves only wait on segments with a smaller index (lower blockIdx: see
// WaveTile::init), every wait is bounded (an expired wait sets the sticky
// error word).
struct SsdLb {
  uint64_t* status;  // [rows][nseg][2] tags: aggregate published, inclusive published
  uint64_t* dec;     // [rows][nseg] decay product of the segment
  uint64_t* agg;     // [rows][nseg][16][64] end state from zero (lane-major)
  uint64_t* inc;     // [rows][nseg][16][64] state after the segment
  WsHeader* hdr;
  uint32_t tag, spin_limit;
};
constexpr int kSsdLbVals = 16;  // state values per lane (H[16 pi + c16][4q + r])

// The 16 words of a lane at `base` (word v at base + 64 v + lane), waited on
// until each carries the tag (bounded).
__device__ inline void settle16(const uint64_t* base, int lane, uint32_t tag, float* v,
                                uint32_t& spins, uint32_t spin_limit, WsHeader* hdr) {
  uint64_t w[kSsdLbVals];
#pragma unroll
  for (int i = 0; i < kSsdLbVals; ++i) w[i] = ld_word(base + 64 * i + lane);
#pragma unroll
  for (int i = 0; i < kSsdLbVals; ++i) {
    w[i] = settle_word(base + 64 * i + lane, w[i], tag, spins, spin_limit, hdr);
    v[i] = word_val(w[i]);
  }
}

// State entering segment c of the row whose segment 0 is `sbase`: fold the
// predecessors' carries newest first -- an inclusive state ends the walk, an
// aggregate (end state X, decay A) is folded in, S = A S_prev + X -- up to
// the row's initial state h0v.  The status of 64 predecessors is read at
// once (lane k: segment c-1-k).  A decay product of exactly zero ends the
// walk too: nothing earlier can contribute.
// h0p: the row's initial state ([P][N], NULL: zero); the lane's values are
// H[16 pi + c16][4q..4q+3].
__device__ inline void load_h0(const float* h0p, int lane, float* v) {
  const int c16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int pi = 0; pi < 4; ++pi) {
    const f32x4 w = h0p ? *reinterpret_cast<const f32x4*>(h0p + (16 * pi + c16) * kMn + 4 * q)
                        : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 4; ++r) v[4 * pi + r] = w[r];
  }
}

__device__ inline void ssd_lookback(const SsdLb& lb, int64_t sbase, int64_t c, int lane,
                                    const float* h0p, float* S) {
  float A = 1.0f, X[kSsdLbVals];
#pragma unroll
  for (int i = 0; i < kSsdLbVals; ++i) X[i] = 0.0f;
  int64_t j = c - 1;  // newest predecessor not folded yet
  uint32_t spins = 0;
  while (true) {
    bool inc_k = false, rdy_k = false;
    if (j - lane < 0) {
      inc_k = rdy_k = true;  // before segment 0 stands h0, an inclusive value
    } else {
      const uint64_t wi = ld_word(lb.status + 2 * (sbase + j - lane) + 1);
      const uint64_t wa = ld_word(lb.status + 2 * (sbase + j - lane));
      inc_k = word_tag(wi) == lb.tag;
      rdy_k = inc_k || word_tag(wa) == lb.tag;
    }
    const uint64_t m_inc = __ballot(inc_k);
    const uint64_t m_rdy = __ballot(rdy_k);
    const int k_inc = m_inc ? __builtin_ctzll(m_inc) : 64;
    const int k_gap = ~m_rdy ? __builtin_ctzll(~m_rdy) : 64;
    const bool resolve = k_inc < k_gap;
    const int n = resolve ? k_inc : k_gap;
    for (int i = 0; i < n; ++i) {  // uniform
      const int64_t sj = sbase + j - i;
      const uint64_t wd = settle_word(lb.dec + sj, ld_word(lb.dec + sj), lb.tag, spins,
                                      lb.spin_limit, lb.hdr);
      float xv[kSsdLbVals];
      settle16(lb.agg + sj * (64 * kSsdLbVals), lane, lb.tag, xv, spins, lb.spin_limit, lb.hdr);
#pragma unroll
      for (int v = 0; v < kSsdLbVals; ++v) X[v] = __builtin_fmaf(A, xv[v], X[v]);
      A *= word_val(wd);
      if (A == 0.0f) {  // uniform: earlier segments cannot contribute
#pragma unroll
        for (int v = 0; v < kSsdLbVals; ++v) S[v] = X[v];
        return;
      }
    }
    if (resolve) {
      const int64_t ji = j - k_inc;
      if (ji < 0) {
        float hv[kSsdLbVals];
        load_h0(h0p, lane, hv);
#pragma unroll
        for (int v = 0; v < kSsdLbVals; ++v) S[v] = __builtin_fmaf(A, hv[v], X[v]);
      } else {
        float iv[kSsdLbVals];
        settle16(lb.inc + (sbase + ji) * (64 * kSsdLbVals), lane, lb.tag, iv, spins,
                 lb.spin_limit, lb.hdr);
#pragma unroll
        for (int v = 0; v < kSsdLbVals; ++v) S[v] = __builtin_fmaf(A, iv[v], X[v]);
      }
      return;
    }
    j -= n;
    if (n == 0) {
      if (++spins > lb.spin_limit) {  // predecessor never published: give up loudly
        flag_error(lb.hdr);
#pragma unroll
        for (int v = 0; v < kSsdLbVals; ++v) S[v] = X[v];
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (spins > lb.spin_limit) {
#pragma unroll
      for (int v = 0; v < kSsdLbVals; ++v) S[v] = X[v];
      return;
    }
  }
}

template <int DISC, bool HAS_D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HAS_D ? 2 : 3))) void ssd_fused_wave_kernel(SsdArgs a, SsdLb lb, uint32_t ngroups) {
  __shared__ __align__(16) uint16_t s_xt[kWaveRows][kWxElems];
  __shared__ __align__(16) uint16_t s_b[kWaveRows][kWsub * kWbRow];
  __shared__ __align__(16) float s_sc[kWaveRows][3][kWsub];  // cum, coef, w
  __shared__ __align__(16) uint16_t s_xr[HAS_D ? kWaveRows : 1][HAS_D ? kWsub * kMp : 4];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, q = lane >> 4, g8 = lane & 7, sq = lane >> 3;
  WaveTile wt;
  if (!wt.init(a, ngroups, wv, lane)) return;  // whole waves; no barriers in this kernel
  const WaveOutLds ld{s_xt[wv], s_b[wv], s_sc[wv][0], s_sc[wv][1], s_sc[wv][2],
                      s_xr[HAS_D ? wv : 0]};
  const float a2 = -expf(a.A_log[wt.h]) * kLog2e;

  // ---- 1. end state from zero, last sub-chunk first, x through the caches
  f32x4 st[4];
#pragma unroll
  for (int pi = 0; pi < 4; ++pi) st[pi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float lsum = 0.0f;  // log2 decay from the end of the current sub-chunk to the segment end
  {
    u32x4 xr[4];
    u32x2 bq[2];
    float dtv;
    wt.template load<0>((wt.nsub - 1) * kWsub, xr, bq, dtv);
#pragma unroll 1
    for (int k = wt.nsub - 1; k >= 0; --k) {
      const int r0 = k * kWsub;
      wave_put_xt(ld.xt, xr, g8, sq);
#pragma unroll
      for (int sg = 0; sg < 2; ++sg)
        *reinterpret_cast<u32x2*>(ld.bs + (16 * sg + c16) * kWbRow + 4 * q) = bq[sg];
      float pre, cf, cumE;
      wave_scalars<DISC>(dtv, wt.tbeg + r0 + (lane & 31) < a.L, a2, pre, cf, cumE);
      if (lane < 32) ld.sw[lane] = exp2_fast(lsum + cumE - pre) * cf;
      lsum += cumE;
      // Once the decay from the segment end to this sub-chunk's start is
      // exactly zero, every earlier step's weight 2^(lsum + cumE' - cum_s)
      // (an exponent at most lsum) is exactly zero too: the earlier
      // sub-chunks add exact zeros to the end state, and the segment's decay
      // product is zero.  They are not read (uniform exit).
      const bool done = k == 0 || exp2_fast(lsum) == 0.0f;
      // the previous sub-chunk's loads overlap everything below
      if (!done) wt.template load<0>(r0 - kWsub, xr, bq, dtv);
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
      s16x4_t xa[4][2];
      wave_get_xa(ld.xt, c16, q, xa);
      wave_state_update(st, xa, ld.bs, ld.sw, c16, q, 1.0f);
      if (done) break;
    }
  }
  // decay product of the segment (uniform; zero when the sweep stopped early)
  const float dseg = exp2_fast(lsum);
  // st now holds X, the end state from zero; X[4 pi + r] = st[pi][r]

  // ---- 2./3. carry out, entry state in
  const int64_t sbase = (int64_t)wt.row * a.nchunks;  // segment 0 of the row
  const int64_t sidx = sbase + wt.c;
  uint64_t* incw = lb.inc + sidx * (64 * kSsdLbVals);
  const float* h0p = a.h0 ? a.h0 + (int64_t)wt.row * (kMp * kMn) : nullptr;
  // Publish the carry before looking back: the inclusive state itself when
  // the segment forgets everything before it (decay product exactly zero),
  // else the aggregate (X, decay product).
  if (wt.c != 0) {
    const bool forget = dseg == 0.0f;  // uniform
    uint64_t* dst = forget ? incw : lb.agg + sidx * (64 * kSsdLbVals);
#pragma unroll
    for (int pi = 0; pi < 4; ++pi)
#pragma unroll
      for (int r = 0; r < 4; ++r) st_word(dst + 64 * (4 * pi + r) + lane, st[pi][r], lb.tag);
    if (lane == 0) {
      if (!forget) st_word(lb.dec + sidx, dseg, lb.tag);
      st_word(lb.status + 2 * sidx + (forget ? 1 : 0), 0.0f, lb.tag);
    }
  }
  float S[kSsdLbVals];  // state entering the segment
  if (wt.c == 0) load_h0(h0p, lane, S);
  else ssd_lookback(lb, sbase, wt.c, lane, h0p, S);
  // state after the segment, O = dseg S + X: published (unless it already
  // was) and, for the row's last segment, the final state
  const bool last = a.h_last && wt.c + 1 == a.nchunks;
  if (wt.c == 0 || dseg != 0.0f || last) {
    float* hp = last ? a.h_last + (int64_t)wt.row * (kMp * kMn) : nullptr;
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      f32x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = __builtin_fmaf(dseg, S[4 * pi + r], st[pi][r]);
      if (wt.c == 0 || dseg != 0.0f) {
#pragma unroll
        for (int r = 0; r < 4; ++r) st_word(incw + 64 * (4 * pi + r) + lane, o[r], lb.tag);
      }
      if (last) *reinterpret_cast<f32x4*>(hp + (16 * pi + c16) * kMn + 4 * q) = o;
    }
    if ((wt.c == 0 || dseg != 0.0f) && lane == 0) st_word(lb.status + 2 * sidx + 1, 0.0f, lb.tag);
  }

  // ---- 4. outputs from the entry state
#pragma unroll
  for (int pi = 0; pi < 4; ++pi)
    st[pi] = f32x4{S[4 * pi], S[4 * pi + 1], S[4 * pi + 2], S[4 * pi + 3]};
  wave_out_sweep<DISC, HAS_D>(a, wt, st, ld, a2, lane);
}

// Tiles per wave of the tile passes: a wave walks ``seg`` consecutive
// 256-step tiles with the state in registers, so the states are passed
// between segments of seg tiles only.  Two tiles per wave when that still
// gives kSegFill waves (4 per SIMD on 256 CUs, one resident generation):
// half the state traffic of one tile per wave and half the passing.
constexpr int64_t kSegFill = 4096;
inline int64_t ssd_wave_seg(int64_t rows, int64_t nchunks) {
  return rows * ((nchunks + 1) / 2) >= kSegFill ? 2 : 1;
}

// The tile passes read rows past L as zero through the buffer range check:
// every row stride must cover one row of the operand, and a segment's rows
// (seg_steps) of every operand must span less than 2^31 bytes.  Outputs leave
// as 16-byte pieces (y rows 16-byte aligned).
inline bool ssd_wave_ok(const SsdArgs& a, int64_t seg_steps) {
  const int64_t lim = (int64_t)1 << 31, q = seg_steps;
  return aligned(a.y, 16) && a.sy_l % 8 == 0 && a.sy_h % 8 == 0 && a.sy_b % 8 == 0 &&
         a.sx_l >= kMp && a.sB_l >= kMn && a.sC_l >= kMn && a.sy_l >= kMp && a.sdt_l >= 1 &&
         (q * a.sx_l + kMp) * 2 < lim && (q * a.sB_l + kMn) * 2 < lim &&
         (q * a.sC_l + kMn) * 2 < lim && (q * a.sy_l + kMp) * 2 < lim &&
         (q * a.sdt_l + 1) * 4 < lim;
}

// ``a.tc`` and ``a.nchunks`` are the segment length and count here; the
// workspace laid out for 256-step chunks holds the fewer segments.
template <int DISC>
int launch_ssd_mfma(bool has_d, int64_t rows, int64_t nchunks, int64_t PN, hipStream_t s,
                    const SsdArgs& a) {
  const uint32_t ngroups = (uint32_t)((rows + kWaveRows - 1) / kWaveRows);
  const dim3 gw((unsigned)(8 * ((nchunks + 7) / 8) * ngroups));
  hipLaunchKernelGGL((ssd_state_wave_kernel<DISC>), gw, dim3(256), 0, s, a, ngroups);
  const int64_t nblk = (PN + kPassEntries - 1) / kPassEntries;
  hipLaunchKernelGGL(ssd_pass_kernel, dim3((unsigned)(rows * nblk)), dim3(kPassEntries * kPassSegs),
                     0, s, a, PN);
  if (has_d) hipLaunchKernelGGL((ssd_out_wave_kernel<DISC, true>), gw, dim3(256), 0, s, a, ngroups);
  else hipLaunchKernelGGL((ssd_out_wave_kernel<DISC, false>), gw, dim3(256), 0, s, a, ngroups);
  return launch_status();
}


inline int64_t cdiv64(int64_t x, int64_t y) { return (x + y - 1) / y; }

template <typename T, int DISC, int N, bool HAS_D>
int launch_ssd_passes(int64_t rows, int64_t nchunks, int64_t PN, hipStream_t s, const SsdArgs& a) {
  const dim3 tiles((unsigned)(rows * nchunks));
  hipLaunchKernelGGL((ssd_state_kernel<T, DISC, N>), tiles, dim3(64), 0, s, a);
  const int64_t nblk = (PN + kPassEntries - 1) / kPassEntries;
  hipLaunchKernelGGL(ssd_pass_kernel, dim3((unsigned)(rows * nblk)), dim3(kPassEntries * kPassSegs),
                     0, s, a, PN);
  hipLaunchKernelGGL((ssd_out_kernel<T, DISC, N, HAS_D>), tiles, dim3(64), 0, s, a);
  return launch_status();
}

template <typename T, int DISC, bool HAS_D>
int launch_ssd_n(int N, int64_t rows, int64_t nchunks, int64_t PN, hipStream_t s, const SsdArgs& a) {
  switch (N) {
    case 8: return launch_ssd_passes<T, DISC, 8, HAS_D>(rows, nchunks, PN, s, a);
    case 16: return launch_ssd_passes<T, DISC, 16, HAS_D>(rows, nchunks, PN, s, a);
    case 32: return launch_ssd_passes<T, DISC, 32, HAS_D>(rows, nchunks, PN, s, a);
    case 64: return launch_ssd_passes<T, DISC, 64, HAS_D>(rows, nchunks, PN, s, a);
    default: return TSSM_ERR_UNSUPPORTED;
  }
}

template <typename T>
int launch_ssd_t(int disc, bool has_d, int N, int64_t rows, int64_t nchunks, int64_t PN,
                 hipStream_t s, const SsdArgs& a) {
  if (disc == TSSM_DISC_ZOH)
    return has_d ? launch_ssd_n<T, TSSM_DISC_ZOH, true>(N, rows, nchunks, PN, s, a)
                 : launch_ssd_n<T, TSSM_DISC_ZOH, false>(N, rows, nchunks, PN, s, a);
  return has_d ? launch_ssd_n<T, TSSM_DISC_EULER, true>(N, rows, nchunks, PN, s, a)
               : launch_ssd_n<T, TSSM_DISC_EULER, false>(N, rows, nchunks, PN, s, a);
}

// Steps per chunk: the `chunk` hint rounded to a multiple of 64 in [64, 1024].
inline int64_t ssd_tc(int64_t chunk) {
  int64_t tc = (chunk + 63) / 64 * 64;
  if (tc < 64) tc = 64;
  if (tc > 1024) tc = 1024;
  return tc;
}

}  // namespace tssm

using namespace tssm;

extern "C" int64_t tssm_ssd_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t H, int64_t P,
                                                 int64_t N, int64_t chunk) {
  if (nbatch <= 0 || L <= 0 || H <= 0 || P <= 0 || P > 64 || N <= 0) return -1;
  const int64_t nchunks = cdiv64(L, ssd_tc(chunk));
  const int64_t rows = nbatch * H;
  // chunk decay products + chunk end states + chunk entry states (fp32)
  return (rows * nchunks * (1 + 2 * P * N)) * 4 + 256;
}

extern "C" int tssm_ssd_scan(int dtype, int disc, const void* x, const float* dt,
                             const float* A_log, const void* B, const void* C, const float* D,
                             const float* h0, void* y, float* h_last, int64_t nbatch, int64_t L,
                             int64_t H, int64_t P, int64_t N, int64_t sx_b, int64_t sx_l,
                             int64_t sx_h, int64_t sdt_b, int64_t sdt_l, int64_t sdt_h,
                             int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sC_b,
                             int64_t sC_l, int64_t sC_h, int64_t sy_b, int64_t sy_l,
                             int64_t sy_h, int64_t chunk, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(x && dt && A_log && B && C && y, TSSM_ERR_NULL);
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16 || dtype == TSSM_F16, TSSM_ERR_DTYPE);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(nbatch > 0 && L > 0 && H > 0 && P > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(P <= 64 && (N == 8 || N == 16 || N == 32 || N == 64), TSSM_ERR_UNSUPPORTED);
  const int64_t need = tssm_ssd_scan_workspace_bytes(nbatch, L, H, P, N, chunk);
  TSSM_CHECK(workspace && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 256), TSSM_ERR_ALIGN);
  const int64_t strides[] = {sx_b, sx_l, sx_h, sdt_b, sdt_l, sdt_h, sB_b, sB_l, sB_h,
                             sC_b, sC_l, sC_h, sy_b, sy_l, sy_h};
  for (int64_t s : strides) TSSM_CHECK(s >= 0, TSSM_ERR_STRIDE);
  const int64_t tc = ssd_tc(chunk);
  const int64_t nchunks = cdiv64(L, tc);
  const int64_t rows = nbatch * H;
  const int64_t PN = P * N;
  TSSM_CHECK(nchunks * rows < (int64_t)INT32_MAX && nchunks * PN < (int64_t)INT32_MAX,
             TSSM_ERR_UNSUPPORTED);
  SsdArgs a;
  a.x = x; a.dt = dt; a.A_log = A_log; a.B = B; a.C = C; a.D = D; a.h0 = h0; a.y = y;
  a.h_last = h_last; a.L = L;
  a.sx_b = sx_b; a.sx_l = sx_l; a.sx_h = sx_h; a.sdt_b = sdt_b; a.sdt_l = sdt_l; a.sdt_h = sdt_h;
  a.sB_b = sB_b; a.sB_l = sB_l; a.sB_h = sB_h; a.sC_b = sC_b; a.sC_l = sC_l; a.sC_h = sC_h;
  a.sy_b = sy_b; a.sy_l = sy_l; a.sy_h = sy_h;
  // The first 256 bytes are the workspace header (sticky error word) shared
  // with the look-back kernels; the three passes use what follows.
  float* ws = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + 256);
  a.chunkX = ws;
  a.entry = ws + rows * nchunks * PN;
  a.chunkA = ws + 2 * rows * nchunks * PN;
  a.H = (uint32_t)H; a.P = (uint32_t)P; a.rows = (uint32_t)rows; a.nchunks = (uint32_t)nchunks;
  a.tc = (uint32_t)tc;
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
  // bf16 at P = 64, N = 16 with 256-step tiles: matrix-core passes (other
  // row strides take the generic passes)
  int64_t wseg = ssd_wave_seg(rows, nchunks);
  if (wseg > 1 && !ssd_wave_ok(a, wseg * kMq)) wseg = 1;  // row strides too long for a segment
  if (dtype == TSSM_BF16 && P == kMp && N == kMn && tc == kMq && ssd_wave_ok(a, wseg * kMq)) {
    TSSM_CHECK(aligned(x, 16) && aligned(B, 16) && aligned(C, 16) && aligned(y, 8), TSSM_ERR_ALIGN);
    TSSM_CHECK(sx_l % 8 == 0 && sx_h % 8 == 0 && sx_b % 8 == 0 && sB_l % 8 == 0 && sB_b % 8 == 0 &&
                   sB_h % 8 == 0 && sC_l % 8 == 0 && sC_b % 8 == 0 && sC_h % 8 == 0 &&
                   sy_l % 4 == 0 && sy_b % 4 == 0 && sy_h % 4 == 0,
               TSSM_ERR_ALIGN);
    const int64_t nseg = cdiv64(nchunks, wseg);
    a.tc = (uint32_t)(wseg * kMq);
    a.nchunks = (uint32_t)nseg;
    return disc == TSSM_DISC_ZOH ? launch_ssd_mfma<TSSM_DISC_ZOH>(has_d, rows, nseg, PN, s, a)
                                 : launch_ssd_mfma<TSSM_DISC_EULER>(has_d, rows, nseg, PN, s, a);
  }
  // bf16 at N = 64 with 16-channel blocks: one matrix-core pass per channel block
  if (dtype == TSSM_BF16 && N == kSqN && P % kSqP == 0 && aligned(x, 16) && aligned(B, 16) &&
      aligned(C, 16) && aligned(y, 8) && sx_l % 8 == 0 && sx_h % 8 == 0 && sx_b % 8 == 0 &&
      sB_l % 8 == 0 && sB_h % 8 == 0 && sB_b % 8 == 0 && sC_l % 8 == 0 && sC_h % 8 == 0 &&
      sC_b % 8 == 0 && sy_l % 4 == 0 && sy_h % 4 == 0 && sy_b % 4 == 0 &&
      rows * (P / kSqP) < (int64_t)INT32_MAX)
    return launch_ssd_seq_any(disc, has_d, rows, P, s, a);
  switch (dtype) {
    case TSSM_BF16: return launch_ssd_t<bf16_t>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
    case TSSM_F16: return launch_ssd_t<f16_t>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
    default: return launch_ssd_t<float>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
  }
}

namespace tssm {
namespace {

// The fused tile kernel applies where the matrix-core tile passes do (bf16,
// P = 64, N = 16, 256-step tiles, row strides that cover a row) and the
// tagged words fit 32-bit segment indices.
bool ssd_fused_ok(int dtype, int64_t P, int64_t N, int64_t tc, const SsdArgs& a, int64_t rows,
                  int64_t nseg, int64_t seg_steps) {
  return dtype == TSSM_BF16 && P == kMp && N == kMn && tc == kMq && ssd_wave_ok(a, seg_steps) &&
         aligned(a.x, 16) && aligned(a.B, 16) && aligned(a.C, 16) && aligned(a.y, 8) &&
         (!a.h0 || aligned(a.h0, 16)) && (!a.h_last || aligned(a.h_last, 16)) &&
         a.sx_l % 8 == 0 && a.sx_h % 8 == 0 && a.sx_b % 8 == 0 && a.sB_l % 8 == 0 &&
         a.sB_b % 8 == 0 && a.sB_h % 8 == 0 && a.sC_l % 8 == 0 && a.sC_b % 8 == 0 &&
         a.sC_h % 8 == 0 && a.sy_l % 4 == 0 && a.sy_b % 4 == 0 && a.sy_h % 4 == 0 &&
         rows * nseg < (int64_t)INT32_MAX;
}

// Look-back words of the fused kernel per (row, segment): 2 status, 1 decay,
// 16 x 64 end-state and 16 x 64 inclusive-state words.
constexpr int64_t kSsdSegWords = 3 + 2 * 64 * kSsdLbVals;

// Segments of 4 tiles (1024 steps) while that still gives 2048 waves, else
// as the wave passes (2 or 1).  At B=1 L=262144 H=8: 4 tiles (2048 waves)
// 157.7 us, 2 tiles (4096 waves) 164.5 us, 8 tiles (1024 waves) 172.5 us
// (later: 4 tiles 148-150 us against 167 us for 3 tiles, 2736 waves) --
// longer segments halve the look-back words and the share of a segment the
// first sweep re-reads, until too few waves remain to keep the memory busy.
constexpr int64_t kFusedSeg4Waves = 2048;
int64_t ssd_fused_segs(int64_t rows, int64_t nchunks, int64_t* wseg) {
  *wseg = rows * cdiv64(nchunks, 4) >= kFusedSeg4Waves ? 4 : ssd_wave_seg(rows, nchunks);
  return cdiv64(nchunks, *wseg);
}

}  // namespace
}  // namespace tssm

extern "C" int64_t tssm_ssd_scan_fused_workspace_bytes(int64_t nbatch, int64_t L, int64_t H,
                                                       int64_t P, int64_t N, int64_t chunk) {
  if (nbatch <= 0 || L <= 0 || H <= 0 || P != kMp || N != kMn || ssd_tc(chunk) != kMq) return -1;
  const int64_t rows = nbatch * H;
  int64_t wseg = 1;
  const int64_t nseg = ssd_fused_segs(rows, cdiv64(L, kMq), &wseg);
  return (int64_t)sizeof(WsHeader) + rows * nseg * kSsdSegWords * 8;
}

namespace tssm {
namespace {
int ssd_fused_setup(int dtype, const void* x, const float* dt, const float* A_log, const void* B,
                    const void* C, const float* D, const float* h0, void* y, float* h_last,
                    int64_t nbatch, int64_t L, int64_t H, int64_t P, int64_t N, int64_t sx_b,
                    int64_t sx_l, int64_t sx_h, int64_t sdt_b, int64_t sdt_l, int64_t sdt_h,
                    int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sC_b, int64_t sC_l,
                    int64_t sC_h, int64_t sy_b, int64_t sy_l, int64_t sy_h, int64_t chunk,
                    SsdArgs* a, int64_t* nseg_out) {
  if (!(x && dt && A_log && B && C && y)) return TSSM_ERR_NULL;
  if (nbatch <= 0 || L <= 0 || H <= 0) return TSSM_ERR_SHAPE;
  const int64_t strides[] = {sx_b, sx_l, sx_h, sdt_b, sdt_l, sdt_h, sB_b, sB_l, sB_h,
                             sC_b, sC_l, sC_h, sy_b, sy_l, sy_h};
  for (int64_t st : strides)
    if (st < 0) return TSSM_ERR_STRIDE;
  const int64_t tc = ssd_tc(chunk);
  const int64_t rows = nbatch * H;
  int64_t wseg = 1;
  const int64_t nseg = ssd_fused_segs(rows, cdiv64(L, kMq), &wseg);
  SsdArgs& r = *a;
  r.x = x; r.dt = dt; r.A_log = A_log; r.B = B; r.C = C; r.D = D; r.h0 = h0; r.y = y;
  r.h_last = h_last; r.L = L;
  r.sx_b = sx_b; r.sx_l = sx_l; r.sx_h = sx_h; r.sdt_b = sdt_b; r.sdt_l = sdt_l; r.sdt_h = sdt_h;
  r.sB_b = sB_b; r.sB_l = sB_l; r.sB_h = sB_h; r.sC_b = sC_b; r.sC_l = sC_l; r.sC_h = sC_h;
  r.sy_b = sy_b; r.sy_l = sy_l; r.sy_h = sy_h;
  r.chunkA = r.chunkX = r.entry = nullptr;
  r.H = (uint32_t)H; r.P = (uint32_t)P; r.rows = (uint32_t)rows;
  r.nchunks = (uint32_t)nseg;
  r.tc = (uint32_t)(wseg * kMq);
  if (!ssd_fused_ok(dtype, P, N, tc, r, rows, nseg, wseg * kMq)) return TSSM_ERR_UNSUPPORTED;
  *nseg_out = nseg;
  return TSSM_OK;
}
}  // namespace
}  // namespace tssm

extern "C" int tssm_ssd_scan_fused_supported(int dtype, const void* x, const float* dt,
                                             const float* A_log, const void* B, const void* C,
                                             const float* D, const float* h0, void* y,
                                             float* h_last, int64_t nbatch, int64_t L, int64_t H,
                                             int64_t P, int64_t N, int64_t sx_b, int64_t sx_l,
                                             int64_t sx_h, int64_t sdt_b, int64_t sdt_l,
                                             int64_t sdt_h, int64_t sB_b, int64_t sB_l,
                                             int64_t sB_h, int64_t sC_b, int64_t sC_l,
                                             int64_t sC_h, int64_t sy_b, int64_t sy_l,
                                             int64_t sy_h, int64_t chunk) {
  SsdArgs a;
  int64_t nseg = 0;
  return ssd_fused_setup(dtype, x, dt, A_log, B, C, D, h0, y, h_last, nbatch, L, H, P, N, sx_b,
                         sx_l, sx_h, sdt_b, sdt_l, sdt_h, sB_b, sB_l, sB_h, sC_b, sC_l, sC_h,
                         sy_b, sy_l, sy_h, chunk, &a, &nseg) == TSSM_OK
             ? 1
             : 0;
}

extern "C" int tssm_ssd_scan_fused(int dtype, int disc, const void* x, const float* dt,
                                   const float* A_log, const void* B, const void* C,
                                   const float* D, const float* h0, void* y, float* h_last,
                                   int64_t nbatch, int64_t L, int64_t H, int64_t P, int64_t N,
                                   int64_t sx_b, int64_t sx_l, int64_t sx_h, int64_t sdt_b,
                                   int64_t sdt_l, int64_t sdt_h, int64_t sB_b, int64_t sB_l,
                                   int64_t sB_h, int64_t sC_b, int64_t sC_l, int64_t sC_h,
                                   int64_t sy_b, int64_t sy_l, int64_t sy_h, int64_t chunk,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  SsdArgs a;
  int64_t nseg = 0;
  const int rc = ssd_fused_setup(dtype, x, dt, A_log, B, C, D, h0, y, h_last, nbatch, L, H, P, N,
                                 sx_b, sx_l, sx_h, sdt_b, sdt_l, sdt_h, sB_b, sB_l, sB_h, sC_b,
                                 sC_l, sC_h, sy_b, sy_l, sy_h, chunk, &a, &nseg);
  if (rc != TSSM_OK) return rc;
  const int64_t need = tssm_ssd_scan_fused_workspace_bytes(nbatch, L, H, P, N, chunk);
  TSSM_CHECK(workspace && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 256), TSSM_ERR_ALIGN);
  const int64_t rows = (int64_t)a.rows;
  SsdLb lb;
  lb.hdr = reinterpret_cast<WsHeader*>(workspace);
  uint64_t* w = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + sizeof(WsHeader));
  lb.status = w;
  lb.dec = lb.status + 2 * rows * nseg;
  lb.agg = lb.dec + rows * nseg;
  lb.inc = lb.agg + rows * nseg * 64 * kSsdLbVals;
  lb.tag = next_epoch(workspace);
  lb.spin_limit = kDefaultSpinLimit;
  const uint32_t ngroups = (uint32_t)((rows + kWaveRows - 1) / kWaveRows);
  const dim3 gw((unsigned)(8 * ((nseg + 7) / 8) * ngroups));
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
#define TSSM_SF(DI, HD) \
  hipLaunchKernelGGL((ssd_fused_wave_kernel<DI, HD>), gw, dim3(256), 0, s, a, lb, ngroups)
  if (disc == TSSM_DISC_ZOH) {
    if (has_d) TSSM_SF(TSSM_DISC_ZOH, true); else TSSM_SF(TSSM_DISC_ZOH, false);
  } else {
    if (has_d) TSSM_SF(TSSM_DISC_EULER, true); else TSSM_SF(TSSM_DISC_EULER, false);
  }
#undef TSSM_SF
  return launch_status();
}

extern "C" int tssm_ssd_stream_step(int disc, const float* x, const float* dt, const float* A_log,
                                    const float* B, const float* C, const float* D, float* state,
                                    float* y, int64_t S, int64_t H, int64_t P, int64_t N,
                                    int64_t sdt_s, int64_t sdt_h, int64_t sx_s, int64_t sx_h,
                                    int64_t sB_s, int64_t sB_h, int64_t sC_s, int64_t sC_h,
                                    int64_t sy_s, int64_t sy_h, void* stream) {
  TSSM_CHECK(x && dt && A_log && B && C && state && y, TSSM_ERR_NULL);
  TSSM_CHECK(disc == TSSM_DISC_EULER || disc == TSSM_DISC_ZOH, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(S > 0 && H > 0 && P > 0 && N > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(N == 16 || N == 32 || N == 64 || N == 128 || N == 256, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(S * H < (int64_t)INT32_MAX, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(aligned(state, 16) && aligned(B, 16) && aligned(C, 16), TSSM_ERR_ALIGN);
  TSSM_CHECK(sB_s % 4 == 0 && sB_h % 4 == 0 && sC_s % 4 == 0 && sC_h % 4 == 0, TSSM_ERR_ALIGN);
  StreamArgs a{x, dt, A_log, B, C, D, state, y, H, P, N, sdt_s, sdt_h, sx_s, sx_h, sB_s, sB_h,
               sC_s, sC_h, sy_s, sy_h};
  const dim3 grid((unsigned)(S * H));
  const hipStream_t s = as_stream(stream);
  const bool zoh = disc == TSSM_DISC_ZOH, has_d = D != nullptr;
#define TSSM_ST(NGV)                                                                           \
  if (zoh) {                                                                                   \
    if (has_d) hipLaunchKernelGGL((ssd_stream_step_kernel<TSSM_DISC_ZOH, true, NGV>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((ssd_stream_step_kernel<TSSM_DISC_ZOH, false, NGV>), grid, dim3(256), 0, s, a);      \
  } else {                                                                                     \
    if (has_d) hipLaunchKernelGGL((ssd_stream_step_kernel<TSSM_DISC_EULER, true, NGV>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((ssd_stream_step_kernel<TSSM_DISC_EULER, false, NGV>), grid, dim3(256), 0, s, a);      \
  }
  switch (N) {
    case 16: TSSM_ST(4); break;
    case 32: TSSM_ST(8); break;
    case 64: TSSM_ST(16); break;
    case 128: TSSM_ST(32); break;
    default: TSSM_ST(64); break;
  }
#undef TSSM_ST
  return launch_status();
}
