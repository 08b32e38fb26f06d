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

constexpr float kRescaleFloor = 5.421010862427522e-20f;  // 2^-64
constexpr int kSsdSub = 16;  // steps staged per sub-block

// Per-step decay and input coefficient for steps [t0, t0+64) of one head,
// computed by lane i for step t0+i and shared through LDS.  Steps at or past
// L get dt = 0, i.e. decay 1 and coefficient 0, so they leave the state alone.
template <int DISC>
__device__ inline void step_scalars(const float* dtp, int64_t sdt_l, int64_t t0, int64_t L,
                                    float a2, float* s_ab, float* s_cf, int lane) {
  const int64_t t = t0 + lane;
  const float d = t < L ? dtp[t * sdt_l] : 0.0f;
  const float arg = d * a2;
  const float ab = exp2_fast(arg);
  s_ab[lane] = ab;
  s_cf[lane] = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(arg * 0.6931471805599453f, ab) * d : d;
}

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

// Stage rows [t0, t0+kSsdSub) of an N-wide operand into LDS as fp32
// (s[i*N + n]); rows at or past L read as zero.
template <typename T, int N>
__device__ inline void stage_rows(const T* __restrict__ base, int64_t sl, int64_t t0, int64_t L,
                                  float* s, int lane) {
#pragma unroll
  for (int k = lane; k < kSsdSub * N; k += 64) {
    const int i = k / N, n = k - (k / N) * N;
    const int64_t t = t0 + i;
    s[k] = t < L ? ldf(base + t * sl + n) : 0.0f;
  }
}

// Stage x_t[lane] for t in [t0, t0+kSsdSub) into s_x[i*64 + lane].
template <typename T>
__device__ inline void stage_x(const T* __restrict__ xp, int64_t sl, int64_t t0, int64_t L,
                               bool act, float* s_x, int lane) {
#pragma unroll
  for (int i = 0; i < kSsdSub; ++i) {
    const int64_t t = t0 + i;
    s_x[i * 64 + lane] = (act && t < L) ? ldf(xp + t * sl) : 0.0f;
  }
}

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
  float Pt = 1.0f, Achunk = 1.0f;
  for (int64_t t0 = tbeg; t0 < tend; t0 += 64) {
    step_scalars<DISC>(dtp, a.sdt_l, t0, a.L, a2, s_ab, s_cf, lane);
    for (int j = 0; j < 64 && t0 + j < tend; j += kSsdSub) {
      stage_x<T>(xp, a.sx_l, t0 + j, a.L, act, s_x, lane);
      stage_rows<T, N>(Bp, a.sB_l, t0 + j, a.L, s_B, lane);
      __syncthreads();
#pragma unroll 2
      for (int i = 0; i < kSsdSub; ++i) {
        const float ab = s_ab[j + i];
        float bv[N];
#pragma unroll
        for (int n = 0; n < N; ++n) bv[n] = s_B[i * N + n];
        rescaled_step<N>(g, Pt, ab, s_cf[j + i] * s_x[i * 64 + lane], bv);
        Achunk *= ab;
      }
      __syncthreads();
    }
  }
  const int64_t PN = (int64_t)P * N;
  if (act) {
    float* out = a.chunkX + ((int64_t)row * a.nchunks + c) * PN + (int64_t)lane * N;
#pragma unroll
    for (int n = 0; n < N; ++n) out[n] = Pt * g[n];
  }
  if (lane == 0) a.chunkA[(int64_t)row * a.nchunks + c] = Achunk;
}

// Pass 2: thread (entry e, segment sg) of a 1024-thread workgroup covering 64
// consecutive state entries of one row and 16 segments of its chunks.
constexpr int kPassEntries = 64, kPassSegs = 16;
__global__ __launch_bounds__(1024) void ssd_pass_kernel(SsdArgs a, int64_t PN) {
  __shared__ float s_a[kPassSegs][kPassEntries], s_x[kPassSegs][kPassEntries];
  const int el = threadIdx.x % kPassEntries;
  const int sg = threadIdx.x / kPassEntries;
  const int64_t nblk = (PN + kPassEntries - 1) / kPassEntries;
  const int64_t row = blockIdx.x / nblk;
  const int64_t e = (blockIdx.x - row * nblk) * kPassEntries + el;
  const bool act = e < PN;
  const int64_t nc = a.nchunks;
  const int64_t seg = (nc + kPassSegs - 1) / kPassSegs;
  const int64_t c0 = sg * seg, c1 = c0 + seg < nc ? c0 + seg : nc;
  const float* cA = a.chunkA + row * nc;
  const float* cX = a.chunkX + row * nc * PN + (act ? e : 0);
  float A = 1.0f, X = 0.0f;
  for (int64_t c = c0; c < c1; ++c) {
    const float ac = cA[c];
    X = __builtin_fmaf(ac, X, cX[c * PN]);
    A *= ac;
  }
  s_a[sg][el] = A;
  s_x[sg][el] = X;
  __syncthreads();
  float S = (act && a.h0) ? a.h0[row * PN + e] : 0.0f;
  for (int k = 0; k < sg; ++k) S = __builtin_fmaf(s_a[k][el], S, s_x[k][el]);
  float* en = a.entry + row * nc * PN + (act ? e : 0);
  for (int64_t c = c0; c < c1; ++c) {
    if (act) en[c * PN] = S;
    S = __builtin_fmaf(cA[c], S, cX[c * PN]);
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
  for (int64_t t0 = tbeg; t0 < tend; t0 += 64) {
    step_scalars<DISC>(dtp, a.sdt_l, t0, a.L, a2, s_ab, s_cf, lane);
    for (int j = 0; j < 64 && t0 + j < tend; j += kSsdSub) {
      const int64_t ts = t0 + j;
      stage_x<T>(xp, a.sx_l, ts, a.L, act, s_x, lane);
      stage_rows<T, N>(Bp, a.sB_l, ts, a.L, s_B, lane);
      stage_rows<T, N>(Cp, a.sC_l, ts, a.L, s_C, lane);
      __syncthreads();
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
  for (int64_t p0 = 0; p0 < a.P; p0 += RPP) {
    const int64_t p = p0 + rp;
    float acc = 0.0f;
    float xv = 0.0f;
    if (p < a.P) {
      xv = a.x[s * a.sx_s + h * a.sx_h + p];
      const float xs = cf * xv;
      f32x4* sp = reinterpret_cast<f32x4*>(st + p * a.N + ng * 4);
      f32x4 v = __builtin_nontemporal_load(sp);
      v.x = __builtin_fmaf(ab, v.x, xs * bq.x);
      v.y = __builtin_fmaf(ab, v.y, xs * bq.y);
      v.z = __builtin_fmaf(ab, v.z, xs * bq.z);
      v.w = __builtin_fmaf(ab, v.w, xs * bq.w);
      __builtin_nontemporal_store(v, sp);
      acc = cq.x * v.x + cq.y * v.y + cq.z * v.z + cq.w * v.w;
    }
    // sum over the NG threads of the row (aligned lane groups)
    for (int o = NG / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (ng == 0 && p < a.P) {
      if (HAS_D) acc = __builtin_fmaf(a.D[h * a.P + p], xv, acc);
      a.y[s * a.sy_s + h * a.sy_h + p] = acc;
    }
  }
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
  TSSM_CHECK(P <= 64 && (N == 8 || N == 16 || N == 32), TSSM_ERR_UNSUPPORTED);
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
  TSSM_CHECK(nchunks * rows < (int64_t)INT32_MAX, TSSM_ERR_UNSUPPORTED);
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
  switch (dtype) {
    case TSSM_BF16: return launch_ssd_t<bf16_t>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
    case TSSM_F16: return launch_ssd_t<f16_t>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
    default: return launch_ssd_t<float>(disc, has_d, (int)N, rows, nchunks, PN, s, a);
  }
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
