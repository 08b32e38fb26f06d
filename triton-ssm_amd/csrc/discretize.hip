// ZOH discretization (discretize_kernel.py:16-94).
//
// Abar = exp(dt*a), Bbar = expm1(dt*a) / (a + 1e-12) * B with a = -exp(A_log).
// Elementwise over (b, t, h): a workgroup covers 256 x 4 consecutive lanes h
// (16-byte accesses where aligned) of 8 rows (b, t), so B/Abar/Bbar rows are
// read and written coalesced and the per-lane constants are computed once.
// expm1 is evaluated accurately (phi1 series below |x| < 0.25) instead of the
// reference's exp(x)-1 / x+x^2/2 branch, which loses ~1e-4 relative accuracy
// for 1e-5 < |x| < 1e-3.
#include "common.h"

namespace tssm {

constexpr int kZohRows = 8;  // rows (b, t) per workgroup

// expm1(x) and exp(x) from the base-2 exponent y = x log2(e): exp(x) =
// exp2(y) (hardware); expm1 = x phi1(x) by phi1's Taylor series (degree 6, in
// y) for |x| < 0.25, else exp(x) - 1 (|exp(x) - 1| >= 0.22: no cancellation).
__device__ inline float expm1_base2(float x, float y, float ex) {
  float p = 2.2005043419116583e-05f;
  p = __builtin_fmaf(p, y, 2.222259691071407e-04f);
  p = __builtin_fmaf(p, y, 1.9236258215256953e-03f);
  p = __builtin_fmaf(p, y, 1.3876027166205394e-02f);
  p = __builtin_fmaf(p, y, 8.007550231970023e-02f);
  p = __builtin_fmaf(p, y, 0.34657359027997264f);
  p = __builtin_fmaf(p, y, 1.0f);
  return __builtin_fabsf(y) < 0.36067376022224085f ? x * p : ex - 1.0f;
}

// Workgroup = 256 threads x V lanes h over kZohRows rows (b, t): the per-lane
// constants a = -exp(A_log[h]), a log2(e) and 1/(a + 1e-12) are computed once
// per workgroup; dt is uniform per row.
template <typename TB, typename TO, int V>
__global__ __launch_bounds__(256) void zoh_discretize_kernel(
    const float* __restrict__ A_log, const TB* __restrict__ B, const float* __restrict__ dt,
    TO* __restrict__ Abar, TO* __restrict__ Bbar, int64_t grid_t, int64_t nrows, int64_t hc,
    int64_t sB_b, int64_t sB_t, int64_t sdt_b, int64_t sdt_t, int64_t sa_b, int64_t sa_t,
    int64_t sb_b, int64_t sb_t) {
  const int64_t h = ((int64_t)blockIdx.y * blockDim.x + threadIdx.x) * V;
  if (h >= hc) return;
  float a[V], a2[V], ia[V];
  {
    float al[V];
    ld_lanes<float, V>(A_log + h, al);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a[v] = -exp_acc(al[v]);
      a2[v] = a[v] * kLog2e;
      ia[v] = 1.0f / (a[v] + 1e-12f);
    }
  }
  const int64_t r0 = (int64_t)blockIdx.x * kZohRows;
  int64_t b = r0 / grid_t, t = r0 - b * grid_t;
  for (int k = 0; k < kZohRows && r0 + k < nrows; ++k) {
    const float d = dt[b * sdt_b + t * sdt_t];
    float bv[V], ab[V], bb[V];
    ld_lanes<TB, V>(B + b * sB_b + t * sB_t + h, bv);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float x = d * a[v], y = d * a2[v];
      ab[v] = exp2_fast(y);
      bb[v] = expm1_base2(x, y, ab[v]) * ia[v] * bv[v];
    }
    st_lanes<TO, V>(Abar + b * sa_b + t * sa_t + h, ab);
    st_lanes<TO, V>(Bbar + b * sb_b + t * sb_t + h, bb);
    if (++t == grid_t) {
      t = 0;
      ++b;
    }
  }
}

}  // namespace tssm

using namespace tssm;

extern "C" int tssm_zoh_discretize(int b_dtype, int out_dtype, const float* A_log, const void* B,
                                   const float* dt, void* Abar, void* Bbar, int64_t nbatch,
                                   int64_t T, int64_t H, int64_t grid_b, int64_t grid_t,
                                   int64_t h_cover, int64_t sB_b, int64_t sB_t, int64_t sdt_b,
                                   int64_t sdt_t, int64_t sa_b, int64_t sa_t, int64_t sb_b,
                                   int64_t sb_t, void* stream) {
  TSSM_CHECK(A_log && B && dt && Abar && Bbar, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && T >= 0 && H >= 0 && grid_b >= 0 && grid_t >= 0 && h_cover >= 0,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_b <= nbatch && grid_t <= T && h_cover <= H, TSSM_ERR_SHAPE);
  const int64_t nrows = grid_b * grid_t;
  if (nrows == 0 || h_cover == 0) return TSSM_OK;
  // 4 lanes per thread when every row and A_log allow 16-byte (fp32) or
  // 8-byte (16-bit) accesses
  const int64_t eb = b_dtype == TSSM_F32 ? 16 : 8, eo = out_dtype == TSSM_F32 ? 16 : 8;
  const bool v4 = h_cover % 4 == 0 && sB_b % 4 == 0 && sB_t % 4 == 0 && sa_b % 4 == 0 &&
                  sa_t % 4 == 0 && sb_b % 4 == 0 && sb_t % 4 == 0 && aligned(A_log, 16) &&
                  aligned(B, eb) && aligned(Abar, eo) && aligned(Bbar, eo);
  const int64_t nthr = v4 ? h_cover / 4 : h_cover;
  const int threads = nthr >= 256 ? 256 : (int)((nthr + 63) / 64 * 64);
  const int64_t n_rg = (nrows + kZohRows - 1) / kZohRows;
  const int64_t n_hb = (nthr + threads - 1) / threads;
  TSSM_CHECK(n_rg <= 2147483647 && n_hb <= 65535, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)n_rg, (unsigned)n_hb);
  const hipStream_t s = as_stream(stream);
#define TSSM_ZOH(TBT, TOT)                                                                      \
  if (v4)                                                                                       \
    hipLaunchKernelGGL((zoh_discretize_kernel<TBT, TOT, 4>), grid, dim3(threads), 0, s, A_log,  \
                       (const TBT*)B, dt, (TOT*)Abar, (TOT*)Bbar, grid_t, nrows, h_cover, sB_b, \
                       sB_t, sdt_b, sdt_t, sa_b, sa_t, sb_b, sb_t);                             \
  else                                                                                          \
    hipLaunchKernelGGL((zoh_discretize_kernel<TBT, TOT, 1>), grid, dim3(threads), 0, s, A_log,  \
                       (const TBT*)B, dt, (TOT*)Abar, (TOT*)Bbar, grid_t, nrows, h_cover, sB_b, \
                       sB_t, sdt_b, sdt_t, sa_b, sa_t, sb_b, sb_t)
#define TSSM_ZOH_OUT(TBT)                          \
  switch (out_dtype) {                             \
    case TSSM_F32: TSSM_ZOH(TBT, float); break;    \
    case TSSM_BF16: TSSM_ZOH(TBT, bf16_t); break;  \
    case TSSM_F16: TSSM_ZOH(TBT, f16_t); break;    \
    default: return TSSM_ERR_DTYPE;                \
  }
  switch (b_dtype) {
    case TSSM_F32: TSSM_ZOH_OUT(float); break;
    case TSSM_BF16: TSSM_ZOH_OUT(bf16_t); break;
    case TSSM_F16: TSSM_ZOH_OUT(f16_t); break;
    default: return TSSM_ERR_DTYPE;
  }
#undef TSSM_ZOH_OUT
#undef TSSM_ZOH
  return launch_status();
}

// ---------------------------------------------------------------- backward
// zoh_discretize_bwd_kernel (discretize_kernel.py:98-162), deterministic:
// the reference adds dA_log with atomics over (b, t) and makes ddt a race
// between a store (hblk 0) and atomics (:156-162).  Here
//   pass 1: workgroup (lane block of up to 256 threads x 4 lanes, group of 64
//           rows r = b*grid_t+t) writes dB, a per-lane partial of dA_log over
//           its rows and, per row, the partial of ddt over its lanes (wave
//           sums + one LDS pass);
//   pass 2: dA[h] += sum of the row-group partials, ddt[r] = sum of the lane-
//           block partials, both in a fixed order.
// The partials live in a caller workspace: [n_rg][hc] then [n_lb][nrows] f32.
namespace tssm {

constexpr int kBwdLanes = 256;   // lanes per workgroup (threads)
constexpr int kBwdRows = 64;     // rows per workgroup
static_assert(kBwdRows <= 64, "the final ddt sum takes one thread per row, and a narrow H "
                              "launches workgroups of only 64 threads");

// psi(x) = (x e^x - expm1(x)) / x^2 = sum_k x^k (k+1)/(k+2)!, the factor of
// d/da [expm1(dt a)/a] = dt^2 psi(dt a).  Series below |x| < 0.5 (the direct
// form cancels there), direct above.
__device__ inline float psi_from_exp(float x, float ex, float em1) {
  float p = 10.0f / 39916800.0f;
  p = __builtin_fmaf(p, x, 9.0f / 3628800.0f);
  p = __builtin_fmaf(p, x, 8.0f / 362880.0f);
  p = __builtin_fmaf(p, x, 7.0f / 40320.0f);
  p = __builtin_fmaf(p, x, 6.0f / 5040.0f);
  p = __builtin_fmaf(p, x, 5.0f / 720.0f);
  p = __builtin_fmaf(p, x, 4.0f / 120.0f);
  p = __builtin_fmaf(p, x, 3.0f / 24.0f);
  p = __builtin_fmaf(p, x, 2.0f / 6.0f);
  p = __builtin_fmaf(p, x, 0.5f);
  const float direct = (x * ex - em1) * __builtin_amdgcn_rcpf(x * x);
  return __builtin_fabsf(x) < 0.5f ? p : direct;
}

template <typename T, int V>
__global__ __launch_bounds__(kBwdLanes) void zoh_bwd_pass1_kernel(
    const float* __restrict__ A_log, const T* __restrict__ B, const float* __restrict__ dt,
    const T* __restrict__ Abar, const T* __restrict__ dAbar, const T* __restrict__ dBbar,
    T* __restrict__ dB, float* __restrict__ part_dA, float* __restrict__ part_ddt, int64_t grid_t,
    int64_t nrows, int64_t hc, int64_t sB_b, int64_t sB_t, int64_t sdt_b, int64_t sdt_t,
    int64_t sa_b, int64_t sa_t, int64_t sb_b, int64_t sb_t) {
  __shared__ float red[kBwdRows][kBwdLanes / 64];
  const int rg = blockIdx.x, lb = blockIdx.y;
  const int64_t h = ((int64_t)lb * blockDim.x + threadIdx.x) * V;
  const bool act = h < hc;
  const int64_t hs = act ? h : 0;  // inactive lanes compute on lane 0 and store nothing
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // per-lane constants: a = -exp(A_log), a log2(e), 1/(a + 1e-12), a^2/(a^2 + 1e-18)
  float a[V], a2[V], ia[V], fac[V], acc_dA[V];
  {
    float al[V];
    ld_lanes<float, V>(A_log + hs, al);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a[v] = -exp_acc(al[v]);
      a2[v] = a[v] * kLog2e;
      ia[v] = 1.0f / (a[v] + 1e-12f);
      const float aa = a[v] * a[v];
      fac[v] = aa / (aa + 1e-18f);
      acc_dA[v] = 0.0f;
    }
  }
  const int64_t r0 = (int64_t)rg * kBwdRows;
  int64_t b = r0 / grid_t, t = r0 - b * grid_t;
  for (int k = 0; k < kBwdRows; ++k) {
    if (r0 + k >= nrows) break;  // uniform over the workgroup
    float ddt = 0.0f;
    if (act) {
      const float d = dt[b * sdt_b + t * sdt_t];
      float bv[V], ab[V], gA[V], gB[V], db[V];
      ld_lanes<T, V>(B + b * sB_b + t * sB_t + h, bv);
      ld_lanes<T, V>(Abar + b * sa_b + t * sa_t + h, ab);
      ld_lanes<T, V>(dAbar + b * sa_b + t * sa_t + h, gA);
      ld_lanes<T, V>(dBbar + b * sb_b + t * sb_t + h, gB);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float x = d * a[v], y = d * a2[v];
        const float ex = exp2_fast(y);
        const float em1 = expm1_base2(x, y, ex);
        ddt += gA[v] * a[v] * ab[v] + gB[v] * ex * bv[v];                     // :130-140
        const float num = d * d * psi_from_exp(x, ex, em1) * fac[v];          // :146
        const float da = gA[v] * d * ab[v] + gB[v] * num * bv[v];             // :143-148
        acc_dA[v] = __builtin_fmaf(da, a[v], acc_dA[v]);                      // :151, :156
        db[v] = gB[v] * em1 * ia[v];                                          // :154, :157
      }
      st_lanes<T, V>(dB + b * sB_b + t * sB_t + h, db);
    }
    for (int o = 32; o > 0; o >>= 1) ddt += __shfl_xor(ddt, o);
    if (lane == 0) red[k][wave] = ddt;
    if (++t == grid_t) {
      t = 0;
      ++b;
    }
  }
  if (act) {
#pragma unroll
    for (int v = 0; v < V; ++v) part_dA[(int64_t)rg * hc + h + v] = acc_dA[v];
  }
  __syncthreads();
  if (threadIdx.x < kBwdRows) {
    const int64_t r = r0 + threadIdx.x;
    if (r < nrows) {
      float s = 0.0f;
      for (int w = 0; w < nw; ++w) s += red[threadIdx.x][w];
      part_ddt[(int64_t)lb * nrows + r] = s;
    }
  }
}

// dA[h] += sum over row groups of part_dA (workgroup = 64 lanes h x 16 waves;
// wave w sums the row groups g = w mod 16 in order, then the 16 wave sums are
// added in wave order); ddt[r] = sum over lane blocks of part_ddt.  Both
// orders are fixed, so results are deterministic.
constexpr int kRedWaves = 16;
constexpr int kRedBatch = 16;  // row-group partials a dA wave loads at once
__global__ __launch_bounds__(64 * kRedWaves) void zoh_bwd_pass2_kernel(
    const float* __restrict__ part_dA, const float* __restrict__ part_ddt, float* __restrict__ dA,
    float* __restrict__ ddt, int64_t grid_t, int64_t nrows, int64_t hc, int64_t n_rg,
    int64_t n_lb, int64_t sdt_b, int64_t sdt_t, int64_t n_hblk) {
  __shared__ float red[kRedWaves][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if ((int64_t)blockIdx.x < n_hblk) {  // uniform: a dA workgroup
    const int64_t h = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.0f;
    if (h < hc) {
      // kRedBatch row groups' partials loaded at once (indices past n_rg
      // re-read the batch's first), then added in the same order as one at
      // a time: g = wave, wave + kRedWaves, ...
      for (int64_t g0 = wave; g0 < n_rg; g0 += (int64_t)kRedWaves * kRedBatch) {
        float v[kRedBatch];
#pragma unroll
        for (int u = 0; u < kRedBatch; ++u) {
          const int64_t g = g0 + (int64_t)u * kRedWaves;
          v[u] = part_dA[(g < n_rg ? g : g0) * hc + h];
        }
#pragma unroll
        for (int u = 0; u < kRedBatch; ++u)
          s = g0 + (int64_t)u * kRedWaves < n_rg ? s + v[u] : s;
      }
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && h < hc) {
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < kRedWaves; ++w) tot += red[w][lane];
      dA[h] += tot;
    }
  } else {
    const int64_t r = ((int64_t)blockIdx.x - n_hblk) * (64 * kRedWaves) + threadIdx.x;
    if (r < nrows) {
      float s = 0.0f;
      for (int64_t g = 0; g < n_lb; ++g) s += part_ddt[g * nrows + r];
      const int64_t b = r / grid_t, t = r - b * grid_t;
      ddt[b * sdt_b + t * sdt_t] = s;
    }
  }
}

inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tssm

extern "C" int64_t tssm_zoh_discretize_bwd_workspace_bytes(int64_t grid_b, int64_t grid_t,
                                                           int64_t h_cover) {
  if (grid_b < 0 || grid_t < 0 || h_cover < 0) return -1;
  const int64_t nrows = grid_b * grid_t;
  const int64_t n_rg = cdiv64(nrows, kBwdRows), n_lb = cdiv64(h_cover, kBwdLanes);
  return (n_rg * h_cover + n_lb * nrows) * (int64_t)sizeof(float);
}

extern "C" int tssm_zoh_discretize_bwd(int dtype, const float* A_log, const void* B,
                                       const float* dt, const void* Abar, const void* dAbar,
                                       const void* dBbar, float* dA, void* dB, float* ddt,
                                       int64_t nbatch, int64_t T, int64_t H, int64_t grid_b,
                                       int64_t grid_t, int64_t h_cover, int64_t sB_b,
                                       int64_t sB_t, int64_t sdt_b, int64_t sdt_t, int64_t sa_b,
                                       int64_t sa_t, int64_t sb_b, int64_t sb_t, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(A_log && B && dt && Abar && dAbar && dBbar && dA && dB && ddt, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && T >= 0 && H >= 0 && grid_b >= 0 && grid_t >= 0 && h_cover >= 0,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_b <= nbatch && grid_t <= T && h_cover <= H, TSSM_ERR_SHAPE);
  const int64_t nrows = grid_b * grid_t;
  if (nrows == 0) return TSSM_OK;
  const int64_t need = tssm_zoh_discretize_bwd_workspace_bytes(grid_b, grid_t, h_cover);
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  // 4 lanes per thread when every row and A_log allow 16-byte (fp32) or
  // 8-byte (16-bit) accesses
  const int64_t ea = dtype == TSSM_F32 ? 16 : 8;
  const bool v4 = h_cover % 4 == 0 && sB_b % 4 == 0 && sB_t % 4 == 0 && sa_b % 4 == 0 &&
                  sa_t % 4 == 0 && sb_b % 4 == 0 && sb_t % 4 == 0 && aligned(A_log, 16) &&
                  aligned(B, ea) && aligned(Abar, ea) && aligned(dAbar, ea) &&
                  aligned(dBbar, ea) && aligned(dB, ea);
  const int V = v4 ? 4 : 1;
  const int64_t nthr = h_cover / V;
  const int threads = nthr >= kBwdLanes ? kBwdLanes : (int)(cdiv64(nthr, 64) * 64);
  const int64_t n_rg = cdiv64(nrows, kBwdRows);
  // lane blocks of threads * V lanes (never more than the workspace's 256-lane blocks)
  const int64_t n_lb = h_cover == 0 ? 0 : cdiv64(h_cover, (int64_t)threads * V);
  TSSM_CHECK(n_rg <= 2147483647 && n_lb <= 65535, TSSM_ERR_UNSUPPORTED);
  float* part_dA = reinterpret_cast<float*>(workspace);
  float* part_ddt = part_dA + n_rg * h_cover;
  const hipStream_t s = as_stream(stream);
  if (h_cover > 0) {
    const dim3 grid1((unsigned)n_rg, (unsigned)n_lb);
#define TSSM_ZOH_BWD(TT)                                                                        \
  if (v4)                                                                                        \
    hipLaunchKernelGGL((zoh_bwd_pass1_kernel<TT, 4>), grid1, dim3(threads), 0, s, A_log,         \
                       (const TT*)B, dt, (const TT*)Abar, (const TT*)dAbar, (const TT*)dBbar,    \
                       (TT*)dB, part_dA, part_ddt, grid_t, nrows, h_cover, sB_b, sB_t, sdt_b,    \
                       sdt_t, sa_b, sa_t, sb_b, sb_t);                                           \
  else                                                                                           \
    hipLaunchKernelGGL((zoh_bwd_pass1_kernel<TT, 1>), grid1, dim3(threads), 0, s, A_log,         \
                       (const TT*)B, dt, (const TT*)Abar, (const TT*)dAbar, (const TT*)dBbar,    \
                       (TT*)dB, part_dA, part_ddt, grid_t, nrows, h_cover, sB_b, sB_t, sdt_b,    \
                       sdt_t, sa_b, sa_t, sb_b, sb_t)
    switch (dtype) {
      case TSSM_F32: TSSM_ZOH_BWD(float); break;
      case TSSM_BF16: TSSM_ZOH_BWD(bf16_t); break;
      case TSSM_F16: TSSM_ZOH_BWD(f16_t); break;
      default: return TSSM_ERR_DTYPE;
    }
#undef TSSM_ZOH_BWD
    const int st = launch_status();
    if (st != TSSM_OK) return st;
  }
  // pass 2: dA workgroups first, then the ddt workgroups (no lanes: ddt = 0)
  const int64_t n_hblk = cdiv64(h_cover, 64);
  const int64_t n2 = n_hblk + cdiv64(nrows, 64 * kRedWaves);
  TSSM_CHECK(n2 <= 2147483647, TSSM_ERR_UNSUPPORTED);
  hipLaunchKernelGGL(zoh_bwd_pass2_kernel, dim3((unsigned)n2), dim3(64 * kRedWaves), 0, s,
                     part_dA, part_ddt, dA, ddt, grid_t, nrows, h_cover, n_rg, n_lb, sdt_b, sdt_t,
                     n_hblk);
  return launch_status();
}

// ---------------------------------------------------------------- dt projection
// dt_project_softplus_kernel (discretize_kernel.py:166-213, evident intent of
// :203): dt[b,t,h] = clamp(softplus(sum_r dt_raw[b,t,r] W[r,h] + bias[h]),
// DT_MIN, DT_MAX).  Workgroup = (lane block of 256 lanes h, group of 16 rows
// (b,t)); each thread keeps 8 rows of W for its lane in registers while the
// rows' dt_raw values (uniform over the workgroup) are broadcast, so W is read
// once per workgroup and dt_raw once per lane block.  Softplus is evaluated as
// max(x,0) + log1p(exp(-|x|)), equal to log(1+exp(x)) wherever that is finite;
// the clamp makes the overflow case agree too.
namespace tssm {

constexpr int kDtRows = 8;
constexpr int kDtRank = 8;

// Workgroup = 256 threads in 256 / LPR row groups of LPR threads (whole
// waves); a thread covers V consecutive lanes h (V = 4: 16-byte W, bias and
// output accesses) of kDtRows rows (b, t).  dt_raw values are uniform over a
// row group's waves (scalar loads); W rows are read in groups of kDtRank.
// Several row groups per workgroup keep short rows (H / V <= 128) from
// launching one-wave workgroups.
template <typename TO, int V, int LPR>
__global__ __launch_bounds__(256) void dt_project_kernel(
    const float* __restrict__ raw, const float* __restrict__ W, const float* __restrict__ bias,
    TO* __restrict__ out, int64_t grid_t, int64_t nrows, int64_t hc, int64_t rank,
    int64_t sr_b, int64_t sr_t, int64_t sw_r, int64_t so_b, int64_t so_t, float dt_min,
    float dt_max) {
  static_assert(LPR % 64 == 0 && 256 % LPR == 0, "row groups of whole waves");
  constexpr int NRG = 256 / LPR;
  const int rg = __builtin_amdgcn_readfirstlane((int)threadIdx.x / LPR);
  const int64_t h = ((int64_t)blockIdx.y * LPR + (int)threadIdx.x % LPR) * V;
  const bool act = h < hc;
  const int64_t hs = act ? h : 0;  // inactive lanes read lane 0 (in bounds), store nothing
  const int64_t r0 = ((int64_t)blockIdx.x * NRG + rg) * kDtRows;
  if (r0 >= nrows) return;  // whole waves; no barrier in this kernel
  const int nr = (int)((nrows - r0) < kDtRows ? (nrows - r0) : kDtRows);
  // offsets of rows r0 .. r0+kDtRows-1 = (b, t) walking t, wrapping into the
  // next batch (uniform: scalar registers)
  int64_t ro_in[kDtRows], ro_out[kDtRows];
  {
    int64_t bb = r0 / grid_t, tt = r0 - bb * grid_t;
#pragma unroll
    for (int k = 0; k < kDtRows; ++k) {
      ro_in[k] = bb * sr_b + tt * sr_t;
      ro_out[k] = bb * so_b + tt * so_t;
      if (++tt == grid_t) {
        tt = 0;
        ++bb;
      }
    }
  }
  float acc[kDtRows][V];
#pragma unroll
  for (int k = 0; k < kDtRows; ++k)
#pragma unroll
    for (int v = 0; v < V; ++v) acc[k][v] = 0.0f;
  for (int64_t q0 = 0; q0 < rank; q0 += kDtRank) {
    const bool full = q0 + kDtRank <= rank;  // uniform: unguarded raw loads
    float w[kDtRank][V];
#pragma unroll
    for (int i = 0; i < kDtRank; ++i) {
      const bool ok = q0 + i < rank;
      const float* wp = W + (ok ? q0 + i : 0) * sw_r + hs;
      if constexpr (V == 4) {
        const float4 q = *reinterpret_cast<const float4*>(wp);
        w[i][0] = ok ? q.x : 0.0f; w[i][1] = ok ? q.y : 0.0f;
        w[i][2] = ok ? q.z : 0.0f; w[i][3] = ok ? q.w : 0.0f;
      } else {
        w[i][0] = ok ? *wp : 0.0f;
      }
    }
    // every row's values of this rank group are loaded before any is used:
    // unconditional loads (rows past the end repeat the last row, columns past
    // rank repeat the last column and are zeroed), so they go out together
    float rv[kDtRows][kDtRank];
    if (full) {
#pragma unroll
      for (int k = 0; k < kDtRows; ++k) {
        const float* rp = raw + ro_in[k < nr ? k : nr - 1] + q0;
#pragma unroll
        for (int i = 0; i < kDtRank; ++i) rv[k][i] = rp[i];
      }
    } else {
      const int64_t lim = rank - 1 - q0;  // last column of this group, >= 0
#pragma unroll
      for (int k = 0; k < kDtRows; ++k) {
        const float* rp = raw + ro_in[k < nr ? k : nr - 1] + q0;
#pragma unroll
        for (int i = 0; i < kDtRank; ++i) {
          const float x = rp[i < lim ? i : lim];
          rv[k][i] = i <= lim ? x : 0.0f;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kDtRows; ++k)
#pragma unroll
      for (int i = 0; i < kDtRank; ++i)
#pragma unroll
        for (int v = 0; v < V; ++v) acc[k][v] = __builtin_fmaf(rv[k][i], w[i][v], acc[k][v]);
  }
  if (!act) return;
  float bv[V];
  if constexpr (V == 4) {
    const float4 q = *reinterpret_cast<const float4*>(bias + h);
    bv[0] = q.x; bv[1] = q.y; bv[2] = q.z; bv[3] = q.w;
  } else {
    bv[0] = bias[h];
  }
#pragma unroll
  for (int k = 0; k < kDtRows; ++k) {
    if (k < nr) {
      float sp[V];
#pragma unroll
      for (int v = 0; v < V; ++v)
        sp[v] = clamp_med3(softplus_fast(acc[k][v] + bv[v]), dt_min, dt_max);
      TO* op = out + ro_out[k] + h;
      if constexpr (V == 4 && sizeof(TO) == 4) {
        *reinterpret_cast<float4*>(op) = make_float4(sp[0], sp[1], sp[2], sp[3]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) stf(op + v, sp[v]);
      }
    }
  }
}

// Matrix-core form for 4-aligned operands: per 16 x 16 tile, out^T = W^T raw^T
// on v_mfma_f32_16x16x4_f32 (fp32 products and sums, like the FMA form).  A
// wave owns (batch b, 32 steps, 32 lanes h): 2 x 2 tiles, 4 MFMAs per tile
// and 16 rank columns.  Lane l = (li = l % 16, lj = l / 16): operand A is
// W^T[h0 + li][q], operand B raw^T[q][t0 + li], and at k-step s the MFMA
// index k = lj stands for rank column q = 4 lj + s, so lane l's raw values for
// one rank block are one 16-byte load.  The accumulator, seeded with the bias,
// gives lane l out[t0 + li][h0 + 4 lj + v], v = 0..3: softplus and clamp on
// the VALU and one 16-byte store.  Every load is clamped in bounds; tiles past grid_t
// or h_cover are computed and not stored.
constexpr int kDpTiles = 2;  // 16-row tiles and 16-lane tiles per wave (2 x 2 measured faster than 4 x 4)

template <typename TO>
__global__ __launch_bounds__(256) void dt_project_mfma_kernel(
    const float* __restrict__ raw, const float* __restrict__ W, const float* __restrict__ bias,
    TO* __restrict__ out, int64_t grid_b, int64_t grid_t, int64_t ntsb, int64_t hc,
    int64_t rank, int64_t sr_b, int64_t sr_t, int64_t sw_r, int64_t so_b, int64_t so_t,
    float dt_min, float dt_max) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wv >= grid_b * ntsb) return;  // whole waves; no barrier in this kernel
  const int64_t b = wv / ntsb;
  const int64_t t0 = (wv - b * ntsb) * (16 * kDpTiles);
  const int64_t h0 = (int64_t)blockIdx.y * (16 * kDpTiles);
  const int li = lane & 15, lj = lane >> 4;
  const float* rb = raw + b * sr_b;

  // the accumulators start from the bias of the lane's 4 h (h_cover % 4 == 0:
  // all 4 in range or none)
  f32x4 acc[kDpTiles][kDpTiles];
#pragma unroll
  for (int ct = 0; ct < kDpTiles; ++ct) {
    const int64_t h = h0 + 16 * ct + 4 * lj;
    const float4 bq = *reinterpret_cast<const float4*>(bias + (h < hc ? h : 0));
#pragma unroll
    for (int rt = 0; rt < kDpTiles; ++rt) acc[rt][ct] = f32x4{bq.x, bq.y, bq.z, bq.w};
  }

  for (int64_t q0 = 0; q0 < rank; q0 += 16) {
    // rank % 4 == 0: lane group lj's 4 columns are all in range or all out
    const bool qok = q0 + 4 * lj < rank;
    const int64_t qa = qok ? q0 + 4 * lj : 0;
    float wa[kDpTiles][4];
#pragma unroll
    for (int ct = 0; ct < kDpTiles; ++ct) {
      const int64_t h = h0 + 16 * ct + li;
      const float* wp = W + (h < hc ? h : hc - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float v = wp[(qa + s) * sw_r];
        wa[ct][s] = qok ? v : 0.0f;
      }
    }
    f32x4 rv[kDpTiles];
#pragma unroll
    for (int rt = 0; rt < kDpTiles; ++rt) {
      const int64_t t = t0 + 16 * rt + li;
      const f32x4 v =
          *reinterpret_cast<const f32x4*>(rb + (t < grid_t ? t : grid_t - 1) * sr_t + qa);
      rv[rt] = qok ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int rt = 0; rt < kDpTiles; ++rt)
#pragma unroll
        for (int ct = 0; ct < kDpTiles; ++ct)
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[ct][s], rv[rt][s], acc[rt][ct],
                                                              0, 0, 0);
  }

  // row by row, so the 64-byte pieces of one output line leave in consecutive
  // store instructions
  TO* ob = out + b * so_b + h0 + 4 * lj;
#pragma unroll
  for (int rt = 0; rt < kDpTiles; ++rt) {
    const int64_t t = t0 + 16 * rt + li;
    if (t >= grid_t) continue;
    TO* orow = ob + t * so_t;
#pragma unroll
    for (int ct = 0; ct < kDpTiles; ++ct) {
      if (h0 + 16 * ct + 4 * lj >= hc) continue;
      float sp[4];
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sp[v] = clamp_med3(softplus_fast(acc[rt][ct][v]), dt_min, dt_max);
      st_lanes<TO, 4>(orow + 16 * ct, sp);
    }
  }
}

}  // namespace tssm

extern "C" int tssm_dt_project_softplus(int out_dtype, const float* dt_raw, const float* W,
                                        const float* bias, void* dt_out, int64_t nbatch,
                                        int64_t T, int64_t H, int64_t rank, int64_t grid_b,
                                        int64_t grid_t, int64_t h_cover, int64_t sr_b,
                                        int64_t sr_t, int64_t sw_r, int64_t so_b, int64_t so_t,
                                        float dt_min, float dt_max, void* stream) {
  TSSM_CHECK(dt_raw && W && bias && dt_out, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && T >= 0 && H >= 0 && rank >= 0 && grid_b >= 0 && grid_t >= 0 &&
                 h_cover >= 0,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_b <= nbatch && grid_t <= T && h_cover <= H, TSSM_ERR_SHAPE);
  TSSM_CHECK(sr_b >= 0 && sr_t >= 0 && sw_r >= 0 && so_b >= 0 && so_t >= 0, TSSM_ERR_STRIDE);
  const int64_t nrows = grid_b * grid_t;
  if (nrows == 0 || h_cover == 0) return TSSM_OK;
  const int64_t n_rg = cdiv64(nrows, kDtRows);
  // 4 lanes per thread when every W row, bias and output row is 16-byte aligned
  const bool v4 = h_cover % 4 == 0 && sw_r % 4 == 0 && so_b % 4 == 0 && so_t % 4 == 0 &&
                  aligned(W, 16) && aligned(bias, 16) &&
                  aligned(dt_out, out_dtype == TSSM_F32 ? 16 : 8);
  // matrix cores when raw rows are 16-byte vectors of a rank that is a
  // multiple of 4 (and the 4-lane output conditions above hold)
  if (v4 && rank % 4 == 0 && rank > 0 && sr_b % 4 == 0 && sr_t % 4 == 0 && aligned(dt_raw, 16)) {
    const int64_t ntsb = cdiv64(grid_t, 16 * kDpTiles);
    const int64_t gx = cdiv64(grid_b * ntsb, 4), gy = cdiv64(h_cover, 16 * kDpTiles);
    TSSM_CHECK(gx <= 2147483647 && gy <= 65535, TSSM_ERR_UNSUPPORTED);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    const hipStream_t s = as_stream(stream);
#define TSSM_DTM(TT)                                                                           \
  hipLaunchKernelGGL(dt_project_mfma_kernel<TT>, grid, dim3(256), 0, s, dt_raw, W, bias,       \
                     (TT*)dt_out, grid_b, grid_t, ntsb, h_cover, rank, sr_b, sr_t, sw_r, so_b, \
                     so_t, dt_min, dt_max)
    switch (out_dtype) {
      case TSSM_F32: TSSM_DTM(float); break;
      case TSSM_BF16: TSSM_DTM(bf16_t); break;
      case TSSM_F16: TSSM_DTM(f16_t); break;
      default: return TSSM_ERR_DTYPE;
    }
#undef TSSM_DTM
    return launch_status();
  }
  const int64_t nthr = v4 ? h_cover / 4 : h_cover;
  const int lpr = nthr > 128 ? 256 : (nthr > 64 ? 128 : 64);  // threads per row group
  const int64_t gx = cdiv64(n_rg, 256 / lpr);
  TSSM_CHECK(gx <= 2147483647 && cdiv64(nthr, lpr) <= 65535, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)gx, (unsigned)cdiv64(nthr, lpr));
  const hipStream_t s = as_stream(stream);
#define TSSM_DTP(TT, VV, LP)                                                                   \
  hipLaunchKernelGGL((dt_project_kernel<TT, VV, LP>), grid, dim3(256), 0, s, dt_raw, W, bias,  \
                     (TT*)dt_out, grid_t, nrows, h_cover, rank, sr_b, sr_t, sw_r, so_b, so_t, \
                     dt_min, dt_max)
#define TSSM_DTP_L(TT, VV)                     \
  if (lpr == 64) TSSM_DTP(TT, VV, 64);         \
  else if (lpr == 128) TSSM_DTP(TT, VV, 128);  \
  else TSSM_DTP(TT, VV, 256)
  switch (out_dtype) {
    case TSSM_F32: if (v4) { TSSM_DTP_L(float, 4); } else { TSSM_DTP_L(float, 1); } break;
    case TSSM_BF16: if (v4) { TSSM_DTP_L(bf16_t, 4); } else { TSSM_DTP_L(bf16_t, 1); } break;
    case TSSM_F16: if (v4) { TSSM_DTP_L(f16_t, 4); } else { TSSM_DTP_L(f16_t, 1); } break;
    default: return TSSM_ERR_DTYPE;
  }
#undef TSSM_DTP_L
#undef TSSM_DTP
  return launch_status();
}
