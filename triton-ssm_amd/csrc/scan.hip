// Elementwise chunked linear scan, phase-exact (ssm_scan.py).
//
// h_t = A_t h_{t-1} + B_t u_t ; y_t = C_t h_t + D u_t over contiguous
// [B, L, H] tensors.  Each Triton program (row = b*H + h, chunk blk) becomes
// one thread; consecutive threads take consecutive lanes h, so every time
// step of a chunk is one coalesced row access.  Intermediates (loc_a, loc_x,
// carry [2, B*H, NBLK]) keep the reference layouts because callers can read
// them.  Arithmetic is fp32; loads/stores convert to the tensor dtype.
#include "common.h"

namespace tssm {

// thread -> (blk, b, h) with h fastest
struct RowMap {
  int64_t blk, b, h, rid;
};
__device__ inline bool map_row(int64_t i, int64_t nb, int64_t H, int64_t grid_rows,
                               int64_t grid_blks, RowMap* m) {
  const int64_t per_blk = nb * H;
  m->blk = i / per_blk;
  const int64_t r = i - m->blk * per_blk;
  m->b = r / H;
  m->h = r - m->b * H;
  m->rid = m->b * H + m->h;
  return m->blk < grid_blks && m->rid < grid_rows;
}

// ssm_fwd_local_kernel, ssm_scan.py:18-50
template <typename T>
__global__ void ssm_fwd_local_kernel(const T* __restrict__ u, const T* __restrict__ A,
                                     const T* __restrict__ Bm, T* __restrict__ loc_a,
                                     T* __restrict__ loc_x, T* __restrict__ carry, int64_t nb,
                                     int64_t L, int64_t H, int64_t blk_sz, int64_t nblk,
                                     int64_t grid_rows, int64_t grid_blks) {
  RowMap m;
  if (!map_row((int64_t)blockIdx.x * blockDim.x + threadIdx.x, nb, H, grid_rows, grid_blks, &m))
    return;
  const int64_t ts = m.blk * blk_sz;
  const int64_t te = ts + blk_sz > L ? L : ts + blk_sz;
  float ar = 1.0f, xr = 0.0f;
  for (int64_t p = ts; p < te; ++p) {
    const int64_t off = m.b * L * H + p * H + m.h;
    const float a = ldf(A + off);
    xr = a * xr + ldf(Bm + off) * ldf(u + off);
    ar = a * ar;
    stf(loc_a + off, ar);
    stf(loc_x + off, xr);
  }
  const int64_t nrows = nb * H;
  stf(carry + m.rid * nblk + m.blk, ar);
  stf(carry + nrows * nblk + m.rid * nblk + m.blk, xr);
}

// ssm_carry_scan_kernel (ssm_scan.py:54-65) and the reverse variant
// ssm_bwd_carry_scan_kernel (:174-185): inclusive scan of NBLK carries per
// row, sequential per thread in fp32, rounded to the carry dtype on store.
template <typename T>
__global__ void carry_scan_kernel(T* __restrict__ carry, int64_t nrows, int64_t nblk,
                                  int reverse, int64_t grid_rows) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= grid_rows) return;
  T* ca = carry + r * nblk;
  T* cx = carry + nrows * nblk + r * nblk;
  // kB carries per batch of loads, all issued before the batch is folded in;
  // reverse order walks k = nblk-1 .. 0.  The first carry is kept as loaded.
  constexpr int kB = 8;
  float A = 1.0f, X = 0.0f;
  for (int64_t k0 = 0; k0 < nblk; k0 += kB) {
    float av[kB], xv[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int64_t i = k0 + j < nblk ? k0 + j : nblk - 1;
      const int64_t k = reverse ? nblk - 1 - i : i;
      av[j] = ldf(ca + k);
      xv[j] = ldf(cx + k);
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (k0 + j >= nblk) break;
      const int64_t k = reverse ? nblk - 1 - (k0 + j) : k0 + j;
      X = __builtin_fmaf(av[j], X, xv[j]);
      A = av[j] * A;
      if (k0 + j > 0) {
        stf(ca + k, A);
        stf(cx + k, X);
      }
    }
  }
}

// ssm_fwd_apply_kernel, ssm_scan.py:69-98
template <typename T>
__global__ void ssm_fwd_apply_kernel(const T* __restrict__ loc_a, const T* __restrict__ loc_x,
                                     const T* __restrict__ carry, T* __restrict__ h_out,
                                     int64_t nb, int64_t L, int64_t H, int64_t blk_sz,
                                     int64_t nblk, int64_t grid_rows, int64_t grid_blks) {
  RowMap m;
  if (!map_row((int64_t)blockIdx.x * blockDim.x + threadIdx.x, nb, H, grid_rows, grid_blks, &m))
    return;
  const int64_t nrows = nb * H;
  const float x_p = m.blk == 0 ? 0.0f : ldf(carry + nrows * nblk + m.rid * nblk + m.blk - 1);
  const int64_t ts = m.blk * blk_sz;
  const int64_t te = ts + blk_sz > L ? L : ts + blk_sz;
  for (int64_t p = ts; p < te; ++p) {
    const int64_t off = m.b * L * H + p * H + m.h;
    stf(h_out + off, ldf(loc_a + off) * x_p + ldf(loc_x + off));
  }
}

// ssm_output_kernel, ssm_scan.py:102-124
template <typename T>
__global__ void ssm_output_kernel(const T* __restrict__ h, const T* __restrict__ C,
                                  const T* __restrict__ D, const T* __restrict__ u,
                                  T* __restrict__ y, int64_t nb, int64_t L, int64_t H,
                                  int64_t blk_sz, int64_t grid_rows, int64_t grid_blks) {
  RowMap m;
  if (!map_row((int64_t)blockIdx.x * blockDim.x + threadIdx.x, nb, H, grid_rows, grid_blks, &m))
    return;
  const float dv = ldf(D + m.h);
  const int64_t ts = m.blk * blk_sz;
  const int64_t te = ts + blk_sz > L ? L : ts + blk_sz;
  for (int64_t p = ts; p < te; ++p) {
    const int64_t off = m.b * L * H + p * H + m.h;
    stf(y + off, ldf(C + off) * ldf(h + off) + dv * ldf(u + off));
  }
}

// ssm_bwd_local_kernel, ssm_scan.py:136-170
template <typename T>
__global__ void ssm_bwd_local_kernel(const T* __restrict__ A, const T* __restrict__ C,
                                     const T* __restrict__ dY, T* __restrict__ loc_a,
                                     T* __restrict__ loc_dh, T* __restrict__ carry, int64_t nb,
                                     int64_t L, int64_t H, int64_t blk_sz, int64_t nblk,
                                     int64_t grid_rows, int64_t grid_blks) {
  RowMap m;
  if (!map_row((int64_t)blockIdx.x * blockDim.x + threadIdx.x, nb, H, grid_rows, grid_blks, &m))
    return;
  const int64_t ts = m.blk * blk_sz;
  const int64_t te = ts + blk_sz > L ? L : ts + blk_sz;
  float ar = 1.0f, xr = 0.0f;
  for (int64_t p = te - 1; p >= ts; --p) {
    const int64_t off = m.b * L * H + p * H + m.h;
    const float a1 = (p + 1 < L) ? ldf(A + off + H) : 0.0f;
    xr = a1 * xr + ldf(C + off) * ldf(dY + off);
    ar = a1 * ar;
    stf(loc_a + off, ar);
    stf(loc_dh + off, xr);
  }
  const int64_t nrows = nb * H;
  stf(carry + m.rid * nblk + m.blk, ar);
  stf(carry + nrows * nblk + m.rid * nblk + m.blk, xr);
}

// ssm_bwd_apply_kernel, ssm_scan.py:189-231
template <typename T>
__global__ void ssm_bwd_apply_kernel(const T* __restrict__ loc_a, const T* __restrict__ loc_dh,
                                     const T* __restrict__ carry, const T* __restrict__ u,
                                     const T* __restrict__ Bm, const T* __restrict__ h,
                                     const T* __restrict__ dY, T* __restrict__ du,
                                     T* __restrict__ dA, T* __restrict__ dB, T* __restrict__ dC,
                                     int64_t nb, int64_t L, int64_t H, int64_t blk_sz,
                                     int64_t nblk, int64_t grid_rows, int64_t grid_blks) {
  RowMap m;
  if (!map_row((int64_t)blockIdx.x * blockDim.x + threadIdx.x, nb, H, grid_rows, grid_blks, &m))
    return;
  const int64_t nrows = nb * H;
  const float x_p =
      m.blk == nblk - 1 ? 0.0f : ldf(carry + nrows * nblk + m.rid * nblk + m.blk + 1);
  const int64_t ts = m.blk * blk_sz;
  const int64_t te = ts + blk_sz > L ? L : ts + blk_sz;
  for (int64_t p = te - 1; p >= ts; --p) {
    const int64_t off = m.b * L * H + p * H + m.h;
    const float dh = ldf(loc_a + off) * x_p + ldf(loc_dh + off);
    const float hv = ldf(h + off);
    stf(dC + off, ldf(dY + off) * hv);
    stf(du + off, ldf(Bm + off) * dh);
    stf(dB + off, ldf(u + off) * dh);
    const float hp = p > 0 ? ldf(h + off - H) : 0.0f;
    stf(dA + off, hp * dh);
  }
}

inline unsigned blocks_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace tssm

using namespace tssm;

#define TSSM_DISPATCH_T(dtype, MACRO) \
  switch (dtype) {                    \
    case TSSM_F32: MACRO(float); break; \
    case TSSM_BF16: MACRO(bf16_t); break; \
    case TSSM_F16: MACRO(f16_t); break; \
    default: return TSSM_ERR_DTYPE;   \
  }

static int check_phase(int64_t nb, int64_t L, int64_t H, int64_t blk, int64_t nblk,
                       int64_t grid_rows, int64_t grid_blks) {
  TSSM_CHECK(nb > 0 && L > 0 && H > 0 && blk > 0 && nblk > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_rows >= 0 && grid_blks >= 0 && grid_rows <= nb * H && grid_blks <= nblk,
             TSSM_ERR_SHAPE);
  return TSSM_OK;
}

extern "C" int tssm_ssm_fwd_local(int dtype, const void* u, const void* A, const void* B,
                                  void* loc_a, void* loc_x, void* carry, int64_t nbatch,
                                  int64_t L, int64_t H, int64_t blk, int64_t nblk,
                                  int64_t grid_rows, int64_t grid_blks, void* stream) {
  TSSM_CHECK(u && A && B && loc_a && loc_x && carry, TSSM_ERR_NULL);
  int st = check_phase(nbatch, L, H, blk, nblk, grid_rows, grid_blks);
  if (st) return st;
  const int64_t n = grid_blks * nbatch * H;
  if (n == 0 || grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_L(T)                                                                              \
  hipLaunchKernelGGL(ssm_fwd_local_kernel<T>, dim3(blocks_for(n, 256)), dim3(256), 0, s,       \
                     (const T*)u, (const T*)A, (const T*)B, (T*)loc_a, (T*)loc_x, (T*)carry,   \
                     nbatch, L, H, blk, nblk, grid_rows, grid_blks)
  TSSM_DISPATCH_T(dtype, TSSM_L)
#undef TSSM_L
  return launch_status();
}

extern "C" int tssm_carry_scan(int dtype, void* carry, int64_t nrows, int64_t nblk, int reverse,
                               int64_t grid_rows, void* stream) {
  TSSM_CHECK(carry, TSSM_ERR_NULL);
  TSSM_CHECK(nrows > 0 && nblk > 0 && grid_rows >= 0 && grid_rows <= nrows, TSSM_ERR_SHAPE);
  if (grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_C(T)                                                                              \
  hipLaunchKernelGGL(carry_scan_kernel<T>, dim3(blocks_for(grid_rows, 64)), dim3(64), 0, s,    \
                     (T*)carry, nrows, nblk, reverse, grid_rows)
  TSSM_DISPATCH_T(dtype, TSSM_C)
#undef TSSM_C
  return launch_status();
}

extern "C" int tssm_ssm_fwd_apply(int dtype, const void* loc_a, const void* loc_x,
                                  const void* carry, void* h_out, int64_t nbatch, int64_t L,
                                  int64_t H, int64_t blk, int64_t nblk, int64_t grid_rows,
                                  int64_t grid_blks, void* stream) {
  TSSM_CHECK(loc_a && loc_x && carry && h_out, TSSM_ERR_NULL);
  int st = check_phase(nbatch, L, H, blk, nblk, grid_rows, grid_blks);
  if (st) return st;
  const int64_t n = grid_blks * nbatch * H;
  if (n == 0 || grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_A(T)                                                                              \
  hipLaunchKernelGGL(ssm_fwd_apply_kernel<T>, dim3(blocks_for(n, 256)), dim3(256), 0, s,       \
                     (const T*)loc_a, (const T*)loc_x, (const T*)carry, (T*)h_out, nbatch, L,  \
                     H, blk, nblk, grid_rows, grid_blks)
  TSSM_DISPATCH_T(dtype, TSSM_A)
#undef TSSM_A
  return launch_status();
}

extern "C" int tssm_ssm_output(int dtype, const void* h, const void* C, const void* D,
                               const void* u, void* y, int64_t nbatch, int64_t L, int64_t H,
                               int64_t blk, int64_t grid_rows, int64_t grid_blks, void* stream) {
  TSSM_CHECK(h && C && D && u && y, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch > 0 && L > 0 && H > 0 && blk > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_rows >= 0 && grid_blks >= 0 && grid_rows <= nbatch * H, TSSM_ERR_SHAPE);
  const int64_t n = grid_blks * nbatch * H;
  if (n == 0 || grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_O(T)                                                                              \
  hipLaunchKernelGGL(ssm_output_kernel<T>, dim3(blocks_for(n, 256)), dim3(256), 0, s,          \
                     (const T*)h, (const T*)C, (const T*)D, (const T*)u, (T*)y, nbatch, L, H,  \
                     blk, grid_rows, grid_blks)
  TSSM_DISPATCH_T(dtype, TSSM_O)
#undef TSSM_O
  return launch_status();
}

extern "C" int tssm_ssm_bwd_local(int dtype, const void* A, const void* C, const void* dY,
                                  void* loc_a, void* loc_dh, void* carry, int64_t nbatch,
                                  int64_t L, int64_t H, int64_t blk, int64_t nblk,
                                  int64_t grid_rows, int64_t grid_blks, void* stream) {
  TSSM_CHECK(A && C && dY && loc_a && loc_dh && carry, TSSM_ERR_NULL);
  int st = check_phase(nbatch, L, H, blk, nblk, grid_rows, grid_blks);
  if (st) return st;
  const int64_t n = grid_blks * nbatch * H;
  if (n == 0 || grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_BL(T)                                                                             \
  hipLaunchKernelGGL(ssm_bwd_local_kernel<T>, dim3(blocks_for(n, 256)), dim3(256), 0, s,       \
                     (const T*)A, (const T*)C, (const T*)dY, (T*)loc_a, (T*)loc_dh, (T*)carry, \
                     nbatch, L, H, blk, nblk, grid_rows, grid_blks)
  TSSM_DISPATCH_T(dtype, TSSM_BL)
#undef TSSM_BL
  return launch_status();
}

extern "C" int tssm_ssm_bwd_apply(int dtype, const void* loc_a, const void* loc_dh,
                                  const void* carry, const void* u, const void* A, const void* B,
                                  const void* h, const void* dY, void* du, void* dA, void* dB,
                                  void* dC, int64_t nbatch, int64_t L, int64_t H, int64_t blk,
                                  int64_t nblk, int64_t grid_rows, int64_t grid_blks,
                                  void* stream) {
  TSSM_CHECK(loc_a && loc_dh && carry && u && A && B && h && dY && du && dA && dB && dC,
             TSSM_ERR_NULL);
  int st = check_phase(nbatch, L, H, blk, nblk, grid_rows, grid_blks);
  if (st) return st;
  const int64_t n = grid_blks * nbatch * H;
  if (n == 0 || grid_rows == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
#define TSSM_BA(T)                                                                             \
  hipLaunchKernelGGL(ssm_bwd_apply_kernel<T>, dim3(blocks_for(n, 256)), dim3(256), 0, s,       \
                     (const T*)loc_a, (const T*)loc_dh, (const T*)carry, (const T*)u,          \
                     (const T*)B, (const T*)h, (const T*)dY, (T*)du, (T*)dA, (T*)dB, (T*)dC,   \
                     nbatch, L, H, blk, nblk, grid_rows, grid_blks)
  TSSM_DISPATCH_T(dtype, TSSM_BA)
#undef TSSM_BA
  return launch_status();
}
