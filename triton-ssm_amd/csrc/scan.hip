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
// row in fp32, rounded to the carry dtype on store.  A wave holds 64 / S rows of S = min(64, pow2 >= nblk)
// carries, lane = (row, carry k); one load round trip, then a segmented
// inclusive scan across the row's lanes (Hillis-Steele, log2 S shuffles,
// earlier carries on the left as in _combine), and one store.  Rows longer
// than 64 carries go in 64-carry segments, each started from the previous
// segment's last state.  reverse walks k = nblk-1 .. 0.  The first carry is
// kept as loaded, as in the sequential form; sums are reassociated like the
// reference's tree-shaped tl.associative_scan.
template <typename T, int S>
__global__ __launch_bounds__(256) void carry_scan_lanes_kernel(T* __restrict__ carry,
                                                               int64_t nrows, int64_t nblk,
                                                               int reverse, int64_t grid_rows) {
  constexpr int RPW = 64 / S;
  const int lane = threadIdx.x & 63;
  const int64_t r = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / S;
  const int j = lane % S;
  const bool row_ok = r < grid_rows;
  T* ca = carry + (row_ok ? r : 0) * nblk;
  T* cx = carry + nrows * nblk + (row_ok ? r : 0) * nblk;
  float Ain = 1.0f, Xin = 0.0f;  // state entering the segment
  for (int64_t i0 = 0; i0 < nblk; i0 += S) {
    const int64_t i = i0 + j;
    const bool ok = row_ok && i < nblk;
    const int64_t k = reverse ? nblk - 1 - (ok ? i : 0) : (ok ? i : 0);
    float A = ok ? ldf(ca + k) : 1.0f;
    float X = ok ? ldf(cx + k) : 0.0f;
#pragma unroll
    for (int d = 1; d < S; d <<= 1) {
      const float Al = __shfl_up(A, d, S), Xl = __shfl_up(X, d, S);
      if (j >= d) {
        X = __builtin_fmaf(A, Xl, X);
        A = A * Al;
      }
    }
    if (i0 > 0) {  // fold in the previous segments
      X = __builtin_fmaf(A, Xin, X);
      A = A * Ain;
    }
    if (ok && i > 0) {
      stf(ca + k, A);
      stf(cx + k, X);
    }
    if (i0 + S < nblk) {  // S == 64 here: the segment's last lane carries on
      Ain = __shfl(A, 63);
      Xin = __shfl(X, 63);
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
  // lanes over carries: rows of S lanes, 4 waves per workgroup
  int S = 1;
  while (S < 64 && S < nblk) S <<= 1;
  const int64_t rows_per_wg = 4 * (64 / S);
  const int64_t nwg = (grid_rows + rows_per_wg - 1) / rows_per_wg;
  TSSM_CHECK(nwg <= 2147483647, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)nwg);
#define TSSM_CS(T, SV)                                                                         \
  hipLaunchKernelGGL((carry_scan_lanes_kernel<T, SV>), grid, dim3(256), 0, s, (T*)carry,       \
                     nrows, nblk, reverse, grid_rows)
#define TSSM_C(T)                      \
  switch (S) {                         \
    case 1: TSSM_CS(T, 1); break;      \
    case 2: TSSM_CS(T, 2); break;      \
    case 4: TSSM_CS(T, 4); break;      \
    case 8: TSSM_CS(T, 8); break;      \
    case 16: TSSM_CS(T, 16); break;    \
    case 32: TSSM_CS(T, 32); break;    \
    default: TSSM_CS(T, 64); break;    \
  }
  TSSM_DISPATCH_T(dtype, TSSM_C)
#undef TSSM_C
#undef TSSM_CS
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
