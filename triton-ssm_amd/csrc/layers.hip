// Model layers around the scan: LayerNorm forward/backward and SwiGLU
// forward/backward (fused_ssm_interp.py:105-217), residual add and inverted
// dropout + residual (multihead_ssm_kernel.py:191-222), the mean-pool logit
// head and the padding mask (streaming_inference_kernel.py:160-214).
//
// All HBM-bound.  Row kernels (LayerNorm) give one wave per row, the row's
// elements strided over the 64 lanes so every load instruction reads 64
// consecutive elements; the 2-3 passes over a row re-read it from L1/L2.
// Elementwise kernels are flat grid-stride loops.  Reductions that the
// reference does with atomics (LayerNorm's dw/db, :169-170) are done in a
// fixed order instead, so results are deterministic:
//   layernorm_bwd_row_kernel   dx per row + the row's (mu, 1/sigma)
//   ln_param_partial_kernel    column partial sums of dout*xhat, dout over
//                              blocks of kLnRowBlock rows
//   ln_param_final_kernel      partials summed in block order, added to dw/db
// mean_pool_logit reduces each batch's T*H products over blocks of rows, then
// the block partials in order.
//
// Arithmetic is fp32 for every I/O dtype (fp32, bf16, fp16).
#include <initializer_list>

#include "common.h"

namespace tssm {
namespace {

constexpr int kThreads = 256;
constexpr int kLnRowBlock = 128;   // rows per column-partial block
constexpr int kPoolRows = 16;      // (t) rows per mean-pool block

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Row r of a (grid_b x grid_l) launch -> element offset of its first element.
struct Rows {
  int64_t grid_l, sb, sl;
  __device__ int64_t base(int64_t r) const {
    const int64_t b = r / grid_l, l = r - b * grid_l;
    return b * sb + l * sl;
  }
};

// mean and 1/sqrt(var + eps) of a row; `pad` = BLOCK_H - H masked lanes of
// the reference's block, which enter the variance as (0 - mu)^2.
template <typename T>
__device__ inline void row_stats(const T* x, int64_t H, int64_t pad, float eps, int lane,
                                 float* mu_out, float* inv_out) {
  float s = 0.0f;
  for (int64_t h = lane; h < H; h += 64) s += ldf(x + h);
  const float mu = wave_sum(s) / (float)H;
  float q = 0.0f;
  for (int64_t h = lane; h < H; h += 64) {
    const float c = ldf(x + h) - mu;
    q = __builtin_fmaf(c, c, q);
  }
  const float var = (wave_sum(q) + (float)pad * mu * mu) / (float)H;
  *mu_out = mu;
  *inv_out = 1.0f / sqrtf(var + eps);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void layernorm_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ out, Rows rows, int64_t nrow, int64_t H, int64_t pad, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = kThreads / 64;
  for (int64_t r = blockIdx.x * wpb + (threadIdx.x >> 6); r < nrow; r += (int64_t)gridDim.x * wpb) {
    const int64_t o = rows.base(r);
    float mu, inv;
    row_stats(x + o, H, pad, eps, lane, &mu, &inv);
    for (int64_t h = lane; h < H; h += 64)
      stf(out + o + h, __builtin_fmaf((ldf(x + o + h) - mu) * inv, ldf(w + h), ldf(bias + h)));
  }
}

// Rows held in registers: NV 4-lane vectors per lane (H <= 256 NV, H % 4 == 0,
// 16-byte / 8-byte aligned rows), so each row is read from HBM once.  Lane
// chunk j of a row covers elements 4 (lane + 64 j) .. +3.
template <typename T, int NV>
struct RowRegs {
  float v[NV][4];
  // chunks past H read chunk 0 (no branch around the loads); every use skips them
  __device__ inline void load(const T* row, int lane, int64_t H) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = 4 * (lane + 64 * (int64_t)j);
      ld_lanes<T, 4>(row + (e < H ? e : 0), v[j]);
    }
  }
};

template <typename T, int NV>
__device__ inline void row_stats_regs(const RowRegs<T, NV>& x, int lane, int64_t H, int64_t pad,
                                      float eps, float* mu_out, float* inv_out) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (4 * (lane + 64 * (int64_t)j) < H) s += (x.v[j][0] + x.v[j][1]) + (x.v[j][2] + x.v[j][3]);
  const float mu = wave_sum(s) / (float)H;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (4 * (lane + 64 * (int64_t)j) >= H) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = x.v[j][e] - mu;
      q = __builtin_fmaf(c, c, q);
    }
  }
  const float var = (wave_sum(q) + (float)pad * mu * mu) / (float)H;
  *mu_out = mu;
  *inv_out = 1.0f / sqrtf(var + eps);
}

template <typename T, int NV>
__global__ __launch_bounds__(kThreads) void layernorm_fwd_reg_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ out, Rows rows, int64_t nrow, int64_t H, int64_t pad, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = kThreads / 64;
  RowRegs<T, NV> wr, br;
  wr.load(w, lane, H);
  br.load(bias, lane, H);
  for (int64_t r = blockIdx.x * wpb + (threadIdx.x >> 6); r < nrow; r += (int64_t)gridDim.x * wpb) {
    const int64_t o = rows.base(r);
    RowRegs<T, NV> xr;
    xr.load(x + o, lane, H);
    float mu, inv;
    row_stats_regs(xr, lane, H, pad, eps, &mu, &inv);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = 4 * (lane + 64 * (int64_t)j);
      if (e >= H) continue;
      float ov[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        ov[k] = __builtin_fmaf((xr.v[j][k] - mu) * inv, wr.v[j][k], br.v[j][k]);
      st_lanes<T, 4>(out + o + e, ov);
    }
  }
}

// Backward with rows in registers: dx per row, and this wave's partial sums of
// dout*xhat and dout over its rows (row r = wave, wave + nwaves, ...) kept in
// registers and written to part[wave][H] / part[nwaves + wave][H].
template <typename T, int NV>
__global__ __launch_bounds__(kThreads) void layernorm_bwd_reg_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const T* __restrict__ w,
    T* __restrict__ dx, float* __restrict__ part, Rows rows, int64_t nrow, int64_t H,
    int64_t pad, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = kThreads / 64;
  const int64_t wv = blockIdx.x * wpb + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * wpb;
  RowRegs<T, NV> wr;
  wr.load(w, lane, H);
  float pw[NV][4], pb[NV][4];
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) pw[j][k] = pb[j][k] = 0.0f;
  for (int64_t r = wv; r < nrow; r += nwaves) {
    const int64_t o = rows.base(r);
    RowRegs<T, NV> xr, gr;
    xr.load(x + o, lane, H);
    gr.load(dout + o, lane, H);
    float mu, inv;
    row_stats_regs(xr, lane, H, pad, eps, &mu, &inv);
    float s_dxc = 0.0f, s_dx = 0.0f, s_xc = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (4 * (lane + 64 * (int64_t)j) >= H) continue;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float xc = xr.v[j][k] - mu;
        const float dxh = gr.v[j][k] * wr.v[j][k];
        s_dxc = __builtin_fmaf(dxh, xc, s_dxc);
        s_dx += dxh;
        s_xc += xc;
        pw[j][k] = __builtin_fmaf(gr.v[j][k], xc * inv, pw[j][k]);
        pb[j][k] += gr.v[j][k];
      }
    }
    s_dxc = wave_sum(s_dxc);
    s_dx = wave_sum(s_dx);
    s_xc = wave_sum(s_xc);
    const float dvar = s_dxc * -0.5f * inv * inv * inv;
    const float sum_m2xc = -2.0f * s_xc + 2.0f * (float)pad * mu;
    const float dmu = -inv * s_dx + dvar * sum_m2xc / (float)H;
    const float k2 = 2.0f * dvar / (float)H, k0 = dmu / (float)H;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = 4 * (lane + 64 * (int64_t)j);
      if (e >= H) continue;
      float dv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float xc = xr.v[j][k] - mu;
        dv[k] = __builtin_fmaf(gr.v[j][k] * wr.v[j][k], inv, __builtin_fmaf(k2, xc, k0));
      }
      st_lanes<T, 4>(dx + o + e, dv);
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t e = 4 * (lane + 64 * (int64_t)j);
    if (e >= H) continue;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      part[wv * H + e + k] = pw[j][k];
      part[(nwaves + wv) * H + e + k] = pb[j][k];
    }
  }
}

// dw[h] += sum_k part[k][h], db[h] += sum_k part[nblk + k][h] in two fixed-
// order levels (deterministic).  Level 1: workgroup (64 lanes h, split y) =
// 16 waves over the partials of split y, wave w taking k = k0 + w, k0 + w + 16,
// ...; the 16 wave sums are added in wave order into part2[y][h] (and
// part2[kSplits + y][h] for db).  Level 2: the kSplits sums in split order.
constexpr int kRedWaves = 16;
constexpr int kSplits = 16;
__global__ __launch_bounds__(64 * kRedWaves) void ln_param_reduce_kernel(
    const float* __restrict__ part, float* __restrict__ part2, int64_t H, int64_t nblk) {
  __shared__ float red[2][kRedWaves][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t h = (int64_t)blockIdx.x * 64 + lane;
  const int64_t per = (nblk + kSplits - 1) / kSplits;
  const int64_t k0 = (int64_t)blockIdx.y * per;
  const int64_t k1 = k0 + per < nblk ? k0 + per : nblk;
  float sw = 0.0f, sb = 0.0f;
  if (h < H) {
    for (int64_t k = k0 + wave; k < k1; k += kRedWaves) {
      sw += part[k * H + h];
      sb += part[(nblk + k) * H + h];
    }
  }
  red[0][wave][lane] = sw;
  red[1][wave][lane] = sb;
  __syncthreads();
  if (wave == 0 && h < H) {
    float tw = 0.0f, tb = 0.0f;
#pragma unroll
    for (int k = 0; k < kRedWaves; ++k) {
      tw += red[0][k][lane];
      tb += red[1][k][lane];
    }
    part2[blockIdx.y * H + h] = tw;
    part2[(kSplits + blockIdx.y) * H + h] = tb;
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void ln_param_add_kernel(const float* __restrict__ part2,
                                                                T* __restrict__ dw,
                                                                T* __restrict__ db, int64_t H) {
  const int64_t h = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (h >= H) return;
  float tw = 0.0f, tb = 0.0f;
#pragma unroll
  for (int k = 0; k < kSplits; ++k) {
    tw += part2[k * H + h];
    tb += part2[(kSplits + k) * H + h];
  }
  stf(dw + h, ldf(dw + h) + tw);
  stf(db + h, ldf(db + h) + tb);
}

// dx of a row (fused_ssm_interp.py:148-166) and its (mu, inv) for the
// parameter-gradient pass.
template <typename T>
__global__ __launch_bounds__(kThreads) void layernorm_bwd_row_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const T* __restrict__ w,
    T* __restrict__ dx, float* __restrict__ stats, Rows rows, int64_t nrow, int64_t H,
    int64_t pad, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = kThreads / 64;
  for (int64_t r = blockIdx.x * wpb + (threadIdx.x >> 6); r < nrow; r += (int64_t)gridDim.x * wpb) {
    const int64_t o = rows.base(r);
    float mu, inv;
    row_stats(x + o, H, pad, eps, lane, &mu, &inv);
    float s_dxc = 0.0f, s_dx = 0.0f, s_xc = 0.0f;
    for (int64_t h = lane; h < H; h += 64) {
      const float xc = ldf(x + o + h) - mu;
      const float dxh = ldf(dout + o + h) * ldf(w + h);
      s_dxc = __builtin_fmaf(dxh, xc, s_dxc);
      s_dx += dxh;
      s_xc += xc;
    }
    s_dxc = wave_sum(s_dxc);
    s_dx = wave_sum(s_dx);
    s_xc = wave_sum(s_xc);
    // (var + eps)^-1.5 = inv^3; the padded lanes hold xc = -mu
    const float dvar = s_dxc * -0.5f * inv * inv * inv;
    const float sum_m2xc = -2.0f * s_xc + 2.0f * (float)pad * mu;
    const float dmu = -inv * s_dx + dvar * sum_m2xc / (float)H;
    const float k2 = 2.0f * dvar / (float)H, k0 = dmu / (float)H;
    for (int64_t h = lane; h < H; h += 64) {
      const float xc = ldf(x + o + h) - mu;
      const float dxh = ldf(dout + o + h) * ldf(w + h);
      stf(dx + o + h, __builtin_fmaf(dxh, inv, __builtin_fmaf(k2, xc, k0)));
    }
    if (lane == 0) {
      stats[2 * r] = mu;
      stats[2 * r + 1] = inv;
    }
  }
}

// Column partials over row block blockIdx.y: part[blk][h] = sum dout*xhat,
// part[nblk + blk][h] = sum dout (rows in ascending order).
template <typename T>
__global__ __launch_bounds__(kThreads) void ln_param_partial_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const float* __restrict__ stats,
    float* __restrict__ part, Rows rows, int64_t nrow, int64_t H, int64_t nblk) {
  const int64_t h = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (h >= H) return;
  const int64_t r0 = (int64_t)blockIdx.y * kLnRowBlock;
  const int64_t r1 = r0 + kLnRowBlock < nrow ? r0 + kLnRowBlock : nrow;
  float sw = 0.0f, sb = 0.0f;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t o = rows.base(r) + h;
    const float d = ldf(dout + o);
    sw = __builtin_fmaf(d, (ldf(x + o) - stats[2 * r]) * stats[2 * r + 1], sw);
    sb += d;
  }
  part[blockIdx.y * H + h] = sw;
  part[(nblk + blockIdx.y) * H + h] = sb;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void ln_param_final_kernel(
    const float* __restrict__ part, T* __restrict__ dw, T* __restrict__ db, int64_t H,
    int64_t nblk) {
  const int64_t h = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (h >= H) return;
  float sw = 0.0f, sb = 0.0f;
  for (int64_t k = 0; k < nblk; ++k) {
    sw += part[k * H + h];
    sb += part[(nblk + k) * H + h];
  }
  stf(dw + h, ldf(dw + h) + sw);
  stf(db + h, ldf(db + h) + sb);
}

__device__ inline float sigmoid(float g) { return 1.0f / (1.0f + expf(-g)); }

// Row-elementwise launch: workgroup = 256 threads x V lanes h (grid y) over
// kRowsWG consecutive rows (grid x); the row's offset advances without a
// division per element.
constexpr int kRowsWG = 2;  // swiglu 69.0 -> 65.4 us cold against 4 rows
template <int V, typename F>
__device__ inline void for_rows(const Rows& rows, int64_t nrow, int64_t H, F&& f) {
  const int64_t h = ((int64_t)blockIdx.y * kThreads + threadIdx.x) * V;
  if (h >= H) return;
  const int64_t r0 = (int64_t)blockIdx.x * kRowsWG;
  int64_t b = r0 / rows.grid_l, l = r0 - b * rows.grid_l;
  for (int k = 0; k < kRowsWG && r0 + k < nrow; ++k) {
    f(r0 + k, b * rows.sb + l * rows.sl + h, h);
    if (++l == rows.grid_l) {
      l = 0;
      ++b;
    }
  }
}

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_kernel(
    const T* __restrict__ gate, const T* __restrict__ up, T* __restrict__ out, Rows rows,
    int64_t nrow, int64_t H) {
  for_rows<V>(rows, nrow, H, [&](int64_t, int64_t o, int64_t) {
    float g[V], u[V], y[V];
    ld_lanes<T, V>(gate + o, g);
    ld_lanes<T, V>(up + o, u);
#pragma unroll
    for (int v = 0; v < V; ++v) y[v] = g[v] * sigmoid(g[v]) * u[v];
    st_lanes<T, V>(out + o, y);
  });
}

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(
    const T* __restrict__ dout, const T* __restrict__ gate, const T* __restrict__ up,
    T* __restrict__ dgate, T* __restrict__ dup, Rows rows, int64_t nrow, int64_t H) {
  for_rows<V>(rows, nrow, H, [&](int64_t, int64_t o, int64_t) {
    float g[V], u[V], d[V], dg[V], du[V];
    ld_lanes<T, V>(gate + o, g);
    ld_lanes<T, V>(up + o, u);
    ld_lanes<T, V>(dout + o, d);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float sg = sigmoid(g[v]);
      du[v] = d[v] * g[v] * sg;
      dg[v] = d[v] * u[v] * sg * __builtin_fmaf(g[v], 1.0f - sg, 1.0f);
    }
    st_lanes<T, V>(dup + o, du);
    st_lanes<T, V>(dgate + o, dg);
  });
}

template <typename T>
__global__ __launch_bounds__(kThreads) void residual_kernel(
    const T* __restrict__ x, const T* __restrict__ res, const uint8_t* __restrict__ keep,
    T* __restrict__ out, int64_t n, float scale) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float xv = keep ? ldf(x + i) * (float)keep[i] * scale : ldf(x + i);
    stf(out + i, xv + ldf(res + i));
  }
}

// Dropout + residual with 4 elements per thread (16-byte fp32 / 8-byte 16-bit
// accesses, one 4-byte keep load): n % 4 == 0 and aligned pointers.  Same
// values as residual_kernel.
template <typename T>
__global__ __launch_bounds__(kThreads) void residual_vec_kernel(
    const T* __restrict__ x, const T* __restrict__ res, const uint8_t* __restrict__ keep,
    T* __restrict__ out, int64_t n4, float scale) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads) {
    float xv[4], rv[4], o[4];
    ld_lanes<T, 4>(x + 4 * i, xv);
    ld_lanes<T, 4>(res + 4 * i, rv);
    if (keep) {
      const uint32_t k = reinterpret_cast<const uint32_t*>(keep)[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = xv[j] * (float)((k >> (8 * j)) & 0xffu) * scale;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = xv[j] + rv[j];
    st_lanes<T, 4>(out + 4 * i, o);
  }
}

// Partial dot products of W with rows [blockIdx.y * kPoolRows, +kPoolRows) of
// batch blockIdx.x.
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void pool_partial_kernel(
    const T* __restrict__ h, const T* __restrict__ W, float* __restrict__ part, int64_t T_,
    int64_t H, int64_t sb, int64_t st, int64_t nblk) {
  __shared__ float s_w[kThreads / 64];
  const int64_t b = blockIdx.x;
  const int64_t t0 = (int64_t)blockIdx.y * kPoolRows;
  const int64_t t1 = t0 + kPoolRows < T_ ? t0 + kPoolRows : T_;
  float acc = 0.0f;
  for (int64_t k = (int64_t)threadIdx.x * V; k < H; k += (int64_t)kThreads * V) {
    float w[V];
    ld_lanes<T, V>(W + k, w);
    // all rows' loads in flight before the (in-order) accumulation; rows past
    // the block re-read its last row and are not accumulated
    float x[kPoolRows][V];
#pragma unroll
    for (int r = 0; r < kPoolRows; ++r) {
      const int64_t t = t0 + r < t1 ? t0 + r : t1 - 1;
      ld_lanes<T, V>(h + b * sb + t * st + k, x[r]);
    }
#pragma unroll
    for (int r = 0; r < kPoolRows; ++r) {
      if (t0 + r < t1) {
#pragma unroll
        for (int v = 0; v < V; ++v) acc = __builtin_fmaf(w[v], x[r][v], acc);
      }
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k) s += s_w[k];
    part[b * nblk + blockIdx.y] = s;
  }
}

// One wave per batch: lane j sums partials j, j + 64, ... in order, then the
// fixed-order wave reduction (deterministic).
template <typename T>
__global__ __launch_bounds__(64) void pool_final_kernel(const float* __restrict__ part,
                                                        const T* __restrict__ bias,
                                                        T* __restrict__ out, int64_t nblk,
                                                        float denom) {
  const int64_t b = blockIdx.x;
  const int lane = threadIdx.x;
  float s = 0.0f;
  for (int64_t k = lane; k < nblk; k += 64) s += part[b * nblk + k];
  s = wave_sum(s);
  if (lane == 0) stf(out + b, s / denom + ldf(bias));
}

// mask codes: 0 f32, 1 bf16, 2 f16 (the library's), 3 i32, 4 u8 / bool
__device__ inline bool mask_on(const void* m, int64_t i, int code) {
  switch (code) {
    case TSSM_F32: return reinterpret_cast<const float*>(m)[i] > 0.0f;
    case TSSM_BF16: return ldf(reinterpret_cast<const bf16_t*>(m) + i) > 0.0f;
    case TSSM_F16: return ldf(reinterpret_cast<const f16_t*>(m) + i) > 0.0f;
    case 3: return reinterpret_cast<const int32_t*>(m)[i] > 0;
    default: return reinterpret_cast<const uint8_t*>(m)[i] > 0;
  }
}

// Rows (b, t) of H contiguous elements; the row's mask value is uniform over
// the workgroup.  Elements at or past n (a partial last row) are not touched.
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void masked_fill_kernel(
    const T* __restrict__ x, const void* __restrict__ mask, int mcode, T* __restrict__ out,
    int64_t n, int64_t H) {
  const Rows rows{(n + H - 1) / H, 0, H};
  for_rows<V>(rows, rows.grid_l, H, [&](int64_t r, int64_t o, int64_t) {
    if (o >= n) return;  // V divides n, so a vector is whole or absent
    const bool on = mask_on(mask, r, mcode);
    float v[V];
    ld_lanes<T, V>(x + o, v);
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] = on ? v[k] : 0.0f;
    st_lanes<T, V>(out + o, v);
  });
}

// Grid of a flat loop over n items: enough workgroups to fill the chip, at
// most one item per thread.
inline unsigned flat_grid(int64_t n) {
  const int64_t g = (n + kThreads - 1) / kThreads;
  return (unsigned)(g < 8192 ? (g < 1 ? 1 : g) : 8192);
}
inline unsigned row_grid(int64_t nrow) {
  const int64_t g = (nrow + kThreads / 64 - 1) / (kThreads / 64);
  return (unsigned)(g < 8192 ? (g < 1 ? 1 : g) : 8192);
}
inline bool io_dtype(int d) { return d == TSSM_F32 || d == TSSM_BF16 || d == TSSM_F16; }

#define TSSM_DISPATCH(dtype, LAUNCH)            \
  switch (dtype) {                              \
    case TSSM_F32: { using T = float; LAUNCH; } break;   \
    case TSSM_BF16: { using T = bf16_t; LAUNCH; } break; \
    default: { using T = f16_t; LAUNCH; } break;         \
  }

// Rows of H elements allow 4-lane vectors: H and the row strides multiples of
// 4, base pointers 16-byte (fp32) / 8-byte (16-bit) aligned.
inline bool vec4_rows(int dtype, int64_t H, int64_t sb, int64_t sl,
                      std::initializer_list<const void*> ptrs) {
  if (H % 4 != 0 || sb % 4 != 0 || sl % 4 != 0) return false;
  const uintptr_t al = dtype == TSSM_F32 ? 16 : 8;
  for (const void* p : ptrs)
    if (!aligned(p, al)) return false;
  return true;
}
// Grid of for_rows: row groups on x, lane blocks of 256 V lanes on y.
inline dim3 rows_grid(int64_t nrow, int64_t H, int V) {
  const int64_t gy = (H + (int64_t)kThreads * V - 1) / ((int64_t)kThreads * V);
  const int64_t gx = (nrow + kRowsWG - 1) / kRowsWG;
  return dim3((unsigned)(gx < 1 ? 1 : gx), (unsigned)(gy < 1 ? 1 : gy));
}

// 4-lane vectors per lane for rows held in registers (0: rows do not qualify).
inline int reg_nv(int dtype, int64_t H, int64_t sb, int64_t sl,
                  std::initializer_list<const void*> ptrs) {
  if (H % 4 != 0 || H > 2048 || sb % 4 != 0 || sl % 4 != 0) return 0;
  const uintptr_t al = dtype == TSSM_F32 ? 16 : 8;
  for (const void* p : ptrs)
    if (!aligned(p, al)) return 0;
  const int64_t nv = (H + 255) / 256;
  return nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : 8;
}
constexpr int64_t kLnBwdMaxWaves = 2048;   // waves of the register backward (partial rows)

}  // namespace
}  // namespace tssm

using namespace tssm;

extern "C" int tssm_layernorm_fwd(int dtype, const void* x, const void* w, const void* bias,
                                  void* out, int64_t nbatch, int64_t L, int64_t H,
                                  int64_t stride_b, int64_t stride_l, float eps,
                                  int64_t block_h, int64_t grid_b, int64_t grid_l,
                                  void* stream) {
  TSSM_CHECK(x && w && bias && out, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(H > 0 && block_h >= H && grid_b >= 0 && grid_l >= 0 && grid_b <= nbatch &&
                 grid_l <= L, TSSM_ERR_SHAPE);
  TSSM_CHECK(stride_b >= 0 && stride_l >= 0, TSSM_ERR_STRIDE);
  const int64_t nrow = grid_b * grid_l;
  if (nrow == 0) return TSSM_OK;
  const Rows rows{grid_l, stride_b, stride_l};
  const hipStream_t s = as_stream(stream);
  const int nv = reg_nv(dtype, H, stride_b, stride_l, {x, w, bias, out});
#define TSSM_LN_REG(NV)                                                                   \
  hipLaunchKernelGGL((layernorm_fwd_reg_kernel<T, NV>), dim3(row_grid(nrow)), dim3(kThreads), \
                     0, s, (const T*)x, (const T*)w, (const T*)bias, (T*)out, rows, nrow, H,  \
                     block_h - H, eps)
  TSSM_DISPATCH(dtype, {
    switch (nv) {
      case 1: TSSM_LN_REG(1); break;
      case 2: TSSM_LN_REG(2); break;
      case 4: TSSM_LN_REG(4); break;
      case 8: TSSM_LN_REG(8); break;
      default:
        hipLaunchKernelGGL((layernorm_fwd_kernel<T>), dim3(row_grid(nrow)), dim3(kThreads), 0, s,
                           (const T*)x, (const T*)w, (const T*)bias, (T*)out, rows, nrow, H,
                           block_h - H, eps);
    }
  });
#undef TSSM_LN_REG
  return launch_status();
}

extern "C" int64_t tssm_layernorm_bwd_workspace_bytes(int64_t grid_b, int64_t grid_l, int64_t H) {
  if (grid_b < 0 || grid_l < 0 || H <= 0) return -1;
  const int64_t nrow = grid_b * grid_l;
  const int64_t nblk = (nrow + kLnRowBlock - 1) / kLnRowBlock;
  const int64_t rows_path = 2 * nrow + 2 * nblk * H;            // stats + column partials
  const int64_t reg_path = 2 * (kLnBwdMaxWaves + kSplits) * H;  // per-wave + split partials
  return (rows_path > reg_path ? rows_path : reg_path) * (int64_t)sizeof(float);
}

extern "C" int tssm_layernorm_bwd(int dtype, const void* dout, const void* x, const void* w,
                                  void* dx, void* dw, void* db, int64_t nbatch, int64_t L,
                                  int64_t H, int64_t stride_b, int64_t stride_l, float eps,
                                  int64_t block_h, int64_t grid_b, int64_t grid_l,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(dout && x && w && dx && dw && db, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(H > 0 && block_h >= H && grid_b >= 0 && grid_l >= 0 && grid_b <= nbatch &&
                 grid_l <= L, TSSM_ERR_SHAPE);
  TSSM_CHECK(stride_b >= 0 && stride_l >= 0, TSSM_ERR_STRIDE);
  const int64_t nrow = grid_b * grid_l;
  if (nrow == 0) return TSSM_OK;
  const int64_t need = tssm_layernorm_bwd_workspace_bytes(grid_b, grid_l, H);
  TSSM_CHECK(workspace && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 16), TSSM_ERR_ALIGN);
  const int64_t nblk = (nrow + kLnRowBlock - 1) / kLnRowBlock;
  TSSM_CHECK(nblk <= 65535, TSSM_ERR_UNSUPPORTED);
  float* stats = reinterpret_cast<float*>(workspace);
  float* part = stats + 2 * nrow;
  const Rows rows{grid_l, stride_b, stride_l};
  const hipStream_t s = as_stream(stream);
  const int nv = reg_nv(dtype, H, stride_b, stride_l, {dout, x, w, dx});
  if (nv > 0) {
    int64_t g = row_grid(nrow);
    if (g * (kThreads / 64) > kLnBwdMaxWaves) g = kLnBwdMaxWaves / (kThreads / 64);
    const int64_t nwaves = g * (kThreads / 64);
    float* wpart = reinterpret_cast<float*>(workspace);
    float* part2 = wpart + 2 * nwaves * H;
    const dim3 gred((unsigned)((H + 63) / 64), (unsigned)kSplits);
    const dim3 gadd((unsigned)((H + kThreads - 1) / kThreads));
#define TSSM_LNB_REG(NV)                                                                      \
  hipLaunchKernelGGL((layernorm_bwd_reg_kernel<T, NV>), dim3((unsigned)g), dim3(kThreads), 0, \
                     s, (const T*)dout, (const T*)x, (const T*)w, (T*)dx, wpart, rows, nrow, H,  \
                     block_h - H, eps)
    TSSM_DISPATCH(dtype, {
      switch (nv) {
        case 1: TSSM_LNB_REG(1); break;
        case 2: TSSM_LNB_REG(2); break;
        case 4: TSSM_LNB_REG(4); break;
        default: TSSM_LNB_REG(8); break;
      }
      hipLaunchKernelGGL(ln_param_reduce_kernel, gred, dim3(64 * kRedWaves), 0, s, wpart, part2,
                         H, nwaves);
      hipLaunchKernelGGL((ln_param_add_kernel<T>), gadd, dim3(kThreads), 0, s, part2, (T*)dw,
                         (T*)db, H);
    });
#undef TSSM_LNB_REG
    return launch_status();
  }
  const dim3 gcol((unsigned)((H + kThreads - 1) / kThreads), (unsigned)nblk);
  const dim3 gfin((unsigned)((H + kThreads - 1) / kThreads));
  TSSM_DISPATCH(dtype, {
    hipLaunchKernelGGL((layernorm_bwd_row_kernel<T>), dim3(row_grid(nrow)), dim3(kThreads), 0, s,
                       (const T*)dout, (const T*)x, (const T*)w, (T*)dx, stats, rows, nrow, H,
                       block_h - H, eps);
    hipLaunchKernelGGL((ln_param_partial_kernel<T>), gcol, dim3(kThreads), 0, s, (const T*)dout,
                       (const T*)x, stats, part, rows, nrow, H, nblk);
    hipLaunchKernelGGL((ln_param_final_kernel<T>), gfin, dim3(kThreads), 0, s, part, (T*)dw,
                       (T*)db, H, nblk);
  });
  return launch_status();
}

extern "C" int tssm_swiglu_fwd(int dtype, const void* gate, const void* up, void* out,
                               int64_t nbatch, int64_t L, int64_t H, int64_t stride_b,
                               int64_t stride_l, int64_t grid_b, int64_t grid_l, void* stream) {
  TSSM_CHECK(gate && up && out, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(H >= 0 && grid_b >= 0 && grid_l >= 0 && grid_b <= nbatch && grid_l <= L,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(stride_b >= 0 && stride_l >= 0, TSSM_ERR_STRIDE);
  const int64_t nrow = grid_b * grid_l;
  if (nrow == 0 || H == 0) return TSSM_OK;
  const Rows rows{grid_l, stride_b, stride_l};
  const int V = vec4_rows(dtype, H, stride_b, stride_l, {gate, up, out}) ? 4 : 1;
  const dim3 grid = rows_grid(nrow, H, V);
  const hipStream_t s = as_stream(stream);
  TSSM_DISPATCH(dtype, {
    if (V == 4)
      hipLaunchKernelGGL((swiglu_fwd_kernel<T, 4>), grid, dim3(kThreads), 0, s, (const T*)gate,
                         (const T*)up, (T*)out, rows, nrow, H);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<T, 1>), grid, dim3(kThreads), 0, s, (const T*)gate,
                         (const T*)up, (T*)out, rows, nrow, H);
  });
  return launch_status();
}

extern "C" int tssm_swiglu_bwd(int dtype, const void* dout, const void* gate, const void* up,
                               void* dgate, void* dup, int64_t nbatch, int64_t L, int64_t H,
                               int64_t stride_b, int64_t stride_l, int64_t grid_b,
                               int64_t grid_l, void* stream) {
  TSSM_CHECK(dout && gate && up && dgate && dup, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(H >= 0 && grid_b >= 0 && grid_l >= 0 && grid_b <= nbatch && grid_l <= L,
             TSSM_ERR_SHAPE);
  TSSM_CHECK(stride_b >= 0 && stride_l >= 0, TSSM_ERR_STRIDE);
  const int64_t nrow = grid_b * grid_l;
  if (nrow == 0 || H == 0) return TSSM_OK;
  const Rows rows{grid_l, stride_b, stride_l};
  const int V = vec4_rows(dtype, H, stride_b, stride_l, {dout, gate, up, dgate, dup}) ? 4 : 1;
  const dim3 grid = rows_grid(nrow, H, V);
  const hipStream_t s = as_stream(stream);
  TSSM_DISPATCH(dtype, {
    if (V == 4)
      hipLaunchKernelGGL((swiglu_bwd_kernel<T, 4>), grid, dim3(kThreads), 0, s, (const T*)dout,
                         (const T*)gate, (const T*)up, (T*)dgate, (T*)dup, rows, nrow, H);
    else
      hipLaunchKernelGGL((swiglu_bwd_kernel<T, 1>), grid, dim3(kThreads), 0, s, (const T*)dout,
                         (const T*)gate, (const T*)up, (T*)dgate, (T*)dup, rows, nrow, H);
  });
  return launch_status();
}

extern "C" int tssm_residual_add(int dtype, const void* x, const void* res, const uint8_t* keep,
                                 void* out, int64_t n, float p_keep, void* stream) {
  TSSM_CHECK(x && res && out, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(n >= 0, TSSM_ERR_SHAPE);
  if (n == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
  const float scale = 1.0f / p_keep;
  // dropout: 4 elements per thread (one 4-byte keep load) measured 97 -> 81 us
  // at 33.5 M fp32 elements; the plain add stays one element per thread (the
  // 4-element form measured 3 us slower there)
  const uintptr_t ve = dtype == TSSM_F32 ? 16 : 8;  // bytes of 4 elements
  if (keep && n % 4 == 0 && aligned(x, ve) && aligned(res, ve) && aligned(out, ve) &&
      aligned(keep, 4)) {
    TSSM_DISPATCH(dtype, hipLaunchKernelGGL((residual_vec_kernel<T>), dim3(flat_grid(n / 4)),
                                            dim3(kThreads), 0, s, (const T*)x, (const T*)res,
                                            keep, (T*)out, n / 4, scale));
    return launch_status();
  }
  TSSM_DISPATCH(dtype, hipLaunchKernelGGL((residual_kernel<T>), dim3(flat_grid(n)),
                                          dim3(kThreads), 0, s, (const T*)x, (const T*)res,
                                          keep, (T*)out, n, scale));
  return launch_status();
}

extern "C" int64_t tssm_mean_pool_logit_workspace_bytes(int64_t grid_b, int64_t T) {
  if (grid_b < 0 || T < 0) return -1;
  return grid_b * ((T + kPoolRows - 1) / kPoolRows) * (int64_t)sizeof(float);
}

extern "C" int tssm_mean_pool_logit(int dtype, const void* h, const void* W, const void* bias,
                                    void* out, int64_t nbatch, int64_t nt, int64_t H,
                                    int64_t stride_b, int64_t stride_t, int64_t grid_b,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(h && W && bias && out, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype), TSSM_ERR_DTYPE);
  TSSM_CHECK(nt > 0 && H > 0 && grid_b >= 0 && grid_b <= nbatch, TSSM_ERR_SHAPE);
  TSSM_CHECK(stride_b >= 0 && stride_t >= 0, TSSM_ERR_STRIDE);
  if (grid_b == 0) return TSSM_OK;
  const int64_t nblk = (nt + kPoolRows - 1) / kPoolRows;
  TSSM_CHECK(nblk <= 65535 && grid_b <= 2147483647, TSSM_ERR_UNSUPPORTED);
  TSSM_CHECK(workspace && workspace_bytes >= tssm_mean_pool_logit_workspace_bytes(grid_b, nt),
             TSSM_ERR_WORKSPACE);
  float* part = reinterpret_cast<float*>(workspace);
  // the reference divides in fp32 by (T * H + 1e-9)
  const float denom = (float)(nt * H) + 1e-9f;
  const hipStream_t s = as_stream(stream);
  TSSM_DISPATCH(dtype, {
    if (vec4_rows(dtype, H, stride_b, stride_t, {h, W}))
      hipLaunchKernelGGL((pool_partial_kernel<T, 4>), dim3((unsigned)grid_b, (unsigned)nblk),
                         dim3(kThreads), 0, s, (const T*)h, (const T*)W, part, nt, H, stride_b,
                         stride_t, nblk);
    else
      hipLaunchKernelGGL((pool_partial_kernel<T, 1>), dim3((unsigned)grid_b, (unsigned)nblk),
                         dim3(kThreads), 0, s, (const T*)h, (const T*)W, part, nt, H, stride_b,
                         stride_t, nblk);
    hipLaunchKernelGGL((pool_final_kernel<T>), dim3((unsigned)grid_b), dim3(64), 0, s, part,
                       (const T*)bias, (T*)out, nblk, denom);
  });
  return launch_status();
}

extern "C" int tssm_masked_fill_zero(int dtype, int mask_code, const void* x, const void* mask,
                                     void* out, int64_t n, int64_t H, void* stream) {
  TSSM_CHECK(x && mask && out, TSSM_ERR_NULL);
  TSSM_CHECK(io_dtype(dtype) && mask_code >= 0 && mask_code <= 4, TSSM_ERR_DTYPE);
  TSSM_CHECK(n >= 0 && H > 0, TSSM_ERR_SHAPE);
  if (n == 0) return TSSM_OK;
  const hipStream_t s = as_stream(stream);
  const int V = (n % 4 == 0 && vec4_rows(dtype, H, 0, 0, {x, out})) ? 4 : 1;
  const dim3 grid = rows_grid((n + H - 1) / H, H, V);
  TSSM_DISPATCH(dtype, {
    if (V == 4)
      hipLaunchKernelGGL((masked_fill_kernel<T, 4>), grid, dim3(kThreads), 0, s, (const T*)x,
                         mask, mask_code, (T*)out, n, H);
    else
      hipLaunchKernelGGL((masked_fill_kernel<T, 1>), grid, dim3(kThreads), 0, s, (const T*)x,
                         mask, mask_code, (T*)out, n, H);
  });
  return launch_status();
}
