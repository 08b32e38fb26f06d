// Time-aware interpolation (fused_interp_kernel.py) and the fused
// interpolation + one SSM step (fused_ssm_interp.py:12-101).
//
// Reference semantics kept exactly (they change results):
//  * "observed" is a per-(b, t, FTILE-wide tile) aggregate: the tile's mask
//    lanes summed > 0.5 (fused_interp_kernel.py:51-54);
//  * prev/next = nearest step within K on each side with an observed tile;
//  * w = clip((tau_t - tau_prev)/(tau_next - tau_prev), 0, 1), 0.5 when the
//    denominator <= 1e-9 (:80-83);
//  * vhat = interp / v_prev / v_next when a neighbour exists, else v_cur --
//    an observed current value is overwritten when any neighbour exists (:94-97).
//
// Two passes:
//  interp_obs_kernel: one wave per (b, t) row computes the row's "any lane
//    observed" flag of every feature tile once (M is read exactly once; the
//    reference re-reads each mask tile 2K+1 times) into a byte workspace
//    obs[b][t][tile];
//  interp_kernel: one workgroup per (b, tile, block of TB steps) resolves
//    neighbours and weights per step from the flags, then all (step, lane)
//    pairs of the block are interpolated at once, 16-byte vectors where the
//    layout allows.
#include "common.h"

namespace tssm {

constexpr int kInterpTB = 64;     // time steps per workgroup
constexpr int kInterpThreads = 256;
// The search window K sizes each kernel's LDS (flags and timestamps of the
// candidate rows), allocated at launch; a launch needing more than this per
// workgroup is refused (K up to ~6500 in every kernel, ~32000 in the offline one).
constexpr int64_t kMaxLds = 64 * 1024;
// Batches launch in slices of at most this many (a grid y/z dimension).
constexpr int64_t kMaxGridYZ = 65535;

// Sum of the tile's mask lanes for one row, by one wave.
__device__ inline float wave_tile_sum(const void* M, int md, int64_t row_off, int64_t f0,
                                      int64_t f1, int lane) {
  float s = 0.0f;
  for (int64_t f = f0 + lane; f < f1; f += 64) s += ld_any(M, row_off + f, md);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  return s;
}

struct InterpArgs {
  const void* V;
  const void* M;
  const void* tau;
  void* Vhat;
  unsigned char* obs;  // [grid_b][rows][ntile] flags
  int md, td;
  int64_t T, F, svb, svt, smb, smt, stb, stt, sob, sot;
  int64_t K, FTILE, grid_t, rows, ntile;
  int64_t b0;  // first batch of this launch (batches launch in slices)
};

__global__ __launch_bounds__(kInterpThreads) void interp_obs_kernel(InterpArgs a, int64_t nrow) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kInterpThreads / 64) + (threadIdx.x >> 6);
  if (r >= nrow) return;  // uniform per wave
  const int64_t b = r / a.rows, t = r - b * a.rows;
  for (int64_t tile = 0; tile < a.ntile; ++tile) {
    const int64_t f0 = tile * a.FTILE;
    const int64_t f1 = f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F;
    const float sum = wave_tile_sum(a.M, a.md, b * a.smb + t * a.smt, f0, f1, lane);
    if (lane == 0) a.obs[r * a.ntile + tile] = sum > 0.5f ? 1 : 0;
  }
}

// E consecutive feature lanes as floats: E = 4 (fp32) or 8 (16-bit) with one
// 16-byte access, or E = 1.
template <typename TV, int E> struct Lanes {
  float v[E];
  __device__ inline void load(const TV* p) {
    if constexpr (E == 1) {
      v[0] = ldf(p);
    } else if constexpr (sizeof(TV) == 4) {
      const float4 q = *reinterpret_cast<const float4*>(p);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
      Vec8<TV> q;
      q.load(p);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = q.get(j);
    }
  }
  __device__ inline void store(TV* p) const {
    if constexpr (E == 1) {
      stf(p, v[0]);
    } else if constexpr (sizeof(TV) == 4) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) stf(p + j, v[j]);
    }
  }
};

// Vectorized flags: each wave walks rows of E-lane vectors (16 bytes per
// lane), all loads of kObsU (row, block) items issued before any reduction.
// A row's tile sums come from a segmented inclusive scan across the wave
// keyed by tile index, carried between 64-vector blocks of one row; the lane
// holding a tile's last vector writes its flag.  Needs FTILE % E == 0 and
// E-aligned rows.
constexpr int kObsRowsPerWave = 4;
constexpr int kObsU = 4;

template <typename TM, int E>
__global__ __launch_bounds__(kInterpThreads) void interp_obs_vec_kernel(InterpArgs a,
                                                                       int64_t nrow) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * (kInterpThreads / 64) + (threadIdx.x >> 6);
  const int64_t r0 = w * kObsRowsPerWave;
  if (r0 >= nrow) return;  // uniform per wave
  const int64_t fc = a.F < a.ntile * a.FTILE ? a.F : a.ntile * a.FTILE;
  const int64_t nvec = fc / E, vpt = a.FTILE / E;
  const int64_t nblk = (nvec + 63) / 64;
  const int64_t nr = nrow - r0 < kObsRowsPerWave ? nrow - r0 : kObsRowsPerWave;
  const int64_t total = nr * nblk;
  const TM* M = reinterpret_cast<const TM*>(a.M);
  float carry = 0.0f;
  int64_t carry_tile = -1;
  for (int64_t i0 = 0; i0 < total; i0 += kObsU) {
    float s[kObsU];
    int64_t vv[kObsU], rr[kObsU];
#pragma unroll
    for (int u = 0; u < kObsU; ++u) {
      const int64_t item = i0 + u;
      const int64_t rl = (int)item / (int)nblk;  // both below 2^31 (launcher checks)
      const int64_t r = r0 + rl;
      const int64_t v = (item - rl * nblk) * 64 + lane;
      const bool ok = item < total && v < nvec;
      const int64_t b = r / a.rows, t = r - b * a.rows;
      // out-of-range lanes read the first vector instead (always in bounds)
      const int64_t off = ok ? b * a.smb + t * a.smt + v * E : 0;
      Lanes<TM, E> q;
      q.load(M + off);
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < E; ++j) sum += q.v[j];
      s[u] = ok ? sum : 0.0f;
      vv[u] = ok ? v : -1;
      rr[u] = r;
    }
#pragma unroll
    for (int u = 0; u < kObsU; ++u) {
      if (i0 + u >= total) break;  // uniform per wave
      const int64_t v = vv[u];
      const int64_t tile = v >= 0 ? (int)v / (int)vpt : -1;
      if ((int)(i0 + u) % (int)nblk == 0) carry_tile = -1;  // a new row starts
      float x = s[u];
      if (lane == 0 && tile == carry_tile) x += carry;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float xo = __shfl_up(x, o);
        const int64_t to = __shfl_up(tile, o);
        if (lane >= o && to == tile) x += xo;
      }
      const bool last = v >= 0 && ((v + 1) % vpt == 0 || v == nvec - 1);
      if (last) a.obs[rr[u] * a.ntile + tile] = x > 0.5f ? 1 : 0;
      carry = __shfl(x, 63);
      carry_tile = __shfl(tile, 63);
    }
  }
}

// Tiles of vpt = 2^lvpt 16-byte vectors (vpt <= 64) line up with aligned
// vpt-lane groups of a 64-vector block, so a tile's sum is the lanes' vector
// sums reduced over their group (xor shuffles) and the group's first lane
// writes the flag.  A wave takes kObsP2Rows (row, block) items per batch, all
// loads issued first; the row's (b, t) advance as wave-uniform counters.
constexpr int kObsP2Rows = 4;

template <typename TM, int E>
__global__ __launch_bounds__(kInterpThreads) void interp_obs_pow2_kernel(InterpArgs a,
                                                                        int64_t nrow, int lvpt) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * (kInterpThreads / 64) +
                    __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int64_t r0 = w * kObsP2Rows;
  if (r0 >= nrow) return;  // uniform per wave
  const int64_t fc = a.F < a.ntile * a.FTILE ? a.F : a.ntile * a.FTILE;
  const int64_t nvec = fc / E;
  const int nblk = (int)((nvec + 63) / 64);
  const int nr = (int)(nrow - r0 < kObsP2Rows ? nrow - r0 : kObsP2Rows);
  const int total = nr * nblk;
  const int vpt = 1 << lvpt;
  const TM* M = reinterpret_cast<const TM*>(a.M);
  int64_t b = r0 / a.rows, t = r0 - b * a.rows;  // (b, t) of the next item's row
  int64_t r = r0;
  int blk = 0;
  for (int i0 = 0; i0 < total; i0 += kObsP2Rows) {
    float s[kObsP2Rows];
    int64_t vv[kObsP2Rows], rr[kObsP2Rows];
#pragma unroll
    for (int u = 0; u < kObsP2Rows; ++u) {
      const int64_t v = (int64_t)blk * 64 + lane;
      const bool ok = i0 + u < total && v < nvec;
      // lanes past the row or the batch read the first vector (in bounds)
      const int64_t off = ok ? b * a.smb + t * a.smt + v * E : 0;
      Lanes<TM, E> q;
      q.load(M + off);
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < E; ++j) sum += q.v[j];
      s[u] = ok ? sum : 0.0f;
      vv[u] = ok ? v : -1;
      rr[u] = r;
      if (++blk == nblk) {  // uniform: next row
        blk = 0;
        ++r;
        if (++t == a.rows) {
          t = 0;
          ++b;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kObsP2Rows; ++u) {
      float x = s[u];
      for (int o = 1; o < vpt; o <<= 1) x += __shfl_xor(x, o);
      if (vv[u] >= 0 && (lane & (vpt - 1)) == 0)
        a.obs[rr[u] * a.ntile + (vv[u] >> lvpt)] = x > 0.5f ? 1 : 0;
    }
  }
}

template <typename TV, int E>
__global__ __launch_bounds__(kInterpThreads) void interp_kernel(InterpArgs a) {
  extern __shared__ unsigned char s_obs[];  // [kInterpTB + 2K]
  __shared__ int s_prev[kInterpTB], s_next[kInterpTB];
  __shared__ float s_w[kInterpTB];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * kInterpTB;
  const int64_t tile = blockIdx.y;
  const int64_t b = a.b0 + blockIdx.z;
  const int64_t f0 = tile * a.FTILE;
  const int64_t f1 = f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F;
  const int K = (int)a.K;
  // 1. flags of rows t0-K .. t0+TB+K-1 (rows outside [0, T) are unobserved)
  for (int i = tid; i < kInterpTB + 2 * K; i += kInterpThreads) {
    const int64_t t = t0 - K + i;
    s_obs[i] = (t >= 0 && t < a.rows) ? a.obs[(b * a.rows + t) * a.ntile + tile] : 0;
  }
  __syncthreads();
  // 2. neighbours and weight per step
  if (tid < kInterpTB) {
    const int64_t t = t0 + tid;
    int prev = -1, next = -1;
    float w = 0.5f;
    if (t < a.grid_t) {
      for (int k = 1; k <= K; ++k)
        if (prev < 0 && s_obs[tid + K - k]) prev = (int)(t - k);
      for (int k = 1; k <= K; ++k)
        if (next < 0 && s_obs[tid + K + k]) next = (int)(t + k);
      const float tau_t = ld_any(a.tau, b * a.stb + t * a.stt, a.td);
      const float tp = prev >= 0 ? ld_any(a.tau, b * a.stb + prev * a.stt, a.td) : 0.0f;
      const float tn = next >= 0 ? ld_any(a.tau, b * a.stb + next * a.stt, a.td) : 0.0f;
      const float den = tn - tp;
      w = den > 1e-9f ? (tau_t - tp) / den : 0.5f;
      w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
    }
    s_prev[tid] = prev;
    s_next[tid] = next;
    s_w[tid] = w;
  }
  __syncthreads();
  // 3. all (step, lane group) pairs of the block, U per thread per batch with
  // every load issued before the stores
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb;
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob;
  const int tmax = (int)((a.grid_t - t0) < kInterpTB ? (a.grid_t - t0) : kInterpTB);
  const int ng = (int)((f1 - f0) / E);  // lane groups per step (E divides the tile)
  const int total = tmax * ng;
  constexpr int U = 2;  // 27.0 us at the a12 shape cold (U = 4: 27.7, U = 8: 27.0)
  for (int q0 = tid; q0 < total; q0 += U * kInterpThreads) {
    Lanes<TV, E> vp[U], vn[U];
    int64_t ot[U], of[U];
    float wt[U];
    int mode[U];  // bit 0: prev exists, bit 1: next exists; -1: no pair
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kInterpThreads;
      mode[u] = -1;
      if (q < total) {
        const int i = q / ng;
        const int64_t f = f0 + (int64_t)(q - i * ng) * E;
        const int prev = s_prev[i], next = s_next[i];
        const int64_t t = t0 + i;
        // row read as "prev" (v_prev, else v_next, else v_cur) and as "next"
        const int64_t rp = prev >= 0 ? prev : (next >= 0 ? next : t);
        const int64_t rn = next >= 0 ? next : rp;
        vp[u].load(V + rp * a.svt + f);
        vn[u].load(V + rn * a.svt + f);
        mode[u] = (prev >= 0 ? 1 : 0) | (next >= 0 ? 2 : 0);
        wt[u] = s_w[i];
        ot[u] = t;
        of[u] = f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (mode[u] < 0) continue;
      Lanes<TV, E> o;
#pragma unroll
      for (int j = 0; j < E; ++j)
        o.v[j] = mode[u] == 3 ? lerp_pair(vp[u].v[j], vn[u].v[j], wt[u]) : vp[u].v[j];
      o.store(O + ot[u] * a.sot + of[u]);
    }
  }
}

// interp_obs_pow2_kernel and interp_kernel in one launch: a workgroup forms
// the flags of its tile's rows t0-K .. t0+TB+K-1 itself from M (same per-lane
// vector sums and xor reduction over the tile's aligned lane group as the
// flags kernel, so the same flags), keeps them in LDS and interpolates as
// interp_kernel.  M is read (TB + 2K) / TB times instead of once, but the
// flags' round trip through memory and a launch are gone.  Needs the
// conditions of both vector paths: tiles of vpt = FTILE / EM mask vectors
// with vpt a power of two <= 64, E-aligned V/Vhat rows.
constexpr int kFusedU = 4;  // mask vectors per lane in flight

template <typename TV, int E, typename TM, int EM>
__global__ __launch_bounds__(kInterpThreads) void interp_fused_kernel(InterpArgs a, int lvpt) {
  extern __shared__ unsigned char s_obs[];  // [kInterpTB + 2K]
  __shared__ int s_prev[kInterpTB], s_next[kInterpTB];
  __shared__ float s_w[kInterpTB];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * kInterpTB;
  const int64_t tile = blockIdx.y;
  const int64_t b = a.b0 + blockIdx.z;
  const int64_t f0 = tile * a.FTILE;
  const int64_t f1 = f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F;
  const int K = (int)a.K;
  const int NR = kInterpTB + 2 * K;
  // 1. flags: item q = (row q >> lvpt, vector q & (vpt - 1)) of the tile
  {
    const int vpt = 1 << lvpt;
    const int nitem = NR << lvpt;
    const TM* M = reinterpret_cast<const TM*>(a.M) + b * a.smb + f0;
    for (int q0 = tid; q0 < nitem; q0 += kFusedU * kInterpThreads) {
      float sv[kFusedU];
#pragma unroll
      for (int u = 0; u < kFusedU; ++u) {
        const int q = q0 + u * kInterpThreads;
        const int i = q >> lvpt, j = q & (vpt - 1);
        const int64_t t = t0 - K + i;
        const bool ok = q < nitem && t >= 0 && t < a.rows && f0 + (int64_t)j * EM < f1;
        Lanes<TM, EM> v;
        v.load(M + (ok ? t * a.smt + (int64_t)j * EM : 0));  // invalid items read vector 0
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < EM; ++k) sum += v.v[k];
        sv[u] = ok ? sum : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kFusedU; ++u) {
        const int q = q0 + u * kInterpThreads;  // uniform per wave in whether q < nitem
        float x = sv[u];
        for (int o = 1; o < vpt; o <<= 1) x += __shfl_xor(x, o);
        if (q < nitem && (q & (vpt - 1)) == 0) s_obs[q >> lvpt] = x > 0.5f ? 1 : 0;
      }
    }
  }
  __syncthreads();
  // 2. neighbours and weight per step (as interp_kernel)
  if (tid < kInterpTB) {
    const int64_t t = t0 + tid;
    int prev = -1, next = -1;
    float w = 0.5f;
    if (t < a.grid_t) {
      for (int k = 1; k <= K; ++k)
        if (prev < 0 && s_obs[tid + K - k]) prev = (int)(t - k);
      for (int k = 1; k <= K; ++k)
        if (next < 0 && s_obs[tid + K + k]) next = (int)(t + k);
      const float tau_t = ld_any(a.tau, b * a.stb + t * a.stt, a.td);
      const float tp = prev >= 0 ? ld_any(a.tau, b * a.stb + prev * a.stt, a.td) : 0.0f;
      const float tn = next >= 0 ? ld_any(a.tau, b * a.stb + next * a.stt, a.td) : 0.0f;
      const float den = tn - tp;
      w = den > 1e-9f ? (tau_t - tp) / den : 0.5f;
      w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
    }
    s_prev[tid] = prev;
    s_next[tid] = next;
    s_w[tid] = w;
  }
  __syncthreads();
  // 3. interpolation (as interp_kernel)
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb;
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob;
  const int tmax = (int)((a.grid_t - t0) < kInterpTB ? (a.grid_t - t0) : kInterpTB);
  const int ng = (int)((f1 - f0) / E);
  const int total = tmax * ng;
  constexpr int U = 2;
  for (int q0 = tid; q0 < total; q0 += U * kInterpThreads) {
    Lanes<TV, E> vp[U], vn[U];
    int64_t ot[U], of[U];
    float wt[U];
    int mode[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kInterpThreads;
      mode[u] = -1;
      if (q < total) {
        const int i = q / ng;
        const int64_t f = f0 + (int64_t)(q - i * ng) * E;
        const int prev = s_prev[i], next = s_next[i];
        const int64_t t = t0 + i;
        const int64_t rp = prev >= 0 ? prev : (next >= 0 ? next : t);
        const int64_t rn = next >= 0 ? next : rp;
        vp[u].load(V + rp * a.svt + f);
        vn[u].load(V + rn * a.svt + f);
        mode[u] = (prev >= 0 ? 1 : 0) | (next >= 0 ? 2 : 0);
        wt[u] = s_w[i];
        ot[u] = t;
        of[u] = f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (mode[u] < 0) continue;
      Lanes<TV, E> o;
#pragma unroll
      for (int j = 0; j < E; ++j)
        o.v[j] = mode[u] == 3 ? lerp_pair(vp[u].v[j], vn[u].v[j], wt[u]) : vp[u].v[j];
      o.store(O + ot[u] * a.sot + of[u]);
    }
  }
}

// interp_fused_kernel with the workgroup's global loads issued in two rounds
// instead of one per loop iteration and phase: first every mask vector of the
// tile's rows t0-K .. t0+TB+K-1 (flags formed exactly as there) and the
// timestamps of those rows (kept in LDS for the weights), then both
// neighbours' V of every (step, vector) item of the thread.  No load sits
// behind a branch (the compiler would sink it there and wait for it alone).
// Same results as interp_fused_kernel.  LDS: tau [TB+2K] floats, flags
// [TB+2K] bytes.
constexpr int kBatMU = 12;  // mask vectors per thread in the first round

template <typename TV, int E, typename TM, int EM>
__global__ __launch_bounds__(kInterpThreads) void interp_batched_kernel(InterpArgs a, int lvpt) {
  extern __shared__ __align__(16) unsigned char s_dyn[];
  __shared__ int s_prev[kInterpTB], s_next[kInterpTB];
  __shared__ float s_w[kInterpTB];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * kInterpTB;
  const int64_t tile = blockIdx.y;
  const int64_t b = a.b0 + blockIdx.z;
  const int64_t f0 = tile * a.FTILE;
  const int64_t f1 = f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F;
  const int K = (int)a.K;
  const int NR = kInterpTB + 2 * K;
  float* s_tau = reinterpret_cast<float*>(s_dyn);
  unsigned char* s_obs = s_dyn + (size_t)NR * 4;
  const TM* M = reinterpret_cast<const TM*>(a.M) + b * a.smb + f0;
  const int vpt = 1 << lvpt;
  const int nitem = NR << lvpt;

  // 1. mask vectors and timestamps.  Invalid items read the tile's first
  // vector of row 0 (in bounds) and count zero.
  auto m_item = [&](int q) {
    const int i = q >> lvpt, j = q & (vpt - 1);
    const int64_t t = t0 - K + i;
    const bool ok = q < nitem && t >= 0 && t < a.rows && f0 + (int64_t)j * EM < f1;
    Lanes<TM, EM> v;
    v.load(M + (ok ? t * a.smt + (int64_t)j * EM : 0));
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < EM; ++k) s += v.v[k];
    return ok ? s : 0.0f;
  };
  {
    float sv[kBatMU];
#pragma unroll
    for (int u = 0; u < kBatMU; ++u) sv[u] = m_item(tid + u * kInterpThreads);
    const int64_t rt = t0 - K + tid;
    const bool tok = tid < NR && rt >= 0 && rt < a.rows;
    const float tv = ld_any_nb(a.tau, b * a.stb + (tok ? rt : 0) * a.stt, a.td);
    // tile sums: the xor butterfly of interp_fused_kernel, level by level
    // over all items so that each level's exchanges issue together
    for (int o = 1; o < vpt; o <<= 1)
#pragma unroll
      for (int u = 0; u < kBatMU; ++u) sv[u] += __shfl_xor(sv[u], o);
#pragma unroll
    for (int u = 0; u < kBatMU; ++u) {
      const int q = tid + u * kInterpThreads;
      if (q < nitem && (q & (vpt - 1)) == 0) s_obs[q >> lvpt] = sv[u] > 0.5f ? 1 : 0;
    }
    if (tid < NR) s_tau[tid] = tok ? tv : 0.0f;
  }
  // items beyond the first round (wide tiles or large K); q0 - tid is
  // uniform, so every lane takes part in the exchanges
  for (int q0 = tid + kBatMU * kInterpThreads; q0 - tid < nitem; q0 += kInterpThreads) {
    float x = m_item(q0);
    for (int o = 1; o < vpt; o <<= 1) x += __shfl_xor(x, o);
    if (q0 < nitem && (q0 & (vpt - 1)) == 0) s_obs[q0 >> lvpt] = x > 0.5f ? 1 : 0;
  }
  for (int i = tid + kInterpThreads; i < NR; i += kInterpThreads) {
    const int64_t r = t0 - K + i;
    s_tau[i] = (r >= 0 && r < a.rows) ? ld_any(a.tau, b * a.stb + r * a.stt, a.td) : 0.0f;
  }
  __syncthreads();
  // 2. neighbours and weight per step (as interp_fused_kernel, timestamps from LDS)
  if (tid < kInterpTB) {
    const int64_t t = t0 + tid;
    int prev = -1, next = -1;
    float w = 0.5f;
    if (t < a.grid_t) {
      // nearest first, without a branch per flag (the reads issue together)
#pragma unroll 8
      for (int k = 1; k <= K; ++k) {
        const int fp = s_obs[tid + K - k], fn = s_obs[tid + K + k];
        prev = (prev < 0 && fp) ? (int)(t - k) : prev;
        next = (next < 0 && fn) ? (int)(t + k) : next;
      }
      const float tau_t = s_tau[tid + K];
      const float tp = prev >= 0 ? s_tau[prev - (t0 - K)] : 0.0f;
      const float tn = next >= 0 ? s_tau[next - (t0 - K)] : 0.0f;
      const float den = tn - tp;
      w = den > 1e-9f ? (tau_t - tp) / den : 0.5f;
      w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
    }
    s_prev[tid] = prev;
    s_next[tid] = next;
    s_w[tid] = w;
  }
  __syncthreads();
  // 3. interpolation, every item's two loads issued before the first use
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb + f0;
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob + f0;
  const int tmax = (int)((a.grid_t - t0) < kInterpTB ? (a.grid_t - t0) : kInterpTB);
  const int ng = (int)((f1 - f0) / E);
  const int total = tmax * ng;
  constexpr int U = 32 / E;  // 32 values of each neighbour in flight per thread
  for (int q0 = tid; q0 < total; q0 += U * kInterpThreads) {
    Lanes<TV, E> vp[U], vn[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kInterpThreads;
      const int i = q < total ? q / ng : 0;  // items past the end load row t0's first vector
      const int j = q < total ? q - i * ng : 0;
      const int prev = s_prev[i], next = s_next[i];
      const int64_t rp = prev >= 0 ? prev : (next >= 0 ? next : t0 + i);
      const int64_t rn = next >= 0 ? next : rp;
      vp[u].load(V + rp * a.svt + (int64_t)j * E);
      vn[u].load(V + rn * a.svt + (int64_t)j * E);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = q0 + u * kInterpThreads;
      if (q >= total) continue;
      const int i = q / ng, j = q - (q / ng) * ng;
      const bool both = s_prev[i] >= 0 && s_next[i] >= 0;
      const float w = s_w[i];
      Lanes<TV, E> o;
#pragma unroll
      for (int e = 0; e < E; ++e)
        o.v[e] = both ? lerp_pair(vp[u].v[e], vn[u].v[e], w) : vp[u].v[e];
      o.store(O + (t0 + i) * a.sot + (int64_t)j * E);
    }
  }
}

// fused_interp_ssm_step_kernel: one workgroup per (b, tile) at step t_cur.
struct StepArgs {
  const void* V;
  const void* M;
  const void* tau;
  const float* A_bar;
  const float* B_bar;
  const float* h_in;
  void* Vhat;
  float* h_out;
  int md, td;
  int64_t nb, T, F, svb, svt, smb, smt, stb, stt, sob, sot, s_hib, s_hob;
  int64_t t_cur, K, FTILE;
  int64_t b0;  // first batch of this launch (batches launch in slices)
};

template <typename TV>
__global__ __launch_bounds__(kInterpThreads) void interp_step_kernel(StepArgs a) {
  extern __shared__ unsigned char s_obs[];  // [2K + 1]
  __shared__ int s_pn[2];
  __shared__ float s_w;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t b = a.b0 + blockIdx.y;
  const int64_t f0 = tile * a.FTILE;
  const int64_t f1 = f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F;
  const int K = (int)a.K;
  for (int i = wave; i < 2 * K + 1; i += kInterpThreads / 64) {
    const int64_t t = a.t_cur - K + i;
    bool obs = false;
    if (t >= 0 && t < a.T) obs = wave_tile_sum(a.M, a.md, b * a.smb + t * a.smt, f0, f1, lane) > 0.5f;
    if (lane == 0) s_obs[i] = obs ? 1 : 0;
  }
  __syncthreads();
  if (tid == 0) {
    int prev = -1, next = -1;
    for (int k = 1; k <= K; ++k)
      if (prev < 0 && s_obs[K - k]) prev = (int)(a.t_cur - k);
    for (int k = 1; k <= K; ++k)
      if (next < 0 && s_obs[K + k]) next = (int)(a.t_cur + k);
    const float tau_t = ld_any(a.tau, b * a.stb + a.t_cur * a.stt, a.td);
    const float tp = prev >= 0 ? ld_any(a.tau, b * a.stb + prev * a.stt, a.td) : 0.0f;
    const float tn = next >= 0 ? ld_any(a.tau, b * a.stb + next * a.stt, a.td) : 0.0f;
    const float den = tn - tp;
    float w = den > 1e-9f ? (tau_t - tp) / den : 0.5f;
    s_w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
    s_pn[0] = prev;
    s_pn[1] = next;
  }
  __syncthreads();
  const int prev = s_pn[0], next = s_pn[1];
  const float w = s_w;
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb;
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob;
  for (int64_t f = f0 + tid; f < f1; f += kInterpThreads) {
    float v;
    if (prev >= 0 && next >= 0)
      v = lerp_pair(ldf(V + prev * a.svt + f), ldf(V + next * a.svt + f), w);
    else if (prev >= 0)
      v = ldf(V + prev * a.svt + f);
    else if (next >= 0)
      v = ldf(V + next * a.svt + f);
    else
      v = ldf(V + a.t_cur * a.svt + f);
    stf(O + a.t_cur * a.sot + f, v);
    // h_in is read as 0 where b*stride_hib + f >= B*F (fused_ssm_interp.py:97-98)
    const int64_t lin = b * a.s_hib + f;
    const float hp = lin < a.nb * a.F ? a.h_in[lin] : 0.0f;
    a.h_out[b * a.s_hob + f] = a.A_bar[f] * hp + a.B_bar[f] * v;
  }
}

// Tiles of at most 256 features: one thread per feature, and every load that
// does not depend on the neighbour search goes out in the first round trip --
// the mask values of all 2K+1 candidate rows (spread flat over the
// workgroup, kStepBatch per thread at a time), tau of every candidate row,
// and h_in, A_bar, B_bar of the thread's feature.  Threads that see an
// observed lane store 1 into the row's flag (the same value: no atomics);
// every thread then searches the flags in LDS, and only the two V rows of
// the chosen neighbours are loaded after that.  Same selection and weights
// as interp_step_kernel (fused_ssm_interp.py:41-101).
constexpr int kStepBatch = 16;

template <typename TM>
__device__ inline void step_mask_batch(const TM* M, int64_t row0, int64_t smt, int64_t f0,
                                       int64_t t_lo, int64_t T, int nf, int total, int base,
                                       int tid, float* mv, int* mi) {
#pragma unroll
  for (int j = 0; j < kStepBatch; ++j) {
    const int idx = base + tid + j * kInterpThreads;
    const int ix = idx < total ? idx : 0;
    const int i = ix / nf, f = ix - i * nf;
    int64_t t = t_lo + i;
    t = t < 0 ? 0 : (t < T ? t : T - 1);  // rows outside [0, T) are never observed
    mv[j] = ldf(M + row0 + t * smt + f0 + f);
    mi[j] = idx < total && t_lo + i >= 0 && t_lo + i < T ? i : -1;
  }
}

// TM: the mask's element type, a template argument so that the mask loads
// are straight-line code (behind a dtype switch each load would be waited on
// before the switch's branches join: one round trip per load).
template <typename TV, typename TM>
__global__ __launch_bounds__(kInterpThreads) void interp_step_fast_kernel(StepArgs a) {
  extern __shared__ float s_tau[];  // [2K + 1], then the flags
  unsigned char* s_obs = reinterpret_cast<unsigned char*>(s_tau + 2 * a.K + 1);  // [2K + 1]
  const int tid = threadIdx.x;
  const int64_t b = a.b0 + blockIdx.y;
  const int64_t f0 = (int64_t)blockIdx.x * a.FTILE;
  const int nf = (int)((f0 + a.FTILE < a.F ? f0 + a.FTILE : a.F) - f0);
  const int K = (int)a.K, nrow = 2 * K + 1;
  const int64_t t_lo = a.t_cur - K;
  const int total = nrow * nf;
  const int64_t mrow = b * a.smb;

  float mv[kStepBatch];
  int mi[kStepBatch];
  const TM* Mt = reinterpret_cast<const TM*>(a.M);
  step_mask_batch(Mt, mrow, a.smt, f0, t_lo, a.T, nf, total, 0, tid, mv, mi);
  // feature side inputs
  const bool fact = tid < nf;
  const int64_t f = f0 + (fact ? tid : 0);
  const int64_t lin = b * a.s_hib + f;  // h_in reads 0 where b*stride_hib + f >= B*F (:97-98)
  const float hp = lin < a.nb * a.F ? a.h_in[lin] : 0.0f;
  const float abar = a.A_bar[f], bbar = a.B_bar[f];
  // timestamps of the candidate rows (rows outside [0, T) read a clamped row
  // and are never a neighbour); branch-free so that the loads stay in flight
  // with the mask loads
  for (int i = tid; i < nrow; i += kInterpThreads) {
    int64_t t = t_lo + i;
    t = t < 0 ? 0 : (t < a.T ? t : a.T - 1);
    s_obs[i] = 0;
    s_tau[i] = ld_any_nb(a.tau, b * a.stb + t * a.stt, a.td);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kStepBatch; ++j)
    if (mi[j] >= 0 && mv[j] > 0.5f) s_obs[mi[j]] = 1;
  for (int base = kStepBatch * kInterpThreads; base < total; base += kStepBatch * kInterpThreads) {
    step_mask_batch(Mt, mrow, a.smt, f0, t_lo, a.T, nf, total, base, tid, mv, mi);
#pragma unroll
    for (int j = 0; j < kStepBatch; ++j)
      if (mi[j] >= 0 && mv[j] > 0.5f) s_obs[mi[j]] = 1;
  }
  __syncthreads();
  // nearest observed row within K on each side (the tile's "any observed")
  int kp = 0, kn = 0;
  for (int k = 1; k <= K; ++k)
    if (kp == 0 && s_obs[K - k]) kp = k;
  for (int k = 1; k <= K; ++k)
    if (kn == 0 && s_obs[K + k]) kn = k;
  if (!fact) return;  // after the last barrier
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb + f;
  float v;
  if (kp > 0 && kn > 0) {
    const float tp = s_tau[K - kp], tn = s_tau[K + kn], den = tn - tp;
    float w = den > 1e-9f ? (s_tau[K] - tp) / den : 0.5f;
    w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
    const float vp = ldf(V + (a.t_cur - kp) * a.svt), vn = ldf(V + (a.t_cur + kn) * a.svt);
    v = lerp_pair(vp, vn, w);
  } else if (kp > 0) {
    v = ldf(V + (a.t_cur - kp) * a.svt);
  } else if (kn > 0) {
    v = ldf(V + (a.t_cur + kn) * a.svt);
  } else {
    v = ldf(V + a.t_cur * a.svt);
  }
  stf(reinterpret_cast<TV*>(a.Vhat) + b * a.sob + a.t_cur * a.sot + f, v);
  a.h_out[b * a.s_hob + f] = abar * hp + bbar * v;
}

// Opt-in corrected interpolation (per-feature neighbours, observed values
// kept; the reference behaviour above stays the default).  Workgroup = (b,
// 64 steps, 64 features): the observed flags (M > 0.5) and tau of rows
// t0-K .. t0+63+K are staged in LDS, lane = feature, wave w takes steps
// t0 + w + 4 i; the nearest observed step within K on each side is found in
// LDS and V is read only at the step itself or at the chosen neighbours.
constexpr int kCorrTB = 64;

template <typename TV>
__global__ __launch_bounds__(kInterpThreads) void interp_corrected_kernel(InterpArgs a) {
  extern __shared__ float s_tau[];  // [kCorrTB + 2K], then the flags [kCorrTB + 2K][64]
  auto s_obs = reinterpret_cast<unsigned char (*)[64]>(s_tau + kCorrTB + 2 * a.K);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kCorrTB;
  const int64_t f = (int64_t)blockIdx.y * 64 + lane;
  const int64_t b = a.b0 + blockIdx.z;
  const int K = (int)a.K;
  const int nrow = kCorrTB + 2 * K;
  const bool fok = f < a.F;
  const int64_t fs = fok ? f : 0;
  for (int i = wave; i < nrow; i += kInterpThreads / 64) {
    const int64_t t = t0 - K + i;
    const bool in = t >= 0 && t < a.T;
    s_obs[i][lane] = (in && fok && ld_any(a.M, b * a.smb + t * a.smt + fs, a.md) > 0.5f) ? 1 : 0;
    if (lane == 0) s_tau[i] = in ? ld_any(a.tau, b * a.stb + t * a.stt, a.td) : 0.0f;
  }
  __syncthreads();
  if (!fok) return;  // after the only barrier
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb + f;
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob + f;
  for (int j = wave; j < kCorrTB; j += kInterpThreads / 64) {
    const int64_t t = t0 + j;
    if (t >= a.grid_t) break;
    const int i = K + j;  // row of step t in the staged window
    float v;
    if (s_obs[i][lane]) {
      v = ldf(V + t * a.svt);
    } else {
      int kp = 0, kn = 0;
      for (int k = 1; k <= K && kp == 0; ++k)
        if (s_obs[i - k][lane]) kp = k;
      for (int k = 1; k <= K && kn == 0; ++k)
        if (s_obs[i + k][lane]) kn = k;
      if (kp > 0 && kn > 0) {
        const float tp = s_tau[i - kp], tn = s_tau[i + kn], den = tn - tp;
        float w = den > 1e-9f ? (s_tau[i] - tp) / den : 0.5f;
        w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
        v = lerp_pair(ldf(V + (t - kp) * a.svt), ldf(V + (t + kn) * a.svt), w);
      } else if (kp > 0) {
        v = ldf(V + (t - kp) * a.svt);
      } else if (kn > 0) {
        v = ldf(V + (t + kn) * a.svt);
      } else {
        v = ldf(V + t * a.svt);
      }
    }
    stf(O + t * a.sot, v);
  }
}

// Staged form for windows whose V rows fit in LDS beside the flags (324 bytes
// per window row, K up to 69): the flags, tau and V of rows t0-K .. t0+63+K are
// loaded as coalesced rows, kCorrBatch rows per wave in flight, and every step
// is then resolved from LDS.  The direct form above reads V behind each step's
// data-dependent branch, one step at a time per wave.  VEC (fp32 V and M,
// 16-byte rows, whole 64-feature tiles): 16 lanes stage a row with 16-byte
// loads, so one wave instruction covers 4 rows.
constexpr int kCorrBatch = 8;

__host__ __device__ constexpr int64_t corr_staged_lds(int64_t K) {
  return ((kCorrTB + 2 * K + 3) / 4 * 4) * 4 + (kCorrTB + 2 * K) * (64 * 4 + 64);
}

template <typename TV, bool VEC>
__global__ __launch_bounds__(kInterpThreads) void interp_corrected_staged_kernel(InterpArgs a) {
  extern __shared__ float s_tau[];  // [nrow (padded)], then V [nrow][64], then flags [nrow][64]
  const int K = (int)a.K;
  const int nrow = kCorrTB + 2 * K;
  const int npad = (nrow + 3) / 4 * 4;
  float (*s_v)[64] = reinterpret_cast<float (*)[64]>(s_tau + npad);
  auto s_obs = reinterpret_cast<unsigned char (*)[64]>(s_tau + npad + nrow * 64);
  constexpr int NW = kInterpThreads / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kCorrTB;
  const int64_t f = (int64_t)blockIdx.y * 64 + lane;
  const int64_t b = a.b0 + blockIdx.z;
  const bool fok = f < a.F;
  const int64_t fs = fok ? f : 0;
  const TV* V = reinterpret_cast<const TV*>(a.V) + b * a.svb + fs;
  if constexpr (VEC) {
    // lane = (row of 4 within the wave instruction, 4 features): rows
    // 4 (wave + NW q) + lane / 16 of the window
    const int rl = lane >> 4, c4 = (lane & 15) * 4;
    const int64_t f0 = (int64_t)blockIdx.y * 64 + c4;
    const float* Vq = reinterpret_cast<const float*>(a.V) + b * a.svb + f0;
    const float* Mq = reinterpret_cast<const float*>(a.M) + b * a.smb + f0;
    // No load sits behind a branch (the compiler would sink it into the
    // branch and wait for it alone): positions past the window take the
    // window's last row, loading and storing exactly what its own lanes do.
    // the first timestamps load with the first batch of rows
    const int64_t tt = t0 - K + tid;
    const bool tok = tid < nrow && tt >= 0 && tt < a.T;
    const float tv = ld_any_nb(a.tau, b * a.stb + (tok ? tt : 0) * a.stt, a.td);
    for (int q0 = 0; q0 * 4 * NW < nrow; q0 += kCorrBatch) {
      f32x4 mv[kCorrBatch], vv[kCorrBatch];
#pragma unroll
      for (int q = 0; q < kCorrBatch; ++q) {  // rows outside [0, T) read row 0 (flags 0)
        const int i = min(4 * (wave + NW * (q0 + q)) + rl, nrow - 1);
        const int64_t t = t0 - K + i;
        const int64_t tc = (t >= 0 && t < a.T) ? t : 0;
        mv[q] = *reinterpret_cast<const f32x4*>(Mq + tc * a.smt);
        vv[q] = *reinterpret_cast<const f32x4*>(Vq + tc * a.svt);
      }
#pragma unroll
      for (int q = 0; q < kCorrBatch; ++q) {
        const int i = min(4 * (wave + NW * (q0 + q)) + rl, nrow - 1);
        const int64_t t = t0 - K + i;
        const bool in = t >= 0 && t < a.T;
        const uint32_t fl = in ? ((mv[q][0] > 0.5f ? 1u : 0u) | (mv[q][1] > 0.5f ? 0x100u : 0u) |
                                  (mv[q][2] > 0.5f ? 0x10000u : 0u) | (mv[q][3] > 0.5f ? 0x1000000u : 0u))
                               : 0u;
        *reinterpret_cast<uint32_t*>(&s_obs[i][c4]) = fl;
        *reinterpret_cast<f32x4*>(&s_v[i][c4]) = vv[q];
      }
    }
    if (tid < nrow) s_tau[tid] = tok ? tv : 0.0f;
    for (int i = tid + kInterpThreads; i < nrow; i += kInterpThreads) {
      const int64_t t = t0 - K + i;
      s_tau[i] = (t >= 0 && t < a.T) ? ld_any(a.tau, b * a.stb + t * a.stt, a.td) : 0.0f;
    }
  } else {
  for (int i0 = wave; i0 < nrow; i0 += NW * kCorrBatch) {
    float mv[kCorrBatch], vv[kCorrBatch], tv[kCorrBatch];
#pragma unroll
    for (int q = 0; q < kCorrBatch; ++q) {  // rows out of range read row 0, discarded below
      const int64_t t = t0 - K + i0 + NW * q;
      const int64_t tc = (t >= 0 && t < a.T) ? t : 0;
      mv[q] = ld_any(a.M, b * a.smb + tc * a.smt + fs, a.md);
      vv[q] = ldf(V + tc * a.svt);
      tv[q] = lane == 0 ? ld_any(a.tau, b * a.stb + tc * a.stt, a.td) : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < kCorrBatch; ++q) {
      const int i = i0 + NW * q;
      if (i < nrow) {
        const int64_t t = t0 - K + i;
        const bool in = t >= 0 && t < a.T;
        s_obs[i][lane] = (in && fok && mv[q] > 0.5f) ? 1 : 0;
        s_v[i][lane] = vv[q];
        if (lane == 0) s_tau[i] = in ? tv[q] : 0.0f;
      }
    }
  }
  }
  __syncthreads();
  if (!fok) return;  // after the only barrier
  TV* O = reinterpret_cast<TV*>(a.Vhat) + b * a.sob + f;
  // value of step t (row i of the window) from the nearest observed rows kp
  // before and kn after it (0: none within K).  The weight's division is a
  // hardware reciprocal (about 1 ulp) times the numerator.
  auto resolve = [&](int i, int kp, int kn) {
    if (kp > 0 && kn > 0) {
      const float tp = s_tau[i - kp], tn = s_tau[i + kn], den = tn - tp;
      float w = den > 1e-9f ? (s_tau[i] - tp) * __builtin_amdgcn_rcpf(den) : 0.5f;
      w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
      return lerp_pair(s_v[i - kp][lane], s_v[i + kn][lane], w);
    }
    return kp > 0 ? s_v[i - kp][lane] : (kn > 0 ? s_v[i + kn][lane] : s_v[i][lane]);
  };
  constexpr int JW = kCorrTB / NW;  // consecutive steps per wave
  const int jw = wave * JW;
  if (JW + 2 * K <= 64) {
    // the wave's rows jw .. jw + JW + 2K - 1 as one observed-bit mask per lane:
    // the nearest observed row on each side is a leading/trailing-zero count
    uint64_t mask = 0;
    for (int r = 0; r < JW + 2 * K; ++r) mask |= (uint64_t)s_obs[jw + r][lane] << r;
    const uint64_t lowK = (uint64_t(1) << K) - 1;
    for (int jj = 0; jj < JW; ++jj) {
      const int64_t t = t0 + jw + jj;
      if (t >= a.grid_t) break;
      const int r = K + jj;  // bit of step t; its row in the window is jw + r
      float v;
      if ((mask >> r) & 1) {
        v = s_v[jw + r][lane];
      } else {
        const uint64_t below = (mask >> (r - K)) & lowK;  // bit p: row r - K + p
        const uint64_t above = (mask >> (r + 1)) & lowK;  // bit p: row r + 1 + p
        const int kp = below ? K - (63 - __builtin_clzll(below)) : 0;
        const int kn = above ? __builtin_ctzll(above) + 1 : 0;
        v = resolve(jw + r, kp, kn);
      }
      stf(O + t * a.sot, v);
    }
  } else {
    for (int j = wave; j < kCorrTB; j += NW) {
      const int64_t t = t0 + j;
      if (t >= a.grid_t) break;
      const int i = K + j;  // row of step t in the staged window
      float v = s_v[i][lane];
      if (!s_obs[i][lane]) {
        int kp = 0, kn = 0;
        for (int k = 1; k <= K && kp == 0; ++k)
          if (s_obs[i - k][lane]) kp = k;
        for (int k = 1; k <= K && kn == 0; ++k)
          if (s_obs[i + k][lane]) kn = k;
        v = resolve(i, kp, kn);
      }
      stf(O + t * a.sot, v);
    }
  }
}

}  // namespace tssm

using namespace tssm;

static bool float_dtype(int d) { return d == TSSM_F32 || d == TSSM_BF16 || d == TSSM_F16; }

static int64_t interp_rows(int64_t T, int64_t grid_t, int64_t K) {
  return grid_t + K < T ? grid_t + K : T;
}

extern "C" int64_t tssm_time_aware_interp_workspace_bytes(int64_t T, int64_t F, int64_t K,
                                                          int64_t FTILE, int64_t grid_b,
                                                          int64_t grid_t, int64_t grid_f) {
  if (T < 0 || F < 0 || K < 0 || FTILE <= 0 || grid_b < 0 || grid_t < 0 || grid_f < 0) return -1;
  const int64_t ntile = (F + FTILE - 1) / FTILE;
  const int64_t gf = grid_f < ntile ? grid_f : ntile;
  return grid_b * interp_rows(T, grid_t, K) * gf;
}

extern "C" int tssm_time_aware_interp(int v_dtype, int m_dtype, int tau_dtype, const void* V,
                                      const void* M, const void* tau, void* Vhat, int64_t nbatch,
                                      int64_t T, int64_t F, int64_t svb, int64_t svt, int64_t smb,
                                      int64_t smt, int64_t stb, int64_t stt, int64_t sob,
                                      int64_t sot, int64_t K, int64_t FTILE, int64_t grid_b,
                                      int64_t grid_t, int64_t grid_f, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(V && M && tau && Vhat, TSSM_ERR_NULL);
  TSSM_CHECK(float_dtype(v_dtype) && float_dtype(m_dtype) && float_dtype(tau_dtype),
             TSSM_ERR_DTYPE);
  TSSM_CHECK(nbatch >= 0 && T >= 0 && F >= 0 && FTILE > 0 && K >= 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_b >= 0 && grid_t >= 0 && grid_f >= 0 && grid_b <= nbatch && grid_t <= T,
             TSSM_ERR_SHAPE);
  // interp_kernel's LDS: flags of kInterpTB + 2K rows after its fixed arrays
  const size_t lds_interp = (size_t)(kInterpTB + 2 * K);
  TSSM_CHECK(K <= kMaxLds && (int64_t)lds_interp + 3 * kInterpTB * 4 <= kMaxLds,
             TSSM_ERR_UNSUPPORTED);
  // interp_batched_kernel adds the window's timestamps (while they fit)
  const size_t lds_batched = lds_interp * 5;
  const int64_t ntile = (F + FTILE - 1) / FTILE;
  const int64_t gf = grid_f < ntile ? grid_f : ntile;
  if (grid_b == 0 || grid_t == 0 || gf == 0) return TSSM_OK;
  TSSM_CHECK(gf <= kMaxGridYZ, TSSM_ERR_UNSUPPORTED);
  const int64_t rows = interp_rows(T, grid_t, K);
  const int64_t need = grid_b * rows * gf;
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  InterpArgs a{V, M, tau, Vhat, reinterpret_cast<unsigned char*>(workspace), m_dtype, tau_dtype,
               T, F, svb, svt, smb, smt, stb, stt, sob, sot, K, FTILE, grid_t, rows, gf, 0};
  const hipStream_t s = as_stream(stream);
  const int64_t nrow = grid_b * rows;
  const int64_t wpb = kInterpThreads / 64;
  TSSM_CHECK((nrow + wpb - 1) / wpb <= 2147483647, TSSM_ERR_UNSUPPORTED);
  // flags: 16-byte mask vectors when tiles and rows are whole vectors
  const int64_t EM = m_dtype == TSSM_F32 ? 4 : 8;
  const int64_t fc = F < gf * FTILE ? F : gf * FTILE;
  const int64_t E = v_dtype == TSSM_F32 ? 4 : 8;
  const bool vec = FTILE % E == 0 && F % E == 0 && svt % E == 0 && sot % E == 0 &&
                   svb % E == 0 && sob % E == 0 && aligned(V, 16) && aligned(Vhat, 16);
  int lvpt = 0;
  while ((int64_t(1) << lvpt) < FTILE / EM) ++lvpt;
  const bool mvec = FTILE % EM == 0 && fc % EM == 0 && smt % EM == 0 && smb % EM == 0 &&
                    aligned(M, 16) && fc / EM < 2147483647 - 64;
  // Both vector paths apply: one launch forms its flags and interpolates.
  if (vec && mvec && (int64_t(1) << lvpt) == FTILE / EM && FTILE / EM <= 64) {
    for (int64_t b0 = 0; b0 < grid_b; b0 += kMaxGridYZ) {  // batches in grid-z slices
      a.b0 = b0;
      const int64_t nb = grid_b - b0 < kMaxGridYZ ? grid_b - b0 : kMaxGridYZ;
      const dim3 grid((unsigned)((grid_t + kInterpTB - 1) / kInterpTB), (unsigned)gf,
                      (unsigned)nb);
#define TSSM_FUSED(TT, EE, MT, ME)                                                             \
  if ((int64_t)lds_batched + 3 * kInterpTB * 4 <= kMaxLds)                                  \
    hipLaunchKernelGGL((interp_batched_kernel<TT, EE, MT, ME>), grid, dim3(kInterpThreads), \
                       lds_batched, s, a, lvpt);                                            \
  else                                                                                      \
    hipLaunchKernelGGL((interp_fused_kernel<TT, EE, MT, ME>), grid, dim3(kInterpThreads),   \
                       lds_interp, s, a, lvpt)
#define TSSM_FUSED_M(TT, EE)                                      \
  switch (m_dtype) {                                              \
    case TSSM_F32: TSSM_FUSED(TT, EE, float, 4); break;            \
    case TSSM_BF16: TSSM_FUSED(TT, EE, bf16_t, 8); break;          \
    default: TSSM_FUSED(TT, EE, f16_t, 8); break;                  \
  }
      switch (v_dtype) {
        case TSSM_F32: TSSM_FUSED_M(float, 4); break;
        case TSSM_BF16: TSSM_FUSED_M(bf16_t, 8); break;
        default: TSSM_FUSED_M(f16_t, 8); break;
      }
#undef TSSM_FUSED_M
#undef TSSM_FUSED
      const int st2 = launch_status();
      if (st2 != TSSM_OK) return st2;
    }
    return TSSM_OK;
  }
  if (mvec) {
    const int64_t vpt = FTILE / EM;
    if ((int64_t(1) << lvpt) == vpt && vpt <= 64) {  // tiles = aligned lane groups
      const int64_t wv = (nrow + kObsP2Rows - 1) / kObsP2Rows;
      const dim3 g((unsigned)((wv + wpb - 1) / wpb));
      switch (m_dtype) {
        case TSSM_F32: hipLaunchKernelGGL((interp_obs_pow2_kernel<float, 4>), g,
                                          dim3(kInterpThreads), 0, s, a, nrow, lvpt); break;
        case TSSM_BF16: hipLaunchKernelGGL((interp_obs_pow2_kernel<bf16_t, 8>), g,
                                           dim3(kInterpThreads), 0, s, a, nrow, lvpt); break;
        default: hipLaunchKernelGGL((interp_obs_pow2_kernel<f16_t, 8>), g,
                                    dim3(kInterpThreads), 0, s, a, nrow, lvpt); break;
      }
    } else {
    const int64_t wv = (nrow + kObsRowsPerWave - 1) / kObsRowsPerWave;
    const dim3 g((unsigned)((wv + wpb - 1) / wpb));
    switch (m_dtype) {
      case TSSM_F32: hipLaunchKernelGGL((interp_obs_vec_kernel<float, 4>), g,
                                        dim3(kInterpThreads), 0, s, a, nrow); break;
      case TSSM_BF16: hipLaunchKernelGGL((interp_obs_vec_kernel<bf16_t, 8>), g,
                                         dim3(kInterpThreads), 0, s, a, nrow); break;
      default: hipLaunchKernelGGL((interp_obs_vec_kernel<f16_t, 8>), g,
                                  dim3(kInterpThreads), 0, s, a, nrow); break;
    }
    }
  } else {
    hipLaunchKernelGGL(interp_obs_kernel, dim3((unsigned)((nrow + wpb - 1) / wpb)),
                       dim3(kInterpThreads), 0, s, a, nrow);
  }
  const int st = launch_status();
  if (st != TSSM_OK) return st;
  // 16-byte lane groups when every tile, row stride and base pointer allows (vec)
  for (int64_t b0 = 0; b0 < grid_b; b0 += kMaxGridYZ) {  // batches in grid-z slices
    a.b0 = b0;
    const int64_t nb = grid_b - b0 < kMaxGridYZ ? grid_b - b0 : kMaxGridYZ;
    const dim3 grid((unsigned)((grid_t + kInterpTB - 1) / kInterpTB), (unsigned)gf,
                    (unsigned)nb);
#define TSSM_INTERP(TT, EE) \
  hipLaunchKernelGGL((interp_kernel<TT, EE>), grid, dim3(kInterpThreads), lds_interp, s, a)
    switch (v_dtype) {
      case TSSM_F32: if (vec) TSSM_INTERP(float, 4); else TSSM_INTERP(float, 1); break;
      case TSSM_BF16: if (vec) TSSM_INTERP(bf16_t, 8); else TSSM_INTERP(bf16_t, 1); break;
      default: if (vec) TSSM_INTERP(f16_t, 8); else TSSM_INTERP(f16_t, 1); break;
    }
#undef TSSM_INTERP
    const int st2 = launch_status();
    if (st2 != TSSM_OK) return st2;
  }
  return TSSM_OK;
}

extern "C" int tssm_interp_ssm_step(int v_dtype, int m_dtype, int tau_dtype, const void* V,
                                    const void* M, const void* tau, const float* A_bar,
                                    const float* B_bar, const float* h_in, void* Vhat,
                                    float* h_out, int64_t nbatch, int64_t T, int64_t F,
                                    int64_t svb, int64_t svt, int64_t smb, int64_t smt,
                                    int64_t stb, int64_t stt, int64_t sob, int64_t sot,
                                    int64_t s_hib, int64_t s_hob, int64_t t_cur, int64_t K,
                                    int64_t FTILE, int64_t grid_b, int64_t grid_f,
                                    void* stream) {
  TSSM_CHECK(V && M && tau && A_bar && B_bar && h_in && Vhat && h_out, TSSM_ERR_NULL);
  TSSM_CHECK(float_dtype(v_dtype) && float_dtype(m_dtype) && float_dtype(tau_dtype),
             TSSM_ERR_DTYPE);
  TSSM_CHECK(nbatch >= 0 && T > 0 && F >= 0 && FTILE > 0 && K >= 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(t_cur >= 0 && t_cur < T, TSSM_ERR_SHAPE);
  TSSM_CHECK(grid_b >= 0 && grid_f >= 0 && grid_b <= nbatch, TSSM_ERR_SHAPE);
  // LDS: the 2K+1 candidate rows' timestamps (fast kernel) and flags
  const bool fast = FTILE <= kInterpThreads;  // one thread per feature: every load up front
  const size_t lds = fast ? (size_t)(2 * K + 1) * 5 : (size_t)(2 * K + 1);
  TSSM_CHECK(K <= kMaxLds && (int64_t)lds + 64 <= kMaxLds, TSSM_ERR_UNSUPPORTED);
  const int64_t ntile = (F + FTILE - 1) / FTILE;
  const int64_t gf = grid_f < ntile ? grid_f : ntile;
  if (grid_b == 0 || gf == 0) return TSSM_OK;
  TSSM_CHECK(gf <= 2147483647, TSSM_ERR_UNSUPPORTED);
  StepArgs a{V, M, tau, A_bar, B_bar, h_in, Vhat, h_out, m_dtype, tau_dtype, nbatch, T, F,
             svb, svt, smb, smt, stb, stt, sob, sot, s_hib, s_hob, t_cur, K, FTILE, 0};
  const hipStream_t s = as_stream(stream);
  for (int64_t b0 = 0; b0 < grid_b; b0 += kMaxGridYZ) {  // batches in grid-y slices
    a.b0 = b0;
    const int64_t nb = grid_b - b0 < kMaxGridYZ ? grid_b - b0 : kMaxGridYZ;
    const dim3 grid((unsigned)gf, (unsigned)nb);
    if (fast) {
#define TSSM_STEP_FAST(TT)                                                                   \
  switch (m_dtype) {                                                                         \
    case TSSM_F32: hipLaunchKernelGGL((interp_step_fast_kernel<TT, float>), grid,             \
                                      dim3(kInterpThreads), lds, s, a); break;               \
    case TSSM_BF16: hipLaunchKernelGGL((interp_step_fast_kernel<TT, bf16_t>), grid,           \
                                       dim3(kInterpThreads), lds, s, a); break;              \
    default: hipLaunchKernelGGL((interp_step_fast_kernel<TT, f16_t>), grid,                   \
                                dim3(kInterpThreads), lds, s, a); break;                     \
  }
      switch (v_dtype) {
        case TSSM_F32: TSSM_STEP_FAST(float); break;
        case TSSM_BF16: TSSM_STEP_FAST(bf16_t); break;
        default: TSSM_STEP_FAST(f16_t); break;
      }
#undef TSSM_STEP_FAST
    } else {
      switch (v_dtype) {
        case TSSM_F32: hipLaunchKernelGGL(interp_step_kernel<float>, grid, dim3(kInterpThreads), lds, s, a); break;
        case TSSM_BF16: hipLaunchKernelGGL(interp_step_kernel<bf16_t>, grid, dim3(kInterpThreads), lds, s, a); break;
        default: hipLaunchKernelGGL(interp_step_kernel<f16_t>, grid, dim3(kInterpThreads), lds, s, a); break;
      }
    }
    const int st = launch_status();
    if (st != TSSM_OK) return st;
  }
  return TSSM_OK;
}

extern "C" int tssm_time_aware_interp_corrected(int v_dtype, int m_dtype, int tau_dtype,
                                                const void* V, const void* M, const void* tau,
                                                void* Vhat, int64_t nbatch, int64_t T, int64_t F,
                                                int64_t svb, int64_t svt, int64_t smb, int64_t smt,
                                                int64_t stb, int64_t stt, int64_t sob, int64_t sot,
                                                int64_t K, void* stream) {
  TSSM_CHECK(V && M && tau && Vhat, TSSM_ERR_NULL);
  TSSM_CHECK(float_dtype(v_dtype) && float_dtype(m_dtype) && float_dtype(tau_dtype),
             TSSM_ERR_DTYPE);
  TSSM_CHECK(nbatch >= 0 && T >= 0 && F >= 0 && K >= 0, TSSM_ERR_SHAPE);
  // LDS: timestamps and per-feature flags of kCorrTB + 2K rows (K up to 449)
  const size_t lds = (size_t)(kCorrTB + 2 * K) * (4 + 64);
  TSSM_CHECK(K <= kMaxLds && (int64_t)lds <= kMaxLds, TSSM_ERR_UNSUPPORTED);
  if (nbatch == 0 || T == 0 || F == 0) return TSSM_OK;
  const int64_t gx = (T + kCorrTB - 1) / kCorrTB, gy = (F + 63) / 64;
  TSSM_CHECK(gx <= 2147483647 && gy <= kMaxGridYZ, TSSM_ERR_UNSUPPORTED);
  InterpArgs a{V, M, tau, Vhat, nullptr, m_dtype, tau_dtype, T, F, svb, svt, smb, smt, stb, stt,
               sob, sot, K, 1, T, T, 0, 0};
  const hipStream_t s = as_stream(stream);
  // V staged in LDS with the flags when the window fits (K up to 69)
  const int64_t lds_st = corr_staged_lds(K);
  const bool staged = lds_st <= kMaxLds;
  // 16-byte staging: fp32 V and M, rows and bases 16-byte aligned, whole tiles
  const bool vec = v_dtype == TSSM_F32 && m_dtype == TSSM_F32 && F % 64 == 0 && svt % 4 == 0 &&
                   svb % 4 == 0 && smt % 4 == 0 && smb % 4 == 0 && aligned(V, 16) && aligned(M, 16);
  for (int64_t b0 = 0; b0 < nbatch; b0 += kMaxGridYZ) {  // batches in grid-z slices
    a.b0 = b0;
    const int64_t nb = nbatch - b0 < kMaxGridYZ ? nbatch - b0 : kMaxGridYZ;
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)nb);
    if (staged && vec) {
      hipLaunchKernelGGL((interp_corrected_staged_kernel<float, true>), grid, dim3(kInterpThreads), lds_st, s, a);
    } else if (staged) {
      switch (v_dtype) {
        case TSSM_F32: hipLaunchKernelGGL((interp_corrected_staged_kernel<float, false>), grid, dim3(kInterpThreads), lds_st, s, a); break;
        case TSSM_BF16: hipLaunchKernelGGL((interp_corrected_staged_kernel<bf16_t, false>), grid, dim3(kInterpThreads), lds_st, s, a); break;
        default: hipLaunchKernelGGL((interp_corrected_staged_kernel<f16_t, false>), grid, dim3(kInterpThreads), lds_st, s, a); break;
      }
    } else {
      switch (v_dtype) {
        case TSSM_F32: hipLaunchKernelGGL(interp_corrected_kernel<float>, grid, dim3(kInterpThreads), lds, s, a); break;
        case TSSM_BF16: hipLaunchKernelGGL(interp_corrected_kernel<bf16_t>, grid, dim3(kInterpThreads), lds, s, a); break;
        default: hipLaunchKernelGGL(interp_corrected_kernel<f16_t>, grid, dim3(kInterpThreads), lds, s, a); break;
      }
    }
    const int st = launch_status();
    if (st != TSSM_OK) return st;
  }
  return TSSM_OK;
}
