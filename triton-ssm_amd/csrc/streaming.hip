// Streaming single-step updates (streaming_inference_kernel.py).
//
// stream_step_kernel: streaming_ssm_inplace_kernel[_bf16] (:7-71) --
//   h <- Abar*h + Bbar*vhat in place, y = C*h_new + D*vhat, y written with
//   vhat's batch stride (:37).  The state dtype is the kernel's dtype (the
//   bf16 variant rounds the state to bf16 on every step, as the reference).
// stream_interp_step_kernel: streaming_interp_then_ssm_kernel (:75-156) with
//   one workgroup per stream, so the ring head is read once by every feature
//   tile and advanced after all of them (the reference reads it in every
//   tile program but advances it from tile 0 only, :106,115-117).
#include "common.h"

namespace tssm {

// Workgroup = 256 threads x V lanes (grid y) of kStepRows streams (grid x):
// no per-element division, 16-byte (fp32) / 8-byte (16-bit) accesses when
// aligned (V = 4).
constexpr int kStepRows = 4;
template <typename T, int V>
__global__ __launch_bounds__(256) void stream_step_kernel(
    const T* __restrict__ vhat, T* __restrict__ h, const T* __restrict__ Abar,
    const T* __restrict__ Bbar, const T* __restrict__ C, const T* __restrict__ D,
    T* __restrict__ y, int64_t hc, int64_t nb, int64_t svb, int64_t shb, int64_t scb) {
  const int64_t k = ((int64_t)blockIdx.y * 256 + threadIdx.x) * V;
  if (k >= hc) return;
  float ab[V], bb[V], dv[V];
  ld_lanes<T, V>(Abar + k, ab);
  ld_lanes<T, V>(Bbar + k, bb);
  ld_lanes<T, V>(D + k, dv);
  // every row's loads first, so the thread makes one round trip to memory
  // instead of one per row (a store's wait would otherwise hold up the next
  // row's loads).  Rows past nb redo row nb - 1 from the same loaded values and
  // store the same results there: no branch, so no load sinks back into one.
  const int64_t b0 = (int64_t)blockIdx.x * kStepRows;
  float v[kStepRows][V], hv[kStepRows][V], cv[kStepRows][V];
  int64_t rb[kStepRows];
#pragma unroll
  for (int r = 0; r < kStepRows; ++r) {
    rb[r] = b0 + r < nb ? b0 + r : nb - 1;
    ld_lanes<T, V>(vhat + rb[r] * svb + k, v[r]);
    ld_lanes<T, V>(h + rb[r] * shb + k, hv[r]);
    ld_lanes<T, V>(C + rb[r] * scb + k, cv[r]);
  }
#pragma unroll
  for (int r = 0; r < kStepRows; ++r) {
    float yv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      hv[r][j] = ab[j] * hv[r][j] + bb[j] * v[r][j];
      yv[j] = cv[r][j] * hv[r][j] + dv[j] * v[r][j];
    }
    st_lanes<T, V>(h + rb[r] * shb + k, hv[r]);
    st_lanes<T, V>(y + rb[r] * svb + k, yv);
  }
}

constexpr int kStreamThreads = 256;
constexpr int kRingFast = 16;  // search slots held in registers (KRING <= 17)

struct RingArgs {
  float* ring_V;
  float* ring_M;
  float* ring_tau;
  int32_t* ring_head;
  const float* v_new;
  const float* m_new;
  const float* tau_new;
  float* h;
  const float* Abar;
  const float* Bbar;
  const float* C;
  const float* D;
  float* y;
  int64_t H, srb, srk, svb, shb, scb, BLOCK_H, KRING;
};

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// One workgroup per stream; feature tiles are spread over its waves, each tile
// searched and updated by one wave with wave-level sums.  The search never
// reads the slot being written (it starts one slot behind it), so the insert
// needs no barrier; one barrier before the head advances.
__global__ __launch_bounds__(kStreamThreads) void stream_interp_step_kernel(RingArgs a) {
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  constexpr int nwaves = kStreamThreads / 64;
  const int64_t KR = a.KRING;
  const int64_t head = a.ring_head[b];
  const int64_t nh = (head + 1) % KR;                                    // :107
  float* rV = a.ring_V + b * a.srb;
  float* rM = a.ring_M + b * a.srb;
  // insert the new observation (:113-114); m_new uses v's batch stride (:110)
  for (int64_t k = tid; k < a.H; k += kStreamThreads) {
    rV[nh * a.srk + k] = a.v_new[b * a.svb + k];
    rM[nh * a.srk + k] = a.m_new[b * a.svb + k];
  }
  const int64_t ntile = (a.H + a.BLOCK_H - 1) / a.BLOCK_H;
  if (a.BLOCK_H <= 64 && KR - 1 <= kRingFast) {
    // one feature per lane.  The search result is used only when the new
    // observation leaves the tile empty (fill, :133,143), so the tile's new
    // mask is summed first and the ring is searched only then, every slot's
    // mask value loaded before the first wave sum.
    for (int64_t tile = wave; tile < ntile; tile += nwaves) {
      const int64_t f = tile * a.BLOCK_H + lane;
      const bool act = lane < a.BLOCK_H && f < a.H;
      const int64_t fs = act ? f : tile * a.BLOCK_H;  // in bounds for idle lanes
      const float vn = a.v_new[b * a.svb + fs];
      const float mn = act ? a.m_new[b * a.svb + fs] : 0.0f;
      const float hv = a.h[b * a.shb + fs], ab = a.Abar[fs], bb = a.Bbar[fs];
      const float cv = a.C[b * a.scb + fs], dv = a.D[fs];
      float v = vn;
      if (wave_sum(mn) < 0.5f) {  // uniform
        float ms[kRingFast];
#pragma unroll
        for (int k = 1; k <= kRingFast; ++k) {
          const int64_t kk = k < KR ? k : KR - 1;  // clamped, zeroed below
          const int64_t rk = (nh - kk + KR) % KR;
          const float m = rM[rk * a.srk + fs];
          ms[k - 1] = (act && k < KR) ? m : 0.0f;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
          for (int k = 0; k < kRingFast; ++k) ms[k] += __shfl_xor(ms[k], o);
        int prev_k = -1;  // nearest earlier slot whose tile has any observation (:124-130)
#pragma unroll
        for (int k = kRingFast; k >= 1; --k)
          if (k < KR && ms[k - 1] > 0.5f) prev_k = (int)((nh - k + KR) % KR);
        if (prev_k >= 0) v = rV[prev_k * a.srk + fs];
      }
      if (act) {
        const float hn = ab * hv + bb * v;                           // :152
        a.h[b * a.shb + f] = hn;
        a.y[b * a.svb + f] = cv * hn + dv * v;                       // :153,156
      }
    }
  } else {
  for (int64_t tile = wave; tile < ntile; tile += nwaves) {
    const int64_t f0 = tile * a.BLOCK_H;
    const int64_t f1 = f0 + a.BLOCK_H < a.H ? f0 + a.BLOCK_H : a.H;
    // backward search over the previous KRING-1 slots (:124-130): nearest slot
    // whose tile has any observation
    int64_t prev_k = -1;
    for (int64_t k = 1; k < KR; ++k) {
      const int64_t rk = (nh - k + KR) % KR;
      float s = 0.0f;
      for (int64_t f = f0 + lane; f < f1; f += 64) s += rM[rk * a.srk + f];
      if (wave_sum(s) > 0.5f) {  // uniform over the wave
        prev_k = rk;
        break;
      }
    }
    float sm = 0.0f;
    for (int64_t f = f0 + lane; f < f1; f += 64) sm += a.m_new[b * a.svb + f];
    const bool fill = prev_k >= 0 && wave_sum(sm) < 0.5f;                // :133,143
    for (int64_t f = f0 + lane; f < f1; f += 64) {
      const float v = fill ? rV[prev_k * a.srk + f] : a.v_new[b * a.svb + f];
      const float hn = a.Abar[f] * a.h[b * a.shb + f] + a.Bbar[f] * v;  // :152
      a.h[b * a.shb + f] = hn;
      a.y[b * a.svb + f] = a.C[b * a.scb + f] * hn + a.D[f] * v;        // :153,156
    }
  }
  }
  __syncthreads();  // every wave has read the head before it advances
  if (tid == 0) {
    a.ring_tau[b * KR + nh] = a.tau_new[b];                              // :116
    a.ring_head[b] = (int32_t)nh;                                        // :117
  }
}

// 16-byte form (BLOCK_H = 4 LPT with LPT in 4 .. 64; H % 4 == 0; aligned
// rows, KRING - 1 <= kRingFast): a lane owns 4 adjacent features, LPT lanes
// one tile, so a wave instruction covers 64 / LPT tiles.  Same steps as
// stream_interp_step_kernel, with every load of a thread issued before the
// first wait: per tile the new observation (inserted into the ring by the
// lanes that own its features: a lane's tile loop covers exactly the features
// the insert loop would give it), the new mask sum (an LPT-lane group sum),
// the ring searched (all slots at once) only when some tile of the wave has no
// new observation, and the in-place step.  Ring slots are uniform and formed
// once, without 64-bit divisions.
template <int LPT>
__global__ __launch_bounds__(kStreamThreads) void stream_interp_step_vec_kernel(RingArgs a) {
  constexpr int TPW = 64 / LPT;  // tiles per wave instruction
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  constexpr int nwaves = kStreamThreads / 64;
  const int KR = (int)a.KRING;
  float* rV = a.ring_V + b * a.srb;
  float* rM = a.ring_M + b * a.srb;
  const int64_t ntile = (a.H + a.BLOCK_H - 1) / a.BLOCK_H;
  for (int64_t tg = (int64_t)wave * TPW; tg < ntile; tg += nwaves * TPW) {
    const int64_t tile = tg + lane / LPT;
    const int64_t f = tile * a.BLOCK_H + 4 * (lane % LPT);
    const bool act = tile < ntile && f < a.H;  // H % 4 == 0: all 4 features or none
    const int64_t fs = act ? f : 0;
    float vn[4], mn[4], hv[4], cv[4], ab[4], bb[4], dv[4];
    ld_lanes<float, 4>(a.v_new + b * a.svb + fs, vn);
    ld_lanes<float, 4>(a.m_new + b * a.svb + fs, mn);
    ld_lanes<float, 4>(a.h + b * a.shb + fs, hv);
    ld_lanes<float, 4>(a.C + b * a.scb + fs, cv);
    ld_lanes<float, 4>(a.Abar + fs, ab);
    ld_lanes<float, 4>(a.Bbar + fs, bb);
    ld_lanes<float, 4>(a.D + fs, dv);
    // the head is read here, after this tile's loads (volatile: read in the
    // loop, so its wait is not hoisted ahead of them)
    const int32_t head = *reinterpret_cast<const volatile int32_t*>(a.ring_head + b);
    const int nh = (int)((((int64_t)head + 1) % KR + KR) % KR);            // :107
    if (act) {  // insert the new observation (:110-114)
      st_lanes<float, 4>(rV + nh * a.srk + f, vn);
      st_lanes<float, 4>(rM + nh * a.srk + f, mn);
    }
    const float sm = group_sum<LPT>(act ? (mn[0] + mn[1]) + (mn[2] + mn[3]) : 0.0f);
    const bool need = act && sm < 0.5f;  // same on every lane of the tile
    float v[4] = {vn[0], vn[1], vn[2], vn[3]};
    if (__ballot(need) != 0) {  // uniform
      int slot[kRingFast];  // slot of the observation k steps back, nearest first
#pragma unroll
      for (int k = 1; k <= kRingFast; ++k) {
        const int kk = k < KR ? k : KR - 1;  // clamped, ignored below
        slot[k - 1] = nh - kk < 0 ? nh - kk + KR : nh - kk;
      }
      float ms[kRingFast];
#pragma unroll
      for (int k = 1; k <= kRingFast; ++k) {
        float m[4];
        ld_lanes<float, 4>(rM + slot[k - 1] * a.srk + fs, m);
        ms[k - 1] = (act && k < KR) ? (m[0] + m[1]) + (m[2] + m[3]) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < kRingFast; ++k) ms[k] = group_sum<LPT>(ms[k]);
      int prev_k = -1;  // nearest earlier slot whose tile has any observation (:124-130)
#pragma unroll
      for (int k = kRingFast; k >= 1; --k)
        if (k < KR && ms[k - 1] > 0.5f) prev_k = slot[k - 1];
      if (need && prev_k >= 0) ld_lanes<float, 4>(rV + prev_k * a.srk + fs, v);  // :133,143
    }
    if (act) {
      float hn[4], yo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hn[j] = ab[j] * hv[j] + bb[j] * v[j];                            // :152
        yo[j] = cv[j] * hn[j] + dv[j] * v[j];                            // :153,156
      }
      st_lanes<float, 4>(a.h + b * a.shb + f, hn);
      st_lanes<float, 4>(a.y + b * a.svb + f, yo);
    }
  }
  __syncthreads();  // every wave has read the head before it advances
  if (tid == 0) {
    const int nh = (int)((((int64_t)a.ring_head[b] + 1) % KR + KR) % KR);
    a.ring_tau[b * KR + nh] = a.tau_new[b];                              // :116
    a.ring_head[b] = (int32_t)nh;                                        // :117
  }
}

// Opt-in corrected streaming interpolation: the same insert and head update
// as stream_interp_step_kernel, then per feature an observed new value is
// kept and an unobserved one is forward-filled from the most recent of the
// previous KRING-1 slots where that feature was observed (a causal step has
// no later neighbour to weight against); none: v_new as given.
__global__ __launch_bounds__(kStreamThreads) void stream_interp_step_corrected_kernel(RingArgs a) {
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t KR = a.KRING;
  const int64_t head = a.ring_head[b];
  const int64_t nh = (head + 1) % KR;
  float* rV = a.ring_V + b * a.srb;
  float* rM = a.ring_M + b * a.srb;
  for (int64_t f = tid; f < a.H; f += kStreamThreads) {
    const float vn = a.v_new[b * a.svb + f];
    const float mn = a.m_new[b * a.svb + f];
    rV[nh * a.srk + f] = vn;  // this thread's own feature: no other thread reads it
    rM[nh * a.srk + f] = mn;
    float v = vn;
    if (!(mn > 0.5f)) {
      int64_t hit = -1;
      if (KR - 1 <= kRingFast) {  // every slot's mask at once, nearest hit kept
        float ms[kRingFast];
#pragma unroll
        for (int k = 1; k <= kRingFast; ++k) {
          const int64_t kk = k < KR ? k : KR - 1;  // clamped, ignored below
          ms[k - 1] = rM[((nh - kk + KR) % KR) * a.srk + f];
        }
#pragma unroll
        for (int k = kRingFast; k >= 1; --k)
          if (k < KR && ms[k - 1] > 0.5f) hit = (nh - k + KR) % KR;
      } else {
        for (int64_t k = 1; k < KR && hit < 0; ++k) {  // nearest first
          const int64_t rk = (nh - k + KR) % KR;
          if (rM[rk * a.srk + f] > 0.5f) hit = rk;
        }
      }
      if (hit >= 0) v = rV[hit * a.srk + f];
    }
    const float hn = a.Abar[f] * a.h[b * a.shb + f] + a.Bbar[f] * v;
    a.h[b * a.shb + f] = hn;
    a.y[b * a.svb + f] = a.C[b * a.scb + f] * hn + a.D[f] * v;
  }
  __syncthreads();  // every thread has read the head before it advances
  if (tid == 0) {
    a.ring_tau[b * KR + nh] = a.tau_new[b];
    a.ring_head[b] = (int32_t)nh;
  }
}

// Vector form for 16-byte-aligned rows (H % 4 == 0, KRING <= 17): a thread
// owns 4 consecutive features and issues every load that does not depend on
// the search -- v_new, m_new, h, the parameters and the masks of all previous
// slots -- at once; only V of the chosen slots follows.  Same results as the
// kernel above.
__device__ inline f32x4 ld4v(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ inline void st4v(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

__global__ __launch_bounds__(kStreamThreads) void stream_interp_step_corrected_vec_kernel(RingArgs a) {
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int KR = (int)a.KRING;  // KRING - 1 <= kRingFast (host)
  const int nh = (int)((((int64_t)a.ring_head[b] + 1) % KR + KR) % KR);
  // slots of the previous observations, nearest first (uniform; k past
  // KRING - 1 repeats the last one and is ignored below)
  int slot[kRingFast];
#pragma unroll
  for (int k = 1; k <= kRingFast; ++k) {
    const int kk = k < KR ? k : KR - 1;
    slot[k - 1] = nh - kk < 0 ? nh - kk + KR : nh - kk;
  }
  float* rV = a.ring_V + b * a.srb;
  float* rM = a.ring_M + b * a.srb;
  for (int64_t f = 4 * tid; f < a.H; f += 4 * kStreamThreads) {
    const f32x4 vn = ld4v(a.v_new + b * a.svb + f);
    const f32x4 mn = ld4v(a.m_new + b * a.svb + f);
    const f32x4 hp = ld4v(a.h + b * a.shb + f);
    const f32x4 ab = ld4v(a.Abar + f), bb = ld4v(a.Bbar + f), dd = ld4v(a.D + f);
    const f32x4 cc = ld4v(a.C + b * a.scb + f);
    f32x4 ms[kRingFast];
#pragma unroll
    for (int k = 0; k < kRingFast; ++k) ms[k] = ld4v(rM + slot[k] * a.srk + f);
    st4v(rV + nh * a.srk + f, vn);  // the new slot: not among the slots searched
    st4v(rM + nh * a.srk + f, mn);
    // per element the nearest observed slot; the four neighbour loads issue
    // together (an unused one reads v_new, in bounds)
    const float* src[4];
    bool fill[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int hit = -1;
#pragma unroll
      for (int k = kRingFast; k >= 1; --k)
        if (k < KR && ms[k - 1][e] > 0.5f) hit = slot[k - 1];
      fill[e] = !(mn[e] > 0.5f) && hit >= 0;
      src[e] = fill[e] ? rV + hit * a.srk + f + e : a.v_new + b * a.svb + f + e;
    }
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = *src[e];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = fill[e] ? v[e] : vn[e];
    f32x4 hn, yo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hn[e] = ab[e] * hp[e] + bb[e] * v[e];
      yo[e] = cc[e] * hn[e] + dd[e] * v[e];
    }
    st4v(a.h + b * a.shb + f, hn);
    st4v(a.y + b * a.svb + f, yo);
  }
  __syncthreads();  // every thread has read the head before it advances
  if (tid == 0) {
    a.ring_tau[b * KR + nh] = a.tau_new[b];
    a.ring_head[b] = (int32_t)nh;
  }
}

}  // namespace tssm

using namespace tssm;

extern "C" int tssm_stream_step(int dtype, const void* vhat, void* h, const void* Abar,
                                const void* Bbar, const void* C, const void* D, void* y,
                                int64_t nbatch, int64_t H, int64_t grid_b, int64_t h_cover,
                                int64_t svb, int64_t shb, int64_t scb, void* stream) {
  TSSM_CHECK(vhat && h && Abar && Bbar && C && D && y, TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && H >= 0 && grid_b >= 0 && h_cover >= 0 && grid_b <= nbatch &&
                 h_cover <= H,
             TSSM_ERR_SHAPE);
  if (grid_b == 0 || h_cover == 0) return TSSM_OK;
  const uintptr_t al = dtype == TSSM_F32 ? 16 : 8;
  const bool v4 = h_cover % 4 == 0 && svb % 4 == 0 && shb % 4 == 0 && scb % 4 == 0 &&
                  aligned(vhat, al) && aligned(h, al) && aligned(Abar, al) && aligned(Bbar, al) &&
                  aligned(C, al) && aligned(D, al) && aligned(y, al);
  const int64_t V = v4 ? 4 : 1;
  const int64_t gy = (h_cover + 256 * V - 1) / (256 * V);
  const int64_t gx = (grid_b + kStepRows - 1) / kStepRows;
  TSSM_CHECK(gy <= 65535 && gx <= 2147483647, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)gx, (unsigned)gy);
  const hipStream_t s = as_stream(stream);
#define TSSM_S(T)                                                                               \
  if (v4)                                                                                       \
    hipLaunchKernelGGL((stream_step_kernel<T, 4>), grid, dim3(256), 0, s, (const T*)vhat, (T*)h, \
                       (const T*)Abar, (const T*)Bbar, (const T*)C, (const T*)D, (T*)y,          \
                       h_cover, grid_b, svb, shb, scb);                                          \
  else                                                                                          \
    hipLaunchKernelGGL((stream_step_kernel<T, 1>), grid, dim3(256), 0, s, (const T*)vhat, (T*)h, \
                       (const T*)Abar, (const T*)Bbar, (const T*)C, (const T*)D, (T*)y,          \
                       h_cover, grid_b, svb, shb, scb)
  switch (dtype) {
    case TSSM_F32: TSSM_S(float); break;
    case TSSM_BF16: TSSM_S(bf16_t); break;
    case TSSM_F16: TSSM_S(f16_t); break;
    default: return TSSM_ERR_DTYPE;
  }
#undef TSSM_S
  return launch_status();
}

extern "C" int tssm_stream_interp_step(float* ring_V, float* ring_M, float* ring_tau,
                                       int32_t* ring_head, const float* v_new,
                                       const float* m_new, const float* tau_new, float* h,
                                       const float* Abar, const float* Bbar, const float* C,
                                       const float* D, float* y, int64_t nbatch, int64_t H,
                                       int64_t srb, int64_t srk, int64_t svb, int64_t shb,
                                       int64_t scb, int64_t BLOCK_H, int64_t KRING,
                                       int64_t grid_b, void* stream) {
  TSSM_CHECK(ring_V && ring_M && ring_tau && ring_head && v_new && m_new && tau_new && h &&
                 Abar && Bbar && C && D && y,
             TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && H >= 0 && BLOCK_H > 0 && KRING > 0 && grid_b >= 0 &&
                 grid_b <= nbatch,
             TSSM_ERR_SHAPE);
  if (grid_b == 0 || H == 0) return TSSM_OK;
  RingArgs a{ring_V, ring_M, ring_tau, ring_head, v_new, m_new, tau_new, h, Abar, Bbar, C, D, y,
             H, srb, srk, svb, shb, scb, BLOCK_H, KRING};
  const bool vec = (BLOCK_H == 16 || BLOCK_H == 32 || BLOCK_H == 64 || BLOCK_H == 128 ||
                    BLOCK_H == 256) && KRING - 1 <= kRingFast &&
                   H % 4 == 0 && srb % 4 == 0 && srk % 4 == 0 && svb % 4 == 0 && shb % 4 == 0 &&
                   scb % 4 == 0 && aligned(ring_V, 16) && aligned(ring_M, 16) &&
                   aligned(v_new, 16) && aligned(m_new, 16) && aligned(h, 16) &&
                   aligned(Abar, 16) && aligned(Bbar, 16) && aligned(C, 16) && aligned(D, 16) &&
                   aligned(y, 16);
  const dim3 grid((unsigned)grid_b), block(kStreamThreads);
  const hipStream_t s = as_stream(stream);
  if (vec) {
    switch (BLOCK_H) {
      case 16: hipLaunchKernelGGL(stream_interp_step_vec_kernel<4>, grid, block, 0, s, a); break;
      case 32: hipLaunchKernelGGL(stream_interp_step_vec_kernel<8>, grid, block, 0, s, a); break;
      case 64: hipLaunchKernelGGL(stream_interp_step_vec_kernel<16>, grid, block, 0, s, a); break;
      case 128: hipLaunchKernelGGL(stream_interp_step_vec_kernel<32>, grid, block, 0, s, a); break;
      default: hipLaunchKernelGGL(stream_interp_step_vec_kernel<64>, grid, block, 0, s, a); break;
    }
  } else {
    hipLaunchKernelGGL(stream_interp_step_kernel, grid, block, 0, s, a);
  }
  return launch_status();
}

extern "C" int tssm_stream_interp_step_corrected(
    float* ring_V, float* ring_M, float* ring_tau, int32_t* ring_head, const float* v_new,
    const float* m_new, const float* tau_new, float* h, const float* Abar, const float* Bbar,
    const float* C, const float* D, float* y, int64_t nbatch, int64_t H, int64_t srb,
    int64_t srk, int64_t svb, int64_t shb, int64_t scb, int64_t KRING, void* stream) {
  TSSM_CHECK(ring_V && ring_M && ring_tau && ring_head && v_new && m_new && tau_new && h &&
                 Abar && Bbar && C && D && y,
             TSSM_ERR_NULL);
  TSSM_CHECK(nbatch >= 0 && H >= 0 && KRING > 0, TSSM_ERR_SHAPE);
  if (nbatch == 0 || H == 0) return TSSM_OK;
  TSSM_CHECK(nbatch <= 2147483647, TSSM_ERR_UNSUPPORTED);
  RingArgs a{ring_V, ring_M, ring_tau, ring_head, v_new, m_new, tau_new, h, Abar, Bbar, C, D, y,
             H, srb, srk, svb, shb, scb, 1, KRING};
  const bool vec = KRING - 1 <= kRingFast && H % 4 == 0 && srb % 4 == 0 && srk % 4 == 0 &&
                   svb % 4 == 0 && shb % 4 == 0 && scb % 4 == 0 && aligned(ring_V, 16) &&
                   aligned(ring_M, 16) && aligned(v_new, 16) && aligned(m_new, 16) &&
                   aligned(h, 16) && aligned(Abar, 16) && aligned(Bbar, 16) && aligned(C, 16) &&
                   aligned(D, 16) && aligned(y, 16);
  if (vec)
    hipLaunchKernelGGL(stream_interp_step_corrected_vec_kernel, dim3((unsigned)nbatch),
                       dim3(kStreamThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(stream_interp_step_corrected_kernel, dim3((unsigned)nbatch),
                       dim3(kStreamThreads), 0, as_stream(stream), a);
  return launch_status();
}
