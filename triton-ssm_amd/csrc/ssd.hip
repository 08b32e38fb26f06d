// SSD selective scan (scalar decay per head, state P x N per (batch, head)).
//
//   h_t[p, n] = exp(dt_t a) h_{t-1}[p, n] + Bbar_t x_t[p] B_t[n]
//   y_t[p]    = sum_n C_t[n] h_t[p, n] + D[p] x_t[p]
// with Bbar_t = dt_t (Euler) or expm1(dt_t a)/a (ZOH) -- the recurrence of
// ssm_scan.py:5-10 with the discretization of discretize_kernel.py:44-54 and
// one decay per head.
//
// ssd_scan_kernel: single pass with decoupled look-back.
//   tile = (row = b*H + h, chunk c of TC = 4*RUN steps), numbered chunk-major
//   (blockIdx = c * rows + row): with few rows and many chunks, a tile's
//   predecessor is a whole layer of rows earlier in launch order.
//   4 waves = 4 runs of RUN steps; lane = channel p with the N state values of
//   its row p in registers.  The per-step decay and input coefficient are
//   computed once per tile into LDS; B_t and C_t are wave-uniform.
//   sweep 1: each run's local state from zero -> runs combined in LDS ->
//   the last wave publishes the tile aggregate (one decay word + P*N state
//   words), looks back for the entry state, publishes the inclusive state ->
//   sweep 2: each run rescans from its exact entry state and writes y.
// ssd_stream_step_kernel: one streaming step with the state [S,H,P,N] fp32
//   resident in HBM, updated in place; one workgroup per (stream, head).
#include "common.h"
#include "lookback.h"

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
  WsHeader* hdr;
  uint64_t* words;
  uint32_t H, P, rows, nchunks, run, tag, spin_limit;
};

constexpr int kSsdWaves = 4;

// B_t[n] / C_t[n] for all n of one step, wave-uniform, converted to fp32.
template <typename T, int N>
__device__ inline void load_row(const T* __restrict__ p, float* out) {
#pragma unroll
  for (int n = 0; n < N; ++n) out[n] = ldf(p + n);
}

template <typename T, int DISC, int N, bool HAS_D>
__global__ __launch_bounds__(256) void ssd_scan_kernel(SsdArgs a) {
  extern __shared__ float s_mem[];
  const int RUN = (int)a.run;
  const int TC = RUN * kSsdWaves;
  const int P = (int)a.P;
  float* s_ab = s_mem;                         // [TC] decay per step
  float* s_cf = s_ab + TC;                     // [TC] input coefficient per step
  float* s_ra = s_cf + TC;                     // [4] run decay products
  float* s_rx = s_ra + kSsdWaves;              // [4][P][N] run local states -> entry prefixes
  float* s_carry = s_rx + kSsdWaves * P * N;   // [P][N] tile entry state

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p = tid & 63;
  const bool act = p < P;
  const uint32_t c = blockIdx.x / a.rows;
  const uint32_t row = blockIdx.x - c * a.rows;
  const uint32_t b = row / a.H;
  const uint32_t h = row - b * a.H;
  const int64_t tile_t0 = (int64_t)c * TC;
  const float a2 = -expf(a.A_log[h]) * kLog2e;

  // ---- per-step decay and input coefficient, once per tile
  const float* dtp = a.dt + b * a.sdt_b + h * a.sdt_h;
  for (int i = tid; i < TC; i += blockDim.x) {
    const int64_t t = tile_t0 + i;
    const float d = t < a.L ? dtp[t * a.sdt_l] : 0.0f;
    const float arg = d * a2;
    const float ab = exp2_fast(arg);
    s_ab[i] = ab;
    s_cf[i] = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(arg * 0.6931471805599453f, ab) * d : d;
  }
  __syncthreads();

  const int64_t t0 = tile_t0 + (int64_t)wave * RUN;
  int nsteps = RUN;
  if (t0 >= a.L) nsteps = 0;
  else if (t0 + RUN > a.L) nsteps = (int)(a.L - t0);
  const T* xp = reinterpret_cast<const T*>(a.x) + b * a.sx_b + h * a.sx_h + (act ? p : 0);
  const T* Bp = reinterpret_cast<const T*>(a.B) + b * a.sB_b + h * a.sB_h;
  const T* Cp = reinterpret_cast<const T*>(a.C) + b * a.sC_b + h * a.sC_h;
  const float* ab_run = s_ab + wave * RUN;
  const float* cf_run = s_cf + wave * RUN;

  // ---- sweep 1: local state of the run from zero
  float st[N];
#pragma unroll
  for (int n = 0; n < N; ++n) st[n] = 0.0f;
  float A_run = 1.0f;
  for (int i = 0; i < nsteps; ++i) {
    const int64_t t = t0 + i;
    const float ab = ab_run[i];
    const float xs = cf_run[i] * ldf(xp + t * a.sx_l);
    float bv[N];
    load_row<T, N>(Bp + t * a.sB_l, bv);
#pragma unroll
    for (int n = 0; n < N; ++n) st[n] = __builtin_fmaf(ab, st[n], xs * bv[n]);
    A_run *= ab;
  }
  if (act) {
#pragma unroll
    for (int n = 0; n < N; ++n) s_rx[(wave * P + p) * N + n] = st[n];
  }
  if (p == 0) s_ra[wave] = A_run;
  __syncthreads();

  // ---- combine runs: entry prefix of each run within the tile; the last
  //      wave resolves the tile's carry
  {
    float PA = 1.0f;
    float PX[N];
#pragma unroll
    for (int n = 0; n < N; ++n) PX[n] = 0.0f;
    for (int w = 0; w < wave; ++w) {
      const float wa = s_ra[w];
#pragma unroll
      for (int n = 0; n < N; ++n)
        PX[n] = __builtin_fmaf(wa, PX[n], act ? s_rx[(w * P + p) * N + n] : 0.0f);
      PA *= wa;
    }
    __syncthreads();  // every wave has read the run states it needs
    if (act) {
#pragma unroll
      for (int n = 0; n < N; ++n) s_rx[(wave * P + p) * N + n] = PX[n];
    }
    if (wave == kSsdWaves - 1) {
      // tile aggregate = (this run) o (prefix of earlier runs)
      const float TA = A_run * PA;
      float TX[N];
#pragma unroll
      for (int n = 0; n < N; ++n) TX[n] = __builtin_fmaf(A_run, PX[n], st[n]);
      const int64_t cw = (int64_t)P * N;  // state words per tile
      uint64_t* tile0 = a.words + (int64_t)row * a.nchunks * (2 * cw + 1);
      // layout per tile: [agg_a (1)] [agg_x (cw)] [inc (cw)]
      uint64_t* mine = tile0 + (int64_t)c * (2 * cw + 1);
      if (c > 0 && act) {
        if (p == 0) st_word(mine, TA, a.tag);
#pragma unroll
        for (int n = 0; n < N; ++n) st_word(mine + 1 + p * N + n, TX[n], a.tag);
      }
      float cin[N];
#pragma unroll
      for (int n = 0; n < N; ++n) cin[n] = (a.h0 && act) ? a.h0[((int64_t)row * P + p) * N + n] : 0.0f;
      if (c > 0 && act) {
        // walk back: all N words of a predecessor must carry the tag
        float Aacc = 1.0f, Xacc[N];
#pragma unroll
        for (int n = 0; n < N; ++n) Xacc[n] = 0.0f;
        int64_t j = (int64_t)c - 1;
        uint32_t spins = 0;
        bool done = false;
        while (j >= 0 && !done) {
          const uint64_t* pj = tile0 + j * (2 * cw + 1);
          uint64_t wi[N], wx[N];
          const uint64_t wa = ld_word(pj);
#pragma unroll
          for (int n = 0; n < N; ++n) {
            wi[n] = ld_word(pj + 1 + cw + p * N + n);
            wx[n] = ld_word(pj + 1 + p * N + n);
          }
          bool inc_ok = true, agg_ok = word_tag(wa) == a.tag;
#pragma unroll
          for (int n = 0; n < N; ++n) {
            inc_ok = inc_ok && word_tag(wi[n]) == a.tag;
            agg_ok = agg_ok && word_tag(wx[n]) == a.tag;
          }
          if (inc_ok) {
#pragma unroll
            for (int n = 0; n < N; ++n) cin[n] = __builtin_fmaf(Aacc, word_val(wi[n]), Xacc[n]);
            done = true;
          } else if (agg_ok) {
            const float ja = word_val(wa);
#pragma unroll
            for (int n = 0; n < N; ++n) Xacc[n] = __builtin_fmaf(Aacc, word_val(wx[n]), Xacc[n]);
            Aacc *= ja;
            --j;
          } else {
            if (++spins > a.spin_limit) {
              flag_error(a.hdr);
#pragma unroll
              for (int n = 0; n < N; ++n) cin[n] = Xacc[n];
              done = true;
            } else {
              __builtin_amdgcn_s_sleep(1);
            }
          }
        }
        if (!done) {  // reached the row start: fold h0
#pragma unroll
          for (int n = 0; n < N; ++n) cin[n] = __builtin_fmaf(Aacc, cin[n], Xacc[n]);
        }
      }
      if (act) {
#pragma unroll
        for (int n = 0; n < N; ++n) {
          const float incl = __builtin_fmaf(TA, cin[n], TX[n]);
          st_word(mine + 1 + cw + p * N + n, incl, a.tag);
          s_carry[p * N + n] = cin[n];
          if (a.h_last && c == a.nchunks - 1) a.h_last[((int64_t)row * P + p) * N + n] = incl;
        }
      }
    }
    __syncthreads();
    // entry state of this run = prefix o carry
    if (act) {
#pragma unroll
      for (int n = 0; n < N; ++n)
        st[n] = __builtin_fmaf(PA, s_carry[p * N + n], s_rx[(wave * P + p) * N + n]);
    }
  }

  // ---- sweep 2: rescan the run from its exact entry state, write y
  const float dv = (HAS_D && act) ? a.D[h * P + p] : 0.0f;
  T* yp = reinterpret_cast<T*>(a.y) + b * a.sy_b + h * a.sy_h + p;
  for (int i = 0; i < nsteps; ++i) {
    const int64_t t = t0 + i;
    const float ab = ab_run[i];
    const float xv = ldf(xp + t * a.sx_l);
    const float xs = cf_run[i] * xv;
    float bv[N], cv[N];
    load_row<T, N>(Bp + t * a.sB_l, bv);
    load_row<T, N>(Cp + t * a.sC_l, cv);
    float acc = HAS_D ? dv * xv : 0.0f;
#pragma unroll
    for (int n = 0; n < N; ++n) {
      st[n] = __builtin_fmaf(ab, st[n], xs * bv[n]);
      acc = __builtin_fmaf(cv[n], st[n], acc);
    }
    if (act) stf(yp + t * a.sy_l, acc);
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

template <typename T, int DISC, bool HAS_D>
int launch_ssd_n(int N, dim3 grid, size_t lds, hipStream_t s, const SsdArgs& a) {
  switch (N) {
    case 8: hipLaunchKernelGGL((ssd_scan_kernel<T, DISC, 8, HAS_D>), grid, dim3(256), lds, s, a); break;
    case 16: hipLaunchKernelGGL((ssd_scan_kernel<T, DISC, 16, HAS_D>), grid, dim3(256), lds, s, a); break;
    case 32: hipLaunchKernelGGL((ssd_scan_kernel<T, DISC, 32, HAS_D>), grid, dim3(256), lds, s, a); break;
    default: return TSSM_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <typename T>
int launch_ssd_t(int disc, bool has_d, int N, dim3 grid, size_t lds, hipStream_t s,
                 const SsdArgs& a) {
  if (disc == TSSM_DISC_ZOH)
    return has_d ? launch_ssd_n<T, TSSM_DISC_ZOH, true>(N, grid, lds, s, a)
                 : launch_ssd_n<T, TSSM_DISC_ZOH, false>(N, grid, lds, s, a);
  return has_d ? launch_ssd_n<T, TSSM_DISC_EULER, true>(N, grid, lds, s, a)
               : launch_ssd_n<T, TSSM_DISC_EULER, false>(N, grid, lds, s, a);
}

inline int ssd_run(int64_t chunk) {
  int64_t run = chunk / kSsdWaves;
  if (run < 16) run = 16;
  if (run > 256) run = 256;
  return (int)run;
}

}  // namespace tssm

using namespace tssm;

extern "C" int64_t tssm_ssd_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t H, int64_t P,
                                                 int64_t N, int64_t chunk) {
  if (nbatch <= 0 || L <= 0 || H <= 0 || P <= 0 || P > 64 || N <= 0) return -1;
  const int64_t tc = (int64_t)ssd_run(chunk) * kSsdWaves;
  const int64_t nchunks = cdiv64(L, tc);
  return (int64_t)sizeof(WsHeader) + nbatch * H * nchunks * (2 * P * N + 1) * 8;
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
  const int run = ssd_run(chunk);
  const int64_t nchunks = cdiv64(L, (int64_t)run * kSsdWaves);
  const int64_t rows = nbatch * H;
  TSSM_CHECK(nchunks * rows < (int64_t)INT32_MAX, TSSM_ERR_UNSUPPORTED);
  SsdArgs a;
  a.x = x; a.dt = dt; a.A_log = A_log; a.B = B; a.C = C; a.D = D; a.h0 = h0; a.y = y;
  a.h_last = h_last; a.L = L;
  a.sx_b = sx_b; a.sx_l = sx_l; a.sx_h = sx_h; a.sdt_b = sdt_b; a.sdt_l = sdt_l; a.sdt_h = sdt_h;
  a.sB_b = sB_b; a.sB_l = sB_l; a.sB_h = sB_h; a.sC_b = sC_b; a.sC_l = sC_l; a.sC_h = sC_h;
  a.sy_b = sy_b; a.sy_l = sy_l; a.sy_h = sy_h;
  a.hdr = reinterpret_cast<WsHeader*>(workspace);
  a.words = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + sizeof(WsHeader));
  a.H = (uint32_t)H; a.P = (uint32_t)P; a.rows = (uint32_t)rows; a.nchunks = (uint32_t)nchunks;
  a.run = (uint32_t)run; a.tag = next_epoch(workspace); a.spin_limit = kDefaultSpinLimit;
  const size_t lds = ((size_t)2 * run * kSsdWaves + kSsdWaves + (size_t)(kSsdWaves + 1) * P * N) *
                     sizeof(float);
  TSSM_CHECK(lds <= 65536, TSSM_ERR_UNSUPPORTED);
  const dim3 grid((unsigned)(nchunks * rows));
  const hipStream_t s = as_stream(stream);
  const bool has_d = D != nullptr;
  switch (dtype) {
    case TSSM_BF16: return launch_ssd_t<bf16_t>(disc, has_d, (int)N, grid, lds, s, a);
    case TSSM_F16: return launch_ssd_t<f16_t>(disc, has_d, (int)N, grid, lds, s, a);
    default: return launch_ssd_t<float>(disc, has_d, (int)N, grid, lds, s, a);
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
