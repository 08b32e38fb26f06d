// Elementwise scan, single pass: the host functions ssm_forward and
// ssm_backward (ssm_scan.py:239-289) without their intermediate arrays.
//
//   forward   h_t = A_t h_{t-1} + B_t u_t,  y_t = C_t h_t + D u_t
//   backward  dh_t = A_{t+1} dh_{t+1} + C_t dY_t (dh_L = 0),
//             du = B dh, dB = u dh, dA = h_{t-1} dh, dC = dY h
//             (du without a D dY term, as the reference, :226)
// over contiguous [B, L, H] tensors.  The reference runs four kernels and
// moves loc_a/loc_x (or loc_dh) and the carries through HBM; here every
// input is read once and every output written once.
//
// Tile = (batch b, block of 64 lanes h, chunk of 64 steps); 256 threads,
// each owning 4 consecutive lanes (one 16-byte fp32 / 8-byte 16-bit access)
// of a run of 4 steps, so one load instruction of a wave reads 4 runs x 256
// contiguous bytes.  Within a tile: a local scan per run in registers, a
// scan over the 16 runs through LDS, then a decoupled look-back over the
// chunks of the (b, lane block) row for the state entering the tile (tagged
// carry words, lookback.h).  The backward kernel runs the same machinery in
// reverse time: chunk c is the logical chunk nchunks-1-c, so every tile still
// waits only on tiles of smaller launch index.
#include "common.h"
#include "lookback.h"

namespace tssm {
namespace {

constexpr int kV = 4;                  // lanes per thread
constexpr int kG = 16;                 // threads per run
constexpr int kR = 4;                  // steps per run
constexpr int kW = 4;                  // waves per workgroup (4: backward 8% faster than 8)
constexpr int kRowsW = 64 / kG;        // runs per wave
constexpr int kRuns = kW * kRowsW;     // runs per tile (16)
constexpr int kTC = kRuns * kR;        // steps per tile (64)
constexpr int kLanes = kG * kV;        // lanes per tile (64)
static_assert(kLanes == 64, "the look-back walks one whole wave per tile");
constexpr int kSeg = 4;                // runs per run-scan segment
constexpr int kSegs = kRuns / kSeg;    // 4: kSegs * kLanes == threads
static_assert(kSegs * kLanes == kW * 64, "run scan covers the workgroup");

struct EwArgs {
  const void* u;
  const void* A;
  const void* B;
  const void* C;
  const void* D;
  const void* h;    // backward: the forward states
  const void* dY;   // backward
  void* o0;         // forward: y;  backward: du
  void* o1;         // forward: h;  backward: dA
  void* o2;         // backward: dB
  void* o3;         // backward: dC
  int64_t L, H, nlb;
  uint32_t nchunks;
  WsHeader* hdr;
  uint64_t* words;
  uint64_t* status;  // TileStatus of every row: [rows][nchunks][2]
  uint32_t tag, spin_limit;
};

// Thread geometry of a tile.
struct EwTile {
  int tid, ch0, run;
  uint32_t row, c;   // c = logical chunk (look-back order)
  int64_t b, h0;
  __device__ EwTile(const EwArgs& a) {
    tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    ch0 = (lane % kG) * kV;
    run = wave * kRowsW + lane / kG;
    row = blockIdx.x / a.nchunks;
    c = blockIdx.x - row * a.nchunks;
    b = row / a.nlb;
    h0 = (int64_t)(row - b * a.nlb) * kLanes + ch0;
  }
};

// Scan over the tile's runs (s_a/s_x hold run aggregates in scan order) and
// the look-back: on return s_a/s_x hold each run's exclusive prefix within
// the tile and s_carry the state entering the tile, per lane.
__device__ inline void tile_scan(const EwArgs& a, const EwTile& t, float (*s_a)[kLanes],
                                 float (*s_x)[kLanes],
                                 float (*s_sa)[kLanes], float (*s_sx)[kLanes], float* s_carry) {
  const int ch = t.tid % kLanes, sg = t.tid / kLanes;
  const int q0 = sg * kSeg;
  float ea[kSeg], ex[kSeg];
  float A = 1.0f, X = 0.0f;
#pragma unroll
  for (int q = 0; q < kSeg; ++q) {
    const float ra = s_a[q0 + q][ch], rx = s_x[q0 + q][ch];
    ea[q] = A;
    ex[q] = X;
    X = __builtin_fmaf(ra, X, rx);
    A = A * ra;
  }
  s_sa[sg][ch] = A;
  s_sx[sg][ch] = X;
  __syncthreads();
  float SA = 1.0f, SX = 0.0f;
  for (int k = 0; k < sg; ++k) {
    const float ka = s_sa[k][ch];
    SX = __builtin_fmaf(ka, SX, s_sx[k][ch]);
    SA = SA * ka;
  }
#pragma unroll
  for (int q = 0; q < kSeg; ++q) {
    s_a[q0 + q][ch] = ea[q] * SA;
    s_x[q0 + q][ch] = __builtin_fmaf(ea[q], SX, ex[q]);
  }
  if (sg == kSegs - 1) {
    const float TA = A * SA, TX = __builtin_fmaf(A, SX, X);
    // every lane publishes; lanes past H (their runs read lane 0) are never stored
    CarrySlot slot{a.words + (int64_t)t.row * a.nchunks * 3 * kLanes, 3 * kLanes, kLanes};
    const TileStatus tst{a.status + (int64_t)t.row * a.nchunks * 2};
    if (t.c > 0) {
      st_word(slot.agg_a(t.c, ch), TA, a.tag);
      st_word(slot.agg_x(t.c, ch), TX, a.tag);
      if (ch == 0) st_word(tst.agg(t.c), 0.0f, a.tag);
    }
    // a tile whose decay product is exactly zero forgets its entry state:
    // its inclusive state is published before the look-back
    const bool forgets = TA == 0.0f;
    if (forgets) st_word(slot.inc(t.c, ch), TX, a.tag);
    // one whole wave (kLanes == 64) walks back by the status words
    const float carry = t.c > 0 ? lookback_wave<16, 4>(slot, tst, t.c, ch, a.tag, 0.0f,
                                                       a.spin_limit, a.hdr)
                                : 0.0f;
    if (!forgets) st_word(slot.inc(t.c, ch), __builtin_fmaf(TA, carry, TX), a.tag);
    if (ch == 0) st_word(tst.inc(t.c), 0.0f, a.tag);
    s_carry[ch] = carry;
  }
  __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(kW * 64) void ew_scan_fwd_kernel(EwArgs a) {
  __shared__ float s_a[kRuns][kLanes], s_x[kRuns][kLanes];
  __shared__ float s_sa[kSegs][kLanes], s_sx[kSegs][kLanes];
  __shared__ float s_carry[kLanes];
  const EwTile t(a);
  const bool lanes_ok = t.h0 < a.H;            // all 4 lanes (H % 4 == 0)
  const int64_t hs = lanes_ok ? t.h0 : 0;      // lanes past H read lane 0, store nothing
  const int64_t t0 = (int64_t)t.c * kTC + (int64_t)t.run * kR;
  const int64_t base = t.b * a.L * a.H + hs;
  // loads, rows past L read row L-1 (no branch around the loads)
  float u[kR][kV], Av[kR][kV], Bv[kR][kV], Cv[kR][kV], Dv[kV];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t tt = t0 + r < a.L ? t0 + r : a.L - 1;
    const int64_t o = base + tt * a.H;
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.u) + o, u[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.A) + o, Av[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.B) + o, Bv[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.C) + o, Cv[r]);
  }
  ld_lanes<T, kV>(reinterpret_cast<const T*>(a.D) + hs, Dv);
  __builtin_amdgcn_sched_barrier(0);
  // local scan of the run; steps past L are identities (A = 1, B u = 0)
  float al[kV], xl[kV], pa[kR][kV], px[kR][kV];
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    al[v] = 1.0f;
    xl[v] = 0.0f;
  }
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const bool ok = t0 + r < a.L;
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      const float av = ok ? Av[r][v] : 1.0f;
      const float bu = ok ? Bv[r][v] * u[r][v] : 0.0f;
      xl[v] = __builtin_fmaf(av, xl[v], bu);
      al[v] = al[v] * av;
      pa[r][v] = al[v];
      px[r][v] = xl[v];
    }
  }
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    s_a[t.run][t.ch0 + v] = al[v];
    s_x[t.run][t.ch0 + v] = xl[v];
  }
  __syncthreads();
  tile_scan(a, t, s_a, s_x, s_sa, s_sx, s_carry);
  float S[kV];
#pragma unroll
  for (int v = 0; v < kV; ++v)
    S[v] = __builtin_fmaf(s_a[t.run][t.ch0 + v], s_carry[t.ch0 + v], s_x[t.run][t.ch0 + v]);
  if (!lanes_ok) return;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (t0 + r >= a.L) break;
    float hv[kV], yv[kV];
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      hv[v] = __builtin_fmaf(pa[r][v], S[v], px[r][v]);
      yv[v] = __builtin_fmaf(Cv[r][v], hv[v], Dv[v] * u[r][v]);
    }
    const int64_t o = base + (t0 + r) * a.H;
    st_lanes<T, kV>(reinterpret_cast<T*>(a.o1) + o, hv);
    st_lanes<T, kV>(reinterpret_cast<T*>(a.o0) + o, yv);
  }
}

template <typename T>
__global__ __launch_bounds__(kW * 64) void ew_scan_bwd_kernel(EwArgs a) {
  __shared__ float s_a[kRuns][kLanes], s_x[kRuns][kLanes];
  __shared__ float s_sa[kSegs][kLanes], s_sx[kSegs][kLanes];
  __shared__ float s_carry[kLanes];
  const EwTile t(a);
  const bool lanes_ok = t.h0 < a.H;
  const int64_t hs = lanes_ok ? t.h0 : 0;
  // logical chunk c covers time chunk nchunks-1-c; runs are scanned latest first
  const int64_t tc = (int64_t)(a.nchunks - 1 - t.c);
  const int64_t t0 = tc * kTC + (int64_t)t.run * kR;
  const int srun = kRuns - 1 - t.run;          // the run's position in scan order
  const int64_t base = t.b * a.L * a.H + hs;
  const int64_t last = a.L - 1;
  auto clamp = [&](int64_t tt) { return tt < 0 ? 0 : (tt > last ? last : tt); };
  // sweep-1 operands: A_{t+1}, C_t, dY_t, h_t
  float An[kR][kV], Cv[kR][kV], dYv[kR][kV], hv[kR][kV];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t o = base + clamp(t0 + r) * a.H;
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.A) + base + clamp(t0 + r + 1) * a.H, An[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.C) + o, Cv[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.dY) + o, dYv[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.h) + o, hv[r]);
  }
  __builtin_amdgcn_sched_barrier(0);
  float al[kV], xl[kV], pa[kR][kV], px[kR][kV];
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    al[v] = 1.0f;
    xl[v] = 0.0f;
  }
#pragma unroll
  for (int r = kR - 1; r >= 0; --r) {
    const bool ok = t0 + r < a.L;
    const bool has_next = t0 + r + 1 < a.L;
    float dC[kV];
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      const float av = ok ? (has_next ? An[r][v] : 0.0f) : 1.0f;
      const float cv = ok ? Cv[r][v] * dYv[r][v] : 0.0f;
      xl[v] = __builtin_fmaf(av, xl[v], cv);
      al[v] = al[v] * av;
      pa[r][v] = al[v];
      px[r][v] = xl[v];
      dC[v] = dYv[r][v] * hv[r][v];
    }
    if (ok && lanes_ok)
      st_lanes<T, kV>(reinterpret_cast<T*>(a.o3) + base + (t0 + r) * a.H, dC);
  }
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    s_a[srun][t.ch0 + v] = al[v];
    s_x[srun][t.ch0 + v] = xl[v];
  }
  // sweep-2 operands, in flight during the scans: u_t, B_t, h_{t-1}
  float uv[kR][kV], Bv[kR][kV], hp[kV];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t o = base + clamp(t0 + r) * a.H;
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.u) + o, uv[r]);
    ld_lanes<T, kV>(reinterpret_cast<const T*>(a.B) + o, Bv[r]);
  }
  ld_lanes<T, kV>(reinterpret_cast<const T*>(a.h) + base + clamp(t0 - 1) * a.H, hp);
  __syncthreads();
  tile_scan(a, t, s_a, s_x, s_sa, s_sx, s_carry);
  float S[kV], hprev[kV];
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    S[v] = __builtin_fmaf(s_a[srun][t.ch0 + v], s_carry[t.ch0 + v], s_x[srun][t.ch0 + v]);
    hprev[v] = t0 > 0 ? hp[v] : 0.0f;
  }
  if (!lanes_ok) return;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (t0 + r >= a.L) break;
    float du[kV], dA[kV], dB[kV];
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      const float dh = __builtin_fmaf(pa[r][v], S[v], px[r][v]);
      du[v] = Bv[r][v] * dh;
      dB[v] = uv[r][v] * dh;
      dA[v] = hprev[v] * dh;
      hprev[v] = hv[r][v];
    }
    const int64_t o = base + (t0 + r) * a.H;
    st_lanes<T, kV>(reinterpret_cast<T*>(a.o0) + o, du);
    st_lanes<T, kV>(reinterpret_cast<T*>(a.o1) + o, dA);
    st_lanes<T, kV>(reinterpret_cast<T*>(a.o2) + o, dB);
  }
}

inline int64_t cdiv(int64_t x, int64_t y) { return (x + y - 1) / y; }

int ew_check(int dtype, int64_t nbatch, int64_t L, int64_t H) {
  TSSM_CHECK(dtype == TSSM_F32 || dtype == TSSM_BF16 || dtype == TSSM_F16, TSSM_ERR_DTYPE);
  TSSM_CHECK(nbatch > 0 && L > 0 && H > 0, TSSM_ERR_SHAPE);
  TSSM_CHECK(H % kV == 0, TSSM_ERR_UNSUPPORTED);
  return TSSM_OK;
}

int ew_setup(EwArgs& a, int64_t nbatch, int64_t L, int64_t H, void* workspace,
             int64_t workspace_bytes, int64_t need, dim3* grid) {
  TSSM_CHECK(workspace != nullptr && workspace_bytes >= need, TSSM_ERR_WORKSPACE);
  TSSM_CHECK(aligned(workspace, 256), TSSM_ERR_ALIGN);
  a.L = L;
  a.H = H;
  a.nlb = cdiv(H, kLanes);
  const int64_t nch = cdiv(L, kTC);
  const int64_t ntiles = nbatch * a.nlb * nch;
  TSSM_CHECK(ntiles <= 2147483647, TSSM_ERR_UNSUPPORTED);
  a.nchunks = (uint32_t)nch;
  a.hdr = reinterpret_cast<WsHeader*>(workspace);
  a.words = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(workspace) + sizeof(WsHeader));
  a.status = a.words + ntiles * 3 * kLanes;
  a.tag = next_epoch(workspace);
  a.spin_limit = kDefaultSpinLimit;
  *grid = dim3((unsigned)ntiles);
  return TSSM_OK;
}

}  // namespace
}  // namespace tssm

using namespace tssm;

extern "C" int64_t tssm_ssm_scan_fused_workspace_bytes(int64_t nbatch, int64_t L, int64_t H) {
  if (nbatch <= 0 || L <= 0 || H <= 0) return -1;
  // header | carry words [tiles][3][kLanes] | status words [tiles][2]
  return (int64_t)sizeof(WsHeader) +
         nbatch * cdiv(H, kLanes) * cdiv(L, kTC) * (3 * kLanes + 2) * (int64_t)sizeof(uint64_t);
}

extern "C" int tssm_ssm_forward_fused(int dtype, const void* u, const void* A, const void* B,
                                      const void* C, const void* D, void* y, void* h,
                                      int64_t nbatch, int64_t L, int64_t H, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  TSSM_CHECK(u && A && B && C && D && y && h, TSSM_ERR_NULL);
  int st = ew_check(dtype, nbatch, L, H);
  if (st != TSSM_OK) return st;
  const int64_t al = dtype == TSSM_F32 ? 16 : 8;
  TSSM_CHECK(aligned(u, al) && aligned(A, al) && aligned(B, al) && aligned(C, al) &&
                 aligned(D, al) && aligned(y, al) && aligned(h, al), TSSM_ERR_ALIGN);
  EwArgs a{};
  a.u = u; a.A = A; a.B = B; a.C = C; a.D = D; a.o0 = y; a.o1 = h;
  dim3 grid;
  st = ew_setup(a, nbatch, L, H, workspace, workspace_bytes,
                tssm_ssm_scan_fused_workspace_bytes(nbatch, L, H), &grid);
  if (st != TSSM_OK) return st;
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case TSSM_F32: hipLaunchKernelGGL(ew_scan_fwd_kernel<float>, grid, dim3(kW * 64), 0, s, a); break;
    case TSSM_BF16: hipLaunchKernelGGL(ew_scan_fwd_kernel<bf16_t>, grid, dim3(kW * 64), 0, s, a); break;
    default: hipLaunchKernelGGL(ew_scan_fwd_kernel<f16_t>, grid, dim3(kW * 64), 0, s, a); break;
  }
  return launch_status();
}

extern "C" int tssm_ssm_backward_fused(int dtype, const void* u, const void* A, const void* B,
                                       const void* C, const void* h, const void* dY, void* du,
                                       void* dA, void* dB, void* dC, int64_t nbatch, int64_t L,
                                       int64_t H, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  TSSM_CHECK(u && A && B && C && h && dY && du && dA && dB && dC, TSSM_ERR_NULL);
  int st = ew_check(dtype, nbatch, L, H);
  if (st != TSSM_OK) return st;
  const int64_t al = dtype == TSSM_F32 ? 16 : 8;
  TSSM_CHECK(aligned(u, al) && aligned(A, al) && aligned(B, al) && aligned(C, al) &&
                 aligned(h, al) && aligned(dY, al) && aligned(du, al) && aligned(dA, al) &&
                 aligned(dB, al) && aligned(dC, al), TSSM_ERR_ALIGN);
  EwArgs a{};
  a.u = u; a.A = A; a.B = B; a.C = C; a.h = h; a.dY = dY;
  a.o0 = du; a.o1 = dA; a.o2 = dB; a.o3 = dC;
  dim3 grid;
  st = ew_setup(a, nbatch, L, H, workspace, workspace_bytes,
                tssm_ssm_scan_fused_workspace_bytes(nbatch, L, H), &grid);
  if (st != TSSM_OK) return st;
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case TSSM_F32: hipLaunchKernelGGL(ew_scan_bwd_kernel<float>, grid, dim3(kW * 64), 0, s, a); break;
    case TSSM_BF16: hipLaunchKernelGGL(ew_scan_bwd_kernel<bf16_t>, grid, dim3(kW * 64), 0, s, a); break;
    default: hipLaunchKernelGGL(ew_scan_bwd_kernel<f16_t>, grid, dim3(kW * 64), 0, s, a); break;
  }
  return launch_status();
}
