// bf16 SSD with N = 64 on the matrix cores: the one-pass kernel and its time
// segments, in a translation unit of their own, built with the scheduler's
// max-ilp strategy (B=8 L=4096 H=16 P=N=64: 118.7-120.0 against 119.1-123.0
// us per scan in alternating runs on one box; the one-launch N = 16 kernel
// of ssd.hip measured slower with that strategy and keeps the default).
#include "ssd_dev.h"

namespace tssm {

// ---------------------------------------------------------------------------
// SSD with N = 64 and bf16 I/O on the matrix cores, in one pass.  With N = 64
// a chunk state is P x 64 fp32 (16 KB per head), so state passing between
// workgroups would move as many bytes as the inputs.  Instead one workgroup
// owns (row, block of 32 channels -- 16 when P is not a multiple of 32) and
// walks the whole sequence in blocks of steps, carrying its slice of the
// state (channels x 64) in LDS: the recurrence of channel p involves only
// state row p, so the channel blocks of a row are independent (they share the
// B, C and dt reads, which the XCD-aware mapping keeps in one L2).  Per block,
// with cum_t the inclusive sum of
// log2(decay) over the block and coef_s the input coefficient:
//   y_t[p]   = sum_{s<=t} 2^(cum_t-cum_s) coef_s (C_t.B_s) x_s[p]
//              + 2^cum_t (C_t . H[p,:])                     (+ D[p] x_t[p])
//   H'[p, n] = 2^cum_e H[p, n] + sum_s 2^(cum_e-cum_s) coef_s x_s[p] B_s[n]
// (cum_e: the sum over the whole block).
// Blocks of 128 steps: output wave w (0-3) produces the outputs of the 16-step
// groups w and 7 - w (9 Gram blocks of the lower triangle each) and state wave
// 4 + w the state columns 16w..16w+15 (the kernel below).  Every decay factor
// is <= 1, so nothing needs rescaling.  Products whose operand is not a raw input (the
// decay-weighted Gram matrix, the weighted x and the state) split it into
// bf16 hi + lo parts.

// LDS element offsets: 16-byte column blocks XORed with the row so that the
// 16 rows read by one operand fetch spread over the banks.
__device__ inline int sq_tix(int row, int col) {  // [row][128] bf16, col = step
  return row * 128 + ((((col >> 3) ^ row ^ (row >> 3)) & 15) << 3) + (col & 7);
}
__device__ inline int sq_bix(int s, int n) {  // [s][64] bf16
  return s * 64 + ((((n >> 3) ^ s) & 7) << 3) + (n & 7);
}
__device__ inline int sq_hix(int p, int n) {  // [16][64] fp32 state slice
  return p * 64 + ((((n >> 2) ^ p) & 15) << 2) + (n & 3);
}

__device__ inline void split_bf16x4(const float* v, s16x4_t& hi, s16x4_t& lo) {
  const uint32_t h0 = pk_bf16(v[0], v[1]), h1 = pk_bf16(v[2], v[3]);
  const uint32_t l0 = pk_bf16(v[0] - bf16_lo(h0), v[1] - bf16_hi(h0));
  const uint32_t l1 = pk_bf16(v[2] - bf16_lo(h1), v[3] - bf16_hi(h1));
  hi = __builtin_bit_cast(s16x4_t, make_uint2(h0, h1));
  lo = __builtin_bit_cast(s16x4_t, make_uint2(l0, l1));
}

// One Gram block: steps 16sb.. of B against the lane's output step t,
// masked (DIAG: the block holds the diagonal, s <= t) and decay-weighted, as
// the bf16 hi/lo parts of the B operand of the product with x.  Factored form
// (FAC): the weight of step s is v_s = 2^(ref - cum_s) coef_s and the caller
// scales the sum by u_t = 2^(cum_t - ref); exact form: each element takes
// 2^(cum_t - cum_s) coef_s.
template <bool FAC, bool DIAG>
__device__ inline void sq_gram_m(const uint16_t* Bn, const float* s_cum, const float* s_coef,
                                 const float* s_v, int sb, int t, float cum_t, u32x4 c0, u32x4 c1,
                                 int q, int c16, s16x4_t& mh, s16x4_t& ml) {
  const int sr = 16 * sb + c16;
  const bf16x8_t g0 = as_bf16x8(*reinterpret_cast<const u32x4*>(Bn + sq_bix(sr, 8 * q)));
  const bf16x8_t g1 = as_bf16x8(*reinterpret_cast<const u32x4*>(Bn + sq_bix(sr, 8 * q + 32)));
  f32x4 g = {0.0f, 0.0f, 0.0f, 0.0f};
  g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(g0, as_bf16x8(c0), g, 0, 0, 0);
  g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(g1, as_bf16x8(c1), g, 0, 0, 0);
  float m[4];
  if constexpr (FAC) {
    const float4 vv = *reinterpret_cast<const float4*>(s_v + 16 * sb + 4 * q);
    const float vs[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) m[v] = g[v] * vs[v];
  } else {
    const float4 cs = *reinterpret_cast<const float4*>(s_cum + 16 * sb + 4 * q);
    const float4 cf = *reinterpret_cast<const float4*>(s_coef + 16 * sb + 4 * q);
    const float csv[4] = {cs.x, cs.y, cs.z, cs.w}, cfv[4] = {cf.x, cf.y, cf.z, cf.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) m[v] = g[v] * exp2_fast(cum_t - csv[v]) * cfv[v];
  }
  if constexpr (DIAG) {
#pragma unroll
    for (int v = 0; v < 4; ++v) m[v] = 16 * sb + 4 * q + v <= t ? m[v] : 0.0f;
  }
  split_bf16x4(m, mh, ml);
}

// acc[k][p][t] += x^T[16k + p][16sb..] . (weighted block), channel blocks k < PB.
template <int PB>
__device__ inline void sq_mx(const uint16_t* xT, int sb, int q, int c16, s16x4_t mh, s16x4_t ml,
                             f32x4* acc) {
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const s16x4_t ax = __builtin_bit_cast(
        s16x4_t, *reinterpret_cast<const uint2*>(xT + sq_tix(16 * k + c16, 16 * sb + 4 * q)));
    acc[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ax, mh, acc[k], 0, 0, 0);
    acc[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ax, ml, acc[k], 0, 0, 0);
  }
}

// Two weighted blocks (steps 16sb.. and 16sb+16..) in one K = 32 product:
// the contraction order is free, so lane l's 8 k-values are its 4 steps of
// each block, and the x operand is read in the same order.
template <int PB>
__device__ inline void sq_mx2(const uint16_t* xT, int sb, int q, int c16, s16x4_t mh, s16x4_t ml,
                              s16x4_t mh2, s16x4_t ml2, f32x4* acc) {
  const bf16x8_t bh = __builtin_bit_cast(
      bf16x8_t, u32x4{__builtin_bit_cast(uint2, mh).x, __builtin_bit_cast(uint2, mh).y,
                      __builtin_bit_cast(uint2, mh2).x, __builtin_bit_cast(uint2, mh2).y});
  const bf16x8_t bl = __builtin_bit_cast(
      bf16x8_t, u32x4{__builtin_bit_cast(uint2, ml).x, __builtin_bit_cast(uint2, ml).y,
                      __builtin_bit_cast(uint2, ml2).x, __builtin_bit_cast(uint2, ml2).y});
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const uint2 x0 = *reinterpret_cast<const uint2*>(xT + sq_tix(16 * k + c16, 16 * sb + 4 * q));
    const uint2 x1 = *reinterpret_cast<const uint2*>(xT + sq_tix(16 * k + c16, 16 * sb + 16 + 4 * q));
    const bf16x8_t ax = as_bf16x8(u32x4{x0.x, x0.y, x1.x, x1.y});
    acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax, bh, acc[k], 0, 0, 0);
    acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax, bl, acc[k], 0, 0, 0);
  }
}

// The Gram blocks 0..tg of one output group: off-diagonal blocks two at a
// time (one K = 32 product per pair), then the diagonal block.
template <bool FAC, int PB>
__device__ inline void sq_group(const uint16_t* Bn, const uint16_t* xT, const float* s_cum,
                                const float* s_coef, const float* s_v, int tg, int st, float cum_t,
                                u32x4 c0, u32x4 c1, int q, int c16, f32x4* acc) {
  s16x4_t mh, ml, mh2, ml2;
  int sb = 0;
  for (; sb + 1 < tg; sb += 2) {
    sq_gram_m<FAC, false>(Bn, s_cum, s_coef, s_v, sb, st, cum_t, c0, c1, q, c16, mh, ml);
    sq_gram_m<FAC, false>(Bn, s_cum, s_coef, s_v, sb + 1, st, cum_t, c0, c1, q, c16, mh2, ml2);
    sq_mx2<PB>(xT, sb, q, c16, mh, ml, mh2, ml2, acc);
  }
  if (sb < tg) {
    sq_gram_m<FAC, false>(Bn, s_cum, s_coef, s_v, sb, st, cum_t, c0, c1, q, c16, mh, ml);
    sq_mx<PB>(xT, sb, q, c16, mh, ml, acc);
  }
  sq_gram_m<FAC, true>(Bn, s_cum, s_coef, s_v, tg, st, cum_t, c0, c1, q, c16, mh, ml);
  sq_mx<PB>(xT, tg, q, c16, mh, ml, acc);
}

// Both output groups of a wave: Gram blocks 0..tA (group A) and 0..tB.
template <bool FAC, int PB>
__device__ inline void sq_groups(const uint16_t* Bn, const uint16_t* xT, const float* s_cum,
                                 const float* s_coef, const float* s_v, int tA, int tB, int sA,
                                 int sB, float cum_a, float cum_b, u32x4 a0, u32x4 a1, u32x4 b0,
                                 u32x4 b1, int q, int c16, f32x4* accA, f32x4* accB) {
  sq_group<FAC, PB>(Bn, xT, s_cum, s_coef, s_v, tA, sA, cum_a, a0, a1, q, c16, accA);
  sq_group<FAC, PB>(Bn, xT, s_cum, s_coef, s_v, tB, sB, cum_b, b0, b1, q, c16, accB);
}

// Carried state H[p,:] . C_t into acc[p][t]; the state slice is kept in LDS
// as bf16 hi and lo parts ([p][n], like B) next to its fp32 values.
__device__ inline void sq_state_c(const uint16_t* Hh, const uint16_t* Hl, int p, u32x4 c0,
                                  u32x4 c1, int q, f32x4& acc) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const bf16x8_t hh = as_bf16x8(*reinterpret_cast<const u32x4*>(Hh + sq_bix(p, 8 * q + 32 * ks)));
    const bf16x8_t hl = as_bf16x8(*reinterpret_cast<const u32x4*>(Hl + sq_bix(p, 8 * q + 32 * ks)));
    const bf16x8_t cb = as_bf16x8(ks == 0 ? c0 : c1);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hh, cb, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hl, cb, acc, 0, 0, 0);
  }
}

// Store one state value: fp32, bf16 hi and bf16 lo.
__device__ inline void sq_put_state(float* Hf, uint16_t* Hh, uint16_t* Hl, int p, int n, float v) {
  const uint32_t hi = pk_bf16(v, 0.0f);
  Hf[sq_hix(p, n)] = v;
  Hh[sq_bix(p, n)] = (uint16_t)hi;
  Hl[sq_bix(p, n)] = (uint16_t)pk_bf16(v - bf16_lo(hi), 0.0f);
}

// Workgroup -> (row, channel block, time segment).  With rows a multiple of 8
// the units of a row share blockIdx mod 8, so they run on one XCD (its L2
// holds the row's B, C and dt) and are dispatched together.
struct SqUnit {
  uint32_t row, pb, seg;
};
__device__ inline SqUnit sq_unit(uint32_t bid, uint32_t rows, uint32_t npb, uint32_t nsg) {
  const uint32_t g = npb * nsg;
  uint32_t row, u;
  if (rows % 8 == 0) {
    const uint32_t j = bid >> 3;
    u = j % g;
    row = (j / g) * 8 + (bid & 7);
  } else {
    row = bid / g;
    u = bid - row * g;
  }
  return {row, u % npb, u / npb};
}

// Time-segmented form, pass 1: the end state, from a zero state, of every
// sub-segment before the last segment (a segment splits into m sub-segments
// so that pass 1 has enough waves).  One wave per workgroup, no state shared
// between waves: wave (row, sub-segment, tile) holds a 16CT-channel x
// 32-column tile of the state in registers and walks the sub-segment in
// 64-step sub-blocks, last sub-block first: H += sum_s w_s x_s B_s^T with
// w_s = 2^(lsum + tot - cum_s) coef_s (lsum: the log2 decay of the later
// sub-blocks), as bf16 hi/lo products on the matrix cores.  Once the decay
// from the sub-segment end has underflowed to exactly zero, every earlier
// step's weight is exactly zero too: the walk stops there (checked every
// kSgAhead sub-blocks) and the sub-segment's decay product is zero.  It
// stages its own x and B slices through LDS (transposed to [column][step],
// the operand layout of the products) and forms the sub-block's weights
// itself, so the only barriers are its own.  kSgAhead sub-blocks of loads
// are in flight.  Writes chunkX[row][sub][p][n] and the sub-segment's decay
// chunkA[row][sub].
constexpr int kSgSteps = 64;   // steps per sub-block
constexpr int kSgAhead = 2;    // sub-blocks of loads in flight
constexpr int kSgStride = kSgSteps + 8;  // LDS row stride (bf16) of the staged slices

template <int DISC, int CT>
__global__ __launch_bounds__(64) void ssd_seg_state_kernel(SsdArgs a, uint32_t tiles,
                                                           uint32_t nsub, uint32_t subb) {
  __shared__ __align__(16) uint16_t xT[16 * CT * kSgStride];
  __shared__ __align__(16) uint16_t BT[32 * kSgStride];
  __shared__ __align__(16) float s_w[kSgSteps];
  const int lane = threadIdx.x, q = lane >> 4, c16 = lane & 15;
  const uint32_t ngrp = a.rows * nsub, bid = blockIdx.x;
  uint32_t grp, tau;
  if (ngrp % 8 == 0) {  // the tiles of a (row, sub-segment) on one XCD
    const uint32_t j = bid >> 3;
    tau = j % tiles;
    grp = (j / tiles) * 8 + (bid & 7);
  } else {
    grp = bid / tiles;
    tau = bid - grp * tiles;
  }
  const uint32_t row = grp / nsub, sub = grp - row * nsub;
  const uint32_t b = row / a.H, h = row - b * a.H;
  const int c0 = (int)(tau >> 1) * 16 * CT, n0 = (int)(tau & 1) * 32;
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x) + b * a.sx_b + h * a.sx_h + c0;
  const uint16_t* Bb = reinterpret_cast<const uint16_t*>(a.B) + b * a.sB_b + h * a.sB_h + n0;
  const float* dtb = a.dt + b * a.sdt_b + h * a.sdt_h;
  const float a2 = -expf(a.A_log[h]) * kLog2e;
  const int64_t last = a.L - 1;
  auto clampt = [&](int64_t t) { return t < last ? t : last; };
  // lane: step pairs sp and sp + 16, 8-column octet oc (x: octets past 2 CT
  // re-read the first ones and are not staged)
  const int sp = lane >> 2, oc = lane & 3;
  const int xoc = oc < 2 * CT ? oc : oc - 2 * CT;
  struct Sub {
    u32x4 xr[4], br[4];  // [2 * half + step of the pair]
    float dl;
  };
  auto load = [&](Sub& r, int64_t t0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = clampt(t0 + 2 * sp + 32 * (j >> 1) + (j & 1));
      r.xr[j] = *reinterpret_cast<const u32x4*>(xb + t * a.sx_l + 8 * xoc);
      r.br[j] = *reinterpret_cast<const u32x4*>(Bb + t * a.sB_l + 8 * oc);
    }
    r.dl = dtb[clampt(t0 + lane) * a.sdt_l];
  };
  // every sub-segment before the last segment is whole: subb sub-blocks of
  // kSgSteps steps, a multiple of kSgAhead (the refills of the last sets
  // read sub-block 0 again and are never staged)
  const int64_t tbeg = (int64_t)sub * subb * kSgSteps;
  auto t0_of = [&](int64_t kb) { return tbeg + kSgSteps * (kb > 0 ? kb : 0); };
  f32x4 st[CT][2];
#pragma unroll
  for (int i = 0; i < CT; ++i) st[i][0] = st[i][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float lsum = 0.0f;  // log2 decay from the end of the current sub-block to the sub-segment end
  Sub rg[kSgAhead];
#pragma unroll
  for (int d = 0; d < kSgAhead; ++d) {
    load(rg[d], t0_of((int64_t)subb - 1 - d));
    __builtin_amdgcn_sched_barrier(0);
  }
  bool done = false;
  for (int64_t kb0 = (int64_t)subb - 1; kb0 >= 0 && !done; kb0 -= kSgAhead) {
#pragma unroll
  for (int d = 0; d < kSgAhead; ++d) {
    {
      const int64_t kb = kb0 - d;
      const int64_t t0 = tbeg + kSgSteps * kb;
      Sub& r = rg[d];
      __syncthreads();  // the previous sub-block's LDS reads are done
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = 2 * sp + 32 * hh;
        if (oc < 2 * CT) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            *reinterpret_cast<uint32_t*>(xT + (8 * oc + 2 * e) * kSgStride + col) =
                perm_lo(r.xr[2 * hh][e], r.xr[2 * hh + 1][e]);
            *reinterpret_cast<uint32_t*>(xT + (8 * oc + 2 * e + 1) * kSgStride + col) =
                perm_hi(r.xr[2 * hh][e], r.xr[2 * hh + 1][e]);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          *reinterpret_cast<uint32_t*>(BT + (8 * oc + 2 * e) * kSgStride + col) =
              perm_lo(r.br[2 * hh][e], r.br[2 * hh + 1][e]);
          *reinterpret_cast<uint32_t*>(BT + (8 * oc + 2 * e + 1) * kSgStride + col) =
              perm_hi(r.br[2 * hh][e], r.br[2 * hh + 1][e]);
        }
      }
      // weights of the sub-block's steps, lane = step
      const float d = t0 + lane < a.L ? r.dl : 0.0f;
      const float l2 = d * a2;
      const float ab = exp2_fast(l2);
      const float coef = (DISC == TSSM_DISC_ZOH) ? phi1_from_exp(l2 * 0.6931471805599453f, ab) * d : d;
      const float cum = scan_incl<64>(l2);
      const float tot = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cum), 63));
      s_w[lane] = exp2_fast(lsum + (tot - cum)) * coef;
      lsum += tot;
      load(r, t0_of(kb - kSgAhead));
      __syncthreads();
#pragma unroll
      for (int kc = 0; kc < kSgSteps / 32; ++kc) {
        const int s0 = 8 * q + 32 * kc;
        const float4 w0 = *reinterpret_cast<const float4*>(s_w + s0);
        const float4 w1 = *reinterpret_cast<const float4*>(s_w + s0 + 4);
        bf16x8_t bt[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bt[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(BT + (16 * j + c16) * kSgStride + s0));
#pragma unroll
        for (int i = 0; i < CT; ++i) {
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xT + (16 * i + c16) * kSgStride + s0);
          const float f[8] = {bf16_lo(xv[0]) * w0.x, bf16_hi(xv[0]) * w0.y, bf16_lo(xv[1]) * w0.z,
                              bf16_hi(xv[1]) * w0.w, bf16_lo(xv[2]) * w1.x, bf16_hi(xv[2]) * w1.y,
                              bf16_lo(xv[3]) * w1.z, bf16_hi(xv[3]) * w1.w};
          bf16x8_t fh, fl;
          split_bf16(f, fh, fl);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            st[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fh, bt[j], st[i][j], 0, 0, 0);
            st[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fl, bt[j], st[i][j], 0, 0, 0);
          }
        }
      }
    }
  }
    // uniform: earlier sub-blocks would add exact zeros
    done = exp2_fast(lsum) == 0.0f;
  }
  const float adec = exp2_fast(lsum);  // zero when the walk stopped early
  const int64_t PN = (int64_t)a.P * kSqN;
  const int64_t slot = (int64_t)row * nsub + sub;
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float* out = a.chunkX + slot * PN + (int64_t)(c0 + 16 * i + 4 * q) * kSqN + n0 + 16 * j + c16;
#pragma unroll
      for (int v = 0; v < 4; ++v) out[v * kSqN] = st[i][j][v];
    }
  if (tau == 0 && lane == 0) a.chunkA[slot] = adec;
}

// Time-segmented form, pass 2: thread (row, state entry e) walks the
// sub-segments in order, S <- decay(k) S + end(k) from h0 (or zero), and
// writes entry[row][s] = S at the start of segment s (every m-th
// sub-segment).  Loads are clamped to the last sub-segment pass 1 formed, so
// every load of a batch is issued at once and stays in bounds.
constexpr int kSegBatch = 32;
__global__ __launch_bounds__(256) void ssd_seg_prefix_kernel(SsdArgs a, uint32_t nsub, uint32_t m,
                                                             int64_t PN) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = i / PN, e = i - row * PN;
  if (row >= (int64_t)a.rows) return;
  const uint32_t nseg = nsub / m + 1;
  float S = a.h0 ? a.h0[row * PN + e] : 0.0f;
  const float* X = a.chunkX + row * nsub * PN + e;
  const float* A = a.chunkA + row * nsub;
  float* E = a.entry + row * nseg * PN + e;
  for (uint32_t s0 = 0; s0 <= nsub; s0 += kSegBatch) {
    float xs[kSegBatch], as[kSegBatch];
#pragma unroll
    for (int k = 0; k < kSegBatch; ++k) {
      const uint32_t sc = min(s0 + k, nsub - 1);
      xs[k] = X[(int64_t)sc * PN];
      as[k] = A[sc];
    }
#pragma unroll
    for (int k = 0; k < kSegBatch; ++k) {
      const uint32_t sk = s0 + k;
      if (sk <= nsub) {
        if (sk % m == 0) E[(int64_t)(sk / m) * PN] = S;
        if (sk < nsub) S = __builtin_fmaf(as[k], S, xs[k]);
      }
    }
  }
}

// Store four state values H[p][n0..n0+3] (n0 a multiple of 4): fp32, bf16 hi
// and bf16 lo, each as one contiguous write.
__device__ inline void sq_put_state4(float* Hf, uint16_t* Hh, uint16_t* Hl, int p, int n0,
                                     f32x4 v) {
  *reinterpret_cast<f32x4*>(Hf + sq_hix(p, n0)) = v;
  const uint32_t h01 = pk_bf16(v[0], v[1]), h23 = pk_bf16(v[2], v[3]);
  const uint32_t l01 = pk_bf16(v[0] - bf16_lo(h01), v[1] - bf16_hi(h01));
  const uint32_t l23 = pk_bf16(v[2] - bf16_lo(h23), v[3] - bf16_hi(h23));
  *reinterpret_cast<uint2*>(Hh + sq_bix(p, n0)) = make_uint2(h01, h23);
  *reinterpret_cast<uint2*>(Hl + sq_bix(p, n0)) = make_uint2(l01, l23);
}

// 8 waves: waves 0-3 form the weighted Gram blocks of their output groups
// once and apply them to every channel block of the workgroup (PB blocks of
// 16), then the carried-state term and the outputs; waves 4-7 update state
// columns 16(w-4).. for every channel block.  Both read the state entering the
// block; the updated state goes to the other buffer.  The staged operands are
// double-buffered, so every wave stages block i+1 (and wave 4 forms its step
// scalars) before it works on block i, with one barrier per block.
//
// Time-segmented form (nseg > 1), pass 3: workgroup (row, channel block,
// segment) starts from the segment's entry state, entry[row][seg] (pass 2
// puts h0, or zero, into segment 0's), and the last segment writes the final
// state.
template <int DISC, bool HAS_D, int PB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void ssd_seq_kernel(
    SsdArgs a, uint32_t npb, uint32_t nseg, uint32_t segb) {
  constexpr int CP = kSqP * PB;  // channels per workgroup
  // staged blocks, double-buffered: block i+1 is staged while block i is used
  __shared__ __align__(16) uint16_t xTb[2][CP * kSqQ];    // x^T [p][s]
  __shared__ __align__(16) uint16_t Bnb[2][kSqQ * kSqN];  // B [s][n]
  __shared__ __align__(16) uint16_t BTb[2][kSqN * kSqQ];  // B^T [n][s]
  __shared__ __align__(16) float sH[2][CP * kSqN];     // state slice, ping-pong
  __shared__ __align__(16) uint16_t sHh[2][CP * kSqN], sHl[2][CP * kSqN];  // its bf16 parts
  __shared__ __align__(16) float s_cumb[2][kSqQ], s_coefb[2][kSqQ], s_wb[2][kSqQ], s_ub[2][kSqQ],
      s_vb[2][kSqQ];
  __shared__ float s_decb[2], s_erefb[2];
  __shared__ int s_facb[2];
  __shared__ float s_D[HAS_D ? CP : 1];  // the skip term of the workgroup's channels
  const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, c16 = lane & 15;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = wv & 3;
  const SqUnit un = sq_unit(blockIdx.x, a.rows, npb, nseg);
  const uint32_t row = un.row, pb = un.pb;
  const uint32_t b = row / a.H, h = row - b * a.H;
  const int p0 = (int)pb * CP;
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x) + b * a.sx_b + h * a.sx_h + p0;
  const uint16_t* Bb = reinterpret_cast<const uint16_t*>(a.B) + b * a.sB_b + h * a.sB_h;
  const uint16_t* Cb = reinterpret_cast<const uint16_t*>(a.C) + b * a.sC_b + h * a.sC_h;
  const float* dtb = a.dt + b * a.sdt_b + h * a.sdt_h;
  uint16_t* yb = reinterpret_cast<uint16_t*>(a.y) + b * a.sy_b + h * a.sy_h + p0;
  const int64_t PN = (int64_t)a.P * kSqN;
  const float* hin = nseg > 1 ? a.entry + ((int64_t)row * nseg + un.seg) * PN
                              : (a.h0 ? a.h0 + row * PN : nullptr);
  for (int k = tid; k < CP * kSqN; k += 512) {
    const int p = k >> 6, n = k & 63;
    sq_put_state(sH[0], sHh[0], sHl[0], p, n, hin ? hin[(int64_t)(p0 + p) * kSqN + n] : 0.0f);
  }
  if constexpr (HAS_D) {
    if (tid < CP) s_D[tid] = a.D[h * a.P + p0 + tid];
  }
  // output groups of an output wave and their steps
  const int tA = w, tB = 7 - w;
  const int sA = 16 * tA + c16, sB = 16 * tB + c16;
  // global loads of one block (rows at or past L read row L-1; their
  // coefficient is 0 and their outputs are not stored)
  const int64_t last = a.L - 1;
  auto clampt = [&](int64_t t) { return t < last ? t : last; };
  constexpr int kXq = CP / 4;             // channel quads
  const bool x_item = tid < 64 * kXq;     // (step pair, channel quad) items
  const int x_sp = tid / kXq, x_pq = tid % kXq;
  uint2 xr[2] = {};
  u32x4 br[2], cA0 = {}, cA1 = {}, cB0 = {}, cB1 = {};
  float dl0 = 0.0f, dl1 = 0.0f;
  // x, B and dt are loaded two blocks ahead of their use (one ahead of their
  // staging), C one block ahead (the output waves read it from registers)
  auto load_xb = [&](int64_t t0) {
    if (x_item) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        xr[k] = *reinterpret_cast<const uint2*>(xb + clampt(t0 + 2 * x_sp + k) * a.sx_l + 4 * x_pq);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)  // steps 2 (tid >> 3) + k, state columns 8 (tid & 7) ..
      br[k] = *reinterpret_cast<const u32x4*>(Bb + clampt(t0 + 2 * (tid >> 3) + k) * a.sB_l +
                                              8 * (tid & 7));
    if (wv == 4) {
      dl0 = dtb[clampt(t0 + 2 * lane) * a.sdt_l];
      dl1 = dtb[clampt(t0 + 2 * lane + 1) * a.sdt_l];
    }
  };
  auto load_c = [&](int64_t t0) {
    if (wv < 4) {
      const int64_t ta = clampt(t0 + sA), tb = clampt(t0 + sB);
      cA0 = *reinterpret_cast<const u32x4*>(Cb + ta * a.sC_l + 8 * q);
      cA1 = *reinterpret_cast<const u32x4*>(Cb + ta * a.sC_l + 8 * q + 32);
      cB0 = *reinterpret_cast<const u32x4*>(Cb + tb * a.sC_l + 8 * q);
      cB1 = *reinterpret_cast<const u32x4*>(Cb + tb * a.sC_l + 8 * q + 32);
    }
  };
  // Stage the block in xr / br / dl (its first step t0) into buffer sb: x^T,
  // B, B^T, and (wave 4) the per-step scalars.
  auto stage = [&](int sb, int64_t t0) {
    uint16_t* xT = xTb[sb];
    uint16_t* Bn = Bnb[sb];
    uint16_t* BT = BTb[sb];
    if (x_item) {
      const int s = 2 * x_sp;
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        const uint32_t w0 = j == 0 ? xr[0].x : xr[0].y, w1 = j == 0 ? xr[1].x : xr[1].y;
        *reinterpret_cast<uint32_t*>(xT + sq_tix(4 * x_pq + j, s)) = perm_lo(w0, w1);
        *reinterpret_cast<uint32_t*>(xT + sq_tix(4 * x_pq + j + 1, s)) = perm_hi(w0, w1);
      }
    }
    {
      const int s = 2 * (tid >> 3), ng = tid & 7;
      const u32x4 b0 = br[0], b1 = br[1];
      *reinterpret_cast<u32x4*>(Bn + sq_bix(s, 8 * ng)) = b0;
      *reinterpret_cast<u32x4*>(Bn + sq_bix(s + 1, 8 * ng)) = b1;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int k = e >> 1;
        *reinterpret_cast<uint32_t*>(BT + sq_tix(8 * ng + e, s)) = perm_lo(b0[k], b1[k]);
        *reinterpret_cast<uint32_t*>(BT + sq_tix(8 * ng + e + 1, s)) = perm_hi(b0[k], b1[k]);
      }
    }
    if (wv == 4) {  // lane: steps 2 lane, 2 lane + 1
      float l2a, ca, l2b, cb;
      mfma_step_scalars<DISC>(a, h, t0, 2 * lane, dl0, &l2a, &ca);
      mfma_step_scalars<DISC>(a, h, t0, 2 * lane + 1, dl1, &l2b, &cb);
      const float cum = scan_incl<64>(l2a + l2b);
      const float tot = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cum), 63));
      const float cum_a = cum - l2b;
      // factored decay about the block's mid-value: every factor stays within
      // 2^+-120 while the block decays by at most 2^-240
      const float ref = 0.5f * tot;
      *reinterpret_cast<float2*>(s_cumb[sb] + 2 * lane) = make_float2(cum_a, cum);
      *reinterpret_cast<float2*>(s_coefb[sb] + 2 * lane) = make_float2(ca, cb);
      *reinterpret_cast<float2*>(s_wb[sb] + 2 * lane) =
          make_float2(exp2_fast(tot - cum_a) * ca, exp2_fast(tot - cum) * cb);
      *reinterpret_cast<float2*>(s_ub[sb] + 2 * lane) =
          make_float2(exp2_fast(cum_a - ref), exp2_fast(cum - ref));
      *reinterpret_cast<float2*>(s_vb[sb] + 2 * lane) =
          make_float2(exp2_fast(ref - cum_a) * ca, exp2_fast(ref - cum) * cb);
      if (lane == 0) {
        s_decb[sb] = exp2_fast(tot);
        s_erefb[sb] = exp2_fast(ref);
        s_facb[sb] = tot >= -240.0f;
      }
    }
  };
  const int64_t nblk = (a.L + kSqQ - 1) / kSqQ;
  const int64_t blk0 = (int64_t)un.seg * segb;
  const int64_t blk1 = blk0 + segb < nblk ? blk0 + segb : nblk;
  load_xb(blk0 * kSqQ);
  load_c(blk0 * kSqQ);
  stage(0, blk0 * kSqQ);
  load_xb((blk0 + 1) * kSqQ);
  __syncthreads();
  int cur = 0, sb = 0;
  // Per block: stage the next block into the other buffer (its loads were
  // issued a block earlier), issue the loads of the block after it, then use
  // this block; one barrier ends the block.  Blocks past the segment stage
  // clamped rows into the buffer that is not read again.
  for (int64_t blk = blk0; blk < blk1; ++blk, sb ^= 1) {
    const int64_t t0 = blk * kSqQ;
    const u32x4 a0 = cA0, a1 = cA1, b0 = cB0, b1 = cB1;
    stage(sb ^ 1, t0 + kSqQ);
    load_xb(t0 + 2 * kSqQ);
    load_c(t0 + kSqQ);
    const uint16_t* xT = xTb[sb];
    const uint16_t* Bn = Bnb[sb];
    const uint16_t* BT = BTb[sb];
    const float* s_cum = s_cumb[sb];
    const float* s_coef = s_coefb[sb];
    const float* s_w = s_wb[sb];
    const float* s_u = s_ub[sb];
    const float* s_v = s_vb[sb];

    if (wv < 4) {
      const float cum_a = s_cum[sA], cum_b = s_cum[sB];
      const bool fac = __builtin_amdgcn_readfirstlane(s_facb[sb]) != 0;
      // decay-weighted Gram blocks and their products with x, both groups
      f32x4 accA[PB], accB[PB], zA[PB], zB[PB];
#pragma unroll
      for (int k = 0; k < PB; ++k) accA[k] = accB[k] = zA[k] = zB[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (fac)
        sq_groups<true, PB>(Bn, xT, s_cum, s_coef, s_v, tA, tB, sA, sB, cum_a, cum_b, a0, a1, b0,
                            b1, q, c16, accA, accB);
      else
        sq_groups<false, PB>(Bn, xT, s_cum, s_coef, s_v, tA, tB, sA, sB, cum_a, cum_b, a0, a1, b0,
                             b1, q, c16, accA, accB);
#pragma unroll
      for (int k = 0; k < PB; ++k) {
        sq_state_c(sHh[cur], sHl[cur], 16 * k + c16, a0, a1, q, zA[k]);
        sq_state_c(sHh[cur], sHl[cur], 16 * k + c16, b0, b1, q, zB[k]);
      }
      // outputs y[t0 + s][p0 + 16k + 4q .. +3]:
      //   factored: y = u_t (acc + 2^ref z);  exact: y = acc + 2^cum_t z
      const float eref = s_erefb[sb];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int s = g == 0 ? sA : sB;
        const float u_t = fac ? s_u[s] : 1.0f;
        const float zs = fac ? eref : exp2_fast(g == 0 ? cum_a : cum_b);
        const int64_t t = t0 + s;
#pragma unroll
        for (int k = 0; k < PB; ++k) {
          const f32x4 acc = g == 0 ? accA[k] : accB[k], z = g == 0 ? zA[k] : zB[k];
          float yv[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            yv[v] = u_t * __builtin_fmaf(zs, z[v], acc[v]);
            if constexpr (HAS_D) {
              const float xv = bf16_bits_to_f32(xT[sq_tix(16 * k + 4 * q + v, s)]);
              yv[v] = __builtin_fmaf(s_D[16 * k + 4 * q + v], xv, yv[v]);
            }
          }
          if (t < a.L)
            *reinterpret_cast<uint2*>(yb + t * a.sy_l + 16 * k + 4 * q) =
                make_uint2(pk_bf16(yv[0], yv[1]), pk_bf16(yv[2], yv[3]));
        }
      }
    } else {
      // state columns 16w..16w+15 of every channel block: H'^T = 2^tot H^T + (w B)^T x,
      // the weighted B^T rows (split into bf16 hi + lo) as the A operand,
      // shared by the channel blocks, and the raw x^T rows as the B operand;
      // lane: channel 16k + c16, state columns 16w + 4q .. +3
      const float dec = s_decb[sb];
      const int p = c16, nq = 16 * w + 4 * q;
      const float* Hc = sH[cur];
      f32x4 st[PB];
#pragma unroll
      for (int k = 0; k < PB; ++k) {
        const f32x4 hv = *reinterpret_cast<const f32x4*>(Hc + sq_hix(16 * k + p, nq));
#pragma unroll
        for (int v = 0; v < 4; ++v) st[k][v] = dec * hv[v];
      }
#pragma unroll
      for (int ks = 0; ks < kSqQ / 32; ++ks) {
        const int s0 = 8 * q + 32 * ks;
        const u32x4 bv = *reinterpret_cast<const u32x4*>(BT + sq_tix(16 * w + c16, s0));
        const float4 w0 = *reinterpret_cast<const float4*>(s_w + s0);
        const float4 w1 = *reinterpret_cast<const float4*>(s_w + s0 + 4);
        const float f[8] = {bf16_lo(bv[0]) * w0.x, bf16_hi(bv[0]) * w0.y, bf16_lo(bv[1]) * w0.z,
                            bf16_hi(bv[1]) * w0.w, bf16_lo(bv[2]) * w1.x, bf16_hi(bv[2]) * w1.y,
                            bf16_lo(bv[3]) * w1.z, bf16_hi(bv[3]) * w1.w};
        bf16x8_t fh, fl;
        split_bf16(f, fh, fl);
#pragma unroll
        for (int k = 0; k < PB; ++k) {
          const bf16x8_t xv = as_bf16x8(*reinterpret_cast<const u32x4*>(xT + sq_tix(16 * k + c16, s0)));
          st[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fh, xv, st[k], 0, 0, 0);
          st[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fl, xv, st[k], 0, 0, 0);
        }
      }
#pragma unroll
      for (int k = 0; k < PB; ++k)
        sq_put_state4(sH[cur ^ 1], sHh[cur ^ 1], sHl[cur ^ 1], 16 * k + p, nq, st[k]);
    }
    cur ^= 1;
    __syncthreads();  // this block's reads and the next block's staging are done
  }
  if (a.h_last && un.seg + 1 == nseg) {
    __syncthreads();
    for (int k = tid; k < CP * kSqN; k += 512) {
      const int p = k >> 6, n = k & 63;
      a.h_last[row * PN + (int64_t)(p0 + p) * kSqN + n] = sH[cur][sq_hix(p, n)];
    }
  }
}

// Time segments of the one-pass kernel: as many (row, channel block, segment)
// workgroups as fit one per CU (the kernel holds one 512-thread workgroup per
// CU), segments of at least two 128-step blocks and no more segments than
// the workspace has chunk slots.  With one segment the kernel walks whole
// rows from h0; with more, pass 1 forms the end states of the sub-segments
// before the last segment (m per segment, m dividing the segment's blocks,
// enough for about kSgWaves waves), pass 2 the segments' entry states (h0 in
// the first), and pass 3 the outputs and the final state.
constexpr int64_t kSeqGroups = 256, kSeqMinSegBlocks = 2, kSgWaves = 2048;
static_assert((kSqQ / kSgSteps) % kSgAhead == 0, "pass-1 sub-segments hold whole sets of sub-blocks");

template <int DISC, bool HAS_D, int PB>
int launch_ssd_seq_pb(int64_t rows, int64_t npb, hipStream_t s, const SsdArgs& a) {
  const int64_t nblk = (a.L + kSqQ - 1) / kSqQ;
  // at most kSeqGroups workgroups: a second, partial round of workgroups
  // would cost a whole segment's time
  int64_t nseg = kSeqGroups / (rows * npb);
  const int64_t by_len = (nblk + kSeqMinSegBlocks - 1) / kSeqMinSegBlocks;
  if (nseg > by_len) nseg = by_len;
  if (nseg > (int64_t)a.nchunks) nseg = a.nchunks;
  if (nseg < 1) nseg = 1;
  const int64_t segb = (nblk + nseg - 1) / nseg;
  nseg = (nblk + segb - 1) / segb;
  if (nseg > 1) {
    constexpr int CT = PB;  // channel tiles of 16 per pass-1 wave
    const int64_t tiles = (a.P / (16 * CT)) * 2;
    const int64_t want = (kSgWaves + rows * (nseg - 1) * tiles - 1) / (rows * (nseg - 1) * tiles);
    int64_t m = want < segb ? want : segb;
    while (m > 1 && (segb % m != 0 || (nseg - 1) * m > (int64_t)a.nchunks)) --m;
    const int64_t nsub = (nseg - 1) * m;
    hipLaunchKernelGGL((ssd_seg_state_kernel<DISC, CT>), dim3((unsigned)(rows * nsub * tiles)),
                       dim3(64), 0, s, a, (uint32_t)tiles, (uint32_t)nsub,
                       (uint32_t)(segb / m * (kSqQ / kSgSteps)));
    const int64_t PN = (int64_t)a.P * kSqN;
    hipLaunchKernelGGL(ssd_seg_prefix_kernel, dim3((unsigned)((rows * PN + 255) / 256)), dim3(256),
                       0, s, a, (uint32_t)nsub, (uint32_t)m, PN);
  }
  hipLaunchKernelGGL((ssd_seq_kernel<DISC, HAS_D, PB>), dim3((unsigned)(rows * npb * nseg)),
                     dim3(512), 0, s, a, (uint32_t)npb, (uint32_t)nseg, (uint32_t)segb);
  return launch_status();
}

template <int DISC, bool HAS_D>
int launch_ssd_seq_d(int64_t rows, int64_t P, hipStream_t s, const SsdArgs& a) {
  if (P % 32 == 0) return launch_ssd_seq_pb<DISC, HAS_D, 2>(rows, P / 32, s, a);
  return launch_ssd_seq_pb<DISC, HAS_D, 1>(rows, P / 16, s, a);
}

template <int DISC>
int launch_ssd_seq(bool has_d, int64_t rows, int64_t P, hipStream_t s, const SsdArgs& a) {
  return has_d ? launch_ssd_seq_d<DISC, true>(rows, P, s, a)
               : launch_ssd_seq_d<DISC, false>(rows, P, s, a);
}

int launch_ssd_seq_any(int disc, bool has_d, int64_t rows, int64_t P, hipStream_t s,
                       const SsdArgs& a) {
  return disc == TSSM_DISC_ZOH ? launch_ssd_seq<TSSM_DISC_ZOH>(has_d, rows, P, s, a)
                               : launch_ssd_seq<TSSM_DISC_EULER>(has_d, rows, P, s, a);
}

}  // namespace tssm
