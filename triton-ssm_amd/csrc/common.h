// Shared device/host helpers for the tssm HIP library (gfx950 only).
//
// * dtype codes and element conversion (bf16 round-to-nearest-even, fp16 via
//   the hardware conversion),
// * 16-byte vector load/store of 8 channels in any of the three dtypes,
// * fast exp2 and an accurate phi1(x) = expm1(x)/x for the ZOH input term,
// * status codes and the argument-check macros every C-ABI entry point uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tssm.h"

namespace tssm {

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- dtypes
enum DType : int { F32 = TSSM_F32, BF16 = TSSM_BF16, F16 = TSSM_F16 };

struct bf16_t { uint16_t bits; };
using f16_t = _Float16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __host__ inline float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
// round-to-nearest-even (gfx950 converts in hardware: v_cvt_pk_bf16_f32)
typedef __bf16 hw_bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
// two floats -> packed bf16 pair (a in the low half), one instruction
__device__ inline uint32_t pk_bf16(float a, float b) {
  const hw_bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ inline float ld(const float* p) { return *p; }
  static __device__ inline void st(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  static __device__ inline float ld(const bf16_t* p) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[0]);
  }
  static __device__ inline void st(bf16_t* p, float v) {
    reinterpret_cast<uint16_t*>(p)[0] = (uint16_t)f32_to_bf16_bits(v);
  }
};
template <> struct Elem<f16_t> {
  static __device__ inline float ld(const f16_t* p) { return (float)*p; }
  static __device__ inline void st(f16_t* p, float v) { *p = (f16_t)v; }
};

template <typename T> __device__ inline float ldf(const T* p) { return Elem<T>::ld(p); }
template <typename T> __device__ inline void stf(T* p, float v) { Elem<T>::st(p, v); }

// Runtime-typed scalar load, for small side inputs (masks, timestamps) whose
// dtype the caller chooses freely.  The switch is wave-uniform.
// ld_any without a branch around the load: two 16-bit loads (the second the
// upper half of an fp32 element, or the same half again), then the value
// selected by dtype.  A load inside a dtype branch must complete before the
// branches join, a round trip of its own; this one waits only where its value
// is used.  Every access stays inside the element.
__device__ inline float ld_any_nb(const void* p, int64_t i, int dt) {
  const int esz = dt == F32 ? 4 : 2;
  const uint16_t* e = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p) + i * esz);
  const uint32_t lo = e[0], hi = e[esz == 4 ? 1 : 0];
  const float f32 = __uint_as_float(lo | (hi << 16));
  const float b16 = __uint_as_float(lo << 16);
  const float h16 = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
  return dt == F32 ? f32 : (dt == BF16 ? b16 : h16);
}

__device__ inline float ld_any(const void* p, int64_t i, int dt) {
  switch (dt) {
    case BF16: return ldf(reinterpret_cast<const bf16_t*>(p) + i);
    case F16: return ldf(reinterpret_cast<const f16_t*>(p) + i);
    default: return reinterpret_cast<const float*>(p)[i];
  }
}

// 8 consecutive channels as one vector load: 16 B for bf16/fp16, 32 B for fp32.
// Raw buffer loads: a descriptor for a uniform base (scalar registers), a
// per-lane byte offset (VGPR) and a uniform byte offset (SGPR), so per-step
// offsets of a tile cost no vector instructions.  The range covers 2^31 bytes
// from the base; callers keep every offset below that.
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
constexpr int kBufNt = 2;  // cache policy bit: non-temporal
__device__ inline uint4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, int32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, soff, kBufNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T> __device__ inline float buf_ldf(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                      int32_t soff);
template <> __device__ inline float buf_ldf<float>(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   int32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, soff, 0));
}
template <> __device__ inline float buf_ldf<bf16_t>(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                    int32_t soff) {
  return bf16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, soff, 0));
}
template <> __device__ inline float buf_ldf<f16_t>(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   int32_t soff) {
  return (float)__builtin_bit_cast(f16_t, __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, soff, 0));
}

template <typename T> struct Vec8;
// load_nt: non-temporal (streamed once, not kept in the caches).
__device__ inline uint4 ld_nt16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <> struct Vec8<bf16_t> {
  uint4 raw;
  __device__ inline void load(const bf16_t* p) { raw = *reinterpret_cast<const uint4*>(p); }
  __device__ inline void load_nt(const bf16_t* p) { raw = ld_nt16(p); }
  __device__ inline void load_nt(__amdgpu_buffer_rsrc_t r, uint32_t vo, int32_t so) {
    raw = buf_ld16_nt(r, vo, so);
  }
  __device__ inline void zero() { raw = make_uint4(0, 0, 0, 0); }
  __device__ inline float get(int j) const {
    uint32_t w = (&raw.x)[j >> 1];
    return (j & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  }
};
template <> struct Vec8<f16_t> {
  uint4 raw;
  __device__ inline void load(const f16_t* p) { raw = *reinterpret_cast<const uint4*>(p); }
  __device__ inline void load_nt(const f16_t* p) { raw = ld_nt16(p); }
  __device__ inline void load_nt(__amdgpu_buffer_rsrc_t r, uint32_t vo, int32_t so) {
    raw = buf_ld16_nt(r, vo, so);
  }
  __device__ inline void zero() { raw = make_uint4(0, 0, 0, 0); }
  __device__ inline float get(int j) const {
    uint32_t w = (&raw.x)[j >> 1];
    uint16_t h = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return (float)__builtin_bit_cast(f16_t, h);
  }
};
template <> struct Vec8<float> {
  float4 lo, hi;
  __device__ inline void load(const float* p) {
    lo = reinterpret_cast<const float4*>(p)[0];
    hi = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ inline void load_nt(const float* p) {
    const uint4 a = ld_nt16(p), b = ld_nt16(p + 4);
    lo = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w));
    hi = make_float4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w));
  }
  __device__ inline void load_nt(__amdgpu_buffer_rsrc_t r, uint32_t vo, int32_t so) {
    const uint4 a = buf_ld16_nt(r, vo, so), b = buf_ld16_nt(r, vo + 16, so);
    lo = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w));
    hi = make_float4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w));
  }
  __device__ inline void zero() { lo = make_float4(0, 0, 0, 0); hi = lo; }
  __device__ inline float get(int j) const { return j < 4 ? (&lo.x)[j] : (&hi.x)[j - 4]; }
};

// Store one value broadcast into 8 consecutive channels.
template <typename T> __device__ inline void store_bcast8(T* p, float v);
template <> __device__ inline void store_bcast8<bf16_t>(bf16_t* p, float v) {
  const uint32_t w = pk_bf16(v, v);
  __builtin_nontemporal_store(u32x4{w, w, w, w}, reinterpret_cast<u32x4*>(p));
}
template <> __device__ inline void store_bcast8<f16_t>(f16_t* p, float v) {
  uint32_t b = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)v);
  uint32_t w = b | (b << 16);
  __builtin_nontemporal_store(u32x4{w, w, w, w}, reinterpret_cast<u32x4*>(p));
}
template <> __device__ inline void store_bcast8<float>(float* p, float v) {
  f32x4 q = {v, v, v, v};
  __builtin_nontemporal_store(q, reinterpret_cast<f32x4*>(p));
  __builtin_nontemporal_store(q, reinterpret_cast<f32x4*>(p) + 1);
}

// ---------------------------------------------------------------- math
// exp(x) for x = y*log2(e) given y pre-scaled: one v_exp_f32.  Results below
// 2^-126 flush to zero (the state simply forgets), which is the intended
// underflow behaviour for exp(dt*a) with very negative arguments.
__device__ inline float exp2_fast(float y) { return __builtin_amdgcn_exp2f(y); }

// phi1(x) = expm1(x)/x, phi1(0) = 1, accurate to a few ulp over all x<=0
// (and moderate x>0).  |x| < 0.5: Taylor series of expm1(x)/x to degree 8
// (truncation < 1e-9); otherwise (exp(x)-1)/x, where |exp(x)-1| >= 0.39 so
// the subtraction loses no significant bits.  ``ex`` is exp(x), which every
// caller has already computed for Abar.
__device__ inline float phi1_from_exp(float x, float ex) {
  float p = 1.0f / 362880.0f;
  p = __builtin_fmaf(p, x, 1.0f / 40320.0f);
  p = __builtin_fmaf(p, x, 1.0f / 5040.0f);
  p = __builtin_fmaf(p, x, 1.0f / 720.0f);
  p = __builtin_fmaf(p, x, 1.0f / 120.0f);
  p = __builtin_fmaf(p, x, 1.0f / 24.0f);
  p = __builtin_fmaf(p, x, 1.0f / 6.0f);
  p = __builtin_fmaf(p, x, 0.5f);
  p = __builtin_fmaf(p, x, 1.0f);
  float big = (ex - 1.0f) * __builtin_amdgcn_rcpf(x);
  return __builtin_fabsf(x) < 0.5f ? p : big;
}
// ---------------------------------------------------------------- DPP helpers
template <int CTRL>
__device__ inline float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
// The value of lane i ^ 16 (within each 32-lane half), one ds_swizzle
// (bitmask mode: and 0x1f, or 0, xor 0x10) without an address computation.
__device__ inline float swizzle_xor16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
// Lane i gets lane i - n of its 16-lane row (row_shr), 0 where that leaves
// the row; or, with the row_bcast controls, lane 15 (0x142) / lane 31 (0x143)
// of the preceding row(s) in the rows ROWS selects, 0 in the others.
template <int CTRL, int ROWS>
__device__ inline float dpp_in(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, true));
}
// Inclusive prefix sum over each 32-lane half of the wave (GROUP 32) or over
// the whole wave (GROUP 64): Hillis-Steele within 16-lane rows by row shifts,
// then the row totals carried by row broadcasts.  All VALU, no LDS round trip.
template <int GROUP>
__device__ inline float scan_incl(float v) {
  static_assert(GROUP == 32 || GROUP == 64, "half-wave or wave scans");
  v += dpp_in<0x111, 0xf>(v);  // row_shr:1
  v += dpp_in<0x112, 0xf>(v);  // row_shr:2
  v += dpp_in<0x114, 0xf>(v);  // row_shr:4
  v += dpp_in<0x118, 0xf>(v);  // row_shr:8
  v += dpp_in<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  if constexpr (GROUP == 64) v += dpp_in<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64; DPP
// within rows of 16, lane shuffles beyond); every lane of the group receives
// the sum.
template <int G>
__device__ inline float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
  if constexpr (G >= 16) v += dpp_mov<0x140>(v); // row_mirror
  if constexpr (G >= 32) v += __shfl_xor(v, 16);
  if constexpr (G >= 64) v += __shfl_xor(v, 32);
  return v;
}

// softplus(x) = max(x, 0) + log1p(exp(-|x|)) with hardware exp2/log2.  With
// e = exp(-|x|) <= 1 and u = 1 + e rounded, c = (u - 1) - e is the rounding
// error exactly (u - 1 and the difference are exact by Sterbenz), and
// log1p(e) = log(u) - c / u + O(c^2).  1/u is replaced by 1 - e + e^2: its
// error e^3 / (1 + e) multiplies c <= 2^-23, negligible at every e (for
// e < 2^-24, u = 1, c = -e and the result is e (1 - e + e^2)).  11 operations,
// two of them transcendental, and no division.
__device__ inline float softplus_fast(float x) {
  const float e = exp2_fast(-__builtin_fabsf(x) * kLog2e);
  const float u = 1.0f + e;
  const float c = (u - 1.0f) - e;
  const float r = __builtin_fmaf(e, e - 1.0f, 1.0f);
  const float lp = __builtin_fmaf(__builtin_amdgcn_logf(u), 0.6931471805599453f, -c * r);
  return fmaxf(x, 0.0f) + lp;
}

// Linear interpolation between a neighbour pair with weight w on the later
// one, (1 - w) a + w b, in one fixed evaluation order (the product of the
// earlier value rounded, then an fma): every interpolation kernel gives the
// same bits whatever the compiler would contract.
__device__ inline float lerp_pair(float a, float b, float w) {
  return __builtin_fmaf(w, b, (1.0f - w) * a);
}

// clamp to [lo, hi] (lo <= hi) in one v_med3_f32
__device__ inline float clamp_med3(float x, float lo, float hi) {
  return __builtin_amdgcn_fmed3f(x, lo, hi);
}

// ZOH input coefficient expm1(dt a) / a for dt >= 0, a < 0, from the base-2
// exponent y = dt a log2(e), e = exp2(y) (already computed for Abar) and
// ia = 1/a.  |dt a| < 0.125: dt phi1(dt a), phi1's Taylor series to degree 4
// written in y (coefficients ln2^k / (k+1)!; truncation < 4.3e-8 relative);
// otherwise (e - 1) / a as one fma, where |e - 1| >= 0.1175 keeps the
// subtraction within ~5e-7 relative.  No reciprocal per call.
__device__ inline float zoh_coef2(float y, float e, float dt, float ia) {
  float p = 1.9236258215256953e-03f;
  p = __builtin_fmaf(p, y, 1.3876027166205394e-02f);
  p = __builtin_fmaf(p, y, 8.007550231970023e-02f);
  p = __builtin_fmaf(p, y, 0.34657359027997264f);
  p = __builtin_fmaf(p, y, 1.0f);
  const float big = __builtin_fmaf(e, ia, -ia);
  return __builtin_fabsf(y) < 0.18033688011112042f ? p * dt : big;
}
__device__ inline float expm1_acc(float x, float ex) {
  return x * phi1_from_exp(x, ex);
}

// Accurate exp for the fp32 paths: ocml expf (correctly range-reduced).
__device__ inline float exp_acc(float x) { return expf(x); }

// V consecutive elements as floats: V = 4 uses one 16-byte (fp32) or 8-byte
// (16-bit) access, V = 1 a scalar one.
template <typename T, int V>
__device__ inline void ld_lanes(const T* p, float* v) {
  if constexpr (V == 1) {
    v[0] = ldf(p);
  } else if constexpr (sizeof(T) == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    T tmp[4];
    *reinterpret_cast<uint2*>(tmp) = *reinterpret_cast<const uint2*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = ldf(tmp + j);
  }
}
template <typename T, int V>
__device__ inline void st_lanes(T* p, const float* v) {
  if constexpr (V == 1) {
    stf(p, v[0]);
  } else if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    T tmp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) stf(tmp + j, v[j]);
    *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(tmp);
  }
}

// ---------------------------------------------------------------- status
#define TSSM_CHECK(cond, code) \
  do {                         \
    if (!(cond)) return (code); \
  } while (0)

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TSSM_OK : (int)e;
}

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace tssm
