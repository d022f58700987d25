// Shared device-side definitions for the gfx950 AFA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/afa.h"

namespace afa {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2_t;

// ------------------------------------------------------------------ element conversions
__device__ __forceinline__ float bf16_lo(unsigned w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(unsigned w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
__device__ __forceinline__ float f16_lo(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}

// Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned pack_f16(float a, float b) {
  f16x2_t v;
  v[0] = (_Float16)a;
  v[1] = (_Float16)b;
  return __builtin_bit_cast(unsigned, v);
}

template <int DT>
struct Elem;
template <>
struct Elem<AFA_BF16> {
  typedef unsigned short storage;
  static __device__ __forceinline__ float lo(unsigned w) { return bf16_lo(w); }
  static __device__ __forceinline__ float hi(unsigned w) { return bf16_hi(w); }
  static __device__ __forceinline__ unsigned pack(float a, float b) { return pack_bf16(a, b); }
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return __builtin_bit_cast(float, (unsigned)((const unsigned short*)p)[i] << 16);
  }
  static __device__ __forceinline__ float round(float x) { return (float)(__bf16)x; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
    ((__bf16*)p)[i] = (__bf16)x;
  }
};
template <>
struct Elem<AFA_F16> {
  typedef unsigned short storage;
  static __device__ __forceinline__ float lo(unsigned w) { return f16_lo(w); }
  static __device__ __forceinline__ float hi(unsigned w) { return f16_hi(w); }
  static __device__ __forceinline__ unsigned pack(float a, float b) { return pack_f16(a, b); }
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return (float)((const _Float16*)p)[i];
  }
  static __device__ __forceinline__ float round(float x) { return (float)(_Float16)x; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
    ((_Float16*)p)[i] = (_Float16)x;
  }
};
template <>
struct Elem<AFA_F32> {
  typedef float storage;
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return ((const float*)p)[i];
  }
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
};

// ------------------------------------------------------------------ rho(s)^8
// Two-branch, cancellation-safe evaluation (src/kernels/pallas_afa.py:39-49):
//   t = 1 + s^2, r = rsqrt(t); s >= 0: rho = s + t r;  s < 0: rho = r / (1 - s r)
// then three squarings.  Here the s < 0 branch is evaluated as 1/rho(|s|)^8, the same
// quantity (rho(s) rho(-s) = 1), so a single rsqrt, fma and squaring chain serves both signs
// and the reciprocal is taken once, after the squarings.
__device__ __forceinline__ float rho8_exact(float s) {
  const float a = __builtin_fabsf(s);
  const float t = __builtin_fmaf(a, a, 1.0f);
  const float r = __builtin_amdgcn_rsqf(t);
  const float rho = __builtin_fmaf(t, r, a);
  const float p2 = rho * rho;
  const float p4 = p2 * p2;
  const float p8 = p4 * p4;
  const float inv = __builtin_amdgcn_rcpf(p8);
  // Select on the sign bit without a compare: mask = s >> 31 (arithmetic).
  const unsigned m = (unsigned)(__builtin_bit_cast(int, s) >> 31);
  const unsigned bits = (__builtin_bit_cast(unsigned, inv) & m) | (__builtin_bit_cast(unsigned, p8) & ~m);
  return __builtin_bit_cast(float, bits);
}

// Branch-free evaluation rho = s + sqrt(1 + s^2) computed as fma(t, rsqrt(t), s) for both
// signs.  Exact for s >= 0 (same expression as the reference's positive branch); for s < 0
// the cancellation adds an absolute error below 1e-8 to rho^8 (about 8 rho(s)^7 |s| 2^-22),
// which the host accepts only when sink_omega makes it negligible against the denominator
// (fast_rho_ok in afa_capi.hip).
__device__ __forceinline__ float rho8_fast(float s) {
  const float t = __builtin_fmaf(s, s, 1.0f);
  const float r = __builtin_amdgcn_rsqf(t);
  const float rho = __builtin_fmaf(t, r, s);
  const float p2 = rho * rho;
  const float p4 = p2 * p2;
  return p4 * p4;
}

// (rho(s)/sqrt(2))^8 = rho(s)^8 / 16 for s = sqrt(2) x, computed from x without forming s:
// rho(s)/sqrt(2) = x + sqrt(x^2 + 1/2).  Used when 1/sqrt(head_dim) is sqrt(2) times a power
// of two (head_dim = 32, 128): the power of two is folded into q exactly and the weights are
// carried scaled by 1/16 (an exact power of two) together with sink_omega.
__device__ __forceinline__ float rho8_fast_half(float x) {
  const float t = __builtin_fmaf(x, x, 0.5f);
  const float r = __builtin_amdgcn_rsqf(t);
  const float rho = __builtin_fmaf(t, r, x);
  const float p2 = rho * rho;
  const float p4 = p2 * p2;
  return p4 * p4;
}

// Reference-faithful double precision evaluation (two branches, IEEE sqrt and division).
__device__ __forceinline__ double rho8_f64(double s) {
  const double rad = 1.0 + s * s;
  const double r = 1.0 / sqrt(rad);
  double rho;
  if (s < 0.0) {
    rho = r / (1.0 - s * r);
  } else {
    rho = s + rad * r;
  }
  const double k2 = rho * rho;
  const double k4 = k2 * k2;
  return k4 * k4;
}

// fp32 two-branch evaluation with IEEE operations, op for op as the reference.  Used by the
// generic kernels (which are not VALU bound) so their fp32 results track the reference
// formula as closely as fp32 allows.
__device__ __forceinline__ float rho8_ref(float s) {
  const float rad = 1.0f + s * s;
  const float r = 1.0f / __builtin_sqrtf(rad);
  float rho;
  if (s < 0.0f) {
    rho = r / (1.0f - s * r);
  } else {
    rho = s + rad * r;
  }
  const float k2 = rho * rho;
  const float k4 = k2 * k2;
  return k4 * k4;
}

// Workgroup id -> (b*h, query block) for the causal/non-causal attention grids
// (B*H*nqb workgroups).  Dispatch order is heaviest query block first across all heads, so list
// scheduling approximates longest-processing-time-first; block id b runs on XCD b mod 8, and
// when the head count allows, the heads of one XCD form one contiguous group (their K/V tiles
// share that XCD's L2).  Non-causal grids use the same order (all blocks weigh the same).
__device__ __forceinline__ void block_item(int bid, int BH, int nqb, int causal, int& bh, int& qblk) {
  int rank;
  if ((BH & 7) == 0) {
    const int hq = BH >> 3, j = bid >> 3;
    bh = (bid & 7) * hq + j % hq;
    rank = j / hq;
  } else {
    bh = bid % BH;
    rank = bid / BH;
  }
  qblk = causal ? nqb - 1 - rank : rank;
}

}  // namespace afa
