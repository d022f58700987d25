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

// ------------------------------------------------------------------ key-shard sums
// One element of a key shard's unnormalised sums: stored (mode 1, ACC_STORE) or added (mode 2,
// ACC_ADD) to what the caller's array holds.
template <typename T>
__device__ __forceinline__ void acc_row(T* p, T x, int mode) {
  *p = mode == 2 ? *p + x : x;
}

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
// signs.  Exact for s >= 0 (same expression as the reference's positive branch).  For s < 0
// the sum cancels: t r = sqrt(1 + s^2) (1 + eta) with eta <= 2^-25 + 1.5 * 2^-23 (the rounding
// of t, halved by the square root, and the hardware rsqrt's rounding and one ulp), so
// fma(t, r, s) carries an absolute error of about |s| eta against rho(s) ~ 1/(2|s|), a relative
// error of 16 s^2 eta in rho^8.  The kernels therefore use this form only in waves whose every
// score is provably within |s| <= kFastRhoMaxScore (fast_rho_safe below), where that is at most
// 16 * 32^2 * 2.1e-7 = 3.4e-3 per weight; other waves, and every wave when the caller sets
// AFA_FLAG_EXACT_TAIL, take rho8_exact.
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

// Two-branch form of rho8_fast_half: (rho(s)/sqrt 2)^8 = rho(s)^8 / 16 for s = sqrt(2) x without
// cancellation.  For s < 0, rho(s) = 1/rho(|s|), so (rho(s)/sqrt 2)^8 = 1 / (256 (rho(|s|)/sqrt 2)^8).
__device__ __forceinline__ float rho8_exact_half(float x) {
  const float a = __builtin_fabsf(x);
  const float t = __builtin_fmaf(a, a, 0.5f);
  const float r = __builtin_amdgcn_rsqf(t);
  const float rho = __builtin_fmaf(t, r, a);
  const float p2 = rho * rho;
  const float p4 = p2 * p2;
  const float p8 = p4 * p4;
  const float inv = __builtin_amdgcn_rcpf(p8 * 256.0f);
  return x < 0.0f ? inv : p8;
}

// ------------------------------------------------------------------ fast-rho guard
// Largest |score| on which the branch-free rho^8 is used (see rho8_fast).
constexpr float kFastRhoMaxScore = 32.0f;

// Sum of squares of the 8 packed 16-bit elements of a 16-byte chunk, in fp32 (v_dot2).
template <int DT>
__device__ __forceinline__ float chunk_norm2(u32x4_t w) {
  float s = 0.0f;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // the element goes through a scalar: this hipcc (clang 22, ROCm 7.2) compiles
    // __builtin_bit_cast(T, w[p]) on a vector element as a cast of w[0] for every p
    const unsigned u = w[p];
    if constexpr (DT == AFA_BF16) {
      const bf16x2_t v = __builtin_bit_cast(bf16x2_t, u);
      s = __builtin_amdgcn_fdot2_f32_bf16(v, v, s, false);
    } else {
      const f16x2_t v = __builtin_bit_cast(f16x2_t, u);
      s = __builtin_amdgcn_fdot2(v, v, s, false);
    }
  }
  return s;
}

// Lane layout of the row-norm producers (afa_rownorm_kernel, afa_krot_kernel): one wave covers
// one block of 64 rows of D elements in CHP iterations; in each, CHP consecutive lanes hold the
// 16-byte chunks of one row (chunks c >= D/8 idle when D/8 is not a power of two), so 64 / CHP
// rows are read as one contiguous span and a row's sum needs log2(CHP) shuffles.
template <int D>
struct RowBlockLayout {
  static constexpr int CH = D / 8;
  static constexpr int CHP = CH <= 4 ? 4 : CH <= 8 ? 8 : CH <= 16 ? 16 : 32;
  static constexpr int RPI = 64 / CHP;  // rows per iteration
  static_assert(D % 8 == 0 && CH <= 32, "row layout");
};

// Sum of v over the n consecutive lanes (n a power of two, aligned) that share it.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = 1; o < N; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane i of the wave
// reads sbase + voff (voff per lane, sbase wave-uniform) and writes LDS bytes lds + 16 i
// (lds wave-uniform, M0).  Issued as inline assembly so that the compiler does not track it:
// this hipcc waits for every LDS-DMA load in flight before each ds_read_b64_tr_b16, whatever
// LDS it reads, which stalls a wave on the tile it has just started loading.  A kernel using
// this orders the loads against its LDS reads itself (s_waitcnt vmcnt, then a barrier, before
// a buffer is read) and waits for them before it ends.
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, const void* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(m0)
               : "memory", "m0");
}

// Buffer resource of a raw byte range [base, base + bytes) for the loads below: stride 0,
// num_records = bytes, dword 3 selecting 32-bit data (gfx9 raw buffer access).  Every field is
// made wave-uniform so the descriptor sits in scalar registers.
typedef __attribute__((ext_vector_type(4))) int i32x4_t;
__device__ __forceinline__ i32x4_t raw_buffer_srd(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// Buffer resource over the byte range [base + off, base + bytes), empty when off >= bytes.  A
// tile's offset goes into the resource's base, never into the instruction's scalar offset: the
// range check of a raw buffer access covers the lane offset and the instruction offset only, and
// the scalar offset is added to the address after the check.  Only a range that starts at the
// tile makes the bytes past `bytes` read as zeros.
__device__ __forceinline__ i32x4_t raw_buffer_srd_at(const void* base, uint32_t bytes, uint32_t off) {
  return raw_buffer_srd((const char*)base + off, bytes > off ? bytes - off : 0u);
}

// 16 bytes per lane from the buffer at voff (per lane) into LDS at lds (the wave's 1 KB
// destination, as above); the scalar offset is 0.  Lanes whose 16 bytes start at or past the
// buffer's range read zeros instead of memory (the range check of a raw buffer), so a tile whose
// resource starts at the tile (raw_buffer_srd_at) and ends with the head's last row needs no
// clamp for the rows past the end of the head.
__device__ __forceinline__ void lds_dma16_buf(i32x4_t srd, uint32_t voff, const void* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(srd), "s"(m0)
               : "memory", "m0");
}

// The same with a full 64-bit address per lane.
__device__ __forceinline__ void lds_dma16(const void* src, const void* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(m0) : "memory", "m0");
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9: vmcnt [3:0] and [15:14]; expcnt and
// lgkmcnt at their no-wait maxima).
__host__ __device__ constexpr int vmcnt_only(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Maximum of a per-lane value over the wave, returned wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o));
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// Choice between rho8_fast and rho8_exact for one wave.  `nb2` holds, for each 64-row block of
// the other operand's head, the largest squared row norm (afa_rownorm_kernel / the rotation
// pre-passes); `vmax2` is the largest squared row norm of this wave's own operand rows as the
// MFMA sees them.  By Cauchy-Schwarz every score formed from block j satisfies
// s^2 <= score_scale^2 * vmax2 * nb2[j], and `lim` is kFastRhoMaxScore^2 / score_scale^2 less a
// margin for rounding (set by the host).  Returns true, wave-uniform, when every block in
// [blk0, blk1) satisfies vmax2 * nb2[j] <= lim (one ballot per 64 blocks; NaN compares false, and
// such waves take the exact form, which propagates the NaN as the reference does);
// nb2 == nullptr gives false.
__device__ __forceinline__ bool fast_rho_safe(const float* nb2, int blk0, int blk1, float vmax2, float lim) {
  if (nb2 == nullptr) return false;
  bool ok = true;
  for (int base = blk0; base < blk1; base += 64) {
    const int j = base + (int)(threadIdx.x & 63);
    const float m = j < blk1 ? nb2[j] : 0.0f;
    ok = ok && __ballot(!(m * vmax2 <= lim)) == 0;
  }
  return ok;
}

// The first 64 bounds of fast_rho_safe's range, one per lane.  They do not depend on the rows
// they are compared with, so a kernel loads them before its q (or k) loads and the guard waits
// for one memory round trip instead of two.
__device__ __forceinline__ float fast_rho_prefetch(const float* nb2, int blk0, int blk1) {
  const int j = blk0 + (int)(threadIdx.x & 63);
  return nb2 != nullptr && j < blk1 ? nb2[j] : 0.0f;
}

// fast_rho_safe with the range's first 64 bounds already loaded (fast_rho_prefetch); the same
// result.
__device__ __forceinline__ bool fast_rho_safe(const float* nb2, int blk0, int blk1, float vmax2, float lim,
                                              float first) {
  if (nb2 == nullptr) return false;
  if (blk0 >= blk1) return true;
  bool ok = __ballot(!(first * vmax2 <= lim)) == 0;
  for (int base = blk0 + 64; base < blk1; base += 64) {
    const int j = base + (int)(threadIdx.x & 63);
    const float m = j < blk1 ? nb2[j] : 0.0f;
    ok = ok && __ballot(!(m * vmax2 <= lim)) == 0;
  }
  return ok;
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
