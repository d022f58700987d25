// Fused AFA forward for head_dim 128 (bf16 / fp16 operands, fp32 accumulate) without rotary
// tables (C5).  Same contract as afa_fwd_mfma.hip (src/kernels/pallas_afa.py:52-151).  At
// head_dim 128 a score costs 512 MFMA FLOPs against the same ~7.5 VALU slots of the rho^8 chain
// as at 64, so the matrix and vector work are about even and must overlap:
//
//   * two waves per SIMD (at most 256 registers per wave): while one wave runs its rho^8 chain on
//     the VALU the other's MFMAs run.  A wave owns 32 queries; unit u (32 keys) first issues
//     S(u+1) = K Q^T (8 x 32x32x16), then rho^8 of S(u), then O += V^T P(u) (8 x 32x32x16); the K
//     and V fragments live only around their own MFMAs, S in two register sets used alternately;
//   * K and V reach LDS by direct global -> LDS loads in tiles of 32 keys (256-byte rows of
//     16-byte chunks): K chunk c of row r at c ^ (r & 7) (conflict-free 32-row fragments), V
//     chunk c at c ^ ((r & 3) << 1) (conflict-free ds_read_tr16_b64 of 4-key column slices,
//     which give the PV MFMA's A operand in the key order of the S^T accumulator);
//   * LDS is a ring of NB tiles: iteration u issues tile u + NB - 1 into the buffer of tile u - 1
//     and waits only for its own loads of tile u + 1; one barrier per tile;
//   * 1/sqrt(128) = 2^-4 sqrt(2): 2^-4 is folded into q exactly, and sqrt(2) is either evaluated
//     inside (rho/sqrt 2)^8 = rho^8/16 (bf16 fast path: weights and sink carry 1/16) or formed
//     explicitly (two-branch path, fp16);
//   * masks only on units that cross the causal diagonal or valid_len; workgroups heaviest first.
#include <type_traits>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

namespace {

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

template <int DT>
__device__ __forceinline__ f32x16_t mma128(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == AFA_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ u32x4_t scale8(u32x4_t w, float scale) {
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = Elem<DT>::pack(Elem<DT>::lo(w[p]) * scale, Elem<DT>::hi(w[p]) * scale);
  return r;
}

__device__ __forceinline__ float tree16x(const float (&p)[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[2 * i] + p[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[2 * i] + a[2 * i + 1];
  a[0] = a[0] + a[1];
  a[2] = a[2] + a[3];
  return a[0] + a[2];
}

__host__ __device__ constexpr int vm_wait(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

}  // namespace

// SM: 1 = s = sqrt(2) x evaluated as (rho/sqrt 2)^8 = rho^8/16 (weights and sink carry 1/16);
//     2 = s = sqrt(2) x formed explicitly.
template <int DT, bool EXACT, int SM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void afa_fwd_d128_kernel(const FwdArgs a) {
  constexpr int D = 128;
  constexpr int KT = 32;                 // keys per tile = one unit
  constexpr int NB = 4;                  // ring of tile buffers
  constexpr int LOADS = 4;               // direct loads per thread per tile (2 K + 2 V)
  __shared__ __attribute__((aligned(16))) unsigned short lds_k[NB][KT * D];
  __shared__ __attribute__((aligned(16))) unsigned short lds_v[NB][KT * D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5, l16 = lane & 15, m16 = (lane >> 4) & 1;

  int bh, qblk;
  block_item(blockIdx.x, a.B * a.H, a.nqb, a.causal, bh, qblk);
  const int b = bh / a.H, h = bh % a.H;
  const int L = a.L, vlen = a.valid_len;
  const int q0_wg = qblk * 128, q0_w = q0_wg + wave * 32;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 128)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 32) : vlen;
  const int ntiles = (kend_wg + KT - 1) / KT;
  const int U = q0_w < L ? (kend_w + KT - 1) / KT : 0;  // units of this wave
  const unsigned short* qp = (const unsigned short*)a.q + b * a.q_b + h * a.q_h;
  const unsigned short* kp = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
  const unsigned short* vp = (const unsigned short*)a.v + b * a.v_b + h * a.v_h;

  // q fragments (B operand of S^T = K Q^T): query q0_w + l32, features kc*16 + 8g .. +7
  const int qi = q0_w + l32;
  u32x4_t qf[8];
#pragma unroll
  for (int kc = 0; kc < 8; ++kc) {
    u32x4_t w = {0u, 0u, 0u, 0u};
    if (qi < L) w = scale8<DT>(*(const u32x4_t*)(qp + (int64_t)qi * a.q_l + kc * 16 + 8 * g), a.q_scale);
    qf[kc] = w;
  }

  // direct loads: slot s = tid + 256 i covers row s >> 4, physical chunk s & 15
  auto issue_tile = [&](int t) {
    unsigned short* kd = &lds_k[t % NB][0];
    unsigned short* vd = &lds_v[t % NB][0];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = tid + 256 * i, r = s >> 4, pc = s & 15;
      const int key = min(t * KT + r, L - 1);  // rows past L: finite data, masked
      const int lk = pc ^ (r & 7), lv = pc ^ ((r & 3) << 1);
      __builtin_amdgcn_global_load_lds((const void*)(kp + (int64_t)key * a.k_l + lk * 8),
                                       (void*)(kd + (256 * i + wave * 64) * 8), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vp + (int64_t)key * a.v_l + lv * 8),
                                       (void*)(vd + (256 * i + wave * 64) * 8), 16, 0, 0);
    }
  };
  u32x4_t kf[8];
  u32x4_t vf[4][2];
  auto read_kf = [&](int u) {
    const unsigned short* base = &lds_k[u % NB][l32 * D];
#pragma unroll
    for (int kc = 0; kc < 8; ++kc) kf[kc] = *(const u32x4_t*)(base + (((2 * kc + g) ^ (l32 & 7)) * 8));
  };
  auto read_vf = [&](int u) {
    const unsigned short* tile = lds_v[u % NB];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int row = kk * 16 + hh * 8 + 4 * g + (l16 >> 2);
          const int col = db * 32 + m16 * 16 + 4 * (l16 & 3);
          const int pc = (col >> 3) ^ ((row & 3) << 1);
          const unsigned short* p = tile + row * D + pc * 8 + (col & 7);
          const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
          const u32x2_t w = __builtin_bit_cast(u32x2_t, v);
          f[2 * hh] = w[0];
          f[2 * hh + 1] = w[1];
        }
        vf[db][kk] = f;
      }
  };

  f32x16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float rowsum = 0.f;
  f32x16_t sA, sB;

  // prologue: tiles 0 .. NB-2 in flight; tile 0 resident; S(0) in registers
  const int npro = min(ntiles, NB - 1);
  for (int t = 0; t < npro; ++t) issue_tile(t);
  if (npro == NB - 1) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * (NB - 2)));
  else __builtin_amdgcn_s_waitcnt(vm_wait(0));
  __syncthreads();
  if (ntiles > 0) {
    read_kf(0);
#pragma unroll
    for (int e = 0; e < 16; ++e) sA[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < 8; ++kc) sA = mma128<DT>(kf[kc], qf[kc], sA);
  }

  // unit u: S(u+1) = K(u+1) Q^T on the MFMA pipe first, then P(u) = rho^8(S(u)) on the VALU, then
  // O += V(u)^T P(u).  The K and V fragments live only around their own MFMAs (two waves per
  // SIMD fit in the registers: one wave's VALU runs while the other's MFMAs do).
  auto unit = [&](int u, f32x16_t& scur, f32x16_t& snxt) {
    if (u >= U) return;
    if (u + 1 < U) {
      read_kf(u + 1);
#pragma unroll
      for (int e = 0; e < 16; ++e) snxt[e] = 0.f;
#pragma unroll
      for (int kc = 0; kc < 8; ++kc) snxt = mma128<DT>(kf[kc], qf[kc], snxt);
    }
    __builtin_amdgcn_sched_barrier(0);
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float x = SM == 2 ? scur[r] * 1.41421356237309515f : scur[r];
      if constexpr (EXACT) p[r] = rho8_exact(x);
      else if constexpr (SM == 1) p[r] = rho8_fast_half(x);
      else p[r] = rho8_fast(x);
    }
    const int key0 = u * KT;
    if ((a.causal && key0 + 31 > q0_w) || key0 + 31 >= vlen) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = key0 + (r >> 2) * 8 + 4 * g + (r & 3);
        const bool keep = (j < vlen) && (!a.causal || j <= qi);
        p[r] = keep ? p[r] : 0.f;
      }
    }
    rowsum += tree16x(p);
    u32x4_t pk[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[kk][e] = Elem<DT>::pack(p[kk * 8 + 2 * e], p[kk * 8 + 2 * e + 1]);
    __builtin_amdgcn_sched_barrier(0);
    read_vf(u);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] = mma128<DT>(vf[db][kk], pk[kk], o[db]);
  };

  for (int u = 0; u < ntiles; ++u) {
    // own loads of tile u+1 done (those of tile u+2 may remain), then publish them; the barrier
    // also ends every wave's unit u-1, the last reader of the buffer reused below
    if (u + 2 < ntiles) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS));
    else __builtin_amdgcn_s_waitcnt(vm_wait(0));
    __syncthreads();
    if (u + NB - 1 < ntiles) issue_tile(u + NB - 1);
    if (u & 1) unit(u, sB, sA);
    else unit(u, sA, sB);
  }

  // epilogue
  const float tot = rowsum + __shfl_xor(rowsum, 32) + a.omega;
  if (qi < L) {
    unsigned short* op = (unsigned short*)a.out + b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
    const float inv = 1.0f / tot;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        u32x2_t w;
        w[0] = Elem<DT>::pack(o[db][r4 * 4 + 0] * inv, o[db][r4 * 4 + 1] * inv);
        w[1] = Elem<DT>::pack(o[db][r4 * 4 + 2] * inv, o[db][r4 * 4 + 3] * inv);
        *(u32x2_t*)(op + db * 32 + r4 * 8 + 4 * g) = w;
      }
    if (a.denom != nullptr && g == 0) a.denom[(int64_t)bh * L + qi] = tot * a.w_unscale;
  }
}

template <int DT, bool EXACT, int SM>
static hipError_t launch_d128(const FwdArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((afa_fwd_d128_kernel<DT, EXACT, SM>), dim3(a.B * a.H * a.nqb), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t d128_fwd_launch(int dtype, FwdArgs a, bool exact, hipStream_t st) {
  a.nqb = (a.L + 127) / 128;
  a.q_scale = 0.0625f;  // 2^-4 of 1/sqrt(128), exact
  a.w_unscale = 1.0f;
  if (dtype == AFA_BF16) {
    if (exact) return launch_d128<AFA_BF16, true, 2>(a, st);
    a.omega *= 0.0625f;
    a.w_unscale = 16.0f;
    return launch_d128<AFA_BF16, false, 1>(a, st);
  }
  return exact ? launch_d128<AFA_F16, true, 2>(a, st) : launch_d128<AFA_F16, false, 2>(a, st);
}

}  // namespace afa
