// Fused AFA forward for gfx950, bf16/fp16 operands with fp32 accumulation on MFMA.
//
// Math and dtype contract of the reference tile kernel (src/kernels/pallas_afa.py:52-151):
//   S = (Q K^T) * scale (fp32 accumulate) -> P = rho(S)^8 -> masks -> O += cast(P) V,
//   D += rowsum(P) (unrounded fp32) -> out = O / (D + Omega), d = D + Omega.
//
// Work decomposition (one workgroup = 4 waves = one block of 4*QW queries of one (b, h)):
//   * each wave owns QW queries (QW/32 column blocks of 32) and sweeps the key axis;
//   * S is computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_{bf16,f16}: lane l holds
//     query (l & 31) and 16 keys of a 32-key block, so the row sums are per-lane partials and
//     the packed P^T feeds the PV MFMA (O^T = V^T P^T) directly from registers;
//   * K and V^T tiles of 64 keys are staged in LDS, double buffered, shared by the 4 waves;
//     V is transposed on its way into LDS with key bits 2 and 3 swapped, which makes the 8 keys
//     a lane group contracts over in the PV MFMA contiguous (one ds_read_b128 per fragment);
//   * the Cayley rotation (AGO) of K is applied between the global load and the LDS store,
//     and of Q once when the wave loads its queries; the power-of-two part of 1/sqrt(D) is
//     folded into Q exactly;
//   * causal: each workgroup stops at its last query, each wave skips 32-key blocks past its
//     own last query, and masks are evaluated only on blocks that cross the diagonal or
//     valid_len.
#include <cmath>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

template <int DT>
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == AFA_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// Rotate the 4 (even, odd) pairs packed in w by (c, s) in fp32, scale by `scale` (a power of
// two) and round back to the element type.  The products and sums are rounded separately
// (no contraction), which is the contract the C restatement follows.
template <int DT>
__device__ __forceinline__ u32x4_t rotate4(u32x4_t w, f32x4_t c, f32x4_t s, float scale) {
#pragma clang fp contract(off)
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = Elem<DT>::lo(w[p]);
    const float x1 = Elem<DT>::hi(w[p]);
    const float y0 = c[p] * x0 - s[p] * x1;
    const float y1 = s[p] * x0 + c[p] * x1;
    r[p] = Elem<DT>::pack(y0 * scale, y1 * scale);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ u32x4_t scale4(u32x4_t w, float scale) {
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = Elem<DT>::pack(Elem<DT>::lo(w[p]) * scale, Elem<DT>::hi(w[p]) * scale);
  return r;
}

// Swap bits 2 and 3 of a key index inside its 32-key block (self-inverse).
__device__ __forceinline__ int swap23(int j) { return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1); }

// SM: how s relates to the MFMA output x.  0: s = x (1/sqrt(D) folded into q exactly);
// 1: s = sqrt(2) x evaluated as (rho/sqrt 2)^8 = rho^8/16 (bf16 only: weights and sink carry 1/16);
// 2: s = sqrt(2) x formed explicitly.
template <int DT, int D, int QW, bool EXACT, int SM, bool ROT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1, D <= 128 ? 2 : 1)))
void afa_fwd_mfma_kernel(const FwdArgs a) {
  constexpr int KT = 64;             // keys per LDS tile
  constexpr int NQB = QW / 32;       // 32-query column blocks per wave
  constexpr int NKC = D / 16;        // K-dim chunks of the QK^T MFMA
  constexpr int NDB = D / 32;        // 32-row blocks of O^T
  constexpr int KSTR = D + 8;        // LDS row stride of K (elements): 16 B pad, no bank conflict
  constexpr int VSTR = KT + 8;       // LDS row stride of V^T
  constexpr int C8 = D / 8;          // 16-byte chunks per row
  constexpr int NCH = KT * C8 / 256; // 16-byte chunks per thread per tile (for K and for V)
  static_assert(NCH >= 1 && (KT * C8) % 256 == 0, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) unsigned short lds_k[2][KT * KSTR];
  __shared__ __attribute__((aligned(16))) unsigned short lds_v[2][D * VSTR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, qblk;
  block_item(blockIdx.x, a.B * a.H, a.nqb, a.causal, bh, qblk);
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int L = a.L;

  const int q0_wg = qblk * (4 * QW);
  const int q0_w = q0_wg + wave * QW;
  const int q_end_wg = min(L, q0_wg + 4 * QW);
  const int kend_wg = a.causal ? min(a.valid_len, q_end_wg) : a.valid_len;
  const int kend_w = a.causal ? min(a.valid_len, q0_w + QW) : a.valid_len;
  const int ntiles = (kend_wg + KT - 1) / KT;

  const unsigned short* qp = (const unsigned short*)a.q + b * a.q_b + h * a.q_h;
  const unsigned short* kp = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
  const unsigned short* vp = (const unsigned short*)a.v + b * a.v_b + h * a.v_h;

  // ---- Q fragments (B operand of S^T = K Q^T): query q0_w + qb*32 + l32, d = kc*16 + 8g .. +7
  u32x4_t qf[NQB][NKC];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int qi = q0_w + qb * 32 + l32;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      const int d0 = kc * 16 + 8 * g;
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (qi < L) {
        w = *(const u32x4_t*)(qp + (int64_t)qi * a.q_l + d0);
        if constexpr (ROT) {
          const f32x4_t c = *(const f32x4_t*)(a.rc + (int64_t)qi * (D / 2) + d0 / 2);
          const f32x4_t s = *(const f32x4_t*)(a.rs + (int64_t)qi * (D / 2) + d0 / 2);
          w = rotate4<DT>(w, c, s, a.q_scale);
        } else {
          w = scale4<DT>(w, a.q_scale);
        }
      }
      qf[qb][kc] = w;
    }
  }
  // fast-rho guard: the largest squared norm of the wave's queries as the MFMA sees them against
  // the key blocks it reads
  bool fast = false;
  if (!EXACT) {
    float m = 0.0f;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float n2 = 0.0f;
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) n2 += chunk_norm2<DT>(qf[qb][kc]);
      m = __builtin_fmaxf(m, n2 + __shfl_xor(n2, 32));
    }
    fast = fast_rho_safe(a.kbm != nullptr ? a.kbm + (int64_t)bh * a.nkb : nullptr, 0, (kend_w + 63) / 64,
                         wave_max(m), a.nb_lim);
  }

  // ---- tile loader (all 256 threads): chunk c = tid + 256 i -> key row c / C8, column c % C8
  u32x4_t kreg[NCH], vreg[NCH];
  f32x4_t creg[NCH], sreg[NCH];
  auto issue_loads = [&](int t) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      const int row = c / C8;
      const int c8 = c % C8;
      const int key = t * KT + row;
      if (key < L) {
        kreg[i] = *(const u32x4_t*)(kp + (int64_t)key * a.k_l + c8 * 8);
        vreg[i] = *(const u32x4_t*)(vp + (int64_t)key * a.v_l + c8 * 8);
        if constexpr (ROT) {
          creg[i] = *(const f32x4_t*)(a.rc + (int64_t)key * (D / 2) + c8 * 4);
          sreg[i] = *(const f32x4_t*)(a.rs + (int64_t)key * (D / 2) + c8 * 4);
        }
      } else {
        kreg[i] = u32x4_t{0u, 0u, 0u, 0u};
        vreg[i] = u32x4_t{0u, 0u, 0u, 0u};
        if constexpr (ROT) {
          creg[i] = f32x4_t{1.f, 1.f, 1.f, 1.f};
          sreg[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      const int row = c / C8;
      const int c8 = c % C8;
      u32x4_t kw = kreg[i];
      if constexpr (ROT) kw = rotate4<DT>(kw, creg[i], sreg[i], 1.0f);
      *(u32x4_t*)&lds_k[buf][row * KSTR + c8 * 8] = kw;
      const int pj = (row & 32) | swap23(row & 31);
      unsigned short* vt = &lds_v[buf][(c8 * 8) * VSTR + pj];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        vt[(2 * p) * VSTR] = (unsigned short)(vreg[i][p] & 0xffffu);
        vt[(2 * p + 1) * VSTR] = (unsigned short)(vreg[i][p] >> 16);
      }
    }
  };

  f32x16_t o[NDB][NQB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[db][qb][e] = 0.f;
  float rowsum[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) rowsum[qb] = 0.f;

  if (ntiles > 0) {
    issue_loads(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) issue_loads(t + 1);

#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key0 = t * KT + kb * 32;
      if (key0 < kend_w) {
        // S^T (32 keys x 32 queries per qb) = K_block Q^T
        f32x16_t s[NQB];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[qb][e] = 0.f;
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const u32x4_t kf = *(const u32x4_t*)&lds_k[buf][(kb * 32 + l32) * KSTR + kc * 16 + 8 * g];
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) s[qb] = mfma32<DT>(kf, qf[qb][kc], s[qb]);
        }
        // P = rho(S)^8 (masked on blocks crossing the diagonal / valid_len), row sums, pack
        u32x4_t pf[NQB][2];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const int qlo = q0_w + qb * 32;
          const bool need_mask = (a.causal && key0 + 31 > qlo) || (key0 + 31 >= a.valid_len);
          float p[16];
          if (fast) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float x = SM == 2 ? s[qb][r] * 1.41421356237309515f : s[qb][r];
              p[r] = SM == 1 ? rho8_fast_half(x) : rho8_fast(x);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float x = SM == 2 ? s[qb][r] * 1.41421356237309515f : s[qb][r];
              p[r] = SM == 1 ? rho8_exact_half(x) : rho8_exact(x);
            }
          }
          if (need_mask) {
            const int qi = qlo + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int j = key0 + (r >> 2) * 8 + 4 * g + (r & 3);
              const bool keep = (j < a.valid_len) && (!a.causal || j <= qi);
              p[r] = keep ? p[r] : 0.f;
            }
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) rowsum[qb] += p[r];
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              pf[qb][kk][e] = Elem<DT>::pack(p[kk * 8 + 2 * e], p[kk * 8 + 2 * e + 1]);
        }
        // O^T += V^T P^T
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const u32x4_t vf =
                *(const u32x4_t*)&lds_v[buf][(db * 32 + l32) * VSTR + kb * 32 + kk * 16 + 8 * g];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) o[db][qb] = mfma32<DT>(vf, pf[qb][kk], o[db][qb]);
          }
        }
      }
    }

    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: combine the two lane groups' row sums, normalise, store
  unsigned short* op = (unsigned short*)a.out + b * a.o_b + h * a.o_h;
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const float tot = rowsum[qb] + __shfl_xor(rowsum[qb], 32) + a.omega;
    const int qi = q0_w + qb * 32 + l32;
    if (qi < L) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d0 = db * 32 + r4 * 8 + 4 * g;
          u32x2_t w;
          w[0] = Elem<DT>::pack(o[db][qb][r4 * 4 + 0] / tot, o[db][qb][r4 * 4 + 1] / tot);
          w[1] = Elem<DT>::pack(o[db][qb][r4 * 4 + 2] / tot, o[db][qb][r4 * 4 + 3] / tot);
          *(u32x2_t*)(op + (int64_t)qi * a.o_l + d0) = w;
        }
      }
      if (a.denom != nullptr && g == 0) a.denom[(int64_t)bh * L + qi] = tot * a.w_unscale;
    }
  }
}

// Host-side launcher (called from afa_capi.cpp after validation).
template <int DT, int D, int QW, bool EXACT, int SM, bool ROT>
static hipError_t launch_one(const FwdArgs& a, hipStream_t stream) {
  const int nblocks = a.B * a.H * a.nqb;
  hipLaunchKernelGGL((afa_fwd_mfma_kernel<DT, D, QW, EXACT, SM, ROT>), dim3(nblocks), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

template <int DT, int D, int QW, bool EXACT, int SM>
static hipError_t launch_rot(const FwdArgs& a, hipStream_t stream) {
  return a.rc != nullptr ? launch_one<DT, D, QW, EXACT, SM, true>(a, stream)
                         : launch_one<DT, D, QW, EXACT, SM, false>(a, stream);
}

// Queries per workgroup for a given head_dim (4 waves x QW).
int mfma_fwd_queries_per_block(int head_dim) { return head_dim == 64 ? 256 : 128; }

bool mfma_fwd_supported(int dtype, int head_dim) {
  return (dtype == AFA_BF16 || dtype == AFA_F16) && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

hipError_t mfma_fwd_launch(int dtype, int head_dim, FwdArgs a, bool exact, hipStream_t stream) {
  // 1/sqrt(64) = 2^-3 folds into q exactly.  1/sqrt(128) = 2^-4 sqrt(2): fold 2^-4 into q and
  // either evaluate (rho/sqrt 2)^8 = rho^8/16 (bf16 fast path; weights and sink carry the
  // exact factor 1/16) or form s = sqrt(2) x per element.
  a.w_unscale = 1.0f;
  // the key bounds come from the unrotated rows when the kernel rotates at tile load; the
  // rounding of the rotated operands stays inside the bound's margin
  a.nb_lim = fast_rho_lim(head_dim == 128 ? std::sqrt(2.0) : 1.0);
  if (head_dim == 64) {
    a.q_scale = 0.125f;
    if (dtype == AFA_BF16)
      return exact ? launch_rot<AFA_BF16, 64, 64, true, 0>(a, stream)
                   : launch_rot<AFA_BF16, 64, 64, false, 0>(a, stream);
    return exact ? launch_rot<AFA_F16, 64, 64, true, 0>(a, stream)
                 : launch_rot<AFA_F16, 64, 64, false, 0>(a, stream);
  }
  a.q_scale = 0.0625f;
  if (head_dim == 256) {  // 1/sqrt(256) = 2^-4, exact in q
    if (dtype == AFA_BF16)
      return exact ? launch_rot<AFA_BF16, 256, 32, true, 0>(a, stream)
                   : launch_rot<AFA_BF16, 256, 32, false, 0>(a, stream);
    return exact ? launch_rot<AFA_F16, 256, 32, true, 0>(a, stream)
                 : launch_rot<AFA_F16, 256, 32, false, 0>(a, stream);
  }
  if (dtype == AFA_BF16) {
    if (exact) return launch_rot<AFA_BF16, 128, 32, true, 2>(a, stream);
    a.omega *= 0.0625f;
    a.w_unscale = 16.0f;
    return launch_rot<AFA_BF16, 128, 32, false, 1>(a, stream);
  }
  return exact ? launch_rot<AFA_F16, 128, 32, true, 2>(a, stream)
               : launch_rot<AFA_F16, 128, 32, false, 2>(a, stream);
}

}  // namespace afa
