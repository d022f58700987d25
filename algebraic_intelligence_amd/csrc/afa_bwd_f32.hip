// fp32 ("HIGHEST") analytical AFA backward on the fp32 matrix cores (v_mfma_f32_32x32x2_f32),
// head_dim 32, 64 and 128.  Contract of tiled_afa_backward (src/kernels/pallas_afa.py:437-522)
// with fp32 operands, as the generic fp32 kernel computes it:
//   E_i = sum_d g_id out_id;  s = (q_i . k_j) * scale;  r = rsqrt(1 + s^2);  w = rho(s)^8 / d_i;
//   ds = 8 scale r w (g_i . v_j - E_i);  dq_i += ds_ij k_j;  dk_j += ds_ij q_i;  dv_j += w_ij g_i,
// with rho^8 by the two-branch form; only the order of the fp32 additions differs.
//
// Three launches, no atomics:
//   * afa_bwd_f32_prep_kernel: E_i and 1/d_i per row into the workspace;
//   * afa_bwd_f32_dq_kernel: one lane per query (32 per wave, 128 per workgroup), the layout of
//     the fp32 forward: q and g stay in registers, lane group g holding head_dim entries
//     [g D/2, (g+1) D/2); S^T = K Q^T and dP^T = V g^T contract K / V rows read as 16-byte LDS
//     fragments; dQ^T += K^T dS^T takes the dS^T accumulator element j as its B operand as it is
//     (element j of lane (query, g) is key 8 (j >> 2) + 4 g + (j & 3));
//   * afa_bwd_f32_dkdv_kernel: one lane per key, the mirror image: k and v in registers, S = Q K^T
//     and dP = g V^T from Q / g rows in LDS, then dV^T += g^T W and dK^T += Q^T dS.
// Tiles of 32 rows are staged through registers into padded, double-buffered LDS (one barrier per
// tile); with Cayley tables q and k are rotated in fp32 as they are staged, and dq, dk are rotated
// back through R^T before they are stored.
#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

namespace {

constexpr int FKT = 32;  // rows per tile

__device__ __forceinline__ f32x16_t fmma(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float frot_first(float c, float s, float x0, float x1) {
#pragma clang fp contract(off)
  return c * x0 - s * x1;
}
__device__ __forceinline__ float frot_second(float c, float s, float x0, float x1) {
#pragma clang fp contract(off)
  return s * x0 + c * x1;
}

// rho(s)^8 (two-branch: rho(|s|)^8, reciprocal for s < 0) and r = rsqrt(1 + s^2)
__device__ __forceinline__ float frho8r(float s, float& r) {
  const float a = __builtin_fabsf(s);
  const float t = __builtin_fmaf(a, a, 1.0f);
  r = __builtin_amdgcn_rsqf(t);
  const float rho = __builtin_fmaf(t, r, a);
  const float p2 = rho * rho;
  const float p4 = p2 * p2;
  const float p8 = p4 * p4;
  return s < 0.0f ? __builtin_amdgcn_rcpf(p8) : p8;
}

// Rotate the gradients of features m .. m+3 (accumulator elements e0 .. e0+3: two (even, odd)
// pairs) back through R^T with the fp32 tables at row `pos`.
template <int D>
__device__ __forceinline__ void f_unrotate4(f32x16_t& acc, int e0, const float* rc, const float* rs, int pos,
                                            int m) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int64_t t = (int64_t)pos * (D / 2) + m / 2 + p;
    const float c = rc[t], s = rs[t];
    const float x0 = acc[e0 + 2 * p], x1 = acc[e0 + 2 * p + 1];
    acc[e0 + 2 * p] = c * x0 + s * x1;
    acc[e0 + 2 * p + 1] = c * x1 - s * x0;
  }
}

}  // namespace

// E_i = sum_d g_id out_id and 1/d_i: 8 lanes per row, 16-byte chunks.  E at e_ws[row], 1/d at
// e_ws[B H L + row].
__global__ __launch_bounds__(256) void afa_bwd_f32_prep_kernel(const GenArgs a) {
  const int64_t rows = (int64_t)a.B * a.H * a.L;
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  float part = 0.f;
  if (row < rows) {
    const float* gr = (const float*)a.g + row * a.D;
    const float* orow = (const float*)a.out_in + row * a.D;
    for (int c = sub; c < a.D / 4; c += 8) {
      const f32x4_t gw = *(const f32x4_t*)(gr + 4 * c);
      const f32x4_t ow = *(const f32x4_t*)(orow + 4 * c);
      part += gw[0] * ow[0] + gw[1] * ow[1] + gw[2] * ow[2] + gw[3] * ow[3];
    }
  }
  part += __shfl_xor(part, 1);
  part += __shfl_xor(part, 2);
  part += __shfl_xor(part, 4);
  if (row < rows && sub == 0) {
    ((float*)a.e_ws)[row] = part;
    ((float*)a.e_ws)[rows + row] = 1.0f / ((const float*)a.dtot)[row];
  }
}

// ------------------------------------------------------------------------------ dQ
template <int D, bool ROT>
__global__ __launch_bounds__(256) void afa_bwd_f32_dq_kernel(const GenArgs a) {
  constexpr int DV = (D + 31) / 32 * 32;  // features in 32-feature output blocks (48 -> 64)
  constexpr int LDR = DV + 4;  // padded LDS row (shifts 16 bytes per row); features [D, DV) zero
  constexpr int KH = D / 2;
  constexpr int NDB = DV / 32;
  constexpr int KJOBS = FKT * (D / 2) / 256;  // K rotation pairs per thread per tile
  constexpr int VJOBS = (FKT * (D / 4) + 255) / 256;  // float4 of V per thread per tile
  static_assert(FKT * (D / 2) % 256 == 0 && KJOBS >= 1, "head_dim does not fit the tile loader");
  __shared__ __attribute__((aligned(16))) float ks[2][FKT * LDR];
  __shared__ __attribute__((aligned(16))) float vs[2][FKT * LDR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int L = a.L, vlen = a.valid_len, BH = a.B * a.H;
  int bh, qblk;
  block_item(blockIdx.x, BH, (L + 127) / 128, a.causal, bh, qblk);
  const int q0_wg = qblk * 128, q0_w = q0_wg + wave * 32;
  const int qi = q0_w + l32;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 128)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 32) : vlen;
  const int ntiles = (kend_wg + FKT - 1) / FKT;
  const int64_t base = (int64_t)bh * L * D;
  const float* qp = (const float*)a.q + base;
  const float* kp = (const float*)a.k + base;
  const float* vp = (const float*)a.v + base;
  const float* gp = (const float*)a.g + base;
  const float* rc = (const float*)a.rc;
  const float* rs = (const float*)a.rs;
  const float scale = (float)a.scale;
  const float c8 = 8.0f * scale;

  float qf[KH], gf[KH];
#pragma unroll
  for (int j = 0; j < KH; j += 2) {
    const int d0 = g * KH + j;
    float x0 = 0.f, x1 = 0.f, y0 = 0.f, y1 = 0.f;
    if (qi < L) {
      x0 = qp[(int64_t)qi * D + d0];
      x1 = qp[(int64_t)qi * D + d0 + 1];
      y0 = gp[(int64_t)qi * D + d0];
      y1 = gp[(int64_t)qi * D + d0 + 1];
      if constexpr (ROT) {
        const float c = rc[(int64_t)qi * (D / 2) + d0 / 2], s = rs[(int64_t)qi * (D / 2) + d0 / 2];
        const float r0 = frot_first(c, s, x0, x1), r1 = frot_second(c, s, x0, x1);
        x0 = r0;
        x1 = r1;
      }
    }
    qf[j] = x0;
    qf[j + 1] = x1;
    gf[j] = y0;
    gf[j + 1] = y1;
  }
  const int64_t rows = (int64_t)BH * L;
  const float ei = qi < L ? ((const float*)a.e_ws)[(int64_t)bh * L + qi] : 0.f;
  const float invd = qi < L ? ((const float*)a.e_ws)[rows + (int64_t)bh * L + qi] : 0.f;

  float kx[KJOBS][2], kc[KJOBS], ksn[KJOBS];
  f32x4_t vx[VJOBS];
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < KJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
      const int key = t * FKT + r;
      kx[i][0] = kx[i][1] = 0.f;
      kc[i] = 1.f;
      ksn[i] = 0.f;
      if (key < L) {
        kx[i][0] = kp[(int64_t)key * D + 2 * p];
        kx[i][1] = kp[(int64_t)key * D + 2 * p + 1];
        if constexpr (ROT) {
          kc[i] = rc[(int64_t)key * (D / 2) + p];
          ksn[i] = rs[(int64_t)key * (D / 2) + p];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
      const int key = t * FKT + r;
      f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      vx[i] = key < L && e < FKT * (D / 4) ? *(const f32x4_t*)(vp + (int64_t)key * D + 4 * c4) : z;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
      float y0 = kx[i][0], y1 = kx[i][1];
      if constexpr (ROT) {
        y0 = frot_first(kc[i], ksn[i], kx[i][0], kx[i][1]);
        y1 = frot_second(kc[i], ksn[i], kx[i][0], kx[i][1]);
      }
      ks[buf][r * LDR + 2 * p] = y0;
      ks[buf][r * LDR + 2 * p + 1] = y1;
    }
#pragma unroll
    for (int i = 0; i < VJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
      if (e < FKT * (D / 4)) *(f32x4_t*)&vs[buf][r * LDR + 4 * c4] = vx[i];
    }
  };
  if constexpr (DV > D) {  // the padding features of every K and V row, once
    for (int e = tid; e < 2 * FKT * (DV - D); e += 256) {
      const int buf = e / (FKT * (DV - D)), r = (e / (DV - D)) % FKT, f = D + e % (DV - D);
      ks[buf][r * LDR + f] = 0.f;
      vs[buf][r * LDR + f] = 0.f;
    }
  }

  f32x16_t dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) dq[db][e] = 0.f;

  if (ntiles > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) load(t + 1);
    const int key0 = t * FKT;
    if (key0 < kend_w && q0_w < L) {
      const float* kt = ks[t & 1];
      const float* vt = vs[t & 1];
      f32x16_t st, pt;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        st[e] = 0.f;
        pt[e] = 0.f;
      }
#pragma unroll
      for (int j4 = 0; j4 < KH / 4; ++j4) {
        const f32x4_t kv = *(const f32x4_t*)(kt + l32 * LDR + g * KH + 4 * j4);
        const f32x4_t vv = *(const f32x4_t*)(vt + l32 * LDR + g * KH + 4 * j4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          st = fmma(kv[u], qf[4 * j4 + u], st);
          pt = fmma(vv[u], gf[4 * j4 + u], pt);
        }
      }
      const bool need_mask = (a.causal && key0 + 31 > q0_w) || key0 + 31 >= vlen || q0_w + 31 >= L;
      float ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float rr;
        const float w = frho8r(st[e] * scale, rr) * invd;
        float d = c8 * rr * w * (pt[e] - ei);
        if (need_mask) {
          const int key = key0 + 8 * (e >> 2) + 4 * g + (e & 3);
          const bool keep = key < vlen && qi < L && (!a.causal || key <= qi);
          d = keep ? d : 0.f;
        }
        ds[e] = d;
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kr = 8 * (j >> 2) + 4 * g + (j & 3);
          dq[db] = fmma(kt[kr * LDR + db * 32 + l32], ds[j], dq[db]);
        }
    }
    // the buffer of tile t+1 was last read in tile t-1, before the previous barrier
    if (t + 1 < ntiles) store((t + 1) & 1);
    __syncthreads();
  }

  if (qi < L) {
    float* op = (float*)a.out + base + (int64_t)qi * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int m = db * 32 + 8 * e4 + 4 * g;  // features m .. m+3 (two rotation pairs)
        if (DV == D || m < D) {
          if constexpr (ROT) f_unrotate4<D>(dq[db], 4 * e4, rc, rs, qi, m);
          f32x4_t w;
#pragma unroll
          for (int u = 0; u < 4; ++u) w[u] = dq[db][4 * e4 + u];
          *(f32x4_t*)(op + m) = w;
        }
      }
  }
}

// ------------------------------------------------------------------------------ dK, dV
template <int D, bool ROT>
__global__ __launch_bounds__(256) void afa_bwd_f32_dkdv_kernel(const GenArgs a) {
  constexpr int DV = (D + 31) / 32 * 32;  // features in 32-feature output blocks (48 -> 64)
  constexpr int LDR = DV + 4;  // features [D, DV) of the q and g rows stay zero
  constexpr int KH = D / 2;
  constexpr int NDB = DV / 32;
  constexpr int QJOBS = FKT * (D / 2) / 256;  // Q rotation pairs per thread per tile
  constexpr int GJOBS = (FKT * (D / 4) + 255) / 256;  // float4 of g per thread per tile
  static_assert(FKT * (D / 2) % 256 == 0 && QJOBS >= 1, "head_dim does not fit the tile loader");
  __shared__ __attribute__((aligned(16))) float qs[2][FKT * LDR];
  __shared__ __attribute__((aligned(16))) float gs[2][FKT * LDR];
  __shared__ float es[2][2 * FKT];  // E, then 1/d of the tile's rows

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int L = a.L, vlen = a.valid_len, BH = a.B * a.H;
  int bh, kblk;
  // heaviest first: for causal grids the low key blocks see the most queries
  block_item(blockIdx.x, BH, (L + 127) / 128, 0, bh, kblk);
  const int k0_wg = kblk * 128, k0_w = k0_wg + wave * 32;
  const int kj = k0_w + l32;
  const bool wave_live = k0_w < L && k0_w < vlen;
  const int t0 = a.causal ? k0_wg / FKT : 0;
  const int ntiles = (L + FKT - 1) / FKT;
  const int64_t base = (int64_t)bh * L * D;
  const float* qp = (const float*)a.q + base;
  const float* kp = (const float*)a.k + base;
  const float* vp = (const float*)a.v + base;
  const float* gp = (const float*)a.g + base;
  const float* rc = (const float*)a.rc;
  const float* rs = (const float*)a.rs;
  const float* ep = (const float*)a.e_ws + (int64_t)bh * L;
  const float* ip = (const float*)a.e_ws + (int64_t)BH * L + (int64_t)bh * L;
  const float scale = (float)a.scale;
  const float c8 = 8.0f * scale;

  float kf[KH], vf[KH];
#pragma unroll
  for (int j = 0; j < KH; j += 2) {
    const int d0 = g * KH + j;
    float x0 = 0.f, x1 = 0.f, y0 = 0.f, y1 = 0.f;
    if (kj < L) {
      x0 = kp[(int64_t)kj * D + d0];
      x1 = kp[(int64_t)kj * D + d0 + 1];
      y0 = vp[(int64_t)kj * D + d0];
      y1 = vp[(int64_t)kj * D + d0 + 1];
      if constexpr (ROT) {
        const float c = rc[(int64_t)kj * (D / 2) + d0 / 2], s = rs[(int64_t)kj * (D / 2) + d0 / 2];
        const float r0 = frot_first(c, s, x0, x1), r1 = frot_second(c, s, x0, x1);
        x0 = r0;
        x1 = r1;
      }
    }
    kf[j] = x0;
    kf[j + 1] = x1;
    vf[j] = y0;
    vf[j + 1] = y1;
  }

  float qx[QJOBS][2], qc[QJOBS], qsn[QJOBS];
  f32x4_t gx[GJOBS];
  float ex = 0.f;
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < QJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
      const int row = t * FKT + r;
      qx[i][0] = qx[i][1] = 0.f;
      qc[i] = 1.f;
      qsn[i] = 0.f;
      if (row < L) {
        qx[i][0] = qp[(int64_t)row * D + 2 * p];
        qx[i][1] = qp[(int64_t)row * D + 2 * p + 1];
        if constexpr (ROT) {
          qc[i] = rc[(int64_t)row * (D / 2) + p];
          qsn[i] = rs[(int64_t)row * (D / 2) + p];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < GJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
      const int row = t * FKT + r;
      f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      gx[i] = row < L && e < FKT * (D / 4) ? *(const f32x4_t*)(gp + (int64_t)row * D + 4 * c4) : z;
    }
    if (tid < 2 * FKT) {
      const int row = t * FKT + (tid & (FKT - 1));
      ex = row < L ? (tid < FKT ? ep : ip)[row] : 0.f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < QJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
      float y0 = qx[i][0], y1 = qx[i][1];
      if constexpr (ROT) {
        y0 = frot_first(qc[i], qsn[i], qx[i][0], qx[i][1]);
        y1 = frot_second(qc[i], qsn[i], qx[i][0], qx[i][1]);
      }
      qs[buf][r * LDR + 2 * p] = y0;
      qs[buf][r * LDR + 2 * p + 1] = y1;
    }
#pragma unroll
    for (int i = 0; i < GJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
      if (e < FKT * (D / 4)) *(f32x4_t*)&gs[buf][r * LDR + 4 * c4] = gx[i];
    }
    if (tid < 2 * FKT) es[buf][tid] = ex;
  };
  if constexpr (DV > D) {  // the padding features of every q and g row, once
    for (int e = tid; e < 2 * FKT * (DV - D); e += 256) {
      const int buf = e / (FKT * (DV - D)), r = (e / (DV - D)) % FKT, f = D + e % (DV - D);
      qs[buf][r * LDR + f] = 0.f;
      gs[buf][r * LDR + f] = 0.f;
    }
  }

  f32x16_t dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      dk[db][e] = 0.f;
      dv[db][e] = 0.f;
    }

  if (t0 < ntiles) {
    load(t0);
    store(t0 & 1);
  }
  __syncthreads();
  for (int t = t0; t < ntiles; ++t) {
    if (t + 1 < ntiles) load(t + 1);
    const int i0 = t * FKT;  // first query of the tile
    const bool live = wave_live && i0 < L && (!a.causal || i0 + 31 >= k0_w);
    if (live) {
      const float* qt = qs[t & 1];
      const float* gt = gs[t & 1];
      const float* et = es[t & 1];
      f32x16_t st, pt;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        st[e] = 0.f;
        pt[e] = 0.f;
      }
#pragma unroll
      for (int j4 = 0; j4 < KH / 4; ++j4) {
        const f32x4_t qv = *(const f32x4_t*)(qt + l32 * LDR + g * KH + 4 * j4);
        const f32x4_t gv = *(const f32x4_t*)(gt + l32 * LDR + g * KH + 4 * j4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          st = fmma(qv[u], kf[4 * j4 + u], st);
          pt = fmma(gv[u], vf[4 * j4 + u], pt);
        }
      }
      const bool need_mask = (a.causal && i0 < k0_w + 31) || k0_w + 31 >= vlen || i0 + 31 >= L;
      float w[16], ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int qr = 8 * (e >> 2) + 4 * g + (e & 3);  // query of element e within the tile
        float rr;
        float we = frho8r(st[e] * scale, rr) * et[FKT + qr];
        float d = c8 * rr * we * (pt[e] - et[qr]);
        if (need_mask) {
          const int i = i0 + qr;
          const bool keep = kj < vlen && i < L && (!a.causal || kj <= i);
          we = keep ? we : 0.f;
          d = keep ? d : 0.f;
        }
        w[e] = we;
        ds[e] = d;
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int qr = 8 * (j >> 2) + 4 * g + (j & 3);
          dv[db] = fmma(gt[qr * LDR + db * 32 + l32], w[j], dv[db]);
          dk[db] = fmma(qt[qr * LDR + db * 32 + l32], ds[j], dk[db]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep each feature block's LDS reads with its MFMAs
      }
    }
    if (t + 1 < ntiles) store((t + 1) & 1);
    __syncthreads();
  }

  if (kj < L) {
    float* kout = (float*)a.dk + base + (int64_t)kj * D;
    float* vout = (float*)a.dv + base + (int64_t)kj * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int m = db * 32 + 8 * e4 + 4 * g;
        if (DV == D || m < D) {
          if constexpr (ROT) f_unrotate4<D>(dk[db], 4 * e4, rc, rs, kj, m);
          f32x4_t wk, wv;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            wk[u] = dk[db][4 * e4 + u];
            wv[u] = dv[db][4 * e4 + u];
          }
          *(f32x4_t*)(kout + m) = wk;
          *(f32x4_t*)(vout + m) = wv;
        }
      }
  }
}

bool f32_bwd_supported(int head_dim) {
  return head_dim == 32 || head_dim == 48 || head_dim == 64 || head_dim == 96 || head_dim == 128;
}

template <int D, bool ROT>
static void f32_bwd_launch_d(const GenArgs& a, hipStream_t st) {
  const int nb = a.B * a.H * ((a.L + 127) / 128);
  hipLaunchKernelGGL((afa_bwd_f32_dq_kernel<D, ROT>), dim3(nb), dim3(256), 0, st, a);
  hipLaunchKernelGGL((afa_bwd_f32_dkdv_kernel<D, ROT>), dim3(nb), dim3(256), 0, st, a);
}

template <int D>
static void f32_bwd_launch_r(const GenArgs& a, hipStream_t st) {
  if (a.rc != nullptr) f32_bwd_launch_d<D, true>(a, st);
  else f32_bwd_launch_d<D, false>(a, st);
}

hipError_t f32_bwd_launch(const GenArgs& a, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.L;
  hipLaunchKernelGGL(afa_bwd_f32_prep_kernel, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, st, a);
  if (a.D == 32) f32_bwd_launch_r<32>(a, st);
  else if (a.D == 48) f32_bwd_launch_r<48>(a, st);
  else if (a.D == 64) f32_bwd_launch_r<64>(a, st);
  else if (a.D == 96) f32_bwd_launch_r<96>(a, st);
  else f32_bwd_launch_r<128>(a, st);
  return hipGetLastError();
}

}  // namespace afa
