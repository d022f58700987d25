// Generic (non-MFMA) AFA forward and backward kernels for every dtype (fp32, bf16, fp16, fp64)
// and head_dim up to 256.
//
// Layout: 8 consecutive lanes cooperate on one row (query for the forward and dQ passes, key
// for the dK/dV pass); lane `sub` owns features d = sub + 8m.  Dot products are per-lane
// partial sums combined by an xor butterfly, which gives every lane of the group the same
// bits (IEEE addition is commutative), so all lanes see identical scores.
//
// Forward contract: src/kernels/pallas_afa.py:104-151 (S in the accumulation type, rho(S)^8,
// masks, P cast to v.dtype for PV, unrounded row sum, out = O / (D + Omega)); with
// AFA_FLAG_EXACT_REF the exact_afa_reference contract (:267-327): q * scale rounded to q.dtype
// before the dot, row sum of the cast P, out = O * (1 / (D + Omega)); for bf16 / fp16 inputs
// every op of that program is rounded to the input dtype as its JAX typing does (the score, each
// step of rho^8, the P V product, the row sum, D + Omega, its reciprocal and the product).
// Backward contract: src/kernels/pallas_afa.py:437-522 (E = rowsum(g * out); w = rho^8 / d;
// ds = 8 scale r w (g.v - E); matmul operands cast to the input dtype, accumulation in the
// accumulation type).
#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

template <int DT>
struct Acc {
  typedef float T;
};
template <>
struct Acc<AFA_F64> {
  typedef double T;
};

template <int DT>
__device__ __forceinline__ typename Acc<DT>::T ld(const void* p, int64_t i) {
  if constexpr (DT == AFA_F64) {
    return ((const double*)p)[i];
  } else {
    return Elem<DT>::load(p, i);
  }
}
template <int DT>
__device__ __forceinline__ typename Acc<DT>::T rnd(typename Acc<DT>::T x) {
  if constexpr (DT == AFA_F64) {
    return x;
  } else {
    return Elem<DT>::round(x);
  }
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, typename Acc<DT>::T x) {
  if constexpr (DT == AFA_F64) {
    ((double*)p)[i] = x;
  } else {
    Elem<DT>::store(p, i, x);
  }
}
template <typename T>
__device__ __forceinline__ T rho8_acc(T s) {
  if constexpr (sizeof(T) == 8) {
    return rho8_f64(s);
  } else {
    return rho8_ref(s);
  }
}
template <typename T>
__device__ __forceinline__ T rsq1p(T s) {
  if constexpr (sizeof(T) == 8) {
    return 1.0 / sqrt(1.0 + s * s);
  } else {
    return 1.0f / __builtin_sqrtf(1.0f + s * s);
  }
}
template <typename T>
__device__ __forceinline__ T group8_sum(T x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  return x;
}

// rho(s)^8 of exact_afa_reference for bf16 / fp16 inputs (src/kernels/pallas_afa.py:32-49 on the
// scores of :284, which are bf16 / fp16): each elementwise op of _vmu_octic_kernel is evaluated in
// fp32 and rounded to the input dtype, as every jnp op on such an array returns that dtype; rsqrt
// is 1 / sqrt, each rounded in fp32.
template <int DT>
__device__ __forceinline__ float rho8_stepwise(float s) {
#pragma clang fp contract(off)
  const float s_sq = Elem<DT>::round(s * s);
  const float rad = Elem<DT>::round(1.0f + s_sq);
  const float r = Elem<DT>::round(1.0f / __builtin_sqrtf(rad));
  const float u = Elem<DT>::round(s * r);
  const float rho = s < 0.0f ? Elem<DT>::round(r / Elem<DT>::round(1.0f - u))
                             : Elem<DT>::round(s + Elem<DT>::round(rad * r));
  const float k2 = Elem<DT>::round(rho * rho);
  const float k4 = Elem<DT>::round(k2 * k2);
  return Elem<DT>::round(k4 * k4);
}

// Cayley rotation of one (even, odd) pair; products and sums rounded separately.
template <typename T>
__device__ __forceinline__ T rot_pair(T c, T s, T x0, T x1, bool odd) {
#pragma clang fp contract(off)
  return odd ? (s * x0 + c * x1) : (c * x0 - s * x1);
}
template <int DT>
__device__ __forceinline__ void table_cs(const void* rc, const void* rs, int64_t idx,
                                         typename Acc<DT>::T& c, typename Acc<DT>::T& s) {
  if constexpr (DT == AFA_F64) {
    c = ((const double*)rc)[idx];
    s = ((const double*)rs)[idx];
  } else {
    c = ((const float*)rc)[idx];
    s = ((const float*)rs)[idx];
  }
}

// Load `rows` rows starting at `row0` of a (L, D) slice into LDS (type T), applying the
// Cayley rotation (fp32/fp64 tables, result rounded to the input dtype) when ROT.
template <int DT, bool ROT, int DMAX, int KTG>
__device__ __forceinline__ void load_tile(typename Acc<DT>::T (*dst)[DMAX], const void* src,
                                          int64_t base, int64_t ld_l, int row0, int L, int D,
                                          const void* rc, const void* rs) {
  typedef typename Acc<DT>::T T;
  if constexpr (ROT) {
    const int P = D / 2;
    for (int e = threadIdx.x; e < KTG * P; e += blockDim.x) {
      const int r = e / P, p = e % P;
      const int row = row0 + r;
      T y0 = 0, y1 = 0;
      if (row < L) {
        const T x0 = ld<DT>(src, base + (int64_t)row * ld_l + 2 * p);
        const T x1 = ld<DT>(src, base + (int64_t)row * ld_l + 2 * p + 1);
        T c, s;
        table_cs<DT>(rc, rs, (int64_t)row * P + p, c, s);
        y0 = rnd<DT>(rot_pair(c, s, x0, x1, false));
        y1 = rnd<DT>(rot_pair(c, s, x0, x1, true));
      }
      dst[r][2 * p] = y0;
      dst[r][2 * p + 1] = y1;
    }
  } else {
    for (int e = threadIdx.x; e < KTG * D; e += blockDim.x) {
      const int r = e / D, d = e % D;
      const int row = row0 + r;
      dst[r][d] = row < L ? ld<DT>(src, base + (int64_t)row * ld_l + d) : T(0);
    }
  }
}

template <int DT, int DMAX>
constexpr int gen_tile_rows() {
  typedef typename Acc<DT>::T T;
  constexpr int r = 32768 / (2 * DMAX * (int)sizeof(T));
  return r > 64 ? 64 : r;
}

// ------------------------------------------------------------------------------ forward
template <int DT, int DMAX, bool ROT>
__global__ __launch_bounds__(256) void afa_fwd_generic_kernel(const GenArgs a) {
  typedef typename Acc<DT>::T T;
  constexpr int M = DMAX / 8;
  constexpr int KTG = gen_tile_rows<DT, DMAX>();
  // bf16 / fp16 under AFA_FLAG_EXACT_REF: every op of exact_afa_reference rounded to the input
  // dtype, in a fixed order (the score as 8 fma chains over features sub + 8m added by the xor
  // butterfly, the P V product as an fma chain and the row sum as a sum in key order)
  constexpr bool HALF = DT == AFA_BF16 || DT == AFA_F16;
  const bool step = HALF && a.exact_ref;
  __shared__ T ks[KTG][DMAX];
  __shared__ T vs[KTG][DMAX];

  const int nq = (a.L + 31) / 32;
  const int bh = blockIdx.x / nq;
  const int qblk = blockIdx.x % nq;
  const int b = bh / a.H, h = bh % a.H;
  const int sub = threadIdx.x & 7;
  const int qi = qblk * 32 + (threadIdx.x >> 3);
  const int D = a.D;
  const int64_t qbase = b * a.q_b + h * a.q_h;
  const int64_t kbase = b * a.k_b + h * a.k_h;
  const int64_t vbase = b * a.v_b + h * a.v_h;
  const T scale = (T)a.scale;

  T qv[M], o[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    qv[m] = 0;
    o[m] = 0;
  }
  if (qi < a.L) {
    if constexpr (ROT) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int d = sub + 8 * m;
        if (d < D) {
          const int p = d >> 1;
          const T x0 = ld<DT>(a.q, qbase + (int64_t)qi * a.q_l + 2 * p);
          const T x1 = ld<DT>(a.q, qbase + (int64_t)qi * a.q_l + 2 * p + 1);
          T c, s;
          table_cs<DT>(a.rc, a.rs, (int64_t)qi * (D / 2) + p, c, s);
          qv[m] = rnd<DT>(rot_pair(c, s, x0, x1, d & 1));
        }
      }
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int d = sub + 8 * m;
        if (d < D) qv[m] = ld<DT>(a.q, qbase + (int64_t)qi * a.q_l + d);
      }
    }
    if (a.exact_ref) {
      // q * scale rounded to q's dtype; the reference's Python float scale takes q's dtype first
      const T sc = HALF ? rnd<DT>(scale) : scale;
#pragma unroll
      for (int m = 0; m < M; ++m) qv[m] = rnd<DT>(qv[m] * sc);
    }
  }

  const int q_last = min(a.L, qblk * 32 + 32) - 1;
  const int kend = a.causal ? min(a.valid_len, q_last + 1) : a.valid_len;
  T dsum = 0;
  for (int k0 = 0; k0 < kend; k0 += KTG) {
    __syncthreads();
    load_tile<DT, ROT, DMAX, KTG>(ks, a.k, kbase, a.k_l, k0, a.L, D, a.rc, a.rs);
    load_tile<DT, false, DMAX, KTG>(vs, a.v, vbase, a.v_l, k0, a.L, D, nullptr, nullptr);
    __syncthreads();
    const int nk = min(KTG, kend - k0);
    for (int jj = 0; jj < nk; ++jj) {
      const int j = k0 + jj;
      T part = 0;
      if (step) {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (sub + 8 * m < D) part = __builtin_fmaf(qv[m], ks[jj][sub + 8 * m], part);
      } else {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (sub + 8 * m < D) part += qv[m] * ks[jj][sub + 8 * m];
      }
      const T sdot = group8_sum(part);
      T p;
      if constexpr (HALF) {
        p = step ? rho8_stepwise<DT>(rnd<DT>(sdot)) : rho8_acc(a.exact_ref ? sdot : sdot * scale);
      } else {
        p = rho8_acc(a.exact_ref ? sdot : sdot * scale);
      }
      if (a.causal && j > qi) p = 0;
      const T pv = rnd<DT>(p);
      if (step) {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (sub + 8 * m < D) o[m] = __builtin_fmaf(pv, vs[jj][sub + 8 * m], o[m]);
      } else {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (sub + 8 * m < D) o[m] += pv * vs[jj][sub + 8 * m];
      }
      dsum += a.exact_ref ? pv : p;
    }
  }
  if (qi < a.L && a.acc) {
    // one key shard: the unnormalised sums, stored (ACC_STORE) or added to the caller's arrays
    const int64_t obase = b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (sub + 8 * m < D) acc_row((T*)a.out + obase + sub + 8 * m, o[m], a.acc);
    if (sub == 0) acc_row((T*)a.denom + (int64_t)bh * a.L + qi, dsum, a.acc);
  } else if (qi < a.L) {
    // under step, the row sum, Omega and their sum are each rounded to the input dtype
    const T tot = step ? rnd<DT>(rnd<DT>(dsum) + rnd<DT>((T)a.omega)) : dsum + (T)a.omega;
    const int64_t obase = b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
    if (a.exact_ref) {
      const T inv = rnd<DT>(T(1) / tot);
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (sub + 8 * m < D) st<DT>(a.out, obase + sub + 8 * m, (step ? rnd<DT>(o[m]) : o[m]) * inv);
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (sub + 8 * m < D) st<DT>(a.out, obase + sub + 8 * m, o[m] / tot);
    }
    if (a.denom != nullptr && sub == 0) ((T*)a.denom)[(int64_t)bh * a.L + qi] = tot;
  }
}

// ------------------------------------------------------------------------------ backward
// E_i = sum_d g_id out_id in the accumulation type (src/kernels/pallas_afa.py:451-452).
template <int DT>
__global__ __launch_bounds__(256) void afa_bwd_e_kernel(const GenArgs a) {
  typedef typename Acc<DT>::T T;
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  const int64_t nrows = (int64_t)a.B * a.H * a.L;
  T part = 0;
  if (row < nrows) {
    for (int d = sub; d < a.D; d += 8) part += ld<DT>(a.g, row * a.D + d) * ld<DT>(a.out_in, row * a.D + d);
  }
  const T e = group8_sum(part);
  if (row < nrows && sub == 0) ((T*)a.e_ws)[row] = e;
}

// Rotate a gradient pair back through R^T: (g0, g1) -> (c g0 + s g1, -s g0 + c g1), then store.
// Called by every lane of the wave (the partner value comes from lane sub ^ 1 of the same
// 8-lane group, which owns feature d ^ 1); `valid` guards the loads and stores only.
template <int DT, int M>
__device__ __forceinline__ void unrotate_store(typename Acc<DT>::T (&acc)[M], void* dst, int64_t base,
                                               int row, int D, int sub, const void* rc, const void* rs,
                                               bool rot, bool valid) {
  typedef typename Acc<DT>::T T;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int d = sub + 8 * m;
    T val = acc[m];
    if (rot) {
      const T other = __shfl_xor(acc[m], 1);
      T c = 0, s = 0;
      if (valid && d < D) table_cs<DT>(rc, rs, (int64_t)row * (D / 2) + (d >> 1), c, s);
      val = (d & 1) ? (c * val - s * other) : (c * val + s * other);
    }
    if (valid && d < D) st<DT>(dst, base + d, val);
  }
}

// dQ pass: one 8-lane group per query, sweeping keys j (<= i when causal).
template <int DT, int DMAX, bool ROT>
__global__ __launch_bounds__(256) void afa_bwd_dq_kernel(const GenArgs a) {
  typedef typename Acc<DT>::T T;
  constexpr int M = DMAX / 8;
  constexpr int KTG = gen_tile_rows<DT, DMAX>();
  __shared__ T ks[KTG][DMAX];
  __shared__ T vs[KTG][DMAX];
  const int nq = (a.L + 31) / 32;
  const int bh = blockIdx.x / nq, qblk = blockIdx.x % nq;
  const int b = bh / a.H, h = bh % a.H;
  const int sub = threadIdx.x & 7;
  const int qi = qblk * 32 + (threadIdx.x >> 3);
  const int D = a.D;
  const int64_t base = (int64_t)bh * a.L * D;  // contiguous backward tensors
  const T scale = (T)a.scale;
  const T c8 = T(8) * scale;

  T qv[M], gv[M], acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) qv[m] = gv[m] = acc[m] = 0;
  T di = 1, ei = 0;
  if (qi < a.L) {
    // rotated q row (tile loader semantics: fp32/fp64 rotation, one rounding)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int d = sub + 8 * m;
      if (d < D) {
        gv[m] = ld<DT>(a.g, base + (int64_t)qi * D + d);
        if constexpr (ROT) {
          const int p = d >> 1;
          const T x0 = ld<DT>(a.q, base + (int64_t)qi * D + 2 * p);
          const T x1 = ld<DT>(a.q, base + (int64_t)qi * D + 2 * p + 1);
          T c, s;
          table_cs<DT>(a.rc, a.rs, (int64_t)qi * (D / 2) + p, c, s);
          qv[m] = rnd<DT>(rot_pair(c, s, x0, x1, d & 1));
        } else {
          qv[m] = ld<DT>(a.q, base + (int64_t)qi * D + d);
        }
      }
    }
    di = ((const T*)a.dtot)[(int64_t)bh * a.L + qi];
    ei = ((const T*)a.e_ws)[(int64_t)bh * a.L + qi];
  }
  const int q_last = min(a.L, qblk * 32 + 32) - 1;
  const int kend = a.causal ? min(a.valid_len, q_last + 1) : a.valid_len;
  for (int k0 = 0; k0 < kend; k0 += KTG) {
    __syncthreads();
    load_tile<DT, ROT, DMAX, KTG>(ks, a.k, base, D, k0, a.L, D, a.rc, a.rs);
    load_tile<DT, false, DMAX, KTG>(vs, a.v, base, D, k0, a.L, D, nullptr, nullptr);
    __syncthreads();
    const int nk = min(KTG, kend - k0);
    for (int jj = 0; jj < nk; ++jj) {
      const int j = k0 + jj;
      T ps = 0, pg = 0;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (sub + 8 * m < D) {
          ps += qv[m] * ks[jj][sub + 8 * m];
          pg += gv[m] * vs[jj][sub + 8 * m];
        }
      }
      const T s = group8_sum(ps) * scale;
      const T gw = group8_sum(pg);
      const T w = rho8_acc(s) / di;
      T ds = c8 * rsq1p(s) * w * (gw - ei);
      if (a.causal && j > qi) ds = 0;
      const T dsr = rnd<DT>(ds);
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (sub + 8 * m < D) acc[m] += dsr * ks[jj][sub + 8 * m];
    }
  }
  unrotate_store<DT, M>(acc, a.out, base + (int64_t)qi * D, qi, D, sub, a.rc, a.rs, ROT, qi < a.L);
}

// dK/dV pass: one 8-lane group per key, sweeping queries i (>= j when causal).
template <int DT, int DMAX, bool ROT>
__global__ __launch_bounds__(256) void afa_bwd_dkdv_kernel(const GenArgs a) {
  typedef typename Acc<DT>::T T;
  constexpr int M = DMAX / 8;
  constexpr int KTG = gen_tile_rows<DT, DMAX>();
  __shared__ T qs[KTG][DMAX];
  __shared__ T gs[KTG][DMAX];
  __shared__ T dis[KTG];
  __shared__ T eis[KTG];
  const int nk = (a.L + 31) / 32;
  const int bh = blockIdx.x / nk, kblk = blockIdx.x % nk;
  const int sub = threadIdx.x & 7;
  const int kj = kblk * 32 + (threadIdx.x >> 3);
  const int D = a.D;
  const int64_t base = (int64_t)bh * a.L * D;
  const T scale = (T)a.scale;
  const T c8 = T(8) * scale;

  T kv[M], vv[M], adk[M], adv[M];
#pragma unroll
  for (int m = 0; m < M; ++m) kv[m] = vv[m] = adk[m] = adv[m] = 0;
  const bool key_ok = kj < a.L && kj < a.valid_len;
  if (kj < a.L) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int d = sub + 8 * m;
      if (d < D) {
        vv[m] = ld<DT>(a.v, base + (int64_t)kj * D + d);
        if constexpr (ROT) {
          const int p = d >> 1;
          const T x0 = ld<DT>(a.k, base + (int64_t)kj * D + 2 * p);
          const T x1 = ld<DT>(a.k, base + (int64_t)kj * D + 2 * p + 1);
          T c, s;
          table_cs<DT>(a.rc, a.rs, (int64_t)kj * (D / 2) + p, c, s);
          kv[m] = rnd<DT>(rot_pair(c, s, x0, x1, d & 1));
        } else {
          kv[m] = ld<DT>(a.k, base + (int64_t)kj * D + d);
        }
      }
    }
  }
  const int k_first = kblk * 32;
  const int qstart = a.causal ? k_first : 0;
  for (int i0 = qstart; i0 < a.L; i0 += KTG) {
    __syncthreads();
    load_tile<DT, ROT, DMAX, KTG>(qs, a.q, base, D, i0, a.L, D, a.rc, a.rs);
    load_tile<DT, false, DMAX, KTG>(gs, a.g, base, D, i0, a.L, D, nullptr, nullptr);
    for (int r = threadIdx.x; r < KTG; r += blockDim.x) {
      const int row = i0 + r;
      dis[r] = row < a.L ? ((const T*)a.dtot)[(int64_t)bh * a.L + row] : T(1);
      eis[r] = row < a.L ? ((const T*)a.e_ws)[(int64_t)bh * a.L + row] : T(0);
    }
    __syncthreads();
    const int nq = min(KTG, a.L - i0);
    for (int ii = 0; ii < nq; ++ii) {
      const int i = i0 + ii;
      T ps = 0, pg = 0;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (sub + 8 * m < D) {
          ps += kv[m] * qs[ii][sub + 8 * m];
          pg += vv[m] * gs[ii][sub + 8 * m];
        }
      }
      const T s = group8_sum(ps) * scale;
      const T gw = group8_sum(pg);
      const bool keep = key_ok && (!a.causal || kj <= i);
      const T w = keep ? rho8_acc(s) / dis[ii] : T(0);
      const T ds = keep ? c8 * rsq1p(s) * w * (gw - eis[ii]) : T(0);
      const T dsr = rnd<DT>(ds), wr = rnd<DT>(w);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (sub + 8 * m < D) {
          adk[m] += dsr * qs[ii][sub + 8 * m];
          adv[m] += wr * gs[ii][sub + 8 * m];
        }
      }
    }
  }
  unrotate_store<DT, M>(adk, a.dk, base + (int64_t)kj * D, kj, D, sub, a.rc, a.rs, ROT, kj < a.L);
  if (kj < a.L) {
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (sub + 8 * m < D) st<DT>(a.dv, base + (int64_t)kj * D + sub + 8 * m, adv[m]);
  }
}

// ------------------------------------------------------------------------------ launchers
static int dmax_for(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }

template <int DT, int DMAX>
static hipError_t gen_fwd_rot(const GenArgs& a, bool rot, hipStream_t st) {
  const int grid = a.B * a.H * ((a.L + 31) / 32);
  if (rot)
    hipLaunchKernelGGL((afa_fwd_generic_kernel<DT, DMAX, true>), dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((afa_fwd_generic_kernel<DT, DMAX, false>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DT>
static hipError_t gen_fwd_dt(const GenArgs& a, bool rot, hipStream_t st) {
  switch (dmax_for(a.D)) {
    case 32: return gen_fwd_rot<DT, 32>(a, rot, st);
    case 64: return gen_fwd_rot<DT, 64>(a, rot, st);
    case 128: return gen_fwd_rot<DT, 128>(a, rot, st);
    default: return gen_fwd_rot<DT, 256>(a, rot, st);
  }
}

hipError_t generic_fwd_launch(int dtype, const GenArgs& a, hipStream_t st) {
  const bool rot = a.rc != nullptr;
  switch (dtype) {
    case AFA_F32: return gen_fwd_dt<AFA_F32>(a, rot, st);
    case AFA_BF16: return gen_fwd_dt<AFA_BF16>(a, rot, st);
    case AFA_F16: return gen_fwd_dt<AFA_F16>(a, rot, st);
    default: return gen_fwd_dt<AFA_F64>(a, rot, st);
  }
}

template <int DT, int DMAX, bool ROT>
static hipError_t gen_bwd_all(const GenArgs& a, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.L;
  hipLaunchKernelGGL((afa_bwd_e_kernel<DT>), dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, st, a);
  const int grid = a.B * a.H * ((a.L + 31) / 32);
  hipLaunchKernelGGL((afa_bwd_dq_kernel<DT, DMAX, ROT>), dim3(grid), dim3(256), 0, st, a);
  hipLaunchKernelGGL((afa_bwd_dkdv_kernel<DT, DMAX, ROT>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DT, int DMAX>
static hipError_t gen_bwd_rot(const GenArgs& a, bool rot, hipStream_t st) {
  return rot ? gen_bwd_all<DT, DMAX, true>(a, st) : gen_bwd_all<DT, DMAX, false>(a, st);
}

template <int DT>
static hipError_t gen_bwd_dt(const GenArgs& a, bool rot, hipStream_t st) {
  switch (dmax_for(a.D)) {
    case 32: return gen_bwd_rot<DT, 32>(a, rot, st);
    case 64: return gen_bwd_rot<DT, 64>(a, rot, st);
    case 128: return gen_bwd_rot<DT, 128>(a, rot, st);
    default: return gen_bwd_rot<DT, 256>(a, rot, st);
  }
}

hipError_t generic_bwd_launch(int dtype, const GenArgs& a, hipStream_t st) {
  const bool rot = a.rc != nullptr;
  switch (dtype) {
    case AFA_F32: return gen_bwd_dt<AFA_F32>(a, rot, st);
    case AFA_BF16: return gen_bwd_dt<AFA_BF16>(a, rot, st);
    case AFA_F16: return gen_bwd_dt<AFA_F16>(a, rot, st);
    default: return gen_bwd_dt<AFA_F64>(a, rot, st);
  }
}

// ------------------------------------------------------------------------------ ring finish
// The final division of a ring's accumulators (src/kernels/pallas_afa.py:660-661):
// out = acc / (denom + sink) in the accumulation type, rounded to the input dtype; total
// (optional) receives denom + sink, the denominator the backward takes.  One thread per output
// element; acc, out and total are strided (b, h, l, and contiguous features for acc and out),
// denom is contiguous over (b, h, l).
template <int DT>
__global__ __launch_bounds__(256) void afa_ring_finish_kernel(const RingFinish r) {
  typedef typename Acc<DT>::T T;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)r.B * r.H * r.L * r.D) return;
  const int64_t row = i / r.D;
  const int64_t f = i - row * r.D;
  const int64_t l = row % r.L, bh = row / r.L;
  const int64_t h = bh % r.H, b = bh / r.H;
  const T d = ((const T*)r.denom)[row] + (T)r.sink;
  const T x = ((const T*)r.acc)[b * r.a_b + h * r.a_h + l * r.a_l + f];
  st<DT>(r.out, b * r.o_b + h * r.o_h + l * r.o_l + f, x / d);
  if (r.total != nullptr && f == 0) ((T*)r.total)[b * r.t_b + h * r.t_h + l * r.t_l] = d;
}

// The same with 8 features per thread and 16-byte loads and stores (head_dim a multiple of 8,
// 16-byte aligned bases, strides multiples of 8 elements): D / 8 threads per row, 256 / (D / 8)
// rows per workgroup, one index decomposition per thread.
template <int DT>
__global__ __launch_bounds__(256) void afa_ring_finish_vec_kernel(const RingFinish r) {
  typedef typename Acc<DT>::T T;
  const int tpr = r.D >> 3;
  const int rpb = 256 / tpr;
  const int t = (int)threadIdx.x / tpr;
  if (t >= rpb) return;
  const int64_t row = (int64_t)blockIdx.x * rpb + t;
  if (row >= (int64_t)r.B * r.H * r.L) return;
  const int c = ((int)threadIdx.x - t * tpr) * 8;
  const int64_t bh = row / r.L, l = row - bh * r.L;
  const int64_t b = bh / r.H, h = bh - b * r.H;
  const T d = ((const T*)r.denom)[row] + (T)r.sink;
  if (r.total != nullptr && c == 0) ((T*)r.total)[b * r.t_b + h * r.t_h + l * r.t_l] = d;
  const T* src = (const T*)r.acc + b * r.a_b + h * r.a_h + l * r.a_l + c;
  const int64_t o = b * r.o_b + h * r.o_h + l * r.o_l + c;
  T x[8];
  if constexpr (DT == AFA_F64) {
    typedef __attribute__((ext_vector_type(2))) double f64x2_t;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f64x2_t v = ((const f64x2_t*)src)[i];
      x[2 * i] = v[0];
      x[2 * i + 1] = v[1];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f64x2_t w;
      w[0] = x[2 * i] / d;
      w[1] = x[2 * i + 1] / d;
      ((f64x2_t*)((double*)r.out + o))[i] = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x4_t v = ((const f32x4_t*)src)[i];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[4 * i + u] = v[u];
    }
    if constexpr (DT == AFA_F32) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f32x4_t w;
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = x[4 * i + u] / d;
        ((f32x4_t*)((float*)r.out + o))[i] = w;
      }
    } else {
      u32x4_t w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = Elem<DT>::pack(x[2 * i] / d, x[2 * i + 1] / d);
      *(u32x4_t*)((unsigned short*)r.out + o) = w;
    }
  }
}

template <int DT>
static void ring_finish_dt(const RingFinish& r, bool vec, hipStream_t st) {
  if (vec) {
    const int64_t rpb = 256 / (r.D / 8);
    const int64_t rows = (int64_t)r.B * r.H * r.L;
    hipLaunchKernelGGL((afa_ring_finish_vec_kernel<DT>), dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0,
                       st, r);
  } else {
    const int64_t n = (int64_t)r.B * r.H * r.L * r.D;
    hipLaunchKernelGGL((afa_ring_finish_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, r);
  }
}

hipError_t ring_finish_launch(int dtype, const RingFinish& r, hipStream_t st) {
  bool vec = r.D % 8 == 0 && r.D <= 2048 && ((uintptr_t)r.acc & 15) == 0 && ((uintptr_t)r.out & 15) == 0;
  for (int64_t s : {r.a_b, r.a_h, r.a_l, r.o_b, r.o_h, r.o_l})
    if (s % 8 != 0) vec = false;
  switch (dtype) {
    case AFA_F32: ring_finish_dt<AFA_F32>(r, vec, st); break;
    case AFA_BF16: ring_finish_dt<AFA_BF16>(r, vec, st); break;
    case AFA_F16: ring_finish_dt<AFA_F16>(r, vec, st); break;
    default: ring_finish_dt<AFA_F64>(r, vec, st); break;
  }
  return hipGetLastError();
}

}  // namespace afa
