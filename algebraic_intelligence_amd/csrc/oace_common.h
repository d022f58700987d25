// Device helpers shared by the OACE kernels (oace.hip, oace_mfma.hip).
#pragma once

#include <type_traits>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

template <typename A>
__device__ __forceinline__ A o_rsq(A x) {
  if constexpr (std::is_same<A, double>::value) return 1.0 / sqrt(x);
  else return __builtin_amdgcn_rsqf(x);
}
template <typename A>
__device__ __forceinline__ A o_rcp(A x) {
  if constexpr (std::is_same<A, double>::value) return 1.0 / x;
  else return __builtin_amdgcn_rcpf(x);
}

template <typename A>
struct Oct {
  A k8, rho7, rho, r;
};

// Two-branch octic parts (pallas_oace.py:38-56): rho = x + (1+x^2) r for x >= 0 and r / (1 - x r)
// for x < 0, which has no cancellation; k8 = rho^8, rho7 = rho k2 k4 as the reference.
template <typename A>
__device__ __forceinline__ Oct<A> octic(A x) {
  const A rad = A(1) + x * x;
  const A r = o_rsq<A>(rad);
  const A pos = x + rad * r;
  const A neg = r * o_rcp<A>(A(1) - x * r);
  Oct<A> o;
  o.rho = x < A(0) ? neg : pos;
  o.r = r;
  const A k2 = o.rho * o.rho;
  const A k4 = k2 * k2;
  o.k8 = k4 * k4;
  o.rho7 = o.rho * k2 * k4;
  return o;
}

// Branch-free fp32 octic parts: rho = fma(1 + x^2, rsqrt(1 + x^2), x) for both signs.  For x < 0
// this cancels, but the absolute error of rho^7, rho^8 stays below ~1e-7 there (rho < 1), far
// below the resolution of sums over a vocabulary of such terms, which is where it is used; the
// target's rho is always taken from the two-branch form.
__device__ __forceinline__ Oct<float> octic_fast(float x) {
  const float t = __builtin_fmaf(x, x, 1.0f);
  Oct<float> o;
  o.r = __builtin_amdgcn_rsqf(t);
  o.rho = __builtin_fmaf(t, o.r, x);
  const float k2 = o.rho * o.rho;
  const float k4 = k2 * k2;
  o.k8 = k4 * k4;
  o.rho7 = o.rho * k2 * k4;
  return o;
}

// Row record from the forward sums (pallas_oace.py:166-187).
template <typename A>
__device__ __forceinline__ void oace_finalize_row(A* rec, A tau, A s0, A s1, A s2, A s3, A rho_t, A rn_t,
                                                  A inv_v, A gamma) {
  const A inv_S = o_rcp<A>(s0);
  const A S8 = o_rsq<A>(o_rsq<A>(o_rsq<A>(inv_S)));
  const A scale = S8 * inv_S;
  const A sum_p78 = scale * s1;
  const A p_c_inv8 = S8 * o_rcp<A>(rho_t);
  const A diff = sum_p78 - p_c_inv8;
  const A radial = (scale * s3 - rn_t * p_c_inv8 - diff * inv_S * s2) * inv_v;
  const A loss = gamma * (A(8) * p_c_inv8 + A(8.0 / 7.0) * sum_p78 - A(64.0 / 7.0));
  rec[OACE_TAU] = tau;
  rec[OACE_INV_S] = inv_S;
  rec[OACE_S8] = S8;
  rec[OACE_SUM_P78] = sum_p78;
  rec[OACE_PC_INV8] = p_c_inv8;
  rec[OACE_RADIAL] = radial;
  rec[OACE_LOSS] = loss;
  rec[7] = A(0);
}

}  // namespace afa
