// A-Softmax row kernels and the elementwise octic weight.
//
// algebraic_softmax (src/attention.py:53-91, AVN from src/primitives.py:56-79), per row of n:
//   z = promote(x);  tau = rsqrt(sum(z^2) * (1/n) + eps);  y = tau z
//   k = rho(y)^8, r = rsqrt(1 + y^2);  p = k / (sum k + Omega);  output cast(p, x.dtype)
// VJP (src/attention.py:75-82, src/primitives.py:73-79):
//   ng = 8 r p (g - sum(p g));  dx = tau (ng - (sum(ng y) / n) y)
// Rows are handled by one wave each; values are promoted to fp32 (fp64 stays fp64) and the
// reference's two-branch rho formula is evaluated op for op.  These kernels are HBM bound.
#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

template <int DT>
struct SAcc {
  typedef float T;
};
template <>
struct SAcc<AFA_F64> {
  typedef double T;
};

template <int DT>
__device__ __forceinline__ typename SAcc<DT>::T sload(const void* p, int64_t i) {
  if constexpr (DT == AFA_F64) {
    return ((const double*)p)[i];
  } else {
    return Elem<DT>::load(p, i);
  }
}
template <int DT>
__device__ __forceinline__ void sstore(void* p, int64_t i, typename SAcc<DT>::T x) {
  if constexpr (DT == AFA_F64) {
    ((double*)p)[i] = x;
  } else {
    Elem<DT>::store(p, i, x);
  }
}

template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// rho(z)^8 and r = rsqrt(1 + z^2), op for op as src/attention.py:18-26.
template <typename T>
__device__ __forceinline__ T octic_ref(T z, T& r_out) {
  const T one = 1;
  const T zz = z * z;
  T r;
  if constexpr (sizeof(T) == 8) {
    r = 1.0 / sqrt(one + zz);
  } else {
    r = 1.0f / __builtin_sqrtf(one + zz);
  }
  const T u = z * r;
  const T rho = z < 0 ? r / (one - u) : z + (one + zz) * r;
  const T k2 = rho * rho;
  const T k4 = k2 * k2;
  r_out = r;
  return k4 * k4;
}

template <typename T>
__device__ __forceinline__ T inv_sqrt(T x) {
  if constexpr (sizeof(T) == 8) {
    return 1.0 / sqrt(x);
  } else {
    return 1.0f / __builtin_sqrtf(x);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void asoftmax_fwd_kernel(int64_t rows, int64_t n, const void* x,
                                                           void* y, double sink, double eps) {
#pragma clang fp contract(off)
  typedef typename SAcc<DT>::T T;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * n;
  T ss = 0;
  for (int64_t i = lane; i < n; i += 64) {
    const T z = sload<DT>(x, base + i);
    ss += z * z;
  }
  ss = wave_sum(ss);
  const T tau = inv_sqrt(ss * (T(1) / (T)n) + (T)eps);
  T ks = 0;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    ks += octic_ref(sload<DT>(x, base + i) * tau, r);
  }
  ks = wave_sum(ks);
  const T den = ks + (T)sink;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    const T k = octic_ref(sload<DT>(x, base + i) * tau, r);
    sstore<DT>(y, base + i, k / den);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void asoftmax_bwd_kernel(int64_t rows, int64_t n, const void* x,
                                                           const void* g, void* dx, double sink,
                                                           double eps) {
#pragma clang fp contract(off)
  typedef typename SAcc<DT>::T T;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * n;
  const T inv_n = T(1) / (T)n;
  T ss = 0;
  for (int64_t i = lane; i < n; i += 64) {
    const T z = sload<DT>(x, base + i);
    ss += z * z;
  }
  ss = wave_sum(ss);
  const T tau = inv_sqrt(ss * inv_n + (T)eps);
  T ks = 0;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    ks += octic_ref(sload<DT>(x, base + i) * tau, r);
  }
  ks = wave_sum(ks);
  const T den = ks + (T)sink;
  // dot = sum(p g)
  T dot = 0;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    const T p = octic_ref(sload<DT>(x, base + i) * tau, r) / den;
    dot += p * sload<DT>(g, base + i);
  }
  dot = wave_sum(dot);
  // radial = sum(ng y) / n
  T rad = 0;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    const T yv = sload<DT>(x, base + i) * tau;
    const T p = octic_ref(yv, r) / den;
    const T ng = T(8) * r * p * (sload<DT>(g, base + i) - dot);
    rad += ng * yv;
  }
  rad = wave_sum(rad) * inv_n;
  for (int64_t i = lane; i < n; i += 64) {
    T r;
    const T yv = sload<DT>(x, base + i) * tau;
    const T p = octic_ref(yv, r) / den;
    const T ng = T(8) * r * p * (sload<DT>(g, base + i) - dot);
    sstore<DT>(dx, base + i, tau * (ng - rad * yv));
  }
}

template <int DT>
__global__ __launch_bounds__(256) void octic_fwd_kernel(int64_t n, const void* x, void* y) {
  typedef typename SAcc<DT>::T T;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  T r;
  sstore<DT>(y, i, octic_ref(sload<DT>(x, i), r));
}

template <int DT>
__global__ __launch_bounds__(256) void octic_bwd_kernel(int64_t n, const void* x, const void* g,
                                                        void* dx) {
#pragma clang fp contract(off)
  typedef typename SAcc<DT>::T T;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  T r;
  const T k = octic_ref(sload<DT>(x, i), r);
  sstore<DT>(dx, i, T(8) * r * k * sload<DT>(g, i));
}

#define AFA_DISPATCH_DT(dtype, FN, ...)            \
  switch (dtype) {                                 \
    case AFA_F32: FN<AFA_F32>(__VA_ARGS__); break; \
    case AFA_BF16: FN<AFA_BF16>(__VA_ARGS__); break; \
    case AFA_F16: FN<AFA_F16>(__VA_ARGS__); break; \
    default: FN<AFA_F64>(__VA_ARGS__); break;      \
  }

template <int DT>
static void sm_fwd(int64_t rows, int64_t n, const void* x, void* y, double sink, double eps, hipStream_t st) {
  hipLaunchKernelGGL((asoftmax_fwd_kernel<DT>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, rows, n, x, y, sink, eps);
}
template <int DT>
static void sm_bwd(int64_t rows, int64_t n, const void* x, const void* g, void* dx, double sink, double eps, hipStream_t st) {
  hipLaunchKernelGGL((asoftmax_bwd_kernel<DT>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, rows, n, x, g, dx, sink, eps);
}
template <int DT>
static void oc_fwd(int64_t n, const void* x, void* y, hipStream_t st) {
  hipLaunchKernelGGL((octic_fwd_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n, x, y);
}
template <int DT>
static void oc_bwd(int64_t n, const void* x, const void* g, void* dx, hipStream_t st) {
  hipLaunchKernelGGL((octic_bwd_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n, x, g, dx);
}

hipError_t asoftmax_fwd_launch(int dtype, int64_t rows, int64_t n, const void* x, void* y, double sink,
                               double eps, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, sm_fwd, rows, n, x, y, sink, eps, st);
  return hipGetLastError();
}
hipError_t asoftmax_bwd_launch(int dtype, int64_t rows, int64_t n, const void* x, const void* g,
                               void* dx, double sink, double eps, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, sm_bwd, rows, n, x, g, dx, sink, eps, st);
  return hipGetLastError();
}
hipError_t octic_fwd_launch(int dtype, int64_t n, const void* x, void* y, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, oc_fwd, n, x, y, st);
  return hipGetLastError();
}
hipError_t octic_bwd_launch(int dtype, int64_t n, const void* x, const void* g, void* dx, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, oc_bwd, n, x, g, dx, st);
  return hipGetLastError();
}

}  // namespace afa
