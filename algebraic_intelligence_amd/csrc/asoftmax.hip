// A-Softmax row kernels and the elementwise octic weight.
//
// algebraic_softmax (src/attention.py:53-91, AVN from src/primitives.py:56-79), per row of n:
//   z = promote(x);  tau = rsqrt(sum(z^2) * (1/n) + eps);  y = tau z
//   k = rho(y)^8, r = rsqrt(1 + y^2);  p = k / (sum k + Omega);  output cast(p, x.dtype)
// VJP (src/attention.py:75-82, src/primitives.py:73-79):
//   ng = 8 r p (g - sum(p g));  dx = tau (ng - (sum(ng y) / n) y)
// Rows are handled by one wave each; values are promoted to fp32 (fp64 stays fp64) and the
// reference's two-branch rho formula is evaluated op for op.  These kernels are HBM bound; rows
// that fit in registers take the single-read kernels further down.
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

// rho(x)^8 and r = rsqrt(1 + x^2), both stored in the accumulation type (fp32, fp64 for fp64
// inputs): src/attention.py:18-26 returns the pair, r being the factor of the VJP 8 r rho^8 g.
template <int DT>
__global__ __launch_bounds__(256) void octic_fwd_r_kernel(int64_t n, const void* x, void* k, void* r) {
  typedef typename SAcc<DT>::T T;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  T rr;
  const T kk = octic_ref(sload<DT>(x, i), rr);
  ((T*)k)[i] = kk;
  ((T*)r)[i] = rr;
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


// rho(z)^8 and r = rsqrt(1 + z^2) with the hardware reciprocal square root and reciprocal
// (1 ulp each), the reference's own operations (src/attention.py:18-26 uses lax.rsqrt; its
// division r / (1 - u) becomes r * rcp(1 - u)).  Used by the register-resident kernels.
__device__ __forceinline__ float octic_hw(float z, float& r_out) {
  const float t = __builtin_fmaf(z, z, 1.0f);
  const float r = __builtin_amdgcn_rsqf(t);
  const float neg = r * __builtin_amdgcn_rcpf(1.0f - z * r);
  const float pos = __builtin_fmaf(t, r, z);
  const float rho = z < 0.0f ? neg : pos;
  const float k2 = rho * rho;
  const float k4 = k2 * k2;
  r_out = r;
  return k4 * k4;
}

// ---------------------------------------------------------------- register-resident row kernels
// One wave per row, the whole row held in registers: 16-byte vector loads (lane l owns chunks
// l, l + 64, ... of EPC elements), one HBM read of x (and g), one write; rho^8 and r are
// evaluated once per element with the hardware rsqrt / reciprocal (octic_hw) and the row is
// normalised with one division and products; the multi-pass kernels above keep IEEE 1/sqrt and
// divisions throughout.  Used when the row fits
// (cols <= 64 * EPC * NCH) and cols is a multiple of the chunk width on 16-byte-aligned rows.
template <int DT>
struct Chunk {
  static constexpr int EPC = DT == AFA_F32 ? 4 : 8;
  static __device__ __forceinline__ void load(const void* p, int64_t e0, float (&v)[8]) {
    const u32x4_t w = *(const u32x4_t*)((const char*)p + e0 * (DT == AFA_F32 ? 4 : 2));
    if constexpr (DT == AFA_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // bind the element first: a bit_cast of a runtime-indexed vector element reads element 0
        const unsigned u = w[i];
        v[i] = __builtin_bit_cast(float, u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = Elem<DT>::lo(w[i]);
        v[2 * i + 1] = Elem<DT>::hi(w[i]);
      }
    }
  }
  static __device__ __forceinline__ void store(void* p, int64_t e0, const float (&v)[8]) {
    u32x4_t w;
    if constexpr (DT == AFA_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = v[i];
        w[i] = __builtin_bit_cast(unsigned, f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = Elem<DT>::pack(v[2 * i], v[2 * i + 1]);
    }
    *(u32x4_t*)((char*)p + e0 * (DT == AFA_F32 ? 4 : 2)) = w;
  }
};

template <int DT, int NCH>
__global__ __launch_bounds__(256) void asoftmax_fwd_reg_kernel(int64_t rows, int64_t n, const void* x,
                                                               void* y, double sink, double eps) {
#pragma clang fp contract(off)
  constexpr int EPC = Chunk<DT>::EPC;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * n;
  float v[NCH][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e0 = (int64_t)(lane + 64 * j) * EPC;
    if (e0 < n) {
      Chunk<DT>::load(x, base + e0, v[j]);
#pragma unroll
      for (int i = 0; i < EPC; ++i) ss += v[j][i] * v[j][i];
    }
  }
  ss = wave_sum(ss);
  const float tau = inv_sqrt(ss * (1.f / (float)n) + (float)eps);
  float ks = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if ((int64_t)(lane + 64 * j) * EPC < n) {
#pragma unroll
      for (int i = 0; i < EPC; ++i) {
        float r;
        v[j][i] = octic_hw(v[j][i] * tau, r);
        ks += v[j][i];
      }
    }
  }
  ks = wave_sum(ks);
  const float inv = 1.0f / (ks + (float)sink);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e0 = (int64_t)(lane + 64 * j) * EPC;
    if (e0 < n) {
#pragma unroll
      for (int i = 0; i < EPC; ++i) v[j][i] = v[j][i] * inv;
      Chunk<DT>::store(y, base + e0, v[j]);
    }
  }
}

template <int DT, int NCH>
__global__ __launch_bounds__(256) void asoftmax_bwd_reg_kernel(int64_t rows, int64_t n, const void* x,
                                                               const void* g, void* dx, double sink,
                                                               double eps) {
#pragma clang fp contract(off)
  // The row's x and g stay in registers as their raw 16-byte chunks and are unpacked where used;
  // one float per element, w = 8 r rho^8, carries the octic between passes.  sum(p g) is taken
  // as sum(rho^8 g) / (sum rho^8 + sink) in the pass that forms sum rho^8, so three wave
  // reductions serve the row, and the kernel holds few enough registers for six or more waves
  // per SIMD to keep loads in flight.
  constexpr int EPC = Chunk<DT>::EPC;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t base = row * n;
  const float inv_n = 1.f / (float)n;
  const int esz = DT == AFA_F32 ? 4 : 2;
  u32x4_t xr[NCH], gr[NCH];
  float w[NCH][8];
  auto unpack = [&](const u32x4_t& c, float (&v)[8]) {
    if constexpr (DT == AFA_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned u = c[i];
        v[i] = __builtin_bit_cast(float, u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = Elem<DT>::lo(c[i]);
        v[2 * i + 1] = Elem<DT>::hi(c[i]);
      }
    }
  };
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e0 = (int64_t)(lane + 64 * j) * EPC;
    if (e0 < n) {
      xr[j] = *(const u32x4_t*)((const char*)x + (base + e0) * esz);
      gr[j] = *(const u32x4_t*)((const char*)g + (base + e0) * esz);
      float z[8];
      unpack(xr[j], z);
#pragma unroll
      for (int i = 0; i < EPC; ++i) ss += z[i] * z[i];
    }
  }
  ss = wave_sum(ss);
  const float tau = inv_sqrt(ss * inv_n + (float)eps);
  float ks = 0.f, pg = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if ((int64_t)(lane + 64 * j) * EPC < n) {
      float z[8], gv[8];
      unpack(xr[j], z);
      unpack(gr[j], gv);
#pragma unroll
      for (int i = 0; i < EPC; ++i) {
        float r;
        const float p = octic_hw(z[i] * tau, r);
        ks += p;
        pg += p * gv[i];
        w[j][i] = 8.f * r * p;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // one chunk's unpacked values live at a time
  }
  ks = wave_sum(ks);
  pg = wave_sum(pg);
  const float inv = 1.0f / (ks + (float)sink);
  const float dot = pg * inv;
  float rad = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if ((int64_t)(lane + 64 * j) * EPC < n) {
      float z[8], gv[8];
      unpack(xr[j], z);
      unpack(gr[j], gv);
#pragma unroll
      for (int i = 0; i < EPC; ++i) {
        w[j][i] = w[j][i] * inv * (gv[i] - dot);  // ng
        rad += w[j][i] * (z[i] * tau);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  rad = wave_sum(rad) * inv_n;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e0 = (int64_t)(lane + 64 * j) * EPC;
    if (e0 < n) {
      float z[8];
      unpack(xr[j], z);
#pragma unroll
      for (int i = 0; i < EPC; ++i) w[j][i] = tau * (w[j][i] - rad * (z[i] * tau));
      Chunk<DT>::store(dx, base + e0, w[j]);
    }
  }
}

// Chunks per lane for the register kernels (0 = the row does not fit: use the multi-pass kernel).
static int reg_chunks(int dtype, int64_t n, const void* a, const void* b, const void* c, int max_nch) {
  if (dtype == AFA_F64) return 0;
  const int epc = dtype == AFA_F32 ? 4 : 8;
  const int esz = dtype == AFA_F32 ? 4 : 2;
  if (n % epc != 0) return 0;
  for (const void* p : {a, b, c})
    if (p != nullptr && ((uintptr_t)p & 15u) != 0) return 0;
  if (((n * esz) & 15) != 0) return 0;
  for (int nch = 1; nch <= max_nch; nch *= 2)
    if (n <= (int64_t)64 * epc * nch) return nch;
  return 0;
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
static void oc_fwd_r(int64_t n, const void* x, void* k, void* r, hipStream_t st) {
  hipLaunchKernelGGL((octic_fwd_r_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n, x, k, r);
}
template <int DT>
static void oc_bwd(int64_t n, const void* x, const void* g, void* dx, hipStream_t st) {
  hipLaunchKernelGGL((octic_bwd_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n, x, g, dx);
}

template <int DT, int NCH>
static void sm_fwd_reg(int64_t rows, int64_t n, const void* x, void* y, double sink, double eps, hipStream_t st) {
  hipLaunchKernelGGL((asoftmax_fwd_reg_kernel<DT, NCH>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, rows, n, x, y, sink, eps);
}
template <int DT, int NCH>
static void sm_bwd_reg(int64_t rows, int64_t n, const void* x, const void* g, void* dx, double sink, double eps,
                       hipStream_t st) {
  hipLaunchKernelGGL((asoftmax_bwd_reg_kernel<DT, NCH>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, rows, n, x, g, dx, sink, eps);
}
template <int DT>
static void sm_fwd_reg_dt(int nch, int64_t rows, int64_t n, const void* x, void* y, double sink, double eps, hipStream_t st) {
  switch (nch) {
    case 1: sm_fwd_reg<DT, 1>(rows, n, x, y, sink, eps, st); break;
    case 2: sm_fwd_reg<DT, 2>(rows, n, x, y, sink, eps, st); break;
    case 4: sm_fwd_reg<DT, 4>(rows, n, x, y, sink, eps, st); break;
    default: sm_fwd_reg<DT, 8>(rows, n, x, y, sink, eps, st); break;
  }
}
template <int DT>
static void sm_bwd_reg_dt(int nch, int64_t rows, int64_t n, const void* x, const void* g, void* dx, double sink,
                          double eps, hipStream_t st) {
  switch (nch) {
    case 1: sm_bwd_reg<DT, 1>(rows, n, x, g, dx, sink, eps, st); break;
    case 2: sm_bwd_reg<DT, 2>(rows, n, x, g, dx, sink, eps, st); break;
    default: sm_bwd_reg<DT, 4>(rows, n, x, g, dx, sink, eps, st); break;
  }
}

hipError_t asoftmax_fwd_launch(int dtype, int64_t rows, int64_t n, const void* x, void* y, double sink,
                               double eps, hipStream_t st) {
  const int nch = reg_chunks(dtype, n, x, y, nullptr, 8);
  if (nch > 0) {
    if (dtype == AFA_F32) sm_fwd_reg_dt<AFA_F32>(nch, rows, n, x, y, sink, eps, st);
    else if (dtype == AFA_BF16) sm_fwd_reg_dt<AFA_BF16>(nch, rows, n, x, y, sink, eps, st);
    else sm_fwd_reg_dt<AFA_F16>(nch, rows, n, x, y, sink, eps, st);
    return hipGetLastError();
  }
  AFA_DISPATCH_DT(dtype, sm_fwd, rows, n, x, y, sink, eps, st);
  return hipGetLastError();
}
hipError_t asoftmax_bwd_launch(int dtype, int64_t rows, int64_t n, const void* x, const void* g,
                               void* dx, double sink, double eps, hipStream_t st) {
  const int nch = reg_chunks(dtype, n, x, g, dx, 4);
  if (nch > 0) {
    if (dtype == AFA_F32) sm_bwd_reg_dt<AFA_F32>(nch, rows, n, x, g, dx, sink, eps, st);
    else if (dtype == AFA_BF16) sm_bwd_reg_dt<AFA_BF16>(nch, rows, n, x, g, dx, sink, eps, st);
    else sm_bwd_reg_dt<AFA_F16>(nch, rows, n, x, g, dx, sink, eps, st);
    return hipGetLastError();
  }
  AFA_DISPATCH_DT(dtype, sm_bwd, rows, n, x, g, dx, sink, eps, st);
  return hipGetLastError();
}
hipError_t octic_fwd_launch(int dtype, int64_t n, const void* x, void* y, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, oc_fwd, n, x, y, st);
  return hipGetLastError();
}
hipError_t octic_fwd_r_launch(int dtype, int64_t n, const void* x, void* k, void* r, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, oc_fwd_r, n, x, k, r, st);
  return hipGetLastError();
}
hipError_t octic_bwd_launch(int dtype, int64_t n, const void* x, const void* g, void* dx, hipStream_t st) {
  AFA_DISPATCH_DT(dtype, oc_bwd, n, x, g, dx, st);
  return hipGetLastError();
}

}  // namespace afa
