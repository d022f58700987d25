// Cayley rotary (AGO) kernels: table construction and pairwise rotation.
//
// Tables (src/attention.py:155-204): with Cayley parameter w_k,
//   c0 = (1 - w^2)/(1 + w^2), s0 = 2w/(1 + w^2);  row 0 = (1, 0);
//   row m+1 = (c0 c - s0 s, s0 c + c0 s) renormalised by rsqrt of its squared norm.
// The recurrence is sequential in position and independent per pair, so one thread owns one
// pair column and walks the positions.  Default w_k = 1/(1 + alpha k)^2 with
// alpha = (sqrt(base) - 1) / max(D/2 - 1, 1), sqrt(base) = base * rsqrt(base) (:180-187).
// Every operation is rounded separately in the table type (no contraction).
//
// Rotation (src/attention.py:142-152): (x0, x1) -> (c x0 - s x1, s x0 + c x1) with c and s
// first cast to the x dtype; computed in fp32 (fp64 for fp64) and rounded once.
#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

template <typename T>
__device__ __forceinline__ T inv_sqrt_ieee(T x) {
  if constexpr (sizeof(T) == 8) {
    return 1.0 / sqrt(x);
  } else {
    return 1.0f / __builtin_sqrtf(x);
  }
}

template <typename T>
__global__ __launch_bounds__(64) void ago_tables_kernel(int pairs, int len, const T* freqs, T base,
                                                        T* c_out, T* s_out) {
#pragma clang fp contract(off)
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= pairs) return;
  T w;
  if (freqs != nullptr) {
    w = freqs[p];
  } else {
    const T sqrt_base = base * inv_sqrt_ieee(base);
    const T denom = pairs - 1 > 1 ? (T)(pairs - 1) : (T)1;
    const T alpha = (sqrt_base - (T)1) / denom;
    const T lin = (T)1 + alpha * (T)p;
    w = (T)1 / (lin * lin);
  }
  const T w2 = w * w;
  const T cb = ((T)1 - w2) / ((T)1 + w2);
  const T sb = ((T)2 * w) / ((T)1 + w2);
  T c = 1, s = 0;
  for (int m = 0; m < len; ++m) {
    c_out[(int64_t)m * pairs + p] = c;
    s_out[(int64_t)m * pairs + p] = s;
    const T cn = cb * c - sb * s;
    const T sn = sb * c + cb * s;
    const T r = inv_sqrt_ieee(cn * cn + sn * sn);
    c = cn * r;
    s = sn * r;
  }
}

hipError_t ago_tables_launch(int table_dtype, int pairs, int len, const void* freqs, double base,
                             void* c_out, void* s_out, hipStream_t st) {
  const int blocks = (pairs + 63) / 64;
  if (table_dtype == AFA_F64) {
    hipLaunchKernelGGL((ago_tables_kernel<double>), dim3(blocks), dim3(64), 0, st, pairs, len,
                       (const double*)freqs, base, (double*)c_out, (double*)s_out);
  } else {
    hipLaunchKernelGGL((ago_tables_kernel<float>), dim3(blocks), dim3(64), 0, st, pairs, len,
                       (const float*)freqs, (float)base, (float*)c_out, (float*)s_out);
  }
  return hipGetLastError();
}

template <int TD>
__device__ __forceinline__ float table_load_f32(const void* t, int64_t i) {
  if constexpr (TD == AFA_F32) return ((const float*)t)[i];
  if constexpr (TD == AFA_F64) return (float)((const double*)t)[i];
  if constexpr (TD == AFA_BF16) return Elem<AFA_BF16>::load(t, i);
  return Elem<AFA_F16>::load(t, i);
}

template <int DT, int TD>
__global__ __launch_bounds__(256) void ago_rotate_kernel(int64_t npairs_total, int64_t seq_len,
                                                         int64_t inner, int pairs, const void* x,
                                                         void* y, const void* rc, const void* rs) {
#pragma clang fp contract(off)
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= npairs_total) return;
  const int p = (int)(e % pairs);
  const int64_t row = e / pairs;               // index over (outer, seq, inner)
  const int64_t t = (row / inner) % seq_len;   // sequence position
  const int64_t tix = t * pairs + p;
  if constexpr (DT == AFA_F64) {
    double c, s;
    if constexpr (TD == AFA_F64) {
      c = ((const double*)rc)[tix];
      s = ((const double*)rs)[tix];
    } else {
      c = table_load_f32<TD>(rc, tix);
      s = table_load_f32<TD>(rs, tix);
    }
    const double x0 = ((const double*)x)[2 * e], x1 = ((const double*)x)[2 * e + 1];
    ((double*)y)[2 * e] = c * x0 - s * x1;
    ((double*)y)[2 * e + 1] = s * x0 + c * x1;
  } else {
    // cast the table to the x dtype first (c.astype(x.dtype))
    const float c = Elem<DT>::round(table_load_f32<TD>(rc, tix));
    const float s = Elem<DT>::round(table_load_f32<TD>(rs, tix));
    const float x0 = Elem<DT>::load(x, 2 * e), x1 = Elem<DT>::load(x, 2 * e + 1);
    const float y0 = c * x0 - s * x1;
    const float y1 = s * x0 + c * x1;
    Elem<DT>::store(y, 2 * e, y0);
    Elem<DT>::store(y, 2 * e + 1, y1);
  }
}

template <int DT>
static hipError_t ago_rotate_dt(int table_dtype, int64_t n, int64_t seq, int64_t inner, int pairs,
                                const void* x, void* y, const void* rc, const void* rs,
                                hipStream_t st) {
  const unsigned blocks = (unsigned)((n + 255) / 256);
  switch (table_dtype) {
    case AFA_F32:
      hipLaunchKernelGGL((ago_rotate_kernel<DT, AFA_F32>), dim3(blocks), dim3(256), 0, st, n, seq, inner, pairs, x, y, rc, rs);
      break;
    case AFA_F64:
      hipLaunchKernelGGL((ago_rotate_kernel<DT, AFA_F64>), dim3(blocks), dim3(256), 0, st, n, seq, inner, pairs, x, y, rc, rs);
      break;
    case AFA_BF16:
      hipLaunchKernelGGL((ago_rotate_kernel<DT, AFA_BF16>), dim3(blocks), dim3(256), 0, st, n, seq, inner, pairs, x, y, rc, rs);
      break;
    default:
      hipLaunchKernelGGL((ago_rotate_kernel<DT, AFA_F16>), dim3(blocks), dim3(256), 0, st, n, seq, inner, pairs, x, y, rc, rs);
      break;
  }
  return hipGetLastError();
}

hipError_t ago_rotate_launch(int dtype, int table_dtype, int64_t outer, int64_t seq, int64_t inner,
                             int dim, const void* x, void* y, const void* rc, const void* rs,
                             hipStream_t st) {
  const int pairs = dim / 2;
  const int64_t n = outer * seq * inner * pairs;
  switch (dtype) {
    case AFA_F32: return ago_rotate_dt<AFA_F32>(table_dtype, n, seq, inner, pairs, x, y, rc, rs, st);
    case AFA_BF16: return ago_rotate_dt<AFA_BF16>(table_dtype, n, seq, inner, pairs, x, y, rc, rs, st);
    case AFA_F16: return ago_rotate_dt<AFA_F16>(table_dtype, n, seq, inner, pairs, x, y, rc, rs, st);
    default: return ago_rotate_dt<AFA_F64>(table_dtype, n, seq, inner, pairs, x, y, rc, rs, st);
  }
}

}  // namespace afa
