// OACE loss head: the octic algebraic cross-entropy over an AVN-normalised A-Softmax, either on
// given logits (fused_oace_softmax_loss, src/model.py:180-240) or fused with the vocabulary
// projection z = h W (fused_linear_oace, src/kernels/pallas_oace.py:59-293).
//
// Per row n of logits z (length V), with calc type A (fp32; fp64 for fp64 inputs):
//   tau = rsqrt(sum z^2 / V + eps);  x = tau z;  r = rsqrt(1 + x^2);  rho = x + (1+x^2) r
//   (rho = r / (1 - x r) for x < 0);  k8 = rho^8;  rho7 = rho^7
//   sums  S0 = sum k8, S1 = sum rho7, S2 = sum (r x) k8, S3 = sum (r x) rho7; target rho_t, (r x)_t
//   inv_S = 1/S0, S8 = rsqrt(rsqrt(rsqrt(inv_S))), scale = S8 inv_S, sum_p78 = scale S1,
//   p_c_inv8 = S8 / rho_t, radial = (scale S3 - (r x)_t p_c_inv8 - (sum_p78 - p_c_inv8) inv_S S2) / V,
//   loss = gamma (8 p_c_inv8 + 8/7 sum_p78 - 64/7)                       (pallas_oace.py:166-187)
// and the backward dz = tau c (r bracket - radial x), c = 8 gamma g / N,
//   bracket = scale rho7 - [v = target] p_c_inv8 - (k8 inv_S)(sum_p78 - p_c_inv8)  (:245-256).
//
// This file holds the generic path (any dtype): row kernels over materialised logits, a tiled
// SIMT GEMM for z = h W, dh = dz W^T and dW = h^T dz, and the transposition of W used by the
// MFMA path (oace_mfma.hip).
#include <algorithm>

#include "oace_common.h"

namespace afa {

namespace {

template <typename A, typename T>
__device__ __forceinline__ A ld_as(const T* p, int64_t i) {
  if constexpr (std::is_same<T, __bf16>::value) return (A)(float)p[i];
  else if constexpr (std::is_same<T, _Float16>::value) return (A)(float)p[i];
  else return (A)p[i];
}
template <typename T, typename A>
__device__ __forceinline__ void st_as(T* p, int64_t i, A x) {
  if constexpr (std::is_same<T, __bf16>::value) p[i] = (__bf16)(float)x;
  else if constexpr (std::is_same<T, _Float16>::value) p[i] = (_Float16)(float)x;
  else p[i] = (T)x;
}

template <typename A>
__device__ __forceinline__ A wave_sum(A x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
  return x;
}

// Sum over a 256-thread block; every thread gets the result.
template <typename A, int K>
__device__ __forceinline__ void block_sum(A (&x)[K], A* sh /* 4*K */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < K; ++i) x[i] = wave_sum(x[i]);
  __syncthreads();
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < K; ++i) sh[wave * K + i] = x[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < K; ++i) x[i] = (sh[i] + sh[K + i]) + (sh[2 * K + i] + sh[3 * K + i]);
}

}  // namespace

// One workgroup per row of z (row stride ldz): both passes, the target capture and the record.
template <typename ZT, typename A>
__global__ __launch_bounds__(256) void oace_rows_fwd_kernel(const ZT* z, int64_t ldz, int64_t V,
                                                            const int64_t* targets, A eps, A gamma, A inv_v,
                                                            A* rows) {
  __shared__ A sh[24];
  const int64_t row = blockIdx.x;
  const ZT* zr = z + row * ldz;
  A ss[1] = {A(0)};
  for (int64_t v = threadIdx.x; v < V; v += 256) {
    const A x = ld_as<A>(zr, v);
    ss[0] += x * x;
  }
  block_sum<A, 1>(ss, sh);
  const A tau = o_rsq<A>(ss[0] * inv_v + eps);
  A s[4] = {A(0), A(0), A(0), A(0)};
  for (int64_t v = threadIdx.x; v < V; v += 256) {
    const A x = ld_as<A>(zr, v) * tau;
    const Oct<A> o = octic(x);
    const A rn = o.r * x;
    s[0] += o.k8;
    s[1] += o.rho7;
    s[2] += rn * o.k8;
    s[3] += rn * o.rho7;
  }
  block_sum<A, 4>(s, sh + 4);
  if (threadIdx.x == 0) {
    const int64_t t = targets[row];
    A rho_t = A(0), rn_t = A(0);  // a target outside [0, V) leaves rho_t = 0 (loss = inf), as the reference
    if (t >= 0 && t < V) {
      const A x = ld_as<A>(zr, t) * tau;
      const Oct<A> o = octic(x);
      rho_t = o.rho;
      rn_t = o.r * x;
    }
    oace_finalize_row<A>(rows + row * OACE_ROW, tau, s[0], s[1], s[2], s[3], rho_t, rn_t, inv_v, gamma);
  }
}

// loss = mean of the per-row losses, in a fixed order (one workgroup).
template <typename A>
__global__ __launch_bounds__(256) void oace_mean_kernel(const A* rows, int64_t N, A* loss) {
  __shared__ A sh[4];
  A s[1] = {A(0)};
  for (int64_t i = threadIdx.x; i < N; i += 256) s[0] += rows[i * OACE_ROW + OACE_LOSS];
  block_sum<A, 1>(s, sh);
  if (threadIdx.x == 0) *loss = s[0] / (A)N;
}

// dz = tau c (r bracket - radial x) for every element of rows (grid.y = row), c = c0 * g.
template <typename ZT, typename OT, typename A>
__global__ __launch_bounds__(256) void oace_rows_bwd_kernel(const ZT* z, int64_t ldz, int64_t V,
                                                            const int64_t* targets, const A* rows,
                                                            const A* g_loss, A c0, OT* dz, int64_t lddz) {
  const int64_t row = blockIdx.y;
  const A* rec = rows + row * OACE_ROW;
  const A tau = rec[OACE_TAU], inv_S = rec[OACE_INV_S], S8 = rec[OACE_S8];
  const A pc = rec[OACE_PC_INV8], radial = rec[OACE_RADIAL];
  const A diff = rec[OACE_SUM_P78] - pc;
  const A scale = S8 * inv_S;
  const A c = c0 * (g_loss ? *g_loss : A(1));
  const int64_t t = targets[row];
  const ZT* zr = z + row * ldz;
  OT* dr = dz + row * lddz;
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < V; v += (int64_t)gridDim.x * 256) {
    const A x = ld_as<A>(zr, v) * tau;
    const Oct<A> o = octic(x);
    const A bracket = scale * o.rho7 - (v == t ? pc : A(0)) - (o.k8 * inv_S) * diff;
    st_as<OT, A>(dr, v, tau * (c * (o.r * bracket - radial * x)));
  }
}

// C[m][n] (+)= sum_k A[m][k] B[k][n] with arbitrary element strides; 64x64 tiles, 4x4 per thread.
template <typename TA, typename TB, typename TC, typename A>
__global__ __launch_bounds__(256) void oace_gemm_generic_kernel(int64_t M, int64_t Nn, int64_t K, const TA* a,
                                                                int64_t sam, int64_t sak, const TB* b,
                                                                int64_t sbk, int64_t sbn, TC* c, int64_t scm,
                                                                int64_t scn, int accumulate) {
  __shared__ A as[16][65];
  __shared__ A bs[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  A acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = A(0);
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = threadIdx.x + 256 * i;  // 1024 = 16 x 64
      const int kk = e >> 6, mm = e & 63;
      const int64_t gm = m0 + mm, gn = n0 + mm, gk = k0 + kk;
      as[kk][mm] = (gm < M && gk < K) ? ld_as<A>(a, gm * sam + gk * sak) : A(0);
      bs[kk][mm] = (gn < Nn && gk < K) ? ld_as<A>(b, gk * sbk + gn * sbn) : A(0);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      A av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = as[kk][ty + 16 * i];
        bv[i] = bs[kk][tx + 16 * i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gm = m0 + ty + 16 * i, gn = n0 + tx + 16 * j;
      if (gm < M && gn < Nn) {
        const int64_t off = gm * scm + gn * scn;
        const A prev = accumulate ? ld_as<A>(c, off) : A(0);
        st_as<TC, A>(c, off, prev + acc[i][j]);
      }
    }
}

// y(k, v) = x[k V + v] for a dense rows x V accumulator, written with strides (sk, sv).
template <typename A, typename E>
__global__ __launch_bounds__(256) void oace_convert_kernel(const A* x, int64_t rows, int64_t V, E* y, int64_t sk,
                                                           int64_t sv) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < rows * V; i += (int64_t)gridDim.x * 256) {
    const int64_t k = i / V, v = i - k * V;
    st_as<E, A>(y, k * sk + v * sv, x[i]);
  }
}

// y (cols x rows, leading dimension ldy) = x^T for a rows x cols matrix x of 2-byte elements
// (leading dimension ldx, rows of any alignment), rows a multiple of 8 and y 16-byte aligned with
// ldy a multiple of 8.  A workgroup stages a 64-row x 128-column tile in LDS: each wave reads 16
// rows, one 2-byte element per lane and column (coalesced along the row); then every 8 lanes
// write 64 consecutive elements of one row of y (one 128-byte line), 16 bytes per lane.
constexpr int TR_ROWS = 64, TR_COLS = 128, TR_PITCH = TR_COLS + 2;
__global__ __launch_bounds__(256) void oace_transpose16_kernel(const unsigned short* x, int64_t rows, int64_t cols,
                                                               int64_t ldx, unsigned short* y, int64_t ldy) {
  __shared__ unsigned short t[TR_ROWS * TR_PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * TR_COLS, r0 = (int64_t)blockIdx.y * TR_ROWS;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t c = c0 + h * 64 + lane;
    unsigned short v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t r = r0 + wave * 16 + i;
      v[i] = c < cols && r < rows ? x[r * ldx + c] : (unsigned short)0;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t[(wave * 16 + i) * TR_PITCH + h * 64 + lane] = v[i];
  }
  __syncthreads();
  const int sg = tid & 7;  // 8-row segment of the tile
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int cl = (tid >> 3) + 32 * k;  // tile column = row of y
    const int64_t c = c0 + cl;
    if (c < cols && r0 + 8 * sg < rows) {
      u32x4_t w;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = (unsigned)t[(8 * sg + 2 * e) * TR_PITCH + cl] | ((unsigned)t[(8 * sg + 2 * e + 1) * TR_PITCH + cl] << 16);
      *(u32x4_t*)(y + c * ldy + r0 + 8 * sg) = w;
    }
  }
}

// ------------------------------------------------------------------------------ launchers
namespace {

template <int DT>
struct OTypes;
template <>
struct OTypes<AFA_F32> { typedef float E; typedef float A; };
template <>
struct OTypes<AFA_BF16> { typedef __bf16 E; typedef float A; };
template <>
struct OTypes<AFA_F16> { typedef _Float16 E; typedef float A; };
template <>
struct OTypes<AFA_F64> { typedef double E; typedef double A; };

template <typename TA, typename TB, typename TC, typename A>
void gemm_generic(int64_t M, int64_t N, int64_t K, const TA* a, int64_t sam, int64_t sak, const TB* b, int64_t sbk,
                  int64_t sbn, TC* c, int64_t scm, int64_t scn, bool accumulate, hipStream_t st) {
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  hipLaunchKernelGGL((oace_gemm_generic_kernel<TA, TB, TC, A>), grid, dim3(256), 0, st, M, N, K, a, sam, sak, b, sbk,
                     sbn, c, scm, scn, accumulate ? 1 : 0);
}

// W element (k, v) strides for a layout.
void w_strides(const OaceArgs& a, int64_t& sk, int64_t& sv) {
  if (a.w_layout == OACE_W_DV) {
    sk = a.ldw;
    sv = 1;
  } else {
    sk = 1;
    sv = a.ldw;
  }
}

template <int DT>
hipError_t rows_fwd_dt(const OaceArgs& a, const void* z, int64_t ldz, bool z_is_acc, void* rows, hipStream_t st) {
  typedef typename OTypes<DT>::E E;
  typedef typename OTypes<DT>::A A;
  const A inv_v = (A)(1.0 / (double)a.V);
  if (z_is_acc)
    hipLaunchKernelGGL((oace_rows_fwd_kernel<A, A>), dim3((unsigned)a.N), dim3(256), 0, st, (const A*)z, ldz, a.V,
                       a.targets, (A)a.eps, (A)a.gamma, inv_v, (A*)rows);
  else
    hipLaunchKernelGGL((oace_rows_fwd_kernel<E, A>), dim3((unsigned)a.N), dim3(256), 0, st, (const E*)z, ldz, a.V,
                       a.targets, (A)a.eps, (A)a.gamma, inv_v, (A*)rows);
  return hipGetLastError();
}

unsigned bwd_grid_x(int64_t V) { return (unsigned)std::min<int64_t>((V + 255) / 256, 64); }

}  // namespace

size_t oace_generic_chunk_rows(int dtype, int64_t N, int64_t V) {
  const size_t acc = dtype == AFA_F64 ? 8 : 4;
  const size_t cap = (size_t)256 << 20;
  int64_t r = (int64_t)(cap / ((size_t)V * acc));
  return (size_t)std::max<int64_t>(1, std::min<int64_t>(N, r));
}

size_t oace_generic_workspace(int dtype, int64_t N, int64_t d, int64_t V, bool backward) {
  const size_t acc = dtype == AFA_F64 ? 8 : 4;
  const int64_t R = (int64_t)oace_generic_chunk_rows(dtype, N, V);
  size_t b = (size_t)R * V * acc;  // z / dz chunk
  b = (b + 255) & ~(size_t)255;
  if (backward && R < N) b += (size_t)d * V * acc;  // dW accumulator
  return b;
}

template <int DT>
static hipError_t linear_fwd_generic_dt(const OaceArgs& a, void* rows, void* ws, hipStream_t st) {
  typedef typename OTypes<DT>::E E;
  typedef typename OTypes<DT>::A A;
  const int64_t R = (int64_t)oace_generic_chunk_rows(DT, a.N, a.V);
  A* z = (A*)ws;
  int64_t sk, sv;
  w_strides(a, sk, sv);
  for (int64_t r0 = 0; r0 < a.N; r0 += R) {
    const int64_t rn = std::min(R, a.N - r0);
    gemm_generic<E, E, A, A>(rn, a.V, a.d, (const E*)a.h + r0 * a.ldh, a.ldh, 1, (const E*)a.w, sk, sv, z, a.V, 1,
                             false, st);
    OaceArgs sub = a;
    sub.N = rn;
    sub.targets = a.targets + r0;
    hipError_t e = rows_fwd_dt<DT>(sub, z, a.V, true, (A*)rows + r0 * OACE_ROW, st);
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

template <int DT>
static hipError_t linear_bwd_generic_dt(const OaceArgs& a, const void* rows, void* ws, hipStream_t st) {
  typedef typename OTypes<DT>::E E;
  typedef typename OTypes<DT>::A A;
  const int64_t R = (int64_t)oace_generic_chunk_rows(DT, a.N, a.V);
  A* z = (A*)ws;
  const bool chunked = R < a.N;
  A* dwacc = chunked ? (A*)((char*)ws + (((size_t)R * a.V * sizeof(A) + 255) & ~(size_t)255)) : nullptr;
  int64_t sk, sv;
  w_strides(a, sk, sv);
  const A c0 = (A)(8.0 * a.gamma / (double)a.N);
  for (int64_t r0 = 0; r0 < a.N; r0 += R) {
    const int64_t rn = std::min(R, a.N - r0);
    const E* hc = (const E*)a.h + r0 * a.ldh;
    gemm_generic<E, E, A, A>(rn, a.V, a.d, hc, a.ldh, 1, (const E*)a.w, sk, sv, z, a.V, 1, false, st);
    hipLaunchKernelGGL((oace_rows_bwd_kernel<A, A, A>), dim3(bwd_grid_x(a.V), (unsigned)rn), dim3(256), 0, st,
                       (const A*)z, a.V, a.V, a.targets + r0, (const A*)rows + r0 * OACE_ROW, (const A*)a.g_loss, c0,
                       z, a.V);
    // dh (rn x d) = dz (rn x V) W^T: element (n, k) = sum_v dz[n][v] W(k, v)
    gemm_generic<A, E, E, A>(rn, a.d, a.V, z, a.V, 1, (const E*)a.w, sv, sk, (E*)a.dh + r0 * a.d, a.d, 1, false, st);
    // dW(k, v) = sum_n h[n][k] dz[n][v], stored in W's layout
    if (chunked)
      gemm_generic<E, A, A, A>(a.d, a.V, rn, hc, 1, a.ldh, z, a.V, 1, dwacc, a.V, 1, r0 > 0, st);
    else
      gemm_generic<E, A, E, A>(a.d, a.V, rn, hc, 1, a.ldh, z, a.V, 1, (E*)a.dw, sk, sv, false, st);
  }
  if (chunked)  // dW from the accumulator, in the element type and W's layout
    hipLaunchKernelGGL((oace_convert_kernel<A, E>), dim3((unsigned)std::min<int64_t>((a.d * a.V + 255) / 256, 65536)),
                       dim3(256), 0, st, (const A*)dwacc, a.d, a.V, (E*)a.dw, sk, sv);
  return hipGetLastError();
}

hipError_t oace_linear_fwd_generic(int dtype, const OaceArgs& a, void* rows, void* ws, hipStream_t st) {
  hipError_t e;
  switch (dtype) {
    case AFA_F32: e = linear_fwd_generic_dt<AFA_F32>(a, rows, ws, st); break;
    case AFA_BF16: e = linear_fwd_generic_dt<AFA_BF16>(a, rows, ws, st); break;
    case AFA_F16: e = linear_fwd_generic_dt<AFA_F16>(a, rows, ws, st); break;
    default: e = linear_fwd_generic_dt<AFA_F64>(a, rows, ws, st); break;
  }
  if (e != hipSuccess) return e;
  return oace_mean_launch(dtype, rows, a.N, a.loss, st);
}

hipError_t oace_linear_bwd_generic(int dtype, const OaceArgs& a, const void* rows, void* ws, hipStream_t st) {
  switch (dtype) {
    case AFA_F32: return linear_bwd_generic_dt<AFA_F32>(a, rows, ws, st);
    case AFA_BF16: return linear_bwd_generic_dt<AFA_BF16>(a, rows, ws, st);
    case AFA_F16: return linear_bwd_generic_dt<AFA_F16>(a, rows, ws, st);
    default: return linear_bwd_generic_dt<AFA_F64>(a, rows, ws, st);
  }
}

hipError_t oace_mean_launch(int dtype, const void* rows, int64_t N, void* loss, hipStream_t st) {
  if (dtype == AFA_F64)
    hipLaunchKernelGGL((oace_mean_kernel<double>), dim3(1), dim3(256), 0, st, (const double*)rows, N, (double*)loss);
  else
    hipLaunchKernelGGL((oace_mean_kernel<float>), dim3(1), dim3(256), 0, st, (const float*)rows, N, (float*)loss);
  return hipGetLastError();
}

hipError_t oace_softmax_fwd_launch(int dtype, const OaceArgs& a, void* rows, hipStream_t st) {
  hipError_t e;
  switch (dtype) {
    case AFA_F32: e = rows_fwd_dt<AFA_F32>(a, a.h, a.ldh, false, rows, st); break;
    case AFA_BF16: e = rows_fwd_dt<AFA_BF16>(a, a.h, a.ldh, false, rows, st); break;
    case AFA_F16: e = rows_fwd_dt<AFA_F16>(a, a.h, a.ldh, false, rows, st); break;
    default: e = rows_fwd_dt<AFA_F64>(a, a.h, a.ldh, false, rows, st); break;
  }
  if (e != hipSuccess) return e;
  return oace_mean_launch(dtype, rows, a.N, a.loss, st);
}

template <int DT>
static hipError_t softmax_bwd_dt(const OaceArgs& a, const void* rows, void* dz, hipStream_t st) {
  typedef typename OTypes<DT>::E E;
  typedef typename OTypes<DT>::A A;
  const A c0 = (A)(8.0 * a.gamma / (double)a.N);
  hipLaunchKernelGGL((oace_rows_bwd_kernel<E, E, A>), dim3(bwd_grid_x(a.V), (unsigned)a.N), dim3(256), 0, st,
                     (const E*)a.h, a.ldh, a.V, a.targets, (const A*)rows, (const A*)a.g_loss, c0, (E*)dz, a.ldh);
  return hipGetLastError();
}

hipError_t oace_softmax_bwd_launch(int dtype, const OaceArgs& a, const void* rows, void* dz, hipStream_t st) {
  switch (dtype) {
    case AFA_F32: return softmax_bwd_dt<AFA_F32>(a, rows, dz, st);
    case AFA_BF16: return softmax_bwd_dt<AFA_BF16>(a, rows, dz, st);
    case AFA_F16: return softmax_bwd_dt<AFA_F16>(a, rows, dz, st);
    default: return softmax_bwd_dt<AFA_F64>(a, rows, dz, st);
  }
}

hipError_t oace_transpose16(const void* x, int64_t rows, int64_t cols, int64_t ldx, void* y, int64_t ldy,
                            hipStream_t st) {
  if (rows % 8 != 0 || ldy % 8 != 0 || ((uintptr_t)y & 15u) != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((cols + TR_COLS - 1) / TR_COLS), (unsigned)((rows + TR_ROWS - 1) / TR_ROWS));
  hipLaunchKernelGGL(oace_transpose16_kernel, grid, dim3(256), 0, st, (const unsigned short*)x, rows, cols, ldx,
                     (unsigned short*)y, ldy);
  return hipGetLastError();
}

}  // namespace afa
