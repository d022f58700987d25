// Row-norm pre-pass of the fast-rho guard (fast_rho_safe in afa_common.h).
//
// For every (b, h) and every block of 64 rows, the largest squared norm of the block's rows,
// sum_d x_ld^2 in fp32 from the bf16 / fp16 elements as stored.  The MFMA kernels bound every
// score of a key tile by Cauchy-Schwarz with it (|q . k| <= |q| |k|) and use the branch-free
// rho^8 only where that bound keeps |s| <= kFastRhoMaxScore.  It reads the tensor once and writes
// B H ceil(L/64) floats; with rotary tables the K rotation pass (afa_krot_kernel) produces the
// same bounds from the rotated rows instead, for the forward's k and the backward's q and k.
#include <cmath>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

// Each wave handles one (b, h, 64-row block) work item (RowBlockLayout): CHP loads per lane
// issued back to back, then the row sums by shuffles and the wave maximum.  No LDS, no barrier.
template <int DT, int D>
__global__ __launch_bounds__(256) void afa_rownorm_kernel(const unsigned short* x, int64_t sb, int64_t sh,
                                                         int64_t sl, int H, int L, int nblk, int nwork,
                                                         float* nb2, int* zero, int nzero) {
  using RL = RowBlockLayout<D>;
  for (int i = blockIdx.x * 256 + (int)threadIdx.x; i < nzero; i += gridDim.x * 256) zero[i] = 0;
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (int)(threadIdx.x >> 6);  // wave-uniform work item
  if (w >= nwork) return;
  const int bh = w / nblk, blk = w - bh * nblk;
  const int b = bh / H, h = bh - b * H;
  const unsigned short* xb = x + b * sb + h * sh;
  const int c = lane % RL::CHP, rsub = lane / RL::CHP;
  u32x4_t v[RL::CHP];
#pragma unroll
  for (int it = 0; it < RL::CHP; ++it) {
    const int row = blk * 64 + it * RL::RPI + rsub;
    v[it] = u32x4_t{0u, 0u, 0u, 0u};
    if (c < RL::CH && row < L) v[it] = *(const u32x4_t*)(xb + (int64_t)row * sl + c * 8);
  }
  float m = 0.0f;
#pragma unroll
  for (int it = 0; it < RL::CHP; ++it) m = __builtin_fmaxf(m, group_sum<RL::CHP>(chunk_norm2<DT>(v[it])));
  m = wave_max(m);
  if (lane == 0) nb2[(int64_t)bh * nblk + blk] = m;
}

template <int DT, int D>
static void rownorm_launch_d(const void* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, float* nb2,
                             hipStream_t stream, int* zero, int nzero) {
  const int nblk = (L + 63) / 64;
  const int nwork = B * H * nblk;
  hipLaunchKernelGGL((afa_rownorm_kernel<DT, D>), dim3((unsigned)((nwork + 3) / 4)), dim3(256), 0, stream,
                     (const unsigned short*)x, sb, sh, sl, H, L, nblk, nwork, nb2, zero, nzero);
}

template <int DT>
static hipError_t rownorm_launch_dt(const void* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                                    int head_dim, float* nb2, hipStream_t stream, int* zero, int nzero) {
  switch (head_dim) {
    case 32: rownorm_launch_d<DT, 32>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    case 48: rownorm_launch_d<DT, 48>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    case 64: rownorm_launch_d<DT, 64>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    case 96: rownorm_launch_d<DT, 96>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    case 128: rownorm_launch_d<DT, 128>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    case 256: rownorm_launch_d<DT, 256>(x, sb, sh, sl, B, H, L, nb2, stream, zero, nzero); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

float fast_rho_lim(double score_per_output) {
  const double s = (double)kFastRhoMaxScore / score_per_output;
  return (float)(s * s / 1.05);
}

hipError_t rownorm_launch(int dtype, const void* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                          int head_dim, float* nb2, hipStream_t stream, int* zero, int nzero) {
  if (x == nullptr || nb2 == nullptr) return hipErrorInvalidValue;
  if (dtype == AFA_BF16) return rownorm_launch_dt<AFA_BF16>(x, sb, sh, sl, B, H, L, head_dim, nb2, stream, zero, nzero);
  if (dtype == AFA_F16) return rownorm_launch_dt<AFA_F16>(x, sb, sh, sl, B, H, L, head_dim, nb2, stream, zero, nzero);
  return hipErrorInvalidValue;
}

}  // namespace afa
