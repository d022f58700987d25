// Row-norm pre-pass of the fast-rho guard (FastGuard in afa_common.h).
//
// For every (b, h) and every block of 64 rows, the largest squared norm of the block's rows,
// sum_d x_ld^2 in fp32 from the bf16 / fp16 elements as stored.  The MFMA kernels bound every
// score of a key tile by Cauchy-Schwarz with it (|q . k| <= |q| |k|) and use the branch-free
// rho^8 only where that bound keeps |s| <= kFastRhoMaxScore.  It reads the tensor once and writes
// B H ceil(L/64) floats; with rotary tables the rotation pre-passes produce the same bounds from
// the rotated rows instead (afa_krot_kernel, afa_bwd_mfma_rotate_kernel).
#include <cmath>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

// Grid (ceil(L / 64), B * H), 256 threads; thread slot e = tid + 256 i covers row e / (D/8) of the
// block and its 16-byte chunk e % (D/8).  Partial sums meet in LDS (the order of the fp32 adds
// does not matter to a bound that carries a margin).
template <int DT>
__global__ __launch_bounds__(256) void afa_rownorm_kernel(const unsigned short* x, int64_t sb, int64_t sh,
                                                         int64_t sl, int H, int L, int D, float* nb2) {
  __shared__ float rn[64];
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int ch = D / 8;
  const unsigned short* xb = x + b * sb + h * sh;
  if (threadIdx.x < 64) rn[threadIdx.x] = 0.0f;
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * ch; e += 256) {
    const int r = e / ch, c = e - r * ch;
    const int l = blockIdx.x * 64 + r;
    if (l < L) atomicAdd(&rn[r], chunk_norm2<DT>(*(const u32x4_t*)(xb + (int64_t)l * sl + c * 8)));
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const float m = wave_max(rn[threadIdx.x]);
    if (threadIdx.x == 0) nb2[(int64_t)bh * gridDim.x + blockIdx.x] = m;
  }
}

float fast_rho_lim(double score_per_output) {
  const double s = (double)kFastRhoMaxScore / score_per_output;
  return (float)(s * s / 1.05);
}

hipError_t rownorm_launch(int dtype, const void* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                          int head_dim, float* nb2, hipStream_t stream) {
  if (x == nullptr || nb2 == nullptr || head_dim % 8 != 0 || head_dim > 256) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((L + 63) / 64), (unsigned)(B * H));
  if (dtype == AFA_BF16)
    hipLaunchKernelGGL((afa_rownorm_kernel<AFA_BF16>), grid, dim3(256), 0, stream, (const unsigned short*)x, sb, sh,
                       sl, H, L, head_dim, nb2);
  else if (dtype == AFA_F16)
    hipLaunchKernelGGL((afa_rownorm_kernel<AFA_F16>), grid, dim3(256), 0, stream, (const unsigned short*)x, sb, sh,
                       sl, H, L, head_dim, nb2);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace afa
