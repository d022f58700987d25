// MFMA path of the fused Linear + OACE head for bf16 / fp16 (src/kernels/pallas_oace.py:59-269).
//
// The vocabulary projection is never materialised in the forward.  Two GEMM sweeps over the
// logits z = h W, each with a fused epilogue, produce per-(vocabulary tile, row) partial sums:
//   MODE_SQ:    sum_v z^2                                  -> tau = rsqrt(mean z^2 + eps)
//   MODE_OCTIC: sum k8, sum rho7, sum (r x) k8, sum (r x) rho7 of x = tau z
// which small kernels reduce in a fixed order into the row records; the MODE_SQ epilogue also keeps
// each row's target logit z[n][t_n], from which the row kernel forms rho and r x.  The reference takes the
// second moment from the Gram matrix W W^T; the sum of squared logits is the same quantity and
// a second sweep costs less than the Gram product whenever rows < d_model, the case of the
// reference's own benchmark (512 x 768).  When the fp32 logits fit the cache bound below, the
// first sweep also stores them (MODE_SQZ) and one workgroup per row then forms tau, the octic
// sums, the target's terms and the record from them in one pass (oace_mfma_row_cached_kernel),
// in place of the second sweep.  The backward recomputes z once:
//   MODE_DZ:    dz = tau c (r bracket - radial x), stored as the element type (rows, V padded)
// and forms dh = dz W^T and dW = h^T dz with the MFMA GEMMs of oace_bwd_gemm.hip.
//
// GEMM tile: z^T = W^T h^T over a 256 (vocabulary) x 128 (rows) tile per workgroup, four waves of
// 64 x 128, each a 2 x 4 grid of 32x32x16 MFMA blocks whose accumulator lanes hold one row and 16
// vocabulary entries, so the row reductions are in-lane.  K (d_model) advances 32 per step
// through a 3-stage LDS ring filled by direct global -> LDS loads (64-byte rows, 16-byte chunks
// swizzled by (row >> 2) & 3: 16 consecutive rows in 16 distinct bank groups), one barrier per
// step.  Tiles of one vocabulary block are dispatched consecutively on one XCD (they share its W tile in L2).
// W is used as W^T (vocab, d_model) with d_model contiguous: a tied embedding already is; the
// (d_model, vocab) output head is transposed once per call into the workspace.
#include <algorithm>
#include <type_traits>

#include "oace_common.h"

namespace afa {

namespace {

constexpr int TV = 256;  // vocabulary entries per workgroup tile
constexpr int TN = 128;  // rows per workgroup tile
constexpr int KS = 32;   // d_model per pipeline step
constexpr int NSTAGE = 3;
constexpr int A_BYTES = TV * KS * 2;
constexpr int B_BYTES = TN * KS * 2;
constexpr int STAGE = A_BYTES + B_BYTES;
constexpr int A_LOADS = A_BYTES / (256 * 16);  // 16-byte direct loads per thread and step
constexpr int B_LOADS = B_BYTES / (256 * 16);
constexpr int LOADS = A_LOADS + B_LOADS;
constexpr int MODE_SQ = 0, MODE_OCTIC = 1, MODE_DZ = 2, MODE_SQZ = 3;

struct GemmArgs {
  const unsigned short* wt;  // (V, d), row stride ldwt
  int64_t ldwt;
  const unsigned short* h;  // (N, d), row stride ldh
  int64_t ldh;
  int N, V, d, nvt, nnt;
  const float* rows;
  const int64_t* targets;
  float* part;  // MODE_SQ: [nvt][N]; MODE_OCTIC: [nvt][N][4]
  unsigned short* dz;  // MODE_DZ: (N, ldz)
  int64_t ldz;
  float* zc;  // MODE_SQZ: the fp32 logits, (N, ldz)
  float* zt;  // MODE_SQ: the target logit of row n at zt[n * OACE_ROW] (the row record's unused last
              // field until the row kernel finalises the record; not written for targets outside [0, V))
  float c0;
  const float* g_loss;
};

template <int DT>
__device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == AFA_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

__host__ __device__ constexpr int vm_only(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Byte offset of logical 16-byte chunk lc of row r in a tile of 64-byte rows.
__device__ __forceinline__ int chunk_off(int r, int lc) { return r * 64 + ((lc ^ ((r >> 2) & 3)) << 4); }

}  // namespace

template <int DT, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void oace_mfma_gemm_kernel(const GemmArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[NSTAGE * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;

  // tiles of one vocabulary block run consecutively on one XCD (block b runs on XCD b mod 8)
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int nt = j % a.nnt, vt = (j / a.nnt) * 8 + xcd;
  if (vt >= a.nvt) return;
  const int v0 = vt * TV, n0 = nt * TN;

  // direct-load sources: thread slot s = 256 i + tid covers row s >> 2, physical chunk s & 3
  const unsigned short* asrc[A_LOADS];
  const unsigned short* bsrc[B_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int s = 256 * i + tid, r = s >> 2, lc = (s & 3) ^ ((r >> 2) & 3);
    asrc[i] = a.wt + (int64_t)min(v0 + r, a.V - 1) * a.ldwt + lc * 8;
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int s = 256 * i + tid, r = s >> 2, lc = (s & 3) ^ ((r >> 2) & 3);
    bsrc[i] = a.h + (int64_t)min(n0 + r, a.N - 1) * a.ldh + lc * 8;
  }
  auto issue = [&](int t) {
    unsigned char* st = lds + (t % NSTAGE) * STAGE;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(asrc[i] + t * KS), (void*)(st + (256 * i + wave * 64) * 16), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(bsrc[i] + t * KS), (void*)(st + A_BYTES + (256 * i + wave * 64) * 16),
                                       16, 0, 0);
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[vb][nb][e] = 0.f;

  // MODE_SQ keeps each row's target logit: the lane that will hold (row n, target) finds its
  // element offset now, so the target loads complete under the main loop
  int toff[4];
  if constexpr (MODE == MODE_SQ) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int n = n0 + nb * 32 + l32;
      const int64_t off = (n < a.N ? a.targets[n] : (int64_t)-1) - (v0 + wave * 64 + 4 * g);
      toff[nb] = off >= 0 && off < 64 && (off & 4) == 0 ? (int)off : -1;
    }
  }

  const int T = a.d / KS;
  issue(0);
  if (T > 1) issue(1);
  if (T > 1) __builtin_amdgcn_s_waitcnt(vm_only(LOADS));
  else __builtin_amdgcn_s_waitcnt(vm_only(0));
  __syncthreads();

  for (int t = 0; t < T; ++t) {
    // the buffer of step t+2 was last read in step t-1, before the previous barrier
    if (t + 2 < T) issue(t + 2);
    const unsigned char* st = lds + (t % NSTAGE) * STAGE;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4_t af[2], bf[4];
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) af[vb] = *(const u32x4_t*)(st + chunk_off(wave * 64 + vb * 32 + l32, 2 * kk + g));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) bf[nb] = *(const u32x4_t*)(st + A_BYTES + chunk_off(nb * 32 + l32, 2 * kk + g));
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[vb][nb] = mma<DT>(af[vb], bf[nb], acc[vb][nb]);
    }
    // own loads of step t+1 complete (only those of step t+2 may remain), then publish them
    if (t + 2 < T) __builtin_amdgcn_s_waitcnt(vm_only(LOADS));
    else __builtin_amdgcn_s_waitcnt(vm_only(0));
    __syncthreads();
  }

  // ---- epilogue.  Element e of acc[vb][nb]: vocabulary v = vw + 32 vb + 8 (e >> 2) + 4 g + (e & 3)
  // (vw = v0 + 64 wave), row n = n0 + 32 nb + l32.
  const int vw = v0 + wave * 64;
  const bool vtail = v0 + TV > a.V;
  float* red = (float*)lds;  // the ring is idle after the last barrier
  if constexpr (MODE == MODE_SQZ) {
    // the logits themselves, 32 rows at a time through LDS (the idle ring): each wave writes its
    // 64 vocabulary columns of the 32 rows, then every wave stores whole 1 KB row segments
    // (a 4-entry group that starts below V ends below the padded row length; its entries past V
    // are finite and never read)
    constexpr int ZP = TV + 4;  // staged row pitch in floats (16-byte aligned rows)
    static_assert(32 * ZP * 4 <= NSTAGE * STAGE, "the staged rows must fit the ring");
    float* zt = (float*)lds;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          f32x4_t w;
#pragma unroll
          for (int u = 0; u < 4; ++u) w[u] = acc[vb][nb][4 * e4 + u];
          *(f32x4_t*)(zt + l32 * ZP + wave * 64 + 32 * vb + 8 * e4 + 4 * g) = w;
        }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 32 * TV / 4 / 256; ++i) {
        const int idx = tid + 256 * i, row = idx / (TV / 4), c4 = idx % (TV / 4);
        const int n = n0 + nb * 32 + row, vs = v0 + 4 * c4;
        if (n < a.N && vs < a.V) *(f32x4_t*)(a.zc + (int64_t)n * a.ldz + vs) = *(const f32x4_t*)(zt + row * ZP + 4 * c4);
      }
      __syncthreads();
    }
  }
  if constexpr (MODE == MODE_SQ || MODE == MODE_SQZ) {
    float s[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      s[nb] = 0.f;
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float z = acc[vb][nb][e];
          const int v = vw + 32 * vb + 8 * (e >> 2) + 4 * g + (e & 3);
          s[nb] += (!vtail || v < a.V) ? z * z : 0.f;
        }
      if constexpr (MODE == MODE_SQ) {
        // the target logit, for the row kernel (offset 32 vb + 8 (e >> 2) + (e & 3) in this lane)
        if (toff[nb] >= 0) {
          const int o = toff[nb], ovb = o >> 5, oe = ((o & 31) >> 3) * 4 + (o & 3);
          float zt = 0.f;
#pragma unroll
          for (int vb = 0; vb < 2; ++vb)
#pragma unroll
            for (int e = 0; e < 16; ++e) zt = (vb == ovb && e == oe) ? acc[vb][nb][e] : zt;
          a.zt[(int64_t)(n0 + nb * 32 + l32) * OACE_ROW] = zt;
        }
      }
      s[nb] += __shfl_xor(s[nb], 32);
      if (g == 0) red[wave * TN + nb * 32 + l32] = s[nb];
    }
    __syncthreads();
    if (tid < TN && n0 + tid < a.N)
      a.part[(int64_t)vt * a.N + n0 + tid] = (red[tid] + red[TN + tid]) + (red[2 * TN + tid] + red[3 * TN + tid]);
  } else if constexpr (MODE == MODE_OCTIC) {
    float tau[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int n = n0 + nb * 32 + l32;
      tau[nb] = n < a.N ? a.rows[(int64_t)n * OACE_ROW + OACE_TAU] : 0.f;
    }
    // Entries past the vocabulary (last tile only) are set to z = 0, whose octic terms are exact:
    // rho = 1, so each adds 1 to sum k8 and sum rho7 and 0 to the r x sums; those counts are
    // subtracted below.  One code path for every tile keeps the epilogue within the registers.
    float nmask = 0.f;
    if (vtail) {
      const int vlim = a.V - vw - 4 * g;  // valid offsets 32 vb + 8 (e >> 2) + (e & 3) < vlim
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const bool out = 32 * vb + 8 * (e >> 2) + (e & 3) >= vlim;
          nmask += out ? 1.f : 0.f;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) acc[vb][nb][e] = out ? 0.f : acc[vb][nb][e];
        }
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float s[4] = {-nmask, -nmask, 0.f, 0.f};
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float x = acc[vb][nb][e] * tau[nb];
          const Oct<float> o = octic_fast(x);
          const float rn = o.r * x;
          s[0] += o.k8;
          s[1] += o.rho7;
          s[2] += rn * o.k8;
          s[3] += rn * o.rho7;
          // bound the octic chains in flight (each holds x and r): 8 at a time fit the registers
          if ((e & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x = s[q] + __shfl_xor(s[q], 32);
        if (g == 0) red[(wave * 4 + q) * TN + nb * 32 + l32] = x;
      }
    }
    __syncthreads();
    for (int i = tid; i < TN * 4; i += 256) {
      const int q = i / TN, nl = i % TN;
      if (n0 + nl < a.N)
        a.part[((int64_t)vt * a.N + n0 + nl) * 4 + q] =
            (red[q * TN + nl] + red[(4 + q) * TN + nl]) + (red[(8 + q) * TN + nl] + red[(12 + q) * TN + nl]);
    }
  } else {  // MODE_DZ
    const float gl = a.g_loss ? *a.g_loss : 1.f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int n = n0 + nb * 32 + l32;
      if (n >= a.N) continue;
      const float* rec = a.rows + (int64_t)n * OACE_ROW;
      const float tau = rec[OACE_TAU], inv_S = rec[OACE_INV_S], pc = rec[OACE_PC_INV8], radial = rec[OACE_RADIAL];
      const float scale = rec[OACE_S8] * inv_S;
      const float diff = rec[OACE_SUM_P78] - pc;
      const float tc = tau * (a.c0 * gl);
      const int64_t t = a.targets[n];
      unsigned short* drow = a.dz + (int64_t)n * a.ldz;
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int vs = vw + 32 * vb + 8 * e4 + 4 * g;
          float dzv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float x = acc[vb][nb][4 * e4 + u] * tau;
            const Oct<float> o = octic_fast(x);  // error far below the rounding of dz to the element type
            const float bracket = scale * o.rho7 - (vs + u == t ? pc : 0.f) - (o.k8 * inv_S) * diff;
            dzv[u] = tc * (o.r * bracket - radial * x);
          }
          if (vs < a.V) {
            u32x2_t w;
            w[0] = Elem<DT>::pack(dzv[0], dzv[1]);
            w[1] = Elem<DT>::pack(dzv[2], dzv[3]);
            *(u32x2_t*)(drow + vs) = w;
          }
        }
    }
  }
}

// tau per row from the MODE_SQ partials, summed over vocabulary tiles in order.
__global__ __launch_bounds__(256) void oace_mfma_tau_kernel(const float* part, int nvt, int N, float inv_v, float eps,
                                                            float* rows) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);  // one wave per row
  if (n >= N) return;
  float ss = 0.f;
  for (int t = lane; t < nvt; t += 64) ss += part[(int64_t)t * N + n];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  if (lane == 0) rows[(int64_t)n * OACE_ROW + OACE_TAU] = o_rsq<float>(ss * inv_v + eps);
}

// One row from the kept logits, in one workgroup: tau from the row's MODE_SQ partials (summed in
// the order of oace_mfma_tau_kernel), the four octic sums over the row (16-byte loads, RC_UNROLL
// of them in flight per lane while the previous group is evaluated), the target's rho and r x
// from its own logit (the value the sums use), and the row record.  A target outside [0, V)
// leaves rho_t = 0 (infinite loss), as the reference.
constexpr int RC_THREADS = 512, RC_UNROLL = 4, RC_SPAN = 4 * RC_THREADS * RC_UNROLL;
__global__ __launch_bounds__(RC_THREADS) void oace_mfma_row_cached_kernel(const float* part, int nvt, const float* zc,
                                                                          int64_t ldz, int N, int V, float inv_v,
                                                                          float eps, float gamma,
                                                                          const int64_t* targets, float* rows) {
  constexpr int NW = RC_THREADS / 64;
  __shared__ float sh[NW * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = blockIdx.x;
  const float* zrow = zc + (int64_t)n * ldz;
  // Groups of RC_SPAN logits alternate between two register sets: the loads of the next group go
  // out before the current one is evaluated.  Loads are unconditional (a lane past the padded row
  // length reads the row's first entries, which are not used), so nothing waits on them early.
  const int ld = (int)ldz;
  auto load = [&](f32x4_t (&z)[RC_UNROLL], int v0) {
#pragma unroll
    for (int u = 0; u < RC_UNROLL; ++u) {
      const int vs = v0 + 4 * (tid + RC_THREADS * u);
      z[u] = *(const f32x4_t*)(zrow + (vs < ld ? vs : 0));
    }
  };
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  float tau;
  auto eval = [&](const f32x4_t (&z)[RC_UNROLL], int v0) {
#pragma unroll
    for (int u = 0; u < RC_UNROLL; ++u) {
      const int vs = v0 + 4 * (tid + RC_THREADS * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (vs + e < V) {
          const float x = z[u][e] * tau;
          const Oct<float> o = octic_fast(x);
          const float rn = o.r * x;
          s[0] += o.k8;
          s[1] += o.rho7;
          s[2] += rn * o.k8;
          s[3] += rn * o.rho7;
        }
      }
    }
  };
  // Every wave sums the row's MODE_SQ partials itself, in the order of oace_mfma_tau_kernel (lane
  // l adds partials l, l + 64, ...), so no barrier stands before the stream; the first chunk of
  // partials is loaded before the first group of logits, whose loads stay in flight while it is
  // added.
  float ss = 0.f;
  f32x4_t za[RC_UNROLL], zb[RC_UNROLL];
  {
    float p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = lane + 64 * u;
      p[u] = part[(int64_t)(t < nvt ? t : 0) * N + n];
    }
    load(za, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) ss += lane + 64 * u < nvt ? p[u] : 0.f;
  }
  for (int t0 = 256; t0 < nvt; t0 += 256) {
    float p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + lane + 64 * u;
      p[u] = t < nvt ? part[(int64_t)t * N + n] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) ss += p[u];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  tau = o_rsq<float>(ss * inv_v + eps);
  for (int v0 = 0; v0 < V; v0 += 2 * RC_SPAN) {
    load(zb, v0 + RC_SPAN);
    eval(za, v0);
    load(za, v0 + 2 * RC_SPAN);
    eval(zb, v0 + RC_SPAN);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s[q] += __shfl_xor(s[q], m);
    if (lane == 0) sh[wave * 4 + q] = s[q];
  }
  __syncthreads();
  if (tid == 0) {
    float t4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float x = 0.f;
      for (int w = 0; w < NW; ++w) x += sh[w * 4 + q];
      t4[q] = x;
    }
    const int64_t t = targets[n];
    float rho_t = 0.f, rn_t = 0.f;
    if (t >= 0 && t < V) {
      const float x = zrow[t] * tau;
      const Oct<float> o = octic(x);
      rho_t = o.rho;
      rn_t = o.r * x;
    }
    oace_finalize_row<float>(rows + (int64_t)n * OACE_ROW, tau, t4[0], t4[1], t4[2], t4[3], rho_t, rn_t, inv_v,
                             gamma);
  }
}

// dz from the cached logits: the MODE_DZ epilogue's arithmetic on the same fp32 logits; entries
// in [V, ldz) are written as zeros.  One wave per 1024 consecutive entries of a row, each lane
// with four groups of 4 entries (all four loads in flight before the arithmetic; every load
// and store instruction covers a contiguous 1 KB / 512 B of the row).
constexpr int DZ_SPAN = 1024;
template <int DT>
__global__ __launch_bounds__(256) void oace_mfma_dz_cached_kernel(const float* zc, int64_t ldz, int N, int V,
                                                                  const float* rows, const int64_t* targets, float c0,
                                                                  const float* g_loss, unsigned short* dz) {
  const int lane = threadIdx.x & 63;
  const int spans = (int)((ldz + DZ_SPAN - 1) / DZ_SPAN);
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)N * spans) return;
  const int n = (int)(w / spans);
  const int v0 = (int)(w % spans) * DZ_SPAN + 4 * lane;
  const float gl = g_loss ? *g_loss : 1.f;
  const float* rec = rows + (int64_t)n * OACE_ROW;
  const float tau = rec[OACE_TAU], inv_S = rec[OACE_INV_S], pc = rec[OACE_PC_INV8], radial = rec[OACE_RADIAL];
  const float scale = rec[OACE_S8] * inv_S;
  const float diff = rec[OACE_SUM_P78] - pc;
  const float tc = tau * (c0 * gl);
  const int64_t t = targets[n];
  const float* zrow = zc + (int64_t)n * ldz;
  unsigned short* drow = dz + (int64_t)n * ldz;
  f32x4_t z4[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int vs = v0 + 256 * u;
    if (vs < V) z4[u] = *(const f32x4_t*)(zrow + vs);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int vs = v0 + 256 * u;
    if (vs >= ldz) continue;
    float dzv[4] = {0.f, 0.f, 0.f, 0.f};
    if (vs < V) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = z4[u][e] * tau;
        const Oct<float> o = octic_fast(x);
        const float bracket = scale * o.rho7 - (vs + e == t ? pc : 0.f) - (o.k8 * inv_S) * diff;
        dzv[e] = vs + e < V ? tc * (o.r * bracket - radial * x) : 0.f;
      }
    }
    u32x2_t wv;
    wv[0] = Elem<DT>::pack(dzv[0], dzv[1]);
    wv[1] = Elem<DT>::pack(dzv[2], dzv[3]);
    *(u32x2_t*)(drow + vs) = wv;
  }
}

// Row records from the MODE_OCTIC partials, one wave per row.  The target logit is the one the
// MODE_SQ sweep kept in the record's last field (the GEMM's own value, as the sums use); a target
// outside [0, V) leaves rho_t = 0 (infinite loss), as the reference.
__global__ __launch_bounds__(256) void oace_mfma_rows_kernel(const float* part, int nvt, int N, float inv_v,
                                                             float gamma, int V, const int64_t* targets, float* rows) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int64_t t = targets[n];
  const bool valid = t >= 0 && t < V;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int vt = lane; vt < nvt; vt += 64)
#pragma unroll
    for (int q = 0; q < 4; ++q) s[q] += part[((int64_t)vt * N + n) * 4 + q];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s[q] += __shfl_xor(s[q], m);
  if (lane == 0) {
    float* rec = rows + (int64_t)n * OACE_ROW;
    const float tau = rec[OACE_TAU];
    float rho_t = 0.f, rn_t = 0.f;
    if (valid) {
      const float x = rec[OACE_ROW - 1] * tau;
      const Oct<float> o = octic(x);
      rho_t = o.rho;
      rn_t = o.r * x;
    }
    oace_finalize_row<float>(rec, tau, s[0], s[1], s[2], s[3], rho_t, rn_t, inv_v, gamma);
  }
}

// ------------------------------------------------------------------------------ host side
namespace {

int64_t nvt_of(int64_t V) { return (V + TV - 1) / TV; }
int64_t nnt_of(int64_t N) { return (N + TN - 1) / TN; }
int64_t ldz_of(int64_t V) { return (V + 63) / 64 * 64; }
size_t al(size_t b) { return (b + 255) & ~(size_t)255; }
bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The forward keeps the fp32 logits (rows x padded vocabulary) when they take at most this many
// bytes -- the reference benchmark's 512 x 50257 take 103 MB, which the 256 MB Infinity Cache
// holds -- and then evaluates the octic sums, and the backward dz, from them instead of a
// second GEMM sweep.  Larger problems recompute z, which keeps the workspace O(rows x d_model).
constexpr size_t ZC_MAX_BYTES = (size_t)256 << 20;
bool z_cached(const OaceArgs& a) {
  return !(a.flags & OACE_FLAG_RECOMPUTE_Z) && (size_t)a.N * ldz_of(a.V) * sizeof(float) <= ZC_MAX_BYTES;
}

// dh (N, d) = dz W^T as D[n][m] = sum_v W^T[v][m] dz[n][v]: A = W^T row-contiguous over the
// model features, B = dz contraction-contiguous.  Its vocabulary contraction is split for this
// many workgroups: a constant, so that the summation order, and the result, do not depend on
// the device.
constexpr int DH_WGS = 256;
OaceGemm dh_gemm(const OaceArgs& a, const unsigned short* wt, int64_t ldwt, const unsigned short* dz) {
  return OaceGemm{wt, ldwt, true, a.d, dz, ldz_of(a.V), false, a.N, a.V, a.dh, a.d};
}

struct Layout {
  size_t wt, zc, part, dz, dhp, total;
};
Layout layout_of(const OaceArgs& a) {
  Layout l;
  l.wt = a.w_layout == OACE_W_DV ? al((size_t)a.V * a.d * 2) : 0;
  l.zc = z_cached(a) ? al((size_t)a.N * ldz_of(a.V) * sizeof(float)) : 0;
  l.part = al((size_t)nvt_of(a.V) * a.N * 4 * sizeof(float));
  l.dz = al((size_t)a.N * ldz_of(a.V) * 2);
  const OaceGemm gh = dh_gemm(a, nullptr, a.d, nullptr);
  l.dhp = al(oace_gemm_part_bytes(gh, oace_gemm_parts(gh, DH_WGS)));  // split-K partials of dh
  l.total = l.wt + l.zc + std::max(l.part, l.dz + l.dhp);
  return l;
}

// W^T (V, d) with d contiguous: the caller's tied embedding, or a transposed copy at the start of
// the workspace -- made here, or left there by a forward call on the same workspace and weights
// (OACE_FLAG_WT_READY, the caller's guarantee).
const unsigned short* wt_of(const OaceArgs& a, void* ws, int64_t& ldwt, hipStream_t st, hipError_t& e) {
  e = hipSuccess;
  if (a.w_layout == OACE_W_VD) {
    ldwt = a.ldw;
    return (const unsigned short*)a.w;
  }
  ldwt = a.d;
  if (!(a.flags & OACE_FLAG_WT_READY)) e = oace_transpose16(a.w, a.d, a.V, a.ldw, ws, a.d, st);
  return (const unsigned short*)ws;
}

GemmArgs gemm_args(const OaceArgs& a, const unsigned short* wt, int64_t ldwt) {
  GemmArgs g = {};
  g.wt = wt;
  g.ldwt = ldwt;
  g.h = (const unsigned short*)a.h;
  g.ldh = a.ldh;
  g.N = (int)a.N;
  g.V = (int)a.V;
  g.d = (int)a.d;
  g.nvt = (int)nvt_of(a.V);
  g.nnt = (int)nnt_of(a.N);
  g.targets = a.targets;
  return g;
}

template <int DT, int MODE>
hipError_t launch_gemm(const GemmArgs& g, hipStream_t st) {
  const unsigned grid = (unsigned)(8 * g.nnt * ((g.nvt + 7) / 8));
  hipLaunchKernelGGL((oace_mfma_gemm_kernel<DT, MODE>), dim3(grid), dim3(256), 0, st, g);
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_gemm_dt(int dtype, const GemmArgs& g, hipStream_t st) {
  return dtype == AFA_BF16 ? launch_gemm<AFA_BF16, MODE>(g, st) : launch_gemm<AFA_F16, MODE>(g, st);
}

}  // namespace

bool oace_mfma_supported(int dtype, const OaceArgs& a) {
  if (dtype != AFA_BF16 && dtype != AFA_F16) return false;
  if (a.d % KS != 0 || a.ldh % 8 != 0 || !al16(a.h)) return false;
  if (a.w_layout == OACE_W_VD && (a.ldw % 8 != 0 || !al16(a.w))) return false;
  if (a.N > (1 << 28) || a.V >= (1 << 24)) return false;
  // 32-bit per-lane offsets of the backward GEMMs' direct loads
  if (a.ldh >= (1 << 26) || (a.w_layout == OACE_W_VD && a.ldw >= (1 << 26))) return false;
  return true;
}

size_t oace_mfma_workspace(int dtype, const OaceArgs& a) {
  (void)dtype;
  return layout_of(a).total;
}

hipError_t oace_linear_fwd_mfma(int dtype, const OaceArgs& a, void* rows, void* ws, hipStream_t st) {
  const Layout l = layout_of(a);
  char* base = (char*)ws;
  hipError_t e;
  int64_t ldwt = 0;
  const unsigned short* wt = wt_of(a, base, ldwt, st, e);
  if (e != hipSuccess) return e;
  float* part = (float*)(base + l.wt + l.zc);
  GemmArgs g = gemm_args(a, wt, ldwt);
  g.rows = (const float*)rows;
  g.part = part;
  const float inv_v = (float)(1.0 / (double)a.V);
  const bool zc = l.zc > 0;
  if (zc) {
    g.zc = (float*)(base + l.wt);
    g.ldz = ldz_of(a.V);
    e = launch_gemm_dt<MODE_SQZ>(dtype, g, st);
  } else {
    g.zt = (float*)rows + (OACE_ROW - 1);
    e = launch_gemm_dt<MODE_SQ>(dtype, g, st);
  }
  if (e != hipSuccess) return e;
  if (zc) {
    hipLaunchKernelGGL(oace_mfma_row_cached_kernel, dim3((unsigned)a.N), dim3(RC_THREADS), 0, st, (const float*)part,
                       g.nvt, (const float*)g.zc, g.ldz, g.N, g.V, inv_v, (float)a.eps, (float)a.gamma, a.targets,
                       (float*)rows);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return oace_mean_launch(dtype, rows, a.N, a.loss, st);
  }
  const unsigned rg = (unsigned)((a.N + 3) / 4);
  hipLaunchKernelGGL(oace_mfma_tau_kernel, dim3(rg), dim3(256), 0, st, (const float*)part, g.nvt, g.N, inv_v,
                     (float)a.eps, (float*)rows);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = launch_gemm_dt<MODE_OCTIC>(dtype, g, st)) != hipSuccess) return e;
  const unsigned wg = (unsigned)((a.N + 3) / 4);
  hipLaunchKernelGGL(oace_mfma_rows_kernel, dim3(wg), dim3(256), 0, st, (const float*)part, g.nvt, g.N, inv_v,
                     (float)a.gamma, g.V, a.targets, (float*)rows);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return oace_mean_launch(dtype, rows, a.N, a.loss, st);
}

hipError_t oace_linear_bwd_mfma(int dtype, const OaceArgs& a, const void* rows, void* ws, hipStream_t st) {
  const Layout l = layout_of(a);
  char* base = (char*)ws;
  hipError_t e;
  int64_t ldwt = 0;
  const unsigned short* wt = wt_of(a, base, ldwt, st, e);
  if (e != hipSuccess) return e;
  char* sbase = base + l.wt + l.zc;  // the region after the cached logits
  unsigned short* dz = (unsigned short*)sbase;
  GemmArgs g = gemm_args(a, wt, ldwt);
  g.rows = (const float*)rows;
  g.dz = dz;
  g.ldz = ldz_of(a.V);
  g.c0 = (float)(8.0 * a.gamma / (double)a.N);
  g.g_loss = (const float*)a.g_loss;
  if (l.zc > 0 && (a.flags & OACE_FLAG_Z_READY)) {
    // the forward's logits are in the workspace: dz elementwise
    const float* zcp = (const float*)(base + l.wt);
    const unsigned dg = (unsigned)(((int64_t)a.N * ((g.ldz + DZ_SPAN - 1) / DZ_SPAN) + 3) / 4);
    if (dtype == AFA_BF16)
      hipLaunchKernelGGL(oace_mfma_dz_cached_kernel<AFA_BF16>, dim3(dg), dim3(256), 0, st, zcp, g.ldz, g.N, g.V,
                         (const float*)rows, a.targets, g.c0, g.g_loss, dz);
    else
      hipLaunchKernelGGL(oace_mfma_dz_cached_kernel<AFA_F16>, dim3(dg), dim3(256), 0, st, zcp, g.ldz, g.N, g.V,
                         (const float*)rows, a.targets, g.c0, g.g_loss, dz);
    e = hipGetLastError();
  } else {
    e = launch_gemm_dt<MODE_DZ>(dtype, g, st);
  }
  if (e != hipSuccess) return e;
  const OaceGemm gh = dh_gemm(a, wt, ldwt, dz);
  if ((e = oace_gemm(dtype, gh, oace_gemm_parts(gh, DH_WGS), (float*)(sbase + l.dz), st)) != hipSuccess) return e;
  const OaceGemm gw = a.w_layout == OACE_W_DV
                          // dW (d, V): D[k][v] = sum_n dz[n][v] h[n][k]
                          ? OaceGemm{dz, g.ldz, true, a.V, a.h, a.ldh, true, a.d, a.N, a.dw, a.ldw}
                          // dW^T (V, d): D[v][k] = sum_n h[n][k] dz[n][v]
                          : OaceGemm{a.h, a.ldh, true, a.d, dz, g.ldz, true, a.V, a.N, a.dw, a.ldw};
  return oace_gemm(dtype, gw, 1, nullptr, st);
}

}  // namespace afa
