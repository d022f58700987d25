// fp32 ("HIGHEST") fused AFA forward on the fp32 matrix cores (v_mfma_f32_32x32x2_f32), for
// head_dim 32, 64 and 128.  Same contract as the generic fp32 path (src/kernels/pallas_afa.py:
// 52-151 with fp32 operands): s = (q . k) scale in fp32, w = rho(s)^8 by the cancellation-safe
// two-branch form, out = sum_j w v_j / (sum_j w + Omega), d = sum_j w + Omega; only the order of
// the fp32 additions differs.
//
// A wave owns 32 queries; a unit is 32 keys x 32 queries.
//   S^T = K Q^T: 32x32x2 steps over head_dim.  The two k-slots of a step are split by lane group
//   g: group g contracts head_dim entries [g D/2, (g+1) D/2), so a lane reads its K row as
//   contiguous 16-byte LDS fragments and keeps its query's half of q in registers.
//   O^T += V^T P^T: the S^T accumulator of lane (query c, group g) holds keys 8 (e >> 2) + 4 g +
//   (e & 3); contracting key (j, g) at step j makes element j of that accumulator the B operand as
//   it is, and the A operand one V element per lane (consecutive lanes, consecutive features).
// K/V tiles of 32 keys are staged through registers into double-buffered, padded LDS rows (the
// Cayley rotation of k is applied in that pass, as the generic kernel does), one barrier per tile.
// Query blocks are dispatched heaviest first (block_item).
// Small grids (fewer workgroups than CUs) split every query block's key tiles over blockIdx.y:
// the numerator and denominator are sums over keys, so each split writes its partial O and row
// sum, and afa_fwd_f32_combine_kernel adds them, adds the sink and divides.
#include <climits>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

namespace {

constexpr int KT = 32;  // keys per tile

__device__ __forceinline__ f32x16_t mma_f32(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float rot_first(float c, float s, float x0, float x1) {
#pragma clang fp contract(off)
  return c * x0 - s * x1;
}
__device__ __forceinline__ float rot_second(float c, float s, float x0, float x1) {
#pragma clang fp contract(off)
  return s * x0 + c * x1;
}

}  // namespace

template <int D, bool ROT, bool SPLIT>
__global__ __launch_bounds__(256) void afa_fwd_f32_kernel(const FwdArgs a) {
  constexpr int LDR = D + 4;   // padded LDS row: consecutive rows shift by 16 bytes (no conflicts)
  constexpr int DV = (D + 31) / 32 * 32;  // V features in 32-feature output blocks (48 -> 64)
  constexpr int LDV = DV + 4;  // V rows; features [D, DV) stay zero
  constexpr int KH = D / 2;    // head_dim entries per lane group
  constexpr int NDB = DV / 32; // 32-feature output blocks
  constexpr int KJOBS = KT * (D / 2) / 256;  // rotation pairs per thread per tile
  constexpr int VJOBS = (KT * (D / 4) + 255) / 256;  // float4 of V per thread per tile
  static_assert(KT * (D / 2) % 256 == 0 && KJOBS >= 1, "head_dim does not fit the tile loader");
  __shared__ __attribute__((aligned(16))) float ks[2][KT * LDR];
  __shared__ __attribute__((aligned(16))) float vs[2][KT * LDV];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  int bh, qblk;
  block_item(blockIdx.x, a.B * a.H, a.nqb, a.causal, bh, qblk);
  const int b = bh / a.H, h = bh % a.H;
  const int L = a.L, vlen = a.valid_len;
  const int q0_wg = qblk * 128, q0_w = q0_wg + wave * 32;
  const int qi = q0_w + l32;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 128)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 32) : vlen;
  const int ntiles_wg = (kend_wg + KT - 1) / KT;
  // this workgroup's key tiles [t_beg, ntiles): all of them, or one of gridDim.y even parts
  int t_beg = 0, ntiles = ntiles_wg;
  if constexpr (SPLIT) {
    const int per = (ntiles_wg + (int)gridDim.y - 1) / (int)gridDim.y;
    t_beg = min(ntiles_wg, (int)blockIdx.y * per);
    ntiles = min(ntiles_wg, t_beg + per);
  }
  const float* qp = (const float*)a.q + b * a.q_b + h * a.q_h;
  const float* kp = (const float*)a.k + b * a.k_b + h * a.k_h;
  const float* vp = (const float*)a.v + b * a.v_b + h * a.v_h;

  // q: lane (query qi, group g) holds features [g KH, (g+1) KH), rotated in fp32 when ROT
  float qf[KH];
#pragma unroll
  for (int j = 0; j < KH; j += 2) {
    const int d0 = g * KH + j;
    float x0 = 0.f, x1 = 0.f;
    if (qi < L) {
      x0 = qp[(int64_t)qi * a.q_l + d0];
      x1 = qp[(int64_t)qi * a.q_l + d0 + 1];
      if constexpr (ROT) {
        const float c = a.rc[(int64_t)qi * (D / 2) + d0 / 2], s = a.rs[(int64_t)qi * (D / 2) + d0 / 2];
        const float y0 = rot_first(c, s, x0, x1), y1 = rot_second(c, s, x0, x1);
        x0 = y0;
        x1 = y1;
      }
    }
    qf[j] = x0;
    qf[j + 1] = x1;
  }

  // tile staging in registers: K as rotation pairs, V as float4.  Each thread's elements sit at
  // the same offsets in every tile: those offsets are formed once, and a tile only moves the
  // (wave-uniform) base pointers by KT rows.
  float kx[KJOBS][2];
  float kc[KJOBS], ksn[KJOBS];
  f32x4_t vx[VJOBS];
  int64_t koff[KJOBS], voff[VJOBS];
  int krow[KJOBS], vrow[VJOBS], toff[KJOBS];
#pragma unroll
  for (int i = 0; i < KJOBS; ++i) {
    const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
    krow[i] = r;
    koff[i] = (int64_t)r * a.k_l + 2 * p;
    toff[i] = r * (D / 2) + p;
  }
#pragma unroll
  for (int i = 0; i < VJOBS; ++i) {
    const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
    vrow[i] = e < KT * (D / 4) ? r : INT_MAX;  // past the tile (head_dim 48): never loaded
    voff[i] = (int64_t)r * a.v_l + 4 * c4;
  }
  auto load = [&](int t) {
    const int rows = L - t * KT;  // rows of tile t inside the sequence
    const float* kt = kp + (int64_t)t * KT * a.k_l;
    const float* vt = vp + (int64_t)t * KT * a.v_l;
#pragma unroll
    for (int i = 0; i < KJOBS; ++i) {
      kx[i][0] = kx[i][1] = 0.f;
      kc[i] = 1.f;
      ksn[i] = 0.f;
      if (krow[i] < rows) {
        kx[i][0] = kt[koff[i]];
        kx[i][1] = kt[koff[i] + 1];
        if constexpr (ROT) {
          kc[i] = a.rc[(int64_t)t * KT * (D / 2) + toff[i]];
          ksn[i] = a.rs[(int64_t)t * KT * (D / 2) + toff[i]];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VJOBS; ++i) {
      f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      vx[i] = vrow[i] < rows ? *(const f32x4_t*)(vt + voff[i]) : z;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 2), p = e % (D / 2);
      float y0 = kx[i][0], y1 = kx[i][1];
      if constexpr (ROT) {
        y0 = rot_first(kc[i], ksn[i], kx[i][0], kx[i][1]);
        y1 = rot_second(kc[i], ksn[i], kx[i][0], kx[i][1]);
      }
      ks[buf][r * LDR + 2 * p] = y0;
      ks[buf][r * LDR + 2 * p + 1] = y1;
    }
#pragma unroll
    for (int i = 0; i < VJOBS; ++i) {
      const int e = tid + 256 * i, r = e / (D / 4), c4 = e % (D / 4);
      if (e < KT * (D / 4)) *(f32x4_t*)&vs[buf][r * LDV + 4 * c4] = vx[i];
    }
  };
  if constexpr (DV > D) {  // the padding features of both V buffers, once
    for (int e = tid; e < 2 * KT * (DV - D); e += 256) {
      const int buf = e / (KT * (DV - D)), r = (e / (DV - D)) % KT, f = D + e % (DV - D);
      vs[buf][r * LDV + f] = 0.f;
    }
  }

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float dsum = 0.f;
  const float scale = a.q_scale;

  if (t_beg < ntiles) {
    load(t_beg);
    store(t_beg & 1);
  }
  __syncthreads();
  for (int t = t_beg; t < ntiles; ++t) {
    if (t + 1 < ntiles) load(t + 1);  // global loads in flight during this tile's MFMAs
    const int key0 = t * KT;
    if (key0 < kend_w && q0_w < L) {
      const float* kt = ks[t & 1];
      const float* vt = vs[t & 1];
      f32x16_t st;
#pragma unroll
      for (int e = 0; e < 16; ++e) st[e] = 0.f;
#pragma unroll
      for (int j4 = 0; j4 < KH / 4; ++j4) {
        const f32x4_t kv = *(const f32x4_t*)(kt + l32 * LDR + g * KH + 4 * j4);
#pragma unroll
        for (int u = 0; u < 4; ++u) st = mma_f32(kv[u], qf[4 * j4 + u], st);
      }
      const bool need_mask = (a.causal && key0 + 31 > q0_w) || key0 + 31 >= vlen || q0_w + 31 >= L;
#pragma unroll
      for (int e = 0; e < 16; ++e) st[e] = rho8_exact(st[e] * scale);
      if (need_mask) {
        // a side effect the compiler cannot move keeps this a branch on the wave-uniform test
        // instead of a compare and a select per score in every tile
        asm volatile("" ::: "memory");
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = key0 + 8 * (e >> 2) + 4 * g + (e & 3);
          const bool keep = key < vlen && qi < L && (!a.causal || key <= qi);
          st[e] = keep ? st[e] : 0.f;
        }
      }
      float ts = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) ts += st[e];
      // two-level sums: the tile's own (row sum and PV from zero), then added to the running
      // ones, as the reference adds one block's dot(p, v) at a time
      // (src/kernels/pallas_afa.py:131-139); a single chain over L keys would carry a rounding
      // error growing with L (4.8e-6 normwise at L = 4096 against 1.3e-6 for 256-key chains)
      dsum += ts;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        f32x16_t ot;
#pragma unroll
        for (int e = 0; e < 16; ++e) ot[e] = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kr = 8 * (j >> 2) + 4 * g + (j & 3);
          ot = mma_f32(vt[kr * LDV + db * 32 + l32], st[j], ot);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] += ot[e];
      }
    }
    // the buffer of tile t+1 was last read in tile t-1, before the previous barrier
    if (t + 1 < ntiles) store((t + 1) & 1);
    __syncthreads();
  }

  dsum += __shfl_xor(dsum, 32);
  if constexpr (SPLIT) {
    // unnormalised partials of split blockIdx.y: the numerators of all splits (each B, H, L, D),
    // then the row sums of all splits (each B, H, L)
    const int64_t rows = (int64_t)a.B * a.H * L;
    float* po = a.part + (int64_t)blockIdx.y * rows * D;
    float* pd = a.part + (int64_t)gridDim.y * rows * D + (int64_t)blockIdx.y * rows;
    if (qi < L) {
      float* op = po + ((int64_t)bh * L + qi) * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          if (DV == D || db * 32 + 8 * e4 + 4 * g < D) {
            f32x4_t w;
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] = o[db][4 * e4 + u];
            *(f32x4_t*)(op + db * 32 + 8 * e4 + 4 * g) = w;
          }
        }
      if (g == 0) pd[(int64_t)bh * L + qi] = dsum;
    }
    return;
  }
  if (qi < L) {
    const float tot = dsum + a.omega;
    float* op = (float*)a.out + b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        if (DV == D || db * 32 + 8 * e4 + 4 * g < D) {
          f32x4_t* p = (f32x4_t*)(op + db * 32 + 8 * e4 + 4 * g);
          f32x4_t w;
          if (a.acc) {
            // one key shard: the unnormalised sums, stored or added to the caller's arrays
            if (a.acc == ACC_ADD) w = *p;
            else w = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] += o[db][4 * e4 + u];
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] = o[db][4 * e4 + u] / tot;
          }
          *p = w;
        }
      }
    if (a.acc && g == 0) acc_row(a.denom + (int64_t)bh * L + qi, dsum, a.acc);
    else if (a.denom != nullptr && g == 0) a.denom[(int64_t)bh * L + qi] = tot;
  }
}

// out = (sum of the split numerators) / (sum of the split row sums + sink), in split order; one
// thread per 4 features of a row.
template <int D>
__global__ __launch_bounds__(256) void afa_fwd_f32_combine_kernel(const FwdArgs a, int nsplit) {
  const int64_t rows = (int64_t)a.B * a.H * a.L;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * (D / 4)) return;
  const int64_t row = idx / (D / 4);
  const int c4 = (int)(idx % (D / 4));
  float tot = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < nsplit; ++sp) {
    tot += a.part[(int64_t)nsplit * rows * D + (int64_t)sp * rows + row];
    const f32x4_t v = *(const f32x4_t*)(a.part + (int64_t)sp * rows * D + row * D + 4 * c4);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += v[u];
  }
  tot += a.omega;
  const int bh = (int)(row / a.L), l = (int)(row % a.L);
  const int b = bh / a.H, h = bh % a.H;
  float* op = (float*)a.out + b * a.o_b + h * a.o_h + (int64_t)l * a.o_l + 4 * c4;
  if (a.acc) {
    // one key shard: the sums, stored or added to the caller's arrays (the sink is 0)
    f32x4_t w = {0.f, 0.f, 0.f, 0.f};
    if (a.acc == ACC_ADD) w = *(const f32x4_t*)op;
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] += acc[u];
    *(f32x4_t*)op = w;
    if (c4 == 0) acc_row(a.denom + row, tot, a.acc);
    return;
  }
  f32x4_t w;
#pragma unroll
  for (int u = 0; u < 4; ++u) w[u] = acc[u] / tot;
  *(f32x4_t*)op = w;
  if (a.denom != nullptr && c4 == 0) a.denom[row] = tot;
}

bool f32_fwd_supported(int head_dim) {
  return head_dim == 32 || head_dim == 48 || head_dim == 64 || head_dim == 96 || head_dim == 128;
}

size_t f32_fwd_part_floats(const FwdArgs& a, int head_dim, int nsplit) {
  return (size_t)nsplit * a.B * a.H * a.L * (head_dim + 1);
}

template <int D, bool SPLIT>
static void f32_launch_s(const FwdArgs& a, int nsplit, hipStream_t st) {
  const dim3 grid((unsigned)(a.B * a.H * a.nqb), (unsigned)nsplit);
  if (a.rc != nullptr)
    hipLaunchKernelGGL((afa_fwd_f32_kernel<D, true, SPLIT>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((afa_fwd_f32_kernel<D, false, SPLIT>), grid, dim3(256), 0, st, a);
}

template <int D>
static hipError_t f32_launch_d(const FwdArgs& a, int nsplit, hipStream_t st) {
  if (nsplit <= 1) {
    f32_launch_s<D, false>(a, 1, st);
    return hipGetLastError();
  }
  if (a.part == nullptr) return hipErrorInvalidValue;
  f32_launch_s<D, true>(a, nsplit, st);
  const int64_t n = (int64_t)a.B * a.H * a.L * (D / 4);
  hipLaunchKernelGGL((afa_fwd_f32_combine_kernel<D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a,
                     nsplit);
  return hipGetLastError();
}

hipError_t f32_fwd_launch(int head_dim, FwdArgs a, int nsplit, hipStream_t st) {
  a.nqb = (a.L + 127) / 128;
  if (head_dim == 32) return f32_launch_d<32>(a, nsplit, st);
  if (head_dim == 48) return f32_launch_d<48>(a, nsplit, st);
  if (head_dim == 64) return f32_launch_d<64>(a, nsplit, st);
  if (head_dim == 96) return f32_launch_d<96>(a, nsplit, st);
  return f32_launch_d<128>(a, nsplit, st);
}

}  // namespace afa
