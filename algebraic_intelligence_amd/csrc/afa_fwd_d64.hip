// Software-pipelined fused AFA forward for head_dim 64 (bf16 / fp16 operands, fp32 accumulate).
//
// Same contract as afa_fwd_mfma.hip (src/kernels/pallas_afa.py:52-151); this kernel is shaped
// for the VALU-bound regime of head_dim 64, where each score costs ~7.5 VALU slots (rho^8
// chain, row sum, bf16 pack) against 256 MFMA FLOPs:
//
//   * a wave owns 64 queries = two 32-query blocks; its key axis is cut into 32-key sub-tiles,
//     and a "unit" is (sub-tile n, query block qb), u = 2n + qb;
//   * unit u evaluates rho^8 of S(u) on the VALU while the MFMA pipe runs S(u+1) = K Q^T and
//     O += V^T P(u-1); S alternates between two register sets, so no copies are made;
//   * K and V tiles reach LDS by direct global -> LDS loads with no register or VALU work: rows
//     of 128 B with XOR-swizzled 16-byte chunks, K read as 32-row fragments, V with
//     ds_read_tr16_b64, which returns 4 consecutive keys of one feature column per lane (two
//     such reads form the PV MFMA's A operand in the key order of the S^T accumulator);
//   * LDS is a ring of 4 tiles of 64 keys: iteration t computes on tiles t and t+1, loads tile
//     t+3 and waits only for its own loads of tile t+2; one barrier per tile;
//   * the Cayley rotation (AGO) of q is applied when a wave loads its queries; k is rotated
//     once per call by afa_krot_kernel (each K tile is read by up to L/256 query blocks, so
//     rotating it at every tile load would repeat the work that many times); both use the
//     same fp32 arithmetic and a single rounding to the element type;
//   * masks (causal diagonal, valid_len) are applied only on units that cross them;
//   * workgroups are dispatched heaviest query block first across all heads, with the heads of
//     one XCD grouped together (shared L2).
#include <type_traits>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

namespace {

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

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

template <int DT>
__device__ __forceinline__ u32x4_t rot4(u32x4_t w, f32x4_t c, f32x4_t s, float scale) {
#pragma clang fp contract(off)
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = Elem<DT>::lo(w[p]);
    const float x1 = Elem<DT>::hi(w[p]);
    const float y0 = c[p] * x0 - s[p] * x1;
    const float y1 = s[p] * x0 + c[p] * x1;
    r[p] = Elem<DT>::pack(y0 * scale, y1 * scale);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ u32x4_t scl4(u32x4_t w, float scale) {
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = Elem<DT>::pack(Elem<DT>::lo(w[p]) * scale, Elem<DT>::hi(w[p]) * scale);
  return r;
}

// Pairwise tree sum of 16 values (shorter dependency chain than a running sum).
__device__ __forceinline__ float tree16(const float (&p)[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[2 * i] + p[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[2 * i] + a[2 * i + 1];
  a[0] = a[0] + a[1];
  a[2] = a[2] + a[3];
  return a[0] + a[2];
}

}  // namespace


// LDS tiles of the head_dim-64 kernel: a ring of D64_NB tiles of D64_KT keys x 64 features.
constexpr int D64_KT = 64;
constexpr int D64_NB = 4;
typedef unsigned short D64Tile[D64_KT * 64];

// Cayley rotation of K, once per call: y (contiguous B, H, L, D) = rotate(x) in fp32 with the
// (L, D/2) fp32 tables, rounded once to the element type -- the values the fused loaders would
// produce (rot4 with scale 1).  Each wave handles one (b, h, 64-row block) work item with the
// lane layout of RowBlockLayout (contiguous 16-byte chunks), and also writes the largest squared
// norm of the block's rotated rows (as rounded) to nb2[bh * nblk + block], the key bound of the
// fast-rho guard (fast_rho_safe).
template <int DT, int D>
__global__ __launch_bounds__(256) void afa_krot_kernel(const FwdArgs a, unsigned short* y, float* nb2, int nblk,
                                                      int nwork, int* zero, int nzero) {
  using RL = RowBlockLayout<D>;
  for (int i = blockIdx.x * 256 + (int)threadIdx.x; i < nzero; i += gridDim.x * 256) zero[i] = 0;
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (int)(threadIdx.x >> 6);  // wave-uniform work item
  if (w >= nwork) return;
  const int bh = w / nblk, blk = w - bh * nblk;
  const int b = bh / a.H, h = bh - b * a.H;
  const unsigned short* xb = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
  unsigned short* yb = y + (int64_t)bh * a.L * D;
  const int c = lane % RL::CHP, rsub = lane / RL::CHP;
  // the loads of G row iterations are issued before their first store: the stores to y could
  // alias the inputs as far as the compiler knows, so a load-rotate-store loop would wait on HBM
  // per row; G = 4 keeps 12 loads per lane in flight at 48 VGPRs of staging
  constexpr int G = RL::CHP < 4 ? RL::CHP : 4;
  float m = 0.0f;
#pragma unroll
  for (int g = 0; g < RL::CHP; g += G) {
    u32x4_t wv[G];
    f32x4_t cc[G], ss[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int l = blk * 64 + (g + i) * RL::RPI + rsub;
      if (c < RL::CH && l < a.L) {
        wv[i] = *(const u32x4_t*)(xb + (int64_t)l * a.k_l + c * 8);
        cc[i] = *(const f32x4_t*)(a.rc + (int64_t)l * (D / 2) + c * 4);
        ss[i] = *(const f32x4_t*)(a.rs + (int64_t)l * (D / 2) + c * 4);
      }
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int l = blk * 64 + (g + i) * RL::RPI + rsub;
      float n2 = 0.0f;
      if (c < RL::CH && l < a.L) {
        const u32x4_t r = rot4<DT>(wv[i], cc[i], ss[i], 1.0f);
        *(u32x4_t*)(yb + (int64_t)l * D + c * 8) = r;
        n2 = chunk_norm2<DT>(r);
      }
      m = __builtin_fmaxf(m, group_sum<RL::CHP>(n2));
    }
  }
  m = wave_max(m);
  if (lane == 0) nb2[(int64_t)bh * nblk + blk] = m;
}

// Tile loop and epilogue of afa_fwd_d64_kernel for one form of rho^8: FAST, the branch-free
// rho8_fast (the wave's scores are all within the fast-rho bound), else the two-branch
// rho8_exact.  The kernel instantiates both and each wave runs one, so the two loops get their
// own register allocation; the barriers count waves, not code locations.
template <int DT, bool FAST>
__device__ __forceinline__ void d64_body(const FwdArgs& a, D64Tile* lds_k, D64Tile* lds_v, const u32x4_t (&qf)[2][4],
                                         int bh, int qblk) {
  constexpr int D = 64;
  constexpr int KT = D64_KT;
  constexpr int NB = D64_NB;
  constexpr int LOADS = 4;      // direct loads per thread per tile (2 K + 2 V chunks)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int l16 = lane & 15;
  const int m16 = (lane >> 4) & 1;
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int L = a.L;
  const int vlen = a.valid_len;

  const int q0_wg = qblk * 256;
  const int q0_w = q0_wg + wave * 64;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 256)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 64) : vlen;
  const int ntiles = (kend_wg + KT - 1) / KT;
  const int nsub = q0_w < L ? (kend_w + 31) / 32 : 0;  // 32-key sub-tiles of this wave
  const int U = 2 * nsub;                                // units of this wave
  const unsigned short* kp = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
  const unsigned short* vp = (const unsigned short*)a.v + b * a.v_b + h * a.v_h;
  // rho^8 of one unit's 16 scores per lane
  auto rho8_unit = [&](float (&p)[16], const f32x16_t& sv) {
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = FAST ? rho8_fast(sv[r]) : rho8_exact(sv[r]);
  };

  // ---- tile staging by direct global -> LDS loads.  Thread chunk c = tid + 256 i covers key
  // row c >> 3 of the tile and physical 16-byte column c & 7; it loads the logical chunk that
  // the swizzle places there.  K arrives already Cayley-rotated (rotated once per call by
  // afa_krot_kernel), so the tiles need no further work after their loads land.
  const int row0 = tid >> 3, c8 = tid & 7;     // chunk 1 is row0 + 32 (same low row bits)
  const int lcv = c8 ^ (((row0 >> 1) & 1) << 2);
  const int lck = c8 ^ (row0 & 7);
  // Each load is a uniform base (the tile's first row) plus a 32-bit lane offset: the caller
  // routes only strides whose in-head byte offsets fit 32 bits here.
  const uint32_t voff = (uint32_t)(row0 * (int)a.v_l + lcv * 8) * 2u;
  const uint32_t koff = (uint32_t)(row0 * (int)a.k_l + lck * 8) * 2u;
  const int64_t v32 = 64 * a.v_l, k32 = 64 * a.k_l;  // bytes of 32 rows
  auto issue_tile = [&](int t) {
    unsigned short* vdst = &lds_v[t & (NB - 1)][wave * 512];
    unsigned short* kdst = &lds_k[t & (NB - 1)][wave * 512];
    if (t * KT + KT <= L) {
      const char* vb = (const char*)vp + (int64_t)t * KT * a.v_l * 2;
      const char* kb = (const char*)kp + (int64_t)t * KT * a.k_l * 2;
      lds_dma16(vb, voff, vdst);
      lds_dma16(vb + v32, voff, vdst + 2048);
      lds_dma16(kb, koff, kdst);
      lds_dma16(kb + k32, koff, kdst + 2048);
    } else {
      // last, partial tile: rows past L read row L-1 (masked keys; the data only has to be finite)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int key = min(t * KT + row0 + 32 * i, L - 1);
        const uint32_t vo = (uint32_t)(key * (int)a.v_l + lcv * 8) * 2u;
        const uint32_t ko = (uint32_t)(key * (int)a.k_l + lck * 8) * 2u;
        lds_dma16(vp, vo, vdst + 2048 * i);
        lds_dma16(kp, ko, kdst + 2048 * i);
      }
    }
  };

  // ---- per-unit fragment readers
  auto read_kf = [&](int n, u32x4_t (&kf)[4]) {
    const unsigned short* base = &lds_k[(n >> 1) & (NB - 1)][((n & 1) * 32 + l32) * D];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) kf[kc] = *(const u32x4_t*)(base + (((2 * kc + g) ^ (l32 & 7)) * 8));
  };
  auto read_vf = [&](int n, u32x4_t (&vf)[2][2]) {
    const unsigned short* tile = lds_v[(n >> 1) & (NB - 1)];
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int row = (n & 1) * 32 + kk * 16 + hh * 8 + 4 * g + (l16 >> 2);
          const int blk = db ^ ((row >> 1) & 1);
          const unsigned short* p = tile + row * D + blk * 32 + m16 * 16 + 4 * (l16 & 3);
          const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
          const u32x2_t w = __builtin_bit_cast(u32x2_t, v);
          f[2 * hh] = w[0];
          f[2 * hh + 1] = w[1];
        }
        vf[db][kk] = f;
      }
    }
  };

  f32x16_t o[2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[db][qb][e] = 0.f;
  float rowsum[2] = {0.f, 0.f};

  // pipeline state; S(u) lives in sA for odd u, in sB for even u
  f32x16_t sA, sB;
  u32x4_t p_prev[2];
  u32x4_t kf[4];
  u32x4_t vf[2][2];

  // prologue: tiles 0..2 in flight; wait for 0 and 1
  const int npro = min(ntiles, 3);
  for (int t = 0; t < npro; ++t) issue_tile(t);
  if (npro == 3) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS));
  else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  __syncthreads();

  auto mask16 = [&](float (&p)[16], int u) {
    const int key0 = (u >> 1) * 32;
    const int qlo = q0_w + (u & 1) * 32;
    if ((a.causal && key0 + 31 > qlo) || key0 + 31 >= vlen) {
      const int qi = qlo + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = key0 + (r >> 2) * 8 + 4 * g + (r & 3);
        const bool keep = (j < vlen) && (!a.causal || j <= qi);
        p[r] = keep ? p[r] : 0.f;
      }
    }
  };
  auto finish_p = [&](float (&p)[16], int qb) {
    rowsum[qb] += tree16(p);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) p_prev[kk][e] = Elem<DT>::pack(p[kk * 8 + 2 * e], p[kk * 8 + 2 * e + 1]);
  };

  // ---- unit 0: S(0), P(0), S(1) -> sA; fragments K(1), V(0)
  if (U > 0) {
    read_kf(0, kf);
    f32x16_t s0;
#pragma unroll
    for (int e = 0; e < 16; ++e) s0[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) s0 = mma<DT>(kf[kc], qf[0][kc], s0);
#pragma unroll
    for (int e = 0; e < 16; ++e) sA[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) sA = mma<DT>(kf[kc], qf[1][kc], sA);
    float p[16];
    rho8_unit(p, s0);
    mask16(p, 0);
    finish_p(p, 0);
    read_kf(1, kf);
    read_vf(0, vf);
  }

  // Unit u = 2n + QB: P(u) from scur = S(u); S(u+1) into snxt and PV(u-1) on the MFMA pipe,
  // interleaved with the rho^8 VALU; even units then read the fragments of sub-tiles n+1 (K)
  // and n (V).  Units past the wave's last one are skipped; masks apply only where needed.
  auto unit = [&](int u, f32x16_t& scur, f32x16_t& snxt, auto qb_tag) {
    constexpr int QB = decltype(qb_tag)::value;
    constexpr int NQ = QB ^ 1;
    constexpr int PQ = QB ^ 1;
    if (u > U) return;
    const int n = u >> 1;
    // S(u+1) unconditionally (past the wave's last unit it is never used; kf holds finite data)
#pragma unroll
    for (int e = 0; e < 16; ++e) snxt[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) snxt = mma<DT>(kf[kc], qf[NQ][kc], snxt);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db][PQ] = mma<DT>(vf[db][kk], p_prev[kk], o[db][PQ]);
    if (u < U) {
      float p[16];
      rho8_unit(p, scur);
      mask16(p, u);
      finish_p(p, QB);
      if constexpr (QB == 0) {
        if (u + 1 < U) read_kf(n + 1, kf);
        read_vf(n, vf);
      }
    }
  };
  // The same unit where it is known to be one of the wave's units, to need no mask and (even
  // units) to have a next sub-tile.  With no branch, the 8 MFMAs, the rho^8 VALU, the row sum,
  // the P packing and the fragment reads form one basic block, and the scheduler spreads the
  // MFMAs through the VALU stream: the wave keeps issuing VALU while its MFMAs run, instead of
  // waiting on the MFMA pipe before a branch.
  auto clean_unit = [&](int u, f32x16_t& scur, f32x16_t& snxt, auto qb_tag) {
    constexpr int QB = decltype(qb_tag)::value;
    constexpr int NQ = QB ^ 1;
    constexpr int PQ = QB ^ 1;
    const int n = u >> 1;
#pragma unroll
    for (int e = 0; e < 16; ++e) snxt[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) snxt = mma<DT>(kf[kc], qf[NQ][kc], snxt);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db][PQ] = mma<DT>(vf[db][kk], p_prev[kk], o[db][PQ]);
    float p[16];
    rho8_unit(p, scur);
    finish_p(p, QB);
    if constexpr (QB == 0) {
      read_kf(n + 1, kf);
      read_vf(n, vf);
    }
  };
  // Units 4t+1 .. 4t+4 of tile iteration t are clean when the last two (the largest key
  // sub-tile 2t+2 against either query half) need no mask and unit 4t+5 is still one of the
  // wave's.  Each condition can only turn false as t grows, so the clean iterations are a prefix
  // [0, tc): they run in a loop of their own (one loop holding both unit forms would not fit
  // the register budget).  Every wave passes ntiles barriers.
  auto tile_clean = [&](int t) {
    const int key_hi = 64 * t + 95;  // last key of sub-tile 2t+2
    return (!a.causal || key_hi <= q0_w) && key_hi < vlen && 4 * t + 5 < U;
  };
  int tc = 0;
  while (tc < ntiles && tile_clean(tc)) ++tc;

  // Iteration t reads tiles t and t+1, issues tile t+3 into the buffer of tile t-1 (last read
  // before the previous barrier) and waits for its own loads of tile t+2, which the barrier then
  // publishes for iteration t+1.
  auto tile_end = [&](int t) {
    if (t + 3 < ntiles) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS));
    else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __syncthreads();
  };
  for (int t = 0; t < tc; ++t) {
    if (t + 3 < ntiles) issue_tile(t + 3);
    clean_unit(4 * t + 1, sA, sB, std::integral_constant<int, 1>{});
    clean_unit(4 * t + 2, sB, sA, std::integral_constant<int, 0>{});
    clean_unit(4 * t + 3, sA, sB, std::integral_constant<int, 1>{});
    clean_unit(4 * t + 4, sB, sA, std::integral_constant<int, 0>{});
    tile_end(t);
  }
  for (int t = tc; t < ntiles; ++t) {
    if (t + 3 < ntiles) issue_tile(t + 3);
    unit(4 * t + 1, sA, sB, std::integral_constant<int, 1>{});
    unit(4 * t + 2, sB, sA, std::integral_constant<int, 0>{});
    unit(4 * t + 3, sA, sB, std::integral_constant<int, 1>{});
    unit(4 * t + 4, sB, sA, std::integral_constant<int, 0>{});
    tile_end(t);
  }

  if (a.acc) {
    // one key shard: the unnormalised sums go to the caller's fp32 arrays, stored (ACC_STORE) or
    // added to what they hold (ACC_ADD)
    float* op = (float*)a.out + b * a.o_b + h * a.o_h;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const float tot = rowsum[qb] + __shfl_xor(rowsum[qb], 32);
      const int qi = q0_w + qb * 32 + l32;
      if (qi < L) {
        // every load before the first store, so that the row's memory latencies overlap
        f32x4_t x[2][4];
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            x[db][r4] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (a.acc == ACC_ADD) x[db][r4] = *(const f32x4_t*)(op + (int64_t)qi * a.o_l + db * 32 + r4 * 8 + 4 * g);
          }
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) x[db][r4][u] += o[db][qb][r4 * 4 + u];
            *(f32x4_t*)(op + (int64_t)qi * a.o_l + db * 32 + r4 * 8 + 4 * g) = x[db][r4];
          }
        if (g == 0) acc_row(a.denom + (int64_t)bh * L + qi, tot, a.acc);
      }
    }
    return;
  }
  // ---- epilogue: one IEEE division per row, then products
  unsigned short* op = (unsigned short*)a.out + b * a.o_b + h * a.o_h;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float tot = rowsum[qb] + __shfl_xor(rowsum[qb], 32) + a.omega;
    const int qi = q0_w + qb * 32 + l32;
    if (qi < L) {
      const float inv = 1.0f / tot;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d0 = db * 32 + r4 * 8 + 4 * g;
          u32x2_t w;
          w[0] = Elem<DT>::pack(o[db][qb][r4 * 4 + 0] * inv, o[db][qb][r4 * 4 + 1] * inv);
          w[1] = Elem<DT>::pack(o[db][qb][r4 * 4 + 2] * inv, o[db][qb][r4 * 4 + 3] * inv);
          *(u32x2_t*)(op + (int64_t)qi * a.o_l + d0) = w;
        }
      }
      if (a.denom != nullptr && g == 0) a.denom[(int64_t)bh * L + qi] = tot * a.w_unscale;
    }
  }
}

template <int DT, bool EXACT, bool ROT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void afa_fwd_d64_kernel(const FwdArgs a) {
  constexpr int D = 64;
  // K and V tiles are row-major, 128 B per key row, 16-byte chunks XOR-swizzled: K chunk
  // c of row r sits at c ^ (r & 7) (conflict-free 32-row fragment reads), V chunk c at
  // c ^ (((r >> 1) & 1) << 2) (conflict-free ds_read_tr16_b64 of 4-key column slices).
  __shared__ __attribute__((aligned(16))) D64Tile lds_k[D64_NB];
  __shared__ __attribute__((aligned(16))) D64Tile lds_v[D64_NB];

  int bh, qblk;
  block_item(blockIdx.x, a.B * a.H, a.nqb, a.causal, bh, qblk);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int L = a.L;
  const int vlen = a.valid_len;

  const int q0_wg = qblk * 256;
  const int q0_w = q0_wg + wave * 64;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 256)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 64) : vlen;
  const unsigned short* qp = (const unsigned short*)a.q + b * a.q_b + h * a.q_h;
  // the fast-rho guard's key-block bounds go out first: they do not depend on q
  const float* kbm = !EXACT && a.kbm != nullptr ? a.kbm + (int64_t)bh * a.nkb : nullptr;
  const int kblk1 = (kend_w + 63) / 64;
  const float kbm_first = fast_rho_prefetch(kbm, 0, kblk1);

  // ---- Q fragments: query q0_w + qb*32 + l32, features kc*16 + 8g .. +7 (scaled, rotated)
  u32x4_t qf[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = q0_w + qb * 32 + l32;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int d0 = kc * 16 + 8 * g;
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (qi < L) {
        w = *(const u32x4_t*)(qp + (int64_t)qi * a.q_l + d0);
        if constexpr (ROT) {
          const f32x4_t c = *(const f32x4_t*)(a.rc + (int64_t)qi * (D / 2) + d0 / 2);
          const f32x4_t s = *(const f32x4_t*)(a.rs + (int64_t)qi * (D / 2) + d0 / 2);
          w = rot4<DT>(w, c, s, a.q_scale);
        } else {
          w = scl4<DT>(w, a.q_scale);
        }
      }
      qf[qb][kc] = w;
    }
  }
  // fast-rho guard: the largest squared norm of the wave's queries (as the MFMA sees them; each
  // lane holds half the features of query l32 of each block) against the key blocks it reads
  bool fast = false;
  if (!EXACT) {
    float m = 0.0f;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float n2 = 0.0f;
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) n2 += chunk_norm2<DT>(qf[qb][kc]);
      m = __builtin_fmaxf(m, n2 + __shfl_xor(n2, 32));
    }
    fast = fast_rho_safe(kbm, 0, kblk1, wave_max(m), a.nb_lim, kbm_first);
  }
  if (fast) d64_body<DT, true>(a, lds_k, lds_v, qf, bh, qblk);
  else d64_body<DT, false>(a, lds_k, lds_v, qf, bh, qblk);
}

template <int DT, bool EXACT, bool ROT>
static hipError_t launch_d64(const FwdArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((afa_fwd_d64_kernel<DT, EXACT, ROT>), dim3(a.B * a.H * a.nqb), dim3(256), 0, stream, a);
  return hipGetLastError();
}

size_t krot_bytes(const FwdArgs& a, int head_dim) { return (size_t)a.B * a.H * a.L * head_dim * 2; }

template <int D>
static void krot_launch_d(int dtype, const FwdArgs& a, void* krot, float* nb2, hipStream_t stream, int* zero,
                          int nzero) {
  const int nblk = (a.L + 63) / 64;
  const int nwork = a.B * a.H * nblk;
  const dim3 grid((unsigned)((nwork + 3) / 4));
  if (dtype == AFA_BF16)
    hipLaunchKernelGGL((afa_krot_kernel<AFA_BF16, D>), grid, dim3(256), 0, stream, a, (unsigned short*)krot, nb2,
                       nblk, nwork, zero, nzero);
  else
    hipLaunchKernelGGL((afa_krot_kernel<AFA_F16, D>), grid, dim3(256), 0, stream, a, (unsigned short*)krot, nb2,
                       nblk, nwork, zero, nzero);
}

hipError_t krot_launch(int dtype, int head_dim, FwdArgs& a, void* krot, float* nb2, hipStream_t stream, int* zero,
                       int nzero) {
  if (krot == nullptr || nb2 == nullptr) return hipErrorInvalidValue;
  switch (head_dim) {
    case 32: krot_launch_d<32>(dtype, a, krot, nb2, stream, zero, nzero); break;
    case 48: krot_launch_d<48>(dtype, a, krot, nb2, stream, zero, nzero); break;
    case 64: krot_launch_d<64>(dtype, a, krot, nb2, stream, zero, nzero); break;
    case 96: krot_launch_d<96>(dtype, a, krot, nb2, stream, zero, nzero); break;
    case 128: krot_launch_d<128>(dtype, a, krot, nb2, stream, zero, nzero); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  a.k = krot;
  a.k_l = head_dim;
  a.k_h = (int64_t)a.L * head_dim;
  a.k_b = (int64_t)a.H * a.L * head_dim;
  a.kbm = nb2;
  a.nkb = (a.L + 63) / 64;
  return hipSuccess;
}

hipError_t d64_fwd_launch(int dtype, FwdArgs a, bool exact, hipStream_t stream) {
  a.q_scale = 0.125f;  // 1/sqrt(64), exact in any binary format
  a.w_unscale = 1.0f;
  a.nb_lim = fast_rho_lim(1.0);  // s is the MFMA output itself
  const bool rot = a.rc != nullptr;
  if (dtype == AFA_BF16) {
    if (exact) return rot ? launch_d64<AFA_BF16, true, true>(a, stream) : launch_d64<AFA_BF16, true, false>(a, stream);
    return rot ? launch_d64<AFA_BF16, false, true>(a, stream) : launch_d64<AFA_BF16, false, false>(a, stream);
  }
  if (exact) return rot ? launch_d64<AFA_F16, true, true>(a, stream) : launch_d64<AFA_F16, true, false>(a, stream);
  return rot ? launch_d64<AFA_F16, false, true>(a, stream) : launch_d64<AFA_F16, false, false>(a, stream);
}

}  // namespace afa
