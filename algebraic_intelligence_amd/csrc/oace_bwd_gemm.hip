// Hand-written MFMA GEMMs of the fused Linear + OACE backward (src/kernels/pallas_oace.py:212-269):
//   dh = dz W^T  (rows x d_model; the contraction runs over the whole vocabulary, so it is split
//                 into parts whose fp32 partials a second kernel adds in part order)
//   dW = h^T dz  (d_model x vocab in W's layout; the contraction runs over the rows)
// for bf16 / fp16 operands with fp32 accumulation, each result rounded once to the element type.
//
// One kernel template: D[n][m] = sum_k A[m][k] B[n][k] over 256 (m) x 128 WN (n) tiles, waves
// of 64 x 128, each a 2 x 4 grid of 32x32x16 MFMA blocks (Cfg below: WN = 1, four waves and two
// workgroups per CU, for a short contraction; WN = 2, eight waves and one workgroup per CU, for a
// long one).  Each operand is read from memory in one of two orientations:
//   K-contiguous (KC): element (r, k) at p[r * ld + k]; the LDS tile holds 64-byte rows (32 k of
//     one r), 16-byte chunks swizzled by (r >> 2) & 3, and a fragment is one 16-byte read;
//   row-contiguous (MC): element (r, k) at p[k * ld + r]; the LDS tile holds the 32 k rows of the
//     tile's r range, 16-byte chunks swizzled by (k & 3) << 2 (conflict-free), and a fragment is
//     two ds_read_tr16_b64, which return 4 k rows of one r column per lane.
// Both give lane (r = lane & 31, group g = lane >> 5) the contraction rows 8g .. 8g+7 of each
// 16-row MFMA step, the MFMA operand layout.  K advances 32 per step through a 3- or 4-stage LDS
// ring filled by direct global -> LDS loads (LDS-DMA), one barrier per step; a last step shorter
// than 32 is loaded through registers, with the entries past the contraction set to zero, and
// taken first.  Rows and columns past the operand extents read the last valid row / 8-column chunk
// (data whose results are never stored).
//
//   dh: A = W^T (V x d, d contiguous) as MC over (m = d_model, k = vocab), B = dz (N x ldz) as KC;
//   dW, (d, V) layout: A = dz as MC over (m = vocab, k = rows), B = h as MC over (n = d_model);
//   dW, (V, d) layout: A = h as MC, B = dz as MC (D[v][k], d contiguous).
#include <algorithm>

#include "oace_common.h"

namespace afa {

namespace {

constexpr int GM = 256;  // A rows (m) per tile
constexpr int GK = 32;   // contraction per step
constexpr int OUT_PART = 0, OUT_ELEM = 1;
constexpr int SPITCH = GM * 2 + 16;  // staged output row pitch in bytes (16-byte aligned rows)
constexpr int LONG_K = 2048;  // contractions longer than this take the 256 x 256 tiles

// Tile configurations.  WN = 1: 256 x 128 tiles, 4 waves, a 3-stage ring of 24 KB stages (two
// workgroups per CU).  WN = 2: 256 x 256 tiles, 8 waves, a 4-stage ring of 32 KB stages (one
// workgroup per CU): half the operand bytes per MFMA and a prefetch three steps deep.
template <int WN>
struct Cfg {
  static constexpr int NT = 256 * WN;  // threads
  static constexpr int NW = 4 * WN;    // waves: 4 along m (64 rows each) x WN along n (128 each)
  static constexpr int TN = 128 * WN;  // B rows (n) per tile
  static constexpr int NST = WN == 1 ? 3 : 4;  // a 5th stage for WN = 2 measured no faster
  static constexpr int A_BYTES = GM * GK * 2;
  static constexpr int B_BYTES = TN * GK * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_LOADS = A_BYTES / (NT * 16);  // 16-byte loads per thread and step
  static constexpr int B_LOADS = B_BYTES / (NT * 16);
  static constexpr int LOADS = A_LOADS + B_LOADS;
  static constexpr int LDS = NST * STAGE;
  static constexpr int CUS_SLOTS = WN == 1 ? 2 : 1;  // workgroups per CU
  static_assert(128 * SPITCH <= LDS, "128 staged output rows must fit the ring");
  static_assert(NST - 2 <= 2, "wait_steps is given at most two later steps");
};

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

struct BgArgs {
  const unsigned short* a;  // A operand, m x K
  int64_t lda;
  int am;
  const unsigned short* b;  // B operand, n x K
  int64_t ldb;
  int bn;
  int K, kpart, parts, mt, nt;
  unsigned short* out;  // OUT_ELEM: D[n][m] at out[n * ldo + m]
  int64_t ldo;
  int own;      // columns per tile that the tile stores (256; 248 for rows that are not dword aligned)
  float* part;  // OUT_PART: fp32 partials, lane-major
};

template <int DT>
__device__ __forceinline__ f32x16_t bg_mma(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == AFA_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// Byte offset in an operand's stage of (tile row, logical 16-byte chunk): KC rows are the R
// operand rows (64 bytes: 4 chunks of k); MC rows are the 32 k rows (R * 2 bytes).
template <bool MC, int R>
__device__ __forceinline__ int bg_off(int row, int c) {
  if constexpr (MC) return row * (R * 2) + ((c ^ ((row & 3) << 2)) << 4);
  else return row * 64 + ((c ^ ((row >> 2) & 3)) << 4);
}

// (tile row, logical chunk) of the 16-byte slot s (physical position s * 16 of the stage).
template <bool MC, int R>
__device__ __forceinline__ void bg_slot(int s, int& row, int& c) {
  if constexpr (MC) {
    constexpr int CPR = R / 8;
    row = s / CPR;
    c = (s % CPR) ^ ((row & 3) << 2);
  } else {
    row = s >> 2;
    c = (s & 3) ^ ((row >> 2) & 3);
  }
}

// Element offset (from the tile's origin: operand row r0, contraction k0) of slot (row, c);
// out-of-range operand rows / chunks read the last valid one.
template <bool MC>
__device__ __forceinline__ int64_t bg_elem(int row, int c, int r0, int rows, int64_t ld) {
  if constexpr (MC) {
    const int col = min(r0 + 8 * c, ((rows + 7) >> 3) * 8 - 8) - r0;
    return (int64_t)row * ld + col;
  } else {
    return (int64_t)(min(r0 + row, rows - 1) - r0) * ld + 8 * c;
  }
}

// Fragment (32 operand rows from blk * 32, contraction rows 16 kk + 8 g .. + 7) of a stage.
template <bool MC, int R>
__device__ __forceinline__ u32x4_t bg_frag(const unsigned char* st, int blk, int kk, int lane) {
  const int l32 = lane & 31, g = lane >> 5;
  if constexpr (MC) {
    const int l16 = lane & 15, m16 = (lane >> 4) & 1;
    u32x4_t f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 16 * kk + 8 * g + 4 * hh + (l16 >> 2);
      const int c = blk * 4 + m16 * 2 + ((l16 & 3) >> 1);
      const unsigned char* p = st + bg_off<true, R>(row, c) + (l16 & 1) * 8;
      const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
      const u32x2_t w = __builtin_bit_cast(u32x2_t, v);
      f[2 * hh] = w[0];
      f[2 * hh + 1] = w[1];
    }
    return f;
  } else {
    return *(const u32x4_t*)(st + bg_off<false, R>(blk * 32 + l32, 2 * kk + g));
  }
}

// The 16 bytes of slot (row, c) for a step starting at contraction k0 whose entries at k >= k1
// are zero (register path of a short last step).
template <bool MC>
__device__ __forceinline__ u32x4_t bg_masked(const unsigned short* p, int64_t ld, int r0, int rows, int k0, int k1,
                                             int row, int c) {
  u32x4_t v = {0u, 0u, 0u, 0u};
  const unsigned short* src = p + bg_elem<MC>(row, c, r0, rows, ld);
  if constexpr (MC) {
    if (k0 + row < k1) v = *(const u32x4_t*)(src + (int64_t)k0 * ld);
  } else {
    const int k = k0 + 8 * c;
    if (k + 8 <= k1) {
      v = *(const u32x4_t*)(src + k0);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k + u < k1) {
          const unsigned e = src[k0 + u];
          v[u >> 1] |= e << (16 * (u & 1));
        }
    }
  }
  return v;
}

}  // namespace

// Waits until the direct loads of at most `later` steps (0..2) issued after the one needed remain.
template <int LOADS>
__device__ __forceinline__ void wait_steps(int later) {
  if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * LOADS));
  else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS));
  else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
}

template <int DT, bool A_MC, bool B_MC, int OUT, int WN>
__global__ __launch_bounds__(256 * WN) __attribute__((amdgpu_waves_per_eu(2, 2)))
void oace_bwd_gemm_kernel(const BgArgs a) {
  using C = Cfg<WN>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[C::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, wn = wave >> 2;
  const int l32 = lane & 31, g = lane >> 5;

  // Workgroups that share an operand slice run consecutively on one XCD (block b runs on XCD
  // b mod 8), each XCD taking an equal contiguous run of work items.  With parts: items in
  // (part, n tile, m tile) order, so that the tiles of one contraction part share both
  // operands' slices.  Without: the n tiles of one m tile (its A slice), m tiles in order, so
  // that neighbouring tiles -- which share the 128-byte lines at the ends of their output row
  // segments when rows are not 128-byte aligned -- write them through the same L2.
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  int part, mi, ni;
  if (a.parts > 1) {
    const int tiles = a.mt * a.nt, ipx = (a.parts * tiles + 7) / 8;  // items per XCD
    const int item = xcd * ipx + j;
    if (j >= ipx || item >= a.parts * tiles) return;
    part = item / tiles;
    mi = (item % tiles) % a.mt;
    ni = (item % tiles) / a.mt;
  } else {
    const int mpx = (a.mt + 7) / 8;  // m tiles per XCD
    part = 0;
    mi = xcd * mpx + j / a.nt;
    ni = j % a.nt;
    if (j / a.nt >= mpx || mi >= a.mt) return;
  }
  const int m0 = mi * a.own, n0 = ni * C::TN;
  const int k_lo = part * a.kpart, k_hi = min(k_lo + a.kpart, a.K);
  const int T = (k_hi - k_lo) / GK;
  const bool tail = (k_hi - k_lo) % GK != 0;

  // per-thread offsets of the direct loads (constant over the steps), wave-uniform bases
  uint32_t aoff[C::A_LOADS], boff[C::B_LOADS];
#pragma unroll
  for (int i = 0; i < C::A_LOADS; ++i) {
    int row, c;
    bg_slot<A_MC, GM>(C::NT * i + tid, row, c);
    aoff[i] = (uint32_t)bg_elem<A_MC>(row, c, m0, a.am, a.lda) * 2u;
  }
#pragma unroll
  for (int i = 0; i < C::B_LOADS; ++i) {
    int row, c;
    bg_slot<B_MC, C::TN>(C::NT * i + tid, row, c);
    boff[i] = (uint32_t)bg_elem<B_MC>(row, c, n0, a.bn, a.ldb) * 2u;
  }
  const char* abase = (const char*)(a.a + (A_MC ? (int64_t)k_lo * a.lda + m0 : (int64_t)m0 * a.lda + k_lo));
  const char* bbase = (const char*)(a.b + (B_MC ? (int64_t)k_lo * a.ldb + n0 : (int64_t)n0 * a.ldb + k_lo));
  const int64_t astep = A_MC ? (int64_t)GK * a.lda * 2 : GK * 2;
  const int64_t bstep = B_MC ? (int64_t)GK * a.ldb * 2 : GK * 2;
  auto issue = [&](int t) {
    unsigned char* st = lds + (t % C::NST) * C::STAGE;
    const char* ab = abase + t * astep;
    const char* bb = bbase + t * bstep;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) lds_dma16(ab, aoff[i], st + (C::NT * i + wave * 64) * 16);
#pragma unroll
    for (int i = 0; i < C::B_LOADS; ++i)
      lds_dma16(bb, boff[i], st + C::A_BYTES + (C::NT * i + wave * 64) * 16);
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[vb][nb][e] = 0.f;

  auto compute = [&](const unsigned char* st) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4_t af[2], bf[4];
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) af[vb] = bg_frag<A_MC, GM>(st, wm * 2 + vb, kk, lane);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) bf[nb] = bg_frag<B_MC, C::TN>(st + C::A_BYTES, wn * 4 + nb, kk, lane);
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[vb][nb] = bg_mma<DT>(af[vb], bf[nb], acc[vb][nb]);
    }
  };

  // prologue: the first NST-1 steps in flight
#pragma unroll
  for (int t = 0; t < C::NST - 1; ++t)
    if (t < T) issue(t);
  if (tail) {
    // the short last step [kt, k_hi), taken first (no accumulator is live yet), through
    // registers into the last stage, which the prologue's loads do not touch
    const int kt = k_lo + T * GK;
    unsigned char* st = lds + (C::NST - 1) * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) {
      int row, c;
      const int s = C::NT * i + tid;
      bg_slot<A_MC, GM>(s, row, c);
      const unsigned short* p = a.a + (A_MC ? (int64_t)m0 : (int64_t)m0 * a.lda);
      *(u32x4_t*)(st + s * 16) = bg_masked<A_MC>(p, a.lda, m0, a.am, kt, k_hi, row, c);
    }
#pragma unroll
    for (int i = 0; i < C::B_LOADS; ++i) {
      int row, c;
      const int s = C::NT * i + tid;
      bg_slot<B_MC, C::TN>(s, row, c);
      const unsigned short* p = a.b + (B_MC ? (int64_t)n0 : (int64_t)n0 * a.ldb);
      *(u32x4_t*)(st + C::A_BYTES + s * 16) = bg_masked<B_MC>(p, a.ldb, n0, a.bn, kt, k_hi, row, c);
    }
    __syncthreads();
    compute(st);
    // the last stage is next written by the load of step NST-1 (issued in step 0) or by the
    // epilogue: both after a barrier that follows this read
    if (T == 0) __syncthreads();
  }
  if (T > 0) {
    wait_steps<C::LOADS>(min(T, C::NST - 1) - 1);
    __syncthreads();
    for (int t = 0; t < T; ++t) {
      // the buffer of step t+NST-1 was last read in step t-1, before the previous barrier
      if (t + C::NST - 1 < T) issue(t + C::NST - 1);
      compute(lds + (t % C::NST) * C::STAGE);
      // own loads of step t+1 complete (only later steps' may remain), then publish them
      wait_steps<C::LOADS>(min(T - 1, t + C::NST - 1) - (t + 1));
      __syncthreads();
    }
  }

  // ---- epilogue.  Element e of acc[vb][nb]: m = m0 + 64 wm + 32 vb + 8 (e >> 2) + 4 g + (e & 3),
  // n = n0 + 128 wn + 32 nb + l32.
  if constexpr (OUT == OUT_PART) {
    // lane-major partial: per wave, 32 groups of 4 values for the 64 lanes (every store covers
    // 1 KB); oace_bwd_gemm_sum_kernel reads the same layout
    const int tile = ni * a.mt + mi;
    f32x4_t* dst = (f32x4_t*)a.part + ((((int64_t)part * a.mt * a.nt + tile) * C::NW + wave) * 32) * 64 + lane;
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4_t w;
#pragma unroll
          for (int u = 0; u < 4; ++u) w[u] = acc[vb][nb][4 * q + u];
          dst[((vb * 4 + nb) * 4 + q) * 64] = w;
        }
  } else {
    // the tile in the element type through LDS (the idle ring), 128 n rows per round, then
    // whole row segments
#pragma unroll
    for (int h = 0; h < WN; ++h) {
      if (wn == h) {
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              u32x2_t w;
              w[0] = Elem<DT>::pack(acc[vb][nb][4 * q], acc[vb][nb][4 * q + 1]);
              w[1] = Elem<DT>::pack(acc[vb][nb][4 * q + 2], acc[vb][nb][4 * q + 3]);
              const int ml = wm * 64 + vb * 32 + q * 8 + 4 * g, nl = nb * 32 + l32;
              *(u32x2_t*)(lds + nl * SPITCH + ml * 2) = w;
            }
      }
      __syncthreads();
      // Row n of the output.  A tile writes whole dwords: those whose first element it owns
      // (columns [m0, m0 + own)); when rows are not dword aligned (an odd row stride, such as
      // a (d_model, vocab) weight's), own = 248 < 256 and the tile's last owned dword takes its
      // second element from the 8 columns it computes past them.  Sub-dword stores are slow
      // (several times the cost of the whole row segment): only an element whose dword starts in
      // the previous row or ends in the next one (at most one at each end of a row) is stored
      // alone.  16-byte stores from the first 16-byte aligned element, then, in a second pass,
      // the at most 3 + 3 dwords before and after them: the cost of a store instruction hardly
      // depends on how many lanes it has, so those go 32 rows to an instruction.
      struct RowSeg {
        unsigned short* rowp;  // element m at rowp + m
        int s0, e1, hb, nbody;
      };
      auto seg = [&](int n) {
        RowSeg q;
        q.rowp = a.out + (int64_t)n * a.ldo;
        auto half = [&](int m) { return (int)(((uint32_t)(uintptr_t)(q.rowp + m) >> 1) & 1u); };
        const int own_end = min(m0 + a.own, a.am);
        q.s0 = m0 + half(m0);
        q.e1 = own_end == a.am ? a.am - half(a.am) : own_end + half(own_end);
        q.hb = q.s0 + (int)(((16u - ((uint32_t)(uintptr_t)(q.rowp + q.s0) & 15u)) & 15u) >> 1);
        q.nbody = q.e1 > q.hb ? (q.e1 - q.hb) >> 3 : 0;
        return q;
      };
#pragma unroll
      for (int i = 0; i < 128 * (GM / 8) / C::NT; ++i) {
        const int idx = tid + C::NT * i, r = idx / (GM / 8), c = idx % (GM / 8);
        const int n = n0 + 128 * h + r;
        if (n < a.bn) {
          const RowSeg q = seg(n);
          if (c < q.nbody) {
            const unsigned char* srow = lds + r * SPITCH;  // staged element m at srow + 2 (m - m0)
            const int e = q.hb - m0 + 8 * c;               // first staged index of this chunk
            u32x4_t v;
            if ((e & 7) == 0) {
              v = *(const u32x4_t*)(srow + 2 * e);
            } else if ((e & 1) == 0) {
              const unsigned* w = (const unsigned*)(srow + 2 * e);
#pragma unroll
              for (int u = 0; u < 4; ++u) v[u] = w[u];
            } else {
              const unsigned* w = (const unsigned*)(srow + 2 * (e - 1));
              unsigned x[5];
#pragma unroll
              for (int u = 0; u < 5; ++u) x[u] = w[u];
#pragma unroll
              for (int u = 0; u < 4; ++u) v[u] = __builtin_amdgcn_alignbit(x[u + 1], x[u], 16);
            }
            *(u32x4_t*)(q.rowp + m0 + e) = v;
          }
        }
      }
      // slots 0..5: the dwords before and after the chunks; 6 and 7: the elements stored alone
#pragma unroll
      for (int i = 0; i < 128 * 8 / C::NT; ++i) {
        const int idx = tid + C::NT * i, r = idx >> 3, c = idx & 7;
        const int n = n0 + 128 * h + r;
        if (n < a.bn) {
          const RowSeg q = seg(n);
          const unsigned char* srow = lds + r * SPITCH;
          auto st16 = [&](int m) { return (unsigned)*(const unsigned short*)(srow + 2 * (m - m0)); };
          const int hend = min(q.hb, q.e1), tstart = max(q.hb + 8 * q.nbody, hend);
          const int nhead = (hend - q.s0) >> 1, ndw = nhead + max(0, (q.e1 - tstart) >> 1);
          if (c < ndw) {
            const int m = c < nhead ? q.s0 + 2 * c : tstart + 2 * (c - nhead);
            *(unsigned*)(q.rowp + m) = st16(m) | (st16(m + 1) << 16);
          } else if (c == 6) {
            if (m0 == 0 && q.s0 == 1) q.rowp[0] = (unsigned short)st16(0);
          } else if (c == 7) {
            if (min(m0 + a.own, a.am) == a.am && q.e1 == a.am - 1 && a.am - 1 >= q.s0)
              q.rowp[a.am - 1] = (unsigned short)st16(a.am - 1);
          }
        }
      }
      if (h + 1 < WN) __syncthreads();
    }
  }
}

// D[n][m] = sum over parts of the lane-major fp32 partials (in part order), rounded once to the
// element type; one thread per 4 consecutive m of one n, the parts' loads four at a time.
template <int DT, int WN>
__global__ __launch_bounds__(256) void oace_bwd_gemm_sum_kernel(const f32x4_t* part, int parts, int mt, int nt, int M,
                                                                int N, unsigned short* out, int64_t ldo) {
  using C = Cfg<WN>;
  const int64_t per_part = (int64_t)mt * nt * C::NW * 32 * 64;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= per_part) return;
  const int lane = (int)(i & 63), grp = (int)((i >> 6) & 31);
  const int wave = (int)((i >> 11) % C::NW), tile = (int)((i >> 11) / C::NW);
  const int mi = tile % mt, ni = tile / mt;
  const int vb = grp >> 4, nb = (grp >> 2) & 3, q = grp & 3;
  const int m = mi * GM + (wave & 3) * 64 + vb * 32 + q * 8 + 4 * (lane >> 5);
  const int n = ni * C::TN + (wave >> 2) * 128 + nb * 32 + (lane & 31);
  if (n >= N || m >= M) return;
  f32x4_t s = part[i];
  int p = 1;
  for (; p + 4 <= parts; p += 4) {
    const f32x4_t x0 = part[p * per_part + i], x1 = part[(p + 1) * per_part + i];
    const f32x4_t x2 = part[(p + 2) * per_part + i], x3 = part[(p + 3) * per_part + i];
    s += x0;
    s += x1;
    s += x2;
    s += x3;
  }
  for (; p < parts; ++p) s += part[p * per_part + i];
  unsigned short* o = out + (int64_t)n * ldo + m;
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (m + u < M) Elem<DT>::store(o, u, s[u]);
}

// ------------------------------------------------------------------------------ host side
namespace {

// Tile configuration of a GEMM: 256 x 256 tiles for a long contraction (split into parts when
// the tiles are few: fewer partials), 256 x 128 tiles with two workgroups per CU for a short
// one (their loops overlap each other's prologue and epilogue).
int wn_of(const OaceGemm& g) { return g.k > LONG_K ? 2 : 1; }

int tiles_m(int64_t m, int own = GM) { return (int)((m + own - 1) / own); }
int tiles_n(int64_t n, int wn) { return (int)((n + 128 * wn - 1) / (128 * wn)); }

// Contraction per part for a split into about `parts` parts (a multiple of the step).
int64_t kpart_of(int64_t K, int parts) {
  const int64_t kp = (K + parts - 1) / parts;
  return std::max<int64_t>(GK, (kp + GK - 1) / GK * GK);
}

template <int DT, bool A_MC, bool B_MC, int OUT, int WN>
hipError_t bg_launch(const BgArgs& g, hipStream_t st) {
  const unsigned grid = (unsigned)(g.parts > 1 ? 8 * ((g.parts * g.mt * g.nt + 7) / 8) : 8 * g.nt * ((g.mt + 7) / 8));
  hipLaunchKernelGGL((oace_bwd_gemm_kernel<DT, A_MC, B_MC, OUT, WN>), dim3(grid), dim3(256 * WN), 0, st, g);
  return hipGetLastError();
}

template <int DT, int WN>
hipError_t bg_run(const OaceGemm& g, BgArgs& b, hipStream_t st) {
  if (b.parts > 1) {
    if (!g.a_mc || g.b_mc) return hipErrorNotSupported;
    hipError_t e = bg_launch<DT, true, false, OUT_PART, WN>(b, st);
    if (e != hipSuccess) return e;
    const int64_t threads = (int64_t)b.mt * b.nt * Cfg<WN>::NW * 32 * 64;
    hipLaunchKernelGGL((oace_bwd_gemm_sum_kernel<DT, WN>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const f32x4_t*)b.part, b.parts, b.mt, b.nt, b.am, b.bn, b.out, b.ldo);
    return hipGetLastError();
  }
  if (g.a_mc && !g.b_mc) return bg_launch<DT, true, false, OUT_ELEM, WN>(b, st);
  if (g.a_mc && g.b_mc) return bg_launch<DT, true, true, OUT_ELEM, WN>(b, st);
  return hipErrorNotSupported;
}

}  // namespace

bool oace_gemm_fits(const OaceGemm& g) {
  // 16-byte aligned operand rows, and 32-bit per-lane byte offsets within a tile
  auto fits = [](const void* p, int64_t ld, bool mc, int rows_per_tile) {
    if (((uintptr_t)p & 15u) != 0 || ld % 8 != 0 || ld <= 0) return false;
    const int64_t span = mc ? (int64_t)(GK - 1) * ld + 256 : (int64_t)(rows_per_tile - 1) * ld + GK;
    return span * 2 < ((int64_t)1 << 32);
  };
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.m >= (1 << 30) || g.n >= (1 << 30) || g.k >= (1 << 30)) return false;
  return fits(g.a, g.lda, g.a_mc, GM) && fits(g.b, g.ldb, g.b_mc, 256);
}

int oace_gemm_parts(const OaceGemm& g, int cus) {
  // The contraction is split into the part count that minimises a model of the time: the
  // rounds of workgroups over the CU slots, each as long as one tile over its share of the
  // contraction, plus writing and reading the parts' fp32 partials.  Rates: a workgroup of
  // 256 x 256 tiles (one per CU) at 6 TFLOP/s, 256 x 128 tiles (two per CU) at 3 TFLOP/s each;
  // partials at 5 TB/s.  Parts hold at least 1024 of the contraction.  Part counts of 8 and
  // more are multiples of 8: at N = 512 (6 tiles), 42 parts -- 32 workgroups on each XCD's 32
  // CUs -- made dh 56.1 us against 51.4 us for 40 (30 per XCD), measured twice on one box.
  const int wn = wn_of(g);
  const int64_t tiles = (int64_t)tiles_m(g.m) * tiles_n(g.n, wn);
  const int64_t slots = (int64_t)cus * (wn == 1 ? Cfg<1>::CUS_SLOTS : Cfg<2>::CUS_SLOTS);
  const double t_tile = 2.0 * GM * 128.0 * wn * (double)g.k / (wn == 1 ? 3e12 : 6e12);
  const double t_part = 2.0 * (double)g.m * (double)g.n * 4.0 / 5e12;
  const int pmax = (int)std::min<int64_t>(64, std::max<int64_t>(1, g.k / 1024));
  int best = 1;
  double best_t = 0.0;
  for (int p = 1; p <= pmax; ++p) {
    const double rounds = (double)((tiles * p + slots - 1) / slots);
    const double t = rounds * t_tile / p + (p > 1 ? p * t_part : 0.0);
    if (p >= 8 && p % 8 != 0) continue;
    if (p == 1 || t < best_t) {
      best = p;
      best_t = t;
    }
  }
  return best <= 1 ? 1 : (int)((g.k + kpart_of(g.k, best) - 1) / kpart_of(g.k, best));
}

size_t oace_gemm_part_bytes(const OaceGemm& g, int parts) {
  const int wn = wn_of(g);
  return parts > 1 ? (size_t)parts * tiles_m(g.m) * tiles_n(g.n, wn) * GM * 128 * wn * sizeof(float) : 0;
}

hipError_t oace_gemm(int dtype, const OaceGemm& g, int parts, float* part, hipStream_t st) {
  if (!oace_gemm_fits(g) || (dtype != AFA_BF16 && dtype != AFA_F16)) return hipErrorNotSupported;
  const int wn = wn_of(g);
  BgArgs b = {};
  b.a = (const unsigned short*)g.a;
  b.lda = g.lda;
  b.am = (int)g.m;
  b.b = (const unsigned short*)g.b;
  b.ldb = g.ldb;
  b.bn = (int)g.n;
  b.K = (int)g.k;
  // columns stored per tile: 248 when the output rows are not dword aligned (overlapping tiles)
  b.own = parts <= 1 && (((g.ldo & 1) != 0) || (((uintptr_t)g.out & 2u) != 0)) ? GM - 8 : GM;
  b.mt = tiles_m(g.m, b.own);
  b.nt = tiles_n(g.n, wn);
  b.parts = parts > 1 ? parts : 1;
  b.kpart = b.parts > 1 ? (int)kpart_of(g.k, b.parts) : (int)g.k;
  if (b.parts > 1 && (int64_t)(b.parts - 1) * b.kpart >= g.k) return hipErrorInvalidValue;
  b.out = (unsigned short*)g.out;
  b.ldo = g.ldo;
  b.part = part;
  if (dtype == AFA_BF16) return wn == 1 ? bg_run<AFA_BF16, 1>(g, b, st) : bg_run<AFA_BF16, 2>(g, b, st);
  return wn == 1 ? bg_run<AFA_F16, 1>(g, b, st) : bg_run<AFA_F16, 2>(g, b, st);
}

}  // namespace afa
