// Fused AFA forward with 32 queries per wave and several waves per SIMD, for head_dim 64 and 128
// (bf16 / fp16 operands, fp32 accumulate).  Same contract as afa_fwd_mfma.hip
// (src/kernels/pallas_afa.py:52-151).  A score costs 4 D MFMA FLOPs against ~7.5 VALU slots of the
// rho^8 chain, row sum and pack; one wave's MFMAs and VALU work barely overlap, so the kernel is
// shaped for overlap ACROSS waves: while one wave runs its rho^8 chain the other waves of its
// SIMD keep the matrix pipe busy.
//
//   * a wave owns 32 queries; unit u (32 keys) first issues S(u+1) = K Q^T (D/16 x 32x32x16),
//     then rho^8 of S(u), then O += V^T P(u) (D/16 x 32x32x16).  The K and V fragments live only
//     around their own MFMAs and S alternates between two register sets, which keeps a wave at
//     <= 256 VGPRs (D = 128: two waves per SIMD) or <= 168 (D = 64: three waves per SIMD);
//   * K and V reach LDS by direct global -> LDS loads in tiles of 32 keys (rows of D/8 16-byte
//     chunks): K chunk c of row r at c ^ k_key(r) (r & 15 for D = 128, (r >> 1) & 7 for D = 64:
//     conflict-free fragment reads); V chunk c at c ^ ((r & 3) << 2) for D = 128 and
//     c ^ (((r >> 1) & 1) << 2) for D = 64 (conflict-free ds_read_tr16_b64 of 4-key column
//     slices, which give the PV MFMA's A operand in the key order of the S^T accumulator);
//   * LDS is a ring of NB tiles: iteration u issues tile u + NB - 1 into the buffer of tile u - 1
//     and waits only for its own loads of tile u + 1; one barrier per tile;
//   * q is scaled by 1/sqrt(D) (and Cayley-rotated in fp32 when rotary tables are given) as it is
//     loaded; k arrives rotated (afa_krot_kernel, once per call).  At D = 128, 1/sqrt(128) =
//     2^-4 sqrt(2): 2^-4 is folded into q exactly, and sqrt(2) is either evaluated inside
//     (rho/sqrt 2)^8 = rho^8/16 (bf16 fast path: weights and sink carry 1/16) or formed
//     explicitly (two-branch path, fp16);
//   * masks only on units that cross the causal diagonal or valid_len; workgroups heaviest first;
//   * head_dim 32, 48 and 96 run as 64, 64 and 128: the padding chunks of every LDS row are
//     loaded from a zero chunk in device memory (so every lane of every direct load is active and
//     the per-tile load counts stay exact), q's padding features are zero, and only the head_dim
//     output features are stored.  1/sqrt(D) is a power of two folded into q exactly times an
//     fp32 factor applied to the score: s = (q 2^-k . k) * (fl(1/sqrt D) 2^k) rounds like the
//     reference's (q . k) * fl(1/sqrt D).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "afa_common.h"
#include "afa_launch.h"

namespace afa {

namespace {

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

template <int DT>
__device__ __forceinline__ f32x16_t mma16(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == AFA_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// 8 consecutive q features (one 16-byte chunk), scaled, and Cayley-rotated in fp32 first when
// ROT: pairs (x0, x1) -> (c x0 - s x1, s x0 + c x1), one rounding to the element type.
template <int DT, bool ROT>
__device__ __forceinline__ u32x4_t q_chunk(u32x4_t w, const float* cc, const float* ss, float scale) {
#pragma clang fp contract(off)
  u32x4_t r;
  f32x4_t c = {1.f, 1.f, 1.f, 1.f}, s = {0.f, 0.f, 0.f, 0.f};
  if constexpr (ROT) {
    c = *(const f32x4_t*)cc;
    s = *(const f32x4_t*)ss;
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = Elem<DT>::lo(w[p]), x1 = Elem<DT>::hi(w[p]);
    float y0 = x0, y1 = x1;
    if constexpr (ROT) {
      y0 = c[p] * x0 - s[p] * x1;
      y1 = s[p] * x0 + c[p] * x1;
    }
    r[p] = Elem<DT>::pack(y0 * scale, y1 * scale);
  }
  return r;
}

__device__ __forceinline__ float tree16x(const float (&p)[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[2 * i] + p[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[2 * i] + a[2 * i + 1];
  a[0] = a[0] + a[1];
  a[2] = a[2] + a[3];
  return a[0] + a[2];
}

// K chunk c of tile row r sits at c ^ k_key(r).  At DP = 128 a 256-byte row is one bank period and
// r & 15 spreads the 16 rows of a fragment read's pass (16 lanes x 16 bytes) over its 16 slots; at
// DP = 64 an even and an odd row share a period, and (r >> 1) & 7 takes all 8 positions over the
// even rows and over the odd ones (r & 7 took them over 8 rows only: 2-way conflicts).
template <int DP>
__device__ __forceinline__ int k_key(int r) {
  if constexpr (DP == 128) return r & 15;
  else return (r >> 1) & 7;
}

template <int D>
__device__ __forceinline__ int v_swizzle(int r, int c) {
  if constexpr (D == 128) return c ^ ((r & 3) << 2);
  else return c ^ (((r >> 1) & 1) << 2);
}

template <int DP>
struct PipeShape {
  static constexpr int NB = 4;                  // ring of tile buffers
  static constexpr int WAVES_PER_EU = DP == 128 ? 2 : 3;
};

constexpr int padded_dim(int d) { return d <= 64 ? 64 : 128; }

}  // namespace

// Source of the padding chunks of LDS rows (head_dim 32, 48, 96).
__device__ __attribute__((aligned(16))) unsigned int afa_pipe_zero_chunk[4];

// SM: 0 = s as formed (q carries 1/sqrt(D) exactly, D = 64);
//     1 = s = sqrt(2) x evaluated as (rho/sqrt 2)^8 = rho^8/16 (weights and sink carry 1/16);
//     2 = s = a.s_mult x formed explicitly.
// Key range of one workgroup: tiles [t0, t1) of its query block, part `part` of `nparts`.
struct PipePart {
  int t0 = 0, t1 = 1 << 30, part = 0, nparts = 1;
};

// 32-key tiles of query block q for the split plan (valid_len = L).
__device__ __forceinline__ int split_block_tiles(const FwdArgs& a, int q) {
  return a.causal ? (min(a.L, 128 * (q + 1)) + 31) / 32 : (a.L + 31) / 32;
}

// Work item of the split grid: the items of one (query block, part) rank are the B * H heads
// (grouped per XCD as in block_item), ranks run from the last query block down (the longest
// parts first); a block from ks_q0 on has ceil(tiles / ks_tiles) parts of an even number of tiles
// each but the last.
__device__ __forceinline__ void split_item(const FwdArgs& a, int bid, int& bh, int& qblk, PipePart& pp) {
  const int BH = a.B * a.H;
  int rank;
  if ((BH & 7) == 0) {
    const int hq = BH >> 3, j = bid >> 3;
    bh = (bid & 7) * hq + j % hq;
    rank = j / hq;
  } else {
    bh = bid % BH;
    rank = bid / BH;
  }
  qblk = 0;
  pp = PipePart();
  for (int q = a.nqb - 1; q >= 0; --q) {
    const int nt = split_block_tiles(a, q);
    const int np = q < a.ks_q0 ? 1 : (nt + a.ks_tiles - 1) / a.ks_tiles;
    if (rank < np) {
      qblk = q;
      pp.part = rank;
      pp.nparts = np;
      pp.t0 = 2 * ((rank * nt) / (2 * np));
      pp.t1 = rank + 1 == np ? nt : 2 * (((rank + 1) * nt) / (2 * np));
      break;
    }
    rank -= np;
  }
}

// LDS tile of the pipelined kernels: 32 keys x the padded head dim.
template <int DP>
using PipeTile = unsigned short[32 * DP];

// Direct global -> LDS loads of key tile t (32 keys of K and of V) of one head into ring buffer
// buf = t % NB: slot s = tid + 256 i covers row s / CH, physical chunk s % CH; K chunk c of row r goes to
// c ^ k_key(r), V chunk c to v_swizzle; rows past L
// read zeros (buffer loads whose range ends with row L - 1) or, at head dims with padding
// chunks, row L - 1: finite data for masked keys.
template <int D>
__device__ __forceinline__ void pipe_issue_tile(const FwdArgs& a, PipeTile<padded_dim(D)>* lds_k,
                                                PipeTile<padded_dim(D)>* lds_v, const unsigned short* kp,
                                                const unsigned short* vp, int t, int buf) {
  constexpr int DP = padded_dim(D);
  constexpr int KT = 32;
  constexpr int NB = PipeShape<DP>::NB;
  constexpr int CH = DP / 8;
  constexpr int CHD = D / 8;
  constexpr int LPT = KT * CH / 256;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  unsigned short* kd = &lds_k[buf][0];
  unsigned short* vd = &lds_v[buf][0];
  if constexpr (CHD == CH) {
    // buffer loads: each resource runs from the tile's first row to the end of the head's row
    // L - 1, so rows past L read zeros (finite, masked keys) and nothing past the head is read;
    // each lane's offset is the same in every tile
    const uint32_t ks0 = __builtin_amdgcn_readfirstlane((uint32_t)(t * KT * (int)a.k_l) * 2u);
    const uint32_t vs0 = __builtin_amdgcn_readfirstlane((uint32_t)(t * KT * (int)a.v_l) * 2u);
    const i32x4_t ksrd = raw_buffer_srd_at(kp, (uint32_t)((a.L - 1) * (int)a.k_l + D) * 2u, ks0);
    const i32x4_t vsrd = raw_buffer_srd_at(vp, (uint32_t)((a.L - 1) * (int)a.v_l + D) * 2u, vs0);
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int s = tid + 256 * i, r = s / CH, pc = s % CH;
      const int lk = pc ^ k_key<DP>(r), lv = v_swizzle<DP>(r, pc);
      lds_dma16_buf(ksrd, (uint32_t)(r * (int)a.k_l + lk * 8) * 2u, kd + (256 * i + wave * 64) * 8);
      lds_dma16_buf(vsrd, (uint32_t)(r * (int)a.v_l + lv * 8) * 2u, vd + (256 * i + wave * 64) * 8);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int s = tid + 256 * i, r = s / CH, pc = s % CH;
    const int key = min(t * KT + r, a.L - 1);
    const int lk = pc ^ k_key<DP>(r), lv = v_swizzle<DP>(r, pc);
    // byte offsets within the head fit 32 bits (checked by the caller): a uniform base plus a
    // 32-bit lane offset per load
    const void* ks = (const void*)((const char*)kp + (uint32_t)(key * (int)a.k_l + lk * 8) * 2u);
    const void* vs = (const void*)((const char*)vp + (uint32_t)(key * (int)a.v_l + lv * 8) * 2u);
    if constexpr (CHD < CH) {
      if (lk >= CHD) ks = (const void*)afa_pipe_zero_chunk;
      if (lv >= CHD) vs = (const void*)afa_pipe_zero_chunk;
    }
    lds_dma16(ks, kd + (256 * i + wave * 64) * 8);
    lds_dma16(vs, vd + (256 * i + wave * 64) * 8);
  }
}

// Tile loop and epilogue of afa_fwd_pipe_kernel for one form of rho^8: FAST, the branch-free
// form (the wave's scores are all within the fast-rho bound), else the two-branch form.  The
// kernel instantiates both and each wave runs one, so the two loops get their own register
// allocation; the barriers count waves, not code locations.
template <int D, int DT, bool FAST, int SM>
__device__ __forceinline__ void pipe_body(const FwdArgs& a, PipeTile<padded_dim(D)>* lds_k,
                                          PipeTile<padded_dim(D)>* lds_v, const u32x4_t (&qf)[padded_dim(D) / 16],
                                          int bh, int qblk, const PipePart& pp) {
  constexpr int DP = padded_dim(D);      // LDS row and MFMA width
  constexpr int KT = 32;                 // keys per tile = one unit
  constexpr int NB = PipeShape<DP>::NB;
  constexpr int CH = DP / 8;             // 16-byte chunks per LDS row
  constexpr int CHD = D / 8;             // chunks that hold data
  constexpr int LPT = KT * CH / 256;     // direct loads per thread per tile, each of K and V
  constexpr int LOADS = 2 * LPT;
  constexpr int NK = DP / 16;            // 16-feature MFMA steps of S
  constexpr int NDB = DP / 32;           // 32-feature output blocks
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5, l16 = lane & 15, m16 = (lane >> 4) & 1;
  const int b = bh / a.H, h = bh % a.H;
  const int L = a.L, vlen = a.valid_len;
  const int q0_wg = qblk * 128, q0_w = q0_wg + wave * 32;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 128)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 32) : vlen;
  // this workgroup's key tiles [t_lo, t_hi): its part of the block's tiles (all of them unsplit)
  const int ntiles = (kend_wg + KT - 1) / KT;
  const int t_hi = min(pp.t1, ntiles), t_lo = min(pp.t0, t_hi);
  const int U = min(q0_w < L ? (kend_w + KT - 1) / KT : 0, t_hi);  // end of this wave's units
  const int qi = q0_w + l32;
  const unsigned short* kp = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
  const unsigned short* vp = (const unsigned short*)a.v + b * a.v_b + h * a.v_h;

  // tile t lives in ring buffer t % NB (t >= 0; NB is a power of two).  The callers pass the
  // buffer: a constant in the loop over aligned groups of NB tiles, so that every LDS address
  // there is a loop-invariant lane offset plus an immediate
  auto issue_tile = [&](int t, int buf) { pipe_issue_tile<D>(a, lds_k, lds_v, kp, vp, t, buf); };
  u32x4_t kf[NK];
  u32x4_t vf[NDB][2];
  auto read_kf = [&](int buf) {
    const unsigned short* base = &lds_k[buf][l32 * DP];
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) kf[kc] = *(const u32x4_t*)(base + (((2 * kc + g) ^ k_key<DP>(l32)) * 8));
  };
  auto read_vf = [&](int buf) {
    const unsigned short* tile = lds_v[buf];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int row = kk * 16 + hh * 8 + 4 * g + (l16 >> 2);
          const int col = db * 32 + m16 * 16 + 4 * (l16 & 3);
          const unsigned short* p = tile + row * DP + v_swizzle<DP>(row, col >> 3) * 8 + (col & 7);
          const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
          const u32x2_t w = __builtin_bit_cast(u32x2_t, v);
          f[2 * hh] = w[0];
          f[2 * hh + 1] = w[1];
        }
        vf[db][kk] = f;
      }
  };

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float rowsum = 0.f;
  f32x16_t sA, sB;

  // prologue: tiles t_lo .. t_lo+NB-2 in flight (issued by the kernel before its q loads); tile
  // t_lo resident; S(t_lo) in registers (t_lo is even, so S(u) is in sA for even u as in the loop)
  const int npro = min(t_hi - t_lo, NB - 1);
  if (npro == NB - 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS * (NB - 2)));
  else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  __syncthreads();
  if (t_lo < t_hi) {
    read_kf(t_lo & (NB - 1));
#pragma unroll
    for (int e = 0; e < 16; ++e) sA[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) sA = mma16<DT>(kf[kc], qf[kc], sA);
  }

  // unit u: S(u+1) on the MFMA pipe first, then P(u) = rho^8(S(u)) on the VALU, then O += V(u)^T P(u)
  auto unit = [&](int u, f32x16_t& scur, f32x16_t& snxt) {
    if (u >= U) return;
    if (u + 1 < U) {
      read_kf((u + 1) & (NB - 1));
#pragma unroll
      for (int e = 0; e < 16; ++e) snxt[e] = 0.f;
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) snxt = mma16<DT>(kf[kc], qf[kc], snxt);
    }
    __builtin_amdgcn_sched_barrier(0);
    float p[16];
    if constexpr (FAST) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = SM == 2 ? scur[r] * a.s_mult : scur[r];
        p[r] = SM == 1 ? rho8_fast_half(x) : rho8_fast(x);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = SM == 2 ? scur[r] * a.s_mult : scur[r];
        p[r] = SM == 1 ? rho8_exact_half(x) : rho8_exact(x);
      }
    }
    const int key0 = u * KT;
    if ((a.causal && key0 + 31 > q0_w) || key0 + 31 >= vlen) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = key0 + (r >> 2) * 8 + 4 * g + (r & 3);
        const bool keep = (j < vlen) && (!a.causal || j <= qi);
        p[r] = keep ? p[r] : 0.f;
      }
    }
    rowsum += tree16x(p);
    u32x4_t pk[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[kk][e] = Elem<DT>::pack(p[kk * 8 + 2 * e], p[kk * 8 + 2 * e + 1]);
    __builtin_amdgcn_sched_barrier(0);
    read_vf(u & (NB - 1));
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] = mma16<DT>(vf[db][kk], pk[kk], o[db]);
  };
  // The same unit where it is known to be one of the wave's units, to have a next one and to
  // need no mask: no branch and no select in its VALU stream (the guarded form's mask test is
  // if-converted into a compare and a select per score).
  auto clean_unit = [&](int buf, f32x16_t& scur, f32x16_t& snxt) {  // buf = u % NB
    read_kf((buf + 1) & (NB - 1));
#pragma unroll
    for (int e = 0; e < 16; ++e) snxt[e] = 0.f;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) snxt = mma16<DT>(kf[kc], qf[kc], snxt);
    // V(u)'s fragments are read here, so their LDS latency runs under the rho^8 chain
    read_vf(buf);
    __builtin_amdgcn_sched_barrier(0);
    float p[16];
    if constexpr (FAST) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = SM == 2 ? scur[r] * a.s_mult : scur[r];
        p[r] = SM == 1 ? rho8_fast_half(x) : rho8_fast(x);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = SM == 2 ? scur[r] * a.s_mult : scur[r];
        p[r] = SM == 1 ? rho8_exact_half(x) : rho8_exact(x);
      }
    }
    rowsum += tree16x(p);
    u32x4_t pk[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[kk][e] = Elem<DT>::pack(p[kk * 8 + 2 * e], p[kk * 8 + 2 * e + 1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] = mma16<DT>(vf[db][kk], pk[kk], o[db]);
  };

  // Step u: own loads of tile u+1 done (those of later tiles may remain), then publish them; the
  // barrier also ends every wave's unit u-1, the last reader of the buffer reused by the issue.
  auto step = [&](int u, int buf) {  // buf = u % NB
    if (u + 2 < t_hi) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS * (NB - 3)));
    else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __syncthreads();
    if (u + NB - 1 < t_hi) issue_tile(u + NB - 1, (buf + NB - 1) & (NB - 1));
  };
  // Units are taken in pairs from the even t_lo, so S(u) sits in sA for even u and in sB for
  // odd u with no register copies.  Unit u is clean when u + 1 < U (a next unit exists) and no
  // key of it needs a mask; both can only turn false as u grows, so the clean units are a prefix
  // [t_lo, uc) of the wave's.  The loop bounds differ between waves, but every wave runs one
  // step, and so one barrier, per tile of [t_lo, t_hi).
  auto clean = [&](int u) {
    const int key0 = u * KT;
    return u + 1 < U && !((a.causal && key0 + 31 > q0_w) || key0 + 31 >= vlen);
  };
  int uc = t_lo;
  while (uc < t_hi && clean(uc)) ++uc;
  int u = t_lo;
  // clean units: one pair up to a multiple of NB, then groups of NB with constant buffers
  static_assert(NB == 4, "the clean loop takes the ring's buffers in groups of four");
  if ((u & (NB - 1)) != 0 && u + 1 < uc) {
    step(u, u & (NB - 1));
    clean_unit(u & (NB - 1), sA, sB);
    step(u + 1, (u + 1) & (NB - 1));
    clean_unit((u + 1) & (NB - 1), sB, sA);
    u += 2;
  }
  for (; u + 3 < uc; u += 4) {
    step(u, 0);
    clean_unit(0, sA, sB);
    step(u + 1, 1);
    clean_unit(1, sB, sA);
    step(u + 2, 2);
    clean_unit(2, sA, sB);
    step(u + 3, 3);
    clean_unit(3, sB, sA);
  }
  for (; u + 1 < uc; u += 2) {
    step(u, u & (NB - 1));
    clean_unit(u & (NB - 1), sA, sB);
    step(u + 1, (u + 1) & (NB - 1));
    clean_unit((u + 1) & (NB - 1), sB, sA);
  }
  for (; u < t_hi; u += 2) {
    step(u, u & (NB - 1));
    unit(u, sA, sB);
    if (u + 1 < t_hi) {
      step(u + 1, (u + 1) & (NB - 1));
      unit(u + 1, sB, sA);
    }
  }

  // key split: every part stores its fp32 partial numerators and row sums, then counts itself
  // in; the last part of the block to arrive adds all parts' partials (in part order, so that
  // the sum does not depend on which part finished last) and stores the block.  The partials go
  // through device-scope relaxed atomic stores and loads (written through to, and read from,
  // the point where every XCD sees them), so no cache-wide write-back or invalidate is needed:
  // a part's stores are complete (vmcnt 0) before its count, and the last part reads after its
  // own count.
  //
  // This hand-off has no release/acquire edge in the HIP memory model; it is correct because of
  // how gfx950 executes these instructions, and the bitwise-repeatability test of the key split
  // guards it:
  //  * an agent-scope relaxed store is a global store with the sc1 bit, written through the
  //    XCD's L2 to memory-side coherent storage, and vmcnt counts it complete only once that
  //    write is acknowledged, so every part's partials are visible device-wide before its
  //    s_waitcnt vmcnt(0) ends and the barrier lets tid 0 issue the counter atomic;
  //  * the counter atomic executes at device scope, and the last part's partial loads are issued
  //    only after it returns (its value decides the branch);
  //  * an agent-scope relaxed load carries sc1 as well and misses the non-coherent cache levels,
  //    so it returns the value written through, not a stale line of this XCD's L2.
  // A target whose stores are acknowledged before they are device-visible, or whose sc1 loads
  // may hit stale lines, would need an acq_rel fetch_add by tid 0 (a whole-L2 write-back and
  // invalidate on gfx950, which made the split 2-4x slower).
  if (pp.nparts > 1) {
    __shared__ int ks_last;
    // a part's partial, lane-major so that every store and load instruction covers 256
    // contiguous bytes: per wave, NDB * 16 accumulator values, then the row sum, each for the 64
    // lanes (the last part's lanes hold the same rows and features as every other part's)
    constexpr int NV = NDB * 16 + 1;
    constexpr int PSTRIDE = 4 * NV * 64;  // floats per part
    const int blk = bh * (a.nqb - a.ks_q0) + (qblk - a.ks_q0);
    float* parts = a.ks_part + (size_t)blk * a.ks_pmax * PSTRIDE + wave * NV * 64 + lane;
    float* mine = parts + (size_t)pp.part * PSTRIDE;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        __hip_atomic_store(mine + (db * 16 + e) * 64, o[db][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(mine + (NV - 1) * 64, rowsum + __shfl_xor(rowsum, 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __syncthreads();
    if (tid == 0) ks_last = atomicAdd(a.ks_cnt + blk, 1) == pp.nparts - 1;
    __syncthreads();
    if (!ks_last) return;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
    float total = 0.f;
    for (int p2 = 0; p2 < pp.nparts; ++p2) {
      const float* part = parts + (size_t)p2 * PSTRIDE;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          o[db][e] += __hip_atomic_load(part + (db * 16 + e) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      total += __hip_atomic_load(part + (NV - 1) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    rowsum = g == 0 ? total : 0.f;
  }

  // epilogue
  const float tot = rowsum + __shfl_xor(rowsum, 32) + a.omega;
  if (a.acc) {
    // one key shard: the unnormalised sums go to the caller's fp32 arrays, stored (ACC_STORE) or
    // added to what they hold (ACC_ADD); every element of this block's rows belongs to one lane
    if (qi < L) {
      float* op = (float*)a.out + b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
      // every load before the first store, so that the row's memory latencies overlap
      f32x4_t x[NDB][4];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int f = db * 32 + r4 * 8 + 4 * g;
          x[db][r4] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          if (a.acc == ACC_ADD && (D == DP || f < D)) x[db][r4] = *(const f32x4_t*)(op + f);
        }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int f = db * 32 + r4 * 8 + 4 * g;
          if (D == DP || f < D) {
#pragma unroll
            for (int u = 0; u < 4; ++u) x[db][r4][u] += o[db][r4 * 4 + u] * a.w_unscale;
            *(f32x4_t*)(op + f) = x[db][r4];
          }
        }
      if (g == 0) acc_row(a.denom + (int64_t)bh * L + qi, (tot - a.omega) * a.w_unscale, a.acc);
    }
    return;
  }
  if (qi < L) {
    unsigned short* op = (unsigned short*)a.out + b * a.o_b + h * a.o_h + (int64_t)qi * a.o_l;
    const float inv = 1.0f / tot;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int f = db * 32 + r4 * 8 + 4 * g;  // features f .. f+3 (D is a multiple of 16)
        if (D == DP || f < D) {
          u32x2_t w;
          w[0] = Elem<DT>::pack(o[db][r4 * 4 + 0] * inv, o[db][r4 * 4 + 1] * inv);
          w[1] = Elem<DT>::pack(o[db][r4 * 4 + 2] * inv, o[db][r4 * 4 + 3] * inv);
          *(u32x2_t*)(op + f) = w;
        }
      }
    if (a.denom != nullptr && g == 0) a.denom[(int64_t)bh * L + qi] = tot * a.w_unscale;
  }
}

template <int D, int DT, bool EXACT, int SM, bool ROT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PipeShape<padded_dim(D)>::WAVES_PER_EU,
                                                                     PipeShape<padded_dim(D)>::WAVES_PER_EU)))
void afa_fwd_pipe_kernel(const FwdArgs a) {
  constexpr int DP = padded_dim(D);      // LDS row and MFMA width
  constexpr int KT = 32;                 // keys per tile = one unit
  constexpr int NB = PipeShape<DP>::NB;
  constexpr int CH = DP / 8;             // 16-byte chunks per LDS row
  constexpr int CHD = D / 8;             // chunks that hold data
  constexpr int LPT = KT * CH / 256;     // direct loads per thread per tile, each of K and V
  constexpr int LOADS = 2 * LPT;
  constexpr int NK = DP / 16;            // 16-feature MFMA steps of S
  constexpr int NDB = DP / 32;           // 32-feature output blocks
  static_assert(D % 16 == 0 && D <= DP, "head_dim");
  static_assert(LPT >= 1 && KT * CH % 256 == 0, "tile loader shape");
  static_assert(NB == 4, "the waits below assume at most one tile in flight beyond the next");
  __shared__ __attribute__((aligned(16))) PipeTile<DP> lds_k[NB];
  __shared__ __attribute__((aligned(16))) PipeTile<DP> lds_v[NB];

  int bh, qblk;
  PipePart pp;
  if (a.ks_tiles == 0) block_item(blockIdx.x, a.B * a.H, a.nqb, a.causal, bh, qblk);
  else split_item(a, (int)blockIdx.x, bh, qblk, pp);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int b = bh / a.H, h = bh % a.H;
  const int L = a.L, vlen = a.valid_len;
  const int q0_wg = qblk * 128, q0_w = q0_wg + wave * 32;
  const int kend_wg = a.causal ? min(vlen, min(L, q0_wg + 128)) : vlen;
  const int kend_w = a.causal ? min(vlen, q0_w + 32) : vlen;
  const unsigned short* qp = (const unsigned short*)a.q + b * a.q_b + h * a.q_h;
  // the fast-rho guard's key-block bounds go out first: they do not depend on q
  const float* kbm = !EXACT && a.kbm != nullptr ? a.kbm + (int64_t)bh * a.nkb : nullptr;
  const int kblk1 = (kend_w + 63) / 64;
  const float kbm_first = fast_rho_prefetch(kbm, 0, kblk1);

  // the first tiles of this workgroup's key range go out before the q loads, so that their
  // memory latencies overlap (pipe_body waits for them)
  {
    const int ntiles = (kend_wg + KT - 1) / KT;
    const int t_hi = min(pp.t1, ntiles), t_lo = min(pp.t0, t_hi);
    const unsigned short* kp = (const unsigned short*)a.k + b * a.k_b + h * a.k_h;
    const unsigned short* vp = (const unsigned short*)a.v + b * a.v_b + h * a.v_h;
    for (int t = t_lo; t < t_lo + min(t_hi - t_lo, NB - 1); ++t)
      pipe_issue_tile<D>(a, lds_k, lds_v, kp, vp, t, t & (NB - 1));
  }

  // q fragments (B operand of S^T = K Q^T): query q0_w + l32, features kc*16 + 8g .. +7
  const int qi = q0_w + l32;
  u32x4_t qf[NK];
#pragma unroll
  for (int kc = 0; kc < NK; ++kc) {
    u32x4_t w = {0u, 0u, 0u, 0u};
    const int d0 = kc * 16 + 8 * g;
    if (qi < L && d0 < D) {
      const float* cc = ROT ? a.rc + (int64_t)qi * (D / 2) + d0 / 2 : nullptr;
      const float* ss = ROT ? a.rs + (int64_t)qi * (D / 2) + d0 / 2 : nullptr;
      w = q_chunk<DT, ROT>(*(const u32x4_t*)(qp + (int64_t)qi * a.q_l + d0), cc, ss, a.q_scale);
    }
    qf[kc] = w;
  }
  // fast-rho guard: the largest squared norm of the wave's queries as the MFMA sees them (each
  // lane holds half the features of query l32) against the key blocks it reads
  bool fast = false;
  if (!EXACT) {
    float n2 = 0.0f;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) n2 += chunk_norm2<DT>(qf[kc]);
    fast = fast_rho_safe(kbm, 0, kblk1, wave_max(n2 + __shfl_xor(n2, 32)), a.nb_lim, kbm_first);
  }

  if (fast) pipe_body<D, DT, true, SM>(a, lds_k, lds_v, qf, bh, qblk, pp);
  else pipe_body<D, DT, false, SM>(a, lds_k, lds_v, qf, bh, qblk, pp);
}

namespace {

template <int D, int DT, bool EXACT, int SM>
hipError_t launch_pipe(const FwdArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.ks_tiles > 0 ? a.ks_items : a.B * a.H * a.nqb));
  if (a.rc != nullptr)
    hipLaunchKernelGGL((afa_fwd_pipe_kernel<D, DT, EXACT, SM, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((afa_fwd_pipe_kernel<D, DT, EXACT, SM, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

PipeSplit pipe_split_plan(int head_dim, int64_t BH, int64_t L, bool causal, int cus) {
  PipeSplit ps;
  const int DP = head_dim <= 64 ? 64 : 128;
  const int64_t slots = (int64_t)cus * (DP == 128 ? PipeShape<128>::WAVES_PER_EU : PipeShape<64>::WAVES_PER_EU);
  const int64_t nqb = (L + 127) / 128;
  auto tiles = [&](int64_t q) { return causal ? (std::min(L, 128 * (q + 1)) + 31) / 32 : (L + 31) / 32; };
  int64_t total = 0;
  for (int64_t q = 0; q < nqb; ++q) total += tiles(q);
  total *= BH;
  // parts of about the balanced load per workgroup slot, at least 16 tiles (512 keys) each, and
  // the partials (fp32 rows of every part of every split block) within 48 MiB.  No split when the
  // longest block is within 50% of a part: storing and adding the partials then costs more than
  // the shorter critical path saves (B=32 H=4 L=1024 D=64 causal, whose longest block is 1.33
  // parts: 334 TFLOP/s split, 353 unsplit; B=4 H=8 L=2048, 2.67 parts: 386 split, 371 unsplit)
  for (int64_t T = std::max<int64_t>((total + slots - 1) / slots, 16); T <= tiles(nqb - 1); T *= 2) {
    T = (T + 1) & ~(int64_t)1;
    if (tiles(nqb - 1) * 2 <= T * 3) return ps;
    int64_t q0 = 0;
    while (tiles(q0) <= T) ++q0;
    const int64_t pmax = (tiles(nqb - 1) + T - 1) / T;
    const size_t part_bytes = (size_t)(BH * (nqb - q0) * pmax) * 4 * (DP / 2 + 1) * 64 * sizeof(float);
    if (part_bytes > ((size_t)48 << 20)) continue;
    int64_t ranks = 0;
    for (int64_t q = 0; q < nqb; ++q) ranks += q < q0 ? 1 : (tiles(q) + T - 1) / T;
    ps.tiles = (int)T;
    ps.q0 = (int)q0;
    ps.pmax = (int)pmax;
    ps.items = (int)(ranks * BH);
    ps.part_bytes = part_bytes;
    ps.cnt_bytes = (size_t)(BH * (nqb - q0)) * sizeof(int);
    return ps;
  }
  return ps;
}

bool pipe_fwd_supported(int dtype, int head_dim) {
  return (dtype == AFA_BF16 || dtype == AFA_F16) &&
         (head_dim == 32 || head_dim == 48 || head_dim == 64 || head_dim == 96 || head_dim == 128);
}

namespace {

// 1/sqrt(D) = 2^-k * c: q carries 2^-k exactly; the score factor c = fl(1/sqrt D) * 2^k
// (exact scaling of the reference's fp32 constant).
template <int D>
hipError_t launch_scaled(int dtype, FwdArgs a, bool exact, int k, hipStream_t st) {
  a.q_scale = std::ldexp(1.0f, -k);
  a.s_mult = std::ldexp((float)(1.0 / std::sqrt((double)D)), k);
  a.nb_lim = fast_rho_lim(a.s_mult);
  if (dtype == AFA_BF16) return exact ? launch_pipe<D, AFA_BF16, true, 2>(a, st) : launch_pipe<D, AFA_BF16, false, 2>(a, st);
  return exact ? launch_pipe<D, AFA_F16, true, 2>(a, st) : launch_pipe<D, AFA_F16, false, 2>(a, st);
}

// 1/sqrt(D) = 2^-k sqrt(2) (D = 32, 128): bf16 fast path evaluates (rho/sqrt 2)^8 = rho^8/16
template <int D>
hipError_t launch_sqrt2(int dtype, FwdArgs a, bool exact, int k, hipStream_t st) {
  if (dtype == AFA_BF16 && !exact) {
    a.q_scale = std::ldexp(1.0f, -k);
    a.omega *= 0.0625f;
    a.w_unscale = 16.0f;
    a.nb_lim = fast_rho_lim(std::sqrt(2.0));  // s = sqrt(2) x
    return launch_pipe<D, AFA_BF16, false, 1>(a, st);
  }
  return launch_scaled<D>(dtype, a, exact, k, st);
}

}  // namespace

hipError_t pipe_fwd_launch(int dtype, int head_dim, FwdArgs a, bool exact, hipStream_t st) {
  a.nqb = (a.L + 127) / 128;
  a.w_unscale = 1.0f;
  a.s_mult = 1.0f;
  switch (head_dim) {
    case 32: return launch_sqrt2<32>(dtype, a, exact, 3, st);
    case 48: return launch_scaled<48>(dtype, a, exact, 3, st);
    case 64:
      a.q_scale = 0.125f;  // 1/sqrt(64), exact in any binary format
      a.nb_lim = fast_rho_lim(1.0);
      if (dtype == AFA_BF16) return exact ? launch_pipe<64, AFA_BF16, true, 0>(a, st) : launch_pipe<64, AFA_BF16, false, 0>(a, st);
      return exact ? launch_pipe<64, AFA_F16, true, 0>(a, st) : launch_pipe<64, AFA_F16, false, 0>(a, st);
    case 96: return launch_scaled<96>(dtype, a, exact, 4, st);
    case 128: return launch_sqrt2<128>(dtype, a, exact, 4, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace afa
