// Kernel argument blocks and launcher prototypes shared by the kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace afa {

// Forward epilogues for one key shard (AFA_FLAG_PARTIAL, AFA_FLAG_ACCUMULATE): none (normalised
// output), store the unnormalised sums, or add them to what the caller's arrays hold.
enum AccMode { ACC_NONE = 0, ACC_STORE = 1, ACC_ADD = 2 };

// Fused MFMA forward (afa_fwd_mfma.hip).
struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* denom;
  const float* rc;
  const float* rs;
  int64_t q_b, q_h, q_l, k_b, k_h, k_l, v_b, v_h, v_l, o_b, o_h, o_l;
  int B, H, L;
  int valid_len;    // keys >= valid_len carry zero weight (valid_len <= L)
  int causal;
  int nqb;          // query blocks per (b, h)
  float q_scale;    // power of two folded into q
  float omega;      // sink_omega times the weight scale
  float w_unscale;  // denominator output = w_unscale * (D' + omega)
  float s_mult;     // fp32 factor of the score after the q_scale fold (kernels that take one)
  float* part;      // split-K partials (afa_fwd_f32.hip): nsplit x B H L D numerators, then nsplit x B H L sums
  // fast-rho guard (FastGuard in afa_common.h): the largest squared norm of the key rows of each
  // 64-row block, nkb blocks per (b, h) (nullptr: every tile takes the two-branch rho), and the
  // bound nb_lim on (squared query-fragment norm) x (key block bound) below which a tile's scores
  // are all within |s| <= kFastRhoMaxScore (set by the launcher for its score scaling)
  const float* kbm;
  int nkb;
  float nb_lim;
  // key split of the pipelined kernel (PipeSplit below): query blocks from ks_q0 on are processed
  // in parts of up to ks_tiles 32-key tiles by ks_items workgroups in all; every part writes its
  // fp32 partial numerators and row sums to ks_part and counts itself in ks_cnt (one int per
  // split block, zero on entry), and the last part of a block to arrive adds the others' partials
  // and stores the block.  ks_tiles = 0: no split.
  int ks_tiles;
  int ks_q0;
  int ks_pmax;
  int ks_items;
  float* ks_part;
  int* ks_cnt;
  // AFA_FLAG_PARTIAL / AFA_FLAG_ACCUMULATE (AccMode): out is fp32 (element strides o_*) and
  // receives the unnormalised numerator, denom the row sum (sink_omega is 0)
  int acc;
};

// Key split of the pipelined kernel for one shape: causal rows near the end of a long sequence,
// or every row of a grid with fewer 128-query blocks than workgroup slots, would otherwise leave
// one workgroup's key loop as the critical path of the whole call.  Planned for valid_len = L;
// with a shorter valid_len some parts have no keys and contribute zero partials.
struct PipeSplit {
  int tiles = 0;       // 32-key tiles per part (0: no split)
  int q0 = 0;          // first split query block
  int pmax = 1;        // parts of the last query block (the most of any block)
  int items = 0;       // workgroups of the launch
  size_t part_bytes = 0, cnt_bytes = 0;
};

// Generic forward / backward (afa_generic.hip).
struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* out_in;  // backward: forward output
  const void* dtot;    // backward: forward denominator (accumulation type)
  const void* g;       // backward: output cotangent
  void* out;           // forward output / backward dq
  void* dk;
  void* dv;
  void* denom;         // forward denominator output (accumulation type), nullable
  void* e_ws;          // backward: E workspace (accumulation type, B*H*L)
  const void* rc;
  const void* rs;
  int64_t q_b, q_h, q_l, k_b, k_h, k_l, v_b, v_h, v_l, o_b, o_h, o_l;
  int B, H, L, D;
  int valid_len;
  int causal;
  int exact_ref;
  int acc;  // forward, AccMode: out and denom (accumulation type) receive the unnormalised sums
  double scale;
  double omega;
  // fast-rho guard of the MFMA backward (as FwdArgs): per 64-row block bounds of q (for the dK/dV
  // kernel, which owns keys) and of k (for the dQ kernel), nkb blocks per (b, h)
  const float* qbm;
  const float* kbm;
  int nkb;
  float nb_lim;
};

// afa_status code of a HIP error (AFA_ERR_HIP, recording it for afa_last_hip_error).
int hip_status_code(hipError_t e);

bool mfma_fwd_supported(int dtype, int head_dim);
int mfma_fwd_queries_per_block(int head_dim);
hipError_t mfma_fwd_launch(int dtype, int head_dim, FwdArgs a, bool exact, hipStream_t stream);
// K rotated once per call (afa_krot_kernel, head_dim 32, 48, 64, 96 or 128) into `krot`
// (krot_bytes bytes, contiguous B, H, L, D); a's k then points at it, and a's key bounds at nb2
// (B H ceil(L/64) floats), which the same launch fills from the rotated rows.
size_t krot_bytes(const FwdArgs& a, int head_dim);
hipError_t krot_launch(int dtype, int head_dim, FwdArgs& a, void* krot, float* nb2, hipStream_t stream,
                       int* zero = nullptr, int nzero = 0);
// Bound of the fast-rho guard: kFastRhoMaxScore^2 / (score / MFMA-output)^2, less a 5% margin for
// the rounding of the norms and of the rotated operands.
float fast_rho_lim(double score_per_output);
// Largest squared row norm of each 64-row block of x (bf16 / fp16; rows of head_dim elements,
// 16-byte aligned, element strides per (b, h, l)) into nb2[bh * ceil(L/64) + block].
// Both norm pre-passes also clear the `nzero` ints at `zero` (the key split's counters; nullptr: none).
hipError_t rownorm_launch(int dtype, const void* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                          int head_dim, float* nb2, hipStream_t stream, int* zero = nullptr, int nzero = 0);
// Software-pipelined head_dim-64 kernel (afa_fwd_d64.hip); 256 queries per workgroup.  q is
// rotated at load when a.rc is set; k must arrive rotated (krot_launch).
hipError_t d64_fwd_launch(int dtype, FwdArgs a, bool exact, hipStream_t stream);
// 32 queries per wave, several waves per SIMD (afa_fwd_pipe.hip): head_dim 32, 48, 64, 96 or
// 128 (rows zero-padded to 64 or 128 in LDS), 128 queries per workgroup; q is rotated at load
// when a.rc is set, k must arrive rotated.
bool pipe_fwd_supported(int dtype, int head_dim);
// Key split for B * H heads of L queries on `cus` compute units (tiles = 0 when none pays off).
PipeSplit pipe_split_plan(int head_dim, int64_t BH, int64_t L, bool causal, int cus);
// a.ks_*: the split (ks_tiles = 0 for none; the counters cleared by a pre-pass of the same call).
hipError_t pipe_fwd_launch(int dtype, int head_dim, FwdArgs a, bool exact, hipStream_t stream);

// fp32 forward on the fp32 MFMA (afa_fwd_f32.hip): head_dim 32/64/128, V and out rows 16-byte
// aligned; q_scale carries 1/sqrt(head_dim) (applied to the fp32 dot product).
bool f32_fwd_supported(int head_dim);
// nsplit > 1: the key range of every query block is split over nsplit workgroups whose partial
// numerators and row sums go to a.part (f32_fwd_part_floats(a, head_dim, nsplit) floats), then
// a combine kernel writes out and denom.
size_t f32_fwd_part_floats(const FwdArgs& a, int head_dim, int nsplit);
hipError_t f32_fwd_launch(int head_dim, FwdArgs a, int nsplit, hipStream_t st);

hipError_t generic_fwd_launch(int dtype, const GenArgs& a, hipStream_t st);
// MFMA backward (afa_bwd_mfma.hip): bf16/fp16, head_dim 32, 48, 64, 96, 128 or 256, any seq_len,
// contiguous tensors.  e_ws holds 2 * B*H*LP floats, LP = seq_len rounded up to 4 (-E, then
// 1/d, per head).  With rotary tables (fp32, 16-byte aligned) q and k are first rotated into
// rot_scratch (mfma_bwd_rot_bytes(a) bytes) and dq, dk are rotated back in the store epilogues.
bool mfma_bwd_supported(int dtype, int head_dim, int64_t seq_len);
size_t mfma_bwd_rot_bytes(const GenArgs& a);
hipError_t mfma_bwd_launch(int dtype, const GenArgs& a, bool exact, void* rot_scratch, hipStream_t st);
// fp32 backward on the fp32 MFMA (afa_bwd_f32.hip): head_dim 32/64/128, contiguous tensors,
// 16-byte aligned.  e_ws holds 2 * B*H*L floats (E, then 1/d).
bool f32_bwd_supported(int head_dim);
hipError_t f32_bwd_launch(const GenArgs& a, hipStream_t st);
hipError_t generic_bwd_launch(int dtype, const GenArgs& a, hipStream_t st);

hipError_t ago_tables_launch(int table_dtype, int pairs, int len, const void* freqs, double base,
                             void* c_out, void* s_out, hipStream_t st);
hipError_t ago_rotate_launch(int dtype, int table_dtype, int64_t outer, int64_t seq, int64_t inner,
                             int dim, const void* x, void* y, const void* rc, const void* rs,
                             hipStream_t st);

hipError_t asoftmax_fwd_launch(int dtype, int64_t rows, int64_t n, const void* x, void* y,
                               double sink, double eps, hipStream_t st);
hipError_t asoftmax_bwd_launch(int dtype, int64_t rows, int64_t n, const void* x, const void* g,
                               void* dx, double sink, double eps, hipStream_t st);
hipError_t octic_fwd_launch(int dtype, int64_t n, const void* x, void* y, hipStream_t st);
hipError_t octic_fwd_r_launch(int dtype, int64_t n, const void* x, void* k, void* r, hipStream_t st);

// Final division of a ring's accumulators (afa_generic.hip); strides in elements.
struct RingFinish {
  const void* acc;    // fp32 (fp64 for AFA_F64) numerators
  const void* denom;  // row sums, contiguous over (b, h, l)
  void* out;          // the input dtype
  void* total;        // nullable: denom + sink in the accumulation type, strides t_*
  int64_t a_b, a_h, a_l, o_b, o_h, o_l, t_b, t_h, t_l;
  int B, H, L, D;
  double sink;
};
hipError_t ring_finish_launch(int dtype, const RingFinish& r, hipStream_t st);
hipError_t octic_bwd_launch(int dtype, int64_t n, const void* x, const void* g, void* dx,
                            hipStream_t st);

// ---- OACE loss head (oace.hip: generic path and row kernels; oace_mfma.hip: bf16/fp16 path).
// Per-row record (OACE_ROW values of the calc type) cached by the forward for the backward.
enum {
  OACE_TAU = 0, OACE_INV_S = 1, OACE_S8 = 2, OACE_SUM_P78 = 3, OACE_PC_INV8 = 4, OACE_RADIAL = 5,
  OACE_LOSS = 6, OACE_ROW = 8
};
struct OaceArgs {
  int64_t N, d, V;
  const void* h;  // (N, d) hidden rows, row stride ldh; the logits (N, V) for the softmax loss
  int64_t ldh;
  const void* w;  // vocabulary projection, element (k, v) per w_layout and ldw
  int w_layout;
  int64_t ldw;
  const int64_t* targets;
  double eps, gamma;
  void* loss;          // calc-type scalar
  const void* g_loss;  // backward: calc-type cotangent of the loss, nullable (= 1)
  void* dh;            // backward: (N, d) contiguous
  void* dw;            // backward: W's layout and ldw
  unsigned flags;
};
size_t oace_generic_chunk_rows(int dtype, int64_t N, int64_t V);
size_t oace_generic_workspace(int dtype, int64_t N, int64_t d, int64_t V, bool backward);
hipError_t oace_linear_fwd_generic(int dtype, const OaceArgs& a, void* rows, void* ws, hipStream_t st);
hipError_t oace_linear_bwd_generic(int dtype, const OaceArgs& a, const void* rows, void* ws, hipStream_t st);
hipError_t oace_mean_launch(int dtype, const void* rows, int64_t N, void* loss, hipStream_t st);
hipError_t oace_softmax_fwd_launch(int dtype, const OaceArgs& a, void* rows, hipStream_t st);
hipError_t oace_softmax_bwd_launch(int dtype, const OaceArgs& a, const void* rows, void* dz, hipStream_t st);
hipError_t oace_transpose16(const void* x, int64_t rows, int64_t cols, int64_t ldx, void* y, int64_t ldy,
                            hipStream_t st);
// MFMA path (oace_mfma.hip): bf16/fp16, d_model a multiple of 32, 16-byte aligned rows of h (and
// of W^T for OACE_W_VD).
bool oace_mfma_supported(int dtype, const OaceArgs& a);
size_t oace_mfma_workspace(int dtype, const OaceArgs& a);
hipError_t oace_linear_fwd_mfma(int dtype, const OaceArgs& a, void* rows, void* ws, hipStream_t st);
hipError_t oace_linear_bwd_mfma(int dtype, const OaceArgs& a, const void* rows, void* ws, hipStream_t st);

// MFMA GEMM of the OACE backward (oace_bwd_gemm.hip): D[n][m] = sum_k A[m][k] B[n][k] in the
// element type at out[n * ldo + m], fp32 accumulation.  An operand is row-contiguous (mc:
// element (r, k) at p[k * ld + r]) or contraction-contiguous (element (r, k) at p[r * ld + k]).
struct OaceGemm {
  const void* a;
  int64_t lda;
  bool a_mc;
  int64_t m;
  const void* b;
  int64_t ldb;
  bool b_mc;
  int64_t n;
  int64_t k;
  void* out;
  int64_t ldo;
};
bool oace_gemm_fits(const OaceGemm& g);
// Contraction parts for about `wgs` workgroups (1: no split); parts > 1 need part_bytes of fp32
// partials, added in part order by a second kernel (row-contiguous A, contiguous B only).
int oace_gemm_parts(const OaceGemm& g, int wgs);
size_t oace_gemm_part_bytes(const OaceGemm& g, int parts);
hipError_t oace_gemm(int dtype, const OaceGemm& g, int parts, float* part, hipStream_t st);

}  // namespace afa
