/*
 * afa.h — C ABI of the MI355X (gfx950) Algebraic FlashAttention library (libafa_hip.so).
 *
 * Every entry point takes plain device pointers, sizes and an optional hipStream_t
 * (passed as void*; NULL = the default stream).  The caller owns every buffer, including the
 * workspaces of the entry points that take one (a NULL workspace makes the call allocate and
 * free its own, stream-ordered, from a memory pool private to this library); calls are
 * stream-ordered, stateless and re-entrant.  They return 0 (AFA_OK) or an afa_status code;
 * afa_status_string() gives the message.
 *
 * Layout: q, k, v, out are (batch, heads, seq_len, head_dim) with head_dim contiguous.
 * `strides` (nullable) holds 12 element strides {q_b, q_h, q_l, k_b, k_h, k_l, v_b, v_h,
 * v_l, o_b, o_h, o_l}; NULL means contiguous.  The denominator output is contiguous
 * (batch, heads, seq_len) fp32 (fp64 for AFA_F64 inputs).
 *
 * Citations are into tasmaikeni13/algebraic-intelligence.
 */
#ifndef ALGEBRAIC_INTELLIGENCE_AMD_AFA_H
#define ALGEBRAIC_INTELLIGENCE_AMD_AFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types; AFA_F64 accumulates in fp64 like the reference (pallas_afa.py:208). */
enum afa_dtype { AFA_F32 = 0, AFA_BF16 = 1, AFA_F16 = 2, AFA_F64 = 3 };

enum afa_status {
  AFA_OK = 0,
  AFA_ERR_NULL = 1,          /* a required pointer is NULL */
  AFA_ERR_DTYPE = 2,         /* unsupported dtype */
  AFA_ERR_SHAPE = 3,         /* non-positive or inconsistent sizes */
  AFA_ERR_HEAD_DIM = 4,      /* head_dim > 128 and not a multiple of 128 (pallas_afa.py:179-180) */
  AFA_ERR_SINK = 5,          /* sink_omega not finite or negative (pallas_afa.py:171-172) */
  AFA_ERR_VALID_LEN = 6,     /* valid_len outside [1, seq_len] (pallas_afa.py:185-186) */
  AFA_ERR_EPS = 7,           /* eps not finite or not positive (attention.py:62-63) */
  AFA_ERR_ROTARY = 8,        /* rotary tables shorter than seq_len, or odd head_dim */
  AFA_ERR_ALIGN = 9,         /* a stride or pointer breaks the required alignment */
  AFA_ERR_WORKSPACE = 10,    /* workspace too small */
  AFA_ERR_UNSUPPORTED = 11,  /* combination this build does not implement */
  AFA_ERR_GAMMA = 12,        /* OACE gamma not finite or not positive (src/loss.py:33-34) */
  AFA_ERR_SCRATCH_LIMIT = 13, /* afa_fwd_noalloc: the call needs more workspace than the fixed
                                 per-device scratch (AFA_NOALLOC_SCRATCH_BYTES) */
  AFA_ERR_HIP = 100          /* a HIP runtime call failed; afa_last_hip_error() has the code */
};

/* Flags for afa_fwd / afa_bwd. */
#define AFA_FLAG_EXACT_TAIL 0x1u   /* always use the cancellation-safe two-branch rho for s < 0
                                      (otherwise only where the fast-rho guard asks for it) */
#define AFA_FLAG_GENERIC 0x2u      /* route to the generic (non-MFMA) kernel */
#define AFA_FLAG_EXACT_REF 0x4u    /* exact_afa_reference contract: q*scale rounded to the input
                                      dtype before the dot, row sum of P cast to v.dtype, and
                                      out = o * (1/(D+Omega)) (pallas_afa.py:283-297) */
#define AFA_FLAG_SIMPLE_SCHEDULE 0x8u /* bf16/fp16 head_dim 64 and 128: use the non-pipelined
                                         MFMA kernel (the reference point for the pipelined ones) */
/* afa_fwd on one key shard, as one hop of distributed_ring_afa (src/kernels/pallas_afa.py:618-662,
   _ring_step) or one part of a split-K sum: out and denom are arrays in the accumulation type
   (fp32; fp64 for AFA_F64), out with the strides given for it, denom contiguous (batch, heads,
   seq_len), and they receive the unnormalised sums num_i = sum_j rho(s_ij)^8 v_j (rho^8 rounded
   to v's dtype as the PV operand) and den_i = sum_j rho(s_ij)^8.  AFA_FLAG_PARTIAL stores them
   (out = num, denom = den: the first hop, or a split-K part), AFA_FLAG_ACCUMULATE adds them to
   what the arrays hold (out += num, denom += den: every later hop).  sink_omega must be 0 (the
   sink enters only the final division, afa_ring_finish) and denom must not be NULL; the two
   flags exclude each other. */
#define AFA_FLAG_ACCUMULATE 0x100u
#define AFA_FLAG_PARTIAL 0x200u

const char* afa_status_string(int status);
int afa_last_hip_error(void);
int afa_version(void);

/*
 * Fused AFA forward.  Replaces pallas_afa_forward (src/kernels/pallas_afa.py:154-264) and its
 * tile kernel afa_kernel (:52-151); also serves tiled_afa_forward (:330-406), whose result is
 * the same function of the inputs.  out = sum_j rho(s_ij)^8 v_j / (sum_j rho(s_ij)^8 + sink),
 * s_ij = q_i.k_j / sqrt(head_dim); keys j > i are masked when causal != 0 and keys
 * j >= valid_len when valid_len > 0.  denom (nullable) receives sum_j rho^8 + sink.
 * rot_cos/rot_sin (nullable, both or neither): Cayley rotary tables (rot_len, head_dim/2),
 * fp32 (fp64 for AFA_F64); q and k rows at position i are rotated by row i (fusing
 * _rotate_tensor, src/attention.py:142-152, as called from src/model.py:262-264): q when the
 * kernel loads it, k at tile load, except on the pipelined bf16/fp16 paths (head_dim 32, 48,
 * 64, 96, 128), where k is rotated once per call into the workspace.
 * On bf16/fp16 inputs rho(s)^8 takes a branch-free form on key tiles where every score is
 * provably within |s| <= 32 (Cauchy-Schwarz with per-block row norms that the call computes into
 * the workspace), and the two-branch form of the reference elsewhere; AFA_FLAG_EXACT_TAIL forces
 * the two-branch form everywhere.  AFA_FLAG_SIMPLE_SCHEDULE selects the fully fused kernel
 * (head_dim 64, 128).
 * workspace: at least afa_fwd_workspace_size() bytes of 16-byte aligned device memory for the
 * same sizes and rotary choice (0 bytes on some paths), or NULL to let the call allocate it
 * stream-ordered from a memory pool of this library and free it on `stream` before returning.
 * The size is that of the call's largest path on the current device (the fp32 split-K partials
 * depend on its compute-unit count).  Calls that share a workspace must be ordered on one stream.
 */
size_t afa_fwd_workspace_size(int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                              int64_t head_dim, int rotary);
int afa_fwd(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
            const void* q, const void* k, const void* v, const int64_t* strides, void* out,
            void* denom, const void* rot_cos, const void* rot_sin, int64_t rot_len,
            double sink_omega, int causal, int64_t valid_len, unsigned flags, void* workspace,
            size_t workspace_bytes, void* stream);

/*
 * Final step of distributed_ring_afa (src/kernels/pallas_afa.py:660-661): out = acc / (denom +
 * sink_omega), divided in the accumulation type (fp32; fp64 for AFA_F64) and rounded to dtype.
 * acc and denom are the sums that afa_fwd calls with AFA_FLAG_PARTIAL / ACCUMULATE filled: acc
 * (batch, heads, seq_len, head_dim), denom contiguous (batch, heads, seq_len).  total (nullable)
 * receives denom + sink_omega in the accumulation type: the d_total that afa_bwd takes, so the
 * ring's gradient is afa_bwd's.  strides (nullable = contiguous): 9 element strides, (b, h, l) of
 * acc, of out, then of total; head_dim contiguous.
 */
int afa_ring_finish(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                    const void* acc, const void* denom, const int64_t* strides, double sink_omega,
                    void* out, void* total, void* stream);

/*
 * afa_fwd without allocation.  No counterpart in the reference: for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as afa_fwd; the workspace is a fixed array of
 * AFA_NOALLOC_SCRATCH_BYTES that the library holds on every device it runs on until the process
 * ends, and the call allocates nothing (no hipMalloc, hipFree or pool allocation).  Calls whose
 * afa_fwd_workspace_size() exceeds the array return AFA_ERR_SCRATCH_LIMIT before any device work
 * (64 MiB holds, e.g., B=8 H=12 L=4096 D=64 bf16 with rotary tables).  Every call on a device
 * shares that device's array: calls that overlap on one device (different streams, or threads
 * without ordering) race; calls ordered on one stream do not.  No part of the array needs to be
 * cleared between calls.
 */
#define AFA_NOALLOC_SCRATCH_BYTES (64u << 20)
int afa_fwd_noalloc(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                    const void* q, const void* k, const void* v, const int64_t* strides, void* out,
                    void* denom, const void* rot_cos, const void* rot_sin, int64_t rot_len,
                    double sink_omega, int causal, int64_t valid_len, unsigned flags, void* stream);

/*
 * Analytical AFA backward.  Replaces tiled_afa_backward (src/kernels/pallas_afa.py:409-522)
 * as used by the pallas_afa custom VJP (:532-615).  Inputs: the forward's q, k, v, out and
 * denom (= d_total, fp32; fp64 for AFA_F64) and the output cotangent g (same layout as q).
 * Outputs dq, dk, dv (contiguous).  With rotary tables the forward rotated q and k, and the
 * returned dq, dk are with respect to the unrotated inputs (the fp32 matrix-core kernels rotate
 * them as tiles are staged; on the bf16/fp16 matrix-core path, head_dim 32, 48, 64, 96, 128 and
 * 256, q and k are rotated once into the workspace).  rho(s)^8 follows the same fast-rho guard
 * as afa_fwd.  workspace: at least afa_bwd_workspace_size() bytes (16-byte aligned) for the same
 * sizes and rotary choice, or NULL to let the call allocate it as afa_fwd does.
 */
size_t afa_bwd_workspace_size(int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                              int64_t head_dim, int rotary);
int afa_bwd(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
            const void* q, const void* k, const void* v, const void* out, const void* denom,
            const void* g, void* dq, void* dk, void* dv, const void* rot_cos,
            const void* rot_sin, int64_t rot_len, double sink_omega, int causal,
            int64_t valid_len, unsigned flags, void* workspace, size_t workspace_bytes,
            void* stream);

/*
 * A-Softmax over the last axis of a (rows, cols) contiguous array: AVN normalisation
 * tau = rsqrt(mean(x^2) + eps), then rho(tau x)^8 / (sum + sink), in fp32 (fp64 for AFA_F64),
 * output in the input dtype.  Replaces algebraic_softmax (src/attention.py:53-91, with AVN from
 * src/primitives.py:56-65).  asoftmax_bwd is its cached VJP (src/attention.py:75-82 with
 * src/primitives.py:73-79).
 */
int asoftmax_fwd(int dtype, int64_t rows, int64_t cols, const void* x, void* y,
                 double sink_omega, double eps, void* stream);
int asoftmax_bwd(int dtype, int64_t rows, int64_t cols, const void* x, const void* g, void* dx,
                 double sink_omega, double eps, void* stream);

/* Elementwise rho(x)^8 and its VJP 8 r rho^8 g.  Replaces octic_kernel / _vmu_octic_kernel
 * (src/attention.py:18-50, src/kernels/pallas_afa.py:32-49). */
int octic_fwd(int dtype, int64_t n, const void* x, void* y, void* stream);
int octic_bwd(int dtype, int64_t n, const void* x, const void* g, void* dx, void* stream);
/* rho(x)^8 and r = rsqrt(1 + x^2) in the same evaluation, both written in the accumulation type
 * (fp32, or fp64 for AFA_F64 inputs).  Replaces _kernel (src/attention.py:18-26), which returns
 * the pair: r is the factor of the VJP 8 r rho^8 g. */
int octic_fwd_r(int dtype, int64_t n, const void* x, void* k, void* r, void* stream);

/*
 * Cayley rotary tables.  Replaces build_cayley_rotary_matrix (src/attention.py:155-204):
 * c, s of shape (max_seq_len, dim/2) in table_dtype (AFA_F32 or AFA_F64, device memory).
 * freqs (nullable, device memory, dim/2 entries of table_dtype) are the Cayley parameters w_k;
 * NULL selects the default w_k = 1/(1 + alpha k)^2, alpha = (sqrt(base) - 1)/max(dim/2 - 1, 1).
 */
int ago_build_tables(int table_dtype, int64_t dim, int64_t max_seq_len, const void* freqs,
                     double base, void* cos_out, void* sin_out, void* stream);

/*
 * Pairwise Cayley rotation of x viewed as (outer, seq_len, inner, dim), contiguous, by the
 * table row of each sequence position.  The tables (rot_len >= seq_len rows, dim/2 columns,
 * table_dtype AFA_F32/AFA_BF16/AFA_F16/AFA_F64) are cast to the x dtype first, as
 * _rotate_tensor does (src/attention.py:142-152); apply_ago_rotations (:207-240) calls this for
 * q and k.  y may alias x.
 */
int ago_rotate(int dtype, int64_t outer, int64_t seq_len, int64_t inner, int64_t dim,
               const void* x, void* y, int table_dtype, const void* rot_cos,
               const void* rot_sin, int64_t rot_len, void* stream);

/*
 * OACE loss head.  Calc type A: fp32, fp64 for AFA_F64 inputs.  targets: int64 class indices
 * (rows of them, device memory); a target outside [0, vocab) gives an infinite loss, as in the
 * reference.  loss: one A (device memory), the mean over rows.  row_cache: rows x
 * OACE_ROW_FIELDS values of A per row, in this order: tau, inv_S, S^(1/8), sum p^(7/8),
 * p_target^(-1/8), radial, loss, (unused) -- the forward writes it and the backward reads it
 * (the cache of the reference's custom VJP).  g_loss (nullable = 1): the loss cotangent, one A
 * in device memory.
 *
 * oace_linear_fwd / oace_linear_bwd replace fused_linear_oace_forward / _backward
 * (src/kernels/pallas_oace.py:59-269) and the custom VJP fused_linear_oace (:272-293):
 * loss = mean_n gamma (8 p_c^(-1/8) + 8/7 sum p^(7/8) - 64/7) of the A-Softmax of
 * z = h W normalised by tau = rsqrt(mean(z^2) + eps_vocab).  h: (rows, d_model), row stride
 * ldh.  w: OACE_W_DV, (d_model, vocab) with row stride ldw (the reference's output_head), or
 * OACE_W_VD, (vocab, d_model) with row stride ldw (a tied token embedding, W = E^T).
 * Backward outputs: dh (rows, d_model) contiguous, in h's dtype; dw in w's layout, dtype and
 * ldw.  The vocabulary chunk size of the reference does not change the result and is not an
 * argument.  workspace: oace_workspace_size() bytes of device memory, or NULL to let the call
 * allocate and free it on `stream`.  AFA_FLAG_GENERIC forces the generic (non-MFMA) kernels.
 */
#define OACE_W_DV 0
#define OACE_W_VD 1
#define OACE_ROW_FIELDS 8
/* oace_linear_bwd: the workspace is the one an oace_linear_fwd call with the same arguments used,
   and the weights have not changed since; the transposed copy of an OACE_W_DV weight that call
   left in it is reused. */
#define OACE_FLAG_WT_READY 0x10u
/* oace_linear_bwd: as OACE_FLAG_WT_READY, and h has not changed either; the fp32 logits that the
   forward keeps in the workspace (bf16/fp16 when rows x vocab x 4 bytes fit 256 MB) are reused,
   so dz is formed elementwise instead of by a second GEMM.  No counterpart in the reference. */
#define OACE_FLAG_Z_READY 0x20u
/* oace_workspace_size / oace_linear_fwd / oace_linear_bwd (the same on all three): never keep
   the logits; the backward recomputes them (a workspace of O(rows x d_model + vocab x d_model)).
   No counterpart in the reference. */
#define OACE_FLAG_RECOMPUTE_Z 0x40u
size_t oace_workspace_size(int dtype, int64_t rows, int64_t d_model, int64_t vocab, int w_layout,
                           unsigned flags);
int oace_linear_fwd(int dtype, int64_t rows, int64_t d_model, int64_t vocab, const void* h,
                    int64_t ldh, const void* w, int w_layout, int64_t ldw, const int64_t* targets,
                    double eps_vocab, double gamma, void* loss, void* row_cache, unsigned flags,
                    void* workspace, size_t workspace_bytes, void* stream);
int oace_linear_bwd(int dtype, int64_t rows, int64_t d_model, int64_t vocab, const void* h,
                    int64_t ldh, const void* w, int w_layout, int64_t ldw, const int64_t* targets,
                    double gamma, const void* row_cache, const void* g_loss, void* dh, void* dw,
                    unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The same loss on given logits (rows, vocab) contiguous, and its VJP dlogits (same shape and
 * dtype).  Replaces fused_oace_softmax_loss and its custom VJP (src/model.py:180-240); the
 * reference evaluates in the logits dtype, this evaluates in A and rounds dlogits once.
 */
int oace_softmax_loss_fwd(int dtype, int64_t rows, int64_t vocab, const void* logits,
                          const int64_t* targets, double eps, double gamma, void* loss,
                          void* row_cache, void* stream);
int oace_softmax_loss_bwd(int dtype, int64_t rows, int64_t vocab, const void* logits,
                          const int64_t* targets, double gamma, const void* row_cache,
                          const void* g_loss, void* dlogits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ALGEBRAIC_INTELLIGENCE_AMD_AFA_H */
