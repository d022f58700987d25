// C ABI of libafa_hip.so (declared in include/afa.h): argument validation mirroring the
// reference's ValueError checks, path selection, and kernel dispatch.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>

#include "../../include/afa.h"
#include "afa_launch.h"

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
  if (e == hipSuccess) return AFA_OK;
  g_last_hip_error = (int)e;
  return AFA_ERR_HIP;
}

bool finite_nonneg(double x) { return x >= 0.0 && x < INFINITY; }  // NaN fails both
bool valid_dtype(int dt) { return dt == AFA_F32 || dt == AFA_BF16 || dt == AFA_F16 || dt == AFA_F64; }
size_t elem_size(int dt) { return dt == AFA_F64 ? 8 : dt == AFA_F32 ? 4 : 2; }
size_t acc_size(int dt) { return dt == AFA_F64 ? 8 : 4; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (cached per device; 256 if the query fails).
int cu_count() {
  static std::once_flag once[64];
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::call_once(once[dev], [dev]() {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  });
  return cus[dev];
}

// Stream-ordered scratch for calls that pass no workspace, from a memory pool of this library
// (one per device, created on first use; its release threshold keeps memory freed by one call for
// the next instead of unmapping it at every synchronisation).  The device's default pool and
// every other pool of the process keep their own settings.  Returns nullptr on failure.
void* scratch_alloc(size_t bytes, hipStream_t s) {
  static std::once_flag once[64];
  static hipMemPool_t pools[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::call_once(once[dev], [dev]() {
    hipMemPoolProps props = {};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    if (hipMemPoolCreate(&pool, &props) == hipSuccess) {
      uint64_t keep = UINT64_MAX;
      (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
      pools[dev] = pool;
    } else {
      (void)hipGetLastError();
      pools[dev] = nullptr;
    }
  });
  if (pools[dev] == nullptr) return nullptr;
  void* p = nullptr;
  if (hipMallocFromPoolAsync(&p, bytes, pools[dev], s) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct Strides {
  int64_t v[12];
};

Strides resolve_strides(const int64_t* s, int64_t H, int64_t L, int64_t D) {
  Strides r;
  if (s == nullptr) {
    for (int t = 0; t < 4; ++t) {
      r.v[3 * t + 0] = H * L * D;
      r.v[3 * t + 1] = L * D;
      r.v[3 * t + 2] = D;
    }
  } else {
    for (int i = 0; i < 12; ++i) r.v[i] = s[i];
  }
  return r;
}

int check_rotary(const void* rc, const void* rs, int64_t rot_len, int64_t L, int64_t D) {
  if ((rc == nullptr) != (rs == nullptr)) return AFA_ERR_ROTARY;
  if (rc != nullptr && (rot_len < L || D % 2 != 0)) return AFA_ERR_ROTARY;
  return AFA_OK;
}

}  // namespace

namespace afa {
int hip_status_code(hipError_t e) { return hip_status(e); }
}  // namespace afa

extern "C" {

const char* afa_status_string(int status) {
  switch (status) {
    case AFA_OK: return "ok";
    case AFA_ERR_NULL: return "a required pointer is NULL";
    case AFA_ERR_DTYPE: return "unsupported dtype";
    case AFA_ERR_SHAPE: return "q, k, and v must all have shape (batch, heads, sequence, dimension) with positive sizes";
    case AFA_ERR_HEAD_DIM: return "head dimensions above 128 must be divisible by 128";
    case AFA_ERR_SINK: return "sink_omega must be finite and nonnegative";
    case AFA_ERR_VALID_LEN: return "valid_seq_len must be in [1, seq_len]";
    case AFA_ERR_EPS: return "eps must be finite and positive (nonnegative for the OACE loss)";
    case AFA_ERR_ROTARY: return "rotary tables must both be given, cover seq_len rows and need an even head dimension";
    case AFA_ERR_ALIGN: return "stride or pointer alignment not supported";
    case AFA_ERR_WORKSPACE: return "workspace too small";
    case AFA_ERR_UNSUPPORTED: return "combination not supported by this build";
    case AFA_ERR_GAMMA: return "gamma must be finite and strictly positive";
    case AFA_ERR_SCRATCH_LIMIT: return "the call needs more workspace than afa_fwd_noalloc's fixed scratch";
    case AFA_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

int afa_last_hip_error(void) { return g_last_hip_error; }

int afa_version(void) { return 1; }

}  // extern "C"

namespace {

// ---------------------------------------------------------------------------------- forward
// Path of an afa_fwd call and the workspace it needs (byte offsets of 256-byte aligned regions):
//   bf16 / fp16 matrix-core kernels: the fast-rho guard's key bounds (B H ceil(L/64) floats),
//     then, with rotary tables on the pipelined kernels, the rotated k (B H L D elements), then,
//     when the 128-query kernel splits long key ranges (PipeSplit), its partials and counters;
//   fp32 matrix-core kernel: the split-K partials when its grid is split;
//   generic kernel: nothing.
enum { FWD_GENERIC = 0, FWD_FUSED = 1, FWD_PIPE = 2, FWD_F32 = 3 };
struct FwdPlan {
  int kind = FWD_GENERIC;
  bool wide = false;  // FWD_PIPE at head_dim 64: the 256-query kernel (afa_fwd_d64.hip)
  bool rotk = false;  // FWD_PIPE with rotary tables: k rotated once into the workspace
  int nsplit = 1;     // FWD_F32: key splits
  afa::PipeSplit ks;  // FWD_PIPE 128-query kernel: key split (ks.tiles = 0: none)
  size_t kbm = 0, krot = 0, part = 0, ks_part = 0, ks_cnt = 0, total = 0;
};

// mfma_layout: 16-byte aligned q, k, v, out (and tables) with 8-element strides; f32_layout: the
// fp32 kernel's float4 rows of v and out; in_head_32: K and V rows addressable by 32-bit byte
// offsets within a head (the pipelined kernels' loads).
// causal < 0 (workspace queries): the larger of the causal and the non-causal needs.
FwdPlan fwd_plan(int dtype, int64_t B, int64_t H, int64_t L, int64_t D, int64_t vlen, bool rotary,
                 bool mfma_layout, bool f32_layout, bool in_head_32, unsigned flags, int causal) {
  FwdPlan p;
  if (flags & (AFA_FLAG_GENERIC | AFA_FLAG_EXACT_REF)) return p;
  // key-shard calls (partial or accumulating) take the kernels with that epilogue: the pipelined
  // bf16/fp16 kernels, the fp32 matrix-core kernel and the generic one
  const bool acc = (flags & (AFA_FLAG_ACCUMULATE | AFA_FLAG_PARTIAL)) != 0;
  const bool fused_ok = !acc && afa::mfma_fwd_supported(dtype, (int)D);
  const bool pipe_ok = afa::pipe_fwd_supported(dtype, (int)D) && in_head_32;
  if ((fused_ok || pipe_ok) && mfma_layout) {
    size_t off = align256((size_t)(B * H * ((L + 63) / 64)) * sizeof(float));
    if (pipe_ok && !(fused_ok && (flags & AFA_FLAG_SIMPLE_SCHEDULE))) {
      p.kind = FWD_PIPE;
      // head_dim 64: 256-query workgroups at two per CU (afa_fwd_d64.hip) when they fill at least
      // one and a half rounds of those slots; otherwise, and at the other head dims, 128-query
      // workgroups with several waves per SIMD (afa_fwd_pipe.hip).  With a single round (C4: 512
      // workgroups on 256 CUs) the finer causal blocks of the 128-query kernel balance better:
      // 0.0545 against 0.0560 ms, measured on one box.
      p.wide = D == 64 && B * H * ((L + 255) / 256) >= 3 * (int64_t)cu_count();
      if (rotary) {
        p.rotk = true;
        p.krot = off;
        off += align256((size_t)(B * H * L * D) * 2);
      }
      // the split's counters are cleared by the norm pre-pass, which runs with rotary tables or
      // under the fast-rho guard
      if (!p.wide && (rotary || !(flags & AFA_FLAG_EXACT_TAIL))) {
        if (causal >= 0) {
          p.ks = afa::pipe_split_plan((int)D, B * H, L, causal != 0, cu_count());
        } else {
          const afa::PipeSplit c = afa::pipe_split_plan((int)D, B * H, L, true, cu_count());
          const afa::PipeSplit n = afa::pipe_split_plan((int)D, B * H, L, false, cu_count());
          p.ks = c.part_bytes + c.cnt_bytes >= n.part_bytes + n.cnt_bytes ? c : n;
          p.ks.part_bytes = std::max(c.part_bytes, n.part_bytes);
          p.ks.cnt_bytes = std::max(c.cnt_bytes, n.cnt_bytes);
        }
        if (p.ks.tiles > 0) {
          p.ks_part = off;
          off += align256(p.ks.part_bytes);
          p.ks_cnt = off;
          off += align256(p.ks.cnt_bytes);
        }
      }
    } else {
      p.kind = FWD_FUSED;
    }
    p.total = off;
    return p;
  }
  if (dtype == AFA_F32 && afa::f32_fwd_supported((int)D) && f32_layout) {
    p.kind = FWD_F32;
    // fewer 128-query workgroups than CUs: split every query block's key tiles over up to
    // 2 * CUs workgroups in all (partials in the workspace, then a combine kernel).  Fewer than
    // the kernel's resident slots (4, 2 and 1 per CU at head_dim 32, 48-64 and 96-128) with rows
    // of at least 1024 keys: split up to the slots.  Shorter rows do not repay the partials'
    // traffic and the combine (a 16-shard ring hop of 256 keys: 31 against 39 us per hop).
    const int64_t nwg = B * H * ((L + 127) / 128);
    const int64_t key_tiles = (vlen + 31) / 32;
    const int64_t cus = cu_count();
    const int64_t slots = cus * (D <= 32 ? 4 : D <= 64 ? 2 : 1);
    if (nwg < cus && key_tiles > 1)
      p.nsplit = (int)std::min<int64_t>(key_tiles, (2 * cus + nwg - 1) / nwg);
    else if (nwg < slots && key_tiles >= 32)
      p.nsplit = (int)std::min<int64_t>(key_tiles, (slots + nwg - 1) / nwg);
    if (p.nsplit > 1) p.total = align256((size_t)p.nsplit * B * H * L * (D + 1) * sizeof(float));
  }
  return p;
}

int fwd_check(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0) return AFA_ERR_SHAPE;
  if (batch * heads > INT32_MAX / 4 || seq_len > (INT32_MAX >> 2)) return AFA_ERR_SHAPE;
  if (head_dim > 128 && head_dim % 128 != 0) return AFA_ERR_HEAD_DIM;
  return AFA_OK;
}

// ---------------------------------------------------------------------------------- backward
// Workspace of afa_bwd (256-byte aligned regions): E and 1/d per row (every path); on the
// bf16 / fp16 matrix-core path the fast-rho guard's q and k bounds (2 B H ceil(L/64) floats) and,
// with rotary tables, the rotated q and k (2 B H L D elements).
struct BwdPlan {
  bool mfma16 = false;
  size_t e = 0, qbm = 0, kbm = 0, rot = 0, total = 0;
};

BwdPlan bwd_plan(int dtype, int64_t B, int64_t H, int64_t L, int64_t D, bool rotary, bool mfma_ok) {
  BwdPlan p;
  // E and 1/d per row; each head's rows padded to a multiple of 4 (the matrix-core kernels load
  // them in 16-byte chunks)
  size_t off = align256((size_t)(B * H * ((L + 3) / 4 * 4)) * acc_size(dtype) * 2);
  if (mfma_ok) {
    p.mfma16 = true;
    const size_t nb = align256((size_t)(B * H * ((L + 63) / 64)) * sizeof(float));
    p.qbm = off;
    p.kbm = off + nb;
    off += 2 * nb;
    if (rotary) {
      p.rot = off;
      off += align256((size_t)(B * H * L * D) * 2 * 2);
    }
  }
  p.total = off;
  return p;
}

}  // namespace

extern "C" {

size_t afa_fwd_workspace_size(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                              int rotary) {
  if (fwd_check(dtype, batch, heads, seq_len, head_dim) != AFA_OK) return 0;
  const bool in_head = (seq_len - 1) * head_dim + head_dim < (int64_t(1) << 31);
  // the larger of the default plan and the key-shard one (which never takes the fully fused
  // kernel, so it may need the pipelined kernels' workspace where the default plan does not)
  return std::max(
      fwd_plan(dtype, batch, heads, seq_len, head_dim, seq_len, rotary != 0, true, true, in_head, 0, -1).total,
      fwd_plan(dtype, batch, heads, seq_len, head_dim, seq_len, rotary != 0, true, true, in_head,
               AFA_FLAG_ACCUMULATE, -1).total);
}

int afa_fwd(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
            const void* q, const void* k, const void* v, const int64_t* strides, void* out,
            void* denom, const void* rot_cos, const void* rot_sin, int64_t rot_len,
            double sink_omega, int causal, int64_t valid_len, unsigned flags, void* workspace,
            size_t workspace_bytes, void* stream) {
  int rc = fwd_check(dtype, batch, heads, seq_len, head_dim);
  if (rc != AFA_OK) return rc;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return AFA_ERR_NULL;
  if (!finite_nonneg(sink_omega)) return AFA_ERR_SINK;
  if (valid_len < 0 || valid_len > seq_len) return AFA_ERR_VALID_LEN;
  rc = check_rotary(rot_cos, rot_sin, rot_len, seq_len, head_dim);
  if (rc != AFA_OK) return rc;
  const unsigned shard_flags = flags & (AFA_FLAG_ACCUMULATE | AFA_FLAG_PARTIAL);
  if (shard_flags == (AFA_FLAG_ACCUMULATE | AFA_FLAG_PARTIAL)) return AFA_ERR_UNSUPPORTED;
  const int acc = shard_flags == AFA_FLAG_PARTIAL ? afa::ACC_STORE : shard_flags ? afa::ACC_ADD : afa::ACC_NONE;
  if (acc && denom == nullptr) return AFA_ERR_NULL;  // the row sums' array
  if (acc && sink_omega != 0.0) return AFA_ERR_SINK;  // the sink belongs to the final division
  const int vlen = valid_len == 0 ? (int)seq_len : (int)valid_len;
  const Strides st = resolve_strides(strides, heads, seq_len, head_dim);
  hipStream_t s = (hipStream_t)stream;

  // 16-byte vector loads/stores: 8-element aligned strides and 16-byte aligned bases
  bool mfma_layout = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                     (rot_cos == nullptr || (aligned16(rot_cos) && aligned16(rot_sin)));
  for (int i = 0; i < 12; ++i)
    if (st.v[i] % 8 != 0) mfma_layout = false;
  bool f32_layout = aligned16(v) && aligned16(out);
  for (int i : {6, 7, 8, 9, 10, 11})
    if (st.v[i] % 4 != 0) f32_layout = false;
  auto in_head_32 = [&](int64_t row_stride) {
    return row_stride >= 0 && (seq_len - 1) * row_stride + head_dim < (int64_t(1) << 31);
  };
  const FwdPlan plan = fwd_plan(dtype, batch, heads, seq_len, head_dim, vlen, rot_cos != nullptr, mfma_layout,
                                f32_layout, in_head_32(st.v[5]) && in_head_32(st.v[8]), flags, causal ? 1 : 0);

  char* ws = (char*)workspace;
  bool owned = false;
  if (plan.total > 0) {
    if (ws == nullptr) {
      ws = (char*)scratch_alloc(plan.total, s);
      if (ws == nullptr) return hip_status(hipErrorOutOfMemory);
      owned = true;
    } else if (workspace_bytes < plan.total) {
      return AFA_ERR_WORKSPACE;
    } else if (!aligned16(ws)) {
      return AFA_ERR_ALIGN;
    }
  }

  afa::FwdArgs a = {};
  a.q = q; a.k = k; a.v = v; a.out = out; a.denom = (float*)denom;
  a.rc = (const float*)rot_cos; a.rs = (const float*)rot_sin;
  a.q_b = st.v[0]; a.q_h = st.v[1]; a.q_l = st.v[2];
  a.k_b = st.v[3]; a.k_h = st.v[4]; a.k_l = st.v[5];
  a.v_b = st.v[6]; a.v_h = st.v[7]; a.v_l = st.v[8];
  a.o_b = st.v[9]; a.o_h = st.v[10]; a.o_l = st.v[11];
  a.B = (int)batch; a.H = (int)heads; a.L = (int)seq_len;
  a.valid_len = vlen;
  a.causal = causal ? 1 : 0;
  a.acc = acc;
  a.omega = (float)sink_omega;
  a.q_scale = 1.0f;
  a.w_unscale = 1.0f;
  a.s_mult = 1.0f;
  // the branch-free rho^8 runs only on tiles the fast-rho guard clears, unless the caller asks
  // for the two-branch form everywhere
  const bool exact = (flags & AFA_FLAG_EXACT_TAIL) != 0;
  hipError_t e = hipSuccess;
  if (plan.kind == FWD_PIPE || plan.kind == FWD_FUSED) {
    float* kbm = (float*)(ws + plan.kbm);
    int* ks_cnt = nullptr;
    int nks_cnt = 0;
    if (plan.ks.tiles > 0) {
      a.ks_tiles = plan.ks.tiles;
      a.ks_q0 = plan.ks.q0;
      a.ks_pmax = plan.ks.pmax;
      a.ks_items = plan.ks.items;
      a.ks_part = (float*)(ws + plan.ks_part);
      a.ks_cnt = ks_cnt = (int*)(ws + plan.ks_cnt);
      nks_cnt = (int)(plan.ks.cnt_bytes / sizeof(int));
    }
    if (plan.rotk) {
      // a.k, a.kbm now the rotated k
      e = afa::krot_launch(dtype, (int)head_dim, a, ws + plan.krot, kbm, s, ks_cnt, nks_cnt);
    } else if (!exact) {
      e = afa::rownorm_launch(dtype, k, st.v[3], st.v[4], st.v[5], a.B, a.H, a.L, (int)head_dim, kbm, s, ks_cnt,
                              nks_cnt);
      a.kbm = kbm;
      a.nkb = (a.L + 63) / 64;
    }
    if (e == hipSuccess) {
      if (plan.kind == FWD_FUSED) {
        a.nqb = (int)((seq_len + afa::mfma_fwd_queries_per_block((int)head_dim) - 1) /
                      afa::mfma_fwd_queries_per_block((int)head_dim));
        e = afa::mfma_fwd_launch(dtype, (int)head_dim, a, exact, s);
      } else if (plan.wide) {
        a.nqb = (int)((seq_len + 255) / 256);
        e = afa::d64_fwd_launch(dtype, a, exact, s);
      } else {
        e = afa::pipe_fwd_launch(dtype, (int)head_dim, a, exact, s);
      }
    }
  } else if (plan.kind == FWD_F32) {
    a.q_scale = (float)(1.0 / std::sqrt((double)head_dim));
    a.part = plan.nsplit > 1 ? (float*)(ws + plan.part) : nullptr;
    e = afa::f32_fwd_launch((int)head_dim, a, plan.nsplit, s);
  } else {
    if (head_dim > 256) {
      if (owned) (void)hipFreeAsync(ws, s);
      return AFA_ERR_UNSUPPORTED;
    }
    afa::GenArgs g = {};
    g.q = q; g.k = k; g.v = v; g.out = out; g.denom = denom;
    g.rc = rot_cos; g.rs = rot_sin;
    g.q_b = st.v[0]; g.q_h = st.v[1]; g.q_l = st.v[2];
    g.k_b = st.v[3]; g.k_h = st.v[4]; g.k_l = st.v[5];
    g.v_b = st.v[6]; g.v_h = st.v[7]; g.v_l = st.v[8];
    g.o_b = st.v[9]; g.o_h = st.v[10]; g.o_l = st.v[11];
    g.B = (int)batch; g.H = (int)heads; g.L = (int)seq_len; g.D = (int)head_dim;
    g.valid_len = vlen;
    g.causal = causal ? 1 : 0;
    g.exact_ref = (flags & AFA_FLAG_EXACT_REF) ? 1 : 0;
    g.acc = acc;
    g.scale = 1.0 / std::sqrt((double)head_dim);
    if (dtype != AFA_F64) g.scale = (double)(float)g.scale;
    g.omega = dtype == AFA_F64 ? sink_omega : (double)(float)sink_omega;
    e = afa::generic_fwd_launch(dtype, g, s);
  }
  if (owned) {
    hipError_t e2 = hipFreeAsync(ws, s);
    if (e == hipSuccess) e = e2;
  }
  return hip_status(e);
}

int afa_ring_finish(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                    const void* acc, const void* denom, const int64_t* strides, double sink_omega,
                    void* out, void* total, void* stream) {
  int rc = fwd_check(dtype, batch, heads, seq_len, head_dim);
  if (rc != AFA_OK) return rc;
  if (acc == nullptr || denom == nullptr || out == nullptr) return AFA_ERR_NULL;
  if (!finite_nonneg(sink_omega)) return AFA_ERR_SINK;
  if ((batch * heads * seq_len * head_dim + 255) / 256 >= (int64_t(1) << 31)) return AFA_ERR_SHAPE;
  afa::RingFinish r = {};
  r.acc = acc; r.denom = denom; r.out = out; r.total = total;
  const int64_t dense[9] = {heads * seq_len * head_dim, seq_len * head_dim, head_dim,
                            heads * seq_len * head_dim, seq_len * head_dim, head_dim,
                            heads * seq_len, seq_len, 1};
  const int64_t* sv = strides != nullptr ? strides : dense;
  r.a_b = sv[0]; r.a_h = sv[1]; r.a_l = sv[2];
  r.o_b = sv[3]; r.o_h = sv[4]; r.o_l = sv[5];
  r.t_b = sv[6]; r.t_h = sv[7]; r.t_l = sv[8];
  r.B = (int)batch; r.H = (int)heads; r.L = (int)seq_len; r.D = (int)head_dim;
  r.sink = sink_omega;
  return hip_status(afa::ring_finish_launch(dtype, r, (hipStream_t)stream));
}

size_t afa_bwd_workspace_size(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                              int rotary) {
  if (!valid_dtype(dtype) || batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  return bwd_plan(dtype, batch, heads, seq_len, head_dim, rotary != 0,
                  afa::mfma_bwd_supported(dtype, (int)head_dim, seq_len)).total;
}

int afa_bwd(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
            const void* q, const void* k, const void* v, const void* out, const void* denom,
            const void* g, void* dq, void* dk, void* dv, const void* rot_cos,
            const void* rot_sin, int64_t rot_len, double sink_omega, int causal,
            int64_t valid_len, unsigned flags, void* workspace, size_t workspace_bytes,
            void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!q || !k || !v || !out || !denom || !g || !dq || !dk || !dv) return AFA_ERR_NULL;
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0) return AFA_ERR_SHAPE;
  if (batch * heads * ((seq_len + 31) / 32) > INT32_MAX) return AFA_ERR_SHAPE;
  if (head_dim > 128 && head_dim % 128 != 0) return AFA_ERR_HEAD_DIM;
  if (head_dim > 256) return AFA_ERR_UNSUPPORTED;
  if (!finite_nonneg(sink_omega)) return AFA_ERR_SINK;
  if (valid_len < 0 || valid_len > seq_len) return AFA_ERR_VALID_LEN;
  int rc = check_rotary(rot_cos, rot_sin, rot_len, seq_len, head_dim);
  if (rc != AFA_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const bool aligned = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(g) &&
                       aligned16(dq) && aligned16(dk) && aligned16(dv) && aligned16(denom) &&
                       (workspace == nullptr || aligned16(workspace));
  const bool use_mfma = !(flags & AFA_FLAG_GENERIC) && aligned &&
                        afa::mfma_bwd_supported(dtype, (int)head_dim, seq_len) &&
                        (rot_cos == nullptr || (aligned16(rot_cos) && aligned16(rot_sin)));
  // fp32: the fp32 matrix-core kernels (q and k rotated as they are staged)
  const bool use_f32 = dtype == AFA_F32 && !(flags & AFA_FLAG_GENERIC) && aligned &&
                       afa::f32_bwd_supported((int)head_dim);
  const BwdPlan plan = bwd_plan(dtype, batch, heads, seq_len, head_dim, rot_cos != nullptr, use_mfma);
  char* ws = (char*)workspace;
  bool owned = false;
  if (ws == nullptr) {
    ws = (char*)scratch_alloc(plan.total, s);
    if (ws == nullptr) return hip_status(hipErrorOutOfMemory);
    owned = true;
  } else if (workspace_bytes < plan.total) {
    return AFA_ERR_WORKSPACE;
  }
  afa::GenArgs a = {};
  a.q = q; a.k = k; a.v = v; a.out_in = out; a.dtot = denom; a.g = g;
  a.out = dq; a.dk = dk; a.dv = dv; a.e_ws = ws + plan.e;
  a.rc = rot_cos; a.rs = rot_sin;
  a.B = (int)batch; a.H = (int)heads; a.L = (int)seq_len; a.D = (int)head_dim;
  a.valid_len = valid_len == 0 ? (int)seq_len : (int)valid_len;
  a.causal = causal ? 1 : 0;
  a.scale = 1.0 / std::sqrt((double)head_dim);
  if (dtype != AFA_F64) a.scale = (double)(float)a.scale;
  a.omega = sink_omega;
  const bool exact = (flags & AFA_FLAG_EXACT_TAIL) != 0;
  hipError_t e;
  if (use_mfma) {
    a.qbm = (const float*)(ws + plan.qbm);
    a.kbm = (const float*)(ws + plan.kbm);
    e = afa::mfma_bwd_launch(dtype, a, exact, rot_cos != nullptr ? ws + plan.rot : nullptr, s);
  } else {
    e = use_f32 ? afa::f32_bwd_launch(a, s) : afa::generic_bwd_launch(dtype, a, s);
  }
  if (owned) {
    hipError_t e2 = hipFreeAsync(ws, s);
    if (e == hipSuccess) e = e2;
  }
  return hip_status(e);
}

int asoftmax_fwd(int dtype, int64_t rows, int64_t cols, const void* x, void* y,
                 double sink_omega, double eps, void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!x || !y) return AFA_ERR_NULL;
  if (rows <= 0 || cols <= 0) return AFA_ERR_SHAPE;
  if (!finite_nonneg(sink_omega)) return AFA_ERR_SINK;
  if (!(eps > 0.0 && eps < INFINITY)) return AFA_ERR_EPS;
  return hip_status(afa::asoftmax_fwd_launch(dtype, rows, cols, x, y, sink_omega, eps, (hipStream_t)stream));
}

int asoftmax_bwd(int dtype, int64_t rows, int64_t cols, const void* x, const void* g, void* dx,
                 double sink_omega, double eps, void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!x || !g || !dx) return AFA_ERR_NULL;
  if (rows <= 0 || cols <= 0) return AFA_ERR_SHAPE;
  if (!finite_nonneg(sink_omega)) return AFA_ERR_SINK;
  if (!(eps > 0.0 && eps < INFINITY)) return AFA_ERR_EPS;
  return hip_status(afa::asoftmax_bwd_launch(dtype, rows, cols, x, g, dx, sink_omega, eps, (hipStream_t)stream));
}

int octic_fwd(int dtype, int64_t n, const void* x, void* y, void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!x || !y) return AFA_ERR_NULL;
  if (n < 0) return AFA_ERR_SHAPE;
  if (n == 0) return AFA_OK;
  return hip_status(afa::octic_fwd_launch(dtype, n, x, y, (hipStream_t)stream));
}

int octic_fwd_r(int dtype, int64_t n, const void* x, void* k, void* r, void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!x || !k || !r) return AFA_ERR_NULL;
  if (n < 0) return AFA_ERR_SHAPE;
  if (n == 0) return AFA_OK;
  return hip_status(afa::octic_fwd_r_launch(dtype, n, x, k, r, (hipStream_t)stream));
}

int octic_bwd(int dtype, int64_t n, const void* x, const void* g, void* dx, void* stream) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!x || !g || !dx) return AFA_ERR_NULL;
  if (n < 0) return AFA_ERR_SHAPE;
  if (n == 0) return AFA_OK;
  return hip_status(afa::octic_bwd_launch(dtype, n, x, g, dx, (hipStream_t)stream));
}

int ago_build_tables(int table_dtype, int64_t dim, int64_t max_seq_len, const void* freqs,
                     double base, void* cos_out, void* sin_out, void* stream) {
  if (table_dtype != AFA_F32 && table_dtype != AFA_F64) return AFA_ERR_DTYPE;
  if (!cos_out || !sin_out) return AFA_ERR_NULL;
  if (dim <= 0 || dim % 2 != 0 || max_seq_len <= 0 || max_seq_len > INT32_MAX) return AFA_ERR_SHAPE;
  return hip_status(afa::ago_tables_launch(table_dtype, (int)(dim / 2), (int)max_seq_len,
                                           freqs, base, cos_out, sin_out,
                                           (hipStream_t)stream));
}

int ago_rotate(int dtype, int64_t outer, int64_t seq_len, int64_t inner, int64_t dim,
               const void* x, void* y, int table_dtype, const void* rot_cos,
               const void* rot_sin, int64_t rot_len, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(table_dtype)) return AFA_ERR_DTYPE;
  if (!x || !y || !rot_cos || !rot_sin) return AFA_ERR_NULL;
  if (outer <= 0 || seq_len <= 0 || inner <= 0 || dim <= 0) return AFA_ERR_SHAPE;
  if (dim % 2 != 0 || rot_len < seq_len) return AFA_ERR_ROTARY;
  return hip_status(afa::ago_rotate_launch(dtype, table_dtype, outer, seq_len, inner, (int)dim, x, y,
                                           rot_cos, rot_sin, (hipStream_t)stream));
}

// ------------------------------------------------------------------------------ OACE
}  // extern "C"

namespace {

int oace_check(int dtype, int64_t rows, int64_t d, int64_t V, const void* h, int64_t ldh, const void* w,
               int layout, int64_t ldw, const int64_t* targets, double eps, double gamma) {
  if (!valid_dtype(dtype)) return AFA_ERR_DTYPE;
  if (!h || !w || !targets) return AFA_ERR_NULL;
  if (rows <= 0 || d <= 0 || V <= 0 || rows > INT32_MAX || V > INT32_MAX || d > INT32_MAX) return AFA_ERR_SHAPE;
  if (layout != OACE_W_DV && layout != OACE_W_VD) return AFA_ERR_SHAPE;
  if (ldh < d || ldw < (layout == OACE_W_DV ? V : d)) return AFA_ERR_SHAPE;
  if (!(eps >= 0.0 && eps < INFINITY)) return AFA_ERR_EPS;
  if (!(gamma > 0.0 && gamma < INFINITY)) return AFA_ERR_GAMMA;
  return AFA_OK;
}

afa::OaceArgs oace_args(int64_t rows, int64_t d, int64_t V, const void* h, int64_t ldh, const void* w, int layout,
                        int64_t ldw, const int64_t* targets, double eps, double gamma) {
  afa::OaceArgs a = {};
  a.N = rows;
  a.d = d;
  a.V = V;
  a.h = h;
  a.ldh = ldh;
  a.w = w;
  a.w_layout = layout;
  a.ldw = ldw;
  a.targets = targets;
  a.eps = eps;
  a.gamma = gamma;
  return a;
}

size_t oace_rows_bytes(int dtype, int64_t rows) {
  return ((size_t)rows * OACE_ROW_FIELDS * acc_size(dtype) + 255) & ~(size_t)255;
}

size_t oace_path_bytes(int dtype, const afa::OaceArgs& a, bool use_mfma) {
  if (use_mfma) return afa::oace_mfma_workspace(dtype, a);
  return std::max(afa::oace_generic_workspace(dtype, a.N, a.d, a.V, false),
                  afa::oace_generic_workspace(dtype, a.N, a.d, a.V, true));
}

// Workspace: [row records | path scratch]; the first part is unused when the caller passes
// row_cache.  Size from the dimensions only, the larger of the two paths.
size_t oace_ws_size(int dtype, const afa::OaceArgs& a) {
  return oace_rows_bytes(dtype, a.N) + std::max(oace_path_bytes(dtype, a, false), oace_path_bytes(dtype, a, true));
}

}  // namespace

extern "C" {

size_t oace_workspace_size(int dtype, int64_t rows, int64_t d_model, int64_t vocab, int w_layout, unsigned flags) {
  if (!valid_dtype(dtype) || rows <= 0 || d_model <= 0 || vocab <= 0) return 0;
  afa::OaceArgs a = oace_args(rows, d_model, vocab, nullptr, d_model, nullptr, w_layout,
                              w_layout == OACE_W_DV ? vocab : d_model, nullptr, 0.0, 1.0);
  a.flags = flags & OACE_FLAG_RECOMPUTE_Z;
  return oace_ws_size(dtype, a);
}

int oace_linear_fwd(int dtype, int64_t rows, int64_t d_model, int64_t vocab, const void* h, int64_t ldh,
                    const void* w, int w_layout, int64_t ldw, const int64_t* targets, double eps_vocab,
                    double gamma, void* loss, void* row_cache, unsigned flags, void* workspace,
                    size_t workspace_bytes, void* stream) {
  int rc = oace_check(dtype, rows, d_model, vocab, h, ldh, w, w_layout, ldw, targets, eps_vocab, gamma);
  if (rc != AFA_OK) return rc;
  if (!loss) return AFA_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  afa::OaceArgs a = oace_args(rows, d_model, vocab, h, ldh, w, w_layout, ldw, targets, eps_vocab, gamma);
  a.loss = loss;
  a.flags = flags & ~OACE_FLAG_WT_READY;
  const size_t need = oace_ws_size(dtype, a);
  void* ws = workspace;
  bool owned = false;
  if (ws == nullptr) {
    ws = scratch_alloc(need, s);
    if (ws == nullptr) return hip_status(hipErrorOutOfMemory);
    owned = true;
  } else if (workspace_bytes < need) {
    return AFA_ERR_WORKSPACE;
  }
  void* recs = row_cache ? row_cache : ws;
  void* scratch = (char*)ws + oace_rows_bytes(dtype, rows);
  const bool mfma = !(flags & AFA_FLAG_GENERIC) && afa::oace_mfma_supported(dtype, a);
  hipError_t e = mfma ? afa::oace_linear_fwd_mfma(dtype, a, recs, scratch, s)
                      : afa::oace_linear_fwd_generic(dtype, a, recs, scratch, s);
  if (owned) {
    hipError_t e2 = hipFreeAsync(ws, s);
    if (e == hipSuccess) e = e2;
  }
  return hip_status(e);
}

int oace_linear_bwd(int dtype, int64_t rows, int64_t d_model, int64_t vocab, const void* h, int64_t ldh,
                    const void* w, int w_layout, int64_t ldw, const int64_t* targets, double gamma,
                    const void* row_cache, const void* g_loss, void* dh, void* dw, unsigned flags, void* workspace,
                    size_t workspace_bytes, void* stream) {
  int rc = oace_check(dtype, rows, d_model, vocab, h, ldh, w, w_layout, ldw, targets, 0.0, gamma);
  if (rc != AFA_OK) return rc;
  if (!row_cache || !dh || !dw) return AFA_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  afa::OaceArgs a = oace_args(rows, d_model, vocab, h, ldh, w, w_layout, ldw, targets, 0.0, gamma);
  a.g_loss = g_loss;
  a.dh = dh;
  a.dw = dw;
  a.flags = workspace != nullptr ? flags : flags & ~(OACE_FLAG_WT_READY | OACE_FLAG_Z_READY);
  const size_t need = oace_ws_size(dtype, a);
  void* ws = workspace;
  bool owned = false;
  if (ws == nullptr) {
    ws = scratch_alloc(need, s);
    if (ws == nullptr) return hip_status(hipErrorOutOfMemory);
    owned = true;
  } else if (workspace_bytes < need) {
    return AFA_ERR_WORKSPACE;
  }
  void* scratch = (char*)ws + oace_rows_bytes(dtype, rows);
  const bool mfma = !(flags & AFA_FLAG_GENERIC) && afa::oace_mfma_supported(dtype, a);
  hipError_t e = mfma ? afa::oace_linear_bwd_mfma(dtype, a, row_cache, scratch, s)
                      : afa::oace_linear_bwd_generic(dtype, a, row_cache, scratch, s);
  if (owned) {
    hipError_t e2 = hipFreeAsync(ws, s);
    if (e == hipSuccess) e = e2;
  }
  return hip_status(e);
}

int oace_softmax_loss_fwd(int dtype, int64_t rows, int64_t vocab, const void* logits, const int64_t* targets,
                          double eps, double gamma, void* loss, void* row_cache, void* stream) {
  int rc = oace_check(dtype, rows, vocab, vocab, logits, vocab, logits, OACE_W_VD, vocab, targets, eps, gamma);
  if (rc != AFA_OK) return rc;
  if (!loss) return AFA_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  afa::OaceArgs a = oace_args(rows, vocab, vocab, logits, vocab, nullptr, OACE_W_VD, vocab, targets, eps, gamma);
  a.loss = loss;
  void* recs = row_cache;
  bool owned = false;
  if (recs == nullptr) {
    recs = scratch_alloc(oace_rows_bytes(dtype, rows), s);
    if (recs == nullptr) return hip_status(hipErrorOutOfMemory);
    owned = true;
  }
  hipError_t e = afa::oace_softmax_fwd_launch(dtype, a, recs, s);
  if (owned) {
    hipError_t e2 = hipFreeAsync(recs, s);
    if (e == hipSuccess) e = e2;
  }
  return hip_status(e);
}

int oace_softmax_loss_bwd(int dtype, int64_t rows, int64_t vocab, const void* logits, const int64_t* targets,
                          double gamma, const void* row_cache, const void* g_loss, void* dlogits, void* stream) {
  int rc = oace_check(dtype, rows, vocab, vocab, logits, vocab, logits, OACE_W_VD, vocab, targets, 0.0, gamma);
  if (rc != AFA_OK) return rc;
  if (!row_cache || !dlogits) return AFA_ERR_NULL;
  afa::OaceArgs a = oace_args(rows, vocab, vocab, logits, vocab, nullptr, OACE_W_VD, vocab, targets, 0.0, gamma);
  a.g_loss = g_loss;
  return hip_status(afa::oace_softmax_bwd_launch(dtype, a, row_cache, dlogits, (hipStream_t)stream));
}

}  // extern "C"
