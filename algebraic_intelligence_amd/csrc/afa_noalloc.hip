// afa_fwd_noalloc: afa_fwd with its workspace in a fixed per-device array of this library, for
// callers that cannot allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).  It allocates nothing: no hipMalloc, hipFree, pool or torch
// allocation, on any call.
//
// The workspace is `scratch`, a file-scope __device__ array of AFA_NOALLOC_SCRATCH_BYTES; every
// GPU the library runs on holds its own copy until the process ends.  Host code never uses the
// array's name as a device address: on the first call on each device (with that device current)
// hipGetSymbolAddress gives the copy's address, which is kept per device and passed to afa_fwd.
// Nothing in the workspace has to start at zero: every region afa_fwd uses (the rotated k, the
// fast-rho key bounds, the fp32 split-K partials) is written in full by the call before it is
// read, and the key split's per-block counters, which do count from zero, are cleared by a kernel
// of the same call (the norm or K-rotation pre-pass) before the attention kernel runs.  All calls
// on one device share its array, so calls that overlap on one device (on
// different streams, or from several threads without ordering) race; calls ordered on one
// stream do not.
#include <mutex>

#include "../../include/afa.h"
#include "afa_launch.h"

static __device__ __align__(256) unsigned char scratch[AFA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// Address of the current device's copy of `scratch`, looked up once per device; nullptr (and the
// HIP error in *err) if the lookup failed.
void* scratch_address(hipError_t* err) {
  static std::once_flag once[kMaxDevices];
  static void* addr[kMaxDevices];
  static hipError_t status[kMaxDevices];
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *err = e != hipSuccess ? e : hipErrorInvalidDevice;
    return nullptr;
  }
  std::call_once(once[dev], [dev]() {
    void* p = nullptr;
    status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr[dev] = status[dev] == hipSuccess ? p : nullptr;
  });
  *err = status[dev];
  return addr[dev];
}

}  // namespace

extern "C" int afa_fwd_noalloc(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                               const void* q, const void* k, const void* v, const int64_t* strides, void* out,
                               void* denom, const void* rot_cos, const void* rot_sin, int64_t rot_len,
                               double sink_omega, int causal, int64_t valid_len, unsigned flags, void* stream) {
  // a call whose workspace would exceed the array is refused before any device work
  const size_t need = afa_fwd_workspace_size(dtype, batch, heads, seq_len, head_dim, rot_cos != nullptr);
  if (need > (size_t)AFA_NOALLOC_SCRATCH_BYTES) return AFA_ERR_SCRATCH_LIMIT;
  hipError_t e = hipSuccess;
  void* ws = scratch_address(&e);
  if (ws == nullptr) {
    (void)hipGetLastError();
    return afa::hip_status_code(e);
  }
  return afa_fwd(dtype, batch, heads, seq_len, head_dim, q, k, v, strides, out, denom, rot_cos, rot_sin,
                 rot_len, sink_omega, causal, valid_len, flags, ws, (size_t)AFA_NOALLOC_SCRATCH_BYTES, stream);
}
