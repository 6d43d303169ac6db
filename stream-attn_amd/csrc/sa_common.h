// Shared host-side helpers of libseqattn_hip: thread-local error text and
// HIP status propagation.  No exception crosses the C ABI: every failure is a
// return code plus a message readable through sa_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "seqattn_hip.h"

namespace sa {

void set_error(const char* fmt, ...);
void clear_error();

// Converts a hipError_t into the ABI convention (0 or a positive code) and
// records a message naming the failing call.
int32_t hip_status(hipError_t err, const char* what);

// Makes `device` current for the lifetime of the guard and restores the
// caller's device afterwards (torch tracks its own current device per thread).
// status() reports a failure to query or select the device; callers return
// it before enqueueing anything.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    status_ = hipGetDevice(&previous_);
    if (status_ == hipSuccess && previous_ != device) {
      status_ = hipSetDevice(device);
      changed_ = status_ == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (changed_) (void)hipSetDevice(previous_);  // nothing to report from a destructor
  }
  hipError_t status() const { return status_; }
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int previous_ = 0;
  bool changed_ = false;
  hipError_t status_ = hipSuccess;
};

}  // namespace sa

#define SA_HIP_RETURN(call)                                  \
  do {                                                       \
    hipError_t sa_err_ = (call);                             \
    if (sa_err_ != hipSuccess) return sa::hip_status(sa_err_, #call); \
  } while (0)

// Kernel entry points shared between the kernel and pipeline translation units.
namespace sa {
// Output of an update launch that also finalizes its rows (launch_update with
// SA_FLAG_INITIALIZE over all keys): out [q_tokens, q_heads, head_dim] with
// strides (so_t, so_h, 1); lse element (h, t) at lse[h * lse_sh + lse_off + t]
// when lse is non-null.
struct FusedOutput {
  void* out;
  int64_t so_t, so_h;
  float* lse;
  int64_t lse_sh, lse_off;
};
int32_t launch_update(const void* q, const void* k, const void* v, float* m, float* l, float* acc,
                      int64_t sq_t, int64_t sq_h, int64_t sk_t, int64_t sk_h, int64_t sv_t,
                      int64_t sv_h, int64_t ss_t, int64_t ss_h, int64_t sa_t, int64_t sa_h,
                      int32_t q_tokens, int32_t kv_tokens, int32_t q_heads, int32_t kv_heads,
                      int32_t head_dim, int32_t q_local_offset, int32_t kv_local_offset,
                      int32_t causal_shift, double softmax_scale, int32_t flags, int32_t dtype,
                      hipStream_t stream, int32_t merge_keys = 0,
                      const FusedOutput* fused = nullptr, bool v_transposed = false,
                      bool tiled_state = false);
// V [kv_tokens, kv_heads, 128] -> vt [kv_heads][128][t_pad] in the key order
// the update kernel's transposed-V variant reads, zero keys up to t_pad.
int32_t launch_transpose_v(const void* v, int64_t sv_t, int64_t sv_h, int32_t kv_tokens, int32_t kv_heads,
                           int32_t head_dim, void* vt, int64_t t_pad, hipStream_t stream);
int32_t launch_update_int8(const void* q, const void* k, const void* v, const void* k_scales,
                           const void* v_scales, float* m, float* l, float* acc, int64_t sq_t,
                           int64_t sq_h, int64_t sk_t, int64_t sk_h, int64_t sv_t, int64_t sv_h,
                           int64_t sks_g, int64_t sks_h, int64_t svs_g, int64_t svs_h,
                           int64_t ss_t, int64_t ss_h, int64_t sa_t, int64_t sa_h,
                           int32_t q_tokens, int32_t kv_tokens, int32_t q_heads, int32_t kv_heads,
                           int32_t head_dim, int32_t q_local_offset, int32_t kv_local_offset,
                           int32_t storage_token_offset, int32_t causal_shift,
                           double softmax_scale, int32_t flags, int32_t dtype,
                           int32_t quant_group_tokens, hipStream_t stream, bool tiled_state = false);
int32_t launch_finalize(const float* acc, const float* m, const float* l, void* out, float* lse,
                        int64_t sa_t, int64_t sa_h, int64_t ss_t, int64_t ss_h, int64_t so_t,
                        int64_t so_h, int64_t lse_sh, int64_t lse_off, int32_t q_tokens,
                        int32_t q_heads, int32_t head_dim, int32_t dtype, hipStream_t stream,
                        bool tiled_state = false);
// tiled_state: m, l and acc are the pipeline's own buffers in the row-group
// layout (16-row groups, lane order; see the update kernels), not strided.

// Queries per workgroup of the update kernel for this head_dim: launches that
// split a Q block split it at a multiple of this.
int32_t update_block_rows(int32_t head_dim);
}  // namespace sa
