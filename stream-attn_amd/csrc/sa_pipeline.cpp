// Transfer pipeline of the streamed exact-attention path: caller-pinned host
// Q/K/V -> HBM workspace (resident Q super-block + K/V ring) -> update and
// finalize kernels -> pinned host output.
//
// The fence graph follows TritonExecutorMixin._run_triton (reference
// src/seqattn_core/streaming/executor.py:18-188) and CudaWorkspace
// (src/seqattn_core/streaming/workspace.py:8-50):
//   H2D stream : [wait q_free] Q copy, record q_ready;
//                per K/V chunk [wait kv_free[slot]] K,V copies, record kv_ready[slot]
//   compute    : wait q_ready; per chunk wait kv_ready[slot], update launch,
//                record kv_free[slot]; record q_free (unless output reuses Q);
//                [wait out_free[slot]] finalize; record out_ready[slot]
//   D2H stream : wait out_ready[slot], output copy, record out_free[slot]
//                (and q_free when the output lives in the Q buffer)
// Copies are hipMemcpyAsync on two dedicated default-priority streams, so
// PCIe traffic in both directions overlaps the kernels on the compute stream.
//
// The FP32 state (m, l, acc) of the pipeline is kept in the update kernel's
// row-group layout (16-row groups in lane order), which the kernels and the
// finalize of this file read and write; the buffers must therefore hold the
// Q block's rows rounded up to a multiple of 16.
//
// Streamed chunks of a Q block of at least 512 rows are applied by two
// launches, one per half of the block's rows: the first on the compute
// stream, the second on the pipeline's own `side` stream (default priority).
// A span forks `side` from the compute stream and joins it back, and a slot
// is refilled only after both halves recorded their kv_free events.  The two
// halves' launches run concurrently, so one launch's partial last round of
// workgroups overlaps the other's work instead of leaving CUs idle.  Every
// row's arithmetic is that of a single launch: results are bit-identical.

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <new>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "sa_common.h"

namespace sa {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int32_t hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return 0;
  set_error("%s failed: %s (%d)", what, hipGetErrorString(err), (int)err);
  return (int32_t)err > 0 ? (int32_t)err : 1;
}

}  // namespace sa

namespace {

// Host-side trace ranges named like the reference's NVTX ranges
// (streaming/executor.py: seqattn:q_h2d, kv_h2d, fused_update,
// fused_finalize, output_d2h), bracketing the enqueue of each stage.  The
// ROCm tracer API is resolved with dlopen when ranges are first enabled, so
// the library has no link-time dependency on it.
struct TraceApi {
  int (*push)(const char*) = nullptr;
  int (*pop)() = nullptr;
};

const TraceApi& trace_api() {
  static const TraceApi api = [] {
    TraceApi a;
    for (const char* name : {"librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so", "libroctx64.so.4",
                             "libroctx64.so"}) {
      void* handle = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (!handle) continue;
      a.push = reinterpret_cast<int (*)(const char*)>(dlsym(handle, "roctxRangePushA"));
      a.pop = reinterpret_cast<int (*)()>(dlsym(handle, "roctxRangePop"));
      if (a.push && a.pop) break;
      a = TraceApi();
    }
    return a;
  }();
  return api;
}

class TraceRange {
 public:
  TraceRange(bool enabled, const char* name) : on_(enabled && trace_api().push) {
    if (on_) trace_api().push(name);
  }
  ~TraceRange() {
    if (on_) trace_api().pop();
  }
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;

 private:
  bool on_;
};

}  // namespace

struct sa_pipeline {
  int device = 0;
  void* q_buffer = nullptr;
  void* k_slots[3] = {nullptr, nullptr, nullptr};
  void* v_slots[3] = {nullptr, nullptr, nullptr};
  int num_kv = 0;
  // INT8 K/V: per ring slot, one fp16 scale per (row, K/V head) for K and V.
  void* ks_slots[3] = {nullptr, nullptr, nullptr};
  void* vs_slots[3] = {nullptr, nullptr, nullptr};
  bool has_scales = false;
  float* m = nullptr;
  float* l = nullptr;
  float* acc = nullptr;
  void* out_slots[2] = {nullptr, nullptr};
  bool has_out_slots = false;
  int num_out = 0;
  int q_chunk = 0, kv_chunk = 0, q_heads = 0, kv_heads = 0, head_dim = 0, dtype = 0;
  int64_t q_row_bytes = 0, kv_row_bytes = 0;

  hipStream_t h2d = nullptr, d2h = nullptr;
  bool owns_streams = false;
  hipEvent_t q_ready = nullptr, q_free = nullptr;
  hipEvent_t kv_ready[3] = {}, kv_free[3] = {};
  // Second half of a split chunk update: its stream, the slot-free events it
  // records, and the span's fork / join events.
  hipStream_t side = nullptr;
  hipEvent_t kv_free_side[3] = {};
  hipEvent_t fork = nullptr, join = nullptr;
  bool kv_side_pending[3] = {false, false, false};
  // Caller-owned device scratch for a transposed copy of V in HBM-resident
  // runs (sa_pipeline_attach_resident_scratch); null when none is attached.
  void* vt_scratch = nullptr;
  int64_t vt_scratch_bytes = 0;
  hipEvent_t out_ready[2] = {}, out_free[2] = {};
  // sa_pipeline_run with one output slot: the Q block buffer and the output
  // slot take turns as a pass's Q block and output (ready: Q copied in;
  // done: output finalized; free: output copied out).
  hipEvent_t alt_ready[2] = {}, alt_done[2] = {}, alt_free[2] = {};
  // sa_pipeline_run without output slots (host_aliased): per row piece of
  // the Q block, its output written (done), copied out (out) and the next
  // block's Q rows copied in (ready).
  static constexpr int kPieces = 4;
  hipEvent_t piece_done[kPieces] = {}, piece_out[kPieces] = {}, piece_ready[kPieces] = {};
  bool q_pending = false;
  bool kv_pending[3] = {false, false, false};
  bool out_pending[2] = {false, false};
  int64_t ring_next = 0;  // next K/V ring slot (rotates across calls)

  // Head-group schedule (sa_pipeline_create_head_groups).  A unit is every
  // token of a group of K/V heads and their query heads; each buffer set
  // holds one unit's Q (then its output), K, V and optionally V transposed.
  // Per set: ready (the unit's copies landed), done (its output written),
  // free (its output copied out).
  bool head_groups = false;
  static constexpr int kMaxSets = 2;
  int num_sets = 0, group_kv = 0;
  int64_t hg_max_q = 0, hg_max_kv = 0, hg_vt_bytes = 0;
  void* set_qo[kMaxSets] = {}, *set_k[kMaxSets] = {}, *set_v[kMaxSets] = {}, *set_vt[kMaxSets] = {};
  hipEvent_t set_ready[kMaxSets] = {}, set_done[kMaxSets] = {}, set_free[kMaxSets] = {};
  bool set_pending[kMaxSets] = {false, false};
  // Page-locked host staging for a pageable output
  // (sa_pipeline_attach_host_staging).
  void* staging = nullptr;
  int64_t staging_bytes = 0;

  // Host-side trace ranges around each stage's enqueue (sa_pipeline_set_trace_ranges).
  bool trace = false;
  // Optional timing of update launches (event pairs on the compute stream).
  bool timing = false;
  std::vector<hipEvent_t> t_start, t_stop;
  size_t t_used = 0;
};

namespace {

void add_stats(sa_pipeline_stats* st, int64_t h2d, int64_t d2h, int64_t qc, int64_t kvt,
               int64_t resident) {
  if (!st) return;
  st->h2d_bytes += h2d;
  st->d2h_bytes += d2h;
  st->q_chunks += qc;
  st->kv_tiles += kvt;
  st->max_resident_q_tokens = std::max(st->max_resident_q_tokens, resident);
}

// Teardown: failures here cannot be acted on, so their codes are dropped.
void release(sa_pipeline* p) {
  if (p->h2d) (void)hipStreamSynchronize(p->h2d);
  if (p->d2h) (void)hipStreamSynchronize(p->d2h);
  if (p->side) (void)hipStreamSynchronize(p->side);
  hipEvent_t* evs[] = {&p->q_ready, &p->q_free, &p->fork, &p->join};
  for (hipEvent_t* e : evs)
    if (*e) (void)hipEventDestroy(*e);
  for (int i = 0; i < 3; ++i) {
    if (p->kv_ready[i]) (void)hipEventDestroy(p->kv_ready[i]);
    if (p->kv_free[i]) (void)hipEventDestroy(p->kv_free[i]);
    if (p->kv_free_side[i]) (void)hipEventDestroy(p->kv_free_side[i]);
  }
  for (int i = 0; i < 2; ++i) {
    if (p->out_ready[i]) (void)hipEventDestroy(p->out_ready[i]);
    if (p->out_free[i]) (void)hipEventDestroy(p->out_free[i]);
    if (p->alt_ready[i]) (void)hipEventDestroy(p->alt_ready[i]);
    if (p->alt_done[i]) (void)hipEventDestroy(p->alt_done[i]);
    if (p->alt_free[i]) (void)hipEventDestroy(p->alt_free[i]);
  }
  for (int i = 0; i < sa_pipeline::kPieces; ++i) {
    if (p->piece_done[i]) (void)hipEventDestroy(p->piece_done[i]);
    if (p->piece_out[i]) (void)hipEventDestroy(p->piece_out[i]);
    if (p->piece_ready[i]) (void)hipEventDestroy(p->piece_ready[i]);
  }
  for (int i = 0; i < sa_pipeline::kMaxSets; ++i) {
    if (p->set_ready[i]) (void)hipEventDestroy(p->set_ready[i]);
    if (p->set_done[i]) (void)hipEventDestroy(p->set_done[i]);
    if (p->set_free[i]) (void)hipEventDestroy(p->set_free[i]);
  }
  for (hipEvent_t e : p->t_start) (void)hipEventDestroy(e);
  for (hipEvent_t e : p->t_stop) (void)hipEventDestroy(e);
  if (p->owns_streams) {
    if (p->h2d) (void)hipStreamDestroy(p->h2d);
    if (p->d2h) (void)hipStreamDestroy(p->d2h);
  }
  if (p->side) (void)hipStreamDestroy(p->side);
}

// Make the H2D stream wait until ring slot `slot` is no longer read by any
// launch (both halves of a split update).
int32_t wait_slot_free(sa_pipeline* p, int slot) {
  if (p->kv_pending[slot]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->kv_free[slot], 0));
  if (p->kv_side_pending[slot]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->kv_free_side[slot], 0));
  return 0;
}

int32_t load_q(sa_pipeline* p, const void* q_host, int32_t q_tokens, hipStream_t compute,
               sa_pipeline_stats* st) {
  if (q_tokens < 0 || q_tokens > p->q_chunk) {
    sa::set_error("q_tokens %d outside [0, q_chunk_tokens=%d]", q_tokens, p->q_chunk);
    return SA_ERR_INVALID_ARGUMENT;
  }
  TraceRange range(p->trace, "seqattn:q_h2d");
  const int64_t bytes = (int64_t)q_tokens * p->q_row_bytes;
  if (p->q_pending) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->q_free, 0));
  if (bytes > 0)
    SA_HIP_RETURN(hipMemcpyAsync(p->q_buffer, q_host, bytes, hipMemcpyHostToDevice, p->h2d));
  SA_HIP_RETURN(hipEventRecord(p->q_ready, p->h2d));
  SA_HIP_RETURN(hipStreamWaitEvent(compute, p->q_ready, 0));
  add_stats(st, bytes, 0, 1, 0, q_tokens);
  return 0;
}

// One update launch over rows [start, start + n) of a K/V span, optionally
// bracketed by timing events.
int32_t launch_timed(sa_pipeline* p, const void* q, int64_t sq_t, int64_t sq_h, const void* k,
                     int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_t, int64_t sv_h,
                     int32_t q_tokens, int32_t kv_tokens, int32_t q_local_offset,
                     int32_t kv_local_offset, int32_t causal_shift, double scale, int32_t flags,
                     hipStream_t compute, int32_t merge_keys = 0,
                     const sa::FusedOutput* fused = nullptr, int32_t state_row = 0,
                     bool v_transposed = false) {
  TraceRange range(p->trace, "seqattn:fused_update");
  if (p->timing) {
    if (p->t_used == p->t_start.size()) {
      hipEvent_t a = nullptr, b = nullptr;
      SA_HIP_RETURN(hipEventCreate(&a));
      SA_HIP_RETURN(hipEventCreate(&b));
      p->t_start.push_back(a);
      p->t_stop.push_back(b);
    }
    SA_HIP_RETURN(hipEventRecord(p->t_start[p->t_used], compute));
  }
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  const int64_t srow = (int64_t)state_row * p->q_heads;
  int32_t rc = sa::launch_update(q, k, v, p->m + srow, p->l + srow, p->acc + srow * p->head_dim, sq_t,
                                 sq_h, sk_t, sk_h, sv_t, sv_h,
                                 p->q_heads, 1, qt, p->head_dim, q_tokens, kv_tokens, p->q_heads,
                                 p->kv_heads, p->head_dim, q_local_offset, kv_local_offset,
                                 causal_shift, scale, flags, p->dtype, compute, merge_keys, fused,
                                 v_transposed, /*tiled_state=*/true);
  if (rc != 0) return rc;
  if (p->timing) SA_HIP_RETURN(hipEventRecord(p->t_stop[p->t_used++], compute));
  return 0;
}

// The INT8 K/V update over ring slot `slot` (int8 rows, per-row scales),
// optionally bracketed by timing events.
int32_t launch_timed_int8(sa_pipeline* p, int slot, int32_t q_tokens, int32_t kv_tokens,
                          int32_t q_local_offset, int32_t kv_local_offset, int32_t causal_shift,
                          double scale, int32_t flags, hipStream_t compute) {
  TraceRange range(p->trace, "seqattn:fused_update");
  if (p->timing) {
    if (p->t_used == p->t_start.size()) {
      hipEvent_t a = nullptr, b = nullptr;
      SA_HIP_RETURN(hipEventCreate(&a));
      SA_HIP_RETURN(hipEventCreate(&b));
      p->t_start.push_back(a);
      p->t_stop.push_back(b);
    }
    SA_HIP_RETURN(hipEventRecord(p->t_start[p->t_used], compute));
  }
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  const int64_t kt = (int64_t)p->kv_heads * p->head_dim;
  int32_t rc = sa::launch_update_int8(
      p->q_buffer, p->k_slots[slot], p->v_slots[slot], p->ks_slots[slot], p->vs_slots[slot], p->m,
      p->l, p->acc, qt, p->head_dim, kt, p->head_dim, kt, p->head_dim, p->kv_heads, 1, p->kv_heads, 1,
      p->q_heads, 1, qt, p->head_dim, q_tokens, kv_tokens, p->q_heads, p->kv_heads, p->head_dim,
      q_local_offset, kv_local_offset, 0, causal_shift, scale, flags, p->dtype, 1, compute,
      /*tiled_state=*/true);
  if (rc != 0) return rc;
  if (p->timing) SA_HIP_RETURN(hipEventRecord(p->t_stop[p->t_used++], compute));
  return 0;
}

// Where the K/V rows of a span live: pinned host rows copied through the ring
// (tensor and paged modes), or device rows read in place (HBM-resident mode).
struct KVSource {
  const char* k;
  const char* v;
  bool on_device;
  int64_t sk_t, sk_h, sv_t, sv_h;  // element strides, used when on_device
};

// Joins the side stream back into the compute stream when a split span ends,
// including an early return on error, so that nothing enqueued later on the
// compute stream can overlap the second half's launches.
struct SideJoin {
  sa_pipeline* p;
  hipStream_t compute;
  bool active = false;
  int32_t finish() {
    if (!active) return 0;
    active = false;
    SA_HIP_RETURN(hipEventRecord(p->join, p->side));
    SA_HIP_RETURN(hipStreamWaitEvent(compute, p->join, 0));
    return 0;
  }
  ~SideJoin() { (void)finish(); }
};

// Apply K/V rows [kv_local_offset, kv_local_offset + kv_tokens) of one segment
// to the resident Q block, kv_chunk_tokens rows per launch.  `initialize` is
// true while the state still has to be defined by the next launch; it is
// cleared by the first launch.  Keys at or beyond `visible_end` are masked for
// every query of the block under the bottom-right causal rule; their chunks
// change nothing and are neither copied nor launched, except that a chunk
// always runs while the state is uninitialized.  `after_copy`, if given, is
// called with the chunk's ordinal once its H2D copies are enqueued, so the
// caller can slot other H2D work between chunks.  `fused_last`, if given,
// describes the output (and LSE) of row 0 of the block: the span's last
// launch then writes acc / l and the LSE in its epilogue instead of storing
// the state, with the finalize kernel's expressions, and *fused_done is set.
// The caller runs the finalize kernel itself when no launch was made.
int32_t apply_span(sa_pipeline* p, const void* q, int64_t sq_t, int64_t sq_h, const KVSource& src,
                   int32_t kv_tokens, int32_t kv_local_offset, bool* initialize,
                   int32_t q_tokens, int32_t q_local_offset, int32_t causal_shift, double scale,
                   int32_t causal, hipStream_t compute, sa_pipeline_stats* st,
                   const std::function<int32_t(int32_t)>* after_copy = nullptr,
                   const sa::FusedOutput* fused_last = nullptr, bool* fused_done = nullptr) {
  if (kv_tokens < 0 || kv_local_offset < 0 || q_tokens < 0 || q_tokens > p->q_chunk) {
    sa::set_error("bad K/V span kv_tokens=%d kv_local_offset=%d q_tokens=%d", kv_tokens,
                  kv_local_offset, q_tokens);
    return SA_ERR_INVALID_ARGUMENT;
  }
  int64_t visible_end = INT64_MAX;
  if (causal) visible_end = std::max<int64_t>(0, (int64_t)q_local_offset + q_tokens + causal_shift);
  const int64_t kt = (int64_t)p->kv_heads * p->head_dim;
  // Rows [0, split) update on the compute stream, [split, q_tokens) on side;
  // split is a multiple of the kernel's workgroup tile.
  const int32_t tile = sa::update_block_rows(p->head_dim);
  const int32_t split = (!src.on_device && q_tokens >= 2 * tile) ? (q_tokens / 2 + tile - 1) / tile * tile : q_tokens;
  const bool two = split < q_tokens && kv_tokens > 0;
  const char* q_second = static_cast<const char*>(q) + (int64_t)split * sq_t * 2;
  // Start of the last chunk the loop below launches (-1: none).
  int64_t last_start = -1;
  {
    bool init = *initialize;
    for (int32_t start = 0; start < kv_tokens; start += p->kv_chunk) {
      if (!init && (int64_t)kv_local_offset + start >= visible_end) break;
      last_start = start;
      init = false;
    }
  }
  sa::FusedOutput out_first{}, out_second{};
  if (fused_last != nullptr) {
    out_first = *fused_last;
    out_second = *fused_last;
    out_second.out = static_cast<char*>(fused_last->out) + (int64_t)split * fused_last->so_t * 2;
    out_second.lse_off = fused_last->lse_off + split;
  }
  SideJoin join{p, compute};
  if (two) {
    SA_HIP_RETURN(hipEventRecord(p->fork, compute));
    SA_HIP_RETURN(hipStreamWaitEvent(p->side, p->fork, 0));
    join.active = true;
  }
  for (int32_t start = 0; start < kv_tokens; start += p->kv_chunk) {
    const int64_t position = (int64_t)kv_local_offset + start;
    if (!*initialize && position >= visible_end) break;
    const int32_t n = std::min(p->kv_chunk, kv_tokens - start);
    const int32_t flags = (causal ? SA_FLAG_CAUSAL : 0) | (*initialize ? SA_FLAG_INITIALIZE : 0);
    const bool fuse = fused_last != nullptr && start == last_start;
    if (fuse && fused_done) *fused_done = true;
    int32_t rc;
    if (src.on_device) {
      rc = launch_timed(p, q, sq_t, sq_h, src.k + start * src.sk_t * 2, src.sk_t, src.sk_h,
                        src.v + start * src.sv_t * 2, src.sv_t, src.sv_h, q_tokens, n,
                        q_local_offset, (int32_t)position, causal_shift, scale, flags, compute, 0,
                        fuse ? &out_first : nullptr);
      if (rc != 0) return rc;
      add_stats(st, 0, 0, 0, 1, 0);
    } else {
      const int slot = (int)(p->ring_next++ % p->num_kv);
      const int64_t bytes = (int64_t)n * p->kv_row_bytes;
      {
        TraceRange range(p->trace, "seqattn:kv_h2d");
        int32_t wrc = wait_slot_free(p, slot);
        if (wrc != 0) return wrc;
        SA_HIP_RETURN(hipMemcpyAsync(p->k_slots[slot], src.k + (int64_t)start * p->kv_row_bytes,
                                     bytes, hipMemcpyHostToDevice, p->h2d));
        SA_HIP_RETURN(hipMemcpyAsync(p->v_slots[slot], src.v + (int64_t)start * p->kv_row_bytes,
                                     bytes, hipMemcpyHostToDevice, p->h2d));
        SA_HIP_RETURN(hipEventRecord(p->kv_ready[slot], p->h2d));
        add_stats(st, 2 * bytes, 0, 0, 1, 0);
      }
      if (after_copy) {
        const int32_t hrc = (*after_copy)(start / p->kv_chunk);
        if (hrc != 0) return hrc;
      }
      SA_HIP_RETURN(hipStreamWaitEvent(compute, p->kv_ready[slot], 0));
      rc = launch_timed(p, q, sq_t, sq_h, p->k_slots[slot], kt, p->head_dim, p->v_slots[slot], kt,
                        p->head_dim, split, n, q_local_offset, (int32_t)position, causal_shift,
                        scale, flags, compute, 0, fuse ? &out_first : nullptr);
      if (rc != 0) return rc;
      SA_HIP_RETURN(hipEventRecord(p->kv_free[slot], compute));
      p->kv_pending[slot] = true;
      if (two) {
        SA_HIP_RETURN(hipStreamWaitEvent(p->side, p->kv_ready[slot], 0));
        rc = launch_timed(p, q_second, sq_t, sq_h, p->k_slots[slot], kt, p->head_dim, p->v_slots[slot], kt,
                          p->head_dim, q_tokens - split, n, q_local_offset + split, (int32_t)position,
                          causal_shift, scale, flags, p->side, 0, fuse ? &out_second : nullptr, split);
        if (rc != 0) return rc;
        SA_HIP_RETURN(hipEventRecord(p->kv_free_side[slot], p->side));
        p->kv_side_pending[slot] = true;
      }
    }
    *initialize = false;
  }
  return join.finish();
}

// Gathered span: consecutive segment positions [kv_local_offset, +total)
// whose host rows are split over `nfrag` contiguous fragments (one per page).
// Ring slots are filled fragment piece by fragment piece (one hipMemcpyAsync
// per piece and tensor), so page-sized host records feed chunk-sized kernel
// launches without a host-side copy.
//
// INT8 mode (ks_frags / vs_frags non-null): fragments hold int8 rows of
// kv_heads * head_dim bytes plus one fp16 scale per (row, K/V head); both are
// gathered into the ring slot and its scale slot, and the launch dequantizes
// in the kernel.
int32_t apply_gather(sa_pipeline* p, const void* const* k_frags, const void* const* v_frags,
                     const void* const* ks_frags, const void* const* vs_frags,
                     const int32_t* frag_tokens, int32_t nfrag, int32_t kv_local_offset,
                     bool* initialize, int32_t q_tokens, int32_t q_local_offset,
                     int32_t causal_shift, double scale, int32_t causal, hipStream_t compute,
                     sa_pipeline_stats* st) {
  const bool int8 = ks_frags != nullptr;
  if (int8 && (!vs_frags || !p->has_scales)) {
    sa::set_error("INT8 K/V gather needs scale fragments and a pipeline with scale slots");
    return SA_ERR_BAD_STATE;
  }
  int64_t total = 0;
  for (int32_t i = 0; i < nfrag; ++i) {
    if (frag_tokens[i] < 0 || (frag_tokens[i] > 0 && (!k_frags[i] || !v_frags[i])) ||
        (int8 && frag_tokens[i] > 0 && (!ks_frags[i] || !vs_frags[i]))) {
      sa::set_error("bad K/V fragment %d (%d tokens)", i, frag_tokens[i]);
      return SA_ERR_INVALID_ARGUMENT;
    }
    total += frag_tokens[i];
  }
  if (total > INT32_MAX || kv_local_offset < 0 || q_tokens < 0 || q_tokens > p->q_chunk) {
    sa::set_error("bad gathered K/V span (%lld tokens at %d, q_tokens %d)", (long long)total,
                  kv_local_offset, q_tokens);
    return SA_ERR_INVALID_ARGUMENT;
  }
  int64_t visible_end = INT64_MAX;
  if (causal) visible_end = std::max<int64_t>(0, (int64_t)q_local_offset + q_tokens + causal_shift);
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  const int64_t kt = (int64_t)p->kv_heads * p->head_dim;
  const int64_t row_bytes = int8 ? kt : p->kv_row_bytes;
  const int64_t scale_row_bytes = (int64_t)p->kv_heads * 2;
  int32_t frag = 0;       // fragment holding the next row
  int64_t frag_row = 0;   // rows of that fragment already consumed
  for (int64_t start = 0; start < total; start += p->kv_chunk) {
    const int64_t position = (int64_t)kv_local_offset + start;
    if (!*initialize && position >= visible_end) break;
    const int32_t n = (int32_t)std::min<int64_t>(p->kv_chunk, total - start);
    const int slot = (int)(p->ring_next++ % p->num_kv);
    char* kd = static_cast<char*>(p->k_slots[slot]);
    char* vd = static_cast<char*>(p->v_slots[slot]);
    {
      TraceRange kv_range(p->trace, "seqattn:kv_h2d");
      int32_t wrc = wait_slot_free(p, slot);
      if (wrc != 0) return wrc;
      int64_t filled = 0;
      while (filled < n) {
        while (frag < nfrag && frag_row >= frag_tokens[frag]) {
          ++frag;
          frag_row = 0;
        }
        const int64_t rows = std::min<int64_t>(n - filled, frag_tokens[frag] - frag_row);
        const int64_t bytes = rows * row_bytes;
        const int64_t src_off = frag_row * row_bytes;
        SA_HIP_RETURN(hipMemcpyAsync(kd + filled * row_bytes,
                                     static_cast<const char*>(k_frags[frag]) + src_off, bytes,
                                     hipMemcpyHostToDevice, p->h2d));
        SA_HIP_RETURN(hipMemcpyAsync(vd + filled * row_bytes,
                                     static_cast<const char*>(v_frags[frag]) + src_off, bytes,
                                     hipMemcpyHostToDevice, p->h2d));
        if (int8) {
          const int64_t sbytes = rows * scale_row_bytes;
          const int64_t ssrc = frag_row * scale_row_bytes;
          SA_HIP_RETURN(hipMemcpyAsync(static_cast<char*>(p->ks_slots[slot]) + filled * scale_row_bytes,
                                       static_cast<const char*>(ks_frags[frag]) + ssrc, sbytes,
                                       hipMemcpyHostToDevice, p->h2d));
          SA_HIP_RETURN(hipMemcpyAsync(static_cast<char*>(p->vs_slots[slot]) + filled * scale_row_bytes,
                                       static_cast<const char*>(vs_frags[frag]) + ssrc, sbytes,
                                       hipMemcpyHostToDevice, p->h2d));
        }
        filled += rows;
        frag_row += rows;
      }
      SA_HIP_RETURN(hipEventRecord(p->kv_ready[slot], p->h2d));
    }
    add_stats(st, 2 * (int64_t)n * (row_bytes + (int8 ? scale_row_bytes : 0)), 0, 0, 1, 0);
    SA_HIP_RETURN(hipStreamWaitEvent(compute, p->kv_ready[slot], 0));
    const int32_t flags = (causal ? SA_FLAG_CAUSAL : 0) | (*initialize ? SA_FLAG_INITIALIZE : 0);
    int32_t rc = int8 ? launch_timed_int8(p, slot, q_tokens, n, q_local_offset, (int32_t)position,
                                          causal_shift, scale, flags, compute)
                      : launch_timed(p, p->q_buffer, qt, p->head_dim, kd, kt, p->head_dim, vd, kt,
                                     p->head_dim, q_tokens, n, q_local_offset, (int32_t)position,
                                     causal_shift, scale, flags, compute);
    if (rc != 0) return rc;
    SA_HIP_RETURN(hipEventRecord(p->kv_free[slot], compute));
    p->kv_pending[slot] = true;
    *initialize = false;
  }
  return 0;
}

// Defines the state of a Q block that sees no keys at all (m = -inf, l = 0,
// acc = 0): an update launch with zero keys and the initialize flag.
int32_t init_state(sa_pipeline* p, const void* q, int64_t sq_t, int64_t sq_h, int32_t q_tokens,
                   int32_t q_local_offset, int32_t causal_shift, double scale,
                   hipStream_t compute) {
  if (q_tokens <= 0) return 0;
  const int64_t kt = (int64_t)p->kv_heads * p->head_dim;
  return launch_timed(p, q, sq_t, sq_h, p->k_slots[0], kt, p->head_dim, p->v_slots[0], kt,
                      p->head_dim, q_tokens, 0, q_local_offset, 0, causal_shift, scale,
                      SA_FLAG_INITIALIZE, compute);
}

// Copy K/V rows [0, n) of k_host / v_host into the next ring slot (after its
// last readers) and record its kv_ready event; *slot_out names the slot.
int32_t prefetch_chunk(sa_pipeline* p, const void* k_host, const void* v_host, int32_t n,
                       sa_pipeline_stats* st, int32_t* slot_out) {
  const int slot = (int)(p->ring_next++ % p->num_kv);
  const int64_t bytes = (int64_t)n * p->kv_row_bytes;
  TraceRange range(p->trace, "seqattn:kv_h2d");
  int32_t rc = wait_slot_free(p, slot);
  if (rc != 0) return rc;
  SA_HIP_RETURN(hipMemcpyAsync(p->k_slots[slot], k_host, bytes, hipMemcpyHostToDevice, p->h2d));
  SA_HIP_RETURN(hipMemcpyAsync(p->v_slots[slot], v_host, bytes, hipMemcpyHostToDevice, p->h2d));
  SA_HIP_RETURN(hipEventRecord(p->kv_ready[slot], p->h2d));
  add_stats(st, 2 * bytes, 0, 0, 1, 0);
  *slot_out = slot;
  return 0;
}

int32_t stream_kv(sa_pipeline* p, const void* k_host, const void* v_host, int32_t k_length,
                  int32_t q_tokens, int32_t q_local_offset, int32_t causal_shift, double scale,
                  int32_t causal, hipStream_t compute, sa_pipeline_stats* st,
                  const void* q_block = nullptr,
                  const std::function<int32_t(int32_t)>* after_copy = nullptr,
                  const sa::FusedOutput* fused_last = nullptr, bool* fused_done = nullptr) {
  if (k_length < 0 || q_tokens < 0 || q_tokens > p->q_chunk) {
    sa::set_error("bad stream_kv sizes k_length=%d q_tokens=%d", k_length, q_tokens);
    return SA_ERR_INVALID_ARGUMENT;
  }
  const void* q = q_block ? q_block : p->q_buffer;
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  KVSource src{static_cast<const char*>(k_host), static_cast<const char*>(v_host), false, 0, 0, 0, 0};
  bool initialize = true;
  int32_t rc = apply_span(p, q, qt, p->head_dim, src, k_length, 0, &initialize, q_tokens, q_local_offset,
                          causal_shift, scale, causal, compute, st, after_copy, fused_last, fused_done);
  if (rc != 0) return rc;
  if (initialize)
    return init_state(p, q, qt, p->head_dim, q_tokens, q_local_offset, causal_shift, scale, compute);
  return 0;
}

int32_t finalize(sa_pipeline* p, int32_t slot, int32_t q_tokens, float* lse, int64_t lse_sh,
                 int64_t lse_off, hipStream_t compute) {
  TraceRange range(p->trace, "seqattn:fused_finalize");
  void* dest;
  if (slot >= 0) {
    if (!p->has_out_slots || slot >= p->num_out) {
      sa::set_error("output slot %d unavailable (%d slots)", slot,
                    p->has_out_slots ? p->num_out : 0);
      return SA_ERR_INVALID_ARGUMENT;
    }
    SA_HIP_RETURN(hipEventRecord(p->q_free, compute));
    p->q_pending = true;
    if (p->out_pending[slot]) SA_HIP_RETURN(hipStreamWaitEvent(compute, p->out_free[slot], 0));
    dest = p->out_slots[slot];
  } else {
    dest = p->q_buffer;
  }
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  return sa::launch_finalize(p->acc, p->m, p->l, dest, lse, qt, p->head_dim, p->q_heads, 1, qt,
                             p->head_dim, lse_sh, lse_off, q_tokens, p->q_heads, p->head_dim,
                             p->dtype, compute, /*tiled_state=*/true);
}

int32_t d2h(sa_pipeline* p, void* dst, const void* src, int64_t bytes, int32_t slot,
            int32_t release_q, hipStream_t compute, sa_pipeline_stats* st) {
  if (slot < 0 || slot >= p->num_out) {
    sa::set_error("event slot %d outside [0, %d)", slot, p->num_out);
    return SA_ERR_INVALID_ARGUMENT;
  }
  TraceRange range(p->trace, "seqattn:output_d2h");
  SA_HIP_RETURN(hipEventRecord(p->out_ready[slot], compute));
  SA_HIP_RETURN(hipStreamWaitEvent(p->d2h, p->out_ready[slot], 0));
  if (bytes > 0) SA_HIP_RETURN(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, p->d2h));
  SA_HIP_RETURN(hipEventRecord(p->out_free[slot], p->d2h));
  p->out_pending[slot] = true;
  if (release_q) {
    SA_HIP_RETURN(hipEventRecord(p->q_free, p->d2h));
    p->q_pending = true;
  }
  add_stats(st, 0, bytes, 0, 0, 0);
  return 0;
}

// One Q block of sa_pipeline_run: rows [qt, qt + n) of the packed Q, with
// its segment's K/V rows [k_start, k_start + k_len).
struct Pass {
  int64_t qt, k_start;
  int32_t n, k_len, q_local, causal_shift;
};

// Rows per pass for a segment of q_length query rows: the pass count of
// q_chunk-row blocks, with the rows spread evenly over the passes in
// multiples of the update kernel's workgroup tile instead of a short last
// block.  A short pass applies every K/V chunk to few rows, so its
// chunk copies outrun its kernels; even passes keep each chunk's copy hidden
// behind its compute.  The pass count, and with it the H2D bytes, is that of
// q_chunk-row blocks.
int64_t pass_rows(int64_t q_length, int32_t q_chunk, int32_t tile) {
  if (q_length <= q_chunk) return q_chunk;
  const int64_t passes = (q_length + q_chunk - 1) / q_chunk;
  const int64_t even = (q_length + passes - 1) / passes;
  return std::min<int64_t>(q_chunk, (even + tile - 1) / tile * tile);
}

// sa_pipeline_run with one output slot.  The plan's two block-sized buffers
// (the Q block and the output slot) take turns: pass i reads its Q block from
// buffer i % 2, is finalized into that same buffer (its Q rows are no longer
// read by then) and copied out from it.  The next pass's Q block is copied
// into the other buffer during pass i, in four pieces placed between K/V
// chunk copies spread over the pass, so each piece fits in the slack of the
// K/V ring.  A pass therefore starts as soon as the previous one is
// finalized: its Q block and first K/V chunks are already in HBM.  Memory and
// decomposition are the plan's; only the order of the copies changes.
int32_t run_alternating(sa_pipeline* p, const char* qh, const char* kh, const char* vh, char* oh,
                        float* lse, int64_t lse_sh, const std::vector<Pass>& passes, double scale,
                        int32_t causal, hipStream_t compute, sa_pipeline_stats* st) {
  constexpr int kPieces = 4;
  void* buf[2] = {p->q_buffer, p->out_slots[0]};
  bool pending[2] = {false, false};  // a copy-out from the buffer was enqueued
  // Work another entry point left on these buffers completes first.
  if (p->q_pending) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->q_free, 0));
  if (p->out_pending[0]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->out_free[0], 0));
  auto copy_piece = [&](size_t i, int j) -> int32_t {
    const Pass& ps = passes[i];
    const int b = (int)(i & 1);
    TraceRange range(p->trace, "seqattn:q_h2d");
    if (j == 0 && pending[b]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->alt_free[b], 0));
    const int64_t r0 = (int64_t)ps.n * j / kPieces, r1 = (int64_t)ps.n * (j + 1) / kPieces;
    const int64_t bytes = (r1 - r0) * p->q_row_bytes;
    if (bytes > 0)
      SA_HIP_RETURN(hipMemcpyAsync(static_cast<char*>(buf[b]) + r0 * p->q_row_bytes,
                                   qh + (ps.qt + r0) * p->q_row_bytes, bytes, hipMemcpyHostToDevice, p->h2d));
    const bool last = j == kPieces - 1;
    add_stats(st, bytes, 0, last ? 1 : 0, 0, last ? ps.n : 0);
    if (last) SA_HIP_RETURN(hipEventRecord(p->alt_ready[b], p->h2d));
    return 0;
  };
  int32_t rc = 0;
  if (!passes.empty()) {
    for (int j = 0; j < kPieces && rc == 0; ++j) rc = copy_piece(0, j);
    if (rc) return rc;
  }
  const int64_t q_stride = (int64_t)p->q_heads * p->head_dim;
  for (size_t i = 0; i < passes.size(); ++i) {
    const Pass& ps = passes[i];
    const int b = (int)(i & 1);
    const bool has_next = i + 1 < passes.size();
    // The next pass's Q block goes into the buffer whose output the previous
    // pass is still copying out, and the H2D stream runs in order, so piece 0
    // waits for that copy and every K/V chunk copy after it waits too.  The
    // pieces therefore follow chunks spread over the pass (after chunk
    // (j + 1) * chunks / 5 for piece j), which leaves the output copy a fifth
    // of the pass to finish before anything waits for it.
    int64_t chunks = 0;
    {
      const int64_t visible_end =
          causal ? std::max<int64_t>(0, (int64_t)ps.q_local + ps.n + ps.causal_shift) : INT64_MAX;
      for (int64_t start = 0; start < ps.k_len; start += p->kv_chunk) {
        if (chunks > 0 && start >= visible_end) break;
        ++chunks;
      }
    }
    int next_piece = 0;
    std::function<int32_t(int32_t)> between_chunks = [&](int32_t ordinal) -> int32_t {
      while (has_next && next_piece < kPieces &&
             ordinal >= std::max<int64_t>(1, (next_piece + 1) * chunks / (kPieces + 1))) {
        const int32_t prc = copy_piece(i + 1, next_piece++);
        if (prc != 0) return prc;
      }
      return 0;
    };
    SA_HIP_RETURN(hipStreamWaitEvent(compute, p->alt_ready[b], 0));
    // The pass's last chunk launches write the output into the pass's own Q
    // buffer (each query row is read and written by one wave only) and the
    // LSE, in place of a state store and a finalize launch.
    const sa::FusedOutput fused{buf[b], q_stride, p->head_dim, lse, lse_sh, ps.qt};
    bool fused_done = false;
    rc = stream_kv(p, kh + ps.k_start * p->kv_row_bytes, vh + ps.k_start * p->kv_row_bytes, ps.k_len, ps.n,
                   ps.q_local, ps.causal_shift, scale, causal, compute, st, buf[b], &between_chunks, &fused,
                   &fused_done);
    if (rc) return rc;
    while (has_next && next_piece < kPieces)
      if ((rc = copy_piece(i + 1, next_piece++)) != 0) return rc;
    {
      TraceRange range(p->trace, "seqattn:fused_finalize");
      if (!fused_done) {
        rc = sa::launch_finalize(p->acc, p->m, p->l, buf[b], lse, q_stride, p->head_dim, p->q_heads, 1, q_stride,
                                 p->head_dim, lse_sh, ps.qt, ps.n, p->q_heads, p->head_dim, p->dtype, compute,
                                 /*tiled_state=*/true);
        if (rc) return rc;
      }
      SA_HIP_RETURN(hipEventRecord(p->alt_done[b], compute));
    }
    const int64_t bytes = (int64_t)ps.n * p->q_row_bytes;
    {
      TraceRange range(p->trace, "seqattn:output_d2h");
      SA_HIP_RETURN(hipStreamWaitEvent(p->d2h, p->alt_done[b], 0));
      if (bytes > 0)
        SA_HIP_RETURN(hipMemcpyAsync(oh + ps.qt * p->q_row_bytes, buf[b], bytes, hipMemcpyDeviceToHost, p->d2h));
      SA_HIP_RETURN(hipEventRecord(p->alt_free[b], p->d2h));
    }
    pending[b] = true;
    add_stats(st, 0, bytes, 0, 0, 0);
  }
  SA_HIP_RETURN(hipStreamSynchronize(p->d2h));
  return 0;
}

// sa_pipeline_run without output slots (output_mode="host_aliased").  A
// pass's output is written into its own Q block and copied out from there,
// and the next pass's Q block is copied into the same buffer, so between two
// passes the block crosses the link twice while no update can run on it.
// That boundary is worked in row pieces of the block (multiples of the
// update kernel's workgroup tile):
//  - the pass's last K/V chunk is applied to one piece at a time, and each
//    piece's output is copied out as soon as its launch ends;
//  - the next pass's first K/V chunk is copied before its Q block, and its Q
//    rows of a piece are copied in as soon as the output rows they overwrite
//    have left;
//  - that first chunk is applied to each piece as its Q rows land.
// The chunks in between are applied to the whole block (apply_span).  Every
// row sees the same chunks in the same order as with one launch per chunk,
// so the results are bit-identical.
int32_t run_aliased(sa_pipeline* p, const char* qh, const char* kh, const char* vh, char* oh, float* lse,
                    int64_t lse_sh, const std::vector<Pass>& passes, double scale, int32_t causal,
                    hipStream_t compute, sa_pipeline_stats* st) {
  constexpr int kP = sa_pipeline::kPieces;
  if (passes.empty()) return 0;
  const int32_t tile = sa::update_block_rows(p->head_dim);
  const int64_t q_stride = (int64_t)p->q_heads * p->head_dim;
  const int64_t kt = (int64_t)p->kv_heads * p->head_dim;
  char* qbuf = static_cast<char*>(p->q_buffer);
  // Row bounds r[0..np] of the pieces of an n-row block (n > 0).
  auto piece_bounds = [&](int32_t n, int32_t* r) -> int {
    const int32_t tiles = (n + tile - 1) / tile;
    const int np = std::max(1, std::min(kP, (int)tiles));
    for (int j = 0; j <= np; ++j)
      r[j] = j == np ? n : std::min<int32_t>(n, (int32_t)((int64_t)tiles * j / np) * tile);
    return np;
  };
  // Work another entry point left on the Q buffer completes first.
  if (p->q_pending) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->q_free, 0));
  int32_t r_out[kP + 1] = {};
  int np_out = 0;  // pieces whose output copies are the last enqueued (0: none)
  auto copy_q = [&](const Pass& ps, const int32_t* r, int np) -> int32_t {
    TraceRange range(p->trace, "seqattn:q_h2d");
    for (int j = 0; j < np; ++j) {
      if (np_out > 0) {
        // The output copies run in order on the D2H stream: waiting for the
        // last one that overlaps rows [r[j], r[j+1]) covers all of them.
        int k = 0;
        while (k + 1 < np_out && r_out[k + 1] < r[j + 1]) ++k;
        SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->piece_out[k], 0));
      }
      const int64_t bytes = (int64_t)(r[j + 1] - r[j]) * p->q_row_bytes;
      if (bytes > 0)
        SA_HIP_RETURN(hipMemcpyAsync(qbuf + r[j] * p->q_row_bytes, qh + (ps.qt + r[j]) * p->q_row_bytes, bytes,
                                     hipMemcpyHostToDevice, p->h2d));
      SA_HIP_RETURN(hipEventRecord(p->piece_ready[j], p->h2d));
    }
    add_stats(st, (int64_t)ps.n * p->q_row_bytes, 0, 1, 0, ps.n);
    return 0;
  };
  // One chunk of K/V rows [start, start + n_k) of pass ps, applied to each
  // piece on the compute stream.  first: each piece first waits for its Q
  // rows; last: each piece writes its output (and LSE) and records
  // piece_done.
  auto pieces_chunk = [&](const Pass& ps, const int32_t* r, int np, int slot, int32_t start, int32_t n_k,
                          bool first, bool last) -> int32_t {
    SA_HIP_RETURN(hipStreamWaitEvent(compute, p->kv_ready[slot], 0));
    const int32_t flags = (causal ? SA_FLAG_CAUSAL : 0) | (first ? SA_FLAG_INITIALIZE : 0);
    for (int j = 0; j < np; ++j) {
      if (first) SA_HIP_RETURN(hipStreamWaitEvent(compute, p->piece_ready[j], 0));
      const sa::FusedOutput fused{qbuf + r[j] * p->q_row_bytes, q_stride, p->head_dim, lse, lse_sh, ps.qt + r[j]};
      const int32_t rc = launch_timed(p, qbuf + r[j] * p->q_row_bytes, q_stride, p->head_dim, p->k_slots[slot], kt,
                                      p->head_dim, p->v_slots[slot], kt, p->head_dim, r[j + 1] - r[j], n_k,
                                      ps.q_local + r[j], start, ps.causal_shift, scale, flags, compute, 0,
                                      last ? &fused : nullptr, r[j]);
      if (rc != 0) return rc;
      if (last) SA_HIP_RETURN(hipEventRecord(p->piece_done[j], compute));
    }
    SA_HIP_RETURN(hipEventRecord(p->kv_free[slot], compute));
    p->kv_pending[slot] = true;
    p->kv_side_pending[slot] = false;
    return 0;
  };
  int32_t rc = 0;
  int32_t r[kP + 1], r_next[kP + 1];
  int np = piece_bounds(passes[0].n, r);
  int32_t slot0 = -1;
  rc = prefetch_chunk(p, kh + passes[0].k_start * p->kv_row_bytes, vh + passes[0].k_start * p->kv_row_bytes,
                      std::min<int32_t>(p->kv_chunk, passes[0].k_len), st, &slot0);
  if (rc) return rc;
  if ((rc = copy_q(passes[0], r, np)) != 0) return rc;
  for (size_t i = 0; i < passes.size(); ++i) {
    const Pass& ps = passes[i];
    const bool has_next = i + 1 < passes.size();
    // Chunks the block applies: the first always, later ones while some row
    // of the block can see them (bottom-right causal rule).
    const int64_t visible_end =
        causal ? std::max<int64_t>(0, (int64_t)ps.q_local + ps.n + ps.causal_shift) : INT64_MAX;
    int32_t last_start = 0;
    for (int32_t start = p->kv_chunk; start < ps.k_len && start < visible_end; start += p->kv_chunk)
      last_start = start;
    const int32_t n_first = std::min<int32_t>(p->kv_chunk, ps.k_len);
    const bool single = last_start == 0;
    if ((rc = pieces_chunk(ps, r, np, slot0, 0, n_first, true, single)) != 0) return rc;
    if (!single) {
      if (last_start > p->kv_chunk) {
        KVSource src{kh + (ps.k_start + p->kv_chunk) * p->kv_row_bytes,
                     vh + (ps.k_start + p->kv_chunk) * p->kv_row_bytes, false, 0, 0, 0, 0};
        bool initialize = false;
        rc = apply_span(p, qbuf, q_stride, p->head_dim, src, last_start - p->kv_chunk, p->kv_chunk, &initialize,
                        ps.n, ps.q_local, ps.causal_shift, scale, causal, compute, st);
        if (rc) return rc;
      }
      int32_t slot = -1;
      rc = prefetch_chunk(p, kh + (ps.k_start + last_start) * p->kv_row_bytes,
                          vh + (ps.k_start + last_start) * p->kv_row_bytes,
                          std::min<int32_t>(p->kv_chunk, ps.k_len - last_start), st, &slot);
      if (rc) return rc;
      rc = pieces_chunk(ps, r, np, slot, last_start, std::min<int32_t>(p->kv_chunk, ps.k_len - last_start), false,
                        true);
      if (rc) return rc;
    }
    int np_next = 0;
    if (has_next) {
      const Pass& nx = passes[i + 1];
      np_next = piece_bounds(nx.n, r_next);
      rc = prefetch_chunk(p, kh + nx.k_start * p->kv_row_bytes, vh + nx.k_start * p->kv_row_bytes,
                          std::min<int32_t>(p->kv_chunk, nx.k_len), st, &slot0);
      if (rc) return rc;
    }
    {
      TraceRange range(p->trace, "seqattn:output_d2h");
      for (int j = 0; j < np; ++j) {
        SA_HIP_RETURN(hipStreamWaitEvent(p->d2h, p->piece_done[j], 0));
        const int64_t bytes = (int64_t)(r[j + 1] - r[j]) * p->q_row_bytes;
        if (bytes > 0)
          SA_HIP_RETURN(hipMemcpyAsync(oh + (ps.qt + r[j]) * p->q_row_bytes, qbuf + r[j] * p->q_row_bytes, bytes,
                                       hipMemcpyDeviceToHost, p->d2h));
        SA_HIP_RETURN(hipEventRecord(p->piece_out[j], p->d2h));
      }
      add_stats(st, 0, (int64_t)ps.n * p->q_row_bytes, 0, 0, 0);
    }
    np_out = np;
    std::copy(r, r + np + 1, r_out);
    if (has_next) {
      if ((rc = copy_q(passes[i + 1], r_next, np_next)) != 0) return rc;
      np = np_next;
      std::copy(r_next, r_next + np_next + 1, r);
    }
  }
  SA_HIP_RETURN(hipStreamSynchronize(p->d2h));
  return 0;
}

// The step API works on a token-block pipeline's Q block, ring and state,
// which a head-group pipeline does not have.
int32_t require_token_blocks(const sa_pipeline* p, const char* what) {
  if (!p->head_groups) return 0;
  sa::set_error("%s: not available on a head-group pipeline (sa_pipeline_run runs its schedule)", what);
  return SA_ERR_BAD_STATE;
}

// Copy `rows` rows of `width` bytes between buffers whose rows start `dpitch`
// and `spitch` bytes apart: one flat copy when both sides are dense, else one
// strided copy, which the copy engines run at the link's rate for rows of
// 1 KB and more (about three quarters of it for 256-byte rows).
int32_t copy_rows(void* dst, int64_t dpitch, const void* src, int64_t spitch, int64_t width, int64_t rows,
                  hipMemcpyKind kind, hipStream_t stream) {
  if (rows <= 0 || width <= 0) return 0;
  if (dpitch == width && spitch == width) {
    SA_HIP_RETURN(hipMemcpyAsync(dst, src, (size_t)(width * rows), kind, stream));
  } else {
    SA_HIP_RETURN(hipMemcpy2DAsync(dst, (size_t)dpitch, src, (size_t)spitch, (size_t)width, (size_t)rows, kind,
                                   stream));
  }
  return 0;
}

// Merge interval of a fused launch over k_length keys: the plan's K/V chunk
// (the row sums merge where the token-block schedule stores and reloads
// them), or none when the chunk is not a multiple of the 64-key tile and the
// whole span fits one chunk.  -1: the span cannot run as one fused launch.
int32_t fused_merge_keys(const sa_pipeline* p, int64_t k_length) {
  if (p->kv_chunk % 64 == 0) return p->kv_chunk;
  return k_length <= p->kv_chunk ? 0 : -1;
}

// One fused update launch of the head-group schedule (initializes, runs over
// every key of a segment, writes the output and the LSE), optionally
// bracketed by timing events.
int32_t launch_unit(sa_pipeline* p, const void* q, int64_t sq_t, const void* k, int64_t sk_t, const void* v,
                    int64_t sv_t, int64_t sv_h, int32_t q_tokens, int32_t kv_tokens, int32_t q_heads,
                    int32_t kv_heads, int32_t causal_shift, double scale, int32_t causal, int32_t merge_keys,
                    const sa::FusedOutput& fused, bool v_transposed, hipStream_t stream) {
  TraceRange range(p->trace, "seqattn:fused_update");
  if (p->timing) {
    if (p->t_used == p->t_start.size()) {
      hipEvent_t a = nullptr, b = nullptr;
      SA_HIP_RETURN(hipEventCreate(&a));
      SA_HIP_RETURN(hipEventCreate(&b));
      p->t_start.push_back(a);
      p->t_stop.push_back(b);
    }
    SA_HIP_RETURN(hipEventRecord(p->t_start[p->t_used], stream));
  }
  const int32_t flags = (causal ? SA_FLAG_CAUSAL : 0) | SA_FLAG_INITIALIZE;
  const int32_t rc = sa::launch_update(q, k, v, nullptr, nullptr, nullptr, sq_t, p->head_dim, sk_t, p->head_dim,
                                       sv_t, sv_h, 0, 0, 0, 0, q_tokens, kv_tokens, q_heads, kv_heads, p->head_dim,
                                       0, 0, causal_shift, scale, flags, p->dtype, stream, merge_keys, &fused,
                                       v_transposed, /*tiled_state=*/false);
  if (rc != 0) return rc;
  if (p->timing) SA_HIP_RETURN(hipEventRecord(p->t_stop[p->t_used++], stream));
  return 0;
}

// One chunk of a staged output: `rows` rows of `width` bytes from the dense
// staging buffer into host rows `pitch` bytes apart.
struct ScatterRows {
  char* dst;
  int64_t pitch;
  const char* src;
  int64_t width, rows;
};

// Host function of the D2H stream (it calls no HIP function).
void scatter_rows(void* arg) {
  const ScatterRows* s = static_cast<const ScatterRows*>(arg);
  for (int64_t r = 0; r < s->rows; ++r) std::memcpy(s->dst + r * s->pitch, s->src + r * s->width, (size_t)s->width);
}

// K/V heads of each unit of a head-group run.  With two sets the sizes ramp
// up 1, 2, 4, ... below group_kv and back down ..., 4, 2, 1 at the end, with
// units of at most group_kv heads, evened out, between: the first unit's
// copies and the last units' output copies are the only ones no launch
// hides (the last two units' launches end together), so they are small.
// With one set (nothing overlaps) every unit but the last has group_kv.
std::vector<int> head_group_unit_sizes(int kv_heads, int group_kv, int num_sets) {
  std::vector<int> sizes;
  if (group_kv <= 0 || kv_heads <= 0) return sizes;
  std::vector<int> ramp;
  if (num_sets > 1)
    for (int size = 1; size < group_kv; size *= 2) ramp.push_back(size);
  int ramp_heads = 0;
  for (const int size : ramp) ramp_heads += size;
  if (2 * ramp_heads > kv_heads) {
    // Too few heads for both ramps: ramp up only, then group_kv.
    for (int done = 0, size = num_sets > 1 ? 1 : group_kv; done < kv_heads;) {
      const int gk = std::min(std::min(size, group_kv), kv_heads - done);
      sizes.push_back(gk);
      done += gk;
      size = std::min(2 * size, group_kv);
    }
    return sizes;
  }
  sizes = ramp;
  const int middle = kv_heads - 2 * ramp_heads;
  const int count = (middle + group_kv - 1) / group_kv;
  for (int i = 0; i < count; ++i) sizes.push_back(middle / count + (i < middle % count ? 1 : 0));
  sizes.insert(sizes.end(), ramp.rbegin(), ramp.rend());
  return sizes;
}

// sa_pipeline_run on a head-group pipeline.  Unit u (a range of K/V heads,
// at most group_kv, with their query heads) uses buffer set u % num_sets
// and, with two sets, compute stream u % 2 (the caller's, then the
// pipeline's second stream):
//   H2D : [wait set_done] K and V columns of every token, [wait set_free] Q
//         columns (strided copies from the host's [token][head][d] rows),
//         record set_ready;
//   compute: wait set_ready; per segment [transpose V], one fused update
//         launch over all its queries and keys that writes the output (over
//         the unit's Q rows) and the LSE; record set_done;
//   D2H : wait set_done; output columns back into the host rows, record
//         set_free.
// Every byte of Q, K and V crosses the link once.  The launch for unit u + 1
// runs on the other stream, so it starts while unit u's last workgroups
// drain, and its copies landed during unit u.  Each launch is the one
// sa_pipeline_run_resident makes for those heads, which the per-chunk
// schedule matches bit for bit.
//
// Units are enqueued num_sets - 1 ahead of the unit whose output is being
// copied out: a unit's copies into a set wait for the set's previous output
// copy, so that copy has to be enqueued first.  With host staging attached
// (a pageable output), the output of a unit goes through the staging buffer
// in row chunks on the D2H stream, each scattered into the host rows by a
// host function once its copy has landed, while later units' launches run.
int32_t run_head_groups(sa_pipeline* p, const char* qh, const char* kh, const char* vh, char* oh, float* lse,
                        int64_t lse_sh, const int64_t* cu_q, const int64_t* cu_k, int32_t num_segments,
                        double scale, int32_t causal, hipStream_t compute, sa_pipeline_stats* st,
                        char* out_dev = nullptr, int64_t so_t = 0, int64_t so_h = 0) {
  for (int32_t s = 0; s < num_segments; ++s) {
    const int64_t q_length = cu_q[s + 1] - cu_q[s], k_length = cu_k[s + 1] - cu_k[s];
    if (cu_q[s] < 0 || cu_k[s] < 0 || q_length < 0 || k_length < 0 || (q_length > 0 && k_length == 0) ||
        cu_q[s + 1] > p->hg_max_q || cu_k[s + 1] > p->hg_max_kv || q_length > INT32_MAX || k_length > INT32_MAX) {
      sa::set_error("sa_pipeline_run: segment %d has invalid bounds for this head-group pipeline", s);
      return SA_ERR_INVALID_ARGUMENT;
    }
    if (q_length > 0 && fused_merge_keys(p, k_length) < 0) {
      sa::set_error("sa_pipeline_run: segment %d has %lld keys, more than one K/V chunk of %d, which is not a "
                    "multiple of 64", s, (long long)k_length, p->kv_chunk);
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  if (num_segments <= 0) return 0;
  const int64_t total_q = cu_q[num_segments], total_k = cu_k[num_segments];
  const int group = p->q_heads / p->kv_heads;
  const int64_t d_bytes = (int64_t)p->head_dim * 2;
  if (p->staging != nullptr && (int64_t)p->group_kv * group * d_bytes > p->staging_bytes) {
    sa::set_error("sa_pipeline_run: host staging of %lld bytes cannot hold one output row of a unit "
                  "(%lld bytes)", (long long)p->staging_bytes, (long long)p->group_kv * group * d_bytes);
    return SA_ERR_INVALID_ARGUMENT;
  }
  const int64_t q_pitch = p->q_heads * d_bytes, kv_pitch = p->kv_heads * d_bytes;
  // Units as K/V head ranges [kv0, kv0 + gk).
  std::vector<std::pair<int, int>> unit_list;
  {
    const std::vector<int> sizes = head_group_unit_sizes(p->kv_heads, p->group_kv, p->num_sets);
    int kv0 = 0;
    for (const int gk : sizes) {
      unit_list.emplace_back(kv0, gk);
      kv0 += gk;
    }
  }
  const int units = (int)unit_list.size();
  hipStream_t streams[sa_pipeline::kMaxSets] = {compute, p->side};
  SideJoin join{p, compute};
  if (p->num_sets > 1 && units > 1) {
    // The second stream starts after the caller's earlier work.
    SA_HIP_RETURN(hipEventRecord(p->fork, compute));
    SA_HIP_RETURN(hipStreamWaitEvent(p->side, p->fork, 0));
    join.active = true;
  }
  // Arguments of the staged output's host functions: they run after this
  // function has enqueued them, and it returns only after the D2H stream has
  // drained, so they live here; reserved in full so none moves.
  std::vector<ScatterRows> scatters;
  if (p->staging != nullptr) {
    int64_t count = 0;
    for (const auto& unit : unit_list) {
      const int64_t wq = (int64_t)unit.second * group * d_bytes;
      count += (total_q + p->staging_bytes / wq - 1) / (p->staging_bytes / wq);
    }
    scatters.reserve((size_t)count);
  }
  // Drains the D2H stream on every return (an error included) before the
  // host functions' arguments above go away.
  struct DrainD2H {
    hipStream_t stream;
    ~DrainD2H() { (void)hipStreamSynchronize(stream); }
  } drain{p->d2h};
  // K/V heads [kv0, kv0 + gk) of unit u and the bytes of one row of its
  // Q/output (wq) and of its K and V (wk).
  auto unit_heads = [&](int u, int* kv0, int* gk, int64_t* wq, int64_t* wk) {
    *kv0 = unit_list[u].first;
    *gk = unit_list[u].second;
    *wq = *gk * group * d_bytes;
    *wk = *gk * d_bytes;
  };
  auto enqueue_unit = [&](int u) -> int32_t {
    const int b = u % p->num_sets;
    hipStream_t cs = streams[b];
    int kv0, gk;
    int64_t wq, wk;
    unit_heads(u, &kv0, &gk, &wq, &wk);
    const int gq = gk * group;
    char* qo = static_cast<char*>(p->set_qo[b]);
    char* kd = static_cast<char*>(p->set_k[b]);
    char* vd = static_cast<char*>(p->set_v[b]);
    // The set's K and V are free once its previous unit's launches have
    // ended; its Q/output buffer only once that unit's output has left.  K
    // and V go first, so that they land while that output is copied out.
    {
      TraceRange range(p->trace, "seqattn:kv_h2d");
      if (p->set_pending[b]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->set_done[b], 0));
      int32_t rc = copy_rows(kd, wk, kh + kv0 * d_bytes, kv_pitch, wk, total_k, hipMemcpyHostToDevice, p->h2d);
      if (rc == 0) rc = copy_rows(vd, wk, vh + kv0 * d_bytes, kv_pitch, wk, total_k, hipMemcpyHostToDevice, p->h2d);
      if (rc != 0) return rc;
    }
    {
      TraceRange range(p->trace, "seqattn:q_h2d");
      if (p->set_pending[b]) SA_HIP_RETURN(hipStreamWaitEvent(p->h2d, p->set_free[b], 0));
      int32_t rc = copy_rows(qo, wq, qh + (int64_t)kv0 * group * d_bytes, q_pitch, wq, total_q,
                             hipMemcpyHostToDevice, p->h2d);
      if (rc != 0) return rc;
      SA_HIP_RETURN(hipEventRecord(p->set_ready[b], p->h2d));
    }
    add_stats(st, total_q * wq + 2 * total_k * wk, 0, 1, 0, total_q);
    SA_HIP_RETURN(hipStreamWaitEvent(cs, p->set_ready[b], 0));
    int64_t chunks = 0;
    for (int32_t s = 0; s < num_segments; ++s) {
      const int64_t q_start = cu_q[s], k_start = cu_k[s];
      const int64_t q_length = cu_q[s + 1] - q_start, k_length = cu_k[s + 1] - k_start;
      if (q_length == 0) continue;
      const int64_t t_pad = (k_length + 63) / 64 * 64;
      const bool vt = p->head_dim == 128 && p->set_vt[b] != nullptr && gk * 128 * t_pad * 2 <= p->hg_vt_bytes &&
                      t_pad < (1 << 24);
      const char* vseg = vd + k_start * wk;
      if (vt) {
        const int32_t rc = sa::launch_transpose_v(vseg, gk * p->head_dim, p->head_dim, (int32_t)k_length, gk,
                                                  p->head_dim, p->set_vt[b], t_pad, cs);
        if (rc != 0) return rc;
      }
      // The output goes over the unit's Q rows (copied out afterwards), or
      // straight into the caller's device rows of the unit's heads.
      const sa::FusedOutput fused =
          out_dev ? sa::FusedOutput{out_dev + (q_start * so_t + (int64_t)kv0 * group * so_h) * 2, so_t, so_h,
                                    lse ? lse + (int64_t)kv0 * group * lse_sh : nullptr, lse_sh, q_start}
                  : sa::FusedOutput{qo + q_start * wq, (int64_t)gq * p->head_dim, p->head_dim,
                                    lse ? lse + (int64_t)kv0 * group * lse_sh : nullptr, lse_sh, q_start};
      const int32_t rc = launch_unit(p, qo + q_start * wq, (int64_t)gq * p->head_dim, kd + k_start * wk,
                                     (int64_t)gk * p->head_dim, vt ? static_cast<const char*>(p->set_vt[b]) : vseg,
                                     vt ? t_pad : (int64_t)gk * p->head_dim, vt ? 128 * t_pad : p->head_dim,
                                     (int32_t)q_length, (int32_t)k_length, gq, gk, (int32_t)(k_length - q_length),
                                     scale, causal, fused_merge_keys(p, k_length), fused, vt, cs);
      if (rc != 0) return rc;
      chunks += (k_length + p->kv_chunk - 1) / p->kv_chunk;
    }
    add_stats(st, 0, 0, 0, chunks, 0);
    SA_HIP_RETURN(hipEventRecord(p->set_done[b], cs));
    return 0;
  };
  auto output_unit = [&](int u) -> int32_t {
    const int b = u % p->num_sets;
    int kv0, gk;
    int64_t wq, wk;
    unit_heads(u, &kv0, &gk, &wq, &wk);
    if (out_dev != nullptr) {
      // The launches wrote the caller's rows: the set is free once they end.
      SA_HIP_RETURN(hipEventRecord(p->set_free[b], streams[b]));
      p->set_pending[b] = true;
      return 0;
    }
    const char* qo = static_cast<const char*>(p->set_qo[b]);
    char* dst = oh + (int64_t)kv0 * group * d_bytes;
    TraceRange range(p->trace, "seqattn:output_d2h");
    SA_HIP_RETURN(hipStreamWaitEvent(p->d2h, p->set_done[b], 0));
    if (p->staging == nullptr) {
      const int32_t rc = copy_rows(dst, q_pitch, qo, wq, wq, total_q, hipMemcpyDeviceToHost, p->d2h);
      if (rc != 0) return rc;
    } else {
      // Row chunks through the staging buffer, in order on the D2H stream:
      // copy a chunk, then scatter it into the host rows with a host
      // function (run by the runtime when the stream reaches it; the stream
      // resumes when it returns), then the next chunk.  Nothing here blocks
      // the calling thread, so later units are enqueued at once.
      const int64_t rows = p->staging_bytes / wq;
      for (int64_t r0 = 0; r0 < total_q; r0 += rows) {
        const int64_t n = std::min(rows, total_q - r0);
        SA_HIP_RETURN(hipMemcpyAsync(p->staging, qo + r0 * wq, (size_t)(n * wq), hipMemcpyDeviceToHost, p->d2h));
        scatters.push_back(ScatterRows{dst + r0 * q_pitch, q_pitch, static_cast<const char*>(p->staging), wq, n});
        SA_HIP_RETURN(hipLaunchHostFunc(p->d2h, scatter_rows, &scatters.back()));
      }
    }
    SA_HIP_RETURN(hipEventRecord(p->set_free[b], p->d2h));
    p->set_pending[b] = true;
    add_stats(st, 0, total_q * wq, 0, 0, 0);
    return 0;
  };
  int next = 0;
  for (int u = 0; u < units; ++u) {
    while (next < units && next <= u + p->num_sets - 1) {
      const int32_t rc = enqueue_unit(next++);
      if (rc != 0) return rc;
    }
    const int32_t rc = output_unit(u);
    if (rc != 0) return rc;
  }
  // Work the caller enqueues on compute_stream later (a read of the LSE or
  // of a device output) follows the second stream's launches.
  const int32_t jrc = join.finish();
  if (jrc != 0) return jrc;
  if (out_dev != nullptr) {
    // The host inputs are no longer read once the last copies have landed;
    // the launches complete in stream order on compute_stream.
    SA_HIP_RETURN(hipStreamSynchronize(p->h2d));
    return 0;
  }
  SA_HIP_RETURN(hipStreamSynchronize(p->d2h));
  return 0;
}

// sa_pipeline_run's schedules, dispatched by the pipeline's kind and output
// slots (the caller's device is current).
int32_t run_host_output(sa_pipeline* p, const void* q_host, const void* k_host, const void* v_host,
                        void* out_host, float* lse, int64_t lse_stride_h, const int64_t* cu_seqlens_q,
                        const int64_t* cu_seqlens_k, int32_t num_segments, double softmax_scale,
                        int32_t causal, void* compute_stream, sa_pipeline_stats* stats) {
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  const char* qh = static_cast<const char*>(q_host);
  const char* kh = static_cast<const char*>(k_host);
  const char* vh = static_cast<const char*>(v_host);
  char* oh = static_cast<char*>(out_host);
  if (p->head_groups)
    return run_head_groups(p, qh, kh, vh, oh, lse, lse_stride_h, cu_seqlens_q, cu_seqlens_k, num_segments,
                           softmax_scale, causal, compute, stats);
  if (!p->has_out_slots || p->num_out == 1) {
    std::vector<Pass> passes;
    for (int32_t s = 0; s < num_segments; ++s) {
      const int64_t q_start = cu_seqlens_q[s], q_stop = cu_seqlens_q[s + 1];
      const int64_t k_start = cu_seqlens_k[s], k_stop = cu_seqlens_k[s + 1];
      const int64_t q_length = q_stop - q_start, k_length = k_stop - k_start;
      if (q_length < 0 || k_length < 0 || (q_length > 0 && k_length == 0)) {
        sa::set_error("sa_pipeline_run: segment %d has invalid bounds", s);
        return SA_ERR_INVALID_ARGUMENT;
      }
      const int64_t block = pass_rows(q_length, p->q_chunk, sa::update_block_rows(p->head_dim));
      for (int64_t qt = q_start; qt < q_stop; qt += block)
        passes.push_back(Pass{qt, k_start, (int32_t)std::min<int64_t>(block, q_stop - qt), (int32_t)k_length,
                              (int32_t)(qt - q_start), (int32_t)(k_length - q_length)});
    }
    if (!p->has_out_slots)
      return run_aliased(p, qh, kh, vh, oh, lse, lse_stride_h, passes, softmax_scale, causal, compute, stats);
    return run_alternating(p, qh, kh, vh, oh, lse, lse_stride_h, passes, softmax_scale, causal, compute, stats);
  }
  int64_t chunk_index = 0;
  for (int32_t s = 0; s < num_segments; ++s) {
    const int64_t q_start = cu_seqlens_q[s], q_stop = cu_seqlens_q[s + 1];
    const int64_t k_start = cu_seqlens_k[s], k_stop = cu_seqlens_k[s + 1];
    const int64_t q_length = q_stop - q_start, k_length = k_stop - k_start;
    if (q_length < 0 || k_length < 0 || (q_length > 0 && k_length == 0)) {
      sa::set_error("sa_pipeline_run: segment %d has invalid bounds", s);
      return SA_ERR_INVALID_ARGUMENT;
    }
    const int32_t causal_shift = (int32_t)(k_length - q_length);
    const int64_t block = pass_rows(q_length, p->q_chunk, sa::update_block_rows(p->head_dim));
    for (int64_t qt = q_start; qt < q_stop; qt += block) {
      const int32_t n = (int32_t)std::min<int64_t>(block, q_stop - qt);
      // Two output slots: the block is finalized into slot i % 2 and copied
      // out while the next block streams.
      int32_t rc = load_q(p, qh + qt * p->q_row_bytes, n, compute, stats);
      if (rc) return rc;
      rc = stream_kv(p, kh + k_start * p->kv_row_bytes, vh + k_start * p->kv_row_bytes,
                     (int32_t)k_length, n, (int32_t)(qt - q_start), causal_shift, softmax_scale,
                     causal, compute, stats);
      if (rc) return rc;
      const int32_t slot = (int32_t)(chunk_index % p->num_out);
      const int64_t bytes = (int64_t)n * p->q_row_bytes;
      rc = finalize(p, slot, n, lse, lse_stride_h, qt, compute);
      if (rc) return rc;
      rc = d2h(p, oh + qt * p->q_row_bytes, p->out_slots[slot], bytes, slot, 0, compute, stats);
      if (rc) return rc;
      ++chunk_index;
    }
  }
  SA_HIP_RETURN(hipStreamSynchronize(p->d2h));
  return 0;
}

// After a failed run, copies enqueued before the failure may still read the
// host inputs or write the host output, and the pipeline's second stream may
// still run launches: wait for them, so that the caller may release its
// buffers once the call returns.  The error reported stays the first one.
void drain_after_error(sa_pipeline* p) {
  if (p->h2d) (void)hipStreamSynchronize(p->h2d);
  if (p->d2h) (void)hipStreamSynchronize(p->d2h);
  if (p->side) (void)hipStreamSynchronize(p->side);
}

}  // namespace

extern "C" {

int32_t sa_abi_version(void) { return SA_ABI_VERSION; }

const char* sa_last_error(void) { return sa::g_last_error.c_str(); }

int32_t sa_pipeline_create(sa_pipeline** out_pipeline, int32_t device, void* q_buffer,
                           void* const* k_slots, void* const* v_slots, int32_t num_kv_buffers,
                           float* running_max, float* running_sum, float* accumulator,
                           void* const* out_slots, int32_t num_output_buffers,
                           int32_t q_chunk_tokens, int32_t kv_chunk_tokens, int32_t q_heads,
                           int32_t kv_heads, int32_t head_dim, int32_t dtype,
                           void* h2d_stream, void* d2h_stream) {
  sa::clear_error();
  if (!out_pipeline) {
    sa::set_error("sa_pipeline_create: null out_pipeline");
    return SA_ERR_INVALID_ARGUMENT;
  }
  *out_pipeline = nullptr;
  if (num_kv_buffers < 1 || num_kv_buffers > 3 || num_output_buffers < 1 || num_output_buffers > 2 ||
      q_chunk_tokens <= 0 || kv_chunk_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || head_dim % 8 != 0) {
    sa::set_error("sa_pipeline_create: invalid plan (kv buffers %d, output buffers %d, q_chunk %d, "
                  "kv_chunk %d, heads %d/%d, head_dim %d)",
                  num_kv_buffers, num_output_buffers, q_chunk_tokens, kv_chunk_tokens, q_heads,
                  kv_heads, head_dim);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    sa::set_error("sa_pipeline_create: unsupported dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (!q_buffer || !k_slots || !v_slots || !running_max || !running_sum || !accumulator) {
    sa::set_error("sa_pipeline_create: null workspace buffer");
    return SA_ERR_INVALID_ARGUMENT;
  }
  sa_pipeline* p = new (std::nothrow) sa_pipeline();
  if (!p) {
    sa::set_error("sa_pipeline_create: out of host memory");
    return SA_ERR_BAD_STATE;
  }
  p->device = device;
  p->q_buffer = q_buffer;
  p->num_kv = num_kv_buffers;
  for (int i = 0; i < num_kv_buffers; ++i) {
    p->k_slots[i] = k_slots[i];
    p->v_slots[i] = v_slots[i];
    if (!k_slots[i] || !v_slots[i]) {
      delete p;
      sa::set_error("sa_pipeline_create: null K/V slot %d", i);
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  p->m = running_max;
  p->l = running_sum;
  p->acc = accumulator;
  p->num_out = num_output_buffers;
  p->has_out_slots = out_slots != nullptr;
  if (p->has_out_slots) {
    for (int i = 0; i < num_output_buffers; ++i) {
      p->out_slots[i] = out_slots[i];
      if (!out_slots[i]) {
        delete p;
        sa::set_error("sa_pipeline_create: null output slot %d", i);
        return SA_ERR_INVALID_ARGUMENT;
      }
    }
  }
  p->q_chunk = q_chunk_tokens;
  p->kv_chunk = kv_chunk_tokens;
  p->q_heads = q_heads;
  p->kv_heads = kv_heads;
  p->head_dim = head_dim;
  p->dtype = dtype;
  p->q_row_bytes = (int64_t)q_heads * head_dim * 2;
  p->kv_row_bytes = (int64_t)kv_heads * head_dim * 2;

  sa::DeviceGuard guard(device);
  hipError_t err = guard.status();
  if (err != hipSuccess) {
    delete p;
    return sa::hip_status(err, "sa_pipeline_create: selecting the device");
  }
  if ((h2d_stream == nullptr) != (d2h_stream == nullptr)) {
    delete p;
    sa::set_error("sa_pipeline_create: pass both copy streams or neither");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (h2d_stream) {
    p->h2d = static_cast<hipStream_t>(h2d_stream);
    p->d2h = static_cast<hipStream_t>(d2h_stream);
  } else {
    p->owns_streams = true;
    err = hipStreamCreateWithFlags(&p->h2d, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&p->d2h, hipStreamNonBlocking);
  }
  const unsigned flags = hipEventDisableTiming;
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->q_ready, flags);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->q_free, flags);
  for (int i = 0; i < num_kv_buffers && err == hipSuccess; ++i) {
    err = hipEventCreateWithFlags(&p->kv_ready[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->kv_free[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->kv_free_side[i], flags);
  }
  if (err == hipSuccess) err = hipStreamCreateWithFlags(&p->side, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->fork, flags);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->join, flags);
  for (int i = 0; i < num_output_buffers && err == hipSuccess; ++i) {
    err = hipEventCreateWithFlags(&p->out_ready[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->out_free[i], flags);
  }
  for (int i = 0; i < 2 && err == hipSuccess; ++i) {
    err = hipEventCreateWithFlags(&p->alt_ready[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->alt_done[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->alt_free[i], flags);
  }
  for (int i = 0; i < sa_pipeline::kPieces && err == hipSuccess; ++i) {
    err = hipEventCreateWithFlags(&p->piece_done[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->piece_out[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->piece_ready[i], flags);
  }
  if (err != hipSuccess) {
    int32_t rc = sa::hip_status(err, "sa_pipeline_create stream/event creation");
    release(p);
    delete p;
    return rc;
  }
  *out_pipeline = p;
  return 0;
}

int32_t sa_pipeline_create_head_groups(sa_pipeline** out_pipeline, int32_t device, void* const* qo_sets,
                                       void* const* k_sets, void* const* v_sets, void* const* vt_sets,
                                       int64_t vt_bytes, int32_t num_sets, int64_t max_q_tokens,
                                       int64_t max_kv_tokens, int32_t group_kv_heads, int32_t kv_chunk_tokens,
                                       int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t dtype,
                                       void* h2d_stream, void* d2h_stream) {
  sa::clear_error();
  if (!out_pipeline) {
    sa::set_error("sa_pipeline_create_head_groups: null out_pipeline");
    return SA_ERR_INVALID_ARGUMENT;
  }
  *out_pipeline = nullptr;
  if (num_sets < 1 || num_sets > sa_pipeline::kMaxSets || max_q_tokens < 0 || max_kv_tokens < 0 ||
      kv_chunk_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || group_kv_heads <= 0 ||
      group_kv_heads > kv_heads || head_dim <= 0 || head_dim % 8 != 0 || vt_bytes < 0) {
    sa::set_error("sa_pipeline_create_head_groups: invalid plan (sets %d, tokens %lld/%lld, kv_chunk %d, heads "
                  "%d/%d, %d K/V heads per group, head_dim %d)",
                  num_sets, (long long)max_q_tokens, (long long)max_kv_tokens, kv_chunk_tokens, q_heads, kv_heads,
                  group_kv_heads, head_dim);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    sa::set_error("sa_pipeline_create_head_groups: unsupported dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (!qo_sets || !k_sets || !v_sets) {
    sa::set_error("sa_pipeline_create_head_groups: null buffer set array");
    return SA_ERR_INVALID_ARGUMENT;
  }
  for (int i = 0; i < num_sets; ++i) {
    const uintptr_t bits = reinterpret_cast<uintptr_t>(qo_sets[i]) | reinterpret_cast<uintptr_t>(k_sets[i]) |
                           reinterpret_cast<uintptr_t>(v_sets[i]) |
                           (vt_sets ? reinterpret_cast<uintptr_t>(vt_sets[i]) : 0);
    if (!qo_sets[i] || !k_sets[i] || !v_sets[i] || (vt_sets && vt_bytes > 0 && !vt_sets[i]) || bits % 16 != 0) {
      sa::set_error("sa_pipeline_create_head_groups: buffer set %d has a null or misaligned buffer", i);
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  sa_pipeline* p = new (std::nothrow) sa_pipeline();
  if (!p) {
    sa::set_error("sa_pipeline_create_head_groups: out of host memory");
    return SA_ERR_BAD_STATE;
  }
  p->device = device;
  p->head_groups = true;
  p->num_sets = num_sets;
  p->group_kv = group_kv_heads;
  p->hg_max_q = max_q_tokens;
  p->hg_max_kv = max_kv_tokens;
  p->hg_vt_bytes = vt_sets ? vt_bytes : 0;
  for (int i = 0; i < num_sets; ++i) {
    p->set_qo[i] = qo_sets[i];
    p->set_k[i] = k_sets[i];
    p->set_v[i] = v_sets[i];
    p->set_vt[i] = vt_sets && vt_bytes > 0 ? vt_sets[i] : nullptr;
  }
  p->kv_chunk = kv_chunk_tokens;
  p->q_heads = q_heads;
  p->kv_heads = kv_heads;
  p->head_dim = head_dim;
  p->dtype = dtype;
  p->q_row_bytes = (int64_t)q_heads * head_dim * 2;
  p->kv_row_bytes = (int64_t)kv_heads * head_dim * 2;

  sa::DeviceGuard guard(device);
  hipError_t err = guard.status();
  if (err != hipSuccess) {
    delete p;
    return sa::hip_status(err, "sa_pipeline_create_head_groups: selecting the device");
  }
  if ((h2d_stream == nullptr) != (d2h_stream == nullptr)) {
    delete p;
    sa::set_error("sa_pipeline_create_head_groups: pass both copy streams or neither");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (h2d_stream) {
    p->h2d = static_cast<hipStream_t>(h2d_stream);
    p->d2h = static_cast<hipStream_t>(d2h_stream);
  } else {
    p->owns_streams = true;
    err = hipStreamCreateWithFlags(&p->h2d, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&p->d2h, hipStreamNonBlocking);
  }
  const unsigned flags = hipEventDisableTiming;
  if (err == hipSuccess) err = hipStreamCreateWithFlags(&p->side, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->fork, flags);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&p->join, flags);
  for (int i = 0; i < num_sets && err == hipSuccess; ++i) {
    err = hipEventCreateWithFlags(&p->set_ready[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->set_done[i], flags);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->set_free[i], flags);
  }
  if (err != hipSuccess) {
    int32_t rc = sa::hip_status(err, "sa_pipeline_create_head_groups stream/event creation");
    release(p);
    delete p;
    return rc;
  }
  *out_pipeline = p;
  return 0;
}

int32_t sa_pipeline_destroy(sa_pipeline* p) {
  sa::clear_error();
  if (!p) return 0;
  {
    sa::DeviceGuard guard(p->device);
    release(p);
  }
  delete p;
  return 0;
}

int32_t sa_pipeline_load_q(sa_pipeline* p, const void* q_host, int32_t q_tokens,
                           void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_load_q")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  return load_q(p, q_host, q_tokens, static_cast<hipStream_t>(compute_stream), stats);
}

int32_t sa_pipeline_stream_kv(sa_pipeline* p, const void* k_host, const void* v_host,
                              int32_t k_length, int32_t q_tokens, int32_t q_local_offset,
                              int32_t causal_shift, double softmax_scale, int32_t causal,
                              void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_stream_kv")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  return stream_kv(p, k_host, v_host, k_length, q_tokens, q_local_offset, causal_shift,
                   softmax_scale, causal, static_cast<hipStream_t>(compute_stream), stats);
}

int32_t sa_pipeline_stream_kv_span(sa_pipeline* p, const void* k_host, const void* v_host,
                                   int32_t kv_tokens, int32_t kv_local_offset,
                                   int32_t* initialize, int32_t q_tokens,
                                   int32_t q_local_offset, int32_t causal_shift,
                                   double softmax_scale, int32_t causal, void* compute_stream,
                                   sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !initialize || (kv_tokens > 0 && (!k_host || !v_host))) {
    sa::set_error("sa_pipeline_stream_kv_span: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_stream_kv_span")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  KVSource src{static_cast<const char*>(k_host), static_cast<const char*>(v_host), false, 0, 0, 0, 0};
  bool init = *initialize != 0;
  int32_t rc;
  if (kv_tokens == 0) {
    rc = init ? init_state(p, p->q_buffer, qt, p->head_dim, q_tokens, q_local_offset,
                           causal_shift, softmax_scale, compute)
              : 0;
    init = false;
  } else {
    rc = apply_span(p, p->q_buffer, qt, p->head_dim, src, kv_tokens, kv_local_offset, &init,
                    q_tokens, q_local_offset, causal_shift, softmax_scale, causal, compute, stats);
  }
  *initialize = init ? 1 : 0;
  return rc;
}

int32_t sa_pipeline_stream_kv_gather(sa_pipeline* p, const void* const* k_fragments,
                                     const void* const* v_fragments,
                                     const int32_t* fragment_tokens, int32_t num_fragments,
                                     int32_t kv_local_offset, int32_t* initialize,
                                     int32_t q_tokens, int32_t q_local_offset,
                                     int32_t causal_shift, double softmax_scale, int32_t causal,
                                     void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !initialize || num_fragments < 0 ||
      (num_fragments > 0 && (!k_fragments || !v_fragments || !fragment_tokens))) {
    sa::set_error("sa_pipeline_stream_kv_gather: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_stream_kv_gather")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  bool init = *initialize != 0;
  int32_t rc = apply_gather(p, k_fragments, v_fragments, nullptr, nullptr, fragment_tokens,
                            num_fragments, kv_local_offset, &init, q_tokens, q_local_offset,
                            causal_shift, softmax_scale, causal, compute, stats);
  *initialize = init ? 1 : 0;
  return rc;
}

int32_t sa_pipeline_attach_int8_scales(sa_pipeline* p, void* const* k_scale_slots,
                                       void* const* v_scale_slots, int32_t num_slots) {
  sa::clear_error();
  if (!p || !k_scale_slots || !v_scale_slots || num_slots != p->num_kv) {
    sa::set_error("sa_pipeline_attach_int8_scales: need %d K and V scale slots",
                  p ? p->num_kv : 0);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_attach_int8_scales")) return hg;
  if (p->head_dim % 16 != 0 || p->head_dim > 128) {
    sa::set_error("sa_pipeline_attach_int8_scales: INT8 K/V needs head_dim a multiple of 16 up to "
                  "128, got %d", p->head_dim);
    return SA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  for (int i = 0; i < num_slots; ++i) {
    if (!k_scale_slots[i] || !v_scale_slots[i] ||
        (reinterpret_cast<uintptr_t>(k_scale_slots[i]) | reinterpret_cast<uintptr_t>(v_scale_slots[i])) % 2) {
      sa::set_error("sa_pipeline_attach_int8_scales: scale slot %d is null or misaligned", i);
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  for (int i = 0; i < num_slots; ++i) {
    p->ks_slots[i] = k_scale_slots[i];
    p->vs_slots[i] = v_scale_slots[i];
  }
  p->has_scales = true;
  return 0;
}

int32_t sa_pipeline_stream_kv_gather_int8(
    sa_pipeline* p, const void* const* k_fragments, const void* const* v_fragments,
    const void* const* k_scale_fragments, const void* const* v_scale_fragments,
    const int32_t* fragment_tokens, int32_t num_fragments, int32_t kv_local_offset,
    int32_t* initialize, int32_t q_tokens, int32_t q_local_offset, int32_t causal_shift,
    double softmax_scale, int32_t causal, void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !initialize || num_fragments < 0 ||
      (num_fragments > 0 && (!k_fragments || !v_fragments || !k_scale_fragments ||
                             !v_scale_fragments || !fragment_tokens))) {
    sa::set_error("sa_pipeline_stream_kv_gather_int8: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_stream_kv_gather_int8")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  bool init = *initialize != 0;
  static const void* const kNoFragment = nullptr;
  int32_t rc = apply_gather(p, k_fragments, v_fragments,
                            num_fragments > 0 ? k_scale_fragments : &kNoFragment,
                            num_fragments > 0 ? v_scale_fragments : &kNoFragment, fragment_tokens,
                            num_fragments, kv_local_offset, &init, q_tokens, q_local_offset,
                            causal_shift, softmax_scale, causal, compute, stats);
  *initialize = init ? 1 : 0;
  return rc;
}

int32_t sa_pipeline_run_resident(sa_pipeline* p, const void* q, const void* k, const void* v,
                                 void* out, float* lse, int64_t stride_qt, int64_t stride_qh,
                                 int64_t stride_kt, int64_t stride_kh, int64_t stride_vt,
                                 int64_t stride_vh, int64_t stride_ot, int64_t stride_oh,
                                 int64_t lse_stride_h, const int64_t* cu_seqlens_q,
                                 const int64_t* cu_seqlens_k, int32_t num_segments,
                                 double softmax_scale, int32_t causal, void* compute_stream,
                                 sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k || num_segments < 0) {
    sa::set_error("sa_pipeline_run_resident: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  const char* qd = static_cast<const char*>(q);
  const char* kd = static_cast<const char*>(k);
  const char* vd = static_cast<const char*>(v);
  char* od = static_cast<char*>(out);
  const int64_t qt_stride = (int64_t)p->q_heads * p->head_dim;
  for (int32_t s = 0; s < num_segments; ++s) {
    const int64_t q_start = cu_seqlens_q[s], q_stop = cu_seqlens_q[s + 1];
    const int64_t k_start = cu_seqlens_k[s], k_stop = cu_seqlens_k[s + 1];
    const int64_t q_length = q_stop - q_start, k_length = k_stop - k_start;
    if (q_length < 0 || k_length < 0 || (q_length > 0 && k_length == 0)) {
      sa::set_error("sa_pipeline_run_resident: segment %d has invalid bounds", s);
      return SA_ERR_INVALID_ARGUMENT;
    }
    const int32_t causal_shift = (int32_t)(k_length - q_length);
    KVSource src{kd + k_start * stride_kt * 2, vd + k_start * stride_vt * 2, true,
                 stride_kt, stride_kh, stride_vt, stride_vh};
    char* seg_out = od + q_start * stride_ot * 2;
    // A head-group pipeline has no Q block or state buffers: only the single
    // fused launch below is available to it.
    const int32_t merge = p->head_groups ? fused_merge_keys(p, k_length) : (p->kv_chunk % 64 == 0 ? p->kv_chunk : -1);
    const bool fused_segment = q_length > 0 && merge >= 0 && q_length <= INT32_MAX && k_length <= INT32_MAX &&
                               stride_ot % 8 == 0 && stride_oh % 8 == 0 &&
                               reinterpret_cast<uintptr_t>(seg_out) % 16 == 0;
    if (p->head_groups && q_length > 0 && !fused_segment) {
      sa::set_error("sa_pipeline_run_resident: segment %d needs the chunked schedule (a 16-byte aligned output "
                    "with strides that are multiples of 8, and at most one K/V chunk unless the chunk is a "
                    "multiple of 64), which a head-group pipeline does not have", s);
      return SA_ERR_BAD_STATE;
    }
    if (fused_segment) {
      // K/V already in HBM: one launch covers every query and key of the
      // segment and finalizes its rows in the epilogue.  The row sums are
      // merged at every kv_chunk boundary exactly as the chunked schedule
      // stores and reloads them, so the output and LSE equal
      // sa_pipeline_run's bit for bit, with no state round trips, no
      // per-launch tails and no finalize launches.  Stats count the Q blocks
      // and chunks of the chunked schedule.
      const sa::FusedOutput fused{seg_out, stride_ot, stride_oh, lse, lse_stride_h, q_start};
      // With head_dim 128 and enough attached scratch, V is first copied
      // transposed (keys padded to whole tiles), which the update kernel
      // reads with half the LDS instructions for the same operands.
      const int64_t t_pad = (k_length + 63) / 64 * 64;
      const int64_t vt_bytes = (int64_t)p->kv_heads * 128 * t_pad * 2;
      const bool vt = p->head_dim == 128 && p->vt_scratch != nullptr && vt_bytes <= p->vt_scratch_bytes &&
                      t_pad < (1 << 24);
      int32_t rc = 0;
      if (vt) {
        rc = sa::launch_transpose_v(src.v, src.sv_t, src.sv_h, (int32_t)k_length, p->kv_heads, p->head_dim,
                                    p->vt_scratch, t_pad, compute);
        if (rc != 0) return rc;
      }
      rc = launch_timed(p, qd + q_start * stride_qt * 2, stride_qt, stride_qh, src.k, src.sk_t, src.sk_h,
                        vt ? static_cast<const char*>(p->vt_scratch) : src.v, vt ? t_pad : src.sv_t,
                        vt ? 128 * t_pad : src.sv_h, (int32_t)q_length, (int32_t)k_length, 0, 0, causal_shift,
                        softmax_scale, (causal ? SA_FLAG_CAUSAL : 0) | SA_FLAG_INITIALIZE, compute, merge,
                        &fused, 0, vt);
      if (rc != 0) return rc;
      const int64_t block = p->head_groups ? q_length
                                           : pass_rows(q_length, p->q_chunk, sa::update_block_rows(p->head_dim));
      for (int64_t qs = q_start; qs < q_stop; qs += block) {
        const int64_t n = std::min<int64_t>(block, q_stop - qs);
        const int64_t visible_end = causal ? std::max<int64_t>(0, qs - q_start + n + causal_shift) : INT64_MAX;
        int64_t chunks = 0;
        for (int64_t start = 0; start < k_length; start += p->kv_chunk) {
          if (chunks > 0 && start >= visible_end) break;
          ++chunks;
        }
        add_stats(stats, 0, 0, 1, chunks, n);
      }
      continue;
    }
    for (int64_t qs = q_start; qs < q_stop; qs += p->q_chunk) {
      const int32_t n = (int32_t)std::min<int64_t>(p->q_chunk, q_stop - qs);
      const char* qblock = qd + qs * stride_qt * 2;
      bool initialize = true;
      int32_t rc = apply_span(p, qblock, stride_qt, stride_qh, src, (int32_t)k_length, 0, &initialize, n,
                              (int32_t)(qs - q_start), causal_shift, softmax_scale, causal, compute, stats);
      if (rc != 0) return rc;
      if (initialize) {
        rc = init_state(p, qblock, stride_qt, stride_qh, n, (int32_t)(qs - q_start), causal_shift,
                        softmax_scale, compute);
        if (rc != 0) return rc;
      }
      rc = sa::launch_finalize(p->acc, p->m, p->l, od + qs * stride_ot * 2, lse, qt_stride,
                               p->head_dim, p->q_heads, 1, stride_ot, stride_oh, lse_stride_h, qs,
                               n, p->q_heads, p->head_dim, p->dtype, compute, /*tiled_state=*/true);
      if (rc != 0) return rc;
      add_stats(stats, 0, 0, 1, 0, n);
    }
  }
  return 0;
}

int32_t sa_pipeline_finalize(sa_pipeline* p, int32_t slot, int32_t q_tokens, float* lse,
                             int64_t lse_stride_h, int64_t lse_token_offset, void* compute_stream) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_finalize")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  return finalize(p, slot, q_tokens, lse, lse_stride_h, lse_token_offset,
                  static_cast<hipStream_t>(compute_stream));
}

int32_t sa_pipeline_finalize_into(sa_pipeline* p, void* dest, int64_t stride_ot,
                                  int64_t stride_oh, int32_t q_tokens, float* lse,
                                  int64_t lse_stride_h, int64_t lse_token_offset,
                                  void* compute_stream) {
  sa::clear_error();
  if (!p || !dest) return SA_ERR_INVALID_ARGUMENT;
  if (q_tokens < 0 || q_tokens > p->q_chunk) {
    sa::set_error("q_tokens %d outside [0, q_chunk_tokens=%d]", q_tokens, p->q_chunk);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_finalize_into")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  hipStream_t compute = static_cast<hipStream_t>(compute_stream);
  TraceRange range(p->trace, "seqattn:fused_finalize");
  SA_HIP_RETURN(hipEventRecord(p->q_free, compute));
  p->q_pending = true;
  const int64_t qt = (int64_t)p->q_heads * p->head_dim;
  return sa::launch_finalize(p->acc, p->m, p->l, dest, lse, qt, p->head_dim, p->q_heads, 1,
                             stride_ot, stride_oh, lse_stride_h, lse_token_offset, q_tokens,
                             p->q_heads, p->head_dim, p->dtype, compute, /*tiled_state=*/true);
}

int32_t sa_pipeline_release_q(sa_pipeline* p, void* compute_stream) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_release_q")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  SA_HIP_RETURN(hipEventRecord(p->q_free, static_cast<hipStream_t>(compute_stream)));
  p->q_pending = true;
  return 0;
}

int32_t sa_pipeline_d2h(sa_pipeline* p, void* dst_host, const void* src, int64_t bytes,
                        int32_t event_slot, int32_t release_q, void* compute_stream,
                        sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (const int32_t hg = require_token_blocks(p, "sa_pipeline_d2h")) return hg;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  return d2h(p, dst_host, src, bytes, event_slot, release_q,
             static_cast<hipStream_t>(compute_stream), stats);
}

int32_t sa_pipeline_synchronize(sa_pipeline* p) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  SA_HIP_RETURN(hipStreamSynchronize(p->d2h));
  return 0;
}

int32_t sa_pipeline_attach_resident_scratch(sa_pipeline* p, void* scratch, int64_t bytes) {
  sa::clear_error();
  if (!p || bytes < 0 || (scratch == nullptr) != (bytes == 0) ||
      (scratch && reinterpret_cast<uintptr_t>(scratch) % 16 != 0)) {
    sa::set_error("sa_pipeline_attach_resident_scratch: need a 16-byte aligned buffer and its size, or NULL and 0");
    return SA_ERR_INVALID_ARGUMENT;
  }
  p->vt_scratch = scratch;
  p->vt_scratch_bytes = bytes;
  return 0;
}

int32_t sa_pipeline_attach_host_staging(sa_pipeline* p, void* staging, int64_t bytes) {
  sa::clear_error();
  if (!p || bytes < 0 || (staging == nullptr) != (bytes == 0)) {
    sa::set_error("sa_pipeline_attach_host_staging: need a page-locked buffer and its size, or NULL and 0");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (!p->head_groups) {
    sa::set_error("sa_pipeline_attach_host_staging: only head-group pipelines stage their output");
    return SA_ERR_BAD_STATE;
  }
  // Earlier runs returned only after their copies and scatters finished, so
  // the previous buffer is no longer read or written.
  p->staging = staging;
  p->staging_bytes = bytes;
  return 0;
}

int32_t sa_pipeline_set_trace_ranges(sa_pipeline* p, int32_t enable) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  if (enable && !trace_api().push) {
    sa::set_error("sa_pipeline_set_trace_ranges: no ROCm tracer library (roctx) could be loaded");
    return SA_ERR_BAD_STATE;
  }
  p->trace = enable != 0;
  return 0;
}

int32_t sa_pipeline_set_kernel_timing(sa_pipeline* p, int32_t enable) {
  sa::clear_error();
  if (!p) return SA_ERR_INVALID_ARGUMENT;
  p->timing = enable != 0;
  p->t_used = 0;
  return 0;
}

int32_t sa_pipeline_kernel_busy(sa_pipeline* p, double* busy_ms, double* total_ms, int64_t* launches) {
  sa::clear_error();
  if (!p || !busy_ms || !total_ms || !launches) return SA_ERR_INVALID_ARGUMENT;
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  // Launch intervals as offsets from the first recorded start; the events of
  // both streams share the device's clock.
  std::vector<std::pair<double, double>> spans;
  spans.reserve(p->t_used);
  double total = 0.0;
  for (size_t i = 0; i < p->t_used; ++i) {
    SA_HIP_RETURN(hipEventSynchronize(p->t_stop[i]));
    float begin = 0.f, end = 0.f;
    SA_HIP_RETURN(hipEventElapsedTime(&begin, p->t_start[0], p->t_start[i]));
    SA_HIP_RETURN(hipEventElapsedTime(&end, p->t_start[0], p->t_stop[i]));
    spans.emplace_back(begin, end);
    total += end - begin;
  }
  std::sort(spans.begin(), spans.end());
  double busy = 0.0, open_begin = 0.0, open_end = -1.0;
  for (const auto& s : spans) {
    if (open_end < open_begin || s.first > open_end) {
      if (open_end >= open_begin) busy += open_end - open_begin;
      open_begin = s.first;
      open_end = s.second;
    } else {
      open_end = std::max(open_end, s.second);
    }
  }
  if (!spans.empty()) busy += open_end - open_begin;
  *busy_ms = busy;
  *total_ms = total;
  *launches = (int64_t)p->t_used;
  p->t_used = 0;
  return 0;
}

int32_t sa_pipeline_kernel_timing(sa_pipeline* p, double* total_ms, int64_t* launches) {
  double busy = 0.0;
  return sa_pipeline_kernel_busy(p, &busy, total_ms, launches);
}

void* sa_pipeline_stream(sa_pipeline* p, int32_t which) {
  if (!p) return nullptr;
  return which == 0 ? static_cast<void*>(p->h2d) : static_cast<void*>(p->d2h);
}

void* sa_pipeline_output_slot(sa_pipeline* p, int32_t index) {
  if (!p || !p->has_out_slots || index < 0 || index >= p->num_out) return nullptr;
  return p->out_slots[index];
}

void* sa_pipeline_q_buffer(sa_pipeline* p) { return p ? p->q_buffer : nullptr; }

int32_t sa_pipeline_run_device_output(sa_pipeline* p, const void* q_host, const void* k_host, const void* v_host,
                                      void* out, int64_t stride_ot, int64_t stride_oh, float* lse,
                                      int64_t lse_stride_h, const int64_t* cu_seqlens_q,
                                      const int64_t* cu_seqlens_k, int32_t num_segments, double softmax_scale,
                                      int32_t causal, void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !q_host || !k_host || !v_host || !out || !cu_seqlens_q || !cu_seqlens_k || num_segments < 0) {
    sa::set_error("sa_pipeline_run_device_output: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (!p->head_groups) {
    sa::set_error("sa_pipeline_run_device_output: only head-group pipelines write a device output from their "
                  "launches (token-block pipelines use the step API)");
    return SA_ERR_BAD_STATE;
  }
  // The fused launches' output rules, checked before anything is enqueued.
  if (stride_ot % 8 != 0 || stride_oh % 8 != 0 || stride_oh < p->head_dim ||
      stride_ot < (int64_t)p->q_heads * stride_oh || reinterpret_cast<uintptr_t>(out) % 16 != 0) {
    sa::set_error("sa_pipeline_run_device_output: out must be 16-byte aligned with strides that are multiples of "
                  "8 and hold [tokens, q_heads, head_dim]");
    return SA_ERR_INVALID_ARGUMENT;
  }
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  const int32_t rc = run_head_groups(p, static_cast<const char*>(q_host), static_cast<const char*>(k_host),
                                     static_cast<const char*>(v_host), nullptr, lse, lse_stride_h, cu_seqlens_q,
                                     cu_seqlens_k, num_segments, softmax_scale, causal,
                                     static_cast<hipStream_t>(compute_stream), stats, static_cast<char*>(out),
                                     stride_ot, stride_oh);
  if (rc != 0) drain_after_error(p);
  return rc;
}

int32_t sa_pipeline_run(sa_pipeline* p, const void* q_host, const void* k_host, const void* v_host,
                        void* out_host, float* lse, int64_t lse_stride_h,
                        const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k,
                        int32_t num_segments, double softmax_scale, int32_t causal,
                        void* compute_stream, sa_pipeline_stats* stats) {
  sa::clear_error();
  if (!p || !q_host || !k_host || !v_host || !out_host || !cu_seqlens_q || !cu_seqlens_k ||
      num_segments < 0) {
    sa::set_error("sa_pipeline_run: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  sa::DeviceGuard guard(p->device);
  SA_HIP_RETURN(guard.status());
  const int32_t rc = run_host_output(p, q_host, k_host, v_host, out_host, lse, lse_stride_h, cu_seqlens_q,
                                     cu_seqlens_k, num_segments, softmax_scale, causal, compute_stream, stats);
  if (rc != 0) drain_after_error(p);
  return rc;
}

}  // extern "C"
