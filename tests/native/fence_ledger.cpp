// Fence ledger: a recording implementation of the HIP calls the transfer
// pipeline (stream-attn_amd/csrc/sa_pipeline.cpp) makes, plus the kernel
// launchers it calls, built with the host compiler against
// hip_stub/hip/hip_runtime.h.  Nothing runs on a GPU: every copy, launch,
// event record, stream wait and host synchronization is appended to a ledger
// with the byte ranges it reads and writes, and ledger_check() verifies the
// schedule by happens-before:
//   * operations on one stream run in enqueue order;
//   * a wait runs after the event record it names (the record most recent
//     at the time of the wait call, HIP's semantics);
//   * everything enqueued after a host synchronization runs after what that
//     synchronization waited for.
// Any two enqueued operations whose byte ranges conflict (a write against a
// read or a write) must be ordered by that relation in their enqueue order;
// and every device-to-host copy must be complete at the last host
// synchronization, where the pipeline returns the host output to its caller.
// ledger_drop_wait(n) makes the n-th stream-wait call a no-op: a planted
// ordering mistake the check must report.  ledger_fail_copy(n) makes the n-th
// copy call fail (nothing is recorded for it): an error in the middle of a
// run, after which ledger_unfinished() counts the copies and host functions
// that were not complete when the call returned.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "sa_common.h"

namespace {

// [lo, hi), or with pitch > 0 the rows [lo + i * pitch, lo + i * pitch +
// width) that start below hi.
struct Range {
  uintptr_t lo, hi;
  uintptr_t pitch = 0, width = 0;
};

enum Kind { kCopyH2D, kCopyD2H, kCopyD2D, kKernel, kRecord, kWait, kStreamSync, kEventSync };

struct Op {
  Kind kind;
  int stream;       // -1: not on a stream (event synchronization)
  int source = -1;  // wait / event sync: index of the record it follows
  std::vector<Range> reads, writes;
  std::string label;
};

struct Ledger {
  std::vector<Op> ops;
  std::map<const void*, int> last_record;  // event -> op index of its latest record
  std::map<const void*, int> stream_ids;
  std::vector<std::unique_ptr<char>> handles;
  long waits_seen = 0;
  long drop_wait = -1;
  long dropped = 0;
  long copies_seen = 0;
  long fail_copy = -1;
};

Ledger g;

// Whether this copy call is the one planted to fail.
bool copy_fails() { return g.copies_seen++ == g.fail_copy; }

int stream_id(hipStream_t s) {
  auto it = g.stream_ids.find(s);
  if (it != g.stream_ids.end()) return it->second;
  const int id = (int)g.stream_ids.size() + 1;
  g.stream_ids.emplace(s, id);
  return id;
}

template <typename T>
T new_handle() {
  g.handles.emplace_back(new char(0));
  return reinterpret_cast<T>(g.handles.back().get());
}

int push(Op op) {
  g.ops.push_back(std::move(op));
  return (int)g.ops.size() - 1;
}

Range span(const void* p, int64_t bytes) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return Range{lo, lo + (uintptr_t)std::max<int64_t>(bytes, 0)};
}

// Rows of `width` bytes, `pitch` apart (`count` of them), from p.
Range strided(const void* p, int64_t width, int64_t pitch, int64_t count) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  if (count <= 0 || width <= 0) return Range{lo, lo};
  if (count == 1 || width >= pitch) return Range{lo, lo + (uintptr_t)((count - 1) * pitch + width)};
  return Range{lo, lo + (uintptr_t)((count - 1) * pitch + width), (uintptr_t)pitch, (uintptr_t)width};
}

// Whether a row range and a contiguous range [a, b) share a byte: some row
// start s = lo + i * pitch with a - width < s < b.
bool rows_meet(const Range& r, uintptr_t a, uintptr_t b) {
  const uintptr_t first = a + 1 > r.lo + r.width ? (a + 1 - r.width - r.lo + r.pitch - 1) / r.pitch : 0;
  const uintptr_t s = r.lo + first * r.pitch;
  return s < b && s < r.hi;
}

bool intersect(const Range& x, const Range& y) {
  if (!(x.lo < y.hi && y.lo < x.hi && x.lo < x.hi && y.lo < y.hi)) return false;
  if (!x.pitch && !y.pitch) return true;
  if (!x.pitch) return rows_meet(y, x.lo, x.hi);
  if (!y.pitch) return rows_meet(x, y.lo, y.hi);
  if (x.pitch != y.pitch) return true;  // different pitches: the bounding ranges decide
  // Same pitch, overlapping extents: the column windows must meet.
  const uintptr_t p = x.pitch, cx = x.lo % p, cy = y.lo % p;
  for (const uintptr_t shift : {(uintptr_t)0, p}) {
    if (cx < cy + shift + y.width && cy + shift < cx + x.width) return true;
    if (cy < cx + shift + x.width && cx + shift < cy + y.width) return true;
  }
  return false;
}

bool overlaps(const std::vector<Range>& a, const std::vector<Range>& b) {
  for (const Range& x : a)
    for (const Range& y : b)
      if (intersect(x, y)) return true;
  return false;
}

// Byte ranges of rows [0, rows) of a token-major tensor with a row stride of
// `stride` elements of `elem` bytes.
Range rows_of(const void* base, int64_t rows, int64_t stride, int elem) { return span(base, rows * stride * elem); }

// Rows of pipeline state a launch over `rows` rows touches: whole 16-row
// groups in the row-group layout.
int64_t state_rows(int64_t rows, bool tiled) { return tiled ? (rows + 15) / 16 * 16 : rows; }

// Per-head ranges of an LSE written for `rows` rows starting at token `off`.
void lse_ranges(std::vector<Range>& out, const float* lse, int64_t sh, int64_t off, int64_t rows, int heads) {
  if (!lse) return;
  for (int h = 0; h < heads; ++h) out.push_back(span(lse + h * sh + off, rows * 4));
}

}  // namespace

// --------------------------------------------------------------- HIP stubs
const char* hipGetErrorString(hipError_t) { return "stub"; }
hipError_t hipGetDevice(int* device) {
  *device = 0;
  return hipSuccess;
}
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int) {
  *stream = new_handle<hipStream_t>();
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t stream) {
  push(Op{kStreamSync, stream_id(stream), -1, {}, {}, "stream sync"});
  return hipSuccess;
}
hipError_t hipStreamWaitEvent(hipStream_t stream, hipEvent_t event, unsigned int) {
  const long n = g.waits_seen++;
  if (n == g.drop_wait) {
    ++g.dropped;
    return hipSuccess;
  }
  auto it = g.last_record.find(event);
  push(Op{kWait, stream_id(stream), it == g.last_record.end() ? -1 : it->second, {}, {}, "wait"});
  return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t* event) {
  *event = new_handle<hipEvent_t>();
  return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned int) { return hipEventCreate(event); }
hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream) {
  g.last_record[event] = push(Op{kRecord, stream_id(stream), -1, {}, {}, "record"});
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t event) {
  auto it = g.last_record.find(event);
  push(Op{kEventSync, -1, it == g.last_record.end() ? -1 : it->second, {}, {}, "event sync"});
  return hipSuccess;
}
hipError_t hipEventElapsedTime(float* ms, hipEvent_t, hipEvent_t) {
  *ms = 0.f;
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t stream) {
  if (copy_fails()) return hipErrorInvalidValue;
  const Kind k = kind == hipMemcpyHostToDevice ? kCopyH2D : kind == hipMemcpyDeviceToHost ? kCopyD2H : kCopyD2D;
  push(Op{k, stream_id(stream), -1, {span(src, (int64_t)bytes)}, {span(dst, (int64_t)bytes)},
          k == kCopyH2D ? "h2d copy" : k == kCopyD2H ? "d2h copy" : "d2d copy"});
  return hipSuccess;
}

// A strided copy reads and writes rows of `width` bytes on each side.
hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                            hipMemcpyKind kind, hipStream_t stream) {
  if (copy_fails()) return hipErrorInvalidValue;
  const Kind k = kind == hipMemcpyHostToDevice ? kCopyH2D : kind == hipMemcpyDeviceToHost ? kCopyD2H : kCopyD2D;
  push(Op{k, stream_id(stream), -1, {strided(src, (int64_t)width, (int64_t)spitch, (int64_t)height)},
          {strided(dst, (int64_t)width, (int64_t)dpitch, (int64_t)height)},
          k == kCopyH2D ? "h2d 2-d copy" : k == kCopyD2H ? "d2h 2-d copy" : "d2d 2-d copy"});
  return hipSuccess;
}

// A host function is an operation of its stream with no device ranges; it
// runs here at once (the tests that enqueue one give it real host memory).
hipError_t hipLaunchHostFunc(hipStream_t stream, hipHostFn_t fn, void* user_data) {
  push(Op{kKernel, stream_id(stream), -1, {}, {}, "host function"});
  fn(user_data);
  return hipSuccess;
}

// ------------------------------------------------------- kernel launchers
namespace sa {

// Same values as the kernels' workgroup tiles.
int32_t update_block_rows(int32_t head_dim) {
  if (head_dim > 64 && head_dim <= 128) return 384;
  return head_dim <= 64 ? 256 : 128;
}

int32_t launch_update(const void* q, const void* k, const void* v, float* m, float* l, float* acc, int64_t sq_t,
                      int64_t, int64_t sk_t, int64_t, int64_t sv_t, int64_t sv_h, int64_t ss_t, int64_t,
                      int64_t sa_t, int64_t, int32_t q_tokens, int32_t kv_tokens, int32_t q_heads,
                      int32_t kv_heads, int32_t head_dim, int32_t, int32_t, int32_t, double, int32_t flags, int32_t,
                      hipStream_t stream, int32_t, const FusedOutput* fused, bool v_transposed, bool tiled) {
  Op op{kKernel, stream_id(stream), -1, {}, {}, "update"};
  op.reads.push_back(rows_of(q, q_tokens, sq_t, 2));
  op.reads.push_back(rows_of(k, kv_tokens, sk_t, 2));
  op.reads.push_back(v_transposed ? span(v, kv_heads * sv_h * 2) : rows_of(v, kv_tokens, sv_t, 2));
  // A state-loading launch reads m, l and acc; a fused one writes the output
  // and the LSE (it may alias q) instead of storing the state.
  std::vector<Range> state;
  if (!fused || !(flags & SA_FLAG_INITIALIZE)) {
    const int64_t rows = state_rows(q_tokens, tiled);
    state = {rows_of(m, rows, ss_t, 4), rows_of(l, rows, ss_t, 4), rows_of(acc, rows, sa_t, 4)};
  }
  if (!(flags & SA_FLAG_INITIALIZE)) op.reads.insert(op.reads.end(), state.begin(), state.end());
  if (fused) {
    // Each head's output columns of every row.
    for (int h = 0; h < q_heads; ++h)
      op.writes.push_back(strided(static_cast<const char*>(fused->out) + h * fused->so_h * 2, head_dim * 2,
                                  fused->so_t * 2, q_tokens));
    lse_ranges(op.writes, fused->lse, fused->lse_sh, fused->lse_off, q_tokens, q_heads);
  } else {
    op.writes = state;
  }
  push(std::move(op));
  return 0;
}

int32_t launch_transpose_v(const void* v, int64_t sv_t, int64_t, int32_t kv_tokens, int32_t kv_heads, int32_t,
                           void* vt, int64_t t_pad, hipStream_t stream) {
  push(Op{kKernel, stream_id(stream), -1, {rows_of(v, kv_tokens, sv_t, 2)}, {span(vt, kv_heads * 128 * t_pad * 2)},
          "transpose v"});
  return 0;
}

int32_t launch_update_int8(const void* q, const void* k, const void* v, const void* k_scales, const void* v_scales,
                           float* m, float* l, float* acc, int64_t sq_t, int64_t, int64_t sk_t, int64_t,
                           int64_t sv_t, int64_t, int64_t sks_g, int64_t, int64_t svs_g, int64_t, int64_t ss_t,
                           int64_t, int64_t sa_t, int64_t, int32_t q_tokens, int32_t kv_tokens, int32_t,
                           int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, double, int32_t flags, int32_t,
                           int32_t, hipStream_t stream, bool tiled) {
  Op op{kKernel, stream_id(stream), -1, {}, {}, "update int8"};
  op.reads = {rows_of(q, q_tokens, sq_t, 2), rows_of(k, kv_tokens, sk_t, 1), rows_of(v, kv_tokens, sv_t, 1),
              rows_of(k_scales, kv_tokens, sks_g, 2), rows_of(v_scales, kv_tokens, svs_g, 2)};
  const int64_t rows = state_rows(q_tokens, tiled);
  std::vector<Range> state = {rows_of(m, rows, ss_t, 4), rows_of(l, rows, ss_t, 4), rows_of(acc, rows, sa_t, 4)};
  if (!(flags & SA_FLAG_INITIALIZE)) op.reads.insert(op.reads.end(), state.begin(), state.end());
  op.writes = state;
  push(std::move(op));
  return 0;
}

int32_t launch_finalize(const float* acc, const float* m, const float* l, void* out, float* lse, int64_t sa_t,
                        int64_t, int64_t ss_t, int64_t, int64_t so_t, int64_t, int64_t lse_sh, int64_t lse_off,
                        int32_t q_tokens, int32_t q_heads, int32_t, int32_t, hipStream_t stream, bool tiled) {
  Op op{kKernel, stream_id(stream), -1, {}, {}, "finalize"};
  const int64_t rows = state_rows(q_tokens, tiled);
  op.reads = {rows_of(acc, rows, sa_t, 4), rows_of(m, rows, ss_t, 4), rows_of(l, rows, ss_t, 4)};
  op.writes = {rows_of(out, q_tokens, so_t, 2)};
  lse_ranges(op.writes, lse, lse_sh, lse_off, q_tokens, q_heads);
  push(std::move(op));
  return 0;
}

}  // namespace sa

// --------------------------------------------------------------- checker
extern "C" {

void ledger_reset(void) {
  g.ops.clear();
  g.last_record.clear();
  g.waits_seen = 0;
  g.drop_wait = -1;
  g.dropped = 0;
  g.copies_seen = 0;
  g.fail_copy = -1;
}

void ledger_drop_wait(long n) { g.drop_wait = n; }

void ledger_fail_copy(long n) { g.fail_copy = n; }

long ledger_copies(void) { return g.copies_seen; }

long ledger_waits(void) { return g.waits_seen; }

long ledger_dropped(void) { return g.dropped; }

// Counts of recorded operations: [copies H2D, copies D2H, kernels, waits].
void ledger_counts(int64_t* out) {
  out[0] = out[1] = out[2] = out[3] = 0;
  for (const Op& op : g.ops) {
    if (op.kind == kCopyH2D) ++out[0];
    if (op.kind == kCopyD2H) ++out[1];
    if (op.kind == kKernel) ++out[2];
    if (op.kind == kWait) ++out[3];
  }
}

// Returns the number of unordered conflicting pairs plus D2H copies not
// complete at the last host synchronization; describes the first few in msg.
int64_t ledger_check(char* msg, int64_t msg_len) {
  const int n = (int)g.ops.size();
  const int words = (n + 63) / 64;
  std::vector<uint64_t> reach((size_t)n * words, 0);  // reach[j] holds i when i happens before j
  std::map<int, int> last_on_stream;
  int barrier = -1;  // latest host synchronization: everything later follows it
  int last_sync = -1;
  for (int j = 0; j < n; ++j) {
    const Op& op = g.ops[j];
    std::vector<int> preds;
    if (op.stream >= 0) {
      auto it = last_on_stream.find(op.stream);
      if (it != last_on_stream.end()) preds.push_back(it->second);
    }
    if ((op.kind == kWait || op.kind == kEventSync) && op.source >= 0) preds.push_back(op.source);
    if (barrier >= 0) preds.push_back(barrier);
    uint64_t* row = &reach[(size_t)j * words];
    for (int p : preds) {
      const uint64_t* prow = &reach[(size_t)p * words];
      for (int w = 0; w < words; ++w) row[w] |= prow[w];
      row[p / 64] |= 1ull << (p % 64);
    }
    if (op.stream >= 0) last_on_stream[op.stream] = j;
    if (op.kind == kStreamSync || op.kind == kEventSync) barrier = last_sync = j;
  }
  auto before = [&](int i, int j) { return (reach[(size_t)j * words + i / 64] >> (i % 64)) & 1ull; };
  int64_t violations = 0;
  std::string text;
  auto note = [&](const std::string& s) {
    if (++violations <= 4) text += s + "; ";
  };
  std::vector<int> accessing;
  for (int i = 0; i < n; ++i)
    if (!g.ops[i].reads.empty() || !g.ops[i].writes.empty()) accessing.push_back(i);
  for (size_t a = 0; a < accessing.size(); ++a) {
    const int i = accessing[a];
    for (size_t b = a + 1; b < accessing.size(); ++b) {
      const int j = accessing[b];
      const Op& x = g.ops[i];
      const Op& y = g.ops[j];
      const bool conflict = overlaps(x.writes, y.reads) || overlaps(x.writes, y.writes) || overlaps(x.reads, y.writes);
      if (conflict && !before(i, j)) {
        char buf[160];
        snprintf(buf, sizeof(buf), "#%d %s (stream %d) and #%d %s (stream %d) unordered", i, x.label.c_str(),
                 x.stream, j, y.label.c_str(), y.stream);
        note(buf);
      }
    }
  }
  for (int i = 0; i < n; ++i) {
    if (g.ops[i].kind != kCopyD2H) continue;
    if (last_sync < i || !before(i, last_sync)) {
      char buf[120];
      snprintf(buf, sizeof(buf), "#%d d2h copy not complete at the last host synchronization", i);
      note(buf);
    }
  }
  if (msg && msg_len > 0) snprintf(msg, (size_t)msg_len, "%s", text.c_str());
  return violations;
}

// Copies and host functions (they touch host memory) not ordered before the
// last host synchronization recorded so far.
int64_t ledger_unfinished(void) {
  const int n = (int)g.ops.size();
  int last_sync = -1;
  for (int j = 0; j < n; ++j)
    if (g.ops[j].kind == kStreamSync || g.ops[j].kind == kEventSync) last_sync = j;
  // Stream order, waits and earlier synchronizations, as in ledger_check.
  std::vector<std::vector<char>> reach(n, std::vector<char>(n, 0));
  std::map<int, int> last_on_stream;
  int barrier = -1;
  for (int j = 0; j < n; ++j) {
    const Op& op = g.ops[j];
    std::vector<int> preds;
    if (op.stream >= 0) {
      auto it = last_on_stream.find(op.stream);
      if (it != last_on_stream.end()) preds.push_back(it->second);
    }
    if ((op.kind == kWait || op.kind == kEventSync) && op.source >= 0) preds.push_back(op.source);
    if (barrier >= 0) preds.push_back(barrier);
    for (int p : preds) {
      for (int i = 0; i < n; ++i) reach[j][i] |= reach[p][i];
      reach[j][p] = 1;
    }
    if (op.stream >= 0) last_on_stream[op.stream] = j;
    if (op.kind == kStreamSync || op.kind == kEventSync) barrier = j;
  }
  int64_t unfinished = 0;
  for (int i = 0; i < n; ++i) {
    const Kind k = g.ops[i].kind;
    const bool host_side = k == kCopyH2D || k == kCopyD2H || (k == kKernel && g.ops[i].label == "host function");
    if (host_side && (last_sync < i || !reach[last_sync][i])) ++unfinished;
  }
  return unfinished;
}

}  // extern "C"
