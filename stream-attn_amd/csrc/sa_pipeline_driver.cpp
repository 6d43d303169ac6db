// Native driver of the pinned-DRAM streamed path: caller-pinned Q/K/V ->
// sa_pipeline_run -> caller-pinned output, with no Python in the process.
// It exists so that copy-engine activity can be traced
// (`rocprofv3 --memory-copy-trace`) on the same C-ABI, plan and kernels the
// Python runner uses (StreamingAttentionRunner.__call__, reference
// src/seqattn_core/streaming/runner.py:80-138).
//
// usage: sa_pipeline_driver TOKENS HEADS HEAD_DIM Q_CHUNK KV_CHUNK NUM_KV NUM_OUT [STEPS]
//   One non-causal bf16 segment of TOKENS tokens with HEADS query and K/V
//   heads; Q_CHUNK / KV_CHUNK / NUM_KV / NUM_OUT are the planner's resident
//   Q block, K/V chunk, ring depth and output slots (build_plan prints them).
//   Inputs are a fixed bf16 pattern of magnitude < 1: the driver measures
//   transfers and time, not values (parity lives in the test suite).
//
// Prints one line per step: seconds, effective TFLOPS (4*H*D*N^2 / s) and the
// logical H2D / D2H bytes the pipeline reports.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "seqattn_hip.h"

namespace {

bool ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
  return false;
}

// Fill n bf16 values with a deterministic pattern in (-1, 1), in parallel.
void fill(uint16_t* dst, size_t n, uint32_t seed) {
  const unsigned workers = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  for (unsigned w = 0; w < workers; ++w) {
    pool.emplace_back([=] {
      const size_t lo = n * w / workers, hi = n * (w + 1) / workers;
      uint32_t x = seed ^ (0x9e3779b9u * (w + 1));
      for (size_t i = lo; i < hi; ++i) {
        x = x * 1664525u + 1013904223u;
        const float f = (float)((int32_t)(x >> 9) - (1 << 22)) / (float)(1 << 22);  // [-1, 1)
        uint32_t bits;
        std::memcpy(&bits, &f, 4);
        dst[i] = (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);  // round to nearest even
      }
    });
  }
  for (auto& t : pool) t.join();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 8) {
    std::fprintf(stderr,
                 "usage: %s TOKENS HEADS HEAD_DIM Q_CHUNK KV_CHUNK NUM_KV NUM_OUT [STEPS]\n", argv[0]);
    return 2;
  }
  const int64_t tokens = std::atoll(argv[1]);
  const int32_t heads = std::atoi(argv[2]), head_dim = std::atoi(argv[3]);
  const int32_t q_chunk = std::atoi(argv[4]), kv_chunk = std::atoi(argv[5]);
  const int32_t num_kv = std::atoi(argv[6]), num_out = std::atoi(argv[7]);
  const int steps = argc > 8 ? std::atoi(argv[8]) : 1;
  if (tokens <= 0 || heads <= 0 || head_dim <= 0 || q_chunk <= 0 || kv_chunk <= 0 || num_kv < 1 ||
      num_kv > 3 || num_out < 1 || num_out > 2 || steps < 1) {
    std::fprintf(stderr, "invalid arguments\n");
    return 2;
  }
  const size_t row = (size_t)heads * head_dim;           // elements per token
  const size_t host_bytes = (size_t)tokens * row * 2;    // one bf16 tensor
  void *qh = nullptr, *kh = nullptr, *vh = nullptr, *oh = nullptr;
  if (!ok(hipHostMalloc(&qh, host_bytes, 0), "hipHostMalloc q") ||
      !ok(hipHostMalloc(&kh, host_bytes, 0), "hipHostMalloc k") ||
      !ok(hipHostMalloc(&vh, host_bytes, 0), "hipHostMalloc v") ||
      !ok(hipHostMalloc(&oh, host_bytes, 0), "hipHostMalloc out"))
    return 1;
  fill(static_cast<uint16_t*>(qh), tokens * row, 1);
  fill(static_cast<uint16_t*>(kh), tokens * row, 2);
  fill(static_cast<uint16_t*>(vh), tokens * row, 3);

  // Workspace with the layout of CudaWorkspace: resident Q block, K/V ring,
  // fp32 state, output slots.
  void* q_buf = nullptr;
  void* k_slots[3] = {nullptr, nullptr, nullptr};
  void* v_slots[3] = {nullptr, nullptr, nullptr};
  void* out_slots[2] = {nullptr, nullptr};
  float *m = nullptr, *l = nullptr, *acc = nullptr;
  const size_t q_bytes = (size_t)q_chunk * row * 2, kv_bytes = (size_t)kv_chunk * row * 2;
  if (!ok(hipMalloc(&q_buf, q_bytes), "hipMalloc q block")) return 1;
  for (int i = 0; i < num_kv; ++i)
    if (!ok(hipMalloc(&k_slots[i], kv_bytes), "hipMalloc k slot") ||
        !ok(hipMalloc(&v_slots[i], kv_bytes), "hipMalloc v slot"))
      return 1;
  for (int i = 0; i < num_out; ++i)
    if (!ok(hipMalloc(&out_slots[i], q_bytes), "hipMalloc output slot")) return 1;
  if (!ok(hipMalloc((void**)&m, (size_t)q_chunk * heads * 4), "hipMalloc m") ||
      !ok(hipMalloc((void**)&l, (size_t)q_chunk * heads * 4), "hipMalloc l") ||
      !ok(hipMalloc((void**)&acc, (size_t)q_chunk * row * 4), "hipMalloc acc"))
    return 1;
  hipStream_t compute = nullptr;
  if (!ok(hipStreamCreate(&compute), "hipStreamCreate")) return 1;

  sa_pipeline* pipe = nullptr;
  int32_t rc = sa_pipeline_create(&pipe, 0, q_buf, k_slots, v_slots, num_kv, m, l, acc,
                                  out_slots, num_out, q_chunk, kv_chunk, heads,
                                  heads, head_dim, SA_DTYPE_BF16, nullptr, nullptr);
  if (rc) {
    std::fprintf(stderr, "sa_pipeline_create: %s\n", sa_last_error());
    return 1;
  }
  const int64_t cu[2] = {0, tokens};
  const double flop = 4.0 * heads * head_dim * (double)tokens * (double)tokens;
  for (int s = 0; s < steps; ++s) {
    sa_pipeline_stats st = {};
    const auto t0 = std::chrono::steady_clock::now();
    rc = sa_pipeline_run(pipe, qh, kh, vh, oh, nullptr, 0, cu, cu, 1, 1.0 / std::sqrt((double)head_dim), 0,
                         compute, &st);
    if (rc == 0 && !ok(hipStreamSynchronize(compute), "hipStreamSynchronize")) rc = 1;
    if (rc) {
      std::fprintf(stderr, "sa_pipeline_run: %s\n", sa_last_error());
      return 1;
    }
    const double sec = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    std::printf("step %d: %.3f s, %.1f TFLOPS, h2d %lld B, d2h %lld B\n", s, sec, flop / sec / 1e12,
                (long long)st.h2d_bytes, (long long)st.d2h_bytes);
    std::fflush(stdout);
  }
  sa_pipeline_destroy(pipe);
  (void)hipStreamDestroy(compute);
  for (void* ptr : {q_buf, k_slots[0], k_slots[1], k_slots[2], v_slots[0], v_slots[1], v_slots[2], out_slots[0],
                    out_slots[1], (void*)m, (void*)l, (void*)acc})
    if (ptr) (void)hipFree(ptr);
  for (void* ptr : {qh, kh, vh, oh}) (void)hipHostFree(ptr);
  return 0;
}
