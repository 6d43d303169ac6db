// Chunk-update and finalize kernels of the streamed exact-attention path for
// MI355X (gfx950, CDNA4), plus their C-ABI launchers.
//
// Semantics follow _streaming_attention_update_kernel and
// _finalize_attention_kernel (reference src/seqattn_core/kernels/streaming.py:19-156
// and :158-202): base-2 online softmax over one K/V chunk, FP32 state
// (m, l, acc) carried in HBM between chunks, P rounded to the input dtype
// before the PV product, out = acc / l (0 where l == 0).  The finalize kernel
// also writes LSE = (m + log2 l) * ln 2, which the reference does not produce.
//
// Work decomposition (update kernel):
//   workgroup = 4 wavefronts = 128 queries of one query head; grid
//   (ceil(q_tokens / 128), q_heads).  Wave w owns queries 32w..32w+31.
//   K/V are streamed through LDS in 64-key tiles: K row-major
//   [key][d], V transposed [d][key], both padded against bank conflicts.
//   The next tile's global loads are issued before the current tile's MFMA
//   work so HBM/L2 latency hides under compute.
//
// MFMA mapping (v_mfma_f32_32x32x16_{bf16,f16}: A 32x16, B 16x32, C 32x32):
//   S^T[key][query] = K . Q^T : A = K rows from LDS, B = Q fragments held in
//   registers for the whole kernel.  In the C layout a lane owns one query
//   column and 16 key rows, so the row max / row sum of the softmax are
//   in-lane reductions plus one exchange with lane ^ 32.
//   O^T[d][query] += V^T . P^T : B = P^T taken straight from the S^T
//   registers (same lane, same query), A = V^T rows from LDS.  The accumulator
//   lane again owns one query, so the alpha rescale is a lane-uniform scalar.
//   The contraction slot (lane half h, element e) -> key assignment only has
//   to agree between A and B, which both sides construct identically.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "sa_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlockM = 32 * kWaves;  // queries per workgroup
constexpr int kBlockN = 64;           // keys per LDS tile
constexpr int kVtPad = 4;             // V^T row padding (elements)
constexpr int kKPad = 8;              // K row padding (elements)

struct BF16 {
  __device__ static inline f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Two floats -> two round-to-nearest-even bf16 packed in one dword (low = a).
  __device__ static inline uint32_t pack2(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct FP16 {
  __device__ static inline f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct UpdateParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* m;
  float* l;
  float* acc;
  int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, ss_t, ss_h, sa_t, sa_h;
  int32_t q_tokens, kv_tokens, group, head_dim;
  int32_t q_local_offset, kv_local_offset, causal_shift;
  float scale_log2;
};

// Row r (0..15) of a 32x32 C tile held in register i of a lane in half h.
__device__ inline int c_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

template <typename Op, int DP, bool CAUSAL, bool INIT>
__global__ __launch_bounds__(kThreads) void update_kernel(const UpdateParams p) {
  constexpr int KROW = DP + kKPad;
  constexpr int VROW = kBlockN + kVtPad;
  constexpr int QC = DP / 16;  // 16-wide d slices of the QK^T contraction
  constexpr int DB = DP / 32;  // 32-row d blocks of the PV output
  constexpr int KL = (kBlockN * DP / 8) / kThreads;  // 16-byte K loads per thread
  constexpr int VBLOCKS = (kBlockN / 4) * (DP / 8);  // 4-key x 8-d V blocks per tile
  constexpr int VL = (VBLOCKS + kThreads - 1) / kThreads;
  static_assert(KL >= 1, "tile too small for the workgroup");

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBlockN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[DP * VROW];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lr = lane & 31;
  const int hf = lane >> 5;

  const int head = blockIdx.y;
  const int kv_head = head / p.group;
  const int q_block = blockIdx.x * kBlockM;
  const int qw0 = q_block + wave * 32;  // first query of this wave
  const int qi = qw0 + lr;              // this lane's query
  const bool q_ok = qi < p.q_tokens;

  const uint16_t* qp = p.q + (int64_t)head * p.sq_h;
  const uint16_t* kp = p.k + (int64_t)kv_head * p.sk_h;
  const uint16_t* vp = p.v + (int64_t)kv_head * p.sv_h;

  // Q fragments (B operand of S^T = K Q^T): query qi, d = 16c + 8h .. +7.
  u32x4 qf[QC];
#pragma unroll
  for (int c = 0; c < QC; ++c) {
    const int d = 16 * c + 8 * hf;
    if (q_ok && d < p.head_dim)
      qf[c] = *reinterpret_cast<const u32x4*>(qp + (int64_t)qi * p.sq_t + d);
    else
      qf[c] = u32x4{0, 0, 0, 0};
  }

  // Online-softmax state of query qi (base-2 domain).
  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x16 acc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) acc[b] = f32x16{};
  const int64_t srow = (int64_t)qi * p.ss_t + (int64_t)head * p.ss_h;
  float* arow = p.acc + (int64_t)qi * p.sa_t + (int64_t)head * p.sa_h;
  if (!INIT && q_ok) {
    m_run = p.m[srow];
    l_run = p.l[srow];
#pragma unroll
    for (int b = 0; b < DB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * b + 8 * g + 4 * hf;
        if (d < p.head_dim) {
          const f32x4 v4 = *reinterpret_cast<const f32x4*>(arow + d);
          acc[b][4 * g + 0] = v4[0];
          acc[b][4 * g + 1] = v4[1];
          acc[b][4 * g + 2] = v4[2];
          acc[b][4 * g + 3] = v4[3];
        }
      }
    }
  }

  // Keys at or beyond kv_end are invisible to every query of this workgroup.
  int kv_end = p.kv_tokens;
  if (CAUSAL) {
    const int q_last = min(p.q_tokens, q_block + kBlockM) - 1;
    const int lim = p.q_local_offset + q_last + p.causal_shift - p.kv_local_offset + 1;
    kv_end = max(0, min(kv_end, lim));
  }
  const int ntiles = (kv_end + kBlockN - 1) / kBlockN;

  // Register staging of the next tile.
  u32x4 kreg[KL];
  u32x4 vreg[VL][4];

  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int c = tid + i * kThreads;
      const int key = c / (DP / 8);
      const int d = (c % (DP / 8)) * 8;
      if (kt + key < p.kv_tokens && d < p.head_dim)
        kreg[i] = *reinterpret_cast<const u32x4*>(kp + (int64_t)(kt + key) * p.sk_t + d);
      else
        kreg[i] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int b = tid + i * kThreads;
      const int k4 = b % (kBlockN / 4);
      const int d = (b / (kBlockN / 4)) * 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kt + 4 * k4 + r;
        if (b < VBLOCKS && key < p.kv_tokens && d < p.head_dim)
          vreg[i][r] = *reinterpret_cast<const u32x4*>(vp + (int64_t)key * p.sv_t + d);
        else
          vreg[i][r] = u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int c = tid + i * kThreads;
      const int key = c / (DP / 8);
      const int d = (c % (DP / 8)) * 8;
      *reinterpret_cast<u32x4*>(&k_lds[key * KROW + d]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int b = tid + i * kThreads;
      if (b < VBLOCKS) {
        const int k4 = b % (kBlockN / 4);
        const int d = (b / (kBlockN / 4)) * 8;
        // vreg[i][r] holds V[key 4*k4 + r][d .. d+7]; emit V^T[d + e][4*k4 .. +3].
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t x0 = vreg[i][0][w], x1 = vreg[i][1][w];
          const uint32_t x2 = vreg[i][2][w], x3 = vreg[i][3][w];
          const u32x2 even = {(x0 & 0xffffu) | (x1 << 16), (x2 & 0xffffu) | (x3 << 16)};
          const u32x2 odd = {(x0 >> 16) | (x1 & 0xffff0000u), (x2 >> 16) | (x3 & 0xffff0000u)};
          *reinterpret_cast<u32x2*>(&vt_lds[(d + 2 * w) * VROW + 4 * k4]) = even;
          *reinterpret_cast<u32x2*>(&vt_lds[(d + 2 * w + 1) * VROW + 4 * k4]) = odd;
        }
      }
    }
  };

  if (ntiles > 0) load_tile(0);

  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * kBlockN;
    __syncthreads();  // every wave is done reading the previous tile
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) load_tile(kt + kBlockN);

    // S^T for the two 32-key halves of the tile.
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int c = 0; c < QC; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&k_lds[(32 * kb + lr) * KROW + 16 * c + 8 * hf]);
        s[kb] = Op::mma(a, qf[c], s[kb]);
      }
    }

    // Scaled logits, masking, tile max.
    bool need_mask = kt + kBlockN > p.kv_tokens;
    if (CAUSAL)
      need_mask = need_mask ||
                  (p.kv_local_offset + kt + kBlockN - 1 > p.q_local_offset + qw0 + p.causal_shift);
    float x[2][16];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float val = s[kb][i] * p.scale_log2;
        if (need_mask) {
          const int key = kt + 32 * kb + c_row(i, hf);
          bool ok = key < p.kv_tokens;
          if (CAUSAL) ok = ok && (p.kv_local_offset + key <= p.q_local_offset + qi + p.causal_shift);
          val = ok ? val : -INFINITY;
        }
        x[kb][i] = val;
        mx = fmaxf(mx, val);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const bool row_ok = m_new != -INFINITY;
    const float alpha = row_ok ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
    const float m_use = row_ok ? m_new : 0.f;

    // P^T (as PV B operands) and its row sum.
    float psum = 0.f;
    u32x4 pf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = __builtin_amdgcn_exp2f(x[kb][8 * half + 2 * e] - m_use);
          const float p1 = __builtin_amdgcn_exp2f(x[kb][8 * half + 2 * e + 1] - m_use);
          psum += p0 + p1;
          pf[2 * kb + half][e] = Op::pack2(p0, p1);
        }
      }
    }
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = row_ok ? m_new : m_run;

    // O^T = O^T * alpha + V^T P^T.
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      acc[b] *= alpha;
      const uint16_t* vrow = &vt_lds[(32 * b + lr) * VROW + 4 * hf];
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const u32x2 a0 = *reinterpret_cast<const u32x2*>(vrow + 16 * kc);
        const u32x2 a1 = *reinterpret_cast<const u32x2*>(vrow + 16 * kc + 8);
        const u32x4 a = {a0[0], a0[1], a1[0], a1[1]};
        acc[b] = Op::mma(a, pf[kc], acc[b]);
      }
    }
  }

  if (q_ok) {
    if (hf == 0) {
      p.m[srow] = m_run;
      p.l[srow] = l_run;
    }
#pragma unroll
    for (int b = 0; b < DB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * b + 8 * g + 4 * hf;
        if (d < p.head_dim) {
          const f32x4 v4 = {acc[b][4 * g + 0], acc[b][4 * g + 1], acc[b][4 * g + 2], acc[b][4 * g + 3]};
          *reinterpret_cast<f32x4*>(arow + d) = v4;
        }
      }
    }
  }
}

struct FinalizeParams {
  const float* acc;
  const float* m;
  const float* l;
  uint16_t* out;
  float* lse;
  int64_t sa_t, sa_h, ss_t, ss_h, so_t, so_h, lse_sh, lse_off;
  int64_t total;  // q_tokens * q_heads * (head_dim / 8)
  int32_t q_heads, groups;
};

template <typename Op>
__global__ __launch_bounds__(256) void finalize_kernel(const FinalizeParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.total) return;
  const int g = (int)(idx % p.groups);
  const int64_t row = idx / p.groups;
  const int h = (int)(row % p.q_heads);
  const int64_t t = row / p.q_heads;
  const float l = p.l[t * p.ss_t + h * p.ss_h];
  const float* a = p.acc + t * p.sa_t + h * p.sa_h + 8 * g;
  const f32x4 a0 = *reinterpret_cast<const f32x4*>(a);
  const f32x4 a1 = *reinterpret_cast<const f32x4*>(a + 4);
  u32x4 o;
  if (l > 0.f) {
    o[0] = Op::pack2(a0[0] / l, a0[1] / l);
    o[1] = Op::pack2(a0[2] / l, a0[3] / l);
    o[2] = Op::pack2(a1[0] / l, a1[1] / l);
    o[3] = Op::pack2(a1[2] / l, a1[3] / l);
  } else {
    o = u32x4{0, 0, 0, 0};
  }
  *reinterpret_cast<u32x4*>(p.out + t * p.so_t + h * p.so_h + 8 * g) = o;
  if (p.lse != nullptr && g == 0) {
    const float m = p.m[t * p.ss_t + h * p.ss_h];
    p.lse[h * p.lse_sh + p.lse_off + t] =
        l > 0.f ? (m + log2f(l)) * 0.69314718055994530942f : -INFINITY;
  }
}

template <typename Op, int DP>
hipError_t launch_update_dp(const UpdateParams& p, bool causal, bool init, dim3 grid, hipStream_t s) {
  if (causal) {
    if (init)
      hipLaunchKernelGGL((update_kernel<Op, DP, true, true>), grid, dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((update_kernel<Op, DP, true, false>), grid, dim3(kThreads), 0, s, p);
  } else {
    if (init)
      hipLaunchKernelGGL((update_kernel<Op, DP, false, true>), grid, dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((update_kernel<Op, DP, false, false>), grid, dim3(kThreads), 0, s, p);
  }
  return hipGetLastError();
}

template <typename Op>
hipError_t launch_update_op(const UpdateParams& p, int dp, bool causal, bool init, dim3 grid,
                            hipStream_t s) {
  switch (dp) {
    case 32: return launch_update_dp<Op, 32>(p, causal, init, grid, s);
    case 64: return launch_update_dp<Op, 64>(p, causal, init, grid, s);
    case 128: return launch_update_dp<Op, 128>(p, causal, init, grid, s);
    default: return launch_update_dp<Op, 256>(p, causal, init, grid, s);
  }
}

inline bool aligned(const void* ptr, uintptr_t n) { return (reinterpret_cast<uintptr_t>(ptr) % n) == 0; }

}  // namespace

namespace sa {

int32_t launch_update(const void* q, const void* k, const void* v, float* m, float* l, float* acc,
                      int64_t sq_t, int64_t sq_h, int64_t sk_t, int64_t sk_h, int64_t sv_t,
                      int64_t sv_h, int64_t ss_t, int64_t ss_h, int64_t sa_t, int64_t sa_h,
                      int32_t q_tokens, int32_t kv_tokens, int32_t q_heads, int32_t kv_heads,
                      int32_t head_dim, int32_t q_local_offset, int32_t kv_local_offset,
                      int32_t causal_shift, double softmax_scale, int32_t flags, int32_t dtype,
                      hipStream_t stream) {
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    set_error("sa_update_attention_state: unsupported dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (head_dim < 16 || head_dim > 256 || head_dim % 8 != 0) {
    set_error("sa_update_attention_state: head_dim must be a multiple of 8 in [16, 256], got %d",
              head_dim);
    return SA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  if (q_tokens < 0 || kv_tokens < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0) {
    set_error("sa_update_attention_state: bad sizes q_tokens=%d kv_tokens=%d q_heads=%d kv_heads=%d",
              q_tokens, kv_tokens, q_heads, kv_heads);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (q_tokens == 0) return 0;
  if (!q || !k || !v || !m || !l || !acc) {
    set_error("sa_update_attention_state: null pointer argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  // 16-byte vector access of 8 elements (inputs) and 4 floats (accumulator).
  const int64_t el_strides[] = {sq_t, sq_h, sk_t, sk_h, sv_t, sv_h};
  for (int64_t st : el_strides) {
    if (st % 8 != 0) {
      set_error("sa_update_attention_state: q/k/v token and head strides must be multiples of 8 elements");
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  if (sa_t % 4 != 0 || sa_h % 4 != 0 || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) ||
      !aligned(acc, 16) || !aligned(m, 4) || !aligned(l, 4)) {
    set_error("sa_update_attention_state: buffers must be 16-byte aligned with vector-aligned strides");
    return SA_ERR_INVALID_ARGUMENT;
  }
  UpdateParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.m = m;
  p.l = l;
  p.acc = acc;
  p.sq_t = sq_t; p.sq_h = sq_h; p.sk_t = sk_t; p.sk_h = sk_h; p.sv_t = sv_t; p.sv_h = sv_h;
  p.ss_t = ss_t; p.ss_h = ss_h; p.sa_t = sa_t; p.sa_h = sa_h;
  p.q_tokens = q_tokens;
  p.kv_tokens = kv_tokens;
  p.group = q_heads / kv_heads;
  p.head_dim = head_dim;
  p.q_local_offset = q_local_offset;
  p.kv_local_offset = kv_local_offset;
  p.causal_shift = causal_shift;
  p.scale_log2 = (float)(softmax_scale * 1.4426950408889634);
  const int dp = head_dim <= 32 ? 32 : head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
  const dim3 grid((q_tokens + kBlockM - 1) / kBlockM, q_heads);
  const bool causal = (flags & SA_FLAG_CAUSAL) != 0;
  const bool init = (flags & SA_FLAG_INITIALIZE) != 0;
  hipError_t err = dtype == SA_DTYPE_BF16 ? launch_update_op<BF16>(p, dp, causal, init, grid, stream)
                                          : launch_update_op<FP16>(p, dp, causal, init, grid, stream);
  return err == hipSuccess ? 0 : hip_status(err, "update kernel launch");
}

int32_t launch_finalize(const float* acc, const float* m, const float* l, void* out, float* lse,
                        int64_t sa_t, int64_t sa_h, int64_t ss_t, int64_t ss_h, int64_t so_t,
                        int64_t so_h, int64_t lse_sh, int64_t lse_off, int32_t q_tokens,
                        int32_t q_heads, int32_t head_dim, int32_t dtype, hipStream_t stream) {
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    set_error("sa_finalize_attention: unsupported dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (head_dim < 8 || head_dim > 256 || head_dim % 8 != 0) {
    set_error("sa_finalize_attention: head_dim must be a multiple of 8 in [8, 256], got %d", head_dim);
    return SA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  if (q_tokens < 0 || q_heads <= 0) {
    set_error("sa_finalize_attention: bad sizes q_tokens=%d q_heads=%d", q_tokens, q_heads);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (q_tokens == 0) return 0;
  if (!acc || !l || !out || (lse && !m)) {
    set_error("sa_finalize_attention: null pointer argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (sa_t % 4 != 0 || sa_h % 4 != 0 || so_t % 8 != 0 || so_h % 8 != 0 || !aligned(acc, 16) ||
      !aligned(out, 16)) {
    set_error("sa_finalize_attention: buffers must be 16-byte aligned with vector-aligned strides");
    return SA_ERR_INVALID_ARGUMENT;
  }
  FinalizeParams p;
  p.acc = acc;
  p.m = m;
  p.l = l;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.sa_t = sa_t; p.sa_h = sa_h; p.ss_t = ss_t; p.ss_h = ss_h; p.so_t = so_t; p.so_h = so_h;
  p.lse_sh = lse_sh;
  p.lse_off = lse_off;
  p.groups = head_dim / 8;
  p.q_heads = q_heads;
  p.total = (int64_t)q_tokens * q_heads * p.groups;
  const dim3 grid((unsigned)((p.total + 255) / 256));
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL(finalize_kernel<BF16>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(finalize_kernel<FP16>, grid, dim3(256), 0, stream, p);
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_status(err, "finalize kernel launch");
}

}  // namespace sa

extern "C" {

int32_t sa_update_attention_state(const void* q, const void* k, const void* v, float* running_max,
                                  float* running_sum, float* accumulator, int64_t stride_qt,
                                  int64_t stride_qh, int64_t stride_kt, int64_t stride_kh,
                                  int64_t stride_vt, int64_t stride_vh, int64_t stride_st,
                                  int64_t stride_sh, int64_t stride_at, int64_t stride_ah,
                                  int32_t q_tokens, int32_t kv_tokens, int32_t q_heads,
                                  int32_t kv_heads, int32_t head_dim, int32_t q_local_offset,
                                  int32_t kv_local_offset, int32_t causal_shift,
                                  double softmax_scale, int32_t flags, int32_t dtype, void* stream) {
  sa::clear_error();
  return sa::launch_update(q, k, v, running_max, running_sum, accumulator, stride_qt, stride_qh,
                           stride_kt, stride_kh, stride_vt, stride_vh, stride_st, stride_sh,
                           stride_at, stride_ah, q_tokens, kv_tokens, q_heads, kv_heads, head_dim,
                           q_local_offset, kv_local_offset, causal_shift, softmax_scale, flags,
                           dtype, static_cast<hipStream_t>(stream));
}

int32_t sa_finalize_attention(const float* accumulator, const float* running_max,
                              const float* running_sum, void* out, float* lse, int64_t stride_at,
                              int64_t stride_ah, int64_t stride_st, int64_t stride_sh,
                              int64_t stride_ot, int64_t stride_oh, int64_t lse_stride_h,
                              int64_t lse_token_offset, int32_t q_tokens, int32_t q_heads,
                              int32_t head_dim, int32_t dtype, void* stream) {
  sa::clear_error();
  return sa::launch_finalize(accumulator, running_max, running_sum, out, lse, stride_at, stride_ah,
                             stride_st, stride_sh, stride_ot, stride_oh, lse_stride_h,
                             lse_token_offset, q_tokens, q_heads, head_dim, dtype,
                             static_cast<hipStream_t>(stream));
}

}  // extern "C"
