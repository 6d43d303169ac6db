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
// Update kernel work decomposition:
//   head_dim 72..128 (update48_kernel): workgroup = 8 wavefronts (two per
//   SIMD), each owning 48 queries of one query head (384 queries per
//   workgroup) as three 16-query blocks of 16x16x32 MFMAs; while one wave of
//   a SIMD waits on LDS or on the MFMA pipe the other issues.  Head dims 16..64
//   and 256 (update_kernel): 4 wavefronts (one per SIMD) owning QB blocks of
//   32 queries (QB = 2 for head_dim <= 64, 1 for 256) with 32x32x16 MFMAs.
//   Either way each K/V fragment read from LDS feeds several MFMAs.
//   Workgroups are numbered head-major and dealt to the 8 XCDs in contiguous
//   runs, so the workgroups resident on one XCD share one head's K/V stream in
//   that XCD's L2.
//   K/V stream through LDS in 64-key tiles, two stages: the tile after the one
//   being computed is fetched by global_load_lds_dwordx4 (HBM/L2 -> LDS with
//   no register staging) while the MFMAs run; one barrier per tile.
//   LDS rows are row-major [key][d] with 16-byte granules XOR-swizzled by the
//   row index, which keeps both the K operand reads (ds_read_b128, 8
//   consecutive keys per phase) and the transposing V reads
//   (ds_read_b64_tr_b16, 4 consecutive keys per 16-lane group) free of bank
//   conflicts.
//
// MFMA mapping of update_kernel (v_mfma_f32_32x32x16_{bf16,f16}: A 32x16,
// B 16x32, C 32x32; update48_kernel's 16x16x32 mapping is described there):
//   S^T[key][query] = K . Q^T : A = K rows (LDS), B = Q fragments held in
//   registers for the whole kernel.  In the C layout a lane owns one query
//   column and 16 key rows, so softmax row reductions are in-lane.
//   O^T[d][query] += V^T . P^T : B = P^T straight from the S^T registers (same
//   lane, same query), A = V^T fragments produced by ds_read_b64_tr_b16 from
//   the row-major V tile.  The contraction slot (lane half h, element e) ->
//   key assignment is the same on both sides: key = 16c + 8(e/4) + 4h + e%4.
//   Each K/V fragment read from LDS feeds QB MFMAs.
//
// Online softmax with a thresholded rescale: a query's running maximum m only
// moves (and its acc, l are rescaled by exp2(m_old - m_new)) when one of its
// logits exceeds m + 8; otherwise p = exp2(s*scale - m) <= 2^8 against the
// kept m.  The decision is per query, so results do not depend on how queries
// are grouped into wavefronts or Q blocks.
// Each step first computes P against the kept m and tests the lane's partial
// row sum: every p <= 2^8 whenever that sum is, so the row maximum (and its
// cross-lane exchange) is only taken on the rare steps that may rescale, and
// the result is the same as deciding on the maximum.
// (m, l, acc) remains an exact representation of the partial softmax:
// out = acc / l and LSE = m + log2(l) are unchanged, and P keeps bf16's
// relative precision.  The row sum l is accumulated per lane half and the two
// halves are combined once when the state is written.
//
// INT8 K/V (update_attention_state_int8, reference kernels/streaming.py:113-120
// and :274-342): int8 rows with one fp16 scale per (token group, K/V head).
// Raw int8 tiles (half the bytes of bf16) arrive by LDS DMA into a staging
// area; one pass per tile turns them into the bf16/fp16 stage layout above as
// dtype(fp32(k) * fp32(scale)), exactly the reference's dequantization, so
// the MFMA loop is shared and the result equals the 16-bit kernel run on
// dequantized K/V bit for bit.  Per tile: DMA of tile t+2, dequantization of
// tile t+1 and the MFMAs of tile t, one barrier.  Each thread's scales for
// the next tile are loaded into registers one tile ahead.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

#include "sa_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

#define SA_LDS __attribute__((address_space(3)))
#define SA_GLOBAL __attribute__((address_space(1)))

constexpr int kSubKeys = 32;   // keys per softmax step
constexpr float kRescaleThreshold = 8.0f;  // log2 units

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
  int32_t q_tokens, kv_tokens, group, head_dim, q_heads;
  int32_t q_local_offset, kv_local_offset, causal_shift;
  int32_t q_blocks;       // workgroups per query head
  int32_t xcd_run;        // ceil(q_blocks * q_heads / 8)
  int32_t deal_blocks;    // causal, q_heads not a multiple of 8: every XCD takes every eighth block
  float scale_log2;
  // INT8 K/V only: fp16 scales, element (group, kv_head) at
  // scales[group * s?s_g + kv_head * s?s_h], group = (scale_offset + key) >> scale_shift.
  const uint16_t* ks;
  const uint16_t* vs;
  int64_t sks_g, sks_h, svs_g, svs_h;
  int32_t scale_offset, scale_shift;
  // 16-bit launches spanning several K/V chunks of the streamed schedule:
  // the tile count of one chunk (0: one chunk).  At each chunk boundary the
  // two lane halves' partial row sums are merged exactly as a chunk launch
  // stores l and the next one reloads it, so the result equals the chunked
  // schedule's bit for bit.
  int32_t merge_tiles = 0;
  // Fused finalize, for the launch that applies the last keys of its rows
  // (with or without loading the state first): when out is non-null the
  // epilogue writes acc / l (0 where l == 0) to out and, when lse is
  // non-null, (m + log2 l) ln 2 (-inf where l == 0) to
  // lse[head * lse_sh + lse_off + query], with the expressions of
  // finalize_kernel, and stores no state.  out may alias q: each query's
  // row of one head is read (at the start) and written (at the end) by the
  // same wave only.
  uint16_t* out = nullptr;
  int64_t so_t = 0, so_h = 0;
  float* lse = nullptr;
  int64_t lse_sh = 0, lse_off = 0;
  // State in the pipeline's row-group layout (state_offset) instead of the
  // strided [token][head] layout given by ss_* / sa_*.
  int32_t tiled_state = 0;
};

// Pipeline-owned FP32 state is kept in the order the update kernels' lanes
// hold it.  Rows form groups of 16; group g of head h is one block of
// 16 * head_dim floats (and 16 floats of m, of l) at block index
// g * q_heads + h, so row r of a buffer sits where the token-major layout
// would put it, rounded to its 16-row group.  Within a block, 4-float chunk c
// (d = 4c .. 4c + 3) of row r is at (c * 16 + r) * 4.  A wave's state
// instruction then covers whole 256-byte runs (16 rows of one chunk) where
// the token-major layout touched one 16- or 32-byte piece per row, rows
// q_heads * head_dim * 4 bytes apart.
__device__ inline int64_t state_block(int64_t row, int head, int q_heads) {
  return (row >> 4) * q_heads + head;
}

// Row r (0..15) of a 32x32 C tile held in register i of a lane in half h.
__device__ inline int c_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// Positive factor applied to raw logits inside the exponent's FMA (so the
// running max can be taken before scaling): |scale|, at least 1e-30.
__device__ inline float scale_factor(float scale_log2) { return fmaxf(fabsf(scale_log2), 1e-30f); }

// Sign-bit mask that negates every 16-bit element of a Q fragment when the
// scale is negative: s * scale == (-q . k) * |scale|, exactly.
__device__ inline u32x4 q_sign(float scale_log2) {
  const uint32_t m = scale_log2 < 0.f ? 0x80008000u : 0u;
  return u32x4{m, m, m, m};
}

template <int DP>
struct Geometry {
  static constexpr int G = DP / 8;             // 16-byte granules per K/V row
  static constexpr int ROW_BYTES = DP * 2;
  // Four wavefronts of 64 queries (32 for head_dim 256), each K/V fragment
  // read from LDS feeding two MFMAs.
  static constexpr int WAVES = 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QB = DP >= 128 ? 1 : 2;  // 32-query blocks per wave
  static constexpr int BLOCK_M = WAVES * 32 * QB;
  static constexpr int TILE_KEYS = 64;                       // keys per LDS stage
  static constexpr int TILE_BYTES = TILE_KEYS * ROW_BYTES;  // K (or V) part of a stage
  static constexpr int ROWS_PER_DMA = 1024 / ROW_BYTES;     // rows per wave-wide 1 KB DMA
  static constexpr int DMA_PER_WAVE = TILE_KEYS / ROWS_PER_DMA / WAVES;
  // K fragments requested ahead of their MFMAs, and V^T d-blocks per batch
  // of transposing reads.
  static constexpr int KB = DP / 16;
  static constexpr int VB = DP / 32 < 4 ? DP / 32 : 4;
  static_assert(DMA_PER_WAVE >= 1, "tile too small for the workgroup");
  // INT8 staging: a tile is 64 rows of DP bytes; a wave-wide 16-byte-per-lane
  // DMA moves 1 KB, I8_GR granules of 16 int8 per row.
  static constexpr int I8_TILE_BYTES = TILE_KEYS * DP;
  static constexpr int I8_GR = DP / 16;
  static constexpr int I8_DMAS = I8_TILE_BYTES / 1024;                // per tensor per tile
  static constexpr int I8_DMA_PER_WAVE = (I8_DMAS + WAVES - 1) / WAVES;
  static constexpr int I8_GRANULES = TILE_KEYS * I8_GR;               // per tensor per tile
  static constexpr int I8_PER_THREAD = (I8_GRANULES + THREADS - 1) / THREADS;
  // Granule swizzle: 8 distinct masks over 8 consecutive rows, so the K
  // reads (ds_read_b128, consecutive rows at one logical granule) and the
  // transposing V reads (4-row blocks) spread over the banks.
  __device__ static inline int swz(int row) {
    return (((row & 3) << 1) | ((row >> 2) & 1)) & (G - 1);
  }
  __device__ static inline int offset(int row, int granule) {
    return row * ROW_BYTES + ((granule ^ swz(row)) << 4);
  }
};

template <typename Op, int DP, bool CAUSAL, bool INIT, bool QUANT>
__global__ __launch_bounds__(Geometry<DP>::THREADS) void update_kernel(const UpdateParams p) {
  using Geo = Geometry<DP>;
  static_assert(DP != 128, "head_dim 128 runs update48_kernel");
  constexpr int QB = Geo::QB;
  constexpr int QC = DP / 16;  // 16-wide d slices of the QK^T contraction
  constexpr int DB = DP / 32;  // 32-row d blocks of the PV output
  constexpr int G = Geo::G;

  // Two LDS stages as distinct objects: every LDS read and every DMA target
  // below names one of them statically, so the compiler can tell that the
  // in-flight prefetch into one stage does not alias reads of the other and
  // need not wait for it.
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a[2 * Geo::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b[2 * Geo::TILE_BYTES];
  // INT8 staging (K then V of one raw tile), also two distinct objects.
  constexpr int kStagingBytes = QUANT ? 2 * Geo::I8_TILE_BYTES : 16;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_qa[kStagingBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_qb[kStagingBytes];

  // XCD-aware numbering: hardware block b runs on XCD b % 8; consecutive
  // logical workgroups (same head, neighbouring query blocks) share an XCD.
  // Under a causal mask later query blocks see more keys: they are dealt
  // first so that the short blocks fill the end of the launch.  Unless the
  // launch's heads are a multiple of 8 (then each XCD's run holds whole
  // heads and the runs are kept), a contiguous run would give some XCD more
  // than its share of long blocks, so in causal launches every XCD takes
  // every eighth block instead (measured: 1.7x the runs' rate on one head,
  // 1.14x on 12).
  const int b = blockIdx.x;
  const int logical = (CAUSAL && p.deal_blocks) ? b : (b & 7) * p.xcd_run + (b >> 3);
  if (logical >= p.q_blocks * p.q_heads) return;
  const int head = logical / p.q_blocks;
  const int qb_index = CAUSAL ? p.q_blocks - 1 - (logical - head * p.q_blocks) : logical - head * p.q_blocks;
  const int q_block = qb_index * Geo::BLOCK_M;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lr = lane & 31;
  const int hf = lane >> 5;
  const int kv_head = head / p.group;
  const int qw0 = q_block + wave * 32 * QB;  // first query of this wave

  const uint16_t* qp = p.q + (int64_t)head * p.sq_h;
  const uint16_t* kp = p.k + (int64_t)kv_head * p.sk_h;
  const uint16_t* vp = p.v + (int64_t)kv_head * p.sv_h;

  // Q fragments (B operand of S^T = K Q^T): query qw0 + 32qb + lr, d = 16c + 8h .. +7.
  u32x4 qf[QB][QC];
  int qi[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qi[qb] = qw0 + 32 * qb + lr;
    const bool ok = qi[qb] < p.q_tokens;
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      const int d = 16 * c + 8 * hf;
      if (ok && d < p.head_dim)
        qf[qb][c] = *reinterpret_cast<const u32x4*>(qp + (int64_t)qi[qb] * p.sq_t + d) ^ q_sign(p.scale_log2);
      else
        qf[qb][c] = u32x4{0, 0, 0, 0};
    }
  }

  // Online-softmax state (base-2 domain).  l_part is this lane half's share of l.
  float m_run[QB], l_part[QB];
  f32x16 acc[QB][DB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_part[qb] = 0.f;
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[qb][d] = f32x16{};
    if (!INIT && qi[qb] < p.q_tokens) {
      const int64_t blk = state_block(qi[qb], head, p.q_heads);
      const int r = qi[qb] & 15;
      const int64_t srow = p.tiled_state ? blk * 16 + r : (int64_t)qi[qb] * p.ss_t + (int64_t)head * p.ss_h;
      m_run[qb] = p.m[srow];
      l_part[qb] = hf == 0 ? p.l[srow] : 0.f;
      const float* arow = p.tiled_state ? p.acc + blk * 16 * p.head_dim + 4 * r
                                        : p.acc + (int64_t)qi[qb] * p.sa_t + (int64_t)head * p.sa_h;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = 32 * d + 8 * g + 4 * hf;
          if (col < p.head_dim) {
            const f32x4 v4 = *reinterpret_cast<const f32x4*>(arow + (p.tiled_state ? 16 * col : col));
            acc[qb][d][4 * g + 0] = v4[0];
            acc[qb][d][4 * g + 1] = v4[1];
            acc[qb][d][4 * g + 2] = v4[2];
            acc[qb][d][4 * g + 3] = v4[3];
          }
        }
      }
    }
  }

  // Keys at or beyond kv_end are invisible to every query of this workgroup.
  int kv_end = p.kv_tokens;
  if (CAUSAL) {
    const int q_last = min(p.q_tokens, q_block + Geo::BLOCK_M) - 1;
    const int lim = p.q_local_offset + q_last + p.causal_shift - p.kv_local_offset + 1;
    kv_end = max(0, min(kv_end, lim));
  }
  const int ntiles = (kv_end + Geo::TILE_KEYS - 1) / Geo::TILE_KEYS;

  // The scale is fused into the exponent's FMA and the max is taken on raw
  // logits, which needs a positive factor: a negative scale was folded into
  // the sign of Q when the fragments were loaded, and a zero scale becomes
  // 1e-30 (every logit then rounds to the same exponent, as with zero).
  const float cf = scale_factor(p.scale_log2);

  // HBM/L2 -> LDS DMA of key tile [kt, kt + 64) into stage st.  Each lane's
  // element offset within a tile is fixed (precomputed below); the tile base
  // is wave-uniform.  In the tail tile, rows past the chunk are clamped to its
  // last row, and granules past head_dim always read granule 0: those values
  // are finite and masked (keys) or multiplied by zero Q / never stored (d),
  // and every address stays inside the caller's buffers.
  int k_off[Geo::DMA_PER_WAVE], v_off[Geo::DMA_PER_WAVE], dma_row[Geo::DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < Geo::DMA_PER_WAVE; ++i) {
    const int chunk = wave * Geo::DMA_PER_WAVE + i;
    const int row = chunk * Geo::ROWS_PER_DMA + lane / G;
    const int lg = (lane % G) ^ Geo::swz(row);
    const int col = (lg * 8 < p.head_dim) ? lg * 8 : 0;
    dma_row[i] = row;
    k_off[i] = row * (int)p.sk_t + col;
    v_off[i] = row * (int)p.sv_t + col;
  }
  auto issue_tile = [&](int kt, uint8_t* stage) {
    uint8_t* k_stage = stage;
    uint8_t* v_stage = stage + Geo::TILE_BYTES;
    const uint16_t* kt_base = kp + (int64_t)kt * p.sk_t;
    const uint16_t* vt_base = vp + (int64_t)kt * p.sv_t;
    const bool tail = kt + Geo::TILE_KEYS > p.kv_tokens;
#pragma unroll
    for (int i = 0; i < Geo::DMA_PER_WAVE; ++i) {
      const int chunk = wave * Geo::DMA_PER_WAVE + i;
      int ko = k_off[i], vo = v_off[i];
      if (tail && kt + dma_row[i] >= p.kv_tokens) {
        const int back = kt + dma_row[i] - (p.kv_tokens - 1);  // rows to step back
        ko -= back * (int)p.sk_t;
        vo -= back * (int)p.sv_t;
      }
      __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(kt_base + ko),
                                       (SA_LDS void*)(k_stage + chunk * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(vt_base + vo),
                                       (SA_LDS void*)(v_stage + chunk * 1024), 16, 0, 0);
    }
  };

  // The MFMA / softmax work of tile t, read from the 16-bit stage `cur`.
  auto compute = [&](int t, const uint8_t* cur) {
    const int kt = t * Geo::TILE_KEYS;
    const uint8_t* k_stage = cur;
    const uint8_t* v_stage = cur + Geo::TILE_BYTES;

#pragma unroll
    for (int sub = 0; sub < Geo::TILE_KEYS / kSubKeys; ++sub) {
      const int rb = sub * kSubKeys;  // tile-relative first key of this step
      const int key0 = kt + rb;

      // S^T for the 32 keys x (32 * QB) queries of this wave.  All K
      // fragments of the step are requested before the first MFMA so the
      // LDS latency is paid once.
      f32x16 s[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[qb] = f32x16{};
      constexpr int KB = Geo::KB;
#pragma unroll
      for (int c0 = 0; c0 < QC; c0 += KB) {
        u32x4 kf[KB];
#pragma unroll
        for (int c = 0; c < KB; ++c)
          kf[c] = *reinterpret_cast<const u32x4*>(k_stage + Geo::offset(rb + lr, 2 * (c0 + c) + hf));
#pragma unroll
        for (int c = 0; c < KB; ++c) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) s[qb] = Op::mma(kf[c], qf[qb][c0 + c], s[qb]);
        }
      }

      bool need_mask = key0 + kSubKeys > p.kv_tokens;
      if (CAUSAL)
        need_mask = need_mask || (p.kv_local_offset + key0 + kSubKeys - 1 >
                                  p.q_local_offset + qw0 + p.causal_shift);
      if (need_mask) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = key0 + c_row(i, hf);
            bool ok = key < p.kv_tokens;
            if (CAUSAL) ok = ok && (p.kv_local_offset + key <= p.q_local_offset + qi[qb] + p.causal_shift);
            s[qb][i] = ok ? s[qb][i] : -INFINITY;
          }
        }
      }

      // P^T (B operands of PV) and this lane's partial row sums, first against
      // the kept maximum m: p = exp2(s * scale - m).  The pairwise sum order
      // is fixed, so a row's sum does not depend on which path computed it.
      auto exps = [&](int qb, float neg_m, u32x4 (&pq)[2]) -> float {
        float sum = 0.f;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[qb][8 * kc + 2 * e], cf, neg_m));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[qb][8 * kc + 2 * e + 1], cf, neg_m));
            sum = (kc == 0 && e == 0) ? p0 + p1 : sum + (p0 + p1);
            pq[kc][e] = Op::pack2(p0, p1);
          }
        }
        return sum;
      };
      u32x4 pf[QB][2];
      float psum[QB];
      bool grow = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        psum[qb] = exps(qb, m_run[qb] == -INFINITY ? 0.f : -m_run[qb], pf[qb]);
        // Every p <= 2^8 (no logit above m + 8) whenever the lane's sum is;
        // a row without a maximum yet always takes the rescale path.
        grow = grow || !(psum[qb] <= 256.f) || m_run[qb] == -INFINITY;
      }
      // Rescale only when some logit of the wave may have left the [.., m + 8]
      // window.  The rule is that of the half-row maxima: m moves to the
      // query's full maximum when that exceeds m + 8.  Each query decides
      // for itself (both lane halves of a query see the same decision), so a
      // query's result never depends on which other queries share its
      // wavefront; where m stays, the values computed above stand.
      if (__ballot(grow) != 0) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          float a = fmaxf(fmaxf(s[qb][0], s[qb][1]), s[qb][2]);
#pragma unroll
          for (int i = 3; i < 15; i += 2) a = fmaxf(fmaxf(a, s[qb][i]), s[qb][i + 1]);
          a = fmaxf(a, s[qb][15]) * cf;
          const float full = fmaxf(a, __shfl_xor(a, 32));
          const float m_new = full > m_run[qb] + kRescaleThreshold ? full : m_run[qb];
          if (m_new != m_run[qb]) {
            const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
            l_part[qb] *= alpha;
#pragma unroll
            for (int d = 0; d < DB; ++d) acc[qb][d] *= alpha;
            m_run[qb] = m_new;
            psum[qb] = exps(qb, -m_new, pf[qb]);
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) l_part[qb] += psum[qb];

      // O^T += V^T P^T; each V^T fragment (two transposing LDS reads) feeds QB
      // MFMAs.  The reads of a batch of up to 4 d-blocks are all issued before
      // the batch's MFMAs.  They are inline asm followed by one explicit
      // lgkmcnt wait: the compiler cannot relate a transposing LDS read to the
      // DMA writing the other stage and would otherwise wait for that prefetch
      // (vmcnt) before every read.  LDS reads complete in order, so the
      // compiler's own lgkmcnt waits around these remain sufficient.
      const int grp = lane >> 4;
      const int gi = lane & 15;
      const uint32_t v_lds = (uint32_t)(uintptr_t)(const SA_LDS uint8_t*)(v_stage);
      constexpr int VB = Geo::VB;
#pragma unroll
      for (int d0 = 0; d0 < DB; d0 += VB) {
        u32x4 vf[VB][2];
#pragma unroll
        for (int dd = 0; dd < VB; ++dd) {
          const int granule = 4 * (d0 + dd) + 2 * (grp & 1) + ((gi & 3) >> 1);
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int row = rb + 16 * kc + 8 * r + 4 * (grp >> 1) + (gi >> 2);
              const uint32_t addr = v_lds + Geo::offset(row, granule) + 8 * (gi & 1);
              u32x2 w;
              asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(w) : "v"(addr));
              vf[dd][kc][2 * r] = w[0];
              vf[dd][kc][2 * r + 1] = w[1];
            }
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int dd = 0; dd < VB; ++dd) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) asm volatile("" : "+v"(vf[dd][kc]));
        }
#pragma unroll
        for (int dd = 0; dd < VB; ++dd) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
              acc[qb][d0 + dd] = Op::mma(vf[dd][kc], pf[qb][kc], acc[qb][d0 + dd]);
          }
        }
      }
    }
  };

  if constexpr (!QUANT) {
    // Tile t is computed from `cur` while tile t+1 streams into `next`.
    int until_merge = p.merge_tiles;  // tiles left in the current K/V chunk
    auto tile = [&](int t, const uint8_t* cur, uint8_t* next) {
      // Every wave waits for its own DMA of tile t before the barrier, so
      // after it all 64 rows of `cur` are in LDS.  LDS DMA is counted by
      // vmcnt, which a workgroup-scope fence does not wait for: without this
      // explicit wait a wave could read rows that another wave's DMA has not
      // written yet.  The barrier also guarantees `next` (tile t-1) is no
      // longer being read.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (t + 1 < ntiles) issue_tile((t + 1) * Geo::TILE_KEYS, next);
      compute(t, cur);
      if (p.merge_tiles > 0 && --until_merge == 0) {
        until_merge = p.merge_tiles;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float full = l_part[qb] + __shfl_xor(l_part[qb], 32);
          l_part[qb] = hf == 0 ? full : 0.f;
        }
      }
    };
    if (ntiles > 0) issue_tile(0, lds_a);
    for (int t = 0; t < ntiles; t += 2) {
      tile(t, lds_a, lds_b);
      if (t + 1 < ntiles) tile(t + 1, lds_b, lds_a);
    }
  } else {
    // Raw int8 tile [kt, kt + 64) of K and V into staging `stg` (K at 0, V at
    // I8_TILE_BYTES), row-major with 16-byte granules; the same tail and
    // head_dim clamps as the 16-bit path keep every address in the buffers.
    const uint8_t* kp8 = reinterpret_cast<const uint8_t*>(p.k) + (int64_t)kv_head * p.sk_h;
    const uint8_t* vp8 = reinterpret_cast<const uint8_t*>(p.v) + (int64_t)kv_head * p.sv_h;
    int k8_off[Geo::I8_DMA_PER_WAVE], v8_off[Geo::I8_DMA_PER_WAVE], row8[Geo::I8_DMA_PER_WAVE];
#pragma unroll
    for (int i = 0; i < Geo::I8_DMA_PER_WAVE; ++i) {
      const int chunk = wave + Geo::WAVES * i;
      const int row = chunk * (1024 / DP) + lane / Geo::I8_GR;
      const int gr = lane % Geo::I8_GR;
      const int col = gr * 16 < p.head_dim ? gr * 16 : 0;
      row8[i] = row;
      k8_off[i] = row * (int)p.sk_t + col;
      v8_off[i] = row * (int)p.sv_t + col;
    }
    auto issue_i8 = [&](int kt, uint8_t* stg) {
      const uint8_t* kt_base = kp8 + (int64_t)kt * p.sk_t;
      const uint8_t* vt_base = vp8 + (int64_t)kt * p.sv_t;
#pragma unroll
      for (int i = 0; i < Geo::I8_DMA_PER_WAVE; ++i) {
        const int chunk = wave + Geo::WAVES * i;
        if (Geo::I8_DMAS % Geo::WAVES != 0 && chunk >= Geo::I8_DMAS) break;
        int ko = k8_off[i], vo = v8_off[i];
        if (kt + row8[i] >= p.kv_tokens) {
          const int back = kt + row8[i] - (p.kv_tokens - 1);
          ko -= back * (int)p.sk_t;
          vo -= back * (int)p.sv_t;
        }
        __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(kt_base + ko),
                                         (SA_LDS void*)(stg + chunk * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(vt_base + vo),
                                         (SA_LDS void*)(stg + Geo::I8_TILE_BYTES + chunk * 1024), 16, 0, 0);
      }
    };
    // This thread's dequantization granules: g = tid + THREADS * j, row g / I8_GR.
    // Their scales (raw fp16 bits) are loaded one tile ahead into registers.
    uint32_t ksc[Geo::I8_PER_THREAD], vsc[Geo::I8_PER_THREAD];
    const uint16_t* ksp = p.ks + (int64_t)kv_head * p.sks_h;
    const uint16_t* vsp = p.vs + (int64_t)kv_head * p.svs_h;
    auto load_scales = [&](int kt) {
#pragma unroll
      for (int j = 0; j < Geo::I8_PER_THREAD; ++j) {
        const int g = tid + Geo::THREADS * j;
        const int key = min(kt + min(g, Geo::I8_GRANULES - 1) / Geo::I8_GR, p.kv_tokens - 1);
        const int64_t group = (int64_t)((p.scale_offset + key) >> p.scale_shift);
        ksc[j] = ksp[group * p.sks_g];
        vsc[j] = vsp[group * p.svs_g];
      }
    };
    // dtype(fp32(k) * fp32(scale)) into the swizzled 16-bit stage.  A signed
    // byte b is (b ^ 0x80) - 128; fma(u, s, -128 s) rounds (u - 128) * s once,
    // the same value as the reference's fp32 product.
    auto dequant = [&](const uint8_t* stg, uint8_t* stage) {
#pragma unroll
      for (int j = 0; j < Geo::I8_PER_THREAD; ++j) {
        const int g = tid + Geo::THREADS * j;
        if (Geo::I8_GRANULES % Geo::THREADS != 0 && g >= Geo::I8_GRANULES) break;
        const int row = g / Geo::I8_GR;
        const int gr = g % Geo::I8_GR;
#pragma unroll
        for (int tensor = 0; tensor < 2; ++tensor) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(stg + tensor * Geo::I8_TILE_BYTES + row * DP + gr * 16);
          const uint16_t bits = (uint16_t)(tensor == 0 ? ksc[j] : vsc[j]);
          const float sc = (float)__builtin_bit_cast(_Float16, bits);
          const float nb = -128.f * sc;
          u32x4 out[2];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t x = raw[w] ^ 0x80808080u;
            const float f0 = fmaf((float)(x & 0xffu), sc, nb);
            const float f1 = fmaf((float)((x >> 8) & 0xffu), sc, nb);
            const float f2 = fmaf((float)((x >> 16) & 0xffu), sc, nb);
            const float f3 = fmaf((float)(x >> 24), sc, nb);
            out[w >> 1][2 * (w & 1)] = Op::pack2(f0, f1);
            out[w >> 1][2 * (w & 1) + 1] = Op::pack2(f2, f3);
          }
          uint8_t* dst = stage + tensor * Geo::TILE_BYTES;
          *reinterpret_cast<u32x4*>(dst + Geo::offset(row, 2 * gr)) = out[0];
          *reinterpret_cast<u32x4*>(dst + Geo::offset(row, 2 * gr + 1)) = out[1];
        }
      }
    };
    // At tile t: `cur` holds tile t (dequantized before the barrier), staging
    // `stg_next` holds raw tile t+1 and `stg_cur` (raw tile t) and `next`
    // (read by tile t-1's MFMAs) are free.  The vmcnt wait covers this wave's
    // DMA and scale loads; the barrier makes every wave's DMA and
    // dequantization writes visible.
    auto tile_q = [&](int t, const uint8_t* cur, uint8_t* next, uint8_t* stg_cur, const uint8_t* stg_next) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (t + 2 < ntiles) issue_i8((t + 2) * Geo::TILE_KEYS, stg_cur);
      if (t + 1 < ntiles) {
        dequant(stg_next, next);
        if (t + 2 < ntiles) load_scales((t + 2) * Geo::TILE_KEYS);
      }
      compute(t, cur);
    };
    if (ntiles > 0) {
      issue_i8(0, lds_qa);
      load_scales(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      dequant(lds_qa, lds_a);
      if (ntiles > 1) {
        issue_i8(Geo::TILE_KEYS, lds_qb);
        load_scales(Geo::TILE_KEYS);
      }
    }
    for (int t = 0; t < ntiles; t += 2) {
      tile_q(t, lds_a, lds_b, lds_qa, lds_qb);
      if (t + 1 < ntiles) tile_q(t + 1, lds_b, lds_a, lds_qb, lds_qa);
    }
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l_full = l_part[qb] + __shfl_xor(l_part[qb], 32);
    if (qi[qb] >= p.q_tokens) continue;
    if (p.out != nullptr) {
      uint16_t* orow = p.out + (int64_t)qi[qb] * p.so_t + (int64_t)head * p.so_h;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = 32 * d + 8 * g + 4 * hf;
          if (col < p.head_dim) {
            const f32x16& a = acc[qb][d];
            u32x2 o = {0, 0};
            if (l_full > 0.f) {
              o[0] = Op::pack2(a[4 * g + 0] / l_full, a[4 * g + 1] / l_full);
              o[1] = Op::pack2(a[4 * g + 2] / l_full, a[4 * g + 3] / l_full);
            }
            *reinterpret_cast<u32x2*>(orow + col) = o;
          }
        }
      }
      if (p.lse != nullptr && hf == 0)
        p.lse[(int64_t)head * p.lse_sh + p.lse_off + qi[qb]] =
            l_full > 0.f ? (m_run[qb] + log2f(l_full)) * 0.69314718055994530942f : -INFINITY;
      continue;
    }
    const int64_t blk = state_block(qi[qb], head, p.q_heads);
    const int r = qi[qb] & 15;
    const int64_t srow = p.tiled_state ? blk * 16 + r : (int64_t)qi[qb] * p.ss_t + (int64_t)head * p.ss_h;
    if (hf == 0) {
      p.m[srow] = m_run[qb];
      p.l[srow] = l_full;
    }
    float* arow = p.tiled_state ? p.acc + blk * 16 * p.head_dim + 4 * r
                                : p.acc + (int64_t)qi[qb] * p.sa_t + (int64_t)head * p.sa_h;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = 32 * d + 8 * g + 4 * hf;
        if (col < p.head_dim) {
          const f32x4 v4 = {acc[qb][d][4 * g + 0], acc[qb][d][4 * g + 1], acc[qb][d][4 * g + 2],
                            acc[qb][d][4 * g + 3]};
          *reinterpret_cast<f32x4*>(arow + (p.tiled_state ? 16 * col : col)) = v4;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// head_dim 72..128: 16x16x32 MFMAs, 48 queries per wavefront.
//
// Eight wavefronts (two per SIMD) own three 16-query blocks each, 384 queries
// per workgroup.  Each K fragment and each V^T fragment read from LDS feeds
// three MFMAs, so a 64-key tile costs two thirds of the LDS bytes per FLOP of
// a 32-query wave, and the tile DMA feeds 384 queries instead of 256.  The
// registers still fit two waves per SIMD: Q 48, O^T 96, S^T 24, P^T 12.
//
// v_mfma_f32_16x16x32_{bf16,f16}: A 16x32 (lane l: row l % 16, k 8 (l / 16)
// .. +7), B 32x16 (lane l: column l % 16, k 8 (l / 16) .. +7), C 16x16 (lane
// l: column l % 16, rows 4 (l / 16) .. +3).  With j = l / 16:
//   S^T[key][query] = K . Q^T: A = K rows (LDS), B = Q (registers for the
//   whole kernel).  The lane holds query l % 16 of each block and keys
//   4j .. 4j + 3 of each 16-key block of the 32-key step.
//   O^T[d][query] += V^T . P^T: B = P^T straight from those registers, k slot
//   8j + e holding key 4j + e (e < 4) or 16 + 4j + e - 4; A = V^T rows in
//   the same slot order, from two transposing LDS reads per fragment (or one
//   16-byte read of the transposed copy of V).
// A query's 32 keys of a step are spread over four lanes (j = 0..3); its
// partial row sums stay per lane and are added in the fixed order
// (l0 + l1) + (l2 + l3) wherever l is stored or merged.  The rescale rule
// is the 32-query kernel's, decided per query from all four of its lanes.
// In the row-group state layout the 64 lanes' chunks of one d block are 1 KB
// of contiguous memory.
struct Geometry48 {
  static constexpr int DP = 128;
  static constexpr int WAVES = 8;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QB = 3;                                 // 16-query blocks per wave
  static constexpr int BLOCK_M = WAVES * 16 * QB;              // 384
  static constexpr int TILE_KEYS = 64;
  static constexpr int TILE_BYTES = TILE_KEYS * DP * 2;        // K (or V) part of a stage
  static constexpr int DMA_PER_WAVE = TILE_BYTES / 1024 / WAVES;
  static constexpr int I8_TILE_BYTES = TILE_KEYS * DP;
  static constexpr int I8_GR = DP / 16;
  static constexpr int I8_DMAS = I8_TILE_BYTES / 1024;
  static constexpr int I8_DMA_PER_WAVE = (I8_DMAS + WAVES - 1) / WAVES;
  static constexpr int I8_GRANULES = TILE_KEYS * I8_GR;
  static constexpr int I8_PER_THREAD = (I8_GRANULES + THREADS - 1) / THREADS;
  static_assert(DMA_PER_WAVE >= 1 && I8_DMAS % WAVES == 0 && I8_GRANULES % THREADS == 0, "tile geometry");
  // LDS layouts of one stage.  Every fragment read is a per-lane base plus a
  // compile-time offset (the instruction's immediate), and every read is free
  // of bank conflicts (measured with SQ_LDS_BANK_CONFLICT).
  //   K: in fragment order.  The 16-key x 32-d A fragment (16-key block kb,
  //   d block c) is 1 KB at (4 kb + c) KB, lane (j, r16)'s 16 bytes (key
  //   16 kb + r16, d 32 c + 8 j .. +7) at 16 * lane: each read is 1 KB of
  //   consecutive bytes.
  //   V: eight blocks of 16 d (64 keys x 32 bytes each).  A transposing read
  //   has each 16-lane group take 4 consecutive keys (128 bytes) of a block:
  //   512 consecutive bytes per read.
  //   V^T (transposed copy): in fragment order, the 16-d x 32-key fragment
  //   (32-key block sb, d block db) at (8 sb + db) KB, lane (j, r16)'s 16
  //   bytes (row 16 db + r16, key granule 4 sb + j) at 16 * lane.
  __device__ static inline int k_offset(int key, int g) {
    return ((key >> 4) * 4 + (g >> 2)) * 1024 + 16 * (((g & 3) << 4) | (key & 15));
  }
  __device__ static inline int v_offset(int key, int g) { return (g >> 1) * 2048 + key * 32 + ((g & 1) << 4); }
};

template <typename Op>
__device__ inline f32x4 mma16(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ inline f32x4 mma16<BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
template <>
__device__ inline f32x4 mma16<FP16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// VT: V transposed per K/V head, [128 rows][keys], each 32-key group in the
// k-slot order above (slot s holds key 16 ((s >> 2) & 1) + 4 (s >> 3) +
// (s & 3)), zero keys up to a multiple of 64.
template <typename Op, bool CAUSAL, bool INIT, bool QUANT, bool VT>
__global__ __launch_bounds__(Geometry48::THREADS) void update48_kernel(const UpdateParams p) {
  using Geo = Geometry48;
  static_assert(!(VT && QUANT), "transposed V is read by the 16-bit kernel only");
  constexpr int QB = Geo::QB;

  __shared__ __attribute__((aligned(1024))) uint8_t lds_a[2 * Geo::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b[2 * Geo::TILE_BYTES];
  constexpr int kStagingBytes = QUANT ? 2 * Geo::I8_TILE_BYTES : 16;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_qa[kStagingBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_qb[kStagingBytes];

  // Workgroup numbering as in the 32-query kernel.
  const int b = blockIdx.x;
  const int logical = (CAUSAL && p.deal_blocks) ? b : (b & 7) * p.xcd_run + (b >> 3);
  if (logical >= p.q_blocks * p.q_heads) return;
  const int head = logical / p.q_blocks;
  const int qb_index = CAUSAL ? p.q_blocks - 1 - (logical - head * p.q_blocks) : logical - head * p.q_blocks;
  const int q_block = qb_index * Geo::BLOCK_M;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r16 = lane & 15;  // query within a 16-query block; key / d row within a 16-row fragment
  const int j = lane >> 4;    // k-slot group
  const int kv_head = head / p.group;
  const int qw0 = q_block + wave * 16 * QB;

  const uint16_t* qp = p.q + (int64_t)head * p.sq_h;
  const uint16_t* kp = p.k + (int64_t)kv_head * p.sk_h;
  const uint16_t* vp = p.v + (int64_t)kv_head * p.sv_h;

  int kv_end = p.kv_tokens;
  if (CAUSAL) {
    const int q_last = min(p.q_tokens, q_block + Geo::BLOCK_M) - 1;
    const int lim = p.q_local_offset + q_last + p.causal_shift - p.kv_local_offset + 1;
    kv_end = max(0, min(kv_end, lim));
  }
  const int ntiles = (kv_end + Geo::TILE_KEYS - 1) / Geo::TILE_KEYS;
  const float cf = scale_factor(p.scale_log2);

  // HBM/L2 -> LDS DMA of key tile [kt, kt + 64), issued by waves 0-3 (the
  // first wave of each SIMD) only.  The second waves of the SIMDs get the
  // smaller share of issue slots while both compute, so they finish a tile
  // last; the first waves wait at the tile barrier meanwhile, and issuing
  // the DMA there takes it off the tile's critical path.
  // A wave-wide DMA writes 1 KB of LDS linearly (16 bytes per lane); piece f
  // (0..15) of a tensor is LDS bytes [f KB, f KB + 1 KB), and each lane loads
  // the global granule the layouts above place at its slot.  The global
  // element offset is a wave-uniform part (f) plus a per-lane part (lane):
  //   K (fragment 4 kb + c = f): key 16 (f / 4) + lane % 16, d 32 (f % 4) + 8 (lane / 16);
  //   V: key (32 f) % 64 + lane / 2, d 16 (f / 2) + 8 (lane % 2);
  //   V^T (fragment 8 sb + db = f): row 16 (f % 8) + lane % 16,
  //   key 32 (f / 8) + 8 (lane / 16).
  // In the tail tile, keys past the chunk read its last key, and V^T keys
  // past the row's padded length read the row's first granule; granules
  // past head_dim read d = 0.  Those values are finite and masked (keys) or
  // multiplied by zero Q / never stored (d), and every address stays inside
  // the caller's buffers.
  constexpr int kPieces = Geo::TILE_BYTES / 1024;   // per tensor per tile
  constexpr int kIssuers = 4;
  const int k_dma_lane = (lane & 15) * (int)p.sk_t + 8 * (lane >> 4);
  const int v_dma_lane = VT ? (lane & 15) * (int)p.sv_t + 8 * (lane >> 4) : (lane >> 1) * (int)p.sv_t + 8 * (lane & 1);
  auto issue_tile = [&](int kt, uint8_t* stage) {
    if (wave >= kIssuers) return;
    uint8_t* k_stage = stage;
    uint8_t* v_stage = stage + Geo::TILE_BYTES;
    const bool tail = kt + Geo::TILE_KEYS > p.kv_tokens;
    const bool narrow = p.head_dim < 128;
#pragma unroll
    for (int i = 0; i < kPieces / kIssuers; ++i) {
      const int f = wave * (kPieces / kIssuers) + i;
      const int k_key0 = 16 * (f >> 2);
      const int k_d0 = 32 * (f & 3);
      int ko = k_dma_lane;
      if (narrow && k_d0 + 8 * (lane >> 4) >= p.head_dim) ko -= k_d0 + 8 * (lane >> 4);
      if (tail) {
        const int key = kt + k_key0 + (lane & 15);
        if (key >= p.kv_tokens) ko -= (key - (p.kv_tokens - 1)) * (int)p.sk_t;
      }
      __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(kp + (int64_t)(kt + k_key0) * p.sk_t + k_d0 + ko),
                                       (SA_LDS void*)(k_stage + f * 1024), 16, 0, 0);
      const uint16_t* vb;
      int vo = v_dma_lane;
      if constexpr (VT) {
        const int row0 = 16 * (f & 7), key0 = 32 * (f >> 3);
        vb = vp + (int64_t)row0 * p.sv_t + kt + key0;
        if (tail && kt + key0 + 8 * (lane >> 4) >= p.sv_t) vo -= kt + key0 + 8 * (lane >> 4);
      } else {
        const int v_key0 = (32 * f) & (Geo::TILE_KEYS - 1);
        const int v_d0 = 16 * ((32 * f) / Geo::TILE_KEYS);
        vb = vp + (int64_t)(kt + v_key0) * p.sv_t + v_d0;
        if (narrow && v_d0 + 8 * (lane & 1) >= p.head_dim) vo -= v_d0 + 8 * (lane & 1);
        if (tail) {
          const int key = kt + v_key0 + (lane >> 1);
          if (key >= p.kv_tokens) vo -= (key - (p.kv_tokens - 1)) * (int)p.sv_t;
        }
      }
      __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(vb + vo), (SA_LDS void*)(v_stage + f * 1024), 16, 0, 0);
    }
  };

  // The first tile's DMA is issued before the Q and state loads, so that it
  // is in flight while they arrive (the 16-bit path; the INT8 path stages
  // its own first tile).
  if constexpr (!QUANT) {
    if (ntiles > 0) issue_tile(0, lds_a);
  }

  // Q fragments: query qw0 + 16 qb + r16, d = 32 c + 8 j .. +7.
  u32x4 qf[QB][4];
  int qi[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qi[qb] = qw0 + 16 * qb + r16;
    const bool ok = qi[qb] < p.q_tokens;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = 32 * c + 8 * j;
      if (ok && d < p.head_dim)
        qf[qb][c] = *reinterpret_cast<const u32x4*>(qp + (int64_t)qi[qb] * p.sq_t + d) ^ q_sign(p.scale_log2);
      else
        qf[qb][c] = u32x4{0, 0, 0, 0};
    }
  }

  // Online-softmax state; acc[db][qb] holds d = 16 db + 4 j .. +3 of query qi[qb].
  float m_run[QB], l_part[QB];
  f32x4 acc[8][QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_part[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!INIT && qi[qb] < p.q_tokens) {
      const int64_t blk = state_block(qi[qb], head, p.q_heads);
      const int64_t srow = p.tiled_state ? blk * 16 + r16 : (int64_t)qi[qb] * p.ss_t + (int64_t)head * p.ss_h;
      m_run[qb] = p.m[srow];
      l_part[qb] = j == 0 ? p.l[srow] : 0.f;
      const float* arow = p.tiled_state ? p.acc + blk * 16 * p.head_dim + 4 * lane
                                        : p.acc + (int64_t)qi[qb] * p.sa_t + (int64_t)head * p.sa_h + 4 * j;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        if (16 * db + 4 * j < p.head_dim)
          acc[db][qb] = *reinterpret_cast<const f32x4*>(arow + (p.tiled_state ? 256 * db : 16 * db));
      }
    }
  }

  // Per-lane parts of the fragment addresses: 16 bytes per lane for the K and
  // V^T fragments, 8 bytes per lane for the transposing V reads.
  const int k_lane = 16 * lane;
  const int v_lane = VT ? 16 * lane : 8 * lane;

  auto compute = [&](int t, const uint8_t* cur) {
    const int kt = t * Geo::TILE_KEYS;
    const uint8_t* k_stage = cur;
    const uint8_t* v_stage = cur + Geo::TILE_BYTES;
#pragma unroll
    for (int sub = 0; sub < Geo::TILE_KEYS / kSubKeys; ++sub) {
      const int rb = sub * kSubKeys;
      const int key0 = kt + rb;

      // S^T: two 16-key blocks x three 16-query blocks, four 32-wide d steps.
      f32x4 s[2][QB];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      {
        // All eight K fragments of the step are read before one wait (the
        // compiler's own schedule waited three times per step, with the
        // second wave of the SIMD usually waiting at the same moment).
        const uint32_t k_addr = (uint32_t)(uintptr_t)(const SA_LDS uint8_t*)(k_stage) + k_lane;
        u32x4 kf[8];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            u32x4 w;
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(w) : "v"(k_addr), "i"(((rb / 16 + kb) * 4 + c) * 1024));
            kf[kb * 4 + c] = w;
          }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int x = 0; x < 8; ++x) asm volatile("" : "+v"(kf[x]));
        // Query blocks in snake order: consecutive MFMAs change only one of
        // their A and B operands except where c changes.  An MFMA whose A
        // and B both differ from the previous one's issues later (measured:
        // up to 1.5x the MFMA's cycles).
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < QB; ++i) {
              const int qb = kb == 0 ? i : QB - 1 - i;
              s[kb][qb] = mma16<Op>(kf[kb * 4 + c], qf[qb][c], s[kb][qb]);
            }
      }

      bool need_mask = key0 + kSubKeys > p.kv_tokens;
      if (CAUSAL)
        need_mask = need_mask || (p.kv_local_offset + key0 + kSubKeys - 1 >
                                  p.q_local_offset + qw0 + p.causal_shift);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = key0 + 16 * kb + 4 * j + i;
              bool ok = key < p.kv_tokens;
              if (CAUSAL) ok = ok && (p.kv_local_offset + key <= p.q_local_offset + qi[qb] + p.causal_shift);
              s[kb][qb][i] = ok ? s[kb][qb][i] : -INFINITY;
            }
      }

      // P^T against the kept maximum, and the lane's partial row sum (8 keys).
      auto exps = [&](int qb, float neg_m, u32x4& pq) -> float {
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kb][qb][2 * e], cf, neg_m));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kb][qb][2 * e + 1], cf, neg_m));
            sum = (kb == 0 && e == 0) ? p0 + p1 : sum + (p0 + p1);
            pq[2 * kb + e] = Op::pack2(p0, p1);
          }
        }
        return sum;
      };
      u32x4 pf[QB];
      float psum[QB];
      bool grow[QB];
      bool any = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        psum[qb] = exps(qb, m_run[qb] == -INFINITY ? 0.f : -m_run[qb], pf[qb]);
        // Every p <= 2^8 (no logit above m + 8) whenever the lane's sum is;
        // a row without a maximum yet always takes the rescale path.
        grow[qb] = !(psum[qb] <= 256.f) || m_run[qb] == -INFINITY;
        any = any || grow[qb];
      }
      if (__ballot(any) != 0) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          // The query's own decision: one of its four lanes saw a partial sum
          // above 2^8 (some logit may exceed m + 8) or it has no maximum yet.
          const uint64_t bal = __ballot(grow[qb]);
          uint32_t fold = (uint32_t)bal | (uint32_t)(bal >> 32);
          fold |= fold >> 16;
          const bool mine = (fold >> r16) & 1u;
          float a = fmaxf(fmaxf(s[0][qb][0], s[0][qb][1]), fmaxf(s[0][qb][2], s[0][qb][3]));
          a = fmaxf(a, fmaxf(fmaxf(s[1][qb][0], s[1][qb][1]), fmaxf(s[1][qb][2], s[1][qb][3]))) * cf;
          float full = fmaxf(a, __shfl_xor(a, 16));
          full = fmaxf(full, __shfl_xor(full, 32));
          const float m_new = (mine && full > m_run[qb] + kRescaleThreshold) ? full : m_run[qb];
          if (m_new != m_run[qb]) {
            const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
            l_part[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < 8; ++db) acc[db][qb] *= alpha;
            m_run[qb] = m_new;
            psum[qb] = exps(qb, -m_new, pf[qb]);
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) l_part[qb] += psum[qb];

      // O^T += V^T P^T, two d blocks per batch of LDS reads.  The reads are
      // inline asm with one explicit lgkmcnt wait, as in the 32-query kernel.
      const uint32_t v_addr = (uint32_t)(uintptr_t)(const SA_LDS uint8_t*)(v_stage) + v_lane;
#pragma unroll
      for (int d0 = 0; d0 < 8; d0 += 2) {
        u32x4 vf[2];
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          const int db = d0 + dd;
          if constexpr (VT) {
            // Rows d = 16 db + r16, key granule j of the step's 32-key block.
            u32x4 w;
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(w) : "v"(v_addr), "i"(((rb / 32) * 8 + db) * 1024));
            vf[dd] = w;
          } else {
            // Lane (j, r16) addresses key 4 j + r16 / 4 of each 16-key block
            // at d = 16 db + 4 (r16 % 4) .. +3; after the transpose it holds
            // d = 16 db + r16 for keys 4 j .. 4 j + 3.
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
              u32x2 w;
              asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                           : "=v"(w) : "v"(v_addr), "i"(db * 2048 + (rb + 16 * kb) * 32));
              vf[dd][2 * kb] = w[0];
              vf[dd][2 * kb + 1] = w[1];
            }
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) asm volatile("" : "+v"(vf[dd]));
#pragma unroll
        for (int dd = 0; dd < 2; ++dd)
#pragma unroll
          for (int i = 0; i < QB; ++i) {
            const int qb = dd == 0 ? i : QB - 1 - i;  // snake order, as in QK^T
            acc[d0 + dd][qb] = mma16<Op>(vf[dd], pf[qb], acc[d0 + dd][qb]);
          }
      }
    }
  };

  // Sum of a query's four partial row sums, identical on all four lanes.
  auto full_l = [&](float x) -> float {
    const float h = x + __shfl_xor(x, 16);
    return h + __shfl_xor(h, 32);
  };

  if constexpr (!QUANT) {
    int until_merge = p.merge_tiles;
    auto tile = [&](int t, const uint8_t* cur, uint8_t* next) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (t + 1 < ntiles) issue_tile((t + 1) * Geo::TILE_KEYS, next);
      compute(t, cur);
      if (p.merge_tiles > 0 && --until_merge == 0) {
        until_merge = p.merge_tiles;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float full = full_l(l_part[qb]);
          l_part[qb] = j == 0 ? full : 0.f;
        }
      }
    };
    for (int t = 0; t < ntiles; t += 2) {
      tile(t, lds_a, lds_b);
      if (t + 1 < ntiles) tile(t + 1, lds_b, lds_a);
    }
  } else {
    const uint8_t* kp8 = reinterpret_cast<const uint8_t*>(p.k) + (int64_t)kv_head * p.sk_h;
    const uint8_t* vp8 = reinterpret_cast<const uint8_t*>(p.v) + (int64_t)kv_head * p.sv_h;
    int k8_off[Geo::I8_DMA_PER_WAVE], v8_off[Geo::I8_DMA_PER_WAVE], row8[Geo::I8_DMA_PER_WAVE];
#pragma unroll
    for (int i = 0; i < Geo::I8_DMA_PER_WAVE; ++i) {
      const int chunk = wave + Geo::WAVES * i;
      const int row = chunk * (1024 / Geo::DP) + lane / Geo::I8_GR;
      const int gr = lane % Geo::I8_GR;
      const int col = gr * 16 < p.head_dim ? gr * 16 : 0;
      row8[i] = row;
      k8_off[i] = row * (int)p.sk_t + col;
      v8_off[i] = row * (int)p.sv_t + col;
    }
    auto issue_i8 = [&](int kt, uint8_t* stg) {
      const uint8_t* kt_base = kp8 + (int64_t)kt * p.sk_t;
      const uint8_t* vt_base = vp8 + (int64_t)kt * p.sv_t;
#pragma unroll
      for (int i = 0; i < Geo::I8_DMA_PER_WAVE; ++i) {
        const int chunk = wave + Geo::WAVES * i;
        int ko = k8_off[i], vo = v8_off[i];
        if (kt + row8[i] >= p.kv_tokens) {
          const int back = kt + row8[i] - (p.kv_tokens - 1);
          ko -= back * (int)p.sk_t;
          vo -= back * (int)p.sv_t;
        }
        __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(kt_base + ko),
                                         (SA_LDS void*)(stg + chunk * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const SA_GLOBAL void*)(vt_base + vo),
                                         (SA_LDS void*)(stg + Geo::I8_TILE_BYTES + chunk * 1024), 16, 0, 0);
      }
    };
    uint32_t ksc[Geo::I8_PER_THREAD], vsc[Geo::I8_PER_THREAD];
    const uint16_t* ksp = p.ks + (int64_t)kv_head * p.sks_h;
    const uint16_t* vsp = p.vs + (int64_t)kv_head * p.svs_h;
    auto load_scales = [&](int kt) {
#pragma unroll
      for (int i = 0; i < Geo::I8_PER_THREAD; ++i) {
        const int g = tid + Geo::THREADS * i;
        const int key = min(kt + g / Geo::I8_GR, p.kv_tokens - 1);
        const int64_t group = (int64_t)((p.scale_offset + key) >> p.scale_shift);
        ksc[i] = ksp[group * p.sks_g];
        vsc[i] = vsp[group * p.svs_g];
      }
    };
    // dtype(fp32(k) * fp32(scale)) into the swizzled 16-bit stage, with the
    // 32-query kernel's arithmetic.
    auto dequant = [&](const uint8_t* stg, uint8_t* stage) {
#pragma unroll
      for (int i = 0; i < Geo::I8_PER_THREAD; ++i) {
        const int g = tid + Geo::THREADS * i;
        const int row = g / Geo::I8_GR;
        const int gr = g % Geo::I8_GR;
#pragma unroll
        for (int tensor = 0; tensor < 2; ++tensor) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(stg + tensor * Geo::I8_TILE_BYTES + row * Geo::DP + gr * 16);
          const uint16_t bits = (uint16_t)(tensor == 0 ? ksc[i] : vsc[i]);
          const float sc = (float)__builtin_bit_cast(_Float16, bits);
          const float nb = -128.f * sc;
          u32x4 out[2];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t x = raw[w] ^ 0x80808080u;
            const float f0 = fmaf((float)(x & 0xffu), sc, nb);
            const float f1 = fmaf((float)((x >> 8) & 0xffu), sc, nb);
            const float f2 = fmaf((float)((x >> 16) & 0xffu), sc, nb);
            const float f3 = fmaf((float)(x >> 24), sc, nb);
            out[w >> 1][2 * (w & 1)] = Op::pack2(f0, f1);
            out[w >> 1][2 * (w & 1) + 1] = Op::pack2(f2, f3);
          }
          if (tensor == 0) {
            *reinterpret_cast<u32x4*>(stage + Geo::k_offset(row, 2 * gr)) = out[0];
            *reinterpret_cast<u32x4*>(stage + Geo::k_offset(row, 2 * gr + 1)) = out[1];
          } else {
            *reinterpret_cast<u32x4*>(stage + Geo::TILE_BYTES + Geo::v_offset(row, 2 * gr)) = out[0];
            *reinterpret_cast<u32x4*>(stage + Geo::TILE_BYTES + Geo::v_offset(row, 2 * gr + 1)) = out[1];
          }
        }
      }
    };
    auto tile_q = [&](int t, const uint8_t* cur, uint8_t* next, uint8_t* stg_cur, const uint8_t* stg_next) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (t + 2 < ntiles) issue_i8((t + 2) * Geo::TILE_KEYS, stg_cur);
      if (t + 1 < ntiles) {
        dequant(stg_next, next);
        if (t + 2 < ntiles) load_scales((t + 2) * Geo::TILE_KEYS);
      }
      compute(t, cur);
    };
    if (ntiles > 0) {
      issue_i8(0, lds_qa);
      load_scales(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      dequant(lds_qa, lds_a);
      if (ntiles > 1) {
        issue_i8(Geo::TILE_KEYS, lds_qb);
        load_scales(Geo::TILE_KEYS);
      }
    }
    for (int t = 0; t < ntiles; t += 2) {
      tile_q(t, lds_a, lds_b, lds_qa, lds_qb);
      if (t + 1 < ntiles) tile_q(t + 1, lds_b, lds_a, lds_qb, lds_qa);
    }
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l_full = full_l(l_part[qb]);
    if (qi[qb] >= p.q_tokens) continue;
    if (p.out != nullptr) {
      uint16_t* orow = p.out + (int64_t)qi[qb] * p.so_t + (int64_t)head * p.so_h + 4 * j;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        if (16 * db + 4 * j < p.head_dim) {
          const f32x4& a = acc[db][qb];
          u32x2 o = {0, 0};
          if (l_full > 0.f) {
            o[0] = Op::pack2(a[0] / l_full, a[1] / l_full);
            o[1] = Op::pack2(a[2] / l_full, a[3] / l_full);
          }
          *reinterpret_cast<u32x2*>(orow + 16 * db) = o;
        }
      }
      if (p.lse != nullptr && j == 0)
        p.lse[(int64_t)head * p.lse_sh + p.lse_off + qi[qb]] =
            l_full > 0.f ? (m_run[qb] + log2f(l_full)) * 0.69314718055994530942f : -INFINITY;
      continue;
    }
    const int64_t blk = state_block(qi[qb], head, p.q_heads);
    const int64_t srow = p.tiled_state ? blk * 16 + r16 : (int64_t)qi[qb] * p.ss_t + (int64_t)head * p.ss_h;
    if (j == 0) {
      p.m[srow] = m_run[qb];
      p.l[srow] = l_full;
    }
    float* arow = p.tiled_state ? p.acc + blk * 16 * p.head_dim + 4 * lane
                                : p.acc + (int64_t)qi[qb] * p.sa_t + (int64_t)head * p.sa_h + 4 * j;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      if (16 * db + 4 * j < p.head_dim)
        *reinterpret_cast<f32x4*>(arow + (p.tiled_state ? 256 * db : 16 * db)) = acc[db][qb];
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
  int32_t q_tokens, q_heads, groups;  // groups = head_dim / 8
  int32_t tiled_state;  // state in the row-group layout (state_block)
};

// One workgroup per (16-row group, head): blockIdx.x is the row group and
// blockIdx.y the head, so no thread divides 64-bit indices.  Item i of the
// group covers row r = i % 16 and output granule g = i / 16 (d = 8g .. 8g +
// 7).  In the row-group layout a wave's 64 items read 2 KB of consecutive
// accumulator bytes (chunks 2g and 2g + 1 of 16 rows) and write 16 rows x 64
// bytes of output.
template <typename Op>
__global__ __launch_bounds__(256) void finalize_kernel(const FinalizeParams p) {
  const int h = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int64_t blk = state_block(row0, h, p.q_heads);
  const int items = 16 * p.groups;
  for (int i = threadIdx.x; i < items; i += 256) {
    const int r = i & 15;
    const int g = i >> 4;
    const int64_t t = row0 + r;
    if (t >= p.q_tokens) continue;
    const int64_t srow = p.tiled_state ? blk * 16 + r : t * p.ss_t + h * p.ss_h;
    const float l = p.l[srow];
    f32x4 a0, a1;
    if (p.tiled_state) {
      // Chunks 2g and 2g + 1 (d = 8g .. 8g + 7) of row r.
      const float* a = p.acc + blk * 16 * (p.groups * 8) + (2 * g * 16 + r) * 4;
      a0 = *reinterpret_cast<const f32x4*>(a);
      a1 = *reinterpret_cast<const f32x4*>(a + 16 * 4);
    } else {
      const float* a = p.acc + t * p.sa_t + h * p.sa_h + 8 * g;
      a0 = *reinterpret_cast<const f32x4*>(a);
      a1 = *reinterpret_cast<const f32x4*>(a + 4);
    }
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
      const float m = p.m[srow];
      p.lse[h * p.lse_sh + p.lse_off + t] = l > 0.f ? (m + log2f(l)) * 0.69314718055994530942f : -INFINITY;
    }
  }
}

// Transposed copy of V for the head_dim-128 update kernel's VT variant.  V is
// [kv_tokens, kv_heads, 128] with element strides (sv_t, sv_h); vt is
// [kv_heads][128][t_pad].  Within each 32-key group, slot s holds key
// 16 ((s >> 2) & 1) + 4 (s >> 3) + (s & 3): slots 8j .. 8j + 7 hold keys
// 4j .. 4j + 3 and 16 + 4j .. 16 + 4j + 3, the k-slot order in which that
// kernel's P^T operand holds the keys of a 16x16x32 MFMA, as laid out by the
// S^T accumulator rows.  Keys kv_tokens .. t_pad-1 are zero.  One workgroup
// per (kv_head, 64 keys), staged through LDS.
struct TransposeParams {
  const uint16_t* v;
  uint16_t* vt;
  int64_t sv_t, sv_h, t_pad;
  int32_t kv_tokens, tiles;
};

__global__ __launch_bounds__(256) void transpose_v_kernel(const TransposeParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][128 + 8];
  const int tid = threadIdx.x;
  const int head = blockIdx.x / p.tiles;
  const int kt = (blockIdx.x - head * p.tiles) * 64;
  {
    // Thread t reads key kt + t / 4, elements 32 (t % 4) .. +31.
    const int key = tid >> 2, d0 = (tid & 3) * 32;
    const bool ok = kt + key < p.kv_tokens;
    const uint16_t* src = p.v + (int64_t)(kt + key) * p.sv_t + (int64_t)head * p.sv_h + d0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 w = ok ? *reinterpret_cast<const u32x4*>(src + 8 * j) : u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&tile[key][d0 + 8 * j]) = w;
    }
  }
  __syncthreads();
  {
    // Thread t writes row d = t / 2, slots 32 (t % 2) .. +31.
    const int d = tid >> 1, s0 = (tid & 1) * 32;
    uint16_t* dst = p.vt + ((int64_t)head * 128 + d) * p.t_pad + kt + s0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sa = s0 + 8 * j + 2 * e, sb = sa + 1;
        const int ka = (sa & 32) | (16 * ((sa >> 2) & 1) + 4 * ((sa >> 3) & 3) + (sa & 3));
        const int kb = (sb & 32) | (16 * ((sb >> 2) & 1) + 4 * ((sb >> 3) & 3) + (sb & 3));
        w[e] = (uint32_t)tile[ka][d] | ((uint32_t)tile[kb][d] << 16);
      }
      *reinterpret_cast<u32x4*>(dst + 8 * j) = w;
    }
  }
}

template <typename Op, bool QUANT, bool VT>
hipError_t launch_update48(UpdateParams p, bool causal, bool init, hipStream_t s) {
  using Geo = Geometry48;
  p.q_blocks = (p.q_tokens + Geo::BLOCK_M - 1) / Geo::BLOCK_M;
  const int64_t total = (int64_t)p.q_blocks * p.q_heads;
  p.xcd_run = (int32_t)((total + 7) / 8);
  p.deal_blocks = causal && p.q_heads % 8 != 0;
  const dim3 grid((unsigned)(8 * (int64_t)p.xcd_run));
  const dim3 block(Geo::THREADS);
  if constexpr (VT) {
    // Transposed V serves launches that start the state (checked by the caller).
    if (causal)
      hipLaunchKernelGGL((update48_kernel<Op, true, true, false, true>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((update48_kernel<Op, false, true, false, true>), grid, block, 0, s, p);
    return hipGetLastError();
  }
  if (causal) {
    if (init)
      hipLaunchKernelGGL((update48_kernel<Op, true, true, QUANT, false>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((update48_kernel<Op, true, false, QUANT, false>), grid, block, 0, s, p);
  } else {
    if (init)
      hipLaunchKernelGGL((update48_kernel<Op, false, true, QUANT, false>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((update48_kernel<Op, false, false, QUANT, false>), grid, block, 0, s, p);
  }
  return hipGetLastError();
}

// The 32-query kernel for head_dim 32, 64 and 256; head_dim 128 uses the
// 48-query kernel.
template <typename Op, int DP, bool QUANT, bool VT = false>
hipError_t launch_update_dp(UpdateParams p, bool causal, bool init, hipStream_t s) {
  if constexpr (DP == 128) {
    return launch_update48<Op, QUANT, VT>(p, causal, init, s);
  } else {
    static_assert(!VT, "transposed V is read by the head_dim-128 kernel only");
    using Geo = Geometry<DP>;
    p.q_blocks = (p.q_tokens + Geo::BLOCK_M - 1) / Geo::BLOCK_M;
    const int64_t total = (int64_t)p.q_blocks * p.q_heads;
    p.xcd_run = (int32_t)((total + 7) / 8);
    p.deal_blocks = causal && p.q_heads % 8 != 0;
    const dim3 grid((unsigned)(8 * (int64_t)p.xcd_run));
    const dim3 block(Geo::THREADS);
    if (causal) {
      if (init)
        hipLaunchKernelGGL((update_kernel<Op, DP, true, true, QUANT>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((update_kernel<Op, DP, true, false, QUANT>), grid, block, 0, s, p);
    } else {
      if (init)
        hipLaunchKernelGGL((update_kernel<Op, DP, false, true, QUANT>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((update_kernel<Op, DP, false, false, QUANT>), grid, block, 0, s, p);
    }
    return hipGetLastError();
  }
}

template <typename Op>
hipError_t launch_update_op(const UpdateParams& p, int dp, bool causal, bool init, hipStream_t s) {
  switch (dp) {
    case 32: return launch_update_dp<Op, 32, false>(p, causal, init, s);
    case 64: return launch_update_dp<Op, 64, false>(p, causal, init, s);
    case 128: return launch_update_dp<Op, 128, false>(p, causal, init, s);
    default: return launch_update_dp<Op, 256, false>(p, causal, init, s);
  }
}

// INT8 K/V covers head_dim <= 128: with head_dim 256 the 16-bit stages and the
// raw staging would not fit in LDS together.
template <typename Op>
hipError_t launch_update_int8_op(const UpdateParams& p, int dp, bool causal, bool init, hipStream_t s) {
  switch (dp) {
    case 32: return launch_update_dp<Op, 32, true>(p, causal, init, s);
    case 64: return launch_update_dp<Op, 64, true>(p, causal, init, s);
    default: return launch_update_dp<Op, 128, true>(p, causal, init, s);
  }
}

inline bool aligned(const void* ptr, uintptr_t n) { return (reinterpret_cast<uintptr_t>(ptr) % n) == 0; }

}  // namespace

namespace sa {

int32_t update_block_rows(int32_t head_dim) {
  if (head_dim > 64 && head_dim <= 128) return Geometry48::BLOCK_M;
  return head_dim <= 64 ? Geometry<64>::BLOCK_M : Geometry<256>::BLOCK_M;
}

int32_t launch_update(const void* q, const void* k, const void* v, float* m, float* l, float* acc,
                      int64_t sq_t, int64_t sq_h, int64_t sk_t, int64_t sk_h, int64_t sv_t,
                      int64_t sv_h, int64_t ss_t, int64_t ss_h, int64_t sa_t, int64_t sa_h,
                      int32_t q_tokens, int32_t kv_tokens, int32_t q_heads, int32_t kv_heads,
                      int32_t head_dim, int32_t q_local_offset, int32_t kv_local_offset,
                      int32_t causal_shift, double softmax_scale, int32_t flags, int32_t dtype,
                      hipStream_t stream, int32_t merge_keys, const FusedOutput* fused,
                      bool v_transposed, bool tiled_state) {
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
  // A fused launch writes the output instead of the state; one that also
  // initializes the state does not touch m, l and acc, which may be null.
  const bool starts_state = (flags & SA_FLAG_INITIALIZE) != 0;
  if (!q || !k || !v || (!(fused != nullptr && starts_state) && (!m || !l || !acc))) {
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
  if (sk_t <= 0 || sv_t <= 0 || sk_t >= (1 << 24) || sv_t >= (1 << 24)) {
    // Per-lane offsets within a 64-key tile are 32-bit.
    set_error("sa_update_attention_state: k/v token strides must be in [1, 2^24) elements");
    return SA_ERR_INVALID_ARGUMENT;
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
  if (merge_keys < 0 || merge_keys % 64 != 0) {
    set_error("merge_keys %d is not a multiple of the 64-key tile", merge_keys);
    return SA_ERR_INVALID_ARGUMENT;
  }
  p.merge_tiles = merge_keys / 64;
  p.tiled_state = tiled_state ? 1 : 0;
  if (fused != nullptr) {
    // Same output layout rules as the finalize kernel.
    if (!fused->out || fused->so_t % 8 != 0 || fused->so_h % 8 != 0 || !aligned(fused->out, 16)) {
      set_error("fused finalize needs a 16-byte aligned output with vector-aligned strides");
      return SA_ERR_INVALID_ARGUMENT;
    }
    p.out = static_cast<uint16_t*>(fused->out);
    p.so_t = fused->so_t;
    p.so_h = fused->so_h;
    p.lse = fused->lse;
    p.lse_sh = fused->lse_sh;
    p.lse_off = fused->lse_off;
  }
  // Workgroup numbering is 32-bit: at least 128 queries per workgroup.
  if (((int64_t)q_tokens + 127) / 128 * q_heads > (int64_t)INT32_MAX / 8) {
    set_error("sa_update_attention_state: q_tokens * q_heads too large for one launch");
    return SA_ERR_INVALID_ARGUMENT;
  }
  const int dp = head_dim <= 32 ? 32 : head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
  p.q_heads = q_heads;
  const bool causal = (flags & SA_FLAG_CAUSAL) != 0;
  const bool init = (flags & SA_FLAG_INITIALIZE) != 0;
  if (v_transposed) {
    // v is transpose_v_kernel's layout: row stride sv_t (keys padded to whole
    // 64-key tiles), head stride sv_h.
    if (head_dim != 128 || !init || sv_t % 64 != 0 || sv_t < kv_tokens || sv_h < 128 * sv_t) {
      set_error("transposed V needs head_dim 128, an initializing launch and a padded [heads][128][keys] layout");
      return SA_ERR_INVALID_ARGUMENT;
    }
    hipError_t err = dtype == SA_DTYPE_BF16 ? launch_update_dp<BF16, 128, false, true>(p, causal, init, stream)
                                            : launch_update_dp<FP16, 128, false, true>(p, causal, init, stream);
    return err == hipSuccess ? 0 : hip_status(err, "update kernel launch");
  }
  hipError_t err = dtype == SA_DTYPE_BF16 ? launch_update_op<BF16>(p, dp, causal, init, stream)
                                          : launch_update_op<FP16>(p, dp, causal, init, stream);
  return err == hipSuccess ? 0 : hip_status(err, "update kernel launch");
}

int32_t launch_update_int8(const void* q, const void* k, const void* v, const void* k_scales,
                           const void* v_scales, float* m, float* l, float* acc, int64_t sq_t,
                           int64_t sq_h, int64_t sk_t, int64_t sk_h, int64_t sv_t, int64_t sv_h,
                           int64_t sks_g, int64_t sks_h, int64_t svs_g, int64_t svs_h,
                           int64_t ss_t, int64_t ss_h, int64_t sa_t, int64_t sa_h,
                           int32_t q_tokens, int32_t kv_tokens, int32_t q_heads, int32_t kv_heads,
                           int32_t head_dim, int32_t q_local_offset, int32_t kv_local_offset,
                           int32_t storage_token_offset, int32_t causal_shift,
                           double softmax_scale, int32_t flags, int32_t dtype,
                           int32_t quant_group_tokens, hipStream_t stream, bool tiled_state) {
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    set_error("sa_update_attention_state_int8: unsupported query dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (head_dim < 16 || head_dim > 128 || head_dim % 16 != 0) {
    set_error("sa_update_attention_state_int8: head_dim must be a multiple of 16 in [16, 128], got %d",
              head_dim);
    return SA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  if (q_tokens < 0 || kv_tokens < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 ||
      storage_token_offset < 0) {
    set_error("sa_update_attention_state_int8: bad sizes q_tokens=%d kv_tokens=%d q_heads=%d kv_heads=%d "
              "storage_token_offset=%d", q_tokens, kv_tokens, q_heads, kv_heads, storage_token_offset);
    return SA_ERR_INVALID_ARGUMENT;
  }
  int shift = 0;
  while (shift < 30 && (1 << shift) < quant_group_tokens) ++shift;
  if (quant_group_tokens <= 0 || (1 << shift) != quant_group_tokens) {
    set_error("sa_update_attention_state_int8: quant_group_tokens must be a power of two, got %d",
              quant_group_tokens);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (q_tokens == 0) return 0;
  if (!q || !k || !v || !k_scales || !v_scales || !m || !l || !acc) {
    set_error("sa_update_attention_state_int8: null pointer argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  // Q: 16-byte vectors of 8 elements; int8 K/V: 16-byte DMA granules.
  if (sq_t % 8 != 0 || sq_h % 8 != 0 || sk_t % 16 != 0 || sk_h % 16 != 0 || sv_t % 16 != 0 ||
      sv_h % 16 != 0) {
    set_error("sa_update_attention_state_int8: q strides must be multiples of 8 elements and int8 "
              "k/v strides multiples of 16");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (sk_t <= 0 || sv_t <= 0 || sk_t >= (1 << 24) || sv_t >= (1 << 24)) {
    set_error("sa_update_attention_state_int8: k/v token strides must be in [1, 2^24) elements");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (sa_t % 4 != 0 || sa_h % 4 != 0 || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) ||
      !aligned(acc, 16) || !aligned(m, 4) || !aligned(l, 4) || !aligned(k_scales, 2) ||
      !aligned(v_scales, 2)) {
    set_error("sa_update_attention_state_int8: buffers must be aligned (16 bytes for q/k/v/acc, 2 for scales)");
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
  p.q_heads = q_heads;
  p.ks = static_cast<const uint16_t*>(k_scales);
  p.vs = static_cast<const uint16_t*>(v_scales);
  p.sks_g = sks_g; p.sks_h = sks_h; p.svs_g = svs_g; p.svs_h = svs_h;
  p.scale_offset = storage_token_offset;
  p.scale_shift = shift;
  p.tiled_state = tiled_state ? 1 : 0;
  const int dp = head_dim <= 32 ? 32 : head_dim <= 64 ? 64 : 128;
  const bool causal = (flags & SA_FLAG_CAUSAL) != 0;
  const bool init = (flags & SA_FLAG_INITIALIZE) != 0;
  hipError_t err = dtype == SA_DTYPE_BF16 ? launch_update_int8_op<BF16>(p, dp, causal, init, stream)
                                          : launch_update_int8_op<FP16>(p, dp, causal, init, stream);
  return err == hipSuccess ? 0 : hip_status(err, "int8 update kernel launch");
}

int32_t launch_transpose_v(const void* v, int64_t sv_t, int64_t sv_h, int32_t kv_tokens, int32_t kv_heads,
                           int32_t head_dim, void* vt, int64_t t_pad, hipStream_t stream) {
  if (head_dim != 128 || kv_tokens < 0 || kv_heads <= 0 || t_pad % 64 != 0 || t_pad < kv_tokens ||
      t_pad >= (1 << 24) || !v || !vt || sv_t % 8 != 0 || sv_h % 8 != 0 || !aligned(v, 16) ||
      !aligned(vt, 16)) {
    set_error("transpose of V: bad arguments (head_dim %d, kv_tokens %d, kv_heads %d, padded keys %lld)",
              head_dim, kv_tokens, kv_heads, (long long)t_pad);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (t_pad == 0) return 0;
  TransposeParams p;
  p.v = static_cast<const uint16_t*>(v);
  p.vt = static_cast<uint16_t*>(vt);
  p.sv_t = sv_t;
  p.sv_h = sv_h;
  p.t_pad = t_pad;
  p.kv_tokens = kv_tokens;
  p.tiles = (int32_t)(t_pad / 64);
  hipLaunchKernelGGL(transpose_v_kernel, dim3((unsigned)((int64_t)kv_heads * p.tiles)), dim3(256), 0, stream, p);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_status(err, "transpose of V");
}

int32_t launch_finalize(const float* acc, const float* m, const float* l, void* out, float* lse,
                        int64_t sa_t, int64_t sa_h, int64_t ss_t, int64_t ss_h, int64_t so_t,
                        int64_t so_h, int64_t lse_sh, int64_t lse_off, int32_t q_tokens,
                        int32_t q_heads, int32_t head_dim, int32_t dtype, hipStream_t stream,
                        bool tiled_state) {
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
  p.q_tokens = q_tokens;
  p.q_heads = q_heads;
  p.tiled_state = tiled_state ? 1 : 0;
  if (q_heads > 65535) {
    set_error("sa_finalize_attention: q_heads %d exceeds the grid's 65,535 heads", q_heads);
    return SA_ERR_INVALID_ARGUMENT;
  }
  const dim3 grid((unsigned)(((int64_t)q_tokens + 15) / 16), (unsigned)q_heads);
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL(finalize_kernel<BF16>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(finalize_kernel<FP16>, grid, dim3(256), 0, stream, p);
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_status(err, "finalize kernel launch");
}

}  // namespace sa

namespace {

// Device scratch of sa_run_resident_noalloc: the transposed copy of V that
// the resident update launch reads.  One array per GPU, held from the first
// load of this library's code object until the process ends.  In host code
// the name is only a stand-in for the symbol: the array's address on a
// device comes from hipGetSymbolAddress with that device current, looked up
// once per device and kept below.
constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

int32_t scratch_on_current_device(void** address) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return sa::hip_status(err, "sa_run_resident_noalloc: hipGetDevice");
  if (device < 0 || device >= kMaxDevices) {
    sa::set_error("sa_run_resident_noalloc: device ordinal %d outside [0, %d)", device, kMaxDevices);
    return SA_ERR_BAD_STATE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* found = nullptr;
    err = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return sa::hip_status(err, "sa_run_resident_noalloc: hipGetSymbolAddress(scratch)");
    if (found == nullptr || reinterpret_cast<uintptr_t>(found) % 256 != 0) {
      sa::set_error("sa_run_resident_noalloc: scratch address %p is not 256-byte aligned", found);
      return SA_ERR_BAD_STATE;
    }
    g_scratch_address[device] = found;
  }
  *address = g_scratch_address[device];
  return 0;
}

}  // namespace

extern "C" {

int32_t sa_run_resident_noalloc(const void* q, const void* k, const void* v, void* out, float* lse,
                                int64_t stride_qt, int64_t stride_qh, int64_t stride_kt,
                                int64_t stride_kh, int64_t stride_vt, int64_t stride_vh,
                                int64_t stride_ot, int64_t stride_oh, int64_t lse_stride_h,
                                const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k,
                                int32_t num_segments, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, int32_t dtype, int32_t kv_chunk_tokens,
                                double softmax_scale, int32_t causal, void* stream) {
  sa::clear_error();
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k || num_segments < 0) {
    sa::set_error("sa_run_resident_noalloc: null argument");
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (head_dim != 128) {
    sa::set_error("sa_run_resident_noalloc: the transposed-V launch needs head_dim 128, got %d", head_dim);
    return SA_ERR_UNSUPPORTED_HEAD_DIM;
  }
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_FP16) {
    sa::set_error("sa_run_resident_noalloc: unsupported dtype code %d", dtype);
    return SA_ERR_UNSUPPORTED_DTYPE;
  }
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || kv_chunk_tokens <= 0 ||
      kv_chunk_tokens % 64 != 0) {
    sa::set_error("sa_run_resident_noalloc: bad heads %d/%d or K/V chunk %d (a positive multiple of 64)",
                  q_heads, kv_heads, kv_chunk_tokens);
    return SA_ERR_INVALID_ARGUMENT;
  }
  if (stride_ot % 8 != 0 || stride_oh % 8 != 0 || !aligned(out, 16)) {
    sa::set_error("sa_run_resident_noalloc: out must be 16-byte aligned with strides that are multiples of 8");
    return SA_ERR_INVALID_ARGUMENT;
  }
  // The launches' own argument rules, checked here so that a call they would
  // reject is rejected before anything is enqueued on the shared scratch.
  const int64_t in_strides[] = {stride_qt, stride_qh, stride_kt, stride_kh, stride_vt, stride_vh};
  for (int64_t st : in_strides) {
    if (st % 8 != 0) {
      sa::set_error("sa_run_resident_noalloc: q/k/v token and head strides must be multiples of 8 elements");
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  if (stride_kt <= 0 || stride_kt >= (1 << 24) || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) ||
      (lse != nullptr && !aligned(lse, 4))) {
    sa::set_error("sa_run_resident_noalloc: q/k/v must be 16-byte aligned (lse 4-byte) and the k token stride "
                  "in [1, 2^24) elements");
    return SA_ERR_INVALID_ARGUMENT;
  }
  // Every segment is checked before anything is enqueued.
  for (int32_t s = 0; s < num_segments; ++s) {
    const int64_t q_length = cu_seqlens_q[s + 1] - cu_seqlens_q[s];
    const int64_t k_length = cu_seqlens_k[s + 1] - cu_seqlens_k[s];
    if (q_length < 0 || k_length < 0 || (q_length > 0 && k_length == 0) || q_length > INT32_MAX ||
        k_length >= (1 << 24)) {
      sa::set_error("sa_run_resident_noalloc: segment %d has invalid bounds", s);
      return SA_ERR_INVALID_ARGUMENT;
    }
    // Workgroup numbering of the update launch is 32-bit.
    if ((q_length + 127) / 128 * q_heads > (int64_t)INT32_MAX / 8) {
      sa::set_error("sa_run_resident_noalloc: segment %d has too many queries x heads for one launch", s);
      return SA_ERR_INVALID_ARGUMENT;
    }
    const int64_t needed = (int64_t)kv_heads * 128 * ((k_length + 63) / 64 * 64) * 2;
    if (q_length > 0 && needed > kNoAllocScratchBytes) {
      sa::set_error("sa_run_resident_noalloc: segment %d needs %lld bytes of transposed-V scratch; this entry "
                    "point has %lld (kv_heads * 128 * keys rounded up to 64 * 2 bytes per segment)",
                    s, (long long)needed, (long long)kNoAllocScratchBytes);
      return SA_ERR_INVALID_ARGUMENT;
    }
  }
  void* vt = nullptr;
  int32_t rc = scratch_on_current_device(&vt);
  if (rc != 0) return rc;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const char* qd = static_cast<const char*>(q);
  const char* kd = static_cast<const char*>(k);
  const char* vd = static_cast<const char*>(v);
  char* od = static_cast<char*>(out);
  for (int32_t s = 0; s < num_segments; ++s) {
    const int64_t q_start = cu_seqlens_q[s], k_start = cu_seqlens_k[s];
    const int64_t q_length = cu_seqlens_q[s + 1] - q_start, k_length = cu_seqlens_k[s + 1] - k_start;
    if (q_length == 0) continue;
    // The launch sequence of sa_pipeline_run_resident's fused path with the
    // scratch in place of the attached one: V transposed (zero keys up to
    // the 64-key tile), then one update launch over the segment that
    // finalizes in its epilogue with the row sums merged at every K/V chunk
    // boundary.  Both launches are on `stream`, so a later segment's
    // transpose starts after this segment's update has read the scratch.
    const int64_t t_pad = (k_length + 63) / 64 * 64;
    const char* v_seg = vd + k_start * stride_vt * 2;
    rc = sa::launch_transpose_v(v_seg, stride_vt, stride_vh, (int32_t)k_length, kv_heads, 128, vt, t_pad, hs);
    if (rc != 0) return rc;
    const sa::FusedOutput fused{od + q_start * stride_ot * 2, stride_ot, stride_oh, lse, lse_stride_h, q_start};
    rc = sa::launch_update(qd + q_start * stride_qt * 2, kd + k_start * stride_kt * 2, vt, nullptr, nullptr,
                           nullptr, stride_qt, stride_qh, stride_kt, stride_kh, t_pad, 128 * t_pad, 0, 0, 0, 0,
                           (int32_t)q_length, (int32_t)k_length, q_heads, kv_heads, 128, 0, 0,
                           (int32_t)(k_length - q_length), softmax_scale,
                           (causal ? SA_FLAG_CAUSAL : 0) | SA_FLAG_INITIALIZE, dtype, hs, kv_chunk_tokens, &fused,
                           true);
    if (rc != 0) return rc;
  }
  return 0;
}

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

int32_t sa_update_attention_state_int8(
    const void* q, const void* k, const void* v, const void* k_scales, const void* v_scales,
    float* running_max, float* running_sum, float* accumulator, int64_t stride_qt,
    int64_t stride_qh, int64_t stride_kt, int64_t stride_kh, int64_t stride_vt, int64_t stride_vh,
    int64_t stride_ksg, int64_t stride_ksh, int64_t stride_vsg, int64_t stride_vsh,
    int64_t stride_st, int64_t stride_sh, int64_t stride_at, int64_t stride_ah, int32_t q_tokens,
    int32_t kv_tokens, int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t q_local_offset,
    int32_t kv_local_offset, int32_t storage_token_offset, int32_t causal_shift,
    double softmax_scale, int32_t flags, int32_t dtype, int32_t quant_group_tokens, void* stream) {
  sa::clear_error();
  return sa::launch_update_int8(q, k, v, k_scales, v_scales, running_max, running_sum, accumulator,
                                stride_qt, stride_qh, stride_kt, stride_kh, stride_vt, stride_vh,
                                stride_ksg, stride_ksh, stride_vsg, stride_vsh, stride_st, stride_sh,
                                stride_at, stride_ah, q_tokens, kv_tokens, q_heads, kv_heads,
                                head_dim, q_local_offset, kv_local_offset, storage_token_offset,
                                causal_shift, softmax_scale, flags, dtype, quant_group_tokens,
                                static_cast<hipStream_t>(stream));
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
