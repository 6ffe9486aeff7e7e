// Batched LFM2.5 pass on gfx950: up to 64 rows (token, sequence, position)
// through all 14 layers, every weight tile read once for all rows and
// multiplied on the matrix cores. This is the reference's batched prompt pass
// (prefill_design, experiments/lfm25_x8.py:341-416: PB tokens per weight load,
// dot4 in kernels/x8/x8p_core.cc:43-60, causal in-batch attention
// attn_block4 :156-227) generalised to rows of several independent sequences.
//
// Rows of one sequence must be consecutive with consecutive positions (a
// prompt chunk); the host checks this. Each sequence has its own conv state
// and KV cache. A pass is one kernel per phase, stream ordered:
//
//   embed -> per layer: norm + in_proj+conv gate | norm + q/k/v+QK-norm+RoPE
//   +append, attention -> out_proj+residual -> norm + w1/w3+SiLU gate ->
//   w2+residual -> (select) final norm + head GEMM + per-block argmax -> pick
//
// GEMM kernels: a block owns NT tiles of 16 weight rows and all batch rows;
// its 8 waves split (tile, K slice), each wave streams its 16 x (K / KS)
// weight slice with 16-byte buffer loads and multiplies it into four 16 x 16
// f32 accumulators (one per 16 batch rows) with v_mfma_f32_16x16x32_bf16; the
// KS partial sums of a tile meet in LDS, summed in slice order, and the
// epilogue of the phase (conv gate, residual, SiLU gate, QK-norm + RoPE + KV
// append, head candidates) runs on the reduced tile. The products whose
// input is the residual stream's RMSNorm stage the normed rows in LDS (the
// norm formed on the way, no pass of its own) and read their activations
// from there. At 4-64 rows the pass is bound by the loads (about B FLOP per
// weight byte), so the matrix cores only have to keep them flowing.
#include <algorithm>
#include <cstring>
#include <vector>

#include "lfm25_host.h"
#include "lfm25_layout.h"
#include "lfm25_stages.h"

namespace lfm25 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to a BF16 pair, low first (one v_cvt_pk_bf16_f32; round to
// nearest even, as f32_to_bf16).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr int kRowsMax = LFM25_BATCH_MAX_ROWS;  // 64
constexpr int kMT = kRowsMax / 16;              // 16-row tiles of the batch
constexpr int kGT = 512;                         // threads of a GEMM block
constexpr int kGW = kGT / kWave;                 // its waves
constexpr int kAT = 256;                         // threads of an attention block
static_assert(kRowsMax % 16 == 0, "whole batch tiles");

// Workspace layout (bytes).
constexpr size_t kBwCtl = 0;                                     // int32 [64]: [0] status
constexpr size_t kBwRows = 256;                                  // int32 [64][4] row table
constexpr size_t kBwStart = kBwRows + kRowsMax * 16;             // int32 [64] decode start positions
constexpr size_t kBwX = 2048;                                    // bf16 [64][1024] residual stream
constexpr size_t kBwXn = kBwX + (size_t)kRowsMax * kHidden * 2;  // bf16 [64][1024] normed rows (above kFoldRows)
constexpr size_t kBwG = kBwXn + (size_t)kRowsMax * kHidden * 2;  // bf16 [64][2560] FFN gate values
constexpr size_t kBwY = kBwG + (size_t)kRowsMax * kFfn * 2;      // bf16 [64][1024] conv out / context
constexpr size_t kBwQ = kBwY + (size_t)kRowsMax * kHidden * 2;   // bf16 [64][1024] queries
constexpr size_t kBwCand = kBwQ + (size_t)kRowsMax * kHidden * 2;  // u64 [head blocks][64]
constexpr int kHeadBlocksMax = 256;  // head blocks (kHeadBlocks)
constexpr int kResSplit = 4;  // K slices of a split residual projection (one block each)
constexpr size_t kBwPart = kBwCand + (size_t)kHeadBlocksMax * kRowsMax * 8;  // f32 [64 tiles][4][64 rows][16]
constexpr size_t kBwCount = kBwPart + (size_t)(kHidden / 16) * kResSplit * kRowsMax * 16 * 4;  // int32 [64 tiles]
constexpr size_t kBwBytes = kBwCount + (size_t)(kHidden / 16) * 4;
// The persistent batched decode's exchange region follows, on a 256-byte
// boundary (batch_persistent_bytes(), lfm25_decode.hip).
constexpr size_t kBwPersist = (kBwBytes + 255) & ~(size_t)255;

// Row table entry: token, sequence, position, and (index within its
// sequence's chunk) | (1 << 16 when it is the chunk's last row).
struct RowInfo {
  int token, seq, pos, chunk;
};
constexpr int kLastRow = 1 << 16;

struct BatchParams {
  const uint16_t* weights;
  const uint16_t* embedding;
  const uint16_t* rope;
  uint16_t* conv_state;   // [seqs][8][1024][3]
  uint16_t* key_cache;    // [seqs][6][8][capacity][64]
  uint16_t* value_cache;
  char* ws;
  int rows, seqs, capacity, vocab;
};

__device__ __forceinline__ int32_t* b_status(const BatchParams& p) {
  return reinterpret_cast<int32_t*>(p.ws + kBwCtl);
}
__device__ __forceinline__ const RowInfo& b_row(const BatchParams& p, int m) {
  return reinterpret_cast<const RowInfo*>(p.ws + kBwRows)[m];
}
__device__ __forceinline__ uint16_t* b_x(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwX); }
__device__ __forceinline__ uint16_t* b_g(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwG); }
__device__ __forceinline__ uint16_t* b_xn(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwXn); }
__device__ __forceinline__ uint16_t* b_y(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwY); }
__device__ __forceinline__ uint16_t* b_q(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwQ); }
// Device-scope (cross-XCD) relaxed loads and stores of one word: they are
// performed at the coherence point, not in one XCD's L2.
__device__ __forceinline__ uint32_t dev_load32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dev_store32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float* b_part(const BatchParams& p) { return reinterpret_cast<float*>(p.ws + kBwPart); }
__device__ __forceinline__ int32_t* b_count(const BatchParams& p) { return reinterpret_cast<int32_t*>(p.ws + kBwCount); }
__device__ __forceinline__ uint64_t* b_cand(const BatchParams& p) {
  return reinterpret_cast<uint64_t*>(p.ws + kBwCand);
}
__device__ __forceinline__ size_t kv_head_base(const BatchParams& p, int seq, int att, int g) {
  return ((size_t)(seq * LFM25_ATTN_LAYERS + att) * kKvHeads + g) * p.capacity * kHeadDim;
}

__device__ __forceinline__ Rsrc rsrc(const void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ bf16x8_t load_bf16x8(Rsrc r, int voff, int soff) {
  return __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// ------------------------------------------------------------------ GEMM core

// Partial tiles of the 8 waves: part[w][m][lane][e] holds, for wave w's tile
// and 16-row batch tile m, the f32 accumulator element e of `lane` (row
// 4 (lane / 16) + e of the weight tile, batch row 16 m + lane % 16).
struct GemmLds {
  f32x4_t part[kGW][kMT][kWave];
};
// The same after a staged product (gemm_tiles_staged): the batch's rows in
// LDS first (padded to kXRow bytes, so that the lanes' 16-byte reads hit
// distinct banks), the partial tiles in the same space once every product
// has read them.
constexpr int kXRow = kHidden * 2 + 16;
struct GemmLdsStaged {
  union {
    char x[kRowsMax][kXRow];
    f32x4_t part[kGW][kMT][kWave];
  };
  float ss[kRowsMax][2];  // the rows' sums of squares, per half (RowStage)
};

// The batch tiles in use (rows past `rows` as zeros) staged into LDS rows of
// kXRow bytes. Up to kFoldRows rows they are RMSNorm'ed on the way
// (Lfm2RMSNorm.forward, modeling_lfm2.py:54-59, two roundings): thread t
// copies the 8 elements of column block t % 128 of rows t / 128 + 4j of every
// tile, so waves 2q and 2q + 1 cover one row: the row's mean square is the
// sum of their two wave sums (each vector's 8 squares added in element
// order, then the wave's tree), in that order. Above that every block would
// repeat too much of the norm (it sits between the loads and the products),
// so k_bx_norm writes the normed rows once and they are copied as they are.
// load() requests the rows and the thread's 8 norm weights; store() (every
// thread of the block) waits for them, exchanges the half-row sums through
// LDS (one block barrier) and writes the rows; the caller's barrier then
// publishes them.
constexpr int kFoldRows = 16;
struct RowStage {
  static constexpr int kPerTile = 16 * (kHidden / 8) / kGT;  // 4 vectors per thread per batch tile
  u32x4_t v[kMT][kPerTile];
  u32x4_t g;
  __device__ __forceinline__ void load(const uint16_t* x, const uint16_t* gamma, int rows, int mt) {
    const Rsrc rx = rsrc(x, (size_t)rows * kHidden * 2);
    if (rows <= kFoldRows) g = reinterpret_cast<const u32x4_t*>(gamma)[threadIdx.x % (kHidden / 8)];
#pragma unroll
    for (int k = 0; k < kMT; ++k) {
      if (k < mt) {
#pragma unroll
        for (int j = 0; j < kPerTile; ++j)
          v[k][j] = __builtin_bit_cast(u32x4_t, load_bf16x8(rx, (row(k, j) * kHidden + col()) * 2, 0));
      }
    }
  }
  __device__ static __forceinline__ int row(int k, int j) { return 16 * k + 4 * j + (int)threadIdx.x / (kHidden / 8); }
  __device__ static __forceinline__ int col() { return 8 * ((int)threadIdx.x % (kHidden / 8)); }
  __device__ __forceinline__ void store(char (*xl)[kXRow], float (*ssl)[2], int mt, bool fold) {
    if (!fold) {
#pragma unroll
      for (int k = 0; k < kMT; ++k) {
        if (k < mt) {
#pragma unroll
          for (int j = 0; j < kPerTile; ++j) *reinterpret_cast<u32x4_t*>(&xl[row(k, j)][2 * col()]) = v[k][j];
        }
      }
      return;
    }
    const int half = wave_id() & 1;
#pragma unroll
    for (int k = 0; k < kMT; ++k) {
      if (k < mt) {
#pragma unroll
        for (int j = 0; j < kPerTile; ++j) {
          float q = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q = fmaf(lo_f32(v[k][j][e]), lo_f32(v[k][j][e]), q);
            q = fmaf(hi_f32(v[k][j][e]), hi_f32(v[k][j][e]), q);
          }
          q = wave_sum(q);
          if (lane_id() == 0) ssl[row(k, j)][half] = q;
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int k = 0; k < kMT; ++k) {
      if (k < mt) {
#pragma unroll
        for (int j = 0; j < kPerTile; ++j) {
          const int r = row(k, j);
          const float sc = 1.0f / sqrtf((ssl[r][0] + ssl[r][1]) * (1.0f / (float)kHidden) + kNormEps);
          u32x4_t o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t xr = pack_bf16(lo_f32(v[k][j][e]) * sc, hi_f32(v[k][j][e]) * sc);
            o[e] = pack_bf16(lo_f32(xr) * lo_f32(g[e]), hi_f32(xr) * hi_f32(g[e]));
          }
          *reinterpret_cast<u32x4_t*>(&xl[r][2 * col()]) = o;
        }
      }
    }
  }
};

// part[w] = W_t[16 x K-slice] . X[rows x K-slice]^T for wave w = t * KS + s:
// tile t of the NT weight tiles (16 rows each, rows of length K starting at
// wt[t]), slice s of KS. Lanes load A (weights: row lane % 16, columns
// 8 (lane / 16) .. + 8 of each 32-column step) and B (activations: batch row
// lane % 16 of the tile, same columns) as 16-byte vectors; rows past `rows`
// read zeros. The wave's whole weight slice is requested before the first
// product (one memory latency per phase instead of one per step).
// `mid` runs in every wave once the wave's loads are requested (before any
// of them is waited for): an epilogue requests its own operands there, so
// their latency hides behind the products. Loads the caller issues before
// the call land first, so `mid` can wait for them without waiting for the
// weights.
struct NoMid {
  __device__ void operator()() const {}
};
// (KLen < K: the product over columns [k0, k0 + KLen) of rows of length K.)
template <int NT, int KS, int K, typename Mid = NoMid, int KLen = K>
__device__ __forceinline__ void gemm_tiles(const uint16_t* const* wt, const uint16_t* x, int rows, GemmLds& sh,
                                           const Mid& mid = Mid{}, int k0 = 0) {
  static_assert(NT * KS <= kGW && KLen % (32 * KS) == 0 && K % KLen == 0, "tile split");
  constexpr int kSteps = KLen / (32 * KS);
  const int w = wave_id(), l = lane_id();
  if (w >= NT * KS) {
    mid();
    return;
  }
  const int t = w / KS, s = w % KS;
  const int mt = (rows + 15) / 16;
  const int col0 = k0 + s * (KLen / KS);
  const Rsrc ra = rsrc(wt[t], (size_t)16 * K * 2);
  const Rsrc rb = rsrc(x, (size_t)rows * K * 2);
  const int a_off = ((l & 15) * K + 8 * (l >> 4)) * 2;
  f32x4_t acc[kMT];
#pragma unroll
  for (int m = 0; m < kMT; ++m) acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  bf16x8_t a[kSteps];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) a[st] = load_bf16x8(ra, a_off, (col0 + 32 * st) * 2);
  // Activations: the slice of batch tile m + 1 is requested before tile m is
  // multiplied (two register buffers, alternating), so each wave waits for
  // the L2 about once per batch tile rather than once per product.
  bf16x8_t bv[2][kSteps];
  const auto load_b = [&](int m, bf16x8_t* dst) {
    const int b_off = ((16 * m + (l & 15)) * K + 8 * (l >> 4)) * 2;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) dst[st] = load_bf16x8(rb, b_off, (col0 + 32 * st) * 2);
  };
  load_b(0, bv[0]);
  // (the scheduler may not move `mid`'s address arithmetic, and the wait for
  // the operands it depends on, in front of the loads above)
  __builtin_amdgcn_sched_barrier(0);
  mid();
#pragma unroll
  for (int m = 0; m < kMT; ++m) {
    if (m < mt) {
      if (m + 1 < mt) load_b(m + 1, bv[(m + 1) & 1]);
#pragma unroll
      for (int st = 0; st < kSteps; ++st)
        acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[st], bv[m & 1][st], acc[m], 0, 0, 0);
    }
  }
#pragma unroll
  for (int m = 0; m < kMT; ++m) sh.part[w][m][l] = acc[m];
}

// Reduced element (tile t, weight row i, batch row m) after gemm_tiles and a
// block barrier: the KS slice partials summed in slice order.
template <int KS, typename Lds>
__device__ __forceinline__ float gemm_at(const Lds& sh, int t, int i, int m) {
  const int lane = (m & 15) + 16 * (i >> 2);
  float v = sh.part[t * KS][m >> 4][lane][i & 3];
#pragma unroll
  for (int s = 1; s < KS; ++s) v += sh.part[t * KS + s][m >> 4][lane][i & 3];
  return v;
}

// gemm_tiles for K = 1,024 over the RMSNorm of the residual stream x with
// norm weights gamma, the normed activations staged in LDS (RowStage): every
// wave reads its B operands from there, so a K slice shared by NT tiles
// crosses the vector cache once instead of NT times (at 64 rows the
// activation reads, not the weights, bound the per-CU load rate), and no
// separate norm pass runs. The weights are requested before the staging
// waits for the rows.
// Weight rows of a tile: row i of tile t lies RowMap::off(t, i) rows after
// wt[t], inside RowMap::span(t) rows (rows at or past the span read zeros).
struct DenseRows {
  __device__ static int off(int, int i) { return i; }
  __device__ static int span(int) { return 16; }
};
template <int NT, int KS, typename RowMap = DenseRows, typename Mid = NoMid>
__device__ __forceinline__ void gemm_tiles_staged(const uint16_t* const* wt, const BatchParams& p, const uint16_t* gamma,
                                                  GemmLdsStaged& sh, const Mid& mid = Mid{}) {
  const int rows = p.rows;
  const bool fold = rows <= kFoldRows;
  constexpr int K = kHidden;
  static_assert(NT * KS <= kGW && K % (32 * KS) == 0, "tile split");
  constexpr int kSteps = K / (32 * KS);
  const int w = wave_id(), l = lane_id();
  const bool active = w < NT * KS;
  const int t = w / KS, s = w % KS;
  const int mt = (rows + 15) / 16;
  const int col0 = s * (K / KS);
  RowStage stage;
  stage.load(fold ? b_x(p) : b_xn(p), gamma, rows, mt);
  bf16x8_t a[kSteps];
  {
    const Rsrc ra = rsrc(wt[active ? t : 0], active ? (size_t)RowMap::span(t) * K * 2 : 0);
    const int a_off = (RowMap::off(t, l & 15) * K + 8 * (l >> 4)) * 2;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) a[st] = load_bf16x8(ra, a_off, (col0 + 32 * st) * 2);
  }
  __builtin_amdgcn_sched_barrier(0);
  mid();
  stage.store(sh.x, sh.ss, mt, fold);
  lds_barrier();
  f32x4_t acc[kMT];
#pragma unroll
  for (int m = 0; m < kMT; ++m) acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (active) {
#pragma unroll
    for (int m = 0; m < kMT; ++m) {
      if (m < mt) {
        const char* xr = &sh.x[16 * m + (l & 15)][2 * col0 + 16 * (l >> 4)];
#pragma unroll
        for (int st = 0; st < kSteps; ++st)
          acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[st], *reinterpret_cast<const bf16x8_t*>(xr + 64 * st),
                                                           acc[m], 0, 0, 0);
      }
    }
  }
  lds_barrier();  // every product has read the rows before the partial tiles overwrite them
  if (active) {
#pragma unroll
    for (int m = 0; m < kMT; ++m) sh.part[w][m][l] = acc[m];
  }
}

// ------------------------------------------------------------------ small phases

// Row m of X = the embedding row of its token (ids outside the table are
// clamped and flagged in status bit 0).
// In a decode step (tokens != nullptr) the block first writes row m of the
// step's table: sequence m consumes tokens[m] at position start[m] + step.
__global__ void __launch_bounds__(kWave) k_bx_embed(BatchParams p, const int32_t* tokens, int step) {
  const int m = blockIdx.x;
  int tok;
  if (tokens != nullptr) {
    tok = tokens[m];
    if (threadIdx.x == 0) {
      const int32_t* start = reinterpret_cast<const int32_t*>(p.ws + kBwStart);
      reinterpret_cast<RowInfo*>(p.ws + kBwRows)[m] = RowInfo{tok, m, start[m] + step, kLastRow};
    }
  } else {
    tok = b_row(p, m).token;
  }
  if (tok < 0 || tok >= p.vocab) {
    if (threadIdx.x == 0) atomicOr(b_status(p), 1);
    tok = tok < 0 ? 0 : p.vocab - 1;
  }
  const uint4* src = reinterpret_cast<const uint4*>(p.embedding + (size_t)tok * kHidden);
  uint4* dst = reinterpret_cast<uint4*>(b_x(p) + (size_t)m * kHidden);
  for (int i = threadIdx.x; i < kHidden / 8; i += kWave) dst[i] = src[i];
}

// RMSNorm of every row (Lfm2RMSNorm.forward, modeling_lfm2.py:54-59, two
// roundings), for passes of more than kFoldRows rows: 128 threads per row,
// thread j holding the 8 elements of column block j, with RowStage's order of
// additions (each block's squares in element order, the wave sums of blocks
// 0..63 and 64..127, then their sum), so a row's normed values are the same
// bits whichever way its pass forms them.
__global__ void __launch_bounds__(2 * kWave) k_bx_norm(BatchParams p, const uint16_t* __restrict__ src,
                                                       const uint16_t* __restrict__ gamma, uint16_t* __restrict__ dst) {
  __shared__ float half_ss[2];
  const int m = blockIdx.x, j = threadIdx.x;
  const u32x4_t x = reinterpret_cast<const u32x4_t*>(src + (size_t)m * kHidden)[j];
  const u32x4_t g = reinterpret_cast<const u32x4_t*>(gamma)[j];
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    q = fmaf(lo_f32(x[e]), lo_f32(x[e]), q);
    q = fmaf(hi_f32(x[e]), hi_f32(x[e]), q);
  }
  q = wave_sum(q);
  if (lane_id() == 0) half_ss[wave_id()] = q;
  __syncthreads();
  const float sc = 1.0f / sqrtf((half_ss[0] + half_ss[1]) * (1.0f / (float)kHidden) + kNormEps);
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t xr = pack_bf16(lo_f32(x[e]) * sc, hi_f32(x[e]) * sc);
    o[e] = pack_bf16(lo_f32(xr) * lo_f32(g[e]), hi_f32(xr) * hi_f32(g[e]));
  }
  reinterpret_cast<u32x4_t*>(dst + (size_t)m * kHidden)[j] = o;
}

// ------------------------------------------------------------------ GEMM phases

// in_proj + gated short conv of 8 channels c0 .. c0 + 7 (rows c, 1024 + c,
// 2048 + c give B, C and x of channel c) for every row, the conv window
// running along each sequence's rows: window [a, b, bx] with a, b the
// previous two bx of the sequence (from its state for the first rows);
// the last row of a chunk leaves its window as the state (conv_gate_channel's
// rounding points). Two weight tiles per block, [B; C] and [x; nothing], so
// the 1,024 channels run on 128 blocks (16 channels and three tiles a block
// left half the CUs idle and each of the rest streaming 96 KB of weights).
struct Conv8Rows {
  __device__ static int off(int t, int i) { return t == 0 && i >= 8 ? kHidden + i - 8 : i; }
  __device__ static int span(int t) { return t == 0 ? kHidden + 8 : 8; }
};
__global__ void __launch_bounds__(kGT) k_bx_conv(BatchParams p, int l) {
  __shared__ GemmLdsStaged sh;
  constexpr int kCh = 8;
  __shared__ float bxs[kCh][kRowsMax];
  __shared__ float cgs[kCh][kRowsMax];
  __shared__ float win[kCh][kRowsMax][2];
  static_assert(kRowsMax * kCh == kGT, "one (channel, row) per thread");
  const int c0 = kCh * blockIdx.x;
  const int n = kCh * p.rows;
  const int ci = conv_before(l);
  // The epilogue's operands: the thread's row and taps before the weights,
  // the conv state (addressed by the row) once the weights are requested.
  const int e = min((int)threadIdx.x, n - 1);
  const int i = e % kCh, m = e / kCh;
  const RowInfo ri = b_row(p, m);
  uint16_t tap[kConvTaps], s1, s2;
  {
    const uint16_t* cw = conv_tensor<C_CONVW>(p.weights, l) + (c0 + i) * kConvTaps;
#pragma unroll
    for (int q = 0; q < kConvTaps; ++q) tap[q] = cw[q];
  }
  const auto states = [&] {
    const uint16_t* st = p.conv_state + ((size_t)(ri.seq * LFM25_CONV_LAYERS + ci) * kHidden + c0 + i) * kConvTaps;
    s1 = st[1];
    s2 = st[2];
  };
  const uint16_t* w_in = conv_tensor<C_IN>(p.weights, l);
  const uint16_t* wt[2] = {w_in + (size_t)c0 * kHidden, w_in + (size_t)(2 * kHidden + c0) * kHidden};
  gemm_tiles_staged<2, 4, Conv8Rows>(wt, p, conv_tensor<C_OPNORM>(p.weights, l), sh, states);
  __syncthreads();
  const bool live = (int)threadIdx.x < n;
  if (live) {
    const float B = round_bf16(gemm_at<4>(sh, 0, i, m));
    const float C = round_bf16(gemm_at<4>(sh, 0, kCh + i, m));
    const float x = round_bf16(gemm_at<4>(sh, 1, i, m));
    bxs[i][m] = round_bf16(B * x);
    cgs[i][m] = C;
  }
  __syncthreads();
  if (live) {
    const int j = ri.chunk & 0xffff;
    const float a = j >= 2 ? bxs[i][m - 2] : j == 1 ? bf16_to_f32(s2) : bf16_to_f32(s1);
    const float b = j >= 1 ? bxs[i][m - 1] : bf16_to_f32(s2);
    const float bx = bxs[i][m];
    const float p0 = round_bf16(a * bf16_to_f32(tap[0]));
    const float p1 = round_bf16(b * bf16_to_f32(tap[1]));
    const float p2 = round_bf16(bx * bf16_to_f32(tap[2]));
    const float c = round_bf16((p0 + p1) + p2);
    b_y(p)[(size_t)m * kHidden + c0 + i] = f32_to_bf16(round_bf16(cgs[i][m] * c));
    win[i][m][0] = a;
    win[i][m][1] = b;
  }
  __syncthreads();  // every read of the old states above precedes the writes below
  if (live && (ri.chunk & kLastRow)) {
    uint16_t* st = p.conv_state + ((size_t)(ri.seq * LFM25_CONV_LAYERS + ci) * kHidden + c0 + i) * kConvTaps;
    st[0] = f32_to_bf16(win[i][m][0]);
    st[1] = f32_to_bf16(win[i][m][1]);
    st[2] = f32_to_bf16(bxs[i][m]);
  }
}

// Residual projection of 16 output rows n0 .. n0 + 15: X[m][n] =
// bf16(X[m][n] + bf16(W[n] . in[m])) (out_proj / o_proj with K = 1024, w2 with
// K = 2560; the residual add of Lfm2DecoderLayer.forward, modeling_lfm2.py:431).
// S blocks per tile (block b: tile b % 64, K slice b / 64), so that S times
// as many CUs share the weights and, above all, the activations (at 64 rows
// a tile reads 128-320 KB of them, which one CU's vector cache takes ~10 us
// to pass); each publishes its partial tile at device scope and counts
// itself in; the last to arrive adds the S partials in slice order and
// applies the residual (no block waits for another). The split is the same
// at every row count, so a row's bits never depend on how many rows share
// its pass (at 4 rows it costs ~4% of the step, at 64 it saves 14%).
// Ordering: the partials are agent-scope stores (written through to the
// device's coherence point, never dirty in an XCD's L2), each thread waits
// for their completion (vmcnt(0)) before the barrier behind which the count
// is incremented, and the last block reads them with agent-scope loads
// issued after its increment returned: the release / acquire pair of the
// memory model without its L2 writeback and invalidate, which only matter
// for data written or read through an XCD's L2.
constexpr int res_ks(int len) { return len % (32 * kGW) == 0 ? kGW : len % (32 * 5) == 0 ? 5 : 4; }
template <int K, int S>
__global__ void __launch_bounds__(kGT) k_bx_residual(BatchParams p, const uint16_t* w, const uint16_t* in) {
  __shared__ GemmLds sh;
  __shared__ int last;
  constexpr int kPer = kRowsMax * 16 / kGT;  // elements per thread
  constexpr int kLen = K / S, KS = res_ks(kLen);
  constexpr int kTiles = kHidden / 16;
  const int tile = blockIdx.x % kTiles, sp = blockIdx.x / kTiles;
  const int n0 = 16 * tile;
  const int n = 16 * p.rows;
  uint16_t* x = b_x(p);
  // the residual values, requested before the weights
  uint16_t h[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int e = min((int)threadIdx.x + kGT * k, n - 1);  // (clamped: no select waits for the load)
    h[k] = x[(size_t)(e >> 4) * kHidden + n0 + (e & 15)];
  }
  const uint16_t* wt[1] = {w + (size_t)n0 * K};
  gemm_tiles<1, KS, K, NoMid, kLen>(wt, in, p.rows, sh, NoMid{}, sp * kLen);
  __syncthreads();
  // partial tile [m][i] of slice sp, then the count
  float* part = b_part(p) + (size_t)tile * S * kRowsMax * 16;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int e = threadIdx.x + kGT * k;
    if (e < n) dev_store32(part + sp * kRowsMax * 16 + e, __float_as_uint(gemm_at<KS>(sh, 0, e & 15, e >> 4)));
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partials have reached device scope
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(b_count(p) + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
  __syncthreads();
  if (!last) return;
  if (threadIdx.x == 0) dev_store32(b_count(p) + tile, 0);  // ready for the next split product
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int e = threadIdx.x + kGT * k;
    if (e >= n) break;
    float sum = __uint_as_float(dev_load32(part + e));
#pragma unroll
    for (int q = 1; q < S; ++q) sum += __uint_as_float(dev_load32(part + q * kRowsMax * 16 + e));
    x[(size_t)(e >> 4) * kHidden + n0 + (e & 15)] = f32_to_bf16(round_bf16(bf16_to_f32(h[k]) + round_bf16(sum)));
  }
}

// w1 / w3 of FFN columns f0 .. f0 + 15 and the SiLU gate (Lfm2MLP.forward,
// modeling_lfm2.py:135-136): g = bf16(bf16(silu(bf16(w1 . n))) * bf16(w3 . n)).
__global__ void __launch_bounds__(kGT) k_bx_silu(BatchParams p, int l) {
  __shared__ GemmLdsStaged sh;
  const int f0 = 16 * blockIdx.x;
  const uint16_t* wt[2] = {layer_tensor<C_W1, A_W1>(p.weights, l) + (size_t)f0 * kHidden,
                           layer_tensor<C_W3, A_W3>(p.weights, l) + (size_t)f0 * kHidden};
  gemm_tiles_staged<2, 4>(wt, p, layer_tensor<C_FFNNORM, A_FFNNORM>(p.weights, l), sh);
  __syncthreads();
  uint16_t* g = b_g(p);
  for (int e = threadIdx.x; e < 16 * p.rows; e += kGT) {
    const int i = e & 15, m = e >> 4;
    const float a = round_bf16(gemm_at<4>(sh, 0, i, m));
    const float b = round_bf16(gemm_at<4>(sh, 1, i, m));
    g[(size_t)m * kFfn + f0 + i] = f32_to_bf16(silu_bf16(a) * b);
  }
}

// q / k / v rows of one head (block b: query head b < 16, key head b - 16,
// value head b - 24), then per row: q and k through QK-RMSNorm + RoPE at the
// row's position (norm_rope_lane), k and v appended to the row's sequence
// cache at that position, q kept for the attention.
__global__ void __launch_bounds__(kGT) k_bx_qkv(BatchParams p, int l) {
  __shared__ GemmLdsStaged sh;
  const int b = blockIdx.x;
  const int row0 = b < 16 ? 64 * b : b < 24 ? kHidden + 64 * (b - 16) : kHidden + 512 + 64 * (b - 24);
  const uint16_t* wq = attn_tensor<A_Q>(p.weights, l) + (size_t)row0 * kHidden;
  const uint16_t* wt[4] = {wq, wq + 16 * kHidden, wq + 32 * kHidden, wq + 48 * kHidden};
  const int w = wave_id(), d = lane_id();
  // The epilogue's operands for the wave's first row: the row and the QK
  // norm weights before the weights, the RoPE row once they are requested.
  const float gq = bf16_to_f32(attn_tensor<A_QLN>(p.weights, l)[d]);
  const float gk = bf16_to_f32(attn_tensor<A_KLN>(p.weights, l)[d]);
  const RowInfo r0 = b_row(p, min(w, p.rows - 1));
  uint16_t cs0 = 0, sn0 = 0;
  const auto rope0 = [&] {
    if (b < 24 && r0.pos >= 0 && r0.pos < p.capacity) {
      cs0 = p.rope[(size_t)r0.pos * 2 * kHeadDim + d];
      sn0 = p.rope[(size_t)r0.pos * 2 * kHeadDim + kHeadDim + d];
    }
  };
  gemm_tiles_staged<4, 2>(wt, p, attn_tensor<A_OPNORM>(p.weights, l), sh, rope0);
  __syncthreads();
  const int att = l - conv_before(l);
  for (int m = w; m < p.rows; m += kGW) {
    const RowInfo r = m == w ? r0 : b_row(p, m);
    if (r.pos < 0 || r.pos >= p.capacity) continue;
    const float raw = round_bf16(gemm_at<2>(sh, d >> 4, d & 15, m));
    if (b < 24) {
      const float cs = bf16_to_f32(m == w ? cs0 : p.rope[(size_t)r.pos * 2 * kHeadDim + d]);
      const float sn = bf16_to_f32(m == w ? sn0 : p.rope[(size_t)r.pos * 2 * kHeadDim + kHeadDim + d]);
      const float o = norm_rope_lane(raw, b < 16 ? gq : gk, cs, sn);
      if (b < 16) b_q(p)[(size_t)m * kHidden + 64 * b + d] = f32_to_bf16(o);
      else p.key_cache[kv_head_base(p, r.seq, att, b - 16) + (size_t)r.pos * kHeadDim + d] = f32_to_bf16(o);
    } else {
      p.value_cache[kv_head_base(p, r.seq, att, b - 24) + (size_t)r.pos * kHeadDim + d] = f32_to_bf16(raw);
    }
  }
}

// Attention of row m (block x) for KV head g (block y): its two query heads
// over positions [0, pos] of its sequence's cache, which k_bx_qkv has filled
// for this row and the chunk's earlier rows (causal inside the batch).
__global__ void __launch_bounds__(kAT) k_bx_attention(BatchParams p, int l) {
  __shared__ AttnSharedT<kAT> sh;
  const int m = blockIdx.x, g = blockIdx.y;
  const RowInfo r = b_row(p, m);
  if (r.pos < 0 || r.pos >= p.capacity) return;
  const int att = l - conv_before(l);
  const uint16_t* keys = p.key_cache + kv_head_base(p, r.seq, att, g);
  const uint16_t* values = p.value_cache + kv_head_base(p, r.seq, att, g);
  const int t = threadIdx.x;
  if (t < 2 * kHeadDim) sh.q[t / kHeadDim][t % kHeadDim] = bf16_to_f32(b_q(p)[(size_t)m * kHidden + 128 * g + t]);
  else if (t < 3 * kHeadDim) sh.k_new[t - 128] = bf16_to_f32(keys[(size_t)r.pos * kHeadDim + t - 128]);
  else sh.v_new[t - 192] = bf16_to_f32(values[(size_t)r.pos * kHeadDim + t - 192]);
  __syncthreads();
  attn_core_t<kAT>(ContiguousRows{keys, values}, r.pos, sh);
  if (t < 2 * kHeadDim) b_y(p)[(size_t)m * kHidden + 128 * g + t] = f32_to_bf16(sh.out[t]);
}

// Head (tied embedding table) in at most kHeadBlocks blocks: a block stages
// the normed rows in LDS once (rows padded to 2,064 bytes, so the lanes'
// 16-byte reads hit distinct banks), then takes rounds of kHeadChunk table
// rows (block b: rounds b, b + grid, ...), each of its 8 waves one 16-row
// tile as one K = 1,024 MFMA chain per batch tile, the next round's rows
// requested while the candidates of this one are formed. The BF16-rounded
// logits keep a running first maximum per batch row
// (kernels/x8/x8_core.cc:126-163); the block's winners go to the candidate
// list. (One block per 64 table rows re-read every batch row's activations
// through the vector cache for each of them: 512 MB per step at 64 rows.)
constexpr int kHeadChunk = kGW * 16;   // table rows per round
constexpr int kHeadBlocks = 256;
struct HeadLds {
  alignas(16) char x[kRowsMax][kXRow];
  float ss[kRowsMax][2];
  float red_v[kGW][kRowsMax];
  int red_i[kGW][kRowsMax];
};
__global__ void __launch_bounds__(kGT) k_bx_head(BatchParams p) {
  __shared__ HeadLds sh;
  constexpr int kSteps = kHidden / 32;
  const int w = wave_id(), l = lane_id();
  const int rows = p.rows, mt = (rows + 15) / 16;
  const int chunks = (p.vocab + kHeadChunk - 1) / kHeadChunk;
  bf16x8_t a[kSteps];
  // the wave's 16 rows of round c (an empty descriptor past the table)
  const auto load_a = [&](int c) {
    const int r0 = c * kHeadChunk + 16 * w;
    const Rsrc ra = rsrc(p.embedding + (size_t)min(r0, p.vocab - 16) * kHidden, r0 < p.vocab ? 16 * kHidden * 2 : 0);
    const int a_off = ((l & 15) * kHidden + 8 * (l >> 4)) * 2;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) a[st] = load_bf16x8(ra, a_off, 64 * st);
  };
  {
    // the final norm of the batch rows into LDS (RowStage), behind the first
    // round's table rows
    const bool fold = rows <= kFoldRows;
    RowStage stage;
    stage.load(fold ? b_x(p) : b_xn(p), final_norm(p.weights), rows, mt);
    load_a(blockIdx.x);
    stage.store(sh.x, sh.ss, mt, fold);
  }
  lds_barrier();
  float bv[kMT];
  int bi[kMT];
#pragma unroll
  for (int m = 0; m < kMT; ++m) {
    bv[m] = -INFINITY;
    bi[m] = 0x7fffffff;
  }
  for (int c = blockIdx.x; c < chunks; c += gridDim.x) {
    const int r0 = c * kHeadChunk + 16 * w;
    f32x4_t acc[kMT];
#pragma unroll
    for (int m = 0; m < kMT; ++m) {
      acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      if (m < mt) {
        const char* xr = &sh.x[16 * m + (l & 15)][16 * (l >> 4)];
#pragma unroll
        for (int st = 0; st < kSteps; ++st)
          acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[st], *reinterpret_cast<const bf16x8_t*>(xr + 64 * st),
                                                           acc[m], 0, 0, 0);
      }
    }
    if (c + (int)gridDim.x < chunks) load_a(c + gridDim.x);
    // lane l holds table rows r0 + 4 (l / 16) + e of batch row 16m + l % 16
    if (r0 < p.vocab) {
#pragma unroll
      for (int m = 0; m < kMT; ++m) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = round_bf16(acc[m][e]);
          const int row = r0 + 4 * (l >> 4) + e;
          if (better(v, row, bv[m], bi[m])) { bv[m] = v; bi[m] = row; }
        }
      }
    }
  }
  // the four lane groups' winners per batch row, then the waves' in order
#pragma unroll
  for (int m = 0; m < kMT; ++m) {
#pragma unroll
    for (int o = 16; o < kWave; o <<= 1) {
      const float ov = __shfl_xor(bv[m], o, kWave);
      const int oi = __shfl_xor(bi[m], o, kWave);
      if (better(ov, oi, bv[m], bi[m])) { bv[m] = ov; bi[m] = oi; }
    }
    if (l < 16) {
      sh.red_v[w][16 * m + l] = bv[m];
      sh.red_i[w][16 * m + l] = bi[m];
    }
  }
  lds_barrier();
  const int t = threadIdx.x;
  if (t >= rows) return;
  float v = sh.red_v[0][t];
  int i = sh.red_i[0][t];
#pragma unroll
  for (int g = 1; g < kGW; ++g)
    if (better(sh.red_v[g][t], sh.red_i[g][t], v, i)) { v = sh.red_v[g][t]; i = sh.red_i[g][t]; }
  b_cand(p)[(size_t)blockIdx.x * kRowsMax + t] = (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)i << 32);
}

// Row m's token: the first maximum over the head blocks' candidates, into
// out[m]; in decode mode also the next input of its sequence.
__global__ void __launch_bounds__(kAT) k_bx_pick(BatchParams p, int blocks, int32_t* out) {
  __shared__ float rv[kAT / kWave];
  __shared__ int ri[kAT / kWave];
  const int m = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = threadIdx.x; b < blocks; b += kAT) {
    const uint64_t c = b_cand(p)[(size_t)b * kRowsMax + m];
    const float v = __uint_as_float((uint32_t)c);
    const int i = (int)(c >> 32);
    if (better(v, i, bv, bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane_id() == 0) { rv[wave_id()] = bv; ri[wave_id()] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = rv[0];
    int i = ri[0];
    for (int w = 1; w < kAT / kWave; ++w)
      if (better(rv[w], ri[w], v, i)) { v = rv[w]; i = ri[w]; }
    out[m] = i;
  }
}

// (status: 0 keeps the status word, which a persistent launch of the same
// call has already cleared and may have flagged)
__global__ void k_bx_status_clear(BatchParams p, int status) {
  if (threadIdx.x == 0 && status) *b_status(p) = 0;
  if (threadIdx.x < kHidden / 16) b_count(p)[threadIdx.x] = 0;
}

// The host's row table (or decode start positions) into the workspace, from
// the kernel's own arguments: stream ordered, with no host buffer that must
// outlive the call.
struct RowTable {
  RowInfo row[kRowsMax];
};
struct StartTable {
  int32_t pos[kRowsMax];
};
__global__ void k_bx_set_rows(BatchParams p, RowTable t) {
  if ((int)threadIdx.x < p.rows) reinterpret_cast<RowInfo*>(p.ws + kBwRows)[threadIdx.x] = t.row[threadIdx.x];
}
__global__ void k_bx_set_starts(BatchParams p, StartTable t) {
  if ((int)threadIdx.x < p.seqs) reinterpret_cast<int32_t*>(p.ws + kBwStart)[threadIdx.x] = t.pos[threadIdx.x];
}

// Y[m][n] = bf16(W[n] . X[m]) for the batch linear test entry point.
template <int K>
__global__ void __launch_bounds__(kGT) k_bx_linear(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows, int n) {
  __shared__ GemmLds sh;
  const int n0 = 16 * blockIdx.x;
  const uint16_t* wt[1] = {w + (size_t)n0 * K};
  gemm_tiles<1, kGW, K>(wt, x, rows, sh);
  __syncthreads();
  for (int e = threadIdx.x; e < 16 * rows; e += kGT) {
    const int i = e & 15, m = e >> 4;
    y[(size_t)m * n + n0 + i] = f32_to_bf16(gemm_at<kGW>(sh, 0, i, m));
  }
}

// ------------------------------------------------------------------ host

uint16_t* b_g_host(const BatchParams& p) { return reinterpret_cast<uint16_t*>(p.ws + kBwG); }

// (decode_tokens != nullptr: a decode step, whose row table the embedding
// kernel writes: sequence m consumes decode_tokens[m] at its start + step.)
int launch_pass(const BatchParams& p, bool select, int32_t* tokens_out, uint16_t* hidden_out, hipStream_t s,
                const int32_t* decode_tokens = nullptr, int step = 0) {
  k_bx_embed<<<p.rows, kWave, 0, s>>>(p, decode_tokens, step);
  uint16_t* x = reinterpret_cast<uint16_t*>(p.ws + kBwX);
  uint16_t* y = reinterpret_cast<uint16_t*>(p.ws + kBwY);
  uint16_t* xn = reinterpret_cast<uint16_t*>(p.ws + kBwXn);
  // above kFoldRows rows the norms run once per phase instead of in every
  // block of the product that reads them
  const bool fold = p.rows <= kFoldRows;
  for (int l = 0; l < kLayers; ++l) {
    const bool attn = is_attn(l);
    const uint16_t* base = p.weights + layer_off(l);
    const uint16_t* op_norm = base + slot_off(attn, attn ? (int)A_OPNORM : (int)C_OPNORM);
    const uint16_t* ffn_norm = base + slot_off(attn, attn ? (int)A_FFNNORM : (int)C_FFNNORM);
    if (!fold) k_bx_norm<<<p.rows, 2 * kWave, 0, s>>>(p, x, op_norm, xn);
    const uint16_t* w_out = base + slot_off(attn, attn ? (int)A_O : (int)C_OUT);
    const uint16_t* w2 = base + slot_off(attn, attn ? (int)A_W2 : (int)C_W2);
    if (attn) {
      k_bx_qkv<<<32, kGT, 0, s>>>(p, l);
      k_bx_attention<<<dim3(p.rows, kKvHeads), kAT, 0, s>>>(p, l);
    } else {
      k_bx_conv<<<kHidden / 8, kGT, 0, s>>>(p, l);
    }
    k_bx_residual<kHidden, kResSplit><<<kResSplit * kHidden / 16, kGT, 0, s>>>(p, w_out, y);
    if (!fold) k_bx_norm<<<p.rows, 2 * kWave, 0, s>>>(p, x, ffn_norm, xn);
    k_bx_silu<<<kFfn / 16, kGT, 0, s>>>(p, l);
    k_bx_residual<kFfn, kResSplit><<<kResSplit * kHidden / 16, kGT, 0, s>>>(p, w2, b_g_host(p));
  }
  int rc = check_launch("batch pass");
  if (rc != LFM25_OK) return rc;
  if (hidden_out != nullptr &&
      hipMemcpyAsync(hidden_out, x, (size_t)p.rows * kHidden * 2, hipMemcpyDeviceToDevice, s) != hipSuccess)
    return set_error(LFM25_EDEVICE, "batch pass: hidden copy failed");
  if (select) {
    const int blocks = std::min(kHeadBlocks, (p.vocab + kHeadChunk - 1) / kHeadChunk);
    if (!fold) k_bx_norm<<<p.rows, 2 * kWave, 0, s>>>(p, x, p.weights + layer_off(kLayers), xn);
    k_bx_head<<<blocks, kGT, 0, s>>>(p);
    k_bx_pick<<<p.rows, kAT, 0, s>>>(p, blocks, tokens_out);
    rc = check_launch("batch head");
  }
  return rc;
}

int check_batch(const lfm25_batch* b) {
  LFM25_REQUIRE(b != nullptr, "batch: null descriptor");
  LFM25_REQUIRE(b->weights && b->embedding && b->rope && b->conv_state && b->key_cache && b->value_cache &&
                    b->workspace,
                "batch: null buffer");
  LFM25_REQUIRE(b->sequences >= 1 && b->sequences <= kRowsMax, "batch: sequences must be in [1, %d], got %d",
                kRowsMax, b->sequences);
  LFM25_REQUIRE(b->capacity >= 1 && b->capacity <= LFM25_MAX_CAPACITY, "batch: capacity must be in [1, %d]",
                LFM25_MAX_CAPACITY);
  LFM25_REQUIRE(b->vocab >= 16 && b->vocab % 16 == 0 && b->vocab <= LFM25_VOCAB,
                "batch: vocab must be a multiple of 16 in [16, %d], got %d", LFM25_VOCAB, b->vocab);
  LFM25_REQUIRE(aligned16(b->weights) && aligned16(b->embedding) && aligned16(b->workspace),
                "batch: weights, embedding and workspace must be 16-byte aligned");
  return LFM25_OK;
}

BatchParams make_batch_params(const lfm25_batch* b, int rows) {
  BatchParams p{};
  p.weights = b->weights;
  p.embedding = b->embedding;
  p.rope = b->rope;
  p.conv_state = b->conv_state;
  p.key_cache = b->key_cache;
  p.value_cache = b->value_cache;
  p.ws = static_cast<char*>(b->workspace);
  p.rows = rows;
  p.seqs = b->sequences;
  p.capacity = b->capacity;
  p.vocab = b->vocab;
  return p;
}

}  // namespace
}  // namespace lfm25

using namespace lfm25;

extern "C" {

size_t lfm25_batch_workspace_bytes(void) { return kBwPersist + batch_persistent_bytes(); }

int lfm25_batch_pass(const lfm25_batch* b, const int32_t* rows, int32_t n_rows, int32_t select,
                     int32_t* tokens_out, uint16_t* hidden_out, lfm25_stream_t stream) {
  int rc = check_batch(b);
  if (rc != LFM25_OK) return rc;
  LFM25_REQUIRE(rows != nullptr && n_rows >= 1 && n_rows <= kRowsMax, "batch pass: rows must be 1..%d, got %d",
                kRowsMax, n_rows);
  LFM25_REQUIRE(!select || tokens_out != nullptr, "batch pass: select needs tokens_out");
  RowTable table{};
  std::vector<char> seen(b->sequences, 0);
  for (int m = 0; m < n_rows; ++m) {
    const int tok = rows[3 * m], seq = rows[3 * m + 1], pos = rows[3 * m + 2];
    LFM25_REQUIRE(tok >= 0 && tok < b->vocab, "batch pass: row %d token %d outside the vocabulary", m, tok);
    LFM25_REQUIRE(seq >= 0 && seq < b->sequences, "batch pass: row %d sequence %d out of range", m, seq);
    LFM25_REQUIRE(pos >= 0 && pos < b->capacity, "batch pass: row %d position %d outside the capacity %d", m, pos,
                  b->capacity);
    const bool cont = m > 0 && rows[3 * (m - 1) + 1] == seq;
    if (cont) {
      LFM25_REQUIRE(pos == rows[3 * (m - 1) + 2] + 1, "batch pass: row %d does not follow row %d's position", m,
                    m - 1);
    } else {
      LFM25_REQUIRE(!seen[seq], "batch pass: sequence %d appears in two separate runs of rows", seq);
      seen[seq] = 1;
    }
    table.row[m] = RowInfo{tok, seq, pos, cont ? (table.row[m - 1].chunk & 0xffff) + 1 : 0};
    if (m + 1 == n_rows || rows[3 * (m + 1) + 1] != seq) table.row[m].chunk |= kLastRow;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const BatchParams p = make_batch_params(b, n_rows);
  k_bx_set_rows<<<1, kRowsMax, 0, s>>>(p, table);
  k_bx_status_clear<<<1, kHidden / 16, 0, s>>>(p, 1);
  return launch_pass(p, select != 0, tokens_out, hidden_out, s);
}

int lfm25_batch_decode(const lfm25_batch* b, const int32_t* tokens_in, const int32_t* positions, int32_t n_steps,
                       int32_t* tokens_out, lfm25_stream_t stream) {
  int rc = check_batch(b);
  if (rc != LFM25_OK) return rc;
  LFM25_REQUIRE(tokens_in != nullptr && positions != nullptr && tokens_out != nullptr,
                "batch decode: null argument");
  LFM25_REQUIRE(n_steps >= 1, "batch decode: n_steps must be positive");
  for (int q = 0; q < b->sequences; ++q)
    LFM25_REQUIRE(positions[q] >= 0 && positions[q] + n_steps <= b->capacity,
                  "batch decode: sequence %d at position %d cannot take %d steps within capacity %d", q,
                  positions[q], n_steps, b->capacity);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // B = 2, 4, 8 within the split attention's positions: one or two
  // persistent launches for the whole call; B = 16: one for the steps below
  // 256 positions, the batched pass for the rest (both keep the same KV and
  // conv state)
  int done = 0;
  rc = batch_decode_persistent(b, static_cast<char*>(b->workspace) + kBwPersist,
                               static_cast<int32_t*>(b->workspace) + kBwCtl / 4, tokens_in, positions, n_steps,
                               tokens_out, nullptr, s, true, &done);
  if (rc != kBatchNotPersistent && (rc != LFM25_OK || done == n_steps)) return rc;
  const BatchParams p = make_batch_params(b, b->sequences);
  StartTable starts{};
  for (int q = 0; q < b->sequences; ++q) starts.pos[q] = positions[q];
  k_bx_set_starts<<<1, kRowsMax, 0, s>>>(p, starts);
  k_bx_status_clear<<<1, kHidden / 16, 0, s>>>(p, done == 0);
  for (int i = done; i < n_steps; ++i) {
    const int32_t* in = i == 0 ? tokens_in : tokens_out + (size_t)(i - 1) * b->sequences;
    rc = launch_pass(p, true, tokens_out + (size_t)i * b->sequences, nullptr, s, in, i);
    if (rc != LFM25_OK) return rc;
  }
  return LFM25_OK;
}

int lfm25_batch_decode_hidden(const lfm25_batch* b, const int32_t* tokens_in, const int32_t* positions,
                              int32_t n_steps, int32_t* tokens_out, uint16_t* hidden_out, lfm25_stream_t stream) {
  int rc = check_batch(b);
  if (rc != LFM25_OK) return rc;
  LFM25_REQUIRE(tokens_in != nullptr && positions != nullptr && tokens_out != nullptr && hidden_out != nullptr,
                "batch decode (hidden): null argument");
  LFM25_REQUIRE((reinterpret_cast<uintptr_t>(hidden_out) & 3u) == 0, "batch decode (hidden): hidden_out must be 4-byte aligned");
  LFM25_REQUIRE(n_steps >= 1, "batch decode (hidden): n_steps must be positive");
  for (int q = 0; q < b->sequences; ++q)
    LFM25_REQUIRE(positions[q] >= 0 && positions[q] + n_steps <= b->capacity,
                  "batch decode (hidden): sequence %d at position %d cannot take %d steps within capacity %d", q,
                  positions[q], n_steps, b->capacity);
  int done = 0;
  rc = batch_decode_persistent(b, static_cast<char*>(b->workspace) + kBwPersist,
                               static_cast<int32_t*>(b->workspace) + kBwCtl / 4, tokens_in, positions, n_steps,
                               tokens_out, hidden_out, reinterpret_cast<hipStream_t>(stream), false, &done);
  if (rc == kBatchNotPersistent)
    return set_error(LFM25_EINVAL, "batch decode (hidden): the persistent path serves 2, 4 or 8 sequences whose "
                     "positions stay below 256 x 16 / sequences, or 16 below 256 (and LFM25_BATCH_PERSISTENT is "
                     "not 0)");
  return rc;
}

int lfm25_batch_linear(const uint16_t* x, const uint16_t* w, uint16_t* y, int32_t rows, int32_t n, int32_t k,
                       lfm25_stream_t stream) {
  LFM25_REQUIRE(x && w && y, "batch linear: null pointer");
  LFM25_REQUIRE(rows >= 1 && rows <= kRowsMax, "batch linear: rows must be in [1, %d], got %d", kRowsMax, rows);
  LFM25_REQUIRE(n >= 16 && n % 16 == 0, "batch linear: n must be a positive multiple of 16, got %d", n);
  LFM25_REQUIRE(k == kHidden || k == kFfn, "batch linear: k must be %d or %d, got %d", kHidden, kFfn, k);
  LFM25_REQUIRE(aligned16(x) && aligned16(w), "batch linear: x and w must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (k == kHidden) k_bx_linear<kHidden><<<n / 16, kGT, 0, s>>>(x, w, y, rows, n);
  else k_bx_linear<kFfn><<<n / 16, kGT, 0, s>>>(x, w, y, rows, n);
  return check_launch("batch linear");
}

}  // extern "C"
