// B independent sequences through the persistent decode in lockstep: the
// batch-1 step's grid, XCD layout, two alternating CU groups and tagged
// exchanges (lfm25_step.h), with every layer's weights held in registers
// once for all B rows. Serves lfm25_batch_decode for B = 2, 4, 8 and 16 (the
// reference's batched pass reads each weight object once for all its rows,
// experiments/lfm25_x8.py:341-416 and dot4 in kernels/x8/x8p_core.cc:43-60;
// independent sequences extend it).
//
// The layer products and the vocabulary head run on the matrix cores, one
// column per sequence, so the weights in registers serve every sequence in
// one instruction stream; norms, the conv gate, attention, residual sums and
// every rounding point are the batch-1 step's per row. The products' FP32
// summation orders are the matrix cores' (K split over the block's waves,
// then summed in a fixed tree), not the batch-1 step's lane reductions, so a
// sequence agrees with the batch-1 decode of it within FP32 summation order.
// Below 256 positions a sequence attends in single blocks; past that, its
// 16 / B blocks split its cache (block i owns passes i, i + 16/B, ... of 64
// positions). B = 16 runs below 256 positions only: one block of a sequence
// per XCD attends for both query heads.
//
// Exchange buffers hold one copy per sequence: a consumer polls the words of
// every sequence with the loads all in flight, and each tag covers all B
// rows of an exchange. Tags run 1 .. 65535 (never 0, the zeroed workspace's
// value), so a never-written word can not pass a poll.
#pragma once
#include "lfm25_step.h"

namespace lfm25 {

constexpr int kBSeqMax = 16;
constexpr int kConvSeqElems = LFM25_CONV_LAYERS * kHidden * kConvTaps;  // one sequence's conv states

// Byte offsets of the persistent region of the batch workspace for kB
// sequences (every region starts on a cache line).
template <int kB>
struct BWs {
  static constexpr size_t ctl = 0;                                             // int32 [64]: [0] epoch, [1] step
  static constexpr size_t lh1 = 256;                                           // u32 [8][kB][1024]: h after R2
  static constexpr size_t lh0 = lh1 + 4ull * kXcds * kB * kHidden;             // u32 [8][kB][1024]: h after R1
  static constexpr size_t ly = lh0 + 4ull * kXcds * kB * kHidden;              // u32 [8][kB][128]
  static constexpr size_t lq = ly + 4ull * kXcds * kB * kLyWords;              // u32 [8][kB][256]
  static constexpr size_t lg = lq + 4ull * kXcds * kB * kLqWords;              // u32 [8][kB][384]
  static constexpr size_t lw = lg + 4ull * kXcds * kB * kLgWords;              // u64 [8][kB][64]
  static constexpr size_t gp = lw + 8ull * kXcds * kB * kLwWords;              // u64 [2][16][8][kB][64]
  static constexpr size_t gw = gp + 8ull * 2 * kGroupBlocks * kXcds * kB * kResRows;  // u64 [kB][16][8]
  static constexpr size_t ls = gw + 8ull * kB * kGroupBlocks * kXcds;          // u64 [8][16][4]
  static constexpr size_t lc = ls + 8ull * kXcds * kLsWords;                   // u64 [8][16][128]
  static constexpr size_t lss = lc + 8ull * kXcds * kLcWords;                  // u64 [2][8][kB][16]: sums of squares
  static constexpr size_t bytes = lss + 8ull * 2 * kXcds * kB * kGroupBlocks;
  static_assert(lh0 % 128 == 0 && ly % 128 == 0 && lq % 128 == 0 && lg % 128 == 0 && lw % 128 == 0 &&
                    gp % 128 == 0 && gw % 128 == 0 && ls % 128 == 0 && lc % 128 == 0 && lss % 128 == 0,
                "every exchange region starts on a cache line");
};
constexpr size_t kBWsBytes = BWs<kBSeqMax>::bytes;  // the largest layout, what the workspace reserves
constexpr int kBCtlEpoch = 0;
constexpr int kBCtlStep = 1;

struct BDecodeParams {
  const uint16_t* weights;
  const uint16_t* embedding;
  const uint16_t* rope;
  uint16_t* conv_state;   // [kB][8][1024][3]
  uint16_t* key_cache;    // [kB][6][8][capacity][64]
  uint16_t* value_cache;
  char* ws;               // the persistent region
  int32_t* status;        // the batch workspace's status word (lfm25_batch_decode's)
  const int32_t* tokens_in;  // [kB]
  int32_t* tokens_out;       // [n_steps][kB]
  uint16_t* hidden_out;      // [n_steps][kB][1024] pre-final-norm states, or null
  int pos0[kBSeqMax];        // position of each sequence at step 0
  int n_steps, capacity, vocab;
};

// Epoch tags 1 .. 65535 of one step, in exchange order.
struct BTags {
  uint32_t base;
  int next = 0;
  __device__ uint32_t take() { return (uint32_t)((base + (uint32_t)(++next)) % 0xffffu) + 1u; }
  __device__ void skip(int n) { next += n; }
  __device__ uint32_t last() const { return (uint32_t)((base + (uint32_t)next) % 0xffffu) + 1u; }
};

// A gathered vector of one sequence in LDS: 512 words of BF16 pairs, rows
// 2,064 bytes apart so that the lanes of a matrix-core step, which read the
// same K range of different sequences, hit different banks.
constexpr int kBVecWords = kNormWords + 4;
typedef uint32_t BVec[kBVecWords];
// Vector buffers: two alternate between the phases; B = 16 has room for one.
// One suffices for the data: each gather writes only words that the waves
// writing them have already read in the phase before (h: a wave's own words;
// y and g: wave w writes words [64w, 64w + 64), which only wave w's P1 / P3
// read), and P2 / P4, which read other waves' words, follow the gathers'
// barrier and finish before bpublish's.
template <int kB> constexpr int kBVecBufs = kB > 8 ? 1 : 2;
template <int kB>
__device__ __forceinline__ int bnext_buf(int buf) { return kBVecBufs<kB> == 1 ? 0 : buf ^ 1; }
// Sequences per wave in the per-sequence phases (R, publish, picks): wave w
// takes sequences w, w + 8, ...
template <int kB> constexpr int kBSeqPerWave = kB > 8 ? kB / 8 : 1;

// The layer products run on the matrix cores (v_mfma_f32_16x16x32_bf16): a
// tile of 16 weight rows x 32 K as the first operand, the gathered vectors of
// up to 16 sequences as the second, K split over the block's waves. Each
// wave leaves its 16 x 16 partial tiles in LDS, rows [tile][16], column =
// sequence, and the sums over waves follow in a fixed order.
constexpr int kMpRows = 48;  // up to three tiles (P3's)
constexpr int kMpCols = 16;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The shared memory of one block.
template <int kB>
struct BShared {
  alignas(16) BVec vec[kBVecBufs<kB>][kB];      // gathered (normed) vectors
  // (a block barrier separates layer 0's norm, the last reader of raw, from
  // the first product's tiles)
  alignas(16) union {
    float mp[kStepWaves][kMpRows][kMpCols];     // every wave's partial product tiles
    uint32_t raw[kB][kNormWords];               // layer 0: the embedding rows before the norm
  };
  float ss[kB][kStepWaves];                     // their sums of squares, per gathering wave
  float hres[kB][kResRows];                     // the block's residual rows of every sequence
  // the next attention layer's cached keys and values of wave w, pass i:
  // kvl[i][w][0][4l ..] the 16 key bytes of lane l, kvl[i][w][1][64e + l]
  // value word e of lane l (the registers of AttnKV, copied by the DMA)
  alignas(16) uint32_t kvl[kAttnPrefetch][kStepWaves][2][4 * kWave];
  AttnSplitShared attn;
  float red_v[kB][kStepWaves];
  int red_i[kB][kStepWaves];
  int tok[kB];                                  // the step's tokens (group 0)
#ifdef LFM25_TRACE
  uint64_t* trace;                              // the timing trace (trace builds)
  int trace_steps;
#endif
};

template <int kB>
struct BBufs {
  char* ws;
  __device__ char* base() const { return as_global(ws); }
  __device__ uint32_t* lh1(int x) const { return reinterpret_cast<uint32_t*>(base() + BWs<kB>::lh1) + (size_t)x * kB * kHidden; }
  __device__ uint32_t* lh0(int x) const { return reinterpret_cast<uint32_t*>(base() + BWs<kB>::lh0) + (size_t)x * kB * kHidden; }
  __device__ uint32_t* ly(int x) const { return reinterpret_cast<uint32_t*>(base() + BWs<kB>::ly) + x * kB * kLyWords; }
  __device__ uint32_t* lq(int x) const { return reinterpret_cast<uint32_t*>(base() + BWs<kB>::lq) + x * kB * kLqWords; }
  __device__ uint32_t* lg(int x) const { return reinterpret_cast<uint32_t*>(base() + BWs<kB>::lg) + x * kB * kLgWords; }
  __device__ uint64_t* lw(int x) const { return reinterpret_cast<uint64_t*>(base() + BWs<kB>::lw) + x * kB * kLwWords; }
  __device__ uint64_t* gp(int k) const {
    return reinterpret_cast<uint64_t*>(base() + BWs<kB>::gp) + (size_t)k * kGroupBlocks * kXcds * kB * kResRows;
  }
  __device__ uint64_t* gw() const { return reinterpret_cast<uint64_t*>(base() + BWs<kB>::gw); }
  __device__ uint64_t* ls(int x) const { return reinterpret_cast<uint64_t*>(base() + BWs<kB>::ls) + x * kLsWords; }
  __device__ uint64_t* lc(int x) const { return reinterpret_cast<uint64_t*>(base() + BWs<kB>::lc) + x * kLcWords; }
  // block jj's sum of squares of its 64 rows of h of sequence s: lss(k, x)[16 s + jj]
  // (k = 0: the h after R1 in lh0, k = 1: after R2 in lh1)
  __device__ uint64_t* lss(int k, int x) const {
    return reinterpret_cast<uint64_t*>(base() + BWs<kB>::lss) + ((size_t)k * kXcds + x) * kB * kGroupBlocks;
  }
};

// ------------------------------------------------------------------ polls of kB rows

// kB 8-byte loads at base + voff + s * stride (s < kB), all in flight, one
// wait (the XCD-local form: non-temporal loads through the XCD's L2).
template <int kB>
__device__ __forceinline__ void nt_load64_rows(const void* base, uint32_t voff, uint32_t stride, uint64_t* w) {
  static_assert(kB == 2 || kB == 4 || kB == 8 || kB == 16, "two, four, eight or sixteen rows");
  if constexpr (kB == 2) {
    asm volatile("global_load_dwordx2 %0, %2, %4 nt\n\t"
                 "global_load_dwordx2 %1, %3, %4 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]) : "v"(voff), "v"(voff + stride), "s"(base) : "memory");
  } else if constexpr (kB == 4) {
    asm volatile("global_load_dwordx2 %0, %4, %8 nt\n\t"
                 "global_load_dwordx2 %1, %5, %8 nt\n\t"
                 "global_load_dwordx2 %2, %6, %8 nt\n\t"
                 "global_load_dwordx2 %3, %7, %8 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
                 : "v"(voff), "v"(voff + stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride), "s"(base)
                 : "memory");
  } else if constexpr (kB == 16) {
    asm volatile("global_load_dwordx2 %0, %16, %32 nt\n\t"
                 "global_load_dwordx2 %1, %17, %32 nt\n\t"
                 "global_load_dwordx2 %2, %18, %32 nt\n\t"
                 "global_load_dwordx2 %3, %19, %32 nt\n\t"
                 "global_load_dwordx2 %4, %20, %32 nt\n\t"
                 "global_load_dwordx2 %5, %21, %32 nt\n\t"
                 "global_load_dwordx2 %6, %22, %32 nt\n\t"
                 "global_load_dwordx2 %7, %23, %32 nt\n\t"
                 "global_load_dwordx2 %8, %24, %32 nt\n\t"
                 "global_load_dwordx2 %9, %25, %32 nt\n\t"
                 "global_load_dwordx2 %10, %26, %32 nt\n\t"
                 "global_load_dwordx2 %11, %27, %32 nt\n\t"
                 "global_load_dwordx2 %12, %28, %32 nt\n\t"
                 "global_load_dwordx2 %13, %29, %32 nt\n\t"
                 "global_load_dwordx2 %14, %30, %32 nt\n\t"
                 "global_load_dwordx2 %15, %31, %32 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]),
                   "=&v"(w[7]), "=&v"(w[8]), "=&v"(w[9]), "=&v"(w[10]), "=&v"(w[11]), "=&v"(w[12]), "=&v"(w[13]),
                   "=&v"(w[14]), "=&v"(w[15])
                 : "v"(voff), "v"(voff + 1 * stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride),
                   "v"(voff + 4 * stride), "v"(voff + 5 * stride), "v"(voff + 6 * stride), "v"(voff + 7 * stride),
                   "v"(voff + 8 * stride), "v"(voff + 9 * stride), "v"(voff + 10 * stride), "v"(voff + 11 * stride),
                   "v"(voff + 12 * stride), "v"(voff + 13 * stride), "v"(voff + 14 * stride), "v"(voff + 15 * stride),
                   "s"(base)
                 : "memory");
  } else {
    asm volatile("global_load_dwordx2 %0, %8, %16 nt\n\t"
                 "global_load_dwordx2 %1, %9, %16 nt\n\t"
                 "global_load_dwordx2 %2, %10, %16 nt\n\t"
                 "global_load_dwordx2 %3, %11, %16 nt\n\t"
                 "global_load_dwordx2 %4, %12, %16 nt\n\t"
                 "global_load_dwordx2 %5, %13, %16 nt\n\t"
                 "global_load_dwordx2 %6, %14, %16 nt\n\t"
                 "global_load_dwordx2 %7, %15, %16 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]),
                   "=&v"(w[7])
                 : "v"(voff), "v"(voff + stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride),
                   "v"(voff + 4 * stride), "v"(voff + 5 * stride), "v"(voff + 6 * stride), "v"(voff + 7 * stride),
                   "s"(base)
                 : "memory");
  }
}

template <int kB, bool kLocal>
__device__ __forceinline__ void load64_rows(const void* base, uint32_t voff, uint32_t stride, uint64_t* w) {
  if constexpr (kLocal) {
    nt_load64_rows<kB>(base, voff, stride, w);
  } else {
#pragma unroll
    for (int s = 0; s < kB; ++s) w[s] = coherent_load64(static_cast<const char*>(base) + voff + s * stride);
  }
}

// Poll the first `words` (<= 128) tagged 32-bit words of kB rows of a local
// buffer (row s at src + s * stride bytes; lane l owns words 2l, 2l + 1)
// until every tag equals `tag`.
template <int kB, bool kLocal>
__device__ __forceinline__ void poll_rows(const uint32_t* src, uint32_t stride, int words, uint32_t tag,
                                          uint64_t* w, int32_t* status) {
  const int l = lane_id();
  const bool in = 2 * l < words;
  Poll poll(status);
  while (true) {
    load64_rows<kB, kLocal>(src, 8 * l, stride, w);
    bool ok = true;
#pragma unroll
    for (int s = 0; s < kB; ++s)
      ok = ok && (!in || (tag_ok((uint32_t)w[s], tag) && tag_ok((uint32_t)(w[s] >> 32), tag)));
    if (__all(ok) || !poll.again()) break;
  }
}

// nt_load64_rows plus kQ = ceil(kB / 4) loads at qbase + qoff + 512 i, all in
// one wait.
template <int kB>
__device__ __forceinline__ void nt_load64_rows_q(const void* base, uint32_t voff, uint32_t stride, const void* qbase,
                                                 uint32_t qoff, uint64_t* w, uint64_t* q) {
  static_assert(kB == 2 || kB == 4 || kB == 8 || kB == 16, "two, four, eight or sixteen rows");
  if constexpr (kB == 2) {
    asm volatile("global_load_dwordx2 %0, %3, %6 nt\n\t"
                 "global_load_dwordx2 %1, %4, %6 nt\n\t"
                 "global_load_dwordx2 %2, %5, %7 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(q[0])
                 : "v"(voff), "v"(voff + stride), "v"(qoff), "s"(base), "s"(qbase)
                 : "memory");
  } else if constexpr (kB == 4) {
    asm volatile("global_load_dwordx2 %0, %5, %10 nt\n\t"
                 "global_load_dwordx2 %1, %6, %10 nt\n\t"
                 "global_load_dwordx2 %2, %7, %10 nt\n\t"
                 "global_load_dwordx2 %3, %8, %10 nt\n\t"
                 "global_load_dwordx2 %4, %9, %11 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(q[0])
                 : "v"(voff), "v"(voff + stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride), "v"(qoff),
                   "s"(base), "s"(qbase)
                 : "memory");
  } else if constexpr (kB == 16) {
    asm volatile("global_load_dwordx2 %0, %20, %37 nt\n\t"
                 "global_load_dwordx2 %1, %21, %37 nt\n\t"
                 "global_load_dwordx2 %2, %22, %37 nt\n\t"
                 "global_load_dwordx2 %3, %23, %37 nt\n\t"
                 "global_load_dwordx2 %4, %24, %37 nt\n\t"
                 "global_load_dwordx2 %5, %25, %37 nt\n\t"
                 "global_load_dwordx2 %6, %26, %37 nt\n\t"
                 "global_load_dwordx2 %7, %27, %37 nt\n\t"
                 "global_load_dwordx2 %8, %28, %37 nt\n\t"
                 "global_load_dwordx2 %9, %29, %37 nt\n\t"
                 "global_load_dwordx2 %10, %30, %37 nt\n\t"
                 "global_load_dwordx2 %11, %31, %37 nt\n\t"
                 "global_load_dwordx2 %12, %32, %37 nt\n\t"
                 "global_load_dwordx2 %13, %33, %37 nt\n\t"
                 "global_load_dwordx2 %14, %34, %37 nt\n\t"
                 "global_load_dwordx2 %15, %35, %37 nt\n\t"
                 "global_load_dwordx2 %16, %36, %38 nt\n\t"
                 "global_load_dwordx2 %17, %36, %38 offset:512 nt\n\t"
                 "global_load_dwordx2 %18, %36, %38 offset:1024 nt\n\t"
                 "global_load_dwordx2 %19, %36, %38 offset:1536 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]),
                   "=&v"(w[7]), "=&v"(w[8]), "=&v"(w[9]), "=&v"(w[10]), "=&v"(w[11]), "=&v"(w[12]), "=&v"(w[13]),
                   "=&v"(w[14]), "=&v"(w[15]), "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
                 : "v"(voff), "v"(voff + 1 * stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride),
                   "v"(voff + 4 * stride), "v"(voff + 5 * stride), "v"(voff + 6 * stride), "v"(voff + 7 * stride),
                   "v"(voff + 8 * stride), "v"(voff + 9 * stride), "v"(voff + 10 * stride), "v"(voff + 11 * stride),
                   "v"(voff + 12 * stride), "v"(voff + 13 * stride), "v"(voff + 14 * stride), "v"(voff + 15 * stride),
                   "v"(qoff), "s"(base), "s"(qbase)
                 : "memory");
  } else {
    asm volatile("global_load_dwordx2 %0, %10, %20 nt\n\t"
                 "global_load_dwordx2 %1, %11, %20 nt\n\t"
                 "global_load_dwordx2 %2, %12, %20 nt\n\t"
                 "global_load_dwordx2 %3, %13, %20 nt\n\t"
                 "global_load_dwordx2 %4, %14, %20 nt\n\t"
                 "global_load_dwordx2 %5, %15, %20 nt\n\t"
                 "global_load_dwordx2 %6, %16, %20 nt\n\t"
                 "global_load_dwordx2 %7, %17, %20 nt\n\t"
                 "global_load_dwordx2 %8, %18, %21 nt\n\t"
                 "global_load_dwordx2 %9, %19, %21 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]),
                   "=&v"(w[7]), "=&v"(q[0]), "=&v"(q[1])
                 : "v"(voff), "v"(voff + stride), "v"(voff + 2 * stride), "v"(voff + 3 * stride),
                   "v"(voff + 4 * stride), "v"(voff + 5 * stride), "v"(voff + 6 * stride), "v"(voff + 7 * stride),
                   "v"(qoff), "v"(qoff + 512), "s"(base), "s"(qbase)
                 : "memory");
  }
}

__device__ __forceinline__ uint32_t pair_of(uint64_t w) {
  return ((uint32_t)w & 0xffffu) | ((uint32_t)(w >> 32) << 16);
}

// An FP32 value as two tagged words (low half, high half), and back.
__device__ __forceinline__ uint64_t tagged_f32(float v, uint32_t tag) {
  const uint32_t b = __float_as_uint(v);
  return (uint64_t)((b & 0xffffu) | (tag << 16)) | ((uint64_t)((b >> 16) | (tag << 16)) << 32);
}
__device__ __forceinline__ float f32_of(uint64_t w) { return __uint_as_float(pair_of(w)); }

// Sequences per interleaved group in the per-sequence VALU work (norms and
// residual sums): G rows run side by side, so their LDS reads and arithmetic
// overlap instead of following each other.
#ifndef LFM25_BGROUP
#define LFM25_BGROUP 2
#endif
template <int kB> constexpr int kBGroup = kB < LFM25_BGROUP ? kB : LFM25_BGROUP;

// ------------------------------------------------------------------ gathers

// Block-wide gather and norm of the kB h vectors of a local buffer (row s =
// sequence s, 1024 words) together with the 16 producer blocks' sums of
// squares of each row (ss[16 s + jj], written with the rows): wave w polls
// words [128w, 128w + 128) of every row and every sum, forms each sequence's
// scale from its 16 sums (a fixed order within a 16-lane row) and norms its
// words straight into vec[s] (norm_words_reg's rounding). With `keep`, wave
// jj / 2 also keeps the block's residual rows; with `raw`, the gathered words
// go there as well ([kB][512]). No barrier: the caller's next one publishes
// vec.
template <int kB, bool kLocal>
__device__ __forceinline__ void bgather_norm(const uint32_t* src, const uint64_t* ss, uint32_t tag, BShared<kB>& sm,
                                             uint32_t gw, BVec* vec, bool keep, uint32_t* raw, int32_t* status) {
  constexpr int kQ = (kB + 3) / 4;  // sums per lane: lane l of load i holds block l % 16 of sequence 4i + l / 16
  const int l = lane_id(), w = wave_id();
  const uint32_t qoff = 8 * (l < kGroupBlocks * kB ? l : 0);
  uint64_t x[kB], q[kQ];
  Poll poll(status);
  while (true) {
    if constexpr (kLocal) {
      nt_load64_rows_q<kB>(src + 128 * w, 8 * l, 4 * kHidden, ss, qoff, x, q);
    } else {
#pragma unroll
      for (int s = 0; s < kB; ++s) x[s] = coherent_load64(src + 128 * w + 2 * l + s * kHidden);
#pragma unroll
      for (int i = 0; i < kQ; ++i) q[i] = coherent_load64(reinterpret_cast<const char*>(ss) + qoff + 512 * i);
    }
    bool ok = true;
#pragma unroll
    for (int s = 0; s < kB; ++s) ok = ok && tag_ok((uint32_t)x[s], tag) && tag_ok((uint32_t)(x[s] >> 32), tag);
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
      const bool in = kWave * i + l < kGroupBlocks * kB;
      ok = ok && (!in || (tag_ok((uint32_t)q[i], tag) && tag_ok((uint32_t)(q[i] >> 32), tag)));
    }
    if (__all(ok) || !poll.again()) break;
  }
  float r_lane[kQ];
#pragma unroll
  for (int i = 0; i < kQ; ++i) {
    const bool in = kWave * i + l < kGroupBlocks * kB;
    r_lane[i] = norm_scale(row16_sum(in ? f32_of(q[i]) : 0.0f));
  }
  const int e = kWave * w + l;  // the lane's word of every row
#pragma unroll
  for (int s = 0; s < kB; ++s) {
    const float r = lane_value(r_lane[s >> 2], 16 * (s & 3));
    const uint32_t word = pair_of(x[s]);
    if (raw != nullptr) raw[s * kNormWords + e] = word;
    const float a = round_bf16(round_bf16(lo_f32(word) * r) * lo_f32(gw));
    const float b = round_bf16(round_bf16(hi_f32(word) * r) * hi_f32(gw));
    vec[s][e] = bf16_pair(a, b);
  }
  if (keep && w == (blk_jj() >> 1)) {
    // rows 64jj + [0, 64) are words 32jj + [0, 32): lanes 32 (jj % 2) + j
    const int j = l - 32 * (blk_jj() & 1);
    if (j >= 0 && j < 32) {
#pragma unroll
      for (int s = 0; s < kB; ++s) {
        const uint32_t word = pair_of(x[s]);
        sm.hres[s][2 * j] = lo_f32(word);
        sm.hres[s][2 * j + 1] = hi_f32(word);
      }
    }
  }
}

// Block-wide: the step's embedding rows (tokens in sm.tok, written before a
// barrier) in sm.raw, wave s % 8 holding row s, with the group sums of
// gather_raw_split's embedding path (the eight wave sums side by side). With
// `requested` wave s's row is already on its way into sm.raw (bpick_global's
// copy); otherwise it is loaded here. Ends with a barrier.
template <int kB>
__device__ __forceinline__ void bgather_rows(const uint16_t* table, BShared<kB>& sm, bool requested) {
  const int l = lane_id(), w = wave_id();
  if (requested) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the copies have landed
#pragma unroll 1
  for (int s = w; s < kB; s += kStepWaves) {
    uint32_t v[8];
    if (requested) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = sm.raw[s][l + 64 * i];
    } else {
      const uint16_t* row = table + (size_t)sm.tok[s] * kHidden;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint32_t*>(row + 2 * l + 128 * i);
#pragma unroll
      for (int i = 0; i < 8; ++i) sm.raw[s][l + 64 * i] = v[i];
    }
    float sw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sw[i] = wave_sum(pair_sq(v[i]));
    if (l == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sm.ss[s][i] = sw[i];
    }
  }
  lds_barrier();
}

// Every wave, after a gather: words [64w, 64w + 64) of each row normed
// (norm_words_reg's arithmetic) into vec[s]; wave s % 8 also keeps the
// block's residual rows of sequence s when `keep` (layer inputs; the head's
// gather does not need them).
template <int kB>
__device__ __forceinline__ void bnorm(BShared<kB>& sm, uint32_t gw, BVec* vec, bool keep) {
  constexpr int G = kBGroup<kB>;
  const int l = lane_id();
  const int i = kWave * wave_id() + l;
  // lane s < kB forms sequence s's scale (norm_scale of group_total, the
  // batch-1 order), broadcast to the wave below: one scale computation a
  // lane instead of kB a thread
  const float r_lane = norm_scale(group_total(sm.ss[l < kB ? l : 0]));
#pragma unroll 1
  for (int s0 = 0; s0 < kB; s0 += G) {
    float r[G];
    uint32_t x[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      r[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r_lane), s0 + g));
      x[g] = sm.raw[s0 + g][i];
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = round_bf16(round_bf16(lo_f32(x[g]) * r[g]) * lo_f32(gw));
      const float b = round_bf16(round_bf16(hi_f32(x[g]) * r[g]) * hi_f32(gw));
      vec[s0 + g][i] = bf16_pair(a, b);
    }
  }
  if (keep) {
    for (int s = wave_id(); s < kB; s += kStepWaves) sm.hres[s][l] = residual_from_raw(sm.raw[s]);
  }
}

// A local vector of `words` (<= 384) values per row into vec: wave w < N
// polls words [128w, 128w + 128) of every row. Ends with a barrier.
template <int kB, int N, bool kLocal>
__device__ __forceinline__ void bgather_plain(const uint32_t* src, int row_words, int words, uint32_t tag,
                                              BVec* vec, int32_t* status) {
  const int l = lane_id(), w = wave_id();
  if (w < N) {
    uint64_t x[kB];
    poll_rows<kB, kLocal>(src + 128 * w, 4 * row_words, words - 128 * w, tag, x, status);
#pragma unroll
    for (int s = 0; s < kB; ++s)
      if (2 * l + 128 * w < words) vec[s][l + 64 * w] = pair_of(x[s]);
  }
  lds_barrier();
}

// ------------------------------------------------------------------ weights

// A layer's weights for wave k (0..7) of block (x, jj) of the layer's group,
// as first operands of v_mfma_f32_16x16x32_bf16: lane l holds row l % 16 of
// a tile and elements 8 (l / 16) .. + 8 of a K step of 32. The block's rows
// are the batch-1 decode's (the same share of every matrix); the K range of a
// row is split over the waves.
//   a: P1 -- conv: tile 0 = in_proj rows c0 + [0, 8) (B) and 1024 + c0 +
//      [0, 8) (C), tile 1 = rows 2048 + c0 + [0, 8) (x), c0 = 128x + 8jj;
//      attention: tile 0 = entries 16jj + [0, 16) of the XCD's q/k/v list,
//      tile 1 rows [0, 8) empty. Rows [8, 16) of tile 1 are P3's: the w1 rows
//      of FFN columns f0 + [16, 20), then their w3 rows (P1 leaves those
//      rows' sums unused). K steps 4k .. 4k + 3 of each (a[j], a[4 + j]);
//   b: P2 -- rows 64jj + 16 (k / 2) + [0, 16) of out_proj / o_proj, K steps
//      2 (k % 2) + [0, 2) of the XCD's 128 columns;
//   c: P3 -- tile t < 2 = w1 rows of FFN columns f0 + 8t + [0, 8) and the
//      w3 rows of the same columns (f0 = 320x + 20jj), K steps 4k .. 4k + 3
//      (c[4t + j]); the block's last four columns are in a[4..7];
//   d: P4 -- rows 64jj + 16 (k / 2) + [0, 16) of w2, K steps 5 (k % 2) +
//      [0, 5) of the XCD's 320 columns.
// Empty rows are out-of-range offsets of their descriptor (zeros, no memory
// touched), so every wave issues the same loads on every layer.
struct BSlabs {
  u32x4 a[8];
  u32x4 b[2];
  u32x4 c[8];
  u32x4 d[5];
};

// The conv epilogue's inputs of thread e = 64k + l < 8 kB (channel c0 + e % 8
// of sequence e / 8): the channel's three taps and the two state taps that
// survive the shift. Loaded at the start of the layer (the gather's poll
// waits for them), so they are held through P1 only.
struct BConvTaps {
  uint32_t taps[3], st[2];
};
template <int kB>
__device__ __forceinline__ void bload_conv_taps(BConvTaps& s, const LayerWeights& L) {
  constexpr int kOutside = 1 << 30;
  const int c0 = kXcdCols * blk_xcd() + kBlockChan * blk_jj();
  const int e = kWave * wave_id() + lane_id(), i = e & 7, q = e >> 3;
  const bool mine = e < kBlockChan * kB;
  const BufRsrc rt = region_rsrc(L.conv_w + c0 * kConvTaps, kBlockChan * kConvTaps * 2, true);
  const BufRsrc rs = region_rsrc(L.state + c0 * kConvTaps, ((kB - 1) * kConvSeqElems + kBlockChan * kConvTaps) * 2, true);
#pragma unroll
  for (int t = 0; t < 3; ++t)
    s.taps[t] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rt, mine ? (i * kConvTaps + t) * 2 : kOutside, 0, 0);
#pragma unroll
  for (int t = 0; t < 2; ++t)
    s.st[t] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
        rs, mine ? (q * kConvSeqElems + i * kConvTaps + 1 + t) * 2 : kOutside, 0, 0);
}

template <int kB>
__device__ __forceinline__ void bload_slabs(BSlabs& s, const LayerWeights& L) {
  constexpr int kOutside = 1 << 30;  // a byte offset past every range below
  const int k = wave_id(), l = lane_id();
  const int x = blk_xcd(), jj = blk_jj();
  const int r = l & 15, grp = l >> 4;
  const int kofs = (128 * k + 8 * grp) * 2;  // the lane's first K element of the wave's range, bytes
  // One descriptor for the layer's P1 and P3 matrices, based at the lowest of
  // them (in_proj or q/k/v, w1, w3: one layer's tensors, element distances
  // far below 2^30).
  const uint16_t* lo = L.wa < L.w1 ? L.wa : L.w1;
  lo = lo < L.w3 ? lo : L.w3;
  const int da = (int)(L.wa - lo), d1 = (int)(L.w1 - lo), d3 = (int)(L.w3 - lo);
  const int f0 = kXcdFfn * x + kBlockFfn * jj;
  const int c0 = kXcdCols * x + kBlockChan * jj;
  int end = da + 3 * kHidden * kHidden;
  end = end > d1 + (f0 + kBlockFfn) * kHidden ? end : d1 + (f0 + kBlockFfn) * kHidden;
  end = end > d3 + (f0 + kBlockFfn) * kHidden ? end : d3 + (f0 + kBlockFfn) * kHidden;
  const BufRsrc rw = region_rsrc(lo, end * 2, true);
  {
    int o0, o1;
    if (L.attn) {
      o0 = (da + (qkv_row(x, kBlockQkv * jj) + r) * kHidden) * 2 + kofs;
    } else {
      o0 = (da + (c0 + (r < 8 ? r : kHidden + r - 8)) * kHidden) * 2 + kofs;
    }
    if (r >= 8) o1 = ((r < 12 ? d1 : d3) + (f0 + 16 + (r & 3)) * kHidden) * 2 + kofs;
    else o1 = L.attn ? kOutside : (da + (c0 + 2 * kHidden + r) * kHidden) * 2 + kofs;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s.a[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, o0 + 64 * j, 0, kBufStream);
      s.a[4 + j] = __builtin_amdgcn_raw_buffer_load_b128(rw, o1 + 64 * j, 0, kBufStream);
    }
  }
  {
    const BufRsrc rb = region_rsrc(L.wb + (size_t)kResRows * jj * kHidden + kXcdCols * x,
                                   ((kResRows - 1) * kHidden + kXcdCols) * 2, true);
    const int ob = ((16 * (k >> 1) + r) * kHidden + 64 * (k & 1) + 8 * grp) * 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) s.b[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, ob + 64 * j, 0, kBufStream);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int oc = ((r < 8 ? d1 : d3) + (f0 + 8 * t + (r & 7)) * kHidden) * 2 + kofs;
#pragma unroll
    for (int j = 0; j < 4; ++j) s.c[4 * t + j] = __builtin_amdgcn_raw_buffer_load_b128(rw, oc + 64 * j, 0, kBufStream);
  }
  {
    const BufRsrc rd = region_rsrc(L.w2 + (size_t)kResRows * jj * kFfn + kXcdFfn * x,
                                   ((kResRows - 1) * kFfn + kXcdFfn) * 2, true);
    const int od = ((16 * (k >> 1) + r) * kFfn + 160 * (k & 1) + 8 * grp) * 2;
#pragma unroll
    for (int j = 0; j < 5; ++j) s.d[j] = __builtin_amdgcn_raw_buffer_load_b128(rd, od + 64 * j, 0, kBufStream);
  }
}

// ------------------------------------------------------------------ compute phases (every wave)

__device__ __forceinline__ f32x4_t mfma_bf16(const u32x4& a, const u32x4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// The second operand's row for this lane: sequence l % 16 (lanes past the
// batch read sequence 0; their columns of the result are never used).
template <int kB>
__device__ __forceinline__ const uint32_t* bcol(BVec* vec) {
  const int col = lane_id() & 15;
  return vec[col < kB ? col : 0];
}

// A wave's partial tile -> mp[row0 + r][sequence] (lane l holds rows
// 4 (l / 16) + i of column l % 16).
__device__ __forceinline__ void bstore_tile(float (*mp)[kMpCols], int row0, f32x4_t acc) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) mp[row0 + 4 * (l >> 4) + i][l & 15] = acc[i];
}

// The sum over the eight waves' partials of one entry, in a fixed tree.
template <int kB>
__device__ __forceinline__ float bsum8(const BShared<kB>& sm, int row, int s) {
  float p[kStepWaves];
#pragma unroll
  for (int k = 0; k < kStepWaves; ++k) p[k] = sm.mp[k][row][s];
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

// P1, conv layer, every sequence: B, C, x of channels c0 + [0, 8) (two tiles
// over the wave's K range), then thread e < 8 kB forms channel c0 + e % 8 of
// sequence e / 8 (the conv gate and state shift) -> ly[s][8jj + e % 8].
template <int kB, bool kLocal>
__device__ __forceinline__ void bcompute_conv(const BSlabs& S, const BConvTaps& T, BShared<kB>& sm, BVec* vec,
                                              uint16_t* state, uint32_t tag, uint32_t* ly) {
  const int k = wave_id(), l = lane_id();
  const uint32_t* xv = bcol<kB>(vec);
  f32x4_t t0 = {0.0f, 0.0f, 0.0f, 0.0f}, t1 = t0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 bx = lds16(xv, 16 * k + 4 * j + (l >> 4));
    t0 = mfma_bf16(S.a[j], bx, t0);
    t1 = mfma_bf16(S.a[4 + j], bx, t1);
  }
  bstore_tile(sm.mp[k], 0, t0);
  bstore_tile(sm.mp[k], 16, t1);
  lds_barrier();
  const int e = threadIdx.x;
  if (e < kBlockChan * kB) {
    const int i = e & 7, s = e >> 3;
    const int c = kXcdCols * blk_xcd() + kBlockChan * blk_jj() + i;
    const uint16_t w[3] = {(uint16_t)T.taps[0], (uint16_t)T.taps[1], (uint16_t)T.taps[2]};
    const uint16_t st[3] = {0, (uint16_t)T.st[0], (uint16_t)T.st[1]};
    const float s01 = conv_state_taps(w, st);
    const float B = round_bf16(bsum8(sm, i, s)), C = round_bf16(bsum8(sm, 8 + i, s));
    const float X = round_bf16(bsum8(sm, 16 + i, s));
    const float yv = conv_gate_channel_from(B, C, X, w, st, s01, state + (size_t)s * kConvSeqElems + c * kConvTaps);
    local_store32<kLocal>(ly + s * kLyWords + kBlockChan * blk_jj() + i, tagged(yv, tag));
  }
}

// P1, attention layer, every sequence: q/k/v entries 16jj + [0, 16) (one
// tile), thread e < 16 kB storing entry 16jj + e % 16 of sequence e / 16.
template <int kB, bool kLocal>
__device__ __forceinline__ void bcompute_qkv(const BSlabs& S, BShared<kB>& sm, BVec* vec, uint32_t tag,
                                             uint32_t* lq) {
  const int k = wave_id(), l = lane_id();
  const uint32_t* xv = bcol<kB>(vec);
  f32x4_t t0 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4; ++j) t0 = mfma_bf16(S.a[j], lds16(xv, 16 * k + 4 * j + (l >> 4)), t0);
  bstore_tile(sm.mp[k], 0, t0);
  lds_barrier();
  const int e = threadIdx.x;
  if (e < kBlockQkv * kB) {
    const int r = e & 15, s = e >> 4;
    local_store32<kLocal>(lq + s * kLqWords + kBlockQkv * blk_jj() + r, tagged(bsum8(sm, r, s), tag));
  }
}

// The block's 64 partial sums of every sequence -> gp[jj][x][s][0..64): row
// 64jj + r is the sum of the tiles of waves 2 (r / 16) and 2 (r / 16) + 1;
// wave s stores sequence s after a barrier (every thread of the block calls it).
template <int kB>
__device__ __forceinline__ void bpublish(BShared<kB>& sm, uint64_t* gp, uint32_t tag) {
  lds_barrier();
  const int w = wave_id(), l = lane_id();
  const int t = l >> 4, r = l & 15;
#pragma unroll
  for (int s = w; s < kB; s += kStepWaves) {
    const float v = sm.mp[2 * t][r][s] + sm.mp[2 * t + 1][r][s];
    coherent_store64(gp + (((size_t)blk_jj() * kXcds + blk_xcd()) * kB + s) * kResRows + l, tagged_partial(v, tag));
  }
}

// P2, every sequence: partial sums of rows 64jj + [0, 64) over the XCD's 128
// columns (wave k: rows 16 (k / 2) + [0, 16), half k % 2 of the columns).
template <int kB>
__device__ __forceinline__ void bcompute_proj(const BSlabs& S, BShared<kB>& sm, BVec* vec,
                                              uint32_t tag, uint64_t* gp) {
  const int k = wave_id(), l = lane_id();
  const uint32_t* xv = bcol<kB>(vec);
  f32x4_t t0 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j) t0 = mfma_bf16(S.b[j], lds16(xv, 8 * (k & 1) + 4 * j + (l >> 4)), t0);
  bstore_tile(sm.mp[k], 0, t0);
  bpublish<kB>(sm, gp, tag);
}

// P3, every sequence: w1 and w3 of the block's 20 FFN columns (two tiles of
// c and the P3 half of a's tile 1, over the wave's K range), then thread
// e < 20 kB forms the gated activation of column e % 20 of sequence e / 20
// -> lg[s][20jj + e % 20].
template <int kB, bool kLocal>
__device__ __forceinline__ void bcompute_up(const BSlabs& S, BShared<kB>& sm, BVec* vec, uint32_t tag,
                                            uint32_t* lg) {
  const int k = wave_id(), l = lane_id();
  const uint32_t* xv = bcol<kB>(vec);
  f32x4_t t[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) t[i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 bx = lds16(xv, 16 * k + 4 * j + (l >> 4));
    t[0] = mfma_bf16(S.c[j], bx, t[0]);
    t[1] = mfma_bf16(S.c[4 + j], bx, t[1]);
    t[2] = mfma_bf16(S.a[4 + j], bx, t[2]);
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) bstore_tile(sm.mp[k], 16 * i, t[i]);
  lds_barrier();
  const int e = threadIdx.x;
  if (e < kBlockFfn * kB) {
    const int s = e / kBlockFfn, f = e % kBlockFfn;
    const int row_a = f < 16 ? 16 * (f >> 3) + (f & 7) : 40 + (f & 3);
    const int row_g = f < 16 ? row_a + 8 : 44 + (f & 3);
    const float a = bsum8(sm, row_a, s), g = bsum8(sm, row_g, s);
    local_store32<kLocal>(lg + s * kLgWords + kBlockFfn * blk_jj() + f,
                          tagged(silu_bf16(round_bf16(a)) * round_bf16(g), tag));
  }
}

// P4, every sequence: partial sums of rows 64jj + [0, 64) over the XCD's 320
// FFN columns (wave k: rows 16 (k / 2) + [0, 16), half k % 2 of the columns).
template <int kB>
__device__ __forceinline__ void bcompute_down(const BSlabs& S, BShared<kB>& sm, BVec* vec,
                                              uint32_t tag, uint64_t* gp) {
  const int k = wave_id(), l = lane_id();
  const uint32_t* xv = bcol<kB>(vec);
  f32x4_t t0 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 5; ++j) t0 = mfma_bf16(S.d[j], lds16(xv, 4 * (5 * (k & 1) + j) + (l >> 4)), t0);
  bstore_tile(sm.mp[k], 0, t0);
  bpublish<kB>(sm, gp, tag);
}

// R phase, every sequence: wave s % 8 polls the partials of sequence s from
// the eight XCDs (eight rows of 512 bytes, all in flight), sums them in
// run_residual_split's order, adds the residual and publishes h rows 64jj +
// lane of sequence s, then their sum of squares -> ss[16 s + jj]. No block
// barrier: the partial tiles that bpublish read are next written by the
// following product, and a wave reaches it only through a gather that has
// polled every sequence's sum of squares from this block, which wave s % 8
// publishes after its last read of the tiles.
template <int kB, bool kLocal>
__device__ __forceinline__ void bresidual(BShared<kB>& sm, const uint64_t* gp, uint32_t tag_gp, uint32_t* dst,
                                          uint64_t* ss, uint32_t tag_out, int32_t* status) {
  constexpr int kPer = kBSeqPerWave<kB>;  // (B = 16: sequences w and w + 8, polled together)
  const int l = lane_id(), w = wave_id();
  if (w >= kB) return;
  // XCD i's partials of sequence s: gp[jj][i][s][0..64)
  const uint64_t* src = gp + ((size_t)blk_jj() * kXcds * kB + w) * kResRows + l;
  Poll poll(status);
  uint64_t x[kPer][kXcds];
  while (true) {
    bool ok = true;
#pragma unroll
    for (int r = 0; r < kPer; ++r)
#pragma unroll
      for (int i = 0; i < kXcds; ++i) x[r][i] = coherent_load64(src + ((size_t)i * kB + 8 * r) * kResRows);
#pragma unroll
    for (int r = 0; r < kPer; ++r)
#pragma unroll
      for (int i = 0; i < kXcds; ++i) ok = ok && (uint32_t)(x[r][i] >> 32) == tag_gp;
    if (__all(ok) || !poll.again()) break;
  }
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int s = w + 8 * r;
    float p[kXcds];
#pragma unroll
    for (int i = 0; i < kXcds; ++i) p[i] = __uint_as_float((uint32_t)x[r][i]);
    const float sum = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    const float h = round_bf16(sm.hres[s][l] + round_bf16(sum));
    sm.hres[s][l] = h;
    local_store32<kLocal>(dst + s * kHidden + kResRows * blk_jj() + l, tagged(h, tag_out));
    const float q = wave_sum(h * h);  // h is BF16, so each square is exact
    if (l == 0) local_store64<kLocal>(ss + s * kGroupBlocks + blk_jj(), tagged_f32(q, tag_out));
  }
}

// ------------------------------------------------------------------ attention (group 0)
//
// Block jj of XCD x serves sequence s = jj / nb (nb = 16 / kB blocks per
// sequence) as its block i = jj % nb. Below 256 positions blocks i = 0, 1
// attend alone, one query head each (attn_single_head, the batch-1 single
// path). Past that the nb blocks split the sequence's cache: block i holds
// passes i, i + nb, i + 2 nb, i + 3 nb (so a sequence has 256 nb positions),
// in attn_prefetch's whole-position layout.

template <int kB>
struct BSeq {
  static constexpr int nb = kGroupBlocks / kB;  // blocks per sequence
  static constexpr int cap = kAttnLocal * nb;   // positions the split path holds
};
template <int kB> __device__ __forceinline__ int bseq() { return blk_jj() / BSeq<kB>::nb; }
template <int kB> __device__ __forceinline__ int bidx() { return blk_jj() % BSeq<kB>::nb; }
// Cache pass of register pass t of this block (split path).
template <int kB> __device__ __forceinline__ int bpass(int t) { return bidx<kB>() + BSeq<kB>::nb * t; }
template <int kB> __device__ __forceinline__ int bwave_base(int w) {
  return bpass<kB>(w >> 1) * kAttnSlots + kSinglePerWave * (w & 1);
}

// The per-lane values of the attention prologue held from the prefetch to
// the attention (the q or k norm weight and the RoPE cos / sin of dimension
// `lane`, waves 0..2).
struct BAttnPre {
  uint32_t gamma, cos, sin;
};

// attn_prefetch for block i of sequence s: `keys` / `values` are that
// sequence's rows of KV head x. The passes go straight to LDS (sm.kvl,
// buffer-to-LDS loads with the same bounds), so nothing is held in
// registers between the layers.
template <int kB, int kPath, bool kLocal>
__device__ __forceinline__ void battn_prefetch(const uint16_t* keys, const uint16_t* values, int past,
                                               const uint16_t* q_gamma, const uint16_t* k_gamma,
                                               const uint16_t* rope_row, BShared<kB>& sm, BAttnPre& pre) {
  typedef __attribute__((address_space(3))) void LdsPtr;
  constexpr bool single = kPath == kAttnOne;
  const int rows = single && bidx<kB>() >= kSingleBlocks ? 0 : past;
  const int w = wave_id(), l = lane_id();
  BufRsrc rk, rv;
  int ok, ov;
  if (single) {
    rk = region_rsrc(keys, rows * kHeadDim * 2, true);
    rv = region_rsrc(values, rows * kHeadDim * 2, true);
    ok = (kSinglePerWave * w + (l & 31)) * kHeadDim * 2 + kHeadDim * (l >> 5);
    ov = (kSinglePerWave * w + kSingleHalf * (l >> 5)) * kHeadDim * 2 + 4 * (l & 31);
  } else {
    const int pass = bpass<kB>(w >> 1);
    rk = kv_pass_rsrc(keys, rows, pass);
    rv = kv_pass_rsrc(values, rows, pass);
    ok = (kSinglePerWave * (w & 1) + (l & 31)) * kHeadDim * 2 + kHeadDim * (l >> 5);
    ov = (kSinglePerWave * (w & 1) + kSingleHalf * (l >> 5)) * kHeadDim * 2 + 4 * (l & 31);
  }
#pragma unroll
  for (int i = 0; i < kAttnPrefetch; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LdsPtr*)&sm.kvl[i][w][0][0], 16, ok + 16 * i, 0, 0,
                                             kKvLoadAux<kLocal>);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (LdsPtr*)&sm.kvl[i][w][1][kWave * e], 4,
                                               ov + (4 * i + e) * kHeadDim * 2, 0, 0, kKvLoadAux<kLocal>);
  }
  const BufRsrc rg = region_rsrc(w < 2 ? q_gamma : k_gamma, kHeadDim * 2, w < 3);
  const BufRsrc rr = region_rsrc(rope_row, 2 * kHeadDim * 2, w < 3);
  pre.gamma = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rg, 2 * l, 0, 0);
  pre.cos = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rr, 2 * l, 0, 0);
  pre.sin = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rr, 2 * l, kHeadDim * 2, 0);
}

// The prefetched passes of this wave back in registers (the DMA has landed:
// every poll since the prefetch waited for all of the wave's loads, and this
// wait covers the rest).
template <int kB>
__device__ __forceinline__ AttnKV battn_kv(const BShared<kB>& sm, const BAttnPre& pre) {
  const int w = wave_id(), l = lane_id();
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  AttnKV kv;
#pragma unroll
  for (int i = 0; i < kAttnPrefetch; ++i) {
    kv.k[i] = *reinterpret_cast<const u32x4*>(&sm.kvl[i][w][0][4 * l]);
#pragma unroll
    for (int e = 0; e < 4; ++e) kv.v[i][e] = sm.kvl[i][w][1][kWave * e + l];
  }
  kv.gamma_rope = pre.gamma;
  kv.cos_sin = pre.cos | (pre.sin << 16);
  return kv;
}

// attn_split_stats over this block's passes of its sequence.
template <int kB>
__device__ __forceinline__ void battn_split_stats(int past, const AttnKV& kv, AttnSplitShared& sh, float* mz) {
  const int w = wave_id(), l = lane_id();
  const int base = bwave_base<kB>(w);
  const bool any = base <= past;
  const int j = base + (l & 31);
  float mw[2] = {-INFINITY, -INFINITY}, zw[2] = {0.0f, 0.0f};
#pragma unroll
  for (int hq = 0; hq < 2; ++hq) {
    float s = -INFINITY;
    if (any) {
      const float full = lane_score(kv, sh, hq, j == past);
      if (j <= past) s = round_bf16(full) * 0.125f;
      if ((l >> 5) == 0) sh.score[hq][kSinglePerWave * w + (l & 31)] = s;
      mw[hq] = wave_max(s);
      const float e = j <= past ? expf(s - mw[hq]) : 0.0f;
      zw[hq] = wave_sum((l >> 5) == 0 ? e : 0.0f);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (l == 0) {
    sh.red[0][w] = mw[0];
    sh.red[1][w] = mw[1];
    sh.red_sum[0][w] = zw[0];
    sh.red_sum[1][w] = zw[1];
  }
  lds_barrier();
#pragma unroll
  for (int hq = 0; hq < 2; ++hq) {
    const float mi = sh.red[hq][l & (kStepWaves - 1)], zi = sh.red_sum[hq][l & (kStepWaves - 1)];
    const float m = wave_max(mi);
    const float ti = zi > 0.0f ? zi * expf(mi - m) : 0.0f;
    float z = lane_value(ti, 0);
#pragma unroll
    for (int i = 1; i < kStepWaves; ++i) z += lane_value(ti, i);
    mz[2 * hq] = m;
    mz[2 * hq + 1] = z;
  }
}

// attn_split_context over this block's passes (one block barrier).
template <int kB>
__device__ __forceinline__ float battn_split_context(int past, const AttnKV& kv, AttnSplitShared& sh, const float* mz) {
  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int half = l >> 5, lo = l & 31;
  const int base = bwave_base<kB>(w);
  const bool any = base <= past;
  const int j = base + lo;
  float c[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  if (any) {
    const uint32_t vnew = sh.vp[lo];
    const int first = base + kSingleHalf * half;
    const bool has_past = past >= first && past < first + kSingleHalf;
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      const float sj = sh.score[hq][kSinglePerWave * w + lo];
      const float p = j <= past ? round_bf16(expf(sj - mz[2 * hq]) / mz[2 * hq + 1]) : 0.0f;
      if (half == 0) sh.score[hq][kSinglePerWave * w + lo] = p;
      float pj[kSingleHalf];
#pragma unroll
      for (int i = 0; i < kSingleHalf / 4; ++i) {
        const u32x4 pv =
            *reinterpret_cast<const u32x4*>(&sh.score[hq][kSinglePerWave * w + kSingleHalf * half + 4 * i]);
        pj[4 * i] = __uint_as_float(pv.x);
        pj[4 * i + 1] = __uint_as_float(pv.y);
        pj[4 * i + 2] = __uint_as_float(pv.z);
        pj[4 * i + 3] = __uint_as_float(pv.w);
      }
#pragma unroll
      for (int i = 0; i < kSingleHalf; ++i) {
        const uint32_t vw = kv.v[i >> 2][i & 3];
        c[hq][0] = fmaf(pj[i], lo_f32(vw), c[hq][0]);
        c[hq][1] = fmaf(pj[i], hi_f32(vw), c[hq][1]);
      }
      if (has_past) {
        const float pp = sh.score[hq][kSinglePerWave * w + (past - base)];
        c[hq][0] = fmaf(pp, lo_f32(vnew), c[hq][0]);
        c[hq][1] = fmaf(pp, hi_f32(vnew), c[hq][1]);
      }
      c[hq][0] = half_swap_sum(c[hq][0]);
      c[hq][1] = half_swap_sum(c[hq][1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (half == 0) {
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      sh.ctx[w][hq][2 * lo] = c[hq][0];
      sh.ctx[w][hq][2 * lo + 1] = c[hq][1];
    }
  }
  lds_barrier();
  float out = 0.0f;
  if (tid < 2 * kHeadDim) {
    const int hq = tid / kHeadDim, d = tid % kHeadDim;
    out = sh.ctx[0][hq][d];
#pragma unroll
    for (int i = 1; i < kStepWaves; ++i) out += sh.ctx[i][hq][d];
  }
  return out;
}

// KV head x for this block's sequence s at position `pos` (run_attention's
// phases): q/k/v of sequence s from lq, QK norm + RoPE, KV append (block i
// = 0), then the single-block head (i < 2) -> ly[s][64 i ..], or the split
// statistics exchange among the sequence's nb blocks and the block's FP32
// context partial -> lc[jj].
template <int kB, bool kLocal, int kPath>
__device__ __forceinline__ void brun_attention(const BBufs<kB>& b, int32_t* status, uint32_t tag_qkv, uint32_t tag_st,
                                               uint32_t tag_out, uint16_t* keys, uint16_t* values, int pos,
                                               BShared<kB>& sm, const BAttnPre& pre) {
  AttnSplitShared& sh = sm.attn;
  constexpr bool single = kPath == kAttnOne;
  constexpr int nb = BSeq<kB>::nb;
  const int w = wave_id(), l = lane_id(), x = blk_xcd(), jj = blk_jj();
  const int s = bseq<kB>(), i = bidx<kB>();
  if (single && i >= kSingleBlocks) return;
  const AttnKV kv = battn_kv<kB>(sm, pre);
  const bool append = i == 0;
  if (w < 4) {
    const int e = kHeadDim * w + l;
    const uint32_t* src = b.lq(x) + s * kLqWords;
    uint64_t wd[1];
    Poll poll(status);
    while (true) {
      local_load64<1, kLocal>(src, 4 * (e & ~1), wd);
      if (__all(tag_ok((uint32_t)(wd[0] >> (32 * (e & 1))), tag_qkv)) || !poll.again()) break;
    }
    const float raw = tagged_value((uint32_t)(wd[0] >> (32 * (e & 1))));
    float val = raw;
    if (w < 3) {
      const float o = norm_rope_lane(raw, lo_f32(kv.gamma_rope), lo_f32(kv.cos_sin), hi_f32(kv.cos_sin));
      val = o;
      if (w < 2) {
        sh.q[w][l] = o;
      } else {
        sh.k_new[l] = o;
        if (append) kv_append<kLocal>(keys + (size_t)pos * kHeadDim + l, f32_to_bf16(o));
      }
    } else {
      sh.v_new[l] = raw;
      if (append) kv_append<kLocal>(values + (size_t)pos * kHeadDim + l, f32_to_bf16(raw));
    }
    const float hi = dpp_f32<kDppQuadXor1>(val);
    if ((l & 1) == 0) {
      uint32_t* dst = w < 2 ? sh.qp[w] : w == 2 ? sh.kp : sh.vp;
      dst[l >> 1] = bf16_pair(val, hi);
    }
  }
  lds_barrier();
  if constexpr (single) {
    // one query head per block; with one block per sequence (B = 16) the
    // block takes both in turn, a barrier apart (the first head's context
    // sums read the shared partials the second one rewrites)
    constexpr int kHeads = nb == 1 ? 2 : 1;
#pragma unroll 1
    for (int t = 0; t < kHeads; ++t) {
      const int hq = nb == 1 ? t : i;
      if (t > 0) lds_barrier();
      const float ctx = attn_single_head<kAttnOne>(pos, hq, kv, sh);
      if (threadIdx.x < kHeadDim)
        local_store32<kLocal>(b.ly(x) + s * kLyWords + kHeadDim * hq + threadIdx.x, tagged(ctx, tag_out));
    }
    return;
  } else {
    static_assert(nb > 1, "the split path needs several blocks per sequence");
    float mz[kAttnStats];
    battn_split_stats<kB>(pos, kv, sh, mz);
    if (threadIdx.x < kAttnStats)
      local_store64<kLocal>(b.ls(x) + kAttnStats * jj + threadIdx.x, tagged_partial(mz[threadIdx.x], tag_st));
    if (w == 0) {
      // lane l < 4 nb: word l % 4 of block s nb + l / 4
      const uint64_t* src = b.ls(x) + kAttnStats * nb * s;
      const bool in = l < kAttnStats * nb;
      uint64_t sw[1];
      Poll poll(status);
      while (true) {
        local_load64<1, kLocal>(src, 8 * (in ? l : 0), sw);
        if (__all(!in || (uint32_t)(sw[0] >> 32) == tag_st) || !poll.again()) break;
      }
      if (in) sh.stats[l] = __uint_as_float((uint32_t)sw[0]);
      if (l < 2) {
        float m = -INFINITY;
        for (int q = 0; q < nb; ++q) m = fmaxf(m, sh.stats[kAttnStats * q + 2 * l]);
        float z = 0.0f;
        for (int q = 0; q < nb; ++q) {
          const float zb = sh.stats[kAttnStats * q + 2 * l + 1];
          if (zb > 0.0f) z += zb * expf(sh.stats[kAttnStats * q + 2 * l] - m);
        }
        sh.mz[2 * l] = m;
        sh.mz[2 * l + 1] = z;
      }
    }
    lds_barrier();
    const float gmz[kAttnStats] = {sh.mz[0], sh.mz[1], sh.mz[2], sh.mz[3]};
    const float part = battn_split_context<kB>(pos, kv, sh, gmz);
    if (threadIdx.x < 2 * kHeadDim)
      local_store64<kLocal>(b.lc(x) + 2 * kHeadDim * jj + threadIdx.x, tagged_partial(part, tag_out));
  }
}

// The contexts of every sequence for P2, from the split path's partials:
// the 16 blocks' FP32 partials (every wave polls two blocks' 256 words), then
// thread t < 64 kB sums the nb partials of sequence t / 64 in block order,
// rounds once and writes vec[s]. Block-wide; ends with a barrier.
template <int kB, bool kLocal>
__device__ __forceinline__ void bgather_context(const BBufs<kB>& b, int32_t* status, uint32_t tag,
                                                BVec* vec, AttnSplitShared& sh) {
  const int w = wave_id(), l = lane_id();
  constexpr int kPerWave = 4 * kWave;
  constexpr int nb = BSeq<kB>::nb;
  {
    const uint64_t* src = b.lc(blk_xcd()) + kPerWave * w;
    uint64_t pw[4];
    Poll poll(status);
    while (true) {
      local_load64<4, kLocal>(src, 8 * l, pw);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) ok = ok && (uint32_t)(pw[i] >> 32) == tag;
      if (__all(ok) || !poll.again()) break;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int word = kPerWave * w + l + kWave * i;
      sh.part[word / (2 * kHeadDim)][word % (2 * kHeadDim)] = __uint_as_float((uint32_t)pw[i]);
    }
  }
  lds_barrier();
  if (threadIdx.x < kHeadDim * kB) {
    const int s = threadIdx.x / kHeadDim, d = threadIdx.x % kHeadDim;
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = 2 * d + u;
      v[u] = sh.part[nb * s][c];
      for (int q = 1; q < nb; ++q) v[u] += sh.part[nb * s + q][c];
    }
    vec[s][d] = bf16_pair(round_bf16(v[0]), round_bf16(v[1]));
  }
  lds_barrier();
}

// ------------------------------------------------------------------ head

// The head on the matrix cores: logits of 16 table rows for up to 16
// sequences per v_mfma_f32_16x16x32_bf16 (the table rows as the first
// operand, lane l holding row l % 16 and 8 of the 32 K of a step, the normed
// vectors as the second, lane l holding sequence l % 16), FP32 accumulation
// over K = 1024 in 32 steps. XCD x scans a contiguous range of 16-row units,
// its 256 waves every 256th unit of it, each unit in four chunks of 256 K
// through two register buffers: the next chunk's loads are in flight while
// one is multiplied (the loop is unrolled by a unit so that no buffer is
// ever copied: a copy would wait for its loads). A lane keeps the first
// maximum of the 4 logits it holds per unit (rows 4 (l / 16) + i of sequence
// l % 16), the four lanes of a sequence are combined at the end, and each
// block's best (value, row) of sequence s -> lw[x][s][j].
constexpr int kBHeadRows = 16;
constexpr int kBHeadChunk = 256;
constexpr int kBHeadSteps = kBHeadChunk / 32;  // MFMA steps per chunk
constexpr int kBHeadChunks = kHidden / kBHeadChunk;
static_assert(kBHeadChunks == 4, "one loop iteration per unit of four chunks");

// Chunk kc of unit u into a (zeros, and no memory touched, when u >= units).
__device__ __forceinline__ void bhead_load(const uint16_t* table, int units, int u, int kc, u32x4* a) {
  const int l = lane_id();
  const BufRsrc r = region_rsrc(table + (size_t)(u < units ? u : 0) * kBHeadRows * kHidden,
                                kBHeadRows * kHidden * 2, u < units);
  const int off = ((l & 15) * kHidden + kc * kBHeadChunk + 8 * (l >> 4)) * 2;
#pragma unroll
  for (int t = 0; t < kBHeadSteps; ++t) a[t] = __builtin_amdgcn_raw_buffer_load_b128(r, off + 64 * t, 0, kBufCached);
}

// The group that computed the last layer scans its units about 30% slower
// than the other group (B = 2, 4, 8; the cause was not found: with the two
// groups' CUs exchanged the slow blocks moved with that role, not with the
// CUs). So each XCD's range is split 5 : 3, the larger part to the other
// group, each group dealing its part round robin to its 128 waves: the scan's
// last block then ends ~3 us sooner at B = 4.
constexpr int kBHeadIdleShare = 320;  // of every 512 units of an XCD's range
constexpr int kBHeadGroupWaves = kGroupBlocks * kStepWaves;  // 128
// The wave's units: u0, u0 + 128, ... below gend; end bounds the XCD's range.
struct BHeadSpan {
  int u0, gend, end;
};
__device__ __forceinline__ BHeadSpan bhead_span(int vocab) {
  const int units = vocab / kBHeadRows;
  const int x = blk_xcd();
  const int base = units / kXcds, rem = units % kXcds;
  int start = 0;
  for (int y = 0; y < x; ++y) start += base + (y < rem ? 1 : 0);
  const int end = start + base + (x < rem ? 1 : 0);
  const bool last = blk_group() == (kLayers - 1) % 2;
  const int split = start + (end - start) * kBHeadIdleShare / 512;
  return BHeadSpan{(last ? split : start) + blk_jj() + kGroupBlocks * wave_id(), last ? end : split, end};
}

// Chunk 0 of the wave's first unit staged in LDS ahead of the head, in the
// register layout of bhead_load (step t: lane l's 16 bytes at word 256 t +
// 4 l of the wave's 8 KB), in the space of the attention prefetch: each group
// issues it behind the weights of its last layer (group 1 computes only conv
// layers; group 0 after its last attention layer), so it lands while the
// other group computes and 1/8 of the table is off the scan's critical path.
// A wave without units stages zeros and touches no memory.
template <int kB>
__device__ __forceinline__ uint32_t* bhead_slot(BShared<kB>& sm) {
  static_assert(sizeof(sm.kvl) >= (size_t)kStepWaves * kBHeadSteps * kWave * 16, "a chunk per wave");
  return &sm.kvl[0][0][0][0] + (size_t)wave_id() * kBHeadSteps * 4 * kWave;
}
template <int kB>
__device__ __forceinline__ void bhead_stage(const uint16_t* table, int vocab, BShared<kB>& sm) {
  typedef __attribute__((address_space(3))) void LdsPtr;
  const BHeadSpan sp = bhead_span(vocab);
  const int l = lane_id();
  const int u = sp.u0 < sp.gend ? sp.u0 : sp.end;
  const BufRsrc r = region_rsrc(table + (size_t)(u < sp.end ? u : 0) * kBHeadRows * kHidden,
                                kBHeadRows * kHidden * 2, u < sp.end);
  const int off = ((l & 15) * kHidden + 8 * (l >> 4)) * 2;
  uint32_t* slot = bhead_slot(sm);
#pragma unroll
  for (int t = 0; t < kBHeadSteps; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr*)(slot + 4 * kWave * t), 16, off + 64 * t, 0, 0, kBufCached);
}

template <int kB, bool kLocal>
__device__ __forceinline__ void brun_head(BShared<kB>& sm, BVec* vec, const uint16_t* table,
                                          int vocab, const BBufs<kB>& b, uint32_t tag) {
  static_assert(kB <= 16, "one MFMA column per sequence");
  const int l = lane_id(), w = wave_id();
  const BHeadSpan sp = bhead_span(vocab);
  const int u0 = sp.u0, gend = sp.gend, end = sp.end;
  const uint32_t* xv = bcol<kB>(vec);
  float best = -INFINITY;
  int best_row = 0x7fffffff;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const auto take = [&](const u32x4* a, int kc) {
#pragma unroll
    for (int t = 0; t < kBHeadSteps; ++t)
      acc = mfma_bf16(a[t], lds16(xv, (kc * kBHeadChunk + 32 * t) / 8 + (l >> 4)), acc);
  };
  u32x4 r0[kBHeadSteps], r1[kBHeadSteps];
  // (the scheduling barriers keep the loads in issue order, so each wait
  // covers only the buffer it needs)
  const auto load = [&](int u, int kc, u32x4* a) { bhead_load(table, end, u < gend ? u : end, kc, a); };
  {
    // chunk 0 of the first unit from bhead_stage's copy (vmcnt(0): landed)
    __builtin_amdgcn_s_waitcnt(0x0F70);
    const uint32_t* slot = bhead_slot(sm);
#pragma unroll
    for (int t = 0; t < kBHeadSteps; ++t) r0[t] = *reinterpret_cast<const u32x4*>(slot + 4 * kWave * t + 4 * l);
  }
  __builtin_amdgcn_sched_barrier(0);
  load(u0, 1, r1);
  __builtin_amdgcn_sched_barrier(0);
  // a unit past the range reads nothing (its loads return zeros)
  for (int u = u0; u < gend; u += kBHeadGroupWaves) {
    const int un = u + kBHeadGroupWaves;
    take(r0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load(u, 2, r0);
    __builtin_amdgcn_sched_barrier(0);
    take(r1, 1);
    __builtin_amdgcn_sched_barrier(0);
    load(u, 3, r1);
    __builtin_amdgcn_sched_barrier(0);
    take(r0, 2);
    __builtin_amdgcn_sched_barrier(0);
    load(un, 0, r0);
    __builtin_amdgcn_sched_barrier(0);
    take(r1, 3);
    __builtin_amdgcn_sched_barrier(0);
    load(un, 1, r1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = round_bf16(acc[i]);
      const int row = u * kBHeadRows + 4 * (l >> 4) + i;
      if (better(v, row, best, best_row)) {
        best = v;
        best_row = row;
      }
    }
    acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // the four lanes of each sequence (l, l ^ 16, l ^ 32, l ^ 48)
#pragma unroll
  for (int o = 16; o < kWave; o <<= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(best_row, o, kWave);
    if (better(ov, oi, best, best_row)) {
      best = ov;
      best_row = oi;
    }
  }
  if (l < kB) {
    sm.red_v[l][w] = best;
    sm.red_i[l][w] = best_row;
  }
  lds_barrier();
  if (threadIdx.x < kB) {
    const int s = threadIdx.x;
    float bv = sm.red_v[s][0];
    int bi = sm.red_i[s][0];
    for (int i = 1; i < kStepWaves; ++i)
      if (better(sm.red_v[s][i], sm.red_i[s][i], bv, bi)) {
        bv = sm.red_v[s][i];
        bi = sm.red_i[s][i];
      }
    local_store64<kLocal>(b.lw(blk_xcd()) + s * kLwWords + blk_j(), tagged_candidate(bv, bi, tag));
  }
}

// A wave of a group-0 block (wave s % 8): sequence s's XCD winner (over the
// XCD's 32 blocks' candidates) -> gw[s][jj][x].
template <int kB, bool kLocal>
__device__ __forceinline__ void bpick_xcd(const BBufs<kB>& b, int32_t* status, uint32_t tag_cand, uint32_t tag_out,
                                          int s) {
  const int l = lane_id(), x = blk_xcd();
  const bool in = l < kXcdBlocks;
  uint64_t w[1];
  Poll poll(status);
  while (true) {
    local_load64<1, kLocal>(b.lw(x) + s * kLwWords, 8 * (in ? l : 0), w);
    if (__all(!in || candidate_ok(w[0], tag_cand)) || !poll.again()) break;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (in) candidate_of(w[0], bv, bi);
  wave_pick(bv, bi);
  if (l == 0)
    coherent_store64(b.gw() + ((size_t)s * kGroupBlocks + blk_jj()) * kXcds + x, tagged_candidate(bv, bi, tag_out));
}

// A wave of a group-0 block (wave s % 8): sequence s's token (first maximum
// over the eight XCD winners) -> sm.tok[s], and to `out[s]` when out is not
// null; its embedding row is requested into sm.raw[s] at once (buffer-to-LDS,
// bounded by the table: a row past it reads zeros) for the next step's first
// gather.
template <int kB>
__device__ __forceinline__ void bpick_global(const BBufs<kB>& b, int32_t* status, uint32_t tag, BShared<kB>& sm,
                                             int32_t* out, const uint16_t* table, int vocab, int s) {
  const int l = lane_id();
  const bool in = l < kXcds;
  uint64_t w = 0;
  Poll poll(status);
  while (true) {
    w = in ? coherent_load64(b.gw() + ((size_t)s * kGroupBlocks + blk_jj()) * kXcds + l) : 0;
    if (__all(!in || candidate_ok(w, tag)) || !poll.again()) break;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (in) candidate_of(w, bv, bi);
  wave_pick(bv, bi);  // (every lane holds the winner)
  typedef __attribute__((address_space(3))) void LdsPtr;
  const int row = __builtin_amdgcn_readfirstlane(bi);
  const BufRsrc r = region_rsrc(table, vocab * kHidden * 2, true);
#pragma unroll
  for (int c = 0; c < 2; ++c)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr*)&sm.raw[s][256 * c], 16,
                                             row * kHidden * 2 + 1024 * c + 16 * l, 0, 0, kBufCached);
  if (l == 0) {
    sm.tok[s] = bi;
    if (out != nullptr) out[s] = bi;
  }
}

}  // namespace lfm25
