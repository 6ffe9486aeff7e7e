// Block-level phases of the LFM2.5 decode step, laid out for the eight XCDs
// of an MI355X.
//
// Grid: 256 blocks of 512 threads (8 waves), one per CU. The hardware deals
// blocks to XCDs round robin, so block b runs on XCD x = b % 8 as its
// j = b / 8-th block there (the host checks this placement once per device,
// the kernel checks it again per block).
//
// Two measured facts shape the design:
//   * an exchange between blocks of one XCD travels through that XCD's L2
//     (plain store, non-temporal load: ~0.45 us round trip) while one across
//     XCDs goes through the fabric (~1.3 us);
//   * a CU returns vector loads in issue order, so a poll issued behind that
//     CU's own in-flight HBM loads waits for them (0.44 us -> 2.5-4.2 us while
//     the CU streams), whereas other CUs streaming barely matters (0.53 us).
//
// So the 32 blocks of each XCD form two groups of 16 (j < 16: group 0,
// j >= 16: group 1) that take turns: group l % 2 computes layer l with that
// layer's weights already in its registers (its polls see an empty load
// queue), then requests the weights of its next layer (l + 2) in one burst,
// which streams in while the other group computes layer l + 1. Each CU holds
// one layer's share of the weights: 184 KB.
//
// Within a layer, the active group's 16 blocks per XCD split the work so most
// exchanges stay inside one XCD:
//
//   XCD x owns conv channels / o_proj input columns [128x, 128x+128), FFN
//   columns [320x, 320x+320) and KV head x; block (x, jj) of the active
//   group owns residual rows [64jj, 64jj+64) on every XCD.
//
//   P1  h (normed) -> in_proj rows of the block's 8 channels + gated conv,
//       or the block's 16 rows of the XCD's q/k/v          -> local y / qkv
//  [ATT blocks (x, 0..1): QK norm, RoPE, KV append, softmax -> local y (ctx)]
//   P2  y[128x..] -> out_proj / o_proj partial sums of rows [64jj, 64jj+64)
//       over the XCD's 128 columns                         -> global partials
//   R1  partials of rows [64jj..] from the 8 XCDs, fixed-order sum, residual
//                                                           -> local h
//   P3  h (normed) -> w1/w3 rows of the block's 20 FFN columns, SiLU gate
//                                                           -> local g
//   P4  g[320x..] -> w2 partial sums of rows [64jj..] over the XCD's 320
//       columns                                             -> global partials
//   R2  as R1                                               -> local h
//
// Every XCD sums the same eight partials in the same order, so all XCDs hold
// bitwise-identical residual rows. Every exchanged value travels as a word
// carrying its epoch tag ([bf16 | tag16] or [f32 | tag32]); a consumer polls
// until every tag equals the producing exchange's epoch, so the data itself
// is the barrier. Each buffer is written once per layer and the all-gathers
// in between order every rewrite after every read of the previous value.
//
// Wave 0 of every block gathers; then all eight waves compute, each with its
// share of the layer's weights in registers (two waves per SIMD leave 256
// registers to a wave).
#pragma once
#include "lfm25_stages.h"

namespace lfm25 {

constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / kWave;    // 8
constexpr int kComputeWaves = kStepWaves;           // 8
constexpr int kXcds = 8;
constexpr int kXcdBlocks = 32;
constexpr int kStepBlocks = kXcds * kXcdBlocks;     // 256
constexpr int kGroupBlocks = kXcdBlocks / 2;        // blocks of one group on one XCD: 16
constexpr int kResRows = kHidden / kGroupBlocks;    // residual rows per block: 64
constexpr int kXcdCols = kHidden / kXcds;           // conv channels / ctx columns per XCD: 128
constexpr int kXcdFfn = kFfn / kXcds;               // FFN columns per XCD: 320
constexpr int kBlockFfn = kXcdFfn / kGroupBlocks;   // FFN columns per block: 20
constexpr int kXcdQkv = 4 * kHeadDim;               // q0, q1, k, v rows of a KV head: 256
constexpr int kBlockQkv = kXcdQkv / kGroupBlocks;   // 16
constexpr int kBlockChan = kXcdCols / kGroupBlocks; // 8
static_assert(kXcds == kKvHeads, "one KV head per XCD");
static_assert(kXcdCols == 2 * kHeadDim, "an XCD's ctx columns are its two query heads");
static_assert(kBlockChan == kComputeWaves && kBlockQkv == 2 * kComputeWaves &&
                  kResRows == 8 * kComputeWaves,
              "one conv channel, two q/k/v rows, eight residual rows per compute wave");

constexpr int kStepStatusTimeout = 4;
constexpr int kStepStatusPlacement = 8;
// Poll time-out in s_memrealtime ticks (100 MHz): 5 s.
constexpr uint64_t kPollTimeout = 500000000ull;

__device__ __forceinline__ int blk_xcd() { return (int)blockIdx.x & (kXcds - 1); }
__device__ __forceinline__ int blk_j() { return (int)blockIdx.x >> 3; }
__device__ __forceinline__ int blk_group() { return blk_j() / kGroupBlocks; }
__device__ __forceinline__ int blk_jj() { return blk_j() % kGroupBlocks; }

__device__ __forceinline__ int hw_xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return (int)(v & 0xf);
}

// ------------------------------------------------------------------ coherent words

__device__ __forceinline__ uint32_t coherent_load32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t coherent_load64(const void* p) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t tagged(float v, uint32_t tag) {
  return (uint32_t)f32_to_bf16(v) | (tag << 16);
}
__device__ __forceinline__ bool tag_ok(uint32_t w, uint32_t tag) { return (w >> 16) == tag; }
__device__ __forceinline__ float tagged_value(uint32_t w) { return __uint_as_float(w << 16); }

// Partial-sum word: [f32 | tag].
__device__ __forceinline__ uint64_t tagged_partial(float v, uint32_t tag) {
  return (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32);
}
// Candidate word: [value f32 | row (16) | tag (16)].
__device__ __forceinline__ uint64_t tagged_candidate(float v, int row, uint32_t tag) {
  return (uint64_t)__float_as_uint(v) | ((uint64_t)(((uint32_t)row << 16) | tag) << 32);
}

// Bounded waiting: false once this wait timed out or any block flagged a
// time-out or a placement error, so every wave of the grid always drains.
struct Poll {
  int32_t* status;
  uint64_t t0;
  uint32_t iter;
  __device__ explicit Poll(int32_t* s) : status(s), t0(0), iter(0) {}
  __device__ bool again() {
    if (iter == 0) t0 = __builtin_amdgcn_s_memrealtime();
    ++iter;
    if ((iter & 15) == 0) {
      if (coherent_load32(status) & (kStepStatusTimeout | kStepStatusPlacement)) return false;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kPollTimeout) {
        __hip_atomic_fetch_or(status, kStepStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    return true;
  }
};

// ------------------------------------------------------------------ XCD-local words
//
// kLocal: producer and consumers of a local buffer share one XCD, so a plain
// store (write-through to that XCD's L2) and a non-temporal load (misses the
// CU's L1, reads the L2) are coherent; the loads are inline assembly so their
// cache bits are exactly these and the poll loop can never be hoisted. The
// other instantiation uses agent-scope atomics (coherent across XCDs) for
// devices or launches where the placement does not hold.

template <bool kLocal>
__device__ __forceinline__ void local_store32(uint32_t* p, uint32_t v) {
  if constexpr (kLocal) *p = v;
  else coherent_store32(p, v);
}
template <bool kLocal>
__device__ __forceinline__ void local_store64(uint64_t* p, uint64_t v) {
  if constexpr (kLocal) *p = v;
  else coherent_store64(p, v);
}

// N 8-byte loads at base + voff + 512 i bytes (i < N), all in flight, one
// wait; base is wave-uniform (SGPR pair), voff the lane's byte offset.
template <int N>
__device__ __forceinline__ void nt_load64(const void* base, uint32_t voff, uint64_t* w) {
  static_assert(N == 1 || N == 2 || N == 3 || N == 4 || N == 8, "load counts used by the phases");
  if constexpr (N == 1) {
    asm volatile("global_load_dwordx2 %0, %1, %2 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]) : "v"(voff), "s"(base) : "memory");
  } else if constexpr (N == 2) {
    asm volatile("global_load_dwordx2 %0, %2, %3 nt\n\t"
                 "global_load_dwordx2 %1, %2, %3 offset:512 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]) : "v"(voff), "s"(base) : "memory");
  } else if constexpr (N == 3) {
    asm volatile("global_load_dwordx2 %0, %3, %4 nt\n\t"
                 "global_load_dwordx2 %1, %3, %4 offset:512 nt\n\t"
                 "global_load_dwordx2 %2, %3, %4 offset:1024 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]) : "v"(voff), "s"(base) : "memory");
  } else if constexpr (N == 4) {
    asm volatile("global_load_dwordx2 %0, %4, %5 nt\n\t"
                 "global_load_dwordx2 %1, %4, %5 offset:512 nt\n\t"
                 "global_load_dwordx2 %2, %4, %5 offset:1024 nt\n\t"
                 "global_load_dwordx2 %3, %4, %5 offset:1536 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]) : "v"(voff), "s"(base) : "memory");
  } else {
    asm volatile("global_load_dwordx2 %0, %8, %9 nt\n\t"
                 "global_load_dwordx2 %1, %8, %9 offset:512 nt\n\t"
                 "global_load_dwordx2 %2, %8, %9 offset:1024 nt\n\t"
                 "global_load_dwordx2 %3, %8, %9 offset:1536 nt\n\t"
                 "global_load_dwordx2 %4, %8, %9 offset:2048 nt\n\t"
                 "global_load_dwordx2 %5, %8, %9 offset:2560 nt\n\t"
                 "global_load_dwordx2 %6, %8, %9 offset:3072 nt\n\t"
                 "global_load_dwordx2 %7, %8, %9 offset:3584 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]),
                   "=&v"(w[6]), "=&v"(w[7])
                 : "v"(voff), "s"(base) : "memory");
  }
}

// base: wave-uniform; the lane reads base + voff + 512 i.
template <int N, bool kLocal>
__device__ __forceinline__ void local_load64(const void* base, uint32_t voff, uint64_t* w) {
  if constexpr (kLocal) {
    nt_load64<N>(base, voff, w);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = coherent_load64(static_cast<const char*>(base) + voff + 512 * i);
  }
}

// Poll the first `words` (<= 128 N) tagged words of a local buffer (lane l
// owns words 2l + 128i, 2l + 1 + 128i) until every tag equals `tag`.
template <int N, bool kLocal>
__device__ __forceinline__ void poll_local(const uint32_t* src, int words, uint32_t tag,
                                           uint64_t* w, int32_t* status) {
  const int l = lane_id();
  Poll poll(status);
  while (true) {
    local_load64<N, kLocal>(src, 8 * l, w);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const bool in = 2 * l + 128 * i < words;
      ok = ok && (!in || (tag_ok((uint32_t)w[i], tag) && tag_ok((uint32_t)(w[i] >> 32), tag)));
    }
    if (__all(ok) || !poll.again()) break;
  }
}

// ------------------------------------------------------------------ gathered vectors in LDS
//
// A gathered vector sits in LDS as BF16 pairs in natural order (word e/2
// holds element e). A lane reading 8 consecutive elements reads 16 bytes.

__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {  // both exact bf16 values
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}
__device__ __forceinline__ u32x4 lds16(const uint32_t* lds, int elem8) {
  return *reinterpret_cast<const u32x4*>(lds + elem8 * 4);
}

// The polled words of poll_local as BF16 pairs into lds (words < `words`).
template <int N>
__device__ __forceinline__ void words_to_lds(const uint64_t* w, int words, uint32_t* lds) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (2 * l + 128 * i < words)
      lds[l + 64 * i] = ((uint32_t)w[i] & 0xffffu) | ((uint32_t)(w[i] >> 32) << 16);
}

// RMSNorm weights are kept in LDS as packed bf16 pairs: word i holds
// elements 2i and 2i + 1.
constexpr int kNormWords = kHidden / 2;
__device__ __forceinline__ void load_norm_lds(uint32_t* dst, const uint16_t* gamma) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(gamma);
  for (int i = threadIdx.x; i < kNormWords; i += blockDim.x) dst[i] = src[i];
}

// ------------------------------------------------------------------ dot products

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// acc + w.lo * x.lo + w.hi * x.hi (bf16 products are exact in fp32).
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x),
                                         acc, false);
}
__device__ __forceinline__ float dot8(const Pack8& w, const u32x4& x, float acc) {
  acc = dot2(w.w[0], x.x, acc);
  acc = dot2(w.w[1], x.y, acc);
  acc = dot2(w.w[2], x.z, acc);
  return dot2(w.w[3], x.w, acc);
}

// Wave reductions that leave results in VGPR lanes: quad butterflies, two
// row rotations and the gfx950 row/half swaps.
constexpr int kDppQuadBcast0 = 0x00;  // quad_perm [0,0,0,0]: every lane of a quad takes lane 0's value
constexpr int kDppQuadBcast1 = 0x55;  // quad_perm [1,1,1,1]
constexpr int kDppQuadBcast2 = 0xAA;  // quad_perm [2,2,2,2]
constexpr int kDppQuadBcast3 = 0xFF;  // quad_perm [3,3,3,3]
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
__device__ __forceinline__ float half_swap_sum(float v) {  // v(l & 31) + v(l | 32), every lane
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float swap_sum(float v) {  // lanes l, l^16, l^32, l^48 summed
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  return half_swap_sum(v);
}
// Sum of v over the wave, in every lane.
__device__ __forceinline__ float wave_total(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowRor4>(v);
  v += dpp_f32<kDppRowRor8>(v);
  return swap_sum(v);
}
// Wave sums of up to four per-lane partials at once: afterwards lane l holds
// the total of p[l % 4] (zero for rows >= R).
template <int R>
__device__ __forceinline__ float wave_totals4(const float* p) {
  static_assert(R >= 2 && R <= 4, "two to four rows");
  const int l = lane_id();
  const bool b0 = (l & 1) != 0, b1 = (l & 2) != 0;
  const float p0 = p[0], p1 = p[1], p2 = R > 2 ? p[2] : 0.0f, p3 = R > 3 ? p[3] : 0.0f;
  const float v01 = (b0 ? p1 : p0) + dpp_f32<kDppQuadXor1>(b0 ? p0 : p1);
  const float v23 = (b0 ? p3 : p2) + dpp_f32<kDppQuadXor1>(b0 ? p2 : p3);
  float v = (b1 ? v23 : v01) + dpp_f32<kDppQuadXor2>(b1 ? v01 : v23);
  v += dpp_f32<kDppRowRor4>(v);
  v += dpp_f32<kDppRowRor8>(v);
  return swap_sum(v);
}

// d[r] = full-row (K = 1024) dot products of R slab rows with the gathered
// vector, as wave-uniform values. Lane l holds elements 512c + 8l .. +8 of
// chunk c of each row.
template <int R>
__device__ __forceinline__ void rows_dot1024(const Pack8* w, const uint32_t* lds, float* d) {
  const u32x4 x0 = lds16(lds, lane_id()), x1 = lds16(lds, 64 + lane_id());
  float p[R];
#pragma unroll
  for (int r = 0; r < R; ++r) p[r] = dot8(w[2 * r + 1], x1, dot8(w[2 * r], x0, 0.0f));
  if constexpr (R == 1) {
    d[0] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_total(p[0]))));
  } else {
    const float v = wave_totals4<R>(p);
#pragma unroll
    for (int r = 0; r < R; ++r) d[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
  }
}

// ------------------------------------------------------------------ register slabs
//
// Weight rows are read with buffer loads: a scalar descriptor per row (or per
// row group), a constant per-lane byte offset and a scalar chunk offset.
// Every wave issues the same loads for every layer; a row the wave does not
// own (the third in_proj row on attention layers, the third FFN column of
// waves 4..7) gets an empty descriptor (reads zeros, touches no memory), so a
// slab lives in the same registers on every path and is never copied (a copy
// would wait for its loads).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw-buffer format word
constexpr int kBufStream = 2;          // cache policy: non-temporal (read once per token)
constexpr int kBufCached = 0;          // default policy (the vocabulary table, also the embedding)
__device__ __forceinline__ BufRsrc region_rsrc(const uint16_t* base, int bytes, bool valid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, valid ? bytes : 0,
                                           kBufWord3);
}
template <int kAux = kBufStream>
__device__ __forceinline__ Pack8 buffer_load8(BufRsrc r, int lane_bytes, int chunk_bytes) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes, chunk_bytes, kAux);
  Pack8 p;
  p.w[0] = v.x; p.w[1] = v.y; p.w[2] = v.z; p.w[3] = v.w;
  return p;
}
// R full rows of 1024 elements into w[2r], w[2r + 1].
template <int R, int kAux = kBufStream>
__device__ __forceinline__ void load_rows1024(Pack8* w, const uint16_t* const* rows, const bool* valid) {
  const int lane_bytes = lane_id() * 16;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const BufRsrc rs = region_rsrc(rows[r], kHidden * 2, valid[r]);
    w[2 * r] = buffer_load8<kAux>(rs, lane_bytes, 0);
    w[2 * r + 1] = buffer_load8<kAux>(rs, lane_bytes, 1024);
  }
}

// The weights of one layer for wave k (0..7) of block
// (x, jj) of the layer's group:
//   a: P1 -- conv: in_proj rows (c, 1024+c, 2048+c) of channel
//      c = 128x + 8jj + k, its conv taps (lanes 0..2) and the two state taps
//      that survive the shift (lanes 3..4); attention: entries 16jj + 2k and
//      16jj + 2k + 1 of the XCD's q/k/v list;
//   b: P2 -- rows 64jj + 8k + [0, 8) of out_proj / o_proj over the XCD's 128
//      columns, two loads of 4 rows x 16 lanes;
//   c: P3 -- w1 and w3 rows of FFN columns 320x + 20jj + fc(k) + [0, nc(k)),
//      fc = 3k and nc = 3 for k < 4, fc = 12 + 2(k - 4) and nc = 2 after;
//   d: P4 -- rows 64jj + 8k + [0, 8) of w2 over the XCD's 320 columns,
//      8 lanes per row, 5 chunks per lane.
struct Slabs {
  Pack8 a[6];
  uint32_t taps, state;
  Pack8 b[2];
  Pack8 c[12];
  Pack8 d[5];
};

__device__ __forceinline__ int ffn_first(int k) { return k < 4 ? 3 * k : 12 + 2 * (k - 4); }
__device__ __forceinline__ int ffn_count(int k) { return k < 4 ? 3 : 2; }

// Row of the packed q/k/v matrix (q [1024], k [512], v [512] rows back to
// back) for entry i of XCD x's list: q rows of heads 2x, 2x+1, k rows of KV
// head x, v rows of KV head x.
__device__ __forceinline__ int qkv_row(int x, int i) {
  return i < 2 * kHeadDim ? 2 * kHeadDim * x + i
       : i < 3 * kHeadDim ? kHidden + kHeadDim * x + (i - 2 * kHeadDim)
                          : kHidden + kKvHeads * kHeadDim + kHeadDim * x + (i - 3 * kHeadDim);
}

// Weight tensors of the layer a block is loading (attention: wa = q/k/v,
// conv_w / state unused; conv: wa = in_proj).
struct LayerWeights {
  bool attn;
  const uint16_t* wa;
  const uint16_t* conv_w;
  const uint16_t* state;
  const uint16_t* wb;  // out_proj / o_proj
  const uint16_t* w1;
  const uint16_t* w3;
  const uint16_t* w2;
};

constexpr int kSlabBBytes = (7 * kHidden + kXcdCols) * 2;
constexpr int kSlabDBytes = (7 * kFfn + kXcdFfn) * 2;

__device__ __forceinline__ void load_slab_a(Slabs& s, const LayerWeights& L) {
  const int k = wave_id();
  const int x = blk_xcd(), jj = blk_jj();
  const int l = lane_id();
  const int c = kXcdCols * x + kBlockChan * jj + k;
  const int r0 = qkv_row(x, kBlockQkv * jj + 2 * k);
  const uint16_t* rows[3] = {L.wa + (size_t)(L.attn ? r0 : c) * kHidden,
                             L.wa + (size_t)(L.attn ? r0 + 1 : kHidden + c) * kHidden,
                             L.wa + (size_t)(2 * kHidden + c) * kHidden};
  const bool valid[3] = {true, true, !L.attn};
  load_rows1024<3>(s.a, rows, valid);
  const BufRsrc taps = region_rsrc(L.conv_w + c * kConvTaps, kConvTaps * 2, !L.attn);
  const BufRsrc st = region_rsrc(L.state + c * kConvTaps, kConvTaps * 2, !L.attn);
  constexpr int kOutside = 1 << 20;  // a byte offset past both 3-element ranges
  s.taps = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(taps, l < 3 ? 2 * l : kOutside, 0, 0);
  s.state = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(st, l == 3 || l == 4 ? 2 * (l - 2) : kOutside,
                                                           0, 0);
}
__device__ __forceinline__ void load_slab_b(Slabs& s, const LayerWeights& L) {
  const int k = wave_id();
  const uint16_t* base = L.wb + (size_t)(kResRows * blk_jj() + 8 * k) * kHidden + kXcdCols * blk_xcd();
  const BufRsrc rs = region_rsrc(base, kSlabBBytes, true);
  const int l = lane_id();
  const int lane_bytes = ((l >> 4) * kHidden + (l & 15) * 8) * 2;
  s.b[0] = buffer_load8(rs, lane_bytes, 0);
  s.b[1] = buffer_load8(rs, lane_bytes, 4 * kHidden * 2);
}
__device__ __forceinline__ void load_slab_c(Slabs& s, const LayerWeights& L) {
  const int k = wave_id();
  const int f = kXcdFfn * blk_xcd() + kBlockFfn * blk_jj() + ffn_first(k);
  const bool three = ffn_count(k) == 3;
  const uint16_t* rows[6] = {L.w1 + (size_t)f * kHidden,       L.w3 + (size_t)f * kHidden,
                             L.w1 + (size_t)(f + 1) * kHidden, L.w3 + (size_t)(f + 1) * kHidden,
                             L.w1 + (size_t)(f + 2) * kHidden, L.w3 + (size_t)(f + 2) * kHidden};
  const bool valid[6] = {true, true, true, true, three, three};
  load_rows1024<6>(s.c, rows, valid);
}
__device__ __forceinline__ void load_slab_d(Slabs& s, const LayerWeights& L) {
  const int k = wave_id();
  const uint16_t* base = L.w2 + (size_t)(kResRows * blk_jj() + 8 * k) * kFfn + kXcdFfn * blk_xcd();
  const BufRsrc rs = region_rsrc(base, kSlabDBytes, true);
  const int l = lane_id();
  const int lane_bytes = ((l >> 3) * kFfn + (l & 7) * 8) * 2;
#pragma unroll
  for (int i = 0; i < 5; ++i) s.d[i] = buffer_load8(rs, lane_bytes, i * 64 * 2);
}
// The whole layer's share of the wave, as one burst.
__device__ __forceinline__ void load_slabs(Slabs& s, const LayerWeights& L) {
  load_slab_a(s, L);
  load_slab_b(s, L);
  load_slab_c(s, L);
  load_slab_d(s, L);
}

// ------------------------------------------------------------------ buffers
//
// The exchange buffers live in the caller's workspace at fixed offsets. Local
// buffers hold one 128-byte-aligned region per XCD.
constexpr int kLhWords = kHidden;
constexpr int kLyWords = kXcdCols;
constexpr int kLqWords = kXcdQkv;
constexpr int kLgWords = 384;
constexpr int kLwWords = 64;
constexpr int kGpWords = kGroupBlocks * kXcds * kResRows;  // [16 jj][8 x][64 rows]
constexpr size_t kWsCtl = 0;                                  // int32[64] control words
constexpr size_t kWsLh1 = 256;                                // u32 [8][1024] layer output h (R2)
constexpr size_t kWsLh0 = kWsLh1 + 4 * kXcds * kLhWords;      // u32 [8][1024] h after the mixer (R1)
constexpr size_t kWsLy = kWsLh0 + 4 * kXcds * kLhWords;       // u32 [8][128] conv output / context
constexpr size_t kWsLq = kWsLy + 4 * kXcds * kLyWords;        // u32 [8][256] q/k/v of the KV head
constexpr size_t kWsLg = kWsLq + 4 * kXcds * kLqWords;        // u32 [8][384] gated FFN activation
constexpr size_t kWsLw = kWsLg + 4 * kXcds * kLgWords;        // u64 [8][64] block head candidates
constexpr size_t kWsGp = kWsLw + 8 * kXcds * kLwWords;        // u64 [2][16][8][64] partial sums
constexpr size_t kWsGw = kWsGp + 8 * 2 * kGpWords;            // u64 [16][8] XCD winners
constexpr int kLsWords = kGroupBlocks * 4;                    // attention (m, z) of two heads per block
constexpr int kLcWords = kGroupBlocks * 2 * kHeadDim;         // attention context partials per block
constexpr size_t kWsLs = kWsGw + 8 * kGroupBlocks * kXcds;    // u64 [8][16][4] attention statistics
constexpr size_t kWsLc = kWsLs + 8 * kXcds * kLsWords;        // u64 [8][16][128] attention context partials
constexpr size_t kWsBytes = kWsLc + 8 * kXcds * kLcWords;
static_assert(kWsLh0 % 128 == 0 && kWsLy % 128 == 0 && kWsLq % 128 == 0 && kWsLg % 128 == 0 &&
                  kWsLw % 128 == 0 && kWsGp % 128 == 0 && kWsGw % 128 == 0 && kWsLs % 128 == 0 &&
                  kWsLc % 128 == 0,
              "every exchange region starts on a cache line");
constexpr int kCtlStatus = 2;  // LFM25_CTL_STATUS

// A pointer the compiler may treat as global memory (so its loads and stores
// become global_* instructions, which the wait-count insertion can order
// precisely, instead of flat_* ones, which force a full vmcnt(0) wait).
template <typename T>
__device__ __forceinline__ T* as_global(T* p) {
  return (T*)((__attribute__((address_space(1))) T*)p);
}
// As as_global, and keeps the compiler from hoisting address arithmetic
// derived from `p` out of the region where it is used.
template <typename T>
__device__ __forceinline__ T* launder(T* p) {
  auto g = (__attribute__((address_space(1))) T*)p;
  asm volatile("" : "+s"(g));
  return (T*)g;
}

struct StepBufs {
  char* ws;
  __device__ char* base() const { return as_global(ws); }
  __device__ int32_t* status() const { return reinterpret_cast<int32_t*>(base() + kWsCtl) + kCtlStatus; }
  __device__ uint64_t* gw() const { return reinterpret_cast<uint64_t*>(base() + kWsGw); }
};

__device__ __forceinline__ uint32_t* lh1_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint32_t*>(b.base() + kWsLh1) + x * kLhWords;
}
__device__ __forceinline__ uint32_t* lh0_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint32_t*>(b.base() + kWsLh0) + x * kLhWords;
}
__device__ __forceinline__ uint32_t* ly_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint32_t*>(b.base() + kWsLy) + x * kLyWords;
}
__device__ __forceinline__ uint32_t* lq_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint32_t*>(b.base() + kWsLq) + x * kLqWords;
}
__device__ __forceinline__ uint32_t* lg_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint32_t*>(b.base() + kWsLg) + x * kLgWords;
}
__device__ __forceinline__ uint64_t* lw_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint64_t*>(b.base() + kWsLw) + x * kLwWords;
}
__device__ __forceinline__ uint64_t* gp_of(const StepBufs& b, int k) {
  return reinterpret_cast<uint64_t*>(b.base() + kWsGp) + k * kGpWords;
}
__device__ __forceinline__ uint64_t* ls_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint64_t*>(b.base() + kWsLs) + x * kLsWords;
}
__device__ __forceinline__ uint64_t* lc_of(const StepBufs& b, int x) {
  return reinterpret_cast<uint64_t*>(b.base() + kWsLc) + x * kLcWords;
}

// Block-local staging of the P2 / P4 partial sums before their one publish
// store (and, in trace builds, the stamp bookkeeping).
struct StepOut {
  float part[kResRows];  // P2 / P4 partial sums of the block's rows
#ifdef LFM25_TRACE
  // Trace builds: the stamp buffers (null: off) and the current slot, kept
  // in LDS so a stamp costs no global load.
  uint64_t* trace_block;
  uint64_t* trace_waves;
  int trace_steps, trace_slots, trace_at;
#endif
};

// Timing trace of the compute waves (built only with -DLFM25_TRACE): lane 0
// of every wave stamps s_memrealtime at point `sub` of the current slot.
#ifdef LFM25_TRACE
__device__ uint64_t* g_trace_waves = nullptr;
__device__ int g_trace_slots = 0;
#define LFM25_TRACE_WAVE(o, sub)                                                                     \
  do {                                                                                               \
    if (lane_id() == 0 && (o).trace_waves != nullptr && (o).trace_at >= 0 &&                         \
        (o).trace_at < (o).trace_slots)                                                              \
      (o).trace_waves[(((size_t)blockIdx.x * (o).trace_slots + (o).trace_at) * kStepWaves +          \
                       wave_id()) * 2 + (sub)] = __builtin_amdgcn_s_memrealtime();                   \
  } while (0)
#else
#define LFM25_TRACE_WAVE(o, sub) \
  do {                           \
  } while (0)
#endif

// Attention timing (built only with -DLFM25_TRACE_ATTN): thread 0 of block 0
// stamps s_memrealtime at fixed points of every attention call it makes into
// g_attn_trace[call][16] (calls counted from each launch's start). The buffer,
// its length and the call index are kept in the attention's LDS (thread 0's
// copies, set by LFM25_ATTN_INIT), so a stamp waits on no memory operation:
// a read of the globals would wait for every load and store the wave has in
// flight and move their latency into the stamp.
#ifdef LFM25_TRACE_ATTN
__device__ uint64_t* g_attn_trace = nullptr;
__device__ int g_attn_calls = 0;
#define LFM25_ATTN_STAMP(k)                                                                      \
  do {                                                                                           \
    if (blockIdx.x == 0 && threadIdx.x == 0 && sh.atrace != nullptr && sh.aat < sh.acalls)       \
      sh.atrace[(size_t)sh.aat * 16 + (k)] = __builtin_amdgcn_s_memrealtime();                   \
  } while (0)
#define LFM25_ATTN_NEXT()                             \
  do {                                                \
    if (blockIdx.x == 0 && threadIdx.x == 0) ++sh.aat; \
  } while (0)
#define LFM25_ATTN_INIT(s)                                                   \
  do {                                                                       \
    if (threadIdx.x == 0) {                                                  \
      (s).atrace = g_attn_trace;                                             \
      (s).acalls = g_attn_calls;                                             \
      (s).aat = 0;                                                           \
    }                                                                        \
  } while (0)
#else
#define LFM25_ATTN_STAMP(k) \
  do {                      \
  } while (0)
#define LFM25_ATTN_NEXT() \
  do {                    \
  } while (0)
#define LFM25_ATTN_INIT(s) \
  do {                     \
  } while (0)
#endif

// ------------------------------------------------------------------ gathers (wave 0)

// A gathered layer input: the values as BF16 pairs in natural order and the
// RMSNorm scale r = 1 / sqrt(mean(x^2) + eps).
struct Gathered {
  uint32_t raw[kNormWords];
  float scale;
  float ss[kStepWaves];  // sums of squares of words [64 i, 64 i + 64) (gather_raw_split)
};

// The RMSNorm sum of squares in a fixed grouping shared by every gather:
// lane l's term of word l + 64 i is hi^2 + lo^2 (one FMA), group i is its
// wave sum, and the eight groups add as ((g0 + g1) + (g2 + g3)) + ((g4 + g5)
// + (g6 + g7)). A gathering wave can so form its group before the block
// barrier instead of every wave summing all 1024 squares after it.
__device__ __forceinline__ float pair_sq(uint32_t w) {
  const float a = lo_f32(w), b = hi_f32(w);
  return fmaf(b, b, a * a);
}
__device__ __forceinline__ float group_total(const float* ss) {
  return ((ss[0] + ss[1]) + (ss[2] + ss[3])) + ((ss[4] + ss[5]) + (ss[6] + ss[7]));
}
__device__ __forceinline__ float norm_scale(float total) {
  return 1.0f / sqrtf(total * (1.0f / (float)kHidden) + kNormEps);
}

// Wave 0: the layer input (the token's embedding row for layer 0, else the
// local h buffer at epoch `tag`) into g.
template <bool kLocal>
__device__ __forceinline__ void gather_raw(const uint16_t* row, const uint32_t* src, uint32_t tag, Gathered& g,
                                           int32_t* status) {
  const int l = lane_id();
  float v[16];
  if (row != nullptr) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 2 * l + 128 * i);
      v[2 * i] = lo_f32(w);
      v[2 * i + 1] = hi_f32(w);
    }
  } else {
    uint64_t w[8];
    poll_local<8, kLocal>(src, kHidden, tag, w, status);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = tagged_value((uint32_t)w[i]);
      v[2 * i + 1] = tagged_value((uint32_t)(w[i] >> 32));
    }
  }
  float ss[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = bf16_pair(v[2 * i], v[2 * i + 1]);
    g.raw[l + 64 * i] = word;
    ss[i] = wave_sum(pair_sq(word));
  }
  if (l == 0) g.scale = norm_scale(group_total(ss));
}

// Block-wide gather_raw (every wave calls it): from a local h buffer, wave
// w polls words [128w, 128w + 128) of it (512 bytes) into g.raw[64w ..
// 64w + 64), so the block's eight polls are in flight at once. An embedding
// row (row != nullptr in every wave) is read by wave 0 alone: the
// persistent decode hands the selected token to wave 0 only, so in the other
// waves `row` may point at another row. Ends with a block barrier. g.scale is not set: every wave
// takes the scale from raw_scale.
// row_lds (wave 0, with a row): the same row already requested into LDS by
// that wave (pick_global), read from there once the copy has landed.
template <bool kLocal>
__device__ __forceinline__ void gather_raw_split(const uint16_t* row, const uint32_t* src, uint32_t tag,
                                                 Gathered& g, int32_t* status, const uint32_t* row_lds = nullptr) {
  const int l = lane_id(), w = wave_id();
  if (row != nullptr) {
    if (w == 0) {
      if (row_lds != nullptr) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the row's LDS copy has landed
#pragma unroll
        for (int i = 0; i < 8; ++i) g.raw[l + 64 * i] = row_lds[l + 64 * i];
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) g.raw[l + 64 * i] = *reinterpret_cast<const uint32_t*>(row + 2 * l + 128 * i);
      }
      // the group sums from the words just stored (LDS keeps a wave's order)
#pragma unroll 1
      for (int i = 0; i < 8; ++i) {
        const float sw = wave_sum(pair_sq(g.raw[l + 64 * i]));
        if (l == 0) g.ss[i] = sw;
      }
    }
  } else {
    uint64_t x[1];
    poll_local<1, kLocal>(src + 128 * w, 128, tag, x, status);
    const uint32_t word = ((uint32_t)x[0] & 0xffffu) | ((uint32_t)(x[0] >> 32) << 16);
    g.raw[l + 64 * w] = word;
    const float sw = wave_sum(pair_sq(word));
    if (l == 0) g.ss[w] = sw;
  }
  lds_barrier();
}

// Every wave, after gather_raw_split: the RMSNorm scale of g.raw from the
// gathering waves' group sums (the grouping gather_raw uses, so both give the
// same bits).
__device__ __forceinline__ float raw_scale(const Gathered& g) { return norm_scale(group_total(g.ss)); }

// Every wave, after a barrier behind the gather: words [64w, 64w + 64) of
// the RMSNorm'ed input (two roundings, Lfm2RMSNorm.forward,
// modeling_lfm2.py:54-59) with scale r into lds.
__device__ __forceinline__ void norm_words(const Gathered& g, float r, const uint32_t* gamma, uint32_t* lds) {
  const int i = kWave * wave_id() + lane_id();
  const uint32_t x = g.raw[i], gw = gamma[i];
  const float a = round_bf16(round_bf16(lo_f32(x) * r) * lo_f32(gw));
  const float b = round_bf16(round_bf16(hi_f32(x) * r) * hi_f32(gw));
  lds[i] = bf16_pair(a, b);
}
__device__ __forceinline__ void norm_words(const Gathered& g, const uint32_t* gamma, uint32_t* lds) {
  norm_words(g, g.scale, gamma, lds);
}
// The same with the thread's weight word gw (norm_word) in a register.
__device__ __forceinline__ void norm_words_reg(const Gathered& g, float r, uint32_t gw, uint32_t* lds) {
  const int i = kWave * wave_id() + lane_id();
  const uint32_t x = g.raw[i];
  const float a = round_bf16(round_bf16(lo_f32(x) * r) * lo_f32(gw));
  const float b = round_bf16(round_bf16(hi_f32(x) * r) * hi_f32(gw));
  lds[i] = bf16_pair(a, b);
}
// The thread's word 64w + lane of a BF16 norm weight vector in global memory
// (the weight stream; it stays in L2 across tokens). Requested before a
// gather's polls, it arrives with them.
__device__ __forceinline__ uint32_t norm_word(const uint16_t* gamma) {
  return reinterpret_cast<const uint32_t*>(gamma)[kWave * wave_id() + lane_id()];
}
static_assert(kStepWaves * kWave == kNormWords, "one normed word per thread");

// The block's residual rows 64jj + lane from the raw copy written by gather_raw
// (same wave, so no barrier is needed).
__device__ __forceinline__ float residual_from_raw(const uint32_t* raw) {
  const int r = kResRows * blk_jj() + lane_id();
  const uint32_t w = raw[r >> 1];
  return (r & 1) ? hi_f32(w) : lo_f32(w);
}

// Waits until a local h buffer holds the whole vector of epoch `tag` (the
// values are not kept).
template <bool kLocal>
__device__ __forceinline__ void wait_h(const uint32_t* src, uint32_t tag, int32_t* status) {
  uint64_t w[8];
  poll_local<8, kLocal>(src, kHidden, tag, w, status);
}

// A local vector of `words` values (no norm) into LDS.
template <int N, bool kLocal>
__device__ __forceinline__ void gather_plain(const uint32_t* src, int words, uint32_t tag, uint32_t* lds,
                                             int32_t* status) {
  uint64_t w[N];
  poll_local<N, kLocal>(src, words, tag, w, status);
  words_to_lds<N>(w, words, lds);
}

// Block-wide gather_plain: wave w < N polls load w of it (words
// [128w, 128w + 128) of the source); ends with a block barrier.
template <int N, bool kLocal>
__device__ __forceinline__ void gather_plain_split(const uint32_t* src, int words, uint32_t tag, uint32_t* lds,
                                                   int32_t* status) {
  const int w = wave_id();
  if (w < N) {
    uint64_t x[1];
    poll_local<1, kLocal>(src + 128 * w, words - 128 * w, tag, x, status);
    words_to_lds<1>(x, words - 128 * w, lds + 64 * w);
  }
  lds_barrier();
}

// R: the partial sums of this block's residual rows from the eight XCDs
// (the blocks (y, jj), y = 0..7, of the active group), summed in a fixed
// order identical on every XCD: ((p0 + p1) + (p2 + p3)) + ((p4 + p5) +
// (p6 + p7)). Returns the sum for row 64jj + lane in every lane.
__device__ __forceinline__ float reduce_partials(const uint64_t* gp, uint32_t tag, int32_t* status) {
  const int l = lane_id();
  const uint64_t* src = gp + (size_t)blk_jj() * kXcds * kResRows;
  Poll poll(status);
  uint64_t w[kXcds];
  while (true) {
#pragma unroll
    for (int i = 0; i < kXcds; ++i) w[i] = coherent_load64(src + l + kResRows * i);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kXcds; ++i) ok = ok && (uint32_t)(w[i] >> 32) == tag;
    if (__all(ok) || !poll.again()) break;
  }
  float p[kXcds];
#pragma unroll
  for (int i = 0; i < kXcds; ++i) p[i] = __uint_as_float((uint32_t)w[i]);
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

// R phase (wave 0): h[r] = bf16(h[r] + bf16(sum of partials)) for the
// block's 64 rows (lane l carries h[64jj + l] in `hres`), published to the
// XCD's local h buffer `dst`.
template <bool kLocal>
__device__ __forceinline__ void run_residual(const uint64_t* gp, uint32_t tag_gp, float& hres,
                                             uint32_t* dst, uint32_t tag_out, int32_t* status) {
  const float s = reduce_partials(gp, tag_gp, status);
  hres = round_bf16(hres + round_bf16(s));
  local_store32<kLocal>(dst + kResRows * blk_jj() + lane_id(), tagged(hres, tag_out));
}

// Block-wide run_residual: wave w polls the partials of XCD w (512 bytes)
// into red[w]; after a block barrier wave 0 sums them in reduce_partials'
// order, adds the residual and publishes (same bits as run_residual).
template <bool kLocal>
__device__ __forceinline__ void run_residual_split(const uint64_t* gp, uint32_t tag_gp, float& hres,
                                                   uint32_t* dst, uint32_t tag_out, int32_t* status,
                                                   float (*red)[kResRows]) {
  const int l = lane_id(), w = wave_id();
  const uint64_t* src = gp + ((size_t)blk_jj() * kXcds + w) * kResRows;
  Poll poll(status);
  uint64_t x;
  while (true) {
    x = coherent_load64(src + l);
    if (__all((uint32_t)(x >> 32) == tag_gp) || !poll.again()) break;
  }
  red[w][l] = __uint_as_float((uint32_t)x);
  lds_barrier();
  if (w == 0) {
    float p[kXcds];
#pragma unroll
    for (int i = 0; i < kXcds; ++i) p[i] = red[i][l];
    const float s = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    hres = round_bf16(hres + round_bf16(s));
    local_store32<kLocal>(dst + kResRows * blk_jj() + l, tagged(hres, tag_out));
  }
}
static_assert(kStepWaves == kXcds, "one wave per XCD's partials");

// The block's residual rows from a complete local h buffer (or the embedding
// row), for callers that do not carry them in registers.
template <bool kLocal>
__device__ __forceinline__ float load_residual(const uint16_t* row, const uint32_t* src, uint32_t tag,
                                               int32_t* status) {
  const int r = kResRows * blk_jj() + lane_id();
  if (row != nullptr) return bf16_to_f32(row[r]);
  uint64_t w[1];
  Poll poll(status);
  while (true) {
    local_load64<1, kLocal>(src, 4 * (r & ~1), w);
    const uint32_t word = (uint32_t)(w[0] >> (32 * (r & 1)));
    if (__all(tag_ok(word, tag)) || !poll.again()) break;
  }
  return tagged_value((uint32_t)(w[0] >> (32 * (r & 1))));
}

// ------------------------------------------------------------------ compute phases (every wave)

// P1 and P3: each wave stores its own outputs as soon as they are computed
// (no block barrier before the publish): the consumer's poll waits for every
// word anyway, and the LDS the waves read stays untouched until the next
// barrier, since the next phase writes the other vector buffer first.

// P1, conv layer: channel c = 128x + 8jj + k: [B, C, x] = in_proj rows . n,
// gated short conv (conv_gate_channel), state update; y -> local ly[8jj + k].
template <bool kLocal>
__device__ __forceinline__ void compute_conv(const Slabs& s, const uint32_t* lds, uint16_t* state,
                                             uint32_t tag_out, StepOut& o, const StepBufs& b) {
  const int k = wave_id();
  const uint16_t w[3] = {(uint16_t)__builtin_amdgcn_readlane(s.taps, 0),
                         (uint16_t)__builtin_amdgcn_readlane(s.taps, 1),
                         (uint16_t)__builtin_amdgcn_readlane(s.taps, 2)};
  uint16_t st[3] = {0, (uint16_t)__builtin_amdgcn_readlane(s.state, 3),
                    (uint16_t)__builtin_amdgcn_readlane(s.state, 4)};
  // the taps over the two kept state values do not depend on the products:
  // formed first, so only the new value's tap follows the dot products
  const float s01 = conv_state_taps(w, st);
  float d[3];
  rows_dot1024<3>(s.a, lds, d);
  const float B = round_bf16(d[0]), C = round_bf16(d[1]), X = round_bf16(d[2]);
  LFM25_TRACE_WAVE(o, 0);
  if (lane_id() == 0) {
    const int c = kXcdCols * blk_xcd() + kBlockChan * blk_jj() + k;
    const float yv = conv_gate_channel_from(B, C, X, w, st, s01, state + c * kConvTaps);
    local_store32<kLocal>(ly_of(b, blk_xcd()) + kBlockChan * blk_jj() + k, tagged(yv, tag_out));
  }
  LFM25_TRACE_WAVE(o, 1);
}

// P1, attention layer: entries 16jj + 2k + {0, 1} of the XCD's q/k/v list,
// qkv = bf16(W . n) -> local lq.
template <bool kLocal>
__device__ __forceinline__ void compute_qkv(const Slabs& s, const uint32_t* lds, uint32_t tag_out,
                                            StepOut& o, const StepBufs& b) {
  const int k = wave_id();
  float d[2];
  rows_dot1024<2>(s.a, lds, d);
  LFM25_TRACE_WAVE(o, 0);
  if (lane_id() < 2)
    local_store32<kLocal>(lq_of(b, blk_xcd()) + kBlockQkv * blk_jj() + 2 * k + lane_id(),
                          tagged(lane_id() == 0 ? d[0] : d[1], tag_out));
  LFM25_TRACE_WAVE(o, 1);
}

// The block's 64 partial sums -> gp[jj][x][0..64): one store instruction
// after a block barrier (every thread of the block calls it). Stores from
// every wave would cost the decode kernels a few registers they do not have.
__device__ __forceinline__ void publish_partials(const StepOut& o, uint64_t* gp, uint32_t tag) {
  LFM25_TRACE_WAVE(o, 0);
  lds_barrier();
  if (wave_id() == 1)
    coherent_store64(gp + ((size_t)blk_jj() * kXcds + blk_xcd()) * kResRows + lane_id(),
                     tagged_partial(o.part[lane_id()], tag));
  LFM25_TRACE_WAVE(o, 1);
}

// P2: partial sums of rows 64jj + 8k + [0, 8) over the XCD's 128 columns;
// lanes 16q .. 16q + 15 hold row 4t + q of load t.
__device__ __forceinline__ void compute_proj(const Slabs& s, const uint32_t* lds, uint32_t tag_out,
                                             StepOut& o, uint64_t* gp) {
  const int k = wave_id();
  const int l = lane_id();
  const u32x4 x = lds16(lds, l & 15);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float v = row16_sum(dot8(s.b[t], x, 0.0f));
    if ((l & 15) == 0) o.part[8 * k + 4 * t + (l >> 4)] = v;
  }
  publish_partials(o, gp, tag_out);
}

// P3: g[f] = bf16(bf16(silu(bf16(w1[f] . n))) * bf16(w3[f] . n)) for the
// wave's FFN columns (Lfm2MLP.forward, modeling_lfm2.py:135-136)
// -> local lg[20jj + ...].
template <bool kLocal>
__device__ __forceinline__ void compute_up(const Slabs& s, const uint32_t* lds, uint32_t tag_out,
                                           StepOut& o, const StepBufs& b) {
  const int k = wave_id();
  float d[6];  // w1[f], w3[f], w1[f + 1], w3[f + 1], w1[f + 2], w3[f + 2]
  rows_dot1024<4>(s.c, lds, d);
  // waves with two columns skip the third (wave-uniform branch)
  if (ffn_count(k) == 3) rows_dot1024<2>(s.c + 8, lds, d + 4);
  else d[4] = d[5] = 0.0f;
  const int l = lane_id();
  LFM25_TRACE_WAVE(o, 0);
  if (l < ffn_count(k)) {
    const float a = l == 0 ? d[0] : l == 1 ? d[2] : d[4];
    const float g = l == 0 ? d[1] : l == 1 ? d[3] : d[5];
    local_store32<kLocal>(lg_of(b, blk_xcd()) + kBlockFfn * blk_jj() + ffn_first(k) + l,
                          tagged(silu_bf16(round_bf16(a)) * round_bf16(g), tag_out));
  }
  LFM25_TRACE_WAVE(o, 1);
}

// P4: partial sums of rows 64jj + 8k + [0, 8) over the XCD's 320 FFN
// columns; lanes 8q .. 8q + 7 hold row q, chunks (l & 7) + 8i, i < 5.
__device__ __forceinline__ void compute_down(const Slabs& s, const uint32_t* lds, uint32_t tag_out,
                                             StepOut& o, uint64_t* gp) {
  const int k = wave_id();
  const int l = lane_id();
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 5; ++i) acc = dot8(s.d[i], lds16(lds, (l & 7) + 8 * i), acc);
  const float v = group_sum<8>(acc);
  if ((l & 7) == 0) o.part[8 * k + (l >> 3)] = v;
  publish_partials(o, gp, tag_out);
}

// ------------------------------------------------------------------ attention (all blocks of the group)
//
// Up to 256 cached positions (four passes of 64), block (x, h) computes
// query head h of KV head x alone (h = 0, 1), as four register passes, and
// publishes that head's BF16 context.
// Beyond that, KV head x runs on the 16 active blocks of XCD x: block jj owns
// the passes jj, jj + 16, jj + 32, jj + 48 of the cache, so the 4,096-position
// capacity is covered by four passes per block. Either way a block's
// positions are loaded into registers a layer ahead (with the QK norm weights
// and the RoPE row), laid out for whole-position work: lane l of wave w holds
// half l >> 5 of the key of one position and two dimensions of the values of
// 16 positions (attn_prefetch), so a score is 16 v_dot2 and one cross-half
// add, and the context needs no reduction over lanes.
// Every block gathers the head's q/k/v and applies the QK norm and RoPE; the
// scores of its positions give a local maximum m_b and sum z_b =
// sum exp(s_j - m_b) per query head, exchanged within the XCD; every block
// then forms the global m = max m_b, z = sum_b z_b exp(m_b - m) (block
// order), and its share of the context with the reference's probabilities
// p_j = bf16(exp(s_j - m) / z), published as FP32 partials that the next
// phase sums in block order before the one BF16 rounding.
constexpr int kAttnSlots = kStepThreads / 8;  // positions per pass: 64
constexpr int kAttnPrefetch = 4;              // passes per block, all held in registers
constexpr int kAttnPassBytes = kAttnSlots * kHeadDim * 2;
constexpr int kAttnLocal = kAttnSlots * kAttnPrefetch;  // positions per block: 256
// Positions below which blocks (x, 0) and (x, 1) attend alone, one query
// head each (at most kAttnLocal, the positions one block holds); from there
// on the 16 blocks split the cache.
#ifndef LFM25_ATTN_SINGLE_BELOW
#define LFM25_ATTN_SINGLE_BELOW kAttnLocal
#endif
constexpr int kAttnSingleBelow = LFM25_ATTN_SINGLE_BELOW;
static_assert(kAttnSingleBelow >= 0 && kAttnSingleBelow <= kAttnLocal, "a block holds at most kAttnLocal");

// Blocks of the single path: block (x, h) takes query head h of KV head x.
constexpr int kSingleBlocks = 2;
// Single path: wave w holds positions [32w, 32w + 32) (kAttnLocal over the
// eight waves); for the context, each half-wave 16 of them.
constexpr int kSinglePerWave = 32;
constexpr int kSingleHalf = 16;
static_assert(kSinglePerWave * kStepWaves == kAttnLocal && 2 * kSingleHalf == kSinglePerWave,
              "the single path covers a block's positions");

// Which attention path code is compiled for: chosen per position at run time,
// or fixed to blocks (x, 0..1) alone / to the split over the 16 blocks. The
// persistent decode compiles a token of each fixed kind, so the registers of
// one path do not burden the other.
enum AttnPath { kAttnAny = 0, kAttnOne = 1, kAttnSplit = 2 };
// Whether position `past` attends on blocks (x, 0..1) alone.
template <int kPath>
__device__ __forceinline__ bool attn_single(int past) {
  if constexpr (kPath == kAttnOne) return true;
  else if constexpr (kPath == kAttnSplit) return false;
  else return past < kAttnSingleBelow;
}
// Cache pass of register pass i of this block.
__device__ __forceinline__ int attn_pass(bool single, int i) { return single ? i : blk_jj() + kGroupBlocks * i; }
static_assert(kMaxCapacity <= kAttnLocal * kGroupBlocks, "every cached position has a block and a register pass");
constexpr int kAttnStats = 4;  // m, z of query head 0, then of query head 1

struct AttnKV {
  u32x4 k[kAttnPrefetch];
  u32x4 v[kAttnPrefetch];
  uint32_t gamma_rope;  // lanes of waves 0..3: q or k norm weight (low half), and
  uint32_t cos_sin;     // the RoPE cos / sin of dimension `lane` (low / high half)
};

struct AttnSplitShared {
  float q[2][kHeadDim];                      // rotated query heads of this KV group
  float k_new[kHeadDim];                     // rotated key of the current position
  float v_new[kHeadDim];                     // value of the current position
  alignas(16) uint32_t qp[2][kHeadDim / 2];  // the same as BF16 pairs (single path)
  alignas(16) uint32_t kp[kHeadDim / 2];
  uint32_t vp[kHeadDim / 2];
  float score[2][kAttnLocal];                // scores of the block's positions
  float red[2][kStepWaves];
  float red_sum[2][kStepWaves];
  float stats[kGroupBlocks * kAttnStats];    // every block's (m, z) pairs
  float mz[4];                               // global m0, z0, m1, z1
  float ctx[kStepWaves][2][kHeadDim];
  float part[kGroupBlocks][2 * kHeadDim];    // the next phase: context partials of the 16 blocks
#ifdef LFM25_TRACE_ATTN
  uint64_t* atrace;                          // attention stamps (thread 0 of block 0)
  int acalls, aat;
#endif
};

// Cached rows [64 pass, 64 pass + 64) of one KV head that lie below `past`,
// as a descriptor over exactly those rows (empty when none is): reads beyond
// them return zeros without touching memory. The pass offset sits in the
// descriptor's base, not in the scalar offset of the load, because the
// hardware range check covers only the per-lane offset.
__device__ __forceinline__ BufRsrc kv_pass_rsrc(const uint16_t* rows, int past, int pass) {
  const int first = pass * kAttnSlots;
  const int n = past <= first ? 0 : min(past - first, kAttnSlots);
  return region_rsrc(rows + (n > 0 ? (size_t)first * kHeadDim : 0), n * kHeadDim * 2, true);
}

// Cache policy of the KV reads: the XCD-local variant reads rows that a
// block of the same XCD appended (through that XCD's L2); the coherent
// variant, whose blocks may sit on other XCDs than the appending block,
// reads them at device scope (sc1: past the reader's L2), as the appends of
// that variant are device-scope stores.
template <bool kLocal>
constexpr int kKvLoadAux = kLocal ? 0 : 16;

// One appended KV element: a plain store in the XCD-local variant (its
// readers share the writer's L2), a device-scope store otherwise.
template <bool kLocal>
__device__ __forceinline__ void kv_append(uint16_t* p, uint16_t v) {
  if constexpr (kLocal) *p = v;
  else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Issues the loads of `kv` for a layer whose attention runs at position
// `past` (block-wide; nothing waits for them here): the block's passes of
// the cached keys / values, the QK norm weights and the RoPE row.
template <int kPath, bool kLocal>
__device__ __forceinline__ void attn_prefetch(const uint16_t* keys, const uint16_t* values, int past,
                                              const uint16_t* q_gamma, const uint16_t* k_gamma,
                                              const uint16_t* rope_row, AttnKV& kv) {
  const bool single = attn_single<kPath>(past);
  // blocks that do not take part read nothing (an empty range)
  const int rows = single && blk_jj() >= kSingleBlocks ? 0 : past;
  const int w = wave_id(), l = lane_id();
  if (single) {
    // lane l of wave w: the key of position 32w + (l & 31), dimensions
    // 32 (l >> 5) .. + 32 (four 16-byte loads), and the values of
    // positions 32w + 16 (l >> 5) + i, i < 16, dimensions 2 (l & 31) and
    // + 1 (one word each). One descriptor over the cached rows: every offset
    // is per lane, so the hardware range check covers it.
    const BufRsrc rk = region_rsrc(keys, rows * kHeadDim * 2, true);
    const BufRsrc rv = region_rsrc(values, rows * kHeadDim * 2, true);
    const int ok = (kSinglePerWave * w + (l & 31)) * kHeadDim * 2 + kHeadDim * (l >> 5);
    const int ov = (kSinglePerWave * w + kSingleHalf * (l >> 5)) * kHeadDim * 2 + 4 * (l & 31);
#pragma unroll
    for (int i = 0; i < kAttnPrefetch; ++i) {
      kv.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, ok + 16 * i, 0, kKvLoadAux<kLocal>);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        kv.v[i][e] = __builtin_amdgcn_raw_buffer_load_b32(rv, ov + (4 * i + e) * kHeadDim * 2, 0, kKvLoadAux<kLocal>);
    }
  } else {
    // the same lane layout over the block's pass attn_pass(false, w / 2),
    // positions 32 (w % 2) .. + 32 of it, through the pass's descriptor
    const int pass = attn_pass(false, w >> 1);
    const BufRsrc rk = kv_pass_rsrc(keys, rows, pass), rv = kv_pass_rsrc(values, rows, pass);
    const int ok = (kSinglePerWave * (w & 1) + (l & 31)) * kHeadDim * 2 + kHeadDim * (l >> 5);
    const int ov = (kSinglePerWave * (w & 1) + kSingleHalf * (l >> 5)) * kHeadDim * 2 + 4 * (l & 31);
#pragma unroll
    for (int i = 0; i < kAttnPrefetch; ++i) {
      kv.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, ok + 16 * i, 0, kKvLoadAux<kLocal>);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        kv.v[i][e] = __builtin_amdgcn_raw_buffer_load_b32(rv, ov + (4 * i + e) * kHeadDim * 2, 0, kKvLoadAux<kLocal>);
    }
  }
  const BufRsrc rg = region_rsrc(w < 2 ? q_gamma : k_gamma, kHeadDim * 2, w < 3);
  const BufRsrc rr = region_rsrc(rope_row, 2 * kHeadDim * 2, w < 3);
  kv.gamma_rope = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rg, 2 * l, 0, 0);
  kv.cos_sin = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rr, 2 * l, 0, 0) |
               ((uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rr, 2 * l, kHeadDim * 2, 0) << 16);
}

// Position of the split path's score lane l of wave w: pass
// attn_pass(false, w / 2), position 32 (w % 2) + (l & 31) in it (the layout
// attn_prefetch loads); a lane's context positions are the 16 from
// 32 (w % 2) + 16 (l >> 5) of the same pass.
__device__ __forceinline__ int split_wave_base(int w) {
  return attn_pass(false, w >> 1) * kAttnSlots + kSinglePerWave * (w & 1);
}

// The score of the lane's position for query head hq (half l >> 5 of the
// dimensions in 16 v_dot2, then both halves added): the current position's
// key from LDS, cached ones from registers.
__device__ __forceinline__ float lane_score(const AttnKV& kv, const AttnSplitShared& sh, int hq, bool current) {
  const int half = lane_id() >> 5;
  const uint32_t* qp = sh.qp[hq] + 16 * half;
  u32x4 qv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 4 * i);
  float a = 0.0f;
  if (current) {
    const uint32_t* kp = sh.kp + 16 * half;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 kk = *reinterpret_cast<const u32x4*>(kp + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) a = dot2(kk[e], qv[i][e], a);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) a = dot2(kv.k[i][e], qv[i][e], a);
  }
  return half_swap_sum(a);
}

// Split path, block-wide: the scores of the block's positions of [0, past]
// for both query heads of the KV group, s_j = bf16(q.k_j) * 0.125 (eager
// semantics, modeling_lfm2.py:184-207), left in s[0..1] (the lane's
// position; -inf past `past`, and in sh.score for the context phase), and
// the block's statistics mz = (m0, z0, m1,
// z1): each wave's (m_w, z_w = sum of exp(s_j - m_w)) through LDS, one block
// barrier, then m = max m_w and z = sum_w z_w exp(m_w - m) in wave order
// (the combination the blocks' statistics take next, over blocks).
template <int kPath>
__device__ __forceinline__ void attn_split_stats(int past, const AttnKV& kv, AttnSplitShared& sh, float* mz,
                                                 float* s) {
  const int w = wave_id(), l = lane_id();
  const int base = split_wave_base(w);
  const bool any = base <= past;  // wave-uniform
  const int j = base + (l & 31);
  float mw[2] = {-INFINITY, -INFINITY}, zw[2] = {0.0f, 0.0f};
#pragma unroll
  for (int hq = 0; hq < 2; ++hq) {
    s[hq] = -INFINITY;
    if (any) {
      const float full = lane_score(kv, sh, hq, j == past);
      if (j <= past) s[hq] = round_bf16(full) * 0.125f;
      if ((l >> 5) == 0) sh.score[hq][kSinglePerWave * w + (l & 31)] = s[hq];
      mw[hq] = wave_max(s[hq]);
      const float e = j <= past ? expf(s[hq] - mw[hq]) : 0.0f;
      zw[hq] = wave_sum((l >> 5) == 0 ? e : 0.0f);
    }
    // one query head at a time: the second's q reads are not hoisted into
    // the first's registers
    __builtin_amdgcn_sched_barrier(0);
  }
  if (l == 0) {
    sh.red[0][w] = mw[0];
    sh.red[1][w] = mw[1];
    sh.red_sum[0][w] = zw[0];
    sh.red_sum[1][w] = zw[1];
  }
  LFM25_ATTN_STAMP(3);
  lds_barrier();
  LFM25_ATTN_STAMP(4);
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

// The block's share of the context of both query heads under the global
// mz = (m0, z0, m1, z1) (the same in every thread): sum over its positions
// of bf16(exp(s_j - m) / z) v_j in FP32, lane-per-dimension (two dimensions
// of 16 positions per lane, with the p_j its wave wrote to LDS), returned per
// thread t < 128 (head t / 64, dimension t % 64). One block barrier.
template <int kPath>
__device__ __forceinline__ float attn_split_context(int past, const AttnKV& kv, AttnSplitShared& sh,
                                                   const float* mz) {
  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int half = l >> 5, lo = l & 31;
  const int base = split_wave_base(w);
  const bool any = base <= past;
  const int j = base + lo;
  float c[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  if (any) {
    const uint32_t vnew = sh.vp[lo];  // the current position's value (not cached yet)
    const int first = base + kSingleHalf * half;
    const bool has_past = past >= first && past < first + kSingleHalf;
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      // the lane's score (from the statistics phase), then p of the wave's
      // positions through LDS in its place (written and read by this wave)
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
      // cached values (zeros from `past` on), then the current position's
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
  LFM25_ATTN_STAMP(11);
  lds_barrier();
  LFM25_ATTN_STAMP(12);
  float out = 0.0f;
  if (tid < 2 * kHeadDim) {
    const int hq = tid / kHeadDim, d = tid % kHeadDim;
    out = sh.ctx[0][hq][d];
#pragma unroll
    for (int i = 1; i < kStepWaves; ++i) out += sh.ctx[i][hq][d];
  }
  return out;
}

// Block (x, hq) alone, hq < 2: query head hq of KV head x over the
// positions [0, past] held in registers (attn_prefetch's single layout),
// block-wide, with the reference's eager semantics (eager_attention_forward,
// modeling_lfm2.py:184-207): s_j = bf16(q.k_j) * 0.125, p_j = bf16(exp(s_j -
// m) / z) with m the maximum and z = sum_j exp(s_j - m), context sum_j p_j v_j
// in FP32, returned for thread d < 64 (dimension d).
//   scores: lane l of wave w takes position 32w + (l & 31), half l >> 5 of
//     the dimensions (16 v_dot2 of BF16 pairs), and the two halves are added
//     across the wave (no reduction over lanes otherwise);
//   softmax: each wave's (m_w, z_w = sum over its positions of
//     exp(s_j - m_w)) in LDS, one barrier, then m = max m_w and z = sum_w
//     z_w exp(m_w - m) in wave order (the combination the split path makes
//     over blocks) and p_j from exp(s_j - m);
//   context: lane l takes dimensions 2 (l & 31), + 1 over 16 of the wave's
//     positions (FMAs with the p_j its wave wrote to LDS), the half-waves are
//     added, and a barrier later thread d sums the eight waves in order.
// Waves whose positions all lie past `past` skip the arithmetic. Two block
// barriers.
template <int kPath>
__device__ __forceinline__ float attn_single_head(int past, int hq, const AttnKV& kv, AttnSplitShared& sh) {
  const int w = wave_id(), l = lane_id();
  const int half = l >> 5, lo = l & 31;
  const int base = kSinglePerWave * w;
  const bool any = base <= past;  // wave-uniform: the wave holds positions
  const int j = base + lo;        // this lane's score position
  float s = -INFINITY;
  if (any) {
    // q of the lane's half of the dimensions as BF16 pairs (broadcast reads)
    const uint32_t* qp = sh.qp[hq] + 16 * half;
    u32x4 qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 4 * i);
    float a = 0.0f;
    if (j == past) {
      // the current position's key is not in the cache yet
      const uint32_t* kp = sh.kp + 16 * half;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 kk = *reinterpret_cast<const u32x4*>(kp + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) a = dot2(kk[e], qv[i][e], a);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) a = dot2(kv.k[i][e], qv[i][e], a);
    }
    const float full = half_swap_sum(a);
    if (j <= past) s = round_bf16(full) * 0.125f;
  }
  LFM25_ATTN_STAMP(3);
  float m_w = -INFINITY, z_w = 0.0f;
  float e = 0.0f;
  if (any) {
    m_w = wave_max(s);
    e = j <= past ? expf(s - m_w) : 0.0f;
    z_w = wave_sum(half == 0 ? e : 0.0f);
  }
  if (l == 0) {
    sh.red[0][w] = m_w;
    sh.red_sum[0][w] = z_w;
  }
  lds_barrier();
  LFM25_ATTN_STAMP(4);
  // m, then z: lane i < 8 forms wave i's term, added in wave order (every
  // aligned group of 8 lanes holds the eight waves' values, so three DPP
  // steps give the maximum)
  const float mi = sh.red[0][l & (kStepWaves - 1)], zi = sh.red_sum[0][l & (kStepWaves - 1)];
  float m = fmaxf(mi, dpp_f32<kDppQuadXor1>(mi));
  m = fmaxf(m, dpp_f32<kDppQuadXor2>(m));
  m = fmaxf(m, dpp_f32<kDppRowHalfMirror>(m));
  const float ti = zi > 0.0f ? zi * expf(mi - m) : 0.0f;
  float z = lane_value(ti, 0);
#pragma unroll
  for (int i = 1; i < kStepWaves; ++i) z += lane_value(ti, i);
  LFM25_ATTN_STAMP(5);
  float c0 = 0.0f, c1 = 0.0f;
  if (any) {
    const uint32_t vnew = sh.vp[lo];  // the current position's value (not cached yet)
    const float p = j <= past ? round_bf16(expf(s - m) / z) : 0.0f;
    // p of the lane's context positions base + 16 half + i, through the
    // wave's own LDS slots (written and read by this wave, so in order)
    if (half == 0) sh.score[0][base + lo] = p;
    float pj[kSingleHalf];
#pragma unroll
    for (int i = 0; i < kSingleHalf / 4; ++i) {
      const u32x4 pv = *reinterpret_cast<const u32x4*>(&sh.score[0][base + kSingleHalf * half + 4 * i]);
      pj[4 * i] = __uint_as_float(pv.x);
      pj[4 * i + 1] = __uint_as_float(pv.y);
      pj[4 * i + 2] = __uint_as_float(pv.z);
      pj[4 * i + 3] = __uint_as_float(pv.w);
    }
    // cached values (zeros from `past` on), then the current position's
#pragma unroll
    for (int i = 0; i < kSingleHalf; ++i) {
      const uint32_t vw = kv.v[i >> 2][i & 3];
      c0 = fmaf(pj[i], lo_f32(vw), c0);
      c1 = fmaf(pj[i], hi_f32(vw), c1);
    }
    const int first = base + kSingleHalf * half;
    const float pp = lane_value(p, past - base < kSinglePerWave ? past - base : 0);
    if (past >= first && past < first + kSingleHalf) {
      c0 = fmaf(pp, lo_f32(vnew), c0);
      c1 = fmaf(pp, hi_f32(vnew), c1);
    }
    c0 = half_swap_sum(c0);
    c1 = half_swap_sum(c1);
  }
  if (half == 0) {
    sh.ctx[w][0][2 * lo] = c0;
    sh.ctx[w][0][2 * lo + 1] = c1;
  }
  LFM25_ATTN_STAMP(6);
  lds_barrier();
  LFM25_ATTN_STAMP(7);
  float ctx = 0.0f;
  if (threadIdx.x < kHeadDim) {
    ctx = sh.ctx[0][0][threadIdx.x];
#pragma unroll
    for (int i = 1; i < kStepWaves; ++i) ctx += sh.ctx[i][0][threadIdx.x];
  }
  return ctx;
}

// KV head x, block-wide, on every block (x, jj) of the active group (from
// kAttnSingleBelow positions on) or on blocks (x, 0..1) alone, one query head
// each: gather q0, q1, k, v of the head from the local lq, QK RMSNorm +
// RoPE, KV append at `pos` (block jj = 0), the block's (m_b, z_b) -> local
// ls (tag_st), the global (m, z), the block's FP32 context partial -> local
// lc (tag_out); alone, the head's BF16 context -> local ly (tag_out) and
// tag_st goes unused. `kv` holds what attn_prefetch loaded for this layer
// and position.
//
// kPart splits the work for launches in which blocks must not wait for each
// other: kAttnWhole does all of it (the persistent decode, whose blocks are
// co-resident by construction); kAttnHalfStats stops after publishing the
// block's statistics (or, alone, after the whole attention) and
// kAttnHalfContext, launched after it, redoes the local part without the append
// or the publish, and finishes from the published statistics. Both halves
// compute the same values, so the results do not depend on the split.
enum AttnPart { kAttnWhole = 0, kAttnHalfStats = 1, kAttnHalfContext = 2 };
template <bool kLocal, int kPath, int kPart = kAttnWhole>
__device__ __forceinline__ void run_attention(uint32_t tag_qkv, uint32_t tag_st, uint16_t* keys, uint16_t* values,
                                              int pos, const StepBufs& b, uint32_t tag_out, const AttnKV& kv,
                                              AttnSplitShared& sh) {
  const int w = wave_id(), l = lane_id(), x = blk_xcd(), jj = blk_jj();
  const bool single = attn_single<kPath>(pos);
  if (single && (jj >= kSingleBlocks || kPart == kAttnHalfContext)) return;
  const bool append = jj == 0 && kPart != kAttnHalfContext;
  LFM25_ATTN_STAMP(0);
  if (w < 4) {
    // wave w polls entry 64 w + lane of the list (q0 | q1 | k | v), 64 each
    const int e = kHeadDim * w + l;
    uint64_t wd[1];
    Poll poll(b.status());
    while (true) {
      local_load64<1, kLocal>(lq_of(b, x), 4 * (e & ~1), wd);
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
    {
      // q, k and v also as BF16 pairs (the lane-per-position products)
      const float hi = dpp_f32<kDppQuadXor1>(val);
      if ((l & 1) == 0) {
        uint32_t* dst = w < 2 ? sh.qp[w] : w == 2 ? sh.kp : sh.vp;
        dst[l >> 1] = bf16_pair(val, hi);
      }
    }
  }
  LFM25_ATTN_STAMP(1);
  lds_barrier();
  LFM25_ATTN_STAMP(2);
  if (single) {
    // block (x, h) holds every position of query head h: its (m, z) are the
    // global ones and its context the whole one (BF16 -> local ly[64h ..],
    // as a conv layer's y)
    const float ctx = attn_single_head<kPath>(pos, jj, kv, sh);
    if (threadIdx.x < kHeadDim)
      local_store32<kLocal>(ly_of(b, x) + kHeadDim * jj + threadIdx.x, tagged(ctx, tag_out));
    LFM25_ATTN_STAMP(13);
    LFM25_ATTN_NEXT();
    return;
  }
  float mz[kAttnStats];
  {
    float sc[2];  // the lane's scores (kept in LDS for the context phase)
    attn_split_stats<kPath>(pos, kv, sh, mz, sc);
  }
  if (kPart != kAttnHalfContext && threadIdx.x < kAttnStats)
    local_store64<kLocal>(ls_of(b, x) + kAttnStats * jj + threadIdx.x, tagged_partial(mz[threadIdx.x], tag_st));
  if constexpr (kPart == kAttnHalfStats) return;
  if (w == 0) {
    // lane l: word l = stat l % 4 of block l / 4
    uint64_t sw[1];
    Poll poll(b.status());
    while (true) {
      local_load64<1, kLocal>(ls_of(b, x), 8 * l, sw);
      if (__all((uint32_t)(sw[0] >> 32) == tag_st) || !poll.again()) break;
    }
    sh.stats[l] = __uint_as_float((uint32_t)sw[0]);
    if (l < 2) {
      // global (m, z) of query head l, summed in block order (blocks without
      // positions report m = -inf, z = 0)
      float m = -INFINITY;
      for (int i = 0; i < kGroupBlocks; ++i) m = fmaxf(m, sh.stats[kAttnStats * i + 2 * l]);
      float z = 0.0f;
      for (int i = 0; i < kGroupBlocks; ++i) {
        const float zb = sh.stats[kAttnStats * i + 2 * l + 1];
        if (zb > 0.0f) z += zb * expf(sh.stats[kAttnStats * i + 2 * l] - m);
      }
      sh.mz[2 * l] = m;
      sh.mz[2 * l + 1] = z;
    }
  }
  lds_barrier();
  const float gmz[kAttnStats] = {sh.mz[0], sh.mz[1], sh.mz[2], sh.mz[3]};
  const float part = attn_split_context<kPath>(pos, kv, sh, gmz);
  if (threadIdx.x < 2 * kHeadDim)
    local_store64<kLocal>(lc_of(b, x) + 2 * kHeadDim * jj + threadIdx.x, tagged_partial(part, tag_out));
}

// The context of XCD x's two query heads for the next phase: the 16 blocks'
// FP32 partials (every wave polls 256 words), summed in block order and
// rounded once -> lds as BF16 pairs (kLyWords / 2 words). Block-wide; ends
// with a block barrier.
template <bool kLocal>
__device__ __forceinline__ void gather_context(const StepBufs& b, uint32_t tag, uint32_t* lds, AttnSplitShared& sh) {
  const int w = wave_id(), l = lane_id();
  constexpr int kPerWave = 4 * kWave;  // words per polling wave: 256 = two blocks' partials
  static_assert(kGroupBlocks * 2 * kHeadDim == kStepWaves * kPerWave, "every wave polls");
  {
    const uint64_t* src = lc_of(b, blk_xcd()) + kPerWave * w;
    uint64_t pw[4];
    Poll poll(b.status());
    while (true) {
      local_load64<4, kLocal>(src, 8 * l, pw);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) ok = ok && (uint32_t)(pw[i] >> 32) == tag;
      if (__all(ok) || !poll.again()) break;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int word = kPerWave * w + l + kWave * i;  // block word / 128, channel word % 128
      sh.part[word / (2 * kHeadDim)][word % (2 * kHeadDim)] = __uint_as_float((uint32_t)pw[i]);
    }
  }
  lds_barrier();
  if (threadIdx.x < kHeadDim) {
    float s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = 2 * threadIdx.x + u;
      s[u] = sh.part[0][c];
#pragma unroll
      for (int i = 1; i < kGroupBlocks; ++i) s[u] += sh.part[i][c];
    }
    lds[threadIdx.x] = bf16_pair(round_bf16(s[0]), round_bf16(s[1]));
  }
  lds_barrier();
}

// ------------------------------------------------------------------ head

// Final RMSNorm + tied head on every block: units of 4 vocabulary rows dealt
// round robin to the 2048 waves of the grid; each block's best (value, row)
// -> local lw[x][j]. A wave's first unit does not depend on h, so head_begin
// requests it ahead of the scan. The table is read with the default cache
// policy: it is also the embedding, and the next token's row is among it.
constexpr int kStepHeadRows = 4;
constexpr int kHeadWaves = kStepBlocks * kStepWaves;  // 2048
constexpr int kXcdWaves = kXcdBlocks * kStepWaves;    // 256
// The units of 4 rows a wave scans: XCD x takes a contiguous range of the
// table, and its 256 waves every 256th unit of it. kHeadOddShare / 1024 of an
// XCD's share can move from each odd XCD to the even one before it: with a
// forward scan every token the odd XCDs finished ~1 us late and 9% helped;
// since the scan direction alternates (L2 reuse), equal shares measure best
// (swept 0, 32, 48, 64, 96: 0 is 0.5% faster than 96). Which wave scans a row
// does not change the pick: candidates carry their row and the first-maximum
// order is total.
constexpr int kHeadOddShare = 0;
struct HeadSpan {
  int first, end;  // units first, first + 256, ... below end
};
__device__ __forceinline__ HeadSpan head_span(int units) {
  const int x = blk_xcd();
  const int base = units / kXcds, rem = units % kXcds;
  const int d = base * kHeadOddShare / 1024;
  int start = 0;
  for (int y = 0; y < x; ++y) start += base + (y < rem ? 1 : 0) + ((y & 1) ? -d : d);
  const int n = base + (x < rem ? 1 : 0) + ((x & 1) ? -d : d);
  return HeadSpan{start + blk_j() + kXcdBlocks * wave_id(), start + n};
}
__device__ __forceinline__ void head_rows(const uint16_t* table, int u, const uint16_t** rows) {
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) rows[r] = table + (size_t)(u * kStepHeadRows + r) * kHidden;
}
__device__ __forceinline__ int clamp_unit(int u, int units) { return u < units ? u : units - 1; }

struct HeadRows {
  Pack8 w[2 * kStepHeadRows];
};
// Unit u's rows (zeros when u is past the table).
__device__ __forceinline__ void head_load(const uint16_t* table, int units, int u, HeadRows& h) {
  const uint16_t* rows[kStepHeadRows];
  head_rows(table, clamp_unit(u, units), rows);
  const bool ok = u < units;
  const bool valid[kStepHeadRows] = {ok, ok, ok, ok};
  load_rows1024<kStepHeadRows, kBufCached>(h.w, rows, valid);
}
__device__ __forceinline__ void head_begin(const uint16_t* table, int vocab, HeadRows& first) {
  const HeadSpan sp = head_span(vocab / kStepHeadRows);
  head_load(table, sp.end, sp.first, first);
}

// A wave's first unit staged in LDS instead of registers (so nothing is held
// in registers while the loads are in flight): words [256c, 256c + 256) of
// rows[r] are chunk c of row r, lane l's 16 bytes at word 256c + 4l, as
// head_load would hold them. head_begin_lds issues the loads (nothing when
// the wave has no unit); head_from_lds waits for them and reads them back.
typedef __attribute__((address_space(3))) void LdsVoid;
typedef __attribute__((address_space(1))) void GlobalVoid;
// kHeadStaged units per wave (its first, first + 256, ...): rows[4k + r]
// holds row r of its k-th unit.
constexpr int kHeadStaged = 2;
// The staged units are copied with the non-temporal policy: read once, they
// should not evict the streamed rows that the next token's scan, running the
// other way, reads first from the XCD's L2.
constexpr int kHeadStageAux = kBufStream;
__device__ __forceinline__ void head_begin_lds(const uint16_t* table, int vocab, uint32_t (*rows)[kNormWords],
                                               int staged = kHeadStaged) {
  const HeadSpan sp = head_span(vocab / kStepHeadRows);
  const int l = lane_id();
  for (int k = 0; k < staged; ++k) {
    const int u = sp.first + kXcdWaves * k;
    if (u >= sp.end) return;
#pragma unroll
    for (int r = 0; r < kStepHeadRows; ++r) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
        __builtin_amdgcn_global_load_lds(
            (GlobalVoid*)(table + (size_t)(u * kStepHeadRows + r) * kHidden + (kHidden / 2) * c + 8 * l),
            (LdsVoid*)&rows[kStepHeadRows * k + r][(kNormWords / 2) * c], 16, 0, kHeadStageAux);
    }
  }
}
__device__ __forceinline__ void head_read_lds(const uint32_t (*rows)[kNormWords], HeadRows& h) {
  const int l = lane_id();
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&rows[r][(kNormWords / 2) * c + 4 * l]);
      h.w[2 * r + c].w[0] = v.x; h.w[2 * r + c].w[1] = v.y; h.w[2 * r + c].w[2] = v.z; h.w[2 * r + c].w[3] = v.w;
    }
  }
}
__device__ __forceinline__ void head_from_lds(const uint32_t (*rows)[kNormWords], HeadRows& h) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS copies have landed
  head_read_lds(rows, h);
}

// The scan of the wave's units: `staged` of them already requested into
// LDS by head_begin_lds (rows; waited for here, before the first streamed
// unit is requested, since both count in vmcnt), or else `first` in
// registers (staged = 0); the rest streamed with the next unit's loads in
// flight during each unit's products.
template <bool kLocal>
__device__ __forceinline__ void run_head(const uint32_t* lds, const uint16_t* table, int vocab,
                                         const StepBufs& b, uint32_t tag_out, float* red_v, int* red_i,
                                         const HeadRows& first, const uint32_t (*rows)[kNormWords] = nullptr,
                                         int staged = 0, bool reverse = false) {
  const int units = vocab / kStepHeadRows;
  float best = -INFINITY;
  int best_row = 0x7fffffff;
  const HeadSpan sp = head_span(units);
  const auto take = [&](const HeadRows& h, int u) {
    float d[kStepHeadRows];
    rows_dot1024<kStepHeadRows>(h.w, lds, d);
#pragma unroll
    for (int r = 0; r < kStepHeadRows; ++r) {
      const float v = round_bf16(d[r]);
      const int row = u * kStepHeadRows + r;
      if (better(v, row, best, best_row)) { best = v; best_row = row; }
    }
  };
  HeadRows cur, nxt;
  int u = sp.first;
  // With `reverse` the streamed units of the XCD's range, [s, sp.end) with
  // s = its start + 256 staged, are taken in decreasing order: every wave
  // maps its unit u to s + (sp.end - 1) - u (wave-uniform arithmetic), which
  // walks the same set of units from the other end.
  const int range_start = sp.first - blk_j() - kXcdBlocks * wave_id();
  const int mirror = reverse ? range_start + kXcdWaves * staged + sp.end - 1 : 0;
  const auto unit = [&](int v) { return reverse ? mirror - v : v; };
  if (staged > 0) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged units have landed
    const int u_stream = sp.first + kXcdWaves * staged;
    if (u_stream < sp.end) head_load(table, units, unit(u_stream), cur);
    for (int k = 0; k < staged && u < sp.end; ++k, u += kXcdWaves) {
      // the products read the staged rows straight from LDS (no wait on the
      // streamed unit, and no second unit's worth of registers)
      const uint32_t (*unit)[kNormWords] = rows + kStepHeadRows * k;
      const int l = lane_id();
      float p[kStepHeadRows];
#pragma unroll
      for (int r = 0; r < kStepHeadRows; ++r) {
        Pack8 w0, w1;
        const u32x4 a = *reinterpret_cast<const u32x4*>(&unit[r][4 * l]);
        const u32x4 c = *reinterpret_cast<const u32x4*>(&unit[r][kNormWords / 2 + 4 * l]);
        w0.w[0] = a.x; w0.w[1] = a.y; w0.w[2] = a.z; w0.w[3] = a.w;
        w1.w[0] = c.x; w1.w[1] = c.y; w1.w[2] = c.z; w1.w[3] = c.w;
        p[r] = dot8(w1, lds16(lds, 64 + l), dot8(w0, lds16(lds, l), 0.0f));
      }
      const float v4 = wave_totals4<kStepHeadRows>(p);
#pragma unroll
      for (int r = 0; r < kStepHeadRows; ++r) {
        const float v = round_bf16(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v4), r)));
        const int row = u * kStepHeadRows + r;
        if (better(v, row, best, best_row)) { best = v; best_row = row; }
      }
    }
  } else {
    cur = first;
  }
  for (; u < sp.end; u += kXcdWaves) {
    if (u + kXcdWaves < sp.end) head_load(table, units, unit(u + kXcdWaves), nxt);
    take(cur, unit(u));
    cur = nxt;
  }
  if (lane_id() == 0) { red_v[wave_id()] = best; red_i[wave_id()] = best_row; }
  lds_barrier();
  if (threadIdx.x == 0) {
    float bv = red_v[0];
    int bi = red_i[0];
    for (int i = 1; i < kStepWaves; ++i)
      if (better(red_v[i], red_i[i], bv, bi)) { bv = red_v[i]; bi = red_i[i]; }
    local_store64<kLocal>(lw_of(b, blk_xcd()) + blk_j(), tagged_candidate(bv, bi, tag_out));
  }
}

// First maximum over the candidates held one per lane (value -INF, row
// INT_MAX for lanes without one); the winner in every lane.
__device__ __forceinline__ void wave_pick(float& bv, int& bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
}

__device__ __forceinline__ bool candidate_ok(uint64_t c, uint32_t tag) {
  return ((uint32_t)(c >> 32) & 0xffffu) == tag;
}
__device__ __forceinline__ void candidate_of(uint64_t c, float& v, int& row) {
  v = __uint_as_float((uint32_t)c);
  row = (int)((uint32_t)(c >> 48));
}

// Wave 0 of a group-0 block: the XCD's 32 block candidates -> the XCD winner
// (same on every block of the XCD) -> global gw[jj][x].
template <bool kLocal>
__device__ __forceinline__ void pick_xcd(const StepBufs& b, uint32_t tag_cand, uint32_t tag_out) {
  const int l = lane_id();
  const int x = blk_xcd();
  uint64_t w[1];
  Poll poll(b.status());
  while (true) {
    local_load64<1, kLocal>(lw_of(b, x), 8 * l, w);
    if (__all(l >= kXcdBlocks || candidate_ok(w[0], tag_cand)) || !poll.again()) break;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (l < kXcdBlocks) candidate_of(w[0], bv, bi);
  wave_pick(bv, bi);
  if (l == 0) coherent_store64(b.gw() + kXcds * blk_jj() + x, tagged_candidate(bv, bi, tag_out));
}

// Wave 0 of a group-0 block: the eight XCD winners -> the token (first
// maximum), every lane. With a table of `vocab` BF16 rows and LDS room for
// eight rows, each XCD winner's row is requested into slot y of `rows` as
// soon as that winner arrives, so the next token's first layer finds its
// input in LDS; *slot is then the winner's slot, or -1 when its row was not
// requested (the row-to-LDS copies are in flight on return:
// gather_raw_split waits for them). An XCD whose waves scanned no rows (a
// table of fewer than 32 rows) reports the placeholder row 0xffff (the
// 16-bit field of INT_MAX); only rows below `vocab` are requested.
__device__ __forceinline__ int pick_global(const StepBufs& b, uint32_t tag, const uint16_t* table = nullptr,
                                           uint32_t (*rows)[kNormWords] = nullptr, int* slot = nullptr,
                                           int vocab = 0) {
  const int l = lane_id();
  const uint64_t* src = b.gw() + kXcds * blk_jj();
  Poll poll(b.status());
  uint64_t w = 0;
  uint32_t seen = 0;  // XCD winners that arrived
  uint32_t have = 0;  // XCD winners whose rows are requested
  while (true) {
    w = l < kXcds ? coherent_load64(src + l) : 0;
    const bool ok = l < kXcds && candidate_ok(w, tag);
    if (table != nullptr) {
      uint32_t fresh = (uint32_t)__ballot(ok) & ~seen;
      seen |= fresh;
      while (fresh != 0) {
        const int y = __builtin_ctz(fresh);
        fresh &= fresh - 1;
        const int row = __builtin_amdgcn_readlane((int)(uint32_t)(w >> 48), y);
        if (row >= vocab) continue;  // wave-uniform: a placeholder, no row to copy
        have |= 1u << y;
#pragma unroll
        for (int c = 0; c < 2; ++c)
          __builtin_amdgcn_global_load_lds((GlobalVoid*)(table + (size_t)row * kHidden + (kHidden / 2) * c + 8 * l),
                                           (LdsVoid*)&rows[y][(kNormWords / 2) * c], 16, 0, 0);
      }
    }
    if (__all(l >= kXcds || ok) || !poll.again()) break;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (l < kXcds) candidate_of(w, bv, bi);
  const int own = bi;
  wave_pick(bv, bi);
  if (slot != nullptr) {
    const uint64_t from = __ballot(l < kXcds && own == bi);
    const int y = from != 0 ? __builtin_ctzll(from) : -1;
    *slot = y >= 0 && ((have >> y) & 1u) != 0 ? y : -1;
  }
  return bi;
}

}  // namespace lfm25
