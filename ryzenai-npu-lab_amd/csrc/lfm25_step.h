// Block-level decode stages that exchange activations through tagged words.
//
// Every activation value that crosses blocks travels as a 32-bit word
// [bf16 value | 16-bit epoch tag], written and read with relaxed agent-scope
// atomics (coherent across the eight XCDs without any L2 writeback or
// invalidate). A consumer polls the words it needs until every tag equals
// the epoch of the stage that produced them, so the data itself is the
// barrier: no counters, no fences, no contention. Epochs advance by one per
// stage and are never reused between two consecutive writes of one buffer.
//
// Each stage is split in two halves so the persistent kernel can run them as
// a software pipeline:
//   prefetch_*  issues the loads of everything the stage needs that does not
//               depend on activations -- its weight rows, conv taps and conv
//               state -- into a register Slab (norm weights sit in LDS);
//   run_*       waits for the input vector (wave 0 polls it into LDS and
//               normalises it when the stage starts with an RMSNorm), then
//               the compute waves finish their rows from registers and LDS.
// A stage's successor is prefetched right after the stage's own dot
// products, so the weight loads overlap the next stage's wait for its input.
// Wave 0 of every block only gathers: vector loads complete in order, so a
// wave with weight loads in flight could not see its polled words any sooner
// than those loads land.
//
// Units are dealt to the compute waves (waves 1..7) block-major
// (cw = block + (wave - 1) * blocks), so every stage spreads over all CUs and
// XCDs. The wave that owns output row r of out_proj / o_proj also owns row r
// of w2, so it carries h[r] in a register from one residual add to the next.
#pragma once
#include "lfm25_stages.h"

namespace lfm25 {

constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / kWave;
constexpr int kStepBlocks = 256;  // grid of every block-level stage
constexpr int kStepStatusTimeout = 4;
// Poll time-out in s_memrealtime ticks (100 MHz): 5 s.
constexpr uint64_t kPollTimeout = 500000000ull;

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

// Candidate word: [value f32 | row (16) | tag (16)].
__device__ __forceinline__ uint64_t tagged_candidate(float v, int row, uint32_t tag) {
  return (uint64_t)__float_as_uint(v) | ((uint64_t)(((uint32_t)row << 16) | tag) << 32);
}

// Bounded waiting: false once this wait timed out or any block flagged a
// time-out (status bit 2), so every wave of the grid always drains.
struct Poll {
  int32_t* status;
  uint64_t t0;
  uint32_t iter;
  __device__ explicit Poll(int32_t* s) : status(s), t0(0), iter(0) {}
  __device__ bool again() {
    if (iter == 0) t0 = __builtin_amdgcn_s_memrealtime();
    ++iter;
    if ((iter & 15) == 0) {
      if (coherent_load32(status) & kStepStatusTimeout) return false;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kPollTimeout) {
        __hip_atomic_fetch_or(status, kStepStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    return true;
  }
};

// ------------------------------------------------------------------ register slabs

// Per-wave registers of one stage: up to 8 x 16 bytes of weight-row chunks
// and a few small operands.
struct Slab {
  Pack8 w[8];
  uint32_t taps;   // conv_in unit: conv tap l in lanes 0..2
  uint32_t state;  // conv_in unit: conv state tap l - 2 in lanes 3..4
};

// RMSNorm weights are kept in LDS as packed bf16 pairs: word i holds
// elements 2i and 2i + 1.
constexpr int kNormWords = kHidden / 2;
__device__ __forceinline__ void load_norm_lds(uint32_t* dst, const uint16_t* gamma) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(gamma);
  for (int i = threadIdx.x; i < kNormWords; i += blockDim.x) dst[i] = src[i];
}

// Weight rows are read with buffer loads: a scalar descriptor per row, the
// chunk offset as a scalar operand and the lane offset (16 bytes per lane) in
// one VGPR that never changes, so no per-lane address arithmetic competes
// with the slab registers (whose reuse would force waits on loads in flight)
// and a row is never read past its end.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw-buffer format word
constexpr int kBufStream = 2;          // cache policy: non-temporal (read once per token)
__device__ __forceinline__ BufRsrc row_rsrc(const uint16_t* row, int elems, bool valid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row), (short)0, valid ? elems * 2 : 0,
                                           kBufWord3);
}
__device__ __forceinline__ Pack8 buffer_load8(BufRsrc r, int lane_bytes, int chunk_bytes) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes, chunk_bytes, kBufStream);
  Pack8 p;
  p.w[0] = v.x; p.w[1] = v.y; p.w[2] = v.z; p.w[3] = v.w;
  return p;
}

// Rows r < R of length K (wave-uniform pointers) into the slab: lane l gets
// elements c*512 + l*8 + [0, 8) of chunk c. Every wave issues the same loads
// in every stage: a row the wave does not own (wave 0, waves past the unit
// count, the unused third row of a q/k/v unit) gets an empty descriptor and
// reads zeros without touching memory. With no branch around the loads a slab
// lives in the same registers on every path, so the compiler never has to copy
// one (a copy would wait for its loads).
template <int K, int R>
__device__ __forceinline__ void slab_load_rows(Slab& s, const uint16_t* const* rows,
                                               const bool* valid) {
  static_assert(R * (K / 512) <= 8, "slab holds 8 chunks");
  const int lane_bytes = lane_id() * 16;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const BufRsrc rs = row_rsrc(rows[r], K, valid[r]);
#pragma unroll
    for (int c = 0; c < K / 512; ++c) s.w[r * (K / 512) + c] = buffer_load8(rs, lane_bytes, c * 1024);
  }
}

// Gathered input vectors sit in LDS as packed bf16 pairs: word i holds
// elements 2i (low half) and 2i + 1. Lane l's 8 elements of chunk c are the 16
// bytes at word c*256 + 4l, which the 64 lanes read without bank conflicts,
// and they line up with the lane's weight chunk for v_dot2_f32_bf16.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {  // both exact bf16 values
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}
__device__ __forceinline__ u32x4 lds_chunk(const uint32_t* lds, int c) {
  return *reinterpret_cast<const u32x4*>(lds + c * 256 + lane_id() * 4);
}

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
// row rotations and the gfx950 row/half swaps (no LDS, no readlane chain).
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
__device__ __forceinline__ float swap_sum(float v) {  // lanes l, l^16, l^32, l^48 summed
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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

// d[r] = row r of the C-chunk weight rows w . x (x: the lane's chunks of the
// gathered vector), as wave-uniform values.
template <int C, int R>
__device__ __forceinline__ void rows_dot(const Pack8* w, const u32x4* x, float* d) {
  float p[R];
#pragma unroll
  for (int r = 0; r < R; ++r) p[r] = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c)
#pragma unroll
    for (int r = 0; r < R; ++r) p[r] = dot8(w[r * C + c], x[c], p[r]);
  if constexpr (R == 1) {
    d[0] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_total(p[0]))));
  } else {
    const float v = wave_totals4<R>(p);
#pragma unroll
    for (int r = 0; r < R; ++r) d[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
  }
}

// Dot products of slab rows [0, R) with the gathered vector in LDS.
template <int K, int R>
__device__ __forceinline__ void slab_dots(const Slab& s, const uint32_t* lds, float* d) {
  constexpr int C = K / 512;
  u32x4 x[C];
#pragma unroll
  for (int c = 0; c < C; ++c) x[c] = lds_chunk(lds, c);
  rows_dot<C, R>(s.w, x, d);
}

// A unit index that is safe to form row pointers from (the row itself is read
// only when the unit exists).
__device__ __forceinline__ int clamp_unit(int u, int units) { return u < units ? u : units - 1; }

// ------------------------------------------------------------------ input gather (wave 0)

// Poll K tagged words (K % 128 == 0; lane l owns words 2l + 128 j) until every
// tag equals `tag`; values land in v[2j], v[2j+1]. (Keeping a second round of
// loads in flight was measured slower: the extra traffic on the few hot lines
// delays the producers' stores more than it shortens detection.)
template <int K>
__device__ __forceinline__ void wave_poll(const uint32_t* src, uint32_t tag, float* v,
                                          int32_t* status) {
  const int l = lane_id();
  Poll poll(status);
  while (true) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < K / 128; ++j) {
      const uint64_t w = coherent_load64(src + 2 * l + 128 * j);
      const uint32_t a = (uint32_t)w, b = (uint32_t)(w >> 32);
      ok = ok && tag_ok(a, tag) && tag_ok(b, tag);
      v[2 * j] = tagged_value(a);
      v[2 * j + 1] = tagged_value(b);
    }
    if (__all(ok) || !poll.again()) break;
  }
}

// As wave_poll, writing the values straight to lds[0, K). Each batch of
// loads is issued back to back before any LDS write: relaxed atomic loads
// stay in program order with the LDS stores, so interleaving them would cost
// one round trip per load.
template <int K, int kBatch = K / 128>
__device__ __forceinline__ void wave_poll_lds(const uint32_t* src, uint32_t tag, uint32_t* lds,
                                              int32_t* status) {
  static_assert((K / 128) % kBatch == 0, "batches split the lane's words evenly");
  const int l = lane_id();
  Poll poll(status);
  while (true) {
    bool ok = true;
#pragma unroll
    for (int j0 = 0; j0 < K / 128; j0 += kBatch) {
      uint64_t w[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) w[j] = coherent_load64(src + 2 * l + 128 * (j0 + j));
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const uint32_t a = (uint32_t)w[j], b = (uint32_t)(w[j] >> 32);
        ok = ok && tag_ok(a, tag) && tag_ok(b, tag);
        lds[l + 64 * (j0 + j)] = (a & 0xffffu) | (b << 16);
      }
    }
    if (__all(ok) || !poll.again()) break;
  }
}

// The untagged embedding row in the same ownership.
__device__ __forceinline__ void wave_row(const uint16_t* row, float* v) {
  const int l = lane_id();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 2 * l + 128 * j);
    v[2 * j] = lo_f32(w);
    v[2 * j + 1] = hi_f32(w);
  }
}

// RMSNorm of a 1024-vector held as 16 values per lane (two roundings,
// modeling_lfm2.py:54-59); gamma is the packed LDS copy.
__device__ __forceinline__ void wave_norm_reg(float* v, const uint32_t* gamma) {
  const int l = lane_id();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ss = fmaf(v[i], v[i], ss);
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss * (1.0f / (float)kHidden) + kNormEps);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t gw = gamma[l + 64 * j];
    v[2 * j] = round_bf16(round_bf16(v[2 * j] * r) * lo_f32(gw));
    v[2 * j + 1] = round_bf16(round_bf16(v[2 * j + 1] * r) * hi_f32(gw));
  }
}

template <int K>
__device__ __forceinline__ void wave_store_lds(const float* v, uint32_t* lds) {
  const int l = lane_id();
#pragma unroll
  for (int j = 0; j < K / 128; ++j) {
    lds[l + 64 * j] = bf16_pair(v[2 * j], v[2 * j + 1]);
  }
}

// ------------------------------------------------------------------ context

struct StepBufs {
  uint32_t* h;      // residual stream, 1024 tagged words
  uint32_t* y;      // conv gate output / attention context, 1024 tagged words
  uint32_t* g;      // gated FFN activation, 2560 tagged words
  uint32_t* qkv;    // 2048 tagged words
  uint64_t* cand;   // one tagged candidate per block
  int32_t* status;
};

// Where a layer's first stage reads its input: the embedding row of the
// token for layer 0, otherwise the tagged residual stream.
struct LayerIn {
  const uint16_t* row;  // non-null for layer 0
  uint32_t tag;         // epoch of h otherwise
};

constexpr int kComputeWavesPerBlock = kStepWaves - 1;
constexpr int kNoUnit = 0x7fffffff;

// Index of this wave among the compute waves of the grid (the head deals its
// units round-robin over them); wave 0 of every block (the gatherer) gets an
// index past every unit count.
__device__ __forceinline__ int compute_wave() {
  const int w = wave_id();
  return w == 0 ? kNoUnit : (int)blockIdx.x + (w - 1) * kStepBlocks;
}

// Units of a layer stage are dealt block-major: block b owns units
// [b * kPer, (b + 1) * kPer), unit b * kPer + k on compute wave k + 1. A
// block's output words are then contiguous and leave in one store
// instruction (publish), instead of one store per wave: 256 stores per
// exchange instead of 1024 cost about 1.3 us less per exchange on MI355X.
// The wave that owns row r of out_proj / o_proj also owns row r of w2.
template <int kUnits>
__device__ __forceinline__ int stage_unit() {
  static_assert(kUnits % kStepBlocks == 0 && kUnits / kStepBlocks <= kComputeWavesPerBlock,
                "units spread evenly over the compute waves");
  constexpr int kPer = kUnits / kStepBlocks;
  const int k = wave_id() - 1;
  return k >= 0 && k < kPer ? (int)blockIdx.x * kPer + k : kNoUnit;
}

// Stage epilogue: the compute waves have left the block's tagged output words
// in out[0, n) (LDS); after a block barrier wave 1 stores them to dst[0, n)
// with one instruction. Every thread of the block calls it.
constexpr int kMaxBlockOut = 16;
__device__ __forceinline__ void publish(const uint32_t* out, int n, uint32_t* dst) {
  __syncthreads();
  if (wave_id() == 1 && lane_id() < n) coherent_store32(dst + lane_id(), out[lane_id()]);
}

// Wave 0: the layer input (embedding row or tagged h), normalised, into LDS.
__device__ __forceinline__ void gather_normed_input(const LayerIn& in, const StepBufs& b,
                                                    const uint32_t* gamma, uint32_t* lds) {
  if (wave_id() != 0) return;
  float v[16];
  if (in.row != nullptr) wave_row(in.row, v);
  else wave_poll<kHidden>(b.h, in.tag, v, b.status);
  wave_norm_reg(v, gamma);
  wave_store_lds<kHidden>(v, lds);
}

// ------------------------------------------------------------------ conv layer stage 1

// The first stage of a layer, prefetched the same way for both layer kinds
// (1024 units): a conv layer's unit c is in_proj rows (c, 1024+c, 2048+c) plus
// its conv operands (lanes 0..2 load the taps, lanes 3..4 the two state taps
// that survive the shift, read back with readlane after the dot products); an
// attention layer's unit u is rows (2u, 2u+1) of the q/k/v projection, whose
// three matrices lie back to back in the weight stream.
constexpr int kFirstUnits = kHidden;
__device__ __forceinline__ void prefetch_first_stage(Slab& s, bool attn, const uint16_t* w,
                                                     const uint16_t* conv_w, const uint16_t* state) {
  const int u = stage_unit<kFirstUnits>();
  const bool ok = u < kFirstUnits;
  const int c = clamp_unit(u, kFirstUnits);
  const uint16_t* rows[3] = {
      w + (size_t)(attn ? 2 * c : c) * kHidden, w + (size_t)(attn ? 2 * c + 1 : kHidden + c) * kHidden,
      w + (size_t)(2 * kHidden + c) * kHidden};
  const bool valid[3] = {ok, ok, ok && !attn};
  slab_load_rows<kHidden, 3>(s, rows, valid);
  const int l = lane_id();
  const bool conv = ok && !attn;
  const BufRsrc taps = row_rsrc(conv_w + c * kConvTaps, kConvTaps, conv);
  const BufRsrc st = row_rsrc(state + c * kConvTaps, kConvTaps, conv);
  constexpr int kOutside = 1 << 20;  // a byte offset past both 3-element ranges
  s.taps = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(taps, l < 3 ? 2 * l : kOutside, 0, 0);
  s.state = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(st, l == 3 || l == 4 ? 2 * (l - 2) : kOutside,
                                                           0, 0);
}

__device__ __forceinline__ void run_conv_in(const Slab& s, const uint32_t* gamma, const LayerIn& in,
                                            uint16_t* state, const StepBufs& b, uint32_t tag_out,
                                            uint32_t* lds, uint32_t* out) {
  __syncthreads();  // poll only once this block has finished its previous stage
  gather_normed_input(in, b, gamma, lds);
  __syncthreads();
  const int c = stage_unit<kFirstUnits>();
  if (c < kFirstUnits) {
    float d[3];
    slab_dots<kHidden, 3>(s, lds, d);
    const float B = round_bf16(d[0]), C = round_bf16(d[1]), X = round_bf16(d[2]);
    const uint16_t w[3] = {(uint16_t)__builtin_amdgcn_readlane(s.taps, 0),
                           (uint16_t)__builtin_amdgcn_readlane(s.taps, 1),
                           (uint16_t)__builtin_amdgcn_readlane(s.taps, 2)};
    uint16_t st[3] = {0, (uint16_t)__builtin_amdgcn_readlane(s.state, 3),
                      (uint16_t)__builtin_amdgcn_readlane(s.state, 4)};
    if (lane_id() == 0) {
      const float yv = conv_gate_channel(B, C, X, w, st, state + c * kConvTaps);
      out[wave_id() - 1] = tagged(yv, tag_out);
    }
  }
  constexpr int kPer = kFirstUnits / kStepBlocks;
  publish(out, kPer, b.y + blockIdx.x * kPer);
}

// ------------------------------------------------------------------ residual projections

// h[r] = bf16(h[r] + bf16(W[r] . v)), K = 1024, row r = global wave; the
// residual h[r] is carried in lane 0's register `hres`.
__device__ __forceinline__ void prefetch_proj(Slab& s, const uint16_t* W) {
  const int u = stage_unit<kHidden>();
  const uint16_t* rows[1] = {W + (size_t)clamp_unit(u, kHidden) * kHidden};
  const bool valid[1] = {u < kHidden};
  slab_load_rows<kHidden, 1>(s, rows, valid);
}

__device__ __forceinline__ void run_proj(const Slab& s, const uint32_t* v, uint32_t tag_v,
                                         float& hres, const StepBufs& b, uint32_t tag_out,
                                         uint32_t* lds, uint32_t* out) {
  __syncthreads();  // poll only once this block has finished its previous stage
  if (wave_id() == 0) {
    float vv[16];
    wave_poll<kHidden>(v, tag_v, vv, b.status);
    wave_store_lds<kHidden>(vv, lds);
  }
  __syncthreads();
  if (stage_unit<kHidden>() < kHidden) {
    float d[1];
    slab_dots<kHidden, 1>(s, lds, d);
    if (lane_id() == 0) {
      hres = round_bf16(hres + round_bf16(d[0]));
      out[wave_id() - 1] = tagged(hres, tag_out);
    }
  }
  constexpr int kPer = kHidden / kStepBlocks;
  publish(out, kPer, b.h + blockIdx.x * kPer);
}

// ------------------------------------------------------------------ MLP

// g[f] = bf16(bf16(silu(bf16(w1[f].n))) * bf16(w3[f].n)), n = RMSNorm(h);
// columns 2u, 2u+1 for unit u = global wave (1280 units).
constexpr int kStepUpUnits = kFfn / 2;
__device__ __forceinline__ void prefetch_up(Slab& s, const uint16_t* w1, const uint16_t* w3) {
  const int u = stage_unit<kStepUpUnits>();
  const int f0 = 2 * clamp_unit(u, kStepUpUnits);
  const uint16_t* rows[4] = {w1 + (size_t)f0 * kHidden, w3 + (size_t)f0 * kHidden,
                             w1 + (size_t)(f0 + 1) * kHidden, w3 + (size_t)(f0 + 1) * kHidden};
  const bool ok = u < kStepUpUnits;
  const bool valid[4] = {ok, ok, ok, ok};
  slab_load_rows<kHidden, 4>(s, rows, valid);
}

__device__ __forceinline__ void run_up(const Slab& s, const uint32_t* gamma, uint32_t tag_h,
                                       const StepBufs& b, uint32_t tag_out, uint32_t* lds,
                                       uint32_t* out) {
  __syncthreads();  // poll only once this block has finished its previous stage
  gather_normed_input(LayerIn{nullptr, tag_h}, b, gamma, lds);
  __syncthreads();
  if (stage_unit<kStepUpUnits>() < kStepUpUnits) {
    float d[4];  // w1[f0], w3[f0], w1[f0 + 1], w3[f0 + 1]
    slab_dots<kHidden, 4>(s, lds, d);
    const float a0 = d[0], b0 = d[1], a1 = d[2], b1 = d[3];
    if (lane_id() < 2) {
      const float a = lane_id() == 0 ? a0 : a1;
      const float g = lane_id() == 0 ? b0 : b1;
      out[2 * (wave_id() - 1) + lane_id()] = tagged(silu_bf16(round_bf16(a)) * round_bf16(g), tag_out);
    }
  }
  constexpr int kPer = 2 * kStepUpUnits / kStepBlocks;
  publish(out, kPer, b.g + blockIdx.x * kPer);
}

// h[r] = bf16(h[r] + bf16(w2[r] . g)), K = 2560, row r = global wave.
__device__ __forceinline__ void prefetch_down(Slab& s, const uint16_t* w2) {
  const int u = stage_unit<kHidden>();
  const uint16_t* rows[1] = {w2 + (size_t)clamp_unit(u, kHidden) * kFfn};
  const bool valid[1] = {u < kHidden};
  slab_load_rows<kFfn, 1>(s, rows, valid);
}

__device__ __forceinline__ void run_down(const Slab& s, uint32_t tag_g, float& hres,
                                         const StepBufs& b, uint32_t tag_out, uint32_t* lds,
                                         uint32_t* out) {
  __syncthreads();  // poll only once this block has finished its previous stage
  if (wave_id() == 0) wave_poll_lds<kFfn>(b.g, tag_g, lds, b.status);
  __syncthreads();
  if (stage_unit<kHidden>() < kHidden) {
    float d[1];
    slab_dots<kFfn, 1>(s, lds, d);
    if (lane_id() == 0) {
      hres = round_bf16(hres + round_bf16(d[0]));
      out[wave_id() - 1] = tagged(hres, tag_out);
    }
  }
  constexpr int kPer = kHidden / kStepBlocks;
  publish(out, kPer, b.h + blockIdx.x * kPer);
}

// ------------------------------------------------------------------ attention layer

// qkv[r] = bf16(W[r] . RMSNorm(x)), rows [0,1024) q, [1024,1536) k,
// [1536,2048) v; rows 2u, 2u+1 for unit u = compute wave (1024 units), loaded
// by prefetch_first_stage.
constexpr int kQkvRowsTotal = kHidden + 2 * kKvHeads * kHeadDim;
static_assert(kQkvRowsTotal / 2 == kFirstUnits, "q/k/v units match conv_in units");
__device__ __forceinline__ void run_qkv(const Slab& s, const uint32_t* gamma, const LayerIn& in,
                                        const StepBufs& b, uint32_t tag_out, uint32_t* lds,
                                        uint32_t* out) {
  __syncthreads();  // poll only once this block has finished its previous stage
  gather_normed_input(in, b, gamma, lds);
  __syncthreads();
  if (stage_unit<kFirstUnits>() < kFirstUnits) {
    float d[2];
    slab_dots<kHidden, 2>(s, lds, d);
    if (lane_id() < 2) out[2 * (wave_id() - 1) + lane_id()] = tagged(lane_id() == 0 ? d[0] : d[1], tag_out);
  }
  constexpr int kPer = 2 * kFirstUnits / kStepBlocks;
  publish(out, kPer, b.qkv + blockIdx.x * kPer);
}

// Attention of KV head `kv` (block-wide, kStepThreads): QK norm + RoPE of the
// gathered projections, KV append at `pos`, softmax, context -> tagged y.
__device__ __forceinline__ void run_attention(int kv, uint32_t tag_qkv, const uint16_t* q_gamma,
                                              const uint16_t* k_gamma, const uint16_t* rope_row,
                                              uint16_t* keys, uint16_t* values, int pos,
                                              const StepBufs& b, uint32_t tag_out,
                                              AttnSharedT<kStepThreads>& sh) {
  const int w = wave_id();
  const int l = lane_id();
  // Wave 0 gathers q head 0, q head 1, k and v of this KV group.
  if (w == 0) {
    const uint32_t* src[4] = {b.qkv + 2 * kv * kHeadDim, b.qkv + (2 * kv + 1) * kHeadDim,
                              b.qkv + kHidden + kv * kHeadDim,
                              b.qkv + kHidden + kKvHeads * kHeadDim + kv * kHeadDim};
    Poll poll(b.status);
    while (true) {
      bool ok = true;
      uint32_t word[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) word[i] = coherent_load32(src[i] + l);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok = ok && tag_ok(word[i], tag_qkv);
        sh.raw[i][l] = tagged_value(word[i]);
      }
      if (__all(ok) || !poll.again()) break;
    }
  }
  __syncthreads();
  if (w < 4) {
    const uint16_t* gam = w == 0 || w == 1 ? q_gamma : k_gamma;
    const float gl = bf16_to_f32(gam[l]);
    const float cl = bf16_to_f32(rope_row[l]);
    const float sl = bf16_to_f32(rope_row[kHeadDim + l]);
    const float raw = sh.raw[w][l];
    if (w < 3) {
      const float o = norm_rope_lane(raw, gl, cl, sl);
      if (w < 2) {
        sh.q[w][l] = o;
      } else {
        sh.k_new[l] = o;
        keys[(size_t)pos * kHeadDim + l] = f32_to_bf16(o);
      }
    } else {
      sh.v_new[l] = raw;
      values[(size_t)pos * kHeadDim + l] = f32_to_bf16(raw);
    }
  }
  __syncthreads();
  attn_core_t<kStepThreads>(keys, values, pos, sh);
  if (threadIdx.x < 2 * kHeadDim)
    coherent_store32(b.y + 2 * kv * kHeadDim + threadIdx.x, tagged(sh.out[threadIdx.x], tag_out));
}

// ------------------------------------------------------------------ head

// Final RMSNorm + tied head: units of 4 vocabulary rows dealt to global waves;
// each block's best (value, row) -> tagged candidate word cand[block]. The
// slab holds the wave's first unit.
constexpr int kStepHeadRows = 4;
__device__ __forceinline__ void head_rows(const uint16_t* table, int u, const uint16_t** rows) {
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) rows[r] = table + (size_t)(u * kStepHeadRows + r) * kHidden;
}

__device__ __forceinline__ void prefetch_head(Slab& s, const uint16_t* table, int vocab) {
  const int units = vocab / kStepHeadRows;
  const int u = compute_wave();
  const uint16_t* rows[kStepHeadRows];
  head_rows(table, clamp_unit(u, units), rows);
  const bool ok = u < units;
  const bool valid[kStepHeadRows] = {ok, ok, ok, ok};
  slab_load_rows<kHidden, kStepHeadRows>(s, rows, valid);
}

__device__ __forceinline__ void run_head(const Slab& s, const uint32_t* gamma, uint32_t tag_h,
                                         const uint16_t* table, int vocab, const StepBufs& b,
                                         uint32_t tag_out, uint32_t* lds, float* red_v, int* red_i) {
  gather_normed_input(LayerIn{nullptr, tag_h}, b, gamma, lds);
  __syncthreads();
  const int waves = kStepBlocks * kComputeWavesPerBlock;
  const int units = vocab / kStepHeadRows;
  const int l = lane_id();
  const u32x4 x[2] = {lds_chunk(lds, 0), lds_chunk(lds, 1)};
  float best = -INFINITY;
  int best_row = 0x7fffffff;
  Pack8 cur[8], nxt[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cur[i] = s.w[i];
  for (int u = compute_wave(); u < units; u += waves) {
    if (u + waves < units) {
      const uint16_t* rows[kStepHeadRows];
      head_rows(table, u + waves, rows);
#pragma unroll
      for (int r = 0; r < kStepHeadRows; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) nxt[r * 2 + c] = load8_stream(rows[r] + c * 512 + l * 8);
    }
    float d[kStepHeadRows];
    rows_dot<2, kStepHeadRows>(cur, x, d);
#pragma unroll
    for (int r = 0; r < kStepHeadRows; ++r) {
      const float v = round_bf16(d[r]);
      const int row = u * kStepHeadRows + r;
      if (better(v, row, best, best_row)) { best = v; best_row = row; }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
  }
  if (lane_id() == 0) { red_v[wave_id()] = best; red_i[wave_id()] = best_row; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = red_v[0];
    int bi = red_i[0];
    for (int i = 1; i < kStepWaves; ++i)
      if (better(red_v[i], red_i[i], bv, bi)) { bv = red_v[i]; bi = red_i[i]; }
    coherent_store64(b.cand + blockIdx.x, tagged_candidate(bv, bi, tag_out));
  }
}

// Every block: wait for all `n` (<= kMaxCandidates) candidates of epoch
// `tag`, return the winner (first maximum) to all threads.
constexpr int kMaxCandidates = 256;
__device__ __forceinline__ int step_pick(const StepBufs& b, int n, uint32_t tag, int* s_winner) {
  if (wave_id() == 0) {
    const int l = lane_id();
    Poll poll(b.status);
    float bv;
    int bi;
    while (true) {
      bool ok = true;
      bv = -INFINITY;
      bi = 0x7fffffff;
      uint64_t cw[kMaxCandidates / kWave];
#pragma unroll
      for (int k = 0; k < kMaxCandidates / kWave; ++k)
        cw[k] = l + k * kWave < n ? coherent_load64(b.cand + l + k * kWave) : 0;
#pragma unroll
      for (int k = 0; k < kMaxCandidates / kWave; ++k) {
        if (l + k * kWave >= n) continue;
        const uint64_t c = cw[k];
        const uint32_t hi = (uint32_t)(c >> 32);
        ok = ok && (hi & 0xffffu) == tag;
        const float v = __uint_as_float((uint32_t)c);
        const int row = (int)(hi >> 16);
        if (better(v, row, bv, bi)) { bv = v; bi = row; }
      }
      if (__all(ok) || !poll.again()) break;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (l == 0) *s_winner = bi;
  }
  __syncthreads();
  return *s_winner;
}

}  // namespace lfm25
