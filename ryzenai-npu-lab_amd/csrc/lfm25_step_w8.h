// 8-bit-weight (w8g32) phases of the persistent decode: the same blocks,
// waves, rows and exchanges as the BF16 phases of lfm25_step.h, with every
// projection and the tied table read as int8 q plus one FP32 scale per row
// and group of 32 inputs (experiments/014_int8_lfm25.py:76-113, the format
// its study ranks first).
//
// A lane holds 16 consecutive weights of a row (one 16-byte load), which lie
// in one group, and the scale of that group. A row's dot product is
// sum over lanes of s * (sum of 16 q x) in FP32: the products q x are exact
// (a BF16 value times an integer of at most 7 bits), the segment sums round
// once per add, then the segment is scaled, as lfm25_w8_gemv computes it.
// The reference's dense form sum_k x (q s)_fp32 rounds each q s instead; both
// lie within the FP32 summation bound of the exact sum.
//
// Converting a byte takes one instruction (v_cvt_f32_i32 with a sign-
// extended byte select) and the product one FMA, where two BF16 weights take
// one v_dot2: the compute phases issue about four times the VALU work of
// the BF16 phases for half the bytes.
#pragma once
#include "lfm25_layout.h"
#include "lfm25_step.h"

namespace lfm25 {

__device__ __forceinline__ BufRsrc byte_rsrc(const void* base, int bytes, bool valid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, valid ? bytes : 0, kBufWord3);
}
// A lane offset past every range a phase uses: the load returns zeros.
constexpr int kOutsideRange = 1 << 24;

// The weights of one layer for wave k (0..7) of block (x, jj) of the layer's
// group, owning the same rows as Slabs:
//   a: P1 rows (conv: in_proj rows c, 1024 + c, 2048 + c of channel
//      c = 128x + 8jj + k; attention: entries 16jj + 2k, + 1 of the XCD's
//      q/k/v list, the third row empty), lane l: bytes [16l, 16l + 16);
//   b: P2 row 64jj + 8k + (l >> 3) of out_proj / o_proj, columns
//      128x + 16 (l & 7) + [0, 16);
//   c: P3 w1 / w3 rows of FFN columns 320x + 20jj + fc(k) + [0, nc(k)), as a;
//   d: P4 row 64jj + 8k + (l >> 3) of w2, chunks (l & 7) + 8i (i < 3, chunk
//      < 20) of 16 columns of the XCD's 320.
// Scales: one per load, of the group the lane's 16 weights lie in.
struct Slabs8 {
  u32x4 a[3];
  float as[3];
  uint32_t taps, state;
  u32x4 b;
  float bs;
  u32x4 c[6];
  float cs[6];
  u32x4 d[3];
  float ds[3];
};

struct LayerWeights8 {
  bool attn;
  const int8_t* qa;  // mixer: in_proj, or q | k | v
  const float* sa;
  const uint16_t* conv_w;
  const uint16_t* state;
  const int8_t* qb;  // out_proj / o_proj
  const float* sb;
  const int8_t* q1;
  const float* s1;
  const int8_t* q3;
  const float* s3;
  const int8_t* q2;
  const float* s2;
};

// R full rows (K = 1024) and their lane's group scale.
template <int R>
__device__ __forceinline__ void load_rows1024_w8(u32x4* q, float* s, const int8_t* const* rows,
                                                 const float* const* scales, const bool* valid) {
  const int l = lane_id();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    q[r] = __builtin_amdgcn_raw_buffer_load_b128(byte_rsrc(rows[r], kHidden, valid[r]), 16 * l, 0, kBufStream);
    s[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(byte_rsrc(scales[r], kW8RowScales * 4, valid[r]),
                                                                4 * (l >> 1), 0, kBufStream));
  }
}

__device__ __forceinline__ void load_slab_a(Slabs8& s, const LayerWeights8& L) {
  const int k = wave_id();
  const int x = blk_xcd(), jj = blk_jj();
  const int l = lane_id();
  const int c = kXcdCols * x + kBlockChan * jj + k;
  const int r0 = qkv_row(x, kBlockQkv * jj + 2 * k);
  const int rows_i[3] = {L.attn ? r0 : c, L.attn ? r0 + 1 : kHidden + c, 2 * kHidden + c};
  const int8_t* rows[3];
  const float* scales[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    rows[r] = L.qa + (size_t)rows_i[r] * kHidden;
    scales[r] = L.sa + (size_t)rows_i[r] * kW8RowScales;
  }
  const bool valid[3] = {true, true, !L.attn};
  load_rows1024_w8<3>(s.a, s.as, rows, scales, valid);
  const BufRsrc taps = region_rsrc(L.conv_w + c * kConvTaps, kConvTaps * 2, !L.attn);
  const BufRsrc st = region_rsrc(L.state + c * kConvTaps, kConvTaps * 2, !L.attn);
  constexpr int kOutside = 1 << 20;
  s.taps = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(taps, l < 3 ? 2 * l : kOutside, 0, 0);
  s.state = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(st, l == 3 || l == 4 ? 2 * (l - 2) : kOutside, 0, 0);
}
__device__ __forceinline__ void load_slab_b(Slabs8& s, const LayerWeights8& L) {
  const int row0 = kResRows * blk_jj() + 8 * wave_id();
  const int x = blk_xcd(), l = lane_id();
  const BufRsrc rq = byte_rsrc(L.qb + (size_t)row0 * kHidden + kXcdCols * x, 7 * kHidden + kXcdCols, true);
  const BufRsrc rs = byte_rsrc(L.sb + (size_t)row0 * kW8RowScales + kXcdCols / kW8Group * x,
                               (7 * kW8RowScales + kXcdCols / kW8Group) * 4, true);
  s.b = __builtin_amdgcn_raw_buffer_load_b128(rq, (l >> 3) * kHidden + 16 * (l & 7), 0, kBufStream);
  s.bs = __uint_as_float(
      __builtin_amdgcn_raw_buffer_load_b32(rs, ((l >> 3) * kW8RowScales + ((l & 7) >> 1)) * 4, 0, kBufStream));
}
__device__ __forceinline__ void load_slab_c(Slabs8& s, const LayerWeights8& L) {
  const int k = wave_id();
  const int f = kXcdFfn * blk_xcd() + kBlockFfn * blk_jj() + ffn_first(k);
  const bool three = ffn_count(k) == 3;
  const int8_t* rows[6] = {L.q1 + (size_t)f * kHidden,       L.q3 + (size_t)f * kHidden,
                           L.q1 + (size_t)(f + 1) * kHidden, L.q3 + (size_t)(f + 1) * kHidden,
                           L.q1 + (size_t)(f + 2) * kHidden, L.q3 + (size_t)(f + 2) * kHidden};
  const float* scales[6] = {L.s1 + (size_t)f * kW8RowScales,       L.s3 + (size_t)f * kW8RowScales,
                            L.s1 + (size_t)(f + 1) * kW8RowScales, L.s3 + (size_t)(f + 1) * kW8RowScales,
                            L.s1 + (size_t)(f + 2) * kW8RowScales, L.s3 + (size_t)(f + 2) * kW8RowScales};
  const bool valid[6] = {true, true, true, true, three, three};
  load_rows1024_w8<6>(s.c, s.cs, rows, scales, valid);
}
// Chunks of 16 columns of the XCD's 320 FFN columns in one w2 row.
constexpr int kW8DownChunks = kXcdFfn / 16;  // 20
constexpr int kW8DownLoads = 3;              // chunk (l & 7) + 8i, i < 3
constexpr int kW8FfnRowScales = kFfn / kW8Group;  // 80
__device__ __forceinline__ void load_slab_d(Slabs8& s, const LayerWeights8& L) {
  const int row0 = kResRows * blk_jj() + 8 * wave_id();
  const int x = blk_xcd(), l = lane_id();
  const BufRsrc rq = byte_rsrc(L.q2 + (size_t)row0 * kFfn + kXcdFfn * x, 7 * kFfn + kXcdFfn, true);
  const BufRsrc rs = byte_rsrc(L.s2 + (size_t)row0 * kW8FfnRowScales + kXcdFfn / kW8Group * x,
                               (7 * kW8FfnRowScales + kXcdFfn / kW8Group) * 4, true);
#pragma unroll
  for (int i = 0; i < kW8DownLoads; ++i) {
    const int c = (l & 7) + 8 * i;
    const bool in = c < kW8DownChunks;
    s.d[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, in ? (l >> 3) * kFfn + 16 * c : kOutsideRange, 0, kBufStream);
    s.ds[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        rs, in ? ((l >> 3) * kW8FfnRowScales + (c >> 1)) * 4 : kOutsideRange, 0, kBufStream));
  }
}
__device__ __forceinline__ void load_slabs(Slabs8& s, const LayerWeights8& L) {
  load_slab_a(s, L);
  load_slab_b(s, L);
  load_slab_c(s, L);
  load_slab_d(s, L);
}

// ------------------------------------------------------------------ dot products

// Elements [16 i, 16 i + 16) of a gathered vector (BF16 pairs in LDS) as FP32.
__device__ __forceinline__ void lds_x16(const uint32_t* lds, int i, float* x) {
  const u32x4 a = lds16(lds, 2 * i), b = lds16(lds, 2 * i + 1);
  x[0] = lo_f32(a.x); x[1] = hi_f32(a.x); x[2] = lo_f32(a.y); x[3] = hi_f32(a.y);
  x[4] = lo_f32(a.z); x[5] = hi_f32(a.z); x[6] = lo_f32(a.w); x[7] = hi_f32(a.w);
  x[8] = lo_f32(b.x); x[9] = hi_f32(b.x); x[10] = lo_f32(b.y); x[11] = hi_f32(b.y);
  x[12] = lo_f32(b.z); x[13] = hi_f32(b.z); x[14] = lo_f32(b.w); x[15] = hi_f32(b.w);
}
// sum_e q_e x_e over one 16-byte segment (exact products, FP32 adds in order).
__device__ __forceinline__ float q8_dot16(const u32x4& q, const float* x) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = q[i];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc = fmaf((float)(int8_t)(w >> (8 * b)), x[4 * i + b], acc);
  }
  return acc;
}

// d[r] = full-row (K = 1024) dot products of R int8 rows with the lane's 16
// elements x of the gathered vector, as wave-uniform values.
template <int R>
__device__ __forceinline__ void rows_dot1024_w8(const u32x4* q, const float* s, const float* x, float* d) {
  float p[R];
#pragma unroll
  for (int r = 0; r < R; ++r) p[r] = s[r] * q8_dot16(q[r], x);
  if constexpr (R == 1) {
    d[0] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_total(p[0]))));
  } else {
    const float v = wave_totals4<R>(p);
#pragma unroll
    for (int r = 0; r < R; ++r) d[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
  }
}

// ------------------------------------------------------------------ compute phases (every wave)

template <bool kLocal>
__device__ __forceinline__ void compute_conv(const Slabs8& s, const uint32_t* lds, uint16_t* state,
                                             uint32_t tag_out, StepOut& o, const StepBufs& b) {
  const int k = wave_id();
  float x[16];
  lds_x16(lds, lane_id(), x);
  float d[3];
  rows_dot1024_w8<3>(s.a, s.as, x, d);
  const float B = round_bf16(d[0]), C = round_bf16(d[1]), X = round_bf16(d[2]);
  const uint16_t w[3] = {(uint16_t)__builtin_amdgcn_readlane(s.taps, 0),
                         (uint16_t)__builtin_amdgcn_readlane(s.taps, 1),
                         (uint16_t)__builtin_amdgcn_readlane(s.taps, 2)};
  uint16_t st[3] = {0, (uint16_t)__builtin_amdgcn_readlane(s.state, 3),
                    (uint16_t)__builtin_amdgcn_readlane(s.state, 4)};
  if (lane_id() == 0) {
    const int c = kXcdCols * blk_xcd() + kBlockChan * blk_jj() + k;
    const float yv = conv_gate_channel(B, C, X, w, st, state + c * kConvTaps);
    local_store32<kLocal>(ly_of(b, blk_xcd()) + kBlockChan * blk_jj() + k, tagged(yv, tag_out));
  }
  (void)o;
}

template <bool kLocal>
__device__ __forceinline__ void compute_qkv(const Slabs8& s, const uint32_t* lds, uint32_t tag_out, StepOut& o,
                                            const StepBufs& b) {
  const int k = wave_id();
  float x[16];
  lds_x16(lds, lane_id(), x);
  float d[2];
  rows_dot1024_w8<2>(s.a, s.as, x, d);
  if (lane_id() < 2)
    local_store32<kLocal>(lq_of(b, blk_xcd()) + kBlockQkv * blk_jj() + 2 * k + lane_id(),
                          tagged(lane_id() == 0 ? d[0] : d[1], tag_out));
  (void)o;
}

// P2: partial sums of rows 64jj + 8k + [0, 8) over the XCD's 128 columns;
// lanes 8r .. 8r + 7 hold row r.
__device__ __forceinline__ void compute_proj(const Slabs8& s, const uint32_t* lds, uint32_t tag_out, StepOut& o,
                                             uint64_t* gp) {
  const int k = wave_id(), l = lane_id();
  float x[16];
  lds_x16(lds, l & 7, x);
  const float v = group_sum<8>(s.bs * q8_dot16(s.b, x));
  if ((l & 7) == 0) o.part[8 * k + (l >> 3)] = v;
  publish_partials(o, gp, tag_out);
}

template <bool kLocal>
__device__ __forceinline__ void compute_up(const Slabs8& s, const uint32_t* lds, uint32_t tag_out, StepOut& o,
                                           const StepBufs& b) {
  const int k = wave_id();
  float x[16];
  lds_x16(lds, lane_id(), x);
  float d[6];  // w1[f], w3[f], w1[f + 1], w3[f + 1], w1[f + 2], w3[f + 2]
  rows_dot1024_w8<4>(s.c, s.cs, x, d);
  if (ffn_count(k) == 3) rows_dot1024_w8<2>(s.c + 4, s.cs + 4, x, d + 4);
  else d[4] = d[5] = 0.0f;
  const int l = lane_id();
  if (l < ffn_count(k)) {
    const float a = l == 0 ? d[0] : l == 1 ? d[2] : d[4];
    const float g = l == 0 ? d[1] : l == 1 ? d[3] : d[5];
    local_store32<kLocal>(lg_of(b, blk_xcd()) + kBlockFfn * blk_jj() + ffn_first(k) + l,
                          tagged(silu_bf16(round_bf16(a)) * round_bf16(g), tag_out));
  }
  (void)o;
}

// P4: partial sums of rows 64jj + 8k + [0, 8) over the XCD's 320 FFN
// columns; lanes 8r .. 8r + 7 hold row r, chunks (l & 7) + 8i.
__device__ __forceinline__ void compute_down(const Slabs8& s, const uint32_t* lds, uint32_t tag_out, StepOut& o,
                                             uint64_t* gp) {
  const int k = wave_id(), l = lane_id();
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kW8DownLoads; ++i) {
    const int c = (l & 7) + 8 * i;
    if (c < kW8DownChunks) {
      float x[16];
      lds_x16(lds, c, x);
      acc = fmaf(s.ds[i], q8_dot16(s.d[i], x), acc);
    }
  }
  const float v = group_sum<8>(acc);
  if ((l & 7) == 0) o.part[8 * k + (l >> 3)] = v;
  publish_partials(o, gp, tag_out);
}

// ------------------------------------------------------------------ layer-0 input

// The token's embedding row of the int8 table, bf16(q s) per element (the
// reference's Weight.rows, 014_int8_lfm25.py:111-112), into g.raw by wave 0
// (lane l: elements 16l .. 16l + 15), or, without a row, the local h buffer
// as gather_raw_split polls it. Ends with a block barrier.
template <bool kLocal>
__device__ __forceinline__ void gather_raw_split_w8(const int8_t* row8, const float* row8_s, const uint32_t* src,
                                                    uint32_t tag, Gathered& g, int32_t* status) {
  if (row8 == nullptr) {
    gather_raw_split<kLocal>(nullptr, src, tag, g, status);
    return;
  }
  if (wave_id() == 0) {
    const int l = lane_id();
    const u32x4 q = *reinterpret_cast<const u32x4*>(row8 + 16 * l);
    const float s = row8_s[l >> 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = q[i];
      const float v0 = round_bf16((float)(int8_t)w * s), v1 = round_bf16((float)(int8_t)(w >> 8) * s);
      const float v2 = round_bf16((float)(int8_t)(w >> 16) * s), v3 = round_bf16((float)(int8_t)(w >> 24) * s);
      g.raw[8 * l + 2 * i] = bf16_pair(v0, v1);
      g.raw[8 * l + 2 * i + 1] = bf16_pair(v2, v3);
    }
    // the group sums of the norm (words l + 64 i, as gather_raw_split forms them)
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's words are in LDS
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sw = wave_sum(pair_sq(g.raw[l + 64 * i]));
      if (l == 0) g.ss[i] = sw;
    }
  }
  lds_barrier();
}

// ------------------------------------------------------------------ head

// A unit of 4 table rows as int8, lane l: bytes [16l, 16l + 16) of each row
// and the scale of group l / 2.
struct HeadRows8 {
  u32x4 w[kStepHeadRows];
  float s[kStepHeadRows];
};
__device__ __forceinline__ void head_load(const int8_t* table, const float* scales, int units, int u, HeadRows8& h) {
  const int l = lane_id();
  const int uu = clamp_unit(u, units);
  const bool ok = u < units;
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) {
    const size_t row = (size_t)uu * kStepHeadRows + r;
    h.w[r] = __builtin_amdgcn_raw_buffer_load_b128(byte_rsrc(table + row * kHidden, kHidden, ok), 16 * l, 0,
                                                  kBufCached);
    h.s[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        byte_rsrc(scales + row * kW8RowScales, kW8RowScales * 4, ok), 4 * (l >> 1), 0, kBufCached));
  }
}

// The wave's first unit staged in LDS (as head_begin_lds): words
// [r][4l, 4l + 4) hold lane l's 16 bytes of row r, word [r][256 + l] its
// scale.
constexpr int kW8HeadScaleWord = kHidden / 4;  // 256
__device__ __forceinline__ void head_begin_lds_w8(const int8_t* table, const float* scales, int vocab,
                                                  uint32_t (*rows)[kNormWords]) {
  const HeadSpan sp = head_span(vocab / kStepHeadRows);
  const int u = sp.first;
  if (u >= sp.end) return;
  const int l = lane_id();
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) {
    const size_t row = (size_t)u * kStepHeadRows + r;
    __builtin_amdgcn_global_load_lds((GlobalVoid*)(table + row * kHidden + 16 * l), (LdsVoid*)&rows[r][0], 16, 0, 0);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)(scales + row * kW8RowScales + (l >> 1)),
                                     (LdsVoid*)&rows[r][kW8HeadScaleWord], 4, 0, 0);
  }
}
static_assert(kW8HeadScaleWord + kWave <= kNormWords, "a staged int8 head row and its scales fit one slot");
__device__ __forceinline__ void head_from_lds(const uint32_t (*rows)[kNormWords], HeadRows8& h) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS copies have landed
  const int l = lane_id();
#pragma unroll
  for (int r = 0; r < kStepHeadRows; ++r) {
    h.w[r] = *reinterpret_cast<const u32x4*>(&rows[r][4 * l]);
    h.s[r] = __uint_as_float(rows[r][kW8HeadScaleWord + l]);
  }
}

// The head of the int8 table (run_head's units, rounding and candidates).
template <bool kLocal>
__device__ __forceinline__ void run_head(const uint32_t* lds, const int8_t* table, const float* scales, int vocab,
                                         const StepBufs& b, uint32_t tag_out, float* red_v, int* red_i,
                                         const HeadRows8& first) {
  const int units = vocab / kStepHeadRows;
  float x[16];
  lds_x16(lds, lane_id(), x);
  float best = -INFINITY;
  int best_row = 0x7fffffff;
  HeadRows8 cur = first, nxt;
  const HeadSpan sp = head_span(units);
  for (int u = sp.first; u < sp.end; u += kXcdWaves) {
    if (u + kXcdWaves < sp.end) head_load(table, scales, units, u + kXcdWaves, nxt);
    float d[kStepHeadRows];
    rows_dot1024_w8<kStepHeadRows>(cur.w, cur.s, x, d);
#pragma unroll
    for (int r = 0; r < kStepHeadRows; ++r) {
      const float v = round_bf16(d[r]);
      const int row = u * kStepHeadRows + r;
      if (better(v, row, best, best_row)) { best = v; best_row = row; }
    }
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

}  // namespace lfm25
