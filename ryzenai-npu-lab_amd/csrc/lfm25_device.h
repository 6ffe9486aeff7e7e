// Device-side building blocks shared by every LFM2.5 decode kernel on gfx950.
//
// BF16 values travel as raw uint16_t bit patterns; arithmetic is FP32 with one
// round-to-nearest-even step wherever the model rounds to BF16 (the CPU
// PyTorch BF16 path: transformers/models/lfm2/modeling_lfm2.py, restated in
// experiments/006_lfm25_cpu_two_recurrent_layers.py:35-55).
//
// Work is organised per wave64: one wave owns whole output rows, each lane
// holds a fixed 16-byte-strided slice of the activation vector in registers,
// weights stream through 128-bit loads, and the 64 per-lane partial sums are
// combined with a butterfly that leaves the bitwise-identical total in every
// lane (the xor-partner pairs add the same two operands), so reduction order
// is fixed and results are deterministic run to run.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lfm25 {

constexpr int kHidden = 1024;
constexpr int kFfn = 2560;
constexpr int kVocab = 65536;
constexpr int kHeads = 16;
constexpr int kKvHeads = 8;
constexpr int kHeadDim = 64;
constexpr int kConvTaps = 3;
constexpr int kWave = 64;
constexpr float kNormEps = 1.0e-5f;

// ------------------------------------------------------------------ BF16

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even FP32 -> BF16; NaNs stay NaN (quiet bit set).
// gfx950 converts in hardware (v_cvt_pk_bf16_f32): round to nearest even,
// NaN kept quiet -- the same bits as u + 0x7fff + ((u >> 16) & 1) >> 16 with
// NaN -> (u >> 16) | 0x40, which the conversion tests check bit for bit.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// Low / high BF16 of a packed 32-bit word as FP32.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ------------------------------------------------------------------ waves

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
// Wave index within the block, as a wave-uniform (scalar) value so branches
// on it and addresses derived from it stay in SGPRs.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
}

// Block barrier for data exchanged through LDS: waits for the wave's own LDS
// operations only. __syncthreads() also waits for every global load and store
// the wave has in flight (its workgroup-scope fence), which puts a store's
// round trip to memory, or a weight prefetch, in front of the barrier; no
// wave of a block reads global memory that another wave of the block wrote
// without a tagged exchange in between, so the LDS order is all that is needed.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// DPP lane moves within a row of 16 lanes (all sources valid, no masking).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, true));
}

// Sum within each row of 16 lanes; every lane of the row gets the same bits
// (each step adds the same two operands in both partner lanes).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);
  v += dpp_f32<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
  return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes in a fixed order (row sums by DPP, then the four
// rows as (r0 + r1) + (r2 + r3)); every lane receives the identical total.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Sum over aligned groups of 8 lanes (quad butterfly then half-row mirror).
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(kWidth == 8, "only groups of 8 lanes are used");
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);
  return v;
}

// ------------------------------------------------------------------ loads

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes = 8 BF16 values.
struct alignas(16) Pack8 {
  uint32_t w[4];
};

__device__ __forceinline__ Pack8 load8(const uint16_t* p) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  Pack8 r;
  r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  return r;
}

// Streaming (read-once) load: weights are used once per token.
__device__ __forceinline__ Pack8 load8_stream(const uint16_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  Pack8 r;
  r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  return r;
}

__device__ __forceinline__ void unpack8(const Pack8& p, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo_f32(p.w[i]);
    f[2 * i + 1] = hi_f32(p.w[i]);
  }
}

// acc += dot(8 BF16 weights, 8 FP32 activations), sequential FMA order.
__device__ __forceinline__ float fma8(const Pack8& w, const float* x, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = fmaf(lo_f32(w.w[i]), x[2 * i], acc);
    acc = fmaf(hi_f32(w.w[i]), x[2 * i + 1], acc);
  }
  return acc;
}

// ------------------------------------------------------------------ vectors
//
// A K-long activation vector is held as K/512 chunks of 8 values per lane:
// lane l owns elements [c*512 + l*8, c*512 + l*8 + 8) of chunk c, so one
// wave-wide 16-byte load of a weight row chunk is 1 KB contiguous.

template <int K>
struct LaneVec {
  static constexpr int kChunks = K / 512;
  float v[kChunks * 8];
};

template <int K>
__device__ __forceinline__ void load_lane_vec(const uint16_t* x, LaneVec<K>& out) {
  const int l = lane_id();
#pragma unroll
  for (int c = 0; c < LaneVec<K>::kChunks; ++c) unpack8(load8(x + c * 512 + l * 8), out.v + c * 8);
}

// FP32 dot product of one BF16 row (K values) with the lane slices; the full
// sum is returned in every lane.
template <int K>
__device__ __forceinline__ float row_dot(const uint16_t* row, const LaneVec<K>& x) {
  const int l = lane_id();
  Pack8 w[LaneVec<K>::kChunks];
#pragma unroll
  for (int c = 0; c < LaneVec<K>::kChunks; ++c) w[c] = load8_stream(row + c * 512 + l * 8);
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < LaneVec<K>::kChunks; ++c) acc = fma8(w[c], x.v + c * 8, acc);
  return wave_sum(acc);
}

// Several rows at once: all loads are issued before any arithmetic so each
// lane keeps R*K/512 16-byte loads in flight.
template <int K, int R>
__device__ __forceinline__ void rows_dot(const uint16_t* const* rows, const LaneVec<K>& x,
                                         float* out) {
  constexpr int C = LaneVec<K>::kChunks;
  const int l = lane_id();
  Pack8 w[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) w[r][c] = load8_stream(rows[r] + c * 512 + l * 8);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) acc = fma8(w[r][c], x.v + c * 8, acc);
    out[r] = wave_sum(acc);
  }
}

// RMSNorm of a 1024-vector held as lane slices (two roundings, as
// Lfm2RMSNorm.forward, modeling_lfm2.py:54-59): s = sum x^2 in FP32,
// r = 1/sqrt(s/N + eps), n = bf16(x*r), y = bf16(n*gamma).
template <int K>
__device__ __forceinline__ void rms_norm_lane_vec(LaneVec<K>& x, const uint16_t* gamma) {
  constexpr int C = LaneVec<K>::kChunks;
  const int l = lane_id();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < C * 8; ++i) ss = fmaf(x.v[i], x.v[i], ss);
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss * (1.0f / (float)K) + kNormEps);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float g[8];
    unpack8(load8(gamma + c * 512 + l * 8), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) x.v[c * 8 + i] = round_bf16(round_bf16(x.v[c * 8 + i] * r) * g[i]);
  }
}

// bf16(silu(h)) with silu evaluated in FP32 as x / (1 + exp(-x)).
__device__ __forceinline__ float silu_bf16(float h) {
  return round_bf16(h / (1.0f + expf(-h)));
}

}  // namespace lfm25
