// Per-operation kernels behind the reference's lfm25_* entry points: one
// C-ABI function per operation, each a single stream-ordered launch (two for
// the argmax reductions). Shapes and pointers are validated on the host
// before anything is launched.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "lfm25_host.h"
#include "lfm25_stages.h"

namespace lfm25 {

static thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

// ------------------------------------------------------------------ RMSNorm

constexpr int kNormThreads = 1024;

__global__ void __launch_bounds__(kNormThreads) k_rms_norm(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ gamma,
                                                           uint16_t* __restrict__ y, int cols) {
  __shared__ float partial[kNormThreads / kWave];
  const int t = threadIdx.x;
  float ss = 0.0f;
  for (int i = t; i < cols; i += kNormThreads) {
    const float v = bf16_to_f32(x[i]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane_id() == 0) partial[wave_id()] = ss;
  __syncthreads();
  float total = partial[0];
  for (int i = 1; i < kNormThreads / kWave; ++i) total += partial[i];
  const float r = 1.0f / sqrtf(total / (float)cols + kNormEps);
  for (int i = t; i < cols; i += kNormThreads)
    y[i] = f32_to_bf16(round_bf16(bf16_to_f32(x[i]) * r) * bf16_to_f32(gamma[i]));
}

// ------------------------------------------------------------------ GEMV

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* y, int row, float v);
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* y, int row, float v) {
  y[row] = f32_to_bf16(v);
}
template <>
__device__ __forceinline__ void store_out<float>(float* y, int row, float v) {
  y[row] = v;
}

// R rows per wave, K fixed at compile time (activation held in registers).
// kNorm: the activation is RMS-normalised with `gamma` first. The first
// unit's weight rows are requested before the activation, so the two memory
// latencies overlap instead of adding up (most waves have one unit).
template <int K, int R, bool kNorm, typename OutT>
__global__ void __launch_bounds__(kGemvThreads) k_gemv_fixed(const uint16_t* __restrict__ w,
                                                             const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gamma,
                                                             OutT* __restrict__ y, int M) {
  constexpr int C = LaneVec<K>::kChunks;
  const WaveGrid g = wave_grid();
  const int units = (M + R - 1) / R;
  if (g.wave >= units) return;
  const int l = lane_id();
  Pack8 first[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c)
      first[r][c] = load8_stream(w + (size_t)min(g.wave * R + r, M - 1) * K + c * 512 + l * 8);
  LaneVec<K> xv;
  load_lane_vec<K>(x, xv);
  if (kNorm) rms_norm_lane_vec<K>(xv, gamma);
  for (int u = g.wave; u < units; u += g.waves) {
    const int r0 = u * R;
    float d[R];
    if (u == g.wave) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) acc = fma8(first[r][c], xv.v + c * 8, acc);
        d[r] = wave_sum(acc);
      }
    } else {
      const uint16_t* rows[R];
#pragma unroll
      for (int r = 0; r < R; ++r) rows[r] = w + (size_t)min(r0 + r, M - 1) * K;
      rows_dot<K, R>(rows, xv, d);
    }
    if (lane_id() < R) {
      float mine = d[0];
#pragma unroll
      for (int r = 1; r < R; ++r) mine = lane_id() == r ? d[r] : mine;
      const int row = r0 + lane_id();
      if (row < M) store_out<OutT>(y, row, mine);
    }
  }
}

// Any K % 8 == 0: one row per wave iteration, activation re-read per row.
template <typename OutT>
__global__ void __launch_bounds__(kGemvThreads) k_gemv_generic(const uint16_t* __restrict__ w,
                                                               const uint16_t* __restrict__ x,
                                                               OutT* __restrict__ y, int M,
                                                               int K) {
  const WaveGrid g = wave_grid();
  const int l = lane_id();
  for (int row = g.wave; row < M; row += g.waves) {
    const uint16_t* wr = w + (size_t)row * K;
    float acc = 0.0f;
    for (int c = l * 8; c < K; c += 512) {
      float xf[8];
      unpack8(load8(x + c), xf);
      acc = fma8(load8_stream(wr + c), xf, acc);
    }
    acc = wave_sum(acc);
    if (l == 0) store_out<OutT>(y, row, acc);
  }
}

template <typename OutT>
static int launch_gemv(const uint16_t* w, const uint16_t* x, const uint16_t* gamma, OutT* y, int M,
                       int K, bool norm, hipStream_t s) {
  auto blocks_for = [](int units) { return (units + kGemvWaves - 1) / kGemvWaves; };
  if (K == 1024) {
    // R rows per wave such that the grid is about one block of 4 waves per
    // CU (1,024 waves): every CU then requests the same bytes at once (with
    // a fixed R = 2 a 3072-row product left half the CUs a second block).
    // A row's sum does not depend on R.
    const int R = std::min(4, std::max(1, (M + 1023) / 1024));
    const int blocks = blocks_for((M + R - 1) / R);
    switch (R * 2 + (norm ? 1 : 0)) {
      case 2: k_gemv_fixed<1024, 1, false, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 3: k_gemv_fixed<1024, 1, true, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 4: k_gemv_fixed<1024, 2, false, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 5: k_gemv_fixed<1024, 2, true, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 6: k_gemv_fixed<1024, 3, false, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 7: k_gemv_fixed<1024, 3, true, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      case 8: k_gemv_fixed<1024, 4, false, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
      default: k_gemv_fixed<1024, 4, true, OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, gamma, y, M); break;
    }
  } else if (K == 2560 && !norm) {
    constexpr int R = 1;
    k_gemv_fixed<2560, R, false, OutT><<<blocks_for(M), kGemvThreads, 0, s>>>(w, x, gamma, y, M);
  } else {
    const int blocks = min(blocks_for(M), 2048);
    k_gemv_generic<OutT><<<blocks, kGemvThreads, 0, s>>>(w, x, y, M, K);
  }
  return check_launch("gemv");
}

// ------------------------------------------------------------------ INT8-weight GEMV
//
// The reference's 8-bit weight formats (experiments/014_int8_lfm25.py:76-113):
// int8 weights q[m][k] with one FP32 scale per row and group of 32 or 64
// inputs (w8g32 / w8g64), or one per row (w8c, applied after the sum of the
// integer-weight products). y[m] = bf16(sum_k x[k] * q[m][k] * s[m][k / g]).
// A wave takes units of kW8Rows consecutive rows, round robin over the grid,
// with the next unit's loads in flight while it computes the current one.
// Lane l reads bytes [16 (l + 64 j), +16) of each row (j < kSeg) with
// 16-byte buffer loads (a 16-byte segment never straddles a group) and keeps
// the matching 16 x values per segment in registers. Loads go through one
// descriptor per row, empty past the last row, so the loop issues the same
// loads every iteration and a finished wave reads nothing.
constexpr int kW8Rows = 4;
typedef __amdgpu_buffer_rsrc_t W8Rsrc;
constexpr int kW8Word3 = 0x00020000;  // gfx9 raw-buffer format word
constexpr int kW8Stream = 2;          // non-temporal: each weight byte is read once

__device__ __forceinline__ W8Rsrc w8_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kW8Word3);
}

__device__ __forceinline__ float dot16_i8(const u32x4& q, const float* x, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = q[i];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc = fmaf((float)(int8_t)(w >> (8 * b)), x[4 * i + b], acc);
  }
  return acc;
}

template <int kSeg, int kGroup>
struct W8Unit {
  u32x4 w[kW8Rows][kSeg];
  float s[kW8Rows][kGroup > 0 ? kSeg : 1];
};

// Issues the loads of unit u (an empty range when u >= units). Every load
// goes through a descriptor over exactly one row (of q, or of its scales),
// empty for rows past M, with the whole offset in the checked per-lane
// offset: the hardware range check covers the lane offset only (not the
// scalar offset), so this is what confines every read to its row. Lanes past
// the row's end (16 c >= K) and rows past M read zeros without touching
// memory.
template <int kSeg, int kGroup>
__device__ __forceinline__ void w8_load(const int8_t* q, const float* scales, int M, int K, int u, int units,
                                        W8Unit<kSeg, kGroup>& t) {
  const int l = lane_id();
  const int r0 = u * kW8Rows;
  const int rows = u < units ? min(kW8Rows, M - r0) : 0;
  const int groups = kGroup > 0 ? K / kGroup : 1;
#pragma unroll
  for (int r = 0; r < kW8Rows; ++r) {
    const bool in = r < rows;
    const size_t row = in ? (size_t)(r0 + r) : 0;
    const W8Rsrc rq = w8_rsrc(q + row * K, in ? K : 0);
    const W8Rsrc rs = w8_rsrc(scales + row * groups, in ? groups * 4 : 0);
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
      const int c = l + kWave * j;
      t.w[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rq, 16 * c, 0, kW8Stream);
      if constexpr (kGroup > 0)
        t.s[r][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * ((16 * c) / kGroup), 0, 0));
    }
    if constexpr (kGroup == 0) t.s[r][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 0, 0, 0));
  }
}

template <int kSeg, int kGroup>
__device__ __forceinline__ void w8_compute(const W8Unit<kSeg, kGroup>& t, const float (&xs)[kSeg][16], int segs,
                                           int M, int u, uint16_t* y) {
  const int l = lane_id();
#pragma unroll
  for (int r = 0; r < kW8Rows; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
      // segments past the row's end (lanes beyond K / 16) read zeros
      const bool in = l + kWave * j < segs;
      const float p = in ? dot16_i8(t.w[r][j], xs[j], 0.0f) : 0.0f;
      if constexpr (kGroup > 0) acc = fmaf(t.s[r][j], p, acc);
      else acc += p;
    }
    acc = wave_sum(acc);
    const int row = u * kW8Rows + r;
    if (l == 0 && row < M) {
      if constexpr (kGroup == 0) acc *= t.s[r][0];
      y[row] = f32_to_bf16(acc);
    }
  }
}

template <int kSeg, int kGroup>
__global__ void __launch_bounds__(kGemvThreads) k_w8_gemv(const int8_t* __restrict__ q,
                                                          const float* __restrict__ scales,
                                                          const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ y, int M, int K) {
  const WaveGrid g = wave_grid();
  const int l = lane_id();
  const int units = (M + kW8Rows - 1) / kW8Rows;
  if (g.wave >= units) return;
  const int segs = K / 16;  // 16-byte segments per row
  W8Unit<kSeg, kGroup> ta, tb;
  int u = g.wave;
  w8_load<kSeg, kGroup>(q, scales, M, K, u, units, ta);
  float xs[kSeg][16];
#pragma unroll
  for (int j = 0; j < kSeg; ++j) {
    const int c = l + kWave * j;
#pragma unroll
    for (int e = 0; e < 16; ++e) xs[j][e] = c < segs ? bf16_to_f32(x[16 * c + e]) : 0.0f;
  }
  while (true) {
    const int u1 = u + g.waves;
    w8_load<kSeg, kGroup>(q, scales, M, K, u1, units, tb);
    w8_compute<kSeg, kGroup>(ta, xs, segs, M, u, y);
    if (u1 >= units) break;
    const int u2 = u1 + g.waves;
    w8_load<kSeg, kGroup>(q, scales, M, K, u2, units, ta);
    w8_compute<kSeg, kGroup>(tb, xs, segs, M, u1, y);
    if (u2 >= units) break;
    u = u2;
  }
}

template <int kGroup>
static void launch_w8(int segs_per_lane, const int8_t* q, const float* s, const uint16_t* x, uint16_t* y, int M,
                      int K, hipStream_t st) {
  // Two blocks per CU, each wave looping over its units: more blocks shorten
  // the loops and lose the prefetch, fewer leave a CU short of loads in
  // flight (65,536 x 1,024, group 32: 128 blocks 27.9 us, 256 17.2, 512 15.0,
  // 1,024 17.9, 4,096 37.2).
  const int units = (M + kW8Rows - 1) / kW8Rows;
  const int blocks = max(1, min((units + kGemvWaves - 1) / kGemvWaves, 512));
  switch (segs_per_lane) {
    case 1: k_w8_gemv<1, kGroup><<<blocks, kGemvThreads, 0, st>>>(q, s, x, y, M, K); break;
    case 2: k_w8_gemv<2, kGroup><<<blocks, kGemvThreads, 0, st>>>(q, s, x, y, M, K); break;
    case 3: k_w8_gemv<3, kGroup><<<blocks, kGemvThreads, 0, st>>>(q, s, x, y, M, K); break;
    default: k_w8_gemv<4, kGroup><<<blocks, kGemvThreads, 0, st>>>(q, s, x, y, M, K); break;
  }
}

// ------------------------------------------------------------------ element-wise

constexpr int kEltThreads = 256;

static int elt_blocks(int n) { return max(1, min((n + kEltThreads - 1) / kEltThreads, 4096)); }

__global__ void k_f32_to_bf16(const float* __restrict__ in, uint16_t* __restrict__ out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = f32_to_bf16(in[i]);
}

__global__ void k_bf16_add(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                           uint16_t* __restrict__ out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

__global__ void k_silu_gate(const uint16_t* __restrict__ w1, const uint16_t* __restrict__ w3,
                            uint16_t* __restrict__ out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = f32_to_bf16(silu_bf16(bf16_to_f32(w1[i])) * bf16_to_f32(w3[i]));
}

// ------------------------------------------------------------------ conv gate

__global__ void k_conv_gate(const uint16_t* __restrict__ proj, const uint16_t* __restrict__ weight,
                            const uint16_t* __restrict__ prev, uint16_t* __restrict__ out,
                            uint16_t* __restrict__ next, uint16_t* __restrict__ weight_copy) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= kHidden) return;
  const float B = bf16_to_f32(proj[c]);
  const float C = bf16_to_f32(proj[kHidden + c]);
  const float x = bf16_to_f32(proj[2 * kHidden + c]);
  uint16_t s[3] = {prev[3 * c], prev[3 * c + 1], prev[3 * c + 2]};
  const float y = conv_gate_channel(B, C, x, weight + 3 * c, s, s);
  next[3 * c] = s[0];
  next[3 * c + 1] = s[1];
  next[3 * c + 2] = s[2];
  out[c] = f32_to_bf16(y);
  if (weight_copy != nullptr) {
    weight_copy[3 * c] = weight[3 * c];
    weight_copy[3 * c + 1] = weight[3 * c + 1];
    weight_copy[3 * c + 2] = weight[3 * c + 2];
  }
}

// ------------------------------------------------------------------ attention

// 24 heads (16 q, 8 k), one wave each, in place.
__global__ void __launch_bounds__(256) k_attention_norm_rope(uint16_t* __restrict__ qkv,
                                                             const uint16_t* __restrict__ aux) {
  const WaveGrid g = wave_grid();
  if (g.wave >= kHeads + kKvHeads) return;
  const int h = g.wave;
  uint16_t* v = qkv + (h < kHeads ? h * kHeadDim : kHidden + (h - kHeads) * kHeadDim);
  const uint16_t* gamma = aux + (h < kHeads ? 0 : kHeadDim);
  const int l = lane_id();
  const float o = norm_rope_lane(bf16_to_f32(v[l]), bf16_to_f32(gamma[l]),
                                 bf16_to_f32(aux[2 * kHeadDim + l]),
                                 bf16_to_f32(aux[3 * kHeadDim + l]));
  v[l] = f32_to_bf16(o);
}

// One block per KV head; cache per head = [keys past x 64 | values past x 64].
__global__ void __launch_bounds__(kAttnThreads) k_attention_context(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ cache,
    uint16_t* __restrict__ ctx, int past) {
  __shared__ AttnShared sh;
  const int h = blockIdx.x;
  attn_prep_plain(qkv + 2 * h * kHeadDim, qkv + kHidden + h * kHeadDim,
                  qkv + kHidden + kKvHeads * kHeadDim + h * kHeadDim, sh);
  const uint16_t* keys = cache + (size_t)h * 2 * past * kHeadDim;
  attn_core(keys, keys + (size_t)past * kHeadDim, past, ctx + 2 * h * kHeadDim, sh);
}

__global__ void k_attention_append(const uint16_t* __restrict__ qkv,
                                   const uint16_t* __restrict__ prior, uint16_t* __restrict__ next,
                                   int past) {
  const int per_head = 2 * (past + 1) * kHeadDim;
  const int total = kKvHeads * per_head;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int h = i / per_head;
    int r = i % per_head;
    const int kv = r / ((past + 1) * kHeadDim);  // 0 keys, 1 values
    r %= (past + 1) * kHeadDim;
    const int j = r / kHeadDim, d = r % kHeadDim;
    uint16_t v;
    if (j < past)
      v = prior[(size_t)h * 2 * past * kHeadDim + (size_t)kv * past * kHeadDim + j * kHeadDim + d];
    else
      v = qkv[kHidden + kv * kKvHeads * kHeadDim + h * kHeadDim + d];
    next[i] = v;
  }
}

// ------------------------------------------------------------------ argmax

constexpr int kScanThreads = 256;
constexpr int kArgmaxChunk = 4096;

static int argmax_blocks(int count) {
  return max(1, min((count + kArgmaxChunk - 1) / kArgmaxChunk, 1024));
}

__global__ void __launch_bounds__(kScanThreads) k_argmax_scan(const uint16_t* __restrict__ logits,
                                                              int count,
                                                              Candidate* __restrict__ cand) {
  __shared__ float red_v[kScanThreads / kWave];
  __shared__ int red_i[kScanThreads / kWave];
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    const float v = bf16_to_f32(logits[i]);
    if (better(v, i, best, best_i)) { best = v; best_i = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(best_i, o, kWave);
    if (better(ov, oi, best, best_i)) { best = ov; best_i = oi; }
  }
  if (lane_id() == 0) { red_v[wave_id()] = best; red_i[wave_id()] = best_i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kScanThreads / kWave; ++i)
      if (better(red_v[i], red_i[i], best, best_i)) { best = red_v[i]; best_i = red_i[i]; }
    cand[blockIdx.x] = {best, best_i};
  }
}

// Merge candidates; optionally copy the winning table row.
__global__ void __launch_bounds__(256) k_pick(const Candidate* __restrict__ cand, int n,
                                              int32_t* __restrict__ token,
                                              const uint16_t* __restrict__ table,
                                              uint16_t* __restrict__ row_out) {
  __shared__ int winner;
  if (wave_id() == 0) {
    const int w = pick_candidates(cand, n);
    if (lane_id() == 0) {
      winner = w;
      token[0] = w;
    }
  }
  __syncthreads();
  if (row_out != nullptr)
    for (int i = threadIdx.x; i < kHidden; i += blockDim.x)
      row_out[i] = table[(size_t)winner * kHidden + i];
}

constexpr int kHeadThreads = 256;

__global__ void __launch_bounds__(kHeadThreads) k_head_scan(const uint16_t* __restrict__ h,
                                                            const uint16_t* __restrict__ gamma,
                                                            const uint16_t* __restrict__ table,
                                                            int vocab, Candidate* __restrict__ cand,
                                                            uint16_t* __restrict__ logits) {
  __shared__ float red_v[kHeadThreads / kWave];
  __shared__ int red_i[kHeadThreads / kWave];
  stage_head_scan(h, gamma, table, vocab, cand, logits, red_v, red_i);
}

static int head_blocks(int vocab) {
  const int units = vocab / kHeadRows;
  return max(1, min((units + kHeadThreads / kWave - 1) / (kHeadThreads / kWave), 1024));
}

// ------------------------------------------------------------------ head without a workspace
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops): the head's per-block candidates live in a static
// device array, one per GPU the library runs on, held until the process ends.
// It holds one candidate per scan block, and head_blocks() never launches
// more than kScratchCandidates blocks (8 KB). Every slot a call reads is
// written by the same call first, so nothing needs clearing; calls that
// overlap on one GPU (two streams at once) race on the array.
constexpr int kScratchCandidates = 1024;
static __device__ __align__(256) Candidate scratch[kScratchCandidates];
constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static Candidate* g_scratch_of[kScratchDevices];  // device address of `scratch` per device

// The current device's copy of `scratch`, looked up once per device. The
// array's name is a host-side stand-in; kernels get this address.
static int scratch_of_current_device(Candidate** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(LFM25_EDEVICE, "fused_vocab_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kScratchDevices)
    return set_error(LFM25_EDEVICE, "fused_vocab_static: device %d beyond the %d supported", dev, kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_of[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t g = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (g != hipSuccess || ptr == nullptr)
      return set_error(LFM25_EDEVICE, "fused_vocab_static: hipGetSymbolAddress: %s", hipGetErrorString(g));
    g_scratch_of[dev] = static_cast<Candidate*>(ptr);
  }
  *out = g_scratch_of[dev];
  return LFM25_OK;
}

// ------------------------------------------------------------------ embedding

__global__ void k_embedding_gather(const uint16_t* __restrict__ table,
                                   const int32_t* __restrict__ token, uint16_t* __restrict__ out,
                                   int vocab, int32_t* __restrict__ status) {
  int t = token[0];
  if (t < 0 || t >= vocab) {
    if (threadIdx.x == 0 && status != nullptr) status[0] |= 1;
    t = t < 0 ? 0 : vocab - 1;
  }
  const int i = threadIdx.x * 8;
  if (i < kHidden)
    *reinterpret_cast<uint4*>(out + i) =
        *reinterpret_cast<const uint4*>(table + (size_t)t * kHidden + i);
}

}  // namespace lfm25

using namespace lfm25;

// ====================================================================== C ABI

extern "C" {

int lfm25_version(void) { return 100; }

const char* lfm25_last_error(void) { return g_error; }

int lfm25_rms_norm(const uint16_t* input, const uint16_t* gamma, uint16_t* output, int32_t cols,
                   lfm25_stream_t stream) {
  LFM25_REQUIRE(input && gamma && output, "rms_norm: null pointer");
  LFM25_REQUIRE(cols >= 1 && cols <= 65536, "rms_norm: cols must be in [1, 65536], got %d", cols);
  k_rms_norm<<<1, kNormThreads, 0, stream>>>(input, gamma, output, cols);
  return check_launch("rms_norm");
}

int lfm25_bf16_bf16_gemv(const uint16_t* weights, const uint16_t* activation, uint16_t* output,
                         int32_t M, int32_t K, lfm25_stream_t stream) {
  LFM25_REQUIRE(weights && activation && output, "bf16_bf16_gemv: null pointer");
  LFM25_REQUIRE(M >= 1 && K >= 8 && K % 8 == 0, "bf16_bf16_gemv: need M >= 1, K %% 8 == 0 (M=%d K=%d)",
                M, K);
  LFM25_REQUIRE(aligned16(weights) && aligned16(activation), "bf16_bf16_gemv: 16-byte alignment");
  return launch_gemv<uint16_t>(weights, activation, nullptr, output, M, K, false, stream);
}

int lfm25_bf16_f32_gemv(const uint16_t* weights, const uint16_t* activation, float* output,
                        int32_t M, int32_t K, lfm25_stream_t stream) {
  LFM25_REQUIRE(weights && activation && output, "bf16_f32_gemv: null pointer");
  LFM25_REQUIRE(M >= 1 && K >= 8 && K % 8 == 0, "bf16_f32_gemv: need M >= 1, K %% 8 == 0 (M=%d K=%d)",
                M, K);
  LFM25_REQUIRE(aligned16(weights) && aligned16(activation), "bf16_f32_gemv: 16-byte alignment");
  return launch_gemv<float>(weights, activation, nullptr, output, M, K, false, stream);
}

int lfm25_norm_bf16_gemv(const uint16_t* hidden, const uint16_t* packed, uint16_t* output,
                         int32_t M, int32_t K, lfm25_stream_t stream) {
  LFM25_REQUIRE(hidden && packed && output, "norm_bf16_gemv: null pointer");
  LFM25_REQUIRE(K == 1024, "norm_bf16_gemv: K must be 1024, got %d", K);
  LFM25_REQUIRE(M >= 1, "norm_bf16_gemv: M must be positive, got %d", M);
  LFM25_REQUIRE(aligned16(hidden) && aligned16(packed), "norm_bf16_gemv: 16-byte alignment");
  return launch_gemv<uint16_t>(packed + 4096, hidden, packed, output, M, K, true, stream);
}

int lfm25_w8_gemv(const int8_t* weights, const float* scales, const uint16_t* activation, uint16_t* output,
                  int32_t M, int32_t K, int32_t group, lfm25_stream_t stream) {
  LFM25_REQUIRE(weights && scales && activation && output, "w8_gemv: null pointer");
  LFM25_REQUIRE(M >= 1 && K >= 64 && K <= 4096 && K % 64 == 0,
                "w8_gemv: need M >= 1 and K a multiple of 64 in [64, 4096] (M=%d K=%d)", M, K);
  LFM25_REQUIRE(group == 0 || group == 32 || group == 64, "w8_gemv: group must be 0, 32 or 64, got %d", group);
  LFM25_REQUIRE(aligned16(weights), "w8_gemv: weights need 16-byte alignment");
  const int segs_per_lane = (K / 16 + kWave - 1) / kWave;
  if (group == 32) launch_w8<32>(segs_per_lane, weights, scales, activation, output, M, K, stream);
  else if (group == 64) launch_w8<64>(segs_per_lane, weights, scales, activation, output, M, K, stream);
  else launch_w8<0>(segs_per_lane, weights, scales, activation, output, M, K, stream);
  return check_launch("w8_gemv");
}

int lfm25_f32_to_bf16(const float* input, uint16_t* output, int32_t count, lfm25_stream_t stream) {
  LFM25_REQUIRE(input && output, "f32_to_bf16: null pointer");
  LFM25_REQUIRE(count >= 1, "f32_to_bf16: count must be positive");
  k_f32_to_bf16<<<elt_blocks(count), kEltThreads, 0, stream>>>(input, output, count);
  return check_launch("f32_to_bf16");
}

int lfm25_bf16_add(const uint16_t* left, const uint16_t* right, uint16_t* output, int32_t count,
                   lfm25_stream_t stream) {
  LFM25_REQUIRE(left && right && output, "bf16_add: null pointer");
  LFM25_REQUIRE(count >= 1, "bf16_add: count must be positive");
  k_bf16_add<<<elt_blocks(count), kEltThreads, 0, stream>>>(left, right, output, count);
  return check_launch("bf16_add");
}

int lfm25_silu_gate(const uint16_t* w1, const uint16_t* w3, uint16_t* output, int32_t count,
                    lfm25_stream_t stream) {
  LFM25_REQUIRE(w1 && w3 && output, "silu_gate: null pointer");
  LFM25_REQUIRE(count >= 1, "silu_gate: count must be positive");
  k_silu_gate<<<elt_blocks(count), kEltThreads, 0, stream>>>(w1, w3, output, count);
  return check_launch("silu_gate");
}

int lfm25_conv_gate(const uint16_t* projection_and_weight, const uint16_t* previous_state,
                    uint16_t* gated_output, uint16_t* next_state, lfm25_stream_t stream) {
  LFM25_REQUIRE(projection_and_weight && previous_state && gated_output && next_state,
                "conv_gate: null pointer");
  k_conv_gate<<<kHidden / 256, 256, 0, stream>>>(projection_and_weight,
                                                  projection_and_weight + 3 * kHidden,
                                                  previous_state, gated_output, next_state, nullptr);
  return check_launch("conv_gate");
}

int lfm25_conv_gate_packed_state(const uint16_t* projection, const uint16_t* state_and_weight,
                                 uint16_t* gated_output, uint16_t* next_state_and_weight,
                                 lfm25_stream_t stream) {
  LFM25_REQUIRE(projection && state_and_weight && gated_output && next_state_and_weight,
                "conv_gate_packed_state: null pointer");
  k_conv_gate<<<kHidden / 256, 256, 0, stream>>>(
      projection, state_and_weight + 3 * kHidden, state_and_weight, gated_output,
      next_state_and_weight, next_state_and_weight + 3 * kHidden);
  return check_launch("conv_gate_packed_state");
}

int lfm25_attention_norm_rope(uint16_t* qkv, const uint16_t* aux, lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv && aux, "attention_norm_rope: null pointer");
  k_attention_norm_rope<<<(kHeads + kKvHeads) / 4, 256, 0, stream>>>(qkv, aux);
  return check_launch("attention_norm_rope");
}

int lfm25_attention_context(const uint16_t* qkv, const uint16_t* past_cache, uint16_t* context,
                            int32_t past_length, lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv && context, "attention_context: null pointer");
  LFM25_REQUIRE(past_length >= 0 && past_length < kMaxCapacity,
                "attention_context: past_length must be in [0, %d), got %d", kMaxCapacity,
                past_length);
  LFM25_REQUIRE(past_length == 0 || (past_cache && aligned16(past_cache)),
                "attention_context: past_cache must be a 16-byte aligned pointer");
  k_attention_context<<<kKvHeads, kAttnThreads, 0, stream>>>(qkv, past_cache, context,
                                                             past_length);
  return check_launch("attention_context");
}

int lfm25_attention_append_cache(const uint16_t* qkv, const uint16_t* prior_cache,
                                 uint16_t* next_cache, int32_t past_length, lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv && next_cache, "attention_append_cache: null pointer");
  LFM25_REQUIRE(past_length >= 0 && past_length < kMaxCapacity,
                "attention_append_cache: past_length must be in [0, %d), got %d", kMaxCapacity,
                past_length);
  LFM25_REQUIRE(past_length == 0 || prior_cache, "attention_append_cache: null prior_cache");
  const int total = kKvHeads * 2 * (past_length + 1) * kHeadDim;
  k_attention_append<<<elt_blocks(total), kEltThreads, 0, stream>>>(qkv, prior_cache, next_cache,
                                                                    past_length);
  return check_launch("attention_append_cache");
}

size_t lfm25_argmax_workspace_bytes(int32_t count) {
  return (size_t)max(argmax_blocks(count), head_blocks(count)) * sizeof(Candidate);
}

int lfm25_argmax(const uint16_t* logits, int32_t count, int32_t* token_id, void* workspace,
                 lfm25_stream_t stream) {
  LFM25_REQUIRE(logits && token_id && workspace, "argmax: null pointer");
  LFM25_REQUIRE(count >= 1, "argmax: count must be positive");
  const int blocks = argmax_blocks(count);
  Candidate* cand = static_cast<Candidate*>(workspace);
  k_argmax_scan<<<blocks, kScanThreads, 0, stream>>>(logits, count, cand);
  k_pick<<<1, 256, 0, stream>>>(cand, blocks, token_id, nullptr, nullptr);
  return check_launch("argmax");
}

int lfm25_fused_vocab(const uint16_t* hidden, const uint16_t* packed, uint16_t* next_embedding,
                      int32_t* token_id, uint16_t* logits, int32_t vocab, void* workspace,
                      lfm25_stream_t stream) {
  LFM25_REQUIRE(hidden && packed && token_id && workspace, "fused_vocab: null pointer");
  LFM25_REQUIRE(vocab >= 4 && vocab % kHeadRows == 0, "fused_vocab: vocab must be a positive "
                "multiple of %d, got %d", kHeadRows, vocab);
  LFM25_REQUIRE(aligned16(hidden) && aligned16(packed), "fused_vocab: 16-byte alignment");
  const int blocks = head_blocks(vocab);
  Candidate* cand = static_cast<Candidate*>(workspace);
  const uint16_t* table = packed + kHidden;
  k_head_scan<<<blocks, kHeadThreads, 0, stream>>>(hidden, packed, table, vocab, cand, logits);
  k_pick<<<1, 256, 0, stream>>>(cand, blocks, token_id, table, next_embedding);
  return check_launch("fused_vocab");
}

int lfm25_fused_vocab_static(const uint16_t* hidden, const uint16_t* packed, uint16_t* next_embedding,
                             int32_t* token_id, uint16_t* logits, int32_t vocab, lfm25_stream_t stream) {
  LFM25_REQUIRE(hidden && packed && token_id, "fused_vocab_static: null pointer");
  LFM25_REQUIRE(vocab >= 4 && vocab % kHeadRows == 0 && vocab <= LFM25_VOCAB,
                "fused_vocab_static: vocab must be a multiple of %d in [4, %d], got %d", kHeadRows, LFM25_VOCAB,
                vocab);
  LFM25_REQUIRE(aligned16(hidden) && aligned16(packed), "fused_vocab_static: 16-byte alignment");
  const int blocks = head_blocks(vocab);
  LFM25_REQUIRE(blocks <= kScratchCandidates, "fused_vocab_static: %d scan blocks exceed the %d-candidate array",
                blocks, kScratchCandidates);
  Candidate* cand = nullptr;
  const int rc = scratch_of_current_device(&cand);
  if (rc != LFM25_OK) return rc;
  const uint16_t* table = packed + kHidden;
  k_head_scan<<<blocks, kHeadThreads, 0, stream>>>(hidden, packed, table, vocab, cand, logits);
  k_pick<<<1, 256, 0, stream>>>(cand, blocks, token_id, table, next_embedding);
  return check_launch("fused_vocab_static");
}

int lfm25_embedding_gather(const uint16_t* table, const int32_t* token_id, uint16_t* embedding,
                           int32_t vocab, int32_t* status, lfm25_stream_t stream) {
  LFM25_REQUIRE(table && token_id && embedding, "embedding_gather: null pointer");
  LFM25_REQUIRE(vocab >= 1, "embedding_gather: vocab must be positive");
  LFM25_REQUIRE(aligned16(table) && aligned16(embedding), "embedding_gather: 16-byte alignment");
  k_embedding_gather<<<1, kHidden / 8, 0, stream>>>(table, token_id, embedding, vocab, status);
  return check_launch("embedding_gather");
}

}  // extern "C"
