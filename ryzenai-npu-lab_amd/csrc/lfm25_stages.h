// The LFM2.5 decode step as a sequence of wave-parallel stages.
//
// Each stage is a device function that processes "units" (a conv channel, an
// output row, an FFN column, a KV head, a block of vocabulary rows) spread
// over all waves of the grid. The same functions are launched one kernel per
// stage (captured in a HIP graph) or called back to back from the persistent
// step kernel with grid barriers between them, so both execution models
// share one set of numerics.
//
// Stage list for one token (reference: the four stages per layer of
// experiments/lfm25_x8.py:248-290 and the head at :292-307):
//   conv layer : conv_in (norm + in_proj + gated short conv) -> proj_residual
//                (out_proj + residual) -> mlp_up (norm + w1/w3 + SiLU gate)
//                -> mlp_down (w2 + residual)
//   attn layer : qkv (norm + q/k/v) -> attention (QK norm, RoPE, KV append,
//                softmax, context) -> proj_residual (o_proj) -> mlp_up ->
//                mlp_down
//   head       : head_scan (final norm + tied head rows + running argmax)
//                -> head_pick (merge per-block candidates)
#pragma once
#include "lfm25_device.h"

namespace lfm25 {

// Largest KV capacity a session may use; the attention stage keeps one FP32
// score per cached position and query head in LDS.
constexpr int kMaxCapacity = 4096;
constexpr int kAttnThreads = 256;

struct WaveGrid {
  int wave;   // global wave index
  int waves;  // waves in the grid
};

__device__ __forceinline__ WaveGrid wave_grid() {
  const int wpb = blockDim.x / kWave;
  return {(int)blockIdx.x * wpb + wave_id(), (int)gridDim.x * wpb};
}

// ------------------------------------------------------------------ conv

// Gated short convolution of one channel (HF Lfm2ShortConv.forward,
// modeling_lfm2.py:350-389, with the per-product rounding of
// experiments/006_lfm25_cpu_two_recurrent_layers.py:41-47 and
// kernels/lfm25_conv_gate.cc:8-43):
//   bx = bf16(B*x); state' = [s1, s2, bx];
//   c  = bf16(bf16(s1*w0) + bf16(s2*w1) + bf16(bx*w2)); y = bf16(C*c).
// `state` points at this channel's three taps [s0, s1, s2] and is updated.
__device__ __forceinline__ float conv_gate_channel(float B, float C, float x, const uint16_t* w,
                                                   uint16_t* state_in, uint16_t* state_out) {
  const float bx = round_bf16(B * x);
  const float s1 = bf16_to_f32(state_in[1]);
  const float s2 = bf16_to_f32(state_in[2]);
  const float p0 = round_bf16(s1 * bf16_to_f32(w[0]));
  const float p1 = round_bf16(s2 * bf16_to_f32(w[1]));
  const float p2 = round_bf16(bx * bf16_to_f32(w[2]));
  const float c = round_bf16((p0 + p1) + p2);
  state_out[0] = f32_to_bf16(s1);
  state_out[1] = f32_to_bf16(s2);
  state_out[2] = f32_to_bf16(bx);
  return round_bf16(C * c);
}

// conv_gate_channel in two parts: the taps over the two kept state values
// (p0 + p1, the first addition of its sum), then the rest from the
// projections. Same operations in the same order, so the same bits.
__device__ __forceinline__ float conv_state_taps(const uint16_t* w, const uint16_t* state_in) {
  const float p0 = round_bf16(bf16_to_f32(state_in[1]) * bf16_to_f32(w[0]));
  const float p1 = round_bf16(bf16_to_f32(state_in[2]) * bf16_to_f32(w[1]));
  return p0 + p1;
}
__device__ __forceinline__ float conv_gate_channel_from(float B, float C, float x, const uint16_t* w,
                                                        const uint16_t* state_in, float p01, uint16_t* state_out) {
  const float bx = round_bf16(B * x);
  const float p2 = round_bf16(bx * bf16_to_f32(w[2]));
  const float c = round_bf16(p01 + p2);
  state_out[0] = f32_to_bf16(bf16_to_f32(state_in[1]));
  state_out[1] = f32_to_bf16(bf16_to_f32(state_in[2]));
  state_out[2] = f32_to_bf16(bx);
  return round_bf16(C * c);
}

// Stage conv_in: one unit per channel c (1024 units). Rows c, 1024+c and
// 2048+c of in_proj give B, C and x of channel c, so the conv gate fuses
// into the projection epilogue (the ownership trick of
// experiments/lfm25_x8.py:452-464).
__device__ __forceinline__ void stage_conv_in(const uint16_t* x_src, const uint16_t* gamma,
                                              const uint16_t* w_in, const uint16_t* conv_w,
                                              uint16_t* state, uint16_t* y_out) {
  const WaveGrid g = wave_grid();
  if (g.wave >= kHidden) return;
  LaneVec<kHidden> x;
  load_lane_vec<kHidden>(x_src, x);
  rms_norm_lane_vec<kHidden>(x, gamma);
  for (int c = g.wave; c < kHidden; c += g.waves) {
    const uint16_t* rows[3] = {w_in + (size_t)c * kHidden, w_in + (size_t)(kHidden + c) * kHidden,
                               w_in + (size_t)(2 * kHidden + c) * kHidden};
    float d[3];
    rows_dot<kHidden, 3>(rows, x, d);
    if (lane_id() == 0) {
      uint16_t* s = state + c * kConvTaps;
      const float y = conv_gate_channel(round_bf16(d[0]), round_bf16(d[1]), round_bf16(d[2]),
                                        conv_w + c * kConvTaps, s, s);
      y_out[c] = f32_to_bf16(y);
    }
  }
}

// Stage proj_residual: h[r] = bf16(h[r] + bf16(W[r] . v)), K = 1024
// (out_proj of the conv block, o_proj of attention; the residual add of
// Lfm2DecoderLayer.forward, modeling_lfm2.py:431).
constexpr int kProjRows = 4;
__device__ __forceinline__ void stage_proj_residual(const uint16_t* v, const uint16_t* w,
                                                    uint16_t* h) {
  const WaveGrid g = wave_grid();
  constexpr int kUnits = kHidden / kProjRows;
  if (g.wave >= kUnits) return;
  LaneVec<kHidden> x;
  load_lane_vec<kHidden>(v, x);
  for (int u = g.wave; u < kUnits; u += g.waves) {
    const int r0 = u * kProjRows;
    const uint16_t* rows[kProjRows];
#pragma unroll
    for (int r = 0; r < kProjRows; ++r) rows[r] = w + (size_t)(r0 + r) * kHidden;
    float d[kProjRows];
    rows_dot<kHidden, kProjRows>(rows, x, d);
    if (lane_id() < kProjRows) {
      float mine = d[0];
#pragma unroll
      for (int r = 1; r < kProjRows; ++r) mine = lane_id() == r ? d[r] : mine;
      const int row = r0 + lane_id();
      h[row] = f32_to_bf16(bf16_to_f32(h[row]) + round_bf16(mine));
    }
  }
}

// Stage mlp_up: g[f] = bf16(bf16(silu(bf16(w1[f].n))) * bf16(w3[f].n)) with
// n = RMSNorm(h) (Lfm2MLP.forward, modeling_lfm2.py:135-136; SiLU in FP32
// then rounded, kernels/lfm25_silu_gate.cc:22-39). Two FFN columns per unit.
constexpr int kUpCols = 2;
__device__ __forceinline__ void stage_mlp_up(const uint16_t* h, const uint16_t* gamma,
                                             const uint16_t* w1, const uint16_t* w3,
                                             uint16_t* g_out) {
  const WaveGrid g = wave_grid();
  constexpr int kUnits = kFfn / kUpCols;
  if (g.wave >= kUnits) return;
  LaneVec<kHidden> x;
  load_lane_vec<kHidden>(h, x);
  rms_norm_lane_vec<kHidden>(x, gamma);
  for (int u = g.wave; u < kUnits; u += g.waves) {
    const int f0 = u * kUpCols;
    const uint16_t* rows[2 * kUpCols];
#pragma unroll
    for (int j = 0; j < kUpCols; ++j) {
      rows[2 * j] = w1 + (size_t)(f0 + j) * kHidden;
      rows[2 * j + 1] = w3 + (size_t)(f0 + j) * kHidden;
    }
    float d[2 * kUpCols];
    rows_dot<kHidden, 2 * kUpCols>(rows, x, d);
    if (lane_id() < kUpCols) {
      float a = d[0], b = d[1];
#pragma unroll
      for (int j = 1; j < kUpCols; ++j)
        if (lane_id() == j) { a = d[2 * j]; b = d[2 * j + 1]; }
      const float s = silu_bf16(round_bf16(a));
      g_out[f0 + lane_id()] = f32_to_bf16(s * round_bf16(b));
    }
  }
}

// Stage mlp_down: h[r] = bf16(h[r] + bf16(w2[r] . g)), K = 2560.
constexpr int kDownRows = 2;
__device__ __forceinline__ void stage_mlp_down(const uint16_t* gvec, const uint16_t* w2,
                                               uint16_t* h) {
  const WaveGrid g = wave_grid();
  constexpr int kUnits = kHidden / kDownRows;
  if (g.wave >= kUnits) return;
  LaneVec<kFfn> x;
  load_lane_vec<kFfn>(gvec, x);
  for (int u = g.wave; u < kUnits; u += g.waves) {
    const int r0 = u * kDownRows;
    const uint16_t* rows[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) rows[r] = w2 + (size_t)(r0 + r) * kFfn;
    float d[kDownRows];
    rows_dot<kFfn, kDownRows>(rows, x, d);
    if (lane_id() < kDownRows) {
      const float mine = lane_id() == 0 ? d[0] : d[1];
      const int row = r0 + lane_id();
      h[row] = f32_to_bf16(bf16_to_f32(h[row]) + round_bf16(mine));
    }
  }
}

// Stage qkv: rows [0,1024) of q, [1024,1536) of k, [1536,2048) of v;
// qkv[r] = bf16(W[r] . RMSNorm(h)).
constexpr int kQkvRows = 4;
__device__ __forceinline__ void stage_qkv(const uint16_t* x_src, const uint16_t* gamma,
                                          const uint16_t* wq, const uint16_t* wk,
                                          const uint16_t* wv, uint16_t* qkv) {
  const WaveGrid g = wave_grid();
  constexpr int kRows = kHidden + 2 * kKvHeads * kHeadDim;  // 2048
  constexpr int kUnits = kRows / kQkvRows;
  if (g.wave >= kUnits) return;
  LaneVec<kHidden> x;
  load_lane_vec<kHidden>(x_src, x);
  rms_norm_lane_vec<kHidden>(x, gamma);
  for (int u = g.wave; u < kUnits; u += g.waves) {
    const int r0 = u * kQkvRows;
    const uint16_t* rows[kQkvRows];
#pragma unroll
    for (int r = 0; r < kQkvRows; ++r) {
      const int row = r0 + r;
      rows[r] = row < kHidden ? wq + (size_t)row * kHidden
              : row < kHidden + 512 ? wk + (size_t)(row - kHidden) * kHidden
                                    : wv + (size_t)(row - kHidden - 512) * kHidden;
    }
    float d[kQkvRows];
    rows_dot<kHidden, kQkvRows>(rows, x, d);
    if (lane_id() < kQkvRows) {
      float mine = d[0];
#pragma unroll
      for (int r = 1; r < kQkvRows; ++r) mine = lane_id() == r ? d[r] : mine;
      qkv[r0 + lane_id()] = f32_to_bf16(mine);
    }
  }
}

// ------------------------------------------------------------------ attention

// Per-head RMSNorm over 64 values then rotary embedding, lane d owning
// element d (Lfm2Attention q/k_layernorm, modeling_lfm2.py:239-240, and
// apply_rotary_pos_emb :147-169; kernels/lfm25_attention_norm_rope.cc:17-54):
//   n = bf16(bf16(x*r)*gamma); out = bf16(bf16(n*cos) + bf16(rot(n)*sin)),
//   rot(n)[d] = d < 32 ? -n[d+32] : n[d-32].
__device__ __forceinline__ float norm_rope_lane(float x, float gamma, float cos_d, float sin_d) {
  const float ss = wave_sum(x * x);
  const float r = 1.0f / sqrtf(ss * (1.0f / (float)kHeadDim) + kNormEps);
  const float n = round_bf16(round_bf16(x * r) * gamma);
  const int d = lane_id();
  const float partner = __shfl_xor(n, 32, kWave);
  const float rot = d < 32 ? -partner : partner;
  return round_bf16(round_bf16(n * cos_d) + round_bf16(rot * sin_d));
}

// Shared-memory layout of the attention stage for a block of kThreads.
template <int kThreads>
struct AttnSharedT {
  float q[2][kHeadDim];         // rotated query heads of this KV group
  float k_new[kHeadDim];        // rotated key of the current position
  float v_new[kHeadDim];        // value of the current position
  float score[2][kMaxCapacity + 1];
  float red[2][kThreads / kWave];
  float red_sum[2][kThreads / kWave];
  float ctx[kThreads / kWave][2][kHeadDim];
  float out[2 * kHeadDim];      // BF16-rounded context of the two query heads
  float raw[4][kHeadDim];       // gathered q0, q1, k, v projections
};
using AttnShared = AttnSharedT<kAttnThreads>;

// Attention prologue for one KV head: QK norm + RoPE of the two query heads
// and the key of the current position (waves 0..2) and the raw value
// (wave 3), into shared memory; appends the rotated key and the value to the
// cache at `pos` when keys/values are given. Must be called by all
// kAttnThreads threads of a block; q_raw/k_raw/v_raw are un-normalised
// projections.
__device__ __forceinline__ void attn_prep_norm_rope(
    const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw, const uint16_t* q_gamma,
    const uint16_t* k_gamma, const uint16_t* cos_row, const uint16_t* sin_row, uint16_t* keys,
    uint16_t* values, int pos, AttnShared& sh) {
  const int w = wave_id();
  const int l = lane_id();
  if (w < 3) {
    const uint16_t* src = w < 2 ? q_raw + w * kHeadDim : k_raw;
    const uint16_t* gam = w < 2 ? q_gamma : k_gamma;
    const float o = norm_rope_lane(bf16_to_f32(src[l]), bf16_to_f32(gam[l]),
                                   bf16_to_f32(cos_row[l]), bf16_to_f32(sin_row[l]));
    if (w < 2) {
      sh.q[w][l] = o;
    } else {
      sh.k_new[l] = o;
      if (keys != nullptr) keys[(size_t)pos * kHeadDim + l] = f32_to_bf16(o);
    }
  } else if (w == 3) {
    sh.v_new[l] = bf16_to_f32(v_raw[l]);
    if (values != nullptr) values[(size_t)pos * kHeadDim + l] = v_raw[l];
  }
  __syncthreads();
}

// Attention prologue when q/k are already normalised and rotated.
__device__ __forceinline__ void attn_prep_plain(const uint16_t* q, const uint16_t* k,
                                                const uint16_t* v, AttnShared& sh) {
  const int t = threadIdx.x;
  if (t < 2 * kHeadDim) sh.q[t / kHeadDim][t % kHeadDim] = bf16_to_f32(q[t]);
  else if (t < 3 * kHeadDim) sh.k_new[t - 2 * kHeadDim] = bf16_to_f32(k[t - 2 * kHeadDim]);
  else if (t < 4 * kHeadDim) sh.v_new[t - 3 * kHeadDim] = bf16_to_f32(v[t - 3 * kHeadDim]);
  __syncthreads();
}

// Where cached position j's key and value rows (64 BF16 each) live.
// ContiguousRows: rows [0, past) back to back per head, 16-byte aligned.
struct ContiguousRows {
  const uint16_t* keys;
  const uint16_t* values;
  static constexpr bool kAligned16 = true;
  __device__ const uint16_t* key(int j) const { return keys + (size_t)j * kHeadDim; }
  __device__ const uint16_t* value(int j) const { return values + (size_t)j * kHeadDim; }
};

// 8 BF16 values of a row: one 16-byte load, or four 4-byte loads for rows
// that are only 4-byte aligned.
template <bool kAligned16>
__device__ __forceinline__ void load_row8(const uint16_t* p, float* f) {
  if constexpr (kAligned16) {
    unpack8(load8(p), f);
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = q[i];
      f[2 * i] = lo_f32(w);
      f[2 * i + 1] = hi_f32(w);
    }
  }
}

// One KV head (two query heads) of GQA decode attention over `past` cached
// positions plus the current one (held in shared memory by a prologue),
// eager semantics (eager_attention_forward, modeling_lfm2.py:184-207;
// kernels/lfm25_attention_context_head.cc:19-82):
//   s_j = bf16(q.k_j) * 0.125 ; p_j = bf16(exp(s_j - max) / sum) ;
//   ctx = bf16(sum_j p_j v_j).
// `rows` locates cached rows [0, past) (see ContiguousRows). Must be called
// by all kThreads threads of a block.
template <int kThreads, typename Rows = ContiguousRows>
__device__ __forceinline__ void attn_core_t(const Rows& rows, int past, AttnSharedT<kThreads>& sh) {
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  constexpr int kWaves = kThreads / kWave;
  constexpr int kPerPass = kThreads / 8;
  constexpr int kAttnThreads = kThreads;
  const int total = past + 1;

  // Scores: eight lanes per position, each lane eight dimensions.
  const int sub = l & 7;
  const int slot = tid >> 3;
  float q0[8], q1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    q0[i] = sh.q[0][sub * 8 + i];
    q1[i] = sh.q[1][sub * 8 + i];
  }
  // Every lane loads a cached row (positions past the cache clamped to its
  // last row, then replaced), with no branch around the load, so that the
  // loads of several passes are in flight together.
  const int last = past > 0 ? past - 1 : 0;
  float kn[8], vn[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kn[i] = sh.k_new[sub * 8 + i];
    vn[i] = sh.v_new[sub * 8 + i];
  }
  const auto score = [&](int j, float* kf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) kf[i] = j < past ? kf[i] : j == past ? kn[i] : 0.0f;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a0 = fmaf(q0[i], kf[i], a0);
      a1 = fmaf(q1[i], kf[i], a1);
    }
    a0 = group_sum<8>(a0);
    a1 = group_sum<8>(a1);
    if (sub == 0 && j < total) {
      sh.score[0][j] = round_bf16(a0) * 0.125f;
      sh.score[1][j] = round_bf16(a1) * 0.125f;
    }
  };
  if (past > 0) {
    // four passes per round, all four rows requested first (the lane sums
    // inside keep the compiler from unrolling a loop of single passes; the
    // passes past the end recompute the last row and store nothing)
    for (int base = 0; base < total; base += 4 * kPerPass) {
      float kf[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        load_row8<Rows::kAligned16>(rows.key(min(base + u * kPerPass + slot, last)) + sub * 8, kf[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u) score(base + u * kPerPass + slot, kf[u]);
    }
  } else {
    float kf[8] = {};
    score(slot, kf);  // the one position: the new key
  }
  lds_barrier();

  // Softmax in FP32 per query head; probabilities rounded to BF16.
  float m0 = -INFINITY, m1 = -INFINITY;
  for (int j = tid; j < total; j += kAttnThreads) {
    m0 = fmaxf(m0, sh.score[0][j]);
    m1 = fmaxf(m1, sh.score[1][j]);
  }
  m0 = wave_max(m0);
  m1 = wave_max(m1);
  if (l == 0) { sh.red[0][w] = m0; sh.red[1][w] = m1; }
  lds_barrier();
  m0 = sh.red[0][0];
  m1 = sh.red[1][0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) { m0 = fmaxf(m0, sh.red[0][i]); m1 = fmaxf(m1, sh.red[1][i]); }
  lds_barrier();
  float z0 = 0.0f, z1 = 0.0f;
  for (int j = tid; j < total; j += kAttnThreads) {
    const float e0 = expf(sh.score[0][j] - m0);
    const float e1 = expf(sh.score[1][j] - m1);
    sh.score[0][j] = e0;
    sh.score[1][j] = e1;
    z0 += e0;
    z1 += e1;
  }
  z0 = wave_sum(z0);
  z1 = wave_sum(z1);
  if (l == 0) { sh.red[0][w] = z0; sh.red[1][w] = z1; }
  lds_barrier();
  z0 = sh.red[0][0];
  z1 = sh.red[1][0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) { z0 += sh.red[0][i]; z1 += sh.red[1][i]; }
  for (int j = tid; j < total; j += kAttnThreads) {
    sh.score[0][j] = round_bf16(sh.score[0][j] / z0);
    sh.score[1][j] = round_bf16(sh.score[1][j] / z1);
  }
  lds_barrier();

  // Context: eight lanes per position, eight dimensions per lane.
  float c0[8], c1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) { c0[i] = 0.0f; c1[i] = 0.0f; }
  const auto context = [&](int j, float* vf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) vf[i] = j < past ? vf[i] : vn[i];
    const int jc = min(j, past);  // (lanes past the last position add nothing)
    const float p0 = sh.score[0][jc], p1 = sh.score[1][jc];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c0[i] = j < total ? fmaf(p0, vf[i], c0[i]) : c0[i];
      c1[i] = j < total ? fmaf(p1, vf[i], c1[i]) : c1[i];
    }
  };
  if (past > 0) {
#pragma unroll 4
    for (int base = 0; base < total; base += kPerPass) {
      float vf[8];
      load_row8<Rows::kAligned16>(rows.value(min(base + slot, last)) + sub * 8, vf);
      context(base + slot, vf);
    }
  } else {
    float vf[8] = {};
    context(slot, vf);
  }
  // Lanes with equal `sub` hold the same dimensions: fold lane groups 8 apart.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int o = 8; o < kWave; o <<= 1) {
      c0[i] += __shfl_xor(c0[i], o, kWave);
      c1[i] += __shfl_xor(c1[i], o, kWave);
    }
  }
  if (l < 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sh.ctx[w][0][l * 8 + i] = c0[i];
      sh.ctx[w][1][l * 8 + i] = c1[i];
    }
  }
  lds_barrier();
  if (tid < 2 * kHeadDim) {
    const int hq = tid / kHeadDim, d = tid % kHeadDim;
    float s = sh.ctx[0][hq][d];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) s += sh.ctx[i][hq][d];
    sh.out[tid] = round_bf16(s);
  }
  lds_barrier();
}

// attn_core_t for 256-thread blocks, context written as BF16 to ctx_out.
__device__ __forceinline__ void attn_core(const uint16_t* keys, const uint16_t* values, int past,
                                          uint16_t* ctx_out, AttnShared& sh) {
  attn_core_t<kAttnThreads>(ContiguousRows{keys, values}, past, sh);
  if (threadIdx.x < 2 * kHeadDim) ctx_out[threadIdx.x] = f32_to_bf16(sh.out[threadIdx.x]);
  __syncthreads();
}

// ------------------------------------------------------------------ head

// Candidate (value, row) ordering: larger value wins, equal values keep the
// lower row, so any merge order yields the first maximum (argmax; the strict
// '>' scan of kernels/x8/x8_core.cc:126-137 and the tie rule of
// kernels/lfm25_vocab_accept_candidate.cc:5-16).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

struct Candidate {
  float value;
  int32_t row;
};

constexpr int kHeadRows = 4;

// Stage head_scan: logits = bf16(E[v] . RMSNorm(h)) for the vocabulary rows
// of this block; writes the block's best (value, row) to cand[blockIdx.x].
// Optionally also stores every BF16 logit.
__device__ __forceinline__ void stage_head_scan(const uint16_t* h, const uint16_t* gamma,
                                                const uint16_t* table, int vocab,
                                                Candidate* cand, uint16_t* logits_out,
                                                float* red_v, int* red_i) {
  const WaveGrid g = wave_grid();
  LaneVec<kHidden> x;
  load_lane_vec<kHidden>(h, x);
  rms_norm_lane_vec<kHidden>(x, gamma);
  float best = -INFINITY;
  int best_row = 0x7fffffff;
  const int units = vocab / kHeadRows;
  for (int u = g.wave; u < units; u += g.waves) {
    const int r0 = u * kHeadRows;
    const uint16_t* rows[kHeadRows];
#pragma unroll
    for (int r = 0; r < kHeadRows; ++r) rows[r] = table + (size_t)(r0 + r) * kHidden;
    float d[kHeadRows];
    rows_dot<kHidden, kHeadRows>(rows, x, d);
#pragma unroll
    for (int r = 0; r < kHeadRows; ++r) {
      const float v = round_bf16(d[r]);
      if (better(v, r0 + r, best, best_row)) { best = v; best_row = r0 + r; }
    }
    if (logits_out != nullptr && lane_id() < kHeadRows) {
      float mine = d[0];
#pragma unroll
      for (int r = 1; r < kHeadRows; ++r) mine = lane_id() == r ? d[r] : mine;
      logits_out[r0 + lane_id()] = f32_to_bf16(mine);
    }
  }
  const int w = wave_id();
  if (lane_id() == 0) { red_v[w] = best; red_i[w] = best_row; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = red_v[0];
    int bi = red_i[0];
    const int wpb = blockDim.x / kWave;
    for (int i = 1; i < wpb; ++i)
      if (better(red_v[i], red_i[i], bv, bi)) { bv = red_v[i]; bi = red_i[i]; }
    cand[blockIdx.x] = {bv, bi};
  }
  __syncthreads();
}

// Merge n candidates (one block); returns the winner in every thread of
// wave 0 and writes it to *token when token != nullptr.
__device__ __forceinline__ int pick_candidates(const Candidate* cand, int n) {
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = lane_id(); i < n; i += kWave) {
    const Candidate c = cand[i];
    if (better(c.value, c.row, bv, bi)) { bv = c.value; bi = c.row; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  return bi;
}

}  // namespace lfm25
