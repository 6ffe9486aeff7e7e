// The whole-token LFM2.5 decode step (the X8Model step of
// experiments/lfm25_x8_model.py:133-148 and the one-submission-per-token
// program of experiments/lfm25_x8.py:227-327) on gfx950.
//
// Two execution models over the same block-level phases (lfm25_step.h), on
// the same 256-block grid and with the same epoch tags, so they are bitwise
// identical:
//   * persistent : cooperative launches that keep the grid across steps run
//                  the steps of a decode call (one launch for a short call,
//                  else one per attention path, see k_decode_persistent);
//                  phases hand activations to each other through tagged
//                  words (the data is the barrier), most of them inside one
//                  XCD, and the token chosen by the head feeds the next step
//                  without returning to the host;
//   * staged     : one kernel per phase (about 100 per token), stream ordered
//                  and capturable in a HIP graph.
// Position, current token, epoch and status live in device control words, so
// neither model needs a host round trip between tokens.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "lfm25_host.h"
#include "lfm25_layout.h"
#include "lfm25_step.h"
#include "lfm25_step_w8.h"
#include "lfm25_bstep.h"

namespace lfm25 {

constexpr int kCtlStep = 3;         // step index within the current decode call
constexpr int kCtlEpoch = 4;        // last epoch tag used (16-bit, wraps)
constexpr int kGrid = kStepBlocks;  // blocks of both execution models
static_assert(kCtlStatus == LFM25_CTL_STATUS, "status word");

struct DecodeParams {
  const uint16_t* weights;  // the packed stream
  const uint16_t* embedding;
  const uint16_t* rope;
  uint16_t* conv_state;
  uint16_t* key_cache;
  uint16_t* value_cache;
  int32_t* ctl;
  StepBufs bufs;
  const int32_t* tokens_in;
  int32_t* tokens_out;
  int n_in, n_gen, capacity, vocab;
  // 8-bit weights (lfm25_decode_w8; null otherwise): the layers' projections
  // and the tied table with its scales. Norms, conv taps and QK-norm weights
  // still come from `weights`.
  const int8_t* w8;
  const int8_t* w8_table;
  const float* w8_table_s;
};

static DecodeParams make_params(const lfm25_decoder* d, const int32_t* tokens_in, int n_in,
                                int n_gen, int32_t* tokens_out) {
  DecodeParams p{};
  p.weights = d->weights;
  p.embedding = d->embedding;
  p.rope = d->rope;
  p.conv_state = d->conv_state;
  p.key_cache = d->key_cache;
  p.value_cache = d->value_cache;
  char* ws = static_cast<char*>(d->workspace);
  p.ctl = reinterpret_cast<int32_t*>(ws + kWsCtl);
  p.bufs.ws = ws;
  p.tokens_in = tokens_in;
  p.tokens_out = tokens_out;
  p.n_in = n_in;
  p.n_gen = n_gen;
  p.capacity = d->capacity;
  p.vocab = d->vocab;
  return p;
}

__device__ __forceinline__ int ctl_load(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ctl_store(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ctl_or(int32_t* p, int v) {
  __hip_atomic_fetch_or(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int clamp_token(int t, int vocab, int32_t* ctl, bool report) {
  if (t < 0 || t >= vocab) {
    if (report) ctl_or(ctl + LFM25_CTL_STATUS, 1);
    t = t < 0 ? 0 : vocab - 1;
  }
  return t;
}

__device__ __forceinline__ uint16_t* conv_state_of(const DecodeParams& p, int conv_index) {
  return p.conv_state + (size_t)conv_index * kHidden * kConvTaps;
}

// RMSNorm weights of a step, n = 0 .. 2 kLayers: op_norm and ffn_norm of
// every layer, then the final norm.
__device__ __forceinline__ const uint16_t* norm_weight(const DecodeParams& p, int n) {
  if (n == 2 * kLayers) return final_norm(p.weights);
  const int l = n / 2;
  return (n & 1) ? layer_tensor<C_FFNNORM, A_FFNNORM>(p.weights, l) : layer_tensor<C_OPNORM, A_OPNORM>(p.weights, l);
}

// Shared memory of one decode block.
struct StepShared {
  alignas(16) uint32_t vec[2][kNormWords];  // double-buffered gathered vectors (bf16 pairs)
  Gathered in;                              // the current gather, before the norm
  StepOut out;                              // a phase's outputs before publish
  AttnSplitShared attn;
  float red_v[kStepWaves];
  int red_i[kStepWaves];
  float red_part[kXcds][kResRows];          // an R phase's partials, one row of them per XCD
  // each wave's first kHeadStaged head units (the 8-bit head stages one)
  alignas(16) uint32_t head_rows[kStepWaves][kHeadStaged * kStepHeadRows][kNormWords];
};

// Eight embedding rows in the head staging area (free from the end of the
// head scan to the next head): pick_global's copies of the XCD winners' rows.
__device__ __forceinline__ uint32_t (*pick_rows(StepShared& sm))[kNormWords] {
  static_assert(sizeof(sm.head_rows) >= kXcds * kNormWords * sizeof(uint32_t), "eight rows fit");
  return reinterpret_cast<uint32_t(*)[kNormWords]>(&sm.head_rows[0][0][0]);
}

// Epoch tags of one step, assigned in exchange order (shared by both
// execution models so they produce identical tags).
struct StepTags {
  uint32_t base;
  int next = 0;
  __device__ __host__ uint32_t take() { return (base + (uint32_t)(++next)) & 0xffffu; }
  __device__ __host__ uint32_t skip(int n) {
    next += n;
    return (base + (uint32_t)next) & 0xffffu;
  }
};

// Exchanges of one step: 6 per conv layer; 8 per attention layer (q/k/v,
// the split attention's statistics, the context, then as a conv layer's
// last five); 2 for the head and the pick.
__host__ __device__ constexpr int layer_exchanges(int l) { return is_attn(l) ? 8 : 6; }
constexpr int kExchangesNoHead = 6 * LFM25_CONV_LAYERS + 8 * LFM25_ATTN_LAYERS;
constexpr int kExchangesHead = 2;

// The group that computes layer l.
__host__ __device__ constexpr int layer_group(int l) { return l & 1; }

// Weight tensors of layer l from (laundered) bases. An attention layer passes
// layer 0's conv operands, which its units load with an empty descriptor and
// never use.
__device__ __forceinline__ LayerWeights layer_weights(const uint16_t* w, const uint16_t* conv_state, int l) {
  const bool attn = is_attn(l);
  LayerWeights L;
  L.attn = attn;
  L.wa = layer_tensor<C_IN, A_Q>(w, l);
  L.conv_w = conv_tensor<C_CONVW>(w, attn ? 0 : l);
  L.state = conv_state + (size_t)(attn ? 0 : conv_before(l)) * kHidden * kConvTaps;
  L.wb = layer_tensor<C_OUT, A_O>(w, l);
  L.w1 = layer_tensor<C_W1, A_W1>(w, l);
  L.w3 = layer_tensor<C_W3, A_W3>(w, l);
  L.w2 = layer_tensor<C_W2, A_W2>(w, l);
  return L;
}

// The 8-bit projections of layer l (same conventions as layer_weights).
__device__ __forceinline__ LayerWeights8 layer_weights8(const int8_t* w8, const uint16_t* w, const uint16_t* conv_state,
                                                        int l) {
  const bool attn = is_attn(l);
  LayerWeights8 L;
  L.attn = attn;
  L.qa = w8_q<P_MIX>(w8, l);
  L.sa = w8_s<P_MIX>(w8, l);
  L.conv_w = conv_tensor<C_CONVW>(w, attn ? 0 : l);
  L.state = conv_state + (size_t)(attn ? 0 : conv_before(l)) * kHidden * kConvTaps;
  L.qb = w8_q<P_OUT>(w8, l);
  L.sb = w8_s<P_OUT>(w8, l);
  L.q1 = w8_q<P_W1>(w8, l);
  L.s1 = w8_s<P_W1>(w8, l);
  L.q3 = w8_q<P_W3>(w8, l);
  L.s3 = w8_s<P_W3>(w8, l);
  L.q2 = w8_q<P_W2>(w8, l);
  L.s2 = w8_s<P_W2>(w8, l);
  return L;
}

// Requests the weights of layer l into the slabs (either format).
__device__ __forceinline__ void load_layer(Slabs& S, const DecodeParams& p, int l) {
  load_slabs(S, layer_weights(launder(p.weights), launder(p.conv_state), l));
}
__device__ __forceinline__ void load_layer(Slabs8& S, const DecodeParams& p, int l) {
  load_slabs(S, layer_weights8(launder(p.w8), launder(p.weights), launder(p.conv_state), l));
}

// Offset of KV head x of attention layer l in the key / value caches.
__device__ __forceinline__ size_t kv_head_offset(const DecodeParams& p, int l, int x) {
  return (size_t)((l - conv_before(l)) * kKvHeads + x) * p.capacity * kHeadDim;
}

// The attention inputs of layer l at position pos that exist before the
// layer runs: cached keys / values of KV head x, QK norm weights, RoPE row.
template <int kPath, bool kLocal>
__device__ __forceinline__ void prefetch_attention(const DecodeParams& p, int l, int pos, AttnKV& kv) {
  const uint16_t* w = launder(p.weights);
  const size_t head = kv_head_offset(p, l, blk_xcd());
  attn_prefetch<kPath, kLocal>(launder(p.key_cache) + head, launder(p.value_cache) + head, pos, attn_tensor<A_QLN>(w, l),
                attn_tensor<A_KLN>(w, l), launder(p.rope) + (size_t)pos * 2 * kHeadDim, kv);
}

// Timing trace (built only with -DLFM25_TRACE, never in the library the
// package ships): wave 0, lane 0 of every block stamps s_memrealtime at fixed
// points of every step into a caller-provided buffer
// [blocks][steps * kTracePerStep].
constexpr int kTracePerLayer = 12;
[[maybe_unused]] constexpr int kTracePerStep = kLayers * kTracePerLayer + 4;
#ifdef LFM25_TRACE
__device__ uint64_t* g_trace = nullptr;
__device__ int g_trace_steps = 0;
#define LFM25_TRACE_AT(o, step, idx)                                                             \
  do {                                                                                           \
    if (wave_id() == 0 && lane_id() == 0 && (o).trace_block != nullptr && (step) < (o).trace_steps) \
      (o).trace_block[((size_t)blockIdx.x * (o).trace_steps + (step)) * kTracePerStep + (idx)] =    \
          __builtin_amdgcn_s_memrealtime();                                                      \
  } while (0)
#define LFM25_TRACE_SLOT(o, step, idx)                                   \
  do {                                                                   \
    if (threadIdx.x == 0) (o).trace_at = (step) * kTracePerStep + (idx); \
  } while (0)
#define LFM25_TRACE_INIT(o, on)                            \
  do {                                                     \
    if (threadIdx.x == 0) {                                \
      (o).trace_block = (on) ? g_trace : nullptr;          \
      (o).trace_steps = g_trace_steps;                     \
      (o).trace_waves = (on) ? g_trace_waves : nullptr;    \
      (o).trace_slots = g_trace_slots;                     \
      (o).trace_at = -1;                                   \
    }                                                      \
  } while (0)
#else
#define LFM25_TRACE_AT(o, step, idx) \
  do {                               \
  } while (0)
#define LFM25_TRACE_SLOT(o, step, idx) \
  do {                                 \
  } while (0)
#define LFM25_TRACE_INIT(o, on) \
  do {                          \
  } while (0)
#endif

// Per-token state of a block in the persistent decode.
struct TokenCtx {
  StepTags tags;
  const uint16_t* row;  // the token's embedding row (layer 0's input)
  float hres;           // wave 0: residual row 64jj + lane of the current layer
  uint32_t t_h;         // tag of the layer input in lh1 (layers > 0)
  int pos;
  int buf;              // last LDS vector buffer used
  int step;             // step index within the decode call (trace builds)
  const int8_t* row8 = nullptr;   // 8-bit weights: the token's int8 table row
  const float* row8_s = nullptr;  // and its 32 group scales
};

__device__ __forceinline__ uint32_t* next_vec(StepShared& sm, TokenCtx& c) {
  c.buf ^= 1;
  return sm.vec[c.buf];
}

// Where one layer's operands live, apart from its weights (in the slabs) and
// the exchange buffers.
struct LayerIO {
  char* ws;                 // the workspace (exchange buffers)
  const uint16_t* in_row;   // the layer input as a BF16 vector, or nullptr: the local h buffer (tag c.t_h)
  const uint16_t* norm_op;  // operator / FFN RMSNorm weights (global memory)
  const uint16_t* norm_ffn;
  uint16_t* conv_state;     // conv layer: the [1024 x 3] state the gated conv writes
  uint16_t* keys;           // attention layer: the cache rows of KV head x
  uint16_t* values;
  const int8_t* in_row8 = nullptr;  // 8-bit weights: layer 0's input as an int8 table row
  const float* in_row8_s = nullptr;
  const uint32_t* in_row_lds = nullptr;  // wave 0: in_row already requested into LDS
};

// Layer l (its kind and its tags) of one token on the group that computes
// it; the layer's weights are in S on entry.
template <bool kLocal, int kPath, typename SlabsT>
__device__ __forceinline__ void decode_layer(const LayerIO& io, StepShared& sm, TokenCtx& c, int l, const SlabsT& S,
                                             const AttnKV& kv) {
  constexpr bool kW8 = std::is_same_v<SlabsT, Slabs8>;
  const StepBufs b{io.ws};
  const int x = blk_xcd();
  const bool w0 = wave_id() == 0;
  const int tr = l * kTracePerLayer;
  (void)tr;
  LFM25_TRACE_AT(sm.out, c.step, tr + 0);
  // P1: normed h -> in_proj + conv (or q/k/v)
  uint32_t* v1 = next_vec(sm, c);
  const uint32_t g_op = norm_word(io.norm_op);
  if constexpr (kW8) gather_raw_split_w8<kLocal>(io.in_row8, io.in_row8_s, lh1_of(b, x), c.t_h, sm.in, b.status());
  else gather_raw_split<kLocal>(io.in_row, lh1_of(b, x), c.t_h, sm.in, b.status(), io.in_row_lds);
  if (w0) c.hres = residual_from_raw(sm.in.raw);
  norm_words_reg(sm.in, raw_scale(sm.in), g_op, v1);
  LFM25_TRACE_AT(sm.out, c.step, tr + 1);
  LFM25_TRACE_SLOT(sm.out, c.step, tr + 1);
  lds_barrier();
  uint32_t t_y;
  if (is_attn(l)) {
    const uint32_t t_qkv = c.tags.take();
    compute_qkv<kLocal>(S, v1, t_qkv, sm.out, b);
    LFM25_TRACE_AT(sm.out, c.step, tr + 2);
    const uint32_t t_st = c.tags.take();
    t_y = c.tags.take();
    run_attention<kLocal, kPath>(t_qkv, t_st, io.keys, io.values, c.pos, b, t_y, kv, sm.attn);
    LFM25_TRACE_AT(sm.out, c.step, tr + 3);
  } else {
    t_y = c.tags.take();
    compute_conv<kLocal>(S, v1, io.conv_state, t_y, sm.out, b);
    LFM25_TRACE_AT(sm.out, c.step, tr + 2);
    LFM25_TRACE_AT(sm.out, c.step, tr + 3);
  }
  // P2: y -> out_proj / o_proj partial sums
  uint32_t* v2 = next_vec(sm, c);
  if (is_attn(l) && !attn_single<kPath>(c.pos)) {
    gather_context<kLocal>(b, t_y, v2, sm.attn);
  } else {
    if (w0) gather_plain<1, kLocal>(ly_of(b, x), kLyWords, t_y, v2, b.status());
  }
  LFM25_TRACE_AT(sm.out, c.step, tr + 4);
  LFM25_TRACE_SLOT(sm.out, c.step, tr + 4);
  lds_barrier();
  const uint32_t t_p1 = c.tags.take();
  compute_proj(S, v2, t_p1, sm.out, gp_of(b, 0));
  LFM25_TRACE_AT(sm.out, c.step, tr + 5);
  // R1, then P3: normed h -> w1/w3 + SiLU gate
  const uint32_t t_h2 = c.tags.take();
  uint32_t* v3 = next_vec(sm, c);
  run_residual_split<kLocal>(gp_of(b, 0), t_p1, c.hres, lh0_of(b, x), t_h2, b.status(), sm.red_part);
  LFM25_TRACE_AT(sm.out, c.step, tr + 6);
  const uint32_t g_ffn = norm_word(io.norm_ffn);
  gather_raw_split<kLocal>(nullptr, lh0_of(b, x), t_h2, sm.in, b.status());
  norm_words_reg(sm.in, raw_scale(sm.in), g_ffn, v3);
  LFM25_TRACE_AT(sm.out, c.step, tr + 7);
  LFM25_TRACE_SLOT(sm.out, c.step, tr + 7);
  lds_barrier();
  const uint32_t t_g = c.tags.take();
  compute_up<kLocal>(S, v3, t_g, sm.out, b);
  LFM25_TRACE_AT(sm.out, c.step, tr + 8);
  // P4: g -> w2 partial sums
  uint32_t* v4 = next_vec(sm, c);
  LFM25_TRACE_SLOT(sm.out, c.step, tr + 9);
  gather_plain_split<3, kLocal>(lg_of(b, x), kXcdFfn, t_g, v4, b.status());
  LFM25_TRACE_AT(sm.out, c.step, tr + 9);
  const uint32_t t_p2 = c.tags.take();
  compute_down(S, v4, t_p2, sm.out, gp_of(b, 1));
  LFM25_TRACE_AT(sm.out, c.step, tr + 10);
  // R2
  c.t_h = c.tags.take();
  run_residual_split<kLocal>(gp_of(b, 1), t_p2, c.hres, lh1_of(b, x), c.t_h, b.status(), sm.red_part);
  LFM25_TRACE_AT(sm.out, c.step, tr + 11);
}

// One token through all layers (and the head when `select`), block-wide.
// Group g computes layers g, g + 2, ...; right after each it requests the
// weights of its next layer (l + 2, or the next token's first layers) into
// S, which stream in while the other group computes. Returns the selected
// token in wave 0 of group-0 blocks (or -1).
//
// Layer 0 needs only the token's embedding row, so nothing would keep group
// 0 from starting it while group 1 still reads the buffers of the previous
// token's last layer, which layer 0 rewrites. After a step without a head
// (whose pick orders this), `fence_tag` is the epoch of that layer's output
// and group 0 first waits for its XCD's copy to be complete: every block of
// the XCD has then passed every read of the layer, and, through the partial
// sums each of them needed, so has every block (y, jj) that shares a partial
// buffer slot with it.
// Stages the wave's first head unit in LDS (either table format).
template <bool kW8>
__device__ __forceinline__ void head_begin(const DecodeParams& p, StepShared& sm) {
  if constexpr (kW8) head_begin_lds_w8(as_global(p.w8_table), as_global(p.w8_table_s), p.vocab, sm.head_rows[wave_id()]);
  else head_begin_lds(as_global(p.embedding), p.vocab, sm.head_rows[wave_id()]);
}

template <bool kLocal, int kPath, bool kRowPick, typename SlabsT>
__device__ __forceinline__ int decode_token(const DecodeParams& p, int token, int pos, bool select, uint32_t base,
                                            bool fence, uint32_t fence_tag, int step, StepShared& sm,
                                            SlabsT& S, AttnKV& kv, int& row_slot) {
  constexpr bool kW8 = std::is_same_v<SlabsT, Slabs8>;
  const bool w0 = wave_id() == 0;
  const int g = blk_group();
  TokenCtx c{StepTags{base}, as_global(p.embedding) + (size_t)token * kHidden, 0.0f, 0u, pos, 0, step};
  if constexpr (kW8) {
    c.row8 = as_global(p.w8_table) + (size_t)token * kHidden;
    c.row8_s = as_global(p.w8_table_s) + (size_t)token * kW8RowScales;
  }
  if (fence && g == 0 && w0) {
    const StepBufs b{launder(p.bufs.ws)};
    wait_h<kLocal>(lh1_of(b, blk_xcd()), fence_tag, b.status());
  }
#pragma unroll 1
  for (int l = 0; l < kLayers; ++l) {
    if (layer_group(l) != g) {
      c.t_h = c.tags.skip(layer_exchanges(l));  // the other group's layer; its last tag is h's
      continue;
    }
    {
      // Every address of the layer derives from bases laundered here, so none
      // of it is computed ahead and kept live across the other layers.
      const size_t head = kv_head_offset(p, l, blk_xcd());
      const LayerIO io{launder(p.bufs.ws), l == 0 ? c.row : nullptr, norm_weight(p, 2 * l), norm_weight(p, 2 * l + 1),
                       launder(p.conv_state) + (size_t)conv_before(l) * kHidden * kConvTaps,
                       launder(p.key_cache) + head, launder(p.value_cache) + head,
                       l == 0 ? c.row8 : nullptr, l == 0 ? c.row8_s : nullptr,
                       l == 0 && row_slot >= 0 ? pick_rows(sm)[row_slot] : nullptr};
      decode_layer<kLocal, kPath>(io, sm, c, l, S, kv);
    }
    // The CU returns loads in order: wave 0's last poll of the layer must not
    // queue behind the next layer's weights.
    lds_barrier();
    if (l + 2 < kLayers && is_attn(l + 2)) prefetch_attention<kPath, kLocal>(p, l + 2, c.pos, kv);
    if (l + 2 < kLayers) {
      load_layer(S, p, l + 2);
      // Group 1's first head rows stream in behind its last layer's weights,
      // through the other group's layer.
      if (select && l + 3 == kLayers) head_begin<kW8>(p, sm);
    } else if (l + 2 == kLayers) {
      load_layer(S, p, 0);
      // Group 0 idles through the last layer: its first head rows arrive
      // meanwhile. Both groups stage them in LDS (registers held across the
      // layer loop would be taken from the layers' own).
      if (select) head_begin<kW8>(p, sm);
    } else if (!select) {
      load_layer(S, p, 1);
    }
  }
  if (!select) return -1;
  // The head on every block; group 0 then picks the token, group 1 requests
  // the next token's layer-1 weights.
  [[maybe_unused]] constexpr int th = kLayers * kTracePerLayer;
  const StepBufs b{launder(p.bufs.ws)};
  const uint32_t t_c = c.tags.take();
  const uint32_t t_w = c.tags.take();
  uint32_t* vh = next_vec(sm, c);
  const uint32_t g_final = norm_word(norm_weight(p, 2 * kLayers));
  gather_raw_split<kLocal>(nullptr, lh1_of(b, blk_xcd()), c.t_h, sm.in, b.status());
  norm_words_reg(sm.in, raw_scale(sm.in), g_final, vh);
  LFM25_TRACE_AT(sm.out, step, th + 0);
  lds_barrier();
  if constexpr (kW8) {
    HeadRows8 first;  // a wave's first head unit
    head_from_lds(sm.head_rows[wave_id()], first);
    run_head<kLocal>(vh, as_global(p.w8_table), as_global(p.w8_table_s), p.vocab, b, t_c, sm.red_v, sm.red_i, first);
  } else {
    const HeadRows none{};
    // Odd positions scan the streamed units backwards: each scan then starts
    // with the rows the previous token's scan read last, which its XCD's L2
    // may still hold (the staged units are copied with the non-temporal
    // policy, so they do not evict them; measured +1.4% tok/s together).
    run_head<kLocal>(vh, as_global(p.embedding), p.vocab, b, t_c, sm.red_v, sm.red_i, none, sm.head_rows[wave_id()],
                     kHeadStaged, (c.pos & 1) != 0);
  }
  LFM25_TRACE_AT(sm.out, step, th + 1);
  int win = -1;
  if (g == 1) {
    load_layer(S, p, 1);
  } else if (w0) {
    pick_xcd<kLocal>(b, t_c, t_w);
    LFM25_TRACE_AT(sm.out, step, th + 2);
    // (the row copies cost the split and combined kernels registers they do
    // not have; the short-context kernel holds most of a call's tokens)
    if constexpr (kW8 || !kRowPick) {
      win = pick_global(b, t_w);
      row_slot = -1;
    } else {
      win = pick_global(b, t_w, as_global(p.embedding), pick_rows(sm), &row_slot, p.vocab);
    }
    LFM25_TRACE_AT(sm.out, step, th + 3);
  }
  return win;
}

// ====================================================================== persistent

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_all_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The persistent decode's state between tokens (every block keeps its own
// copy; the token lives in wave 0 of group-0 blocks).
struct LoopState {
  int pos, token;
  int row_slot;    // wave 0 of group-0 blocks: the LDS slot of the selected token's row (pick_global), or -1
  int i;           // step of the call
  uint32_t epoch;
  bool fence;      // the previous step of this launch had no head
};

// Steps st.i .. steps - 1 of a call (kAttnOne: while the position is below
// kAttnSingleBelow).
template <bool kLocal, int kPath, bool kRowPick = kPath == kAttnOne, typename SlabsT>
__device__ __forceinline__ void token_loop(const DecodeParams& p, StepShared& sm, SlabsT& S, AttnKV& kv,
                                           LoopState& st, int steps, bool lead) {
  int pos = st.pos, token = st.token, row_slot = st.row_slot, i = st.i;
  uint32_t epoch = st.epoch;
  bool fence = st.fence;
  for (; i < steps; ++i) {
    if (kPath == kAttnOne && pos >= kAttnSingleBelow) break;
    // Nothing is in flight across the token boundary that a group would not
    // wait for anyway before its first poll, so the compiler's view of the
    // pending loads inside a token is exact.
    wait_all_loads();
    if (p.tokens_in != nullptr && i < p.n_in) {
      token = p.tokens_in[i];
      row_slot = -1;
    }
    const int chosen = token;
    token = clamp_token(token, p.vocab, p.ctl, lead);
    if (token != chosen) row_slot = -1;
    if (pos >= p.capacity) {
      if (lead) ctl_or(p.ctl + LFM25_CTL_STATUS, 2);
      break;
    }
    const bool select = p.n_gen > 0 && i >= p.n_in - 1;
    // After a step without a head the epoch advanced by exactly its layer
    // exchanges, so the previous step's last h carries the current base tag.
    const int w = decode_token<kLocal, kPath, kRowPick>(p, token, pos, select, epoch, fence, epoch & 0xffffu, i, sm, S, kv,
                                              row_slot);
    fence = !select;
    epoch += kExchangesNoHead + (select ? kExchangesHead : 0);
    if (select) {
      token = w;  // wave 0 of group-0 blocks carries the token; nothing else reads it
      const int o = i - (p.n_in - 1);
      if (lead && p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = token;
    }
    ++pos;
  }
  st = LoopState{pos, token, row_slot, i, epoch, fence};
}

// Compiled into one token loop, the single-block and the split attention
// need a few more registers than a lane has (the compiler spilled some,
// among them prefetched KV passes). kPath = kAttnAny therefore runs two
// sequential loops -- the positions below kAttnSingleBelow, then the rest --
// each keeping the registers of its own path, with no scratch; it serves
// calls of fewer than kSplitLaunchSteps steps in one launch. Longer calls run
// as two launches of the kernels compiled for one path each (kAttnOne while
// the position is below kAttnSingleBelow, then kAttnSplit resuming at the
// step count the first left in the control word; either returns at once when
// it has nothing to do): measured ~1% faster per token than the two-loop
// kernel, which is worth the second launch (~25 us) from 8 steps on.
constexpr int kSplitLaunchSteps = 8;
template <bool kLocal, int kPath, bool kW8 = false>
__global__ void __launch_bounds__(kStepThreads) k_decode_persistent(DecodeParams p) {
  __shared__ StepShared sm;
  p.ctl = as_global(p.ctl);
  p.tokens_in = as_global(p.tokens_in);
  p.tokens_out = as_global(p.tokens_out);
  p.embedding = as_global(p.embedding);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  // The local exchanges rely on block b running on XCD b % 8; a block that
  // finds itself elsewhere stops the run (every poll checks this flag).
  if (kLocal && threadIdx.x == 0 && hw_xcc_id() != blk_xcd())
    ctl_or(p.ctl + LFM25_CTL_STATUS, kStepStatusPlacement);
  int pos = ctl_load(p.ctl + LFM25_CTL_POSITION);
  const int steps = p.n_in + max(p.n_gen - 1, 0);
  const int first = kPath == kAttnSplit ? ctl_load(p.ctl + kCtlStep) : 0;
  if ((kPath == kAttnOne && pos >= kAttnSingleBelow) || first >= steps) {
    if (kPath == kAttnOne && lead) ctl_store(p.ctl + kCtlStep, 0);
    return;
  }
  int token = ctl_load(p.ctl + LFM25_CTL_TOKEN);
  uint32_t epoch = (uint32_t)ctl_load(p.ctl + kCtlEpoch);
  LFM25_TRACE_INIT(sm.out, true);
  LFM25_ATTN_INIT(sm.attn);
  std::conditional_t<kW8, Slabs8, Slabs> S;
  AttnKV kv;  // group 0: the next attention layer's prefetched inputs
  load_layer(S, p, blk_group());
  lds_barrier();
  LoopState st{pos, token, -1, first, epoch, false};
  if constexpr (kPath == kAttnAny) {
    // the positions below kAttnSingleBelow, then the rest: the two loops are
    // sequential, so each keeps the registers of its own attention path
    // (no row copies in the pick: calls this short gain nothing from them,
    // and the registers they take would spill)
    token_loop<kLocal, kAttnOne, false>(p, sm, S, kv, st, steps, lead);
    // Every attention layer prefetches its own inputs before it reads them;
    // clearing them here tells the compiler that nothing of the first loop's
    // prefetches is read by the second, which otherwise keeps them live
    // through the first loop and spills.
    kv = AttnKV{};
    token_loop<kLocal, kAttnSplit, false>(p, sm, S, kv, st, steps, lead);
  } else {
    token_loop<kLocal, kPath>(p, sm, S, kv, st, steps, lead);
  }
  pos = st.pos;
  token = st.token;
  epoch = st.epoch;
  const int i = st.i;
  if (lead) {
    ctl_store(p.ctl + LFM25_CTL_POSITION, pos);
    ctl_store(p.ctl + LFM25_CTL_TOKEN, token);
    ctl_store(p.ctl + kCtlEpoch, (int)(epoch & 0xffffu));
    ctl_store(p.ctl + kCtlStep, i);
  }
}

// ====================================================================== one layer

// One decoder layer as one launch of the decode's group 0 (blocks b < 128,
// block b taking the part of block b / 8 of XCD b % 8): the layer's weights are loaded
// into registers at the start (there is no previous layer to hide them
// behind), then the same phases and exchanges as inside the persistent
// decode. The input is a BF16 vector, the output the layer's last h,
// written by XCD 0's blocks.
struct LayerParams {
  LayerWeights w;
  const uint16_t* op_norm;
  const uint16_t* ffn_norm;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const uint16_t* rope_row;  // attention: cos | sin at `position`
  const uint16_t* in;
  uint16_t* out;
  uint16_t* conv_state_out;
  uint16_t* keys;            // attention: [8 x capacity x 64]
  uint16_t* values;
  char* ws;
  int capacity, position;
};

constexpr int kLayerGrid = kXcds * kGroupBlocks;  // group 0: blocks 0 .. 127
template <bool kLocal, int kPath>
__global__ void __launch_bounds__(kStepThreads) k_decode_layer(LayerParams p) {
  __shared__ StepShared sm;
  int32_t* ctl = reinterpret_cast<int32_t*>(as_global(p.ws) + kWsCtl);
  const int x = blk_xcd();
  // (the placement test is block-uniform; only its report is per thread, so
  // nothing derived from x is merged out of a divergent branch)
  const bool misplaced = kLocal && hw_xcc_id() != x;
  if (misplaced && threadIdx.x == 0) ctl_or(ctl + LFM25_CTL_STATUS, kStepStatusPlacement);
  const bool attn = p.w.attn;
  const int l = attn ? 2 : 0;  // a layer of this kind: its exchange count and trace slots
  const size_t head = (size_t)x * p.capacity * kHeadDim;
  LFM25_TRACE_INIT(sm.out, false);
  LFM25_ATTN_INIT(sm.attn);
  Slabs S;
  AttnKV kv;
  load_slabs(S, p.w);
  if (attn) attn_prefetch<kPath, kLocal>(p.keys + head, p.values + head, p.position, p.q_norm, p.k_norm, p.rope_row, kv);
  const uint32_t epoch = (uint32_t)ctl_load(ctl + kCtlEpoch);
  lds_barrier();
  TokenCtx c{StepTags{epoch}, as_global(p.in), 0.0f, 0u, p.position, 0, 0};
  const LayerIO io{launder(p.ws), c.row, p.op_norm, p.ffn_norm, p.conv_state_out, p.keys + head,
                   p.values + head};
  decode_layer<kLocal, kPath>(io, sm, c, l, S, kv);
  if (x == 0 && wave_id() == 0) p.out[kResRows * blk_jj() + lane_id()] = f32_to_bf16(c.hres);
  // Every block of the group read the epoch before its first exchange, and
  // block 0's last phase needed (through the partial sums) every block's
  // first one, so no block can still be about to read it.
  if (blockIdx.x == 0 && threadIdx.x == 0) ctl_store(ctl + kCtlEpoch, (int)((epoch + layer_exchanges(l)) & 0xffffu));
}

// Cooperative launch feasibility per device (0 unknown, -1 unsupported, 1 ok)
// and whether the placement block b -> XCD b % 8 holds there (checked once
// with a launch of the same shape as the decode).
__global__ void __launch_bounds__(kStepThreads) k_placement(int32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = hw_xcc_id();
}

struct DeviceInfo {
  int coop = 0;
  int local = 0;
};

// Resident blocks per CU of the persistent decode kernels (the smallest).
template <bool kLocal>
static bool occupancy(int* per_cu) {
  void (*const fns[6])(DecodeParams) = {
      k_decode_persistent<kLocal, kAttnAny>,       k_decode_persistent<kLocal, kAttnOne>,
      k_decode_persistent<kLocal, kAttnSplit>,     k_decode_persistent<kLocal, kAttnAny, true>,
      k_decode_persistent<kLocal, kAttnOne, true>, k_decode_persistent<kLocal, kAttnSplit, true>};
  void (*const layer_fns[2])(LayerParams) = {k_decode_layer<false, kAttnOne>, k_decode_layer<false, kAttnSplit>};
  *per_cu = 1 << 30;
  for (auto fn : fns) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kStepThreads, 0) != hipSuccess) return false;
    *per_cu = std::min(*per_cu, n);
  }
  for (auto fn : layer_fns) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kStepThreads, 0) != hipSuccess) return false;
    *per_cu = std::min(*per_cu, n);
  }
  return true;
}

static int device_info(DeviceInfo* info) {
  static std::mutex mu;
  static std::vector<DeviceInfo> per_device;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return LFM25_EDEVICE;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)per_device.size() <= dev) per_device.resize(dev + 1);
  DeviceInfo& d = per_device[dev];
  if (d.coop == 0) {
    int cus = 0, coop = 0, per_cu = 0, per_cu_c = 0;
    d.coop = -1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) == hipSuccess &&
        occupancy<true>(&per_cu) && occupancy<false>(&per_cu_c) &&
        coop && per_cu >= 1 && per_cu_c >= 1 && cus * per_cu >= kGrid && cus * per_cu_c >= kGrid)
      d.coop = 1;
    d.local = 0;
    if (d.coop == 1) {
      // One-time placement probe on a private stream.
      int32_t* buf = nullptr;
      hipStream_t s = nullptr;
      std::vector<int32_t> xcc(kGrid, -1);
      if (hipMalloc(&buf, kGrid * sizeof(int32_t)) == hipSuccess &&
          hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess) {
        void* args[] = {&buf};
        if (hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_placement), dim3(kGrid),
                                       dim3(kStepThreads), args, 0, s) == hipSuccess &&
            hipMemcpyAsync(xcc.data(), buf, kGrid * sizeof(int32_t), hipMemcpyDeviceToHost, s) ==
                hipSuccess &&
            hipStreamSynchronize(s) == hipSuccess) {
          bool ok = true;
          for (int i = 0; i < kGrid; ++i) ok = ok && xcc[i] == i % kXcds;
          d.local = ok ? 1 : 0;
        }
      }
      if (s != nullptr) (void)hipStreamDestroy(s);
      if (buf != nullptr) (void)hipFree(buf);
      (void)hipGetLastError();
    }
  }
  *info = d;
  return d.coop > 0 ? LFM25_OK : LFM25_EDEVICE;
}

// LFM25_XCD_LOCAL=0 in the environment forces the cross-XCD-coherent
// exchanges everywhere (same results, slower).
static bool local_allowed() {
  const char* e = getenv("LFM25_XCD_LOCAL");
  return e == nullptr || strcmp(e, "0") != 0;
}

static int run_persistent(DecodeParams p, hipStream_t s) {
  DeviceInfo info;
  if (device_info(&info) != LFM25_OK)
    return set_error(LFM25_EDEVICE, "decode: a cooperative launch of %d blocks of %d threads is "
                     "not possible on this device", kGrid, kStepThreads);
  const bool local = info.local == 1 && local_allowed();
  const bool w8 = p.w8 != nullptr;
  void* args[] = {&p};
  const bool two = p.n_in + std::max(p.n_gen - 1, 0) >= kSplitLaunchSteps;
  const void* fns[2];
  if (two && w8) {
    fns[0] = local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnOne, true>)
                   : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnOne, true>);
    fns[1] = local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnSplit, true>)
                   : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnSplit, true>);
  } else if (two) {
    fns[0] = local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnOne>)
                   : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnOne>);
    fns[1] = local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnSplit>)
                   : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnSplit>);
  } else {
    fns[0] = w8 ? (local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnAny, true>)
                         : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnAny, true>))
                : (local ? reinterpret_cast<const void*>(k_decode_persistent<true, kAttnAny>)
                         : reinterpret_cast<const void*>(k_decode_persistent<false, kAttnAny>));
  }
  for (int k = 0; k < (two ? 2 : 1); ++k) {
    const hipError_t e = hipLaunchCooperativeKernel(fns[k], dim3(kGrid), dim3(kStepThreads), args, 0, s);
    if (e != hipSuccess) return set_error(LFM25_EDEVICE, "decode (persistent): %s", hipGetErrorString(e));
  }
  return LFM25_OK;
}

static int run_layer(const LayerParams& p, hipStream_t s) {
  DeviceInfo info;
  if (device_info(&info) != LFM25_OK)
    return set_error(LFM25_EDEVICE, "decode_layer: a cooperative launch of %d blocks of %d threads is "
                     "not possible on this device", kGrid, kStepThreads);
  const bool one = !p.w.attn || p.position < kAttnSingleBelow;
  const void* fn = one ? reinterpret_cast<const void*>(k_decode_layer<false, kAttnOne>)
                       : reinterpret_cast<const void*>(k_decode_layer<false, kAttnSplit>);
  // Only group 0 (blocks 0..127, one per CU) computes, so the grid is those
  // 128 blocks, launched as an ordinary kernel: a cooperative launch costs
  // ~18 us more per call on MI355X. An ordinary launch may start while the
  // previous kernel's last blocks still occupy some XCDs, and then its blocks
  // do not land on XCD blockIdx % 8 (seen on MI355X), so the layer always
  // uses the cross-XCD-coherent exchanges. On an otherwise idle device the
  // 128 blocks are resident together; if other work kept some of them
  // waiting, the bounded polls end the call with status bit 2 instead of
  // hanging.
  LayerParams q = p;
  void* args[] = {&q};
  const hipError_t e = hipLaunchKernel(fn, dim3(kLayerGrid), dim3(kStepThreads), args, 0, s);
  if (e != hipSuccess) return set_error(LFM25_EDEVICE, "decode_layer: %s", hipGetErrorString(e));
  return LFM25_OK;
}

// ====================================================================== staged
//
// The same phases, one kernel each, on the same grid, with tags derived from
// the control words: every kernel reads the step's base epoch and gets its
// own and its inputs' offsets within the step from the host. Blocks of the
// group that does not compute a layer return at once. Every input a phase
// polls was written by an earlier kernel, so the cross-XCD-coherent exchange
// variant serves here (the results do not depend on it).

__global__ void k_decode_init(int32_t* ctl) { ctl[kCtlStep] = 0; }

__global__ void k_step_begin(DecodeParams p) {
  if (threadIdx.x != 0) return;
  const int i = p.ctl[kCtlStep];
  int t = (p.tokens_in != nullptr && i < p.n_in) ? p.tokens_in[i] : p.ctl[LFM25_CTL_TOKEN];
  t = clamp_token(t, p.vocab, p.ctl, true);
  p.ctl[LFM25_CTL_TOKEN] = t;
  if (p.ctl[LFM25_CTL_POSITION] >= p.capacity) p.ctl[LFM25_CTL_STATUS] |= 2;
}

struct StagedCtx {
  int pos;
  uint32_t base;
  const uint16_t* row;
  bool halted;
};

__device__ __forceinline__ StagedCtx staged_ctx(DecodeParams& p) {
  p.ctl = as_global(p.ctl);
  p.embedding = as_global(p.embedding);
  StagedCtx c;
  c.pos = p.ctl[LFM25_CTL_POSITION];
  c.base = (uint32_t)p.ctl[kCtlEpoch];
  c.row = p.embedding + (size_t)clamp_token(p.ctl[LFM25_CTL_TOKEN], p.vocab, p.ctl, false) * kHidden;
  c.halted = c.pos >= p.capacity;
  return c;
}

__device__ __forceinline__ uint32_t tag_at(uint32_t base, int off) {
  return (base + (uint32_t)off) & 0xffffu;
}

struct StagedLds {
  alignas(16) uint32_t vec[kNormWords];
  uint32_t gamma[kNormWords];
  Gathered in;
  StepOut out;
  AttnSplitShared attn;  // the attention context partials gathered by k_st_proj
};

// Wave 0 gathers the layer input (see gather_raw), then every wave norms its
// words into sh.vec.
__device__ __forceinline__ void staged_gather_norm(const uint16_t* row, const uint32_t* src, uint32_t tag,
                                                   StagedLds& sh, int32_t* status) {
  if (wave_id() == 0) gather_raw<false>(row, src, tag, sh.in, status);
  lds_barrier();
  norm_words(sh.in, sh.gamma, sh.vec);
  lds_barrier();
}

// P1 of layer l; off_in < 0: the input is the embedding row.
__global__ void __launch_bounds__(kStepThreads) k_st_first(DecodeParams p, int l, int off_in, int off_out) {
  __shared__ StagedLds sh;
  LFM25_TRACE_INIT(sh.out, false);
  if (blk_group() != layer_group(l)) return;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const bool attn = is_attn(l);
  load_norm_lds(sh.gamma, layer_tensor<C_OPNORM, A_OPNORM>(p.weights, l));
  Slabs s;
  load_slab_a(s, layer_weights(p.weights, p.conv_state, l));
  lds_barrier();
  staged_gather_norm(off_in < 0 ? c.row : nullptr, lh1_of(p.bufs, blk_xcd()), tag_at(c.base, off_in), sh,
                     p.bufs.status());
  if (attn) compute_qkv<false>(s, sh.vec, tag_at(c.base, off_out), sh.out, p.bufs);
  else compute_conv<false>(s, sh.vec, conv_state_of(p, conv_before(l)), tag_at(c.base, off_out), sh.out, p.bufs);
}

// Attention of KV head x on the blocks (x, jj) of group 0 (grid of the 128
// blocks of group 0; attention layers are even, so group 0 computes them),
// as two launches (kPart = kAttnHalfStats, then kAttnHalfContext) so that no block
// waits within a launch for another that may not be resident yet.
static_assert(layer_group(2) == 0 && layer_group(12) == 0, "attention layers belong to group 0");
constexpr int kAttnGrid = kXcds * kGroupBlocks;
template <int kPart>
__global__ void __launch_bounds__(kStepThreads)
    k_st_attention(DecodeParams p, int l, int off_qkv, int off_st, int off_out) {
  __shared__ AttnSplitShared sh;
  LFM25_ATTN_INIT(sh);
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const size_t head = kv_head_offset(p, l, blk_xcd());
  AttnKV kv;
  prefetch_attention<kAttnAny, false>(p, l, c.pos, kv);
  run_attention<false, kAttnAny, kPart>(tag_at(c.base, off_qkv), tag_at(c.base, off_st), p.key_cache + head,
                                        p.value_cache + head, c.pos, p.bufs, tag_at(c.base, off_out), kv, sh);
}

__global__ void __launch_bounds__(kStepThreads) k_st_proj(DecodeParams p, int l, int off_y, int off_out) {
  __shared__ StagedLds sh;
  LFM25_TRACE_INIT(sh.out, false);
  if (blk_group() != layer_group(l)) return;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  Slabs s;
  load_slab_b(s, layer_weights(p.weights, p.conv_state, l));
  if (is_attn(l) && !attn_single<kAttnAny>(c.pos)) {
    gather_context<false>(p.bufs, tag_at(c.base, off_y), sh.vec, sh.attn);
  } else {
    if (wave_id() == 0)
      gather_plain<1, false>(ly_of(p.bufs, blk_xcd()), kLyWords, tag_at(c.base, off_y), sh.vec, p.bufs.status());
    lds_barrier();
  }
  compute_proj(s, sh.vec, tag_at(c.base, off_out), sh.out, gp_of(p.bufs, 0));
}

// R phase of layer l: k = 0 adds the mixer's partials to the layer input
// (the embedding row when off_res < 0, else lh1) into lh0; k = 1 adds the
// FFN's partials to lh0 into lh1.
__global__ void __launch_bounds__(kWave) k_st_residual(DecodeParams p, int l, int k, int off_res, int off_gp,
                                                      int off_out) {
  if (blk_group() != layer_group(l)) return;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const int x = blk_xcd();
  const uint32_t* src = k == 0 ? lh1_of(p.bufs, x) : lh0_of(p.bufs, x);
  float hres = load_residual<false>(k == 0 && off_res < 0 ? c.row : nullptr, src,
                                    tag_at(c.base, off_res), p.bufs.status());
  run_residual<false>(gp_of(p.bufs, k), tag_at(c.base, off_gp), hres,
                      k == 0 ? lh0_of(p.bufs, x) : lh1_of(p.bufs, x), tag_at(c.base, off_out),
                      p.bufs.status());
}

__global__ void __launch_bounds__(kStepThreads) k_st_up(DecodeParams p, int l, int off_h, int off_out) {
  __shared__ StagedLds sh;
  LFM25_TRACE_INIT(sh.out, false);
  if (blk_group() != layer_group(l)) return;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  load_norm_lds(sh.gamma, layer_tensor<C_FFNNORM, A_FFNNORM>(p.weights, l));
  Slabs s;
  load_slab_c(s, layer_weights(p.weights, p.conv_state, l));
  lds_barrier();
  staged_gather_norm(nullptr, lh0_of(p.bufs, blk_xcd()), tag_at(c.base, off_h), sh, p.bufs.status());
  compute_up<false>(s, sh.vec, tag_at(c.base, off_out), sh.out, p.bufs);
}

__global__ void __launch_bounds__(kStepThreads) k_st_down(DecodeParams p, int l, int off_g, int off_out) {
  __shared__ StagedLds sh;
  LFM25_TRACE_INIT(sh.out, false);
  if (blk_group() != layer_group(l)) return;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  Slabs s;
  load_slab_d(s, layer_weights(p.weights, p.conv_state, l));
  if (wave_id() == 0)
    gather_plain<3, false>(lg_of(p.bufs, blk_xcd()), kXcdFfn, tag_at(c.base, off_g), sh.vec, p.bufs.status());
  lds_barrier();
  compute_down(s, sh.vec, tag_at(c.base, off_out), sh.out, gp_of(p.bufs, 1));
}

// The head on every block, as in the persistent kernel.
__global__ void __launch_bounds__(kStepThreads) k_st_head(DecodeParams p, int off_h, int off_out) {
  __shared__ StagedLds sh;
  LFM25_TRACE_INIT(sh.out, false);
  __shared__ float red_v[kStepWaves];
  __shared__ int red_i[kStepWaves];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  HeadRows first;
  head_begin(p.embedding, p.vocab, first);
  load_norm_lds(sh.gamma, final_norm(p.weights));
  lds_barrier();
  staged_gather_norm(nullptr, lh1_of(p.bufs, blk_xcd()), tag_at(c.base, off_h), sh, p.bufs.status());
  run_head<false>(sh.vec, p.embedding, p.vocab, p.bufs, tag_at(c.base, off_out), red_v, red_i, first);
}

// One wave: the first maximum over all 256 block candidates (the same winner
// as the two-level pick of the persistent kernel: the order on (value, row)
// is total, so any merge order gives the first maximum), then the control
// words of the next step.
__global__ void __launch_bounds__(kWave) k_step_end(DecodeParams p, int select, int off_cand, int stages) {
  p.ctl = as_global(p.ctl);
  const int i = p.ctl[kCtlStep];
  const bool halted = p.ctl[LFM25_CTL_POSITION] >= p.capacity;
  if (select && !halted) {
    const uint32_t tag = tag_at((uint32_t)p.ctl[kCtlEpoch], off_cand);
    const int l = lane_id();
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    Poll poll(p.bufs.status());
    while (true) {
      bool ok = true;
      bv = -INFINITY;
      bi = 0x7fffffff;
#pragma unroll
      for (int k = 0; k < kStepBlocks / kWave; ++k) {
        const int n = l + k * kWave;  // candidate of block n: lw[n % 8][n / 8]
        const uint64_t w = coherent_load64(lw_of(p.bufs, n % kXcds) + n / kXcds);
        ok = ok && candidate_ok(w, tag);
        float v;
        int row;
        candidate_of(w, v, row);
        if (better(v, row, bv, bi)) { bv = v; bi = row; }
      }
      if (__all(ok) || !poll.again()) break;
    }
    wave_pick(bv, bi);
    if (l == 0) {
      p.ctl[LFM25_CTL_TOKEN] = bi;
      const int o = i - (p.n_in - 1);
      if (p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = bi;
    }
  }
  if (threadIdx.x == 0 && !halted) {
    p.ctl[LFM25_CTL_POSITION] += 1;
    p.ctl[kCtlEpoch] = (int)(((uint32_t)p.ctl[kCtlEpoch] + (uint32_t)stages) & 0xffffu);
  }
  if (threadIdx.x == 0) p.ctl[kCtlStep] = i + 1;
}

static int run_staged(const DecodeParams& p, hipStream_t s) {
  const int steps = p.n_in + max(p.n_gen - 1, 0);
  k_decode_init<<<1, 1, 0, s>>>(p.ctl);
  for (int i = 0; i < steps; ++i) {
    const bool select = p.n_gen > 0 && i >= p.n_in - 1;
    k_step_begin<<<1, 64, 0, s>>>(p);
    int off = 0, off_in = -1;
    for (int l = 0; l < kLayers; ++l) {
      int off_y;
      if (is_attn(l)) {
        const int off_qkv = ++off;
        k_st_first<<<kGrid, kStepThreads, 0, s>>>(p, l, off_in, off_qkv);
        const int off_st = ++off;
        off_y = ++off;
        k_st_attention<kAttnHalfStats><<<kAttnGrid, kStepThreads, 0, s>>>(p, l, off_qkv, off_st, off_y);
        k_st_attention<kAttnHalfContext><<<kAttnGrid, kStepThreads, 0, s>>>(p, l, off_qkv, off_st, off_y);
      } else {
        off_y = ++off;
        k_st_first<<<kGrid, kStepThreads, 0, s>>>(p, l, off_in, off_y);
      }
      const int off_p1 = ++off;
      k_st_proj<<<kGrid, kStepThreads, 0, s>>>(p, l, off_y, off_p1);
      const int off_h2 = ++off;
      k_st_residual<<<kGrid, kWave, 0, s>>>(p, l, 0, off_in, off_p1, off_h2);
      const int off_g = ++off;
      k_st_up<<<kGrid, kStepThreads, 0, s>>>(p, l, off_h2, off_g);
      const int off_p2 = ++off;
      k_st_down<<<kGrid, kStepThreads, 0, s>>>(p, l, off_g, off_p2);
      const int off_h = ++off;
      k_st_residual<<<kGrid, kWave, 0, s>>>(p, l, 1, off_h2, off_p2, off_h);
      off_in = off_h;
    }
    int off_cand = 0;
    if (select) {
      off_cand = ++off;
      k_st_head<<<kGrid, kStepThreads, 0, s>>>(p, off_in, off_cand);
      ++off;  // the tag of the XCD-winner exchange of the persistent kernel
    }
    k_step_end<<<1, kWave, 0, s>>>(p, select ? 1 : 0, off_cand, off);
    const int rc = check_launch("decode (staged)");
    if (rc != LFM25_OK) return rc;
  }
  return LFM25_OK;
}

__global__ void k_decoder_reset(uint16_t* conv_state, uint32_t* workspace_words) {
  constexpr int n = LFM25_CONV_LAYERS * kHidden * kConvTaps;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    conv_state[i] = 0;
  constexpr int words = (int)(kWsBytes / 4);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x)
    workspace_words[i] = 0;
}

// ====================================================================== B sequences

// Timing trace of the batched kernel (trace builds only, -DLFM25_TRACE): the
// batch-1 trace's slots, stamped by wave 0 lane 0 of every block. The trace
// buffer and its step count are copied to the block's LDS at launch, so a
// stamp waits on nothing but LDS (a read of the globals would wait for every
// store the wave has in flight, and move their latency into the stamp).
#ifdef LFM25_TRACE
#define LFM25_BTRACE(step, idx)                                                                    \
  do {                                                                                             \
    if (wave_id() == 0 && lane_id() == 0 && sm.trace != nullptr && (step) < sm.trace_steps)        \
      sm.trace[((size_t)blockIdx.x * sm.trace_steps + (step)) * kTracePerStep + (idx)] =           \
          __builtin_amdgcn_s_memrealtime();                                                        \
  } while (0)
#else
#define LFM25_BTRACE(step, idx) \
  do {                          \
  } while (0)
#endif

// RMSNorm weights n = 0 .. 2 kLayers of a weight stream (norm_weight's order).
__device__ __forceinline__ const uint16_t* bnorm_weight(const uint16_t* w, int n) {
  if (n == 2 * kLayers) return final_norm(w);
  const int l = n / 2;
  return (n & 1) ? layer_tensor<C_FFNNORM, A_FFNNORM>(w, l) : layer_tensor<C_OPNORM, A_OPNORM>(w, l);
}

// Position at step `step` of sequence s (s block-uniform; no dynamic index
// into the parameter array).
template <int kB>
__device__ __forceinline__ int bpos(const BDecodeParams& p, int s, int step) {
  int pos = p.pos0[0];
#pragma unroll
  for (int q = 1; q < kB; ++q)
    if (q == s) pos = p.pos0[q];
  return pos + step;
}

// Rows of KV head x of attention layer l of sequence s in the batch caches
// ([kB][6][8][capacity][64]).
__device__ __forceinline__ size_t bkv_offset(const BDecodeParams& p, int s, int l, int x) {
  return (((size_t)s * LFM25_ATTN_LAYERS + (size_t)(l - conv_before(l))) * kKvHeads + x) * p.capacity * kHeadDim;
}

template <int kB>
__device__ __forceinline__ void bload_layer(BSlabs& S, const BDecodeParams& p, int l) {
  bload_slabs<kB>(S, layer_weights(launder(p.weights), launder(p.conv_state), l));
}

template <int kB, int kPath, bool kLocal>
__device__ __forceinline__ void bprefetch_attention(const BDecodeParams& p, int l, int step, BShared<kB>& sm,
                                                    BAttnPre& pre) {
  const uint16_t* w = launder(p.weights);
  const int s = bseq<kB>();
  const int pos = bpos<kB>(p, s, step);
  const size_t head = bkv_offset(p, s, l, blk_xcd());
  battn_prefetch<kB, kPath, kLocal>(launder(p.key_cache) + head, launder(p.value_cache) + head, pos,
                                    attn_tensor<A_QLN>(w, l), attn_tensor<A_KLN>(w, l),
                                    launder(p.rope) + (size_t)pos * 2 * kHeadDim, sm, pre);
}

// Layer l of every sequence on the group that computes it (decode_layer's
// phases and exchanges, each for kB rows); the layer's weights are in S.
template <int kB, bool kLocal, int kPath>
__device__ __forceinline__ void bdecode_layer(const BDecodeParams& p, int step, BShared<kB>& sm, BTags& tags,
                                              uint32_t& t_h, int l, const BSlabs& S, const BAttnPre& pre, int& buf,
                                              bool rows) {
  const BBufs<kB> b{launder(p.ws)};
  int32_t* status = as_global(p.status);
  const int x = blk_xcd();
  // P1: normed h -> in_proj + conv (or q/k/v)
  buf = bnext_buf<kB>(buf);
  BVec* v1 = sm.vec[buf];
  const int tr = l * kTracePerLayer;
  (void)tr;
  LFM25_BTRACE(step, tr + 0);
  const uint32_t g_op = norm_word(bnorm_weight(launder(p.weights), 2 * l));
  BConvTaps T;
  if (!is_attn(l)) bload_conv_taps<kB>(T, layer_weights(launder(p.weights), launder(p.conv_state), l));
  if (l == 0) {
    bgather_rows<kB>(as_global(p.embedding), sm, rows);
    bnorm<kB>(sm, g_op, v1, true);
  } else {
    bgather_norm<kB, kLocal>(b.lh1(x), b.lss(1, x), t_h, sm, g_op, v1, true, nullptr, status);
  }
  LFM25_BTRACE(step, tr + 1);
  // Past layer 0 no block barrier: wave k's products read words [64k, 64k +
  // 64) of every vector, the words it normed itself. Layer 0's norm reads
  // sm.raw, which shares its LDS with the partial tiles the products write.
  if (l == 0) lds_barrier();
  uint32_t t_y;
  if (is_attn(l)) {
    const uint32_t t_qkv = tags.take();
    bcompute_qkv<kB, kLocal>(S, sm, v1, t_qkv, b.lq(x));
    LFM25_BTRACE(step, tr + 2);
    const uint32_t t_st = tags.take();
    t_y = tags.take();
    const int s = bseq<kB>();
    const size_t head = bkv_offset(p, s, l, x);
    brun_attention<kB, kLocal, kPath>(b, status, t_qkv, t_st, t_y, launder(p.key_cache) + head,
                                      launder(p.value_cache) + head, bpos<kB>(p, s, step), sm, pre);
    LFM25_BTRACE(step, tr + 3);
  } else {
    t_y = tags.take();
    bcompute_conv<kB, kLocal>(S, T, sm, v1, launder(p.conv_state) + (size_t)conv_before(l) * kHidden * kConvTaps, t_y,
                              b.ly(x));
    LFM25_BTRACE(step, tr + 2);
    LFM25_BTRACE(step, tr + 3);
  }
  // P2: y -> out_proj / o_proj partial sums
  buf = bnext_buf<kB>(buf);
  BVec* v2 = sm.vec[buf];
  if (is_attn(l) && kPath == kAttnSplit) bgather_context<kB, kLocal>(b, status, t_y, v2, sm.attn);
  else bgather_plain<kB, 1, kLocal>(b.ly(x), kLyWords, kLyWords, t_y, v2, status);
  LFM25_BTRACE(step, tr + 4);
  const uint32_t t_p1 = tags.take();
  bcompute_proj<kB>(S, sm, v2, t_p1, b.gp(0));
  LFM25_BTRACE(step, tr + 5);
  // R1, then P3: normed h -> w1/w3 + SiLU gate
  const uint32_t t_h2 = tags.take();
  bresidual<kB, kLocal>(sm, b.gp(0), t_p1, b.lh0(x), b.lss(0, x), t_h2, status);
  LFM25_BTRACE(step, tr + 6);
  buf = bnext_buf<kB>(buf);
  BVec* v3 = sm.vec[buf];
  const uint32_t g_ffn = norm_word(bnorm_weight(launder(p.weights), 2 * l + 1));
  bgather_norm<kB, kLocal>(b.lh0(x), b.lss(0, x), t_h2, sm, g_ffn, v3, false, nullptr, status);
  LFM25_BTRACE(step, tr + 7);
  const uint32_t t_g = tags.take();  // (P3 reads only the wave's own words, as P1)
  bcompute_up<kB, kLocal>(S, sm, v3, t_g, b.lg(x));
  LFM25_BTRACE(step, tr + 8);
  // P4: g -> w2 partial sums, then R2
  buf = bnext_buf<kB>(buf);
  BVec* v4 = sm.vec[buf];
  bgather_plain<kB, 3, kLocal>(b.lg(x), kLgWords, kXcdFfn, t_g, v4, status);
  LFM25_BTRACE(step, tr + 9);
  const uint32_t t_p2 = tags.take();
  bcompute_down<kB>(S, sm, v4, t_p2, b.gp(1));
  LFM25_BTRACE(step, tr + 10);
  t_h = tags.take();
  bresidual<kB, kLocal>(sm, b.gp(1), t_p2, b.lh1(x), b.lss(1, x), t_h, status);
  LFM25_BTRACE(step, tr + 11);
}

// One step of every sequence (decode_token's layer loop and head); the
// tokens of the step are in sm.tok of group-0 blocks on entry, and the
// selected ones there on return. `rows`: on entry, whether the step's
// embedding rows were requested into sm.raw by the previous step's pick; on
// return, whether this step's pick requested the next ones.
template <int kB, bool kLocal, int kPath>
__device__ __forceinline__ void bdecode_token(const BDecodeParams& p, int step, uint32_t base, BShared<kB>& sm,
                                              BSlabs& S, BAttnPre& pre, bool& rows) {
  const int g = blk_group();
  BTags tags{base};
  uint32_t t_h = 0;
  int buf = 0;
#pragma unroll 1
  for (int l = 0; l < kLayers; ++l) {
    if (layer_group(l) != g) {
      tags.skip(layer_exchanges(l));
      t_h = tags.last();
      continue;
    }
    bdecode_layer<kB, kLocal, kPath>(p, step, sm, tags, t_h, l, S, pre, buf, rows);
    lds_barrier();
    if (l + 2 < kLayers && is_attn(l + 2)) bprefetch_attention<kB, kPath, kLocal>(p, l + 2, step, sm, pre);
    if (l + 2 < kLayers) bload_layer<kB>(S, p, l + 2);
    else if (l + 2 == kLayers) bload_layer<kB>(S, p, 0);
    // the head's first chunk of each wave, behind the group's last weights
    if (l + 2 == kLayers - 1 || l + 2 == kLayers) bhead_stage<kB>(as_global(p.embedding), p.vocab, sm);
  }
  // The head on every block; group 0 then picks the tokens, group 1
  // requests the next step's layer-1 weights.
  const BBufs<kB> b{launder(p.ws)};
  int32_t* status = as_global(p.status);
  const uint32_t t_c = tags.take();
  const uint32_t t_w = tags.take();
  buf = bnext_buf<kB>(buf);
  BVec* vh = sm.vec[buf];
  const uint32_t g_final = norm_word(bnorm_weight(launder(p.weights), 2 * kLayers));
  // block 0 also writes every sequence's pre-final-norm state (BF16 pairs)
  uint32_t* raw = p.hidden_out != nullptr && blockIdx.x == 0
                      ? reinterpret_cast<uint32_t*>(as_global(p.hidden_out)) + (size_t)step * kB * kNormWords
                      : nullptr;
  bgather_norm<kB, kLocal>(b.lh1(blk_xcd()), b.lss(1, blk_xcd()), t_h, sm, g_final, vh, false, raw, status);
  [[maybe_unused]] constexpr int th = kLayers * kTracePerLayer;
  LFM25_BTRACE(step, th + 0);
  lds_barrier();
  brun_head<kB, kLocal>(sm, vh, as_global(p.embedding), p.vocab, b, t_c);
  LFM25_BTRACE(step, th + 1);
  if (g == 1) {
    bload_layer<kB>(S, p, 1);
  } else if (wave_id() < kB) {
    // one wave per sequence (B = 16: wave w takes w and w + 8); block 0 also
    // records the step's tokens
#pragma unroll 1
    for (int s = wave_id(); s < kB; s += kStepWaves) bpick_xcd<kB, kLocal>(b, status, t_c, t_w, s);
    LFM25_BTRACE(step, th + 2);
#pragma unroll 1
    for (int s = wave_id(); s < kB; s += kStepWaves)
      bpick_global<kB>(b, status, t_w, sm, blockIdx.x == 0 ? as_global(p.tokens_out) + (size_t)step * kB : nullptr,
                       as_global(p.embedding), p.vocab, s);
    rows = true;
    LFM25_BTRACE(step, th + 3);
  }
}

// Steps st .. n_steps - 1 of a batched call, every sequence advancing one
// token per step (kAttnOne: while every position is below 256; kAttnSplit
// resumes at the step the first launch left in the control word).
template <int kB, bool kLocal, int kPath>
__global__ void __launch_bounds__(kStepThreads) k_bdecode(BDecodeParams p) {
  __shared__ BShared<kB> sm;
  LFM25_ATTN_INIT(sm.attn);
#ifdef LFM25_TRACE
  if (threadIdx.x == 0) {
    sm.trace = g_trace;
    sm.trace_steps = g_trace_steps;
  }
#endif
  int32_t* status = as_global(p.status);
  int32_t* ctl = reinterpret_cast<int32_t*>(as_global(p.ws) + BWs<kB>::ctl);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  if (kLocal && threadIdx.x == 0 && hw_xcc_id() != blk_xcd()) ctl_or(status, kStepStatusPlacement);
  const int first = kPath == kAttnSplit ? ctl_load(ctl + kBCtlStep) : 0;
  int maxpos0 = p.pos0[0];
#pragma unroll
  for (int q = 1; q < kB; ++q) maxpos0 = max(maxpos0, p.pos0[q]);
  if ((kPath == kAttnOne && maxpos0 >= kAttnSingleBelow) || first >= p.n_steps) {
    if (kPath == kAttnOne && lead) ctl_store(ctl + kBCtlStep, 0);
    return;
  }
  uint32_t epoch = (uint32_t)ctl_load(ctl + kBCtlEpoch);
  // the step's tokens: the call's inputs, or the selections of the step
  // before (written by the launch that ran it)
  if (threadIdx.x < kB) {
    int t = first == 0 ? p.tokens_in[threadIdx.x] : p.tokens_out[(size_t)(first - 1) * kB + threadIdx.x];
    if (t < 0 || t >= p.vocab) {
      if (blockIdx.x == 0) ctl_or(status, 1);
      t = t < 0 ? 0 : p.vocab - 1;
    }
    sm.tok[threadIdx.x] = t;
  }
  BSlabs S;
  BAttnPre pre;
  bool rows = false;  // the first step's embedding rows are loaded by its gather
  bload_layer<kB>(S, p, blk_group());
  lds_barrier();
  int i = first;
  for (; i < p.n_steps; ++i) {
    if (kPath == kAttnOne && maxpos0 + i >= kAttnSingleBelow) break;
    if (maxpos0 + i >= p.capacity) {
      if (lead) ctl_or(status, 2);
      break;
    }
    wait_all_loads();
    lds_barrier();  // the step's tokens in sm.tok are visible to every wave
    bdecode_token<kB, kLocal, kPath>(p, i, epoch, sm, S, pre, rows);
    epoch = (epoch + kExchangesNoHead + kExchangesHead) % 0xffffu;
  }
  wait_all_loads();  // the last pick's row copies land before the block's LDS is released
  if (lead) {
    ctl_store(ctl + kBCtlEpoch, (int)epoch);
    ctl_store(ctl + kBCtlStep, i);
  }
}

static bool batch_persistent_allowed() {
  const char* e = getenv("LFM25_BATCH_PERSISTENT");
  return e == nullptr || strcmp(e, "0") != 0;
}

__global__ void k_bdecode_status_clear(int32_t* status) {
  if (threadIdx.x == 0) *status = 0;
}

template <int kB>
static int run_bdecode(const lfm25_batch* b, void* region, int32_t* status, const int32_t* tokens_in,
                       const int32_t* positions, int n_steps, int32_t* tokens_out, uint16_t* hidden_out,
                       hipStream_t s, bool local) {
  BDecodeParams p{};
  p.weights = b->weights;
  p.embedding = b->embedding;
  p.rope = b->rope;
  p.conv_state = b->conv_state;
  p.key_cache = b->key_cache;
  p.value_cache = b->value_cache;
  p.ws = static_cast<char*>(region);
  p.status = status;
  p.tokens_in = tokens_in;
  p.tokens_out = tokens_out;
  p.hidden_out = hidden_out;
  for (int q = 0; q < kB; ++q) p.pos0[q] = positions[q];
  p.n_steps = n_steps;
  p.capacity = b->capacity;
  p.vocab = b->vocab;
  k_bdecode_status_clear<<<1, kWave, 0, s>>>(status);
  int rc = check_launch("batch decode (persistent)");
  if (rc != LFM25_OK) return rc;
  // B = 16 runs below 256 positions only (the single-block attention)
  constexpr int kPaths = kB == 16 ? 1 : 2;
  const void* fns[2] = {local ? reinterpret_cast<const void*>(k_bdecode<kB, true, kAttnOne>)
                              : reinterpret_cast<const void*>(k_bdecode<kB, false, kAttnOne>),
                        nullptr};
  if constexpr (kPaths == 2)
    fns[1] = local ? reinterpret_cast<const void*>(k_bdecode<kB, true, kAttnSplit>)
                   : reinterpret_cast<const void*>(k_bdecode<kB, false, kAttnSplit>);
  void* args[] = {&p};
  for (int k = 0; k < kPaths; ++k) {
    const hipError_t e = hipLaunchCooperativeKernel(fns[k], dim3(kGrid), dim3(kStepThreads), args, 0, s);
    if (e != hipSuccess) return set_error(LFM25_EDEVICE, "batch decode (persistent): %s", hipGetErrorString(e));
  }
  return LFM25_OK;
}

size_t batch_persistent_bytes() { return kBWsBytes; }

int batch_decode_persistent(const lfm25_batch* b, void* region, int32_t* status, const int32_t* tokens_in,
                            const int32_t* positions, int32_t n_steps, int32_t* tokens_out, uint16_t* hidden_out,
                            hipStream_t s, bool prefix, int32_t* done) {
  const int B = b->sequences;
  *done = 0;
  if ((B != 2 && B != 4 && B != 8 && B != 16) || !batch_persistent_allowed()) return kBatchNotPersistent;
  int maxpos = 0;
  for (int q = 0; q < B; ++q) maxpos = std::max(maxpos, positions[q]);
  // every sequence's cache must fit the split path's passes (256 positions
  // per block of a sequence) unless the whole call stays below 256; B = 16
  // has no split path: with `prefix` it takes the steps below 256
  int steps = n_steps;
  if (B == 16) {
    if (maxpos + n_steps > kAttnSingleBelow) steps = prefix ? kAttnSingleBelow - maxpos : 0;
  } else {
    const int cap = kAttnLocal * (kGroupBlocks / B);
    if (maxpos + n_steps > kAttnSingleBelow && maxpos + n_steps > cap) steps = 0;
  }
  if (steps <= 0) return kBatchNotPersistent;
  DeviceInfo info;
  if (device_info(&info) != LFM25_OK) return kBatchNotPersistent;
  const bool local = info.local == 1 && local_allowed();
  int rc;
  switch (B) {
    case 2: rc = run_bdecode<2>(b, region, status, tokens_in, positions, steps, tokens_out, hidden_out, s, local); break;
    case 4: rc = run_bdecode<4>(b, region, status, tokens_in, positions, steps, tokens_out, hidden_out, s, local); break;
    case 8: rc = run_bdecode<8>(b, region, status, tokens_in, positions, steps, tokens_out, hidden_out, s, local); break;
    default: rc = run_bdecode<16>(b, region, status, tokens_in, positions, steps, tokens_out, hidden_out, s, local); break;
  }
  if (rc == LFM25_OK) *done = steps;
  return rc;
}

}  // namespace lfm25

using namespace lfm25;

extern "C" {

size_t lfm25_weights_elems(void) { return (size_t)kStreamElems; }

int32_t lfm25_weights_offsets(int64_t* offsets, int32_t n) {
  int k = 0;
  for (int l = 0; l <= kLayers; ++l)
    for (int t = 0; t < tensor_count(l); ++t, ++k)
      if (offsets != nullptr && k < n) offsets[k] = tensor_off(l, t);
  return k;
}


size_t lfm25_decoder_workspace_bytes(void) { return kWsBytes; }

#ifdef LFM25_TRACE
// Trace builds only: where the persistent decode stamps its timing trace
// (nullptr: off) and for how many steps.
int lfm25_trace_set(uint64_t* buf, int32_t steps) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_trace_steps), &steps, sizeof(steps)) != hipSuccess)
    return LFM25_EDEVICE;
  return LFM25_OK;
}
int32_t lfm25_trace_per_step(void) { return kTracePerStep; }
#ifdef LFM25_TRACE_ATTN
// Attention stamps of block 0: buf [calls][16].
int lfm25_trace_attn_set(uint64_t* buf, int32_t calls) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_attn_trace), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_attn_calls), &calls, sizeof(calls)) != hipSuccess)
    return LFM25_EDEVICE;
  return LFM25_OK;
}
#endif
// Per-wave stamps: buf [blocks][slots][8 waves][2], slots = steps * per_step.
int lfm25_trace_waves_set(uint64_t* buf, int32_t slots) {
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace_waves), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_trace_slots), &slots, sizeof(slots)) != hipSuccess)
    return LFM25_EDEVICE;
  return LFM25_OK;
}
#endif

int32_t lfm25_decode_exchange(void) {
  DeviceInfo info;
  if (device_info(&info) != LFM25_OK) return -1;
  return info.local == 1 && local_allowed() ? 1 : 0;
}

int lfm25_init(void) {
  DeviceInfo info;
  if (device_info(&info) != LFM25_OK)
    return set_error(LFM25_EDEVICE, "init: a cooperative launch of %d blocks of %d threads is not possible "
                     "on this device", kGrid, kStepThreads);
  return LFM25_OK;
}

static int check_decoder(const lfm25_decoder* d) {
  LFM25_REQUIRE(d != nullptr, "decoder: null descriptor");
  LFM25_REQUIRE(d->weights && d->embedding && d->rope && d->conv_state && d->key_cache &&
                    d->value_cache && d->workspace,
                "decoder: null buffer in descriptor");
  LFM25_REQUIRE(d->capacity >= 1 && d->capacity <= kMaxCapacity,
                "decoder: capacity must be in [1, %d], got %d", kMaxCapacity, d->capacity);
  LFM25_REQUIRE(d->vocab >= kStepHeadRows && d->vocab % kStepHeadRows == 0 && d->vocab <= 65536,
                "decoder: vocab must be a multiple of %d in [%d, 65536], got %d", kStepHeadRows,
                kStepHeadRows, d->vocab);
  // A cached KV row (64 BF16) is one 128-byte line when the caches are
  // 128-byte aligned, so no reader ever holds a line into which a later
  // append lands (a block reads only rows below the current position).
  LFM25_REQUIRE(aligned16(d->weights) && aligned16(d->embedding) &&
                    (reinterpret_cast<uintptr_t>(d->key_cache) & 127u) == 0 &&
                    (reinterpret_cast<uintptr_t>(d->value_cache) & 127u) == 0 &&
                    (reinterpret_cast<uintptr_t>(d->workspace) & 255u) == 0,
                "decoder: buffers must be 16-byte aligned (KV caches 128-byte, workspace 256-byte)");
  return LFM25_OK;
}

int lfm25_decoder_reset(const lfm25_decoder* d, lfm25_stream_t stream) {
  const int rc = check_decoder(d);
  if (rc != LFM25_OK) return rc;
  k_decoder_reset<<<24, 256, 0, stream>>>(d->conv_state, static_cast<uint32_t*>(d->workspace));
  return check_launch("decoder_reset");
}

int lfm25_decode_layer(const lfm25_layer* L, const uint16_t* hidden_in, uint16_t* hidden_out, int32_t position,
                       void* workspace, lfm25_stream_t stream) {
  LFM25_REQUIRE(L != nullptr && hidden_in && hidden_out && workspace, "decode_layer: null argument");
  LFM25_REQUIRE(L->kind == LFM25_LAYER_CONV || L->kind == LFM25_LAYER_ATTN, "decode_layer: unknown kind %d",
                L->kind);
  const bool attn = L->kind == LFM25_LAYER_ATTN;
  LFM25_REQUIRE(L->op_norm && L->mixer && L->out && L->ffn_norm && L->w1 && L->w3 && L->w2,
                "decode_layer: null weight pointer");
  LFM25_REQUIRE(aligned16(L->mixer) && aligned16(L->out) && aligned16(L->w1) && aligned16(L->w3) &&
                    aligned16(L->w2) && aligned16(hidden_in) &&
                    (reinterpret_cast<uintptr_t>(L->op_norm) & 3u) == 0 &&
                    (reinterpret_cast<uintptr_t>(L->ffn_norm) & 3u) == 0 &&
                    (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
                "decode_layer: matrices and hidden_in must be 16-byte aligned, norms 4-byte, workspace 256-byte");
  if (attn) {
    LFM25_REQUIRE(L->q_norm && L->k_norm && L->key_cache && L->value_cache && L->rope,
                  "decode_layer: attention needs q_norm, k_norm, the caches and the rope table");
    LFM25_REQUIRE(L->capacity >= 1 && L->capacity <= kMaxCapacity, "decode_layer: capacity must be in [1, %d]",
                  kMaxCapacity);
    LFM25_REQUIRE(position >= 0 && position < L->capacity, "decode_layer: position %d outside the capacity %d",
                  position, L->capacity);
    LFM25_REQUIRE((reinterpret_cast<uintptr_t>(L->key_cache) & 127u) == 0 &&
                      (reinterpret_cast<uintptr_t>(L->value_cache) & 127u) == 0,
                  "decode_layer: KV caches must be 128-byte aligned");
  } else {
    LFM25_REQUIRE(L->conv_weight && L->conv_state_in && L->conv_state_out, "decode_layer: conv needs its weight "
                  "and state");
  }
  LayerParams p{};
  p.w.attn = attn;
  p.w.wa = L->mixer;
  p.w.conv_w = attn ? L->mixer : L->conv_weight;  // unread by attention (empty descriptors)
  p.w.state = attn ? L->mixer : L->conv_state_in;
  p.w.wb = L->out;
  p.w.w1 = L->w1;
  p.w.w3 = L->w3;
  p.w.w2 = L->w2;
  p.op_norm = L->op_norm;
  p.ffn_norm = L->ffn_norm;
  p.q_norm = attn ? L->q_norm : L->op_norm;
  p.k_norm = attn ? L->k_norm : L->op_norm;
  p.rope_row = attn ? L->rope + (size_t)position * 2 * kHeadDim : L->op_norm;
  p.in = hidden_in;
  p.out = hidden_out;
  p.conv_state_out = attn ? nullptr : L->conv_state_out;
  p.keys = attn ? L->key_cache : nullptr;
  p.values = attn ? L->value_cache : nullptr;
  p.ws = static_cast<char*>(workspace);
  p.capacity = attn ? L->capacity : 1;
  p.position = attn ? position : 0;
  return run_layer(p, reinterpret_cast<hipStream_t>(stream));
}

int lfm25_decode(const lfm25_decoder* d, const int32_t* tokens_in, int32_t n_in, int32_t n_gen,
                 int32_t* tokens_out, int32_t exec, lfm25_stream_t stream) {
  const int rc = check_decoder(d);
  if (rc != LFM25_OK) return rc;
  LFM25_REQUIRE(n_in >= 1, "decode: n_in must be at least 1, got %d", n_in);
  LFM25_REQUIRE(tokens_in != nullptr || n_in == 1,
                "decode: tokens_in may be NULL only with n_in == 1");
  LFM25_REQUIRE(n_gen >= 0, "decode: n_gen must be non-negative");
  LFM25_REQUIRE(n_gen == 0 || tokens_out != nullptr, "decode: tokens_out is NULL");
  LFM25_REQUIRE(exec == LFM25_EXEC_STAGED || exec == LFM25_EXEC_PERSISTENT,
                "decode: unknown exec mode %d", exec);
  const DecodeParams p = make_params(d, tokens_in, n_in, n_gen, tokens_out);
  return exec == LFM25_EXEC_STAGED ? run_staged(p, stream) : run_persistent(p, stream);
}

size_t lfm25_w8_layers_bytes(void) { return (size_t)kW8LayersBytes; }

int32_t lfm25_w8_layers_offsets(int64_t* offsets, int32_t n) {
  int k = 0;
  for (int l = 0; l < kLayers; ++l)
    for (int pr = 0; pr < P_COUNT; ++pr) {
      const bool attn = is_attn(l);
      if (offsets != nullptr && k < n) offsets[k] = w8_layer_off(l) + w8_slot_q(attn, pr);
      ++k;
      if (offsets != nullptr && k < n) offsets[k] = w8_layer_off(l) + w8_slot_s(attn, pr);
      ++k;
    }
  return k;
}

int lfm25_decode_w8(const lfm25_decoder* d, const lfm25_w8_model* w, const int32_t* tokens_in, int32_t n_in,
                    int32_t n_gen, int32_t* tokens_out, lfm25_stream_t stream) {
  const int rc = check_decoder(d);
  if (rc != LFM25_OK) return rc;
  LFM25_REQUIRE(w != nullptr && w->layers && w->table && w->table_scales, "decode_w8: null 8-bit weights");
  LFM25_REQUIRE(aligned16(w->layers) && (reinterpret_cast<uintptr_t>(w->layers) & 255u) == 0 &&
                    aligned16(w->table) && aligned16(w->table_scales),
                "decode_w8: the 8-bit layers must be 256-byte aligned, the table and its scales 16-byte");
  LFM25_REQUIRE(n_in >= 1, "decode_w8: n_in must be at least 1, got %d", n_in);
  LFM25_REQUIRE(tokens_in != nullptr || n_in == 1, "decode_w8: tokens_in may be NULL only with n_in == 1");
  LFM25_REQUIRE(n_gen >= 0, "decode_w8: n_gen must be non-negative");
  LFM25_REQUIRE(n_gen == 0 || tokens_out != nullptr, "decode_w8: tokens_out is NULL");
  DecodeParams p = make_params(d, tokens_in, n_in, n_gen, tokens_out);
  p.w8 = w->layers;
  p.w8_table = w->table;
  p.w8_table_s = w->table_scales;
  return run_persistent(p, stream);
}

}  // extern "C"
