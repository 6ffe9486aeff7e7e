// The whole-token LFM2.5 decode step (the X8Model step of
// experiments/lfm25_x8_model.py:133-148 and the one-submission-per-token
// program of experiments/lfm25_x8.py:227-327) on gfx950.
//
// Two execution models over the same block-level stages (lfm25_step.h), on
// the same 256-block grid and with the same epoch tags, so they are bitwise
// identical:
//   * persistent : one cooperative launch runs every step of a decode call;
//                  stages hand activations to each other through tagged
//                  words (the data is the barrier), and the token chosen by
//                  the head feeds the next step without returning to the host;
//   * staged     : one kernel per stage (63 per token), stream ordered and
//                  capturable in a HIP graph.
// Position, current token, epoch and status live in device control words, so
// neither model needs a host round trip between tokens.
#include <cstring>
#include <mutex>
#include <vector>

#include "lfm25_host.h"
#include "lfm25_step.h"

namespace lfm25 {

constexpr int kLayers = 14;
// Layer kinds (modeling_lfm2.py layer_types of LFM2.5-230M): attention at
// layers 2, 4, ..., 12, gated short conv elsewhere. Written as arithmetic so
// device code never loads a table for it.
__host__ __device__ constexpr bool is_attn(int l) { return l >= 2 && l <= 12 && (l & 1) == 0; }
// Conv layers before layer l (its conv index when it is a conv layer).
__host__ __device__ constexpr int conv_before(int l) { return l < 2 ? l : (l + 2) >> 1; }
static_assert(conv_before(kLayers - 1) + 1 == LFM25_CONV_LAYERS, "conv layer count");
static_assert(kLayers - LFM25_CONV_LAYERS == LFM25_ATTN_LAYERS, "attention layer count");

// Tensor slots of a layer in the packed stream.
enum ConvSlot { C_OPNORM, C_IN, C_CONVW, C_OUT, C_FFNNORM, C_W1, C_W3, C_W2, C_COUNT };
enum AttnSlot { A_OPNORM, A_Q, A_K, A_V, A_QLN, A_KLN, A_O, A_FFNNORM, A_W1, A_W3, A_W2, A_COUNT };

struct Layout {
  int64_t off[kLayers * A_COUNT + 1];
  int count;
  int64_t total;
};

// The q, k and v matrices of an attention layer are placed back to back
// (their sizes are multiples of the 128-element alignment), so q/k/v row r is
// row r of one 2048 x 1024 matrix starting at the q slot.
static_assert((1LL * kHidden * kHidden) % 128 == 0 && (512LL * kHidden) % 128 == 0,
              "q/k/v stay contiguous in the packed stream");

static Layout build_layout() {
  static const int64_t conv_sizes[C_COUNT] = {kHidden,          3LL * kHidden * kHidden,
                                              3LL * kHidden,    1LL * kHidden * kHidden,
                                              kHidden,          1LL * kFfn * kHidden,
                                              1LL * kFfn * kHidden, 1LL * kHidden * kFfn};
  static const int64_t attn_sizes[A_COUNT] = {kHidden,
                                              1LL * kHidden * kHidden,
                                              512LL * kHidden,
                                              512LL * kHidden,
                                              kHeadDim,
                                              kHeadDim,
                                              1LL * kHidden * kHidden,
                                              kHidden,
                                              1LL * kFfn * kHidden,
                                              1LL * kFfn * kHidden,
                                              1LL * kHidden * kFfn};
  Layout L{};
  int64_t at = 0;
  auto place = [&](int64_t n) {
    L.off[L.count++] = at;
    at += (n + 127) / 128 * 128;
  };
  for (int l = 0; l < kLayers; ++l) {
    if (is_attn(l))
      for (int i = 0; i < A_COUNT; ++i) place(attn_sizes[i]);
    else
      for (int i = 0; i < C_COUNT; ++i) place(conv_sizes[i]);
  }
  place(kHidden);  // embedding_norm
  L.total = at;
  return L;
}

static const Layout& layout() {
  static const Layout L = build_layout();
  return L;
}

struct LayerPtrs {
  const uint16_t* t[A_COUNT];
};

// Workspace byte offsets (tagged activation words, see lfm25_step.h).
constexpr size_t kWsCtl = 0;        // int32[64] control words
constexpr size_t kWsH = 256;        // uint32[1024] residual stream
constexpr size_t kWsY = 4352;       // uint32[1024] conv gate output / attention context
constexpr size_t kWsG = 8448;       // uint32[2560] gated FFN activation
constexpr size_t kWsQkv = 18688;    // uint32[2048]
constexpr size_t kWsCand = 26880;   // uint64[1024] head candidates
constexpr size_t kWsBytes = 40960;
constexpr int kCtlStep = 3;         // step index within the current decode call
constexpr int kCtlEpoch = 4;        // last epoch tag used (16-bit, wraps)
constexpr int kGrid = kStepBlocks;  // blocks of both execution models
static_assert(kGrid <= kMaxCandidates, "one head candidate per block");

struct DecodeParams {
  LayerPtrs layer[kLayers];
  const uint16_t* final_norm;
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
};

static DecodeParams make_params(const lfm25_decoder* d, const int32_t* tokens_in, int n_in,
                                int n_gen, int32_t* tokens_out) {
  const Layout& L = layout();
  DecodeParams p{};
  int slot = 0;
  for (int l = 0; l < kLayers; ++l) {
    const int n = is_attn(l) ? A_COUNT : C_COUNT;
    for (int i = 0; i < n; ++i) p.layer[l].t[i] = d->weights + L.off[slot++];
  }
  p.final_norm = d->weights + L.off[slot];
  p.embedding = d->embedding;
  p.rope = d->rope;
  p.conv_state = d->conv_state;
  p.key_cache = d->key_cache;
  p.value_cache = d->value_cache;
  char* ws = static_cast<char*>(d->workspace);
  p.ctl = reinterpret_cast<int32_t*>(ws + kWsCtl);
  p.bufs.h = reinterpret_cast<uint32_t*>(ws + kWsH);
  p.bufs.y = reinterpret_cast<uint32_t*>(ws + kWsY);
  p.bufs.g = reinterpret_cast<uint32_t*>(ws + kWsG);
  p.bufs.qkv = reinterpret_cast<uint32_t*>(ws + kWsQkv);
  p.bufs.cand = reinterpret_cast<uint64_t*>(ws + kWsCand);
  p.bufs.status = p.ctl + LFM25_CTL_STATUS;
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

__device__ __forceinline__ uint16_t* head_keys(const DecodeParams& p, int att_index, int kv) {
  return p.key_cache + (size_t)(att_index * kKvHeads + kv) * p.capacity * kHeadDim;
}
__device__ __forceinline__ uint16_t* head_values(const DecodeParams& p, int att_index, int kv) {
  return p.value_cache + (size_t)(att_index * kKvHeads + kv) * p.capacity * kHeadDim;
}

// RMSNorm weights of a step: op_norm and ffn_norm of every layer, then the
// final norm.
constexpr int kNorms = 2 * kLayers + 1;
__device__ __forceinline__ const uint16_t* norm_weight(const DecodeParams& p, int n) {
  if (n == 2 * kLayers) return p.final_norm;
  const int l = n / 2;
  const int slot = (n & 1) ? (is_attn(l) ? A_FFNNORM : C_FFNNORM) : (is_attn(l) ? A_OPNORM : C_OPNORM);
  return p.layer[l].t[slot];
}

// Shared memory of one decode block.
// The gathered vectors come first so every dot-product read addresses them
// with a lane offset plus an immediate.
struct StepShared {
  alignas(16) uint32_t lds[2][kFfn / 2];  // double-buffered gathered vectors (bf16 pairs)
  AttnSharedT<kStepThreads> attn;
  float red_v[kStepWaves];
  int red_i[kStepWaves];
  int winner;
  uint32_t out[kMaxBlockOut];         // a stage's output words before publish
  uint32_t norms[kNorms][kNormWords]; // every norm weight of the step, loaded once
};

// Epoch tags of one step, assigned in stage order (shared by both execution
// models so they produce identical tags).
struct StepTags {
  uint32_t base;
  int next = 0;
  __device__ __host__ uint32_t take() { return (base + (uint32_t)(++next)) & 0xffffu; }
};

__device__ __forceinline__ uint16_t* conv_state_of(const DecodeParams& p, int conv_index) {
  return p.conv_state + (size_t)conv_index * kHidden * kConvTaps;
}

// Prefetch of a layer's first stage (in_proj + conv, or q/k/v), without a
// branch on the layer kind: an attention layer passes layer 0's conv operands,
// which its units load but never use.
static_assert(C_IN == A_Q, "in_proj and q share the first weight slot");
__device__ __forceinline__ void prefetch_first(Slab& s, const DecodeParams& p, int l) {
  const bool attn = is_attn(l);
  const int conv_index = attn ? 0 : conv_before(l);
  prefetch_first_stage(s, attn, p.layer[l].t[C_IN], p.layer[attn ? 0 : l].t[C_CONVW],
                       conv_state_of(p, conv_index));
}

// One token through all layers (and the head when `select`), block-wide, as
// a software pipeline over a ring of two register slabs: S0 carries the
// first stage (in_proj + conv, or q/k/v) and the up projection of every
// layer, S1 the residual projection and w2. A slab is refilled with the
// weights of the stage two steps ahead as soon as its own dot products are
// done, so every stage's weights have had a whole stage to arrive. On entry
// S0/S1 hold layer 0's first stage and out_proj; on exit they hold the next
// token's. The layer loop is unrolled so the slab roles and load counts are
// static. Returns the selected token in every thread (or -1).
__device__ int decode_token(const DecodeParams& p, int token, int pos, bool select, uint32_t base,
                            StepShared& sm, Slab& S0, Slab& S1) {
  const StepBufs& b = p.bufs;
  StepTags tags{base};
  int buf = 0;
  auto lds = [&]() {
    buf ^= 1;
    return sm.lds[buf];
  };
  const uint16_t* row = p.embedding + (size_t)token * kHidden;
  const int hr = stage_unit<kHidden>();
  float hres = 0.0f;  // h[hr] in lane 0 of the wave owning residual row hr
  if (hr < kHidden && lane_id() == 0) hres = bf16_to_f32(row[hr]);
  LayerIn in{row, 0};
#pragma unroll
  for (int l = 0; l < kLayers; ++l) {
    const LayerPtrs& L = p.layer[l];
    const int conv_index = conv_before(l), att_index = l - conv_before(l);
    const int ffn = is_attn(l) ? A_FFNNORM : C_FFNNORM;
    uint32_t t_y;
    if (is_attn(l)) {
      const uint32_t t_qkv = tags.take();
      run_qkv(S0, sm.norms[2 * l], in, b, t_qkv, lds(), sm.out);
      t_y = tags.take();
      if ((int)blockIdx.x < kKvHeads) {
        const int kv = blockIdx.x;
        run_attention(kv, t_qkv, L.t[A_QLN], L.t[A_KLN], p.rope + (size_t)pos * 2 * kHeadDim,
                      head_keys(p, att_index, kv), head_values(p, att_index, kv), pos, b, t_y,
                      sm.attn);
      }
    } else {
      t_y = tags.take();
      run_conv_in(S0, sm.norms[2 * l], in, conv_state_of(p, conv_index), b, t_y, lds(), sm.out);
    }
    // Slab loads stay outside the branches on the layer kind (see prefetch_first).
    prefetch_up(S0, L.t[ffn + 1], L.t[ffn + 2]);
    const uint32_t t_h1 = tags.take();
    run_proj(S1, b.y, t_y, hres, b, t_h1, lds(), sm.out);
    prefetch_down(S1, L.t[ffn + 3]);
    const uint32_t t_g = tags.take();
    run_up(S0, sm.norms[2 * l + 1], t_h1, b, t_g, lds(), sm.out);
    const int nl = l + 1 < kLayers ? l + 1 : 0;
    prefetch_first(S0, p, nl);
    const uint32_t t_h2 = tags.take();
    run_down(S1, t_g, hres, b, t_h2, lds(), sm.out);
    prefetch_proj(S1, p.layer[nl].t[is_attn(nl) ? A_O : C_OUT]);
    in = LayerIn{nullptr, t_h2};
  }
  if (!select) return -1;
  const uint32_t t_c = tags.take();
  Slab H;
  prefetch_head(H, p.embedding, p.vocab);
  run_head(H, sm.norms[2 * kLayers], in.tag, p.embedding, p.vocab, b, t_c, lds(), sm.red_v,
           sm.red_i);
  return step_pick(b, kGrid, t_c, &sm.winner);
}

// Stages of one step: 4 per conv layer, 5 per attention layer, 1 head.
constexpr int kStagesNoHead = 4 * LFM25_CONV_LAYERS + 5 * LFM25_ATTN_LAYERS;

// ====================================================================== persistent

__global__ void __launch_bounds__(kStepThreads) k_decode_persistent(DecodeParams p) {
  __shared__ StepShared sm;
  int pos = ctl_load(p.ctl + LFM25_CTL_POSITION);
  int token = ctl_load(p.ctl + LFM25_CTL_TOKEN);
  uint32_t epoch = (uint32_t)ctl_load(p.ctl + kCtlEpoch);
  const int steps = p.n_in + max(p.n_gen - 1, 0);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  for (int n = 0; n < kNorms; ++n) load_norm_lds(sm.norms[n], norm_weight(p, n));
  Slab S0, S1;
  prefetch_first(S0, p, 0);
  prefetch_proj(S1, p.layer[0].t[is_attn(0) ? A_O : C_OUT]);
  for (int i = 0; i < steps; ++i) {
    if (p.tokens_in != nullptr && i < p.n_in) token = p.tokens_in[i];
    token = clamp_token(token, p.vocab, p.ctl, lead);
    if (pos >= p.capacity) {
      if (lead) ctl_or(p.ctl + LFM25_CTL_STATUS, 2);
      break;
    }
    const bool select = p.n_gen > 0 && i >= p.n_in - 1;
    const int w = decode_token(p, token, pos, select, epoch, sm, S0, S1);
    epoch += kStagesNoHead + (select ? 1 : 0);
    if (select) {
      token = w;
      const int o = i - (p.n_in - 1);
      if (lead && p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = token;
    }
    ++pos;
  }
  if (lead) {
    ctl_store(p.ctl + LFM25_CTL_POSITION, pos);
    ctl_store(p.ctl + LFM25_CTL_TOKEN, token);
    ctl_store(p.ctl + kCtlEpoch, (int)(epoch & 0xffffu));
  }
}

static int persistent_grid(int* grid) {
  static std::mutex mu;
  static std::vector<int> per_device;  // 0 unknown, -1 unsupported, else grid
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return LFM25_EDEVICE;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)per_device.size() <= dev) per_device.resize(dev + 1, 0);
  int& g = per_device[dev];
  if (g == 0) {
    int cus = 0, coop = 0, per_cu = 0;
    g = -1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_persistent, kStepThreads,
                                                     0) == hipSuccess &&
        coop && per_cu >= 1 && cus * per_cu >= kGrid)
      g = kGrid;
  }
  *grid = g;
  return g > 0 ? LFM25_OK : LFM25_EDEVICE;
}

static int run_persistent(DecodeParams p, hipStream_t s) {
  int grid = 0;
  if (persistent_grid(&grid) != LFM25_OK)
    return set_error(LFM25_EDEVICE, "decode: a cooperative launch of %d blocks of %d threads is "
                     "not possible on this device", kGrid, kStepThreads);
  void* args[] = {&p};
  const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_decode_persistent),
                                                  dim3(grid), dim3(kStepThreads), args, 0, s);
  if (e != hipSuccess)
    return set_error(LFM25_EDEVICE, "decode (persistent): %s", hipGetErrorString(e));
  return LFM25_OK;
}

// ====================================================================== staged
//
// The same stages, one kernel each, on the same grid, with tags derived from
// the control words: every stage kernel reads the step's base epoch and gets
// its own and its inputs' offsets within the step from the host.

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

__device__ __forceinline__ StagedCtx staged_ctx(const DecodeParams& p) {
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

// off_in < 0: the layer input is the embedding row.
__device__ __forceinline__ LayerIn staged_in(const StagedCtx& c, int off_in) {
  return off_in < 0 ? LayerIn{c.row, 0} : LayerIn{nullptr, tag_at(c.base, off_in)};
}

// Residual h[gw] for the staged kernels: the embedding value for layer 0
// (off_h < 0), otherwise the tagged word written by the previous stage.
__device__ __forceinline__ float staged_hres(const DecodeParams& p, const StagedCtx& c, int off_h) {
  const int gw = stage_unit<kHidden>();
  if (gw >= kHidden || lane_id() != 0) return 0.0f;
  if (off_h < 0) return bf16_to_f32(c.row[gw]);
  const uint32_t tag = tag_at(c.base, off_h);
  Poll poll(p.bufs.status);
  uint32_t w = coherent_load32(p.bufs.h + gw);
  while (!tag_ok(w, tag) && poll.again()) w = coherent_load32(p.bufs.h + gw);
  return tagged_value(w);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_conv_in(DecodeParams p, int l, int conv_index, int off_in, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ uint32_t out[kMaxBlockOut];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const LayerPtrs& L = p.layer[l];
  __shared__ uint32_t gamma[kNormWords];
  load_norm_lds(gamma, L.t[C_OPNORM]);
  Slab s;
  prefetch_first_stage(s, false, L.t[C_IN], L.t[C_CONVW], conv_state_of(p, conv_index));
  run_conv_in(s, gamma, staged_in(c, off_in), conv_state_of(p, conv_index), p.bufs,
              tag_at(c.base, off_out), lds, out);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_qkv(DecodeParams p, int l, int off_in, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ uint32_t out[kMaxBlockOut];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const LayerPtrs& L = p.layer[l];
  __shared__ uint32_t gamma[kNormWords];
  load_norm_lds(gamma, L.t[A_OPNORM]);
  Slab s;
  prefetch_first_stage(s, true, L.t[A_Q], p.layer[0].t[C_CONVW], conv_state_of(p, 0));
  run_qkv(s, gamma, staged_in(c, off_in), p.bufs, tag_at(c.base, off_out), lds, out);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_attention(DecodeParams p, int l, int att_index, int off_qkv, int off_out) {
  __shared__ AttnSharedT<kStepThreads> sh;
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const LayerPtrs& L = p.layer[l];
  const int kv = blockIdx.x;
  run_attention(kv, tag_at(c.base, off_qkv), L.t[A_QLN], L.t[A_KLN],
                p.rope + (size_t)c.pos * 2 * kHeadDim, head_keys(p, att_index, kv),
                head_values(p, att_index, kv), c.pos, p.bufs, tag_at(c.base, off_out), sh);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_proj(DecodeParams p, int l, int slot, int off_res, int off_v, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ uint32_t out[kMaxBlockOut];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  Slab s;
  prefetch_proj(s, p.layer[l].t[slot]);
  float hres = staged_hres(p, c, off_res);
  run_proj(s, p.bufs.y, tag_at(c.base, off_v), hres, p.bufs, tag_at(c.base, off_out), lds, out);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_mlp_up(DecodeParams p, int l, int norm_slot, int off_h, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ uint32_t out[kMaxBlockOut];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  const LayerPtrs& L = p.layer[l];
  __shared__ uint32_t gamma[kNormWords];
  load_norm_lds(gamma, L.t[norm_slot]);
  Slab s;
  prefetch_up(s, L.t[norm_slot + 1], L.t[norm_slot + 2]);
  run_up(s, gamma, tag_at(c.base, off_h), p.bufs, tag_at(c.base, off_out), lds, out);
}

__global__ void __launch_bounds__(kStepThreads)
    k_st_mlp_down(DecodeParams p, int l, int w2_slot, int off_g, int off_h, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ uint32_t out[kMaxBlockOut];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  Slab s;
  prefetch_down(s, p.layer[l].t[w2_slot]);
  float hres = staged_hres(p, c, off_h);
  run_down(s, tag_at(c.base, off_g), hres, p.bufs, tag_at(c.base, off_out), lds, out);
}

__global__ void __launch_bounds__(kStepThreads) k_st_head(DecodeParams p, int off_h, int off_out) {
  __shared__ alignas(16) uint32_t lds[kFfn / 2];
  __shared__ float red_v[kStepWaves];
  __shared__ int red_i[kStepWaves];
  const StagedCtx c = staged_ctx(p);
  if (c.halted) return;
  __shared__ uint32_t gamma[kNormWords];
  load_norm_lds(gamma, p.final_norm);
  Slab s;
  prefetch_head(s, p.embedding, p.vocab);
  __syncthreads();  // the head gathers without a leading block sync
  run_head(s, gamma, tag_at(c.base, off_h), p.embedding, p.vocab, p.bufs, tag_at(c.base, off_out),
           lds, red_v, red_i);
}

__global__ void k_step_end(DecodeParams p, int select, int off_head, int stages) {
  __shared__ int winner;
  const int i = p.ctl[kCtlStep];
  const bool halted = p.ctl[LFM25_CTL_POSITION] >= p.capacity;
  if (select && !halted) {
    const int w = step_pick(p.bufs, kGrid, tag_at((uint32_t)p.ctl[kCtlEpoch], off_head), &winner);
    if (threadIdx.x == 0) {
      p.ctl[LFM25_CTL_TOKEN] = w;
      const int o = i - (p.n_in - 1);
      if (p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = w;
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
    int conv_index = 0, att_index = 0;
    for (int l = 0; l < kLayers; ++l) {
      int off_h1, ffn;
      if (is_attn(l)) {
        const int off_qkv = ++off;
        k_st_qkv<<<kGrid, kStepThreads, 0, s>>>(p, l, off_in, off_qkv);
        const int off_y = ++off;
        k_st_attention<<<kKvHeads, kStepThreads, 0, s>>>(p, l, att_index++, off_qkv, off_y);
        off_h1 = ++off;
        k_st_proj<<<kGrid, kStepThreads, 0, s>>>(p, l, A_O, off_in, off_y, off_h1);
        ffn = A_FFNNORM;
      } else {
        const int off_y = ++off;
        k_st_conv_in<<<kGrid, kStepThreads, 0, s>>>(p, l, conv_index++, off_in, off_y);
        off_h1 = ++off;
        k_st_proj<<<kGrid, kStepThreads, 0, s>>>(p, l, C_OUT, off_in, off_y, off_h1);
        ffn = C_FFNNORM;
      }
      const int off_g = ++off;
      k_st_mlp_up<<<kGrid, kStepThreads, 0, s>>>(p, l, ffn, off_h1, off_g);
      const int off_h2 = ++off;
      k_st_mlp_down<<<kGrid, kStepThreads, 0, s>>>(p, l, ffn + 3, off_g, off_h1, off_h2);
      off_in = off_h2;
    }
    int off_head = 0;
    if (select) {
      off_head = ++off;
      k_st_head<<<kGrid, kStepThreads, 0, s>>>(p, off_in, off_head);
    }
    k_step_end<<<1, 64, 0, s>>>(p, select ? 1 : 0, off_head, off);
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

}  // namespace lfm25

using namespace lfm25;

extern "C" {

size_t lfm25_weights_elems(void) { return (size_t)layout().total; }

int32_t lfm25_weights_offsets(int64_t* offsets, int32_t n) {
  const Layout& L = layout();
  if (offsets != nullptr)
    for (int i = 0; i < n && i < L.count; ++i) offsets[i] = L.off[i];
  return L.count;
}

size_t lfm25_decoder_workspace_bytes(void) { return kWsBytes; }

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
  LFM25_REQUIRE(aligned16(d->weights) && aligned16(d->embedding) && aligned16(d->key_cache) &&
                    aligned16(d->value_cache) &&
                    (reinterpret_cast<uintptr_t>(d->workspace) & 255u) == 0,
                "decoder: buffers must be 16-byte aligned (workspace 256-byte)");
  return LFM25_OK;
}

int lfm25_decoder_reset(const lfm25_decoder* d, lfm25_stream_t stream) {
  const int rc = check_decoder(d);
  if (rc != LFM25_OK) return rc;
  k_decoder_reset<<<24, 256, 0, stream>>>(d->conv_state, static_cast<uint32_t*>(d->workspace));
  return check_launch("decoder_reset");
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

}  // extern "C"
