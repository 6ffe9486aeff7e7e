// The whole-token LFM2.5 decode step (the X8Model step of
// experiments/lfm25_x8_model.py:133-148 and the one-submission-per-token
// program of experiments/lfm25_x8.py:227-327) on gfx950.
//
// Two execution models over the same stage functions (lfm25_stages.h):
//   * staged     : one kernel per stage, ~60 launches per token, stream
//                  ordered and capturable in a HIP graph;
//   * persistent : one cooperative launch runs every step of a decode call;
//                  stages are separated by grid-wide barriers (an agent-scope
//                  release/acquire counter), and the token chosen by the
//                  head feeds the next step without returning to the host.
// Position, current token and status live in device control words, so
// neither model needs a host round trip between tokens.
#include <cstring>
#include <mutex>
#include <vector>

#include "lfm25_host.h"
#include "lfm25_stages.h"

namespace lfm25 {

constexpr int kLayers = 14;
constexpr bool kIsAttn[kLayers] = {false, false, true,  false, true,  false, true,
                                   false, true,  false, true,  false, true,  false};

// Tensor slots of a layer in the packed stream.
enum ConvSlot { C_OPNORM, C_IN, C_CONVW, C_OUT, C_FFNNORM, C_W1, C_W3, C_W2, C_COUNT };
enum AttnSlot { A_OPNORM, A_Q, A_K, A_V, A_QLN, A_KLN, A_O, A_FFNNORM, A_W1, A_W3, A_W2, A_COUNT };

struct Layout {
  int64_t off[kLayers * A_COUNT + 1];
  int count;
  int64_t total;
};

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
    if (kIsAttn[l])
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

// Workspace byte offsets.
constexpr size_t kWsCtl = 0;          // int32[64]
constexpr size_t kWsBarrier = 256;    // uint32[64]
constexpr size_t kWsH = 512;          // bf16[1024] residual stream
constexpr size_t kWsY = 2560;         // bf16[1024] conv gate output / attention context
constexpr size_t kWsG = 4608;         // bf16[2560] gated FFN activation
constexpr size_t kWsQkv = 9728;       // bf16[2048]
constexpr size_t kWsCand = 13824;     // Candidate[1024]
constexpr size_t kWsBytes = 32768;
constexpr int kMaxCand = 1024;
constexpr int kCtlStep = 3;           // step index within the current decode call

struct DecodeParams {
  LayerPtrs layer[kLayers];
  const uint16_t* final_norm;
  const uint16_t* embedding;
  const uint16_t* rope;
  uint16_t* conv_state;
  uint16_t* key_cache;
  uint16_t* value_cache;
  int32_t* ctl;
  uint32_t* barrier;
  uint16_t* h;
  uint16_t* y;
  uint16_t* g;
  uint16_t* qkv;
  Candidate* cand;
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
    const int n = kIsAttn[l] ? A_COUNT : C_COUNT;
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
  p.barrier = reinterpret_cast<uint32_t*>(ws + kWsBarrier);
  p.h = reinterpret_cast<uint16_t*>(ws + kWsH);
  p.y = reinterpret_cast<uint16_t*>(ws + kWsY);
  p.g = reinterpret_cast<uint16_t*>(ws + kWsG);
  p.qkv = reinterpret_cast<uint16_t*>(ws + kWsQkv);
  p.cand = reinterpret_cast<Candidate*>(ws + kWsCand);
  p.tokens_in = tokens_in;
  p.tokens_out = tokens_out;
  p.n_in = n_in;
  p.n_gen = n_gen;
  p.capacity = d->capacity;
  p.vocab = d->vocab;
  return p;
}

__device__ __forceinline__ int ctl_load(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Copy the 1024-element embedding row to the residual stream (block-wide).
__device__ __forceinline__ void copy_row(const uint16_t* src, uint16_t* dst) {
  for (int i = threadIdx.x * 8; i < kHidden; i += blockDim.x * 8)
    *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
}

// One KV head of the attention stage at position `pos` (block-wide).
__device__ __forceinline__ void attention_block(const DecodeParams& p, int layer, int att_index,
                                                int kv_head, int pos, AttnShared& sh) {
  const LayerPtrs& L = p.layer[layer];
  const size_t head_rows = (size_t)(att_index * kKvHeads + kv_head) * p.capacity;
  uint16_t* keys = p.key_cache + head_rows * kHeadDim;
  uint16_t* values = p.value_cache + head_rows * kHeadDim;
  const uint16_t* rope_row = p.rope + (size_t)pos * 2 * kHeadDim;
  attn_prep_norm_rope(p.qkv + 2 * kv_head * kHeadDim, p.qkv + kHidden + kv_head * kHeadDim,
                      p.qkv + kHidden + kKvHeads * kHeadDim + kv_head * kHeadDim, L.t[A_QLN],
                      L.t[A_KLN], rope_row, rope_row + kHeadDim, keys, values, pos, sh);
  attn_core(keys, values, pos, p.y + 2 * kv_head * kHeadDim, sh);
}

// ====================================================================== staged

constexpr int kStageThreads = 256;
constexpr int kStageWaves = kStageThreads / kWave;

__global__ void k_decode_init(int32_t* ctl) { ctl[kCtlStep] = 0; }

__global__ void k_step_begin(DecodeParams p) {
  if (threadIdx.x != 0) return;
  const int i = p.ctl[kCtlStep];
  int t = (p.tokens_in != nullptr && i < p.n_in) ? p.tokens_in[i] : p.ctl[LFM25_CTL_TOKEN];
  t = clamp_token(t, p.vocab, p.ctl, true);
  p.ctl[LFM25_CTL_TOKEN] = t;
  if (p.ctl[LFM25_CTL_POSITION] >= p.capacity) p.ctl[LFM25_CTL_STATUS] |= 2;
}

// First stage of a layer: input is the embedding row for layer 0.
__device__ __forceinline__ const uint16_t* layer_input(const DecodeParams& p, bool first) {
  if (!first) return p.h;
  const int t = clamp_token(p.ctl[LFM25_CTL_TOKEN], p.vocab, p.ctl, false);
  const uint16_t* row = p.embedding + (size_t)t * kHidden;
  if (blockIdx.x == 0) copy_row(row, p.h);
  return row;
}

__global__ void __launch_bounds__(kStageThreads) k_conv_in(DecodeParams p, int layer, int conv_index) {
  const uint16_t* x = layer_input(p, layer == 0);
  const LayerPtrs& L = p.layer[layer];
  stage_conv_in(x, L.t[C_OPNORM], L.t[C_IN], L.t[C_CONVW],
                p.conv_state + (size_t)conv_index * kHidden * kConvTaps, p.y);
}

__global__ void __launch_bounds__(kStageThreads) k_qkv(DecodeParams p, int layer) {
  const uint16_t* x = layer_input(p, layer == 0);
  const LayerPtrs& L = p.layer[layer];
  stage_qkv(x, L.t[A_OPNORM], L.t[A_Q], L.t[A_K], L.t[A_V], p.qkv);
}

__global__ void __launch_bounds__(kAttnThreads) k_attention(DecodeParams p, int layer, int att_index) {
  __shared__ AttnShared sh;
  const int pos = p.ctl[LFM25_CTL_POSITION];
  if (pos >= p.capacity) return;
  attention_block(p, layer, att_index, blockIdx.x, pos, sh);
}

__global__ void __launch_bounds__(kStageThreads) k_proj_residual(DecodeParams p, int layer, int slot) {
  stage_proj_residual(p.y, p.layer[layer].t[slot], p.h);
}

__global__ void __launch_bounds__(kStageThreads) k_mlp_up(DecodeParams p, int layer, int norm_slot) {
  const LayerPtrs& L = p.layer[layer];
  stage_mlp_up(p.h, L.t[norm_slot], L.t[norm_slot + 1], L.t[norm_slot + 2], p.g);
}

__global__ void __launch_bounds__(kStageThreads) k_mlp_down(DecodeParams p, int layer, int w2_slot) {
  stage_mlp_down(p.g, p.layer[layer].t[w2_slot], p.h);
}

__global__ void __launch_bounds__(kStageThreads) k_head(DecodeParams p) {
  __shared__ float red_v[kStageWaves];
  __shared__ int red_i[kStageWaves];
  stage_head_scan(p.h, p.final_norm, p.embedding, p.vocab, p.cand, nullptr, red_v, red_i);
}

__global__ void k_step_end(DecodeParams p, int n_cand, int select) {
  const int i = p.ctl[kCtlStep];
  if (select) {
    const int w = pick_candidates(p.cand, n_cand);
    if (threadIdx.x == 0) {
      p.ctl[LFM25_CTL_TOKEN] = w;
      const int o = i - (p.n_in - 1);
      if (p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = w;
    }
  }
  if (threadIdx.x == 0) {
    p.ctl[LFM25_CTL_POSITION] += 1;
    p.ctl[kCtlStep] = i + 1;
  }
}

static int head_grid(int vocab) {
  const int units = vocab / kHeadRows;
  return max(1, min((units + kStageWaves - 1) / kStageWaves, kMaxCand));
}

static int run_staged(const DecodeParams& p, hipStream_t s) {
  const int steps = p.n_in + max(p.n_gen - 1, 0);
  k_decode_init<<<1, 1, 0, s>>>(p.ctl);
  const int hg = head_grid(p.vocab);
  for (int i = 0; i < steps; ++i) {
    const bool select = p.n_gen > 0 && i >= p.n_in - 1;
    k_step_begin<<<1, 64, 0, s>>>(p);
    int conv_index = 0, att_index = 0;
    for (int l = 0; l < kLayers; ++l) {
      if (kIsAttn[l]) {
        k_qkv<<<kHidden * 2 / kQkvRows / kStageWaves, kStageThreads, 0, s>>>(p, l);
        k_attention<<<kKvHeads, kAttnThreads, 0, s>>>(p, l, att_index++);
        k_proj_residual<<<kHidden / kProjRows / kStageWaves, kStageThreads, 0, s>>>(p, l, A_O);
        k_mlp_up<<<kFfn / kUpCols / kStageWaves, kStageThreads, 0, s>>>(p, l, A_FFNNORM);
        k_mlp_down<<<kHidden / kDownRows / kStageWaves, kStageThreads, 0, s>>>(p, l, A_W2);
      } else {
        k_conv_in<<<kHidden / kStageWaves, kStageThreads, 0, s>>>(p, l, conv_index++);
        k_proj_residual<<<kHidden / kProjRows / kStageWaves, kStageThreads, 0, s>>>(p, l, C_OUT);
        k_mlp_up<<<kFfn / kUpCols / kStageWaves, kStageThreads, 0, s>>>(p, l, C_FFNNORM);
        k_mlp_down<<<kHidden / kDownRows / kStageWaves, kStageThreads, 0, s>>>(p, l, C_W2);
      }
    }
    if (select) k_head<<<hg, kStageThreads, 0, s>>>(p);
    k_step_end<<<1, 64, 0, s>>>(p, hg, select ? 1 : 0);
    const int rc = check_launch("decode (staged)");
    if (rc != LFM25_OK) return rc;
  }
  return LFM25_OK;
}

// ====================================================================== persistent

constexpr int kPersistThreads = 256;
// Barrier time-out in s_memrealtime ticks (100 MHz): 5 s.
constexpr uint64_t kBarrierTimeout = 500000000ull;

// Grid-wide barrier on a monotonically increasing arrival counter: the
// n-th barrier of a launch completes when the counter reaches n * blocks.
// Agent-scope release on arrival / acquire on the final read make every
// block's prior global writes visible to every other block (all XCDs).
// A stuck barrier gives up after kBarrierTimeout, sets status bit 2 and
// releases every other waiter, so the grid always drains.
__device__ __forceinline__ void grid_barrier(uint32_t* counter, uint32_t target, int32_t* ctl) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if ((ctl_load(ctl + LFM25_CTL_STATUS) & 4) != 0) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kBarrierTimeout) {
        ctl_or(ctl + LFM25_CTL_STATUS, 4);
        break;
      }
    }
  }
  __syncthreads();
}

__global__ void k_reset_barrier(uint32_t* counter) { counter[0] = 0; }

__global__ void __launch_bounds__(kPersistThreads) k_decode_persistent(DecodeParams p) {
  __shared__ AttnShared sh;
  __shared__ float red_v[kPersistThreads / kWave];
  __shared__ int red_i[kPersistThreads / kWave];
  __shared__ int s_winner;
  const uint32_t nb = gridDim.x;
  uint32_t target = 0;
  auto sync = [&]() {
    target += nb;
    grid_barrier(p.barrier, target, p.ctl);
  };

  int pos = ctl_load(p.ctl + LFM25_CTL_POSITION);
  int token = ctl_load(p.ctl + LFM25_CTL_TOKEN);
  const int steps = p.n_in + max(p.n_gen - 1, 0);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  for (int i = 0; i < steps; ++i) {
    if (p.tokens_in != nullptr && i < p.n_in) token = p.tokens_in[i];
    token = clamp_token(token, p.vocab, p.ctl, lead);
    if (pos >= p.capacity) {
      if (lead) ctl_or(p.ctl + LFM25_CTL_STATUS, 2);
      break;
    }
    const bool select = p.n_gen > 0 && i >= p.n_in - 1;
    const uint16_t* row = p.embedding + (size_t)token * kHidden;
    int conv_index = 0, att_index = 0;
    for (int l = 0; l < kLayers; ++l) {
      const LayerPtrs& L = p.layer[l];
      const uint16_t* x = l == 0 ? row : p.h;
      if (l == 0 && blockIdx.x == 0) copy_row(row, p.h);
      if (kIsAttn[l]) {
        stage_qkv(x, L.t[A_OPNORM], L.t[A_Q], L.t[A_K], L.t[A_V], p.qkv);
        sync();
        if ((int)blockIdx.x < kKvHeads) attention_block(p, l, att_index, blockIdx.x, pos, sh);
        ++att_index;
        sync();
        stage_proj_residual(p.y, L.t[A_O], p.h);
        sync();
        stage_mlp_up(p.h, L.t[A_FFNNORM], L.t[A_W1], L.t[A_W3], p.g);
        sync();
        stage_mlp_down(p.g, L.t[A_W2], p.h);
        sync();
      } else {
        stage_conv_in(x, L.t[C_OPNORM], L.t[C_IN], L.t[C_CONVW],
                      p.conv_state + (size_t)conv_index * kHidden * kConvTaps, p.y);
        ++conv_index;
        sync();
        stage_proj_residual(p.y, L.t[C_OUT], p.h);
        sync();
        stage_mlp_up(p.h, L.t[C_FFNNORM], L.t[C_W1], L.t[C_W3], p.g);
        sync();
        stage_mlp_down(p.g, L.t[C_W2], p.h);
        sync();
      }
    }
    if (select) {
      stage_head_scan(p.h, p.final_norm, p.embedding, p.vocab, p.cand, nullptr, red_v, red_i);
      sync();
      // Every block merges the candidates itself (same data, same order), so
      // the next step starts without another barrier.
      if (wave_id() == 0) {
        const int w = pick_candidates(p.cand, nb);
        if (lane_id() == 0) s_winner = w;
      }
      __syncthreads();
      token = s_winner;
      if (lead) {
        const int o = i - (p.n_in - 1);
        if (p.tokens_out != nullptr && o >= 0 && o < p.n_gen) p.tokens_out[o] = token;
      }
    }
    ++pos;
  }
  if (lead) {
    ctl_store(p.ctl + LFM25_CTL_POSITION, pos);
    ctl_store(p.ctl + LFM25_CTL_TOKEN, token);
  }
}

struct PersistentConfig {
  int grid = 0;
  int error = 0;
};

static PersistentConfig persistent_config() {
  static std::mutex mu;
  static std::vector<PersistentConfig> per_device;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return {0, 1};
  std::lock_guard<std::mutex> lock(mu);
  if ((int)per_device.size() <= dev) per_device.resize(dev + 1);
  PersistentConfig& c = per_device[dev];
  if (c.grid == 0 && c.error == 0) {
    int cus = 0, coop = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_persistent, kPersistThreads,
                                                     0) != hipSuccess ||
        !coop || per_cu < 1) {
      c.error = 1;
    } else {
      c.grid = min(cus, kMaxCand);
    }
  }
  return c;
}

static int run_persistent(DecodeParams p, hipStream_t s) {
  const PersistentConfig c = persistent_config();
  if (c.error || c.grid < kKvHeads)
    return set_error(LFM25_EDEVICE, "decode: cooperative launch unavailable on this device");
  k_reset_barrier<<<1, 1, 0, s>>>(p.barrier);
  int rc = check_launch("decode (barrier reset)");
  if (rc != LFM25_OK) return rc;
  void* args[] = {&p};
  const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_decode_persistent),
                                                  dim3(c.grid), dim3(kPersistThreads), args, 0, s);
  if (e != hipSuccess)
    return set_error(LFM25_EDEVICE, "decode (persistent): %s", hipGetErrorString(e));
  return LFM25_OK;
}

__global__ void k_decoder_reset(uint16_t* conv_state, int32_t* ctl) {
  constexpr int n = LFM25_CONV_LAYERS * kHidden * kConvTaps;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    conv_state[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x < 64) ctl[threadIdx.x] = 0;
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
  LFM25_REQUIRE(d->vocab >= kHeadRows && d->vocab % kHeadRows == 0,
                "decoder: vocab must be a positive multiple of %d, got %d", kHeadRows, d->vocab);
  LFM25_REQUIRE(aligned16(d->weights) && aligned16(d->embedding) && aligned16(d->key_cache) &&
                    aligned16(d->value_cache) &&
                    (reinterpret_cast<uintptr_t>(d->workspace) & 255u) == 0,
                "decoder: buffers must be 16-byte aligned (workspace 256-byte)");
  return LFM25_OK;
}

int lfm25_decoder_reset(const lfm25_decoder* d, lfm25_stream_t stream) {
  const int rc = check_decoder(d);
  if (rc != LFM25_OK) return rc;
  int32_t* ctl = reinterpret_cast<int32_t*>(static_cast<char*>(d->workspace) + kWsCtl);
  k_decoder_reset<<<24, 256, 0, stream>>>(d->conv_state, ctl);
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
