// The reference's remaining per-operation entry points on gfx950: the
// attention programs over its fixed-capacity and chunked cache layouts, the
// first-position attention, the packing programs that assemble the NPU's
// input buffers, and the BF16 x BF16 -> FP32 matrix product.
//
// Cache layouts (reference: experiments/lfm25_attention_fixed_cache_kernel.py
// :17-28, lfm25_attention_fixed64_cache_kernel.py:16-28,
// lfm25_attention_chunked_cache_kernel.py:16-18, and their kernels
// kernels/lfm25_attention_fixed_head.cc, _fixed64_head.cc, _chunked_head.cc):
// a head region of 2 + 2 * cap * 64 BF16 values holds its filled length as a
// BF16 number in element 0 (element 1 unused), then cap key rows, then cap
// value rows; a cache is 8 such regions, one per KV head, and a chunked cache
// is `blocks` such caches of cap = 64 back to back, the new position appended
// to the last block. The numbers follow the CPU path the decode follows
// (eager attention with BF16 probabilities, the same kernel as
// lfm25_attention_context), not the NPU kernels' polynomial exp.
#include "lfm25_host.h"
#include "lfm25_stages.h"

namespace lfm25 {
namespace {

constexpr int kMaxBlocks = 64;  // chunked caches: 64 blocks of 64 positions = the 4,096-position capacity

__host__ __device__ constexpr int head_elems(int cap) { return 2 + 2 * cap * kHeadDim; }

// Rows of KV head h in a headered cache of `blocks` blocks of capacity cap;
// starts[b] = first position of block b (starts[blocks] = the total length).
struct HeaderedRows {
  const uint16_t* cache;
  const int* starts;
  int head, cap, blocks;
  static constexpr bool kAligned16 = false;  // rows sit 4 bytes past an 8-byte boundary
  __device__ const uint16_t* region(int j, int& within) const {
    int lo = 0, hi = blocks - 1;  // the block b with starts[b] <= j < starts[b + 1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (starts[mid] <= j) lo = mid;
      else hi = mid - 1;
    }
    within = j - starts[lo];
    return cache + ((size_t)lo * kKvHeads + head) * head_elems(cap);
  }
  __device__ const uint16_t* key(int j) const {
    int w;
    const uint16_t* r = region(j, w);
    return r + 2 + (size_t)w * kHeadDim;
  }
  __device__ const uint16_t* value(int j) const {
    int w;
    const uint16_t* r = region(j, w);
    return r + 2 + (size_t)(cap + w) * kHeadDim;
  }
};

struct HeaderedShared {
  AttnShared attn;
  int starts[kMaxBlocks + 1];
  int bad;
};

// One KV head per block (8 blocks): the context of its two query heads over
// the cached positions of `past` (NULL: an empty cache, the first position)
// plus the current one, into tail[1024 + ...]; tail[0:1024] = the hidden
// half of qkv_and_hidden; `next` = the cache with the current key / value
// appended and the last block's length raised by one (next may be past).
// A length outside [0, cap) (or a full block before the last) sets status
// bit 0 and leaves the head's outputs unwritten.
__global__ void __launch_bounds__(kAttnThreads) k_attention_headered(const uint16_t* __restrict__ qkv, const uint16_t* past,
                                                                     uint16_t* __restrict__ tail, uint16_t* next,
                                                                     int cap, int blocks, int32_t* status) {
  __shared__ HeaderedShared sh;
  const int h = blockIdx.x;
  const int he = head_elems(cap);
  if (threadIdx.x == 0) {
    int at = 0, bad = 0;
    for (int b = 0; b < blocks; ++b) {
      sh.starts[b] = at;
      const int len = past == nullptr ? 0 : (int)bf16_to_f32(past[((size_t)b * kKvHeads + h) * he]);
      const bool last = b == blocks - 1;
      if (len < 0 || len > cap || (last && len >= cap) || (!last && len != cap)) bad = 1;
      at += len;
    }
    sh.starts[blocks] = at;
    sh.bad = bad;
    if (bad && status != nullptr) atomicOr(status, 1);
  }
  __syncthreads();
  if (sh.bad) return;
  const int total_past = sh.starts[blocks];
  const int last_len = total_past - sh.starts[blocks - 1];
  attn_prep_plain(qkv + 2 * h * kHeadDim, qkv + kHidden + h * kHeadDim,
                  qkv + kHidden + kKvHeads * kHeadDim + h * kHeadDim, sh.attn);
  attn_core_t<kAttnThreads>(HeaderedRows{past, sh.starts, h, cap, blocks}, total_past, sh.attn);
  const int t = threadIdx.x;
  if (t < 2 * kHeadDim) tail[kHidden + 2 * h * kHeadDim + t] = f32_to_bf16(sh.attn.out[t]);
  for (int i = t; i < kHidden / kKvHeads; i += blockDim.x) {
    const int e = h * (kHidden / kKvHeads) + i;  // every block copies its eighth of the hidden half
    tail[e] = qkv[2 * kHidden + e];
  }
  // the next cache: every block of this head copied (unless in place), the
  // new row and the new length in the last block
  for (int b = 0; b < blocks; ++b) {
    const size_t base = ((size_t)b * kKvHeads + h) * he;
    const bool last = b == blocks - 1;
    for (int i = t; i < he; i += blockDim.x) {
      uint16_t v;
      if (past == nullptr) {
        v = 0;
      } else {
        if (next == past) continue;
        v = past[base + i];
      }
      next[base + i] = v;
    }
    __syncthreads();
    if (last) {
      if (t == 0) next[base] = f32_to_bf16((float)(last_len + 1));
      if (t < kHeadDim) {
        next[base + 2 + (size_t)last_len * kHeadDim + t] = qkv[kHidden + h * kHeadDim + t];
        next[base + 2 + (size_t)(cap + last_len) * kHeadDim + t] = qkv[kHidden + kKvHeads * kHeadDim + h * kHeadDim + t];
      }
    }
  }
}

// Position 0: the softmax over one key is 1, so each query head's context is
// its KV head's value. first_cache = per KV head [key (64) | value (64)];
// tail = [hidden | context] (kernels/lfm25_attention_first_context.cc).
__global__ void k_attention_first(const uint16_t* __restrict__ qkv, uint16_t* __restrict__ tail,
                                  uint16_t* __restrict__ first_cache) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;  // 0 .. 1023
  if (i >= kHidden) return;
  const int h = i / (2 * kHeadDim), d = i % (2 * kHeadDim);
  const uint16_t v = d < kHeadDim ? qkv[kHidden + h * kHeadDim + d] : qkv[kHidden + kKvHeads * kHeadDim + h * kHeadDim + d - kHeadDim];
  first_cache[i] = v;
  const int hq = i / kHeadDim, dd = i % kHeadDim;
  tail[kHidden + i] = qkv[kHidden + kKvHeads * kHeadDim + (hq / 2) * kHeadDim + dd];
  tail[i] = qkv[2 * kHidden + i];
}

// ------------------------------------------------------------------ packing

// Up to four copies (src NULL: zeros) in one launch.
struct Segments {
  const uint16_t* src[4];
  uint16_t* dst[4];
  int n[4];
};
__global__ void k_segments(Segments s, int count) {
  for (int k = 0; k < count; ++k)
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < s.n[k]; i += gridDim.x * blockDim.x)
      s.dst[k][i] = s.src[k] != nullptr ? s.src[k][i] : (uint16_t)0;
}

int run_segments(const Segments& s, int count, hipStream_t st, const char* what) {
  int most = 0;
  for (int k = 0; k < count; ++k) most = s.n[k] > most ? s.n[k] : most;
  k_segments<<<(most + 255) / 256, 256, 0, st>>>(s, count);
  return check_launch(what);
}

// ------------------------------------------------------------------ BF16 x BF16 -> FP32 product

// C[M x N] = A[M x K] . B[K x N], all row-major, FP32 sums in k order. A
// block computes a 16 x 64 tile of C with 256 threads (4 outputs each), the
// A and B tiles staged through LDS 64 k at a time.
constexpr int kMmM = 16, kMmN = 64, kMmK = 64;
__global__ void __launch_bounds__(256) k_bf16_f32_matmul(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                                         float* __restrict__ c, int M, int K, int N) {
  __shared__ float sa[kMmM][kMmK + 1];
  __shared__ float sb[kMmK][kMmN + 1];
  const int t = threadIdx.x;
  const int m0 = blockIdx.y * kMmM, n0 = blockIdx.x * kMmN;
  const int row = t / 16, col = (t % 16) * 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < K; k0 += kMmK) {
    for (int e = t; e < kMmM * kMmK; e += 256) sa[e / kMmK][e % kMmK] = bf16_to_f32(a[(size_t)(m0 + e / kMmK) * K + k0 + e % kMmK]);
    for (int e = t; e < kMmK * kMmN; e += 256) sb[e / kMmN][e % kMmN] = bf16_to_f32(b[(size_t)(k0 + e / kMmN) * N + n0 + e % kMmN]);
    __syncthreads();
    for (int k = 0; k < kMmK; ++k) {
      const float x = sa[row][k];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = fmaf(x, sb[k][col + j], acc[j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) c[(size_t)(m0 + row) * N + n0 + col + j] = acc[j];
}

}  // namespace
}  // namespace lfm25

using namespace lfm25;

extern "C" {

int lfm25_attention_first_context(const uint16_t* qkv_and_hidden, uint16_t* packed_tail_input, uint16_t* first_cache,
                                  lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv_and_hidden && packed_tail_input && first_cache, "attention_first_context: null pointer");
  k_attention_first<<<kHidden / 256, 256, 0, stream>>>(qkv_and_hidden, packed_tail_input, first_cache);
  return check_launch("attention_first_context");
}

int lfm25_attention_fixed(const uint16_t* qkv_and_hidden, const uint16_t* past_cache, uint16_t* packed_tail_input,
                          uint16_t* next_cache, int32_t capacity, int32_t blocks, int32_t* status,
                          lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv_and_hidden && packed_tail_input && next_cache, "attention_fixed: null pointer");
  LFM25_REQUIRE(capacity == 32 || capacity == 64, "attention_fixed: capacity must be 32 or 64, got %d", capacity);
  LFM25_REQUIRE(blocks >= 1 && blocks <= kMaxBlocks && (blocks == 1 || capacity == 64),
                "attention_fixed: blocks must be 1, or 1..%d of capacity 64, got %d", kMaxBlocks, blocks);
  LFM25_REQUIRE(past_cache != nullptr || blocks == 1, "attention_fixed: a chunked cache needs past_cache");
  LFM25_REQUIRE((reinterpret_cast<uintptr_t>(past_cache) & 3u) == 0 &&
                    (reinterpret_cast<uintptr_t>(next_cache) & 3u) == 0,
                "attention_fixed: caches must be 4-byte aligned");
  LFM25_REQUIRE(past_cache == nullptr || past_cache == next_cache ||
                    past_cache + (size_t)blocks * kKvHeads * head_elems(capacity) <= next_cache ||
                    next_cache + (size_t)blocks * kKvHeads * head_elems(capacity) <= past_cache,
                "attention_fixed: next_cache must be past_cache or not overlap it");
  k_attention_headered<<<kKvHeads, kAttnThreads, 0, stream>>>(qkv_and_hidden, past_cache, packed_tail_input,
                                                              next_cache, capacity, blocks, status);
  return check_launch("attention_fixed");
}

int lfm25_pack_block_input(const uint16_t* hidden, const uint16_t* state_and_weight, uint16_t* packed,
                           lfm25_stream_t stream) {
  LFM25_REQUIRE(hidden && state_and_weight && packed, "pack_block_input: null pointer");
  Segments s{{hidden, nullptr, state_and_weight}, {packed, packed + kHidden, packed + 6144}, {kHidden, 6144 - kHidden, 6144}};
  return run_segments(s, 3, stream, "pack_block_input");
}

int lfm25_pack_conv(const uint16_t* projection, const uint16_t* weight, uint16_t* packed, lfm25_stream_t stream) {
  LFM25_REQUIRE(projection && weight && packed, "pack_conv: null pointer");
  Segments s{{projection, weight}, {packed, packed + 3 * kHidden}, {3 * kHidden, 3 * kHidden}};
  return run_segments(s, 2, stream, "pack_conv");
}

int lfm25_pack_attention_tail(const uint16_t* hidden, const uint16_t* context, uint16_t* packed,
                              lfm25_stream_t stream) {
  LFM25_REQUIRE(hidden && context && packed, "pack_attention_tail: null pointer");
  Segments s{{hidden, context}, {packed, packed + kHidden}, {kHidden, kHidden}};
  return run_segments(s, 2, stream, "pack_attention_tail");
}

int lfm25_concat_hidden_pair(const uint16_t* first, const uint16_t* second, uint16_t* pair, lfm25_stream_t stream) {
  LFM25_REQUIRE(first && second && pair, "concat_hidden_pair: null pointer");
  Segments s{{first, second}, {pair, pair + kHidden}, {kHidden, kHidden}};
  return run_segments(s, 2, stream, "concat_hidden_pair");
}

int lfm25_split_hidden_pair(const uint16_t* pair, uint16_t* first, uint16_t* second, lfm25_stream_t stream) {
  LFM25_REQUIRE(pair && first && second, "split_hidden_pair: null pointer");
  Segments s{{pair, pair + kHidden}, {first, second}, {kHidden, kHidden}};
  return run_segments(s, 2, stream, "split_hidden_pair");
}

int lfm25_pack_recurrent_pair(const uint16_t* pair, const uint16_t* state_and_weight, uint16_t* packed,
                              lfm25_stream_t stream) {
  LFM25_REQUIRE(pair && state_and_weight && packed, "pack_recurrent_pair: null pointer");
  // [h0 | zeros to 6144 | h1 | zeros to 12288 | state and weight (6144)]
  Segments s{{pair, nullptr, pair + kHidden, nullptr},
             {packed, packed + kHidden, packed + 6144, packed + 6144 + kHidden},
             {kHidden, 6144 - kHidden, kHidden, 6144 - kHidden}};
  const int rc = run_segments(s, 4, stream, "pack_recurrent_pair");
  if (rc != LFM25_OK) return rc;
  Segments t{{state_and_weight}, {packed + 12288}, {6144}};
  return run_segments(t, 1, stream, "pack_recurrent_pair");
}

int lfm25_bf16_f32_matmul(const uint16_t* a, const uint16_t* b, float* c, int32_t M, int32_t K, int32_t N,
                          lfm25_stream_t stream) {
  LFM25_REQUIRE(a && b && c, "bf16_f32_matmul: null pointer");
  LFM25_REQUIRE(M >= kMmM && M % kMmM == 0 && K >= kMmK && K % kMmK == 0 && N >= kMmN && N % kMmN == 0,
                "bf16_f32_matmul: needs M %% 16 == 0, K %% 64 == 0, N %% 64 == 0, got %d x %d x %d", M, K, N);
  k_bf16_f32_matmul<<<dim3(N / kMmN, M / kMmM), 256, 0, stream>>>(a, b, c, M, K, N);
  return check_launch("bf16_f32_matmul");
}

}  // extern "C"
