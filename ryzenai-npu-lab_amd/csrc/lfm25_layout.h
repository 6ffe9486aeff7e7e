// Layout of the packed LFM2.5 weight stream: every tensor of every layer in
// layer order, each on a 128-element boundary, then the final norm. The
// layer order and each layer's tensor order follow the model
// (experiments/lfm25_x8.py:55-57 for the kinds; modeling_lfm2.py for the
// tensors), so the stream is built from an HF checkpoint by concatenation.
#pragma once
#include <cstdint>

#include "lfm25_hip.h"
#include "lfm25_device.h"

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

// The q, k and v matrices of an attention layer are placed back to back
// (their sizes are multiples of the 128-element alignment), so q/k/v row r is
// row r of one 2048 x 1024 matrix starting at the q slot.
static_assert((1LL * kHidden * kHidden) % 128 == 0 && (512LL * kHidden) % 128 == 0,
              "q/k/v stay contiguous in the packed stream");

// Elements of tensor `slot` of layer l (l == kLayers: the final norm).
__host__ __device__ constexpr int64_t tensor_elems(int l, int slot) {
  if (l == kLayers) return kHidden;
  if (is_attn(l)) {
    switch (slot) {
      case A_OPNORM: case A_FFNNORM: return kHidden;
      case A_Q: case A_O: return 1LL * kHidden * kHidden;
      case A_K: case A_V: return 512LL * kHidden;
      case A_QLN: case A_KLN: return kHeadDim;
      case A_W1: case A_W3: return 1LL * kFfn * kHidden;
      default: return 1LL * kHidden * kFfn;  // A_W2
    }
  }
  switch (slot) {
    case C_OPNORM: case C_FFNNORM: return kHidden;
    case C_IN: return 3LL * kHidden * kHidden;
    case C_CONVW: return 3LL * kHidden;
    case C_OUT: return 1LL * kHidden * kHidden;
    case C_W1: case C_W3: return 1LL * kFfn * kHidden;
    default: return 1LL * kHidden * kFfn;  // C_W2
  }
}
__host__ __device__ constexpr int tensor_count(int l) {
  return l == kLayers ? 1 : is_attn(l) ? A_COUNT : C_COUNT;
}
__host__ __device__ constexpr int64_t align128(int64_t n) { return (n + 127) / 128 * 128; }
// Start (in elements) of tensor `slot` of layer l in the packed stream: every
// tensor of every layer in order, each on a 128-element boundary, then the
// final norm (l == kLayers, slot 0).
__host__ __device__ constexpr int64_t tensor_off(int l, int slot) {
  int64_t at = 0;
  for (int i = 0; i < l; ++i)
    for (int t = 0; t < tensor_count(i); ++t) at += align128(tensor_elems(i, t));
  for (int t = 0; t < slot; ++t) at += align128(tensor_elems(l, t));
  return at;
}
constexpr int64_t kStreamElems = tensor_off(kLayers, 1);
constexpr int kStreamTensors = 8 * LFM25_CONV_LAYERS + 11 * LFM25_ATTN_LAYERS + 1;

// Elements of a whole conv / attention layer and the start of tensor `slot`
// within its layer; every layer starts at
// (conv layers before it) * kConvLayerElems + (attention layers before it) *
// kAttnLayerElems, so a runtime layer index costs two multiply-adds.
__host__ __device__ constexpr int64_t slot_off(bool attn, int slot) {
  return tensor_off(attn ? 2 : 0, slot) - tensor_off(attn ? 2 : 0, 0);
}
constexpr int64_t kConvLayerElems = tensor_off(1, 0);
constexpr int64_t kAttnLayerElems = tensor_off(3, 0) - tensor_off(2, 0);
__host__ __device__ constexpr int64_t layer_off(int l) {
  return conv_before(l) * kConvLayerElems + (l - conv_before(l)) * kAttnLayerElems;
}
static_assert(layer_off(13) == tensor_off(13, 0) && layer_off(14) == tensor_off(14, 0) &&
                  layer_off(6) == tensor_off(6, 0) && layer_off(5) == tensor_off(5, 0),
              "closed-form layer offsets");
static_assert(slot_off(true, A_W2) == tensor_off(12, A_W2) - tensor_off(12, 0) &&
                  slot_off(false, C_W2) == tensor_off(13, C_W2) - tensor_off(13, 0),
              "slot offsets are the same in every layer of a kind");

// Tensor of layer l (from a laundered stream base) whose slot depends only on
// the layer's kind: conv slot kConv or attention slot kAttn. The slot offsets
// are compile-time constants, so a runtime layer index costs a select.
template <int kConv, int kAttn>
__device__ __forceinline__ const uint16_t* layer_tensor(const uint16_t* w, int l) {
  constexpr int64_t oc = slot_off(false, kConv), oa = slot_off(true, kAttn);
  return w + layer_off(l) + (is_attn(l) ? oa : oc);
}
template <int kAttn>
__device__ __forceinline__ const uint16_t* attn_tensor(const uint16_t* w, int l) {
  constexpr int64_t oa = slot_off(true, kAttn);
  return w + layer_off(l) + oa;
}
template <int kConv>
__device__ __forceinline__ const uint16_t* conv_tensor(const uint16_t* w, int l) {
  constexpr int64_t oc = slot_off(false, kConv);
  return w + layer_off(l) + oc;
}
__device__ __forceinline__ const uint16_t* final_norm(const uint16_t* w) { return w + layer_off(kLayers); }
static_assert(layer_off(kLayers) == tensor_off(kLayers, 0), "final norm offset");

// ------------------------------------------------------------------ 8-bit weights (w8g32)
//
// The projections of every layer in the reference's w8g32 format
// (experiments/014_int8_lfm25.py:76-93 with bits 8, group 32): int8 q [M x K]
// row-major, then FP32 scales [M x K / 32], each region on a 256-byte
// boundary. Projections of a layer, in order: the mixer (conv: in_proj
// [3072 x 1024]; attention: q | k | v as one [2048 x 1024] matrix), its output
// projection (out_proj / o_proj [1024 x 1024]), w1, w3 [2560 x 1024], w2
// [1024 x 2560]. Norms, conv taps and QK-norm weights stay BF16 (as in the
// reference's study) and are read from the BF16 stream.
enum W8Proj { P_MIX, P_OUT, P_W1, P_W3, P_W2, P_COUNT };
constexpr int kW8Group = 32;
__host__ __device__ constexpr int w8_rows(bool attn, int p) {
  return p == P_MIX ? (attn ? 2 * kHidden : 3 * kHidden) : (p == P_OUT || p == P_W2) ? kHidden : kFfn;
}
__host__ __device__ constexpr int w8_cols(int p) { return p == P_W2 ? kFfn : kHidden; }
__host__ __device__ constexpr int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }
__host__ __device__ constexpr int64_t w8_q_bytes(bool attn, int p) { return (int64_t)w8_rows(attn, p) * w8_cols(p); }
__host__ __device__ constexpr int64_t w8_s_bytes(bool attn, int p) {
  return (int64_t)w8_rows(attn, p) * (w8_cols(p) / kW8Group) * 4;
}
__host__ __device__ constexpr int64_t w8_proj_bytes(bool attn, int p) {
  return align256(w8_q_bytes(attn, p)) + align256(w8_s_bytes(attn, p));
}
// Byte offset of projection p's q within a layer of the kind.
__host__ __device__ constexpr int64_t w8_slot_q(bool attn, int p) {
  int64_t at = 0;
  for (int i = 0; i < p; ++i) at += w8_proj_bytes(attn, i);
  return at;
}
__host__ __device__ constexpr int64_t w8_slot_s(bool attn, int p) { return w8_slot_q(attn, p) + align256(w8_q_bytes(attn, p)); }
constexpr int64_t kW8ConvLayerBytes = w8_slot_q(false, P_COUNT);
constexpr int64_t kW8AttnLayerBytes = w8_slot_q(true, P_COUNT);
__host__ __device__ constexpr int64_t w8_layer_off(int l) {
  return conv_before(l) * kW8ConvLayerBytes + (l - conv_before(l)) * kW8AttnLayerBytes;
}
constexpr int64_t kW8LayersBytes = w8_layer_off(kLayers);
// Rows per group of 32 scales of the tied table ([vocab x 1024] int8, [vocab x 32] FP32).
constexpr int kW8RowScales = kHidden / kW8Group;

// Projection kProj of layer l: q rows and their scales.
template <int kProj>
__device__ __forceinline__ const int8_t* w8_q(const int8_t* w8, int l) {
  constexpr int64_t oc = w8_slot_q(false, kProj), oa = w8_slot_q(true, kProj);
  return w8 + w8_layer_off(l) + (is_attn(l) ? oa : oc);
}
template <int kProj>
__device__ __forceinline__ const float* w8_s(const int8_t* w8, int l) {
  constexpr int64_t oc = w8_slot_s(false, kProj), oa = w8_slot_s(true, kProj);
  return reinterpret_cast<const float*>(w8 + w8_layer_off(l) + (is_attn(l) ? oa : oc));
}

}  // namespace lfm25
