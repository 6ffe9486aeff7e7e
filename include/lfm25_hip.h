/*
 * lfm25_hip.h - C ABI of the MI355X (gfx950) LFM2.5-230M decode hot path.
 *
 * Every entry point takes caller-owned DEVICE pointers, plain sizes and a HIP
 * stream, enqueues its kernels on that stream and returns without waiting.
 * BF16 tensors are passed as uint16_t bit patterns. Return value: LFM25_OK
 * (0), LFM25_EINVAL (bad shape / null or misaligned pointer; nothing was
 * launched) or LFM25_EDEVICE (the HIP runtime refused a launch);
 * lfm25_last_error() describes the last failure of the calling thread.
 * Vectors read with 128-bit loads must be 16-byte aligned.
 *
 * Rounding follows the reference's CPU PyTorch BF16 path: FP32 arithmetic,
 * one round-to-nearest-even BF16 step at every model rounding point.
 *
 * Each function names the reference symbol or entry point it replaces
 * (paths relative to the reference repository's experiments/ directory).
 */
#ifndef LFM25_HIP_H
#define LFM25_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t* lfm25_stream_t;

#define LFM25_OK 0
#define LFM25_EINVAL 1
#define LFM25_EDEVICE 2

#define LFM25_HIDDEN 1024
#define LFM25_FFN 2560
#define LFM25_VOCAB 65536
#define LFM25_HEADS 16
#define LFM25_KV_HEADS 8
#define LFM25_HEAD_DIM 64
#define LFM25_LAYERS 14
#define LFM25_CONV_LAYERS 8
#define LFM25_ATTN_LAYERS 6
#define LFM25_MAX_CAPACITY 4096

/* Library version (major*10000 + minor*100 + patch). */
int lfm25_version(void);

/* Message for the last non-OK return on the calling thread. */
const char* lfm25_last_error(void);

/* ---------------------------------------------------------------- per-op
 * One function per reference operation (the @iron.jit entry points of
 * lfm25_*_kernel.py and the AIE kernels behind them).
 */

/* y = bf16(bf16(x * rsqrt(mean(x^2) + 1e-5)) * gamma), 1 <= cols <= 65536.
 * Replaces kernels/lfm25_rms_norm.cc:21-41 (lfm25_rms_norm) and the entry
 * rms_norm(input0, gamma0, output, *, N) of lfm25_rms_norm_kernel.py:16-53. */
int lfm25_rms_norm(const uint16_t* input, const uint16_t* gamma, uint16_t* output, int32_t cols,
                   lfm25_stream_t stream);

/* output[M] = bf16(W[M x K] . activation[K]), FP32 accumulation; K % 8 == 0.
 * Replaces entry bf16_bf16_gemv(weights, activation, output, *, M, K, n_cores)
 * of lfm25_bf16_gemv_kernel.py:18-114 (kernels/lfm25_bf16_gemv.cc:7-19 +
 * kernels/lfm25_f32_to_bf16.cc:8-14). */
int lfm25_bf16_bf16_gemv(const uint16_t* weights, const uint16_t* activation, uint16_t* output,
                         int32_t M, int32_t K, lfm25_stream_t stream);

/* output[M] = W[M x K] . activation[K] in FP32 (no rounding); K % 8 == 0.
 * Replaces entry bf16_f32_gemv of lfm25_gemv_kernel.py:21-109. */
int lfm25_bf16_f32_gemv(const uint16_t* weights, const uint16_t* activation, float* output,
                        int32_t M, int32_t K, lfm25_stream_t stream);

/* Fused RMSNorm + GEMV: output = bf16(W . rms_norm(hidden, gamma)), K == 1024.
 * packed_gamma_and_weight = [gamma (1024) | zero pad to 4096 | W row-major
 * M x 1024], the layout of 006_lfm25_npu_norm_gemv.py:26-28.
 * Replaces entry norm_bf16_gemv(hidden, packed_gamma_and_weight, output, *, M, K)
 * of lfm25_norm_gemv_kernel.py:18-122. */
int lfm25_norm_bf16_gemv(const uint16_t* hidden, const uint16_t* packed_gamma_and_weight,
                         uint16_t* output, int32_t M, int32_t K, lfm25_stream_t stream);

/* INT8-weight GEMV in the reference's 8-bit formats (experiments/
 * 014_int8_lfm25.py:76-113, class Weight): output[M] = bf16(sum_k
 * activation[k] * weights[m][k] * scales[m][k / group]), FP32 sums, with
 * weights int8 [M x K] row-major (16-byte aligned) and scales FP32
 * [M x K / group] for group 32 or 64 (w8g32 / w8g64), or FP32 [M] for
 * group 0 (w8c: one scale per row, applied after the sum). K % 64 == 0,
 * K <= 4096. The reference evaluates these formats on the CPU only
 * (Weight.linear, :99-105); this is the decode-side product they need. */
int lfm25_w8_gemv(const int8_t* weights, const float* scales, const uint16_t* activation, uint16_t* output,
                  int32_t M, int32_t K, int32_t group, lfm25_stream_t stream);

/* output = bf16(input), round to nearest even.
 * Replaces kernels/lfm25_f32_to_bf16.cc:8-14 (entry f32_to_bf16,
 * lfm25_cast_kernel.py:16-45). */
int lfm25_f32_to_bf16(const float* input, uint16_t* output, int32_t count, lfm25_stream_t stream);

/* output = bf16(left + right).
 * Replaces kernels/lfm25_bf16_add.cc:7-15 (entry bf16_add, lfm25_add_kernel.py:16-53). */
int lfm25_bf16_add(const uint16_t* left, const uint16_t* right, uint16_t* output, int32_t count,
                   lfm25_stream_t stream);

/* output = bf16(bf16(silu(w1)) * w3), SiLU in FP32.
 * Replaces kernels/lfm25_silu_gate.cc:22-39 (entry silu_gate,
 * lfm25_silu_gate_kernel.py:16-51). */
int lfm25_silu_gate(const uint16_t* w1, const uint16_t* w3, uint16_t* output, int32_t count,
                    lfm25_stream_t stream);

/* One-token gated short convolution over 1024 channels.
 * projection_and_weight = [B (1024) | C (1024) | x (1024) | w (1024 x 3)],
 * previous_state / next_state = HF conv state [1024 x 3].
 * Replaces kernels/lfm25_conv_gate.cc:8-43 (entry conv_gate,
 * lfm25_conv_gate_kernel.py:16-73). */
int lfm25_conv_gate(const uint16_t* projection_and_weight, const uint16_t* previous_state,
                    uint16_t* gated_output, uint16_t* next_state, lfm25_stream_t stream);

/* As lfm25_conv_gate with state_and_weight = [state (1024 x 3) | w (1024 x 3)];
 * next_state_and_weight receives [new state | w].
 * Replaces kernels/lfm25_conv_gate_packed_state.cc:8-45 (entry
 * conv_gate_packed_state, lfm25_conv_gate_packed_state_kernel.py:16-63). */
int lfm25_conv_gate_packed_state(const uint16_t* projection, const uint16_t* state_and_weight,
                                 uint16_t* gated_output, uint16_t* next_state_and_weight,
                                 lfm25_stream_t stream);

/* In place on qkv = [q (16 x 64) | k (8 x 64) | v (8 x 64)]: per-head RMSNorm
 * (eps 1e-5) of the 24 q and k heads then RoPE.
 * aux = [q_gamma (64) | k_gamma (64) | cos (64) | sin (64)].
 * Replaces kernels/lfm25_attention_norm_rope.cc:17-54. */
int lfm25_attention_norm_rope(uint16_t* qkv, const uint16_t* aux, lfm25_stream_t stream);

/* Decode attention for all 8 KV heads, q/k already normalised and rotated.
 * qkv = [q | k | v] of the current position (2048 values); past_cache per
 * KV head h at h * 2 * past_length * 64: [keys (past_length x 64) |
 * values (past_length x 64)]; context [16 x 64]. 0 <= past_length < 4096.
 * Replaces kernels/lfm25_attention_context_head.cc:19-82
 * (lfm25_attention_context_head_dynamic; entry attention_context,
 * lfm25_attention_context_kernel.py:20-72). */
int lfm25_attention_context(const uint16_t* qkv, const uint16_t* past_cache, uint16_t* context,
                            int32_t past_length, lfm25_stream_t stream);

/* next_cache (per head: keys (past_length+1) x 64 | values) = prior cache with
 * the current key/value of qkv appended.
 * Replaces kernels/lfm25_attention_append_cache.cc:5-39
 * (lfm25_attention_append_cache_dynamic; entry append_attention_cache). */
int lfm25_attention_append_cache(const uint16_t* qkv, const uint16_t* prior_cache,
                                 uint16_t* next_cache, int32_t past_length, lfm25_stream_t stream);

/* Position 0 of a prompt: softmax over one key gives its value. From
 * qkv_and_hidden = [q (1024) | k (512) | v (512) | hidden (1024)] (q and k
 * normed and rotated): first_cache = per KV head [key (64) | value (64)],
 * packed_tail_input = [hidden | context (1024)].
 * Replaces kernels/lfm25_attention_first_context.cc (entry
 * attention_first_context, experiments/lfm25_attention_first_context_kernel.py:16-17). */
int lfm25_attention_first_context(const uint16_t* qkv_and_hidden, uint16_t* packed_tail_input,
                                  uint16_t* first_cache, lfm25_stream_t stream);

/* Attention over the reference's headered cache layouts. A head region is
 * 2 + 2 * capacity * 64 BF16 values: element 0 = its filled length (as a BF16
 * number), then `capacity` key rows, then `capacity` value rows; a cache is 8
 * regions (one per KV head), a chunked cache `blocks` such caches of capacity
 * 64, positions in block order, the new one appended to the last block.
 * past_cache NULL = the first position (the next cache starts empty). Writes
 * packed_tail_input = [hidden | context] and next_cache = the cache with the
 * current key / value appended (next_cache may be past_cache). Eager
 * attention with BF16 probabilities, as lfm25_attention_context. A length
 * the layout cannot hold sets *status bit 0 (status may be NULL) and leaves
 * that head unwritten.
 * Replaces kernels/lfm25_attention_fixed_head.cc (capacity 32; entries
 * attention_first_fixed / attention_context_fixed,
 * experiments/lfm25_attention_fixed_cache_kernel.py:30-31,81-82),
 * kernels/lfm25_attention_fixed64_head.cc (capacity 64; attention_first_fixed64 /
 * attention_context_fixed64, lfm25_attention_fixed64_cache_kernel.py:31,82) and
 * kernels/lfm25_attention_chunked_head.cc (blocks > 1; attention_context_chunked,
 * lfm25_attention_chunked_cache_kernel.py:22-24). */
int lfm25_attention_fixed(const uint16_t* qkv_and_hidden, const uint16_t* past_cache, uint16_t* packed_tail_input,
                          uint16_t* next_cache, int32_t capacity, int32_t blocks, int32_t* status,
                          lfm25_stream_t stream);

/* packed[12288] = [hidden (1024) | zeros to 6144 | state_and_weight (6144)].
 * Replaces kernels/lfm25_pack_block_input.cc (entry pack_block_input,
 * experiments/lfm25_pack_block_input_kernel.py:17). */
int lfm25_pack_block_input(const uint16_t* hidden, const uint16_t* state_and_weight, uint16_t* packed,
                           lfm25_stream_t stream);

/* packed[6144] = [projection (3072) | weight (3072)].
 * Replaces kernels/lfm25_pack_conv.cc (entry pack_conv,
 * experiments/lfm25_pack_conv_kernel.py:17). */
int lfm25_pack_conv(const uint16_t* projection, const uint16_t* weight, uint16_t* packed, lfm25_stream_t stream);

/* packed[2048] = [hidden (1024) | context (1024)].
 * Replaces kernels/lfm25_pack_attention_tail.cc (entry pack_attention_tail,
 * experiments/lfm25_pack_attention_tail_kernel.py:17). */
int lfm25_pack_attention_tail(const uint16_t* hidden, const uint16_t* context, uint16_t* packed,
                              lfm25_stream_t stream);

/* pair = [first | second], and back; packed[18432] = [first | zeros to 6144 |
 * second | zeros to 12288 | state_and_weight (6144)]. Replace the two-position
 * prompt programs concat_hidden_pair, split_hidden_pair and
 * pack_recurrent_pair (experiments/lfm25_prefill_pair_data_kernel.py:11,42,73). */
int lfm25_concat_hidden_pair(const uint16_t* first, const uint16_t* second, uint16_t* pair, lfm25_stream_t stream);
int lfm25_split_hidden_pair(const uint16_t* pair, uint16_t* first, uint16_t* second, lfm25_stream_t stream);
int lfm25_pack_recurrent_pair(const uint16_t* pair, const uint16_t* state_and_weight, uint16_t* packed,
                              lfm25_stream_t stream);

/* c[M x N] (FP32) = a[M x K] . b[K x N] (BF16, row-major), FP32 sums;
 * M % 16 == 0, K % 64 == 0, N % 64 == 0.
 * Replaces entry bf16_f32_matmul (experiments/lfm25_matmul_kernel.py:16-27). */
int lfm25_bf16_f32_matmul(const uint16_t* a, const uint16_t* b, float* c, int32_t M, int32_t K, int32_t N,
                          lfm25_stream_t stream);

/* Bytes of device workspace lfm25_argmax / lfm25_fused_vocab need for `count` rows. */
size_t lfm25_argmax_workspace_bytes(int32_t count);

/* token_id[0] = first index of the maximum BF16 logit (count % 4 == 0).
 * Replaces kernels/lfm25_argmax_chunk.cc:5-20 (entry vocab_argmax,
 * lfm25_argmax_kernel.py:18-68). */
int lfm25_argmax(const uint16_t* logits, int32_t count, int32_t* token_id, void* workspace,
                 lfm25_stream_t stream);

/* Final RMSNorm, tied-head logits bf16(E . n), argmax (first maximum) and the
 * winning embedding row. packed_gamma_and_embedding = [gamma (1024) |
 * E (vocab x 1024)]; vocab % 4 == 0. logits may be NULL.
 * Replaces entry fused_vocab(hidden, packed_gamma_and_embedding, next_embedding,
 * token_id) of lfm25_fused_vocab_kernel.py:22-110 (kernels
 * lfm25_vocab_score_keep_row.cc, lfm25_vocab_pack_candidate.cc,
 * lfm25_vocab_accept_candidate.cc). */
int lfm25_fused_vocab(const uint16_t* hidden, const uint16_t* packed_gamma_and_embedding,
                      uint16_t* next_embedding, int32_t* token_id, uint16_t* logits,
                      int32_t vocab, void* workspace, lfm25_stream_t stream);

/* lfm25_fused_vocab without a workspace argument: the per-block candidates
 * live in a static device array of the library (8 KB per GPU, held until the
 * process ends), so the call allocates nothing. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops). vocab % 4 == 0 and vocab <= 65536
 * (LFM25_EINVAL otherwise). Calls that overlap on one GPU race on the array. */
int lfm25_fused_vocab_static(const uint16_t* hidden, const uint16_t* packed_gamma_and_embedding,
                             uint16_t* next_embedding, int32_t* token_id, uint16_t* logits, int32_t vocab,
                             lfm25_stream_t stream);

/* embedding[1024] = table[token_id[0]] with the id read from device memory
 * (ids outside [0, vocab) are clamped and flagged in *status when non-NULL).
 * Replaces entries embedding_dma (lfm25_embedding_dma_kernel.py:11-39) and
 * embedding_dma_dynamic (lfm25_embedding_dynamic_kernel.py:22-68). */
int lfm25_embedding_gather(const uint16_t* table, const int32_t* token_id, uint16_t* embedding,
                           int32_t vocab, int32_t* status, lfm25_stream_t stream);

/* ---------------------------------------------------------------- decoder
 * The whole-token step behind the X8Model layer/step API
 * (lfm25_x8_model.py:33-148): embedding gather, 14 layers in the order
 * conv,conv,attn,conv,attn,conv,attn,conv,attn,conv,attn,conv,attn,conv
 * (lfm25_x8.py:55-57), final norm, tied head and argmax.
 *
 * Packed weight stream (BF16, lfm25_weights_elems() values): per layer, in
 * order, each tensor row-major as in the HF checkpoint and starting on a
 * 128-element boundary (lfm25_weights_offsets() lists every start):
 *   conv layer: operator_norm (1024), in_proj (3072 x 1024), conv (1024 x 3),
 *               out_proj (1024 x 1024), ffn_norm (1024), w1 (2560 x 1024),
 *               w3 (2560 x 1024), w2 (1024 x 2560)
 *   attn layer: operator_norm, q_proj (1024 x 1024), k_proj (512 x 1024),
 *               v_proj (512 x 1024), q_layernorm (64), k_layernorm (64),
 *               out_proj (1024 x 1024), ffn_norm, w1, w3, w2
 *   then embedding_norm (1024).
 * The embedding table [vocab x 1024] is separate (tied with the head).
 */

#define LFM25_TENSORS_PER_CONV 8
#define LFM25_TENSORS_PER_ATTN 11

typedef struct lfm25_decoder {
  const uint16_t* weights;    /* packed weight stream */
  const uint16_t* embedding;  /* [vocab x 1024] */
  const uint16_t* rope;       /* [capacity x 128]: bf16 cos (64) | sin (64) per position */
  uint16_t* conv_state;       /* [8 x 1024 x 3], HF layout */
  uint16_t* key_cache;        /* [6 x 8 x capacity x 64], 128-byte aligned */
  uint16_t* value_cache;      /* [6 x 8 x capacity x 64], 128-byte aligned */
  void* workspace;            /* lfm25_decoder_workspace_bytes() bytes, 256-byte aligned */
  int32_t capacity;           /* KV positions, 1..4096 */
  int32_t vocab;              /* rows of the embedding table, % 4 == 0 */
} lfm25_decoder;

/* Number of BF16 values in the packed weight stream. */
size_t lfm25_weights_elems(void);

/* Start offsets (in elements) of every tensor of the packed stream, in stream
 * order: 8 or 11 per layer then embedding_norm. Writes min(n, total) values
 * and returns the total number of tensors. */
int32_t lfm25_weights_offsets(int64_t* offsets, int32_t n);

size_t lfm25_decoder_workspace_bytes(void);

/* 1 when the persistent decode on the current device exchanges activations
 * inside each XCD through its L2 (blocks land on XCD blockIdx % 8, checked
 * once per device), 0 when it uses cross-XCD-coherent exchanges everywhere
 * (same results; forced by LFM25_XCD_LOCAL=0 in the environment), -1 when the
 * device cannot run the persistent decode. No counterpart in the reference
 * (an NPU has no XCDs); it lets callers and tests see which variant runs. */
int32_t lfm25_decode_exchange(void);

/* One-time set-up of the persistent decode on the current device: checks
 * that a cooperative launch of 256 blocks x 512 threads fits there, and runs
 * the placement probe behind lfm25_decode_exchange (one cooperative launch
 * on a private stream into a 1 KB device buffer; buffer and stream are
 * released before it returns). lfm25_decode, lfm25_decode_w8,
 * lfm25_decode_layer and lfm25_decode_exchange run it themselves on their
 * first call on a device when the caller has not -- that first call then
 * allocates and synchronizes -- so callers that capture streams or may not
 * allocate call lfm25_init once per device beforehand (X8Model does so in
 * its constructor). Returns LFM25_OK or LFM25_EDEVICE. No counterpart in
 * the reference: its NPU runtime does its set-up when the program is
 * loaded (experiments/lfm25_x8_model.py:38-51). */
int lfm25_init(void);

/* Device control words inside the workspace (int32):
 * [0] position = tokens held in the caches, [1] current token,
 * [2] status flags (bit 0: token id out of range, bit 1: capacity reached,
 * bit 2: exchange time-out, bit 3: a block ran off its XCD). */
#define LFM25_CTL_POSITION 0
#define LFM25_CTL_TOKEN 1
#define LFM25_CTL_STATUS 2

/* Zero the conv states and set position = 0 (KV rows are overwritten before
 * they are read, so the caches are not cleared). */
int lfm25_decoder_reset(const lfm25_decoder* d, lfm25_stream_t stream);

/* Run n_in + max(n_gen - 1, 0) decode steps: the first n_in take their token
 * from tokens_in (device int32 [n_in]; NULL with n_in == 1 means "the token
 * held in the control word", i.e. the last one selected), the last of them
 * selects a token when n_gen > 0, and n_gen - 1 further steps each consume the
 * previously selected token. Selected ids go to tokens_out (device int32
 * [n_gen]); may be NULL when n_gen == 0.
 * exec: LFM25_EXEC_STAGED launches one kernel per stage (graph capturable),
 * LFM25_EXEC_PERSISTENT runs the steps in cooperative launches that keep the
 * grid across steps: one launch for a call of fewer than 8 steps, otherwise
 * one for the positions below 256 and one for the rest.
 * Positions beyond the capacity set status bit 1 and stop the run. */
#define LFM25_EXEC_STAGED 0
#define LFM25_EXEC_PERSISTENT 1
int lfm25_decode(const lfm25_decoder* d, const int32_t* tokens_in, int32_t n_in, int32_t n_gen,
                 int32_t* tokens_out, int32_t exec, lfm25_stream_t stream);

/* ------------------------------------------------------------ 8-bit weights
 *
 * The decode with every projection and the tied table in the reference's
 * w8g32 format (experiments/014_int8_lfm25.py:76-113, Weight with bits 8 and
 * group 32: int8 q and one FP32 scale per row and 32 inputs; the embedding
 * row is bf16(q s), Weight.rows :111-112). The reference evaluates this
 * format on the CPU only and names the decode it would need
 * (experiments/014_headroom_leads.md:405-420); this is that decode, on the
 * persistent kernel.
 *
 * layers: lfm25_w8_layers_bytes() bytes, 256-byte aligned: per layer, in
 * order, per projection -- conv: in_proj [3072 x 1024]; attention: q | k | v as
 * one [2048 x 1024] matrix -- then out_proj [1024 x 1024], w1, w3 [2560 x 1024],
 * w2 [1024 x 2560]: int8 q row-major, then FP32 scales [rows x cols / 32],
 * each on a 256-byte boundary (lfm25_w8_layers_offsets() lists every start:
 * q then scales, per projection, per layer).
 * table: [vocab x 1024] int8 and table_scales [vocab x 32] FP32 (tied:
 * embedding rows and the head).
 * The decoder's BF16 stream supplies the norms, conv taps and QK-norm
 * weights (its projection slots are not read); its embedding is not read. */
typedef struct lfm25_w8_model {
  const int8_t* layers;
  const int8_t* table;
  const float* table_scales;
} lfm25_w8_model;

size_t lfm25_w8_layers_bytes(void);
int32_t lfm25_w8_layers_offsets(int64_t* offsets, int32_t n);

/* lfm25_decode (persistent execution) with the 8-bit weights; same tokens,
 * control words, caches and errors. Replaces the per-token forward the
 * reference's INT8 study drives (experiments/014_int8_lfm25.py:158-199,
 * Model.forward / greedy). */
int lfm25_decode_w8(const lfm25_decoder* d, const lfm25_w8_model* w, const int32_t* tokens_in, int32_t n_in,
                    int32_t n_gen, int32_t* tokens_out, lfm25_stream_t stream);

/* ------------------------------------------------------------ one decoder layer
 *
 * One decode layer (conv or attention) of one token as one launch of 128
 * blocks (one per CU, which must be resident together: on an idle device they
 * are; otherwise the bounded waits end the call with status bit 2), with the
 * phases and exchanges of the persistent decode. Replaces
 * the reference's single-program layer entry point recurrent_block
 * (experiments/lfm25_single_program_block_kernel.py:32-284) and, for an
 * attention layer, the three calls attention_prefix -> attention_context_cache
 * -> attention_tail (experiments/006_lfm25_npu_layer_stack.py:181-190).
 * Tensor pointers may point anywhere (e.g. into the reference's packed
 * layouts); q, k and v must be one contiguous [2048 x 1024] matrix. */
#define LFM25_LAYER_CONV 0
#define LFM25_LAYER_ATTN 1
typedef struct lfm25_layer {
  int32_t kind;                   /* LFM25_LAYER_CONV or LFM25_LAYER_ATTN */
  const uint16_t* op_norm;        /* operator_norm [1024] */
  const uint16_t* mixer;          /* conv: in_proj [3072 x 1024]; attention: q | k | v [2048 x 1024] */
  const uint16_t* conv_weight;    /* conv: [1024 x 3] */
  const uint16_t* conv_state_in;  /* conv: HF state [1024 x 3] before the token */
  uint16_t* conv_state_out;       /* conv: the state after it (may equal conv_state_in) */
  const uint16_t* q_norm;         /* attention: q_layernorm [64] */
  const uint16_t* k_norm;         /* attention: k_layernorm [64] */
  uint16_t* key_cache;            /* attention: [8 x capacity x 64], 128-byte aligned */
  uint16_t* value_cache;          /* attention: [8 x capacity x 64], 128-byte aligned */
  const uint16_t* rope;           /* attention: [capacity x 128] cos (64) | sin (64) per position */
  int32_t capacity;               /* attention: KV positions, 1..4096 */
  const uint16_t* out;            /* conv out_proj / attention out_proj [1024 x 1024] */
  const uint16_t* ffn_norm;       /* [1024] */
  const uint16_t* w1;             /* [2560 x 1024] */
  const uint16_t* w3;             /* [2560 x 1024] */
  const uint16_t* w2;             /* [1024 x 2560] */
} lfm25_layer;

/* hidden_out[1024] = the layer applied to hidden_in[1024] at `position`
 * (attention: the token's key / value row is appended there and positions
 * [0, position] are attended; conv: conv_state_out gets the shifted state).
 * workspace: lfm25_decoder_workspace_bytes() bytes, 256-byte aligned, zeroed
 * before the first call and then kept by the caller (its control words carry
 * the exchange epoch from call to call; int32 [2] holds the status flags of
 * lfm25_decode). Calls sharing a workspace must not overlap.
 * The call is one ordinary launch of 128 blocks of 512 threads that hand
 * values to each other, so it makes progress only when all 128 are resident
 * at once (one per CU; an otherwise idle MI355X always holds them). When
 * other work on the device keeps some of them waiting, the blocks already
 * running give up after 5 s: the call then ends with status bit 2 (exchange
 * time-out) and a garbage hidden_out, never a hang. Callers that share the
 * device with other kernels use lfm25_decode (a cooperative launch, which the
 * runtime admits only when the whole grid fits). */
int lfm25_decode_layer(const lfm25_layer* layer, const uint16_t* hidden_in, uint16_t* hidden_out, int32_t position,
                       void* workspace, lfm25_stream_t stream);

/* ------------------------------------------------------------ batched pass (MFMA)
 *
 * Up to LFM25_BATCH_MAX_ROWS rows (token, sequence, position) through the
 * whole model in one pass, every weight tile read once for all rows and
 * multiplied on the matrix cores. Replaces the reference's batched prompt
 * pass: prefill_design (experiments/lfm25_x8.py:341-416), X8Model.prefill_batch
 * (experiments/lfm25_x8_model.py:94-115), dot4 / finish_row / attn_block4
 * (kernels/x8/x8p_core.cc:43-68, :156-227); extended to several independent
 * sequences (each with its own conv state and KV cache), which the reference
 * does not have. Rows of one sequence are consecutive with consecutive
 * positions and attend causally to each other. */
#define LFM25_BATCH_MAX_ROWS 64

typedef struct lfm25_batch {
  const uint16_t* weights;    /* packed weight stream (as lfm25_decoder) */
  const uint16_t* embedding;  /* [vocab x 1024] */
  const uint16_t* rope;       /* [capacity x 128] */
  uint16_t* conv_state;       /* [sequences x 8 x 1024 x 3] */
  uint16_t* key_cache;        /* [sequences x 6 x 8 x capacity x 64] */
  uint16_t* value_cache;      /* [sequences x 6 x 8 x capacity x 64] */
  void* workspace;            /* lfm25_batch_workspace_bytes() bytes, 256-byte aligned, zeroed before first use */
  int32_t sequences;          /* 1..64 */
  int32_t capacity;           /* KV positions per sequence, 1..4096 */
  int32_t vocab;              /* rows of the embedding table, % 16 == 0 */
} lfm25_batch;

size_t lfm25_batch_workspace_bytes(void);

/* One pass over n_rows rows given in host memory as int32 [n_rows x 3]
 * (token, sequence, position). Writes each row's K/V and advances its
 * sequence's conv state. select != 0: each row's greedy next token (first
 * maximum of the BF16 logits) -> tokens_out (device int32 [n_rows]).
 * hidden_out (device bf16 [n_rows x 1024], may be NULL): the last layer's
 * output of each row (before the final norm). Workspace int32 [0] holds status
 * bit 0 when a token id had to be clamped. */
int lfm25_batch_pass(const lfm25_batch* b, const int32_t* rows, int32_t n_rows, int32_t select,
                     int32_t* tokens_out, uint16_t* hidden_out, lfm25_stream_t stream);

/* n_steps greedy steps of all b->sequences sequences in lockstep: at step i
 * sequence s consumes a token at position positions[s] + i (positions: host
 * int32 [sequences]) -- tokens_in[s] (device) at step 0, its own selection
 * of step i - 1 afterwards -- and selects tokens_out[i][s] (device int32
 * [n_steps x sequences]). No counterpart in the reference (independent
 * sequences extend the reference's batched pass, which reads each weight
 * object once for all its rows: experiments/lfm25_x8.py:341-416).
 * With 2, 4 or 8 sequences the call runs as one or two cooperative launches
 * of the persistent decode's grid for all its steps, every layer's weights
 * read once per step for all sequences and their products on the matrix
 * cores (each sequence agrees with lfm25_decode on it alone within FP32
 * summation order); it needs every sequence's last position below 256 x 16
 * / sequences (or below 256) and a workspace that was zeroed before its
 * first use. With 16 sequences the steps below 256 positions run that way
 * (one launch) and the rest on the batched pass. Otherwise, or with
 * LFM25_BATCH_PERSISTENT=0 in the environment, each step is one batched
 * pass (one kernel per phase). Status flags in workspace int32 [0]:
 * bit 0 a token id was clamped, bit 1 capacity, bit 2 exchange time-out,
 * bit 3 a block ran off its XCD. */
int lfm25_batch_decode(const lfm25_batch* b, const int32_t* tokens_in, const int32_t* positions,
                       int32_t n_steps, int32_t* tokens_out, lfm25_stream_t stream);

/* lfm25_batch_decode on the persistent path only (LFM25_EINVAL when the
 * call does not fit it), also writing each step's pre-final-norm hidden
 * states to hidden_out (device BF16 [n_steps x sequences x 1024]): the
 * states X8Model.hidden() returns, for parity checks. No counterpart in
 * the reference. */
int lfm25_batch_decode_hidden(const lfm25_batch* b, const int32_t* tokens_in, const int32_t* positions,
                              int32_t n_steps, int32_t* tokens_out, uint16_t* hidden_out, lfm25_stream_t stream);

/* y = bf16(x . w^T) for x [rows x k], w [n x k] (rows <= 64, n % 16 == 0,
 * k in {1024, 2560}) on the batched pass's MFMA tiles: the GEMM core of
 * dot4 (kernels/x8/x8p_core.cc:43-60) + finish_row (:63-68), exposed for
 * parity tests. */
int lfm25_batch_linear(const uint16_t* x, const uint16_t* w, uint16_t* y, int32_t rows, int32_t n, int32_t k,
                       lfm25_stream_t stream);

/* ------------------------------------------------------------ Parakeet encoder
 *
 * The FastConformer encoder of the reference's all-NPU Parakeet path
 * (experiments/pk_model.py, pk_engine.py, kernels/pk/pk_core.cc, pk_fast.cc):
 * d = 1024, 8 heads of 128, FFN 4096, depthwise conv k = 9, 128-frame blocks
 * (T = 128, `valid` real frames), batches of independent sequences stacked as
 * [batch x 128 x 1024] BF16 rows. Matrices are output-major: W^T, [out x in]. */

/* c = bf16(epi(a . bt^T + bias)): a [m x k] (row stride lda), bt [n x k]
 * (row stride ldb), c [m x n] (row stride ldc); epi 0: none, 1: + bias[n],
 * 2: Swish x * sigmoid(x). n % 128 == 0, k % 64 == 0. splits > 1 divides K
 * into that many equal ranges (each a multiple of 64) whose FP32 partial
 * products go through `workspace` (splits * m * n floats, 16-byte aligned;
 * unused and may be null when splits == 1) and are summed in range order.
 * Replaces gemm_step / pk_wx / epilogue (kernels/pk/pk_fast.cc:167-231,
 * pk_core.cc:169-183) and the Gemm phase (experiments/pk_engine.py:192-220). */
int lfm25_pk_gemm(const uint16_t* a, int32_t lda, const uint16_t* bt, int32_t ldb, const uint16_t* bias,
                  uint16_t* c, int32_t ldc, int32_t m, int32_t n, int32_t k, int32_t epi, int32_t splits,
                  void* workspace, lfm25_stream_t stream);

/* Per 1024-row: x' = y ? bf16(x + scale * y) : x; normed_x == 0: x <- x'
 * (when y), a <- LN1(x'); normed_x != 0: x <- LN1(x') and, with gamma2,
 * a <- LN2(x). LN(v) = bf16((v - mean) / sqrt(var + 1e-5) * gamma + beta).
 * Replaces layer_norm / residual / ln_frame (kernels/pk/pk_core.cc:55-116)
 * and the Ln phase (experiments/pk_engine.py:223-242). */
int lfm25_pk_layer_norm(uint16_t* x, const uint16_t* y, float scale, const uint16_t* gamma1,
                        const uint16_t* beta1, const uint16_t* gamma2, const uint16_t* beta2,
                        int32_t normed_x, uint16_t* a, int32_t rows, lfm25_stream_t stream);

/* Relative-position attention: qkv [batch*128 x 3072] (q scaled by 1/sqrt(128)
 * with bias_v folded in, k, v), pos [8 x 256 x 128] (each head's projected
 * position table, transposed, offsets 127 .. -127 then a zero row), delta
 * [8 x 128] ((bias_u - bias_v) / sqrt(128)) -> out [batch*128 x 1024]; the
 * position scores q . P are formed inside; keys >= valid masked. Replaces
 * att_queries / att_bd / att_keys / att_finish (kernels/pk/pk_core.cc:126-203,
 * pk_fast.cc:71-116), the position-score GEMMs (experiments/pk_model.py:
 * 145-147) and the Att phase (experiments/pk_engine.py:245-281). */
int lfm25_pk_attention(const uint16_t* qkv, const uint16_t* pos, const uint16_t* delta, uint16_t* out,
                       int32_t batch, int32_t frames, int32_t valid, lfm25_stream_t stream);

/* Conv module core: c [batch*128 x 2048] (pointwise1 output) -> GLU, zero for
 * frames >= valid, 9-tap depthwise (dw [1024 x 9], bias [1024]), Swish ->
 * out [batch*128 x 1024]. Replaces conv_frames (kernels/pk/pk_fast.cc:119-154),
 * the Conv phase (experiments/pk_engine.py:284-297). */
int lfm25_pk_conv(const uint16_t* c, const uint16_t* dw, const uint16_t* dw_b, uint16_t* out, int32_t batch,
                  int32_t frames, int32_t valid, lfm25_stream_t stream);

/* One layer's device tensors (BF16). ln: [5 x 2 x 1024] (gamma, beta) of
 * norm_feed_forward1, norm_self_att, norm_conv, norm_feed_forward2, norm_out. */
typedef struct lfm25_pk_layer {
  const uint16_t* ln;
  const uint16_t* ff1_w1;     /* [4096 x 1024] */
  const uint16_t* ff1_w2;     /* [1024 x 4096] */
  const uint16_t* qkv;        /* [3072 x 1024]: wq^T / sqrt(128), wk^T, wv^T */
  const uint16_t* qkv_bias;   /* [3072]: bias_v / sqrt(128), 0, 0 */
  const uint16_t* att_delta;  /* [8 x 128] */
  const uint16_t* pos;        /* [8 x 256 x 128]: P_h^T for relative offsets 127 .. -127, then zero */
  const uint16_t* out;        /* [1024 x 1024] */
  const uint16_t* pw1;        /* [2048 x 1024] */
  const uint16_t* dw;         /* [1024 x 9] (batch norm folded) */
  const uint16_t* dw_b;       /* [1024] */
  const uint16_t* pw2;        /* [1024 x 1024] */
  const uint16_t* ff2_w1;     /* [4096 x 1024] */
  const uint16_t* ff2_w2;     /* [1024 x 4096] */
} lfm25_pk_layer;

size_t lfm25_pk_workspace_bytes(int32_t batch, int32_t frames);

/* n_layers Conformer blocks over x [batch x 128 x 1024] in place (the 22-phase
 * block order of build_phases, experiments/pk_model.py:132-161, and
 * PkEncoder.run :243-258): Macaron FFN/2, relative-position MHSA, conv module,
 * FFN/2, output LayerNorm. layers: host array of n_layers descriptors. */
int lfm25_pk_encoder(const lfm25_pk_layer* layers, int32_t n_layers, uint16_t* x, int32_t batch,
                     int32_t frames, int32_t valid, void* workspace, lfm25_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LFM25_HIP_H */
