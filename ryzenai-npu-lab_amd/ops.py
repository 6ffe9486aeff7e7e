"""Per-operation entry points with the reference's names and call shapes.

Each function mirrors one @iron.jit entry point of the reference's
experiments/lfm25_*_kernel.py: the same positional tensors (inputs first,
preallocated outputs written in place, no return value) and the same
keyword-only compile-time integers. Tensors are torch tensors on the GPU
(BF16 as torch.bfloat16, ids as torch.int32), contiguous. Shape and dtype
errors raise ValueError before anything is launched; device errors raise
RuntimeError. Calls are stream-ordered on torch's current stream and return
without waiting; NPU-only knobs such as n_cores are validated and ignored.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

HIDDEN, FFN, VOCAB = 1024, 2560, 65536
GAMMA_TILE = 4096  # the reference pads every norm weight to one 64x64 tile


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: torch.Tensor, name: str, dtype: torch.dtype, numel: int | None = None) -> int:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name} must hold {numel} values, got {t.numel()}")
    return t.data_ptr()


def _bf(t, name, numel=None):
    return _check(t, name, torch.bfloat16, numel)


def _f32(t, name, numel=None):
    return _check(t, name, torch.float32, numel)


def _i32(t, name, numel=None):
    return _check(t, name, torch.int32, numel)


def _cores(n_cores: int) -> None:
    if n_cores not in (1, 2, 4):
        raise ValueError("n_cores must be 1, 2 or 4")


# ---------------------------------------------------------------- norms / GEMV

def rms_norm(input0, gamma0, output, *, N: int) -> None:
    """Reference: lfm25_rms_norm_kernel.py:16-53 (kernels/lfm25_rms_norm.cc)."""
    if not 1 <= N <= 65536:
        raise ValueError("N must be in [1, 65536]")
    _lib.call("lfm25_rms_norm", _bf(input0, "input0", N), _bf(gamma0, "gamma0", N),
              _bf(output, "output", N), N, _stream())


def bf16_bf16_gemv(weights, activation, output, *, M: int, K: int, n_cores: int = 4) -> None:
    """Reference: lfm25_bf16_gemv_kernel.py:18-114."""
    _cores(n_cores)
    if M < 1 or K < 8 or K % 8:
        raise ValueError("Needs M >= 1 and K divisible by 8")
    _lib.call("lfm25_bf16_bf16_gemv", _bf(weights, "weights", M * K),
              _bf(activation, "activation", K), _bf(output, "output", M), M, K, _stream())


def bf16_f32_gemv(weights, activation, output, *, M: int, K: int, n_cores: int = 4) -> None:
    """Reference: lfm25_gemv_kernel.py:21-109 (FP32 output)."""
    _cores(n_cores)
    if M < 1 or K < 8 or K % 8:
        raise ValueError("Needs M >= 1 and K divisible by 8")
    _lib.call("lfm25_bf16_f32_gemv", _bf(weights, "weights", M * K),
              _bf(activation, "activation", K), _f32(output, "output", M), M, K, _stream())


def norm_bf16_gemv(hidden, packed_gamma_and_weight, output, *, M: int, K: int) -> None:
    """Reference: lfm25_norm_gemv_kernel.py:18-122; packed = [gamma | pad to
    4096 | W row-major M x K] (006_lfm25_npu_norm_gemv.py:26-28)."""
    if K != 1024 or M < 1:
        raise ValueError("Needs K=1024 and M >= 1")
    _lib.call("lfm25_norm_bf16_gemv", _bf(hidden, "hidden", K),
              _bf(packed_gamma_and_weight, "packed_gamma_and_weight", GAMMA_TILE + M * K),
              _bf(output, "output", M), M, K, _stream())


def w8_gemv(weights, scales, activation, output, *, M: int, K: int, group: int) -> None:
    """INT8-weight GEMV in the formats of experiments/014_int8_lfm25.py:76-113
    (w8g32 / w8g64: group 32 / 64, FP32 scales [M, K / group]; w8c: group 0,
    FP32 scales [M]); weights int8 [M, K] as weights.quantize_w8 makes them."""
    if M < 1 or K < 64 or K > 4096 or K % 64:
        raise ValueError("Needs M >= 1 and K a multiple of 64 in [64, 4096]")
    if group not in (0, 32, 64):
        raise ValueError("group must be 0, 32 or 64")
    _lib.call("lfm25_w8_gemv", _check(weights, "weights", torch.int8, M * K),
              _f32(scales, "scales", M * (K // group if group else 1)),
              _bf(activation, "activation", K), _bf(output, "output", M), M, K, group, _stream())


def f32_to_bf16(input0, output, *, N: int) -> None:
    """Reference: lfm25_cast_kernel.py:16-45."""
    if N < 1:
        raise ValueError("N must be positive")
    _lib.call("lfm25_f32_to_bf16", _f32(input0, "input0", N), _bf(output, "output", N), N,
              _stream())


def bf16_add(left, right, output, *, N: int) -> None:
    """Reference: lfm25_add_kernel.py:16-53."""
    if N < 1:
        raise ValueError("N must be positive")
    _lib.call("lfm25_bf16_add", _bf(left, "left", N), _bf(right, "right", N),
              _bf(output, "output", N), N, _stream())


def silu_gate(w1, w3, output, *, N: int) -> None:
    """Reference: lfm25_silu_gate_kernel.py:16-51."""
    if N < 1:
        raise ValueError("N must be positive")
    _lib.call("lfm25_silu_gate", _bf(w1, "w1", N), _bf(w3, "w3", N), _bf(output, "output", N), N,
              _stream())


# ---------------------------------------------------------------- conv

def conv_gate(projection_and_weight, state, output, next_state) -> None:
    """Reference: lfm25_conv_gate_kernel.py:16-73; projection_and_weight =
    [B | C | x | w (1024 x 3)], state/next_state the HF [1024 x 3] state."""
    _lib.call("lfm25_conv_gate", _bf(projection_and_weight, "projection_and_weight", 6 * HIDDEN),
              _bf(state, "state", 3 * HIDDEN), _bf(output, "output", HIDDEN),
              _bf(next_state, "next_state", 3 * HIDDEN), _stream())


def conv_gate_packed_state(projection, state_and_weight, output, next_state_and_weight) -> None:
    """Reference: lfm25_conv_gate_packed_state_kernel.py:16-63."""
    _lib.call("lfm25_conv_gate_packed_state", _bf(projection, "projection", 3 * HIDDEN),
              _bf(state_and_weight, "state_and_weight", 6 * HIDDEN),
              _bf(output, "output", HIDDEN),
              _bf(next_state_and_weight, "next_state_and_weight", 6 * HIDDEN), _stream())


def _layer_workspace(device) -> torch.Tensor:
    """A zeroed lfm25_decode_layer workspace for one call (its exchange epochs
    start from zero, so concurrent calls never share one)."""
    return torch.zeros(int(_lib.load().lfm25_decoder_workspace_bytes()), dtype=torch.uint8, device=device)


def recurrent_block(packed_hidden_and_state, packed_weights, next_state_and_weight,
                    block_output) -> None:
    """One conv decoder layer in one launch (lfm25_decode_layer).
    Reference: lfm25_single_program_block_kernel.py:32-284.
    packed_hidden_and_state = [hidden (1024) | pad to 6144 | state (1024 x 3) |
    conv w (1024 x 3)]; packed_weights = [operator gamma tile | in_proj |
    out_proj | ffn gamma tile | w1 | w3 | w2]; next_state_and_weight =
    [next state (1024 x 3) | conv w (1024 x 3)]."""
    hp = _bf(packed_hidden_and_state, "packed_hidden_and_state", 2 * 6144)
    n_w = 2 * GAMMA_TILE + (3 * HIDDEN + HIDDEN + 2 * FFN) * HIDDEN + HIDDEN * FFN
    wp = _bf(packed_weights, "packed_weights", n_w)
    nxt = _bf(next_state_and_weight, "next_state_and_weight", 6144)
    out = _bf(block_output, "block_output", HIDDEN)
    at = lambda elems: wp + 2 * elems  # noqa: E731  (byte address of element `elems`)
    o_out = GAMMA_TILE + 3 * HIDDEN * HIDDEN
    o_ffn = o_out + HIDDEN * HIDDEN
    o_w1 = o_ffn + GAMMA_TILE
    layer = _lib.Layer(kind=_lib.LAYER_CONV, op_norm=wp, mixer=at(GAMMA_TILE),
                       conv_weight=hp + 2 * (6144 + 3 * HIDDEN), conv_state_in=hp + 2 * 6144,
                       conv_state_out=nxt, out=at(o_out), ffn_norm=at(o_ffn), w1=at(o_w1),
                       w3=at(o_w1 + FFN * HIDDEN), w2=at(o_w1 + 2 * FFN * HIDDEN))
    ws = _layer_workspace(block_output.device)
    _lib.call("lfm25_decode_layer", ctypes.byref(layer), hp, out, 0, ws.data_ptr(), _stream())
    next_state_and_weight[3 * HIDDEN:].copy_(packed_hidden_and_state[6144 + 3 * HIDDEN:])


def _mlp_tail(residual, projection_input, weights, block_output) -> None:
    """[out (1024 x 1024) | ffn gamma tile | w1 | w3 | w2] applied as
    h = residual + out.x; block_output = h + w2.(silu(w1.n) * w3.n), n = norm(h)."""
    dev = block_output.device
    proj = torch.empty(HIDDEN, dtype=torch.bfloat16, device=dev)
    bf16_bf16_gemv(weights[:HIDDEN * HIDDEN], projection_input, proj, M=HIDDEN, K=HIDDEN)
    h = torch.empty(HIDDEN, dtype=torch.bfloat16, device=dev)
    bf16_add(residual, proj, h, N=HIDDEN)
    off = HIDDEN * HIDDEN
    up = torch.empty(2 * FFN, dtype=torch.bfloat16, device=dev)
    norm_bf16_gemv(h, weights[off:off + GAMMA_TILE + 2 * FFN * HIDDEN], up, M=2 * FFN, K=HIDDEN)
    gate = torch.empty(FFN, dtype=torch.bfloat16, device=dev)
    silu_gate(up[:FFN], up[FFN:], gate, N=FFN)
    off += GAMMA_TILE + 2 * FFN * HIDDEN
    down = torch.empty(HIDDEN, dtype=torch.bfloat16, device=dev)
    bf16_bf16_gemv(weights[off:off + HIDDEN * FFN], gate, down, M=HIDDEN, K=FFN)
    bf16_add(h, down, block_output, N=HIDDEN)


# ---------------------------------------------------------------- attention

_QKV = HIDDEN + 2 * 512  # 2048


def attention_prefix(hidden, packed_weights, qkv_output, *, include_hidden: bool = False) -> None:
    """Operator norm, Q/K/V, per-head QK norm and RoPE.
    Reference: lfm25_attention_prefix_kernel.py:22-140; packed_weights =
    [gamma tile | q | k | v | aux tile = q_gamma (64) | k_gamma (64) | cos (64) |
    sin (64)]."""
    n_w = 2 * GAMMA_TILE + _QKV * HIDDEN
    _bf(packed_weights, "packed_weights", n_w)
    _bf(qkv_output, "qkv_output", _QKV + (HIDDEN if include_hidden else 0))
    norm_bf16_gemv(hidden, packed_weights[:GAMMA_TILE + _QKV * HIDDEN], qkv_output[:_QKV],
                   M=_QKV, K=HIDDEN)
    aux = packed_weights[GAMMA_TILE + _QKV * HIDDEN:GAMMA_TILE + _QKV * HIDDEN + 256]
    _lib.call("lfm25_attention_norm_rope", _bf(qkv_output, "qkv_output"), aux.data_ptr(),
              _stream())
    if include_hidden:
        qkv_output[_QKV:].copy_(hidden)


def _past_length(cache, name: str) -> int:
    per = 2 * 8 * 64
    if cache.numel() % per:
        raise ValueError(f"{name} must hold 8 heads x 2 x past_length x 64 values")
    return cache.numel() // per


def attention_context(qkv, past_cache, context) -> None:
    """Reference: lfm25_attention_context_kernel.py:20-72 (past length taken
    from the cache size: 8 heads x [keys P x 64 | values P x 64])."""
    past = _past_length(past_cache, "past_cache")
    _lib.call("lfm25_attention_context", _bf(qkv, "qkv", _QKV), _bf(past_cache, "past_cache"),
              _bf(context, "context", HIDDEN), past, _stream())


def append_attention_cache(qkv, prior_cache, next_cache) -> None:
    """Reference: lfm25_attention_append_cache_kernel.py:20 (prior length P from
    prior_cache; next_cache holds P + 1 positions)."""
    past = _past_length(prior_cache, "prior_cache")
    _lib.call("lfm25_attention_append_cache", _bf(qkv, "qkv"), _bf(prior_cache, "prior_cache"),
              _bf(next_cache, "next_cache", 2 * 8 * (past + 1) * 64), past, _stream())


def attention_context_cache(qkv_and_hidden, past_cache, packed_tail_input, next_cache, *,
                            past_length: int = 21) -> None:
    """Context, KV append and tail-input packing in one call.
    Reference: lfm25_attention_context_cache_kernel.py:16-106;
    packed_tail_input = [hidden (1024) | context (1024)]."""
    if not 1 <= past_length < 4096:
        raise ValueError("past_length must be in [1, 4096)")
    _bf(qkv_and_hidden, "qkv_and_hidden", _QKV + HIDDEN)
    _bf(past_cache, "past_cache", 2 * 8 * past_length * 64)
    _bf(packed_tail_input, "packed_tail_input", 2 * HIDDEN)
    _bf(next_cache, "next_cache", 2 * 8 * (past_length + 1) * 64)
    attention_context(qkv_and_hidden[:_QKV], past_cache, packed_tail_input[HIDDEN:])
    append_attention_cache(qkv_and_hidden[:_QKV], past_cache, next_cache)
    packed_tail_input[:HIDDEN].copy_(qkv_and_hidden[_QKV:])


def attention_tail(packed_hidden_and_context, packed_weights, block_output) -> None:
    """o_proj + residual + SwiGLU MLP + residual.
    Reference: lfm25_attention_tail_kernel.py:29-208; packed_weights = [o |
    ffn gamma tile | w1 | w3 | w2]."""
    _bf(packed_hidden_and_context, "packed_hidden_and_context", 2 * HIDDEN)
    n_w = HIDDEN * HIDDEN + GAMMA_TILE + 3 * FFN * HIDDEN
    _bf(packed_weights, "packed_weights", n_w)
    _bf(block_output, "block_output", HIDDEN)
    _mlp_tail(packed_hidden_and_context[:HIDDEN], packed_hidden_and_context[HIDDEN:],
              packed_weights, block_output)


# ---------------------------------------------------------------- head / embedding

def _workspace(count: int, device) -> torch.Tensor:
    n = int(_lib.load().lfm25_argmax_workspace_bytes(count))
    return torch.empty(n, dtype=torch.uint8, device=device)


def vocab_argmax(logits, token_id) -> None:
    """First index of the maximum BF16 logit. Reference: lfm25_argmax_kernel.py:18-68."""
    n = logits.numel()
    ws = _workspace(n, logits.device)
    _lib.call("lfm25_argmax", _bf(logits, "logits"), n, _i32(token_id, "token_id", 1),
              ws.data_ptr(), _stream())


def fused_vocab(hidden, packed_gamma_and_embedding, next_embedding, token_id, *,
                logits=None) -> None:
    """Final norm, tied head, argmax and the winning embedding row.
    Reference: lfm25_fused_vocab_kernel.py:22-110; packed = [gamma (1024) |
    E (vocab x 1024)] (vocab = 65536 in the reference; any multiple of 4 here)."""
    total = packed_gamma_and_embedding.numel()
    if total < HIDDEN or (total - HIDDEN) % HIDDEN:
        raise ValueError("packed_gamma_and_embedding must be [gamma | E (vocab x 1024)]")
    vocab = (total - HIDDEN) // HIDDEN
    if vocab < 4 or vocab % 4:
        raise ValueError("vocab must be a positive multiple of 4")
    ws = _workspace(vocab, hidden.device)
    lp = 0 if logits is None else _bf(logits, "logits", vocab)
    _lib.call("lfm25_fused_vocab", _bf(hidden, "hidden", HIDDEN),
              _bf(packed_gamma_and_embedding, "packed_gamma_and_embedding"),
              _bf(next_embedding, "next_embedding", HIDDEN), _i32(token_id, "token_id", 1), lp,
              vocab, ws.data_ptr(), _stream())


def embedding_dma_dynamic(table, embedding, token_id) -> None:
    """Reference: lfm25_embedding_dynamic_kernel.py:22-68 (id read on device)."""
    if table.dim() != 2 or table.shape[1] != HIDDEN:
        raise ValueError("table must be [vocab, 1024]")
    _lib.call("lfm25_embedding_gather", _bf(table, "table"), _i32(token_id, "token_id", 1),
              _bf(embedding, "embedding", HIDDEN), table.shape[0], 0, _stream())


def embedding_dma(table, embedding, *, token_id: int) -> None:
    """Reference: lfm25_embedding_dma_kernel.py:11-39 (id fixed at call time)."""
    if table.dim() != 2 or table.shape[1] != HIDDEN:
        raise ValueError("table must be [vocab, 1024]")
    if not 0 <= token_id < table.shape[0]:
        raise ValueError("Token ID outside vocabulary")
    tid = torch.tensor([token_id], dtype=torch.int32, device=table.device)
    embedding_dma_dynamic(table, embedding, tid)


def embedding_pair_dynamic(table, pair, token_ids) -> None:
    """Two embedding rows, ids read on the device: pair = [table[ids[0]] |
    table[ids[1]]]. Reference: lfm25_prefill_pair_embedding_kernel.py:18."""
    if table.dim() != 2 or table.shape[1] != HIDDEN:
        raise ValueError("table must be [vocab, 1024]")
    _bf(pair, "pair", 2 * HIDDEN)
    _i32(token_ids, "token_ids", 2)
    for i in range(2):
        _lib.call("lfm25_embedding_gather", table.data_ptr(), token_ids[i:i + 1].data_ptr(),
                  pair[i * HIDDEN:(i + 1) * HIDDEN].data_ptr(), table.shape[0], 0, _stream())


# ---------------------------------------------------------------- packing programs

def pack_block_input(hidden, state_and_weight, packed) -> None:
    """packed = [hidden | zeros to 6144 | state_and_weight (6144)].
    Reference: lfm25_pack_block_input_kernel.py:17 (kernels/lfm25_pack_block_input.cc)."""
    _lib.call("lfm25_pack_block_input", _bf(hidden, "hidden", HIDDEN),
              _bf(state_and_weight, "state_and_weight", 6144), _bf(packed, "packed", 12288), _stream())


def pack_conv(projection, weight, packed) -> None:
    """packed = [projection (3072) | weight (3072)].
    Reference: lfm25_pack_conv_kernel.py:17 (kernels/lfm25_pack_conv.cc)."""
    _lib.call("lfm25_pack_conv", _bf(projection, "projection", 3 * HIDDEN), _bf(weight, "weight", 3 * HIDDEN),
              _bf(packed, "packed", 6 * HIDDEN), _stream())


def pack_attention_tail(hidden, context, packed) -> None:
    """packed = [hidden | context].
    Reference: lfm25_pack_attention_tail_kernel.py:17 (kernels/lfm25_pack_attention_tail.cc)."""
    _lib.call("lfm25_pack_attention_tail", _bf(hidden, "hidden", HIDDEN), _bf(context, "context", HIDDEN),
              _bf(packed, "packed", 2 * HIDDEN), _stream())


def concat_hidden_pair(first, second, pair) -> None:
    """pair = [first | second]. Reference: lfm25_prefill_pair_data_kernel.py:11."""
    _lib.call("lfm25_concat_hidden_pair", _bf(first, "first", HIDDEN), _bf(second, "second", HIDDEN),
              _bf(pair, "pair", 2 * HIDDEN), _stream())


def split_hidden_pair(pair, first, second) -> None:
    """first, second = pair. Reference: lfm25_prefill_pair_data_kernel.py:42."""
    _lib.call("lfm25_split_hidden_pair", _bf(pair, "pair", 2 * HIDDEN), _bf(first, "first", HIDDEN),
              _bf(second, "second", HIDDEN), _stream())


def pack_recurrent_pair(pair, state, packed) -> None:
    """packed = [first | zeros to 6144 | second | zeros to 12288 | state (6144)].
    Reference: lfm25_prefill_pair_data_kernel.py:73."""
    _lib.call("lfm25_pack_recurrent_pair", _bf(pair, "pair", 2 * HIDDEN), _bf(state, "state", 6144),
              _bf(packed, "packed", 18432), _stream())


# ---------------------------------------------------------------- more layer programs

def norm_proj_conv(packed_hidden_and_state, packed_gamma_and_projection_weight, gate_output,
                   next_state_and_weight) -> None:
    """Operator norm, in_proj and the gated conv of a conv layer.
    Reference: lfm25_norm_proj_conv_kernel.py:24-148; packed_hidden_and_state =
    [hidden | pad to 6144 | state (1024 x 3) | conv w (1024 x 3)];
    packed_gamma_and_projection_weight = [gamma tile | in_proj (3072 x 1024)]."""
    _bf(packed_hidden_and_state, "packed_hidden_and_state", 2 * 6144)
    _bf(packed_gamma_and_projection_weight, "packed_gamma_and_projection_weight", GAMMA_TILE + 3 * HIDDEN * HIDDEN)
    _bf(gate_output, "gate_output", HIDDEN)
    _bf(next_state_and_weight, "next_state_and_weight", 6144)
    proj = torch.empty(3 * HIDDEN, dtype=torch.bfloat16, device=gate_output.device)
    norm_bf16_gemv(packed_hidden_and_state[:HIDDEN], packed_gamma_and_projection_weight, proj,
                   M=3 * HIDDEN, K=HIDDEN)
    conv_gate_packed_state(proj, packed_hidden_and_state[6144:], gate_output, next_state_and_weight)


def _pair_layer(hiddens, state_in, conv_w, packed_weights, next_state_and_weight, block_output) -> None:
    """Two consecutive positions through one conv layer: the second starts
    from the state the first left (lfm25_decode_layer twice, in place)."""
    n_w = 2 * GAMMA_TILE + (3 * HIDDEN + HIDDEN + 2 * FFN) * HIDDEN + HIDDEN * FFN
    wp = _bf(packed_weights, "packed_weights", n_w)
    nxt = _bf(next_state_and_weight, "next_state_and_weight", 6144)
    _bf(block_output, "block_output", 2 * HIDDEN)
    at = lambda elems: wp + 2 * elems  # noqa: E731
    o_out = GAMMA_TILE + 3 * HIDDEN * HIDDEN
    o_ffn = o_out + HIDDEN * HIDDEN
    o_w1 = o_ffn + GAMMA_TILE
    ws = _layer_workspace(block_output.device)
    for i, h in enumerate(hiddens):
        layer = _lib.Layer(kind=_lib.LAYER_CONV, op_norm=wp, mixer=at(GAMMA_TILE), conv_weight=conv_w.data_ptr(),
                           conv_state_in=state_in.data_ptr() if i == 0 else nxt, conv_state_out=nxt,
                           out=at(o_out), ffn_norm=at(o_ffn), w1=at(o_w1), w3=at(o_w1 + FFN * HIDDEN),
                           w2=at(o_w1 + 2 * FFN * HIDDEN))
        _lib.call("lfm25_decode_layer", ctypes.byref(layer), h.data_ptr(),
                  block_output[i * HIDDEN:(i + 1) * HIDDEN].data_ptr(), 0, ws.data_ptr(), _stream())
    next_state_and_weight[3 * HIDDEN:].copy_(conv_w)


def recurrent_pair_block(packed_hidden_and_state, packed_weights, next_state_and_weight, block_output) -> None:
    """Two prompt positions through one conv layer. Reference:
    lfm25_prefill_pair_block_kernel.py:33; packed_hidden_and_state = [first |
    pad to 6144 | second | pad to 12288 | state (1024 x 3) | conv w (1024 x 3)]
    (pack_recurrent_pair); packed_weights as recurrent_block; block_output =
    [first | second]."""
    _bf(packed_hidden_and_state, "packed_hidden_and_state", 3 * 6144)
    p = packed_hidden_and_state
    _pair_layer([p[:HIDDEN], p[6144:6144 + HIDDEN]], p[12288:12288 + 3 * HIDDEN], p[12288 + 3 * HIDDEN:],
                packed_weights, next_state_and_weight, block_output)


def recurrent_pair_direct(hidden_pair, prior_state_and_weight, packed_weights, next_state_and_weight,
                          block_output) -> None:
    """recurrent_pair_block with the pair and the state in separate buffers.
    Reference: lfm25_prefill_pair_direct_kernel.py:33."""
    _bf(hidden_pair, "hidden_pair", 2 * HIDDEN)
    _bf(prior_state_and_weight, "prior_state_and_weight", 6144)
    _pair_layer([hidden_pair[:HIDDEN], hidden_pair[HIDDEN:]], prior_state_and_weight[:3 * HIDDEN],
                prior_state_and_weight[3 * HIDDEN:], packed_weights, next_state_and_weight, block_output)


def attention_prefix_pair(hidden_pair, packed_weights_and_aux0, aux1, qkv_pair) -> None:
    """attention_prefix of two positions: qkv_pair = [q|k|v|hidden of the first
    (3072) | the same of the second]; aux0 (the first position's QK-norm and
    RoPE tile) ends packed_weights_and_aux0, aux1 is the second's.
    Reference: lfm25_prefill_pair_attention_prefix_kernel.py:23."""
    _bf(hidden_pair, "hidden_pair", 2 * HIDDEN)
    _bf(aux1, "aux1", GAMMA_TILE)
    _bf(qkv_pair, "qkv_pair", 2 * (_QKV + HIDDEN))
    w = packed_weights_and_aux0
    _bf(w, "packed_weights_and_aux0", 2 * GAMMA_TILE + _QKV * HIDDEN)
    attention_prefix(hidden_pair[:HIDDEN], w, qkv_pair[:_QKV + HIDDEN], include_hidden=True)
    second = qkv_pair[_QKV + HIDDEN:]
    norm_bf16_gemv(hidden_pair[HIDDEN:], w[:GAMMA_TILE + _QKV * HIDDEN], second[:_QKV], M=_QKV, K=HIDDEN)
    _lib.call("lfm25_attention_norm_rope", second.data_ptr(), aux1.data_ptr(), _stream())
    second[_QKV:].copy_(hidden_pair[HIDDEN:])


def attention_tail_pair(packed_hidden_and_context, packed_weights, block_output) -> None:
    """attention_tail of two positions: [hidden | context] of each in turn ->
    block_output = [first | second]. Reference:
    lfm25_prefill_pair_attention_tail_kernel.py:30."""
    _bf(packed_hidden_and_context, "packed_hidden_and_context", 4 * HIDDEN)
    _bf(block_output, "block_output", 2 * HIDDEN)
    for i in range(2):
        attention_tail(packed_hidden_and_context[2 * i * HIDDEN:2 * (i + 1) * HIDDEN], packed_weights,
                       block_output[i * HIDDEN:(i + 1) * HIDDEN])


# ---------------------------------------------------------------- headered KV caches

def _head_elems(capacity: int) -> int:
    return 2 + 2 * capacity * 64


def _attention_fixed(qkv_and_hidden, past_cache, packed_tail_input, next_cache, capacity: int,
                     blocks: int = 1) -> None:
    n = blocks * 8 * _head_elems(capacity)
    _bf(qkv_and_hidden, "qkv_and_hidden", _QKV + HIDDEN)
    _bf(packed_tail_input, "packed_tail_input", 2 * HIDDEN)
    _bf(next_cache, "next_cache", n)
    past = 0 if past_cache is None else _bf(past_cache, "past_cache", n)
    # The kernel reports a full or malformed block in bit 0 of a status word
    # and then leaves packed_tail_input and next_cache unwritten.
    status = torch.zeros(1, dtype=torch.int32, device=qkv_and_hidden.device)
    _lib.call("lfm25_attention_fixed", qkv_and_hidden.data_ptr(), past, packed_tail_input.data_ptr(),
              next_cache.data_ptr(), capacity, blocks, status.data_ptr(), _stream())
    if int(status.item()) & 1:
        raise ValueError(f"attention: a headered KV cache block (capacity {capacity}) is full or holds "
                         "a length outside [0, capacity); nothing was written")


def attention_first_context(qkv_and_hidden, packed_tail_input, first_cache) -> None:
    """Position 0: context = each KV head's value; first_cache = per head [k | v].
    Reference: lfm25_attention_first_context_kernel.py:16-17."""
    _lib.call("lfm25_attention_first_context", _bf(qkv_and_hidden, "qkv_and_hidden", _QKV + HIDDEN),
              _bf(packed_tail_input, "packed_tail_input", 2 * HIDDEN), _bf(first_cache, "first_cache", HIDDEN),
              _stream())


def attention_first_fixed(qkv_and_hidden, packed_tail_input, first_cache) -> None:
    """Position 0 into a capacity-32 headered cache.
    Reference: lfm25_attention_fixed_cache_kernel.py:30-31."""
    _attention_fixed(qkv_and_hidden, None, packed_tail_input, first_cache, 32)


def attention_context_fixed(qkv_and_hidden, past_cache, packed_tail_input, next_cache) -> None:
    """Attention and append over a capacity-32 headered cache.
    Reference: lfm25_attention_fixed_cache_kernel.py:81-82."""
    _attention_fixed(qkv_and_hidden, past_cache, packed_tail_input, next_cache, 32)


def attention_first_fixed64(qkv_and_hidden, packed_tail_input, first_cache) -> None:
    """Position 0 into a capacity-64 headered cache.
    Reference: lfm25_attention_fixed64_cache_kernel.py:31."""
    _attention_fixed(qkv_and_hidden, None, packed_tail_input, first_cache, 64)


def attention_context_fixed64(qkv_and_hidden, past_cache, packed_tail_input, next_cache) -> None:
    """Attention and append over a capacity-64 headered cache.
    Reference: lfm25_attention_fixed64_cache_kernel.py:82."""
    _attention_fixed(qkv_and_hidden, past_cache, packed_tail_input, next_cache, 64)


def attention_context_chunked(qkv_and_hidden, past_cache, packed_tail_input, next_cache, *,
                              block_count: int = 1) -> None:
    """Attention and append over `block_count` capacity-64 blocks (positions
    in block order, the new one appended to the last block).
    Reference: lfm25_attention_chunked_cache_kernel.py:22-24."""
    if not 1 <= block_count <= 64:
        raise ValueError("block_count must be in [1, 64]")
    _attention_fixed(qkv_and_hidden, past_cache, packed_tail_input, next_cache, 64, block_count)


def attention_pair_context_fixed64(qkv_pair, past_cache, tail_pair, next_cache) -> None:
    """Two causal positions over a capacity-64 headered cache: the second
    attends to the first. tail_pair = [hidden | context of the first | the
    same of the second]. Reference: lfm25_prefill_pair_attention_context_kernel.py:22."""
    _bf(qkv_pair, "qkv_pair", 2 * (_QKV + HIDDEN))
    _bf(tail_pair, "tail_pair", 4 * HIDDEN)
    step = _QKV + HIDDEN
    _attention_fixed(qkv_pair[:step], past_cache, tail_pair[:2 * HIDDEN], next_cache, 64)
    _attention_fixed(qkv_pair[step:], next_cache, tail_pair[2 * HIDDEN:], next_cache, 64)


# ---------------------------------------------------------------- vocabulary, matmul

def fused_vocab_4core(hidden, packed_gamma_and_embedding, next_embedding, token_id) -> None:
    """fused_vocab over the full 65,536-row vocabulary (the NPU's four-core
    shard split has no counterpart: the GPU scans every row in one launch).
    Reference: lfm25_fused_vocab_4core_kernel.py:24-26."""
    if packed_gamma_and_embedding.numel() != HIDDEN + VOCAB * HIDDEN:
        raise ValueError("packed_gamma_and_embedding must be [gamma | E (65536 x 1024)]")
    fused_vocab(hidden, packed_gamma_and_embedding, next_embedding, token_id)


def bf16_f32_matmul(input0, input1, output, *, M: int, K: int, N: int, n_cores: int = 1,
                    reuse_weights: bool = False) -> None:
    """output[M x N] (FP32) = input0[M x K] . input1[K x N] (BF16, row-major).
    Reference: lfm25_matmul_kernel.py:16-27 (same shape checks)."""
    if M < 16 or M % 16 or K % 64 or n_cores not in (1, 2, 4) or N % (64 * n_cores):
        raise ValueError("Needs M%16=0, K%64=0, N%(64*n_cores)=0, cores in 1/2/4")
    if reuse_weights and M != 48:
        raise ValueError("Weight reuse probe requires M=48")
    _lib.call("lfm25_bf16_f32_matmul", _bf(input0, "input0", M * K), _bf(input1, "input1", K * N),
              _f32(output, "output", M * N), M, K, N, _stream())
