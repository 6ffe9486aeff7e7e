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
