"""The reference's remaining per-operation entry points (ops.*) on the GPU:
the headered-cache attention programs, first-position attention, packing and
two-position programs, and the BF16 x BF16 -> FP32 product.

Bars (stated per test): layout programs are bit-exact copies; the attention
programs over the reference's fixed / chunked cache layouts give bit for bit
the context of lfm25_attention_context on the same positions in a contiguous
cache (the same arithmetic, other addressing), and that kernel is held to
the oracle in test_gpu_ops.py; two-position programs equal two one-position
calls bit for bit, and the layers among them are held to the oracle; the
matrix product is within the FP32 summation bound of the exact sum.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import lfm25 as O
from parity_helpers import attention_interval

pytestmark = pytest.mark.gpu

rs = np.random.RandomState(20261202)
HE32, HE64 = 2 + 2 * 32 * 64, 2 + 2 * 64 * 64


def dev(bits) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16).reshape(-1)).cuda().view(
        torch.bfloat16)


def dev_f(x) -> torch.Tensor:
    return dev(O.bf16_bits(np.asarray(x, np.float32)))


def bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def empty(n: int) -> torch.Tensor:
    return torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")


def bf(x):
    return O._bf(np.asarray(x, np.float32))


def qkv_hidden() -> np.ndarray:
    return O.bf16_bits(rs.standard_normal(3072).astype(np.float32))


def headered(keys: np.ndarray, values: np.ndarray, cap: int) -> np.ndarray:
    """keys/values bits [8, n, 64] -> one headered cache of capacity cap."""
    n = keys.shape[1]
    he = 2 + 2 * cap * 64
    out = np.zeros((8, he), np.uint16)
    out[:, 0] = O.bf16_bits(np.float32([n]))[0]
    out[:, 2:2 + n * 64] = keys.reshape(8, -1)
    out[:, 2 + cap * 64:2 + cap * 64 + n * 64] = values.reshape(8, -1)
    return out.reshape(-1)


def contiguous_context(lab, qkv: np.ndarray, keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """lfm25_attention_context over the reference's contiguous layout."""
    past = keys.shape[1]
    cache = np.concatenate([keys, values], axis=1).reshape(-1)
    ctx = empty(1024)
    cache_t = dev(cache) if past else torch.zeros(8, dtype=torch.bfloat16, device="cuda")
    qkv_t = dev(qkv[:2048])  # held until the call is done
    lab._lib.call("lfm25_attention_context", qkv_t.data_ptr(), cache_t.data_ptr(), ctx.data_ptr(), past,
                  torch.cuda.current_stream().cuda_stream)
    return bits(ctx)


def test_attention_first_context_is_exact(gpu, lab):
    qkv = qkv_hidden()
    tail, cache = empty(2048), empty(1024)
    lab.ops.attention_first_context(dev(qkv), tail, cache)
    t, c = bits(tail), bits(cache).reshape(8, 128)
    k, v = qkv[1024:1536].reshape(8, 64), qkv[1536:2048].reshape(8, 64)
    assert np.array_equal(c[:, :64], k) and np.array_equal(c[:, 64:], v)
    assert np.array_equal(t[:1024], qkv[2048:])
    assert np.array_equal(t[1024:].reshape(16, 64), np.repeat(v, 2, axis=0))
    assert np.array_equal(t[1024:], contiguous_context(lab, qkv, np.zeros((8, 0, 64), np.uint16),
                                                       np.zeros((8, 0, 64), np.uint16)))


@pytest.mark.parametrize("cap,first,context", [(32, "attention_first_fixed", "attention_context_fixed"),
                                               (64, "attention_first_fixed64", "attention_context_fixed64")])
def test_fixed_cache_sequence(gpu, lab, cap, first, context):
    """Position 0 into an empty headered cache, then every later position up
    to the capacity: each context bit for bit that of the contiguous-layout
    kernel over the same positions, the next cache exactly the previous with
    the new row appended and the length raised (header element 0)."""
    keys = np.zeros((8, 0, 64), np.uint16)
    values = np.zeros((8, 0, 64), np.uint16)
    cache = None
    for pos in range(cap):
        qkv = qkv_hidden()
        tail, nxt = empty(2048), empty(8 * (2 + 2 * cap * 64))
        if pos == 0:
            getattr(lab.ops, first)(dev(qkv), tail, nxt)
        else:
            getattr(lab.ops, context)(dev(qkv), dev(cache), tail, nxt)
        want_ctx = contiguous_context(lab, qkv, keys, values)
        t = bits(tail)
        assert np.array_equal(t[:1024], qkv[2048:]), pos
        assert np.array_equal(t[1024:], want_ctx), pos
        keys = np.concatenate([keys, qkv[1024:1536].reshape(8, 1, 64)], axis=1)
        values = np.concatenate([values, qkv[1536:2048].reshape(8, 1, 64)], axis=1)
        cache = bits(nxt)
        assert np.array_equal(cache, headered(keys, values, cap)), pos


def test_fixed_context_matches_the_oracle(gpu, lab):
    """One capacity-64 step at 40 cached positions against the oracle's
    attention, with the bar of lfm25_attention_context: every value inside
    the interval the oracle's algorithm allows for FP32 sums in another order
    (parity_helpers.attention_interval), at most 5% of them differing."""
    keys = O.bf16_bits(rs.standard_normal((8, 40, 64)).astype(np.float32))
    values = O.bf16_bits(rs.standard_normal((8, 40, 64)).astype(np.float32))
    qkv = qkv_hidden()
    tail, nxt = empty(2048), empty(8 * HE64)
    lab.ops.attention_context_fixed64(dev(qkv), dev(headered(keys, values, 64)), tail, nxt)
    f = O.f32
    k_all = np.concatenate([f(keys), f(qkv[1024:1536]).reshape(8, 1, 64)], axis=1)
    v_all = np.concatenate([f(values), f(qkv[1536:2048]).reshape(8, 1, 64)], axis=1)
    want = O.attention(f(qkv[:1024]).reshape(16, 64), k_all, v_all)
    got = O.f32(bits(tail)[1024:])
    lo, hi = attention_interval(f(qkv[:1024]).reshape(16, 64), k_all, v_all, 41 + 64)
    g = got.astype(np.float64)
    assert not np.any((g < lo) | (g > hi)), np.flatnonzero((g < lo) | (g > hi))[:8]
    assert np.mean(got != want) <= 0.05


@pytest.mark.parametrize("blocks,last", [(1, 0), (2, 17), (3, 63)])
def test_chunked_cache(gpu, lab, blocks, last):
    """`blocks` capacity-64 blocks, all full but the last (`last` rows): the
    context bit for bit that of the contiguous kernel over the concatenated
    positions; the new row lands in the last block; the others are copied."""
    n = 64 * (blocks - 1) + last
    keys = O.bf16_bits(rs.standard_normal((8, n, 64)).astype(np.float32))
    values = O.bf16_bits(rs.standard_normal((8, n, 64)).astype(np.float32))
    parts = []
    for b in range(blocks):
        lo, hi = 64 * b, min(64 * (b + 1), n)
        parts.append(headered(keys[:, lo:hi], values[:, lo:hi], 64))
    past = np.concatenate(parts)
    qkv = qkv_hidden()
    tail, nxt = empty(2048), empty(blocks * 8 * HE64)
    lab.ops.attention_context_chunked(dev(qkv), dev(past), tail, nxt, block_count=blocks)
    t = bits(tail)
    assert np.array_equal(t[1024:], contiguous_context(lab, qkv, keys, values))
    got = bits(nxt).reshape(blocks, 8 * HE64)
    for b in range(blocks - 1):
        assert np.array_equal(got[b], parts[b]), b
    lo = 64 * (blocks - 1)
    k2 = np.concatenate([keys[:, lo:], qkv[1024:1536].reshape(8, 1, 64)], axis=1)
    v2 = np.concatenate([values[:, lo:], qkv[1536:2048].reshape(8, 1, 64)], axis=1)
    assert np.array_equal(got[-1], headered(k2, v2, 64))


def test_headered_length_errors_set_status(gpu, lab):
    """A full last block (no room to append) is reported in status bit 0 and
    the head is left unwritten."""
    keys = O.bf16_bits(rs.standard_normal((8, 32, 64)).astype(np.float32))
    past = dev(headered(keys, keys, 32))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    tail, nxt = empty(2048), empty(8 * HE32)
    qkv_t = dev(qkv_hidden())  # held until the call is done
    lab._lib.call("lfm25_attention_fixed", qkv_t.data_ptr(), past.data_ptr(), tail.data_ptr(),
                  nxt.data_ptr(), 32, 1, status.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert int(status.item()) == 1
    assert np.all(np.isnan(O.f32(bits(tail))))
    with pytest.raises(ValueError):
        lab.ops.attention_context_chunked(dev(qkv_hidden()), past, tail, nxt, block_count=65)
    # the Python entry points raise instead of returning stale outputs
    with pytest.raises(ValueError, match="full"):
        lab.ops.attention_context_fixed(dev(qkv_hidden()), past, tail, nxt)
    assert np.all(np.isnan(O.f32(bits(tail)))) and np.all(np.isnan(O.f32(bits(nxt))))
    keys64 = O.bf16_bits(rs.standard_normal((8, 64, 64)).astype(np.float32))
    full64 = dev(headered(keys64, keys64, 64))
    with pytest.raises(ValueError, match="full"):
        lab.ops.attention_context_fixed64(dev(qkv_hidden()), full64, tail, empty(8 * HE64))
    with pytest.raises(ValueError, match="full"):
        lab.ops.attention_pair_context_fixed64(dev(np.concatenate([qkv_hidden(), qkv_hidden()])), full64,
                                               empty(4096), empty(8 * HE64))


def test_packing_programs_are_exact(gpu, lab):
    h = O.bf16_bits(rs.standard_normal(1024).astype(np.float32))
    h2 = O.bf16_bits(rs.standard_normal(1024).astype(np.float32))
    sw = O.bf16_bits(rs.standard_normal(6144).astype(np.float32))
    p3 = O.bf16_bits(rs.standard_normal(3072).astype(np.float32))
    out = empty(12288)
    lab.ops.pack_block_input(dev(h), dev(sw), out)
    assert np.array_equal(bits(out), np.concatenate([h, np.zeros(5120, np.uint16), sw]))
    out = empty(6144)
    lab.ops.pack_conv(dev(p3), dev(sw[:3072]), out)
    assert np.array_equal(bits(out), np.concatenate([p3, sw[:3072]]))
    out = empty(2048)
    lab.ops.pack_attention_tail(dev(h), dev(h2), out)
    assert np.array_equal(bits(out), np.concatenate([h, h2]))
    pair = empty(2048)
    lab.ops.concat_hidden_pair(dev(h), dev(h2), pair)
    assert np.array_equal(bits(pair), np.concatenate([h, h2]))
    a, b = empty(1024), empty(1024)
    lab.ops.split_hidden_pair(pair, a, b)
    assert np.array_equal(bits(a), h) and np.array_equal(bits(b), h2)
    out = empty(18432)
    lab.ops.pack_recurrent_pair(pair, dev(sw), out)
    z = np.zeros(5120, np.uint16)
    assert np.array_equal(bits(out), np.concatenate([h, z, h2, z, sw]))


def test_embedding_pair(gpu, lab):
    table = O.bf16_bits(rs.standard_normal((300, 1024)).astype(np.float32))
    pair = empty(2048)
    lab.ops.embedding_pair_dynamic(dev(table).view(300, 1024), pair,
                                   torch.tensor([7, 299], dtype=torch.int32, device="cuda"))
    assert np.array_equal(bits(pair), np.concatenate([table[7], table[299]]))


@pytest.mark.parametrize("M,K,N", [(16, 64, 64), (48, 1024, 3072), (64, 2560, 128)])
def test_bf16_f32_matmul(gpu, lab, M, K, N):
    """Within the FP32 summation bound K 2^-24 sum|a b| of the exact product;
    small-integer operands exactly."""
    a = O.bf16_bits(rs.standard_normal((M, K)).astype(np.float32))
    b = O.bf16_bits((0.02 * rs.standard_normal((K, N))).astype(np.float32))
    c = torch.empty(M * N, dtype=torch.float32, device="cuda")
    lab.ops.bf16_f32_matmul(dev(a), dev(b), c, M=M, K=K, N=N)
    got = c.cpu().numpy().reshape(M, N).astype(np.float64)
    fa, fb = O.f32(a).astype(np.float64), O.f32(b).astype(np.float64)
    exact = fa @ fb
    bound = K * 2.0 ** -24 * (np.abs(fa) @ np.abs(fb))
    assert np.all(np.abs(got - exact) <= bound + 1e-30)
    ai = rs.randint(-4, 5, size=(M, K)).astype(np.float32)
    bi = rs.randint(-4, 5, size=(K, N)).astype(np.float32)
    lab.ops.bf16_f32_matmul(dev_f(ai), dev_f(bi), c, M=M, K=K, N=N)
    assert np.array_equal(c.cpu().numpy().reshape(M, N), (ai.astype(np.float64) @ bi).astype(np.float32))
    with pytest.raises(ValueError):
        lab.ops.bf16_f32_matmul(dev(a), dev(b), c, M=M, K=K, N=N, n_cores=3)


def _conv_layer(lab, seed=23):
    ck = lab.weights.synthetic_checkpoint(seed, vocab=8, layers=3)
    names = O.layer_tensor_names(0)
    t = {n.split("layers.0.")[1]: ck[n] for n in names}
    pad = lambda a: np.concatenate([a.reshape(-1), np.zeros(4096 - a.size, np.uint16)])  # noqa: E731
    weights = np.concatenate([pad(t["operator_norm.weight"]), t["conv.in_proj.weight"].reshape(-1),
                              t["conv.out_proj.weight"].reshape(-1), pad(t["ffn_norm.weight"]),
                              t["feed_forward.w1.weight"].reshape(-1), t["feed_forward.w3.weight"].reshape(-1),
                              t["feed_forward.w2.weight"].reshape(-1)])
    return ck, t, weights


def _ulps(got, want) -> float:
    s = float(np.max(np.abs(want)))
    u = 2.0 ** (math.floor(math.log2(s)) - 7) if s > 0 else 1.0
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))) / u)


def test_norm_proj_conv(gpu, lab):
    """Norm, in_proj and gated conv: the gate within 2 ulps of its scale of the
    oracle's, the next state's shifted taps exact, the new tap within 2 ulps,
    the conv weight copied."""
    ck, t, _ = _conv_layer(lab)
    pad = np.zeros(4096 - 1024, np.uint16)
    packed_w = np.concatenate([t["operator_norm.weight"], pad, t["conv.in_proj.weight"].reshape(-1)])
    hidden = O.bf16_bits((0.5 * rs.standard_normal(1024)).astype(np.float32))
    state = O.bf16_bits(rs.standard_normal((1024, 3)).astype(np.float32))
    data = np.concatenate([hidden, np.zeros(5120, np.uint16), state.reshape(-1), t["conv.conv.weight"].reshape(-1)])
    gate, nxt = empty(1024), empty(6144)
    lab.ops.norm_proj_conv(dev(data), dev(packed_w), gate, nxt)
    n = O.rms_norm(O.f32(hidden), O.f32(t["operator_norm.weight"]))
    bcx = O.linear(t["conv.in_proj.weight"], n)
    y, new = O.conv_gate(bcx[:1024], bcx[1024:2048], bcx[2048:], O.f32(t["conv.conv.weight"]).reshape(1024, 3),
                         O.f32(state).reshape(1024, 3))
    assert _ulps(O.f32(bits(gate)), y) <= 2
    g = O.f32(bits(nxt))
    st = g[:3072].reshape(1024, 3)
    assert np.array_equal(st[:, :2], O.f32(state).reshape(1024, 3)[:, 1:])
    assert _ulps(st[:, 2], new[:, 2]) <= 2
    assert np.array_equal(bits(nxt)[3072:], t["conv.conv.weight"].reshape(-1))


@pytest.mark.parametrize("direct", [False, True])
def test_recurrent_pair(gpu, lab, direct):
    """Two positions through one conv layer: each output within 4 ulps of its
    scale of the oracle layer applied in turn (the second after the first's
    state), the final state within 2 ulps, and bit for bit two
    recurrent_block calls."""
    ck, t, weights = _conv_layer(lab)
    h0 = O.bf16_bits((0.5 * rs.standard_normal(1024)).astype(np.float32))
    h1 = O.bf16_bits((0.5 * rs.standard_normal(1024)).astype(np.float32))
    state = O.bf16_bits(rs.standard_normal((1024, 3)).astype(np.float32)).reshape(-1)
    conv_w = t["conv.conv.weight"].reshape(-1)
    nxt, out = empty(6144), empty(2048)
    if direct:
        lab.ops.recurrent_pair_direct(dev(np.concatenate([h0, h1])), dev(np.concatenate([state, conv_w])),
                                      dev(weights), nxt, out)
    else:
        z = np.zeros(5120, np.uint16)
        packed = np.concatenate([h0, z, h1, z, state, conv_w])
        lab.ops.recurrent_pair_block(dev(packed), dev(weights), nxt, out)
    orc = O.Oracle(ck, capacity=4, layers=3)
    orc.conv_states[0] = O.f32(state).reshape(1024, 3)
    want0 = orc.layer(0, O.f32(h0), 0, 0)
    want1 = orc.layer(0, O.f32(h1), 0, 0)
    got = O.f32(bits(out))
    assert _ulps(got[:1024], want0) <= 4 and _ulps(got[1024:], want1) <= 4
    assert _ulps(O.f32(bits(nxt)[:3072]).reshape(1024, 3), orc.conv_states[0]) <= 2
    assert np.array_equal(bits(nxt)[3072:], conv_w)
    # the same two positions as two one-position calls
    z = np.zeros(5120, np.uint16)
    s1, o0 = empty(6144), empty(1024)
    lab.ops.recurrent_block(dev(np.concatenate([h0, z, state, conv_w])), dev(weights), s1, o0)
    s2, o1 = empty(6144), empty(1024)
    lab.ops.recurrent_block(dev(np.concatenate([h1, z, bits(s1)])), dev(weights), s2, o1)
    assert np.array_equal(bits(out), np.concatenate([bits(o0), bits(o1)]))
    assert np.array_equal(bits(nxt), bits(s2))


def _attention_weights(lab, seed=29):
    ck = lab.weights.synthetic_checkpoint(seed, vocab=8, layers=3)
    names = O.layer_tensor_names(2)
    t = {n.split("layers.2.")[1]: ck[n] for n in names}
    pad = lambda a: np.concatenate([a.reshape(-1), np.zeros(4096 - a.size, np.uint16)])  # noqa: E731
    qkv = np.concatenate([t["self_attn.q_proj.weight"].reshape(-1), t["self_attn.k_proj.weight"].reshape(-1),
                          t["self_attn.v_proj.weight"].reshape(-1)])

    def aux(pos):
        cos, sin = O.rope_table([pos])
        return pad(np.concatenate([t["self_attn.q_layernorm.weight"], t["self_attn.k_layernorm.weight"],
                                   O.bf16_bits(cos[0]), O.bf16_bits(sin[0])]))

    prefix = lambda pos: np.concatenate([pad(t["operator_norm.weight"]), qkv, aux(pos)])  # noqa: E731
    tail = np.concatenate([t["self_attn.out_proj.weight"].reshape(-1), pad(t["ffn_norm.weight"]),
                           t["feed_forward.w1.weight"].reshape(-1), t["feed_forward.w3.weight"].reshape(-1),
                           t["feed_forward.w2.weight"].reshape(-1)])
    return prefix, aux, tail


def test_attention_pair_programs(gpu, lab):
    """attention_prefix_pair, attention_pair_context_fixed64 and
    attention_tail_pair at positions 5 and 6 of a capacity-64 headered cache
    give bit for bit the outputs of the one-position programs called in turn."""
    prefix, aux, tail_w = _attention_weights(lab)
    h = [O.bf16_bits((0.5 * rs.standard_normal(1024)).astype(np.float32)) for _ in range(2)]
    keys = O.bf16_bits(rs.standard_normal((8, 5, 64)).astype(np.float32))
    values = O.bf16_bits(rs.standard_normal((8, 5, 64)).astype(np.float32))
    cache = dev(headered(keys, values, 64))
    qkv_pair = empty(6144)
    lab.ops.attention_prefix_pair(dev(np.concatenate(h)), dev(prefix(5)), dev(aux(6)), qkv_pair)
    tail_pair, nxt = empty(4096), empty(8 * HE64)
    lab.ops.attention_pair_context_fixed64(qkv_pair, cache, tail_pair, nxt)
    out_pair = empty(2048)
    lab.ops.attention_tail_pair(tail_pair, dev(tail_w), out_pair)
    # one position at a time
    cur, outs, tails = cache, [], []
    for i, pos in enumerate((5, 6)):
        q = empty(3072)
        lab.ops.attention_prefix(dev(h[i]), dev(prefix(pos)), q, include_hidden=True)
        assert np.array_equal(bits(q), bits(qkv_pair)[3072 * i:3072 * (i + 1)]), i
        t, n = empty(2048), empty(8 * HE64)
        lab.ops.attention_context_fixed64(q, cur, t, n)
        tails.append(bits(t))
        o = empty(1024)
        lab.ops.attention_tail(t, dev(tail_w), o)
        outs.append(bits(o))
        cur = n
    assert np.array_equal(bits(tail_pair), np.concatenate(tails))
    assert np.array_equal(bits(nxt), bits(cur))
    assert np.array_equal(bits(out_pair), np.concatenate(outs))


def test_fused_vocab_4core_equals_fused_vocab(gpu, lab):
    table = lab.rng.normal_bf16(4, "v4.E", 65536 * 1024, 0.0, 0.02)
    gamma = lab.rng.normal_bf16(4, "v4.g", 1024, 1.0, 0.02)
    hidden = lab.rng.normal_bf16(4, "v4.h", 1024)
    packed = dev(np.concatenate([gamma, table]))
    res = []
    for fn in (lab.ops.fused_vocab, lab.ops.fused_vocab_4core):
        nxt, tok = empty(1024), torch.zeros(1, dtype=torch.int32, device="cuda")
        fn(dev(hidden), packed, nxt, tok)
        res.append((int(tok.item()), bits(nxt)))
    assert res[0][0] == res[1][0] and np.array_equal(res[0][1], res[1][1])
    assert np.array_equal(res[0][1], table.reshape(65536, 1024)[res[0][0]])
    with pytest.raises(ValueError):
        lab.ops.fused_vocab_4core(dev(hidden), packed[:1024 + 4 * 1024], nxt, tok)
