"""Per-operation parity on the GPU: each reference entry point (ops.*) against
the CPU oracle on identical seeded inputs.

Bars (the tolerance is stated in each test):
  * element-wise ops (add, cast, SiLU gate, conv gate, QK norm + RoPE, KV
    append, embedding gather) perform the same FP32 operations as the oracle
    in the same order and must be bit-exact;
  * dot products accumulate in FP32 in the kernel's fixed order while the
    oracle takes exact sums, so outputs must be bit-exact on small-integer
    inputs (every partial sum exact) and, on random data, differ on at most
    1% of elements and never by more than one BF16 ulp plus the FP32
    summation error bound K * 2**-24 * sum|w x| (assert_dot_parity);
  * argmax must pick the oracle's index unless the oracle's top-2 BF16
    logits are within one ulp (a near-tie), and must keep the first index
    on exact ties.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import lfm25 as O
from parity_helpers import attention_interval

pytestmark = pytest.mark.gpu

# Shared by the tests below in file order, so a test's inputs depend on the
# draws of every test before it: new tests take a generator of their own.
rs = np.random.RandomState(20260101)


def dev(bits: np.ndarray) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16).reshape(-1))
    return t.cuda().view(torch.bfloat16)


def dev_f(x: np.ndarray) -> torch.Tensor:
    return dev(O.bf16_bits(x))


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return O.f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def empty(n: int) -> torch.Tensor:
    return torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")


def bf(x):
    return O._bf(np.asarray(x, np.float32))


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ua = O.bf16_bits(a).astype(np.int32)
    ub = O.bf16_bits(b).astype(np.int32)
    ua = np.where(ua & 0x8000, 0x8000 - ua, ua)
    ub = np.where(ub & 0x8000, 0x8000 - ub, ub)
    return np.abs(ua - ub)


def assert_dot_parity(got: np.ndarray, want: np.ndarray, w_bits: np.ndarray, x: np.ndarray,
                      what: str):
    """GPU bf16(FP32-accumulated W.x) vs oracle bf16(exact W.x): the FP32 sum
    of K terms is within K * 2**-24 * sum|w x| of the exact sum (the standard
    recursive-summation bound), and each side rounds once to BF16, so
    |got - want| <= ulp(want) + K * 2**-24 * sum_k |w_k x_k| for every row;
    beyond that, at most 1% of the rows may differ at all, and all rows meet
    the target's relative tolerance 1e-2 (or that bound, near zero)."""
    k = x.size
    mag = np.abs(O.f32(w_bits).reshape(-1, k)).astype(np.float64) @ np.abs(x).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    bound = ulp + k * 2.0 ** -24 * mag
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound), (what, float((err / bound).max()))
    assert np.all((err <= 1e-2 * np.abs(want)) | (err <= bound)), what
    assert np.mean(got != want) <= 0.01, (what, float(np.mean(got != want)))


# ------------------------------------------------------------------ norms / GEMV


def test_rms_norm(gpu, lab):
    for n in (1024, 64, 2560):
        x = bf(rs.standard_normal(n))
        g = bf(1 + 0.02 * rs.standard_normal(n))
        out = empty(n)
        lab.ops.rms_norm(dev_f(x), dev_f(g), out, N=n)
        got, want = host(out), O.rms_norm(x, g)
        d = ulp_diff(got, want)
        assert d.max() <= 1 and np.mean(d > 0) <= 0.002, (n, np.mean(d > 0))
    # small integers: the sum of squares is exact, so bits match exactly
    x = rs.randint(-6, 7, size=1024).astype(np.float32)
    out = empty(1024)
    lab.ops.rms_norm(dev_f(x), dev_f(np.ones(1024)), out, N=1024)
    assert np.array_equal(host(out), O.rms_norm(x, np.ones(1024, np.float32)))


@pytest.mark.parametrize("M,K", [(3072, 1024), (1024, 2560), (1000, 1024), (96, 704), (7, 8)])
def test_bf16_gemv_small_integers_bit_exact(gpu, lab, M, K):
    w = rs.randint(-3, 4, size=(M, K)).astype(np.float32)
    x = rs.randint(-3, 4, size=K).astype(np.float32)
    out = empty(M)
    lab.ops.bf16_bf16_gemv(dev_f(w), dev_f(x), out, M=M, K=K)
    assert np.array_equal(host(out), O.linear(O.bf16_bits(w), x))
    out32 = torch.empty(M, dtype=torch.float32, device="cuda")
    lab.ops.bf16_f32_gemv(dev_f(w), dev_f(x), out32, M=M, K=K)
    torch.cuda.synchronize()
    assert np.array_equal(out32.cpu().numpy(), O.linear_f32(O.bf16_bits(w), x))


@pytest.mark.parametrize("M,K", [(3072, 1024), (1024, 2560), (512, 704)])
def test_bf16_gemv_random(gpu, lab, M, K):
    w = bf(0.02 * rs.standard_normal((M, K)))
    x = bf(rs.standard_normal(K))
    out = empty(M)
    lab.ops.bf16_bf16_gemv(dev_f(w), dev_f(x), out, M=M, K=K)
    assert_dot_parity(host(out), O.linear(O.bf16_bits(w), x), O.bf16_bits(w), x, f"gemv {M}x{K}")
    out32 = torch.empty(M, dtype=torch.float32, device="cuda")
    lab.ops.bf16_f32_gemv(dev_f(w), dev_f(x), out32, M=M, K=K)
    torch.cuda.synchronize()
    assert np.allclose(out32.cpu().numpy(), O.linear_f32(O.bf16_bits(w), x), rtol=1e-5, atol=1e-6)


def _config1(lab, seed=1):
    """Fused RMSNorm + GEMV workload: x[1024] ~ N(0,1), gamma ~ 1+N(0,0.02),
    W[3072x1024] ~ N(0,0.02), all from one seed."""
    x = lab.rng.normal_bf16(seed, "c1.x", 1024)
    g = lab.rng.normal_bf16(seed, "c1.gamma", 1024, 1.0, 0.02)
    w = lab.rng.normal_bf16(seed, "c1.w", 3072 * 1024, 0.0, 0.02).reshape(3072, 1024)
    return x, g, w


def test_norm_bf16_gemv_config1(gpu, lab):
    x, g, w = _config1(lab)
    packed = np.concatenate([g, np.zeros(4096 - 1024, np.uint16), w.reshape(-1)])
    out = empty(3072)
    lab.ops.norm_bf16_gemv(dev(x), dev(packed), out, M=3072, K=1024)
    n = O.rms_norm(O.f32(x), O.f32(g))
    assert_dot_parity(host(out), O.linear(w, n), w, n, "norm_bf16_gemv config 1")


def test_norm_bf16_gemv_small_integers_bit_exact(gpu, lab):
    x = rs.randint(-2, 3, size=1024).astype(np.float32)
    x[0] = 2.0
    w = rs.randint(-2, 3, size=(256, 1024)).astype(np.float32)
    packed = np.concatenate([O.bf16_bits(np.ones(1024, np.float32)), np.zeros(3072, np.uint16),
                             O.bf16_bits(w).reshape(-1)])
    out = empty(256)
    lab.ops.norm_bf16_gemv(dev_f(x), dev(packed), out, M=256, K=1024)
    want = O.linear(O.bf16_bits(w), O.rms_norm(x, np.ones(1024, np.float32)))
    assert np.array_equal(host(out), want)


# K = 1024 takes R = ceil(M / 1024) rows per wave, at most 4 (the tests above
# run R = 1 and 3): 2048 and 1537 / 2047 run R = 2, 4099 R = 4, and 1537,
# 2047 and 4099 end on a partial unit, whose missing rows are read clamped
# and never stored. Own generator, so the inputs of the other tests do not
# depend on these cases.
@pytest.mark.parametrize("M,norm", [(2048, False), (1537, False), (4099, False), (2047, True), (4099, True)])
def test_gemv_rows_per_wave_forms_bit_exact(gpu, lab, M, norm):
    r = np.random.RandomState(M + 7 * norm)
    x = r.randint(-2, 3, size=1024).astype(np.float32)
    w = r.randint(-2, 3, size=(M, 1024)).astype(np.float32)
    out = empty(M)
    if norm:
        x[0] = 2.0
        packed = np.concatenate([O.bf16_bits(np.ones(1024, np.float32)), np.zeros(3072, np.uint16),
                                 O.bf16_bits(w).reshape(-1)])
        lab.ops.norm_bf16_gemv(dev_f(x), dev(packed), out, M=M, K=1024)
        assert np.array_equal(host(out), O.linear(O.bf16_bits(w), O.rms_norm(x, np.ones(1024, np.float32))))
    else:
        lab.ops.bf16_bf16_gemv(dev_f(w), dev_f(x), out, M=M, K=1024)
        assert np.array_equal(host(out), O.linear(O.bf16_bits(w), x))
        out32 = torch.empty(M, dtype=torch.float32, device="cuda")
        lab.ops.bf16_f32_gemv(dev_f(w), dev_f(x), out32, M=M, K=1024)
        torch.cuda.synchronize()
        assert np.array_equal(out32.cpu().numpy(), O.linear_f32(O.bf16_bits(w), x))


# ------------------------------------------------------------------ element-wise


def test_f32_to_bf16_and_add_exact(gpu, lab):
    x = (rs.standard_normal(4099) * 1000).astype(np.float32)
    specials = np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x00000001, 0x80000000],
                        np.uint32).view(np.float32)
    x[:5] = specials
    out = empty(x.size)
    lab.ops.f32_to_bf16(torch.from_numpy(x).cuda(), out, N=x.size)
    assert np.array_equal(host(out).view(np.uint32), O._bf(x).view(np.uint32))
    # Every exponent (denormals, Inf and NaN payloads included) with the
    # rounding-boundary mantissas (ties to even and odd, one above and below)
    # and random mantissas, both signs.
    exps = np.arange(256, dtype=np.uint32) << 23
    mant = np.concatenate([np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0x17FFF, 0x18000, 0x18001,
                                     0x400000, 0x7FFFFF, 0x7F8000, 0x7FFFFE], np.uint32),
                           rs.randint(0, 1 << 23, 52).astype(np.uint32)])
    bits = (exps[:, None] | mant[None, :]).reshape(-1)
    bits = np.concatenate([bits, bits | 0x80000000])
    x = bits.view(np.float32)
    out = empty(x.size)
    lab.ops.f32_to_bf16(torch.from_numpy(x.copy()).cuda(), out, N=x.size)
    assert np.array_equal(host(out).view(np.uint32), O._bf(x).view(np.uint32))
    a, b = bf(rs.standard_normal(3000)), bf(rs.standard_normal(3000) * 1e-3)
    out = empty(3000)
    lab.ops.bf16_add(dev_f(a), dev_f(b), out, N=3000)
    assert np.array_equal(host(out), O.bf16_add(a, b))


def test_silu_gate_exhaustive(gpu, lab):
    """All 65,536 BF16 gate inputs (the reference's SiLU table domain)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = O.f32(bits)
    fin = np.isfinite(x)
    w1 = bits[fin]
    ones = O.bf16_bits(np.ones(w1.size, np.float32))
    out = empty(w1.size)
    lab.ops.silu_gate(dev(w1), dev(ones), out, N=w1.size)
    got, want = host(out), O.silu_gate(O.f32(w1), np.ones(w1.size, np.float32))
    mism = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    # GPU expf and numpy's float32 exp may differ in the last FP32 ulp, which
    # can move a BF16 rounding only at a handful of inputs
    assert mism.size <= 8, (mism.size, [hex(int(w1[i])) for i in mism[:8]])
    assert ulp_diff(got[mism], want[mism]).max(initial=0) <= 1
    w3 = bf(rs.standard_normal(2560))
    g = bf(rs.standard_normal(2560) * 3)
    out = empty(2560)
    lab.ops.silu_gate(dev_f(g), dev_f(w3), out, N=2560)
    assert np.array_equal(host(out), O.silu_gate(g, w3))


def test_conv_gate_exact(gpu, lab):
    B, C, xs = (bf(rs.standard_normal(1024)) for _ in range(3))
    w = bf(0.3 * rs.standard_normal((1024, 3)))
    s = bf(rs.standard_normal((1024, 3)))
    y_want, s_want = O.conv_gate(B, C, xs, w, s)
    packed = np.concatenate([B, C, xs, w.reshape(-1)])
    out, nxt = empty(1024), empty(3072)
    lab.ops.conv_gate(dev_f(packed), dev_f(s), out, nxt)
    assert np.array_equal(host(out), y_want)
    assert np.array_equal(host(nxt).reshape(1024, 3), s_want)
    out, nxt = empty(1024), empty(6144)
    lab.ops.conv_gate_packed_state(dev_f(np.concatenate([B, C, xs])),
                                   dev_f(np.concatenate([s.reshape(-1), w.reshape(-1)])), out, nxt)
    assert np.array_equal(host(out), y_want)
    got = host(nxt)
    assert np.array_equal(got[:3072].reshape(1024, 3), s_want)
    assert np.array_equal(got[3072:], w.reshape(-1))


# ------------------------------------------------------------------ attention


def _rope(pos):
    cos, sin = O.rope_table([pos])
    return cos[0], sin[0]


def test_attention_norm_rope_exact(gpu, lab):
    qkv = bf(rs.standard_normal(2048))
    qg, kg = bf(1 + 0.02 * rs.standard_normal(64)), bf(1 + 0.02 * rs.standard_normal(64))
    cos, sin = _rope(777)
    aux = np.concatenate([qg, kg, cos, sin])
    t = dev_f(qkv)
    aux_t = dev_f(aux)  # held until the call is done
    lab._lib.call("lfm25_attention_norm_rope", t.data_ptr(), aux_t.data_ptr(),
                  torch.cuda.current_stream().cuda_stream)
    got = host(t)
    q = O.norm_rope(qkv[:1024].reshape(16, 64), qg, cos, sin).reshape(-1)
    k = O.norm_rope(qkv[1024:1536].reshape(8, 64), kg, cos, sin).reshape(-1)
    d = ulp_diff(got[:1536], np.concatenate([q, k]))
    # the 64-term sum of squares is the only reordered reduction
    assert d.max() <= 1 and np.mean(d > 0) <= 0.01
    assert np.array_equal(got[1536:], qkv[1536:])


@pytest.mark.parametrize("past", [0, 1, 21, 127, 1023, 4095])
def test_attention_context(gpu, lab, past):
    qkv = bf(rs.standard_normal(2048))
    keys, vals = bf(rs.standard_normal((8, past, 64))), bf(rs.standard_normal((8, past, 64)))
    cache = np.concatenate([keys, vals], axis=1).reshape(-1)       # per head [K | V]
    ctx = empty(1024)
    cache_t = dev_f(cache) if past else torch.zeros(8, dtype=torch.bfloat16, device="cuda")
    qkv_t = dev_f(qkv)
    lab._lib.call("lfm25_attention_context", qkv_t.data_ptr(), cache_t.data_ptr(),
                  ctx.data_ptr(), past, torch.cuda.current_stream().cuda_stream)
    k_all = np.concatenate([keys, qkv[1024:1536].reshape(8, 1, 64)], axis=1)
    v_all = np.concatenate([vals, qkv[1536:].reshape(8, 1, 64)], axis=1)
    want = O.attention(qkv[:1024].reshape(16, 64), k_all, v_all)
    got = host(ctx)
    assert np.allclose(got, want, rtol=1e-2, atol=1e-3), past
    # every element inside the interval the oracle's algorithm allows for FP32
    # sums in another order (past + 1 terms and up to 64 partials per sum)
    lo, hi = attention_interval(qkv[:1024].reshape(16, 64), k_all, v_all, past + 1 + 64)
    g = got.astype(np.float64)
    outside = np.flatnonzero((g < lo) | (g > hi))
    d = ulp_diff(got, want)
    assert outside.size == 0, (past, outside[:8], int(d.max()))
    assert np.mean(d > 0) <= 0.05, (past, int(d.max()), float(np.mean(d > 0)))


@pytest.mark.parametrize("past", [1, 127, 1023, 4095])
@pytest.mark.parametrize("seed", [11, 12])
def test_attention_context_inside_interval(gpu, lab, past, seed):
    """Inputs of their own (not the module's shared generator), held only to
    the derived interval: no allowance tuned to particular data."""
    r = np.random.RandomState(1000 * seed + past)
    qkv = bf(r.standard_normal(2048))
    keys, vals = bf(r.standard_normal((8, past, 64))), bf(r.standard_normal((8, past, 64)))
    cache = np.concatenate([keys, vals], axis=1).reshape(-1)
    ctx = empty(1024)
    # every device tensor held until the call is done (a temporary freed right
    # after its data_ptr() hands its block to the next allocation)
    qkv_t, cache_t = dev_f(qkv), dev_f(cache)
    lab._lib.call("lfm25_attention_context", qkv_t.data_ptr(), cache_t.data_ptr(),
                  ctx.data_ptr(), past, torch.cuda.current_stream().cuda_stream)
    k_all = np.concatenate([keys, qkv[1024:1536].reshape(8, 1, 64)], axis=1)
    v_all = np.concatenate([vals, qkv[1536:].reshape(8, 1, 64)], axis=1)
    lo, hi = attention_interval(qkv[:1024].reshape(16, 64), k_all, v_all, past + 1 + 64)
    g = host(ctx).astype(np.float64)
    outside = np.flatnonzero((g < lo) | (g > hi))
    assert outside.size == 0, (past, seed, outside[:8])


def test_append_attention_cache_exact(gpu, lab):
    past = 21
    qkv = bf(rs.standard_normal(2048))
    prior = bf(rs.standard_normal(8 * 2 * past * 64))
    nxt = empty(8 * 2 * (past + 1) * 64)
    lab.ops.append_attention_cache(dev_f(qkv), dev_f(prior), nxt)
    got = host(nxt).reshape(8, 2, past + 1, 64)
    p = prior.reshape(8, 2, past, 64)
    assert np.array_equal(got[:, :, :past], p)
    assert np.array_equal(got[:, 0, past], qkv[1024:1536].reshape(8, 64))
    assert np.array_equal(got[:, 1, past], qkv[1536:].reshape(8, 64))


# ------------------------------------------------------------------ head / argmax / embedding


def test_vocab_argmax_ties_and_random(gpu, lab):
    logits = bf(rs.standard_normal(65536))
    logits[[40000, 123, 65535]] = 7.0
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    lab.ops.vocab_argmax(dev_f(logits), tok)
    assert int(tok.item()) == 123
    logits = bf(rs.standard_normal(65536))
    lab.ops.vocab_argmax(dev_f(logits), tok)
    assert int(tok.item()) == O.argmax_first(logits)


def test_fused_vocab(gpu, lab):
    table = lab.rng.normal_bf16(3, "head.E", 65536 * 1024, 0.0, 0.02).reshape(65536, 1024)
    gamma = lab.rng.normal_bf16(3, "head.g", 1024, 1.0, 0.02)
    hidden = lab.rng.normal_bf16(3, "head.h", 1024)
    packed = dev(np.concatenate([gamma, table.reshape(-1)]))
    nxt, tok, logits = empty(1024), torch.zeros(1, dtype=torch.int32, device="cuda"), empty(65536)
    lab.ops.fused_vocab(dev(hidden), packed, nxt, tok, logits=logits)
    n = O.rms_norm(O.f32(hidden), O.f32(gamma))
    want = O.linear(table, n)
    got = host(logits)
    assert_dot_parity(got, want, table, n, "head logits")
    t = int(tok.item())
    assert t == O.argmax_first(got)                 # first maximum of its own logits
    best = want.max()
    ulp = 2.0 ** (math.floor(math.log2(abs(best))) - 7)
    assert want[t] >= best - ulp                    # oracle argmax unless a near-tie
    assert np.array_equal(host(nxt), O.f32(table[t]))


def test_embedding_gather(gpu, lab):
    table = bf(rs.standard_normal((300, 1024)))
    out = empty(1024)
    lab.ops.embedding_dma(dev_f(table).view(300, 1024), out, token_id=299)
    assert np.array_equal(host(out), table[299])
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    tid = torch.tensor([1000], dtype=torch.int32, device="cuda")
    table_t = dev_f(table)  # held until the call is done
    lab._lib.call("lfm25_embedding_gather", table_t.data_ptr(), tid.data_ptr(),
                  out.data_ptr(), 300, status.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert int(status.item()) == 1 and np.array_equal(host(out), table[299])


# ------------------------------------------------------------------ composite entry points


def _layer_ck(lab, kind, seed=9):
    ck = lab.weights.synthetic_checkpoint(seed, vocab=8, layers=3)
    idx = 0 if kind == "conv" else 2
    return ck, idx


def test_recurrent_block(gpu, lab):
    ck, idx = _layer_ck(lab, "conv")
    names = O.layer_tensor_names(idx)
    t = {n.split(f"layers.{idx}.")[1]: ck[n] for n in names}
    hidden = bf(rs.standard_normal(1024) * 0.5)
    state = bf(rs.standard_normal((1024, 3)))
    pad = lambda a: np.concatenate([a.reshape(-1), np.zeros(4096 - a.size, np.uint16)])  # noqa: E731
    weights = np.concatenate([pad(t["operator_norm.weight"]), t["conv.in_proj.weight"].reshape(-1),
                              t["conv.out_proj.weight"].reshape(-1), pad(t["ffn_norm.weight"]),
                              t["feed_forward.w1.weight"].reshape(-1),
                              t["feed_forward.w3.weight"].reshape(-1),
                              t["feed_forward.w2.weight"].reshape(-1)])
    data = np.concatenate([O.bf16_bits(hidden), np.zeros(6144 - 1024, np.uint16),
                           O.bf16_bits(state).reshape(-1), t["conv.conv.weight"].reshape(-1)])
    nxt, out = empty(6144), empty(1024)
    lab.ops.recurrent_block(dev(data), dev(weights), nxt, out)
    orc = O.Oracle(ck, capacity=4, layers=3)
    orc.conv_states[0] = state.copy()
    want = orc.layer(idx, hidden, 0, 0)
    got = host(out)
    assert np.allclose(got, want, rtol=1e-2, atol=2e-2)
    scale = float(np.abs(want).max())
    assert np.abs(got - want).max() <= 4 * 2.0 ** (math.floor(math.log2(scale)) - 7)
    assert np.array_equal(host(nxt)[:3072].reshape(1024, 3)[:, :2], state[:, 1:])


# ------------------------------------------------------------------ 8-bit weights


def _w8_dev(q, s):
    return torch.from_numpy(q).cuda(), torch.from_numpy(np.ascontiguousarray(s, np.float32)).cuda()


@pytest.mark.parametrize("group", [0, 32, 64])
def test_w8_gemv_small_integers_bit_exact(gpu, lab, group):
    """Small-integer activations and weights with power-of-two scales: every
    sum is exact, so the GPU matches the oracle bit for bit."""
    M, K = 512, 1024
    q = rs.randint(-6, 7, size=(M, K)).astype(np.int8)
    x = rs.randint(-3, 4, size=K).astype(np.float32)
    shape = (M, K // group) if group else (M,)
    s = (np.float32(2.0) ** rs.randint(-4, 2, size=shape)).astype(np.float32)
    out = empty(M)
    qd, sd = _w8_dev(q, s)
    lab.ops.w8_gemv(qd, sd, dev_f(x), out, M=M, K=K, group=group)
    assert np.array_equal(host(out), O.linear_w8(q, s, group, x))


@pytest.mark.parametrize("M,K", [(3072, 1024), (1024, 2560), (8192, 1024), (192, 4096)])
@pytest.mark.parametrize("group", [0, 32, 64])
def test_w8_gemv_random(gpu, lab, M, K, group):
    """Weights ~ N(0, 0.02) quantized as the reference does, x ~ N(0, 1):
    within one BF16 ulp plus the FP32 summation bound (K + 4) 2^-24 sum|w x|
    of the oracle's exactly summed result (the GPU sums q x per 16-input
    segment, scales, then accumulates); at most 1% of rows differ."""
    w = O.bf16_bits((0.02 * rs.standard_normal((M, K))).astype(np.float32))
    q, s = lab.weights.quantize_w8(w, group)
    x = bf(rs.standard_normal(K))
    out = empty(M)
    qd, sd = _w8_dev(q, s)
    lab.ops.w8_gemv(qd, sd, dev_f(x), out, M=M, K=K, group=group)
    got, want = host(out), O.linear_w8(q, s, group, x)
    mag = np.abs(O.dequantize_w8(q, s, group)).astype(np.float64) @ np.abs(x).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= ulp + (K + 4) * 2.0 ** -24 * mag), float((err / (ulp + (K + 4) * 2.0 ** -24 * mag)).max())
    assert np.mean(got != want) <= 0.01, float(np.mean(got != want))


def test_w8_gemv_close_to_bf16_weights(gpu, lab):
    """The 8-bit GEMV tracks the BF16 GEMV of the unquantized weights within
    the quantization error (relative RMS < 1% at group 32, as the reference
    reports for w8g32)."""
    M, K = 3072, 1024
    w = O.bf16_bits((0.02 * rs.standard_normal((M, K))).astype(np.float32))
    x = bf(rs.standard_normal(K))
    q, s = lab.weights.quantize_w8(w, 32)
    out, ref = empty(M), empty(M)
    qd, sd = _w8_dev(q, s)
    lab.ops.w8_gemv(qd, sd, dev_f(x), out, M=M, K=K, group=32)
    lab.ops.bf16_bf16_gemv(dev(w), dev_f(x), ref, M=M, K=K)
    a, b = host(out).astype(np.float64), host(ref).astype(np.float64)
    assert np.sqrt(np.mean((a - b) ** 2) / np.mean(b ** 2)) < 0.01


def _attention_layer_inputs(lab, past, seed=11):
    """A synthetic attention layer (layer 2), its reference packings and a
    pre-filled cache of `past` positions (per KV head [keys P x 64 | values P
    x 64], the reference's past_cache layout)."""
    ck, idx = _layer_ck(lab, "attention", seed)
    names = O.layer_tensor_names(idx)
    t = {n.split(f"layers.{idx}.")[1]: ck[n] for n in names}
    pad = lambda a: np.concatenate([a.reshape(-1), np.zeros(4096 - a.size, np.uint16)])  # noqa: E731
    cos, sin = _rope(past)
    aux = np.concatenate([t["self_attn.q_layernorm.weight"], t["self_attn.k_layernorm.weight"],
                          O.bf16_bits(cos), O.bf16_bits(sin)])
    prefix_w = np.concatenate([pad(t["operator_norm.weight"]), t["self_attn.q_proj.weight"].reshape(-1),
                               t["self_attn.k_proj.weight"].reshape(-1), t["self_attn.v_proj.weight"].reshape(-1),
                               pad(aux)])
    tail_w = np.concatenate([t["self_attn.out_proj.weight"].reshape(-1), pad(t["ffn_norm.weight"]),
                             t["feed_forward.w1.weight"].reshape(-1), t["feed_forward.w3.weight"].reshape(-1),
                             t["feed_forward.w2.weight"].reshape(-1)])
    keys, vals = bf(rs.standard_normal((8, past, 64))), bf(rs.standard_normal((8, past, 64)))
    return ck, idx, t, prefix_w, tail_w, keys, vals


@pytest.mark.parametrize("past", [21, 300])
def test_attention_layer_composites(gpu, lab, past):
    """The reference's three-call attention layer (006_lfm25_npu_layer_stack.py:
    181-190): attention_prefix -> attention_context_cache -> attention_tail,
    against Oracle.layer at position `past`. Each stage is held to its own bar:
    q / k / v within 2 ulps of each head's scale (a dot product, then QK norm
    and RoPE), the context within 2 ulps of the oracle's attention over the
    GPU's own q / k / v, the next cache and the tail input bit-exact copies,
    the block output within 4 ulps of its scale (as recurrent_block)."""
    ck, idx, t, prefix_w, tail_w, keys, vals = _attention_layer_inputs(lab, past)
    hidden = bf(rs.standard_normal(1024) * 0.5)
    qkv = empty(2048 + 1024)
    lab.ops.attention_prefix(dev_f(hidden), dev(prefix_w), qkv, include_hidden=True)
    orc = O.Oracle(ck, capacity=past + 1, layers=3)
    orc.keys[0][:, :past] = keys
    orc.values[0][:, :past] = vals
    orc.position = past
    n = O.rms_norm(hidden, O.f32(t["operator_norm.weight"]))
    cos, sin = _rope(past)
    q_w = O.norm_rope(O.linear(t["self_attn.q_proj.weight"], n).reshape(16, 64),
                      O.f32(t["self_attn.q_layernorm.weight"]), cos, sin)
    k_w = O.norm_rope(O.linear(t["self_attn.k_proj.weight"], n).reshape(8, 64),
                      O.f32(t["self_attn.k_layernorm.weight"]), cos, sin)
    v_w = O.linear(t["self_attn.v_proj.weight"], n).reshape(8, 64)
    got_qkv = host(qkv)
    for h in range(16):
        assert scale_ulps_vec(got_qkv[64 * h:64 * h + 64], q_w[h]) <= 2, ("q", h)
    for h in range(8):
        assert scale_ulps_vec(got_qkv[1024 + 64 * h:1088 + 64 * h], k_w[h]) <= 2, ("k", h)
        assert scale_ulps_vec(got_qkv[1536 + 64 * h:1600 + 64 * h], v_w[h]) <= 2, ("v", h)
    assert np.array_equal(got_qkv[2048:], hidden)
    cache = np.concatenate([keys, vals], axis=1).reshape(-1)
    tail_in, nxt = empty(2048), empty(8 * 2 * (past + 1) * 64)
    lab.ops.attention_context_cache(qkv, dev_f(cache), tail_in, nxt, past_length=past)
    g_q, g_k, g_v = got_qkv[:1024].reshape(16, 64), got_qkv[1024:1536].reshape(8, 64), got_qkv[1536:2048].reshape(8, 64)
    ctx_want = O.attention(g_q, np.concatenate([keys, g_k[:, None]], axis=1),
                           np.concatenate([vals, g_v[:, None]], axis=1))
    got_tail_in = host(tail_in)
    assert np.array_equal(got_tail_in[:1024], hidden)
    d = ulp_diff(got_tail_in[1024:], ctx_want)
    assert d.max() <= 2 and np.mean(d > 0) <= 0.05, (int(d.max()), float(np.mean(d > 0)))
    got_next = host(nxt).reshape(8, 2, past + 1, 64)
    assert np.array_equal(got_next[:, 0, :past], keys) and np.array_equal(got_next[:, 1, :past], vals)
    assert np.array_equal(got_next[:, 0, past], g_k) and np.array_equal(got_next[:, 1, past], g_v)
    out = empty(1024)
    lab.ops.attention_tail(tail_in, dev(tail_w), out)
    want = orc.layer(idx, hidden, 0, 0)
    got = host(out)
    assert np.allclose(got, want, rtol=1e-2, atol=2e-2)
    assert scale_ulps_vec(got, want) <= 4


def scale_ulps_vec(got, want) -> float:
    s = float(np.max(np.abs(want)))
    u = 2.0 ** (math.floor(math.log2(s)) - 7) if s > 0 else 1.0
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))) / u)


@pytest.mark.parametrize("M,K", [(5, 1024), (4097, 1024), (3, 2560)])
@pytest.mark.parametrize("group", [0, 32])
def test_w8_gemv_ragged_rows(gpu, lab, M, K, group):
    """Row counts that leave the last 4-row unit partly empty: the missing
    rows read nothing and every present row meets the small-integer bar
    (bit-exact with power-of-two scales)."""
    q = rs.randint(-6, 7, size=(M, K)).astype(np.int8)
    x = rs.randint(-3, 4, size=K).astype(np.float32)
    shape = (M, K // group) if group else (M,)
    s = (np.float32(2.0) ** rs.randint(-4, 2, size=shape)).astype(np.float32)
    out = empty(M + 4)
    qd, sd = _w8_dev(q, s)
    lab.ops.w8_gemv(qd, sd, dev_f(x), out[:M], M=M, K=K, group=group)
    got = host(out)
    assert np.array_equal(got[:M], O.linear_w8(q, s, group, x))
    assert np.all(np.isnan(got[M:]))  # nothing written past row M - 1


@pytest.mark.parametrize("past,capacity", [(0, 64), (21, 64), (300, 512), (4000, 4096)])
def test_decode_layer_attention(gpu, lab, past, capacity):
    """One attention layer in one launch (lfm25_decode_layer) at position
    `past` over a cache pre-filled N(0, 1), against Oracle.layer: the output
    within 4 ulps of its scale (as recurrent_block), the appended key / value
    rows within 2 ulps of their scale, the other cache rows untouched. Past
    256 positions the split attention runs (16 blocks per KV head)."""
    ck, idx = _layer_ck(lab, "attention", 17)
    names = O.layer_tensor_names(idx)
    t = {n.split(f"layers.{idx}.")[1]: ck[n] for n in names}
    qkv = np.concatenate([t["self_attn.q_proj.weight"].reshape(-1), t["self_attn.k_proj.weight"].reshape(-1),
                          t["self_attn.v_proj.weight"].reshape(-1)])
    keys = O.bf16_bits(rs.standard_normal((8, capacity, 64)).astype(np.float32))
    vals = O.bf16_bits(rs.standard_normal((8, capacity, 64)).astype(np.float32))
    d = {k: dev(v) for k, v in {"qkv": qkv, "keys": keys, "vals": vals,
                                "rope": lab.weights.rope_table(capacity)}.items()}
    w = {k: dev(t[k]) for k in ("operator_norm.weight", "self_attn.q_layernorm.weight", "self_attn.k_layernorm.weight",
                                "self_attn.out_proj.weight", "ffn_norm.weight", "feed_forward.w1.weight",
                                "feed_forward.w3.weight", "feed_forward.w2.weight")}
    layer = lab._lib.Layer(kind=lab._lib.LAYER_ATTN, op_norm=w["operator_norm.weight"].data_ptr(),
                           mixer=d["qkv"].data_ptr(), q_norm=w["self_attn.q_layernorm.weight"].data_ptr(),
                           k_norm=w["self_attn.k_layernorm.weight"].data_ptr(), key_cache=d["keys"].data_ptr(),
                           value_cache=d["vals"].data_ptr(), rope=d["rope"].data_ptr(), capacity=capacity,
                           out=w["self_attn.out_proj.weight"].data_ptr(), ffn_norm=w["ffn_norm.weight"].data_ptr(),
                           w1=w["feed_forward.w1.weight"].data_ptr(), w3=w["feed_forward.w3.weight"].data_ptr(),
                           w2=w["feed_forward.w2.weight"].data_ptr())
    hidden = bf(rs.standard_normal(1024) * 0.5)
    out = empty(1024)
    ws = torch.zeros(int(lab._lib.load().lfm25_decoder_workspace_bytes()), dtype=torch.uint8, device="cuda")
    import ctypes
    hidden_t = dev_f(hidden)  # held until the call is done
    lab._lib.call("lfm25_decode_layer", ctypes.byref(layer), hidden_t.data_ptr(), out.data_ptr(), past,
                  ws.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert int(ws[:12].view(torch.int32)[2].item()) == 0
    orc = O.Oracle(ck, capacity=capacity, layers=3)
    orc.keys[0][:, :past] = O.f32(keys)[:, :past]
    orc.values[0][:, :past] = O.f32(vals)[:, :past]
    orc.position = past
    want = orc.layer(idx, hidden, 0, 0)
    got = host(out)
    assert np.allclose(got, want, rtol=1e-2, atol=2e-2)
    assert scale_ulps_vec(got, want) <= 4, scale_ulps_vec(got, want)
    gk = host(d["keys"]).reshape(8, capacity, 64)
    gv = host(d["vals"]).reshape(8, capacity, 64)
    assert scale_ulps_vec(gk[:, past], orc.keys[0][:, past]) <= 2
    assert scale_ulps_vec(gv[:, past], orc.values[0][:, past]) <= 2
    others = np.ones(capacity, bool)
    others[past] = False
    assert np.array_equal(gk[:, others], O.f32(keys)[:, others])
    assert np.array_equal(gv[:, others], O.f32(vals)[:, others])


def test_decode_layer_conv_in_place_state(gpu, lab):
    """The conv layer with conv_state_out == conv_state_in (the decode's own
    use) equals the same layer with a separate output state, and two calls
    in a row shift the state twice (teacher-forced against the oracle)."""
    import ctypes
    ck, idx = _layer_ck(lab, "conv", 19)
    names = O.layer_tensor_names(idx)
    t = {n.split(f"layers.{idx}.")[1]: dev(ck[n]) for n in names}
    state0 = O.bf16_bits(rs.standard_normal((1024, 3)).astype(np.float32))
    st = dev(state0)
    layer = lab._lib.Layer(kind=lab._lib.LAYER_CONV, op_norm=t["operator_norm.weight"].data_ptr(),
                           mixer=t["conv.in_proj.weight"].data_ptr(), conv_weight=t["conv.conv.weight"].data_ptr(),
                           conv_state_in=st.data_ptr(), conv_state_out=st.data_ptr(),
                           out=t["conv.out_proj.weight"].data_ptr(), ffn_norm=t["ffn_norm.weight"].data_ptr(),
                           w1=t["feed_forward.w1.weight"].data_ptr(), w3=t["feed_forward.w3.weight"].data_ptr(),
                           w2=t["feed_forward.w2.weight"].data_ptr())
    ws = torch.zeros(int(lab._lib.load().lfm25_decoder_workspace_bytes()), dtype=torch.uint8, device="cuda")
    orc = O.Oracle(ck, capacity=4, layers=3)
    orc.conv_states[0] = O.f32(state0).reshape(1024, 3)
    for k in range(2):
        hidden = bf(rs.standard_normal(1024) * 0.5)
        out = empty(1024)
        hidden_t = dev_f(hidden)  # held until the call is done
        lab._lib.call("lfm25_decode_layer", ctypes.byref(layer), hidden_t.data_ptr(), out.data_ptr(), 0,
                      ws.data_ptr(), torch.cuda.current_stream().cuda_stream)
        want = orc.layer(idx, hidden, 0, 0)
        got = host(out)
        assert scale_ulps_vec(got, want) <= 4, k
        assert scale_ulps_vec(host(st).reshape(1024, 3), orc.conv_states[0]) <= 2, k
