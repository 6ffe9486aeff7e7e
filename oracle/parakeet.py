"""numpy restatement of the Parakeet (FastConformer) encoder block -- TEST INFRASTRUCTURE ONLY.

Two independent restatements of one Conformer layer (d = 1024, 8 heads of 128,
FFN 4096, depthwise conv k = 9, relative-position attention):

  block_bf16   the reference's BF16-boundary mirror of its NPU encoder
               (experiments/012_layer_test.py:45-114 `mirror`): FP32 math,
               BF16 rounding exactly where the NPU stores a field; q/k/v with
               the 1/sqrt(128) scale and bias_v folded into the projection
               (experiments/pk_model.py:82-90).
  block_f32    the reference's FP32 CPU layer (experiments/parakeet_hybrid.py:
               262-321 `rel_shift`, `conformer_layer`), no rounding, NeMo
               rel_shift on the full position table.

Each is a check on the other (they agree to BF16 precision). Weights are a
dict with the reference's names and layouts ([in, out] matrices, x @ W):
feed_forward{1,2}.w1 [1024, 4096], .w2 [4096, 1024], att.wq/wk/wv/wout
[1024, 1024], att.bias_u/bias_v [8, 128], conv.pw1 [1024, 2048], conv.dw
[1024, 9], conv.dw_b [1024], conv.pw2 [1024, 1024], and {name}.w / {name}.b for
the LayerNorms norm_feed_forward1, norm_self_att, norm_conv,
norm_feed_forward2, norm_out. `pos` is the projected relative-position table
of the layer, [8 heads, 128, 2T - 1] for relative offsets T-1 .. -(T-1)
(experiments/pk_model.py:34-44 keeps the [.., c - T + 1 : c + T] slice of a
longer export).
"""

from __future__ import annotations

import numpy as np

D = 1024
HEADS, DK = 8, 128
FFN = 4096
CONV_K = 9
EPS = np.float32(1e-5)
SCALE = np.float32(1.0 / np.sqrt(128.0))
LN_NAMES = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")


def _r(x) -> np.ndarray:
    """As r(), but may return x itself when it already holds BF16 values
    (for read-only operands such as the weights)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    if not np.any(u & np.uint32(0xFFFF)):
        return f  # already BF16 values: rounding is the identity
    # u + 0x7FFF + lsb wraps around 2^32 only for NaN patterns, fixed below
    out = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)).view(np.float32)
    nan = f != f
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def r(x) -> np.ndarray:
    """float32 -> nearest-even BF16 value, kept as float32 (ml_dtypes' cast);
    always a new array."""
    out = _r(x)
    return out.copy() if out is x or np.shares_memory(out, np.asarray(x)) else out


def bits(x) -> np.ndarray:
    """BF16 bit patterns (uint16) of float32 values (rounded to nearest even)."""
    return (r(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def sig(x):
    """experiments/012_layer_test.py:42-43 (FP32)."""
    return np.float32(1) / (np.float32(1) + np.exp(-x))


def ln(x, w, b):
    """LayerNorm with the mirror's operation order (012_layer_test.py:36-39):
    bf16((x - mu) / sqrt(var + eps) * w + b), mean and variance in FP32."""
    mu = x.mean(-1, keepdims=True, dtype=np.float32)
    v = ((x - mu) ** 2).mean(-1, keepdims=True, dtype=np.float32)
    return r((x - mu) / np.sqrt(v + EPS) * w + b)


def mm(a, w):
    """FP32 product of BF16 operands (the mirror's `r(a) @ r(w)`)."""
    return np.matmul(_r(a), _r(w), dtype=np.float32)


def folded_qkv(w):
    """q/k/v weights [1024, 3072] with the 1/sqrt(dk) scale folded into q, the
    bias [3072] (bias_v * scale, 0, 0) and delta = bf16((bias_u - bias_v) *
    scale) [8, 128] (experiments/pk_model.py:82-90)."""
    qkv_w = np.concatenate([w["att.wq"] * SCALE, w["att.wk"], w["att.wv"]], axis=1).astype(np.float32)
    bias = np.concatenate([w["att.bias_v"].reshape(-1) * SCALE, np.zeros(2 * D, np.float32)]).astype(np.float32)
    delta = r((w["att.bias_u"] - w["att.bias_v"]) * SCALE)
    return qkv_w, bias, delta


def pos_slice(pos, T):
    """The mirror's per-head table P [8, 128, 2T]: offsets T-1 .. -(T-1), then
    a zero column (pk_model.pos_tables)."""
    return np.concatenate([pos, np.zeros((HEADS, DK, 1), np.float32)], axis=2)


def gemm(a, w_in_out, bias=None, swish=False):
    """bf16(epi(a @ W + bias)) with the mirror's operation order: the FP32
    product, + the BF16 bias, Swish z * sigmoid(z) on the FP32 value, one
    rounding (012_layer_test.py:57,62,72)."""
    z = mm(a, w_in_out)
    if bias is not None:
        z = z + r(bias)
    if swish:
        z = z * sig(z)
    return r(z)


def residual_ln(x, y, s, g, b):
    """x' = bf16(x + s * y), a = LN(x') (pk_core.cc residual + layer_norm)."""
    x = r(x + np.float32(s) * y)
    return x, ln(x, g, b)


def position_scores(q, P):
    """bd[h] = bf16(q_h @ P_h) for the 8 heads (012_layer_test.py:67)."""
    return np.stack([r(mm(q[:, hh * DK:(hh + 1) * DK], P[hh])) for hh in range(HEADS)])


def attention(qkv, bd, delta, valid):
    """Relative-position attention with q scaled and bias_v folded in
    (012_layer_test.py:70-80): qu = bf16(q + delta_h); s = qu . k_j +
    bd[h][i, T-1-i+j]; keys >= valid masked; FP32 softmax; o = bf16(p . v)."""
    T = qkv.shape[0]
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    o = np.zeros((T, D), np.float32)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    for hh in range(HEADS):
        qu = r(q[:, hh * DK:(hh + 1) * DK] + delta[hh])
        sc = np.matmul(qu, k[:, hh * DK:(hh + 1) * DK].T, dtype=np.float32)
        sc = sc + bd[hh][i, T - 1 - i + j]
        sc[:, valid:] = -np.inf
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        o[:, hh * DK:(hh + 1) * DK] = r(np.matmul(p, v[:, hh * DK:(hh + 1) * DK], dtype=np.float32))
    return o


def conv_module(c, dw, dw_b, valid):
    """GLU over pointwise1's 2048 outputs, frames >= valid zeroed, 9-tap
    depthwise conv (zero outside the frames) summed tap by tap, + bias,
    Swish (012_layer_test.py:92-98)."""
    T = c.shape[0]
    g = r(c[:, :D] * sig(c[:, D:]))
    g[valid:] = 0
    gp = np.pad(g, ((4, 4), (0, 0)))
    dw = r(dw)
    yc = np.float32(0)
    for jj in range(CONV_K):
        yc = yc + gp[jj:jj + T] * dw[:, jj]
    yc = yc + r(dw_b)
    return r(yc * sig(yc))


def block_bf16(x, w, pos, valid):
    """One Conformer layer, BF16 at the NPU's field boundaries
    (012_layer_test.py:45-114). x [T, 1024] BF16 values (rows >= valid are
    padding that still flows through, as on the NPU); returns the new x and
    the named intermediate fields."""
    T = x.shape[0]
    out = {}
    a = ln(x, w["norm_feed_forward1.w"], w["norm_feed_forward1.b"])
    out["a_ff1"] = a
    h = gemm(a, w["feed_forward1.w1"], swish=True)
    out["ff1_h"] = h
    y = gemm(h, w["feed_forward1.w2"])
    out["ff1_y"] = y
    x, a = residual_ln(x, y, 0.5, w["norm_self_att.w"], w["norm_self_att.b"])
    out["a_att"] = a
    qkv_w, bias, delta = folded_qkv(w)
    qkv = gemm(a, qkv_w, bias)
    out["qkv"] = qkv
    bd = position_scores(qkv[:, :D], pos_slice(pos, T))
    out["bd"] = bd
    o = attention(qkv, bd, delta, valid)
    out["att_o"] = o
    y = gemm(o, w["att.wout"])
    x, a = residual_ln(x, y, 1.0, w["norm_conv.w"], w["norm_conv.b"])
    out["a_conv"] = a
    c = gemm(a, w["conv.pw1"])
    out["pw1"] = c
    sconv = conv_module(c, w["conv.dw"], w["conv.dw_b"], valid)
    out["conv_o"] = sconv
    y = gemm(sconv, w["conv.pw2"])
    x, a = residual_ln(x, y, 1.0, w["norm_feed_forward2.w"], w["norm_feed_forward2.b"])
    out["a_ff2"] = a
    h = gemm(a, w["feed_forward2.w1"], swish=True)
    y = gemm(h, w["feed_forward2.w2"])
    x = ln(r(x + np.float32(0.5) * y), w["norm_out.w"], w["norm_out.b"])
    out["x"] = x
    return x, out


# ------------------------------------------------------------------ FP32 restatement

def layer_norm_f32(x, w, b):
    """experiments/parakeet_hybrid.py:65-69."""
    mu = x.mean(-1, keepdims=True)
    xc = x - mu
    var = (xc * xc).mean(-1, keepdims=True)
    return xc / np.sqrt(var + EPS) * w + b


def rel_shift(x):
    """NeMo RelPositionMultiHeadAttention.rel_shift (parakeet_hybrid.py:262-266)."""
    h, t, n = x.shape
    x = np.pad(x, ((0, 0), (0, 0), (1, 0)))
    return x.reshape(h, n + 1, t)[:, 1:].reshape(h, t, n)


def block_f32(x, w, pos, valid):
    """One Conformer layer in FP32 (parakeet_hybrid.py:269-321), with the
    attention mask of `valid` real frames."""
    t = x.shape[0]
    swish = lambda z: z * sig(z)  # noqa: E731
    res = x.astype(np.float32)
    h = swish(layer_norm_f32(res, w["norm_feed_forward1.w"], w["norm_feed_forward1.b"]) @ w["feed_forward1.w1"])
    res = res + 0.5 * (h @ w["feed_forward1.w2"])
    a = layer_norm_f32(res, w["norm_self_att.w"], w["norm_self_att.b"])
    q = (a @ w["att.wq"]).reshape(t, HEADS, DK)
    k = (a @ w["att.wk"]).reshape(t, HEADS, DK).transpose(1, 2, 0)
    v = (a @ w["att.wv"]).reshape(t, HEADS, DK).transpose(1, 0, 2)
    qu = (q + w["att.bias_u"]).transpose(1, 0, 2)
    qv = (q + w["att.bias_v"]).transpose(1, 0, 2)
    att = np.empty((t, HEADS, DK), np.float32)
    keep = np.zeros((t, t), bool)
    keep[:, :valid] = True
    for hd in range(HEADS):
        bd = rel_shift((qv[hd] @ pos[hd])[None])[0, :, :t]
        sc = (qu[hd] @ k[hd] + bd) * SCALE
        sc = np.where(keep, sc, np.float32(-10000.0))
        sc -= sc.max(-1, keepdims=True)
        pr = np.exp(sc)
        pr /= pr.sum(-1, keepdims=True)
        pr *= keep
        att[:, hd] = pr @ v[hd]
    res = res + att.reshape(t, D) @ w["att.wout"]
    c = layer_norm_f32(res, w["norm_conv.w"], w["norm_conv.b"]) @ w["conv.pw1"]
    cp = np.zeros((t + 8, D), np.float32)
    cp[4:t + 4] = c[:, :D] * sig(c[:, D:])
    cp[4 + valid:] = 0.0
    acc = cp[0:t] * w["conv.dw"][:, 0]
    for j in range(1, CONV_K):
        acc = acc + cp[j:j + t] * w["conv.dw"][:, j]
    res = res + swish(acc + w["conv.dw_b"]) @ w["conv.pw2"]
    h = swish(layer_norm_f32(res, w["norm_feed_forward2.w"], w["norm_feed_forward2.b"]) @ w["feed_forward2.w1"])
    res = res + 0.5 * (h @ w["feed_forward2.w2"])
    return layer_norm_f32(res, w["norm_out.w"], w["norm_out.b"])


def encoder_bf16(x, layers, pos_tables, valid):
    """Several layers of block_bf16 (the input is rounded to BF16 first)."""
    x = r(x)
    for w, pos in zip(layers, pos_tables):
        x, _ = block_bf16(x, w, pos, valid)
    return x


def compare(ref, got):
    """The reference's field comparison (012_layer_test.py:117-121)."""
    a, b = np.ravel(ref).astype(np.float64), np.ravel(got).astype(np.float64)
    return {"cosine": float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30)),
            "rel_rms": float(np.sqrt(np.mean((a - b) ** 2) / (np.mean(a ** 2) + 1e-30))),
            "max_abs": float(np.abs(a - b).max())}
