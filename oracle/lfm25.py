"""numpy restatement of the LFM2.5-230M decode step -- TEST INFRASTRUCTURE ONLY.

Conventions: BF16 tensors are uint16 bit arrays; float32 arrays hold values
computed in FP32; `_bf` rounds FP32 to BF16 (nearest even), as torch's
`.to(torch.bfloat16)` does. Element-wise steps are FP32 operations followed
by one BF16 rounding, exactly like a torch BF16 op on the CPU. Dot products
(F.linear / matmul with FP32 accumulation) are taken as the exact sum
rounded to FP32 and then to BF16 -- the limit of FP32 accumulation in any
order (the C helper, or numpy float64 when it is not built).

Reference semantics followed (paths in the reference repository, or in
transformers/models/lfm2/modeling_lfm2.py as "HF"):
  rms_norm       HF :54-59; experiments/006_lfm25_cpu_two_recurrent_layers.py:35-38
  linear         HF nn.Linear BF16; experiments/014_int8_lfm25.py:104-109
  conv_gate      experiments/006_lfm25_cpu_two_recurrent_layers.py:41-47
                 (HF :350-389 with per-product rounding); kernels/lfm25_conv_gate.cc:8-43
  silu_gate      HF :135-136 (Lfm2MLP); kernels/lfm25_silu_gate.cc:22-39
  rope_table     HF :100,108-116; experiments/lfm25_x8_model.py:23-30
  norm_rope      HF :239-240,147-169; kernels/lfm25_attention_norm_rope.cc:17-54
  attention      HF eager_attention_forward :184-207;
                 kernels/lfm25_attention_context_head.cc:19-82
  head/argmax    HF :528,596 + experiments/010_cpu_greedy.py:57,63;
                 kernels/x8/x8_core.cc:126-163 (first maximum wins)
  decode step    HF Lfm2DecoderLayer.forward :405-434, Lfm2Model.forward :477-535
  quantize_w8    experiments/014_int8_lfm25.py:84-93 (Weight.__init__, 8 bits)
  linear_w8      experiments/014_int8_lfm25.py:95-105 (Weight.dense / linear)
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

HIDDEN, FFN, VOCAB = 1024, 2560, 65536
HEADS, KV_HEADS, HEAD_DIM = 16, 8, 64
EPS = np.float32(1e-5)
THETA = 1_000_000.0
KINDS = ("conv", "conv", "attention", "conv", "attention", "conv", "attention", "conv",
         "attention", "conv", "attention", "conv", "attention", "conv")

# Functions whose exact BF16 bits against the third-party CPU path are not
# pinned by a closed form, a brute-force check or a committed vector: the
# FP32 transcendental functions differ between libm implementations in the
# last FP32 ulp, which can move a BF16 rounding.
UNPINNED = {
    "silu_gate": "bf16(silu) uses numpy float32 exp; torch uses SLEEF expf",
    "rope_table": "float32 pow/cos/sin of numpy vs torch",
    "attention": "float32 exp of numpy vs torch in the softmax",
}

# ------------------------------------------------------------------ BF16


def bf16_bits(x) -> np.ndarray:
    """float32 -> BF16 bits, round to nearest even (NaN kept)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (f != f)
    if nan.any():
        r[nan] = ((f.view(np.uint32)[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def f32(bits) -> np.ndarray:
    """BF16 bits -> float32 values."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _bf(x) -> np.ndarray:
    """Round float32 values to BF16, returned as float32."""
    return f32(bf16_bits(x))


# ------------------------------------------------------------------ GEMV

_HELPER = None
_HELPER_PATH = Path(__file__).resolve().parent / "_build" / "liblfm25_oracle.so"


def _helper():
    global _HELPER
    if _HELPER is None:
        if _HELPER_PATH.exists():
            lib = ctypes.CDLL(str(_HELPER_PATH))
            lib.oracle_gemv.restype = None
            lib.oracle_gemv.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_void_p]
            _HELPER = lib
        else:
            _HELPER = False
    return _HELPER


def gemv_exact(w_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Exact-sum W.x in float64 (W BF16 bits [M, K], x float32 [K])."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    m, k = w.shape
    if xv.size != k:
        raise ValueError("shape mismatch")
    lib = _helper()
    if lib:
        y = np.empty(m, dtype=np.float64)
        lib.oracle_gemv(w.ctypes.data, xv.ctypes.data, m, k, y.ctypes.data)
        return y
    return f32(w).astype(np.float64) @ xv.astype(np.float64)


def linear(w_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """bf16(W . x) with FP32 accumulation; returns float32 BF16 values."""
    return _bf(gemv_exact(w_bits, x).astype(np.float32))


def linear_f32(w_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """W . x in FP32 (no BF16 rounding)."""
    return gemv_exact(w_bits, x).astype(np.float32)


# ------------------------------------------------------------------ 8-bit weights


def quantize_w8(w_bits: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    """int8 weights with FP32 scales (014_int8_lfm25.py:84-93, bits 8): for
    each row and each group of `group` consecutive inputs (group 0: the whole
    row), s = max|w| / 127 in FP32, 1 for an all-zero group, and
    q = clamp(round_half_even(w / s), -127, 127) with the division in FP32.
    Returns q int8 [M, K] and s float32 [M, K // group] ([M] for group 0)."""
    w = f32(np.asarray(w_bits, dtype=np.uint16))
    m, k = w.shape
    g = group or k
    if k % g:
        raise ValueError("K must be a multiple of the group")
    q = np.empty((m, k), dtype=np.int8)
    scales = np.empty((m, k // g), dtype=np.float32)
    for j in range(k // g):
        block = w[:, j * g:(j + 1) * g]
        sj = np.max(np.abs(block), axis=1) / np.float32(127)
        sj = np.where(sj == 0, np.float32(1), sj).astype(np.float32)
        ratio = (block / sj[:, None]).astype(np.float32)
        q[:, j * g:(j + 1) * g] = np.clip(np.rint(ratio), -127, 127).astype(np.int8)
        scales[:, j] = sj
    return q, (scales if group else scales[:, 0].copy())


def dequantize_w8(q: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    """FP32 weights q * s (014_int8_lfm25.py:95-103, Weight.dense)."""
    m, k = q.shape
    if group == 0:
        return (q.astype(np.float32) * scales.astype(np.float32)[:, None]).astype(np.float32)
    s = np.repeat(scales.astype(np.float32), group, axis=1)
    return (q.astype(np.float32) * s).astype(np.float32)


def linear_w8(q: np.ndarray, scales: np.ndarray, group: int, x: np.ndarray) -> np.ndarray:
    """bf16 of Weight.linear (014_int8_lfm25.py:104-109) for a BF16-valued x:
    group 0 (w8c) -> bf16(fp32(sum_k q x) * s); groups -> bf16(fp32(sum_k x *
    (q s)_fp32)), each sum exact before its FP32 rounding (float64 here: the
    products are exact and K is small)."""
    xv = np.asarray(x, dtype=np.float32).astype(np.float64)
    if group == 0:
        acc = (q.astype(np.float64) @ xv).astype(np.float32)
        return _bf((acc * scales.astype(np.float32)).astype(np.float32))
    return linear_dense64(dequantize_w8(q, scales, group).astype(np.float64), x)


def linear_dense64(dense: np.ndarray, x: np.ndarray) -> np.ndarray:
    """bf16(fp32(dense . x)) for FP32-exact weights held as float64 (the group
    branch of linear_w8 on a dequantized matrix kept across calls)."""
    return _bf((dense @ np.asarray(x, dtype=np.float32).astype(np.float64)).astype(np.float32))


# ------------------------------------------------------------------ ops


def rms_norm(x: np.ndarray, gamma: np.ndarray, eps=EPS) -> np.ndarray:
    """HF Lfm2RMSNorm: n = bf16(x * rsqrt(mean(x^2) + eps)); y = bf16(gamma * n).
    x, gamma: float32 BF16 values (last axis normalised)."""
    x = np.asarray(x, dtype=np.float32)
    var = (np.square(x.astype(np.float64)).sum(-1, keepdims=True) / x.shape[-1]).astype(np.float32)
    r = np.float32(1) / np.sqrt(var + np.float32(eps))
    n = _bf(x * r)
    return _bf(np.asarray(gamma, dtype=np.float32) * n)


def bf16_add(a, b) -> np.ndarray:
    return _bf(np.asarray(a, np.float32) + np.asarray(b, np.float32))


def silu(h: np.ndarray) -> np.ndarray:
    """bf16(silu(h)) computed in FP32 as h / (1 + exp(-h))."""
    h = np.asarray(h, dtype=np.float32)
    with np.errstate(over="ignore"):
        return _bf(h / (np.float32(1) + np.exp(-h)))


def silu_gate(w1: np.ndarray, w3: np.ndarray) -> np.ndarray:
    """bf16(bf16(silu(w1)) * w3)."""
    return _bf(silu(w1) * np.asarray(w3, np.float32))


def conv_gate(B, C, x, weight, state):
    """Gated short conv, one token. B, C, x: [1024]; weight [1024, 3];
    state [1024, 3] (HF conv_state). Returns (y [1024], new state [1024, 3]).
      bx = bf16(B*x); state' = [s1, s2, bx];
      conv = bf16(sum_j bf16(state'_j * w_j)) (FP32 sum, j in order);
      y = bf16(C * conv)."""
    B, C, x = (np.asarray(a, np.float32) for a in (B, C, x))
    w = np.asarray(weight, np.float32).reshape(HIDDEN, 3)
    s = np.asarray(state, np.float32).reshape(HIDDEN, 3)
    bx = _bf(B * x)
    new = np.stack([s[:, 1], s[:, 2], bx], axis=1)
    p = _bf(new * w)
    conv = _bf((p[:, 0] + p[:, 1]) + p[:, 2])
    return _bf(C * conv), new


def rope_table(positions, theta: float = THETA) -> tuple[np.ndarray, np.ndarray]:
    """(cos, sin) as float32 BF16 values [len(positions), 64]:
    inv_freq = 1 / theta^(2i/64) in FP32, phase = p * inv_freq (FP32),
    cos/sin in FP32 then rounded to BF16; the 32 frequencies repeat twice."""
    exps = np.arange(0, HEAD_DIM, 2, dtype=np.float32) / np.float32(HEAD_DIM)
    inv = np.float32(1) / np.power(np.float32(theta), exps)
    p = np.asarray(positions, dtype=np.float32).reshape(-1, 1)
    f = p * inv[None, :]
    emb = np.concatenate([f, f], axis=1)
    return _bf(np.cos(emb)), _bf(np.sin(emb))


def norm_rope(v: np.ndarray, gamma: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Per-head RMSNorm over 64 then RoPE: out = bf16(bf16(n*cos) + bf16(rot(n)*sin)),
    rot(n) = [-n[32:], n[:32]]. v: [heads, 64]."""
    n = rms_norm(v, gamma)
    rot = np.concatenate([-n[..., 32:], n[..., :32]], axis=-1)
    return _bf(_bf(n * cos) + _bf(rot * sin))


def attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """Eager GQA decode attention for one position.
    q [16, 64]; keys/values [8, T, 64] (all positions including the current).
      s = bf16(q.k) * 0.125; p = bf16(exp(s - max) / sum) (FP32);
      ctx = bf16(sum p * v) (FP32 accumulation). Returns [16 * 64]."""
    out = np.empty((HEADS, HEAD_DIM), dtype=np.float32)
    for hq in range(HEADS):
        kv = hq // (HEADS // KV_HEADS)
        k = keys[kv]
        v = values[kv]
        s = (k.astype(np.float64) @ q[hq].astype(np.float64)).astype(np.float32)
        s = _bf(s) * np.float32(0.125)
        e = np.exp(s - s.max())
        z = np.float32(e.astype(np.float64).sum())  # exact-sum FP32 accumulation
        p = _bf(e / z)
        ctx = (p.astype(np.float64) @ v.astype(np.float64)).astype(np.float32)
        out[hq] = _bf(ctx)
    return out.reshape(-1)


def argmax_first(logits: np.ndarray) -> int:
    """Index of the first maximum (numpy argmax returns the first)."""
    return int(np.argmax(np.asarray(logits, np.float32)))


# ------------------------------------------------------------------ model


def layer_tensor_names(index: int) -> list[str]:
    p = f"model.layers.{index}."
    if KINDS[index] == "conv":
        return [p + n for n in ("operator_norm.weight", "conv.in_proj.weight", "conv.conv.weight",
                                "conv.out_proj.weight", "ffn_norm.weight",
                                "feed_forward.w1.weight", "feed_forward.w3.weight",
                                "feed_forward.w2.weight")]
    return [p + n for n in ("operator_norm.weight", "self_attn.q_proj.weight",
                            "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                            "self_attn.q_layernorm.weight", "self_attn.k_layernorm.weight",
                            "self_attn.out_proj.weight", "ffn_norm.weight",
                            "feed_forward.w1.weight", "feed_forward.w3.weight",
                            "feed_forward.w2.weight")]


@dataclass
class StepRecord:
    token_in: int
    hidden: np.ndarray            # pre-final-norm hidden state (float32 BF16 values)
    logits: np.ndarray | None     # BF16 logits as float32, when the head ran
    token_out: int | None


W8_GROUP = 32


@dataclass
class Oracle:
    """Token-by-token decode with conv/KV caches, as 010_cpu_greedy.py:46-63
    drives the HF model. `ck` maps HF tensor names to BF16 bit arrays.

    w8=True runs the reference's w8g32 model instead (014_int8_lfm25.py:
    133-199 with fmt (8, 32)): every projection and the tied table quantized
    by quantize_w8 (group 32), linear_w8 for each product, embedding rows
    bf16(q s) (Weight.rows :111-112); norms, conv taps and QK norms stay BF16.
    The logits are bf16(linear_w8), the rounding point of every other
    projection (the reference's study keeps its head in FP32, :201-212; a
    head rounding decides only exact BF16 ties)."""

    ck: dict
    capacity: int = 4096
    layers: int = 14
    position: int = 0
    conv_states: list = field(default_factory=list)
    keys: list = field(default_factory=list)
    values: list = field(default_factory=list)
    w8: bool = False

    def __post_init__(self):
        self.reset()
        self._cos, self._sin = rope_table(np.arange(self.capacity))
        self._q8 = {}
        self._d8 = {}  # dequantized float64 matrices, built on first use
        if self.w8:
            for name, t in self.ck.items():
                if t.ndim == 2 and ("_proj." in name or "feed_forward." in name or name.endswith("embed_tokens.weight")):
                    self._q8[name] = quantize_w8(t, W8_GROUP)

    def _lin(self, name, x):
        if self.w8:
            if name not in self._d8:
                q, s = self._q8[name]
                self._d8[name] = dequantize_w8(q, s, W8_GROUP).astype(np.float64)
            return linear_dense64(self._d8[name], x)
        return linear(self._t(name), x)

    def embedding_row(self, token: int) -> np.ndarray:
        """Layer 0's input: the table row (BF16), or bf16(q s) of the int8 row."""
        name = "model.embed_tokens.weight"
        if self.w8:
            q, s = self._q8[name]
            return _bf(dequantize_w8(q[token:token + 1], s[token:token + 1], W8_GROUP)[0])
        return f32(self.ck[name][token])

    def reset(self):
        self.position = 0
        n_conv = sum(1 for k in KINDS[:self.layers] if k == "conv")
        n_att = self.layers - n_conv
        self.conv_states = [np.zeros((HIDDEN, 3), np.float32) for _ in range(n_conv)]
        self.keys = [np.zeros((KV_HEADS, self.capacity, HEAD_DIM), np.float32)
                     for _ in range(n_att)]
        self.values = [np.zeros((KV_HEADS, self.capacity, HEAD_DIM), np.float32)
                       for _ in range(n_att)]

    def _t(self, name):
        return self.ck[name]

    def _g(self, name):
        return f32(self.ck[name]).reshape(-1)

    def layer(self, index: int, h: np.ndarray, conv_i: int, att_i: int) -> np.ndarray:
        names = layer_tensor_names(index)
        n = rms_norm(h, self._g(names[0]))
        if KINDS[index] == "conv":
            bcx = self._lin(names[1], n)
            w = f32(self._t(names[2])).reshape(HIDDEN, 3)
            y, self.conv_states[conv_i] = conv_gate(bcx[:HIDDEN], bcx[HIDDEN:2 * HIDDEN],
                                                    bcx[2 * HIDDEN:], w,
                                                    self.conv_states[conv_i])
            o = self._lin(names[3], y)
            ffn = names[4:]
        else:
            pos = self.position
            q = self._lin(names[1], n).reshape(HEADS, HEAD_DIM)
            k = self._lin(names[2], n).reshape(KV_HEADS, HEAD_DIM)
            v = self._lin(names[3], n).reshape(KV_HEADS, HEAD_DIM)
            cos, sin = self._cos[pos], self._sin[pos]
            q = norm_rope(q, self._g(names[4]), cos, sin)
            k = norm_rope(k, self._g(names[5]), cos, sin)
            self.keys[att_i][:, pos] = k
            self.values[att_i][:, pos] = v
            ctx = attention(q, self.keys[att_i][:, :pos + 1], self.values[att_i][:, :pos + 1])
            o = self._lin(names[6], ctx)
            ffn = names[7:]
        h = bf16_add(h, o)
        n2 = rms_norm(h, self._g(ffn[0]))
        g = silu_gate(self._lin(ffn[1], n2), self._lin(ffn[2], n2))
        return bf16_add(h, self._lin(ffn[3], g))

    def step(self, token: int, select: bool = True) -> StepRecord:
        if self.position >= self.capacity:
            raise ValueError(f"KV capacity {self.capacity} reached")
        h = self.embedding_row(token)
        conv_i = att_i = 0
        for index in range(self.layers):
            h = self.layer(index, h, conv_i, att_i)
            if KINDS[index] == "conv":
                conv_i += 1
            else:
                att_i += 1
        self.position += 1
        if not select:
            return StepRecord(token, h, None, None)
        n = rms_norm(h, self._g("model.embedding_norm.weight"))
        logits = self._lin("model.embed_tokens.weight", n)
        return StepRecord(token, h, logits, argmax_first(logits))

    def greedy(self, prompt, n_gen: int, force=None):
        """Prompt token by token, then n_gen greedy tokens. `force` (optional
        list) replaces the fed-back token at each generated position (teacher
        forcing). Returns the list of StepRecords of the selecting steps."""
        records = []
        for t in prompt[:-1]:
            self.step(int(t), select=False)
        tok = int(prompt[-1])
        for i in range(n_gen):
            rec = self.step(tok, select=True)
            records.append(rec)
            tok = rec.token_out if force is None else int(force[i])
        return records
