"""LFM2.5-230M weights: synthetic seeded checkpoints, the device weight stream
and the rotary table.

A checkpoint is a dict of HF tensor names -> BF16 bit arrays (uint16) with HF
shapes. `pack_stream` lays the layer tensors out in the order of the C ABI's
packed weight stream (include/lfm25_hip.h): per layer, each tensor row-major
as in the checkpoint and starting on a 128-element boundary, then
embedding_norm. This is the GPU counterpart of the reference's pack_weights
(experiments/lfm25_x8.py:428-502), without its per-core slicing: on the GPU
every wave indexes rows of the unsliced matrices directly.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from .bf16 import f32_to_bf16_bits
from .rng import normal_bf16

HIDDEN, FFN, VOCAB = 1024, 2560, 65536
HEADS, KV_HEADS, HEAD_DIM = 16, 8, 64
KINDS = ("conv", "conv", "attention", "conv", "attention", "conv", "attention", "conv",
         "attention", "conv", "attention", "conv", "attention", "conv")
ALIGN = 128

CONV_TENSORS = (
    ("operator_norm.weight", (HIDDEN,)),
    ("conv.in_proj.weight", (3 * HIDDEN, HIDDEN)),
    ("conv.conv.weight", (HIDDEN, 1, 3)),
    ("conv.out_proj.weight", (HIDDEN, HIDDEN)),
    ("ffn_norm.weight", (HIDDEN,)),
    ("feed_forward.w1.weight", (FFN, HIDDEN)),
    ("feed_forward.w3.weight", (FFN, HIDDEN)),
    ("feed_forward.w2.weight", (HIDDEN, FFN)),
)
ATTN_TENSORS = (
    ("operator_norm.weight", (HIDDEN,)),
    ("self_attn.q_proj.weight", (HEADS * HEAD_DIM, HIDDEN)),
    ("self_attn.k_proj.weight", (KV_HEADS * HEAD_DIM, HIDDEN)),
    ("self_attn.v_proj.weight", (KV_HEADS * HEAD_DIM, HIDDEN)),
    ("self_attn.q_layernorm.weight", (HEAD_DIM,)),
    ("self_attn.k_layernorm.weight", (HEAD_DIM,)),
    ("self_attn.out_proj.weight", (HIDDEN, HIDDEN)),
    ("ffn_norm.weight", (HIDDEN,)),
    ("feed_forward.w1.weight", (FFN, HIDDEN)),
    ("feed_forward.w3.weight", (FFN, HIDDEN)),
    ("feed_forward.w2.weight", (HIDDEN, FFN)),
)
NORMS = ("operator_norm.weight", "ffn_norm.weight", "self_attn.q_layernorm.weight",
         "self_attn.k_layernorm.weight")


def stream_tensors() -> list[tuple[str, tuple]]:
    """(HF name, shape) of every tensor of the packed stream, in order."""
    out = []
    for i, kind in enumerate(KINDS):
        for name, shape in (ATTN_TENSORS if kind == "attention" else CONV_TENSORS):
            out.append((f"model.layers.{i}.{name}", shape))
    out.append(("model.embedding_norm.weight", (HIDDEN,)))
    return out


def stream_offsets() -> tuple[list[int], int]:
    offs, at = [], 0
    for _, shape in stream_tensors():
        offs.append(at)
        n = int(np.prod(shape))
        at += (n + ALIGN - 1) // ALIGN * ALIGN
    return offs, at


def all_tensors(vocab: int = VOCAB) -> list[tuple[str, tuple]]:
    return [("model.embed_tokens.weight", (vocab, HIDDEN))] + stream_tensors()


def synthetic_checkpoint(seed: int, vocab: int = VOCAB, std: float = 0.02,
                         layers: int | None = None) -> dict[str, np.ndarray]:
    """Random-init LFM2.5-230M-shape checkpoint: matrices (and the 3-tap conv
    weights, and the embedding table) ~ N(0, std), norm weights ~ 1 + N(0, std),
    each tensor from its own seeded stream (rng.normal_bf16)."""
    ck = {}
    for name, shape in all_tensors(vocab):
        if layers is not None and name.startswith("model.layers."):
            if int(name.split(".")[2]) >= layers:
                continue
        n = int(np.prod(shape))
        mean = 1.0 if name.endswith(NORMS) or name == "model.embedding_norm.weight" else 0.0
        ck[name] = normal_bf16(seed, name, n, mean, std).reshape(shape)
    return ck


def pack_stream(ck: dict[str, np.ndarray]) -> np.ndarray:
    """The packed weight stream (uint16 BF16 bits) of a full 14-layer checkpoint."""
    offs, total = stream_offsets()
    out = np.zeros(total, dtype=np.uint16)
    for (name, shape), off in zip(stream_tensors(), offs):
        t = np.ascontiguousarray(ck[name], dtype=np.uint16).reshape(-1)
        if t.size != int(np.prod(shape)):
            raise ValueError(f"{name}: expected shape {shape}, got {ck[name].shape}")
        out[off:off + t.size] = t
    return out


_FREQUENCIES = np.float32(1) / np.power(
    np.float32(1_000_000), np.arange(0, HEAD_DIM, 2, dtype=np.float32) / np.float32(HEAD_DIM))


def quantize_w8(w_bits: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    """Weights for ops.w8_gemv in the 8-bit formats of
    experiments/014_int8_lfm25.py:84-93: per row and group of `group` inputs
    (32, 64, or 0 for the whole row) s = max|w| / 127 in FP32 (1 for an
    all-zero group) and q = clamp(round_half_even(w / s), -127, 127). w_bits:
    BF16 bits [M, K]. Returns (q int8 [M, K], s float32 [M, K // group] or
    [M])."""
    bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    m, k = bits.shape
    g = group or k
    if group not in (0, 32, 64) or k % g:
        raise ValueError("group must be 0, 32 or 64 and divide K")
    w = (bits.astype(np.uint32) << 16).view(np.float32).reshape(m, k // g, g)
    s = (np.abs(w).max(axis=2) / np.float32(127)).astype(np.float32)
    s[s == 0] = np.float32(1)
    q = np.clip(np.rint(w / s[:, :, None]), -127, 127).astype(np.int8).reshape(m, k)
    return q, (s if group else s[:, 0].copy())


W8_GROUP = 32
W8_ALIGN = 256


def w8_projections(index: int) -> list[tuple[tuple[str, ...], int, int]]:
    """Projections of layer `index` in the 8-bit stream (include/lfm25_hip.h,
    lfm25_w8_model): (HF names stacked by rows, rows, cols). Attention's q, k
    and v form one [2048 x 1024] matrix."""
    p = f"model.layers.{index}."
    if KINDS[index] == "conv":
        mix = ((p + "conv.in_proj.weight",), 3 * HIDDEN, HIDDEN)
        out = ((p + "conv.out_proj.weight",), HIDDEN, HIDDEN)
    else:
        mix = (tuple(p + f"self_attn.{n}_proj.weight" for n in "qkv"), 2 * HIDDEN, HIDDEN)
        out = ((p + "self_attn.out_proj.weight",), HIDDEN, HIDDEN)
    ffn = [((p + f"feed_forward.{n}.weight",), r, c)
           for n, r, c in (("w1", FFN, HIDDEN), ("w3", FFN, HIDDEN), ("w2", HIDDEN, FFN))]
    return [mix, out] + ffn


def w8_offsets() -> tuple[list[tuple[int, int]], int]:
    """(q, scales) byte offsets of every projection of the 8-bit stream, in
    order, and its total size: each region on a 256-byte boundary."""
    al = lambda n: (n + W8_ALIGN - 1) // W8_ALIGN * W8_ALIGN  # noqa: E731
    offs, at = [], 0
    for i in range(len(KINDS)):
        for _, rows, cols in w8_projections(i):
            q = at
            at += al(rows * cols)
            offs.append((q, at))
            at += al(rows * (cols // W8_GROUP) * 4)
    return offs, at


def pack_w8(ck: dict[str, np.ndarray]) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The w8g32 model of a BF16 checkpoint for lfm25_decode_w8: (layers
    uint8 [lfm25_w8_layers_bytes()], table int8 [vocab, 1024], table scales
    float32 [vocab, 32]), quantized as quantize_w8 does (the reference's
    Weight with bits 8, group 32: every projection and the tied table,
    experiments/014_int8_lfm25.py:133-147)."""
    offs, total = w8_offsets()
    out = np.zeros(total, dtype=np.uint8)
    k = 0
    for i in range(len(KINDS)):
        for names, rows, cols in w8_projections(i):
            w = np.concatenate([np.asarray(ck[n], dtype=np.uint16).reshape(-1, cols) for n in names], axis=0)
            if w.shape != (rows, cols):
                raise ValueError(f"{names}: expected {rows} x {cols}, got {w.shape}")
            q, s = quantize_w8(w, W8_GROUP)
            qo, so = offs[k]
            out[qo:qo + q.size] = q.reshape(-1).view(np.uint8)
            out[so:so + 4 * s.size] = s.reshape(-1).view(np.uint8)
            k += 1
    tq, ts = quantize_w8(np.asarray(ck["model.embed_tokens.weight"], dtype=np.uint16), W8_GROUP)
    return out, tq, ts


def rope_table(capacity: int) -> np.ndarray:
    """[capacity, 128] BF16 bits: cos (64) | sin (64) of position p, computed in
    FP32 on the host as the reference's rotary() (experiments/lfm25_x8_model.py:23-30)."""
    p = np.arange(capacity, dtype=np.float32)[:, None]
    values = p * _FREQUENCIES[None, :]
    phase = np.concatenate([values, values], axis=1)
    return np.concatenate([f32_to_bf16_bits(np.cos(phase)), f32_to_bf16_bits(np.sin(phase))],
                          axis=1)


def load_safetensors(path: str | Path) -> dict[str, np.ndarray]:
    """BF16 tensors of a safetensors file as uint16 arrays (memory-mapped).
    Checks the header, dtype and byte lengths like the reference's
    BF16Checkpoint (experiments/lfm25_checkpoint.py:10-36), and that every
    tensor lies inside the file; `__metadata__` is skipped."""
    path = Path(path)
    size = path.stat().st_size
    with path.open("rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError("checkpoint is missing its safetensors header")
        n = int.from_bytes(head, "little")
        if n > size - 8:
            raise ValueError(f"safetensors header of {n} bytes runs past the end of the file")
        header = json.loads(f.read(n))
    data_bytes = size - 8 - n
    data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + n) if data_bytes > 0 else np.zeros(0, np.uint8)
    out = {}
    for name, spec in header.items():
        if name == "__metadata__":
            continue
        if spec["dtype"] != "BF16":
            raise ValueError(f"{name}: expected BF16, got {spec['dtype']}")
        a, b = spec["data_offsets"]
        shape = tuple(spec["shape"])
        if b - a != 2 * int(np.prod(shape)):
            raise ValueError(f"{name}: byte length {b - a} does not match shape {shape}")
        if not 0 <= a <= b <= data_bytes:
            raise ValueError(f"{name}: bytes [{a}, {b}) lie outside the {data_bytes}-byte data section")
        out[name] = data[a:b].view(np.uint16).reshape(shape)
    return out


def save_safetensors(path: str | Path, tensors: dict[str, np.ndarray], metadata: dict[str, str] | None = None) -> None:
    """Writes BF16 tensors (uint16 bit arrays) as a safetensors file: an
    8-byte little-endian header length, a JSON header padded with spaces to
    8 bytes (name -> dtype, shape, data_offsets; optional `__metadata__` of
    strings), then the tensors back to back in the header's order."""
    header: dict = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    at = 0
    arrays = []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        if a.dtype != np.uint16:
            raise ValueError(f"{name}: expected BF16 bits as uint16, got {a.dtype}")
        header[name] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [at, at + a.nbytes]}
        at += a.nbytes
        arrays.append(a)
    raw = json.dumps(header, separators=(",", ":")).encode()
    raw += b" " * (-len(raw) % 8)
    with Path(path).open("wb") as f:
        f.write(len(raw).to_bytes(8, "little"))
        f.write(raw)
        for a in arrays:
            f.write(a.tobytes())
