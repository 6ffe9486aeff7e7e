"""Parakeet (FastConformer) encoder on the gfx950 matrix cores (lfm25_pk_* in include/lfm25_hip.h).

`PkEncoder` mirrors the reference's all-NPU encoder class
(experiments/pk_model.py:199-258 PkEncoder: construct with the layer count,
`run(hidden, valid)` -> the encoder output of the valid frames), for 128-frame
blocks and batches of independent sequences. Only PkEncoder imports torch;
the synthetic layers and the packing serve torch-free callers of the C-ABI
too. Weights come from a seeded synthetic generator (the reference's
exported npz files are not available here) or from a list of per-layer dicts
with the reference's names and layouts (experiments/011_export_weights.py:
[in, out] matrices, `x @ W`).

The host packing follows pk_model.pack_weights (experiments/pk_model.py:69-116):
q/k/v concatenated with the 1/sqrt(128) scale and bias_v folded into q,
delta = (bias_u - bias_v) / sqrt(128); matrices are stored output-major for
the GEMM kernel; the position table of each head is stored transposed.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .bf16 import bf16_bits_to_f32
from . import rng as _rng

D = 1024
HEADS, DK = 8, 128
FFN = 4096
FRAMES = 128
LN_NAMES = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")
SCALE = np.float32(1.0 / np.sqrt(128.0))
EPI_NONE, EPI_BIAS, EPI_SWISH = 0, 1, 2


PkLayer = _lib.PkLayer


def _bf16_round(x: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def _bits(x: np.ndarray) -> np.ndarray:
    """BF16 bit patterns of float32 values (nearest even); values that are
    already BF16 are taken as they are."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    if not (u & 0xFFFF).any():
        return (u >> 16).astype(np.uint16)
    return (_bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def synthetic_layer(seed: int, index: int, frames: int = FRAMES) -> tuple[dict, np.ndarray]:
    """Random-init BF16 weights of Conformer layer `index` (reference names and
    layouts) and its projected relative-position table [8, 128, 2T - 1]
    (float32 arrays holding BF16 values). Linear weights N(0, 0.02); norm
    gains 1 + N(0, 0.02), norm biases N(0, 0.02); attention biases N(0, 0.02);
    depthwise taps N(0, 0.1); the position table N(0, 0.45), the scale of
    sinusoidal embeddings through a N(0, 0.02) projection."""
    def g(name, shape, mean=0.0, std=0.02):
        n = int(np.prod(shape))
        b = _rng.normal_bf16(seed, f"pk.{index}.{name}", n, mean, std)
        return bf16_bits_to_f32(b).reshape(shape)
    w = {
        "feed_forward1.w1": g("ff1.w1", (D, FFN)), "feed_forward1.w2": g("ff1.w2", (FFN, D)),
        "att.wq": g("wq", (D, D)), "att.wk": g("wk", (D, D)), "att.wv": g("wv", (D, D)),
        "att.wout": g("wout", (D, D)),
        "att.bias_u": g("bias_u", (HEADS, DK)), "att.bias_v": g("bias_v", (HEADS, DK)),
        "conv.pw1": g("pw1", (D, 2 * D)), "conv.dw": g("dw", (D, 9), std=0.1), "conv.dw_b": g("dw_b", (D,)),
        "conv.pw2": g("pw2", (D, D)),
        "feed_forward2.w1": g("ff2.w1", (D, FFN)), "feed_forward2.w2": g("ff2.w2", (FFN, D)),
    }
    for name in LN_NAMES:
        w[f"{name}.w"] = g(f"{name}.w", (D,), 1.0, 0.02)
        w[f"{name}.b"] = g(f"{name}.b", (D,))
    pos = g(f"pos{frames}", (HEADS, DK, 2 * frames - 1), std=0.45)
    return w, pos


def pack_layer(w: dict, pos: np.ndarray, frames: int = FRAMES) -> dict[str, np.ndarray]:
    """Device layout of one layer (BF16 bit arrays), as lfm25_pk_layer documents."""
    if pos.shape != (HEADS, DK, 2 * frames - 1):
        raise ValueError(f"position table must be [{HEADS}, {DK}, {2 * frames - 1}]")
    qkv = np.concatenate([w["att.wq"] * SCALE, w["att.wk"], w["att.wv"]], axis=1)
    bias = np.concatenate([w["att.bias_v"].reshape(-1) * SCALE, np.zeros(2 * D, np.float32)])
    delta = (w["att.bias_u"] - w["att.bias_v"]) * SCALE
    pt = np.concatenate([pos, np.zeros((HEADS, DK, 1), np.float32)], axis=2).transpose(0, 2, 1)  # [8, 2T, 128]
    ln = np.stack([np.stack([w[f"{n}.w"], w[f"{n}.b"]]) for n in LN_NAMES])
    t = lambda m: np.ascontiguousarray(_bits(m).T)  # noqa: E731  [in, out] -> [out, in]
    return {
        "ln": _bits(ln), "ff1_w1": t(w["feed_forward1.w1"]), "ff1_w2": t(w["feed_forward1.w2"]),
        "qkv": t(qkv), "qkv_bias": _bits(bias), "att_delta": _bits(delta), "pos": _bits(pt),
        "out": t(w["att.wout"]), "pw1": t(w["conv.pw1"]), "dw": _bits(w["conv.dw"]),
        "dw_b": _bits(w["conv.dw_b"]), "pw2": t(w["conv.pw2"]),
        "ff2_w1": t(w["feed_forward2.w1"]), "ff2_w2": t(w["feed_forward2.w2"]),
    }


def _dev(bits: np.ndarray, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16).reshape(-1)).to(device)


def to_f32(t) -> np.ndarray:
    import torch
    return bf16_bits_to_f32(t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


class PkEncoder:
    """n_layers Conformer blocks for batches of 128-frame sequences.

    layers: None (seeded synthetic layers) or a list of (weights dict,
    position table) pairs as synthetic_layer returns them."""

    def __init__(self, n_layers: int = 24, *, seed: int = 0, layers=None, device="cuda"):
        import torch
        self.device = torch.device(device)
        _lib.load()
        if layers is None:
            layers = [synthetic_layer(seed, i) for i in range(n_layers)]
        self.n_layers = len(layers)
        self._tensors = []
        descs = []
        for w, pos in layers:
            packed = {k: _dev(v, self.device) for k, v in pack_layer(w, pos).items()}
            self._tensors.append(packed)
            descs.append(PkLayer(*[packed[f].data_ptr() for f, _ in PkLayer._fields_]))
        self._descs = (PkLayer * self.n_layers)(*descs)
        self.weight_bytes = sum(v.numel() * 2 for p in self._tensors for k, v in p.items() if k != "pos")
        self._ws = {}

    def _stream(self) -> int:
        import torch
        return torch.cuda.current_stream(self.device).cuda_stream

    def workspace(self, batch: int):
        import torch
        if batch not in self._ws:
            n = _lib.load().lfm25_pk_workspace_bytes(batch, FRAMES)
            self._ws[batch] = torch.empty(n, dtype=torch.uint8, device=self.device)
        return self._ws[batch]

    def run_device(self, x, batch: int, valid: int) -> None:
        """In place on x (bf16 [batch * 128 * 1024] on the device)."""
        _lib.call("lfm25_pk_encoder", self._descs, self.n_layers, x.data_ptr(), batch, FRAMES, valid,
                  self.workspace(batch).data_ptr(), self._stream())

    def run(self, hidden: np.ndarray, valid: int) -> np.ndarray:
        """hidden [T, 1024] or [B, T, 1024] float32 (T <= 128; padded with zero
        frames) -> the encoder output of the valid frames, [valid, 1024] or
        [B, valid, 1024] float32 holding BF16 values (PkEncoder.run,
        experiments/pk_model.py:243-258)."""
        h = np.asarray(hidden, np.float32)
        single = h.ndim == 2
        if single:
            h = h[None]
        b, t, d = h.shape
        if d != D or t > FRAMES or not 1 <= valid <= t:
            raise ValueError(f"hidden must be [B, T <= {FRAMES}, {D}] with 1 <= valid <= T")
        x = np.zeros((b, FRAMES, D), np.float32)
        x[:, :t] = h
        xd = _dev(_bits(x), self.device)
        self.run_device(xd, b, valid)
        out = to_f32(xd).reshape(b, FRAMES, D)[:, :valid]
        return out[0] if single else out
