"""Batched LFM2.5 passes on the matrix cores (lfm25_batch_* in include/lfm25_hip.h).

`BatchDecoder` holds B independent sequences that share one weight stream:
prompts go through passes of up to 64 rows (several sequences per pass), and
greedy decoding advances every sequence by one token per pass, each weight
tile read once for all B rows. It extends the reference's batched prompt
pass (experiments/lfm25_x8.py:341-416,
X8Model.prefill_batch experiments/lfm25_x8_model.py:94-115), which only ever
batched PB = 4 positions of one sequence; `X8Model.prefill_batch` runs on the
same kernels with one sequence.

Arrays come back as float32 numpy arrays holding BF16 values, in the HF
layouts (conv state [1024, 3], keys/values [8, positions, 64]).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .bf16 import bf16_bits_to_f32
from .weights import (HEAD_DIM, HIDDEN, KINDS, KV_HEADS, VOCAB, load_safetensors, pack_stream,
                      rope_table, synthetic_checkpoint)

MAX_ROWS = _lib.BATCH_MAX_ROWS
CONV_LAYERS = KINDS.count("conv")
ATT_LAYERS = KINDS.count("attention")


def _u16_to_device(a: np.ndarray, device) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16).reshape(-1))
    return t.to(device).view(torch.bfloat16)


def _to_f32(t: torch.Tensor) -> np.ndarray:
    return bf16_bits_to_f32(t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def run_pass(desc: _lib.Batch, rows: list[tuple[int, int, int]], select: bool, tokens_out: torch.Tensor | None,
             hidden_out: torch.Tensor | None, stream: int) -> None:
    """One lfm25_batch_pass over `rows` = [(token, sequence, position), ...]."""
    table = np.ascontiguousarray(np.asarray(rows, dtype=np.int32).reshape(-1, 3))
    _lib.call("lfm25_batch_pass", ctypes.byref(desc), table.ctypes.data, len(table), 1 if select else 0,
              tokens_out.data_ptr() if tokens_out is not None else None,
              hidden_out.data_ptr() if hidden_out is not None else None, stream)


class BatchDecoder:
    """B independent sequences decoded in lockstep on shared weights.

    weights: None (seeded synthetic checkpoint), a checkpoint dict, or a
    safetensors path; `share` may pass an existing X8Model or BatchDecoder
    whose device weights, table and rope table are reused."""

    def __init__(self, sequences: int, capacity: int = 4096, *, weights=None, seed: int = 0,
                 vocab: int = VOCAB, device="cuda", share=None):
        if not 1 <= sequences <= MAX_ROWS:
            raise ValueError(f"sequences must be in [1, {MAX_ROWS}]")
        if not 1 <= capacity <= 4096:
            raise ValueError("capacity must be in [1, 4096]")
        self.sequences = sequences
        self.capacity = capacity
        self.device = torch.device(device)
        lib = _lib.load()
        if share is not None:
            if share.capacity < capacity:
                raise ValueError("the shared rope table is shorter than the capacity")
            self.weights, self.table, self.rope, self.vocab = share.weights, share.table, share.rope, share.vocab
        else:
            if weights is None:
                ck = synthetic_checkpoint(seed, vocab)
            elif isinstance(weights, dict):
                ck = weights
            else:
                ck = load_safetensors(weights)
            table = ck["model.embed_tokens.weight"]
            self.vocab = int(table.shape[0])
            stream = pack_stream(ck)
            if stream.size != lib.lfm25_weights_elems():
                raise ValueError("packed weight stream does not match the library layout")
            self.weights = _u16_to_device(stream, self.device)
            self.table = _u16_to_device(table, self.device)
            self.rope = _u16_to_device(rope_table(capacity), self.device)
        if self.vocab % 16:
            raise ValueError("the batched pass needs a vocabulary size that is a multiple of 16")
        bf = dict(dtype=torch.bfloat16, device=self.device)
        self.conv_states = torch.zeros(sequences * CONV_LAYERS * HIDDEN * 3, **bf)
        kv = sequences * ATT_LAYERS * KV_HEADS * capacity * HEAD_DIM
        self.keys = torch.zeros(kv, **bf)
        self.values = torch.zeros(kv, **bf)
        self.workspace = torch.zeros(lib.lfm25_batch_workspace_bytes(), dtype=torch.uint8, device=self.device)
        self._tokens = torch.zeros(MAX_ROWS, dtype=torch.int32, device=self.device)
        self._desc = _lib.Batch(self.weights.data_ptr(), self.table.data_ptr(), self.rope.data_ptr(),
                                self.conv_states.data_ptr(), self.keys.data_ptr(), self.values.data_ptr(),
                                self.workspace.data_ptr(), sequences, capacity, self.vocab)
        self.reset()

    # ------------------------------------------------------------ control

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def reset(self, sequence: int | None = None):
        """Forget every sequence (or one): conv state zeroed, position 0."""
        if sequence is None:
            self.conv_states.zero_()
            self.positions = [0] * self.sequences
        else:
            n = CONV_LAYERS * HIDDEN * 3
            self.conv_states[sequence * n:(sequence + 1) * n].zero_()
            self.positions[sequence] = 0

    def _status(self) -> int:
        return int(self.workspace[:4].view(torch.int32).item())

    # ------------------------------------------------------------ passes

    def run_rows(self, rows: list[tuple[int, int, int]], select: bool = False, hidden: bool = False):
        """One pass over explicit (token, sequence, position) rows. Returns
        (tokens or None, hidden [rows, 1024] float32 or None). Positions must
        continue each sequence (checked on the host)."""
        n = len(rows)
        if not 1 <= n <= MAX_ROWS:
            raise ValueError(f"a pass takes 1..{MAX_ROWS} rows")
        for tok, seq, pos in rows:
            if not 0 <= tok < self.vocab:
                raise ValueError(f"token id {tok} outside the vocabulary")
            if pos >= self.capacity:
                raise ValueError(f"KV capacity {self.capacity} reached")
        out = self._tokens if select else None
        h = torch.empty(n * HIDDEN, dtype=torch.bfloat16, device=self.device) if hidden else None
        run_pass(self._desc, rows, select, out, h, self._stream())
        for _, seq, pos in rows:
            self.positions[seq] = max(self.positions[seq], pos + 1)
        tokens = [int(t) for t in self._tokens[:n].cpu().tolist()] if select else None
        if self._status():
            raise RuntimeError(f"batched pass ended with status 0x{self._status():x}")
        return tokens, (_to_f32(h).reshape(n, HIDDEN) if hidden else None)

    def prefill(self, prompts: list[list[int]]) -> list[int]:
        """Run every sequence's prompt from its current position; returns each
        sequence's greedy next token (selected by its prompt's last row)."""
        if len(prompts) != self.sequences:
            raise ValueError(f"expected {self.sequences} prompts")
        pending = [(s, list(p)) for s, p in enumerate(prompts)]
        for s, p in pending:
            if not p:
                raise ValueError(f"prompt {s} is empty")
            if self.positions[s] + len(p) > self.capacity:
                raise ValueError(f"KV capacity {self.capacity} reached")
        nxt = [0] * self.sequences
        queue = [(s, i, t) for s, p in pending for i, t in enumerate(p)]
        start = list(self.positions)
        while queue:
            chunk, queue = queue[:MAX_ROWS], queue[MAX_ROWS:]
            rows = [(t, s, start[s] + i) for s, i, t in chunk]
            tokens, _ = self.run_rows(rows, select=True)
            for (s, i, _), tok in zip(chunk, tokens):
                if i == len(prompts[s]) - 1:
                    nxt[s] = tok
        return nxt

    def decode(self, tokens: list[int], n_steps: int) -> np.ndarray:
        """n_steps lockstep greedy steps: sequence s first consumes tokens[s].
        Returns the selected ids, int32 [n_steps, sequences]."""
        if len(tokens) != self.sequences:
            raise ValueError(f"expected {self.sequences} tokens")
        if n_steps < 1:
            raise ValueError("n_steps must be positive")
        for s, t in enumerate(tokens):
            if not 0 <= t < self.vocab:
                raise ValueError(f"token id {t} outside the vocabulary")
            if self.positions[s] + n_steps > self.capacity:
                raise ValueError(f"KV capacity {self.capacity} reached")
        tin = torch.tensor(tokens, dtype=torch.int32).to(self.device)
        out = torch.empty(n_steps * self.sequences, dtype=torch.int32, device=self.device)
        pos = np.ascontiguousarray(np.asarray(self.positions, dtype=np.int32))
        _lib.call("lfm25_batch_decode", ctypes.byref(self._desc), tin.data_ptr(), pos.ctypes.data, n_steps,
                  out.data_ptr(), self._stream())
        res = out.cpu().numpy().reshape(n_steps, self.sequences)
        if self._status():
            raise RuntimeError(f"batched decode ended with status 0x{self._status():x}")
        self.positions = [p + n_steps for p in self.positions]
        return res

    def decode_hidden(self, tokens: list[int], n_steps: int) -> tuple[np.ndarray, np.ndarray]:
        """As decode, on the persistent path only (2, 4 or 8 sequences; 16 below
        256 positions), also
        returning each step's pre-final-norm hidden states, float32
        [n_steps, sequences, 1024] holding BF16 values (what X8Model.hidden()
        returns after a step)."""
        if len(tokens) != self.sequences:
            raise ValueError(f"expected {self.sequences} tokens")
        if n_steps < 1:
            raise ValueError("n_steps must be positive")
        for s, t in enumerate(tokens):
            if not 0 <= t < self.vocab:
                raise ValueError(f"token id {t} outside the vocabulary")
            if self.positions[s] + n_steps > self.capacity:
                raise ValueError(f"KV capacity {self.capacity} reached")
        tin = torch.tensor(tokens, dtype=torch.int32).to(self.device)
        out = torch.empty(n_steps * self.sequences, dtype=torch.int32, device=self.device)
        hid = torch.empty(n_steps * self.sequences * HIDDEN, dtype=torch.bfloat16, device=self.device)
        pos = np.ascontiguousarray(np.asarray(self.positions, dtype=np.int32))
        _lib.call("lfm25_batch_decode_hidden", ctypes.byref(self._desc), tin.data_ptr(), pos.ctypes.data, n_steps,
                  out.data_ptr(), hid.data_ptr(), self._stream())
        res = out.cpu().numpy().reshape(n_steps, self.sequences)
        if self._status():
            raise RuntimeError(f"batched decode ended with status 0x{self._status():x}")
        self.positions = [p + n_steps for p in self.positions]
        return res, _to_f32(hid).reshape(n_steps, self.sequences, HIDDEN)

    def generate(self, prompts: list[list[int]], n_gen: int) -> list[list[int]]:
        """Prompts, then n_gen greedy tokens per sequence (n_gen - 1 lockstep steps)."""
        if n_gen < 1:
            raise ValueError("n_gen must be at least 1")
        first = self.prefill(prompts)
        if n_gen == 1:
            return [[t] for t in first]
        rest = self.decode(first, n_gen - 1)
        return [[first[s]] + [int(t) for t in rest[:, s]] for s in range(self.sequences)]

    # ------------------------------------------------------------ state

    def conv_state(self, sequence: int, conv_index: int) -> np.ndarray:
        """HF conv state [1024, 3] of conv layer `conv_index` of a sequence."""
        n = HIDDEN * 3
        o = (sequence * CONV_LAYERS + conv_index) * n
        return _to_f32(self.conv_states[o:o + n]).reshape(HIDDEN, 3)

    def kv(self, sequence: int, att_index: int, position: int):
        """(keys, values) [8, position + 1, 64] of one attention layer of a sequence."""
        n = KV_HEADS * self.capacity * HEAD_DIM
        o = (sequence * ATT_LAYERS + att_index) * n
        k = self.keys[o:o + n].view(KV_HEADS, self.capacity, HEAD_DIM)[:, :position + 1]
        v = self.values[o:o + n].view(KV_HEADS, self.capacity, HEAD_DIM)[:, :position + 1]
        return _to_f32(k.contiguous()).reshape(KV_HEADS, position + 1, HEAD_DIM), \
            _to_f32(v.contiguous()).reshape(KV_HEADS, position + 1, HEAD_DIM)
