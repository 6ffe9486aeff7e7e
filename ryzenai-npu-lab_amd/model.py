"""X8Model: the reference's LFM2.5 layer/step API over the gfx950 decoder.

Same methods, arguments, return types and errors as
experiments/lfm25_x8_model.py:33-148 (X8Model): reset / step / prefill /
prefill_batch / hidden / conv_state / kv / prefill_hidden, attributes
position / capacity / tiers, ValueError("KV capacity ... reached") before a
run that would overflow, RuntimeError when a device run fails. Arrays come
back as float32 numpy arrays holding the BF16 values (ml_dtypes is not
available), in the unpacked HF layouts.

Differences a caller can see: the constructor also takes the weight source
(a seeded synthetic checkpoint, a checkpoint dict or a safetensors path),
the device, the execution mode, whether prompts use the batched pass and the
weight format ("bf16", or "w8g32": every projection and the tied table as
int8 with one FP32 scale per row and 32 inputs, the format the reference's
INT8 study ranks first, experiments/014_int8_lfm25.py); KV tiers are accepted for compatibility
but the GPU streams exactly the filled positions, so only the largest tier
(the capacity) matters. `generate(prompt, n)` runs the prompt as prefill does
and then the greedy tokens in one device call, with no host round trip per
token. A prompt's tokens before the last go through matrix-core passes of up
to 64 positions, as the reference's prefill sends its full PB batches
through prefill_batch.
"""

from __future__ import annotations

import time

import numpy as np
import torch

from . import _lib
from .batch import run_pass
from .bf16 import bf16_bits_to_f32
from .weights import (HEAD_DIM, HIDDEN, KINDS, KV_HEADS, VOCAB, load_safetensors, pack_stream, pack_w8,
                      rope_table, synthetic_checkpoint)

TIERS = (64, 256, 1024, 4096)
MAX_CAPACITY = 4096
PB = 4  # prompt tokens per batched call (experiments/lfm25_x8.py:79)
PASS_ROWS = 64  # prompt positions per matrix-core pass (LFM25_BATCH_MAX_ROWS)
CONV_LAYERS = KINDS.count("conv")
ATT_LAYERS = KINDS.count("attention")


def _u16_to_device(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    if not a.flags.writeable:  # a memory-mapped checkpoint tensor
        a = a.copy()
    t = torch.from_numpy(a.view(np.int16).reshape(-1))
    return t.to(device).view(torch.bfloat16)


def _to_f32(t: torch.Tensor) -> np.ndarray:
    return bf16_bits_to_f32(t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


class X8Model:
    def __init__(self, tiers=TIERS, log=print, *, weights=None, seed: int = 0,
                 vocab: int = VOCAB, device="cuda", exec_mode: str = "persistent",
                 batched_prefill: bool = True, weight_format: str = "bf16"):
        self.tiers = tuple(sorted(tiers))
        self.capacity = self.tiers[-1]
        if not 1 <= self.capacity <= MAX_CAPACITY:
            raise ValueError(f"capacity must be in [1, {MAX_CAPACITY}]")
        if exec_mode not in ("persistent", "staged"):
            raise ValueError("exec_mode must be 'persistent' or 'staged'")
        self.exec = _lib.EXEC_PERSISTENT if exec_mode == "persistent" else _lib.EXEC_STAGED
        if weight_format not in ("bf16", "w8g32"):
            raise ValueError("weight_format must be 'bf16' or 'w8g32'")
        # 8-bit weights run on the persistent decode only (the batched pass
        # and the staged kernels are BF16), so prompts go token by token
        self.w8 = weight_format == "w8g32"
        if self.w8 and exec_mode != "persistent":
            raise ValueError("weight_format 'w8g32' needs exec_mode 'persistent'")
        # prompts in matrix-core passes (False: token by token through the
        # decode, so that any split of a transcript into turns gives the same bits)
        self.batched_prefill = bool(batched_prefill) and not self.w8
        self.device = torch.device(device)
        lib = _lib.load()
        t0 = time.perf_counter()
        if weights is None:
            ck = synthetic_checkpoint(seed, vocab)
        elif isinstance(weights, dict):
            ck = weights
        else:
            ck = load_safetensors(weights)
        table = ck["model.embed_tokens.weight"]
        self.vocab = int(table.shape[0])
        if self.vocab % 4:
            raise ValueError("vocabulary size must be a multiple of 4")
        stream = pack_stream(ck)
        if stream.size != lib.lfm25_weights_elems():
            raise ValueError("packed weight stream does not match the library layout")
        self.weights = _u16_to_device(stream, self.device)
        self.table = _u16_to_device(table, self.device)
        self.rope = _u16_to_device(rope_table(self.capacity), self.device)
        bf = dict(dtype=torch.bfloat16, device=self.device)
        self.conv_states = torch.zeros(CONV_LAYERS * HIDDEN * 3, **bf)
        kv = ATT_LAYERS * KV_HEADS * self.capacity * HEAD_DIM
        self.keys = torch.zeros(kv, **bf)
        self.values = torch.zeros(kv, **bf)
        self.workspace = torch.zeros(lib.lfm25_decoder_workspace_bytes(), dtype=torch.uint8,
                                     device=self.device)
        self.ctl = self.workspace[:256].view(torch.int32)
        # residual stream: 1024 words of [bf16 value | 16-bit epoch tag]
        self._h_words = self.workspace[256:256 + 4 * HIDDEN].view(torch.int32)
        self._tokens_in = torch.zeros(MAX_CAPACITY, dtype=torch.int32, device=self.device)
        self._tokens_out = torch.zeros(MAX_CAPACITY, dtype=torch.int32, device=self.device)
        self._desc = _lib.Decoder(
            self.weights.data_ptr(), self.table.data_ptr(), self.rope.data_ptr(),
            self.conv_states.data_ptr(), self.keys.data_ptr(), self.values.data_ptr(),
            self.workspace.data_ptr(), self.capacity, self.vocab)
        if self.exec == _lib.EXEC_PERSISTENT:
            # the persistent decode's one-time device set-up (its placement
            # probe allocates), here rather than inside the first step
            with torch.cuda.device(self.device):
                _lib.call("lfm25_init")
        self._w8 = None
        if self.w8:
            layers, tq, ts = pack_w8(ck)
            if layers.size != lib.lfm25_w8_layers_bytes():
                raise ValueError("8-bit weight stream does not match the library layout")
            self.w8_layers = torch.from_numpy(layers).to(self.device)
            self.w8_table = torch.from_numpy(tq.reshape(-1)).to(self.device)
            self.w8_table_scales = torch.from_numpy(ts.reshape(-1)).to(self.device)
            self._w8 = _lib.W8Model(self.w8_layers.data_ptr(), self.w8_table.data_ptr(),
                                    self.w8_table_scales.data_ptr())
        self._last_prompt_hidden = []
        self._batch = None
        self._hidden_from_batch = False
        self.reset()
        torch.cuda.synchronize(self.device)
        log(f"weights ready in {time.perf_counter() - t0:.1f} s")

    # ------------------------------------------------------------ control

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def reset(self):
        self.position = 0
        self._hidden_from_batch = False
        _lib.call("lfm25_decoder_reset", self._desc, self._stream())

    def _run(self, tokens, n_gen: int) -> list[int]:
        tokens = [int(t) for t in tokens]
        steps = len(tokens) + max(n_gen - 1, 0)
        if self.position + steps > self.capacity:
            raise ValueError(f"KV capacity {self.capacity} reached")
        for t in tokens:
            if not 0 <= t < self.vocab:
                raise ValueError(f"token id {t} outside the vocabulary")
        if len(tokens) > self._tokens_in.numel() or n_gen > self._tokens_out.numel():
            raise ValueError("too many tokens for one call")
        src = torch.tensor(tokens, dtype=torch.int32)
        self._tokens_in[:len(tokens)].copy_(src, non_blocking=False)
        if self.w8:
            _lib.call("lfm25_decode_w8", self._desc, self._w8, self._tokens_in.data_ptr(), len(tokens), n_gen,
                      self._tokens_out.data_ptr() if n_gen else None, self._stream())
        else:
            _lib.call("lfm25_decode", self._desc, self._tokens_in.data_ptr(), len(tokens), n_gen,
                      self._tokens_out.data_ptr() if n_gen else None, self.exec, self._stream())
        out = self._tokens_out[:n_gen].cpu().tolist() if n_gen else []
        status = int(self.ctl[_lib.CTL_STATUS].item())
        if status:
            raise RuntimeError(f"decode run ended with status 0x{status:x}")
        self.position += steps
        self._hidden_from_batch = False
        return [int(t) for t in out]

    # ------------------------------------------------------------ reference API

    def step(self, token_id, select=True):
        """Run one position. Returns the selected next token id when `select`."""
        if self.position >= self.capacity:
            raise ValueError(f"KV capacity {self.capacity} reached")
        out = self._run([token_id], 1 if select else 0)
        return out[0] if select else None

    def _batch_desc(self):
        if self._batch is None:
            lib = _lib.load()
            self._batch_ws = torch.zeros(lib.lfm25_batch_workspace_bytes(), dtype=torch.uint8,
                                         device=self.device)
            self._batch = _lib.Batch(
                self.weights.data_ptr(), self.table.data_ptr(), self.rope.data_ptr(),
                self.conv_states.data_ptr(), self.keys.data_ptr(), self.values.data_ptr(),
                self._batch_ws.data_ptr(), 1, self.capacity, self.vocab)
        return self._batch

    def _check_tokens(self, tokens, steps: int) -> None:
        if self.position + steps > self.capacity:
            raise ValueError(f"KV capacity {self.capacity} reached")
        for t in tokens:
            if not 0 <= int(t) < self.vocab:
                raise ValueError(f"token id {t} outside the vocabulary")

    def _prefill_rows(self, tokens) -> None:
        """Prompt positions without a selection, in matrix-core passes of up
        to 64 rows on the decoder's own caches (lfm25_batch_pass), then the
        position control word the decode continues from."""
        batch = self._batch_desc()
        for start in range(0, len(tokens), PASS_ROWS):
            chunk = tokens[start:start + PASS_ROWS]
            rows = [(int(t), 0, self.position + i) for i, t in enumerate(chunk)]
            run_pass(batch, rows, False, None, None, self._stream())
            self.position += len(chunk)
        self.ctl[_lib.CTL_POSITION] = self.position
        status = int(self._batch_ws[:4].view(torch.int32).item())
        if status:
            raise RuntimeError(f"batched pass ended with status 0x{status:x}")
        self._hidden_from_batch = False

    def _prompt(self, token_ids, n_gen: int) -> list[int]:
        """A prompt and n_gen greedy tokens, the way the reference's prefill
        runs a prompt (experiments/lfm25_x8_model.py:117-126): every token but
        the last in matrix-core passes (when there are at least PB of them;
        shorter bodies go token by token, one launch beating a pass), then the
        last token and the generated ones in one decode call."""
        tokens = [int(t) for t in token_ids]
        self._check_tokens(tokens, len(tokens) + max(n_gen - 1, 0))
        body = tokens[:-1]
        if len(body) < PB or not self.batched_prefill:
            return self._run(tokens, n_gen)
        self._prefill_rows(body)
        return self._run(tokens[-1:], n_gen)

    def prefill_batch(self, token_ids):
        """PB prompt positions in one batched pass, no token selection (the
        reference's prefill_design): every weight tile is read once for the PB
        rows and multiplied on the matrix cores (lfm25_batch_pass)."""
        if self.w8:
            raise ValueError("prefill_batch runs the BF16 weights; this model uses w8g32")
        if len(token_ids) != PB:
            raise ValueError(f"prefill_batch takes exactly {PB} tokens")
        if self.position + PB > self.capacity:
            raise ValueError(f"KV capacity {self.capacity} reached")
        for t in token_ids:
            if not 0 <= int(t) < self.vocab:
                raise ValueError(f"token id {t} outside the vocabulary")
        rows = [(int(t), 0, self.position + i) for i, t in enumerate(token_ids)]
        h = torch.empty(PB * HIDDEN, dtype=torch.bfloat16, device=self.device)
        run_pass(self._batch_desc(), rows, False, None, h, self._stream())
        status = int(self._batch_ws[:4].view(torch.int32).item())
        if status:
            raise RuntimeError(f"batched pass ended with status 0x{status:x}")
        self.position += PB
        self.ctl[_lib.CTL_POSITION] = self.position
        hidden = _to_f32(h).reshape(PB, HIDDEN)
        self._last_prompt_hidden = [hidden[t] for t in range(PB)]
        self._hidden_from_batch = True

    def prefill(self, token_ids):
        """Process prompt tokens; the last one also selects the next token.
        Returns the selected token id. The tokens before the last run in
        matrix-core passes of up to 64 positions (at least PB of them)."""
        if len(token_ids) < 1:
            raise ValueError("prefill needs at least one token")
        return self._prompt(token_ids, 1)[0]

    def generate(self, prompt, n_gen: int) -> list[int]:
        """Prompt (as prefill runs it) plus n_gen greedy tokens, the tokens in
        one device call."""
        if n_gen < 1:
            raise ValueError("n_gen must be at least 1")
        if len(prompt) < 1:
            raise ValueError("generate needs at least one prompt token")
        return self._prompt(prompt, n_gen)

    def hidden(self) -> np.ndarray:
        """Pre-final-norm output of the last layer for the latest position."""
        if self._hidden_from_batch:
            return self._last_prompt_hidden[-1]
        words = self._h_words.cpu().numpy().view(np.uint32)
        return bf16_bits_to_f32((words & 0xFFFF).astype(np.uint16))

    def prefill_hidden(self, token):
        """Last-layer output of token t of the most recent prefill_batch."""
        return self._last_prompt_hidden[token]

    def conv_state(self, conv_index) -> np.ndarray:
        """HF conv state [1024, 3] of recurrent layer `conv_index`."""
        if not 0 <= conv_index < CONV_LAYERS:
            raise ValueError("conv_index out of range")
        s = self.conv_states[conv_index * HIDDEN * 3:(conv_index + 1) * HIDDEN * 3]
        return _to_f32(s).reshape(HIDDEN, 3)

    def kv(self, att_index, position):
        """(keys, values) of shape (8, position + 1, 64) for one attention layer."""
        if not 0 <= att_index < ATT_LAYERS:
            raise ValueError("att_index out of range")
        if not 0 <= position < self.capacity:
            raise ValueError("position out of range")
        n = KV_HEADS * self.capacity * HEAD_DIM
        k = self.keys[att_index * n:(att_index + 1) * n].view(KV_HEADS, self.capacity, HEAD_DIM)
        v = self.values[att_index * n:(att_index + 1) * n].view(KV_HEADS, self.capacity, HEAD_DIM)
        return (_to_f32(k[:, :position + 1].contiguous()).reshape(KV_HEADS, position + 1, HEAD_DIM),
                _to_f32(v[:, :position + 1].contiguous()).reshape(KV_HEADS, position + 1, HEAD_DIM))
