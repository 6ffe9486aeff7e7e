"""Multi-turn greedy chat on the GPU decoder with state reuse across turns.

`Chat` mirrors the reference's chat runner (experiments/010_lfm25_npu_chat.py:
32-79, `NPUChat.respond`): each turn renders the transcript, and when the new
token ids strictly extend the ids the decoder has already consumed, only the
new suffix is prefilled; otherwise the decoder is reset first. Greedy reply
tokens are stepped one at a time until EOS (id 7) or the token limit, and
every token fed to the decoder is appended to the consumed list, so the
device's conv state and KV cache always hold exactly that prefix.

Tokenization needs the model's tokenizer.json (`tokenizers` package); the
id-level entry point `respond_ids` needs neither, and is what the tests use.
"""

from __future__ import annotations

import time

EOS_ID = 7


def render_chat(messages) -> str:
    """The LFM2.5 chat template the reference renders
    (010_lfm25_npu_chat.py:23-28): a start token, one im_start/im_end block per
    message, then the opening of the assistant's turn."""
    out = ["<|startoftext|>"]
    out.extend(f"<|im_start|>{m['role']}\n{m['content']}<|im_end|>\n" for m in messages)
    out.append("<|im_start|>assistant\n")
    return "".join(out)


class Chat:
    """model: an X8Model (or anything with its reset / prefill / step API and
    a `capacity`); tokenizer: a tokenizers.Tokenizer, or a path to a
    tokenizer.json, or None for the id-level API only."""

    def __init__(self, model, tokenizer=None, eos_id: int = EOS_ID):
        self.model = model
        if isinstance(tokenizer, (str, bytes)) or hasattr(tokenizer, "__fspath__"):
            from tokenizers import Tokenizer
            tokenizer = Tokenizer.from_file(str(tokenizer))
        self.tokenizer = tokenizer
        self.eos_id = eos_id
        self.consumed: list[int] = []

    def reset(self):
        self.model.reset()
        self.consumed = []

    def respond_ids(self, ids, max_new_tokens: int) -> dict:
        """One turn over the token ids of the whole transcript. Returns the
        reference's result fields (generated ids, how many prompt tokens were
        processed, whether the device state was reused, timings)."""
        ids = [int(t) for t in ids]
        if not ids:
            raise ValueError("the transcript has no tokens")
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be at least 1")
        if len(ids) + max_new_tokens > self.model.capacity:
            raise ValueError(f"Transcript needs {len(ids) + max_new_tokens} positions; "
                             f"the KV cache holds {self.model.capacity}.")
        n = len(self.consumed)
        reuse = 0 < n < len(ids) and ids[:n] == self.consumed
        if not reuse:
            self.reset()
        t0 = time.perf_counter()
        pending = ids[len(self.consumed):]
        next_id = self.model.prefill(pending)
        self.consumed = list(ids)
        first = time.perf_counter() - t0
        generated = []
        steps = 0
        t1 = time.perf_counter()
        while next_id != self.eos_id and len(generated) < max_new_tokens:
            generated.append(next_id)
            if len(generated) == max_new_tokens:
                break
            self.consumed.append(next_id)
            next_id = self.model.step(next_id)
            steps += 1
        decode = time.perf_counter() - t1
        return {
            "generated_ids": generated,
            "prompt_tokens": len(ids),
            "prompt_tokens_processed": len(pending),
            "reused_state": reuse,
            "generated_tokens": len(generated),
            "time_to_first_token_s": round(first, 4),
            "decode_tokens_per_s": round(steps / decode, 1) if steps else None,
            "stopped_on_eos": next_id == self.eos_id,
        }

    def respond(self, messages, max_new_tokens: int) -> dict:
        """One turn over chat messages ([{"role": ..., "content": ...}]):
        render, tokenize, respond_ids, and decode the reply text."""
        if self.tokenizer is None:
            raise RuntimeError("respond needs a tokenizer (the model's tokenizer.json)")
        ids = self.tokenizer.encode(render_chat(messages), add_special_tokens=False).ids
        out = self.respond_ids(ids, max_new_tokens)
        out["response"] = self.tokenizer.decode(out["generated_ids"])
        return out
