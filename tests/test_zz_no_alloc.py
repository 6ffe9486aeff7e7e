"""lfm25_fused_vocab_static (the head with its candidates in the library's
static device array, no workspace) against lfm25_fused_vocab (caller
workspace), bit for bit, on two calls in a row, the second with a smaller
vocabulary; and its argument checks."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).cuda().view(torch.bfloat16)


def _head(lab, vocab, seed):
    table = lab.rng.normal_bf16(seed, "noalloc.E", vocab * 1024, 0.0, 0.02)
    gamma = lab.rng.normal_bf16(seed, "noalloc.g", 1024, 1.0, 0.02)
    hidden = lab.rng.normal_bf16(seed, "noalloc.h", 1024)
    return _dev(np.concatenate([gamma, table])), _dev(hidden)


def _run(lab, entry, packed, hidden, vocab, workspace=None):
    s = torch.cuda.current_stream().cuda_stream
    nxt = torch.full((1024,), float("nan"), dtype=torch.bfloat16, device="cuda")
    logits = torch.full((vocab,), float("nan"), dtype=torch.bfloat16, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    args = [hidden.data_ptr(), packed.data_ptr(), nxt.data_ptr(), tok.data_ptr(), logits.data_ptr(), vocab]
    if workspace is not None:
        args.append(workspace.data_ptr())
    lab._lib.call(entry, *args, s)
    torch.cuda.synchronize()
    return int(tok.item()), nxt.view(torch.int16).cpu().numpy(), logits.view(torch.int16).cpu().numpy()


def test_static_head_equals_workspace_head_twice(gpu, lab):
    lib = lab._lib.load()
    for vocab, seed in ((65536, 1), (4100, 2)):       # the second call is smaller
        packed, hidden = _head(lab, vocab, seed)
        ws = torch.empty(int(lib.lfm25_argmax_workspace_bytes(vocab)), dtype=torch.uint8, device="cuda")
        want = _run(lab, "lfm25_fused_vocab", packed, hidden, vocab, ws)
        got = _run(lab, "lfm25_fused_vocab_static", packed, hidden, vocab)
        assert got[0] == want[0] and 0 <= got[0] < vocab, (vocab, got[0], want[0])
        assert np.array_equal(got[1], want[1]), vocab
        assert np.array_equal(got[2], want[2]), vocab


def test_static_head_rejects_sizes_beyond_its_array(gpu, lab):
    packed, hidden = _head(lab, 8, 3)
    with pytest.raises(ValueError):
        _run(lab, "lfm25_fused_vocab_static", packed, hidden, 65540)
    with pytest.raises(ValueError):
        _run(lab, "lfm25_fused_vocab_static", packed, hidden, 6)
