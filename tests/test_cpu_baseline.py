"""The CPU baseline that bench.py times beside the GPU figures
(oracle/torch_cpu.py: the model op by op in PyTorch-CPU BF16, as the
reference's CPU path runs transformers' LFM2, experiments/010_cpu_greedy.py:
39-63) computes the same model as the oracle: on a small-vocabulary model
the greedy tokens are the oracle's and the hidden states stay within the
bound the GPU decode is held to (16 BF16 ulps of the vector's scale: the two
sum in different FP32 orders, and the baseline's SDPA keeps the attention
probabilities in FP32 where the oracle's eager path rounds them to BF16)."""

from __future__ import annotations

import importlib
import math

import numpy as np
import pytest

from oracle import lfm25 as O

torch = pytest.importorskip("torch")


def scale_ulps(got, want):
    s = float(np.max(np.abs(want)))
    ulp = 2.0 ** (math.floor(math.log2(s)) - 7)
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))) / ulp)


def test_torch_cpu_baseline_decodes_like_the_oracle():
    lab = importlib.import_module("ryzenai-npu-lab_amd")
    tc = importlib.import_module("oracle.torch_cpu")
    ck = lab.weights.synthetic_checkpoint(11, vocab=1024)
    prompt = [int(t) for t in lab.rng.uniform_ints(0, "baseline.prompt", 6, 10)]
    n_gen = 6
    torch.set_num_threads(4)
    dec = tc.TorchCpuDecoder(ck, capacity=64)
    orc = O.Oracle(ck, capacity=64)
    # prompt, teacher-forced on both
    for t in prompt[:-1]:
        dec.step(t, select=False)
        rec = orc.step(t, select=False)
        assert scale_ulps(dec.last_hidden.float().numpy(), rec.hidden) <= 16
    tok = prompt[-1]
    got, want, errs = [], [], []
    for _ in range(n_gen):
        g = dec.step(tok, select=True)
        rec = orc.step(tok, select=True)
        err = scale_ulps(dec.last_hidden.float().numpy(), rec.hidden)
        assert err <= 16, (len(got), err)
        errs.append(round(err, 2))
        got.append(g)
        want.append(rec.token_out)
        tok = rec.token_out
    assert got == want, (got, want)
    print("torch-CPU vs oracle: tokens", got, "hidden ulps", errs)
