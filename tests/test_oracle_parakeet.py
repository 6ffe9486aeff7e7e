"""Pinning the Parakeet oracle (oracle/parakeet.py) on the CPU.

The reference commits no encoder fixtures (its weights and outputs live in a
git-ignored cache/), so the two restatements pin each other and closed forms
pin their parts: the BF16-boundary mirror (012_layer_test.py) and the FP32
layer (parakeet_hybrid.py) agree to BF16 precision on a whole layer;
LayerNorm of a constant row is its bias; the mirror's position-score index
T-1-i+j is NeMo's rel_shift; a delta depthwise kernel passes the gate through;
identical keys give the mean of the values; small-integer products are exact.
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest

from oracle import parakeet as P


@pytest.fixture(scope="module")
def layer():
    pk = importlib.import_module("ryzenai-npu-lab_amd.parakeet")
    return pk.synthetic_layer(0, 0, 16)


def test_mirror_and_fp32_layer_agree(layer):
    w, pos = layer
    rng = np.random.default_rng(1)
    x = P.r(rng.standard_normal((16, 1024)).astype(np.float32))
    x[13:] = 0
    xb, _ = P.block_bf16(x, w, pos, 13)
    xf = P.block_f32(x, w, pos, 13)
    c = P.compare(xf[:13], xb[:13])
    assert c["cosine"] > 0.99995 and c["rel_rms"] < 0.01, c


def test_layer_norm_of_constant_row_is_its_bias():
    g = P.r(np.linspace(0.5, 1.5, 1024).astype(np.float32))
    b = P.r(np.linspace(-1, 1, 1024).astype(np.float32))
    x = np.full((3, 1024), 2.5, np.float32)
    assert np.array_equal(P.ln(x, g, b), np.broadcast_to(b, (3, 1024)))


def test_position_index_is_nemo_rel_shift():
    rng = np.random.default_rng(2)
    T = 9
    X = rng.standard_normal((8, T, 2 * T - 1)).astype(np.float32)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    shifted = P.rel_shift(X)[:, :, :T]
    assert np.array_equal(shifted, X[:, i, T - 1 - i + j])


def test_delta_depthwise_kernel_passes_the_gate():
    rng = np.random.default_rng(3)
    c = P.r(rng.standard_normal((12, 2048)).astype(np.float32))
    dw = np.zeros((1024, 9), np.float32)
    dw[:, 4] = 1.0
    out = P.conv_module(c, dw, np.zeros(1024, np.float32), 10)
    g = P.r(c[:, :1024] * P.sig(c[:, 1024:]))
    g[10:] = 0
    assert np.array_equal(out, P.r(g * P.sig(g)))
    dw[:, 4] = 0.0
    dw[:, 5] = 1.0     # tap 5 reads the next frame
    out = P.conv_module(c, dw, np.zeros(1024, np.float32), 10)
    nxt = np.vstack([g[1:], np.zeros((1, 1024), np.float32)])
    assert np.array_equal(out, P.r(nxt * P.sig(nxt)))


def test_identical_keys_average_the_values():
    rng = np.random.default_rng(4)
    T, valid = 8, 6
    qkv = P.r(rng.standard_normal((T, 3072)).astype(np.float32))
    qkv[:, 1024:2048] = qkv[0, 1024:2048]          # every key equal
    bd = np.zeros((8, T, 2 * T), np.float32)
    o = P.attention(qkv, bd, np.zeros((8, 128), np.float32), valid)
    want = P.r(qkv[:valid, 2048:].mean(0, dtype=np.float64).astype(np.float32))
    assert np.abs(o - want).max() <= 2.0 ** -7 * np.abs(want).max()


def test_small_integer_gemm_is_exact():
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 4, (5, 64)).astype(np.float32)
    w = rng.integers(-3, 4, (64, 32)).astype(np.float32)
    assert np.array_equal(P.gemm(a, w), P.r((a.astype(np.int64) @ w.astype(np.int64)).astype(np.float32)))
