"""Acceptance helpers shared by the GPU parity tests (not collected by pytest).

`head_pick_check` is the argmax bar of the target: given the GPU's own final
hidden state, the GPU's token must be the first maximum of the BF16 logits
except where the FP32 accumulation order can change which logit is largest.
It bounds every logit rigorously instead of allowing a fixed number of ulps:

  * final RMSNorm: the GPU's FP32 sum of 1024 squares is within
    gamma_1024 = 1024 u / (1 - 1024 u) (u = 2^-24) of the exact sum, and the
    scale, square root and reciprocal add a few u, so the scale r lies in
    [r0 (1 - d), r0 (1 + d)]; each normalised element n_k = bf16(bf16(x_k r)
    gamma_k) then takes one of the (at most two) values at the ends of that
    range (rounding is monotone);
  * head row t: the FP32 sum of the 1024 exact BF16 products is within
    gamma_1024 * sum_k |E_tk n_k| of the exact sum, and the elements whose
    n_k may differ move it by at most sum_k |E_tk| |n_k^hi - n_k^lo|;
  * the logit is BF16(FP32 sum), so it lies in [bf16(lo_t), bf16(hi_t)].

The GPU's pick g is acceptable when it can be the first maximum for some
logits inside those intervals: hi_g >= lo_t for every t > g and hi_g > lo_t
for every t < g (the first-index tie rule). The check also returns how many
rows could be the first maximum (1 for an unambiguous position).
"""

from __future__ import annotations

import math

import numpy as np

from oracle import lfm25 as O

U = 2.0 ** -24
GAMMA_1024 = 1024 * U / (1 - 1024 * U)


def scale_ulps(got, want) -> float:
    """Largest difference in BF16 ulps of the vector's largest magnitude."""
    s = float(np.max(np.abs(want)))
    ulp = 2.0 ** (math.floor(math.log2(s)) - 7) if s > 0 else 1.0
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))) / ulp)


def logit_ulp(logits: np.ndarray) -> float:
    best = float(np.max(np.abs(logits)))
    return 2.0 ** (math.floor(math.log2(best)) - 7)


def top2_gap_ulps(logits: np.ndarray, token: int) -> float:
    """(max logit - logit[token]) in BF16 ulps of the largest logit."""
    return float((float(np.max(logits)) - float(logits[token])) / logit_ulp(logits))


def _bf_f32(x) -> np.ndarray:
    return O._bf(np.asarray(x, np.float32))


def head_pick_check(table_bits: np.ndarray, gamma_bits: np.ndarray, hidden: np.ndarray, pick: int,
                    dense: np.ndarray | None = None):
    """(ok, n_feasible, oracle_first_max) for the GPU's pick from its own
    pre-final-norm hidden state (float32 BF16 values [1024]).

    dense: the head as FP32-exact float64 values instead of the BF16 table
    (the dequantized q s of an 8-bit table, table_bits unused). The 8-bit
    head sums 16 exact products q x per lane, scales each segment sum once
    and adds the 64 segments in FP32: within (gamma_1024 + 2 u) sum |q s x|
    of the exact sum, the bound used for it."""
    x = np.asarray(hidden, np.float32)
    g = O.f32(gamma_bits).astype(np.float32)
    ss = float(np.sum(x.astype(np.float64) ** 2))
    r0 = 1.0 / math.sqrt(ss / 1024.0 + 1e-5)
    d = GAMMA_1024 + 8 * U
    ends = []
    for r in (np.float32(r0 * (1 - d)), np.float32(r0), np.float32(r0 * (1 + d))):
        ends.append(_bf_f32(_bf_f32(x * r) * g))
    y_lo = np.minimum(np.minimum(ends[0], ends[1]), ends[2])
    y_hi = np.maximum(np.maximum(ends[0], ends[1]), ends[2])
    y_mid = ends[1]
    y_abs = np.maximum(np.abs(y_lo), np.abs(y_hi))
    width = (y_hi - y_lo).astype(np.float64)
    idx = np.nonzero(width)[0]
    if dense is None:
        s_mid = O.gemv_exact(table_bits, y_mid)
        mag = O.gemv_exact(table_bits & np.uint16(0x7FFF), y_abs)
        cols = lambda: np.abs(O.f32(table_bits[:, idx]).astype(np.float64))  # noqa: E731
        gamma = GAMMA_1024
    else:
        s_mid = dense @ y_mid.astype(np.float64)
        mag = np.abs(dense) @ y_abs.astype(np.float64)
        cols = lambda: np.abs(dense[:, idx])  # noqa: E731
        gamma = GAMMA_1024 + 2 * U
    delta = np.zeros_like(s_mid)
    if idx.size:
        delta = cols() @ width[idx]
    slack = gamma * mag + delta
    lo32 = np.nextafter((s_mid - slack).astype(np.float32), np.float32(-np.inf))
    hi32 = np.nextafter((s_mid + slack).astype(np.float32), np.float32(np.inf))
    lo, hi = _bf_f32(lo32).astype(np.float64), _bf_f32(hi32).astype(np.float64)
    n = lo.size

    def feasible(t: int) -> bool:
        before = lo[:t].max() if t > 0 else -np.inf
        after = lo[t + 1:].max() if t + 1 < n else -np.inf
        return bool(hi[t] > before and hi[t] >= after)

    # rows that could be the first maximum: hi_t must reach the largest lo
    cand = np.nonzero(hi >= lo.max())[0]
    n_feasible = sum(1 for t in cand if feasible(int(t)))
    oracle_pick = int(np.argmax(_bf_f32(s_mid.astype(np.float32))))
    return feasible(int(pick)), n_feasible, oracle_pick

