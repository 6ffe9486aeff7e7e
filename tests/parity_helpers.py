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


def _rb(x) -> np.ndarray:
    """BF16 rounding (round to nearest even) of values first rounded to FP32,
    as the oracle rounds."""
    return O.f32(O.bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)


def attention_interval(q, k_all, v_all, n_sum):
    """Where the GPU's BF16 decode attention context may lie, element by
    element, when it follows the oracle's algorithm (O.attention: s =
    bf16(q.k) * 0.125, p = bf16(exp(s - max) / sum), ctx = bf16(sum p v))
    with FP32 sums in another order (at most n_sum roundings on any path):
      * a score is the BF16 rounding of an FP32 dot product within 64 * 2**-24
        * sum |q k| of the exact one, so it can differ from the oracle's by
        ds_j > 0 only where that interval reaches a BF16 rounding boundary;
      * p = softmax(s) does not depend on the maximum subtracted, and scores
        moved by d_i (|d_i| <= ds_i) scale p_j by exp(d_j) / sum_i p_i
        exp(d_i), so p_j before its rounding lies within a relative delta_j
        of the oracle's (with expf's error, the FP32 sum of the exp terms and
        the quotient's rounding on top), and the rounded p may differ from
        the oracle's by dp_j (zero unless a boundary is in reach);
      * the context before its rounding is then within B = sum dp |v| +
        n_sum * 2**-24 * sum (p + dp) |v| of the oracle's exact sum, and BF16
        rounding is monotonic, so the GPU value lies in [bf16(c - B), bf16(c + B)].
    Returns (lo, hi) over [16 * 64]."""
    lo, hi = [], []
    fp = 4 * 2.0 ** -22 + n_sum * 2.0 ** -24   # exp terms, their sum, the quotient
    for hq in range(q.shape[0]):
        kv = hq // (q.shape[0] // k_all.shape[0])
        k, v = k_all[kv].astype(np.float64), v_all[kv].astype(np.float64)
        qq = q[hq].astype(np.float64)
        qk = k @ qq
        err = 1.01 * 64 * 2.0 ** -24 * (np.abs(k) @ np.abs(qq))
        s = _rb(qk) * 0.125
        ds = np.maximum(s - _rb(qk - err) * 0.125, _rb(qk + err) * 0.125 - s)
        e = np.exp(s - s.max())
        p_exact = e / e.sum()
        up = np.exp(ds) / np.sum(p_exact * np.exp(-ds))
        down = np.exp(-ds) / np.sum(p_exact * np.exp(ds))
        delta = np.maximum(up - 1, 1 - down) + fp
        p = _rb(p_exact)
        dp = np.maximum(np.abs(_rb(p_exact * (1 + delta)) - p), np.abs(p - _rb(p_exact * (1 - delta))))
        c = p @ v
        bound = dp @ np.abs(v) + n_sum * 2.0 ** -24 * ((p + dp) @ np.abs(v)) + 2.0 ** -23 * np.abs(c)
        lo.append(_rb(c - bound))
        hi.append(_rb(c + bound))
    return np.concatenate(lo), np.concatenate(hi)


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


def _logit_intervals(table_bits, gamma_bits, h_lo, h_hi, h_mid, dense=None):
    """Rigorous [lo_t, hi_t] of every BF16 logit over hidden states inside
    the element-wise box [h_lo, h_hi] (h_mid a point of it), with the FP32
    slack of the final norm and the head's sums. Returns (lo, hi, s_mid),
    s_mid the exact head sums at h_mid's normed vector."""
    x_lo = np.asarray(h_lo, np.float64)
    x_hi = np.asarray(h_hi, np.float64)
    x = np.asarray(h_mid, np.float32)
    g = O.f32(gamma_bits).astype(np.float32)
    # sum of squares over the box, then the scale's range with its FP32 slack
    sq_max = np.maximum(x_lo ** 2, x_hi ** 2)
    sq_min = np.where((x_lo <= 0) & (x_hi >= 0), 0.0, np.minimum(x_lo ** 2, x_hi ** 2))
    d = GAMMA_1024 + 8 * U
    r_lo = np.float32(1.0 / math.sqrt(float(np.sum(sq_max)) / 1024.0 + 1e-5) * (1 - d))
    r_hi = np.float32(1.0 / math.sqrt(float(np.sum(sq_min)) / 1024.0 + 1e-5) * (1 + d))
    ss = float(np.sum(x.astype(np.float64) ** 2))
    r_mid = np.float32(1.0 / math.sqrt(ss / 1024.0 + 1e-5))
    # n_k = bf16(bf16(x_k r) g_k) is monotone in x_k r, which is bilinear in
    # (x_k, r): its extremes are at the corners of the box
    corners = [_bf_f32(_bf_f32(np.float32(xv) * rv) * g)
               for xv in (x_lo.astype(np.float32), x_hi.astype(np.float32)) for rv in (r_lo, r_hi)]
    y_mid = _bf_f32(_bf_f32(x * r_mid) * g)
    y_lo = np.minimum.reduce(corners + [y_mid])
    y_hi = np.maximum.reduce(corners + [y_mid])
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
    return _bf_f32(lo32).astype(np.float64), _bf_f32(hi32).astype(np.float64), s_mid


def _first_max_check(lo, hi, s_mid, pick):
    n = lo.size

    def feasible(t: int) -> bool:
        before = lo[:t].max() if t > 0 else -np.inf
        after = lo[t + 1:].max() if t + 1 < n else -np.inf
        return bool(hi[t] > before and hi[t] >= after)

    # rows that could be the first maximum: hi_t must reach the largest lo
    cand = np.nonzero(hi >= lo.max())[0]
    n_feasible = sum(1 for t in cand if feasible(int(t)))
    first = int(np.argmax(_bf_f32(s_mid.astype(np.float32))))
    return feasible(int(pick)), n_feasible, first


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
    lo, hi, s_mid = _logit_intervals(table_bits, gamma_bits, x, x, x, dense)
    return _first_max_check(lo, hi, s_mid, pick)


def drift_pick_check(table_bits: np.ndarray, gamma_bits: np.ndarray, h_ref: np.ndarray, h_gpu: np.ndarray,
                     pick: int, dense: np.ndarray | None = None):
    """The stream bar against a teacher-forced reference: (ok, n_feasible,
    ref_first_max). The GPU's hidden state h_gpu differs from the
    reference's h_ref (the oracle's, on the same tokens) by the FP32 order
    of 14 layers of sums; d = |h_gpu - h_ref| per element is measured, not
    assumed. The GPU's pick is accepted when it can be the first maximum of
    the head's BF16 logits for some hidden state in the box
    [h_ref - d, h_ref + d] (which holds both states), with head_pick_check's
    slack for the final norm and the head's FP32 sums: a pick may differ from
    the reference's argmax only where that interval of logits contains both
    candidates, not by a fixed number of ulps."""
    ref = np.asarray(h_ref, np.float64)
    d = np.abs(np.asarray(h_gpu, np.float64) - ref)
    lo, hi, s_mid = _logit_intervals(table_bits, gamma_bits, ref - d, ref + d, np.asarray(h_ref, np.float32),
                                     dense)
    return _first_max_check(lo, hi, s_mid, pick)


# ------------------------------------------------------------------ batched streams


def stream_with_hidden(bd, prompts, n_gen):
    """Each sequence's prompt in one pass (hidden of every row), then n_gen - 1
    lockstep steps as one-row-per-sequence passes: (tokens, hidden) per
    sequence, hidden[i] the pre-final-norm state that selected tokens[i]."""
    rows = [(t, s, bd.positions[s] + i) for s, p in enumerate(prompts) for i, t in enumerate(p)]
    toks, h = [], []
    for c in range(0, len(rows), 64):  # passes of at most 64 rows (a row's bits do not depend on its pass)
        tc, hc = bd.run_rows(rows[c:c + 64], select=True, hidden=True)
        toks += tc
        h.append(hc)
    h = np.concatenate(h)
    last = np.cumsum([len(p) for p in prompts]) - 1
    out = [[toks[r]] for r in last]
    hid = [[h[r]] for r in last]
    for _ in range(n_gen - 1):
        rows = [(out[s][-1], s, bd.positions[s]) for s in range(len(prompts))]
        toks, h = bd.run_rows(rows, select=True, hidden=True)
        for s in range(len(prompts)):
            out[s].append(toks[s])
            hid[s].append(h[s])
    return out, hid


def oracle_stream_check(ck, prompt, toks, hidden, tag):
    """Teacher-forced oracle run of one sequence: every state within 16 ulps,
    and a pick other than the oracle's argmax only where the measured drift
    between the two states makes it a possible first maximum. Returns the
    number of exact picks and the explained others."""
    table, gamma = ck["model.embed_tokens.weight"], ck["model.embedding_norm.weight"]
    orc = O.Oracle(ck, capacity=64)
    recs = orc.greedy(prompt, len(toks), force=toks)
    exact, explained = 0, []
    for i, (t, rec, h) in enumerate(zip(toks, recs, hidden)):
        assert scale_ulps(h, rec.hidden) <= 16, (tag, i)
        if t == rec.token_out:
            exact += 1
            continue
        ok, n_feasible, _ = drift_pick_check(table, gamma, rec.hidden, h, t)
        assert ok, (tag, i, t, rec.token_out, n_feasible)
        explained.append((i, n_feasible))
    return exact, explained, orc
