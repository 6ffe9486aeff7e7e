"""The bars of the GPU tests checked on the CPU against the oracle: the argmax
bar (parity_helpers.head_pick_check) accepts the oracle's own first maximum,
rejects planted wrong picks and keeps the first-index rule on exact ties; the
attention interval (parity_helpers.attention_interval) holds the oracle's
context and an FP32-order restatement of it, and rejects planted mistakes."""

from __future__ import annotations

import numpy as np

from oracle import lfm25 as O
from parity_helpers import attention_interval, head_pick_check


def _head(lab, vocab=4096, seed=5):
    table = lab.rng.normal_bf16(seed, "helper.E", vocab * 1024, 0.0, 0.02).reshape(vocab, 1024)
    gamma = lab.rng.normal_bf16(seed, "helper.g", 1024, 1.0, 0.02)
    hidden = O.f32(lab.rng.normal_bf16(seed, "helper.h", 1024))
    return table, gamma, hidden


def _logits(table, gamma, hidden):
    return O.linear(table, O.rms_norm(hidden, O.f32(gamma)))


def test_accepts_the_oracle_pick_and_rejects_others(lab):
    table, gamma, hidden = _head(lab)
    logits = _logits(table, gamma, hidden)
    best = O.argmax_first(logits)
    ok, n, first = head_pick_check(table, gamma, hidden, best)
    assert ok and first == best and n >= 1
    order = np.argsort(-logits.astype(np.float64), kind="stable")
    far = int(order[len(order) // 2])   # a median logit
    assert not head_pick_check(table, gamma, hidden, far)[0]
    # a runner-up two or more BF16 steps below the top is never acceptable
    for t in (int(v) for v in order[1:40]):
        steps = (int(O.bf16_bits(logits[best:best + 1])[0]) - int(O.bf16_bits(logits[t:t + 1])[0]))
        if logits[best] > 0 and logits[t] > 0 and steps >= 2:
            assert not head_pick_check(table, gamma, hidden, t)[0], (t, steps)
            break
    else:
        raise AssertionError("no runner-up two steps below the maximum")


def test_exact_tie_keeps_the_first_index(lab):
    table, gamma, hidden = _head(lab)
    logits = _logits(table, gamma, hidden)
    best = O.argmax_first(logits)
    tied = table.copy()
    low = 7 if best > 7 else best + 1
    tied[low] = table[best]           # identical rows: identical sums in any order
    first = min(low, best)
    ok, n, oracle_first = head_pick_check(tied, gamma, hidden, first)
    assert ok and oracle_first == first and n >= 2


def test_planted_shift_of_a_row_is_rejected(lab):
    """A pick whose logit is several ulps below the maximum fails, however
    the accumulation order went."""
    table, gamma, hidden = _head(lab)
    logits = _logits(table, gamma, hidden)
    best = O.argmax_first(logits)
    shifted = table.copy()
    row = (best + 1) % table.shape[0]
    shifted[row] = table[best]
    # scale the copied row down by 1/8: its logit drops far below the maximum
    shifted[row] = O.bf16_bits(O.f32(table[best]) * np.float32(0.875))
    assert head_pick_check(shifted, gamma, hidden, best)[0]
    assert not head_pick_check(shifted, gamma, hidden, row)[0]


def test_drift_bar_reduces_to_the_head_check_without_drift(lab):
    from parity_helpers import drift_pick_check
    table, gamma, hidden = _head(lab)
    logits = _logits(table, gamma, hidden)
    best = O.argmax_first(logits)
    order = np.argsort(-logits.astype(np.float64), kind="stable")
    for t in (best, int(order[1]), int(order[len(order) // 2])):
        assert drift_pick_check(table, gamma, hidden, hidden, t) == head_pick_check(table, gamma, hidden, t)


def test_drift_bar_widens_only_with_the_measured_drift(lab):
    """Planted runners-up 4 and 8 BF16 steps below the maximum: with the GPU
    state equal to the reference both are rejected; a drift of 2 ulps on 16
    elements does not reach the nearer one, on 64 it does; the farther one
    stays out of reach with 128 drifted elements, and a median pick is never
    accepted. (A drift on every element widens the box far more: the bound is
    rigorous, so its width follows the measured drift.)"""
    from parity_helpers import drift_pick_check
    table, gamma, hidden = _head(lab)
    logits = _logits(table, gamma, hidden)
    best = O.argmax_first(logits)
    order = np.argsort(-logits.astype(np.float64), kind="stable")
    row, median = int(order[len(order) // 3]), int(order[len(order) // 2])
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(hidden), 1e-30))) - 7)
    perm = np.random.RandomState(0).permutation(1024)

    def drifted(m):
        idx = perm[:m]
        out = hidden.copy()
        out[idx] = O.f32(O.bf16_bits((hidden[idx] + 2 * ulp[idx] * np.sign(hidden[idx])).astype(np.float32)))
        return out

    for frac, reach in ((0.98, (16, 64)), (0.95, (128, None))):
        planted = table.copy()
        planted[row] = O.bf16_bits(O.f32(table[best]) * np.float32(frac))
        lg = _logits(planted, gamma, hidden)
        assert O.argmax_first(lg) == best and lg[row] < lg[best]
        assert not drift_pick_check(planted, gamma, hidden, hidden, row)[0]
        short, long_ = reach
        assert not drift_pick_check(planted, gamma, hidden, drifted(short), row)[0], (frac, short)
        if long_ is not None:
            ok, n_feasible, first = drift_pick_check(planted, gamma, hidden, drifted(long_), row)
            assert ok and n_feasible == 2 and first == best, (frac, long_)
        assert not drift_pick_check(planted, gamma, hidden, drifted(128), median)[0]


# ------------------------------------------------------------------ attention interval


def _attention_case(seed, positions):
    r = np.random.RandomState(seed)
    q = O._bf(r.standard_normal((16, 64)).astype(np.float32))
    k = O._bf(r.standard_normal((8, positions, 64)).astype(np.float32))
    v = O._bf(r.standard_normal((8, positions, 64)).astype(np.float32))
    return q, k, v


def _attention_fp32(q, k, v, round_p=True, scale=np.float32(0.125)):
    """The oracle's algorithm with every sum in FP32 (numpy's order, not the
    oracle's exact one); round_p / scale plant mistakes."""
    out = []
    for hq in range(16):
        kk, vv = k[hq // 2], v[hq // 2]
        s = O._bf(kk @ q[hq]) * scale
        e = np.exp(s - s.max())
        p = e / e.sum(dtype=np.float32)
        if round_p:
            p = O._bf(p)
        out.append(O._bf(p.astype(np.float32) @ vv))
    return np.concatenate(out)


def test_attention_interval_holds_fp32_orders_and_rejects_mistakes():
    for seed, positions in ((1, 1), (2, 22), (3, 1024), (4, 4096)):
        q, k, v = _attention_case(seed, positions)
        lo, hi = attention_interval(q, k, v, positions + 64)
        inside = lambda c: np.all((c >= lo) & (c <= hi))  # noqa: E731
        assert inside(O.attention(q, k, v).astype(np.float64)), positions
        assert inside(_attention_fp32(q, k, v).astype(np.float64)), positions
        if positions > 1:
            # the current position left out, probabilities not rounded to BF16,
            # and the wrong score scale each leave the interval
            assert not inside(O.attention(q, k[:, :-1], v[:, :-1]).astype(np.float64)), positions
            if positions <= 1024:
                # (at 4,096 terms the worst-case FP32 sum error, 2.5e-4 of the
                # sum, leaves a boundary in reach of ~13% of the probabilities,
                # wider than the ~0.4-ulp effect of not rounding them)
                assert not inside(_attention_fp32(q, k, v, round_p=False).astype(np.float64)), positions
            assert not inside(_attention_fp32(q, k, v, scale=np.float32(0.125 * 1.01)).astype(np.float64)), positions
