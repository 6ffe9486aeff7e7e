"""Host-side checker of the persistent decode's exchange schedule.

The persistent decode (csrc/lfm25_decode.hip, csrc/lfm25_step.h) hands every
activation between blocks through tagged words: a consumer polls a buffer
until each word carries the epoch tag of the exchange that produced it, and
the next writer of a buffer relies on the exchanges in between to know that
every reader of the previous value is done. This module restates that
schedule (which block writes and reads which words of which buffer, in what
order, with what tag) and checks it before anything runs on a GPU, the way
the reference checks its NPU schedules statically (experiments/pk_engine.py:
365-425, `check`): it returns a list of problems, empty when the schedule is
sound. It is a scheduling check of the modelled order, not a proof about the
hardware.

Checked, for every word of every exchange buffer, over a run of decode steps:
  * read after write: a poll for tag t reads words whose last write in the
    schedule carries t (else the poll could never end), and whose previous
    value (or the zeroed workspace, tag 0) does not carry t (else a stale word
    could end it early);
  * write after read: every block that read the previous value of a word has
    finished that read before the next writer's store, through a chain of
    exchanges (vector clocks over the blocks' program order and the
    producer -> consumer edges);
  * placement: the XCD-local buffers (plain stores, non-temporal loads through
    one XCD's L2) have every producer and consumer on that XCD;
  * untagged data: each KV-cache row a block prefetches was appended before
    the prefetch through such a chain, and no prefetch reaches a row that is
    not appended yet (the KV loads may hit the CU's vector L1, which is not
    coherent within a launch: a line read before the append could be served
    stale after it; rows of earlier calls are ordered by the launch, at whose
    start the L1 is invalidated);
  * coverage of the split attention: every position of [0, pos] is scored
    by a block that takes part (gathers q/k/v), so no term of the softmax is
    dropped;
  * tag accounting: the exchanges of a step take consecutive tags from the
    step's epoch, and the epoch advances by the constants the kernels use.

Layout of the grid: block b runs on XCD b % 8 as block j = b // 8 there;
group j // 16 computes layers of that parity, block jj = j % 16 of its group
owning residual rows [64jj, 64jj + 64) and, on XCD x, conv channels
128x + 8jj .. + 8, q/k/v entries 16jj .. + 16, FFN columns 320x + 20jj .. + 20.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

XCDS = 8
GROUP_BLOCKS = 16
BLOCKS = 256
LAYERS = 14
ATTN_LAYERS = (2, 4, 6, 8, 10, 12)  # lfm25_x8.py:55-57
ATTN_SINGLE_BELOW = 256             # kAttnSingleBelow: positions below attend on blocks (x, 0..1)
ATTN_SLOTS = 64                     # positions per register pass
CONV_EXCHANGES, ATTN_EXCHANGES, HEAD_EXCHANGES = 6, 8, 2
TAG_MASK = 0xFFFF


def xcd(b: int) -> int:
    return b % XCDS


def group(b: int) -> int:
    return (b // XCDS) // GROUP_BLOCKS


def jj_of(b: int) -> int:
    return (b // XCDS) % GROUP_BLOCKS


def block(x: int, g: int, jj: int) -> int:
    return (g * GROUP_BLOCKS + jj) * XCDS + x


def group_blocks(g: int, x: int | None = None) -> list[int]:
    xs = range(XCDS) if x is None else (x,)
    return [block(xx, g, jj) for xx in xs for jj in range(GROUP_BLOCKS)]


# Exchange buffers: name -> (words, local). Local buffers exist once per XCD.
BUFFERS = {
    "lh0": (1024, True), "lh1": (1024, True), "ly": (128, True), "lq": (256, True),
    "ls": (64, True), "lc": (GROUP_BLOCKS * 128, True), "lg": (384, True), "lw": (64, True),
    "gp0": (GROUP_BLOCKS * XCDS * 64, False), "gp1": (GROUP_BLOCKS * XCDS * 64, False),
    "gw": (GROUP_BLOCKS * XCDS, False),
}


@dataclass
class Options:
    """Schedule variants. The defaults are the kernels' schedule; the others
    exist so tests can plant mistakes and see `check` reject them."""
    fence: bool = True                  # group 0 waits for the last h after a step without a head
    residual_buffers: tuple = ("lh0", "lh1")  # R1 -> first, R2 -> second
    partial_buffers: tuple = ("gp0", "gp1")   # P2 -> first, P4 -> second
    head_exchanges: int = HEAD_EXCHANGES      # epoch advance of a step with a head
    local_gather_xcd: int = 0           # added to the XCD a local gather reads (0: its own)
    # split attention: which blocks publish an empty share at once, without
    # gathering q/k/v: "none" (every block takes part: the kernels),
    # "cached" (blocks whose passes hold no cached position, i.e. none
    # below the current one), "scored" (blocks that score no position of
    # [0, pos]); with either rule a block that alone takes part skips the
    # statistics exchange
    empty_split: str = "none"
    single_below: int = ATTN_SINGLE_BELOW  # positions below attend on blocks (x, 0..1)
    prefetch_past: int = 0              # KV rows prefetched beyond the cached ones (kernels: 0)


@dataclass
class _Buf:
    tag: np.ndarray               # tag of each word's last write (the zeroed workspace: 0)
    prev: np.ndarray              # the tag before that
    writer: np.ndarray            # snapshot id of each word's last write (-1: reset)
    reads: np.ndarray             # [word][block]: event index of the block's last read since the write (0: none)


class Checker:
    def __init__(self, opts: Options | None = None):
        self.opts = opts or Options()
        self.problems: list[str] = []
        self.vc = np.zeros((BLOCKS, BLOCKS), np.int32)   # current vector clock per block
        self.n = np.zeros(BLOCKS, np.int32)              # events so far per block
        self.snaps: dict[int, np.ndarray] = {}
        self.next_snap = 0
        self.bufs: dict[tuple, _Buf] = {}
        self.kv: dict[tuple, tuple] = {}                 # (layer, x, position) -> (block, event index)
        self.epoch = 0
        self.step_no = 0

    # ------------------------------------------------------------------ primitives

    def _buf(self, name: str, x: int | None) -> _Buf:
        key = (name, x)
        if key not in self.bufs:
            words = BUFFERS[name][0]
            self.bufs[key] = _Buf(np.zeros(words, np.int64), np.zeros(words, np.int64),
                                  np.full(words, -1, np.int64), np.zeros((words, BLOCKS), np.int32))
        return self.bufs[key]

    def _event(self, b: int) -> int:
        self.n[b] += 1
        self.vc[b, b] = self.n[b]
        return int(self.n[b])

    def _check_local(self, name: str, x: int | None, b: int, what: str) -> None:
        if BUFFERS[name][1] and xcd(b) != x:
            self.problems.append(f"step {self.step_no}: block {b} (XCD {xcd(b)}) {what} local buffer "
                                 f"{name}[{x}]")

    def write(self, b: int, name: str, x: int | None, lo: int, hi: int, tag: int, where: str) -> None:
        self._check_local(name, x, b, "writes")
        buf = self._buf(name, x)
        self._event(b)
        snap = self.vc[b].copy()
        late = buf.reads[lo:hi] > snap[None, :]
        late[:, b] = False  # the writer's own reads precede it in program order
        if late.any():
            w, c = np.argwhere(late)[0]
            self.problems.append(
                f"step {self.step_no} {where}: block {b} rewrites {name}[{x}] word {lo + w} before "
                f"block {c} has finished reading it")
        buf.reads[lo:hi] = 0
        sid = self.next_snap
        self.next_snap += 1
        self.snaps[sid] = snap
        buf.prev[lo:hi] = buf.tag[lo:hi]
        buf.tag[lo:hi] = tag
        buf.writer[lo:hi] = sid

    def read(self, b: int, name: str, x: int | None, lo: int, hi: int, tag: int, where: str) -> None:
        self._check_local(name, x, b, "reads")
        buf = self._buf(name, x)
        cur = buf.tag[lo:hi]
        if np.any(cur != tag):
            self.problems.append(f"step {self.step_no} {where}: block {b} polls {name}[{x}] "
                                 f"[{lo}, {hi}) for tag {tag} before it is written there")
        if np.any(buf.prev[lo:hi] == tag):
            self.problems.append(f"step {self.step_no} {where}: a stale word of {name}[{x}] "
                                 f"[{lo}, {hi}) already carries tag {tag}")
        for sid in np.unique(buf.writer[lo:hi]):
            if sid >= 0:
                np.maximum(self.vc[b], self.snaps[int(sid)], out=self.vc[b])
        buf.reads[lo:hi, b] = self._event(b)

    def kv_append(self, b: int, layer: int, position: int) -> None:
        self.kv[(layer, xcd(b), position)] = (b, self._event(b))

    def kv_prefetch(self, b: int, layer: int, positions, pos: int) -> None:
        for p in positions:
            if p >= pos:
                # untagged data read before it exists: the loads are default-
                # policy (they may hit the CU's vector L1), so the line read now
                # can still be served from the L1 after the row is appended
                self.problems.append(f"step {self.step_no}: block {b} prefetches the KV row {p} of layer {layer} "
                                     f"at position {pos}, before it is appended (its line can stay stale in the "
                                     f"block's L1)")
                continue
            w = self.kv.get((layer, xcd(b), p))
            if w is None:
                continue  # a row of an earlier call: ordered by the launch boundary (L1 invalidated at launch)
            writer, widx = w
            if writer != b and self.vc[b, writer] < widx:
                self.problems.append(f"step {self.step_no}: block {b} prefetches the KV row {p} of "
                                     f"layer {layer} before block {writer}'s append of it is ordered before")
        self._event(b)

    # ------------------------------------------------------------------ the step

    def _tags(self):
        base, k = self.epoch, 0

        def take():
            nonlocal k
            k += 1
            return (base + k) & TAG_MASK
        return take, lambda: k

    def _gather_all(self, name: str, readers, tag: int, where: str) -> None:
        words = BUFFERS[name][0]
        for b in readers:
            self.read(b, name, xcd(b) + self.opts.local_gather_xcd if BUFFERS[name][1] else None,
                      0, words, tag, where)

    def _residual(self, g: int, gp: str, lh: str, tag_p: int, tag_h: int, where: str) -> None:
        for b in group_blocks(g):
            j = jj_of(b)
            self.read(b, gp, None, j * XCDS * 64, (j + 1) * XCDS * 64, tag_p, where)
            self.write(b, lh, xcd(b), 64 * j, 64 * j + 64, tag_h, where)

    def _mlp(self, g: int, take, where: str) -> tuple[int, int]:
        o = self.opts
        t_p1 = take()
        for b in group_blocks(g):
            self.write(b, o.partial_buffers[0], None, (jj_of(b) * XCDS + xcd(b)) * 64,
                       (jj_of(b) * XCDS + xcd(b)) * 64 + 64, t_p1, where + " P2")
        t_h2 = take()
        self._residual(g, o.partial_buffers[0], o.residual_buffers[0], t_p1, t_h2, where + " R1")
        self._gather_all(o.residual_buffers[0], group_blocks(g), t_h2, where + " P3 gather")
        t_g = take()
        for b in group_blocks(g):
            self.write(b, "lg", xcd(b), 20 * jj_of(b), 20 * jj_of(b) + 20, t_g, where + " P3")
        for b in group_blocks(g):
            self.read(b, "lg", xcd(b), 0, 320, t_g, where + " P4 gather")
        t_p2 = take()
        for b in group_blocks(g):
            self.write(b, o.partial_buffers[1], None, (jj_of(b) * XCDS + xcd(b)) * 64,
                       (jj_of(b) * XCDS + xcd(b)) * 64 + 64, t_p2, where + " P4")
        t_h = take()
        self._residual(g, o.partial_buffers[1], o.residual_buffers[1], t_p2, t_h, where + " R2")
        return t_h2, t_h

    def _attention(self, l: int, pos: int, take, where: str) -> None:
        """q/k/v (P1 output), the split statistics, the context (ly or lc)."""
        o = self.opts
        t_qkv, t_st, t_y = take(), take(), take()
        g = l % 2
        for b in group_blocks(g):
            self.write(b, "lq", xcd(b), 16 * jj_of(b), 16 * jj_of(b) + 16, t_qkv, where + " q/k/v")
        single = pos < o.single_below
        for x in range(XCDS):
            blocks = group_blocks(g, x)
            if single:
                for b in blocks[:2]:
                    self.read(b, "lq", x, 0, 256, t_qkv, where + " attention")
                    if jj_of(b) == 0:
                        self.kv_append(b, l, pos)
                    h = jj_of(b)
                    self.write(b, "ly", x, 64 * h, 64 * h + 64, t_y, where + " context")
                for b in blocks:
                    self.read(b, "ly", x, 0, 128, t_y, where + " P2 gather")
                continue
            # the positions each block scores: those of its passes up to and
            # including the current one (whose key and value come from the
            # q/k/v gather, the cached ones from its registers)
            scored = {b: [p for i in range(4) for p in range(64 * (jj_of(b) + 16 * i), 64 * (jj_of(b) + 16 * i) + 64)
                          if p <= pos] for b in blocks}
            if o.empty_split == "cached":
                part = {b: any(p < pos for p in scored[b]) for b in blocks}
            elif o.empty_split == "scored":
                part = {b: bool(scored[b]) for b in blocks}
            else:
                part = {b: True for b in blocks}
            covered = set()
            for b in blocks:
                if not part[b]:
                    continue
                covered.update(scored[b])
                self.read(b, "lq", x, 0, 256, t_qkv, where + " attention")
                if jj_of(b) == 0:
                    self.kv_append(b, l, pos)
            missing = [p for p in range(pos + 1) if p not in covered]
            if missing:
                owners = sorted({jj_of(b) for b in blocks if any(p in scored[b] for p in missing)})
                self.problems.append(f"step {self.step_no} {where}: positions {missing[0]}..{missing[-1]} on XCD {x} "
                                     f"are scored by no block (block(s) jj = {owners} publish an empty share)")
            lone = sum(part.values()) == 1 and o.empty_split != "none"
            for b in blocks:
                self.write(b, "ls", x, 4 * jj_of(b), 4 * jj_of(b) + 4, t_st, where + " statistics")
            for b in blocks:
                if lone and part[b]:
                    continue  # the only block with positions uses its own statistics
                self.read(b, "ls", x, 0, 64, t_st, where + " statistics gather")
            for b in blocks:
                self.write(b, "lc", x, 128 * jj_of(b), 128 * jj_of(b) + 128, t_y, where + " context")
            for b in blocks:
                self.read(b, "lc", x, 0, GROUP_BLOCKS * 128, t_y, where + " P2 gather")

    def _prefetch(self, l: int, pos: int) -> None:
        """Group 0 after layer l - 2: the KV rows [0, pos) of attention layer l
        (plus `prefetch_past` rows beyond them when a mistake is planted)."""
        single = pos < self.opts.single_below
        end = pos + self.opts.prefetch_past
        for b in group_blocks(0):
            j = jj_of(b)
            if single:
                rows = range(end) if j < 2 else range(0)
            else:
                rows = [p for i in range(4) for p in range(64 * (j + 16 * i), 64 * (j + 16 * i) + 64) if p < end]
            self.kv_prefetch(b, l, rows, pos)

    def step(self, pos: int, select: bool, fence_tag: int | None) -> int | None:
        """One decode step at position `pos`; returns the tag of its last h
        when it has no head (the fence of the next step)."""
        take, count = self._tags()
        where0 = f"pos {pos}"
        if fence_tag is not None and self.opts.fence:
            self._gather_all("lh1", group_blocks(0), fence_tag, where0 + " layer-0 fence")
        t_h = None
        for l in range(LAYERS):
            g = l % 2
            where = f"{where0} layer {l}"
            if l > 0:
                self._gather_all(self.opts.residual_buffers[1], group_blocks(g), t_h, where + " P1 gather")
            if l in ATTN_LAYERS:
                self._attention(l, pos, take, where)
            else:
                t_y = take()
                for b in group_blocks(g):
                    self.write(b, "ly", xcd(b), 8 * jj_of(b), 8 * jj_of(b) + 8, t_y, where + " P1")
                for b in group_blocks(g):
                    self.read(b, "ly", xcd(b), 0, 128, t_y, where + " P2 gather")
            _, t_h = self._mlp(g, take, where)
            if l + 2 in ATTN_LAYERS and g == 0:
                self._prefetch(l + 2, pos)
        expect = CONV_EXCHANGES * (LAYERS - len(ATTN_LAYERS)) + ATTN_EXCHANGES * len(ATTN_LAYERS)
        if count() != expect:
            self.problems.append(f"{where0}: {count()} layer exchanges, the kernels advance {expect}")
        if not select:
            self.epoch = (self.epoch + expect) & TAG_MASK
            return t_h
        # the head: every block reads the final h, publishes its candidate;
        # group 0 picks the XCD winner, then the token
        t_c, t_w = take(), take()
        self._gather_all(self.opts.residual_buffers[1], range(BLOCKS), t_h, where0 + " head gather")
        for b in range(BLOCKS):
            self.write(b, "lw", xcd(b), b // XCDS, b // XCDS + 1, t_c, where0 + " head")
        for b in group_blocks(0):
            self.read(b, "lw", xcd(b), 0, 32, t_c, where0 + " pick (XCD)")
            self.write(b, "gw", None, jj_of(b) * XCDS + xcd(b), jj_of(b) * XCDS + xcd(b) + 1, t_w,
                       where0 + " pick (XCD)")
        for b in group_blocks(0):
            self.read(b, "gw", None, jj_of(b) * XCDS, jj_of(b) * XCDS + XCDS, t_w, where0 + " pick")
        if count() - expect != HEAD_EXCHANGES:
            self.problems.append(f"{where0}: {count() - expect} head exchanges, the kernels take {HEAD_EXCHANGES}")
        self.epoch = (self.epoch + expect + self.opts.head_exchanges) & TAG_MASK
        return None

    def _prune(self) -> None:
        live = set()
        for buf in self.bufs.values():
            live.update(int(s) for s in np.unique(buf.writer) if s >= 0)
        for sid in list(self.snaps):
            if sid not in live:
                del self.snaps[sid]

    def run(self, positions, selects) -> list[str]:
        fence = None
        for pos, sel in zip(positions, selects):
            fence = self.step(pos, sel, fence)
            self.step_no += 1
            self._prune()
        return self.problems


def decode_call(first_position: int, n_in: int, n_gen: int):
    """Positions and head flags of the steps of one lfm25_decode call (the
    kernel's loop: n_in + max(n_gen - 1, 0) steps, the last prompt token and
    every generated one select)."""
    steps = n_in + max(n_gen - 1, 0)
    positions = list(range(first_position, first_position + steps))
    selects = [n_gen > 0 and i >= n_in - 1 for i in range(steps)]
    return positions, selects


def check(positions, selects, opts: Options | None = None, max_problems: int = 20) -> list[str]:
    """Problems of the schedule over the given steps (empty when sound)."""
    problems = Checker(opts).run(positions, selects)
    return problems[:max_problems]


def tag_reuse(positions, selects, head_exchanges: int = HEAD_EXCHANGES) -> list[str]:
    """Tag freshness over a long run (thousands of steps, no vector clocks):
    every poll waits for a tag its buffer did not hold before (the zeroed
    workspace holds tag 0), in the kernels' tag order."""
    problems = []
    last: dict[str, int] = {}
    epoch = 0
    for pos, sel in zip(positions, selects):
        k = 0
        uses = []
        for l in range(LAYERS):
            if l in ATTN_LAYERS:
                qkv, st, y = epoch + k + 1, epoch + k + 2, epoch + k + 3
                k += 3
                uses.append(("lq", qkv))
                uses += [("ly", y)] if pos < ATTN_SINGLE_BELOW else [("ls", st), ("lc", y)]
            else:
                k += 1
                uses.append(("ly", epoch + k))
            for name in ("gp0", "lh0", "lg", "gp1", "lh1"):
                k += 1
                uses.append((name, epoch + k))
        if sel:
            uses += [("lw", epoch + k + 1), ("gw", epoch + k + 2)]
        for name, tag in uses:
            tag &= TAG_MASK
            if last.get(name, 0) == tag:
                problems.append(f"pos {pos}: {name} polled for tag {tag}, which it already holds")
            last[name] = tag
        epoch = (epoch + k + (head_exchanges if sel else 0)) & TAG_MASK
    return problems
