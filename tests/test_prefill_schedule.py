"""CPU model of the persistent prefill kernel's schedule
(varlen_prefill_dma_kernel in nano_qwen_amd/csrc/varlen_prefill.hip).

The model restates, step by step, the kernel's wave-uniform state machine:
the work queue (item indices and their description), the K/V copy stream
that runs across items (`issue`: tile of the item being copied, the queued
item started when the current one runs out, empty entries otherwise), the
per-item prologue and tile loop, and each wave's sequence of vector memory
operations (copies, Q loads, output stores).  A change to one must be
mirrored in the other.  For every workgroup of a launch it checks:

- every copied row range stays in bounds: within the sequence's packed keys,
  or within one existing cache block, and every block-table read within the
  table's width;
- a ring slot is only overwritten once every read of the tile it held is
  complete (behind a barrier);
- a tile is only read after the wait and barrier that complete its copies,
  and holds the keys of the item and tile that read it;
- every `s_waitcnt vmcnt(N)` the kernel issues is safe (at least N of the
  wave's memory operations are younger than the awaited copies) and tight
  (exactly N) -- in the waves that only copy, load and store, and safe in
  wave 0, whose work-queue fetch (an atomic) is one more operation;
- the wait for Q (vmcnt(PAD) after the prologue) leaves only the padding
  stores and later operations outstanding, so the Q loads and the fetch
  before them are complete.

Sizes follow the launch shapes built for 16-bit K/V (waves per workgroup,
16-row blocks per wave, ring slots).
"""
import math
import random
from dataclasses import dataclass

import pytest
import torch

from oracle.inputs import make_prefill_case

KKEYS = 32  # keys per tile
NKK, NJ = 4, 8  # head_dim 128: QK operand steps, output column blocks


@dataclass(frozen=True)
class Shape:
    NW: int  # waves per workgroup
    QS: int  # 16-row query blocks per wave
    SLOTS: int  # K/V ring slots
    WG_PER_CU: int

    @property
    def AHEAD(self):
        return self.SLOTS - 1

    @property
    def COPS(self):
        return (KKEYS // self.NW) // 4

    @property
    def QOPS(self):
        return self.QS * NKK

    @property
    def SOPS(self):
        return self.QS * NJ // 2

    @property
    def PAD(self):  # stores that write nothing, after the Q loads
        return 2 * self.COPS * self.AHEAD

    @property
    def EOPS(self):
        return self.QOPS + self.SOPS + self.PAD

    @property
    def RING_BYTES(self):  # K and V tiles of 32 keys, 2 bytes x head_dim 128
        return self.SLOTS * 2 * KKEYS * 2 * 128

    @property
    def MAX_ITEMS(self):  # queue items listed in what the CU's LDS has left (PShape::MAX_ITEMS)
        fixed = self.RING_BYTES + 32 + 4 * QUEUE_LEVELS + 8 * (MAX_SEQS + 1)
        free = (160 * 1024 // self.WG_PER_CU - fixed) // 4
        return 4096 if free > 4096 else free & ~63


SHAPES = {"a": Shape(8, 2, 5, 1), "c": Shape(4, 2, 4, 2)}


QUEUE_LEVELS, MAX_SEQS = 16, 1024  # kQueueLevels, kMaxSeqs


class Launch:
    """Host-side launch parameters (launch_prefill_dma) and the item map."""

    def __init__(self, S, lq, lk, bt, num_blocks, bs, hkv, hq, causal=True, cus=256, by_cost=None):
        self.S, self.lq, self.lk, self.bt = S, lq, lk, bt
        self.num_blocks, self.bs, self.hkv, self.hq, self.causal = num_blocks, bs, hkv, hq, causal
        G = hq // hkv
        self.G4 = G if G < 4 else 4
        self.quads = 1 if G < 4 else G // 4
        self.G = G
        self.rows = 16 * S.QS * (S.NW // self.G4)  # query rows per item
        self.n_x = math.ceil(max(lq) / self.rows)
        self.n_y = hkv * self.quads
        self.U = self.n_y * len(lq)
        self.pin = self.U >= 8
        total = 8 * ((self.U + 7) // 8) * self.n_x if self.pin else self.U * self.n_x
        self.grid = min((cus * S.WG_PER_CU + 7) // 8 * 8, total)
        self.cu_q, self.cu_k = [0], [0]
        for a, b in zip(lq, lk):
            self.cu_q.append(self.cu_q[-1] + a)
            self.cu_k.append(self.cu_k[-1] + b)
        self.max_blocks = bt.shape[1] if bt is not None else 0
        n = len(lq)
        self.by_cost = (n <= MAX_SEQS and n * self.n_x <= 65536) if by_cost is None else by_cost
        nkt_max = (max(lk) + KKEYS - 1) // KKEYS
        self.level_shift = 0
        while (nkt_max >> self.level_shift) + 1 > QUEUE_LEVELS:
            self.level_shift += 1
        self.n_levels = (nkt_max >> self.level_shift) + 1
        self.ystep = 8 if self.pin else 1
        cx_max = (self.U + 7) // 8 if self.pin else self.U
        # launch_prefill_dma: each queue's items listed in LDS at launch (by_cost == 2)
        self.use_table = bool(self.by_cost and cx_max * self.n_x <= S.MAX_ITEMS
                              and n * self.n_levels * 4 <= S.RING_BYTES and self.n_y <= 256 and self.n_x <= 16384)
        self.lev = {}  # queue x -> level starts (what each workgroup builds in LDS)
        self.n_live = {}
        if self.by_cost:
            for x in range(8 if self.pin else 1):
                cnt = [0] * self.n_levels
                for sq in range(n):
                    w = self.n_slots(self.first_slot(x, sq))
                    for qt in range(self.n_x):
                        if qt * self.rows < lq[sq] and w > 0:
                            cnt[self.cost_level(qt, lq[sq], lk[sq])] += w
                start, carry = [0] * self.n_levels, 0
                for L in range(self.n_levels - 1, -1, -1):
                    start[L] = carry
                    carry += cnt[L]
                self.lev[x], self.n_live[x] = start, carry

    # ---- helpers of the cost order (first_slot, n_slots, first_tile_with, cost_level)
    def first_slot(self, x, s):
        return ((x - s * self.n_y) & 7) if self.ystep == 8 else 0

    def n_slots(self, y0):
        return (self.n_y - 1 - y0) // self.ystep + 1 if y0 < self.n_y else 0

    def first_tile_with(self, v, nq, Lk, P):
        if v <= 0:
            return 0
        if not self.causal:
            return 0 if (Lk + KKEYS - 1) // KKEYS >= v else nq
        t = KKEYS * (v - 1)
        if Lk <= t:
            return nq
        need = t - P
        return 0 if need < 0 else min(need // self.rows, nq)

    def key_end(self, qt, Lq, Lk):
        row_last = min((qt + 1) * self.rows, Lq) - 1
        return max(0, min(Lk, row_last + Lk - Lq + 1)) if self.causal else Lk

    def cost_level(self, qt, Lq, Lk):
        nkt = (self.key_end(qt, Lq, Lk) + KKEYS - 1) // KKEYS
        return min(nkt >> self.level_shift, self.n_levels - 1)

    def queue_of(self, wg):
        x = wg & 7 if self.pin else 0
        cx = (self.U - x + 7) >> 3 if self.pin else self.U
        return x, cx, (self.n_live[x] if self.by_cost else cx * self.n_x)

    def item(self, idx, s, y, qt):
        Lq, Lk = self.lq[s], self.lk[s]
        if qt * self.rows >= Lq:
            return None
        key_end = self.key_end(qt, Lq, Lk)
        return dict(idx=idx, s=s, y=y, qt=qt, kvh=y // self.quads, key_end=key_end,
                    n_kt=(key_end + KKEYS - 1) // KKEYS)

    def table(self, x):
        """The list of queue x's items the kernel builds in LDS at launch: the
        first queue index of each (level, sequence), a level's sequences in
        order, then each live (sequence, query tile) placing its items (one
        per kv-head slot) by slot, then query tile from the last down."""
        start, n = self.lev[x], len(self.lq)
        first = {}
        for L in range(self.n_levels):
            carry = start[L]
            for s in range(n):
                Lq, Lk = self.lq[s], self.lk[s]
                nq = (Lq + self.rows - 1) // self.rows if Lq > 0 else 0
                qlo = self.first_tile_with(L << self.level_shift, nq, Lk, Lk - Lq)
                qhi = nq if L == self.n_levels - 1 else self.first_tile_with((L + 1) << self.level_shift, nq, Lk, Lk - Lq)
                first[L, s] = carry
                carry += max(0, qhi - qlo) * self.n_slots(self.first_slot(x, s))
        tab = [None] * self.n_live[x]
        for s in range(n):
            Lq, Lk = self.lq[s], self.lk[s]
            y0 = self.first_slot(x, s)
            w = self.n_slots(y0)
            for qt in range(self.n_x):
                if qt * self.rows < Lq and w > 0:
                    L = self.cost_level(qt, Lq, Lk)
                    nq = (Lq + self.rows - 1) // self.rows
                    qlo = self.first_tile_with(L << self.level_shift, nq, Lk, Lk - Lq)
                    qhi = nq if L == self.n_levels - 1 else self.first_tile_with((L + 1) << self.level_shift, nq,
                                                                                   Lk, Lk - Lq)
                    for yi in range(w):
                        pos = first[L, s] + yi * (qhi - qlo) + (qhi - 1 - qt)
                        assert tab[pos] is None, "two items at one place"
                        tab[pos] = (s << 22) | ((y0 + self.ystep * yi) << 14) | qt
        return tab

    def describe(self, idx, x, cx, n_items):
        """Item idx of queue x (describe_by_cost / describe_by_tile): None when not live."""
        if idx >= n_items:
            return None
        if not self.by_cost:
            qt = self.n_x - 1 - idx // cx
            u = x + 8 * (idx % cx) if self.pin else idx % cx
            return self.item(idx, u // self.n_y, u % self.n_y, qt)
        start = self.lev[x]
        L = min(l for l in range(self.n_levels) if start[l] <= idx)  # the level search
        r = idx - start[L]
        lo_v = L << self.level_shift
        hi_v = (L + 1) << self.level_shift
        for s in range(len(self.lq)):  # 64 sequences per step in the kernel; one by one here
            Lq, Lk = self.lq[s], self.lk[s]
            nq = (Lq + self.rows - 1) // self.rows if Lq > 0 else 0
            qlo = self.first_tile_with(lo_v, nq, Lk, Lk - Lq)
            qhi = nq if L == self.n_levels - 1 else self.first_tile_with(hi_v, nq, Lk, Lk - Lq)
            n_t = max(0, qhi - qlo)
            y0 = self.first_slot(x, s)
            cnt = n_t * self.n_slots(y0)
            if r < cnt:
                return self.item(idx, s, y0 + self.ystep * (r // n_t), qlo + n_t - 1 - r % n_t)
            r -= cnt
        raise AssertionError("queue index past the live items")


class Workgroup:
    """One workgroup's run over the item indices it fetched, in order."""

    def __init__(self, L, indices, x, cx, n_items, wave0=False):
        self.L, self.S = L, L.S
        self.wave0 = wave0  # the wave whose lane 0 runs the work-queue fetch
        self.x, self.cx, self.n_items = x, cx, n_items
        self.indices = indices
        self.ops = []  # one wave's vector memory operations, in issue order
        self.copied = {}  # stream index -> (item idx or None, tile, first row, rows)
        self.last_op = {}  # stream index -> position of its last operation in `ops`
        self.landed = -1  # stream entries up to this one completed (behind a barrier)
        self.pending_reads = set()  # stream indices read since the last barrier
        self.done_reads = set()  # stream indices all of whose reads completed
        self.pos = 0
        self.rem = self.left = self.bidx = self.blk_next = 0
        self.run_left = self.nrows = 0
        self.run_item = None
        self.off = 0
        self.seq = None
        self.item_idx = None
        self.jt = 0
        self.nx = None
        self.nx_first = 0
        self.any_bad = False
        self.waits = 0

    # ---------------------------------------------------------------- stream
    def entry(self, s, b):
        assert b >= 0
        if b >= self.L.max_blocks:
            return -1
        return int(self.L.bt[s, b])

    def next_run(self):
        """next_run: the next run of entries sharing a descriptor shape."""
        L = self.L
        paged = L.bt is not None
        if self.rem <= 0 and self.nx is not None:  # start the queued item
            it, self.nx = self.nx, None
            self.rem = it["key_end"]
            self.key_end = it["key_end"]
            self.seq = it["s"]
            self.item_idx = it["idx"]
            self.jt = 0
            self.off = 0 if paged else L.cu_k[it["s"]]
            self.blk_next = it["blk0"]
            self.bidx = 0
            self.left = 0 if paged else 1 << 30
            self.nx_first = self.pos
        if self.rem <= 0:  # one empty entry
            self.nrows, self.run_left, self.run_item = 0, 1, None
            return
        ok = True
        if self.left == 0:  # entering the next block
            blk = self.blk_next
            self.blk_next = self.entry(self.seq, self.bidx + 1)
            self.bidx += 1
            ok = 0 <= blk < L.num_blocks
            self.any_bad |= not ok
            self.off = (blk if ok else 0) * L.bs
            self.left = L.bs // KKEYS
        elif paged:
            ok = self.nrows != 0
        full = min(self.left, self.rem // KKEYS)
        self.run_item = self.item_idx
        if full > 0:
            self.run_left, self.left, self.rem = full, self.left - full, self.rem - full * KKEYS
            self.nrows = KKEYS if ok else 0
        else:  # the partial last tile
            self.run_left, self.left = 1, self.left - 1
            self.nrows = self.rem if ok else 0
            self.rem = 0

    def issue(self):
        L, S = self.L, self.S
        paged = L.bt is not None
        if self.run_left == 0:
            self.next_run()
        # the ring slot of this entry held entry pos - SLOTS: its reads are done
        old = self.pos - S.SLOTS
        if old >= 0 and self.copied[old][0] is not None:  # every tile of an item is read
            assert old in self.done_reads, f"slot of stream entry {old} overwritten before its reads completed"
        rows = self.nrows
        if rows:
            lo, hi = self.off, self.off + rows
            if paged:
                assert 0 <= lo and hi <= L.num_blocks * L.bs
                assert lo // L.bs == (hi - 1) // L.bs, "a tile crosses a cache block"
            else:
                assert L.cu_k[self.seq] <= lo and hi <= L.cu_k[self.seq + 1]
        if self.run_item is not None:
            # a tile copies its valid keys (all of them, or none in a missing block)
            assert rows in (0, min(KKEYS, self.key_end - self.jt * KKEYS)), (rows, self.jt, self.key_end)
            self.copied[self.pos] = (self.run_item, self.jt, self.off, rows)
            self.jt += 1
        else:
            self.copied[self.pos] = (None, None, 0, 0)
        self.ops += [("c", self.pos)] * (2 * S.COPS)
        self.last_op[self.pos] = len(self.ops) - 1
        self.off += KKEYS
        self.run_left -= 1
        self.pos += 1

    # ------------------------------------------------------------ checks
    def wait(self, p, n):
        """s_waitcnt vmcnt(n) meant to complete stream entry p, then a barrier."""
        last = self.last_op[p]
        younger = len(self.ops) - 1 - last
        assert n <= younger, f"vmcnt({n}) with only {younger} younger operations: entry {p} may be in flight"
        fetches = sum(1 for op in self.ops[last + 1:] if op[0] == "a") if self.wave0 else 0
        assert n == younger - fetches, f"vmcnt({n}) stricter than needed ({younger} younger operations)"
        assert n < 64
        self.waits += 1
        self.barrier()
        # vmcnt completes in order, and entries are issued in stream order
        self.landed = max(self.landed, p)

    def barrier(self):
        self.done_reads |= self.pending_reads
        self.pending_reads = set()

    def queue_copy(self, it):
        """queue_copy: the item the stream starts when the current one runs
        out (None: nothing queued), with its first block-table entry read now."""
        if it is None or it["n_kt"] == 0:
            self.nx = None
            return
        self.nx = dict(it, blk0=self.entry(it["s"], 0) if self.L.bt is not None else 0)

    def fetch(self):
        if self.wave0:
            self.ops.append(("a",))
            self.fetch_at = len(self.ops) - 1

    def wait_q(self):
        """wait_vmcnt<PAD> after the prologue barrier: at most PAD operations
        outstanding, so everything before the padding -- the Q loads and the
        fetch -- is complete."""
        n = self.S.PAD
        last_q = max(i for i, op in enumerate(self.ops) if op[0] == "q")
        assert all(op[0] == "p" for op in self.ops[last_q + 1:last_q + 1 + n]), "padding follows the Q loads"
        assert len(self.ops) - 1 - last_q >= n, "fewer than PAD operations after the Q loads"
        if self.wave0:
            assert self.fetch_at < last_q, "the fetch precedes the Q loads"

    def read(self, p, item, jt):
        assert p <= self.landed, f"stream entry {p} read before its copies completed"
        assert self.copied[p][:2] == (item, jt), f"entry {p} holds {self.copied[p][:2]}, read as {(item, jt)}"
        self.pending_reads.add(p)

    # ------------------------------------------------------------ kernel
    def run(self):
        L, S = self.L, self.S
        idx = list(self.indices)
        idx_cur, idx_nxt = idx[0], idx[1]
        nxt_fetch = 2
        desc = lambda i: L.describe(i, self.x, self.cx, self.n_items)
        cur, nxt, prev = desc(idx_cur), desc(idx_nxt), None
        self.queue_copy(cur)
        items = 0
        while True:
            epi_pos = -1
            if prev is not None:  # the previous item's output
                self.ops += [("s",)] * S.SOPS
                epi_pos = self.pos
            if idx_cur >= self.n_items:
                break
            self.fetch()
            self.ops += [("q",)] * S.QOPS  # this item's Q
            self.ops += [("p",)] * S.PAD  # padding
            if cur is not None:
                items += 1
                p0 = self.pos
                if cur["n_kt"] > 0:
                    if self.nx is not None:
                        self.issue()
                    p0 = self.nx_first
                self.queue_copy(nxt)
                while self.pos < p0 + S.AHEAD:
                    self.issue()
                assert self.pos == p0 + S.AHEAD
                n_kt = cur["n_kt"]
                self.wait(p0, 2 * S.COPS * (S.AHEAD - 1) + (S.EOPS if p0 < epi_pos else 0))
                self.wait_q()
                if n_kt > 0:
                    self.read(p0, idx_cur, 0)  # K of tile 0
                for jt in range(n_kt):
                    assert self.pos == p0 + S.AHEAD + jt
                    t = p0 + jt + 1
                    self.wait(t, 2 * S.COPS * (S.AHEAD - 2) + (S.EOPS if t < epi_pos else 0))
                    self.issue()
                    if jt + 1 < n_kt:
                        self.read(t, idx_cur, jt + 1)  # K of the next tile
                    self.read(p0 + jt, idx_cur, jt)  # V of this tile
            else:
                self.queue_copy(nxt)
            self.barrier()  # end of item
            idx_new = idx[nxt_fetch]
            nxt_fetch += 1
            prev, cur, nxt = cur, nxt, desc(idx_new)
            idx_cur, idx_nxt = idx_nxt, idx_new
        return items


def split_queue(L, seed):
    """Item indices each workgroup fetches: queue x's counter hands out
    0, 1, 2, ... to its workgroups in an arbitrary interleaving."""
    rng = random.Random(seed)
    per_wg = {}
    queues = {}
    for wg in range(L.grid):
        x, cx, n = L.queue_of(wg)
        queues.setdefault(x, (cx, n, []))[2].append(wg)
    for x, (cx, n, wgs) in queues.items():
        lists = {wg: [] for wg in wgs}
        active = list(wgs)
        i = 0
        while active:  # a workgroup fetches until it has two indices past the end
            wg = rng.choice(active)
            lists[wg].append(i)
            i += 1
            if sum(v >= n for v in lists[wg]) >= 2:
                active.remove(wg)
        for wg in wgs:
            per_wg[wg] = (x, cx, n, lists[wg])
    return per_wg


def run_launch(S, lq, lk, bt, num_blocks, bs, hkv, hq, seed=0, causal=True, cus=256, by_cost=None):
    L = Launch(S, lq, lk, bt, num_blocks, bs, hkv, hq, causal=causal, cus=cus, by_cost=by_cost)
    n_items = 0
    tiles = 0
    for wg, (x, cx, n, indices) in split_queue(L, seed).items():
        w = Workgroup(L, indices, x, cx, n)
        n_items += w.run()
        tiles += sum(1 for v in w.copied.values() if v[0] is not None)
        Workgroup(L, indices, x, cx, n, wave0=True).run()
    # every live item ran exactly once over the launch
    live = 0
    for wg in range(min(L.grid, 8 if L.pin else 1)):
        x, cx, n = L.queue_of(wg)
        live += sum(L.describe(i, x, cx, n) is not None for i in range(n))
    assert n_items == live
    return n_items, tiles


CASES = [dict(nseq=5, lq=(1, 400), prefix_blocks=(0, 0)), dict(nseq=4, lq=(1, 700), prefix_blocks=(1, 3)),
         dict(nseq=16), dict(nseq=3, lq=(20, 300), prefix_blocks=(1, 1), hq=16, hkv=1),
         dict(nseq=3, lq=(20, 300), prefix_blocks=(1, 1), hq=4, hkv=4)]


@pytest.mark.parametrize("by_cost", [True, False])
@pytest.mark.parametrize("shape", sorted(SHAPES))
@pytest.mark.parametrize("kw", CASES)
def test_schedule(shape, kw, by_cost):
    c = make_prefill_case("cfg3", seed=0, device="cpu", **kw)
    items, tiles = run_launch(SHAPES[shape], c["lq"], c["lk"], c["block_tables"], c["num_blocks"],
                              c["block_size"], c["hkv"], c["hq"], seed=1, cus=16, by_cost=by_cost)
    assert items > 0 and tiles > 0


@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_schedule_edges_and_missing_block(shape):
    S = SHAPES[shape]
    lens = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129]
    run_launch(S, lens, lens, None, 0, 256, 8, 32, cus=4)
    run_launch(S, lens, lens, None, 0, 256, 8, 32, causal=False, cus=4)
    run_launch(S, [5, 40], [0, 40], None, 0, 256, 1, 2, cus=1)  # a sequence without keys
    pre, lq = [37, 0, 300], [60, 200, 150]
    lk = [p + q for p, q in zip(pre, lq)]
    W = max((x + 255) // 256 for x in lk)
    bt = torch.full((3, W), -1, dtype=torch.int32)
    perm = torch.randperm(20, generator=torch.Generator().manual_seed(2))
    off = 0
    for i in range(3):
        k = (lk[i] + 255) // 256
        bt[i, :k] = perm[off:off + k]
        off += k
    run_launch(S, lq, lk, bt, 20, 256, 8, 32, cus=2)
    bt[2, 0] = -1  # a missing block: its tiles read as zeros, nothing is copied from it
    run_launch(S, lq, lk, bt, 20, 256, 8, 32, cus=2)


def test_model_catches_a_loose_wait():
    """The checker itself: counting the previous item's epilogue among the
    younger operations where it is not (a wait the kernel must not issue)
    is reported as unsafe."""
    S = SHAPES["c"]
    lens = [300, 300]
    L = Launch(S, lens, lens, None, 0, 256, 1, 4, cus=1)
    x, cx, n, indices = max(split_queue(L, 0).values(), key=lambda v: sum(i < v[2] for i in v[3]))

    class AlwaysEpilogue(Workgroup):
        def wait(self, p, n_):
            if n_ < S.EOPS:
                n_ += S.EOPS
            return super().wait(p, n_)

    Workgroup(L, indices, x, cx, n).run()
    with pytest.raises(AssertionError, match="in flight"):
        AlwaysEpilogue(L, indices, x, cx, n).run()


def cost_order_cases():
    yield dict(lq=[1124, 2023, 1379, 743, 1067, 545, 1602, 1950], lk=[1380, 2023, 2147, 743, 1835, 545, 2626, 1950],
               hkv=8, hq=32)
    yield dict(lq=[1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129], lk=[1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129],
               hkv=8, hq=32)
    yield dict(lq=[5, 40, 300], lk=[0, 40, 900], hkv=1, hq=2)  # a sequence without keys; GQA 2
    yield dict(lq=[20, 300, 77], lk=[276, 300, 77], hkv=1, hq=16)  # 4 head quads
    yield dict(lq=[20, 300], lk=[20, 300], hkv=4, hq=4)  # MHA: 128-row items
    yield dict(lq=[3000, 10], lk=[40000, 10], hkv=2, hq=8)  # levels coarsened past QUEUE_LEVELS


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_cost_order_covers_live_items_longest_first(shape, causal):
    """The cost-ordered queue lists every live item of its XCD exactly once,
    by non-increasing cost level, then sequence, kv-head slot and query tile
    from the last down;
    the arithmetic select matches a plain sort of the live items."""
    for c in cost_order_cases():
        L = Launch(SHAPES[shape], c["lq"], c["lk"], None, 0, 256, c["hkv"], c["hq"], causal=causal, cus=1,
                   by_cost=True)
        for x in range(8 if L.pin else 1):
            _, cx, n = L.queue_of(x)
            got = [L.describe(i, x, cx, n) for i in range(n)]
            assert all(it is not None for it in got)
            keys = [(-L.cost_level(it["qt"], L.lq[it["s"]], L.lk[it["s"]]), it["s"], it["y"], -it["qt"]) for it in got]
            live = sorted((-L.cost_level(qt, L.lq[s_], L.lk[s_]), s_, y, -qt)
                          for s_ in range(len(L.lq)) for y in range(L.n_y) for qt in range(L.n_x)
                          if qt * L.rows < L.lq[s_] and (not L.pin or (s_ * L.n_y + y) % 8 == x))
            assert keys == live
        assert L.level_shift == 0 or L.n_levels <= QUEUE_LEVELS


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_item_list_matches_cost_order(shape, causal):
    """The list of each queue's items built at launch (describe_by_table)
    holds, at every index, the item describe_by_cost derives there, each
    field within its bits of the packed word."""
    for c in cost_order_cases():
        L = Launch(SHAPES[shape], c["lq"], c["lk"], None, 0, 256, c["hkv"], c["hq"], causal=causal, cus=1,
                   by_cost=True)
        for x in range(8 if L.pin else 1):
            _, cx, n = L.queue_of(x)
            tab = L.table(x)
            assert len(tab) == n and all(e is not None for e in tab)
            for i, e in enumerate(tab):
                it = L.describe(i, x, cx, n)
                assert (e >> 22, (e >> 14) & 255, e & 16383) == (it["s"], it["y"], it["qt"])


def test_item_list_chosen_for_the_bench_shapes():
    """launch_prefill_dma lists the items at launch for cfg3's and cfg3_long's
    batches (every queue's bound fits the LDS left by the ring), and falls
    back to deriving them when a queue could outgrow the list."""
    S = SHAPES["c"]
    c = make_prefill_case("cfg3", seed=0, device="cpu")
    assert Launch(S, c["lq"], c["lk"], None, 0, 256, c["hkv"], c["hq"]).use_table
    assert Launch(S, [8192] * 4, [8192] * 4, None, 0, 256, 8, 32).use_table
    assert not Launch(S, [8192] * 64, [8192] * 64, None, 0, 256, 8, 32).use_table
