"""CPU model of the prefill kernel's K/V copy schedule (prefill_item's
`issue` in nano_qwen_amd/csrc/varlen_prefill.hip): every block-table read and
every copied row range stays in bounds -- within the sequence's packed keys,
or within one existing cache block -- for the shapes the GPU tests use.

The model restates the kernel's scalar state machine step by step (tile
index, block-table index, tiles left in the block, the entry fetched one
block ahead); a change to one must be mirrored in the other.  It guards the
class of bug where the packed (table-less) path touched the block table.
"""
import math

import pytest
import torch

from oracle.inputs import make_prefill_case

KKEYS, KAHEAD, KROWS, KNW = 32, 4, 32, 8  # kKeys, kAhead, kRows, kNW


def copy_schedule(lq, lk, bt, num_blocks, bs, hkv, hq, causal=True):
    """Yield (seq, first_row, rows) of every copy the kernel issues."""
    G = hq // hkv
    G4 = G if G < 4 else 4
    rb = KNW // G4
    n_x = math.ceil(max(lq) / (KROWS * rb))
    paged = bt is not None
    max_blocks = bt.shape[1] if paged else 0
    cu_k = [0]
    for x in lk:
        cu_k.append(cu_k[-1] + x)
    for s in range(len(lq)):
        Lq, Lk = lq[s], lk[s]
        P, k0 = Lk - Lq, cu_k[s]
        for qt in range(n_x):
            row_begin = qt * KROWS * rb
            if row_begin >= Lq:
                continue
            row_last = min(row_begin + KROWS * rb, Lq) - 1
            key_end = max(0, min(Lk, row_last + P + 1)) if causal else Lk
            n_kt = (key_end + KKEYS - 1) // KKEYS

            def entry(b):
                return int(bt[s, b]) if b < max_blocks else -1

            jt, left, bidx, ok = 0, 0, 0, True
            off = 0 if paged else k0
            blk_next = entry(0) if paged else 0
            for _ in range(n_kt + KAHEAD):  # kAhead in the prologue, then one per tile
                rows = 0
                if jt < n_kt:
                    if paged and left == 0:
                        blk, blk_next = blk_next, entry(bidx + 1)
                        bidx += 1
                        ok = 0 <= blk < num_blocks
                        off = (blk if ok else 0) * bs
                        left = bs // KKEYS
                    nvalid = min(KKEYS, key_end - jt * KKEYS)
                    assert nvalid >= 1
                    rows = nvalid if ok else 0
                if rows:
                    yield s, off, rows
                off += KKEYS
                if paged:
                    left -= 1
                jt += 1


def assert_in_bounds(lq, lk, bt, num_blocks, bs, hkv, hq):
    total_k = sum(lk)
    cu_k = [0]
    for x in lk:
        cu_k.append(cu_k[-1] + x)
    n = 0
    for s, lo, rows in copy_schedule(lq, lk, bt, num_blocks, bs, hkv, hq):
        hi = lo + rows
        if bt is not None:
            assert 0 <= lo and hi <= num_blocks * bs
            assert lo // bs == (hi - 1) // bs, "a tile crosses a cache block"
        else:
            assert cu_k[s] <= lo and hi <= cu_k[s + 1] <= total_k
        n += 1
    return n


CASES = [dict(nseq=5, lq=(1, 400), prefix_blocks=(0, 0)), dict(nseq=4, lq=(1, 700), prefix_blocks=(1, 3)),
         dict(nseq=16), dict(nseq=3, lq=(20, 300), prefix_blocks=(1, 1), hq=16, hkv=1),
         dict(nseq=3, lq=(20, 300), prefix_blocks=(1, 1), hq=4, hkv=4)]


@pytest.mark.parametrize("kw", CASES)
@pytest.mark.parametrize("seed", [0, 1])
def test_copy_schedule_in_bounds(kw, seed):
    c = make_prefill_case("cfg3", seed=seed, device="cpu", **kw)
    assert assert_in_bounds(c["lq"], c["lk"], c["block_tables"], c["num_blocks"], c["block_size"], c["hkv"],
                            c["hq"]) > 0


def test_copy_schedule_edges_and_missing_block():
    lens = [1, 2, 63, 64, 65, 127, 128, 129]
    assert_in_bounds(lens, lens, None, 0, 256, 8, 32)
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
    assert_in_bounds(lq, lk, bt, 20, 256, 8, 32)
    full = [c for c in copy_schedule(lq, lk, bt, 20, 256, 8, 32) if c[0] == 2]
    first = int(bt[2, 0])
    bt[2, 0] = -1  # a missing block: its tiles are not copied (they read as zeros)
    holed = [c for c in copy_schedule(lq, lk, bt, 20, 256, 8, 32) if c[0] == 2]
    assert_in_bounds(lq, lk, bt, 20, 256, 8, 32)
    assert len(holed) < len(full)
    assert all(lo // 256 != first for _, lo, _ in holed)
