"""CPU model of the stream-K decode schedule (csrc/paged_decode.hip).

The decode kernel's multi-split path lays the batch's contexts end to end
and gives workgroup w of the W ranges in use the tokens [B(w), B(w + 1)),
where B(w) is token floor(w * T / W) rounded down to a multiple of 32 within
its sequence (paged_decode_sk_kernel / sk_boundary); W is at least one range
per CU, keeps ranges at 2048 tokens or more where the batch has them and
each within 61 blocks, and the grid's other workgroups record an empty range.  A sequence inside one range is
written whole; a workgroup writes at most two partial pieces (slot 0: the
sequence began in an earlier range, slot 1: it continues into a later one);
decode_merge_sk_kernel finds a sequence's pieces by searching the recorded
range starts.  This module restates those integer rules and checks, for
random and edge-case batches, that every token is computed exactly once,
that no slot is written twice, that the merge collects exactly the partial
pieces of each sequence with their slots, and that no range spans more than
the 63 block-table entries a wave holds.
"""
import random

import pytest


MIN_PIECE = 2048


def ranges_in_use(total, grid_w, w_min, block_size):
    """W of paged_decode_sk_kernel: at least w_min ranges, none shorter than
    MIN_PIECE tokens where the batch has them, enough to keep each within 61
    blocks, at most the grid."""
    return min(grid_w, max(w_min, max(total // MIN_PIECE, -(-total // (61 * block_size)))))


def boundaries(ctx, grid_w, w_min=1, block_size=256):
    """Recorded range starts B(0..grid_w) as (sequence, token); workgroups
    past the ranges in use record (len(ctx), 0), as does the end."""
    total = sum(ctx)
    W = ranges_in_use(total, grid_w, w_min, block_size)
    starts = [0]
    for c in ctx:
        starts.append(starts[-1] + c)
    out = []
    for w in range(grid_w):
        if w >= W:
            out.append((len(ctx), 0))
            continue
        g = w * total // W
        b = next(i for i in range(len(ctx)) if starts[i + 1] > g)
        out.append((b, (g - starts[b]) & ~31))
    out.append((len(ctx), 0))
    return out


def kernel_pieces(ctx, W, w_min=1, block_size=256):
    """The pieces each workgroup computes, as the kernel's loop enumerates them."""
    bnd = boundaries(ctx, W, w_min, block_size)
    pieces = []  # (w, b, t0, t1, complete, slot)
    for w in range(W):
        lo, hi = bnd[w], bnd[w + 1]
        b = lo[0]
        while b < len(ctx) and (b < hi[0] or (b == hi[0] and hi[1] > 0)):
            t0 = lo[1] if b == lo[0] else 0
            t1 = hi[1] if b == hi[0] else ctx[b]
            if t1 > t0:
                complete = t0 == 0 and t1 == ctx[b]
                pieces.append((w, b, t0, t1, complete, None if complete else (0 if t0 > 0 else 1)))
            b += 1
    return pieces, bnd


def merge_rows(ctx, bnd, b):
    """(w, slot) rows decode_merge_sk_kernel reads for sequence b, or None
    when the sequence was written whole."""
    W = len(bnd) - 1

    def last_le(t):
        lo, hi = 0, W - 1
        while lo < hi:
            mid = (lo + hi + 1) >> 1
            s = bnd[mid]
            if s[0] < b or (s[0] == b and s[1] <= t):
                lo = mid
            else:
                hi = mid - 1
        return lo

    ws, we = last_le(0), last_le(ctx[b] - 1)
    if ws == we:
        return None
    rows = []
    for w in range(ws, we + 1):
        if w + 1 < W and bnd[w] == bnd[w + 1]:
            continue
        rows.append((w, 1 if w == ws else 0))
    return rows


def sk_workgroups(cus, occ, groups, batch, max_tokens, block_size):
    """Host rule (sk_workgroups): every resident slot, and enough ranges that
    none exceeds 61 blocks."""
    W = max(1, cus * occ // groups)
    W = max(W, (batch * max_tokens + 61 * block_size - 1) // (61 * block_size))
    return min(W, 65535)


def sk_eligible(batch, max_tokens, block_size):
    """Host rule (sk_eligible): stream-K only where 65535 ranges of at most 61
    blocks cover batch x max_tokens; split-K otherwise."""
    total = batch * max_tokens
    return batch <= 4096 and total < 2 ** 31 and -(-total // (61 * block_size)) <= 65535


def check(ctx, W, block_size=256, w_min=1):
    pieces, bnd = kernel_pieces(ctx, W, w_min, block_size)
    # every token of every sequence exactly once
    cover = {b: [] for b in range(len(ctx))}
    for w, b, t0, t1, complete, slot in pieces:
        assert t0 % 32 == 0 and 0 <= t0 < t1 <= ctx[b]
        cover[b].append((t0, t1))
        n_blk = (t1 - 1) // block_size - t0 // block_size + 1
        assert n_blk <= 63, (w, b, t0, t1)
    for b, segs in cover.items():
        segs.sort()
        pos = 0
        for t0, t1 in segs:
            assert t0 == pos, (b, segs)
            pos = t1
        assert pos == ctx[b], (b, segs, ctx[b])
    # at most one piece per (workgroup, slot)
    used = {}
    for w, b, t0, t1, complete, slot in pieces:
        if slot is not None:
            assert (w, slot) not in used, (w, slot)
            used[(w, slot)] = b
    # the merge reads exactly the partial pieces of each sequence
    for b in range(len(ctx)):
        if ctx[b] == 0:
            continue
        rows = merge_rows(ctx, bnd, b)
        mine = [(w, slot) for w, bb, t0, t1, complete, slot in pieces if bb == b]
        complete = [p for p in pieces if p[1] == b and p[4]]
        if rows is None:
            assert len(complete) == 1 and len(mine) == 1, (b, mine)
        else:
            assert not complete
            assert sorted(rows) == sorted(mine), (b, rows, mine)
            assert all(used[r] == b for r in rows)


@pytest.mark.parametrize("seed", range(40))
def test_random_batches(seed):
    rng = random.Random(seed)
    B = rng.choice([1, 2, 3, 7, 64, 128, 300])
    hi = rng.choice([1, 40, 600, 4096, 8192, 32768])
    ctx = [rng.randint(0, hi) for _ in range(B)]
    if rng.random() < 0.3:  # padded graph rows
        for i in rng.sample(range(B), k=max(1, B // 4)):
            ctx[i] = 0
    if sum(ctx) == 0:
        ctx[0] = 1
    groups = rng.choice([1, 2])
    W = sk_workgroups(256, rng.choice([1, 2, 3]), groups, B, max(ctx), 256)
    check(ctx, W, w_min=max(1, 256 // groups))
    check(ctx, W, w_min=1)


def test_bench_shapes():
    rng = random.Random(0)
    cfg5 = [rng.randint(2048, 8192) for _ in range(128)]
    check(cfg5, sk_workgroups(256, 1, 1, 128, 8192, 256), w_min=256)
    cfg2 = [rng.randint(1024, 4096) for _ in range(64)]
    check(cfg2, sk_workgroups(256, 2, 2, 64, 4096, 256), w_min=128)
    check([32768] * 8, sk_workgroups(256, 2, 2, 8, 32768, 256), w_min=128)
    # ranges in use: cfg5 one per slot (its ranges exceed 2048 tokens), cfg4
    # 2048-token ranges, cfg2 one per CU
    assert ranges_in_use(sum(cfg5), 256, 256, 256) == 256
    assert ranges_in_use(8 * 32768, 256, 128, 256) == 128
    assert ranges_in_use(sum(cfg2), 256, 128, 256) == 128


def test_edge_cases():
    check([1], 256)              # one token, 255 empty ranges
    check([31, 0, 33], 7)        # ranges shorter than the 32-token rounding
    check([0, 0, 5000, 0], 3)
    check([64] * 1000, 256)      # many whole sequences per range
    W = sk_workgroups(256, 1, 1, 2, 200000, 256)
    check([200000, 200000], W)   # long contexts: the 61-block rule sets W
    check([5000, 3], 256, block_size=32, w_min=1)  # 61 blocks of 32 < 2048 tokens


def test_block_cap_needs_host_rule():
    # Without the host rule a range could span more than 63 blocks.
    pieces, _ = kernel_pieces([64 * 256 * 2], 1, 1)
    (w, b, t0, t1, complete, slot), = pieces
    assert (t1 - 1) // 256 - t0 // 256 + 1 > 63


def test_range_cap_falls_back_to_split_k():
    # block_size 32, 2048 sequences of 65536 tokens: 2^27 tokens need more
    # than 65535 ranges of 61 blocks.  Capped at 65535 workgroups a range
    # would span 65 blocks (past the 63 table entries a wave holds), so the
    # host rule sends this plan to split-K.
    batch, ctx, bs = 2048, 65536, 32
    W = sk_workgroups(256, 1, 1, batch, ctx, bs)
    assert W == 65535
    with pytest.raises(AssertionError):
        check([ctx] * batch, W, block_size=bs, w_min=256)
    assert not sk_eligible(batch, ctx, bs)
    # the largest batch the rule keeps on stream-K stays within 63 blocks
    b_ok = max(b for b in range(1, batch + 1) if sk_eligible(b, ctx, bs))
    assert b_ok < batch
    check([ctx] * b_ok, sk_workgroups(256, 1, 1, b_ok, ctx, bs), block_size=bs, w_min=256)
    # every plan the rule accepts at these sizes gets W within the cap
    for b in (1, 64, 512, b_ok):
        assert -(-(b * ctx) // (61 * bs)) <= sk_workgroups(256, 1, 1, b, ctx, bs) <= 65535
