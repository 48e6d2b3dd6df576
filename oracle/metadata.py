"""Attention metadata closed forms (oracle; test infrastructure only).

Restates how the reference's model runner turns scheduled sequences into the
``Context`` fields the attention path reads.  A "sequence" here is any object
with ``token_ids`` (list), ``num_cached_tokens``, ``num_scheduled_tokens`` and
``block_table`` (list of block ids), as in engine/sequence.py:18-31.
"""
from __future__ import annotations


def prepare_block_tables(seqs):
    """engine/model_runner.py:236-240: rows padded with -1 to the longest."""
    width = max(len(s.block_table) for s in seqs)
    return [list(s.block_table) + [-1] * (width - len(s.block_table)) for s in seqs]


def prepare_prefill(seqs, block_size):
    """engine/model_runner.py:242-283 as plain lists.

    Per sequence: ``start = num_cached_tokens``, ``Lq = num_scheduled_tokens``,
    ``end = start + Lq``, ``Lk = end``; slots cover positions [start, end)
    through the block table; ``block_tables`` only when some ``Lk > Lq``.
    Sequences without a block table (warmup) contribute no slots (:262-263).
    """
    input_ids, positions, slot_mapping = [], [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    for s in seqs:
        start = s.num_cached_tokens
        lq = s.num_scheduled_tokens
        end = start + lq
        input_ids.extend(s.token_ids[start:end])
        positions.extend(range(start, end))
        cu_q.append(cu_q[-1] + lq)
        cu_k.append(cu_k[-1] + end)
        max_q, max_k = max(max_q, lq), max(max_k, end)
        if not s.block_table:
            continue
        for pos in range(start, end):
            slot_mapping.append(s.block_table[pos // block_size] * block_size + pos % block_size)
    tables = prepare_block_tables(seqs) if cu_k[-1] > cu_q[-1] else None
    return dict(input_ids=input_ids, positions=positions, cu_seqlens_q=cu_q,
                cu_seqlens_k=cu_k, max_seqlen_q=max_q, max_seqlen_k=max_k,
                slot_mapping=slot_mapping, block_tables=tables)


def prepare_decode(seqs, block_size, sampled_token_ids=None, batch_slots=None):
    """engine/model_runner.py:285-306 + engine/decode_init.py:29-36.

    ``positions = len-1``, ``context_lens = len``,
    ``slot_mapping = block_table[-1]*block_size + (len-1) % block_size``,
    ``input_ids = sampled_token_ids[batch_slots[i]]``.
    """
    n = len(seqs)
    seq_lens = [len(s.token_ids) for s in seqs]
    last = [s.block_table[-1] for s in seqs]
    out = dict(
        positions=[L - 1 for L in seq_lens],
        context_lens=list(seq_lens),
        slot_mapping=[lb * block_size + (L - 1) % block_size for lb, L in zip(last, seq_lens)],
        block_tables=prepare_block_tables(seqs),
    )
    if sampled_token_ids is not None:
        slots = list(batch_slots) if batch_slots is not None else list(range(n))
        out["input_ids"] = [int(sampled_token_ids[slots[i]]) for i in range(n)]
    return out
