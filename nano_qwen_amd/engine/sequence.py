"""The part of the reference's ``Sequence`` (engine/sequence.py:14-83) that
the attention metadata builders read: token ids, the block table, and the
cached / scheduled token counts."""
from __future__ import annotations

from itertools import count


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], block_table: list[int] | None = None,
                 num_cached_tokens: int = 0, num_scheduled_tokens: int = 0):
        self.seq_id = next(Sequence.counter)
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_cached_tokens = num_cached_tokens
        self.num_scheduled_tokens = num_scheduled_tokens
        self.block_table = list(block_table or [])

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
