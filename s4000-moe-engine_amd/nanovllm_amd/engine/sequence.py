"""Sequence state the KV path reads.

Mirrors the fields and block arithmetic of nanovllm/engine/sequence.py:16-119
that the block manager and the batch preparation use (token ids, cached and
scheduled token counts, block table, block(i), num_blocks,
last_block_num_tokens).  Sampling state is outside this path and is kept
only as opaque attributes.
"""
from __future__ import annotations

from itertools import count


class Sequence:
    block_size = 256
    _ids = count()

    def __init__(self, token_ids: list[int], sampling_params=None):
        self.seq_id = next(Sequence._ids)
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table: list[int] = []
        self.sampling_params = sampling_params

    def __len__(self) -> int:
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_blocks(self) -> int:
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        if not 0 <= i < self.num_blocks:
            raise IndexError(f"block {i} of a {self.num_blocks}-block sequence")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
