"""Block-granular KV export/import between a device pool and pinned staging.

Same API as nanovllm/pd/kv_channel.py:28-82 — KVBlockBuffer (pinned k/v
[n_blocks, L, block_size, kv_heads, head_dim]), extract_kv(kv_cache,
block_table, buf), import_kv(kv_cache, block_table, buf) — with the byte
moves done by libkvc: one gather kernel per pool writes straight into the
pinned buffer (no index_select temporary, no permute copy, no device-wide
synchronise), and one scatter kernel reads it back.  The round trip is a
bitwise copy.
"""
from __future__ import annotations

import torch

from ..engine.kv_runner import BlockMover


class KVBlockBuffer:
    """Pinned staging for n whole blocks: k/v [n_blocks, L, block_size, kv_heads, head_dim]."""

    def __init__(self, n_blocks: int, n_layers: int, block_size: int, kv_heads: int,
                 head_dim: int, dtype=torch.bfloat16):
        shape = (n_blocks, n_layers, block_size, kv_heads, head_dim)
        self.k = torch.empty(shape, dtype=dtype, pin_memory=True)
        self.v = torch.empty(shape, dtype=dtype, pin_memory=True)
        self.n_blocks = n_blocks

    @classmethod
    def from_pool(cls, kv_cache: torch.Tensor, n_blocks: int) -> "KVBlockBuffer":
        _, n_layers, _, block_size, kv_heads, head_dim = kv_cache.shape
        return cls(n_blocks, n_layers, block_size, kv_heads, head_dim, dtype=kv_cache.dtype)

    @property
    def nbytes(self) -> int:
        return self.k.element_size() * self.k.numel() + self.v.element_size() * self.v.numel()


def _movers(kv_cache: torch.Tensor):
    # kv_cache[0:1] / kv_cache[1:2] are the K and V pools as [1, L, blocks, ...].
    return BlockMover(kv_cache[0:1]), BlockMover(kv_cache[1:2])


def _items(t: torch.Tensor, n: int) -> torch.Tensor:
    # [n, L, bs, kvh, d] staging viewed as the mover's [n, 1, L, bs, kvh, d] items
    return t[:n].unsqueeze(1)


def extract_kv(kv_cache: torch.Tensor, block_table: list[int], buf: KVBlockBuffer,
               sync: bool = True) -> None:
    """buf.k[i] / buf.v[i] = the blocks block_table[i] of the K / V pools.

    Like the reference's blocking pinned copy, the call returns with the
    bytes in `buf` (it waits for the current stream); sync=False leaves the
    copy in flight, ordered on the current stream."""
    assert len(block_table) <= buf.n_blocks
    n = len(block_table)
    mk, mv = _movers(kv_cache)
    mk.gather(block_table, out=_items(buf.k, n))
    mv.gather(block_table, out=_items(buf.v, n))
    if sync and n:
        torch.cuda.current_stream(kv_cache.device).synchronize()


def import_kv(kv_cache: torch.Tensor, block_table: list[int], buf: KVBlockBuffer,
              sync: bool = True) -> None:
    """Blocks block_table[i] of the K / V pools = buf.k[i] / buf.v[i].

    Returns once `buf` may be reused by the host (sync=False: the kernels
    may still be reading it)."""
    assert len(block_table) <= buf.n_blocks
    n = len(block_table)
    mk, mv = _movers(kv_cache)
    mk.scatter(_items(buf.k, n), block_table)
    mv.scatter(_items(buf.v, n), block_table)
    if sync and n:
        torch.cuda.current_stream(kv_cache.device).synchronize()
