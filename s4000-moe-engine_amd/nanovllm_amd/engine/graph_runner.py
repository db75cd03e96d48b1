"""Bucketed HIP-graph replay of the decode step's KV work.

Follows the engine's decode graph protocol (nanovllm/engine/model_runner.py:
842-871 for replay, :1130-1200 for capture):
* batch-size buckets 1, 2, 4, 8, 16, 32, ... up to max_bs; a batch runs the
  graph of the smallest bucket that holds it;
* rows past the batch still execute inside the graph, so they are aimed at
  the pool's reserved scratch block: slot_mapping = scratch slot,
  context_lens = 1, block-table rows = the scratch block id.  They write and
  read only that block, never a live one;
* graph inputs are static buffers refreshed before each replay; the padding
  fills and copies run eagerly, outside the graph.  Padded q/k/v rows are
  zeros, so the padded rows' appends (all to the one scratch slot) store the
  same bytes whichever lands last.

What is captured is the path's part of a decode step, per layer:
store_kvcache(k, v, k_cache, v_cache, slot_mapping) then the paged decode,
as one paged_decode_append call (the append rides in the decode launch; a
padded row's slot is position 0 of its scratch-block table row, as the fused
append requires).  Nothing records a host synchronisation or a memset: loop
bounds come from the device context_lens, and the split-K workspace is taken
from torch's caching allocator (the graph's private pool during capture).
"""
from __future__ import annotations

import torch

from ..kernels.paged_attention import paged_decode_append


def default_buckets(max_bs: int) -> list[int]:
    """The engine's buckets (model_runner.py:1154): 1, 2, 4, 8, then every 16."""
    return [b for b in [1, 2, 4, 8] if b <= max_bs] + list(range(16, max_bs + 1, 16))


def pad_decode_inputs(slot_mapping: torch.Tensor, context_lens: torch.Tensor,
                      block_tables: torch.Tensor, slot_buf: torch.Tensor,
                      lens_buf: torch.Tensor, tables_buf: torch.Tensor,
                      scratch_slot: int, scratch_block_id: int) -> None:
    """Fill a bucket's static buffers: live rows from the batch, padded rows at
    the scratch block (model_runner.py:864-869)."""
    bs = slot_mapping.numel()
    slot_buf.fill_(scratch_slot)
    slot_buf[:bs] = slot_mapping
    lens_buf.fill_(1)
    lens_buf[:bs] = context_lens
    tables_buf.fill_(scratch_block_id)
    tables_buf[:bs, :block_tables.size(1)] = block_tables


class DecodeGraphRunner:
    """Graph-captured decode KV work for `num_layers` layers sharing one block
    table.  k_caches / v_caches: per-layer pools [num_blocks + 1, page, KVH, D]
    (the last block is the scratch block).  run(q, k, v, ...) takes
    q [L, bs, H, D], k / v [L, bs, KVH, D] and returns the attention outputs
    [L, bs, H, D] (a view into the static output buffer, valid until the
    next run).

    fence: the pool owner's ordering call, run on the current stream before
    every capture and every replay (KVCacheRunner.fence: with asynchronous
    offload, a put may still be reading a block that the replay appends
    into after the block manager reallocated it, and a replayed graph holds
    none of the eager per-layer waits).  from_kv_runner binds it; a runner
    built without one is for pools that no asynchronous move touches."""

    def __init__(self, k_caches, v_caches, num_heads: int, max_bs: int, max_blocks_per_seq: int,
                 scale: float, buckets: list[int] | None = None, fence=None):
        assert len(k_caches) == len(v_caches) and len(k_caches) > 0
        self.fence = fence
        self.k_caches, self.v_caches = list(k_caches), list(v_caches)
        kc = self.k_caches[0]
        self.num_layers = len(self.k_caches)
        self.page = kc.size(1)
        self.num_kv_heads = kc.size(2)
        self.head_dim = kc.size(3)
        self.num_heads = num_heads
        self.scratch_block_id = kc.size(0) - 1
        self.scratch_slot = self.scratch_block_id * self.page
        self.max_bs = max_bs
        self.scale = scale
        self.buckets = buckets or default_buckets(max_bs)
        assert max(self.buckets) <= max_bs
        dev, dt = kc.device, kc.dtype
        L, D = self.num_layers, self.head_dim
        self.q = torch.zeros(L, max_bs, num_heads, D, dtype=dt, device=dev)
        self.k = torch.zeros(L, max_bs, self.num_kv_heads, D, dtype=dt, device=dev)
        self.v = torch.zeros_like(self.k)
        self.out = torch.zeros_like(self.q)
        self.slot_mapping = torch.full((max_bs,), self.scratch_slot, dtype=torch.int32, device=dev)
        self.context_lens = torch.ones(max_bs, dtype=torch.int32, device=dev)
        self.block_tables = torch.full((max_bs, max_blocks_per_seq), self.scratch_block_id,
                                       dtype=torch.int32, device=dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.pool = None

    @classmethod
    def from_kv_runner(cls, kv_runner, num_heads: int, max_bs: int, max_blocks_per_seq: int,
                       scale: float, buckets: list[int] | None = None) -> "DecodeGraphRunner":
        """A runner over every layer of a KVCacheRunner's bf16 pool, fenced by
        that runner (its asynchronous offload copies, if any, are ordered
        before each capture and replay)."""
        if kv_runner.kv_int8 is not None:
            raise ValueError("the captured decode step runs on a bf16 pool")
        k_caches = [kv_runner.kv_cache[0, i] for i in range(kv_runner.num_layers)]
        v_caches = [kv_runner.kv_cache[1, i] for i in range(kv_runner.num_layers)]
        return cls(k_caches, v_caches, num_heads, max_bs, max_blocks_per_seq, scale, buckets,
                   fence=kv_runner.fence)

    def _step(self, bs: int) -> None:
        sm, cl, bt = self.slot_mapping[:bs], self.context_lens[:bs], self.block_tables[:bs]
        for layer in range(self.num_layers):
            kc, vc = self.k_caches[layer], self.v_caches[layer]
            self.out[layer, :bs] = paged_decode_append(
                self.q[layer, :bs], self.k[layer, :bs], self.v[layer, :bs], kc, vc, sm, bt, cl,
                self.scale)

    def capture(self) -> None:
        """Capture every bucket, small first (model_runner.py:1169-1175): a
        warm-up run on the padded (scratch) inputs, then the capture."""
        for bs in sorted(self.buckets):
            if self.fence is not None:
                self.fence()
            self._step(bs)  # warm-up on the side: scratch rows only
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.pool):
                self._step(bs)
            if self.pool is None:
                self.pool = graph.pool()
            self.graphs[bs] = graph
        torch.cuda.synchronize()

    def bucket_of(self, bs: int) -> int:
        for b in sorted(self.buckets):
            if b >= bs:
                return b
        raise ValueError(f"batch {bs} exceeds the largest bucket {max(self.buckets)}")

    def run(self, q, k, v, slot_mapping, context_lens, block_tables) -> torch.Tensor:
        """One replay, after the runner's fence (asynchronous block moves
        issued so far are ordered before the replay's pool reads and
        appends)."""
        bs = q.size(1)
        if self.fence is not None:
            self.fence()
        b = self.bucket_of(bs)
        self.q[:, :bs] = q
        self.k[:, :bs] = k
        self.v[:, :bs] = v
        # Padded rows all append to the one scratch slot; zeroing them makes
        # every such write the same bytes, so the scratch block's contents do
        # not depend on which row lands last.
        self.q[:, bs:b].zero_()
        self.k[:, bs:b].zero_()
        self.v[:, bs:b].zero_()
        pad_decode_inputs(slot_mapping, context_lens, block_tables, self.slot_mapping[:b],
                          self.context_lens[:b], self.block_tables[:b], self.scratch_slot,
                          self.scratch_block_id)
        self.graphs[b].replay()
        return self.out[:, :bs]
