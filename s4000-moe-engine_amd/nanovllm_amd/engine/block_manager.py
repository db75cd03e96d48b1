"""Paged KV block allocator with prefix caching, LRU reuse and host offload.

Behaviour-compatible with nanovllm/engine/block_manager.py:34-342 (same public
methods, victim order, hash chain, metrics names and executor protocol), so
the scheduler and the runner drive it unchanged:

* victim choice (`_pop_free`, :98-125): never-cached ("fresh") blocks first,
  then the least recently used cached-unreferenced block; with LRU disabled
  the plain FIFO head of the free list;
* prefix hash: xxh64 over the previous block's hash (8 bytes, little endian)
  followed by the block's token ids as int64 (:90-96);
* evict-to-host (:127-153): when an evicted block still owns its hash and an
  executor is set, `call("offload_put", block_id)` returns a host slot (or
  -1: the eviction degrades to a drop, counted in host_drops);
* revive (:155-166): a prefix hit in the host map allocates a fresh device
  block and issues `call("offload_get", slot, block_id)` then
  `call("offload_release", slot)`;
* host map and device hash map never describe the same hash (:76-88, :305).

The executor is any object with `call(name, *args)` — the engine's runner,
nanovllm_amd.engine.kv_runner.KVCacheRunner, or a test double.
"""
from __future__ import annotations

import os
from collections import OrderedDict, deque

import numpy as np
import xxhash

_LRU_DEFAULT = os.environ.get("NANOVLLM_LRU_EVICT", "1") == "1"


class Block:

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []

    def update(self, hash: int, token_ids: list[int]):
        self.hash = hash
        self.token_ids = token_ids

    def reset(self):
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        # Both victim classes are subsets of free_block_ids with ref_count 0.
        self._fresh: deque[int] = deque(range(num_blocks))
        self._fresh_set: set[int] = set(range(num_blocks))
        self._lru: OrderedDict[int, None] = OrderedDict()   # oldest first
        self.lru_enabled = _LRU_DEFAULT
        self.prefix_cache_hit_tokens = 0
        self.allocations = 0
        self.reclaims = 0
        self.evictions = 0
        self._offload_exec = None
        self._host_map: dict[int, tuple[int, list[int]]] = {}   # hash -> (slot, token ids)
        self.host_puts = 0
        self.host_revives = 0
        self.host_drops = 0

    # -- offload wiring --------------------------------------------------------
    def set_offload_executor(self, runner):
        self._offload_exec = runner

    def _release_host_entry(self, hash_key: int):
        entry = self._host_map.pop(hash_key, None)
        if entry is not None:
            self._offload_exec.call("offload_release", entry[0])

    # -- hashing ---------------------------------------------------------------
    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1):
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.asarray(token_ids, dtype=np.int64).tobytes())
        return h.intdigest()

    # -- block lifecycle -------------------------------------------------------
    def _take_from_free_list(self, block_id: int) -> None:
        if self.free_block_ids and self.free_block_ids[0] == block_id:
            self.free_block_ids.popleft()
        else:
            self.free_block_ids.remove(block_id)

    def _pop_free(self) -> int:
        if not self.lru_enabled:
            block_id = self.free_block_ids.popleft()
            if block_id in self._fresh_set:
                if self._fresh[0] == block_id:
                    self._fresh.popleft()
                else:
                    self._fresh.remove(block_id)
                self._fresh_set.discard(block_id)
            else:
                self._lru.pop(block_id, None)
            return block_id
        if self._fresh:
            block_id = self._fresh.popleft()
            self._fresh_set.discard(block_id)
        elif self._lru:
            block_id = next(iter(self._lru))
            self.evictions += 1
        else:
            block_id = self.free_block_ids[0]
        self._take_from_free_list(block_id)
        return block_id

    def _allocate_block(self) -> int:
        block_id = self._pop_free()
        block = self.blocks[block_id]
        assert block.ref_count == 0
        self._lru.pop(block_id, None)
        self._fresh_set.discard(block_id)
        owns_hash = block.hash != -1 and self.hash_to_block_id.get(block.hash) == block_id
        if owns_hash:
            if self._offload_exec is not None:
                slot = self._offload_exec.call("offload_put", block_id)
                if slot == -1:
                    self.host_drops += 1
                else:
                    self._release_host_entry(block.hash)
                    self._host_map[block.hash] = (slot, list(block.token_ids))
                    self.host_puts += 1
            del self.hash_to_block_id[block.hash]
        block.reset()
        self.used_block_ids.add(block_id)
        self.allocations += 1
        return block_id

    def _revive_from_host(self, hash_key: int) -> int:
        slot, token_ids = self._host_map.pop(hash_key)
        block_id = self._allocate_block()
        self._offload_exec.call("offload_get", slot, block_id)
        self._offload_exec.call("offload_release", slot)
        self.blocks[block_id].update(hash_key, token_ids)
        self.hash_to_block_id[hash_key] = block_id
        self.host_revives += 1
        return block_id

    def _deallocate_block(self, block_id: int):
        block = self.blocks[block_id]
        assert block.ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)
        if block.hash == -1:
            self._fresh.append(block_id)
            self._fresh_set.add(block_id)
        else:
            self._lru[block_id] = None   # enters at the MRU end
        self.reclaims += 1

    # -- sequence-level API ----------------------------------------------------
    def can_allocate(self, seq, touch: bool = True) -> int:
        """Number of leading cached blocks (device or host) for `seq`, or -1
        when the free list cannot hold the blocks it still needs."""
        h = -1
        cached = 0
        need = seq.num_blocks
        for i in range(seq.num_blocks - 1):      # the last block is never shared
            token_ids = seq.block(i)
            h = self.compute_hash(token_ids, h)
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id != -1 and self.blocks[block_id].token_ids == token_ids:
                cached += 1
                if touch and self.lru_enabled and block_id in self._lru:
                    self._lru.move_to_end(block_id)
                if block_id in self.used_block_ids:
                    need -= 1
                continue
            if self._offload_exec is not None:
                entry = self._host_map.get(h)
                if entry is not None and entry[1] == token_ids:
                    cached += 1             # revived into a fresh block: still needs one
                    continue
            break
        if len(self.free_block_ids) < need:
            return -1
        return cached

    def allocate(self, seq, num_cached_blocks: int):
        assert num_cached_blocks >= 0, "can_allocate returned -1 (insufficient KV)"
        assert not seq.block_table
        self.prefix_cache_hit_tokens += num_cached_blocks * self.block_size
        h = -1
        for i in range(num_cached_blocks):
            h = self.compute_hash(seq.block(i), h)
            if h not in self.hash_to_block_id:
                seq.block_table.append(self._revive_from_host(h))
                continue
            block_id = self.hash_to_block_id[h]
            block = self.blocks[block_id]
            if block_id in self.used_block_ids:
                block.ref_count += 1
            else:
                block.ref_count = 1
                self.free_block_ids.remove(block_id)
                self.used_block_ids.add(block_id)
                self._lru.pop(block_id, None)
            seq.block_table.append(block_id)
        for _ in range(num_cached_blocks, seq.num_blocks):
            seq.block_table.append(self._allocate_block())
        seq.num_cached_tokens = num_cached_blocks * self.block_size

    def deallocate(self, seq):
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq):
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._allocate_block())

    def _blocks_needed(self, seq, launch_len: int) -> int:
        need = (launch_len - 1) // self.block_size + 1
        return max(0, need - len(seq.block_table))

    def can_append_at(self, seq, launch_len: int) -> bool:
        return len(self.free_block_ids) >= self._blocks_needed(seq, launch_len)

    def total_launch_shortfall(self, seqs, launch_lens) -> int:
        return sum(self._blocks_needed(s, n) for s, n in zip(seqs, launch_lens))

    def may_append_at(self, seq, launch_len: int):
        while self._blocks_needed(seq, launch_len) > 0:
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq, num_new_tokens: int | None = None):
        """Hash the blocks the step just filled (num_new_tokens defaults to
        the sequence's scheduled tokens)."""
        q = seq.num_scheduled_tokens if num_new_tokens is None else num_new_tokens
        start = seq.num_cached_tokens // self.block_size
        end = (seq.num_cached_tokens + q) // self.block_size
        if start == end:
            return
        h = self.blocks[seq.block_table[start - 1]].hash if start > 0 else -1
        for i in range(start, end):
            block = self.blocks[seq.block_table[i]]
            token_ids = seq.block(i)
            h = self.compute_hash(token_ids, h)
            block.update(h, token_ids)
            if h in self._host_map:           # the device copy supersedes the host one
                self._release_host_entry(h)
            self.hash_to_block_id[h] = block.block_id

    def metrics(self):
        capacity = len(self.blocks)
        used = len(self.used_block_ids)
        return {
            "kv_blocks_capacity": capacity,
            "kv_blocks_used": used,
            "kv_cache_utilization": used / capacity if capacity else 0.0,
            "kv_prefix_hit_tokens_total": self.prefix_cache_hit_tokens,
            "kv_block_allocations_total": self.allocations,
            "kv_block_reclaims_total": self.reclaims,
            "kv_lru_size": len(self._lru),
            "kv_lru_evictions_total": self.evictions,
            "kv_lru_enabled": 1 if self.lru_enabled else 0,
            "kv_offload_host_entries": len(self._host_map),
            "kv_offload_puts_total": self.host_puts,
            "kv_offload_revives_total": self.host_revives,
            "kv_offload_drops_total": self.host_drops,
        }

    def clear_prefix_cache(self):
        if self._offload_exec is not None:
            for hash_key in list(self._host_map):
                self._release_host_entry(hash_key)
        self._host_map.clear()
        self.hash_to_block_id.clear()
        for block in self.blocks:
            block.hash = -1
            block.token_ids = []
        for block_id in self._lru:
            self._fresh.append(block_id)
            self._fresh_set.add(block_id)
        self._lru.clear()
