"""Paged KV block allocator: prefix cache, two-tier reuse, host offload.

Drop-in for nanovllm/engine/block_manager.py:34-342.  The scheduler, the
runner and the engine's own tests see the same surface — public methods and
their results, `blocks[i].ref_count/hash/token_ids`, `free_block_ids`,
`used_block_ids`, `hash_to_block_id`, the metric names, the executor
protocol `call("offload_put" | "offload_get" | "offload_release", ...)` —
and every observable decision is the engine's, because those callers depend
on it:
  * reuse order: never-hashed free blocks first, in the order they were
    freed; then the least recently used hashed free block (one eviction);
    with LRU off, the oldest free block whatever its tier (:98-125);
  * a reused block that still owns its hash is offered to the host pool
    first (put, then the release of any stale host copy of that hash), its
    hash forgotten, then the block reset (:127-153);
  * a prefix found only on the host is revived into a newly reused block:
    get, then release of the slot (:155-166);
  * hash_blocks' device copy supersedes a host copy of the same hash
    (:284-307); clear_prefix_cache releases every host entry and demotes
    the hashed free blocks to the fresh tier, in recency order (:329-342).

The state is kept differently.  Per-block fields live in Block objects
indexed by id plus a tier tag per block (in use, free and never hashed,
free and hashed).  Free blocks are threaded on two intrusive doubly linked
lists that share index arrays: the free queue (every free block, in the
order it was freed) and the tier queues (fresh blocks in free order, hashed
blocks in recency order; a block is on at most one).  Each insertion,
removal, move to the back and pop is O(1) — the engine's deque.remove and
OrderedDict bookkeeping are O(n) or hash lookups.  `free_block_ids`,
`used_block_ids`, `_fresh`, `_fresh_set` and `_lru` are read-only views over
that state with the containers' iteration order and membership.

Prefix hash: xxh64 of the previous block's hash (8 bytes, little endian,
absent for the first block) followed by the block's token ids as int64
(:90-96).
"""
from __future__ import annotations

import operator
import os
from collections.abc import Set
from typing import NamedTuple

import numpy as np
import xxhash

_LRU_DEFAULT = os.environ.get("NANOVLLM_LRU_EVICT", "1") == "1"

# tier tags
_USED, _FRESH, _CACHED = 0, 1, 2


class Block:
    __slots__ = ("block_id", "ref_count", "hash", "token_ids")

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


class HostEntry(NamedTuple):
    """A prefix block parked in a host slot: (slot, token ids)."""
    slot: int
    token_ids: list


def _as_id(x):
    try:
        return operator.index(x)
    except TypeError:
        return None


class _Rings:
    """Doubly linked rings over ids 0..n-1, one sentinel per ring (ids n,
    n+1, ...).  An id is on at most one ring of a given _Rings."""

    __slots__ = ("n", "prev", "next", "ring", "size")

    def __init__(self, n: int, rings: int):
        self.n = n
        self.prev = list(range(n + rings))
        self.next = list(range(n + rings))
        self.ring = [-1] * n
        self.size = [0] * rings

    def append(self, r: int, i: int) -> None:
        s = self.n + r
        last = self.prev[s]
        self.next[last] = i
        self.prev[i] = last
        self.next[i] = s
        self.prev[s] = i
        self.ring[i] = r
        self.size[r] += 1

    def unlink(self, i: int) -> None:
        r = self.ring[i]
        if r < 0:
            return
        a, b = self.prev[i], self.next[i]
        self.next[a] = b
        self.prev[b] = a
        self.ring[i] = -1
        self.size[r] -= 1

    def first(self, r: int) -> int:
        i = self.next[self.n + r]
        return i if i < self.n else -1

    def to_back(self, i: int) -> None:
        r = self.ring[i]
        self.unlink(i)
        self.append(r, i)

    def walk(self, r: int):
        i = self.next[self.n + r]
        while i < self.n:
            yield i
            i = self.next[i]


class _RingView:
    """Read-only view of one ring: len, iteration in ring order, membership,
    index 0 (the head)."""

    def __init__(self, rings: _Rings, r: int):
        self._rings, self._r = rings, r

    def __len__(self) -> int:
        return self._rings.size[self._r]

    def __bool__(self) -> bool:
        return self._rings.size[self._r] > 0

    def __iter__(self):
        return self._rings.walk(self._r)

    def __contains__(self, i) -> bool:
        i = _as_id(i)
        return i is not None and 0 <= i < self._rings.n and self._rings.ring[i] == self._r

    def __getitem__(self, k: int) -> int:
        if k != 0:
            return list(self)[k]
        head = self._rings.first(self._r)
        if head < 0:
            raise IndexError("empty")
        return head

    def keys(self):
        return list(self)

    def __repr__(self) -> str:
        return f"{type(self).__name__}({list(self)})"


class _UsedView(Set):
    """The set of referenced block ids (a read-only Set)."""

    def __init__(self, mgr: "BlockManager"):
        self._mgr = mgr

    @classmethod
    def _from_iterable(cls, it):
        return set(it)

    def __contains__(self, i) -> bool:
        t = self._mgr._tier
        i = _as_id(i)
        return i is not None and 0 <= i < len(t) and t[i] == _USED

    def __iter__(self):
        return (i for i, t in enumerate(self._mgr._tier) if t == _USED)

    def __len__(self) -> int:
        return self._mgr._n_used


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self._tier = [_FRESH] * num_blocks
        self._n_used = 0
        self._freeq = _Rings(num_blocks, 1)      # ring 0: free queue
        self._tiers = _Rings(num_blocks, 2)      # ring 0: fresh, ring 1: hashed (LRU order)
        for i in range(num_blocks):
            self._freeq.append(0, i)
            self._tiers.append(0, i)
        self.free_block_ids = _RingView(self._freeq, 0)
        self.used_block_ids = _UsedView(self)
        self._fresh = _RingView(self._tiers, 0)
        self._lru = _RingView(self._tiers, 1)
        self.lru_enabled = _LRU_DEFAULT
        self.prefix_cache_hit_tokens = 0
        self.allocations = 0
        self.reclaims = 0
        self.evictions = 0
        self._offload_exec = None
        self._host_map: dict[int, HostEntry] = {}
        self.host_puts = 0
        self.host_revives = 0
        self.host_drops = 0

    @property
    def _fresh_set(self) -> set[int]:
        return set(self._fresh)

    # -- executor ---------------------------------------------------------------
    def set_offload_executor(self, runner):
        """runner.call(name, *args) moves the bytes (None: offload off)."""
        self._offload_exec = runner

    def _drop_host_copy(self, h: int) -> None:
        entry = self._host_map.pop(h, None)
        if entry is not None:
            self._offload_exec.call("offload_release", entry.slot)

    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1):
        x = xxhash.xxh64()
        if prefix != -1:
            x.update(prefix.to_bytes(8, "little"))
        x.update(np.asarray(token_ids, dtype=np.int64).tobytes())
        return x.intdigest()

    # -- free-block state -----------------------------------------------------
    def _mark_free(self, bid: int) -> None:
        self._tier[bid] = _FRESH if self.blocks[bid].hash == -1 else _CACHED
        self._n_used -= 1
        self._freeq.append(0, bid)
        self._tiers.append(0 if self._tier[bid] == _FRESH else 1, bid)

    def _mark_used(self, bid: int) -> None:
        self._freeq.unlink(bid)
        self._tiers.unlink(bid)
        self._tier[bid] = _USED
        self._n_used += 1

    def _victim(self) -> int:
        """Which free block the next allocation reuses."""
        if not self.lru_enabled:
            bid = self._freeq.first(0)
        else:
            bid = self._tiers.first(0)
            if bid < 0:
                bid = self._tiers.first(1)
                if bid >= 0:
                    self.evictions += 1
                else:
                    bid = self._freeq.first(0)
        if bid < 0:
            raise IndexError("no free KV block")
        return bid

    def _claim(self) -> int:
        """Reuse a free block: offload or drop what it caches, hand it out
        with one reference."""
        bid = self._victim()
        block = self.blocks[bid]
        assert block.ref_count == 0
        self._mark_used(bid)
        h = block.hash
        if h != -1 and self.hash_to_block_id.get(h) == bid:
            if self._offload_exec is not None:
                slot = self._offload_exec.call("offload_put", bid)
                if slot != -1:
                    self._drop_host_copy(h)
                    self._host_map[h] = HostEntry(slot, list(block.token_ids))
                    self.host_puts += 1
                else:
                    self.host_drops += 1
            del self.hash_to_block_id[h]
        block.reset()
        self.allocations += 1
        return bid

    def _revive(self, h: int) -> int:
        entry = self._host_map.pop(h)
        bid = self._claim()
        self._offload_exec.call("offload_get", entry.slot, bid)
        self._offload_exec.call("offload_release", entry.slot)
        self.blocks[bid].update(h, entry.token_ids)
        self.hash_to_block_id[h] = bid
        self.host_revives += 1
        return bid

    def _unref(self, bid: int) -> None:
        block = self.blocks[bid]
        block.ref_count -= 1
        if block.ref_count == 0:
            self._mark_free(bid)
            self.reclaims += 1

    # -- the engine's API ---------------------------------------------------
    def can_allocate(self, seq, touch: bool = True) -> int:
        """Leading cached blocks of `seq` (on the device, or parked on the
        host), or -1 if the free blocks cannot cover the rest.  The last
        block is never matched.  touch moves device hits to the recent end."""
        h, hits, need = -1, 0, seq.num_blocks
        for i in range(seq.num_blocks - 1):
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            bid = self.hash_to_block_id.get(h, -1)
            if bid != -1 and self.blocks[bid].token_ids == toks:
                hits += 1
                tier = self._tier[bid]
                if touch and self.lru_enabled and tier == _CACHED:
                    self._tiers.to_back(bid)
                if tier == _USED:
                    need -= 1
                continue
            if self._offload_exec is not None:
                entry = self._host_map.get(h)
                if entry is not None and entry.token_ids == toks:
                    hits += 1          # revived into a reused block: still needs one
                    continue
            break
        return -1 if self._freeq.size[0] < need else hits

    def allocate(self, seq, num_cached_blocks: int):
        assert num_cached_blocks >= 0, "can_allocate returned -1 (insufficient KV)"
        assert not seq.block_table
        self.prefix_cache_hit_tokens += num_cached_blocks * self.block_size
        table = seq.block_table
        h = -1
        for i in range(num_cached_blocks):
            h = self.compute_hash(seq.block(i), h)
            bid = self.hash_to_block_id.get(h)
            if bid is None:
                table.append(self._revive(h))
                continue
            block = self.blocks[bid]
            if self._tier[bid] == _USED:
                block.ref_count += 1
            else:
                block.ref_count = 1
                self._mark_used(bid)
            table.append(bid)
        for _ in range(num_cached_blocks, seq.num_blocks):
            table.append(self._claim())
        seq.num_cached_tokens = num_cached_blocks * self.block_size

    def deallocate(self, seq):
        for bid in reversed(seq.block_table):
            self._unref(bid)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq) -> bool:
        return self._freeq.size[0] >= (len(seq) % self.block_size == 1)

    def may_append(self, seq):
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._claim())

    def _blocks_needed(self, seq, launch_len: int) -> int:
        """Table shortfall of a decode row whose input token is at index
        launch_len - 1 (block_manager.py:258-263)."""
        return max(0, (launch_len - 1) // self.block_size + 1 - len(seq.block_table))

    def can_append_at(self, seq, launch_len: int) -> bool:
        return self._freeq.size[0] >= self._blocks_needed(seq, launch_len)

    def total_launch_shortfall(self, seqs, launch_lens) -> int:
        return sum(self._blocks_needed(s, n) for s, n in zip(seqs, launch_lens))

    def may_append_at(self, seq, launch_len: int):
        for _ in range(self._blocks_needed(seq, launch_len)):
            seq.block_table.append(self._claim())

    def hash_blocks(self, seq, num_new_tokens: int | None = None):
        """Hash the blocks the step filled (num_new_tokens: the step's query
        length, default the sequence's scheduled tokens)."""
        new = seq.num_scheduled_tokens if num_new_tokens is None else num_new_tokens
        bs = self.block_size
        first, stop = seq.num_cached_tokens // bs, (seq.num_cached_tokens + new) // bs
        if first == stop:
            return
        h = self.blocks[seq.block_table[first - 1]].hash if first else -1
        for i in range(first, stop):
            bid = seq.block_table[i]
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            self.blocks[bid].update(h, toks)
            if h in self._host_map:
                self._drop_host_copy(h)
            self.hash_to_block_id[h] = bid

    def metrics(self):
        n = len(self.blocks)
        return {
            "kv_blocks_capacity": n,
            "kv_blocks_used": self._n_used,
            "kv_cache_utilization": self._n_used / n if n else 0.0,
            "kv_prefix_hit_tokens_total": self.prefix_cache_hit_tokens,
            "kv_block_allocations_total": self.allocations,
            "kv_block_reclaims_total": self.reclaims,
            "kv_lru_size": self._tiers.size[1],
            "kv_lru_evictions_total": self.evictions,
            "kv_lru_enabled": int(bool(self.lru_enabled)),
            "kv_offload_host_entries": len(self._host_map),
            "kv_offload_puts_total": self.host_puts,
            "kv_offload_revives_total": self.host_revives,
            "kv_offload_drops_total": self.host_drops,
        }

    def clear_prefix_cache(self):
        """Forget every hash (live blocks keep their contents and owners)."""
        if self._offload_exec is not None:
            for h in list(self._host_map):
                self._drop_host_copy(h)
        self._host_map.clear()
        self.hash_to_block_id.clear()
        for block in self.blocks:
            block.hash = -1
            block.token_ids = []
        for bid in list(self._tiers.walk(1)):
            self._tiers.unlink(bid)
            self._tiers.append(0, bid)
            self._tier[bid] = _FRESH
