"""BlockManager known answers (CPU).

The scenarios and exact expected block ids restate the reference's own
tests: tests/p16_lru_evict.py:67-185 (victim order, touch-on-hit, FIFO
fallback, clear, invariant fuzz) and tests/p30_kv_offload_hostmap.py:131-235
(host map / pool slot exclusivity across a dropped eviction, with a fake
executor that mirrors HostBlockPool's slot accounting).
"""
import random

import pytest

from nanovllm_amd.engine.block_manager import BlockManager
from nanovllm_amd.engine.sequence import Sequence


def seq_of(tokens):
    return Sequence(list(tokens))


def commit(mgr, seq):
    seq.num_scheduled_tokens = seq.num_tokens - seq.num_cached_tokens
    mgr.hash_blocks(seq)
    seq.num_scheduled_tokens = 0


def check_invariants(mgr):
    for bid in mgr._lru:
        b = mgr.blocks[bid]
        assert b.ref_count == 0 and b.hash != -1 and bid in mgr.free_block_ids
    for bid in mgr._fresh:
        b = mgr.blocks[bid]
        assert b.ref_count == 0 and b.hash == -1 and bid in mgr.free_block_ids
    assert not (set(mgr._fresh) & set(mgr._lru))
    assert set(mgr._fresh) == mgr._fresh_set
    assert not (set(mgr.free_block_ids) & mgr.used_block_ids)
    assert len(mgr.free_block_ids) + len(mgr.used_block_ids) == len(mgr.blocks)


def test_hash_is_xxh64_chain_over_int64_tokens():
    import numpy as np
    import xxhash
    toks = [1, 2, 3, 70000]
    h0 = BlockManager.compute_hash(toks)
    assert h0 == xxhash.xxh64(np.array(toks, dtype=np.int64).tobytes()).intdigest()
    h1 = BlockManager.compute_hash([5], h0)
    assert h1 == xxhash.xxh64(h0.to_bytes(8, "little") + np.array([5], np.int64).tobytes()).intdigest()


def test_only_ref0_victims_fresh_first():
    mgr = BlockManager(6, 256)
    a = seq_of(range(1000, 1512))
    mgr.allocate(a, mgr.can_allocate(a))
    commit(mgr, a)
    c = seq_of(range(2000, 2512))
    mgr.allocate(c, mgr.can_allocate(c))
    commit(mgr, c)
    mgr.deallocate(c)
    d = seq_of(range(3000, 3512))
    mgr.allocate(d, mgr.can_allocate(d))
    assert a.block_table == [0, 1]
    assert d.block_table == [4, 5]
    assert mgr.hash_to_block_id.get(mgr.compute_hash(list(range(2000, 2256)), -1)) == 2


def test_touch_on_hit_protects_hot_prefix():
    hot_tokens = list(range(5000, 6024))           # 4 blocks, 3 hashable

    def build(lru_on):
        mgr = BlockManager(8, 256)
        mgr.lru_enabled = lru_on
        seqs = []
        for toks in (hot_tokens, range(7000, 7512), range(8000, 8512)):   # [0-3] [4,5] [6,7]
            s = seq_of(toks)
            mgr.allocate(s, mgr.can_allocate(s))
            commit(mgr, s)
            seqs.append(s)
        for s in seqs:                              # all free, all cached
            mgr.deallocate(s)
        if lru_on:
            mgr.can_allocate(seq_of(hot_tokens))    # a queued hitter touches 0, 1, 2
        d = seq_of(range(9000, 9512))
        mgr.allocate(d, mgr.can_allocate(d))
        h0 = mgr.compute_hash(hot_tokens[:256], -1)
        h1 = mgr.compute_hash(hot_tokens[256:512], h0)
        h2 = mgr.compute_hash(hot_tokens[512:768], h1)
        return mgr, h0, h1, h2

    mgr, h0, h1, _ = build(True)
    assert mgr.hash_to_block_id.get(h0) == 0
    assert mgr.hash_to_block_id.get(h1) == 1
    mgr, h0, _, h2 = build(False)
    assert mgr.hash_to_block_id.get(h2) is None     # FIFO sacrifices hot block 2
    assert mgr.hash_to_block_id.get(h0) == 0


def test_disabled_lru_is_fifo():
    mgr = BlockManager(4, 256)
    mgr.lru_enabled = False
    a = seq_of(range(1000, 1256))
    mgr.allocate(a, mgr.can_allocate(a))
    commit(mgr, a)
    mgr.deallocate(a)
    b = seq_of(range(1000, 1256))
    mgr.allocate(b, mgr.can_allocate(b))
    assert b.block_table == [1]


def test_clear_prefix_cache_empties_lru():
    mgr = BlockManager(4, 256)
    a = seq_of(range(1000, 1256))
    mgr.allocate(a, mgr.can_allocate(a))
    commit(mgr, a)
    mgr.deallocate(a)
    assert mgr._lru
    mgr.clear_prefix_cache()
    assert not mgr._lru and not mgr.hash_to_block_id
    assert all(b.hash == -1 for b in mgr.blocks)


@pytest.mark.parametrize("lru_on", [True, False])
def test_invariant_fuzz(lru_on):
    random.seed(11)
    mgr = BlockManager(8, 256)
    mgr.lru_enabled = lru_on
    live = []
    for _ in range(300):
        if live and random.random() < 0.4:
            mgr.deallocate(live.pop(random.randrange(len(live))))
        else:
            seed = random.randrange(3)
            n = random.choice([256, 512])
            s = Sequence([seed] * n)
            cached = mgr.can_allocate(s)
            if cached == -1:
                continue
            mgr.allocate(s, cached)
            s.num_cached_tokens = cached * 256
            commit(mgr, s)
            live.append(s)
        check_invariants(mgr)
    for s in live:
        mgr.deallocate(s)
    check_invariants(mgr)
    assert len(mgr.free_block_ids) == 8


class FakePool:
    """HostBlockPool slot accounting without bytes (LIFO slots, -1 when full)."""

    def __init__(self, capacity):
        self.free = list(range(capacity - 1, -1, -1))
        self.in_use = {}
        self.full = 0

    def call(self, name, *args):
        if name == "offload_put":
            if not self.free:
                self.full += 1
                return -1
            slot = self.free.pop()
            self.in_use[slot] = args[0]
            return slot
        if name == "offload_get":
            slot, block_id = args
            assert slot in self.in_use
            self.in_use[slot] = block_id
            return None
        if name == "offload_release":
            assert args[0] in self.in_use
            del self.in_use[args[0]]
            self.free.append(args[0])
            return None
        raise AssertionError(name)


def test_host_map_and_slots_stay_exclusive_across_drop_and_recompute():
    bm = BlockManager(num_blocks=8, block_size=256)
    pool = FakePool(capacity=2)
    bm.set_offload_executor(pool)

    def state():
        return len(bm._host_map), len(pool.in_use), bm.host_drops

    def donor(tokens):
        s = Sequence(tokens)
        bm.allocate(s, 0)
        bm.hash_blocks(s, len(s))
        bm.deallocate(s)

    tok_x = list(range(1000, 1257))
    tok_a = list(range(2000, 2513))
    donor(tok_x)
    donor(tok_a)
    assert len(bm.hash_to_block_id) == 3
    pressure = Sequence(list(range(3000, 4793)))
    bm.allocate(pressure, 0)
    bm.deallocate(pressure)
    assert state() == (2, 2, 1)              # X0, A1 pooled; A0 dropped
    rerun_x = Sequence(tok_x)
    cached = bm.can_allocate(rerun_x)
    assert cached == 1
    bm.allocate(rerun_x, cached)
    bm.hash_blocks(rerun_x, len(rerun_x))
    assert state()[:2] == (1, 1)
    rerun_a = Sequence(tok_a)
    assert bm.can_allocate(rerun_a) == 0     # block 0 was dropped: the chain breaks
    bm.allocate(rerun_a, 0)
    bm.hash_blocks(rerun_a, len(rerun_a))
    assert state()[:2] == (0, 0)             # stale A1 host entry released
    bm.deallocate(rerun_a)
    pressure = Sequence(list(range(5000, 6025)))
    bm.allocate(pressure, 0)
    bm.deallocate(pressure)
    assert state()[:2] == (1, 1)             # no orphaned slot
    bm.clear_prefix_cache()
    assert state()[:2] == (0, 0)


def test_metrics_names():
    m = BlockManager(4, 256).metrics()
    assert set(m) == {
        "kv_blocks_capacity", "kv_blocks_used", "kv_cache_utilization",
        "kv_prefix_hit_tokens_total", "kv_block_allocations_total", "kv_block_reclaims_total",
        "kv_lru_size", "kv_lru_evictions_total", "kv_lru_enabled", "kv_offload_host_entries",
        "kv_offload_puts_total", "kv_offload_revives_total", "kv_offload_drops_total"}


def test_append_and_launch_shortfall():
    bm = BlockManager(4, 256)
    s = Sequence(list(range(256)))
    bm.allocate(s, bm.can_allocate(s))
    s.append_token(7)                         # len 257 -> needs a new block
    assert bm.can_append(s)
    bm.may_append(s)
    assert len(s.block_table) == 2
    assert bm._blocks_needed(s, 513) == 1
    assert bm.total_launch_shortfall([s, s], [513, 769]) == 3
    bm.may_append_at(s, 769)
    assert len(s.block_table) == 4
