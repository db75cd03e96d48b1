"""HostBlockPool accounting (CPU): the gates of tests/p30_kv_offload_unit.py
t1-t4 and t6, plus the batching helpers' slot bookkeeping."""
import pytest
import torch

from nanovllm_amd.engine.kv_offload import HostBlockPool
from nanovllm_amd.workloads import build_block_tables

SHAPE = (2, 4, 8, 2, 16)


def rand():
    return torch.randn(*SHAPE).to(torch.bfloat16)


def test_roundtrip_bitwise():
    pool = HostBlockPool(3, SHAPE, pin=False)
    src = rand()
    slot = pool.put(src, key="h1")
    out = torch.empty(*SHAPE, dtype=torch.bfloat16)
    pool.get(slot, out)
    assert torch.equal(src, out)


def test_release_and_lifo_reuse():
    pool = HostBlockPool(2, SHAPE, pin=False)
    a = pool.put(rand(), "a")
    b = pool.put(rand(), "b")
    pool.release(a)
    a2 = pool.put(rand(), "a2")
    m = pool.metrics()
    assert a2 == a and b != a
    assert m["kv_offload_slots_in_use"] == 2 and m["kv_offload_releases_total"] == 1
    assert m["kv_offload_puts_total"] == 3 and m["kv_offload_slots_capacity"] == 2


def test_full_pool_returns_minus_one_then_recovers():
    pool = HostBlockPool(2, SHAPE, pin=False)
    s1 = pool.put(rand(), "1")
    s2 = pool.put(rand(), "2")
    assert pool.put(rand(), "3") == -1
    assert pool.metrics()["kv_offload_full_total"] == 1
    pool.release(s1)
    assert pool.put(rand(), "3") != -1 and s2 != -1


def test_shape_mismatch_raises():
    pool = HostBlockPool(1, SHAPE, pin=False)
    with pytest.raises(ValueError):
        pool.put(torch.randn(1, 2, 3), "x")
    pool.put(rand(), "k")
    with pytest.raises(ValueError):
        pool.get(0, torch.empty(1, 2, 3))
    with pytest.raises(KeyError):
        pool.release(5)


def test_no_room_fast_path_and_disabled_pool():
    pool = HostBlockPool(1, SHAPE, pin=False)
    assert pool.has_room()
    slot = pool.put(rand(), "a")
    assert not pool.has_room()
    assert pool.note_full() == -1 and pool.metrics()["kv_offload_full_total"] == 1
    disabled = HostBlockPool(0, SHAPE, pin=False)
    assert not disabled.has_room() and disabled.note_full() == -1
    assert disabled.put(rand(), "x") == -1
    pool.release(slot)
    assert pool.has_room()


def test_negative_capacity_rejected():
    with pytest.raises(ValueError):
        HostBlockPool(-1, SHAPE, pin=False)


def test_block_tables_are_disjoint_permutations():
    g = torch.Generator().manual_seed(5)
    bt = build_block_tables([300, 1, 513], 16, 256, g)
    used = bt[bt >= 0].tolist()
    assert len(used) == len(set(used)) == 2 + 1 + 3
    assert (bt[1, 1:] == -1).all()


def test_runner_refuses_offload_with_an_int8_pool():
    # nanovllm/config.py:75-78: offload moves kv_cache blocks only, so an int8
    # pool's scales / side pool would not follow; refused before any allocation.
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    for mode in ("tokhead", "chan"):
        with pytest.raises(AssertionError, match="bf16"):
            KVCacheRunner(2, 4, 256, 4, 128, kv_int8=mode, kv_offload_host_blocks=2)
