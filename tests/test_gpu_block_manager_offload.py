"""The engine's BlockManager driving the GPU runner's offload executor
(nanovllm/engine/block_manager.py evict-to-host and revive,
model_runner.py:284-308): a hashed block evicted under pressure goes to a
pinned slot, its device block is reused and overwritten, and a later prompt
with the same prefix revives the bytes into a fresh block bit for bit, with
the blocking moves and with the asynchronous pipeline."""
import numpy as np
import pytest
import torch

from nanovllm_amd.engine.block_manager import BlockManager
from nanovllm_amd.engine.kv_runner import KVCacheRunner
from nanovllm_amd.engine.sequence import Sequence

pytestmark = pytest.mark.gpu
L, NB, PAGE, KVH = 4, 8, 256, 4


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("groups", [0, 2])
def test_evict_to_host_and_revive_bitwise(groups):
    print(f"[bm-offload] groups={groups}", flush=True)
    runner = KVCacheRunner(L, NB, PAGE, KVH, 128, kv_offload_host_blocks=2,
                           async_offload_groups=groups)
    g = torch.Generator(device="cuda").manual_seed(7)
    runner.kv_cache.normal_(generator=g)
    bm = BlockManager(NB, PAGE)
    bm.set_offload_executor(runner)
    tok_x = list(range(1000, 1000 + PAGE + 1))       # one full (hashed) block + 1 token
    donor = Sequence(tok_x)
    bm.allocate(donor, 0)
    bm.hash_blocks(donor, len(donor))
    x0 = donor.block_table[0]
    snap = _u16(runner.kv_cache[:, :, x0])
    bm.deallocate(donor)
    # Pressure for every block: the hashed block is evicted to a host slot.
    pressure = Sequence(list(range(5000, 5000 + NB * PAGE)))
    bm.allocate(pressure, 0)
    assert bm.metrics()["kv_offload_puts_total"] == 1
    runner.fence()                                    # device writes follow the offload
    runner.kv_cache.normal_(generator=g)              # the pressure prompt's KV
    bm.deallocate(pressure)
    rerun = Sequence(tok_x)
    cached = bm.can_allocate(rerun)
    assert cached == 1
    bm.allocate(rerun, cached)
    assert bm.metrics()["kv_offload_revives_total"] == 1
    runner.fence()
    torch.cuda.synchronize()
    revived = rerun.block_table[0]
    assert np.array_equal(_u16(runner.kv_cache[:, :, revived]), snap)
    bm.deallocate(rerun)
    bm.clear_prefix_cache()
    assert runner.kv_offloader.metrics()["kv_offload_slots_in_use"] == 0


@pytest.mark.parametrize("groups,engine", [(0, "kernel"), (2, "kernel"), (8, "kernel"),
                                           (3, "dma")])
def test_revive_into_the_block_its_own_eviction_frees(groups, engine):
    """A revive whose fresh block is the LRU victim of the same allocation:
    _revive_from_host -> _allocate_block evicts hashed block B
    (offload_put(B)) and then brings the host copy back into B
    (offload_get(slot, B)).  The put must read B before the get overwrites
    it: the new slot holds B's old bytes, B holds the revived bytes."""
    print(f"[bm-offload] revive into the evicted block groups={groups} engine={engine}",
          flush=True)
    runner = KVCacheRunner(L, NB, PAGE, KVH, 128, kv_offload_host_blocks=2,
                           async_offload_groups=groups, async_copy_engine=engine)
    g = torch.Generator(device="cuda").manual_seed(11)
    runner.kv_cache.normal_(generator=g)
    bm = BlockManager(NB, PAGE)
    bm.set_offload_executor(runner)
    tok_x = list(range(1000, 1000 + PAGE + 1))
    donor = Sequence(tok_x)
    bm.allocate(donor, 0)
    bm.hash_blocks(donor, len(donor))
    x_bytes = _u16(runner.kv_cache[:, :, donor.block_table[0]])
    bm.deallocate(donor)
    # Y takes every block (X's block goes to host slot 0), writes its KV and
    # hashes every block: afterwards each free block is a cached LRU block.
    y = Sequence(list(range(7000, 7000 + NB * PAGE)))
    bm.allocate(y, 0)
    assert bm.metrics()["kv_offload_puts_total"] == 1
    runner.fence()
    runner.kv_cache.normal_(generator=g)
    bm.hash_blocks(y, len(y))
    # deallocated last block first: the LRU order is Y's table reversed
    victim, second = y.block_table[-1], y.block_table[-2]
    y_bytes = _u16(runner.kv_cache[:, :, victim])
    y2_bytes = _u16(runner.kv_cache[:, :, second])
    bm.deallocate(y)
    rerun = Sequence(tok_x)
    cached = bm.can_allocate(rerun)
    assert cached == 1
    # block 0: put(victim) -> slot 1, get(slot 0 -> victim), release slot 0;
    # block 1: put(second) -> slot 0 again, which the get above still reads
    bm.allocate(rerun, cached)
    m = bm.metrics()
    assert m["kv_offload_revives_total"] == 1 and m["kv_offload_puts_total"] == 3
    assert rerun.block_table == [victim, second]
    runner.fence()
    if runner.kv_async is not None:
        runner.kv_async.wait_host()
    torch.cuda.synchronize()
    host = runner.kv_offloader.buffer
    assert np.array_equal(_u16(host[1]), y_bytes), \
        "the evicted block's host copy is not its old bytes"
    assert np.array_equal(_u16(host[0]), y2_bytes), "the reused slot's copy is not block 1's"
    assert np.array_equal(_u16(runner.kv_cache[:, :, victim]), x_bytes), \
        "the revived block is not the host copy"
    bm.deallocate(rerun)
    bm.clear_prefix_cache()
    assert runner.kv_offloader.metrics()["kv_offload_slots_in_use"] == 0


def _trace(seed):
    import gzip
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "block_manager_trace.json.gz")
    with gzip.open(path, "rt") as f:
        return next(t for t in json.load(f)["traces"] if t["seed"] == seed)


@pytest.mark.parametrize("seed", [1, 4, 6])
@pytest.mark.parametrize("groups", [0, 4])
def test_replay_reference_executor_logs_bitwise(seed, groups):
    """The offload_put / offload_get / offload_release calls the reference's
    BlockManager made on a recorded trace, replayed in order against the GPU
    runner.  Between ops the blocks the op reused and did not revive are
    overwritten on the compute stream (the next prefill's KV).  Every slot
    number must be the reference executor's, and the bytes of every host slot
    and device block must follow the calls: put copies a block to its slot,
    get copies a slot back."""
    tr = _trace(seed)
    nb, slots = tr["num_blocks"], tr["host_slots"]
    print(f"[bm-offload] replay seed={seed} blocks={nb} slots={slots} groups={groups}",
          flush=True)
    Lr = 2
    runner = KVCacheRunner(Lr, nb, PAGE, KVH, 128, kv_offload_host_blocks=slots,
                           async_offload_groups=groups)
    planes = torch.arange(2 * Lr, device="cuda", dtype=torch.int32).view(2, Lr, 1, 1, 1)

    def write(b, tag):
        # every plane of block b: (tag * 8 + plane) in each 16-bit element
        val = ((tag * 8 + planes) & 0x7FFF).to(torch.int16)
        runner.kv_cache.view(torch.int16)[:, :, b] = val.expand(2, Lr, PAGE, KVH, 128)

    dev_tag = {b: b + 1 for b in range(nb)}
    runner.fence()
    for b, t in dev_tag.items():
        write(b, t)
    slot_tag = {}
    next_tag = nb + 1
    calls = 0

    def expected(tag):
        return ((tag * 8 + torch.arange(2 * Lr, dtype=torch.int32).view(2, Lr, 1, 1, 1))
                & 0x7FFF).to(torch.int16).expand(2, Lr, PAGE, KVH, 128)

    def check():
        runner.fence()
        if runner.kv_async is not None:
            runner.kv_async.wait_host()
        torch.cuda.synchronize()
        pool = runner.kv_cache.view(torch.int16).cpu()
        for b, t in dev_tag.items():
            assert torch.equal(pool[:, :, b], expected(t)), f"block {b} after {calls} calls"
        host = runner.kv_offloader.buffer.view(torch.int16)
        for s_, t in slot_tag.items():
            assert torch.equal(host[s_], expected(t)), f"slot {s_} after {calls} calls"

    for i, rec in enumerate(tr["records"]):
        reused = []
        for call in rec["exec_log"]:
            name = call[0]
            calls += 1
            if name == "offload_put":
                b = call[1]
                got = runner.call("offload_put", b)
                reused.append(b)
                if got != -1:
                    slot_tag[got] = dev_tag[b]
            elif name == "offload_get":
                s, b = call[1], call[2]
                runner.call("offload_get", s, b)
                dev_tag[b] = slot_tag[s]
                if b in reused:
                    reused.remove(b)
            else:
                s = call[1]
                runner.call("offload_release", s)
                del slot_tag[s]
        # the slot numbers are the reference executor's (both hand them out LIFO)
        assert sorted(slot_tag) == rec["host_in_use"], f"op {i}: host slots in use"
        if reused:
            runner.fence()
            for b in reused:
                assert next_tag < 4000          # tags stay distinct in 15 bits
                dev_tag[b] = next_tag
                write(b, next_tag)
                next_tag += 1
        if i % 100 == 99:
            check()
    check()
    assert calls == sum(len(r["exec_log"]) for r in tr["records"]) > 0
