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
