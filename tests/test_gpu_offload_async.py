"""Asynchronous offload (puts and gets on copy streams, fenced per layer
group) against the blocking offload of nanovllm/engine/model_runner.py:
284-305, bit for bit.  Every test enqueues compute-stream work that
overwrites or reads the moved blocks right after the put / get, with only
the layer fences between them, so a missing or misplaced wait shows up as
mixed contents."""
import numpy as np
import pytest
import torch

from nanovllm_amd.engine.kv_offload import HostBlockPool
from nanovllm_amd.engine.kv_runner import KVCacheRunner
from nanovllm_amd.engine.offload_pipeline import AsyncOffloader
from nanovllm_amd.layers.attention import Attention
from nanovllm_amd.utils.context import reset_context, set_context
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"
L, PAGE, KVH = 8, 256, 4


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _setup(blocks=24, slots=8, groups=4, seed=0, engine="kernel"):
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(2, L, blocks, PAGE, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    host = HostBlockPool(slots, tuple(pool[:, :, 0].shape), dtype=pool.dtype)
    return pool, host, AsyncOffloader(pool, host, layer_groups=groups, copy_engine=engine)


@pytest.mark.parametrize("engine", ["kernel", "dma"])
@pytest.mark.parametrize("groups", [1, 3, 8])
def test_put_then_overwrite_per_layer(groups, engine):
    pool, host, off = _setup(groups=groups, seed=groups, engine=engine)
    orig = _u16(pool).copy()
    ids = [3, 7, 11, 20]
    print(f"[offload-async] put+overwrite groups={groups} engine={engine}", flush=True)
    slots = off.put_many(ids)
    assert sorted(slots) == [0, 1, 2, 3]
    g = torch.Generator(device=DEV).manual_seed(5)
    idx = torch.tensor(ids, device=DEV)
    for layer in range(L):          # the next step's appends, layer by layer
        off.fence_layer(layer)
        new = torch.randn(2, len(ids), PAGE, KVH, 128, generator=g, device=DEV)
        pool[:, layer].index_copy_(1, idx, new.to(torch.bfloat16))
    after = _u16(pool).copy()
    off.wait_host()
    buf = _u16(host.buffer)
    for s, b in zip(slots, ids):
        assert np.array_equal(buf[s], orig[:, :, b]), f"slot {s} (block {b})"
    assert not np.array_equal(after[:, :, ids], orig[:, :, ids])


@pytest.mark.parametrize("engine", ["kernel", "dma"])
def test_get_then_read_and_slot_reuse_order(engine):
    pool, host, off = _setup(seed=9, engine=engine)
    orig = _u16(pool).copy()
    print("[offload-async] put/get/release/put", flush=True)
    s = off.put_many([4, 5])
    # get while the put may still be in flight: must wait for it
    off.get_many(s, [14, 15])
    reads = []
    for layer in range(L):
        off.fence_layer(layer)
        reads.append(pool[:, layer, [14, 15]].clone())
    # release slot s[0] and take it again: the new put must not overwrite
    # the slot before the get above has read it
    off.release(s[0])
    s2 = off.put_many([9])
    assert s2 == [s[0]]
    off.get_many(s2, [16])
    off.fence()
    read16 = pool[:, :, 16].clone()
    off.wait_host()
    got = np.stack([_u16(r) for r in reads], axis=1)      # [2, L, 2, ...]
    assert np.array_equal(got, orig[:, :, [4, 5]])
    assert np.array_equal(_u16(pool)[:, :, [14, 15]], orig[:, :, [4, 5]])
    assert np.array_equal(_u16(read16), orig[:, :, 9])
    assert np.array_equal(_u16(host.buffer)[s2[0]], orig[:, :, 9])
    untouched = [b for b in range(pool.size(2)) if b not in (14, 15, 16)]
    assert np.array_equal(_u16(pool)[:, :, untouched], orig[:, :, untouched])


def test_full_pool_moves_nothing():
    pool, host, off = _setup(slots=2, seed=3)
    slots = off.put_many([1, 2, 3, 4])
    assert slots[2:] == [-1, -1] and host.full_count == 2 and host.puts == 2
    off.wait_host()
    orig = _u16(pool)
    assert np.array_equal(_u16(host.buffer)[slots[0]], orig[:, :, 1])
    with pytest.raises(KeyError):
        off.get_many([5], [0])
    with pytest.raises(IndexError):
        off.put_many([pool.size(2)])


def _layers(runner, n_layers, H):
    mods = [Attention(H, 128, 128 ** -0.5, KVH) for _ in range(n_layers)]
    assert runner.bind(mods) == n_layers
    return mods


def test_runner_async_equals_blocking():
    """A step that evicts blocks, reuses them for new prompt rows and revives
    others, through bound attention layers: the async runner's outputs, pool
    and host slots equal the blocking runner's bit for bit."""
    H, NB = 32, 12
    results = []
    g0 = torch.Generator().manual_seed(77)
    init = torch.randn(2, L, NB + 1, PAGE, KVH, 128, generator=g0).to(torch.bfloat16)
    q = torch.randn(PAGE, H, 128, generator=g0).to(torch.bfloat16).to(DEV)
    kv = torch.randn(2, L, PAGE, KVH, 128, generator=g0).to(torch.bfloat16).to(DEV)
    for groups, engine in ((0, "kernel"), (4, "kernel"), (3, "dma")):
        print(f"[offload-async] runner groups={groups} engine={engine}", flush=True)
        r = KVCacheRunner(L, NB, PAGE, KVH, 128, kv_offload_host_blocks=6,
                          async_offload_groups=groups, async_copy_engine=engine)
        r.kv_cache.copy_(init.to(DEV))
        mods = _layers(r, L, H)
        slots = r.offload_put_many([2, 5])            # evict blocks 2 and 5
        r.offload_get_many([slots[0]], [9])           # revive block 2's bytes into 9
        # a prompt of PAGE tokens written into the evicted block 5, attending
        # over [block 9 (revived), block 5]
        table = torch.tensor([[9, 5]], dtype=torch.int32, device=DEV)
        slot_map = torch.arange(5 * PAGE, 6 * PAGE, dtype=torch.int32, device=DEV)
        cq = torch.tensor([0, PAGE], dtype=torch.int32)
        ck = torch.tensor([0, 2 * PAGE], dtype=torch.int32)
        set_context(True, cq.to(DEV), ck.to(DEV), PAGE, 2 * PAGE, slot_map, None, table,
                    cu_seqlens_q_list=cq.tolist(), cu_seqlens_k_list=ck.tolist())
        outs = [m.forward(q, kv[0, i], kv[1, i]) for i, m in enumerate(mods)]
        reset_context()
        torch.cuda.synchronize()
        if r.kv_async is not None:
            r.kv_async.wait_host()
        results.append(([o.cpu() for o in outs], _u16(r.kv_cache).copy(),
                        _u16(r.kv_offloader.buffer)[slots].copy(), slots))
    (o0, p0, h0, s0) = results[0]
    assert np.array_equal(h0[1], ko.torch_bf16_bits(init)[:, :, 5])
    for o1, p1, h1, s1 in results[1:]:
        assert s0 == s1
        assert np.array_equal(h0, h1)
        assert np.array_equal(p0, p1)
        for a, b in zip(o0, o1):
            assert np.array_equal(_u16(a), _u16(b))
