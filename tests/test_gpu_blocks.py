"""Whole-block movement parity (bit-exact): gather, scatter, compaction copy and
the DMA offload moves, on the engine's [2, L, blocks, page, KVH, D] pool."""
import numpy as np
import pytest
import torch

from nanovllm_amd.engine.kv_runner import BlockMover
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pool(L=3, blocks=20, kvh=4, seed=0, page=256):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(2, L, blocks, page, kvh, 128, generator=g).to(torch.bfloat16).to(DEV)


def _np(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def test_gather_into_device_staging_and_pinned_host():
    pool = _pool()
    mover = BlockMover(pool)
    ids = [7, 0, 19, 3, 3]
    print("[blocks] gather", flush=True)
    dev = mover.gather(ids)                      # [n, 2, L, page, KVH, D] device
    host = torch.empty((len(ids),) + tuple(pool[:, :, 0].shape), dtype=pool.dtype, pin_memory=True)
    mover.gather(ids, out=host)                  # kernel writes pinned host memory
    torch.cuda.synchronize()
    ref = ko.block_gather(_np(pool).reshape(2 * pool.size(1), pool.size(2), -1), ids)
    assert np.array_equal(_np(dev).reshape(ref.shape), ref)
    assert np.array_equal(_np(host).reshape(ref.shape), ref)


def test_scatter_from_pinned_host():
    pool = _pool(seed=1)
    mover = BlockMover(pool)
    ids = [2, 11, 5]
    g = torch.Generator().manual_seed(2)
    items = torch.randn((3,) + tuple(pool[:, :, 0].shape), generator=g).to(torch.bfloat16).pin_memory()
    expect = _np(pool).reshape(2 * pool.size(1), pool.size(2), -1).copy()
    ko.block_scatter(expect, ids, _np(items).reshape(3, 2 * pool.size(1), -1))
    print("[blocks] scatter", flush=True)
    mover.scatter(items, ids)
    torch.cuda.synchronize()
    assert np.array_equal(_np(pool).reshape(expect.shape), expect)


def test_compaction_copy_disjoint_and_overlapping():
    pool = _pool(seed=3, blocks=32)
    mover = BlockMover(pool)
    expect = _np(pool).reshape(2 * pool.size(1), pool.size(2), -1).copy()
    src, dst = [1, 5, 9, 30], [2, 6, 10, 31]
    ko.block_copy(expect, src, dst)
    print("[blocks] copy disjoint", flush=True)
    mover.copy(src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(_np(pool).reshape(expect.shape), expect)
    # A chain (dst of one pair is the src of another) must behave as a
    # simultaneous copy, like pool[:, :, dst] = pool[:, :, src].
    src, dst = [3, 4, 8], [4, 8, 12]
    ko.block_copy(expect, src, dst)
    print("[blocks] copy overlapping", flush=True)
    mover.copy(src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(_np(pool).reshape(expect.shape), expect)


def test_dma_offload_roundtrip():
    pool = _pool(seed=4)
    mover = BlockMover(pool)
    ids = [4, 17, 0]
    host = torch.empty((3,) + tuple(pool[:, :, 0].shape), dtype=pool.dtype, pin_memory=True)
    print("[blocks] d2h dma", flush=True)
    mover.d2h(ids, host)
    torch.cuda.synchronize()
    ref = ko.block_gather(_np(pool).reshape(2 * pool.size(1), pool.size(2), -1), ids)
    assert np.array_equal(_np(host).reshape(ref.shape), ref)
    new_ids = [9, 1, 13]
    expect = _np(pool).reshape(2 * pool.size(1), pool.size(2), -1).copy()
    ko.block_scatter(expect, new_ids, _np(host).reshape(ref.shape))
    print("[blocks] h2d dma", flush=True)
    mover.h2d(host, new_ids)
    torch.cuda.synchronize()
    assert np.array_equal(_np(pool).reshape(expect.shape), expect)


def test_overlapped_swap_step_matches_sequential_moves():
    # One offload step with its moves on two copy-engine streams plus the
    # compaction on the current stream: the result equals the closed forms
    # (victims land in the host buffer, revived blocks come from the other host
    # buffer, compaction copies src -> dst); overlapping id sets are rejected.
    pool = _pool(L=2, blocks=24, seed=5)
    before = _np(pool).reshape(2 * pool.size(1), pool.size(2), -1).copy()
    mover = BlockMover(pool)
    out_ids, in_ids, src, dst = [3, 17, 8], [0, 21, 12], [5, 6, 22, 1], [9, 10, 2, 23]
    shape = (3,) + tuple(pool[:, :, 0].shape)
    host_out = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
    g = torch.Generator().manual_seed(6)
    host_in = torch.randn(shape, generator=g).to(torch.bfloat16).pin_memory()
    print("[blocks] overlapped swap", flush=True)
    mover.swap(out_ids, host_out, in_ids, host_in, src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(_np(host_out).reshape(3, *before.shape[:1], -1),
                          ko.block_gather(before, out_ids))
    expect = before.copy()
    ko.block_scatter(expect, in_ids, _np(host_in).reshape(3, before.shape[0], -1))
    ko.block_copy(expect, src, dst)
    assert np.array_equal(_np(pool).reshape(expect.shape), expect)
    with pytest.raises(ValueError):
        mover.swap([1], host_out[:1], [1], host_in[:1])
