"""Argument validation of the shim's newer entry points, on the CPU: the
errors the engine's own functions raise for the same misuse, before any
device work."""
import pytest
import torch

from nanovllm_amd.engine.kv_offload import HostBlockPool
from nanovllm_amd.engine.offload_pipeline import AsyncOffloader
from nanovllm_amd.kernels.paged_attention import paged_decode_append


def _decode_args(head_dim=128, page=256, dtype=torch.bfloat16, heads=32, kvh=4):
    q = torch.zeros(2, heads, head_dim, dtype=dtype)
    k = torch.zeros(2, kvh, head_dim, dtype=dtype)
    cache = torch.zeros(4, page, kvh, head_dim, dtype=dtype)
    return (q, k, k.clone(), cache, cache.clone(), torch.zeros(2, dtype=torch.int32),
            torch.zeros(2, 1, dtype=torch.int32), torch.ones(2, dtype=torch.int32), 0.1)


@pytest.mark.parametrize("bad", [dict(head_dim=64), dict(page=48), dict(heads=30),
                                 dict(dtype=torch.float16)])
def test_paged_decode_append_rejects_unsupported_shapes(bad):
    with pytest.raises(ValueError):
        paged_decode_append(*_decode_args(**bad))


def test_paged_decode_append_needs_device_tensors():
    with pytest.raises(RuntimeError, match="device"):
        paged_decode_append(*_decode_args())


def test_async_offloader_validates_before_the_device():
    pool = torch.zeros(2, 3, 4, 8, 2, 128, dtype=torch.bfloat16)
    host = HostBlockPool(2, tuple(pool[:, :, 0].shape), dtype=pool.dtype, pin=False)
    with pytest.raises(ValueError):
        AsyncOffloader(pool, host, copy_engine="sdma")
    with pytest.raises(AssertionError):
        AsyncOffloader(pool[:, :, :, :, :, :64], host)   # not contiguous
    with pytest.raises(RuntimeError, match="device"):
        AsyncOffloader(pool, host)
