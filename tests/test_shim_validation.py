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


def _decode_meta(lens, page=32, width=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randperm(len(lens) * width, generator=g).view(len(lens), width).to(torch.int32)
    last = torch.tensor(lens) - 1
    slots = (ids.long().gather(1, (last // page).unsqueeze(1)).squeeze(1) * page + last % page)
    return slots.to(torch.int32), ids, torch.tensor(lens, dtype=torch.int32)


def test_append_contract_accepts_engine_decode_slots():
    from nanovllm_amd.kernels.paged_attention import check_append_contract
    sm, bt, cl = _decode_meta([1, 32, 33, 100, 128])
    check_append_contract(sm, bt, cl, 32, 20 * 32)
    # int64 slots given as negative (Python-index) forms are the same slots
    check_append_contract(sm.long() - 20 * 32, bt, cl, 32, 20 * 32)
    # empty rows append nothing and are not checked
    cl0 = cl.clone()
    cl0[1] = 0
    check_append_contract(sm, bt, cl0, 32, 20 * 32)


def test_append_contract_rejects_a_slot_off_the_last_position():
    from nanovllm_amd.kernels.paged_attention import check_append_contract
    sm, bt, cl = _decode_meta([40, 64, 90])
    sm[1] += 1
    with pytest.raises(AssertionError, match="row 1"):
        check_append_contract(sm, bt, cl, 32, 20 * 32)


def test_append_contract_rejects_a_slot_another_row_reads():
    from nanovllm_amd.kernels.paged_attention import check_append_contract
    sm, bt, cl = _decode_meta([40, 64, 90])
    bt[2, 0] = bt[0, 1]                 # row 2 reads row 0's last block at position 7
    with pytest.raises(AssertionError, match="row 2 reads row 0"):
        check_append_contract(sm, bt, cl, 32, 20 * 32)


def test_append_contract_allows_padded_rows_sharing_the_scratch_slot():
    from nanovllm_amd.kernels.paged_attention import check_append_contract
    sm, bt, cl = _decode_meta([40, 64])
    scratch = 19
    pad = torch.full((3, 4), scratch, dtype=torch.int32)
    bt = torch.cat([bt, pad])
    sm = torch.cat([sm, torch.full((3,), scratch * 32, dtype=torch.int32)])
    cl = torch.cat([cl, torch.ones(3, dtype=torch.int32)])
    check_append_contract(sm, bt, cl, 32, 20 * 32)


def test_attention_bound_is_the_bare_bound_below_eight():
    import numpy as np
    from helpers import MAX_ABS, attention_bound, half_ulp_bf16
    x = np.array([0.0, 1.0, 1.99, 4.0, 7.99, 8.0, 15.9, 16.0, -100.0])
    assert np.array_equal(half_ulp_bf16(x),
                          [0, 2**-8, 2**-8, 2**-6, 2**-6, 2**-5, 2**-5, 2**-4, 2**-2])
    b = attention_bound(x)
    assert np.all(b[:5] == MAX_ABS)
    assert np.allclose(b[5:], MAX_ABS + half_ulp_bf16(x[5:]))
    # half an ulp bounds torch's bf16 rounding of every fp32 value of a binade
    g = torch.Generator().manual_seed(1)
    v = torch.randn(100000, generator=g) * 50
    err = (v.to(torch.bfloat16).float() - v).abs().numpy()
    assert np.all(err <= half_ulp_bf16(v.numpy()))


def test_bound_layer_observes_k_v_before_the_store():
    """The calibration hook runs on every forward, before the append (the
    reference's forward pre-hook, model_runner.py:519-535)."""
    from nanovllm_amd.layers.attention import Attention
    from nanovllm_amd.utils.context import reset_context, set_context
    seen = []
    m = Attention(4, 128, 0.1, 2)
    m.k_cache = torch.zeros(2, 256, 2, 128, dtype=torch.int8)
    m.v_cache = torch.zeros_like(m.k_cache)
    m.kv_cache_is_int8 = True
    m.k_scale = m.v_scale = torch.ones(2, 128)
    m.kv_layer = 3
    m.kv_observe = lambda layer, k, v: seen.append((layer, k.shape, v.shape))
    set_context(False, slot_mapping=torch.zeros(5, dtype=torch.int32),
                context_lens=torch.ones(5, dtype=torch.int32),
                block_tables=torch.zeros(5, 1, dtype=torch.int32), max_context_len=1)
    try:
        with pytest.raises(RuntimeError, match="device"):
            m.forward(torch.zeros(5, 4, 128, dtype=torch.bfloat16),
                      torch.zeros(5, 2, 128, dtype=torch.bfloat16),
                      torch.zeros(5, 2, 128, dtype=torch.bfloat16))
    finally:
        reset_context()
    assert seen == [(3, (5, 2, 128), (5, 2, 128))]


def test_calibration_needs_a_per_channel_pool():
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    r = KVCacheRunner.__new__(KVCacheRunner)
    r.kv_int8 = "tokhead"
    with pytest.raises(ValueError, match="per-channel"):
        r.kv_calibrate_begin()
    r._calib = None
    with pytest.raises(RuntimeError, match="begin"):
        r.kv_calibrate_freeze()
