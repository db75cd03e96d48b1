"""KV append parity (bit-exact) — HIP store_kvcache vs the oracle."""
import numpy as np
import pytest
import torch

from helpers import bits
from nanovllm_amd.layers.attention import store_kvcache
from nanovllm_amd.workloads import decode_workload, uniform_lengths
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run_and_check(key, value, k_cache, v_cache, slots, label):
    print(f"[store] {label}: N={key.shape[0]} KVH={key.shape[1]} slots={slots.dtype}", flush=True)
    kc_ref = bits(k_cache).copy()
    vc_ref = bits(v_cache).copy()
    ko.store_kvcache(bits(key), bits(value), kc_ref, vc_ref, slots.cpu().numpy())
    store_kvcache(key, value, k_cache, v_cache, slots)
    torch.cuda.synchronize()
    assert np.array_equal(bits(k_cache), kc_ref), f"{label}: K cache differs"
    assert np.array_equal(bits(v_cache), vc_ref), f"{label}: V cache differs"


def test_decode_append_qwen3_06b_shape():
    # 0.6B-shaped layer: KVH=8, 64 blocks of 256, batch 8, ctx U[128, 1024].
    lens = uniform_lengths(8, 128, 1024, seed=11)
    wl = decode_workload(8, 16, 8, 64, lens, seed=12, device=DEV)
    _run_and_check(wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping, "decode-0.6B")


def test_decode_append_30b_shape_int64_slots():
    lens = uniform_lengths(64, 512, 4096, seed=21)
    wl = decode_workload(64, 32, 4, 1100, lens, seed=22, device=DEV)
    _run_and_check(wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping.long(),
                   "decode-30B-int64")


def test_prefill_append_strided_v_from_fused_qkv():
    # V is a strided view of a fused [N, (H + 2 KVH) * D] projection
    # (nanovllm/models/qwen3.py:77-81): row stride (H + 2 KVH) * D.
    g = torch.Generator().manual_seed(31)
    H, KVH, D, N, blocks = 32, 4, 128, 1084, 16
    qkv = torch.randn(N, (H + 2 * KVH) * D, generator=g).to(torch.bfloat16).to(DEV)
    k = qkv[:, H * D:(H + KVH) * D].view(N, KVH, D)
    v = qkv[:, (H + KVH) * D:].view(N, KVH, D)
    assert v.stride(0) == (H + 2 * KVH) * D
    k_cache = torch.randn(blocks, 256, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    v_cache = torch.randn(blocks, 256, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(blocks * 256, generator=g)[:N].to(torch.int32).to(DEV)
    _run_and_check(k, v, k_cache, v_cache, slots, "prefill-strided-v")


def test_negative_slot_wraps_like_index_put():
    g = torch.Generator().manual_seed(41)
    KVH, D = 2, 128
    k_cache = torch.zeros(3, 256, KVH, D, dtype=torch.bfloat16, device=DEV)
    v_cache = torch.zeros_like(k_cache)
    key = torch.randn(3, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    value = torch.randn(3, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    slots = torch.tensor([5, -1, 700], dtype=torch.int32, device=DEV)
    _run_and_check(key, value, k_cache, v_cache, slots, "negative-slot")
    assert torch.equal(k_cache.view(-1, KVH, D)[-1].cpu(), key[1].cpu())


def test_empty_append_is_a_noop():
    k_cache = torch.ones(2, 256, 2, 128, dtype=torch.bfloat16, device=DEV)
    v_cache = torch.ones_like(k_cache)
    key = torch.empty(0, 2, 128, dtype=torch.bfloat16, device=DEV)
    store_kvcache(key, key, k_cache, v_cache, torch.empty(0, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert bool((k_cache == 1).all()) and bool((v_cache == 1).all())


def test_stride_precondition_raises_assertion():
    k_cache = torch.zeros(2, 256, 2, 128, dtype=torch.bfloat16, device=DEV)
    key = torch.zeros(4, 2, 256, dtype=torch.bfloat16, device=DEV)[:, :, :128]
    with pytest.raises(AssertionError):
        store_kvcache(key, key, k_cache, k_cache, torch.zeros(4, dtype=torch.int32, device=DEV))

