"""Paged decode parity — HIP kvc_paged_decode vs the fp32 oracle.

Tolerance: max-abs 2e-2 and mean-abs 2e-3 against fp32 (bf16 outputs).
Cases follow the reference's kernel tests: NaN-poisoned page tails
(tests/archive/p5_paged_attention.py:40-63), the page-boundary length matrix
with scrambled pages (:66-95), plus GQA groupings, split-K lengths, empty
contexts and the full 32q/4kv batch-64 decode shape.
"""
import math

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, gathered_pool
from nanovllm_amd.kernels.paged_attention import paged_decode_attention
from nanovllm_amd.layers.attention import store_kvcache
from nanovllm_amd.workloads import decode_workload, uniform_lengths
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(params=["stream-k-lds", "fixed-chunk", "register"])
def decode_path(request, monkeypatch):
    """Every decode launch form: the stream-K launch with LDS-staged segments
    (the default), the fixed-chunk launch of one workgroup per (row, chunk)
    (KVC_DECODE_STREAMK=0), and the stream-K launch with register segments
    for every grouping (KVC_DECODE_LDS=0)."""
    monkeypatch.setenv("KVC_DECODE_STREAMK", "0" if request.param == "fixed-chunk" else "1")
    monkeypatch.setenv("KVC_DECODE_LDS", "0" if request.param == "register" else "1")
    return request.param


def _check(q, k_cache, v_cache, block_tables, lens, scale, label):
    print(f"[decode] {label}: B={q.shape[0]} H={q.shape[1]} KVH={k_cache.shape[2]} "
          f"max_ctx={int(lens.max()) if lens.numel() else 0}", flush=True)
    out = paged_decode_attention(q, k_cache, v_cache, block_tables, lens, scale,
                                 int(lens.max()) if lens.numel() else 0)
    torch.cuda.synchronize()
    kc, bt = gathered_pool(k_cache, block_tables)
    vc, _ = gathered_pool(v_cache, block_tables)
    ref = ko.paged_decode_ref(bits(q), ko.bf16_to_f32(bits(kc)), ko.bf16_to_f32(bits(vc)), bt,
                              lens.cpu().numpy(), scale)
    return assert_attention_close(out, ref, label)


def test_small_poison_tail(decode_path):
    torch.manual_seed(20261026)
    page = 256
    lengths = torch.tensor([127, 256, 385, 512], dtype=torch.int32, device=DEV)
    block_tables = torch.tensor([[7, 0], [3, 0], [6, 1], [4, 2]], dtype=torch.int32, device=DEV)
    k_cache = torch.randn(8, page, 2, 128, dtype=torch.bfloat16, device=DEV)
    v_cache = torch.randn_like(k_cache)
    q = torch.randn(4, 16, 128, dtype=torch.bfloat16, device=DEV)
    for row, length in enumerate(lengths.cpu().tolist()):
        tail = length % page
        if tail:
            page_id = int(block_tables[row, length // page])
            k_cache[page_id, tail:] = float("nan")
            v_cache[page_id, tail:] = float("nan")
    out_max, _ = _check(q, k_cache, v_cache, block_tables, lengths, 128 ** -0.5, "poison-tail")
    assert out_max <= 2e-2


def test_page_boundary_matrix(decode_path):
    torch.manual_seed(20261027)
    lengths_cpu = [255, 256, 257, 511, 512, 513, 2047, 2048, 2049]
    page = 256
    per_row = [math.ceil(n / page) for n in lengths_cpu]
    bt = torch.zeros(len(lengths_cpu), max(per_row), dtype=torch.int32)
    nxt = 0
    for row, cnt in enumerate(per_row):
        pages = list(range(nxt, nxt + cnt))
        pages[::2] = list(reversed(pages[::2]))
        bt[row, :cnt] = torch.tensor(pages, dtype=torch.int32)
        nxt += cnt
    k_cache = torch.randn(nxt, page, 2, 128, dtype=torch.bfloat16, device=DEV)
    v_cache = torch.randn_like(k_cache)
    q = torch.randn(len(lengths_cpu), 16, 128, dtype=torch.bfloat16, device=DEV)
    for row, n in enumerate(lengths_cpu):
        tail = n % page
        if tail:
            pid = int(bt[row, n // page])
            k_cache[pid, tail:] = float("nan")
            v_cache[pid, tail:] = float("nan")
    lens = torch.tensor(lengths_cpu, dtype=torch.int32, device=DEV)
    _check(q, k_cache, v_cache, bt.to(DEV), lens, 128 ** -0.5, "page-boundary")


@pytest.mark.parametrize("heads,kv_heads", [(16, 8), (32, 4), (32, 32), (32, 2), (64, 2), (12, 4)])
def test_gqa_groupings(heads, kv_heads, decode_path):
    lens = uniform_lengths(6, 1, 1500, seed=heads * 100 + kv_heads)
    wl = decode_workload(6, heads, kv_heads, 48, lens, seed=7, device=DEV)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale,
           f"gqa-{heads}/{kv_heads}")


def test_qwen3_06b_shape_after_append():
    # 0.6B-shaped layer: 16 q / 8 kv heads, 64 blocks, batch 8, ctx U[128, 1024];
    # one appended token per sequence, then decode with scale 1/sqrt(128).
    lens = uniform_lengths(8, 128, 1024, seed=101)
    wl = decode_workload(8, 16, 8, 64, lens, seed=102, device=DEV)
    store_kvcache(wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale, "0.6B-step")


def test_long_context_split_k(decode_path):
    lens = [32768, 20000, 4097, 1]
    wl = decode_workload(4, 32, 4, 256, lens, seed=9, device=DEV)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale, "long-split-k")


def test_zero_length_context_gives_nan_row(decode_path):
    lens = [0, 300]
    wl = decode_workload(2, 32, 4, 8, [1, 300], seed=3, device=DEV)
    wl.context_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale, "zero-ctx")


def test_full_30b_decode_shape_batch64(decode_path):
    # 32 q / 4 kv heads, batch 64, ctx U[512, 4096], non-contiguous tables over
    # an 8192-block pool, one appended token per sequence.
    lens = uniform_lengths(64, 512, 4096, seed=2)
    wl = decode_workload(64, 32, 4, 8192, lens, seed=3, device=DEV, pool_device_fill=True)
    store_kvcache(wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale, "30B-b64")


def test_strided_q_and_graph_width_tables():
    # q as a strided view and block tables wider than any context (a captured
    # graph's padded table): entries past the context are never read.
    lens = uniform_lengths(5, 100, 900, seed=77)
    wl = decode_workload(5, 32, 4, 40, lens, seed=78, device=DEV)
    wide = torch.full((5, 17), 10**6, dtype=torch.int32, device=DEV)
    wide[:, :wl.block_tables.size(1)] = wl.block_tables
    wide = torch.where(wide == -1, torch.full_like(wide, 10**6), wide)
    big = torch.randn(5, 48, 128, dtype=torch.bfloat16, device=DEV)
    big[:, 8:40] = wl.q
    q = big[:, 8:40]
    assert not q.is_contiguous()
    out = paged_decode_attention(q, wl.k_cache, wl.v_cache, wide, wl.context_lens, wl.scale, 0)
    ref = paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens,
                                 wl.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) or float((out.float() - ref.float()).abs().max()) <= 2e-2


def test_shape_errors_match_reference():
    q = torch.zeros(2, 16, 64, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(4, 256, 2, 64, dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros(2, 1, dtype=torch.int32, device=DEV)
    lens = torch.ones(2, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        paged_decode_attention(q, kc, kc, bt, lens, 1.0, 1)
    with pytest.raises(ValueError):
        paged_decode_attention(q[:, :, None], kc, kc, bt, lens, 1.0, 1)
    q2 = torch.zeros(2, 15, 128, dtype=torch.bfloat16, device=DEV)
    kc2 = torch.zeros(4, 256, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        paged_decode_attention(q2, kc2, kc2, bt, lens, 1.0, 1)


@pytest.mark.parametrize("page", [32, 64, 128])
def test_pages_smaller_than_256(page, decode_path):
    lens = [1, page - 1, page, page + 1, 5 * page + 3, 4000]
    blocks = sum((n + page - 1) // page for n in lens) + 4
    wl = decode_workload(len(lens), 32, 4, blocks, lens, seed=page, device=DEV, page=page)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale,
           f"page-{page}")


@pytest.mark.parametrize("case", ["b64x4096", "ragged-with-empty", "int64-negative-slots",
                                  "unaligned-key-fallback", "two-kv-heads", "eight-kv-heads"])
def test_decode_append_equals_store_then_decode(case, decode_path, deterministic_decode):
    """paged_decode_append (the store inside the decode launch where the
    layout allows) against store_kvcache then paged_decode_attention: the
    same output bits and the same pool bytes."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_append
    heads, kvh = {"two-kv-heads": (16, 2), "eight-kv-heads": (16, 8)}.get(case, (32, 4))
    if case == "b64x4096":
        lens, nb = [4096] * 64, 1100
    elif case == "ragged-with-empty":
        lens, nb = [1, 0, 33, 4096, 257, 0, 9000, 31], 80
    else:
        lens, nb = uniform_lengths(20, 1, 5000, seed=61), 600
    wl = decode_workload(len(lens), heads, kvh, nb, [max(1, n) for n in lens], seed=len(lens),
                         device=DEV, pool_device_fill=True)
    wl.context_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    slots = wl.slot_mapping.clone()
    num_slots = wl.k_cache.size(0) * wl.k_cache.size(1)
    if case == "int64-negative-slots":
        slots = slots.long()
        slots[::3] -= num_slots            # wraps back to the same slot
    key, value = wl.new_k, wl.new_v
    if case == "unaligned-key-fallback":
        big = torch.randn(len(lens), kvh * 128 + 4, dtype=torch.bfloat16, device=DEV)
        big[:, 4:] = key.reshape(len(lens), -1)
        key = big[:, 4:].view(len(lens), kvh, 128)   # 8-byte aligned rows
    print(f"[decode] append fused {case}: B={len(lens)}", flush=True)
    kc0, vc0 = wl.k_cache.clone(), wl.v_cache.clone()
    store_kvcache(key, value, kc0, vc0, slots)
    ref = paged_decode_attention(wl.q, kc0, vc0, wl.block_tables, wl.context_lens, wl.scale, 0)
    kc1, vc1 = wl.k_cache.clone(), wl.v_cache.clone()
    out = paged_decode_append(wl.q, key, value, kc1, vc1, slots, wl.block_tables,
                              wl.context_lens, wl.scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(ref)), "outputs differ from store + decode"
    assert np.array_equal(bits(kc1), bits(kc0)) and np.array_equal(bits(vc1), bits(vc0))


# The reference's published decode grid (benchmarks/archive/P15-pd-autotune.md:
# 10-15) is at the engine's 2-way tensor-parallel shard, 16 q / 2 kv heads:
# batch 1 / 8 / 16 / 32 x context 512-4096; plus the batch-64 x 4096 step.
@pytest.mark.parametrize("batch,ctx", [(1, 512), (1, 4096), (8, 1024), (16, 2048), (32, 4096),
                                       (64, 4096)])
def test_tp2_shard_grid(batch, ctx, decode_path):
    nb = batch * ctx // 256 + 8
    wl = decode_workload(batch, 16, 2, nb, [ctx] * batch, seed=batch * 7 + ctx, device=DEV,
                         pool_device_fill=True)
    store_kvcache(wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping)
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale,
           f"tp2 b{batch} ctx{ctx}")


def test_tp2_shard_ragged_fused_append(deterministic_decode):
    """16q/2kv, batch 64 x U[512, 4096] over an 8192-block pool: the decode
    step with the append fused (2-kv-head LDS segments) gives the same output
    bits and pool bytes as store + decode, and matches the oracle."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_append
    lens = uniform_lengths(64, 512, 4096, seed=21)
    wl = decode_workload(64, 16, 2, 8192, lens, seed=22, device=DEV, pool_device_fill=True)
    kc0, vc0 = wl.k_cache.clone(), wl.v_cache.clone()
    store_kvcache(wl.new_k, wl.new_v, kc0, vc0, wl.slot_mapping)
    ref = paged_decode_attention(wl.q, kc0, vc0, wl.block_tables, wl.context_lens, wl.scale, 0)
    out = paged_decode_append(wl.q, wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping,
                              wl.block_tables, wl.context_lens, wl.scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(ref))
    assert torch.equal(wl.k_cache.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(wl.v_cache.view(torch.int16), vc0.view(torch.int16))
    _check(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens, wl.scale,
           "tp2 ragged after fused append")


def test_decode_stamps_record_every_workgroup(monkeypatch):
    """KVC_DECODE_STAMPS=1: every workgroup of the stream-K decode launch
    records a start and an end stamp (end >= start, all within the launch),
    kvc_decode_stamps reports one pair per workgroup, and the outputs are the
    same bits as without the stamps."""
    import ctypes
    from nanovllm_amd import _native as nat
    lens = uniform_lengths(12, 1, 3000, seed=4)
    wl = decode_workload(len(lens), 32, 4, 200, lens, seed=6, device=DEV)
    monkeypatch.setenv("KVC_DECODE_STREAMK", "1")
    monkeypatch.delenv("KVC_DECODE_STAMPS", raising=False)
    ref = paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.block_tables,
                                 wl.context_lens, wl.scale, max(lens))
    monkeypatch.setenv("KVC_DECODE_STAMPS", "1")
    print("[decode-stamps] B=12", flush=True)
    out = paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.block_tables,
                                 wl.context_lens, wl.scale, max(lens))
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(ref))
    buf = (ctypes.c_ulonglong * (2 * 4096))()
    n, khz = ctypes.c_int(0), ctypes.c_int(0)
    nat.call("kvc_decode_stamps", ctypes.addressof(buf), 4096, ctypes.addressof(n),
             ctypes.addressof(khz))
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert n.value == cus and khz.value > 0
    starts = [buf[2 * v] for v in range(n.value)]
    ends = [buf[2 * v + 1] for v in range(n.value)]
    assert all(s > 0 and e >= s for s, e in zip(starts, ends))
    assert (max(ends) - min(starts)) / khz.value < 1000.0  # under a second
