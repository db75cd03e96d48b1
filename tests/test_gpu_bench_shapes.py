"""Parity at the exact shapes and inputs the benchmark lines time.

* The headline step: paged_decode_append at batch 64 x 4096 over the
  8192-block pool, with bench.py's seeds — outputs against the fp32 oracle
  (nanovllm/kernels/paged_attention.py:193-245 semantics), pool bytes against
  oracle.store_kvcache (nanovllm/layers/attention.py:9-30), and every block
  the step must not touch unchanged.
* The int8 workload as written: batch 16 x 32768, K ~ N(0,1) with 1 % of
  entries x20 and V ~ N(0,1), every token appended through the per-token-head
  quantiser (scripts/archive/p14_int8_kv_probe.py:37-41) — codes and scales
  bit-exact against the oracle's quantiser, the decode against the fp32
  oracle over the stored codes.
* The offload / compaction step at the scaled pool (8192 blocks of
  [2, 48, 256, 4, 128] bf16 = 192 GiB, byte offsets far above 2^32): 128
  blocks out to pinned memory, 128 back in, a 1024-block compaction
  (nanovllm/engine/model_runner.py:284-305 byte moves).  Every 4-byte word of
  the pool carries a tag derived from (plane, block, word); the expected tags
  of moved, revived and untouched blocks are regenerated on the device and
  compared with torch.equal, plane by plane.

Tolerance for attention: max-abs 2e-2 (plus half a bf16 ulp where that is
larger) and mean-abs 2e-3 against fp32.
"""
import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits
from nanovllm_amd.kernels.kv_int8 import store_kvcache_int8_tokhead
from nanovllm_amd.kernels.paged_attention import paged_decode_append, paged_decode_attention
from nanovllm_amd.workloads import decode_workload, int8_tokhead_decode_workload
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _local_tables(bt: torch.Tensor):
    """The blocks a table references, and the table renumbered 0.. over them."""
    used = torch.unique(bt[bt >= 0])
    remap = torch.full((int(used.max()) + 1,), -1, dtype=torch.int64, device=bt.device)
    remap[used.long()] = torch.arange(used.numel(), device=bt.device)
    local = torch.where(bt >= 0, remap[bt.clamp(min=0).long()], torch.full_like(bt.long(), -1))
    return used, local


def test_headline_decode_append_b64x4096_pool8192():
    """bench.py's default step: decode_workload(64, 32, 4, 8192, [4096] * 64,
    seed=3, pool_device_fill=True), then one paged_decode_append."""
    lens = [4096] * 64
    wl = decode_workload(64, 32, 4, 8192, lens, seed=3, device=DEV, pool_device_fill=True)
    print("[bench-shapes] headline decode append 64 x 4096, 8192-block pool", flush=True)
    used, local_bt = _local_tables(wl.block_tables)
    assert used.numel() == 64 * 16
    untouched = torch.ones(wl.k_cache.size(0), dtype=torch.bool, device=DEV)
    untouched[used.long()] = False
    k_rest = wl.k_cache[untouched].clone()
    v_rest = wl.v_cache[untouched].clone()
    kb = bits(wl.k_cache.index_select(0, used))
    vb = bits(wl.v_cache.index_select(0, used))
    out = paged_decode_append(wl.q, wl.new_k, wl.new_v, wl.k_cache, wl.v_cache, wl.slot_mapping,
                              wl.block_tables, wl.context_lens, wl.scale)
    torch.cuda.synchronize()
    # pool bytes: the oracle's store on the referenced blocks, nothing else moved
    page = wl.k_cache.size(1)
    last = np.array(lens) - 1
    bt_h = wl.block_tables.cpu().numpy().astype(np.int64)
    # the engine's decode slots (model_runner.py:685), as the fused append requires
    assert np.array_equal(wl.slot_mapping.cpu().numpy(),
                          bt_h[np.arange(64), last // page] * page + last % page)
    local_slots = local_bt.cpu().numpy()[np.arange(64), last // page] * page + last % page
    ko.store_kvcache(bits(wl.new_k), bits(wl.new_v), kb, vb, local_slots)
    assert np.array_equal(bits(wl.k_cache.index_select(0, used)), kb), "K pool bytes differ"
    assert np.array_equal(bits(wl.v_cache.index_select(0, used)), vb), "V pool bytes differ"
    assert torch.equal(wl.k_cache[untouched].view(torch.int16), k_rest.view(torch.int16))
    assert torch.equal(wl.v_cache[untouched].view(torch.int16), v_rest.view(torch.int16))
    del k_rest, v_rest
    ref = ko.paged_decode_ref(bits(wl.q), ko.bf16_to_f32(kb), ko.bf16_to_f32(vb),
                              local_bt.cpu().numpy(), np.array(lens), wl.scale)
    assert_attention_close(out, ref, "headline 64x4096 decode append")


def test_config4_int8_tokhead_b16x32k_outliers():
    """The int8 line's workload and step: history appended through the
    quantiser, then the step in one call (quantise-on-append inside the
    decode launch)."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_append_int8_tokhead
    lens = [32768] * 16
    wl = int8_tokhead_decode_workload(16, 32, 4, 2048 + 16, lens, seed=3, device=DEV,
                                      keep_raw=True)
    print("[bench-shapes] int8 per-token-head 16 x 32768 with x20 key outliers", flush=True)
    out = paged_decode_append_int8_tokhead(wl.q, wl.new_k, wl.new_v, wl.k_cache, wl.v_cache,
                                           wl.k_scale, wl.v_scale, wl.slot_mapping,
                                           wl.block_tables, wl.context_lens, wl.scale)
    torch.cuda.synchronize()
    kvh, d = 4, 128
    flat_k = wl.k_cache.view(-1, kvh, d)
    flat_v = wl.v_cache.view(-1, kvh, d)
    flat_ks = wl.k_scale.view(-1, kvh)
    flat_vs = wl.v_scale.view(-1, kvh)
    # codes and scales: every token of the step, and a seeded sample of the history
    g = torch.Generator().manual_seed(11)
    pick = torch.randperm(wl.history_slots.numel(), generator=g)[:65536].to(DEV)
    cases = [("step", wl.new_k, wl.new_v, wl.slot_mapping.long()),
             ("history", wl.raw_k[pick], wl.raw_v[pick], wl.history_slots[pick].long())]
    saturated = 0
    for name, xk, xv, slots in cases:
        for side, x, codes, scales in (("K", xk, flat_k, flat_ks), ("V", xv, flat_v, flat_vs)):
            want_c, want_s = ko.quant_tokhead(bits(x))
            got_c = codes[slots].cpu().numpy()
            got_s = scales[slots].cpu().numpy()
            assert np.array_equal(got_c, want_c), f"{name} {side} codes differ"
            assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32)), \
                f"{name} {side} scales differ"
            if side == "K":
                saturated += int((np.abs(want_c) == 127).sum())
    print(f"[bench-shapes] int8 codes/scales bit-exact; {saturated} saturated K codes in the "
          f"sample", flush=True)
    assert saturated > 0
    # decode against the fp32 oracle over the stored codes, one sequence at a time
    got = out.float().cpu().numpy()
    worst = 0.0
    for i in range(16):
        row_bt = wl.block_tables[i:i + 1]
        used, local = _local_tables(row_bt)
        kf = ko.kv_float(wl.k_cache.index_select(0, used).cpu().numpy(), "int8_tokhead",
                         wl.k_scale.index_select(0, used).cpu().numpy())
        vf = ko.kv_float(wl.v_cache.index_select(0, used).cpu().numpy(), "int8_tokhead",
                         wl.v_scale.index_select(0, used).cpu().numpy())
        ref = ko.paged_decode_ref(bits(wl.q[i:i + 1]), kf, vf, local.cpu().numpy(),
                                  np.array([lens[i]]), wl.scale)
        mx, _ = assert_attention_close(out[i:i + 1], ref, f"int8 16x32k row {i}")
        worst = max(worst, mx)
    assert got.shape == (16, 32, 128)
    print(f"[bench-shapes] int8 decode max_abs over rows {worst:.3e}", flush=True)


def _plane_tag(p: int, salt: int) -> int:
    return (p * 2654435761 + salt * 40503 + 12345) & 0x7FFFFFFF


def _tags(p: int, blocks: torch.Tensor, words: torch.Tensor, salt: int = 0) -> torch.Tensor:
    """int32 [len(blocks), words] tag of each 4-byte word of plane p."""
    return torch.bitwise_xor(blocks.to(torch.int32).unsqueeze(1) * words.numel()
                             + words.unsqueeze(0), _plane_tag(p, salt))


def test_config5_swap_compaction_scaled_pool_tags():
    """bench.py --workload swap's step (BlockMover.swap with the bench's seeded
    ids) on the 8192 x 24 MiB pool, checked word by word on the device."""
    L, kvh, NB, active, n_swap, n_copy = 48, 4, 8192, 512, 128, 1024
    item_bytes = 2 * L * 256 * kvh * 128 * 2
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info()
    if free < NB * item_bytes + (16 << 30):
        pytest.skip(f"needs {NB * item_bytes / 2**30:.0f} GiB + 16 GiB free on the device "
                    f"({free / 2**30:.0f} GiB free)")
    from nanovllm_amd.engine.kv_runner import BlockMover
    print("[bench-shapes] offload/compaction step on the 192 GiB pool", flush=True)
    pool = torch.empty(2, L, NB, 256, kvh, 128, device=DEV, dtype=torch.bfloat16)
    planes = 2 * L
    words = torch.arange(item_bytes // planes // 4, dtype=torch.int32, device=DEV)
    pv = pool.view(torch.int32).view(planes, NB, words.numel())
    all_ids = torch.arange(NB, device=DEV)
    for p in range(planes):
        pv[p] = _tags(p, all_ids, words)
    mover = BlockMover(pool)
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(NB, generator=g).tolist()
    victims = perm[:n_swap]
    revived = perm[active:active + n_swap]
    src = perm[active + n_swap:active + n_swap + n_copy]
    dst = perm[active + n_swap + n_copy:active + n_swap + 2 * n_copy]
    host_out = torch.empty((n_swap,) + mover.item_shape, dtype=pool.dtype, pin_memory=True)
    host_in = torch.empty((n_swap,) + mover.item_shape, dtype=pool.dtype, pin_memory=True)
    hin = host_in.view(torch.int32).view(n_swap, planes, words.numel())
    rev_t = torch.tensor(revived, device=DEV)
    for p in range(planes):
        hin[:, p] = _tags(p, rev_t, words, salt=1).cpu()
    mover.swap(victims, host_out, revived, host_in, src, dst)
    torch.cuda.synchronize()
    # the offloaded blocks' bytes in the pinned buffer
    hout = host_out.view(torch.int32).view(n_swap, planes, words.numel())
    vic_t = torch.tensor(victims, device=DEV)
    for p in range(planes):
        assert torch.equal(hout[:, p].to(DEV), _tags(p, vic_t, words)), f"d2h plane {p}"
    # the pool: revived blocks from the host, compaction targets from their
    # sources, everything else (victims included) unchanged
    src_t, dst_t = torch.tensor(src, device=DEV), torch.tensor(dst, device=DEV)
    for p in range(planes):
        want = _tags(p, all_ids, words)
        want[rev_t] = _tags(p, rev_t, words, salt=1)
        want[dst_t] = _tags(p, src_t, words)
        assert torch.equal(pv[p], want), f"pool plane {p}"
        del want
    print(f"[bench-shapes] swap step bit-exact on all {planes} planes of the "
          f"{pool.numel() * 2 / 2**30:.0f} GiB pool", flush=True)
    del pool, pv, host_out, host_in
    torch.cuda.empty_cache()
