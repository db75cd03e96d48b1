"""Paged GQA decode attention on MI355X (libkvc `kvc_paged_decode`).

Drop-in for nanovllm/kernels/paged_attention.py:193-245: same signature, same
output allocation (torch.empty_like(q)), same ValueError conditions, and the
same graph-capture contract (the loop bound is the device-side context_lens;
max_context_len is accepted and ignored, paged_attention.py:212-214).

Differences that only widen what is accepted:
  * page sizes that are multiples of 32 (the reference insists on 256);
  * int8 pools in either encoding: per-channel read scales [KVH, D] with the
    bf16 outlier side pool (the engine's current layout), or per-token-head
    scales [blocks, page, KVH] (k_scale.dim() == 3);
  * the side pool is used without the reference's host sync on
    int(head_n_out.max()) (paged_attention.py:218): the kernel reads
    head_n_out on the device.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from .. import _native as nat


def _check_append_enabled() -> bool:
    """KVC_CHECK_APPEND=1 (read at every call): paged_decode_append checks on
    the host that the decode slots satisfy the fused append's contract before
    it launches (reads the metadata back, so it synchronises; for debugging,
    never under capture)."""
    return os.environ.get("KVC_CHECK_APPEND", "0") == "1"


def set_paged_config(value: str | None) -> None:
    """Accepted for API compatibility (paged_attention.py:50); the HIP kernel
    plans its own split-K launch from the batch shape."""
    del value


def _kv_encoding(k_cache: torch.Tensor, k_scale: torch.Tensor | None) -> int:
    if k_cache.dtype == torch.int8:
        if k_scale is None:
            raise ValueError("an int8 KV pool needs k_scale/v_scale")
        return nat.KVC_KV_INT8_TOKHEAD if k_scale.dim() == 3 else nat.KVC_KV_INT8_CHAN
    if k_cache.dtype != torch.bfloat16:
        raise ValueError(f"KV pool dtype {k_cache.dtype} is not supported (bf16 or int8)")
    if k_scale is not None:
        raise ValueError("k_scale given for a bf16 KV pool")
    return nat.KVC_KV_BF16


def paged_decode_attention(
    q, k_cache, v_cache, block_tables, context_lens, scale, max_context_len,
    k_scale=None, v_scale=None, side_k=None, side_v=None,
    out_idx2d=None, head_n_out=None,
):
    if q.ndim != 3 or k_cache.ndim != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("expected q=[batch,heads,dim], kv=[pages,page,kv_heads,dim]")
    batch, num_heads, head_dim = q.shape
    page_size = k_cache.size(1)
    num_kv_heads = k_cache.size(2)
    if head_dim != 128 or page_size % 32 or num_heads % num_kv_heads:
        raise ValueError(
            "paged decode requires head_dim=128, page_size a multiple of 32 and "
            "GQA-divisible heads")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16 (got {q.dtype})")
    nat.require_device(q, k_cache, v_cache, block_tables, context_lens)
    enc = _kv_encoding(k_cache, k_scale)
    if q.stride(2) != 1:
        q = q.contiguous()
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise AssertionError("KV pools must be contiguous [pages, page, kv_heads, dim]")
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
        context_lens = context_lens.to(torch.int32).contiguous()
    del max_context_len
    output = torch.empty_like(q)
    if output.stride(2) != 1:
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if batch == 0:
        return output
    has_side = enc == nat.KVC_KV_INT8_CHAN and side_k is not None and head_n_out is not None
    if enc == nat.KVC_KV_INT8_TOKHEAD:
        k_scale = k_scale.contiguous()
        v_scale = v_scale.contiguous()
    elif enc == nat.KVC_KV_INT8_CHAN:
        k_scale = k_scale.to(torch.float32).contiguous()
        v_scale = v_scale.to(torch.float32).contiguous()
    max_blocks = block_tables.size(1)
    ws_bytes = nat.query("kvc_paged_decode_workspace_bytes", batch, num_heads, num_kv_heads,
                         head_dim, page_size, max_blocks)
    ws = nat.workspace(ws_bytes, q.device)
    nat.call(
        "kvc_paged_decode",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.size(0), page_size, num_kv_heads,
        head_dim, enc,
        nat.ptr(k_scale), nat.ptr(v_scale),
        nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
        nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
        side_k.size(-1) if has_side else 0,
        block_tables.data_ptr(), block_tables.stride(0), max_blocks,
        context_lens.data_ptr(), batch, num_heads, float(scale),
        output.data_ptr(), output.stride(0), output.stride(1),
        nat.ptr(ws), ws_bytes, nat.stream_of(q),
    )
    return output


def check_append_contract(slot_mapping, block_tables, context_lens, page_size: int,
                          num_slots: int) -> None:
    """The decode-slot contract the fused append relies on, checked on the
    host (AssertionError naming the first offending row):
    * every row b with context_lens[b] > 0 appends at the slot of its own
      last position, block_tables[b][(ctx-1) // page] * page + (ctx-1) % page
      (nanovllm/engine/model_runner.py:685), after the same negative-slot
      wrap the store applies;
    * no row reads another row's new slot at a position before its own last
      one (a row whose last position is that slot replaces it with its own
      token, as the padded scratch rows of a graph replay do)."""
    sm = slot_mapping.detach().to("cpu", torch.int64).numpy()
    bt = block_tables.detach().to("cpu", torch.int64).numpy()
    cl = context_lens.detach().to("cpu", torch.int64).numpy()
    sm = np.where(sm < 0, sm + num_slots, sm)
    live = np.nonzero(cl > 0)[0]
    for b in live:
        last = int(cl[b]) - 1
        blk = int(bt[b, last // page_size])
        want = blk * page_size + last % page_size
        assert int(sm[b]) == want, (
            f"paged_decode_append: row {b} appends at slot {int(sm[b])}, but its last position "
            f"{last} is slot {want} (block {blk}); use store_kvcache + paged_decode_attention")
    for b in live:
        blk, off = divmod(int(sm[b]), page_size)
        for c in live:
            if c == b:
                continue
            nblk = (int(cl[c]) + page_size - 1) // page_size
            hits = np.nonzero(bt[c, :nblk] == blk)[0]
            pos = hits * page_size + off
            early = pos[pos < int(cl[c]) - 1]
            assert early.size == 0, (
                f"paged_decode_append: row {c} reads row {b}'s new slot {int(sm[b])} at "
                f"position {int(early[0])} before its own last one")


def paged_decode_append(q, key, value, k_cache, v_cache, slot_mapping, block_tables,
                        context_lens, scale):
    """The decode step's KV work on a bf16 pool in one call:
    store_kvcache(key, value, k_cache, v_cache, slot_mapping) then
    paged_decode_attention(q, ...) (nanovllm/layers/attention.py:9-30,
    :239-245), with the store inside the decode launch where the layout
    allows.  That needs the engine's decode slots (slot_mapping[b] is
    position context_lens[b] - 1 of row b, read by no other row).  Same
    results and pool contents as the two calls."""
    if q.ndim != 3 or key.ndim != 3 or value.shape != key.shape or k_cache.ndim != 4 \
            or v_cache.shape != k_cache.shape:
        raise ValueError("expected q=[batch,heads,dim], key/value=[batch,kv_heads,dim], "
                         "kv=[pages,page,kv_heads,dim]")
    batch, num_heads, head_dim = q.shape
    page_size = k_cache.size(1)
    num_kv_heads = k_cache.size(2)
    if head_dim != 128 or page_size % 32 or num_heads % num_kv_heads:
        raise ValueError(
            "paged decode requires head_dim=128, page_size a multiple of 32 and "
            "GQA-divisible heads")
    if not (q.dtype == key.dtype == value.dtype == k_cache.dtype == torch.bfloat16):
        raise ValueError("paged_decode_append takes a bf16 pool and bf16 q/k/v")
    assert key.size(0) == batch and key.size(1) == num_kv_heads and slot_mapping.numel() == batch
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    nat.require_device(q, key, value, k_cache, v_cache, slot_mapping, block_tables, context_lens)
    if q.stride(2) != 1:
        q = q.contiguous()
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise AssertionError("KV pools must be contiguous [pages, page, kv_heads, dim]")
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
        context_lens = context_lens.to(torch.int32).contiguous()
    if slot_mapping.dtype == torch.int64:
        sb = 8
    else:
        slot_mapping = slot_mapping.to(torch.int32)
        sb = 4
    slot_mapping = slot_mapping.contiguous()
    output = torch.empty_like(q)
    if output.stride(2) != 1:
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if batch == 0:
        return output
    if _check_append_enabled():
        check_append_contract(slot_mapping, block_tables, context_lens, page_size,
                              k_cache.size(0) * page_size)
    max_blocks = block_tables.size(1)
    ws_bytes = nat.query("kvc_paged_decode_workspace_bytes", batch, num_heads, num_kv_heads,
                         head_dim, page_size, max_blocks)
    ws = nat.workspace(ws_bytes, q.device)
    qs, ks, vs, os_ = q.stride(), key.stride(), value.stride(), output.stride()
    nat.call(
        "kvc_paged_decode_append",
        q.data_ptr(), qs[0], qs[1],
        key.data_ptr(), ks[0], ks[1],
        value.data_ptr(), vs[0], vs[1],
        slot_mapping.data_ptr(), sb,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.size(0), page_size, num_kv_heads,
        head_dim, block_tables.data_ptr(), block_tables.stride(0), max_blocks,
        context_lens.data_ptr(), batch, num_heads, float(scale),
        output.data_ptr(), os_[0], os_[1],
        nat.ptr(ws), ws_bytes, nat.stream_of(q),
    )
    return output


def paged_decode_append_int8_tokhead(q, key, value, k_cache, v_cache, k_scale, v_scale,
                                     slot_mapping, block_tables, context_lens, scale):
    """The decode step over a per-token-head int8 pool in one call:
    store_kvcache_int8_tokhead(key, value, k_cache, v_cache, k_scale, v_scale,
    slot_mapping) then paged_decode_attention(q, ..., k_scale=k_scale,
    v_scale=v_scale) (scripts/archive/p14_int8_kv_probe.py:37-46), with the
    quantiser inside the decode launch where the layout allows (the engine's
    decode slots, as paged_decode_append).  Same codes, scales and outputs
    as the two calls."""
    if q.ndim != 3 or key.ndim != 3 or value.shape != key.shape or k_cache.ndim != 4 \
            or v_cache.shape != k_cache.shape:
        raise ValueError("expected q=[batch,heads,dim], key/value=[batch,kv_heads,dim], "
                         "kv=[pages,page,kv_heads,dim]")
    batch, num_heads, head_dim = q.shape
    page_size = k_cache.size(1)
    num_kv_heads = k_cache.size(2)
    if head_dim != 128 or page_size % 32 or num_heads % num_kv_heads:
        raise ValueError(
            "paged decode requires head_dim=128, page_size a multiple of 32 and "
            "GQA-divisible heads")
    if not (q.dtype == key.dtype == value.dtype == torch.bfloat16
            and k_cache.dtype == v_cache.dtype == torch.int8):
        raise ValueError("paged_decode_append_int8_tokhead takes an int8 pool and bf16 q/k/v")
    if k_scale.shape != k_cache.shape[:3] or v_scale.shape != k_scale.shape \
            or k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        raise ValueError("per-token-head scales are fp32 [pages, page, kv_heads]")
    assert key.size(0) == batch and key.size(1) == num_kv_heads and slot_mapping.numel() == batch
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    nat.require_device(q, key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping,
                       block_tables, context_lens)
    if q.stride(2) != 1:
        q = q.contiguous()
    if not (k_cache.is_contiguous() and v_cache.is_contiguous() and k_scale.is_contiguous()
            and v_scale.is_contiguous()):
        raise AssertionError("KV pools and scales must be contiguous")
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
        context_lens = context_lens.to(torch.int32).contiguous()
    if slot_mapping.dtype == torch.int64:
        sb = 8
    else:
        slot_mapping = slot_mapping.to(torch.int32)
        sb = 4
    slot_mapping = slot_mapping.contiguous()
    output = torch.empty_like(q)
    if output.stride(2) != 1:
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if batch == 0:
        return output
    if _check_append_enabled():
        check_append_contract(slot_mapping, block_tables, context_lens, page_size,
                              k_cache.size(0) * page_size)
    max_blocks = block_tables.size(1)
    ws_bytes = nat.query("kvc_paged_decode_workspace_bytes", batch, num_heads, num_kv_heads,
                         head_dim, page_size, max_blocks)
    ws = nat.workspace(ws_bytes, q.device)
    nat.call(
        "kvc_paged_decode_append_int8",
        q.data_ptr(), q.stride(0), q.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        slot_mapping.data_ptr(), sb,
        k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
        k_cache.size(0), page_size, num_kv_heads, head_dim,
        block_tables.data_ptr(), block_tables.stride(0), max_blocks,
        context_lens.data_ptr(), batch, num_heads, float(scale),
        output.data_ptr(), output.stride(0), output.stride(1),
        nat.ptr(ws), ws_bytes, nat.stream_of(q),
    )
    return output


def paged_decode_append_int8_chan(q, key, value, k_cache, v_cache, k_scale, v_scale,
                                  k_dscale, v_dscale, side_k, side_v, out_idx2d, head_n_out,
                                  slot_mapping, block_tables, context_lens, scale):
    """The decode step over a per-channel int8 pool in one call:
    store_kvcache_int8(key, value, k_cache, v_cache, k_scale, v_scale,
    side_k, side_v, out_idx2d, head_n_out, slot_mapping) then
    paged_decode_attention(q, ..., k_scale=k_dscale, v_scale=v_dscale,
    side_k=side_k, side_v=side_v, out_idx2d=out_idx2d,
    head_n_out=head_n_out) (the engine's int8 step,
    nanovllm/layers/attention.py:130-177 with nanovllm/kernels/kv_int8.py:
    29-93 and paged_attention.py:101-172).  Same codes, side values and
    outputs as the two calls."""
    if q.ndim != 3 or key.ndim != 3 or value.shape != key.shape or k_cache.ndim != 4 \
            or v_cache.shape != k_cache.shape:
        raise ValueError("expected q=[batch,heads,dim], key/value=[batch,kv_heads,dim], "
                         "kv=[pages,page,kv_heads,dim]")
    batch, num_heads, head_dim = q.shape
    pages, page_size, num_kv_heads = k_cache.shape[:3]
    if head_dim != 128 or page_size % 32 or num_heads % num_kv_heads:
        raise ValueError(
            "paged decode requires head_dim=128, page_size a multiple of 32 and "
            "GQA-divisible heads")
    if not (q.dtype == key.dtype == value.dtype == torch.bfloat16
            and k_cache.dtype == v_cache.dtype == torch.int8):
        raise ValueError("paged_decode_append_int8_chan takes an int8 pool and bf16 q/k/v")
    for t in (k_scale, v_scale, k_dscale, v_dscale):
        if t.shape != (num_kv_heads, head_dim) or t.dtype != torch.float32:
            raise ValueError("per-channel store / read scales are fp32 [kv_heads, dim]")
    n_out_max = out_idx2d.size(-1)
    if side_k.shape != (pages, page_size, num_kv_heads, n_out_max) or side_v.shape != side_k.shape \
            or side_k.dtype != torch.bfloat16 or side_v.dtype != torch.bfloat16:
        raise ValueError("side pools are bf16 [pages, page, kv_heads, n_out_max]")
    assert key.size(0) == batch and key.size(1) == num_kv_heads and slot_mapping.numel() == batch
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    nat.require_device(q, key, value, k_cache, v_cache, k_scale, v_scale, k_dscale, v_dscale,
                       side_k, side_v, out_idx2d, head_n_out, slot_mapping, block_tables,
                       context_lens)
    if q.stride(2) != 1:
        q = q.contiguous()
    for t in (k_cache, v_cache, k_scale, v_scale, k_dscale, v_dscale, side_k, side_v):
        if not t.is_contiguous():
            raise AssertionError("KV pools, scales and side pools must be contiguous")
    out_idx2d = out_idx2d.to(torch.int32).contiguous()
    head_n_out = head_n_out.to(torch.int32).contiguous()
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.dtype != torch.int32 or not context_lens.is_contiguous():
        context_lens = context_lens.to(torch.int32).contiguous()
    if slot_mapping.dtype == torch.int64:
        sb = 8
    else:
        slot_mapping = slot_mapping.to(torch.int32)
        sb = 4
    slot_mapping = slot_mapping.contiguous()
    output = torch.empty_like(q)
    if output.stride(2) != 1:
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if batch == 0:
        return output
    max_blocks = block_tables.size(1)
    ws_bytes = nat.query("kvc_paged_decode_workspace_bytes", batch, num_heads, num_kv_heads,
                         head_dim, page_size, max_blocks)
    ws = nat.workspace(ws_bytes, q.device)
    nat.call(
        "kvc_paged_decode_append_int8_chan",
        q.data_ptr(), q.stride(0), q.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        slot_mapping.data_ptr(), sb,
        k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
        k_dscale.data_ptr(), v_dscale.data_ptr(), side_k.data_ptr(), side_v.data_ptr(),
        out_idx2d.data_ptr(), head_n_out.data_ptr(), n_out_max,
        pages, page_size, num_kv_heads, head_dim,
        block_tables.data_ptr(), block_tables.stride(0), max_blocks,
        context_lens.data_ptr(), batch, num_heads, float(scale),
        output.data_ptr(), output.stride(0), output.stride(1),
        nat.ptr(ws), ws_bytes, nat.stream_of(q),
    )
    return output


def paged_decode_append_static(q, key, value, k_cache, v_cache, slot_mapping, block_tables,
                               context_lens, scale, out):
    """paged_decode_append for callers that cannot allocate device memory:
    the split-K workspace is the library's per-GPU static scratch
    (kvc_paged_decode_append_static) and the output goes to the caller's
    `out` [batch, heads, 128] bf16.  Nothing is converted or copied, so every
    argument must already be in the launch's form (int32 tables and lengths,
    int32 or int64 slots, unit inner strides); ValueError when the launch
    needs more scratch than the library holds.  Calls that overlap on one GPU
    share that scratch and must be ordered by the caller."""
    if q.ndim != 3 or key.ndim != 3 or value.shape != key.shape or k_cache.ndim != 4 \
            or v_cache.shape != k_cache.shape or out.shape != q.shape:
        raise ValueError("expected q/out=[batch,heads,dim], key/value=[batch,kv_heads,dim], "
                         "kv=[pages,page,kv_heads,dim]")
    batch, num_heads, head_dim = q.shape
    page_size = k_cache.size(1)
    num_kv_heads = k_cache.size(2)
    if head_dim != 128 or page_size % 32 or num_heads % num_kv_heads:
        raise ValueError(
            "paged decode requires head_dim=128, page_size a multiple of 32 and "
            "GQA-divisible heads")
    if not (q.dtype == key.dtype == value.dtype == k_cache.dtype == out.dtype == torch.bfloat16):
        raise ValueError("paged_decode_append_static takes a bf16 pool and bf16 q/k/v/out")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError("block_tables and context_lens must be int32 (no conversion here)")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("slot_mapping must be int32 or int64")
    assert key.size(0) == batch and key.size(1) == num_kv_heads and slot_mapping.numel() == batch
    assert q.stride(2) == 1 and out.stride(2) == 1 and key.stride(-1) == 1 \
        and value.stride(-1) == 1
    assert block_tables.stride(1) == 1 and context_lens.is_contiguous() \
        and slot_mapping.is_contiguous()
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise AssertionError("KV pools must be contiguous [pages, page, kv_heads, dim]")
    nat.require_device(q, key, value, k_cache, v_cache, slot_mapping, block_tables, context_lens,
                       out)
    nat.call(
        "kvc_paged_decode_append_static",
        q.data_ptr(), q.stride(0), q.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        slot_mapping.data_ptr(), slot_mapping.element_size(),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.size(0), page_size, num_kv_heads,
        head_dim, block_tables.data_ptr(), block_tables.stride(0), block_tables.size(1),
        context_lens.data_ptr(), batch, num_heads, float(scale),
        out.data_ptr(), out.stride(0), out.stride(1), nat.stream_of(q),
    )
    return out
