"""One-launch mixed decode + chunked-prefill attention (libkvc
`kvc_varlen_attention`).

Replaces the two sub-paths of a mixed step — paged decode for the first
`num_decode_rows` rows, then a per-sequence gather + SDPA loop for the prefill
chunks (nanovllm/layers/attention.py:146-166, :179-213) — with one kernel
launch over a unit list covering both, plus a split-K merge pass.  Row order
and masking are the reference's: decode rows first; prefill chunk i holds
sq_i queries at positions sk_i - sq_i .. sk_i - 1, each seeing keys
j <= its position (attention.py:210-212).
"""
from __future__ import annotations

import os

import numpy as np
import torch

from .. import _native as nat
from .paged_attention import _kv_encoding


def _host_list(lst, dev_tensor):
    if lst is not None:
        return list(lst)
    if dev_tensor is None:
        return None
    return dev_tensor.tolist()   # host sync, as the reference does when lists are absent


def _prefill_kq_pairs(cu_q, cu_k) -> int:
    """Query-key pairs per head of the prefill chunks (the work hint of
    kvc_varlen_attention): chunk i's query r sees sk - sq + r + 1 keys."""
    pairs = 0
    for i in range(len(cu_q) - 1):
        sq = cu_q[i + 1] - cu_q[i]
        sk = cu_k[i + 1] - cu_k[i]
        if sq > 0 and sk > 0:
            pairs += sq * (sk - sq) + sq * (sq + 1) // 2
    return pairs


class _Call:
    """The checked, converted arguments shared by both entry points."""


def _prepare(q, k_cache, v_cache, block_tables, num_decode_rows, decode_context_lens,
             decode_context_lens_list, cu_seqlens_q, cu_seqlens_k, cu_seqlens_q_list,
             cu_seqlens_k_list, k, v, k_scale):
    c = _Call()
    T, num_heads, head_dim = q.shape
    if head_dim != 128:
        raise ValueError("varlen attention requires head_dim=128")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16 (got {q.dtype})")
    c.fresh = block_tables is None
    if c.fresh:
        if k is None or v is None:
            raise ValueError("without block_tables the keys come from k/v")
        c.num_kv_heads = k.size(1)
        c.page_size = 0
        c.enc = nat.KVC_KV_BF16
    else:
        c.num_kv_heads = k_cache.size(2)
        c.page_size = k_cache.size(1)
        if c.page_size % 32:
            raise ValueError("page_size must be a multiple of 32")
        c.enc = _kv_encoding(k_cache, k_scale)
        assert k_cache.is_contiguous() and v_cache.is_contiguous()
    if num_heads % c.num_kv_heads:
        raise ValueError("num_heads must be a multiple of num_kv_heads")
    nat.require_device(q)
    if q.stride(2) != 1:
        q = q.contiguous()
    c.q = q
    c.out = torch.empty((T, num_heads, head_dim), dtype=q.dtype, device=q.device)
    c.T, c.num_heads, c.head_dim = T, num_heads, head_dim
    if T == 0:
        return c

    cu_q = _host_list(cu_seqlens_q_list, cu_seqlens_q) or [0]
    cu_k = _host_list(cu_seqlens_k_list, cu_seqlens_k) or [0]
    c.num_prefill = len(cu_q) - 1
    if num_decode_rows + cu_q[-1] != T:
        raise ValueError(f"{T} query rows but {num_decode_rows} decode rows + "
                         f"{cu_q[-1]} prefill tokens")
    sq = [cu_q[i + 1] - cu_q[i] for i in range(c.num_prefill)]
    sk = [cu_k[i + 1] - cu_k[i] for i in range(c.num_prefill)]
    for a, b in zip(sq, sk):
        if a > 0 and b < a:
            raise ValueError("a prefill chunk has fewer keys than queries")
    c.max_seqlen_k = max(sk) if sk else 0
    c.total_keys = cu_k[-1]
    c.cu_k_list = cu_k
    cu_q_np = np.asarray(cu_q, dtype=np.int32)
    cu_k_np = np.asarray(cu_k, dtype=np.int32)
    c.pre_units = nat.query("kvc_varlen_prefill_units", cu_q_np.ctypes.data, cu_k_np.ctypes.data,
                            c.num_prefill, num_heads, c.num_kv_heads, c.max_seqlen_k)
    if c.num_prefill:
        if cu_seqlens_q is None or cu_seqlens_q.device != q.device:
            cu_seqlens_q = torch.from_numpy(cu_q_np).to(q.device, non_blocking=True)
        if cu_seqlens_k is None or cu_seqlens_k.device != q.device:
            cu_seqlens_k = torch.from_numpy(cu_k_np).to(q.device, non_blocking=True)
        cu_seqlens_q = cu_seqlens_q.to(torch.int32).contiguous()
        cu_seqlens_k = cu_seqlens_k.to(torch.int32).contiguous()
    c.cu_seqlens_q, c.cu_seqlens_k = cu_seqlens_q, cu_seqlens_k
    # Work hints for the CU split of a mixed call (0: none).
    c.decode_ctx_tokens = int(sum(decode_context_lens_list)) \
        if num_decode_rows and decode_context_lens_list is not None else 0
    c.prefill_kq_pairs = _prefill_kq_pairs(cu_q, cu_k) if num_decode_rows else 0

    c.max_blocks = 0
    if not c.fresh:
        if block_tables.dtype != torch.int32:
            block_tables = block_tables.to(torch.int32)
        if block_tables.stride(1) != 1:
            block_tables = block_tables.contiguous()
        c.max_blocks = block_tables.size(1)
    c.block_tables = block_tables
    if num_decode_rows:
        decode_context_lens = decode_context_lens.to(torch.int32).contiguous()
    c.decode_context_lens = decode_context_lens
    c.ws_bytes = nat.query("kvc_varlen_workspace_bytes", T, num_heads, c.num_kv_heads, head_dim,
                           num_decode_rows, c.max_seqlen_k, c.page_size, c.max_blocks)
    c.ws = nat.workspace(c.ws_bytes, q.device)
    return c


def gather_kv(k_cache, v_cache, block_tables, cu_seqlens_k, cu_seqlens_k_list, *,
              block_table_row0=0, k_scale=None, v_scale=None, side_k=None, side_v=None,
              out_idx2d=None, head_n_out=None):
    """_gather_kv (nanovllm/layers/attention.py:33-51) for every prefill chunk
    of a step in one launch (kvc_gather_kv): chunk i's keys, read through
    block table row block_table_row0 + i and dequantised as the reference
    does for an int8 pool, at rows cu_seqlens_k[i] .. of the returned bf16
    (K, V), each [cu_seqlens_k[-1], KVH, D]."""
    enc = _kv_encoding(k_cache, k_scale)
    cu_k = list(cu_seqlens_k_list)
    total = cu_k[-1]
    kvh, page = k_cache.size(2), k_cache.size(1)
    out_k = torch.empty((total, kvh, k_cache.size(3)), dtype=torch.bfloat16, device=k_cache.device)
    out_v = torch.empty_like(out_k)
    if total == 0:
        return out_k, out_v
    nat.require_device(k_cache, v_cache, block_tables, cu_seqlens_k)
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    bt = block_tables.to(torch.int32)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    cu = cu_seqlens_k.to(torch.int32).contiguous()
    has_side = enc == nat.KVC_KV_INT8_CHAN and side_k is not None and head_n_out is not None
    if enc == nat.KVC_KV_INT8_TOKHEAD:
        k_scale, v_scale = k_scale.contiguous(), v_scale.contiguous()
    elif enc == nat.KVC_KV_INT8_CHAN:
        k_scale = k_scale.to(torch.float32).contiguous()
        v_scale = v_scale.to(torch.float32).contiguous()
    nat.call(
        "kvc_gather_kv", nat.ptr(k_cache), nat.ptr(v_cache), k_cache.size(0), page, kvh,
        k_cache.size(3), enc, nat.ptr(k_scale), nat.ptr(v_scale),
        nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
        nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
        side_k.size(-1) if has_side else 0, nat.ptr(bt), bt.stride(0), bt.size(1),
        block_table_row0, len(cu_k) - 1, nat.ptr(cu), total, nat.ptr(out_k), nat.ptr(out_v),
        nat.stream_of(out_k),
    )
    return out_k, out_v


def _gathered_prefill(c, q, nd, k_cache, v_cache, scale, k_scale, v_scale, side_k, side_v,
                      out_idx2d, head_n_out):
    """Prefill rows (query rows nd ..) over an int8 pool as the reference reads
    them: the chunks' keys gathered and dequantised to bf16 (gather_kv,
    block table rows nd + i), then the bf16 stream-K prefill over those rows,
    whose outlier dims (a per-channel pool) take the residue product."""
    kg, vg = gather_kv(k_cache, v_cache, c.block_tables, c.cu_seqlens_k, c.cu_k_list,
                       block_table_row0=nd, k_scale=k_scale, v_scale=v_scale, side_k=side_k,
                       side_v=side_v, out_idx2d=out_idx2d, head_n_out=head_n_out)
    has_side = c.enc == nat.KVC_KV_INT8_CHAN and side_k is not None and head_n_out is not None
    qp, op = q[nd:], c.out[nd:]
    nat.call(
        "kvc_varlen_attention",
        qp.data_ptr(), q.stride(0), q.stride(1), c.T - nd, c.num_heads, None, None, 0, 0,
        c.num_kv_heads, c.head_dim, nat.KVC_KV_BF16, None, None, None, None,
        nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
        side_k.size(-1) if has_side else 0,
        nat.ptr(kg), kg.stride(0), kg.stride(1), nat.ptr(vg), vg.stride(0), vg.stride(1),
        None, 0, 0, 0, None, c.num_prefill, nat.ptr(c.cu_seqlens_q), nat.ptr(c.cu_seqlens_k),
        c.pre_units, c.max_seqlen_k, 0, 0,
        float(scale), op.data_ptr(), c.out.stride(0), c.out.stride(1),
        nat.ptr(c.ws), c.ws_bytes, nat.stream_of(q),
    )
    return c.out


def _paged_rows(c, q, nd, k_cache, v_cache, scale, k_scale, v_scale, side_k, side_v, out_idx2d,
                head_n_out, has_side):
    """The decode rows 0 .. nd - 1 of a mixed call alone (no prefill chunks)."""
    nat.call(
        "kvc_varlen_attention",
        q.data_ptr(), q.stride(0), q.stride(1), nd, c.num_heads,
        nat.ptr(k_cache), nat.ptr(v_cache), k_cache.size(0), c.page_size, c.num_kv_heads,
        c.head_dim, c.enc, nat.ptr(k_scale), nat.ptr(v_scale),
        nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
        nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
        side_k.size(-1) if has_side else 0, None, 0, 0, None, 0, 0,
        nat.ptr(c.block_tables), c.block_tables.stride(0), c.max_blocks,
        nd, nat.ptr(c.decode_context_lens), 0, None, None, 0, 0, 0, 0,
        float(scale), c.out.data_ptr(), c.out.stride(0), c.out.stride(1),
        nat.ptr(c.ws), c.ws_bytes, nat.stream_of(q),
    )


def varlen_attention(q, k_cache, v_cache, *, scale, block_tables=None,
                     num_decode_rows=0, decode_context_lens=None,
                     cu_seqlens_q=None, cu_seqlens_k=None,
                     cu_seqlens_q_list=None, cu_seqlens_k_list=None,
                     k=None, v=None,
                     k_scale=None, v_scale=None, side_k=None, side_v=None,
                     out_idx2d=None, head_n_out=None, decode_context_lens_list=None):
    """q: [T, H, D] bf16 with T = num_decode_rows + prefill tokens.
    k/v: the step's fresh [T_k, KVH, D] bf16 keys/values, used only when
    block_tables is None (pure prefill without a prefix cache); rows that
    gather_kv read from a per-channel int8 pool may come with that pool's
    out_idx2d / head_n_out, which give its outlier dims the residue product.
    decode_context_lens_list: the decode rows' context lengths as host ints
    (optional; with them a mixed call over a bf16 pool sizes its CU split to
    the work of both sides).
    Returns out [T, H, D] bf16."""
    c = _prepare(q, k_cache, v_cache, block_tables, num_decode_rows, decode_context_lens,
                 decode_context_lens_list, cu_seqlens_q, cu_seqlens_k, cu_seqlens_q_list,
                 cu_seqlens_k_list, k, v, k_scale)
    if c.T == 0:
        return c.out
    enc, fresh, q = c.enc, c.fresh, c.q
    gathered = (enc != nat.KVC_KV_BF16 and not fresh and c.num_prefill
                and os.environ.get("KVC_PREFILL_SK", "1") != "0")
    has_side = enc == nat.KVC_KV_INT8_CHAN and side_k is not None and head_n_out is not None
    # fresh rows gathered from a per-channel pool name its outlier dims
    fresh_out = fresh and out_idx2d is not None and head_n_out is not None
    if enc == nat.KVC_KV_INT8_TOKHEAD:
        k_scale, v_scale = k_scale.contiguous(), v_scale.contiguous()
    elif enc == nat.KVC_KV_INT8_CHAN:
        k_scale = k_scale.to(torch.float32).contiguous()
        v_scale = v_scale.to(torch.float32).contiguous()
    if gathered:
        # Int8 pool: the decode rows (if any) through the paged decode alone,
        # then the prefill rows over their gathered, dequantised keys.
        if num_decode_rows:
            _paged_rows(c, q, num_decode_rows, k_cache, v_cache, scale, k_scale, v_scale,
                        side_k, side_v, out_idx2d, head_n_out, has_side)
        return _gathered_prefill(c, q, num_decode_rows, k_cache, v_cache, scale, k_scale, v_scale,
                                 side_k, side_v, out_idx2d, head_n_out)
    nat.call(
        "kvc_varlen_attention",
        q.data_ptr(), q.stride(0), q.stride(1), c.T, c.num_heads,
        nat.ptr(k_cache) if not fresh else None, nat.ptr(v_cache) if not fresh else None,
        k_cache.size(0) if not fresh else 0, c.page_size, c.num_kv_heads, c.head_dim, enc,
        nat.ptr(k_scale), nat.ptr(v_scale),
        nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
        nat.ptr(out_idx2d) if has_side or fresh_out else None,
        nat.ptr(head_n_out) if has_side or fresh_out else None,
        side_k.size(-1) if has_side else (out_idx2d.size(1) if fresh_out else 0),
        nat.ptr(k) if fresh else None, k.stride(0) if fresh else 0, k.stride(1) if fresh else 0,
        nat.ptr(v) if fresh else None, v.stride(0) if fresh else 0, v.stride(1) if fresh else 0,
        nat.ptr(c.block_tables) if not fresh else None,
        c.block_tables.stride(0) if not fresh else 0, c.max_blocks,
        num_decode_rows, nat.ptr(c.decode_context_lens) if num_decode_rows else None,
        c.num_prefill, nat.ptr(c.cu_seqlens_q) if c.num_prefill else None,
        nat.ptr(c.cu_seqlens_k) if c.num_prefill else None, c.pre_units, c.max_seqlen_k,
        c.decode_ctx_tokens, c.prefill_kq_pairs,
        float(scale), c.out.data_ptr(), c.out.stride(0), c.out.stride(1),
        nat.ptr(c.ws), c.ws_bytes, nat.stream_of(q),
    )
    return c.out


def varlen_attention_append(q, key, value, k_cache, v_cache, slot_mapping, *, scale,
                            block_tables, num_decode_rows=0, decode_context_lens=None,
                            cu_seqlens_q=None, cu_seqlens_k=None,
                            cu_seqlens_q_list=None, cu_seqlens_k_list=None,
                            decode_context_lens_list=None):
    """store_kvcache(key, value, k_cache, v_cache, slot_mapping) followed by
    varlen_attention over a bf16 pool (nanovllm/layers/attention.py:138-140,
    :146-173), in kvc_varlen_attention_append: the prefill rows' k/v are
    stored ahead of the attention, the decode rows' k/v are appended inside
    the decode launch.  key / value [T, KVH, 128] bf16 (strided views of the
    qkv projection are fine); slot_mapping [T] int32 or int64.  The decode
    rows must use the engine's decode slots (row i's slot is position
    decode_context_lens[i] - 1 of its own table row), as for
    paged_decode_append.  Same results and pool contents as the two calls."""
    if block_tables is None:
        raise ValueError("varlen_attention_append needs a paged pool and block_tables")
    if not (q.dtype == key.dtype == value.dtype == k_cache.dtype == torch.bfloat16):
        raise ValueError("varlen_attention_append takes a bf16 pool and bf16 q/k/v")
    if key.ndim != 3 or value.shape != key.shape or key.size(0) != q.size(0) \
            or key.size(1) != k_cache.size(2) or slot_mapping.numel() != q.size(0):
        raise ValueError("expected key/value=[T,kv_heads,dim] and slot_mapping=[T] for q=[T,...]")
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    c = _prepare(q, k_cache, v_cache, block_tables, num_decode_rows, decode_context_lens,
                 decode_context_lens_list, cu_seqlens_q, cu_seqlens_k, cu_seqlens_q_list,
                 cu_seqlens_k_list, None, None, None)
    if c.T == 0:
        return c.out
    nat.require_device(key, value, k_cache, v_cache, slot_mapping)
    if slot_mapping.dtype == torch.int64:
        sb = 8
    else:
        slot_mapping = slot_mapping.to(torch.int32)
        sb = 4
    slot_mapping = slot_mapping.contiguous()
    q = c.q
    nat.call(
        "kvc_varlen_attention_append",
        q.data_ptr(), q.stride(0), q.stride(1), c.T, c.num_heads,
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        slot_mapping.data_ptr(), sb,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.size(0), c.page_size, c.num_kv_heads,
        c.head_dim, c.block_tables.data_ptr(), c.block_tables.stride(0), c.max_blocks,
        num_decode_rows, nat.ptr(c.decode_context_lens) if num_decode_rows else None,
        c.num_prefill, nat.ptr(c.cu_seqlens_q) if c.num_prefill else None,
        nat.ptr(c.cu_seqlens_k) if c.num_prefill else None, c.pre_units, c.max_seqlen_k,
        c.decode_ctx_tokens, c.prefill_kq_pairs,
        float(scale), c.out.data_ptr(), c.out.stride(0), c.out.stride(1),
        nat.ptr(c.ws), c.ws_bytes, nat.stream_of(q),
    )
    return c.out


def varlen_decode_cus(num_decode_rows, num_prefill_tokens, num_heads, num_kv_heads,
                      decode_context_lens_list=None, cu_seqlens_q_list=None,
                      cu_seqlens_k_list=None, kv_dtype=nat.KVC_KV_BF16) -> int:
    """CUs the decode side of a mixed call's one launch gets (0: the decode and
    prefill launches run in turn), from the same hints varlen_attention
    passes (kvc_varlen_decode_cus)."""
    dec = int(sum(decode_context_lens_list)) if decode_context_lens_list is not None else 0
    pairs = _prefill_kq_pairs(list(cu_seqlens_q_list), list(cu_seqlens_k_list)) \
        if cu_seqlens_q_list is not None else 0
    return nat.query("kvc_varlen_decode_cus", num_decode_rows, num_prefill_tokens, num_heads,
                     num_kv_heads, kv_dtype, dec, pairs)
