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


def varlen_attention(q, k_cache, v_cache, *, scale, block_tables=None,
                     num_decode_rows=0, decode_context_lens=None,
                     cu_seqlens_q=None, cu_seqlens_k=None,
                     cu_seqlens_q_list=None, cu_seqlens_k_list=None,
                     k=None, v=None,
                     k_scale=None, v_scale=None, side_k=None, side_v=None,
                     out_idx2d=None, head_n_out=None):
    """q: [T, H, D] bf16 with T = num_decode_rows + prefill tokens.
    k/v: the step's fresh [T_k, KVH, D] bf16 keys/values, used only when
    block_tables is None (pure prefill without a prefix cache).
    Returns out [T, H, D] bf16."""
    T, num_heads, head_dim = q.shape
    if head_dim != 128:
        raise ValueError("varlen attention requires head_dim=128")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16 (got {q.dtype})")
    fresh = block_tables is None
    if fresh:
        if k is None or v is None:
            raise ValueError("without block_tables the keys come from k/v")
        num_kv_heads = k.size(1)
        page_size = 0
        enc = nat.KVC_KV_BF16
    else:
        num_kv_heads = k_cache.size(2)
        page_size = k_cache.size(1)
        if page_size % 32:
            raise ValueError("page_size must be a multiple of 32")
        enc = _kv_encoding(k_cache, k_scale)
        assert k_cache.is_contiguous() and v_cache.is_contiguous()
    if num_heads % num_kv_heads:
        raise ValueError("num_heads must be a multiple of num_kv_heads")
    nat.require_device(q)
    if q.stride(2) != 1:
        q = q.contiguous()
    out = torch.empty((T, num_heads, head_dim), dtype=q.dtype, device=q.device)
    if T == 0:
        return out

    cu_q = _host_list(cu_seqlens_q_list, cu_seqlens_q) or [0]
    cu_k = _host_list(cu_seqlens_k_list, cu_seqlens_k) or [0]
    num_prefill = len(cu_q) - 1
    if num_decode_rows + cu_q[-1] != T:
        raise ValueError(f"{T} query rows but {num_decode_rows} decode rows + "
                         f"{cu_q[-1]} prefill tokens")
    sq = [cu_q[i + 1] - cu_q[i] for i in range(num_prefill)]
    sk = [cu_k[i + 1] - cu_k[i] for i in range(num_prefill)]
    for a, b in zip(sq, sk):
        if a > 0 and b < a:
            raise ValueError("a prefill chunk has fewer keys than queries")
    max_seqlen_k = max(sk) if sk else 0
    cu_q_np = np.asarray(cu_q, dtype=np.int32)
    cu_k_np = np.asarray(cu_k, dtype=np.int32)
    pre_units = nat.query("kvc_varlen_prefill_units", cu_q_np.ctypes.data, cu_k_np.ctypes.data,
                          num_prefill, num_heads, num_kv_heads, max_seqlen_k)
    if num_prefill:
        if cu_seqlens_q is None or cu_seqlens_q.device != q.device:
            cu_seqlens_q = torch.from_numpy(cu_q_np).to(q.device, non_blocking=True)
        if cu_seqlens_k is None or cu_seqlens_k.device != q.device:
            cu_seqlens_k = torch.from_numpy(cu_k_np).to(q.device, non_blocking=True)
        cu_seqlens_q = cu_seqlens_q.to(torch.int32).contiguous()
        cu_seqlens_k = cu_seqlens_k.to(torch.int32).contiguous()

    max_blocks = 0
    if not fresh:
        if block_tables.dtype != torch.int32:
            block_tables = block_tables.to(torch.int32)
        if block_tables.stride(1) != 1:
            block_tables = block_tables.contiguous()
        max_blocks = block_tables.size(1)
    if num_decode_rows:
        decode_context_lens = decode_context_lens.to(torch.int32).contiguous()
    has_side = enc == nat.KVC_KV_INT8_CHAN and side_k is not None and head_n_out is not None
    if enc == nat.KVC_KV_INT8_TOKHEAD:
        k_scale, v_scale = k_scale.contiguous(), v_scale.contiguous()
    elif enc == nat.KVC_KV_INT8_CHAN:
        k_scale = k_scale.to(torch.float32).contiguous()
        v_scale = v_scale.to(torch.float32).contiguous()
    ws_bytes = nat.query("kvc_varlen_workspace_bytes", T, num_heads, num_kv_heads, head_dim,
                         num_decode_rows, max_seqlen_k, page_size, max_blocks)
    ws = nat.workspace(ws_bytes, q.device)
    nat.call(
        "kvc_varlen_attention",
        q.data_ptr(), q.stride(0), q.stride(1), T, num_heads,
        nat.ptr(k_cache) if not fresh else None, nat.ptr(v_cache) if not fresh else None,
        k_cache.size(0) if not fresh else 0, page_size, num_kv_heads, head_dim, enc,
        nat.ptr(k_scale), nat.ptr(v_scale),
        nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
        nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
        side_k.size(-1) if has_side else 0,
        nat.ptr(k) if fresh else None, k.stride(0) if fresh else 0, k.stride(1) if fresh else 0,
        nat.ptr(v) if fresh else None, v.stride(0) if fresh else 0, v.stride(1) if fresh else 0,
        nat.ptr(block_tables) if not fresh else None,
        block_tables.stride(0) if not fresh else 0, max_blocks,
        num_decode_rows, nat.ptr(decode_context_lens) if num_decode_rows else None,
        num_prefill, nat.ptr(cu_seqlens_q) if num_prefill else None,
        nat.ptr(cu_seqlens_k) if num_prefill else None, pre_units, max_seqlen_k,
        float(scale), out.data_ptr(), out.stride(0), out.stride(1),
        nat.ptr(ws), ws_bytes, nat.stream_of(q),
    )
    return out
