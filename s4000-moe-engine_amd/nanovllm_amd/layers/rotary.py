"""Rotary embedding and the fused step in front of the paged KV path, backed
by libkvc (`kvc_qk_norm_rope_store`).

`RotaryEmbedding` keeps the constructor, the fp32 `cos_sin_cache` buffer and
the `forward(positions, query, key) -> (query, key)` contract of
nanovllm/layers/rotary_embedding.py:18-49 (neox halves, fp32 arithmetic,
results in the input dtype).  `qk_norm_rope_store` is the one-launch form of
what Qwen3Attention.forward does between the qkv projection and attention
(nanovllm/models/qwen3.py:77-86): q_norm / k_norm (RMSNorm over head_dim,
nanovllm/layers/layernorm.py:18-26), the rotation, and store_kvcache of the
rotated k and the raw v (nanovllm/layers/attention.py:9-30).
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as nat


def build_cos_sin_cache(head_size: int, max_position: int, base: float,
                        device: torch.device | str | None = None) -> torch.Tensor:
    """fp32 [max_position, head_size]: cos of position x inv_freq in the first
    half, sin in the second, computed as RotaryEmbedding does
    (rotary_embedding.py:30-35), on the CPU, then moved."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1)
    return cache.to(device) if device is not None else cache


def _index_arg(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    if t.dtype == torch.int64:
        return t.contiguous(), 8
    return t.to(torch.int32).contiguous(), 4


def qk_norm_rope_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None,
                       positions: torch.Tensor, cos_sin_cache: torch.Tensor,
                       q_norm_weight: torch.Tensor | None = None,
                       k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, return_k: bool = True,
                       q_out: torch.Tensor | None = None):
    """q [N, H, D], k/v [N, KVH, D] bf16 (views of the fused projection are
    fine); positions [N]; cos_sin_cache fp32 [max_position, D].  Returns
    (q_rot, k_rot) with k_rot None when return_k is False.  With k_cache /
    v_cache / slot_mapping the rotated k and the unchanged v are also
    appended to the pool (the engine's store_kvcache semantics)."""
    N, H, D = q.shape
    KVH = k.size(1)
    if D != 128:
        raise ValueError("qk_norm_rope_store requires head_dim=128")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise ValueError("q and k must be bf16")
    assert q.stride(-1) == 1 and k.stride(-1) == 1
    assert cos_sin_cache.dtype == torch.float32 and cos_sin_cache.dim() == 2
    assert cos_sin_cache.size(1) == D and cos_sin_cache.is_contiguous()
    nat.require_device(q, k, v, positions, cos_sin_cache, k_cache, v_cache, slot_mapping,
                       q_norm_weight, k_norm_weight)
    if q_out is None:
        q_out = torch.empty((N, H, D), dtype=q.dtype, device=q.device)
    k_out = torch.empty((N, KVH, D), dtype=k.dtype, device=k.device) if return_k else None
    pos, pb = _index_arg(positions)
    cache = k_cache is not None
    num_slots, slots, sb = 0, None, 4
    if cache:
        if v is None or v_cache is None or slot_mapping is None:
            raise ValueError("appending needs v, v_cache and slot_mapping")
        assert v.stride(-1) == 1 and v.dtype == torch.bfloat16
        assert k_cache.is_contiguous() and v_cache.is_contiguous()
        assert k_cache.dtype == v_cache.dtype == torch.bfloat16
        assert slot_mapping.numel() == N
        num_slots = k_cache.numel() // (KVH * D)
        slots, sb = _index_arg(slot_mapping)
    qw = q_norm_weight.to(torch.bfloat16).contiguous() if q_norm_weight is not None else None
    kw = k_norm_weight.to(torch.bfloat16).contiguous() if k_norm_weight is not None else None
    nat.call(
        "kvc_qk_norm_rope_store",
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        nat.ptr(v), v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0,
        N, H, KVH, D, pos.data_ptr(), pb, nat.ptr(qw), nat.ptr(kw), float(eps),
        cos_sin_cache.data_ptr(), cos_sin_cache.size(0),
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        nat.ptr(k_out), k_out.stride(0) if k_out is not None else 0,
        k_out.stride(1) if k_out is not None else 0,
        nat.ptr(k_cache), nat.ptr(v_cache), num_slots, nat.ptr(slots), sb,
        nat.stream_of(q))
    return q_out, k_out


class RotaryEmbedding(nn.Module):
    """nanovllm/layers/rotary_embedding.py:18-49: same constructor, same fp32
    `cos_sin_cache` ([max_position, 1, D] there, [max_position, D] here:
    the same bytes), same forward contract."""

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int,
                 base: float) -> None:
        super().__init__()
        self.head_size = head_size
        assert rotary_dim == head_size
        self.register_buffer("cos_sin_cache",
                             build_cos_sin_cache(head_size, max_position_embeddings, base),
                             persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        N = positions.numel()
        q = query.view(N, -1, self.head_size)
        k = key.view(N, -1, self.head_size)
        q_rot, k_rot = qk_norm_rope_store(q, k, None, positions, self.cos_sin_cache)
        return q_rot.view_as(query), k_rot.view_as(key)
