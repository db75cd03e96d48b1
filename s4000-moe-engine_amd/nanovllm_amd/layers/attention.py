"""Attention layer of the paged KV path, backed by libkvc.

store_kvcache and Attention keep the signatures, attributes and tensor layouts
of nanovllm/layers/attention.py:9-279, so the model (Qwen3Attention) and the
runner (which assigns k_cache/v_cache and the int8 tensors per layer) do not
change.  What changes is underneath:

* append is one HIP launch for K and V (V read through its own strides, so the
  strided V view of a fused qkv projection is not copied first);
* decode is the split-K paged kernel regardless of `attention_backend` (the
  reference's "sdpa" decode gathers and expands the whole padded table,
  attention.py:239-279; both backends compute the same function); on a bf16
  pool the step's append rides in the decode launch (paged_decode_append),
  with the same results and pool bytes as store + decode;
* prefill and mixed batches are ONE varlen launch instead of a Python loop
  over sequences plus torch.cat (attention.py:146-166, :179-213).
"""
from __future__ import annotations

from contextlib import nullcontext

import torch
from torch import nn

from .. import _native as nat
from ..kernels.kv_int8 import store_kvcache_int8
from ..kernels.paged_attention import (paged_decode_append, paged_decode_append_int8_chan,
                                       paged_decode_append_int8_tokhead,
                                       paged_decode_attention)
from ..kernels.varlen import varlen_attention, varlen_attention_append
from ..utils.context import get_context
from .rotary import qk_norm_rope_store


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor):
    """k_cache.view(-1, KVH*D)[slot_mapping] = key.reshape(N, KVH*D); same for V.

    Same preconditions as attention.py:12-15.  A negative slot indexes from
    the end like the reference's integer index_put; no host synchronisation,
    so the call is graph-capturable."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    nat.require_device(key, value, k_cache, v_cache, slot_mapping)
    if slot_mapping.dtype == torch.int64:
        sb = 8
    else:
        slot_mapping = slot_mapping.to(torch.int32)
        sb = 4
    slot_mapping = slot_mapping.contiguous()
    num_slots = k_cache.numel() // D
    nat.call("kvc_store_kv",
             key.data_ptr(), key.stride(0), key.stride(1),
             value.data_ptr(), value.stride(0), value.stride(1),
             k_cache.data_ptr(), v_cache.data_ptr(), num_slots,
             slot_mapping.data_ptr(), sb, N, num_heads, head_dim, key.element_size(),
             nat.stream_of(key))


class Attention(nn.Module):
    """Attention(num_heads, head_dim, scale, num_kv_heads) with the runner-set
    attributes of attention.py:108-123."""

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.block_size = None
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = self.v_scale = None      # int8 store scales
        self.k_dscale = self.v_dscale = None    # int8 per-channel read scales
        self.side_k = self.side_v = None        # bf16 outlier side pools
        self.out_idx2d = None
        self.head_n_out = None
        self.kv_cache_is_int8 = False
        self.attention_backend = "triton_paged"
        self.profiler = None
        self.layer_id = -1
        # Set by a runner whose block moves run asynchronously: called with
        # kv_layer before this layer first touches its pool planes in a step.
        self.kv_fence = None
        self.kv_layer = -1
        # Set by a runner with a per-channel int8 pool: called with
        # (kv_layer, k, v) on every forward; it records calibration
        # statistics between kv_calibrate_begin and kv_calibrate_freeze.
        self.kv_observe = None

    def _profile(self, name):
        if self.profiler is None:
            return nullcontext()
        return self.profiler.range(name, layer=self.layer_id)

    def _int8_tokhead(self) -> bool:
        return self.kv_cache_is_int8 and self.k_scale is not None and self.k_scale.dim() == 3

    def _int8_chan_step(self) -> bool:
        """A per-channel pool with its side pools and read scales bound: the
        decode step is one call (store, then decode)."""
        return (self.kv_cache_is_int8 and not self._int8_tokhead() and self.k_scale is not None
                and self.k_dscale is not None and self.side_k is not None
                and self.out_idx2d is not None and self.head_n_out is not None)

    def _read_scales(self):
        """Scales the read path needs: per-slot scales (per-token-head) or the
        per-channel read scales (0 at outlier dims)."""
        if not self.kv_cache_is_int8:
            return None, None
        if self._int8_tokhead():
            return self.k_scale, self.v_scale
        return self.k_dscale, self.v_dscale

    def forward_fused(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, cos_sin_cache: torch.Tensor,
                      q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None,
                      eps: float):
        """Qwen3Attention.forward's q_norm, k_norm and rotary_emb
        (nanovllm/models/qwen3.py:82-85) fused with this layer's append
        (one launch on a bf16 pool), then attention.  q [N, H*D] or
        [N, H, D]; k, v [N, KVH*D] or [N, KVH, D] (views of the qkv
        projection are fine)."""
        context = get_context()
        if self.kv_fence is not None:
            self.kv_fence(self.kv_layer)
        N = positions.numel()
        q3 = q.view(N, self.num_heads, self.head_dim)
        k3 = k.view(N, self.num_kv_heads, self.head_dim)
        v3 = v.view(N, self.num_kv_heads, self.head_dim)
        k_cache, v_cache = self.k_cache, self.v_cache
        bf16_pool = bool(k_cache.numel() and v_cache.numel()) and not self.kv_cache_is_int8
        need_k = not bf16_pool or context.block_tables is None
        with self._profile("attention.qk_norm_rope_store"):
            q_rot, k_rot = qk_norm_rope_store(
                q3, k3, v3, positions, cos_sin_cache, q_norm_weight, k_norm_weight, eps,
                k_cache if bf16_pool else None, v_cache if bf16_pool else None,
                context.slot_mapping if bf16_pool else None, return_k=need_k)
        if k_rot is None:
            k_rot = k3  # not read: the rows are in the pool
        return self.forward(q_rot, k_rot, v3, kv_stored=bf16_pool)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_stored: bool = False):
        """attention.py:130-177.  kv_stored: the step's k/v rows are already
        in the pool (appended by forward_fused), so the store is skipped."""
        context = get_context()
        if self.kv_fence is not None and not kv_stored:
            self.kv_fence(self.kv_layer)
        if self.kv_observe is not None:
            self.kv_observe(self.kv_layer, k, v)
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() and self.block_size is None:
            self.block_size = k_cache.size(1)
        # A decode step appends inside the decode call (bf16 and per-token-head
        # int8 pools inside the decode launch; per-channel int8 in the same
        # call, as a store launch ahead of the decode).
        fuse_append = (not kv_stored and not (context.is_mixed or context.is_prefill)
                       and bool(k_cache.numel() and v_cache.numel())
                       and (not self.kv_cache_is_int8 or self._int8_tokhead()
                            or self._int8_chan_step()))
        # A mixed (or prefix-cached prefill) step on a bf16 pool stores and
        # attends in one call: the decode rows append inside the decode launch.
        varlen_append = (not kv_stored and (context.is_mixed or context.is_prefill)
                         and context.block_tables is not None
                         and bool(k_cache.numel() and v_cache.numel())
                         and not self.kv_cache_is_int8)
        if varlen_append:
            with self._profile("attention.mixed" if context.is_mixed else "attention.prefill"):
                return varlen_attention_append(
                    q.view(-1, self.num_heads, self.head_dim),
                    k.view(-1, self.num_kv_heads, self.head_dim),
                    v.view(-1, self.num_kv_heads, self.head_dim), k_cache, v_cache,
                    context.slot_mapping, scale=self.scale, block_tables=context.block_tables,
                    num_decode_rows=context.num_decode_rows if context.is_mixed else 0,
                    decode_context_lens=context.decode_context_lens if context.is_mixed else None,
                    cu_seqlens_q=context.cu_seqlens_q, cu_seqlens_k=context.cu_seqlens_k,
                    cu_seqlens_q_list=context.cu_seqlens_q_list,
                    cu_seqlens_k_list=context.cu_seqlens_k_list,
                    decode_context_lens_list=(context.decode_context_lens_list
                                              if context.is_mixed else None))
        if k_cache.numel() and v_cache.numel() and not kv_stored and not fuse_append:
            with self._profile("attention.kv_store"):
                if self.kv_cache_is_int8:
                    store_kvcache_int8(k, v, k_cache, v_cache, self.k_scale, self.v_scale,
                                       self.side_k, self.side_v, self.out_idx2d,
                                       self.head_n_out, context.slot_mapping)
                else:
                    store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        rk, rv = self._read_scales()
        side = self.kv_cache_is_int8 and not self._int8_tokhead()
        if context.is_mixed or context.is_prefill:
            q3 = q.view(-1, self.num_heads, self.head_dim)
            with self._profile("attention.mixed" if context.is_mixed else "attention.prefill"):
                return varlen_attention(
                    q3, k_cache, v_cache, scale=self.scale,
                    block_tables=context.block_tables,
                    num_decode_rows=context.num_decode_rows if context.is_mixed else 0,
                    decode_context_lens=context.decode_context_lens if context.is_mixed else None,
                    cu_seqlens_q=context.cu_seqlens_q, cu_seqlens_k=context.cu_seqlens_k,
                    cu_seqlens_q_list=context.cu_seqlens_q_list,
                    cu_seqlens_k_list=context.cu_seqlens_k_list,
                    k=k.view(-1, self.num_kv_heads, self.head_dim),
                    v=v.view(-1, self.num_kv_heads, self.head_dim),
                    k_scale=rk, v_scale=rv,
                    side_k=self.side_k if side else None,
                    side_v=self.side_v if side else None,
                    out_idx2d=self.out_idx2d if side else None,
                    head_n_out=self.head_n_out if side else None,
                    decode_context_lens_list=(context.decode_context_lens_list
                                              if context.is_mixed else None),
                )
        if fuse_append and self.kv_cache_is_int8 and not self._int8_tokhead():
            with self._profile("attention.paged_decode"):
                return paged_decode_append_int8_chan(
                    q.view(-1, self.num_heads, self.head_dim),
                    k.view(-1, self.num_kv_heads, self.head_dim),
                    v.view(-1, self.num_kv_heads, self.head_dim), k_cache, v_cache,
                    self.k_scale, self.v_scale, self.k_dscale, self.v_dscale, self.side_k,
                    self.side_v, self.out_idx2d, self.head_n_out, context.slot_mapping,
                    context.block_tables, context.context_lens, self.scale)
        if fuse_append and self.kv_cache_is_int8:
            with self._profile("attention.paged_decode"):
                return paged_decode_append_int8_tokhead(
                    q.view(-1, self.num_heads, self.head_dim),
                    k.view(-1, self.num_kv_heads, self.head_dim),
                    v.view(-1, self.num_kv_heads, self.head_dim), k_cache, v_cache,
                    self.k_scale, self.v_scale, context.slot_mapping, context.block_tables,
                    context.context_lens, self.scale)
        if fuse_append:
            with self._profile("attention.paged_decode"):
                return paged_decode_append(
                    q.view(-1, self.num_heads, self.head_dim),
                    k.view(-1, self.num_kv_heads, self.head_dim),
                    v.view(-1, self.num_kv_heads, self.head_dim), k_cache, v_cache,
                    context.slot_mapping, context.block_tables, context.context_lens, self.scale)
        with self._profile("attention.paged_decode"):
            return paged_decode_attention(
                q, k_cache, v_cache, context.block_tables, context.context_lens, self.scale,
                context.max_context_len, k_scale=rk, v_scale=rv,
                side_k=self.side_k if side else None,
                side_v=self.side_v if side else None,
                out_idx2d=self.out_idx2d if side else None,
                head_n_out=self.head_n_out if side else None,
            )
