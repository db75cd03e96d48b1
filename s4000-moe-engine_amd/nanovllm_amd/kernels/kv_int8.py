"""int8 KV cache: quantise on append, dequantise on read (libkvc).

Two encodings share the int8 pool layout [blocks, page, KVH, D]:

* per-channel with a bf16 outlier side pool — the engine's current layout and
  the signature of nanovllm/kernels/kv_int8.py:72-107:
    code = clamp(floor(x / s[h, d] + 0.5), -127, 127), outlier dims zeroed,
    exact bf16 outlier values in side[slot, h, :head_n_out[h]];
* per-token-per-head — the layout of benchmarks/archive/P17-kv-int8.md:9-11
  with the arithmetic of scripts/archive/p14_int8_kv_probe.py:37-46:
    s = max(amax_d |x|, 1e-6) / 127 (fp32), code = clamp(rint(x / s), -127, 127)
  with rint rounding half to even; scales [blocks, page, KVH] fp32.

store_kvcache_int8 picks the encoding from k_scale: [KVH, D] is per-channel,
[blocks, page, KVH] is per-token-head (side pools then unused).
"""
from __future__ import annotations

import torch

from .. import _native as nat


def _slots(slot_mapping: torch.Tensor) -> tuple[torch.Tensor, int]:
    if slot_mapping.dtype == torch.int64:
        return slot_mapping.contiguous(), 8
    if slot_mapping.dtype != torch.int32:
        slot_mapping = slot_mapping.to(torch.int32)
    return slot_mapping.contiguous(), 4


def _check_rows(key: torch.Tensor, value: torch.Tensor) -> None:
    # Same preconditions as kv_int8.py:79-80 (per-row contiguity of [KVH, D]).
    N, KVH, D = key.shape
    assert key.stride(2) == 1 and value.stride(2) == 1
    assert key.stride(1) == D and value.stride(1) == D
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise ValueError("int8 append takes bf16 key/value")


def store_kvcache_int8_tokhead(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping):
    """Per-token-per-head append: codes into k_cache/v_cache [blocks, page, KVH, D]
    int8, scales into k_scale/v_scale [blocks, page, KVH] fp32."""
    _check_rows(key, value)
    N, KVH, D = key.shape
    nat.require_device(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)
    assert slot_mapping.numel() == N
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    assert k_scale.is_contiguous() and v_scale.is_contiguous()
    if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        raise ValueError("per-token-head scales are fp32")
    num_slots = k_cache.numel() // (KVH * D)
    slots, sb = _slots(slot_mapping)
    nat.call("kvc_store_int8_tokhead",
             key.data_ptr(), key.stride(0), key.stride(1),
             value.data_ptr(), value.stride(0), value.stride(1),
             k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
             num_slots, slots.data_ptr(), sb, N, KVH, D, nat.stream_of(key))


def store_kvcache_int8(key, value, k_cache, v_cache, k_scale, v_scale,
                       side_k, side_v, out_idx2d, head_n_out, slot_mapping):
    """key/value: [N, KVH, D] bf16; k/v_cache: int8 per-layer [blocks, page, KVH, D].

    Per-channel mode (k_scale [KVH, D]): side_k/side_v bf16 [blocks, page, KVH,
    N_OUT_MAX], out_idx2d int32 [KVH, N_OUT_MAX], head_n_out int32 [KVH].
    Per-token-head mode (k_scale [blocks, page, KVH]): side arguments ignored.
    """
    if k_scale is not None and k_scale.dim() == 3:
        return store_kvcache_int8_tokhead(key, value, k_cache, v_cache, k_scale, v_scale,
                                          slot_mapping)
    _check_rows(key, value)
    N, KVH, D = key.shape
    nat.require_device(key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)
    assert slot_mapping.numel() == N
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    k_scale = k_scale.to(torch.float32).contiguous()
    v_scale = v_scale.to(torch.float32).contiguous()
    has_side = side_k is not None and head_n_out is not None
    n_out_max = side_k.shape[-1] if has_side else 0
    if has_side:
        assert side_k.is_contiguous() and side_v.is_contiguous()
        out_idx2d = out_idx2d.to(torch.int32).contiguous()
        head_n_out = head_n_out.to(torch.int32).contiguous()
    num_slots = k_cache.numel() // (KVH * D)
    slots, sb = _slots(slot_mapping)
    nat.call("kvc_store_int8_chan",
             key.data_ptr(), key.stride(0), key.stride(1),
             value.data_ptr(), value.stride(0), value.stride(1),
             k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
             nat.ptr(side_k) if has_side else None, nat.ptr(side_v) if has_side else None,
             n_out_max,
             nat.ptr(out_idx2d) if has_side else None, nat.ptr(head_n_out) if has_side else None,
             num_slots, slots.data_ptr(), sb, N, KVH, D, nat.stream_of(key))


def dequant_gathered(kv_i8, dscale, side, out_idx2d, head_n_out):
    """kv_i8 [T, KVH, D] int8; dscale [KVH, D] (0 at outlier dims); side
    [T, KVH, N_OUT_MAX] bf16; out_idx2d [KVH, N_OUT_MAX] -> bf16 [T, KVH, D]
    (kv_int8.py:96-107, without its per-head host loop)."""
    T, KVH, D = kv_i8.shape
    nat.require_device(kv_i8, dscale)
    kv_i8 = kv_i8.contiguous()
    dscale = dscale.to(torch.float32).contiguous()
    out = torch.empty((T, KVH, D), dtype=torch.bfloat16, device=kv_i8.device)
    has_side = side is not None and head_n_out is not None
    if has_side:
        side = side.contiguous()
        out_idx2d = out_idx2d.to(torch.int32).contiguous()
        head_n_out = head_n_out.to(torch.int32).contiguous()
    nat.call("kvc_dequant_chan", kv_i8.data_ptr(), dscale.data_ptr(),
             nat.ptr(side) if has_side else None,
             nat.ptr(out_idx2d) if has_side else None,
             nat.ptr(head_n_out) if has_side else None,
             side.shape[-1] if has_side else 0, T, KVH, D, out.data_ptr(),
             nat.stream_of(kv_i8))
    return out


def dequant_tokhead(kv_i8, scale):
    """kv_i8 [T, KVH, D] int8, scale [T, KVH] fp32 -> bf16 (code * scale)
    (p14_int8_kv_probe.py:45-46)."""
    T, KVH, D = kv_i8.shape
    nat.require_device(kv_i8, scale)
    kv_i8 = kv_i8.contiguous()
    scale = scale.to(torch.float32).contiguous()
    out = torch.empty((T, KVH, D), dtype=torch.bfloat16, device=kv_i8.device)
    nat.call("kvc_dequant_tokhead", kv_i8.data_ptr(), scale.data_ptr(), T, KVH, D,
             out.data_ptr(), nat.stream_of(kv_i8))
    return out


def kv_calib_observe(key, value, amax, abs_sum):
    """Fold one forward's key/value rows [N, KVH, 128] (bf16, views fine)
    into a layer's per-channel statistics: amax [2, KVH, 128] fp32 (running
    max of |x|) and abs_sum (running sum of |x|), K in [0], V in [1]."""
    if key.ndim != 3 or value.shape != key.shape:
        raise ValueError("expected key/value [tokens, kv_heads, dim]")
    N, KVH, D = key.shape
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise ValueError("calibration observes bf16 key/value")
    assert key.stride(2) == 1 and value.stride(2) == 1
    assert amax.shape == (2, KVH, D) and abs_sum.shape == (2, KVH, D)
    assert amax.dtype == abs_sum.dtype == torch.float32
    assert amax.is_contiguous() and abs_sum.is_contiguous()
    nat.require_device(key, value, amax, abs_sum)
    nat.call("kvc_kv_calib_observe", key.data_ptr(), key.stride(0), key.stride(1),
             value.data_ptr(), value.stride(0), value.stride(1), N, KVH, D, amax.data_ptr(),
             abs_sum.data_ptr(), nat.stream_of(key))


def kv_calib_freeze(amax, abs_sum, count, k_scale, v_scale, k_dscale, v_dscale, out_idx2d,
                    head_n_out):
    """Freeze one layer's statistics over `count` tokens into store scales,
    read scales (0 at outlier dims) and the per-head outlier dims (ratio
    amax / mean|x| > 10 for K or V, the first out_idx2d.size(-1) of them per
    head), all in place, on the device."""
    KVH, D = k_scale.shape
    n_out_max = out_idx2d.size(-1)
    for t in (k_scale, v_scale, k_dscale, v_dscale):
        assert t.shape == (KVH, D) and t.dtype == torch.float32 and t.is_contiguous()
    assert out_idx2d.shape == (KVH, n_out_max) and out_idx2d.dtype == torch.int32
    assert head_n_out.shape == (KVH,) and head_n_out.dtype == torch.int32
    assert out_idx2d.is_contiguous() and head_n_out.is_contiguous()
    assert amax.shape == abs_sum.shape == (2, KVH, D)
    nat.require_device(amax, abs_sum, k_scale, v_scale, k_dscale, v_dscale, out_idx2d,
                       head_n_out)
    nat.call("kvc_kv_calib_freeze", amax.data_ptr(), abs_sum.data_ptr(), int(count), KVH, D,
             n_out_max, k_scale.data_ptr(), v_scale.data_ptr(), k_dscale.data_ptr(),
             v_dscale.data_ptr(), out_idx2d.data_ptr(), head_n_out.data_ptr(),
             nat.stream_of(amax))
