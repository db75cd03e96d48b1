"""Shared helpers of the parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import kv_oracle as ko

# Attention tolerance against the fp32 reference (bf16 outputs).
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def bits(t: torch.Tensor) -> np.ndarray:
    return ko.torch_bf16_bits(t)


def half_ulp_bf16(x: np.ndarray) -> np.ndarray:
    """Half a bf16 ulp at |x|: 2^(floor(log2|x|) - 8) (8 significant bits),
    the most that rounding a value of that binade to bf16 can move it."""
    ax = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(ax > 0, ax, 1.0)))
    return np.where(ax > 0, np.exp2(e - 8.0), 0.0)


def attention_bound(ref: np.ndarray, max_abs: float = MAX_ABS) -> np.ndarray:
    """Per-element max-abs bound: the bare max_abs, plus half a bf16 ulp of
    the reference only where that half ulp itself exceeds max_abs (|ref| >= 8
    for 2e-2: the output is bf16, and its rounding alone can cost that much)."""
    h = half_ulp_bf16(ref)
    return max_abs + np.where(h > max_abs, h, 0.0)


def assert_attention_close(out: torch.Tensor, ref: np.ndarray, label: str,
                           max_abs: float = MAX_ABS, mean_abs: float = MEAN_ABS) -> tuple[float, float]:
    got = out.detach().float().cpu().numpy()
    assert got.shape == ref.shape, (label, got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{label}: NaN pattern differs"
    finite = ~nan_ref
    if not finite.any():
        print(f"[tol] {label}: every row NaN (as the reference)", flush=True)
        return 0.0, 0.0
    err = np.abs(got[finite] - ref[finite])
    bound = attention_bound(ref[finite], max_abs)
    worst = float((err - bound).max())
    mx, mn = float(err.max()), float(err.mean())
    widened = int((bound > max_abs).sum())
    print(f"[tol] {label}: max_abs {mx:.3e} mean_abs {mn:.3e} "
          f"({widened} of {err.size} elements have |ref| >= 8)", flush=True)
    assert worst <= 0.0, (f"{label}: max_abs {mx:.3e} exceeds {max_abs} "
                          f"(+ half a bf16 ulp where that exceeds {max_abs})")
    assert mn <= mean_abs, f"{label}: mean_abs {mn:.3e} > {mean_abs}"
    return mx, mn


def gathered_pool(cache: torch.Tensor, block_tables: torch.Tensor):
    """Copy only the blocks the tables reference to the host, renumbered, so the
    oracle can run on multi-GiB pools.  Returns (pool_np_bits_or_values, tables)."""
    bt = block_tables.cpu()
    used = torch.unique(bt[bt >= 0])
    remap = torch.full((cache.size(0),), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    small = cache.index_select(0, used.to(cache.device)).cpu()
    new_bt = torch.where(bt >= 0, remap[bt.clamp(min=0).long()], torch.full_like(bt, -1, dtype=torch.int64))
    return small, new_bt.numpy()


def kv_float_from_torch(cache: torch.Tensor) -> np.ndarray:
    if cache.dtype == torch.bfloat16:
        return ko.bf16_to_f32(bits(cache))
    raise TypeError(cache.dtype)


def p17_unit_inputs():
    """The per-channel int8 unit case of tests/p17_kv_int8.py:64-136 (N=512,
    KVH=8, D=128, seed 7, 4 outlier dims per head at most): key, value, the
    write scales s_k/s_v, the read scales ds_k/ds_v (0 at outlier dims),
    out_idx2d and head_n_out."""
    N, KVH, D, N_OUT_MAX = 512, 8, 128, 4
    g = torch.Generator(device="cpu").manual_seed(7)
    key = (torch.randn(N, KVH, D, generator=g) * 0.7).to(torch.bfloat16)
    value = (torch.randn(N, KVH, D, generator=g) * 0.7).to(torch.bfloat16)
    key[:8] *= 8.0
    key[:, 0, :4] *= 60.0
    key[:, 1, 10] *= 120.0
    value[:, 2, :4] *= 60.0
    kf, vf = key.float(), value.float()
    amax_k, amax_v = kf.abs().amax(0), vf.abs().amax(0)
    typ_k = kf.abs().mean(0).clamp_min(1e-6)
    typ_v = vf.abs().mean(0).clamp_min(1e-6)
    s_k = (amax_k / 127.0).clamp_min(1e-6)
    s_v = (amax_v / 127.0).clamp_min(1e-6)
    ratio = torch.maximum(amax_k / typ_k, amax_v / typ_v)
    out_idx2d = torch.zeros(KVH, N_OUT_MAX, dtype=torch.int32)
    head_n_out = torch.zeros(KVH, dtype=torch.int32)
    for h in range(KVH):
        dims = ratio[h].nonzero().flatten()
        dims = dims[ratio[h, dims] > 10.0][:N_OUT_MAX]
        out_idx2d[h, :dims.numel()] = dims.to(torch.int32)
        head_n_out[h] = dims.numel()
    ds_k, ds_v = s_k.clone(), s_v.clone()
    for h in range(KVH):
        n_h = int(head_n_out[h])
        ds_k[h, out_idx2d[h, :n_h].long()] = 0.0
        ds_v[h, out_idx2d[h, :n_h].long()] = 0.0
    return key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out
