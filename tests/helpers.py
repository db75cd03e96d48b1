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


def assert_attention_close(out: torch.Tensor, ref: np.ndarray, label: str,
                           max_abs: float = MAX_ABS, mean_abs: float = MEAN_ABS) -> tuple[float, float]:
    got = out.detach().float().cpu().numpy()
    assert got.shape == ref.shape, (label, got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{label}: NaN pattern differs"
    finite = ~nan_ref
    if not finite.any():
        return 0.0, 0.0
    err = np.abs(got[finite] - ref[finite])
    # The output is bf16: rounding it alone costs up to half a bf16 ulp
    # (2^-9 relative), which exceeds an absolute 2e-2 once |out| > 10 (the int8
    # outlier-channel cases).  The max-abs bound therefore carries that term.
    bound = max_abs + np.abs(ref[finite]) * 2.0 ** -8
    worst = float((err - bound).max())
    mx, mn = float(err.max()), float(err.mean())
    assert worst <= 0.0, f"{label}: max_abs {mx:.3e} exceeds {max_abs} + 2^-8|ref|"
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
