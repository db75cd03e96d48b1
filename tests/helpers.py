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


def _column(n: int, counts: dict) -> torch.Tensor:
    """A column of n tokens holding `counts[value]` copies of each value
    (every value exact in bf16), zeros elsewhere."""
    vals = [v for v, c in counts.items() for _ in range(c)]
    assert len(vals) <= n
    return torch.tensor(vals + [0.0] * (n - len(vals)))


# Forward lengths of the ratio-flip calibration case and, per flip dim, each
# forward's column: one 8.0 (the amax) plus 2.0 / 1.0 / 0.75 terms.  Over the
# 900 tokens a dim is an outlier iff its sum of |x| < 720 (ratio 8 * 900 /
# sum > 10).
#   dim "hook_in":  sums 239.75 + 199.75 + 279.75 = 719.25 in fp32 (outlier);
#                   each rounds up to bf16: 240 + 200 + 280 = 720 (ratio 10: not)
#   dim "hook_out": sums 239.25 + 200.25 + 280.5 = 720.0 in fp32 (ratio 10: not);
#                   each rounds down: 239 + 200 + 280 = 719 (outlier)
CALIB_FLIP_LENGTHS = (300, 250, 350)
CALIB_FLIP_COLUMNS = {
    "hook_in": ({8.0: 1, 1.0: 30, 0.75: 269}, {8.0: 1, 2.0: 4, 0.75: 245},
                {8.0: 1, 2.0: 8, 0.75: 341}),
    "hook_out": ({8.0: 1, 2.0: 5, 1.0: 3, 0.75: 291}, {8.0: 1, 2.0: 4, 1.0: 2, 0.75: 243},
                 {8.0: 1, 2.0: 8, 1.0: 3, 0.75: 338}),
}


def calib_flip_forwards(kvh: int = 4, d: int = 128, seed: int = 21):
    """Three calibration forwards (key, value bf16 [n_i, kvh, d]) with two
    dims of head 0 whose outlier decision flips between fp32 sums and the
    engine's bf16-rounded per-forward sums (CALIB_FLIP_COLUMNS), a 60x
    outlier channel in head 1, and N(0, 0.7^2) elsewhere (ratio about 4.5).
    Returns (forwards, dims) with dims = {"hook_in": 3, "hook_out": 77}."""
    g = torch.Generator().manual_seed(seed)
    dims = {"hook_in": 3, "hook_out": 77}
    forwards = []
    for i, n in enumerate(CALIB_FLIP_LENGTHS):
        key = torch.randn(n, kvh, d, generator=g) * 0.7
        value = torch.randn(n, kvh, d, generator=g) * 0.7
        key[n // 2, 1, 40] = 40.0
        for name, dim in dims.items():
            col = _column(n, CALIB_FLIP_COLUMNS[name][i])
            key[:, 0, dim] = col[torch.randperm(n, generator=g)]
            value[:, 0, dim] = 0.5        # V ratio 1: K alone decides
        forwards.append((key.to(torch.bfloat16), value.to(torch.bfloat16)))
    return forwards, dims


def torch_hook_stats(forwards):
    """The engine's forward pre-hook statements (model_runner.py:527-533),
    run in CPU torch on the observed rows: per-forward amax and bf16 sum of
    |x|, folded with torch.maximum and fp32 adds.  Returns
    (amax_k, amax_v, sum_k, sum_v, n) as fp32 numpy."""
    buf = {"k": None, "v": None, "k_sum": None, "v_sum": None, "n": 0}
    for k, v in forwards:
        kf = k.detach().abs().amax(dim=0).float()
        vf = v.detach().abs().amax(dim=0).float()
        buf["k"] = kf if buf["k"] is None else torch.maximum(buf["k"], kf)
        buf["v"] = vf if buf["v"] is None else torch.maximum(buf["v"], vf)
        ks = k.detach().abs().sum(dim=0)
        vs = v.detach().abs().sum(dim=0)
        assert ks.dtype == torch.bfloat16        # the hook's sum is bf16
        buf["k_sum"] = ks.float() if buf["k_sum"] is None else buf["k_sum"] + ks.float()
        buf["v_sum"] = vs.float() if buf["v_sum"] is None else buf["v_sum"] + vs.float()
        buf["n"] += k.shape[0]
    return (buf["k"].numpy(), buf["v"].numpy(), buf["k_sum"].numpy(), buf["v_sum"].numpy(),
            buf["n"])
