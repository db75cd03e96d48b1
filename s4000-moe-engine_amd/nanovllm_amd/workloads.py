"""Seeded synthetic workloads for the paged KV path (inputs only).

Shapes follow the engine's production geometry (Qwen3-0.6B / Qwen3-30B-A3B
attention, page 256).  Everything is generated with explicit torch.Generator
seeds so a GPU run, the CPU oracle and the CPU baseline see the same bytes:
random data is drawn on the CPU, then moved to the target device.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

PAGE = 256
HEAD_DIM = 128


@dataclass
class DecodeWorkload:
    q: torch.Tensor               # [B, H, D] bf16
    k_cache: torch.Tensor         # [blocks, page, KVH, D]
    v_cache: torch.Tensor
    block_tables: torch.Tensor    # [B, max_blocks] int32, -1 padded
    context_lens: torch.Tensor    # [B] int32 (after the step's append)
    slot_mapping: torch.Tensor    # [B] int32, slot of each sequence's new token
    new_k: torch.Tensor           # [B, KVH, D] bf16 token appended this step
    new_v: torch.Tensor
    scale: float
    k_scale: torch.Tensor | None = None   # int8 per-token-head scales [blocks, page, KVH]
    v_scale: torch.Tensor | None = None

    @property
    def batch(self) -> int:
        return self.q.size(0)


def _randn(shape, gen, dtype=torch.bfloat16, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(dtype)


def build_block_tables(context_lens: list[int], num_blocks: int, page: int,
                       gen: torch.Generator, contiguous: bool = False) -> torch.Tensor:
    """Non-contiguous tables: a seeded permutation of the pool, consumed in
    order (every sequence owns distinct blocks)."""
    need = [max(1, (n + page - 1) // page) for n in context_lens]
    total = sum(need)
    if total > num_blocks:
        raise ValueError(f"{total} blocks needed, pool has {num_blocks}")
    order = torch.arange(num_blocks) if contiguous else torch.randperm(num_blocks, generator=gen)
    width = max(need)
    bt = torch.full((len(context_lens), width), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(need):
        bt[i, :n] = order[pos:pos + n].to(torch.int32)
        pos += n
    return bt


def slots_for_last_token(block_tables: torch.Tensor, context_lens: list[int], page: int) -> torch.Tensor:
    """slot = block_table[(len-1)//page] * page + (len-1) % page
    (the decode slot of nanovllm/engine/model_runner.py:685)."""
    out = []
    for i, n in enumerate(context_lens):
        out.append(int(block_tables[i, (n - 1) // page]) * page + (n - 1) % page)
    return torch.tensor(out, dtype=torch.int32)


def decode_workload(batch: int, num_heads: int, num_kv_heads: int, num_blocks: int,
                    context_lens: list[int], seed: int, device: str | torch.device = "cpu",
                    page: int = PAGE, fill_std: float = 1.0, pool_device_fill: bool = False,
                    kv_dtype: str = "bf16") -> DecodeWorkload:
    """A decode step: every sequence appends one token at position len-1 and
    then attends over len tokens (context_lens are the lengths after append).

    pool_device_fill draws the pool with a device generator (multi-GiB pools
    at full size); the small parity cases draw on the CPU."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    bt = build_block_tables(context_lens, num_blocks, page, gen)
    slots = slots_for_last_token(bt, context_lens, page)
    q = _randn((batch, num_heads, HEAD_DIM), gen)
    new_k = _randn((batch, num_kv_heads, HEAD_DIM), gen)
    new_v = _randn((batch, num_kv_heads, HEAD_DIM), gen)
    shape = (num_blocks, page, num_kv_heads, HEAD_DIM)
    sshape = (num_blocks, page, num_kv_heads)
    k_scale = v_scale = None
    if pool_device_fill:
        dgen = torch.Generator(device=device).manual_seed(seed + 1)
        if kv_dtype == "int8_tokhead":
            k_cache = torch.randint(-127, 128, shape, generator=dgen, device=device, dtype=torch.int8)
            v_cache = torch.randint(-127, 128, shape, generator=dgen, device=device, dtype=torch.int8)
            k_scale = torch.rand(sshape, generator=dgen, device=device) * 0.03 + 0.005
            v_scale = torch.rand(sshape, generator=dgen, device=device) * 0.03 + 0.005
        else:
            k_cache = torch.randn(shape, generator=dgen, device=device, dtype=torch.bfloat16)
            v_cache = torch.randn(shape, generator=dgen, device=device, dtype=torch.bfloat16)
            if fill_std != 1.0:
                k_cache.mul_(fill_std)
                v_cache.mul_(fill_std)
    elif kv_dtype == "int8_tokhead":
        k_cache = torch.randint(-127, 128, shape, generator=gen, dtype=torch.int8).to(device)
        v_cache = torch.randint(-127, 128, shape, generator=gen, dtype=torch.int8).to(device)
        k_scale = (torch.rand(sshape, generator=gen) * 0.03 + 0.005).to(device)
        v_scale = (torch.rand(sshape, generator=gen) * 0.03 + 0.005).to(device)
    else:
        k_cache = _randn(shape, gen, std=fill_std).to(device)
        v_cache = _randn(shape, gen, std=fill_std).to(device)
    return DecodeWorkload(
        q=q.to(device), k_cache=k_cache, v_cache=v_cache, block_tables=bt.to(device),
        context_lens=torch.tensor(context_lens, dtype=torch.int32).to(device),
        slot_mapping=slots.to(device), new_k=new_k.to(device), new_v=new_v.to(device),
        scale=HEAD_DIM ** -0.5, k_scale=k_scale, v_scale=v_scale)


def uniform_lengths(batch: int, lo: int, hi: int, seed: int) -> list[int]:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()


def outlier_keys(shape, seed: int, frac: float = 0.01, mult: float = 20.0) -> torch.Tensor:
    """K ~ N(0,1) with a fraction of entries scaled by `mult` (the int8 KV
    workload's outliers)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(shape, generator=gen)
    mask = torch.rand(shape, generator=gen) < frac
    x = torch.where(mask, x * mult, x)
    return x.to(torch.bfloat16)


@dataclass
class Int8DecodeWorkload(DecodeWorkload):
    raw_k: torch.Tensor | None = None     # [history tokens, KVH, D] bf16 appended before the step
    raw_v: torch.Tensor | None = None
    history_slots: torch.Tensor | None = None   # [history tokens] int32, their slots


def int8_tokhead_decode_workload(batch: int, num_heads: int, num_kv_heads: int,
                                 num_blocks: int, context_lens: list[int], seed: int,
                                 device, page: int = PAGE, outlier_frac: float = 0.01,
                                 outlier_mult: float = 20.0, keep_raw: bool = False
                                 ) -> Int8DecodeWorkload:
    """The per-token-head int8 decode workload: K ~ N(0,1) with a fraction
    `outlier_frac` of entries scaled by `outlier_mult`, V ~ N(0,1), drawn in
    bf16 on the device with a seeded generator and appended through the
    quantiser (kvc_store_int8_tokhead), so the pool holds the codes and
    scales the append produces.  Positions 0 .. len-2 of every sequence are
    the history; position len-1 is the step's own append (new_k / new_v,
    slot_mapping), left to the caller.  keep_raw keeps the history's bf16
    rows and slots for checking."""
    from .kernels.kv_int8 import store_kvcache_int8_tokhead
    gen = torch.Generator(device="cpu").manual_seed(seed)
    bt = build_block_tables(context_lens, num_blocks, page, gen)
    slots = slots_for_last_token(bt, context_lens, page)
    q = _randn((batch, num_heads, HEAD_DIM), gen).to(device)
    dgen = torch.Generator(device=device).manual_seed(seed + 1)

    def draw(n, outliers):
        x = torch.randn((n, num_kv_heads, HEAD_DIM), generator=dgen, device=device)
        if outliers:
            hit = torch.rand(x.shape, generator=dgen, device=device) < outlier_frac
            x = torch.where(hit, x * outlier_mult, x)
        return x.to(torch.bfloat16)

    shape = (num_blocks, page, num_kv_heads, HEAD_DIM)
    k_cache = torch.zeros(shape, dtype=torch.int8, device=device)
    v_cache = torch.zeros(shape, dtype=torch.int8, device=device)
    k_scale = torch.ones(shape[:3], dtype=torch.float32, device=device)
    v_scale = torch.ones(shape[:3], dtype=torch.float32, device=device)
    # history slots, sequence by sequence
    hist = []
    bt_dev = bt.to(device)
    for i, n in enumerate(context_lens):
        if n > 1:
            pos = torch.arange(n - 1, device=device)
            hist.append((bt_dev[i, pos // page].long() * page + pos % page).to(torch.int32))
    hslots = torch.cat(hist) if hist else torch.zeros(0, dtype=torch.int32, device=device)
    raw_k = draw(hslots.numel(), True)
    raw_v = draw(hslots.numel(), False)
    if hslots.numel():
        store_kvcache_int8_tokhead(raw_k, raw_v, k_cache, v_cache, k_scale, v_scale, hslots)
    new_k = draw(batch, True)
    new_v = draw(batch, False)
    if not keep_raw:
        raw_k = raw_v = hslots = None
    return Int8DecodeWorkload(
        q=q, k_cache=k_cache, v_cache=v_cache, block_tables=bt_dev,
        context_lens=torch.tensor(context_lens, dtype=torch.int32).to(device),
        slot_mapping=slots.to(device), new_k=new_k, new_v=new_v, scale=HEAD_DIM ** -0.5,
        k_scale=k_scale, v_scale=v_scale, raw_k=raw_k, raw_v=raw_v, history_slots=hslots)
