"""CPU restatement of the reference's paged-KV algorithms (test infrastructure).

bf16 tensors travel as uint16 bit patterns (numpy has no bfloat16); helpers
convert with round-to-nearest-even, the rounding torch's .to(bfloat16) uses.
"""
from __future__ import annotations

import math

import numpy as np
import torch

# ---------------------------------------------------------------------------
# bf16 <-> fp32 bit helpers
# ---------------------------------------------------------------------------


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def torch_bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_torch_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16)


# ---------------------------------------------------------------------------
# P1 — append through slot_mapping
# ---------------------------------------------------------------------------


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping: np.ndarray) -> None:
    """nanovllm/layers/attention.py:9-30: flat_k[slot_mapping] = key.reshape(N, KVH*D).

    Arrays are raw element bits of any width ([N, KVH, D] and
    [blocks, page, KVH, D]); negative slots index from the end, as the
    reference's integer index_put does."""
    n = key.shape[0]
    row = key.shape[1] * key.shape[2]
    flat_k = k_cache.reshape(-1, row)
    flat_v = v_cache.reshape(-1, row)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    flat_k[slots] = key.reshape(n, row)
    flat_v[slots] = value.reshape(n, row)


# ---------------------------------------------------------------------------
# P3 — int8 quantise / dequantise
# ---------------------------------------------------------------------------


def quant_tokhead(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token-per-head symmetric int8 (scripts/archive/p14_int8_kv_probe.py:37-41):
    amax = |x|.amax(-1) (bf16, exact) -> fp32 -> clamp_min(1e-6); s = amax / 127;
    code = round_half_even(x / s).clamp(-127, 127).  x_bits [..., D] bf16 bits.
    Returns (codes int8 [..., D], scales fp32 [...])."""
    x = bf16_to_f32(x_bits)
    amax = np.abs(x).max(axis=-1)
    amax = np.maximum(amax, np.float32(1e-6)).astype(np.float32)
    s = (amax / np.float32(127.0)).astype(np.float32)
    q = np.rint((x / s[..., None]).astype(np.float32))
    q = np.clip(q, -127, 127)
    return q.astype(np.int8), s


def store_int8_tokhead(key_bits, value_bits, k_codes, v_codes, k_scale, v_scale, slot_mapping):
    """Per-token-head append into the P17 layout (benchmarks/archive/P17-kv-int8.md:9-11):
    codes [blocks, page, KVH, D] int8, scales [blocks, page, KVH] fp32."""
    kq, ks = quant_tokhead(key_bits)
    vq, vs = quant_tokhead(value_bits)
    kvh, d = key_bits.shape[1], key_bits.shape[2]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    k_codes.reshape(-1, kvh, d)[slots] = kq
    v_codes.reshape(-1, kvh, d)[slots] = vq
    k_scale.reshape(-1, kvh)[slots] = ks
    v_scale.reshape(-1, kvh)[slots] = vs


def quant_chan(x_bits: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Per-channel int8 (nanovllm/kernels/kv_int8.py:53-60, tests/p17_kv_int8.py:47-48):
    code = clamp(floor(x / s + 0.5), -127, 127), all in fp32."""
    x = bf16_to_f32(x_bits)
    q = np.floor((x / scale).astype(np.float32) + np.float32(0.5))
    return np.clip(q, -127, 127).astype(np.int8)


def store_int8_chan(key_bits, value_bits, k_codes, v_codes, k_scale, v_scale, side_k, side_v,
                    out_idx2d, head_n_out, slot_mapping):
    """tests/p17_kv_int8.py:39-61 (the bitwise spec of kv_int8.py:29-69):
    per-channel codes, outlier dims zeroed, exact bf16 outlier values in the
    compacted per-head side row.  side_* are bf16 bits [blocks, page, KVH, NOUT]."""
    n, kvh, d = key_bits.shape
    kq = quant_chan(key_bits, k_scale)
    vq = quant_chan(value_bits, v_scale)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    nout = side_k.shape[-1] if side_k is not None else 0
    for h in range(kvh):
        n_h = int(head_n_out[h]) if head_n_out is not None else 0
        if n_h:
            dims = np.asarray(out_idx2d[h, :n_h], dtype=np.int64)
            kq[:, h, dims] = 0
            vq[:, h, dims] = 0
            side_k.reshape(-1, kvh, nout)[slots, h, :n_h] = key_bits[:, h, dims]
            side_v.reshape(-1, kvh, nout)[slots, h, :n_h] = value_bits[:, h, dims]
    k_codes.reshape(-1, kvh, d)[slots] = kq
    v_codes.reshape(-1, kvh, d)[slots] = vq


def dequant_chan(codes: np.ndarray, dscale: np.ndarray, side_bits, out_idx2d, head_n_out):
    """nanovllm/kernels/kv_int8.py:96-107: bf16(fp32(code) * dscale), then the
    head's outlier dims take the side values.  Returns bf16 bits [T, KVH, D]."""
    out = f32_to_bf16(codes.astype(np.float32) * dscale.astype(np.float32))
    if side_bits is not None and head_n_out is not None:
        for h in range(codes.shape[1]):
            n_h = int(head_n_out[h])
            for j in range(n_h):
                out[:, h, int(out_idx2d[h, j])] = side_bits[:, h, j]
    return out


def dequant_tokhead(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """scripts/archive/p14_int8_kv_probe.py:45-46: bf16(fp32(code) * scale)."""
    return f32_to_bf16(codes.astype(np.float32) * scale.astype(np.float32)[..., None])


def f64_to_bf16_value(x: np.ndarray) -> np.ndarray:
    """Correctly rounded (ties to even) bf16 value of non-negative finite
    float64 numbers, returned as float32.  bf16 keeps 8 significant bits and
    fp32's exponent range: below 2^-126 its spacing is fixed at 2^-133."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty(x.shape, np.float32)
    flat, res = x.ravel(), out.ravel()
    for i, v in enumerate(flat):
        if v == 0.0:
            res[i] = 0.0
            continue
        e = max(math.frexp(v)[1] - 8, -133)       # bf16 spacing at v is 2^e
        q, r = divmod(v, math.ldexp(1.0, e))      # exact: v and 2^e are doubles
        half = math.ldexp(1.0, e - 1)
        if r > half or (r == half and int(q) % 2 == 1):
            q += 1.0
        y = math.ldexp(q, e)
        res[i] = np.float32(y) if y < 2.0 ** 128 else np.float32(np.inf)
    return out


def calib_stats(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The calibration hook's per-channel statistics of one forward's rows
    (nanovllm/engine/model_runner.py:522-532): x_bits [N, KVH, D] bf16 bits ->
    (amax of |x| over tokens, sum of |x| over tokens), fp32 [KVH, D].

    The hook sums a bf16 tensor (`k.abs().sum(dim=0)`), which torch returns
    in bf16 before `.float()`: the sum here is the exact one (float64 holds
    every partial sum of bf16 terms exactly while they span < 2^45) rounded
    once to bf16.  The caller adds these per-forward sums in fp32, as the
    hook's `buf["k_sum"] + ...` does."""
    a = np.abs(bf16_to_f32(x_bits))
    return a.max(axis=0), f64_to_bf16_value(a.astype(np.float64).sum(axis=0))


def calib_fold(forwards: list) -> tuple[np.ndarray, np.ndarray, int]:
    """The hook over several forwards (model_runner.py:527-533): running
    max of the per-forward amax, running fp32 sum of the per-forward
    (bf16-rounded) sums, token count.  forwards: list of [N_i, KVH, D] bf16
    bits."""
    amax, total, n = None, None, 0
    for x_bits in forwards:
        a, s = calib_stats(x_bits)
        amax = a if amax is None else np.maximum(amax, a)
        total = s if total is None else (total + s).astype(np.float32)
        n += x_bits.shape[0]
    return amax, total, n


def calib_freeze(amax_k, amax_v, sum_k, sum_v, count: int, n_out_max: int):
    """ModelRunner.kv_calibrate_freeze (model_runner.py:541-577) for one
    layer: scale = max(amax / 127, 1e-6); typ = max(sum / count, 1e-6);
    ratio = max(amax_k / typ_k, amax_v / typ_v); a head's outlier dims are
    its first n_out_max dims (index order) with ratio > 10; read scales are
    the scales with 0 at those dims.  All fp32.  Returns
    (s_k, s_v, ds_k, ds_v, out_idx2d [KVH, n_out_max] int32 (0 past
    head_n_out), head_n_out [KVH] int32)."""
    f = np.float32
    s_k = np.maximum((amax_k / f(127.0)).astype(f), f(1e-6))
    s_v = np.maximum((amax_v / f(127.0)).astype(f), f(1e-6))
    typ_k = np.maximum((sum_k / f(count)).astype(f), f(1e-6))
    typ_v = np.maximum((sum_v / f(count)).astype(f), f(1e-6))
    ratio = np.maximum((amax_k / typ_k).astype(f), (amax_v / typ_v).astype(f))
    kvh = amax_k.shape[0]
    out_idx2d = np.zeros((kvh, n_out_max), dtype=np.int32)
    head_n_out = np.zeros(kvh, dtype=np.int32)
    ds_k, ds_v = s_k.copy(), s_v.copy()
    for h in range(kvh):
        dims = np.nonzero(ratio[h] > f(10.0))[0][:n_out_max]
        out_idx2d[h, :dims.size] = dims
        head_n_out[h] = dims.size
        ds_k[h, dims] = 0.0
        ds_v[h, dims] = 0.0
    return s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out


# ---------------------------------------------------------------------------
# P2 — attention references (fp32)
# ---------------------------------------------------------------------------


def _gather_rows(cache: np.ndarray, block_row: np.ndarray, length: int) -> np.ndarray:
    page = cache.shape[1]
    nblk = (length + page - 1) // page
    blocks = np.asarray(block_row[:nblk], dtype=np.int64)
    return cache[blocks].reshape(-1, *cache.shape[2:])[:length]


def kv_float(cache, fmt: str, scale=None, side=None, out_idx2d=None, head_n_out=None):
    """Pool -> fp32 values as the reference's read path sees them
    (paged_attention.py:138-145 and :169-172: int8 * scale kept in fp32; the
    side pool supplies exact outlier values)."""
    if fmt == "bf16":
        return bf16_to_f32(cache)
    if fmt == "int8_tokhead":
        return cache.astype(np.float32) * scale.astype(np.float32)[..., None]
    if fmt == "int8_chan":
        x = cache.astype(np.float32) * scale.astype(np.float32)
        if side is not None and head_n_out is not None:
            sf = bf16_to_f32(side)
            for h in range(cache.shape[-2]):
                for j in range(int(head_n_out[h])):
                    x[..., h, int(out_idx2d[h, j])] = sf[..., h, j]
        return x
    raise ValueError(fmt)


def kv_float_prefill(cache, fmt: str, scale=None, side=None, out_idx2d=None, head_n_out=None):
    """Pool -> fp32 values as the reference's prefill reads them
    (nanovllm/layers/attention.py:33-51, _gather_kv): an int8 pool is
    dequantised to bf16 (bf16(fp32(code) * scale), the side pool's exact
    values at the outlier dims) before the bf16 attention, i.e.
    dequant_chan / dequant_tokhead over the whole pool."""
    if fmt == "bf16":
        return bf16_to_f32(cache)
    if fmt == "int8_tokhead":
        return bf16_to_f32(dequant_tokhead(cache, scale))
    if fmt == "int8_chan":
        kvh, d = cache.shape[-2:]
        sb = None if side is None else side.reshape(-1, kvh, side.shape[-1])
        bits = dequant_chan(cache.reshape(-1, kvh, d), scale, sb, out_idx2d, head_n_out)
        return bf16_to_f32(bits.reshape(cache.shape))
    raise ValueError(fmt)


def attend_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                allowed: np.ndarray | None = None) -> np.ndarray:
    """softmax(q k^T * scale) v per head in fp32.  q [Sq, H, D]; k, v [Sk, KVH, D]
    fp32; allowed [Sq, Sk] bool or None.  GQA: q head h reads kv head h // G."""
    sq, nh, d = q.shape
    kvh = k.shape[1]
    g = nh // kvh
    out = np.empty((sq, nh, d), dtype=np.float32)
    for h in range(nh):
        kh = k[:, h // g]
        vh = v[:, h // g]
        logits = (q[:, h] @ kh.T).astype(np.float32) * np.float32(scale)
        if allowed is not None:
            logits = np.where(allowed, logits, -np.inf)
        m = logits.max(axis=1, keepdims=True)
        p = np.exp(logits - m)
        out[:, h] = (p @ vh) / p.sum(axis=1, keepdims=True)
    return out


def paged_decode_ref(q_bits, k_f32, v_f32, block_tables, context_lens, scale) -> np.ndarray:
    """Per-(sequence, head) fp32 decode reference (tests/archive/p5_paged_attention.py:9-27;
    semantics of paged_attention.py:92-190).  q_bits [B, H, D] bf16 bits;
    k_f32/v_f32 [blocks, page, KVH, D] fp32 (kv_float).  Returns fp32 [B, H, D];
    a zero-length context gives NaN rows, like the reference kernel's 0/0."""
    q = bf16_to_f32(q_bits)
    b, nh, d = q.shape
    out = np.empty((b, nh, d), dtype=np.float32)
    for i in range(b):
        n = int(context_lens[i])
        if n == 0:
            out[i] = np.nan
            continue
        k = _gather_rows(k_f32, block_tables[i], n)
        v = _gather_rows(v_f32, block_tables[i], n)
        out[i] = attend_rows(q[i][None], k, v, scale)[0]
    return out


def prefill_ref(q_bits, k_f32, v_f32, block_tables, cu_q, cu_k, scale, row_offset=0,
                fresh_k=None, fresh_v=None) -> np.ndarray:
    """nanovllm/layers/attention.py:179-213: per chunk i, queries at positions
    sk - sq .. sk - 1 attend keys j <= position (prefix mask :210-212); without
    block tables (fresh_k/fresh_v given) the keys are the chunk's own rows and
    the mask is causal (:195-199).  q_bits [T, H, D]; block_tables rows start at
    row_offset.  Returns fp32 [cu_q[-1], H, D]."""
    q = bf16_to_f32(q_bits)
    total = cu_q[-1]
    out = np.full((total, q.shape[1], q.shape[2]), np.nan, dtype=np.float32)
    for i in range(len(cu_q) - 1):
        sq, sk = cu_q[i + 1] - cu_q[i], cu_k[i + 1] - cu_k[i]
        if sq == 0 or sk == 0:
            continue
        if fresh_k is not None:
            k = fresh_k[cu_k[i]:cu_k[i + 1]]
            v = fresh_v[cu_k[i]:cu_k[i + 1]]
        else:
            k = _gather_rows(k_f32, block_tables[row_offset + i], sk)
            v = _gather_rows(v_f32, block_tables[row_offset + i], sk)
        pos = np.arange(sk - sq, sk)[:, None]
        allowed = np.arange(sk)[None, :] <= pos
        out[cu_q[i]:cu_q[i + 1]] = attend_rows(q[cu_q[i]:cu_q[i + 1]], k, v, scale, allowed)
    return out


def mixed_ref(q_bits, k_f32, v_f32, block_tables, num_decode_rows, decode_context_lens, cu_q, cu_k,
              scale, k_pre=None, v_pre=None) -> np.ndarray:
    """Mixed batch (attention.py:146-166): decode rows through the decode
    reference, then prefill rows with block table rows num_decode_rows + i.
    k_pre / v_pre: the pool as the prefill reads it, when that differs from
    the decode's read (an int8 pool: kv_float_prefill against kv_float)."""
    n = num_decode_rows
    dec = paged_decode_ref(q_bits[:n], k_f32, v_f32, block_tables[:n], decode_context_lens, scale)
    pre = prefill_ref(q_bits[n:], k_f32 if k_pre is None else k_pre,
                      v_f32 if v_pre is None else v_pre, block_tables, cu_q, cu_k, scale,
                      row_offset=n)
    return np.concatenate([dec, pre], axis=0)


def _masked_sdpa_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """attention.py:264-279 on gathered rows k, v [B, kv_len, KVH, D]: zero the
    rows past each context, expand the GQA heads, masked SDPA."""
    nh = q.shape[1]
    kv_len = k.size(1)
    valid = torch.arange(kv_len).unsqueeze(0) < context_lens.unsqueeze(1)
    kvh = k.size(2)
    idx = torch.arange(kvh).repeat_interleave(nh // kvh)
    qh = q.transpose(0, 1).unsqueeze(2)
    k = k.index_select(2, idx).permute(2, 0, 1, 3)
    v = v.index_select(2, idx).permute(2, 0, 1, 3)
    kv_valid = valid.unsqueeze(0).unsqueeze(-1)
    k = torch.where(kv_valid, k, torch.zeros((), dtype=k.dtype))
    v = torch.where(kv_valid, v, torch.zeros((), dtype=v.dtype))
    mask = valid.unsqueeze(0).unsqueeze(2)
    o = torch.nn.functional.scaled_dot_product_attention(qh, k, v, attn_mask=mask, scale=scale)
    return o.squeeze(2).permute(1, 0, 2)


def gather_sdpa_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                       max_context_len: int) -> torch.Tensor:
    """The reference's torch decode path (nanovllm/layers/attention.py:239-279) on
    CPU tensors: gather the padded block tables, zero invalid rows, expand GQA
    heads, masked SDPA.  This is the CPU baseline bench.py times."""
    bs = q.shape[0]
    page = k_cache.size(1)
    blocks = block_tables.clamp(min=0).long()
    full = block_tables.size(1) * page
    kv_len = max_context_len or full
    k = k_cache[blocks].view(bs, full, *k_cache.shape[-2:])[:, :kv_len]
    v = v_cache[blocks].view(bs, full, *v_cache.shape[-2:])[:, :kv_len]
    return _masked_sdpa_decode(q, k, v, context_lens, scale)


def _expand_heads(kv: torch.Tensor, num_heads: int, dim: int) -> torch.Tensor:
    """GQA expansion by index_select (nanovllm/layers/attention.py:54-61)."""
    kvh = kv.size(dim)
    if kvh == num_heads:
        return kv
    return kv.index_select(dim, torch.arange(kvh).repeat_interleave(num_heads // kvh))


def prefill_loop_torch(q: torch.Tensor, k_fresh: torch.Tensor, v_fresh: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, cu_q: list, cu_k: list,
                       block_tables: torch.Tensor | None, scale: float) -> torch.Tensor:
    """The reference's per-sequence prefill (nanovllm/layers/attention.py:179-213)
    on CPU tensors: for chunk i, without block tables causal SDPA over the
    chunk's own expanded k/v (:195-199); with them, gather sk cached tokens
    (_gather_kv :33-51 without the int8 branch), expand the kv heads and run
    SDPA under allowed[r, j] = j <= (sk - sq) + r (:200-212); outputs are
    concatenated in chunk order.  q [T, H, D]."""
    nh = q.size(1)
    page = k_cache.size(1)
    outs = []
    for i in range(len(cu_q) - 1):
        sq, sk = cu_q[i + 1] - cu_q[i], cu_k[i + 1] - cu_k[i]
        if sq == 0 or sk == 0:
            continue
        qi = q[cu_q[i]:cu_q[i + 1]].transpose(0, 1).contiguous()
        if block_tables is None:
            ki = _expand_heads(k_fresh[cu_k[i]:cu_k[i + 1]], nh, 1).transpose(0, 1).contiguous()
            vi = _expand_heads(v_fresh[cu_k[i]:cu_k[i + 1]], nh, 1).transpose(0, 1).contiguous()
            o = torch.nn.functional.scaled_dot_product_attention(
                qi.unsqueeze(0), ki.unsqueeze(0), vi.unsqueeze(0), scale=scale, is_causal=True)
        else:
            nblk = (sk + page - 1) // page
            blocks = block_tables[i][:nblk].long()
            kg = k_cache[blocks].view(-1, *k_cache.shape[-2:])[:sk]
            vg = v_cache[blocks].view(-1, *v_cache.shape[-2:])[:sk]
            ki = _expand_heads(kg, nh, 1).transpose(0, 1).contiguous()
            vi = _expand_heads(vg, nh, 1).transpose(0, 1).contiguous()
            pos = torch.arange(sk - sq, sk)
            allowed = torch.arange(sk) <= pos.unsqueeze(1)
            o = torch.nn.functional.scaled_dot_product_attention(
                qi.unsqueeze(0), ki.unsqueeze(0), vi.unsqueeze(0),
                attn_mask=allowed.unsqueeze(0), scale=scale)
        outs.append(o.squeeze(0))
    return torch.cat(outs, dim=1).transpose(0, 1)


def mixed_torch(q, k_cache, v_cache, block_tables, num_decode_rows, decode_context_lens,
                decode_max_context_len, cu_q, cu_k, scale) -> torch.Tensor:
    """The reference's mixed batch (attention.py:146-166) on CPU tensors: decode
    rows through the gather + SDPA decode, prefill rows through the
    per-sequence loop with block table rows num_decode_rows + i, then cat."""
    n = num_decode_rows
    out_dec = gather_sdpa_decode(q[:n], k_cache, v_cache, block_tables[:n], decode_context_lens,
                                 scale, decode_max_context_len)
    out_pre = prefill_loop_torch(q[n:], None, None, k_cache, v_cache, cu_q, cu_k,
                                 block_tables[n:], scale)
    return torch.cat([out_dec, out_pre], dim=0)


def quant_tokhead_torch(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """scripts/archive/p14_int8_kv_probe.py:37-41 as torch ops: amax over D
    (bf16) -> fp32 -> clamp_min(1e-6); s = amax / 127; codes =
    round(x / s) (half to even) clamped to +-127.  Returns (codes int8,
    scales fp32 [..., 1])."""
    amax = x.abs().amax(dim=-1, keepdim=True).float().clamp_min_(1e-6)
    s = amax / 127.0
    return (x.float() / s).round().clamp_(-127, 127).to(torch.int8), s


def gather_sdpa_decode_int8_tokhead(q, k_codes, v_codes, k_scale, v_scale, block_tables,
                                    context_lens, scale, max_context_len) -> torch.Tensor:
    """The torch decode path over a per-token-head int8 pool: gather the padded
    block tables' codes and scales (attention.py:251-254), dequantise with the
    p14 read path bf16(fp32(code) * scale) (p14_int8_kv_probe.py:45-46), then
    the masked SDPA of attention.py:264-279.  codes [blocks, page, KVH, D]
    int8, scales [blocks, page, KVH] fp32."""
    bs = q.size(0)
    page = k_codes.size(1)
    full = block_tables.size(1) * page
    kv_len = max_context_len or full
    blocks = block_tables.clamp(min=0).long()

    def deq(codes, sc):
        c = codes[blocks].view(bs, full, *codes.shape[-2:])[:, :kv_len]
        f = sc[blocks].view(bs, full, sc.size(-1))[:, :kv_len]
        return (c.float() * f.unsqueeze(-1)).to(torch.bfloat16)

    return _masked_sdpa_decode(q, deq(k_codes, k_scale), deq(v_codes, v_scale), context_lens,
                               scale)


# ---------------------------------------------------------------------------
# P4 — whole-block movement
# ---------------------------------------------------------------------------


def block_gather(pool: np.ndarray, ids) -> np.ndarray:
    """[planes, blocks, ...] -> [n, planes, ...]: kv_cache.index_select(2, idx)
    of ModelRunner.offload_put (nanovllm/engine/model_runner.py:284-298) and
    the per-pool index_select + permute of extract_kv (nanovllm/pd/kv_channel.py:54-69)."""
    ids = np.asarray(ids, dtype=np.int64)
    return np.ascontiguousarray(np.moveaxis(pool[:, ids], 1, 0))


def block_scatter(pool: np.ndarray, ids, items: np.ndarray) -> None:
    """pool[:, ids] = items moved back to [planes, n, ...]: index_copy_ of
    offload_get (model_runner.py:300-305) and import_kv (kv_channel.py:72-82)."""
    ids = np.asarray(ids, dtype=np.int64)
    pool[:, ids] = np.moveaxis(items, 0, 1)


def block_copy(pool: np.ndarray, src_ids, dst_ids) -> None:
    """Compaction pool[:, dst] = pool[:, src] with the right-hand side read
    first (no reference function; the closed form of the copy)."""
    src = np.asarray(src_ids, dtype=np.int64)
    dst = np.asarray(dst_ids, dtype=np.int64)
    pool[:, dst] = pool[:, src].copy()


def offload_put_torch(kv_cache: torch.Tensor, block_id: int, slot_buf: torch.Tensor) -> None:
    """ModelRunner.offload_put's byte move (nanovllm/engine/model_runner.py:284-298,
    HostBlockPool.put kv_offload.py:72-88): index_select one block of the
    [2, L, blocks, page, KVH, D] pool along dim 2, copy it into the slot."""
    idx = torch.tensor([block_id], dtype=torch.long)
    slot_buf.copy_(kv_cache.index_select(2, idx).squeeze(2))


def offload_get_torch(kv_cache: torch.Tensor, slot_buf: torch.Tensor, block_id: int) -> None:
    """ModelRunner.offload_get's byte move (model_runner.py:300-305):
    index_copy_ of the slot back into block block_id along dim 2."""
    idx = torch.tensor([block_id], dtype=torch.long)
    kv_cache.index_copy_(2, idx, slot_buf.unsqueeze(2))


def compact_torch(kv_cache: torch.Tensor, src_ids, dst_ids) -> None:
    """The compaction copy pool[:, :, dst] = pool[:, :, src] in the engine's
    torch idiom (index_select, then index_copy_ along the block axis)."""
    src = torch.as_tensor(list(src_ids), dtype=torch.long)
    dst = torch.as_tensor(list(dst_ids), dtype=torch.long)
    kv_cache.index_copy_(2, dst, kv_cache.index_select(2, src))


def decode_kv_bytes(context_lens, kvh: int, d: int, elem_bytes: int) -> int:
    """Algorithmic KV bytes one decode launch must read: every context token's
    K and V row for every kv head."""
    return int(np.sum(np.asarray(context_lens, dtype=np.int64))) * 2 * kvh * d * elem_bytes


def log2e() -> float:
    return 1.0 / math.log(2.0)


# ---------------------------------------------------------------------------
# The step in front of the path: q/k RMSNorm + rotary embedding.  CPU torch in
# the engine's own op order (its arithmetic is torch's), bf16 in and out.
# ---------------------------------------------------------------------------


def cos_sin_cache_ref(head_size: int, max_position: int, base: float) -> torch.Tensor:
    """nanovllm/layers/rotary_embedding.py:30-35: fp32 [max_position, D],
    cos(t * inv_freq) then sin(t * inv_freq)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def rms_norm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """nanovllm/layers/layernorm.py:18-26 (rms_forward), bf16 x and weight."""
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(var + eps)).to(x.dtype).mul_(weight)


def apply_rotary_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """nanovllm/layers/rotary_embedding.py:7-15 (neox halves, fp32 arithmetic)."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def qk_norm_rope_ref(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor,
                     cos_sin_cache: torch.Tensor, q_w: torch.Tensor | None,
                     k_w: torch.Tensor | None, eps: float):
    """nanovllm/models/qwen3.py:80-85 on CPU tensors: q/k [N, heads, D] bf16
    -> (rotated q, rotated k).  Norms are skipped when the weight is None."""
    if q_w is not None:
        q = rms_norm_ref(q, q_w, eps)
    if k_w is not None:
        k = rms_norm_ref(k, k_w, eps)
    cos_sin = cos_sin_cache[positions.long()].unsqueeze(1)
    cos, sin = cos_sin.chunk(2, dim=-1)
    return apply_rotary_ref(q, cos, sin), apply_rotary_ref(k, cos, sin)


# ---------------------------------------------------------------------------
# PD wire format (nanovllm/pd/kv_channel.py:110-220)
# ---------------------------------------------------------------------------


def kv_frame_ref(kv_pool: np.ndarray, block_table) -> bytes:
    """The frame TcpKVChannel.send_blocks (kv_channel.py:137-154) writes for
    `block_table` of a pool [2, L, blocks, page, kvh, d] (any element type,
    little endian): header (n, k_bytes, v_bytes) as three u32 LE, then for
    each side every named block's [L, page, kvh, d] slab in table order —
    extract_kv's buf.k[:n] / buf.v[:n] (kv_channel.py:54-69) taken as bytes
    (_tensor_to_bytes, :110-112)."""
    ids = [int(b) for b in block_table]
    sides = []
    for side in (0, 1):
        slabs = [np.ascontiguousarray(kv_pool[side, :, b]).tobytes() for b in ids]
        sides.append(b"".join(slabs))
    n, k, v = len(ids), sides[0], sides[1]
    header = (n.to_bytes(4, "little") + len(k).to_bytes(4, "little")
              + len(v).to_bytes(4, "little"))
    return header + k + v


def split_frames_ref(stream: bytes) -> tuple[list, bytes]:
    """Cut a byte stream into complete frames (n, k_bytes, v_bytes), the
    reassembly rule of KVFrameAssembler (kv_channel.py:181-220); returns the
    frames and the unconsumed tail."""
    frames, pos = [], 0
    while len(stream) - pos >= 12:
        n = int.from_bytes(stream[pos:pos + 4], "little")
        kl = int.from_bytes(stream[pos + 4:pos + 8], "little")
        vl = int.from_bytes(stream[pos + 8:pos + 12], "little")
        if len(stream) - pos - 12 < kl + vl:
            break
        body = pos + 12
        frames.append((n, stream[body:body + kl], stream[body + kl:body + kl + vl]))
        pos = body + kl + vl
    return frames, stream[pos:]
