"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something other than its own
formula: hand-computed known answers, closed forms, Python's round() or
torch's bf16 cast as independent rounding implementations, and float64 torch
scaled_dot_product_attention as an independent attention routine.  The
known answers are chosen so that plausible mistakes (half-up instead of
half-even, amax/128, a missing clamp, a prefix mask off by one, a transposed
GQA mapping) fail.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kv_oracle as ko


def bf16_bits(x):
    return ko.torch_bf16_bits(torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16))


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def test_f32_to_bf16_matches_torch_cast():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(20000, generator=g) * torch.exp(torch.randn(20000, generator=g) * 8)
    x[:4] = torch.tensor([0.0, -0.0, float("inf"), float("-inf")])
    ref = ko.torch_bf16_bits(x.to(torch.bfloat16))
    assert np.array_equal(ko.f32_to_bf16(x.numpy()), ref)
    # ties: 1 + 2^-8 sits half-way between two bf16 values -> even (1.0)
    assert ko.f32_to_bf16(np.float32([1 + 2 ** -8]))[0] == 0x3F80
    assert ko.f32_to_bf16(np.float32([1 + 3 * 2 ** -8]))[0] == 0x3F82


# ---------------------------------------------------------------------------
# store_kvcache
# ---------------------------------------------------------------------------
def test_store_closed_form_and_brute_force():
    rng = np.random.default_rng(1)
    N, KVH, D, blocks, page = 37, 3, 8, 5, 16
    key = rng.integers(0, 2 ** 16, (N, KVH, D), dtype=np.uint16)
    val = rng.integers(0, 2 ** 16, (N, KVH, D), dtype=np.uint16)
    kc = rng.integers(0, 2 ** 16, (blocks, page, KVH, D), dtype=np.uint16)
    vc = kc.copy()
    slots = rng.permutation(blocks * page)[:N]
    k0, v0 = kc.copy(), vc.copy()
    ko.store_kvcache(key, val, kc, vc, slots)
    flat_k, flat_v = k0.reshape(-1, KVH, D).copy(), v0.reshape(-1, KVH, D).copy()
    for j, s in enumerate(slots):          # brute force
        flat_k[s] = key[j]
        flat_v[s] = val[j]
    assert np.array_equal(kc.reshape(-1, KVH, D), flat_k)
    assert np.array_equal(vc.reshape(-1, KVH, D), flat_v)
    untouched = np.setdiff1d(np.arange(blocks * page), slots)
    assert np.array_equal(kc.reshape(-1, KVH, D)[untouched], k0.reshape(-1, KVH, D)[untouched])


def test_store_negative_slot_is_python_indexing():
    key = np.arange(2 * 4, dtype=np.uint16).reshape(2, 1, 4)
    kc = np.zeros((2, 4, 1, 4), dtype=np.uint16)
    vc = kc.copy()
    ko.store_kvcache(key, key, kc, vc, np.array([-1, 0]))
    assert list(kc.reshape(-1, 4)[7]) == [0, 1, 2, 3]
    assert list(kc.reshape(-1, 4)[0]) == [4, 5, 6, 7]


# ---------------------------------------------------------------------------
# per-token-head int8 (round half to even)
# ---------------------------------------------------------------------------
def test_tokhead_known_answers():
    D = 16
    row = np.zeros(D, np.float32)
    row[:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 127.0]   # amax 127 -> s = 1
    zero = np.zeros(D, np.float32)
    tiny = np.full(D, 3e-7, np.float32)
    x = np.stack([row, zero, tiny])[:, None, :]
    codes, scales = ko.quant_tokhead(bf16_bits(x))
    assert codes[0, 0, :9].tolist() == [0, 2, 2, 0, -2, -2, 126, -126, 127]
    assert scales[0, 0] == np.float32(1.0)
    assert scales[1, 0] == np.float32(np.float32(1e-6) / np.float32(127))   # clamp before /127
    assert codes[1].max() == 0
    tiny_b = float(ko.bf16_to_f32(bf16_bits(np.float32(3e-7))))
    assert codes[2, 0, 0] == round(np.float32(tiny_b) / scales[2, 0])


def test_tokhead_matches_python_round_half_even():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 4, 128, generator=g) * 3
    xb = ko.torch_bf16_bits(x.to(torch.bfloat16))
    codes, scales = ko.quant_tokhead(xb)
    xf = ko.bf16_to_f32(xb)
    for t in range(0, 64, 9):
        for h in range(4):
            amax = max(float(np.abs(xf[t, h]).max()), 1e-6)
            s = np.float32(np.float32(amax) / np.float32(127.0))
            assert scales[t, h] == s
            for d in range(0, 128, 7):
                q = np.float32(xf[t, h, d]) / s           # fp32 IEEE quotient
                want = max(-127, min(127, round(float(q))))  # Python round: half to even
                assert codes[t, h, d] == want


def test_tokhead_saturates_and_dequant_roundtrip():
    x = np.zeros((1, 1, 8), np.float32)
    x[0, 0, 0] = 5.0
    codes, scales = ko.quant_tokhead(bf16_bits(x))
    assert codes[0, 0, 0] == 127 and abs(codes).max() == 127
    deq = ko.dequant_tokhead(codes, scales)
    assert ko.bf16_to_f32(deq)[0, 0, 0] == np.float32(5.0)


# ---------------------------------------------------------------------------
# per-channel int8 (floor(x / s + 0.5)) with the outlier side pool
# ---------------------------------------------------------------------------
def test_chan_known_answers():
    x = np.float32([[[0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 200.0, -200.0]]])
    s = np.ones((1, 8), np.float32)
    assert ko.quant_chan(bf16_bits(x), s)[0, 0].tolist() == [1, 2, 3, 0, -1, -2, 127, -127]


def test_chan_store_outliers_zeroed_and_side_exact():
    KVH, D, NOUT = 2, 8, 3
    x = np.float32(np.arange(KVH * D).reshape(1, KVH, D) - 5) / np.float32(4)
    xb = bf16_bits(x)
    scale = np.full((KVH, D), np.float32(0.25), np.float32)
    out_idx = np.array([[6, 1, 0], [3, 0, 0]], np.int32)
    n_out = np.array([2, 1], np.int32)
    kc = np.full((1, 4, KVH, D), 99, np.int8)
    vc = kc.copy()
    sk = np.zeros((1, 4, KVH, NOUT), np.uint16)
    sv = sk.copy()
    ko.store_int8_chan(xb, xb, kc, vc, scale, scale, sk, sv, out_idx, n_out, np.array([2]))
    expect = np.clip(np.floor(x / 0.25 + 0.5), -127, 127).astype(np.int8)[0]
    expect[0, [6, 1]] = 0
    expect[1, [3]] = 0
    assert np.array_equal(kc[0, 2], expect) and np.array_equal(vc[0, 2], expect)
    assert sk[0, 2, 0, :2].tolist() == [xb[0, 0, 6], xb[0, 0, 1]] and sk[0, 2, 0, 2] == 0
    assert sk[0, 2, 1, 0] == xb[0, 1, 3]
    assert (kc[0, [0, 1, 3]] == 99).all()


def test_chan_dequant_against_torch():
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(-127, 128, (10, 2, 16), generator=g, dtype=torch.int8)
    ds = torch.rand(2, 16, generator=g)
    side = torch.randn(10, 2, 4, generator=g).to(torch.bfloat16)
    idx = torch.tensor([[3, 7, 0, 0], [15, 0, 0, 0]], dtype=torch.int32)
    nout = torch.tensor([2, 1], dtype=torch.int32)
    ref = (codes.float() * ds).to(torch.bfloat16)
    ref[:, 0, 3] = side[:, 0, 0]
    ref[:, 0, 7] = side[:, 0, 1]
    ref[:, 1, 15] = side[:, 1, 0]
    got = ko.dequant_chan(codes.numpy(), ds.numpy(), ko.torch_bf16_bits(side), idx.numpy(),
                          nout.numpy())
    assert np.array_equal(got, ko.torch_bf16_bits(ref))


def test_prefill_read_of_an_int8_pool_is_the_gather_dequantisation():
    # attention.py:33-51 (_gather_kv) restated in torch over a paged pool: the
    # blocks of a table row, (code.float() * dscale).to(bf16), then each
    # head's outlier dims from the side pool; and the per-token-head form
    # bf16(code * scale).  kv_float_prefill must read every slot the same way.
    g = torch.Generator().manual_seed(8)
    blocks, page, kvh, d, nout = 3, 32, 2, 16, 4
    codes = torch.randint(-127, 128, (blocks, page, kvh, d), generator=g, dtype=torch.int8)
    ds = torch.rand(kvh, d, generator=g) * 0.05
    side = torch.randn(blocks, page, kvh, nout, generator=g).to(torch.bfloat16)
    idx = torch.tensor([[3, 9, 1, 0], [14, 0, 0, 0]], dtype=torch.int32)
    nh = torch.tensor([3, 1], dtype=torch.int32)
    table = torch.tensor([2, 0, 1])
    kv = (codes[table].float() * ds).to(torch.bfloat16).view(-1, kvh, d)
    s = side[table].view(-1, kvh, nout)
    for h in range(kvh):
        kv[:, h, idx[h, :nh[h]].long()] = s[:, h, :nh[h]]
    got = ko.kv_float_prefill(codes.numpy(), "int8_chan", ds.numpy(), ko.torch_bf16_bits(side),
                              idx.numpy(), nh.numpy())
    assert np.array_equal(got[table.numpy()].reshape(-1, kvh, d), kv.float().numpy())
    sc = torch.rand(blocks, page, kvh, generator=g) * 0.05
    want = (codes.float() * sc.unsqueeze(-1)).to(torch.bfloat16).float()
    got = ko.kv_float_prefill(codes.numpy(), "int8_tokhead", sc.numpy())
    assert np.array_equal(got, want.numpy())


# ---------------------------------------------------------------------------
# attention references
# ---------------------------------------------------------------------------
def _sdpa64(q, k, v, scale, mask=None):
    """float64 torch SDPA per kv group: q [Sq, H, D], k/v [Sk, KVH, D]."""
    H, KVH = q.shape[1], k.shape[1]
    kk = torch.from_numpy(k).double().repeat_interleave(H // KVH, dim=1).transpose(0, 1)
    vv = torch.from_numpy(v).double().repeat_interleave(H // KVH, dim=1).transpose(0, 1)
    qq = torch.from_numpy(q).double().transpose(0, 1)
    m = None if mask is None else torch.from_numpy(mask)[None]
    o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=m, scale=scale)
    return o.transpose(0, 1).numpy()


def _paged_case(B, H, KVH, lens, seed, page=16, D=32):
    rng = np.random.default_rng(seed)
    nblk = [max(1, math.ceil(n / page)) for n in lens]
    blocks = sum(nblk) + 2
    perm = rng.permutation(blocks)
    bt = -np.ones((B, max(nblk)), np.int64)
    pos = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[pos:pos + n]
        pos += n
    q = bf16_bits(rng.standard_normal((B, H, D)).astype(np.float32))
    k = ko.bf16_to_f32(bf16_bits(rng.standard_normal((blocks, page, KVH, D)).astype(np.float32)))
    v = ko.bf16_to_f32(bf16_bits(rng.standard_normal((blocks, page, KVH, D)).astype(np.float32)))
    return q, k, v, bt


@pytest.mark.parametrize("H,KVH", [(8, 2), (4, 4), (6, 3)])
def test_paged_decode_against_float64_sdpa(H, KVH):
    lens = [1, 15, 16, 17, 40]
    q, k, v, bt = _paged_case(len(lens), H, KVH, lens, seed=H * 10 + KVH)
    out = ko.paged_decode_ref(q, k, v, bt, lens, 0.3)
    for b, n in enumerate(lens):
        nb = math.ceil(n / 16)
        kk = k[bt[b, :nb]].reshape(-1, KVH, k.shape[-1])[:n]
        vv = v[bt[b, :nb]].reshape(-1, KVH, v.shape[-1])[:n]
        want = _sdpa64(ko.bf16_to_f32(q[b:b + 1]), kk, vv, 0.3)[0]
        assert np.abs(out[b] - want).max() < 1e-5


def test_paged_decode_closed_forms_and_poison():
    q, k, v, bt = _paged_case(3, 4, 2, [1, 20, 20], seed=9)
    # identical keys -> uniform softmax -> output is the mean of V
    blk = bt[1, :2]
    k[blk] = k[blk][0:1, 0:1]
    # NaN tail past the context is never read
    k[bt[2, 1], 4:] = np.nan
    v[bt[2, 1], 4:] = np.nan
    out = ko.paged_decode_ref(q, k, v, bt, [1, 20, 20], 0.5)
    assert np.allclose(out[0, 0], v[bt[0, 0], 0, 0])         # one key -> its V row (GQA head 0)
    assert np.allclose(out[0, 3], v[bt[0, 0], 0, 1])         # head 3 reads kv head 1
    vv = v[blk].reshape(-1, 2, v.shape[-1])[:20]
    assert np.allclose(out[1, 0], vv[:, 0].mean(0), atol=1e-6)
    assert np.isfinite(out[2]).all()
    assert np.isnan(ko.paged_decode_ref(q[:1], k, v, bt[:1], [0], 0.5)).all()


def test_prefill_prefix_mask_against_sdpa():
    rng = np.random.default_rng(4)
    H, KVH, D = 4, 2, 32
    chunks = [(0, 5), (7, 3), (16, 10)]          # (cached prefix, new queries)
    lens = [p + c for p, c in chunks]
    q_all, k, v, bt = _paged_case(len(chunks), H, KVH, lens, seed=4, D=D)
    T = sum(c for _, c in chunks)
    q = bf16_bits(rng.standard_normal((T, H, D)).astype(np.float32))
    cu_q = [0]
    cu_k = [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    out = ko.prefill_ref(q, k, v, bt, cu_q, cu_k, 0.25)
    for i, (p, c) in enumerate(chunks):
        sk = p + c
        nb = math.ceil(sk / 16)
        kk = k[bt[i, :nb]].reshape(-1, KVH, D)[:sk]
        vv = v[bt[i, :nb]].reshape(-1, KVH, D)[:sk]
        mask = np.arange(sk)[None, :] <= (p + np.arange(c))[:, None]
        want = _sdpa64(ko.bf16_to_f32(q[cu_q[i]:cu_q[i + 1]]), kk, vv, 0.25, mask)
        assert np.abs(out[cu_q[i]:cu_q[i + 1]] - want).max() < 1e-5
        if p == 0:   # no prefix: plain causal attention
            qq = torch.from_numpy(ko.bf16_to_f32(q[cu_q[i]:cu_q[i + 1]])).double().transpose(0, 1)
            kk2 = torch.from_numpy(kk).double().repeat_interleave(2, 1).transpose(0, 1)
            vv2 = torch.from_numpy(vv).double().repeat_interleave(2, 1).transpose(0, 1)
            causal = F.scaled_dot_product_attention(qq, kk2, vv2, is_causal=True, scale=0.25)
            assert np.abs(out[cu_q[i]:cu_q[i + 1]] - causal.transpose(0, 1).numpy()).max() < 1e-5


def test_mixed_is_decode_rows_then_prefill_rows():
    lens_dec = [9, 30]
    chunks = [(5, 4)]
    q, k, v, bt = _paged_case(3, 4, 2, lens_dec + [9], seed=12)
    rng = np.random.default_rng(1)
    qq = bf16_bits(rng.standard_normal((2 + 4, 4, 32)).astype(np.float32))
    out = ko.mixed_ref(qq, k, v, bt, 2, lens_dec, [0, 4], [0, 9], 0.2)
    dec = ko.paged_decode_ref(qq[:2], k, v, bt[:2], lens_dec, 0.2)
    pre = ko.prefill_ref(qq[2:], k, v, bt, [0, 4], [0, 9], 0.2, row_offset=2)
    assert np.array_equal(out, np.concatenate([dec, pre]))


def test_gather_sdpa_decode_matches_decode_reference():
    lens = [5, 16, 33]
    q, k, v, bt = _paged_case(3, 4, 2, lens, seed=21)
    kt = torch.from_numpy(k)
    vt = torch.from_numpy(v)
    out = ko.gather_sdpa_decode(torch.from_numpy(ko.bf16_to_f32(q)), kt, vt,
                                torch.from_numpy(bt).to(torch.int32),
                                torch.tensor(lens), 0.4, max(lens))
    ref = ko.paged_decode_ref(q, k, v, bt, lens, 0.4)
    assert np.abs(out.numpy() - ref).max() < 1e-5


# ---------------------------------------------------------------------------
# whole-block movement
# ---------------------------------------------------------------------------
def test_block_gather_scatter_roundtrip_and_copy_semantics():
    rng = np.random.default_rng(7)
    pool = rng.integers(0, 2 ** 16, (6, 10, 32), dtype=np.uint16)
    ids = [7, 2, 9]
    items = ko.block_gather(pool, ids)
    assert items.shape == (3, 6, 32)
    assert np.array_equal(items[1], pool[:, 2])
    dst = pool.copy()
    ko.block_scatter(dst, [0, 1, 3], items)
    assert np.array_equal(dst[:, 3], pool[:, 9])
    chain = pool.copy()
    ko.block_copy(chain, [1, 2], [2, 3])          # simultaneous: 3 gets the OLD block 2
    assert np.array_equal(chain[:, 2], pool[:, 1]) and np.array_equal(chain[:, 3], pool[:, 2])


# ---------------------------------------------------------------------------
# q/k RMSNorm + rotary embedding (the step in front of the path)
# ---------------------------------------------------------------------------
def test_cos_sin_cache_matches_closed_form():
    cache = ko.cos_sin_cache_ref(128, 64, 10000.0)
    assert cache.shape == (64, 128) and cache.dtype == torch.float32
    t = np.arange(64)[:, None]
    inv = 10000.0 ** (-np.arange(0, 128, 2) / 128.0)
    np.testing.assert_allclose(cache[:, :64].numpy(), np.cos(t * inv), atol=2e-5)
    np.testing.assert_allclose(cache[:, 64:].numpy(), np.sin(t * inv), atol=2e-5)


def test_rotary_at_position_zero_is_the_identity():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 4, 128, generator=g).to(torch.bfloat16)
    cache = ko.cos_sin_cache_ref(128, 16, 10000.0)
    q, k = ko.qk_norm_rope_ref(x, x[:, :2], torch.zeros(5, dtype=torch.long), cache, None, None,
                               1e-6)
    assert torch.equal(q, x) and torch.equal(k, x[:, :2])


def test_rotary_is_multiplication_by_the_phase():
    # (x1 + i x2) * exp(i p theta_j), theta_j = base^(-2j/D), in float64: a
    # swapped sign or half fails by O(1).
    g = torch.Generator().manual_seed(4)
    x = torch.randn(7, 3, 128, generator=g).to(torch.bfloat16)
    pos = torch.tensor([1, 5, 17, 100, 511, 1000, 2047])
    cache = ko.cos_sin_cache_ref(128, 2048, 10000.0)
    q, _ = ko.qk_norm_rope_ref(x, x[:, :1], pos, cache, None, None, 1e-6)
    xf = x.double().numpy()
    theta = 10000.0 ** (-np.arange(0, 128, 2) / 128.0)
    ph = pos.double().numpy()[:, None, None] * theta[None, None, :]
    z = (xf[..., :64] + 1j * xf[..., 64:]) * np.exp(1j * ph)
    want = np.concatenate([z.real, z.imag], axis=-1)
    got = q.double().numpy()
    assert np.abs(got - want).max() <= 2.0 ** -7 * np.abs(want).max() + 2e-3
    # The rotation keeps each (x1_j, x2_j) pair's length.
    n_in = xf[..., :64] ** 2 + xf[..., 64:] ** 2
    n_out = got[..., :64] ** 2 + got[..., 64:] ** 2
    assert np.abs(n_out - n_in).max() <= 2.0 ** -6 * n_in.max()


def test_rms_norm_closed_forms():
    # A constant row c normalises to c / sqrt(c^2 + eps) = 1 (after the bf16
    # rounding), so the output is the weight itself.
    w = torch.tensor(np.linspace(-2, 2, 128), dtype=torch.float32).to(torch.bfloat16)
    for c in (0.75, -3.0, 40.0):
        x = torch.full((1, 1, 128), c).to(torch.bfloat16)
        y = ko.rms_norm_ref(x, w, 1e-6)
        assert torch.equal(y[0, 0], w * math.copysign(1.0, c))
    # A random row comes out with unit RMS (unit weight), to bf16 precision.
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 128, generator=g) * 7).to(torch.bfloat16)
    y = ko.rms_norm_ref(x, torch.ones(128, dtype=torch.bfloat16), 1e-6).double()
    rms = y.pow(2).mean(-1).sqrt()
    assert torch.all((rms - 1).abs() < 2.0 ** -7)


# ---------------------------------------------------------------------------
# torch restatements timed as the CPU baselines
# ---------------------------------------------------------------------------
def _small_pool(seed, blocks=24, page=32, kvh=2):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(blocks, page, kvh, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(blocks, page, kvh, 128, generator=g).to(torch.bfloat16)
    return g, kc, vc


def test_prefill_loop_torch_matches_prefill_reference():
    g, kc, vc = _small_pool(31)
    cu_q, cu_k = [0, 5, 5, 37], [0, 40, 41, 100]          # prefixes 35, (empty), 27
    bt = torch.randperm(24, generator=g)[:12].view(3, 4).to(torch.int32)
    q = torch.randn(37, 8, 128, generator=g).to(torch.bfloat16)
    got = ko.prefill_loop_torch(q, None, None, kc, vc, cu_q, cu_k, bt, 0.09)
    ref = ko.prefill_ref(ko.torch_bf16_bits(q), ko.bf16_to_f32(ko.torch_bf16_bits(kc)),
                         ko.bf16_to_f32(ko.torch_bf16_bits(vc)), bt.numpy(), cu_q, cu_k, 0.09)
    assert got.shape == (37, 8, 128)
    assert np.abs(got.float().numpy() - ref).max() < 2e-2
    # without block tables: causal over the chunk's own rows
    kf = torch.randn(37, 2, 128, generator=g).to(torch.bfloat16)
    vf = torch.randn(37, 2, 128, generator=g).to(torch.bfloat16)
    got = ko.prefill_loop_torch(q, kf, vf, kc, vc, [0, 5, 37], [0, 5, 37], None, 0.09)
    ref = ko.prefill_ref(ko.torch_bf16_bits(q), None, None, None, [0, 5, 37], [0, 5, 37], 0.09,
                         fresh_k=ko.bf16_to_f32(ko.torch_bf16_bits(kf)),
                         fresh_v=ko.bf16_to_f32(ko.torch_bf16_bits(vf)))
    assert np.abs(got.float().numpy() - ref).max() < 2e-2


def test_mixed_torch_matches_mixed_reference():
    g, kc, vc = _small_pool(32)
    bt = torch.randperm(24, generator=g)[:15].view(5, 3).to(torch.int32)
    dlen = torch.tensor([1, 70, 96], dtype=torch.int32)
    cu_q, cu_k = [0, 4, 10], [0, 30, 90]
    q = torch.randn(13, 8, 128, generator=g).to(torch.bfloat16)
    got = ko.mixed_torch(q, kc, vc, bt, 3, dlen, 96, cu_q, cu_k, 0.09)
    ref = ko.mixed_ref(ko.torch_bf16_bits(q), ko.bf16_to_f32(ko.torch_bf16_bits(kc)),
                       ko.bf16_to_f32(ko.torch_bf16_bits(vc)), bt.numpy(), 3, dlen.numpy(),
                       cu_q, cu_k, 0.09)
    assert np.abs(got.float().numpy() - ref).max() < 2e-2


def test_quant_tokhead_torch_equals_numpy_restatement():
    g = torch.Generator().manual_seed(33)
    x = (torch.randn(300, 4, 128, generator=g) * torch.where(
        torch.rand(300, 4, 128, generator=g) < 0.01, 20.0, 1.0)).to(torch.bfloat16)
    x[0, 0] = 0.0                                          # the 1e-6 clamp
    codes, s = ko.quant_tokhead_torch(x)
    want_c, want_s = ko.quant_tokhead(ko.torch_bf16_bits(x))
    assert np.array_equal(codes.numpy(), want_c)
    assert np.array_equal(s.squeeze(-1).numpy().view(np.uint32), want_s.view(np.uint32))


def test_int8_tokhead_decode_is_the_bf16_decode_of_the_dequantised_pool():
    g, kc, vc = _small_pool(34)
    kq, ks = ko.quant_tokhead_torch(kc)
    vq, vs = ko.quant_tokhead_torch(vc)
    bt = torch.randperm(24, generator=g)[:12].view(3, 4).to(torch.int32)
    lens = torch.tensor([1, 77, 128], dtype=torch.int32)
    q = torch.randn(3, 8, 128, generator=g).to(torch.bfloat16)
    got = ko.gather_sdpa_decode_int8_tokhead(q, kq, vq, ks.squeeze(-1), vs.squeeze(-1), bt, lens,
                                             0.09, 128)
    kd = ko.bits_to_torch_bf16(ko.dequant_tokhead(kq.numpy(), ks.squeeze(-1).numpy()))
    vd = ko.bits_to_torch_bf16(ko.dequant_tokhead(vq.numpy(), vs.squeeze(-1).numpy()))
    want = ko.gather_sdpa_decode(q, kd, vd, bt, lens, 0.09, 128)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_block_moves_torch_match_closed_forms():
    g = torch.Generator().manual_seed(35)
    pool = torch.randint(-2**15, 2**15, (2, 3, 10, 4, 2, 8), generator=g, dtype=torch.int16)
    orig = pool.clone()
    slot = torch.empty_like(pool[:, :, 0])
    ko.offload_put_torch(pool, 7, slot)
    assert torch.equal(slot, orig[:, :, 7])
    ko.offload_get_torch(pool, slot, 2)
    assert torch.equal(pool[:, :, 2], orig[:, :, 7])
    ko.compact_torch(pool, [0, 1, 9], [4, 5, 6])
    want = orig.numpy().reshape(6, 10, -1).copy()
    ko.block_scatter(want, [2], ko.block_gather(orig.numpy().reshape(6, 10, -1), [7]))
    ko.block_copy(want, [0, 1, 9], [4, 5, 6])
    assert np.array_equal(pool.numpy().reshape(6, 10, -1), want)


# ---------------------------------------------------------------------------
# per-channel int8 calibration
# ---------------------------------------------------------------------------
def test_calib_freeze_matches_p17_unit_calibration():
    """tests/p17_kv_int8.py:80-101 (torch, restated in helpers) against the
    oracle's statistics + freeze on the same seeded unit case."""
    from helpers import p17_unit_inputs
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    ak, sk = ko.calib_stats(ko.torch_bf16_bits(key))
    av, sv = ko.calib_stats(ko.torch_bf16_bits(value))
    got = ko.calib_freeze(ak, av, sk, sv, key.shape[0], out_idx2d.shape[1])
    for g, w in zip(got[:4], (s_k, s_v, ds_k, ds_v)):
        assert np.array_equal(g.view(np.uint32), w.numpy().view(np.uint32))
    assert np.array_equal(got[4], out_idx2d.numpy())
    assert np.array_equal(got[5], head_n_out.numpy())
    assert got[5].sum() > 0


def test_calib_freeze_known_answers():
    f = np.float32
    kvh, d = 2, 128
    amax_k = np.ones((kvh, d), f)
    amax_v = np.ones((kvh, d), f)
    sum_k = np.full((kvh, d), 4.0, f)      # typ = 4 / 4 = 1 -> ratio 1
    sum_v = np.full((kvh, d), 4.0, f)
    amax_k[0, 5] = 10.0                     # ratio exactly 10: not an outlier
    amax_k[0, 9] = 10.5                     # > 10
    amax_v[0, 2] = 40.0                     # V alone decides (joint ratio)
    amax_k[1, :] = 50.0                     # every dim of head 1: first 3 in index order
    amax_k[1, 0] = 0.0                      # scale clamps to 1e-6, ratio 0
    s_k, s_v, ds_k, ds_v, idx, n = ko.calib_freeze(amax_k, amax_v, sum_k, sum_v, 4, 3)
    assert n.tolist() == [2, 3]
    assert idx[0].tolist() == [2, 9, 0] and idx[1].tolist() == [1, 2, 3]
    assert s_k[1, 0] == f(1e-6) and s_k[0, 9] == f(10.5) / f(127)
    assert ds_k[0, 2] == 0 and ds_v[0, 9] == 0 and ds_k[0, 5] == s_k[0, 5]
    # typ clamps at 1e-6: an all-zero column has ratio 0
    z = np.zeros((1, d), f)
    assert ko.calib_freeze(z, z, z, z, 7, 8)[5].tolist() == [0]


def test_f64_to_bf16_value_single_rounding():
    """The per-forward sum's rounding: against torch's fp32 -> bf16 cast on
    fp32-exact inputs (ties included), and known answers that a double
    rounding through fp32 would get wrong."""
    g = torch.Generator().manual_seed(5)
    x = (torch.rand(4000, generator=g) * torch.exp2(torch.randint(-140, 120, (4000,),
                                                                     generator=g).float()))
    x[:6] = torch.tensor([0.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 2.0 ** -130, 3 * 2.0 ** -134,
                          3.3895e38])
    want = ko.bf16_to_f32(ko.torch_bf16_bits(x.to(torch.bfloat16)))
    got = ko.f64_to_bf16_value(x.double().numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # just above a tie: the exact value rounds up; via fp32 it would tie to even
    assert ko.f64_to_bf16_value(np.float64([1 + 2 ** -8 + 2 ** -40]))[0] == np.float32(1 + 2 ** -7)
    assert ko.f64_to_bf16_value(np.float64([239.75, 239.25, 280.5, 281.01])).tolist() == \
        [240.0, 239.0, 280.0, 282.0]
    assert ko.f64_to_bf16_value(np.float64([2.0 ** 128 - 2.0 ** 119]))[0] == np.inf


def test_calib_stats_match_the_engine_hook_in_torch():
    """Per-forward statistics folded over forwards of different lengths equal
    the hook's own torch statements (model_runner.py:527-533) bit for bit:
    amax, and the bf16 sums torch returns, added in fp32."""
    from helpers import torch_hook_stats
    g = torch.Generator().manual_seed(44)
    forwards = []
    for n in (300, 17, 512, 1):
        k = (torch.randn(n, 4, 128, generator=g) * 3).to(torch.bfloat16)
        v = (torch.randn(n, 4, 128, generator=g) * torch.exp2(
            torch.randint(-6, 6, (n, 4, 128), generator=g).float())).to(torch.bfloat16)
        forwards.append((k, v))
    ak, av, sk, sv, n = torch_hook_stats(forwards)
    ak2, sk2, n2 = ko.calib_fold([ko.torch_bf16_bits(k) for k, _ in forwards])
    av2, sv2, _ = ko.calib_fold([ko.torch_bf16_bits(v) for _, v in forwards])
    assert n2 == n == 830
    for got, want in ((ak2, ak), (av2, av), (sk2, sk), (sv2, sv)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the per-forward rounding is visible: fp32 sums differ from the hook's
    exact = sum(np.abs(ko.bf16_to_f32(ko.torch_bf16_bits(k))).astype(np.float64).sum(0)
                for k, _ in forwards)
    assert (np.abs(exact - sk) > 0).mean() > 0.5


def test_calib_outlier_flip_follows_the_hook():
    """Two dims whose outlier decision depends on the bf16 rounding of each
    forward's sum (tests/helpers.CALIB_FLIP_COLUMNS): the oracle's freeze
    follows the hook's torch statistics, and the fp32-sum statistics would
    decide both dims the other way."""
    from helpers import calib_flip_forwards, torch_hook_stats
    forwards, dims = calib_flip_forwards()
    ak, av, sk, sv, n = torch_hook_stats(forwards)
    assert n == 900
    assert sk[0, dims["hook_in"]] == 720.0 and sk[0, dims["hook_out"]] == 719.0
    a_k, s_k, _ = ko.calib_fold([ko.torch_bf16_bits(k) for k, _ in forwards])
    a_v, s_v, _ = ko.calib_fold([ko.torch_bf16_bits(v) for _, v in forwards])
    assert np.array_equal(s_k, sk) and np.array_equal(s_v, sv)
    got = ko.calib_freeze(a_k, a_v, s_k, s_v, n, 4)
    want = ko.calib_freeze(ak, av, sk, sv, n, 4)
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_, w_)
    idx, n_out = got[4], got[5]
    head0 = set(idx[0, :n_out[0]].tolist())
    assert dims["hook_out"] in head0 and dims["hook_in"] not in head0
    assert idx[1, :n_out[1]].tolist() == [40]
    # with plain fp32 sums of |x| (no per-forward rounding) both flip
    f32_sum = lambda side: np.sum([np.abs(ko.bf16_to_f32(ko.torch_bf16_bits(f[side])))
                                   .astype(np.float64).sum(0) for f in forwards],
                                  axis=0).astype(np.float32)
    alt = ko.calib_freeze(a_k, a_v, f32_sum(0), f32_sum(1), n, 4)
    head0_alt = set(alt[4][0, :alt[5][0]].tolist())
    assert dims["hook_in"] in head0_alt and dims["hook_out"] not in head0_alt