"""q/k RMSNorm + rotary embedding + KV append in one launch, against the
oracle (the engine's own torch ops on the CPU, nanovllm/models/qwen3.py:80-86).

Bars:
* the rotation alone (no norm) and the v append are bit-exact: every step is
  an IEEE fp32 multiply/add rounded once to bf16, as in torch;
* with the norm, the only freedom is the order of the 128-term sum of
  squares, which moves 1 / sqrt(var + eps) by an ulp at most, and so very
  rarely flips one bf16 rounding: at most 1 element in 1000 may differ, each
  by at most 2^-5 max(1, |ref|) (a couple of bf16 ulps after the rotation);
* the appended k rows are the returned k rows, bit for bit; rows of other
  slots are untouched.
"""
import numpy as np
import pytest
import torch

from helpers import bits
from nanovllm_amd.layers.rotary import RotaryEmbedding, build_cos_sin_cache, qk_norm_rope_store
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(N, H, KVH, seed, max_pos=40960, pos_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(N, (H + 2 * KVH) * 128, generator=g) * 2).to(torch.bfloat16)
    q = qkv[:, :H * 128].view(N, H, 128)
    k = qkv[:, H * 128:(H + KVH) * 128].view(N, KVH, 128)
    v = qkv[:, (H + KVH) * 128:].view(N, KVH, 128)
    pos = torch.randint(0, max_pos, (N,), generator=g).to(pos_dtype)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    return qkv, q, k, v, pos, qw, kw


def _assert_close_bf16(got: torch.Tensor, ref: torch.Tensor, label: str):
    gb, rb = bits(got), bits(ref)
    diff = gb != rb
    frac = diff.mean()
    assert frac <= 1e-3, f"{label}: {frac:.2e} of elements differ"
    if diff.any():
        g = ko.bf16_to_f32(gb[diff]).astype(np.float64)
        r = ko.bf16_to_f32(rb[diff]).astype(np.float64)
        bound = 2.0 ** -5 * np.maximum(1.0, np.abs(r))
        assert np.all(np.abs(g - r) <= bound), f"{label}: max diff {np.abs(g - r).max():.3e}"


@pytest.mark.parametrize("N,H,KVH", [(64, 32, 4), (1037, 32, 4), (300, 16, 8)])
def test_norm_rope_append_matches_reference(N, H, KVH):
    print(f"[rope] N={N} H={H} KVH={KVH}", flush=True)
    qkv, q, k, v, pos, qw, kw = _case(N, H, KVH, seed=N + H)
    cache = build_cos_sin_cache(128, 40960, 1000000.0)
    ref_q, ref_k = ko.qk_norm_rope_ref(q, k, pos, cache, qw, kw, 1e-6)
    blocks = (N + 255) // 256 + 2
    slots = torch.randperm(blocks * 256, generator=torch.Generator().manual_seed(9))[:N]
    sentinel = torch.full((blocks, 256, KVH, 128), 7.0).to(torch.bfloat16)
    kc, vc = sentinel.clone().to(DEV), sentinel.clone().to(DEV)
    qd, kd, vd = qkv.to(DEV), None, None
    qv = qd[:, :H * 128].view(N, H, 128)
    kv_ = qd[:, H * 128:(H + KVH) * 128].view(N, KVH, 128)
    vv = qd[:, (H + KVH) * 128:].view(N, KVH, 128)
    q_out, k_out = qk_norm_rope_store(qv, kv_, vv, pos.to(DEV), cache.to(DEV), qw.to(DEV),
                                      kw.to(DEV), 1e-6, kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    _assert_close_bf16(q_out.cpu(), ref_q, "q")
    _assert_close_bf16(k_out.cpu(), ref_k, "k")
    kc_h, vc_h = kc.cpu().view(-1, KVH, 128), vc.cpu().view(-1, KVH, 128)
    assert np.array_equal(bits(kc_h[slots]), bits(k_out.cpu()))
    assert np.array_equal(bits(vc_h[slots]), bits(v))
    untouched = torch.ones(blocks * 256, dtype=torch.bool)
    untouched[slots] = False
    assert np.array_equal(bits(kc_h[untouched]), bits(sentinel.view(-1, KVH, 128)[untouched]))
    assert np.array_equal(bits(vc_h[untouched]), bits(sentinel.view(-1, KVH, 128)[untouched]))


def test_rotary_embedding_module_is_bit_exact():
    # No norm: every output is one IEEE product pair and one add/sub, rounded
    # once, exactly as torch computes it.
    N, H, KVH = 777, 32, 4
    _, q, k, _, pos, _, _ = _case(N, H, KVH, seed=11, pos_dtype=torch.int32)
    rope = RotaryEmbedding(128, 128, 40960, 1000000.0)
    ref_q, ref_k = ko.qk_norm_rope_ref(q, k, pos, rope.cos_sin_cache, None, None, 1e-6)
    rope = rope.to(DEV)
    got_q, got_k = rope(pos.to(DEV), q.reshape(N, H * 128).to(DEV), k.reshape(N, KVH * 128).to(DEV))
    torch.cuda.synchronize()
    assert got_q.shape == (N, H * 128) and got_k.shape == (N, KVH * 128)
    assert np.array_equal(bits(got_q.cpu().view(N, H, 128)), bits(ref_q))
    assert np.array_equal(bits(got_k.cpu().view(N, KVH, 128)), bits(ref_k))


def test_slots_wrap_skip_and_positions_out_of_range():
    N, H, KVH = 6, 8, 2
    qkv, q, k, v, pos, qw, kw = _case(N, H, KVH, seed=5, max_pos=64)
    pos[3] = -1      # wraps to the last position, like cache[positions] in torch
    pos[4] = 64      # past the cache: torch raises; the kernel yields NaN rows
    cache = build_cos_sin_cache(128, 64, 10000.0)
    slots = torch.tensor([0, 5, -1, 9, 10, 10_000], dtype=torch.int64)  # -1 -> last slot; 10000 skipped
    kc = torch.zeros(4, 4, KVH, 128, dtype=torch.bfloat16, device=DEV)  # 16 slots
    vc = torch.zeros_like(kc)
    q_out, k_out = qk_norm_rope_store(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), cache.to(DEV),
                                      qw.to(DEV), kw.to(DEV), 1e-6, kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    ok = torch.tensor([True, True, True, True, False, True])
    ref_q, ref_k = ko.qk_norm_rope_ref(q[ok], k[ok], pos[ok], cache, qw, kw, 1e-6)
    _assert_close_bf16(q_out.cpu()[ok], ref_q, "q")
    _assert_close_bf16(k_out.cpu()[ok], ref_k, "k")
    assert torch.isnan(q_out[4].float()).all() and torch.isnan(k_out[4].float()).all()
    kf, vf = kc.cpu().view(16, KVH, 128), vc.cpu().view(16, KVH, 128)
    for n, s in [(0, 0), (1, 5), (2, 15), (3, 9), (4, 10)]:
        assert np.array_equal(bits(kf[s]), bits(k_out.cpu()[n]))
        assert np.array_equal(bits(vf[s]), bits(v[n]))
    assert not bool(kf[[1, 2, 3, 4, 6, 7, 8, 11, 12, 13, 14]].float().abs().sum())


def test_empty_batch_and_no_cache():
    H, KVH = 32, 4
    cache = build_cos_sin_cache(128, 16, 10000.0).to(DEV)
    q = torch.empty(0, H, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(0, KVH, 128, dtype=torch.bfloat16, device=DEV)
    q_out, k_out = qk_norm_rope_store(q, k, None, torch.empty(0, dtype=torch.int64, device=DEV),
                                      cache)
    assert q_out.shape == (0, H, 128) and k_out.shape == (0, KVH, 128)
    with pytest.raises(ValueError):
        qk_norm_rope_store(q[:, :, :64], k, None, torch.empty(0, dtype=torch.int64, device=DEV),
                           cache)


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_attention_forward_fused_equals_prologue_then_forward(mode, deterministic_decode):
    """Attention.forward_fused (norm + rope + append in one launch, then
    attention without a second store) == the prologue without the append
    followed by the layer's ordinary forward (which appends), bit for bit."""
    from nanovllm_amd.layers.attention import Attention
    from nanovllm_amd.utils.context import reset_context, set_context
    from nanovllm_amd.workloads import build_block_tables
    H, KVH = 32, 4
    g = torch.Generator().manual_seed(21)
    if mode == "decode":
        lens = [1, 300, 2000]
        N = len(lens)
    else:
        lens = [700]          # one chunk of 64 tokens after a 636-token prefix
        N = 64
    bt = build_block_tables(lens, 16, 256, g)
    qkv = torch.randn(N, (H + 2 * KVH) * 128, generator=g).to(torch.bfloat16).to(DEV)
    q = qkv[:, :H * 128]
    k = qkv[:, H * 128:(H + KVH) * 128]
    v = qkv[:, (H + KVH) * 128:]
    if mode == "decode":
        pos = torch.tensor([n - 1 for n in lens])
        slots = torch.tensor([int(bt[i, (n - 1) // 256]) * 256 + (n - 1) % 256
                              for i, n in enumerate(lens)], dtype=torch.int32)
    else:
        pos = torch.arange(lens[0] - N, lens[0])
        slots = torch.tensor([int(bt[0, p // 256]) * 256 + p % 256 for p in pos.tolist()],
                             dtype=torch.int32)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV)
    cache = build_cos_sin_cache(128, 4096, 1000000.0, DEV)
    pool_k = torch.randn(17, 256, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    pool_v = torch.randn(17, 256, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    outs, pools = [], []
    for fused in (True, False):
        layer = Attention(H, 128, 128 ** -0.5, KVH)
        layer.k_cache, layer.v_cache = pool_k.clone(), pool_v.clone()
        if mode == "decode":
            set_context(False, slot_mapping=slots.to(DEV),
                        context_lens=torch.tensor(lens, dtype=torch.int32).to(DEV),
                        block_tables=bt.to(DEV), max_context_len=max(lens))
        else:
            cq = torch.tensor([0, N], dtype=torch.int32)
            ck = torch.tensor([0, lens[0]], dtype=torch.int32)
            set_context(True, cq.to(DEV), ck.to(DEV), N, lens[0], slots.to(DEV), None, bt.to(DEV),
                        cu_seqlens_q_list=cq.tolist(), cu_seqlens_k_list=ck.tolist())
        if fused:
            o = layer.forward_fused(pos.to(DEV), q, k, v, cache, qw, kw, 1e-6)
        else:
            qr, kr = qk_norm_rope_store(q.view(N, H, 128), k.view(N, KVH, 128), None, pos.to(DEV),
                                        cache, qw, kw, 1e-6)
            o = layer.forward(qr, kr, v.view(N, KVH, 128))
        torch.cuda.synchronize()
        reset_context()
        outs.append(o.cpu())
        pools.append((layer.k_cache.cpu(), layer.v_cache.cpu()))
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    assert np.array_equal(bits(pools[0][0]), bits(pools[1][0]))
    assert np.array_equal(bits(pools[0][1]), bits(pools[1][1]))
