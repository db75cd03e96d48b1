"""int8 KV parity: codes and scales bit-exact, int8 decode within tolerance.

Per-token-head (round half to even, fp32 scale = max(amax, 1e-6) / 127) and
the engine's per-channel encoding with a bf16 outlier side pool
(tests/p17_kv_int8.py:64-136 geometry: N=512, KVH=8, D=128, seed 7).
"""
import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, gathered_pool, p17_unit_inputs
from nanovllm_amd.kernels.kv_int8 import (dequant_gathered, dequant_tokhead, store_kvcache_int8,
                                          store_kvcache_int8_tokhead)
from nanovllm_amd.kernels.paged_attention import paged_decode_attention
from nanovllm_amd.workloads import build_block_tables, decode_workload, outlier_keys, uniform_lengths
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(params=["stream-k-lds", "fixed-chunk", "register"])
def decode_path(request, monkeypatch):
    """The int8 decode launch forms: stream-K with the LDS int8 segment (the
    default for 4 kv heads per workgroup), the fixed-chunk launch
    (KVC_DECODE_STREAMK=0) and stream-K with register segments
    (KVC_DECODE_LDS=0)."""
    monkeypatch.setenv("KVC_DECODE_STREAMK", "0" if request.param == "fixed-chunk" else "1")
    monkeypatch.setenv("KVC_DECODE_LDS", "0" if request.param == "register" else "1")
    return request.param


def _tokhead_store(key, value, blocks, label, slots=None):
    N, KVH, D = key.shape
    print(f"[int8-tokhead] {label}: N={N} KVH={KVH}", flush=True)
    kc = torch.zeros(blocks, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(blocks, 256, KVH, dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    if slots is None:
        slots = torch.randperm(blocks * 256, generator=torch.Generator().manual_seed(N))[:N]
    slots = slots.to(torch.int32).to(DEV)
    store_kvcache_int8_tokhead(key, value, kc, vc, ks, vs, slots)
    torch.cuda.synchronize()
    rkc, rvc = np.zeros(kc.shape, np.int8), np.zeros(vc.shape, np.int8)
    rks, rvs = np.zeros(ks.shape, np.float32), np.zeros(vs.shape, np.float32)
    ko.store_int8_tokhead(bits(key), bits(value), rkc, rvc, rks, rvs, slots.cpu().numpy())
    assert np.array_equal(kc.cpu().numpy(), rkc), f"{label}: K codes differ"
    assert np.array_equal(vc.cpu().numpy(), rvc), f"{label}: V codes differ"
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), rks.view(np.uint32)), f"{label}: K scales"
    assert np.array_equal(vs.cpu().numpy().view(np.uint32), rvs.view(np.uint32)), f"{label}: V scales"
    return kc, vc, ks, vs, slots


def test_tokhead_store_outlier_keys_bitwise():
    # K ~ N(0,1) with 1% outliers x20, V ~ N(0,1) (the int8 KV workload).
    key = outlier_keys((1024, 4, 128), seed=1).to(DEV)
    value = torch.randn(1024, 4, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    _tokhead_store(key, value, 8, "outliers")


def test_tokhead_store_half_way_ties_and_clamps():
    # amax 127 -> s = 1 exactly: x = k + 0.5 are exact ties (half to even);
    # an all-zero row and a tiny row exercise the 1e-6 clamp.
    D = 128
    ties = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], dtype=torch.float32)
    row = torch.zeros(D)
    row[:8] = ties
    row[8] = 127.0
    rows = torch.stack([row, torch.zeros(D), torch.full((D,), 3e-7), -row])
    key = rows.view(4, 1, D).to(torch.bfloat16).to(DEV)
    kc, _, ks, _, slots = _tokhead_store(key, key.clone(), 1, "ties", slots=torch.arange(4))
    codes = kc.view(-1, 1, D)[:4, 0, :9].cpu().tolist()
    assert codes[0] == [0, 2, 2, 0, -2, -2, 126, -126, 127]


def test_tokhead_dequant_bitwise():
    key = outlier_keys((256, 4, 128), seed=5).to(DEV)
    kc, _, ks, _, slots = _tokhead_store(key, key.clone(), 2, "dequant")
    codes = kc.view(-1, 4, 128)[slots.long()]
    scales = ks.view(-1, 4)[slots.long()]
    out = dequant_tokhead(codes, scales)
    torch.cuda.synchronize()
    ref = ko.dequant_tokhead(codes.cpu().numpy(), scales.cpu().numpy())
    assert np.array_equal(bits(out), ref)


def test_chan_store_matches_p17_unit_bitwise():
    key, value, s_k, s_v, _, _, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape
    assert int(head_n_out.sum()) > 0
    print(f"[int8-chan] p17 unit: outliers per head {head_n_out.tolist()}", flush=True)
    blocks, nout = 9, out_idx2d.shape[1]
    slot = torch.arange(N, dtype=torch.int32)
    kc = torch.zeros(blocks, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(blocks, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    store_kvcache_int8(key.to(DEV), value.to(DEV), kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv,
                       out_idx2d.to(DEV), head_n_out.to(DEV), slot.to(DEV))
    torch.cuda.synchronize()
    rkc, rvc = np.zeros(kc.shape, np.int8), np.zeros(vc.shape, np.int8)
    rsk, rsv = np.zeros(sk.shape, np.uint16), np.zeros(sv.shape, np.uint16)
    ko.store_int8_chan(bits(key), bits(value), rkc, rvc, s_k.numpy(), s_v.numpy(), rsk, rsv,
                       out_idx2d.numpy(), head_n_out.numpy(), slot.numpy())
    for name, a, b in (("k_payload", kc.cpu().numpy(), rkc), ("v_payload", vc.cpu().numpy(), rvc),
                       ("k_side", bits(sk), rsk), ("v_side", bits(sv), rsv)):
        assert np.array_equal(a, b), f"{name} differs"


def test_chan_store_strided_v():
    # The reference kernel reads V with K's strides; this path takes V's own.
    key, value, s_k, s_v, _, _, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape
    fused = torch.cat([key.view(N, -1), value.view(N, -1)], dim=1).to(DEV)
    k_view = fused[:, :KVH * D].view(N, KVH, D)
    v_view = fused[:, KVH * D:].view(N, KVH, D)
    nout = out_idx2d.shape[1]
    kc = torch.zeros(3, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(3, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    slot = torch.arange(N, dtype=torch.int32, device=DEV)
    store_kvcache_int8(k_view, v_view, kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv,
                       out_idx2d.to(DEV), head_n_out.to(DEV), slot)
    torch.cuda.synchronize()
    rvc = np.zeros(vc.shape, np.int8)
    rkc = np.zeros(kc.shape, np.int8)
    rsk, rsv = np.zeros(sk.shape, np.uint16), np.zeros(sv.shape, np.uint16)
    ko.store_int8_chan(bits(key), bits(value), rkc, rvc, s_k.numpy(), s_v.numpy(), rsk, rsv,
                       out_idx2d.numpy(), head_n_out.numpy(), slot.cpu().numpy())
    assert np.array_equal(vc.cpu().numpy(), rvc)
    assert np.array_equal(bits(sv), rsv)


def test_chan_dequant_gathered_bitwise_and_relerr():
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape
    nout = out_idx2d.shape[1]
    rkc = np.zeros((3, 256, KVH, D), np.int8)
    rvc = np.zeros_like(rkc)
    rsk = np.zeros((3, 256, KVH, nout), np.uint16)
    rsv = np.zeros_like(rsk)
    slot = np.arange(N)
    ko.store_int8_chan(bits(key), bits(value), rkc, rvc, s_k.numpy(), s_v.numpy(), rsk, rsv,
                       out_idx2d.numpy(), head_n_out.numpy(), slot)
    gq = torch.from_numpy(rkc.reshape(-1, KVH, D)[:N].copy()).to(DEV)
    gside = torch.from_numpy(rsk.reshape(-1, KVH, nout)[:N].view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    out = dequant_gathered(gq, ds_k.to(DEV), gside, out_idx2d.to(DEV), head_n_out.to(DEV))
    torch.cuda.synchronize()
    ref = ko.dequant_chan(gq.cpu().numpy(), ds_k.numpy(), bits(gside), out_idx2d.numpy(),
                          head_n_out.numpy())
    assert np.array_equal(bits(out), ref)
    rel = float((out.float().cpu() - key.float()).abs().mean() / key.float().abs().mean())
    assert rel < 0.03


def _decode_int8_tokhead_case(batch, lens, blocks, seed, label):
    wl = decode_workload(batch, 32, 4, blocks, lens, seed=seed, device=DEV, kv_dtype="int8_tokhead")
    print(f"[int8-decode] {label}: B={batch} max_ctx={max(lens)}", flush=True)
    out = paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.block_tables, wl.context_lens,
                                 wl.scale, max(lens), k_scale=wl.k_scale, v_scale=wl.v_scale)
    torch.cuda.synchronize()
    kc, bt = gathered_pool(wl.k_cache, wl.block_tables)
    vc, _ = gathered_pool(wl.v_cache, wl.block_tables)
    ksc, _ = gathered_pool(wl.k_scale, wl.block_tables)
    vsc, _ = gathered_pool(wl.v_scale, wl.block_tables)
    kf = ko.kv_float(kc.numpy(), "int8_tokhead", ksc.numpy())
    vf = ko.kv_float(vc.numpy(), "int8_tokhead", vsc.numpy())
    ref = ko.paged_decode_ref(bits(wl.q), kf, vf, bt, np.asarray(lens), wl.scale)
    assert_attention_close(out, ref, label)


def test_int8_tokhead_decode_small(decode_path):
    _decode_int8_tokhead_case(6, uniform_lengths(6, 1, 3000, seed=4), 80, 5, "tokhead-small")


def test_int8_tokhead_decode_long_context(decode_path):
    _decode_int8_tokhead_case(2, [32768, 12345], 200, 6, "tokhead-32k")


def test_int8_tokhead_end_to_end_quantised_decode(decode_path):
    # Append real activations through the quantiser, then decode the int8 pool.
    B, H, KVH, D, blocks = 4, 32, 4, 128, 24
    lens = [700, 1, 1500, 256]
    g = torch.Generator().manual_seed(8)
    bt = build_block_tables(lens, blocks, 256, g)
    kc = torch.zeros(blocks, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(blocks, 256, KVH, dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    slots = []
    for i, n in enumerate(lens):
        for t in range(n):
            slots.append(int(bt[i, t // 256]) * 256 + t % 256)
    N = len(slots)
    key = outlier_keys((N, KVH, D), seed=9).to(DEV)
    value = torch.randn(N, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    store_kvcache_int8_tokhead(key, value, kc, vc, ks, vs,
                               torch.tensor(slots, dtype=torch.int32, device=DEV))
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = paged_decode_attention(q, kc, vc, bt.to(DEV), lens_t, D ** -0.5, max(lens),
                                 k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.cpu().numpy(), "int8_tokhead", ks.cpu().numpy())
    vf = ko.kv_float(vc.cpu().numpy(), "int8_tokhead", vs.cpu().numpy())
    ref = ko.paged_decode_ref(bits(q), kf, vf, bt.numpy(), np.asarray(lens), D ** -0.5)
    assert_attention_close(out, ref, "tokhead-e2e")


def test_int8_chan_decode_with_side_pool(decode_path):
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape   # 512 tokens, 8 kv heads
    H = 16
    nout = out_idx2d.shape[1]
    blocks = 4
    lens = [512, 300]
    bt = torch.tensor([[2, 0], [1, 3]], dtype=torch.int32)
    slots = [int(bt[0, t // 256]) * 256 + t % 256 for t in range(512)]
    kc = torch.zeros(blocks, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(blocks, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    store_kvcache_int8(key.to(DEV), value.to(DEV), kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv,
                       out_idx2d.to(DEV), head_n_out.to(DEV),
                       torch.tensor(slots, dtype=torch.int32, device=DEV))
    slots2 = [int(bt[1, t // 256]) * 256 + t % 256 for t in range(300)]
    store_kvcache_int8(key[:300].flip(0).contiguous().to(DEV), value[:300].to(DEV), kc, vc,
                       s_k.to(DEV), s_v.to(DEV), sk, sv, out_idx2d.to(DEV), head_n_out.to(DEV),
                       torch.tensor(slots2, dtype=torch.int32, device=DEV))
    q = torch.randn(2, H, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
    print("[int8-chan-decode] side pool", flush=True)
    out = paged_decode_attention(q, kc, vc, bt.to(DEV), lens_t, D ** -0.5, 512,
                                 k_scale=ds_k.to(DEV), v_scale=ds_v.to(DEV), side_k=sk, side_v=sv,
                                 out_idx2d=out_idx2d.to(DEV), head_n_out=head_n_out.to(DEV))
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.cpu().numpy(), "int8_chan", ds_k.numpy(), bits(sk), out_idx2d.numpy(),
                     head_n_out.numpy())
    vf = ko.kv_float(vc.cpu().numpy(), "int8_chan", ds_v.numpy(), bits(sv), out_idx2d.numpy(),
                     head_n_out.numpy())
    ref = ko.paged_decode_ref(bits(q), kf, vf, bt.numpy(), np.asarray(lens), D ** -0.5)
    assert_attention_close(out, ref, "chan-side")


@pytest.mark.parametrize("n_out_max", [1, 2, 4, 8])
def test_int8_chan_decode_side_widths(decode_path, n_out_max):
    """Per-channel decode at every side-pool width the reference kernel admits
    (tl.arange(0, N_OUT_MAX) needs a power of two; paged_attention.py:107):
    kv heads with 0, 1, ..., n_out_max outlier dims, contexts across page and
    tile boundaries, and NaN in the side slots past each head's count (no
    such slot may reach the output)."""
    B, H, KVH, D, page, blocks = 5, 32, 4, 128, 256, 48
    lens = [4097, 300, 1, 2500, 256 * 7 + 31]
    g = torch.Generator().manual_seed(40 + n_out_max)
    bt = build_block_tables(lens, blocks, page, g)
    kc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    counts = [n_out_max, 0, max(n_out_max - 1, 1), n_out_max // 2]
    head_n_out = torch.tensor(counts, dtype=torch.int32)
    out_idx2d = torch.zeros(KVH, n_out_max, dtype=torch.int32)
    ds_k = torch.rand(KVH, D, generator=g) * 0.02 + 0.01
    ds_v = torch.rand(KVH, D, generator=g) * 0.02 + 0.01
    for h in range(KVH):
        dims = torch.randperm(D, generator=g)[:n_out_max].to(torch.int32)
        out_idx2d[h] = dims
        ds_k[h, dims[:counts[h]].long()] = 0.0
        ds_v[h, dims[:counts[h]].long()] = 0.0
    sk = (torch.randn(blocks, page, KVH, n_out_max, generator=g) * 4).to(torch.bfloat16)
    sv = (torch.randn(blocks, page, KVH, n_out_max, generator=g) * 4).to(torch.bfloat16)
    for h in range(KVH):
        sk[:, :, h, counts[h]:] = float("nan")
        sv[:, :, h, counts[h]:] = float("nan")
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    print(f"[int8-chan-widths] n_out_max={n_out_max} counts={counts} lens={lens}", flush=True)
    out = paged_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV),
                                 torch.tensor(lens, dtype=torch.int32, device=DEV), D ** -0.5,
                                 max(lens), k_scale=ds_k.to(DEV), v_scale=ds_v.to(DEV),
                                 side_k=sk.to(DEV), side_v=sv.to(DEV),
                                 out_idx2d=out_idx2d.to(DEV), head_n_out=head_n_out.to(DEV))
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.numpy(), "int8_chan", ds_k.numpy(), bits(sk), out_idx2d.numpy(),
                     head_n_out.numpy())
    vf = ko.kv_float(vc.numpy(), "int8_chan", ds_v.numpy(), bits(sv), out_idx2d.numpy(),
                     head_n_out.numpy())
    ref = ko.paged_decode_ref(bits(q), kf, vf, bt.numpy(), np.asarray(lens), D ** -0.5)
    assert_attention_close(out, ref, f"chan-widths-{n_out_max}")


def test_chan_calibration_on_device_matches_p17_unit_case():
    """KVCacheRunner.kv_calibrate_begin / the bound layer's kv_observe hook /
    kv_calibrate_freeze (model_runner.py:510-577) on the seeded unit case of
    tests/p17_kv_int8.py:64-101, observed as three forwards of 200, 300 and
    12 tokens: store scales, read scales, out_idx2d and head_n_out equal the
    unit case's calibration bit for bit; the append with the frozen scales is
    the oracle's, and dequantisation is within 3 % (p17_kv_int8.py:126-134)."""
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    from nanovllm_amd.layers.attention import Attention
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape
    n_out = out_idx2d.shape[1]
    print(f"[int8-calib] p17 unit case N={N} KVH={KVH} n_out_max={n_out}", flush=True)
    runner = KVCacheRunner(1, 8, 256, KVH, D, kv_int8="chan", n_out_max=n_out)
    mod = Attention(16, D, D ** -0.5, KVH)
    assert runner.bind([mod]) == 1 and mod.kv_observe is not None
    mod.kv_observe(0, key.to(DEV), value.to(DEV))          # before begin: ignored
    runner.kv_calibrate_begin()
    kd, vd = key.to(DEV), value.to(DEV)
    for a, b in ((0, 200), (200, 500), (500, 512)):
        mod.kv_observe(0, kd[a:b], vd[a:b])
    summary = runner.kv_calibrate_freeze()
    assert summary["outlier_dims"] == int(head_n_out.sum())
    u32 = lambda t: t.cpu().contiguous().view(torch.int32).numpy()
    for got, want, name in ((runner.kv_scales[0, 0], s_k, "k_scale"),
                            (runner.kv_scales[1, 0], s_v, "v_scale"),
                            (runner.kv_dscales[0, 0], ds_k, "k_dscale"),
                            (runner.kv_dscales[1, 0], ds_v, "v_dscale")):
        assert np.array_equal(u32(got), u32(want)), name
    assert torch.equal(runner.kv_head_n_out[0].cpu(), head_n_out)
    for h in range(KVH):
        n_h = int(head_n_out[h])
        assert torch.equal(runner.kv_out_idx2d[0, h, :n_h].cpu(), out_idx2d[h, :n_h])
    # append with the frozen scales through the bound views, against the oracle
    runner.kv_cache.zero_()           # the runner's pool starts uninitialised
    slot = torch.arange(N, dtype=torch.int32, device=DEV)
    store_kvcache_int8(kd, vd, mod.k_cache, mod.v_cache, mod.k_scale, mod.v_scale, mod.side_k,
                       mod.side_v, mod.out_idx2d, mod.head_n_out, slot)
    torch.cuda.synchronize()
    kc = np.zeros((9, 256, KVH, D), np.int8)
    vc = np.zeros_like(kc)
    sdk = np.zeros((9, 256, KVH, n_out), np.uint16)
    sdv = np.zeros_like(sdk)
    ko.store_int8_chan(bits(key), bits(value), kc, vc, s_k.numpy(), s_v.numpy(), sdk, sdv,
                       out_idx2d.numpy(), head_n_out.numpy(), np.arange(N))
    assert np.array_equal(mod.k_cache.cpu().numpy(), kc)
    assert np.array_equal(mod.v_cache.cpu().numpy(), vc)
    assert np.array_equal(bits(mod.side_k), sdk) and np.array_equal(bits(mod.side_v), sdv)
    deq = dequant_gathered(mod.k_cache.view(-1, KVH, D)[:N], mod.k_dscale,
                           mod.side_k.view(-1, KVH, n_out)[:N], mod.out_idx2d, mod.head_n_out)
    rel = float((deq.float().cpu() - key.float()).abs().mean() / key.float().abs().mean())
    print(f"[int8-calib] dequant rel err {rel:.4%}", flush=True)
    assert rel < 0.03


def test_chan_calibration_follows_the_engine_hook_over_forwards():
    """Calibration over three forwards of 300, 250 and 350 tokens whose
    per-forward sums of |x| round to bf16 (model_runner.py:529-532): the
    device statistics equal the oracle's fold bit for bit (amax, fp32 sum of
    bf16-rounded forward sums), and the frozen store scales, read scales,
    out_idx2d and head_n_out equal the oracle's freeze.  Two dims of head 0
    are outliers under the hook's rounding and not under fp32 sums (or the
    reverse), so a kernel that skips the rounding fails here."""
    from helpers import calib_flip_forwards
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    from nanovllm_amd.layers.attention import Attention
    forwards, dims = calib_flip_forwards()
    KVH, D, n_out = 4, 128, 4
    print(f"[int8-calib] flip case: forwards {[k.shape[0] for k, _ in forwards]}, "
          f"dims {dims}", flush=True)
    runner = KVCacheRunner(1, 4, 256, KVH, D, kv_int8="chan", n_out_max=n_out)
    mod = Attention(32, D, D ** -0.5, KVH)
    assert runner.bind([mod]) == 1
    runner.kv_calibrate_begin()
    for k, v in forwards:
        mod.kv_observe(0, k.to(DEV), v.to(DEV))
    amax_dev, sum_dev = runner._calib[0][0].cpu().numpy(), runner._calib[1][0].cpu().numpy()
    a_k, s_k, n = ko.calib_fold([bits(k) for k, _ in forwards])
    a_v, s_v, _ = ko.calib_fold([bits(v) for _, v in forwards])
    u32 = lambda a: np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    assert np.array_equal(u32(amax_dev[0]), u32(a_k)) and np.array_equal(u32(amax_dev[1]), u32(a_v))
    assert np.array_equal(u32(sum_dev[0]), u32(s_k)) and np.array_equal(u32(sum_dev[1]), u32(s_v))
    runner.kv_calibrate_freeze()
    want = ko.calib_freeze(a_k, a_v, s_k, s_v, n, n_out)
    for got, w, name in ((runner.kv_scales[0, 0], want[0], "k_scale"),
                         (runner.kv_scales[1, 0], want[1], "v_scale"),
                         (runner.kv_dscales[0, 0], want[2], "k_dscale"),
                         (runner.kv_dscales[1, 0], want[3], "v_dscale")):
        assert np.array_equal(u32(got.cpu().numpy()), u32(w)), name
    n_got = runner.kv_head_n_out[0].cpu().numpy()
    assert np.array_equal(n_got, want[5])
    for h in range(KVH):
        assert np.array_equal(runner.kv_out_idx2d[0, h, :n_got[h]].cpu().numpy(),
                              want[4][h, :n_got[h]])
    head0 = set(want[4][0, :want[5][0]].tolist())
    assert dims["hook_out"] in head0 and dims["hook_in"] not in head0


@pytest.mark.parametrize("case", ["b16x4096", "ragged-with-empty", "int64-negative-slots",
                                  "unaligned-key-refused", "two-kv-heads-fallback",
                                  "eight-kv-heads"])
def test_int8_tokhead_decode_append_equals_store_then_decode(case, decode_path):
    """paged_decode_append_int8_tokhead (the per-token-head quantiser inside
    the decode launch where the layout allows) against
    store_kvcache_int8_tokhead then paged_decode_attention: the same output
    bits, codes and scales, and the codes and scales of the new tokens are
    the oracle's (scripts/archive/p14_int8_kv_probe.py:37-41)."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_append_int8_tokhead
    heads, kvh = {"two-kv-heads-fallback": (16, 2), "eight-kv-heads": (16, 8)}.get(case, (32, 4))
    if case == "b16x4096":
        lens, nb = [4096] * 16, 300
    elif case == "ragged-with-empty":
        lens, nb = [1, 0, 33, 4096, 257, 0, 9000, 31], 80
    else:
        lens, nb = uniform_lengths(20, 1, 5000, seed=63), 600
    wl = decode_workload(len(lens), heads, kvh, nb, [max(1, n) for n in lens], seed=len(lens) + 5,
                         device=DEV, pool_device_fill=True, kv_dtype="int8_tokhead")
    wl.context_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    slots = wl.slot_mapping.clone()
    num_slots = wl.k_cache.size(0) * wl.k_cache.size(1)
    if case == "int64-negative-slots":
        slots = slots.long()
        slots[::3] -= num_slots
    g = torch.Generator(device=DEV).manual_seed(9)
    key = (torch.randn(wl.new_k.shape, generator=g, device=DEV) *
           torch.where(torch.rand(wl.new_k.shape, generator=g, device=DEV) < 0.02, 20.0, 1.0)
           ).to(torch.bfloat16)
    value = wl.new_v
    if case == "unaligned-key-refused":
        big = torch.randn(len(lens), kvh * 128 + 4, dtype=torch.bfloat16, device=DEV)
        big[:, 4:] = key.reshape(len(lens), -1)
        key = big[:, 4:].view(len(lens), kvh, 128)
    print(f"[int8-tokhead] fused append {case}: B={len(lens)} {heads}q/{kvh}kv", flush=True)
    if case == "unaligned-key-refused":
        # the quantiser reads 16-byte vectors: both forms refuse 8-byte aligned rows
        with pytest.raises(AssertionError, match="16-byte aligned"):
            store_kvcache_int8_tokhead(key, value, wl.k_cache, wl.v_cache, wl.k_scale,
                                       wl.v_scale, slots)
        with pytest.raises(AssertionError, match="16-byte aligned"):
            paged_decode_append_int8_tokhead(wl.q, key, value, wl.k_cache, wl.v_cache,
                                             wl.k_scale, wl.v_scale, slots, wl.block_tables,
                                             wl.context_lens, wl.scale)
        return
    kc0, vc0 = wl.k_cache.clone(), wl.v_cache.clone()
    ks0, vs0 = wl.k_scale.clone(), wl.v_scale.clone()
    store_kvcache_int8_tokhead(key, value, kc0, vc0, ks0, vs0, slots)
    ref = paged_decode_attention(wl.q, kc0, vc0, wl.block_tables, wl.context_lens, wl.scale, 0,
                                 k_scale=ks0, v_scale=vs0)
    out = paged_decode_append_int8_tokhead(wl.q, key, value, wl.k_cache, wl.v_cache, wl.k_scale,
                                           wl.v_scale, slots, wl.block_tables, wl.context_lens,
                                           wl.scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(ref)), "outputs differ from store + decode"
    assert torch.equal(wl.k_cache, kc0) and torch.equal(wl.v_cache, vc0)
    assert torch.equal(wl.k_scale.view(torch.int32), ks0.view(torch.int32))
    assert torch.equal(wl.v_scale.view(torch.int32), vs0.view(torch.int32))
    sl = slots.long() % num_slots
    for x, codes, sc in ((key, wl.k_cache, wl.k_scale), (value, wl.v_cache, wl.v_scale)):
        want_c, want_s = ko.quant_tokhead(bits(x))
        assert np.array_equal(codes.view(-1, kvh, 128)[sl].cpu().numpy(), want_c)
        assert np.array_equal(sc.view(-1, kvh)[sl].cpu().numpy().view(np.uint32),
                              want_s.view(np.uint32))


@pytest.mark.parametrize("n_out_max", [8, 4, 1])
def test_int8_chan_decode_append_equals_store_then_decode(n_out_max, decode_path):
    """paged_decode_append_int8_chan (the engine's per-channel int8 step in one
    call) against store_kvcache_int8 then paged_decode_attention: the same
    codes and side values in the pools and the same output bits, with heads
    holding 0 .. n_out_max outlier dims, ragged contexts with an empty row,
    and int64 slots given in Python's negative form."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_append_int8_chan
    B, H, KVH, D, page, blocks = 7, 32, 4, 128, 256, 70
    lens = [1, 0, 4097, 300, 2600, 33, 1800]
    g = torch.Generator().manual_seed(70 + n_out_max)
    bt = build_block_tables([max(1, n) for n in lens], blocks, page, g)
    kc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    counts = [n_out_max, 0, max(n_out_max - 1, 1), n_out_max // 2]
    head_n_out = torch.tensor(counts, dtype=torch.int32)
    out_idx2d = torch.zeros(KVH, n_out_max, dtype=torch.int32)
    s_k = torch.rand(KVH, D, generator=g) * 0.02 + 0.01
    s_v = torch.rand(KVH, D, generator=g) * 0.02 + 0.01
    ds_k, ds_v = s_k.clone(), s_v.clone()
    for h in range(KVH):
        dims = torch.randperm(D, generator=g)[:n_out_max].to(torch.int32)
        out_idx2d[h] = dims
        ds_k[h, dims[:counts[h]].long()] = 0.0
        ds_v[h, dims[:counts[h]].long()] = 0.0
    sk = (torch.randn(blocks, page, KVH, n_out_max, generator=g) * 4).to(torch.bfloat16)
    sv = (torch.randn(blocks, page, KVH, n_out_max, generator=g) * 4).to(torch.bfloat16)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    key = (torch.randn(B, KVH, D, generator=g) * 0.5).to(torch.bfloat16)
    value = (torch.randn(B, KVH, D, generator=g) * 0.5).to(torch.bfloat16)
    slots = torch.tensor([int(bt[i, (max(1, n) - 1) // page]) * page + (max(1, n) - 1) % page
                          for i, n in enumerate(lens)], dtype=torch.int64)
    slots[::2] -= blocks * page
    dev = {k: v.to(DEV) for k, v in dict(kc=kc, vc=vc, sk=sk, sv=sv, s_k=s_k, s_v=s_v,
                                         ds_k=ds_k, ds_v=ds_v, oi=out_idx2d, hn=head_n_out,
                                         q=q, key=key, value=value, slots=slots,
                                         bt=bt).items()}
    lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
    print(f"[int8-chan] step in one call: n_out_max={n_out_max} counts={counts}", flush=True)
    kc0, vc0, sk0, sv0 = dev["kc"].clone(), dev["vc"].clone(), dev["sk"].clone(), dev["sv"].clone()
    store_kvcache_int8(dev["key"], dev["value"], kc0, vc0, dev["s_k"], dev["s_v"], sk0, sv0,
                       dev["oi"], dev["hn"], dev["slots"])
    ref = paged_decode_attention(dev["q"], kc0, vc0, dev["bt"], lens_t, D ** -0.5, 0,
                                 k_scale=dev["ds_k"], v_scale=dev["ds_v"], side_k=sk0,
                                 side_v=sv0, out_idx2d=dev["oi"], head_n_out=dev["hn"])
    kc1, vc1, sk1, sv1 = dev["kc"].clone(), dev["vc"].clone(), dev["sk"].clone(), dev["sv"].clone()
    out = paged_decode_append_int8_chan(dev["q"], dev["key"], dev["value"], kc1, vc1, dev["s_k"],
                                        dev["s_v"], dev["ds_k"], dev["ds_v"], sk1, sv1,
                                        dev["oi"], dev["hn"], dev["slots"], dev["bt"], lens_t,
                                        D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0), "codes differ"
    assert torch.equal(sk1.view(torch.int16), sk0.view(torch.int16)), "K side values differ"
    assert torch.equal(sv1.view(torch.int16), sv0.view(torch.int16)), "V side values differ"
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), "outputs differ"
    # and the stored token itself is the oracle's per-channel quantisation
    rk, rv = np.zeros((B, KVH, D), np.int8), np.zeros((B, KVH, D), np.int8)
    rsk, rsv = np.zeros((B, KVH, n_out_max), np.uint16), np.zeros((B, KVH, n_out_max), np.uint16)
    for i in range(B):
        ko.store_int8_chan(bits(key[i:i + 1]), bits(value[i:i + 1]), rk[i:i + 1], rv[i:i + 1],
                           s_k.numpy(), s_v.numpy(), rsk[i:i + 1], rsv[i:i + 1],
                           out_idx2d.numpy(), head_n_out.numpy(), np.zeros(1, np.int64))
    flat = lambda t: t.reshape(-1, KVH, t.shape[-1])
    sl = (slots % (blocks * page)).numpy()
    assert np.array_equal(flat(kc1.cpu()).numpy()[sl], rk)
    assert np.array_equal(flat(vc1.cpu()).numpy()[sl], rv)
    for h in range(KVH):
        n = counts[h]
        assert np.array_equal(bits(flat(sk1.cpu())[sl])[:, h, :n], rsk[:, h, :n])
        assert np.array_equal(bits(flat(sv1.cpu())[sl])[:, h, :n], rsv[:, h, :n])


def test_chan_layer_decode_step_is_store_then_decode():
    """Attention.forward's decode step over a bound per-channel pool (after a
    calibration freeze) runs the one-call step, and its output, codes and
    side values equal the engine's two calls, store_kvcache_int8 then
    paged_decode_attention with the read scales (attention.py:130-177)."""
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    from nanovllm_amd.layers.attention import Attention
    from nanovllm_amd.utils.context import reset_context, set_context
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    N, KVH, D = key.shape
    n_out = out_idx2d.shape[1]
    H, B = 16, 3
    runner = KVCacheRunner(1, 12, 256, KVH, D, kv_int8="chan", n_out_max=n_out)
    mod = Attention(H, D, D ** -0.5, KVH)
    assert runner.bind([mod]) == 1
    runner.kv_calibrate_begin()
    mod.kv_observe(0, key.to(DEV), value.to(DEV))
    runner.kv_calibrate_freeze()
    assert mod._int8_chan_step()
    runner.kv_cache.zero_()
    runner.kv_side.zero_()
    # three sequences of 512 / 300 / 700 tokens already in the pool, then one step
    lens = [512, 300, 700]
    g = torch.Generator().manual_seed(31)
    bt = build_block_tables([n + 1 for n in lens], 12, 256, g)
    prior = torch.randn(sum(lens), KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    pslots = torch.tensor([int(bt[i, t // 256]) * 256 + t % 256
                           for i, n in enumerate(lens) for t in range(n)],
                          dtype=torch.int32, device=DEV)
    store_kvcache_int8(prior, prior.flip(0).contiguous(), mod.k_cache, mod.v_cache, mod.k_scale,
                       mod.v_scale, mod.side_k, mod.side_v, mod.out_idx2d, mod.head_n_out, pslots)
    slots = torch.tensor([int(bt[i, n // 256]) * 256 + n % 256 for i, n in enumerate(lens)],
                         dtype=torch.int32, device=DEV)
    ctx = torch.tensor([n + 1 for n in lens], dtype=torch.int32, device=DEV)
    q = torch.randn(B, H * D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, KVH * D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, KVH * D, generator=g).to(torch.bfloat16).to(DEV)
    kc0, vc0 = mod.k_cache.clone(), mod.v_cache.clone()
    sk0, sv0 = mod.side_k.clone(), mod.side_v.clone()
    store_kvcache_int8(k.view(B, KVH, D), v.view(B, KVH, D), kc0, vc0, mod.k_scale, mod.v_scale,
                       sk0, sv0, mod.out_idx2d, mod.head_n_out, slots)
    ref = paged_decode_attention(q.view(B, H, D), kc0, vc0, bt.to(DEV), ctx, D ** -0.5, 0,
                                 k_scale=mod.k_dscale, v_scale=mod.v_dscale, side_k=sk0,
                                 side_v=sv0, out_idx2d=mod.out_idx2d, head_n_out=mod.head_n_out)
    print("[int8-chan] layer decode step", flush=True)
    try:
        set_context(False, slot_mapping=slots, context_lens=ctx, block_tables=bt.to(DEV),
                    max_context_len=max(lens) + 1)
        out = mod.forward(q, k, v)
    finally:
        reset_context()
    torch.cuda.synchronize()
    assert torch.equal(mod.k_cache, kc0) and torch.equal(mod.v_cache, vc0)
    assert torch.equal(mod.side_k.view(torch.int16), sk0.view(torch.int16))
    assert torch.equal(mod.side_v.view(torch.int16), sv0.view(torch.int16))
    assert torch.equal(out.view(B, H, D).view(torch.int16), ref.view(torch.int16))
