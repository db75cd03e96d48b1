"""The dynamic tail hand-out of the stream-K paged decode (bf16, 4 kv heads
per workgroup; opt-in with KVC_DECODE_STEAL=1): every share's last segment
ends in up to KVC_DECODE_TAIL tiles that its owner claims from the front
while workgroups done with their own shares take single tiles from the
back, each as a partial of its own.

The share skew between even and odd workgroups (KVC_XCD_SKEW, here 0.25:
even shares get 5/3 of the odd shares' tiles) makes the odd workgroups
finish early, so tiles are certainly taken; the layout query then shows how
many.  Outputs are checked against the fp32 oracle (2e-2 max / 2e-3 mean),
pool bytes of the fused append against a store, and a second launch on the
same stream reuses the claim words the first launch's merge reset.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, gathered_pool
from nanovllm_amd import _native as nat
from nanovllm_amd.layers.attention import store_kvcache
from nanovllm_amd.workloads import decode_workload, uniform_lengths
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _decode(wl, append=False, key=None, value=None, slots=None, zero_ws=False):
    """kvc_paged_decode (or kvc_paged_decode_append) with a workspace this
    test keeps: returns (out, workspace)."""
    B, H, D = wl.q.shape
    KVH = wl.k_cache.size(2)
    mb = wl.block_tables.size(1)
    ws_bytes = nat.query("kvc_paged_decode_workspace_bytes", B, H, KVH, D, 256, mb)
    ws = (torch.zeros if zero_ws else torch.empty)(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(wl.q)
    st = torch.cuda.current_stream().cuda_stream
    q, bt, cl = wl.q, wl.block_tables, wl.context_lens
    if append:
        nat.call("kvc_paged_decode_append", q.data_ptr(), q.stride(0), q.stride(1),
                 key.data_ptr(), key.stride(0), key.stride(1),
                 value.data_ptr(), value.stride(0), value.stride(1), slots.data_ptr(), 4,
                 wl.k_cache.data_ptr(), wl.v_cache.data_ptr(), wl.k_cache.size(0), 256, KVH, D,
                 bt.data_ptr(), bt.stride(0), mb, cl.data_ptr(), B, H, float(wl.scale),
                 out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws_bytes, st)
    else:
        nat.call("kvc_paged_decode", q.data_ptr(), q.stride(0), q.stride(1),
                 wl.k_cache.data_ptr(), wl.v_cache.data_ptr(), wl.k_cache.size(0), 256, KVH, D,
                 nat.KVC_KV_BF16, None, None, None, None, None, None, 0,
                 bt.data_ptr(), bt.stride(0), mb, cl.data_ptr(), B, H, float(wl.scale),
                 out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws_bytes, st)
    return out, ws


def _taken_tiles(wl, ws):
    """Tail tiles other workgroups took in the launch that used `ws`
    (every piece's count is written once per kv slice of its row unit)."""
    B, H, _ = wl.q.shape
    KVH = wl.k_cache.size(2)
    lay = (ctypes.c_int64 * 4)()
    nat.call("kvc_paged_decode_layout", B, H, KVH, 128, 256, wl.block_tables.size(1), lay)
    off_nseg, off_taken, ms, kvs = list(lay)
    assert off_taken > 0
    w = ws.cpu()
    nseg = w[off_nseg:off_nseg + B * kvs * 4].view(torch.int32).reshape(B, kvs) & 0xffff
    taken = w[off_taken:off_taken + B * kvs * ms * 4].view(torch.int32).reshape(B, kvs, ms)
    live = torch.arange(ms)[None, None, :] < nseg[:, :, None]
    return int((taken * live).sum()) // 4


def _oracle_check(wl, out, label):
    kc, bt = gathered_pool(wl.k_cache, wl.block_tables)
    vc, _ = gathered_pool(wl.v_cache, wl.block_tables)
    ref = ko.paged_decode_ref(bits(wl.q), ko.bf16_to_f32(bits(kc)), ko.bf16_to_f32(bits(vc)), bt,
                              wl.context_lens.cpu().numpy(), wl.scale)
    assert_attention_close(out, ref, label)


CASES = {
    "b64x4096": ([4096] * 64, 8192),
    "b64-ragged": (uniform_lengths(64, 512, 4096, seed=2), 8192),
    "b200-short": (uniform_lengths(200, 1, 700, seed=5), 1200),
    "b4-32k": ([32768, 30000, 20001, 32768], 700),
}


@pytest.mark.parametrize("case", list(CASES))
def test_handout_under_skew_matches_oracle(case, monkeypatch):
    monkeypatch.setenv("KVC_DECODE_STEAL", "1")
    monkeypatch.setenv("KVC_XCD_SKEW", "0.25")
    lens, nb = CASES[case]
    wl = decode_workload(len(lens), 32, 4, nb, lens, seed=len(lens) + 7, device=DEV,
                         pool_device_fill=True)
    print(f"[handout] {case}: B={len(lens)} skew 0.25", flush=True)
    taken = []
    for rep in range(2):      # the second launch reuses the claim words the first reset
        out, ws = _decode(wl)
        torch.cuda.synchronize()
        taken.append(_taken_tiles(wl, ws))
        _oracle_check(wl, out, f"{case} rep {rep}")
    print(f"[handout] {case}: tiles taken per launch {taken}", flush=True)
    if case in ("b64x4096", "b64-ragged", "b4-32k"):
        assert min(taken) > 0, "no tile was handed out under a 5:3 share skew"


def test_handout_off_takes_nothing(monkeypatch):
    monkeypatch.setenv("KVC_XCD_SKEW", "0.25")
    monkeypatch.setenv("KVC_DECODE_STEAL", "0")
    lens, nb = CASES["b64x4096"]
    wl = decode_workload(64, 32, 4, nb, lens, seed=71, device=DEV, pool_device_fill=True)
    out, ws = _decode(wl, zero_ws=True)      # the counts are not written: they stay 0
    torch.cuda.synchronize()
    assert _taken_tiles(wl, ws) == 0
    _oracle_check(wl, out, "handout off")


@pytest.mark.parametrize("case", ["b64x4096", "b64-ragged"])
def test_handout_with_fused_append(case, monkeypatch):
    """The fused append under hand-out: the row's last tile may be taken, and
    then its taker appends.  Pool bytes equal a store of the new tokens; the
    outputs match the oracle on the appended pool."""
    monkeypatch.setenv("KVC_DECODE_STEAL", "1")
    monkeypatch.setenv("KVC_XCD_SKEW", "0.25")
    lens, nb = CASES[case]
    wl = decode_workload(len(lens), 32, 4, nb, lens, seed=13, device=DEV, pool_device_fill=True)
    print(f"[handout] fused append {case}", flush=True)
    kc0, vc0 = wl.k_cache.clone(), wl.v_cache.clone()
    store_kvcache(wl.new_k, wl.new_v, kc0, vc0, wl.slot_mapping)
    out, ws = _decode(wl, append=True, key=wl.new_k, value=wl.new_v, slots=wl.slot_mapping)
    torch.cuda.synchronize()
    taken = _taken_tiles(wl, ws)
    print(f"[handout] fused append {case}: tiles taken {taken}", flush=True)
    assert torch.equal(wl.k_cache.view(torch.int16), kc0.view(torch.int16))
    assert torch.equal(wl.v_cache.view(torch.int16), vc0.view(torch.int16))
    _oracle_check(wl, out, f"fused append {case}")
    assert taken > 0
