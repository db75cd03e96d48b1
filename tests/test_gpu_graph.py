"""Capture-safe decode step: the decode KV work (append + paged decode, per
layer) captured once per batch bucket and replayed with padded rows aimed at
the scratch block (nanovllm/engine/model_runner.py:842-871).

Every replay is checked bit for bit against the same padded batch run
eagerly on a copy of the pools (same kernels, same launch plan), the live
rows also against the oracle (2e-2 max / 2e-3 mean), and the pools must
differ from their previous state only at the live slots and in the scratch
block.  Replays are interleaved with eager work and synchronisations.
"""
import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits
from nanovllm_amd.engine.graph_runner import DecodeGraphRunner, pad_decode_inputs
from nanovllm_amd.kernels.paged_attention import paged_decode_attention
from nanovllm_amd.layers.attention import store_kvcache
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"
L, H, KVH, PAGE, NB, MAXB = 2, 32, 4, 256, 72, 8


def _batch(bs, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, MAXB * PAGE + 1, (bs,), generator=g).tolist()
    perm = torch.randperm(NB, generator=g).tolist()
    tables = torch.full((bs, MAXB), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(lens):
        nb = (n + PAGE - 1) // PAGE
        tables[i, :nb] = torch.tensor(perm[pos:pos + nb], dtype=torch.int32)
        pos += nb
    slots = torch.tensor([int(tables[i, (n - 1) // PAGE]) * PAGE + (n - 1) % PAGE
                          for i, n in enumerate(lens)], dtype=torch.int32)
    q = torch.randn(L, bs, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(L, bs, KVH, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(L, bs, KVH, 128, generator=g).to(torch.bfloat16)
    return (q.to(DEV), k.to(DEV), v.to(DEV), slots.to(DEV),
            torch.tensor(lens, dtype=torch.int32).to(DEV), tables.to(DEV), lens)


def _eager_padded(kcs, vcs, q, k, v, slots, lens, tables, bucket, runner):
    """The bucket's padded batch run eagerly on the given pools."""
    bs = q.size(1)
    sb = torch.empty(bucket, dtype=torch.int32, device=DEV)
    lb = torch.empty(bucket, dtype=torch.int32, device=DEV)
    tb = torch.empty(bucket, MAXB, dtype=torch.int32, device=DEV)
    pad_decode_inputs(slots, lens, tables, sb, lb, tb, runner.scratch_slot, runner.scratch_block_id)
    qp = torch.zeros_like(runner.q[:, :bucket])
    kp = torch.zeros_like(runner.k[:, :bucket])
    vp = torch.zeros_like(runner.v[:, :bucket])
    qp[:, :bs], kp[:, :bs], vp[:, :bs] = q, k, v  # padded rows are zeros
    outs = []
    for layer in range(L):
        store_kvcache(kp[layer], vp[layer], kcs[layer], vcs[layer], sb)
        outs.append(paged_decode_attention(qp[layer], kcs[layer], vcs[layer], tb, lb,
                                           128 ** -0.5, MAXB * PAGE))
    return torch.stack(outs)[:, :bs]


def test_graph_replays_match_eager_and_touch_only_live_slots_and_scratch(
        deterministic_decode):
    g = torch.Generator().manual_seed(0)
    kcs = [torch.randn(NB + 1, PAGE, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
           for _ in range(L)]
    vcs = [torch.randn(NB + 1, PAGE, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
           for _ in range(L)]
    runner = DecodeGraphRunner(kcs, vcs, H, max_bs=16, max_blocks_per_seq=MAXB,
                               scale=128 ** -0.5)
    runner.capture()
    print(f"[graph] captured buckets {sorted(runner.graphs)}", flush=True)
    scratch = runner.scratch_block_id
    for rnd, bs in enumerate([5, 8, 3, 5]):
        print(f"[graph] replay {rnd}: batch {bs}", flush=True)
        q, k, v, slots, lens, tables, lens_list = _batch(bs, seed=100 + rnd)
        before_k = [c.clone() for c in kcs]
        before_v = [c.clone() for c in vcs]
        ek = [c.clone() for c in kcs]
        ev = [c.clone() for c in vcs]
        bucket = runner.bucket_of(bs)
        want = _eager_padded(ek, ev, q, k, v, slots, lens, tables, bucket, runner)
        # eager work between replays
        junk = torch.randn(512, 512, device=DEV)
        junk = (junk * 2 + 1).sum()
        torch.cuda.synchronize()
        got = runner.run(q, k, v, slots, lens, tables).clone()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), f"replay {rnd}: outputs differ from eager"
        for layer in range(L):
            assert np.array_equal(bits(kcs[layer]), bits(ek[layer]))
            assert np.array_equal(bits(vcs[layer]), bits(ev[layer]))
            # Only the live slots and the scratch block changed.
            flat_b = before_k[layer].view(-1, KVH * 128)
            flat_a = kcs[layer].view(-1, KVH * 128)
            changed = (bits(flat_a) != bits(flat_b)).any(axis=1)
            allowed = np.zeros(changed.shape, dtype=bool)
            allowed[slots.cpu().numpy()] = True
            allowed[scratch * PAGE:(scratch + 1) * PAGE] = True
            assert not (changed & ~allowed).any(), "a live slot outside the batch changed"
            assert np.array_equal(bits(kcs[layer].view(-1, KVH, 128)[slots.long()]),
                                  bits(k[layer]))
            # Live rows against the oracle.
            kc = ko.bf16_to_f32(bits(kcs[layer]))
            vc = ko.bf16_to_f32(bits(vcs[layer]))
            ref = ko.paged_decode_ref(bits(q[layer]), kc, vc, tables.cpu().numpy(),
                                      np.asarray(lens_list), 128 ** -0.5)
            assert_attention_close(got[layer], ref, f"replay {rnd} layer {layer}")
        del before_k, before_v, ek, ev


def _runner_with_pool(init, async_groups):
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    L_, nb = init.size(1), init.size(2) - 1
    r = KVCacheRunner(L_, nb, PAGE, KVH, 128, kv_offload_host_blocks=4,
                      async_offload_groups=async_groups, async_copy_engine="dma")
    r.kv_cache.copy_(init)
    return r


def test_graph_replay_after_async_eviction_of_the_appended_block(deterministic_decode):
    """An eviction put of block B on the copy streams, then a graph replay
    whose appends land in B (the block manager reallocated it): the runner
    built by from_kv_runner fences before the replay, so the host slot holds
    B as it was before the append, and the pool and outputs equal the same
    sequence with blocking offload."""
    Lg, nb = 8, 40
    g = torch.Generator().manual_seed(3)
    init = torch.randn(2, Lg, nb + 1, PAGE, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    bs, B = 3, 17
    lens = [PAGE + 1, 700, 2 * PAGE + 5]
    # row 0 appends at position PAGE of its table -> the first token of block B
    tables = torch.tensor([[5, B, -1], [9, 10, 11], [20, 21, 22]], dtype=torch.int32)
    slots = torch.tensor([B * PAGE, 11 * PAGE + 699 - 2 * PAGE, 22 * PAGE + 4], dtype=torch.int32)
    q = torch.randn(Lg, bs, H, 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(Lg, bs, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(Lg, bs, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    results = {}
    for groups in (0, 4):
        print(f"[graph-offload] async groups {groups}: put block {B}, replay batch {bs}",
              flush=True)
        r = _runner_with_pool(init, groups)
        gr = DecodeGraphRunner.from_kv_runner(r, H, max_bs=4, max_blocks_per_seq=3,
                                              scale=128 ** -0.5, buckets=[4])
        gr.capture()
        torch.cuda.synchronize()
        r.kv_cache.copy_(init)                      # capture wrote the scratch block only
        torch.cuda.synchronize()
        slot = r.offload_put(B)
        out = gr.run(q, k, v, slots.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                     tables.to(DEV)).clone()
        if r.kv_async is not None:
            r.kv_async.wait_host()
        torch.cuda.synchronize()
        host = bits(r.kv_offloader.buffer[slot])
        results[groups] = (bits(out), bits(r.kv_cache), host)
        assert np.array_equal(host, bits(init[:, :, B])), "host slot is not B before the append"
    for a, b in zip(results[0], results[4]):
        assert np.array_equal(a, b)
    flat = r.kv_cache.view(2, Lg, -1, KVH, 128)
    assert np.array_equal(bits(flat[0][:, slots.long().to(DEV)]), bits(k))
    assert np.array_equal(bits(flat[1][:, slots.long().to(DEV)]), bits(v))
