"""kvc_paged_decode_append_static (the decode step with the library's static
per-GPU scratch instead of a caller workspace) called through the C ABI,
against kvc_paged_decode_append with a workspace: the same output bits and
the same pool bytes, on two calls in a row (the headline batch 64 x 4096,
then a smaller ragged batch that reuses the scratch the first call left
behind), the Python wrapper captured into a graph and replayed with new
inputs, and a clear error for a launch the scratch cannot hold."""
import numpy as np
import pytest
import torch

from helpers import bits
from nanovllm_amd import _native as nat
from nanovllm_amd.kernels.paged_attention import paged_decode_append, paged_decode_append_static
from nanovllm_amd.workloads import decode_workload, uniform_lengths

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _static_call(wl, k_cache, v_cache, out):
    q, key, value = wl.q, wl.new_k, wl.new_v
    sm, bt, cl = wl.slot_mapping, wl.block_tables, wl.context_lens
    assert sm.dtype == bt.dtype == cl.dtype == torch.int32
    nat.call("kvc_paged_decode_append_static",
             q.data_ptr(), q.stride(0), q.stride(1),
             key.data_ptr(), key.stride(0), key.stride(1),
             value.data_ptr(), value.stride(0), value.stride(1),
             sm.data_ptr(), 4, k_cache.data_ptr(), v_cache.data_ptr(), k_cache.size(0),
             k_cache.size(1), k_cache.size(2), 128, bt.data_ptr(), bt.stride(0), bt.size(1),
             cl.data_ptr(), q.size(0), q.size(1), float(wl.scale),
             out.data_ptr(), out.stride(0), out.stride(1),
             torch.cuda.current_stream().cuda_stream)


def test_static_scratch_equals_workspace_entry_point_twice(deterministic_decode):
    cases = [("64x4096", [4096] * 64, 1100, 3),
             ("ragged-smaller", uniform_lengths(9, 1, 2500, seed=5), 120, 4)]
    for label, lens, blocks, seed in cases:
        print(f"[no-alloc] {label}: B={len(lens)} blocks={blocks}", flush=True)
        wl = decode_workload(len(lens), 32, 4, blocks, lens, seed=seed, device=DEV,
                             pool_device_fill=True)
        kc0, vc0 = wl.k_cache.clone(), wl.v_cache.clone()
        ref = paged_decode_append(wl.q, wl.new_k, wl.new_v, kc0, vc0, wl.slot_mapping,
                                  wl.block_tables, wl.context_lens, wl.scale)
        kc1, vc1 = wl.k_cache.clone(), wl.v_cache.clone()
        out = torch.full_like(wl.q, float("nan"))
        _static_call(wl, kc1, vc1, out)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), bits(ref)), f"{label}: outputs differ"
        assert torch.equal(kc1.view(torch.int16), kc0.view(torch.int16)), f"{label}: K pool"
        assert torch.equal(vc1.view(torch.int16), vc0.view(torch.int16)), f"{label}: V pool"
        print(f"[no-alloc] {label}: bit-exact", flush=True)


def test_static_entry_point_in_a_graph_replays_like_the_workspace_path(deterministic_decode):
    """paged_decode_append_static captured once into a torch CUDA graph (its
    first call, which resolves the scratch, made eagerly beforehand), then
    replayed with new q / key / value written into the captured buffers
    between replays: every replay's output bits and pool bytes equal
    paged_decode_append's (with a workspace) on the same inputs."""
    lens = uniform_lengths(13, 1, 3000, seed=8)
    wl = decode_workload(len(lens), 32, 4, 200, lens, seed=9, device=DEV, pool_device_fill=True)
    kc_init, vc_init = wl.k_cache.clone(), wl.v_cache.clone()
    q, key, value = wl.q.clone(), wl.new_k.clone(), wl.new_v.clone()
    out = torch.empty_like(q)

    def step():
        paged_decode_append_static(q, key, value, wl.k_cache, wl.v_cache, wl.slot_mapping,
                                   wl.block_tables, wl.context_lens, wl.scale, out)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(21)
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=g).to(torch.bfloat16))
        key.copy_(torch.randn(key.shape, generator=g).to(torch.bfloat16))
        value.copy_(torch.randn(value.shape, generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        print(f"[no-alloc] graph replay {rep}: B={len(lens)}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        kc_ref, vc_ref = kc_init.clone(), vc_init.clone()
        ref = paged_decode_append(q, key, value, kc_ref, vc_ref, wl.slot_mapping,
                                  wl.block_tables, wl.context_lens, wl.scale)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), bits(ref)), f"replay {rep}: outputs differ"
        assert torch.equal(wl.k_cache.view(torch.int16), kc_ref.view(torch.int16)), \
            f"replay {rep}: K pool"
        assert torch.equal(wl.v_cache.view(torch.int16), vc_ref.view(torch.int16)), \
            f"replay {rep}: V pool"
    del graph


def test_static_scratch_rejects_launches_it_cannot_hold():
    need = nat.query("kvc_paged_decode_workspace_bytes", 256, 32, 4, 128, 256, 64)
    assert need > nat.STATIC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="static scratch"):
        nat.call("kvc_paged_decode_append_static", 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 4, 0, 0, 1,
                 256, 4, 128, 0, 64, 64, 0, 256, 32, 1.0, 0, 0, 0,
                 torch.cuda.current_stream().cuda_stream)
