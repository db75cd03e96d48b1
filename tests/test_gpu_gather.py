"""Gather of the prefill chunks' keys (kvc_gather_kv) against the oracle.

The reference reads a prefill chunk's keys with _gather_kv
(nanovllm/layers/attention.py:33-51): the chunk's blocks in table order, cut
at sk, and for an int8 pool dequantised to bf16 with the side pool's values
at the outlier dims.  The gather must be bit-exact.
"""
import numpy as np
import pytest
import torch

from helpers import bits, p17_unit_inputs
from nanovllm_amd.kernels.kv_int8 import store_kvcache_int8
from nanovllm_amd.kernels.varlen import gather_kv
from nanovllm_amd.workloads import build_block_tables
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _expected(pool_bits, bt, cu_k, row0):
    """Rows of every chunk, chunk i through table row row0 + i (bf16 bits)."""
    parts = []
    for i in range(len(cu_k) - 1):
        sk = cu_k[i + 1] - cu_k[i]
        parts.append(ko._gather_rows(pool_bits, bt[row0 + i], sk))
    return np.concatenate(parts, axis=0)


@pytest.mark.parametrize("kv,nom", [("bf16", 8), ("int8_tokhead", 8), ("int8_chan", 8),
                                    ("int8_chan", 3), ("int8_chan", 1)])
@pytest.mark.parametrize("page", [32, 256])
def test_gather_kv_is_the_reference_gather(kv, nom, page):
    # Ragged chunks (an empty one, one key, a page edge, several pages), a
    # table row offset (rows of decode sequences ahead of the chunks).
    KVH, D = 4, 128
    g = torch.Generator().manual_seed(31)
    sks = [0, 1, page, 300, 2 * page + 17]
    lens = [700] + sks
    blocks = sum(max(1, (n + page - 1) // page) for n in lens) + 3
    bt = build_block_tables(lens, blocks, page, g)
    cu_k = [0]
    for n in sks:
        cu_k.append(cu_k[-1] + n)
    kw = {}
    if kv == "bf16":
        kc = torch.randn(blocks, page, KVH, D, generator=g).to(torch.bfloat16)
        vc = torch.randn(blocks, page, KVH, D, generator=g).to(torch.bfloat16)
        ek, ev = bits(kc), bits(vc)
    else:
        kc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
        vc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
        if kv == "int8_tokhead":
            ks = torch.rand(blocks, page, KVH, generator=g) * 0.03 + 0.005
            vs = torch.rand(blocks, page, KVH, generator=g) * 0.03 + 0.005
            ek = ko.dequant_tokhead(kc.numpy(), ks.numpy())
            ev = ko.dequant_tokhead(vc.numpy(), vs.numpy())
            kw = dict(k_scale=ks.to(DEV), v_scale=vs.to(DEV))
        else:
            ks = torch.rand(KVH, D, generator=g) * 0.03 + 0.005
            vs = torch.rand(KVH, D, generator=g) * 0.03 + 0.005
            # any side width up to 8 (the attention takes powers of two)
            oi = torch.zeros(KVH, nom, dtype=torch.int32)
            full = {0: [5, 77, 127], 1: [9, 9], 3: list(range(0, 128, 16))}  # 9, 9: the later slot wins
            hn = torch.zeros(KVH, dtype=torch.int32)
            for h, dims in full.items():
                n_h = min(len(dims), nom)
                oi[h, :n_h] = torch.tensor(dims[:n_h])
                hn[h] = n_h
            for h in range(KVH):
                ks[h, oi[h, :int(hn[h])].long()] = 0.0
                vs[h, oi[h, :int(hn[h])].long()] = 0.0
            sk_ = (torch.randn(blocks, page, KVH, nom, generator=g) * 40).to(torch.bfloat16)
            sv_ = (torch.randn(blocks, page, KVH, nom, generator=g) * 40).to(torch.bfloat16)
            flat = lambda t: t.reshape(-1, KVH, t.shape[-1])
            ek = ko.dequant_chan(flat(kc).numpy(), ks.numpy(), flat(bits(sk_)), oi.numpy(),
                                 hn.numpy()).reshape(blocks, page, KVH, D)
            ev = ko.dequant_chan(flat(vc).numpy(), vs.numpy(), flat(bits(sv_)), oi.numpy(),
                                 hn.numpy()).reshape(blocks, page, KVH, D)
            kw = dict(k_scale=ks.to(DEV), v_scale=vs.to(DEV), side_k=sk_.to(DEV),
                      side_v=sv_.to(DEV), out_idx2d=oi.to(DEV), head_n_out=hn.to(DEV))
    print(f"[gather] {kv} side slots={nom} page={page} keys={cu_k[-1]}", flush=True)
    gk, gv = gather_kv(kc.to(DEV), vc.to(DEV), bt.to(DEV),
                       torch.tensor(cu_k, dtype=torch.int32, device=DEV), cu_k,
                       block_table_row0=1, **kw)
    torch.cuda.synchronize()
    assert gk.shape == (cu_k[-1], KVH, D)
    np.testing.assert_array_equal(bits(gk.cpu()), _expected(ek, bt.numpy(), cu_k, 1))
    np.testing.assert_array_equal(bits(gv.cpu()), _expected(ev, bt.numpy(), cu_k, 1))


def test_gather_kv_of_the_stored_p17_pool():
    # The engine's per-channel pool as store_kvcache_int8 writes it
    # (tests/p17_kv_int8.py:64-136 inputs): gathered rows equal dequant_chan
    # of the stored codes and side rows.
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    KVH, D = key.shape[1], key.shape[2]
    nout = out_idx2d.shape[1]
    kc = torch.zeros(2, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(2, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    oi, hn = out_idx2d.to(DEV), head_n_out.to(DEV)
    slots = torch.arange(512, dtype=torch.int32, device=DEV)
    store_kvcache_int8(key.to(DEV), value.to(DEV), kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv, oi,
                       hn, slots)
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    cu_k = [0, 400]
    gk, gv = gather_kv(kc, vc, bt.to(DEV), torch.tensor(cu_k, dtype=torch.int32, device=DEV),
                       cu_k, k_scale=ds_k.to(DEV), v_scale=ds_v.to(DEV), side_k=sk, side_v=sv,
                       out_idx2d=oi, head_n_out=hn)
    torch.cuda.synchronize()
    for got, pool, side, ds in ((gk, kc, sk, ds_k), (gv, vc, sv, ds_v)):
        rows = torch.cat([pool[1], pool[0]])[:400].cpu().numpy()
        srows = bits(torch.cat([side[1], side[0]])[:400].cpu())
        exp = ko.dequant_chan(rows, ds.numpy(), srows, out_idx2d.numpy(), head_n_out.numpy())
        np.testing.assert_array_equal(bits(got.cpu()), exp)
