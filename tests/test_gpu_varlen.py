"""Mixed decode + chunked-prefill parity — one varlen launch vs the oracle.

The oracle follows the reference's two sub-paths: paged decode for the decode
rows and the per-chunk prefix-masked attention of
nanovllm/layers/attention.py:179-213 for the prefill rows.
"""
import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, gathered_pool, p17_unit_inputs
from nanovllm_amd.kernels.kv_int8 import store_kvcache_int8
from nanovllm_amd.kernels.varlen import (gather_kv, varlen_attention, varlen_attention_append,
                                         varlen_decode_cus)
from nanovllm_amd.layers.attention import Attention, store_kvcache
from nanovllm_amd.utils.context import reset_context, set_context
from nanovllm_amd.workloads import build_block_tables, uniform_lengths
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"


_HINTS = {"on": False}


@pytest.fixture(params=["prefill-sk", "hinted", "split-64", "serial", "units"])
def partition(request, monkeypatch):
    """Every launch partition: prefill rows over bf16 keys as one stream-K
    prefill launch and a mixed call's decode and prefill rows as one launch
    over a static CU split with the default decode share (the defaults), the
    same with the split sized from the host's work hints (the decode rows'
    context lengths as host ints), the split with 64 decode CUs
    (KVC_MIXED_DECODE_CUS=64), the decode launch and then the prefill launch
    (KVC_MIXED_DECODE_CUS=0), and one workgroup per prefill unit
    (KVC_PREFILL_SK=0; a mixed call then runs its decode launch and its unit
    launch in turn)."""
    monkeypatch.setitem(_HINTS, "on", request.param == "hinted")
    monkeypatch.setenv("KVC_PREFILL_SK", "0" if request.param == "units" else "1")
    if request.param == "split-64":
        monkeypatch.setenv("KVC_MIXED_DECODE_CUS", "64")
    elif request.param == "serial":
        monkeypatch.setenv("KVC_MIXED_DECODE_CUS", "0")
    else:
        monkeypatch.delenv("KVC_MIXED_DECODE_CUS", raising=False)
    return request.param


def _mixed_case(H, KVH, dec_lens, chunks, seed, kv="bf16", page=256):
    """chunks: list of (prefix, chunk_len).  Returns inputs on the device."""
    g = torch.Generator().manual_seed(seed)
    pre_total = [p + c for p, c in chunks]
    all_lens = list(dec_lens) + pre_total
    blocks = sum(max(1, (n + page - 1) // page) for n in all_lens) + 3
    bt = build_block_tables(all_lens, blocks, page, g)
    shape = (blocks, page, KVH, 128)
    k_cache = torch.randn(shape, generator=g).to(torch.bfloat16)
    v_cache = torch.randn(shape, generator=g).to(torch.bfloat16)
    T = len(dec_lens) + sum(c for _, c in chunks)
    q = torch.randn(T, H, 128, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    return dict(q=q.to(DEV), k_cache=k_cache.to(DEV), v_cache=v_cache.to(DEV), bt=bt.to(DEV),
                dec_lens=torch.tensor(dec_lens, dtype=torch.int32).to(DEV), cu_q=cu_q, cu_k=cu_k,
                n_dec=len(dec_lens))


def _check_mixed(c, label, scale=128 ** -0.5):
    print(f"[varlen] {label}: rows={c['q'].shape[0]} dec={c['n_dec']} chunks={len(c['cu_q']) - 1}",
          flush=True)
    out = varlen_attention(
        c["q"], c["k_cache"], c["v_cache"], scale=scale, block_tables=c["bt"],
        num_decode_rows=c["n_dec"], decode_context_lens=c["dec_lens"] if c["n_dec"] else None,
        cu_seqlens_q=torch.tensor(c["cu_q"], dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(c["cu_k"], dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=c["cu_q"], cu_seqlens_k_list=c["cu_k"],
        decode_context_lens_list=c["dec_lens"].tolist() if _HINTS["on"] and c["n_dec"] else None)
    torch.cuda.synchronize()
    kc, bt = gathered_pool(c["k_cache"], c["bt"])
    vc, _ = gathered_pool(c["v_cache"], c["bt"])
    ref = ko.mixed_ref(bits(c["q"]), ko.bf16_to_f32(bits(kc)), ko.bf16_to_f32(bits(vc)), bt,
                       c["n_dec"], c["dec_lens"].cpu().numpy(), c["cu_q"], c["cu_k"], scale)
    return assert_attention_close(out, ref, label)


def test_prefill_chunks_with_prefixes_small(partition):
    c = _mixed_case(32, 4, [], [(0, 40), (300, 17), (1000, 256)], seed=1)
    _check_mixed(c, "prefill-only")


def test_mixed_decode_plus_prefill_small(partition):
    c = _mixed_case(32, 4, [1, 255, 256, 257, 3000], [(0, 33), (512, 64), (2048, 100)], seed=2)
    _check_mixed(c, "mixed-small")


@pytest.mark.parametrize("dec,chunks", [([1], [(0, 1)]), ([5000], [(4096, 1)]),
                                        ([3, 4096], [(0, 1), (0, 300)])])
def test_mixed_extremes_of_the_split(dec, chunks, partition):
    """One or two decode rows spread over the decode side's shares (most of
    them empty) and one-token chunks (a prefill item of one query column)."""
    c = _mixed_case(32, 4, dec, chunks, seed=len(dec) + 7 * len(chunks))
    _check_mixed(c, f"extremes dec={dec} chunks={chunks}")


@pytest.mark.parametrize("heads,kv_heads", [(16, 8), (32, 32), (12, 4), (64, 2)])
def test_mixed_gqa_groupings(heads, kv_heads, partition):
    c = _mixed_case(heads, kv_heads, [900, 17], [(0, 20), (700, 45)], seed=heads + kv_heads)
    _check_mixed(c, f"mixed-gqa-{heads}/{kv_heads}")


def test_stall_free_mixed_batch_full_shape(partition):
    # Four prefill chunks of 256 tokens with cached prefixes 0/512/2048/8192
    # plus 60 decode rows with contexts U[256, 4096], 32q/4kv, page 256.
    dec = uniform_lengths(60, 256, 4096, seed=3)
    c = _mixed_case(32, 4, dec, [(0, 256), (512, 256), (2048, 256), (8192, 256)], seed=4)
    _check_mixed(c, "stall-free-full")


def test_stall_free_mixed_batch_repeats_bit_for_bit(partition):
    # The same call three times on the same inputs gives the same bits: the
    # launches have no order-dependent arithmetic, so a difference means a
    # read raced with a load or an MFMA result.
    dec = uniform_lengths(60, 256, 4096, seed=3)
    c = _mixed_case(32, 4, dec, [(0, 256), (512, 256), (2048, 256), (8192, 256)], seed=4)
    outs = []
    for _ in range(3):
        outs.append(bits(varlen_attention(
            c["q"], c["k_cache"], c["v_cache"], scale=128 ** -0.5, block_tables=c["bt"],
            num_decode_rows=c["n_dec"], decode_context_lens=c["dec_lens"],
            cu_seqlens_q=torch.tensor(c["cu_q"], dtype=torch.int32, device=DEV),
            cu_seqlens_k=torch.tensor(c["cu_k"], dtype=torch.int32, device=DEV),
            cu_seqlens_q_list=c["cu_q"], cu_seqlens_k_list=c["cu_k"])))
    for i in (1, 2):
        diff = int((outs[i] != outs[0]).sum())
        print(f"[varlen] repeat {i} ({partition}): {diff} differing elements", flush=True)
        assert diff == 0


def test_many_chunks_empty_chunks_and_empty_context(partition):
    # 70 prefill chunks (more than one 64-chunk pass of the stream-K scan),
    # every ninth of them empty (prefix only), plus decode rows with an empty
    # context (NaN row) between non-empty ones.
    rng = np.random.default_rng(11)
    chunks = [(int(rng.integers(0, 300)), 0 if i % 9 == 4 else int(rng.integers(1, 24)))
              for i in range(70)]
    c = _mixed_case(32, 4, [40, 0, 700], chunks, seed=11)
    _check_mixed(c, "many-chunks")


@pytest.mark.parametrize("enc", ["int8_tokhead", "int8_chan"])
def test_int8_many_chunks_empty_chunks_and_empty_context(enc, partition):
    # The many-chunks case over int8 pools: 70 chunks (every ninth empty),
    # decode rows with an empty context, prefixes of any length; the prefill
    # rows' keys are gathered with empty chunks in between.
    rng = np.random.default_rng(13)
    chunks = [(int(rng.integers(0, 300)), 0 if i % 9 == 4 else int(rng.integers(1, 24)))
              for i in range(70)]
    H, KVH, D = 32, 4, 128
    dec_lens = [40, 0, 700]
    g = torch.Generator().manual_seed(13)
    all_lens = dec_lens + [p + c for p, c in chunks]
    blocks = sum(max(1, (n + 255) // 256) for n in all_lens) + 3
    bt = build_block_tables(all_lens, blocks, 256, g)
    kc = torch.randint(-127, 128, (blocks, 256, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, 256, KVH, D), generator=g, dtype=torch.int8)
    kw, side = {}, (None, None, None, None)
    if enc == "int8_tokhead":
        ks = torch.rand(blocks, 256, KVH, generator=g) * 0.03 + 0.005
        vs = torch.rand(blocks, 256, KVH, generator=g) * 0.03 + 0.005
        kw = dict(k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    else:
        ks = torch.rand(KVH, D, generator=g) * 0.03 + 0.005
        vs = torch.rand(KVH, D, generator=g) * 0.03 + 0.005
        oi = torch.tensor([[7, 64, 0, 0], [1, 2, 3, 127], [50, 0, 0, 0], [9, 33, 100, 0]],
                          dtype=torch.int32)
        hn = torch.tensor([2, 4, 0, 3], dtype=torch.int32)
        for h in range(KVH):
            ks[h, oi[h, :int(hn[h])].long()] = 0.0
            vs[h, oi[h, :int(hn[h])].long()] = 0.0
        sk_ = (torch.randn(blocks, 256, KVH, 4, generator=g) * 3).to(torch.bfloat16)
        sv_ = (torch.randn(blocks, 256, KVH, 4, generator=g) * 3).to(torch.bfloat16)
        kw = dict(k_scale=ks.to(DEV), v_scale=vs.to(DEV), side_k=sk_.to(DEV), side_v=sv_.to(DEV),
                  out_idx2d=oi.to(DEV), head_n_out=hn.to(DEV))
        side = (bits(sk_), bits(sv_), oi.numpy(), hn.numpy())
    T = len(dec_lens) + sum(c for _, c in chunks)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    print(f"[varlen] {enc} many chunks ({partition})", flush=True)
    out = varlen_attention(
        q.to(DEV), kc.to(DEV), vc.to(DEV), scale=D ** -0.5, block_tables=bt.to(DEV),
        num_decode_rows=len(dec_lens),
        decode_context_lens=torch.tensor(dec_lens, dtype=torch.int32, device=DEV),
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, **kw)
    torch.cuda.synchronize()
    if enc == "int8_tokhead":
        kf = ko.kv_float(kc.numpy(), enc, ks.numpy())
        vf = ko.kv_float(vc.numpy(), enc, vs.numpy())
        kp = ko.kv_float_prefill(kc.numpy(), enc, ks.numpy())
        vp = ko.kv_float_prefill(vc.numpy(), enc, vs.numpy())
    else:
        sk_b, sv_b, oi_n, hn_n = side
        kf = ko.kv_float(kc.numpy(), enc, ks.numpy(), sk_b, oi_n, hn_n)
        vf = ko.kv_float(vc.numpy(), enc, vs.numpy(), sv_b, oi_n, hn_n)
        kp = ko.kv_float_prefill(kc.numpy(), enc, ks.numpy(), sk_b, oi_n, hn_n)
        vp = ko.kv_float_prefill(vc.numpy(), enc, vs.numpy(), sv_b, oi_n, hn_n)
    ref = ko.mixed_ref(bits(q), kf, vf, bt.numpy(), len(dec_lens), np.asarray(dec_lens), cu_q,
                       cu_k, D ** -0.5, k_pre=kp, v_pre=vp)
    assert_attention_close(out, ref, f"{enc}-many-chunks")


@pytest.mark.parametrize("seed", range(6))
def test_int8_chan_random_mixes(seed):
    # Seeded random mixes over a per-channel pool: head groupings, pages,
    # side widths, outlier counts per head (distinct dims), decode rows and
    # chunks with and without prefixes; decode rows read the pool in fp32,
    # prefill rows through the bf16 gather (both against the oracle).
    rng = np.random.default_rng(100 + seed)
    H, KVH = [(32, 4), (16, 8), (64, 2), (32, 8), (12, 4), (32, 32)][seed]
    D = 128
    page = int(rng.choice([64, 128, 256]))
    nom = int(rng.choice([1, 2, 4, 8]))
    n_dec = int(rng.integers(0, 5))
    dec_lens = [int(rng.integers(1, 1500)) for _ in range(n_dec)]
    chunks = [(int(rng.integers(0, 900)), int(rng.integers(1, 200)))
              for _ in range(int(rng.integers(1, 6)))]
    g = torch.Generator().manual_seed(200 + seed)
    all_lens = dec_lens + [p + c for p, c in chunks]
    blocks = sum(max(1, (n + page - 1) // page) for n in all_lens) + 2
    bt = build_block_tables(all_lens, blocks, page, g)
    kc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    ks = torch.rand(KVH, D, generator=g) * 0.02 + 0.004
    vs = torch.rand(KVH, D, generator=g) * 0.02 + 0.004
    oi = torch.zeros(KVH, nom, dtype=torch.int32)
    hn = torch.zeros(KVH, dtype=torch.int32)
    for h in range(KVH):
        n_h = int(rng.integers(0, nom + 1))
        oi[h, :n_h] = torch.from_numpy(rng.choice(D, n_h, replace=False).astype(np.int32))
        hn[h] = n_h
        ks[h, oi[h, :n_h].long()] = 0.0
        vs[h, oi[h, :n_h].long()] = 0.0
    sk_ = (torch.randn(blocks, page, KVH, nom, generator=g) * 4).to(torch.bfloat16)
    sv_ = (torch.randn(blocks, page, KVH, nom, generator=g) * 4).to(torch.bfloat16)
    T = n_dec + sum(c for _, c in chunks)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    print(f"[varlen] int8 chan random mix {seed}: H={H} KVH={KVH} page={page} slots={nom} "
          f"dec={dec_lens} chunks={chunks}", flush=True)
    out = varlen_attention(
        q.to(DEV), kc.to(DEV), vc.to(DEV), scale=D ** -0.5, block_tables=bt.to(DEV),
        num_decode_rows=n_dec,
        decode_context_lens=torch.tensor(dec_lens, dtype=torch.int32, device=DEV) if n_dec else None,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, k_scale=ks.to(DEV), v_scale=vs.to(DEV),
        side_k=sk_.to(DEV), side_v=sv_.to(DEV), out_idx2d=oi.to(DEV), head_n_out=hn.to(DEV))
    torch.cuda.synchronize()
    args = (bits(sk_), oi.numpy(), hn.numpy())
    kf = ko.kv_float(kc.numpy(), "int8_chan", ks.numpy(), *args)
    vf = ko.kv_float(vc.numpy(), "int8_chan", vs.numpy(), bits(sv_), oi.numpy(), hn.numpy())
    kp = ko.kv_float_prefill(kc.numpy(), "int8_chan", ks.numpy(), *args)
    vp = ko.kv_float_prefill(vc.numpy(), "int8_chan", vs.numpy(), bits(sv_), oi.numpy(),
                             hn.numpy())
    ref = ko.mixed_ref(bits(q), kf, vf, bt.numpy(), n_dec, np.asarray(dec_lens), cu_q, cu_k,
                       D ** -0.5, k_pre=kp, v_pre=vp)
    assert_attention_close(out, ref, f"int8-chan-random-{seed}")


@pytest.mark.parametrize("seed", range(4))
def test_int8_tokhead_random_mixes(seed):
    # The same kind of seeded random mixes over a per-token-head int8 pool.
    rng = np.random.default_rng(300 + seed)
    H, KVH = [(32, 4), (16, 2), (64, 8), (8, 8)][seed]
    D = 128
    page = int(rng.choice([32, 128, 256]))
    n_dec = int(rng.integers(0, 5))
    dec_lens = [int(rng.integers(1, 1500)) for _ in range(n_dec)]
    chunks = [(int(rng.integers(0, 900)), int(rng.integers(1, 200)))
              for _ in range(int(rng.integers(1, 6)))]
    g = torch.Generator().manual_seed(400 + seed)
    all_lens = dec_lens + [p + c for p, c in chunks]
    blocks = sum(max(1, (n + page - 1) // page) for n in all_lens) + 2
    bt = build_block_tables(all_lens, blocks, page, g)
    kc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, page, KVH, D), generator=g, dtype=torch.int8)
    ks = torch.rand(blocks, page, KVH, generator=g) * 0.03 + 0.005
    vs = torch.rand(blocks, page, KVH, generator=g) * 0.03 + 0.005
    T = n_dec + sum(c for _, c in chunks)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    print(f"[varlen] int8 tokhead random mix {seed}: H={H} KVH={KVH} page={page} "
          f"dec={dec_lens} chunks={chunks}", flush=True)
    out = varlen_attention(
        q.to(DEV), kc.to(DEV), vc.to(DEV), scale=D ** -0.5, block_tables=bt.to(DEV),
        num_decode_rows=n_dec,
        decode_context_lens=torch.tensor(dec_lens, dtype=torch.int32, device=DEV) if n_dec else None,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.numpy(), "int8_tokhead", ks.numpy())
    vf = ko.kv_float(vc.numpy(), "int8_tokhead", vs.numpy())
    kp = ko.kv_float_prefill(kc.numpy(), "int8_tokhead", ks.numpy())
    vp = ko.kv_float_prefill(vc.numpy(), "int8_tokhead", vs.numpy())
    ref = ko.mixed_ref(bits(q), kf, vf, bt.numpy(), n_dec, np.asarray(dec_lens), cu_q, cu_k,
                       D ** -0.5, k_pre=kp, v_pre=vp)
    assert_attention_close(out, ref, f"int8-tokhead-random-{seed}")


def test_long_chunk_many_query_tiles(partition):
    # 64 q / 2 kv heads: 16-head slices and 16-token query tiles, so a
    # 1100-token chunk spans 69 query tiles (the item search crosses a
    # 64-tile pass).
    c = _mixed_case(64, 2, [300], [(100, 1100), (0, 5)], seed=12)
    _check_mixed(c, "long-chunk")


def test_fresh_kv_prefill_without_block_tables(partition):
    # No prefix cache: keys are the step's own k/v rows, causal inside each
    # sequence (attention.py:195-199).
    g = torch.Generator().manual_seed(5)
    H, KVH, lens = 32, 4, [1, 77, 300]
    T = sum(lens)
    q = torch.randn(T, H, 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(T, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(T, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    print("[varlen] fresh-kv prefill", flush=True)
    out = varlen_attention(q, None, None, scale=128 ** -0.5, block_tables=None, k=k, v=v,
                           cu_seqlens_q_list=cu, cu_seqlens_k_list=cu)
    torch.cuda.synchronize()
    ref = ko.prefill_ref(bits(q), None, None, None, cu, cu, 128 ** -0.5,
                         fresh_k=ko.bf16_to_f32(bits(k)), fresh_v=ko.bf16_to_f32(bits(v)))
    assert_attention_close(out, ref, "fresh-kv")


@pytest.mark.parametrize("rows", ["mixed", "prefill-only"])
def test_mixed_int8_tokhead_pool(rows, partition):
    # Decode rows and prefix-cached prefill chunks over a per-token-head int8
    # pool (codes + fp32 scale per slot and kv head): the decode rows read the
    # pool as codes x scale in fp32 (paged_attention.py:138-145), the prefill
    # rows through the bf16 dequantisation the reference's prefill gathers
    # with (attention.py:33-51).  Prefill rows alone take the gathered form
    # (gather_kv, then the bf16 stream-K prefill) unless KVC_PREFILL_SK=0.
    H, KVH, D = 32, 4, 128
    dec_lens = [900, 1, 2500] if rows == "mixed" else []
    chunks = [(0, 40), (700, 90), (3000, 33)]
    g = torch.Generator().manual_seed(21)
    all_lens = dec_lens + [p + c for p, c in chunks]
    blocks = sum(max(1, (n + 255) // 256) for n in all_lens) + 2
    bt = build_block_tables(all_lens, blocks, 256, g)
    kc = torch.randint(-127, 128, (blocks, 256, KVH, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, 256, KVH, D), generator=g, dtype=torch.int8)
    ks = torch.rand(blocks, 256, KVH, generator=g) * 0.03 + 0.005
    vs = torch.rand(blocks, 256, KVH, generator=g) * 0.03 + 0.005
    T = len(dec_lens) + sum(c for _, c in chunks)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    print(f"[varlen] int8 tokhead {rows}: rows={T} ({partition})", flush=True)
    out = varlen_attention(
        q.to(DEV), kc.to(DEV), vc.to(DEV), scale=D ** -0.5, block_tables=bt.to(DEV),
        num_decode_rows=len(dec_lens),
        decode_context_lens=torch.tensor(dec_lens, dtype=torch.int32, device=DEV)
        if dec_lens else None,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.numpy(), "int8_tokhead", ks.numpy())
    vf = ko.kv_float(vc.numpy(), "int8_tokhead", vs.numpy())
    kp = ko.kv_float_prefill(kc.numpy(), "int8_tokhead", ks.numpy())
    vp = ko.kv_float_prefill(vc.numpy(), "int8_tokhead", vs.numpy())
    ref = ko.mixed_ref(bits(q), kf, vf, bt.numpy(), len(dec_lens), np.asarray(dec_lens), cu_q,
                       cu_k, D ** -0.5, k_pre=kp, v_pre=vp)
    assert_attention_close(out, ref, "mixed-int8-tokhead")


@pytest.mark.parametrize("rows", ["mixed", "prefill-only"])
def test_mixed_int8_channel_pool_with_side(rows, partition):
    # The engine's per-channel int8 pool with the bf16 outlier side pool
    # (tests/p17_kv_int8.py:64-136 geometry, 16 q / 8 kv heads): one decode
    # row over 512 stored tokens plus a 100-token chunk after a 200-token
    # prefix; the outlier dims come from the side pool exactly.  Head 2's
    # value outliers (x60) hold the prefill rows to the fp32 reference only
    # with the residue product on the bf16 P operand.
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    KVH, D, H = key.shape[1], key.shape[2], 16
    nout = out_idx2d.shape[1]
    blocks = 4
    bt = torch.tensor([[2, 0], [1, 3]], dtype=torch.int32)
    kc = torch.zeros(blocks, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(blocks, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    oi, hn = out_idx2d.to(DEV), head_n_out.to(DEV)
    slots_a = [int(bt[0, t // 256]) * 256 + t % 256 for t in range(512)]
    store_kvcache_int8(key.to(DEV), value.to(DEV), kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv, oi,
                       hn, torch.tensor(slots_a, dtype=torch.int32, device=DEV))
    slots_b = [int(bt[1, t // 256]) * 256 + t % 256 for t in range(300)]
    store_kvcache_int8(key[:300].flip(0).contiguous().to(DEV), value[:300].to(DEV), kc, vc,
                       s_k.to(DEV), s_v.to(DEV), sk, sv, oi, hn,
                       torch.tensor(slots_b, dtype=torch.int32, device=DEV))
    q = torch.randn(101, H, D, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    cu_q, cu_k = [0, 100], [0, 300]
    nd = 1 if rows == "mixed" else 0
    q, bt = q[1 - nd:], bt[1 - nd:]
    print(f"[varlen] int8 channel {rows} + side pool ({partition})", flush=True)
    out = varlen_attention(
        q.to(DEV), kc, vc, scale=D ** -0.5, block_tables=bt.to(DEV), num_decode_rows=nd,
        decode_context_lens=torch.tensor([512], dtype=torch.int32, device=DEV) if nd else None,
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, k_scale=ds_k.to(DEV),
        v_scale=ds_v.to(DEV), side_k=sk, side_v=sv, out_idx2d=oi, head_n_out=hn)
    torch.cuda.synchronize()
    kf = ko.kv_float(kc.cpu().numpy(), "int8_chan", ds_k.numpy(), bits(sk), out_idx2d.numpy(),
                     head_n_out.numpy())
    vf = ko.kv_float(vc.cpu().numpy(), "int8_chan", ds_v.numpy(), bits(sv), out_idx2d.numpy(),
                     head_n_out.numpy())
    kp = ko.kv_float_prefill(kc.cpu().numpy(), "int8_chan", ds_k.numpy(), bits(sk),
                             out_idx2d.numpy(), head_n_out.numpy())
    vp = ko.kv_float_prefill(vc.cpu().numpy(), "int8_chan", ds_v.numpy(), bits(sv),
                             out_idx2d.numpy(), head_n_out.numpy())
    ref = ko.mixed_ref(bits(q), kf, vf, bt.numpy(), nd, np.asarray([512][:nd]), cu_q, cu_k,
                       D ** -0.5, k_pre=kp, v_pre=vp)
    assert_attention_close(out, ref, "mixed-int8-chan-side")


def test_fresh_rows_gathered_from_a_channel_pool(partition):
    # The two calls an int8 prefill makes, by hand: gather_kv of the p17
    # per-channel pool, then a no-prefix-cache call over the gathered rows
    # naming the pool's outlier dims (the residue product on both prefill
    # launch forms).  Same result as the paged call against the oracle.
    key, value, s_k, s_v, ds_k, ds_v, out_idx2d, head_n_out = p17_unit_inputs()
    KVH, D, H = key.shape[1], key.shape[2], 16
    nout = out_idx2d.shape[1]
    kc = torch.zeros(2, 256, KVH, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(2, 256, KVH, nout, dtype=torch.bfloat16, device=DEV)
    sv = torch.zeros_like(sk)
    oi, hn = out_idx2d.to(DEV), head_n_out.to(DEV)
    slots = torch.tensor([256 + t if t < 256 else t - 256 for t in range(512)], dtype=torch.int32,
                         device=DEV)
    store_kvcache_int8(key.to(DEV), value.to(DEV), kc, vc, s_k.to(DEV), s_v.to(DEV), sk, sv, oi,
                       hn, slots)
    bt = torch.tensor([[1, 0], [1, 0]], dtype=torch.int32)
    cu_q, cu_k = [0, 60, 160], [0, 300, 812]   # chunk 0: 60 queries after 240 keys; chunk 1: 100 after 412
    cuk = torch.tensor(cu_k, dtype=torch.int32, device=DEV)
    kg, vg = gather_kv(kc, vc, bt.to(DEV), cuk, cu_k, k_scale=ds_k.to(DEV), v_scale=ds_v.to(DEV),
                       side_k=sk, side_v=sv, out_idx2d=oi, head_n_out=hn)
    q = torch.randn(160, H, D, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    print(f"[varlen] fresh rows from a channel pool ({partition})", flush=True)
    out = varlen_attention(q.to(DEV), None, None, scale=D ** -0.5, block_tables=None, k=kg, v=vg,
                           cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
                           cu_seqlens_k=cuk, cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k,
                           out_idx2d=oi, head_n_out=hn)
    torch.cuda.synchronize()
    ref = ko.prefill_ref(bits(q), None, None, None, cu_q, cu_k, D ** -0.5,
                         fresh_k=ko.bf16_to_f32(bits(kg.cpu())),
                         fresh_v=ko.bf16_to_f32(bits(vg.cpu())))
    assert_attention_close(out, ref, "fresh-from-channel-pool")


def test_attention_forward_mixed_matches_decode_and_prefill_paths():
    # Attention.forward on a mixed Context: store, then one varlen launch; the
    # result must match the oracle for both row groups.
    H, KVH, D = 32, 4, 128
    g = torch.Generator().manual_seed(6)
    dec_lens = [129, 512]
    chunks = [(0, 31), (256, 20)]
    all_lens = dec_lens + [p + c for p, c in chunks]
    blocks = 12
    bt = build_block_tables(all_lens, blocks, 256, g)
    k_cache = torch.randn(blocks, 256, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    v_cache = torch.randn(blocks, 256, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    # rows: each decode row's new token is its last position; prefill rows are
    # the chunk's tokens (positions prefix .. prefix + c - 1).
    slots = []
    for i, n in enumerate(dec_lens):
        slots.append(int(bt[i, (n - 1) // 256]) * 256 + (n - 1) % 256)
    for j, (p, c) in enumerate(chunks):
        row = len(dec_lens) + j
        for t in range(p, p + c):
            slots.append(int(bt[row, t // 256]) * 256 + t % 256)
    T = len(slots)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(T, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(T, KVH, D, generator=g).to(torch.bfloat16).to(DEV)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    attn = Attention(H, D, D ** -0.5, KVH)
    attn.k_cache, attn.v_cache = k_cache, v_cache
    set_context(True, torch.tensor(cu_q, dtype=torch.int32, device=DEV),
                torch.tensor(cu_k, dtype=torch.int32, device=DEV), max(c for _, c in chunks),
                max(cu_k[i + 1] - cu_k[i] for i in range(len(chunks))),
                torch.tensor(slots, dtype=torch.int32, device=DEV), None, bt.to(DEV),
                cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, is_mixed=True,
                num_decode_rows=len(dec_lens),
                decode_context_lens=torch.tensor(dec_lens, dtype=torch.int32, device=DEV),
                decode_max_context_len=max(dec_lens))
    try:
        print("[varlen] Attention.forward mixed", flush=True)
        out = attn(q, k, v)
        torch.cuda.synchronize()
    finally:
        reset_context()
    kc, btn = gathered_pool(k_cache, bt.to(DEV))
    vc, _ = gathered_pool(v_cache, bt.to(DEV))
    ref = ko.mixed_ref(bits(q), ko.bf16_to_f32(bits(kc)), ko.bf16_to_f32(bits(vc)), btn,
                       len(dec_lens), np.asarray(dec_lens), cu_q, cu_k, D ** -0.5)
    assert_attention_close(out, ref, "forward-mixed")


def _step_slots(c, page=256):
    """The engine's slots for a mixed step: decode row i appends at its last
    position ctx_i - 1, prefill chunk j's tokens sit at positions
    prefix_j .. prefix_j + sq_j - 1 of table row n_dec + j."""
    bt = c["bt"].cpu()
    slots = []
    for i, n in enumerate(c["dec_lens"].tolist()):
        slots.append(int(bt[i, (n - 1) // page]) * page + (n - 1) % page)
    for j in range(len(c["cu_q"]) - 1):
        sq = c["cu_q"][j + 1] - c["cu_q"][j]
        sk = c["cu_k"][j + 1] - c["cu_k"][j]
        row = c["n_dec"] + j
        for t in range(sk - sq, sk):
            slots.append(int(bt[row, t // page]) * page + t % page)
    return slots


@pytest.mark.parametrize("case", ["small", "mix16", "decode-only", "prefill-only",
                                  "int64-slots", "tp2-shard"])
@pytest.mark.parametrize("hinted", [False, True])
def test_varlen_append_equals_store_then_varlen(case, hinted):
    """varlen_attention_append (the prefill rows stored ahead, the decode rows
    appended inside the decode launch or the split launch's decode side)
    against store_kvcache of every row then varlen_attention with the same
    hints: the same output bits and the same pool bytes."""
    H, KVH = (16, 2) if case == "tp2-shard" else (32, 4)
    if case == "mix16":
        dec = uniform_lengths(16, 256, 4096, seed=3)
        chunks = [(0, 512), (512, 512), (2048, 512), (8192, 512)]
    elif case == "decode-only":
        dec, chunks = [1, 31, 32, 33, 700, 4096], []
    elif case == "prefill-only":
        dec, chunks = [], [(0, 40), (300, 17), (1000, 256)]
    else:
        dec, chunks = [1, 255, 256, 257, 3000], [(0, 33), (512, 64), (2048, 100)]
    c = _mixed_case(H, KVH, dec, chunks, seed=17 + len(case))
    slots = torch.tensor(_step_slots(c), dtype=torch.int64 if case == "int64-slots"
                         else torch.int32, device=DEV)
    T = c["q"].shape[0]
    g = torch.Generator().manual_seed(99)
    qkv = torch.randn(T, H + 2 * KVH, 128, generator=g).to(torch.bfloat16).to(DEV)
    q, key, value = qkv[:, :H].contiguous(), qkv[:, H:H + KVH], qkv[:, H + KVH:]
    nd = c["n_dec"]
    kw = dict(scale=128 ** -0.5, block_tables=c["bt"], num_decode_rows=nd,
              decode_context_lens=c["dec_lens"] if nd else None,
              cu_seqlens_q_list=c["cu_q"], cu_seqlens_k_list=c["cu_k"],
              decode_context_lens_list=c["dec_lens"].tolist() if hinted and nd else None)
    kc0, vc0 = c["k_cache"].clone(), c["v_cache"].clone()
    print(f"[varlen-append] {case} hinted={hinted}: T={T} dec={nd}", flush=True)
    store_kvcache(key, value, kc0, vc0, slots)
    ref = varlen_attention(q, kc0, vc0, **kw)
    kc1, vc1 = c["k_cache"].clone(), c["v_cache"].clone()
    out = varlen_attention_append(q, key, value, kc1, vc1, slots, **kw)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(ref)), f"{case}: outputs differ"
    assert torch.equal(kc1.view(torch.int16), kc0.view(torch.int16)), f"{case}: K pool"
    assert torch.equal(vc1.view(torch.int16), vc0.view(torch.int16)), f"{case}: V pool"


def test_hinted_split_follows_the_mix(monkeypatch):
    """The decode side's CUs from the host hints on the device's CU count:
    about 3/8 for 60 decode rows and four 256-token chunks (the measured
    balance), few for 16 rows and four 512-token chunks, most for 128 rows
    and two 128-token chunks."""
    monkeypatch.delenv("KVC_MIXED_DECODE_CUS", raising=False)
    cus = torch.cuda.get_device_properties(0).multi_processor_count

    def split(n, chunks):
        dec = uniform_lengths(n, 256, 4096, seed=3)
        cq, ck = [0], [0]
        for p, c in chunks:
            cq.append(cq[-1] + c)
            ck.append(ck[-1] + p + c)
        return varlen_decode_cus(n, cq[-1], 32, 4, dec, cq, ck)

    a = split(60, [(0, 256), (512, 256), (2048, 256), (8192, 256)])
    b = split(16, [(0, 512), (512, 512), (2048, 512), (8192, 512)])
    d = split(128, [(0, 128), (4096, 128)])
    assert 8 <= b < a < d <= cus - 8, (a, b, d)
    assert abs(a - cus * 3 // 8) <= 16


@pytest.mark.parametrize("page", [32, 64, 128])
def test_pages_smaller_than_256(page, partition):
    # The reference insists on 256-token pages; the kernels take any multiple
    # of 32 (a 32-key tile never straddles a page).
    c = _mixed_case(32, 4, [1, page - 1, page, page + 1, 700],
                    [(0, 40), (page + 3, 33), (5 * page, 64)], seed=page, page=page)
    _check_mixed(c, f"page-{page}")


@pytest.mark.parametrize("case", ["decode-side-8", "prefill-side-8"])
def test_hinted_split_at_its_extremes(case, monkeypatch):
    """A mixed call whose hints give one side the minimum of 8 CUs: one short
    decode row beside two long chunks, and 200 decode rows beside one
    16-token chunk; both against the oracle."""
    monkeypatch.delenv("KVC_MIXED_DECODE_CUS", raising=False)
    monkeypatch.setitem(_HINTS, "on", True)
    if case == "decode-side-8":
        dec, chunks = [100], [(0, 1024), (4096, 1024)]
    else:
        dec, chunks = uniform_lengths(200, 256, 4096, seed=12), [(100, 16)]
    cq, ck = [0], [0]
    for p, c in chunks:
        cq.append(cq[-1] + c)
        ck.append(ck[-1] + p + c)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = varlen_decode_cus(len(dec), cq[-1], 32, 4, dec, cq, ck)
    assert n == (8 if case == "decode-side-8" else cus - 8), n
    c = _mixed_case(32, 4, dec, chunks, seed=31 + len(dec))
    _check_mixed(c, f"hinted-{case}")
