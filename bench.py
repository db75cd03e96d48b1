"""Paged-KV decode benchmark on one MI355X.

Default workload (the headline): Qwen3-30B-A3B full attention shape — 32 q
heads, 4 kv heads, head_dim 128, bf16, page 256 — batch 64 at context 4096
over an 8192-block pool with non-contiguous block tables.  One step = append
one token per sequence through slot_mapping, then one paged decode launch.

Prints ONE JSON line: decode tokens/s (value), the decode kernel's achieved
KV-read bandwidth against the 8 TB/s HBM peak (roofline), and the engine's
torch CPU decode path (gather + GQA expand + masked SDPA) timed on a bounded
sample of the same workload on this host (cpu_baseline).

    python bench.py [--gpus 1] [--steps 50] [--warmup 10]
    python bench.py --workload mixed|mixed16|int8|prefill-int8|decode-dist|append|swap|copy|rope|
                     decode-graph|offload-overlap|pd-wire      (extra lines)
"""
from __future__ import annotations

import argparse
import math
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "s4000-moe-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode attn tokens/s + achieved KV-read HBM GB/s (% of peak), bs64×4k ctx"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode-dist", "decode-tp2", "decode-cold", "cfg1",
                             "p15-grid", "int8", "mixed", "mixed16", "append", "swap", "copy",
                             "rope", "decode-graph", "offload-overlap", "pd-wire",
                             "block-manager", "int8-chan", "prefill-int8", "prefill-scale"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--stamps", action="store_true",
                    help="decode workloads: also report the per-workgroup end times of the "
                         "decode kernel (KVC_DECODE_STAMPS), measured after the timed region")
    ap.add_argument("--mixed-call-only", action="store_true",
                    help="mixed workloads: run only the hinted call in every timed slot (for "
                         "kernel traces of that call; the other fields then repeat it)")
    ap.add_argument("--side-slots", type=int, default=8, choices=[1, 2, 4, 8],
                    help="int8-chan: side-pool slots per kv head (the engine's KV_N_OUT_MAX "
                         "is 8), half of them holding outlier dims")
    ap.add_argument("--cpu-sample", type=int, default=0,
                    help="sequences of the workload the CPU baseline runs (default: 64 of "
                         "the bf16 decode batch, 2 of the 32k-context int8 batch)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------
class EventTimer:
    """Pairs of HIP events recorded on the stream libkvc launches on (torch's
    current stream), created with hipEventDisableSystemFence so that a record
    does not add a system-scope cache flush between the kernels it brackets
    (torch.cuda.Event records one).  Durations are read after the timed
    region ends.  The events come from the HIP runtime already loaded in the
    process (the one torch and libkvc share, soname libamdhip64.so.7)."""

    _DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, torch):
        import ctypes
        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                                     ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float),
                                                 ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.stream = torch.cuda.current_stream().cuda_stream
        self.pairs = []

    def _record(self):
        ev = self.ct.c_void_p()
        rc = self.hip.hipEventCreateWithFlags(self.ct.byref(ev), self._DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        rc = self.hip.hipEventRecord(ev, self.stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")
        return ev

    def start(self):
        return self._record()

    def stop(self, s):
        self.pairs.append((s, self._record()))

    def mean_ms(self):
        out = []
        for s, e in self.pairs:
            self.hip.hipEventSynchronize(e)
            ms = self.ct.c_float()
            rc = self.hip.hipEventElapsedTime(self.ct.byref(ms), s, e)
            if rc != 0:
                raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
            out.append(ms.value)
            self.hip.hipEventDestroy(s)
            self.hip.hipEventDestroy(e)
        self.pairs = []
        return statistics.fmean(out)


def cpu_threads():
    return len(os.sched_getaffinity(0))


def profiled_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel for `workload`, from the
    committed rocprofv3 counter summaries: a line
    `bench-traffic: <workload> <bytes>` in profiles/*.md (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by what the counter reads for a copy
    kernel of known size).  None when no summary covers the workload."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(REPO, "profiles", "*.md"))):
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*bench-traffic:\s*(\S+)\s+(\d+)", line)
                if m and m.group(1) == workload:
                    return int(m.group(2))
    return None


# ---------------------------------------------------------------------------
# CPU baseline: the engine's torch decode path on the host
# ---------------------------------------------------------------------------
def _median_cv(times):
    med = statistics.median(times)
    return med, statistics.pstdev(times) / statistics.fmean(times)


def _peak_rss_gb():
    import resource
    return resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1e6   # KiB -> GB


def _timed_reps(fn, reps):
    fn()   # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return _median_cv(times)


def _host_blocks(torch, cache, bt, used):
    """The blocks `used` of a device pool on the host, renumbered 0.."""
    return cache.index_select(0, used.to(cache.device)).cpu()


def cpu_decode_baseline(torch, wl, sample: int, tok_bytes: int, reps: int = 5,
                        int8: bool = False):
    """The engine's torch CPU decode step on a bounded sample of the
    workload's sequences: bf16, append (index_put, attention.py:9-30) + the
    gather + expand + masked SDPA decode (attention.py:239-279); int8
    per-token-head, the p14 quantise-on-append (p14_int8_kv_probe.py:37-41)
    + gather + dequantise (:45-46) + the same SDPA.  Reported as tokens/s and
    as effective GB/s over the sample's algorithmic KV bytes."""
    from oracle import kv_oracle as ko
    threads = cpu_threads()
    torch.set_num_threads(threads)
    b = min(sample, wl.batch)
    bt = wl.block_tables[:b].cpu()
    used = torch.unique(bt[bt >= 0])
    remap = torch.full((wl.k_cache.size(0),), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    kc = _host_blocks(torch, wl.k_cache, bt, used)
    vc = _host_blocks(torch, wl.v_cache, bt, used)
    bt_small = torch.where(bt >= 0, remap[bt.clamp(min=0).long()], torch.full_like(bt, -1,
                           dtype=torch.int64)).to(torch.int32)
    q = wl.q[:b].cpu()
    lens = wl.context_lens[:b].cpu()
    max_len = int(lens.max())
    page = kc.size(1)
    last = lens.long() - 1
    slots = (bt_small.long().gather(1, (last // page).unsqueeze(1)).squeeze(1) * page
             + last % page)
    nk, nv = wl.new_k[:b].cpu(), wl.new_v[:b].cpu()
    if int8:
        ks = _host_blocks(torch, wl.k_scale, bt, used)
        vs = _host_blocks(torch, wl.v_scale, bt, used)
        row = kc.size(2) * kc.size(3)

        def step():
            for x, codes, sc in ((nk, kc, ks), (nv, vc, vs)):
                c, s_ = ko.quant_tokhead_torch(x)
                codes.view(-1, row)[slots] = c.reshape(b, row)
                sc.view(-1, sc.size(-1))[slots] = s_.squeeze(-1)
            ko.gather_sdpa_decode_int8_tokhead(q, kc, vc, ks, vs, bt_small, lens, wl.scale,
                                               max_len)
        what = ("p14 int8 quantise-on-append + gather + dequantise + expand + masked SDPA "
                "decode")
    else:
        row = kc.size(2) * kc.size(3)

        def step():
            kc.view(-1, row)[slots] = nk.reshape(b, row)
            vc.view(-1, row)[slots] = nv.reshape(b, row)
            ko.gather_sdpa_decode(q, kc, vc, bt_small, lens, wl.scale, max_len)
        what = "torch append (index_put) + gather + expand + masked SDPA decode"
    med, cv = _timed_reps(step, reps)
    kv_bytes = int(lens.sum()) * tok_bytes
    return {
        "value": round(b / med, 1),
        "unit": "tokens/s",
        "GBps_effective": round(kv_bytes / med / 1e9, 3),
        "cores": threads,
        "kind": "port",
        "sample": (f"{b} of the {wl.batch} sequences (same q, block tables and KV bytes), "
                   f"{what}, median of {reps} reps ({med * 1e3:.1f} ms, cv {cv:.2f}); "
                   f"process peak RSS {_peak_rss_gb():.1f} GB"),
    }


def cpu_mixed_baseline(torch, q, kc, vc, bt, dec, dlen, cu_q, cu_k, flops, reps=3):
    """The engine's torch mixed batch on the host (attention.py:146-166):
    gather + SDPA decode of the decode rows, the per-sequence prefill loop
    with the prefix mask (:179-213), torch.cat.  The whole workload (it is
    bounded: about a second per call on 16 cores)."""
    from oracle import kv_oracle as ko
    threads = cpu_threads()
    torch.set_num_threads(threads)
    bt_h = bt.cpu()
    used = torch.unique(bt_h[bt_h >= 0])
    remap = torch.full((kc.size(0),), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    kch = kc.index_select(0, used.to(kc.device)).cpu()
    vch = vc.index_select(0, used.to(vc.device)).cpu()
    bt_small = torch.where(bt_h >= 0, remap[bt_h.clamp(min=0).long()],
                           torch.full_like(bt_h, -1, dtype=torch.int64)).to(torch.int32)
    qh = q.cpu()
    dl = dlen.cpu()
    nd = len(dec)

    def call():
        ko.mixed_torch(qh, kch, vch, bt_small, nd, dl, int(dl.max()), cu_q, cu_k, 128 ** -0.5)
    med, cv = _timed_reps(call, reps)
    T = q.size(0)
    return {"value": round(T / med, 1), "unit": "tokens/s",
            "prefill_TFLOPs": round(flops / med / 1e12, 3),
            "decode_kv_GBps_effective": round(sum(dec) * 2048 / med / 1e9, 3),
            "cores": threads, "kind": "port",
            "sample": (f"the whole mixed call ({nd} decode rows + {len(cu_q) - 1} prefill "
                       f"chunks), torch gather + SDPA decode rows, per-sequence prefix-masked "
                       f"SDPA prefill loop, cat; median of {reps} reps ({med * 1e3:.1f} ms, "
                       f"cv {cv:.2f}); process peak RSS {_peak_rss_gb():.1f} GB")}


def cpu_swap_baseline(torch, L, kvh, reps=3):
    """The engine's torch block moves on the host (model_runner.py:284-305
    offload_put / offload_get, and the compaction as index_select +
    index_copy_) on a host pool scaled to host memory: 96 blocks of
    [2, L, 256, kvh, 128] bf16 (24 MiB each at 48 layers x 4 kv heads),
    8 puts into pinned-size host slots, 8 gets back, a 32-block compaction
    (the config's 128 / 128 / 1024 scaled by 1/16 and 1/32)."""
    from oracle import kv_oracle as ko
    threads = cpu_threads()
    torch.set_num_threads(threads)
    nb, n_swap, n_copy = 96, 8, 32
    g = torch.Generator().manual_seed(7)
    pool = torch.empty(2, L, nb, 256, kvh, 128, dtype=torch.bfloat16)
    pool.view(torch.int16).random_(generator=g)
    perm = torch.randperm(nb, generator=g).tolist()
    out_ids, in_ids = perm[:n_swap], perm[n_swap:2 * n_swap]
    src, dst = perm[2 * n_swap:2 * n_swap + n_copy], perm[2 * n_swap + n_copy:2 * n_swap + 2 * n_copy]
    slots = torch.empty(n_swap, 2, L, 256, kvh, 128, dtype=torch.bfloat16)

    def step():
        for i, b in enumerate(out_ids):
            ko.offload_put_torch(pool, b, slots[i])
        for i, b in enumerate(in_ids):
            ko.offload_get_torch(pool, slots[i], b)
        ko.compact_torch(pool, src, dst)
    med, cv = _timed_reps(step, reps)
    item = 2 * L * 256 * kvh * 128 * 2
    moved = 2 * n_swap * item + 2 * n_copy * item
    return {"value": round(moved / med / 1e9, 3), "unit": "GB/s (moved bytes: put + get + "
            "2 x compaction)", "cores": threads, "kind": "port",
            "sample": (f"host pool of {nb} x {item / 2 ** 20:.0f} MiB blocks: {n_swap} "
                       f"offload_put (index_select + slot copy), {n_swap} offload_get "
                       f"(index_copy_), {n_copy}-block compaction; median of {reps} reps "
                       f"({med * 1e3:.1f} ms, cv {cv:.2f})")}


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
# Decode workloads: (batch, q heads, kv heads, pool blocks, context lengths,
# description of the lengths).
def decode_shape(workload: str):
    from nanovllm_amd.workloads import uniform_lengths
    if workload == "decode-dist":
        return 64, 32, 4, 8192, uniform_lengths(64, 512, 4096, seed=2), "ctx U[512,4096]"
    if workload == "decode-tp2":
        # the engine's per-rank shape under 2-way tensor parallelism
        # (nanovllm/models/qwen3.py:29-35, model_runner.py:407)
        return 64, 16, 2, 8192, [4096] * 64, "ctx 4096"
    if workload == "cfg1":
        # Qwen3-0.6B-shaped layer: 16 q / 8 kv heads, batch 8 of U[128,1024]
        # over a 64-block pool
        return 8, 16, 8, 64, uniform_lengths(8, 128, 1024, seed=1), "ctx U[128,1024]"
    return 64, 32, 4, 8192, [4096] * 64, "ctx 4096"


def run_decode(args, torch, dist: bool, int8: bool = False):
    from nanovllm_amd.kernels.paged_attention import (paged_decode_append,
                                                      paged_decode_append_int8_tokhead)
    from nanovllm_amd.workloads import decode_workload, int8_tokhead_decode_workload

    dev = torch.device("cuda:0")
    if int8:
        # K ~ N(0,1) with 1 % of entries x20, V ~ N(0,1), every context token
        # appended through the per-token-head quantiser before the timed steps
        batch, heads, kvh, blocks = 16, 32, 4, 2048 + 16
        lens = [32768] * batch
        ctx_desc = f"ctx {lens[0]}"
        wl = int8_tokhead_decode_workload(batch, heads, kvh, blocks, lens, seed=3, device=dev)
    else:
        batch, heads, kvh, blocks, lens, ctx_desc = decode_shape(args.workload)
        # a 64-block pool is small enough to draw on the CPU (as the CPU path would)
        wl = decode_workload(batch, heads, kvh, blocks, lens, seed=3, device=dev,
                             pool_device_fill=blocks > 64)
    # decode-cold: the steps cycle through 8 disjoint block-table sets that
    # cover the 8192-block pool, so a step never reads KV that one of the 7
    # steps before it read (8 x 537 MB per cycle against a 256 MB Infinity
    # Cache); every set is a seeded random permutation of its blocks.
    sets = [(wl.block_tables, wl.slot_mapping)]
    if args.workload == "decode-cold":
        gen = torch.Generator().manual_seed(11)
        perm = torch.randperm(blocks, generator=gen).to(torch.int32)
        per = batch * (lens[0] // 256)
        sets = []
        for i in range(blocks // per):
            bt = perm[i * per:(i + 1) * per].view(batch, -1).contiguous()
            sm = bt[:, -1] * 256 + (lens[0] - 1) % 256
            sets.append((bt.to(dev), sm.to(torch.int32).to(dev)))
        ctx_desc += f", {len(sets)} disjoint table sets in turn"
    cycle = [0]

    def step(timer=None):
        if int8:
            # the per-token-head step (quantise-on-append + decode) in one call:
            # the quantiser rides in the decode launch
            s = timer.start() if timer else None
            out = paged_decode_append_int8_tokhead(wl.q, wl.new_k, wl.new_v, wl.k_cache,
                                                   wl.v_cache, wl.k_scale, wl.v_scale,
                                                   wl.slot_mapping, wl.block_tables,
                                                   wl.context_lens, wl.scale)
        else:
            # the engine's decode step (store_kvcache + paged decode) in one call:
            # the append rides in the decode launch
            bt, sm = sets[cycle[0] % len(sets)]
            cycle[0] += 1
            s = timer.start() if timer else None
            out = paged_decode_append(wl.q, wl.new_k, wl.new_v, wl.k_cache, wl.v_cache,
                                      sm, bt, wl.context_lens, wl.scale)
        if timer:
            timer.stop(s)
        return out

    for _ in range(args.warmup):
        step()
    # Throughput: exactly K steps, nothing else in the stream (the per-call
    # events below add command-processor work between the steps).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    # Roofline: the decode call's own duration, from HIP events around it on
    # its stream, in a second pass of K steps.
    timer = EventTimer(torch)
    for _ in range(args.steps):
        step(timer)
    torch.cuda.synchronize()
    kernel_ms = timer.mean_ms()

    tok_bytes = 2 * kvh * 128 * (1 if int8 else 2) + (2 * kvh * 4 if int8 else 0)
    kv_bytes = sum(lens) * tok_bytes
    other = 2 * batch * heads * 128 * 2 + wl.block_tables.numel() * 4 + batch * 4
    if int8:
        # the quantise-on-append: bf16 rows in, codes and fp32 scales out, slots
        other += 2 * batch * kvh * 128 * 2 + 2 * batch * kvh * (128 + 4) + batch * 4
    else:
        other += 2 * 2 * batch * kvh * 128 * 2 + batch * 4  # the append: new rows in and out, slots
    algo = kv_bytes + other
    achieved = algo / (kernel_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": round(batch / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if int8 else "bf16",
        "data": ("synthetic (seeded N(0,1) q/v, K N(0,1) with 1% x20 outliers quantised "
                 "through the append, random non-contiguous block tables)" if int8 else
                 "synthetic (seeded N(0,1) q/k/v, random non-contiguous block tables)"),
        "config": {
            "workload": (f"paged decode step (append 1 token/seq + decode), {heads}q/{kvh}kv/128 "
                         f"{'int8 per-token-head' if int8 else 'bf16'}, batch {batch} x "
                         f"{ctx_desc}, page 256, {blocks}-block pool"),
            "batch": batch,
            "context": ctx_desc[4:],
            "heads": heads,
            "kv_heads": kvh,
            "head_dim": 128,
            "page": 256,
            # HIP events around the decode call: the decode kernel + its split
            # merge (the kernel alone is in the committed kernel trace)
            "decode_call_us": round(kernel_ms * 1e3, 2),
            "kv_read_GBps": round(kv_bytes / (kernel_ms * 1e-3) / 1e9, 1),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": profiled_traffic(args.workload),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE of the same workload, "
                              "committed under profiles/ (not measured in this run)",
        },
    }
    if args.stamps:
        res["workgroup_end_us"] = decode_stamps(torch, step)
    if not args.no_cpu_baseline:
        sample = args.cpu_sample if args.cpu_sample else (2 if int8 else 64)
        res["cpu_baseline"] = cpu_decode_baseline(torch, wl, sample, tok_bytes, int8=int8)
    return res


def run_int8_chan(args, torch):
    """The per-channel int8 decode step (the engine's int8 mode,
    nanovllm/kernels/kv_int8.py:29-93, paged_attention.py:101-172) at the
    int8 configuration's shape: batch 16 x context 32768, 32 q / 4 kv heads,
    page 256.  The pool holds random codes, per-channel store / read scales
    and a side pool of --side-slots slots per kv head (8 in the engine,
    nanovllm/engine/model_runner.py:100), half of them holding outlier dims.
    One step =
    store_kvcache_int8 of one token per sequence (quantise, outlier dims to
    the side pool) + paged decode (the per-channel LDS ring: the read scales
    folded into the query, outlier values from the side pool)."""
    from nanovllm_amd.kernels.kv_int8 import store_kvcache_int8
    from nanovllm_amd.kernels.paged_attention import paged_decode_attention
    from nanovllm_amd.workloads import build_block_tables, slots_for_last_token
    dev = torch.device("cuda:0")
    batch, heads, kvh, ctx, n_out = 16, 32, 4, 32768, args.side_slots
    used = max(1, n_out // 2)
    blocks = batch * ctx // 256 + 16
    lens = [ctx] * batch
    gen = torch.Generator().manual_seed(9)
    bt = build_block_tables(lens, blocks, 256, gen)
    slots = slots_for_last_token(bt, lens, 256).to(dev)
    bt = bt.to(dev)
    cl = torch.tensor(lens, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(10)
    kc = torch.randint(-127, 128, (blocks, 256, kvh, 128), generator=g, device=dev,
                       dtype=torch.int8)
    vc = torch.randint(-127, 128, (blocks, 256, kvh, 128), generator=g, device=dev,
                       dtype=torch.int8)
    s_k = (torch.rand(kvh, 128, generator=g, device=dev) * 0.02 + 0.01)
    s_v = (torch.rand(kvh, 128, generator=g, device=dev) * 0.02 + 0.01)
    dims = [3, 77, 20, 101, 45, 64, 9, 120][:n_out]
    out_idx2d = torch.tensor([dims] * kvh, dtype=torch.int32, device=dev)
    head_n_out = torch.full((kvh,), used, dtype=torch.int32, device=dev)
    ds_k, ds_v = s_k.clone(), s_v.clone()
    for d in dims[:used]:
        ds_k[:, d] = 0.0
        ds_v[:, d] = 0.0
    sk = torch.randn(blocks, 256, kvh, n_out, generator=g, device=dev).to(torch.bfloat16)
    sv = torch.randn(blocks, 256, kvh, n_out, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(batch, heads, 128, generator=g, device=dev).to(torch.bfloat16)
    nk = torch.randn(batch, kvh, 128, generator=g, device=dev).to(torch.bfloat16)
    nv = torch.randn(batch, kvh, 128, generator=g, device=dev).to(torch.bfloat16)

    def step(timer=None):
        s = timer.start() if timer else None
        store_kvcache_int8(nk, nv, kc, vc, s_k, s_v, sk, sv, out_idx2d, head_n_out, slots)
        out = paged_decode_attention(q, kc, vc, bt, cl, 128 ** -0.5, ctx, k_scale=ds_k,
                                     v_scale=ds_v, side_k=sk, side_v=sv, out_idx2d=out_idx2d,
                                     head_n_out=head_n_out)
        if timer:
            timer.stop(s)
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    timer = EventTimer(torch)
    for _ in range(args.steps):
        step(timer)
    torch.cuda.synchronize()
    call_ms = timer.mean_ms()
    # codes, and the side pool's rows (every slot: the rows are read whole),
    # of every context token
    kv_bytes = batch * ctx * (2 * kvh * 128 + 2 * kvh * n_out * 2)
    res = {"workload": f"int8 per-channel decode step (store_kvcache_int8 + paged decode), "
                       f"{heads}q/{kvh}kv/128, batch {batch} x ctx {ctx}, page 256, side pool of "
                       f"{n_out} slots per kv head, {used} outlier dims in use",
           "tokens_per_s": round(batch / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
           "step_call_us": round(call_ms * 1e3, 2), "kv_bytes": kv_bytes,
           "kv_read_GBps_at_call": round(kv_bytes / (call_ms * 1e-3) / 1e9, 1)}
    if args.stamps:
        res["workgroup_end_us"] = decode_stamps(torch, step)
    return res


def decode_stamps(torch, step, reps=20):
    """Per-workgroup end times of the decode kernel (after the timed region):
    KVC_DECODE_STAMPS=1 makes every workgroup record its start and end
    wall-clock stamps; per step, times are taken from the earliest start.
    Returns the medians over `reps` steps of the first, median and last
    workgroup end, the spread (last - first), and each XCD's median end
    (workgroup v runs on XCD v mod 8)."""
    import ctypes
    from nanovllm_amd import _native as nat
    os.environ["KVC_DECODE_STAMPS"] = "1"
    buf = (ctypes.c_ulonglong * (2 * 4096))()
    n, khz = ctypes.c_int(0), ctypes.c_int(0)
    rows = []
    try:
        for _ in range(reps):
            step()
            torch.cuda.synchronize()
            nat.call("kvc_decode_stamps", ctypes.addressof(buf), 4096, ctypes.addressof(n),
                     ctypes.addressof(khz))
            g = n.value
            us_per_tick = 1e3 / khz.value
            t0 = min(buf[2 * v] for v in range(g))
            ends = [(buf[2 * v + 1] - t0) * us_per_tick for v in range(g)]
            srt = sorted(ends)
            xcd = [statistics.median(ends[x::8]) for x in range(8)]
            rows.append((srt[0], srt[g // 2], srt[-1], xcd))
    finally:
        del os.environ["KVC_DECODE_STAMPS"]
    med = lambda i: round(statistics.median(r[i] for r in rows), 2)
    return {"first": med(0), "median": med(1), "last": med(2),
            "spread": round(statistics.median(r[2] - r[0] for r in rows), 2),
            "xcd_median": [round(statistics.median(r[3][x] for r in rows), 2) for x in range(8)],
            "workgroups": n.value, "clock_khz": khz.value, "steps": reps}


# The reference's published decode grid (benchmarks/archive/P15-pd-autotune.md:
# 10-15, Triton on an MTT S4000, geomean over contexts 512/1024/2048/4096 per
# batch, 16 q / 2 kv heads, head_dim 128, page 256): default config and
# autotuned per-batch config, in ms per kernel.
P15_REFERENCE_MS = {1: (0.311, 0.180), 8: (0.487, 0.307), 16: (0.806, 0.365),
                    32: (1.586, 0.547)}


def run_p15_grid(args, torch):
    """Paged decode (no append: the reference times the kernel) at the
    reference's published grid: batch 1 / 8 / 16 / 32 x context 512 / 1024 /
    2048 / 4096 at 16 q / 2 kv heads.  Each point: the decode call captured
    in a HIP graph (as the engine replays its decode steps, so host
    submission is not in the time), HIP events around each replay, mean over
    the timed replays; the geomean over contexts per batch sits beside the
    reference's (other hardware)."""
    from nanovllm_amd.kernels.paged_attention import paged_decode_attention
    from nanovllm_amd.workloads import decode_workload
    dev = torch.device("cuda:0")
    grid, geo = {}, {}
    steps = max(5, args.steps)
    for batch in (1, 8, 16, 32):
        logs = []
        for ctx in (512, 1024, 2048, 4096):
            wl = decode_workload(batch, 16, 2, batch * ctx // 256 + 8, [ctx] * batch,
                                 seed=batch + ctx, device=dev, pool_device_fill=True)

            def call():
                return paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.block_tables,
                                              wl.context_lens, wl.scale, ctx)
            for _ in range(max(1, args.warmup)):
                call()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                call()
            torch.cuda.synchronize()
            for _ in range(3):
                graph.replay()
            timer = EventTimer(torch)
            for _ in range(steps):
                s = timer.start()
                graph.replay()
                timer.stop(s)
            torch.cuda.synchronize()
            del graph
            us = timer.mean_ms() * 1e3
            kv = batch * ctx * 2 * 2 * 128 * 2
            grid[f"b{batch}x{ctx}"] = {"us": round(us, 2), "kv_GBps": round(kv / us / 1e3, 1)}
            logs.append(math.log(us))
            del wl
        geo[batch] = math.exp(sum(logs) / len(logs))
    out_geo = {f"b{b}": {"geomean_us": round(v, 2),
                         "reference_default_us": P15_REFERENCE_MS[b][0] * 1e3,
                         "reference_tuned_us": P15_REFERENCE_MS[b][1] * 1e3}
               for b, v in geo.items()}
    b32 = grid["b32x4096"]
    return {
        "metric": "paged decode call time at the reference's published grid (16q/2kv/128)",
        "value": b32["us"],
        "unit": "us (b32 x 4096)",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(b32["us"] / 1e3, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, random non-contiguous block tables)",
        "config": {"workload": "paged decode call (graph replay), 16q/2kv/128 bf16, page 256, "
                               "batch 1/8/16/32 x ctx 512/1024/2048/4096",
                   "grid": grid, "geomean_by_batch": out_geo},
    }


MIXES = {
    # name: (decode rows, their context range, prefill chunks as (prefix, tokens))
    "mixed": (60, (256, 4096), [(0, 256), (512, 256), (2048, 256), (8192, 256)]),
    "mixed16": (16, (256, 4096), [(0, 512), (512, 512), (2048, 512), (8192, 512)]),
}


def run_mixed(args, torch, mix="mixed"):
    from nanovllm_amd.kernels.varlen import (varlen_attention, varlen_attention_append,
                                             varlen_decode_cus)
    from nanovllm_amd.layers.attention import store_kvcache
    from nanovllm_amd.workloads import build_block_tables, uniform_lengths

    dev = torch.device("cuda:0")
    heads, kvh = 32, 4
    n_dec, (lo, hi), chunks = MIXES[mix]
    dec = uniform_lengths(n_dec, lo, hi, seed=3)
    all_lens = dec + [p + c for p, c in chunks]
    g = torch.Generator().manual_seed(4)
    blocks = sum((n + 255) // 256 for n in all_lens) + 8
    bt_cpu = build_block_tables(all_lens, blocks, 256, g)
    bt = bt_cpu.to(dev)
    dg = torch.Generator(device=dev).manual_seed(5)
    kc = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    T = len(dec) + sum(c for _, c in chunks)
    q = torch.randn(T, heads, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    dlen = torch.tensor(dec, dtype=torch.int32, device=dev)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    # The step's new rows: decode row i at its last position, chunk j's tokens
    # at positions prefix_j .. prefix_j + c_j - 1.
    slots = [int(bt_cpu[i, (n - 1) // 256]) * 256 + (n - 1) % 256 for i, n in enumerate(dec)]
    for j, (p, c) in enumerate(chunks):
        row = len(dec) + j
        slots += [int(bt_cpu[row, t // 256]) * 256 + t % 256 for t in range(p, p + c)]
    slot_t = torch.tensor(slots, dtype=torch.int32, device=dev)
    kv_new = torch.randn(T, 2, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    key, value = kv_new[:, 0], kv_new[:, 1]
    kw = dict(scale=128 ** -0.5, block_tables=bt, num_decode_rows=len(dec),
              decode_context_lens=dlen, cu_seqlens_q=cq, cu_seqlens_k=ck,
              cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k)

    def call():
        return varlen_attention(q, kc, vc, decode_context_lens_list=dec, **kw)

    def call_unhinted():
        return varlen_attention(q, kc, vc, **kw)

    def step_store_then_call():
        store_kvcache(key, value, kc, vc, slot_t)
        return varlen_attention(q, kc, vc, decode_context_lens_list=dec, **kw)

    def step_append():
        return varlen_attention_append(q, key, value, kc, vc, slot_t,
                                       decode_context_lens_list=dec, **kw)

    # The same prefill rows alone (their block-table rows and queries), to
    # price the prefill launch against the MFMA roofline.
    nd = len(dec)
    q_pre, bt_pre = q[nd:], bt[nd:]

    def call_prefill():
        return varlen_attention(q_pre, kc, vc, scale=128 ** -0.5, block_tables=bt_pre,
                                cu_seqlens_q=cq, cu_seqlens_k=ck, cu_seqlens_q_list=cu_q,
                                cu_seqlens_k_list=cu_k)

    # Every form is timed in each step, one after the other, so that all see
    # the same clocks and caches (a form timed alone after another one ran
    # at a different clock state).
    forms = [call, call_unhinted, step_store_then_call, step_append, call_prefill]
    if args.mixed_call_only:
        forms = [call] * len(forms)  # kernel traces of the hinted call alone
    for _ in range(args.warmup):
        for fn in forms:
            fn()
    torch.cuda.synchronize()
    timers = [EventTimer(torch) for _ in forms]
    for _ in range(args.steps):
        for fn, timer in zip(forms, timers):
            s = timer.start()
            fn()
            timer.stop(s)
    torch.cuda.synchronize()
    ms, ms_unhinted, ms_step_store, ms_step_append, ms_pre = (t.mean_ms() for t in timers)
    flops = 0
    for p, c in chunks:
        for r in range(c):
            flops += 4 * 128 * heads * (p + r + 1)
    kv = sum(dec) * 2 * kvh * 128 * 2
    pre_tflops = flops / (ms_pre * 1e-3) / 1e12
    split = varlen_decode_cus(nd, T - nd, heads, kvh, dec, cu_q, cu_k)
    chunk_desc = "/".join(str(p) for p, _ in chunks)
    res = {"workload": f"{mix}: {nd} decode rows ctx U[{lo},{hi}] + {len(chunks)}x"
                       f"{chunks[0][1]}-token prefill chunks (prefix {chunk_desc}): one launch "
                       "over a CU split sized from the host's work hints (stream-K decode + "
                       "stream-K prefill) + one merge launch",
            "ms": round(ms, 4), "decode_cus": split,
            "ms_fixed_3_8_split": round(ms_unhinted, 4),
            "step_store_then_call_ms": round(ms_step_store, 4),
            "step_append_ms": round(ms_step_append, 4),
            "prefill_gflop": round(flops / 1e9, 2),
            "prefill_only_ms": round(ms_pre, 4),
            "prefill_TFLOPs": round(pre_tflops, 1),
            "prefill_mfma_frac": round(pre_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "decode_kv_GB": round(kv / 1e9, 3),
            "tokens_per_s": round(T / (ms * 1e-3), 1)}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_mixed_baseline(torch, q, kc, vc, bt, dec, dlen, cu_q, cu_k,
                                                 flops)
    return res


def run_prefill_int8(args, torch):
    """The prefill rows of the mixed workload (4 chunks of 256 tokens after
    prefixes 0 / 512 / 2048 / 8192, 32 q / 4 kv heads) over a bf16 pool, a
    per-token-head int8 pool and a per-channel int8 pool (read scales, a side
    pool of 8 slots per kv head with 4 outlier dims in use): one varlen call
    each, timed in turn within every step.  The int8 calls read the pool as
    the reference's prefill does (nanovllm/layers/attention.py:33-51): keys
    gathered and dequantised to bf16, then the bf16 prefill."""
    from nanovllm_amd.kernels.varlen import varlen_attention
    from nanovllm_amd.workloads import build_block_tables

    dev = torch.device("cuda:0")
    heads, kvh = 32, 4
    chunks = MIXES["mixed"][2]
    lens = [p + c for p, c in chunks]
    g = torch.Generator().manual_seed(4)
    blocks = sum((n + 255) // 256 for n in lens) + 8
    bt = build_block_tables(lens, blocks, 256, g).to(dev)
    dg = torch.Generator(device=dev).manual_seed(5)
    T = sum(c for _, c in chunks)
    q = torch.randn(T, heads, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    cu_q, cu_k = [0], [0]
    for p, c in chunks:
        cu_q.append(cu_q[-1] + c)
        cu_k.append(cu_k[-1] + p + c)
    kw = dict(scale=128 ** -0.5, block_tables=bt, num_decode_rows=0,
              cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=dev),
              cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=dev),
              cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k)
    kcb = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    vcb = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
    kc8 = torch.randint(-127, 128, (blocks, 256, kvh, 128), generator=dg, device=dev,
                        dtype=torch.int8)
    vc8 = torch.randint(-127, 128, (blocks, 256, kvh, 128), generator=dg, device=dev,
                        dtype=torch.int8)
    ksc = torch.rand(blocks, 256, kvh, generator=dg, device=dev) * 0.02
    vsc = torch.rand(blocks, 256, kvh, generator=dg, device=dev) * 0.02
    nom = 8
    oi = torch.tensor([[3, 77, 20, 101, 45, 64, 9, 120]] * kvh, dtype=torch.int32, device=dev)
    hn = torch.full((kvh,), 4, dtype=torch.int32, device=dev)
    ds = torch.rand(kvh, 128, generator=dg, device=dev) * 0.02 + 0.01
    ds[:, oi[0, :4].long()] = 0.0
    side = torch.randn(blocks, 256, kvh, nom, generator=dg, device=dev).to(torch.bfloat16)
    forms = {
        "bf16": lambda: varlen_attention(q, kcb, vcb, **kw),
        "int8_tokhead": lambda: varlen_attention(q, kc8, vc8, k_scale=ksc, v_scale=vsc, **kw),
        "int8_chan": lambda: varlen_attention(q, kc8, vc8, k_scale=ds, v_scale=ds, side_k=side,
                                              side_v=side, out_idx2d=oi, head_n_out=hn, **kw),
    }
    for _ in range(args.warmup):
        for fn in forms.values():
            fn()
    torch.cuda.synchronize()
    timers = {k: EventTimer(torch) for k in forms}
    for _ in range(args.steps):
        for k, fn in forms.items():
            s = timers[k].start()
            fn()
            timers[k].stop(s)
    torch.cuda.synchronize()
    flops = 0
    for p, c in chunks:
        for r in range(c):
            flops += 4 * 128 * heads * (p + r + 1)
    out = {"workload": "prefill rows of the mixed workload (4x256-token chunks after prefixes "
                       "0/512/2048/8192, 32q/4kv/128) over bf16 / int8 per-token-head / int8 "
                       "per-channel (8 side slots, 4 in use) pools, one varlen call each",
           "prefill_gflop": round(flops / 1e9, 2)}
    for k, t in timers.items():
        ms = t.mean_ms()
        out[f"{k}_us"] = round(ms * 1e3, 1)
        out[f"{k}_TFLOPs"] = round(flops / (ms * 1e-3) / 1e12, 1)
        out[f"{k}_mfma_frac"] = round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
    return out


def run_prefill_scale(args, torch):
    """The stream-K prefill (prefill rows only, bf16 pool) over four chunks
    after prefixes 0 / 512 / 2048 / 8192 whose length runs 64 .. 1024 tokens
    (256 is the mixed workload's): the call time against the FLOPs, fitted
    as fixed + FLOPs / rate, and the per-workgroup start and end stamps of
    the prefill launch (KVC_PREFILL_STAMPS) at each length."""
    import ctypes
    from nanovllm_amd import _native as nat
    from nanovllm_amd.kernels.varlen import varlen_attention
    from nanovllm_amd.workloads import build_block_tables

    dev = torch.device("cuda:0")
    heads, kvh = 32, 4
    points = []
    for c in (64, 128, 256, 512, 1024):
        chunks = [(0, c), (512, c), (2048, c), (8192, c)]
        lens = [p + n for p, n in chunks]
        g = torch.Generator().manual_seed(4)
        blocks = sum((n + 255) // 256 for n in lens) + 8
        bt = build_block_tables(lens, blocks, 256, g).to(dev)
        dg = torch.Generator(device=dev).manual_seed(5)
        T = sum(n for _, n in chunks)
        q = torch.randn(T, heads, 128, generator=dg, device=dev, dtype=torch.bfloat16)
        kc = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(blocks, 256, kvh, 128, generator=dg, device=dev, dtype=torch.bfloat16)
        cu_q, cu_k = [0], [0]
        for p, n in chunks:
            cu_q.append(cu_q[-1] + n)
            cu_k.append(cu_k[-1] + p + n)
        kw = dict(scale=128 ** -0.5, block_tables=bt, num_decode_rows=0,
                  cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=dev),
                  cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=dev),
                  cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k)
        for _ in range(args.warmup):
            varlen_attention(q, kc, vc, **kw)
        torch.cuda.synchronize()
        timer = EventTimer(torch)
        for _ in range(args.steps):
            st = timer.start()
            varlen_attention(q, kc, vc, **kw)
            timer.stop(st)
        torch.cuda.synchronize()
        us = timer.mean_ms() * 1e3
        flops = sum(4 * 128 * heads * (p + r + 1) for p, n in chunks for r in range(n))
        # Stamps of the prefill launch (the slice merge is a launch of its own).
        buf = (ctypes.c_ulonglong * 8192)()
        nwg, khz = ctypes.c_int(), ctypes.c_int()
        os.environ["KVC_PREFILL_STAMPS"] = "1"
        rows = []
        try:
            for _ in range(5):
                varlen_attention(q, kc, vc, **kw)
                torch.cuda.synchronize()
                nat.call("kvc_decode_stamps", ctypes.addressof(buf), 4096,
                         ctypes.addressof(nwg), ctypes.addressof(khz))
                n_wg, tick = nwg.value, 1e3 / khz.value
                t0 = min(buf[2 * v] for v in range(n_wg))
                ends = sorted((buf[2 * v + 1] - t0) * tick for v in range(n_wg))
                busy = [e for e in ends if e > 5.0] or ends
                rows.append((busy[len(busy) // 10], ends[n_wg // 2], ends[-1]))
        finally:
            del os.environ["KVC_PREFILL_STAMPS"]
        med = [round(statistics.median(r[i] for r in rows), 2) for i in range(3)]
        points.append({"chunk": c, "gflop": round(flops / 1e9, 2), "call_us": round(us, 1),
                       "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1),
                       "end_p10_us": med[0], "end_median_us": med[1], "end_last_us": med[2]})
    # Least-squares fit of call_us = fixed + gflop / rate over the five points.
    xs = [pt["gflop"] for pt in points]
    ys = [pt["call_us"] for pt in points]
    mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    return {"workload": "stream-K prefill rows only (bf16 pool, 32q/4kv/128, page 256), four "
                        "chunks after prefixes 0/512/2048/8192, chunk length 64..1024 tokens",
            "points": points,
            "fit_fixed_us": round(my - slope * mx, 1),
            "fit_marginal_TFLOPs": round(1e3 / slope, 1),
            "fit_marginal_mfma_frac": round(1e3 / slope / MFMA_BF16_PEAK_TFLOPS, 4)}


def run_append(args, torch):
    from nanovllm_amd.layers.attention import store_kvcache
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1)
    N, kvh = 16384, 4
    k = torch.randn(N, kvh, 128, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(N, kvh, 128, generator=g, device=dev, dtype=torch.bfloat16)
    kc = torch.empty(1024, 256, kvh, 128, device=dev, dtype=torch.bfloat16)
    vc = torch.empty_like(kc)
    slots = torch.randperm(1024 * 256, device=dev)[:N].to(torch.int32)
    for _ in range(args.warmup):
        store_kvcache(k, v, kc, vc, slots)
    timer = EventTimer(torch)
    for _ in range(args.steps):
        s = timer.start()
        store_kvcache(k, v, kc, vc, slots)
        timer.stop(s)
    torch.cuda.synchronize()
    ms = timer.mean_ms()
    byts = 2 * 2 * N * kvh * 128 * 2 + N * 4
    return {"workload": f"append {N} tokens x 4kv x 128 bf16 (K and V)", "ms": round(ms, 4),
            "GBps": round(byts / (ms * 1e-3) / 1e9, 1)}


def run_rope(args, torch):
    """q/k RMSNorm + rotary embedding + KV append in one launch at the
    Qwen3-30B-A3B attention shape (32 q / 4 kv heads x 128, page 256): a
    decode step (64 tokens) and a 16384-token prefill batch.  HBM bytes per
    token: the fused qkv row read (40 x 256 B) + q out (32 x 256 B) + K and V
    rows appended (2 x 4 x 256 B) + the token's fp32 cos/sin row (512 B) +
    its position and slot (16 B)."""
    from nanovllm_amd.layers.rotary import build_cos_sin_cache, qk_norm_rope_store
    dev = torch.device("cuda:0")
    H, KVH = 32, 4
    per_token = (H + 2 * KVH) * 256 + H * 256 + 2 * KVH * 256 + 512 + 16
    cache = build_cos_sin_cache(128, 40960, 1000000.0, dev)
    qw = torch.ones(128, dtype=torch.bfloat16, device=dev)
    kw = torch.ones(128, dtype=torch.bfloat16, device=dev)
    out = {"workload": "q/k RMSNorm + RoPE + KV append, 32q/4kv/128 bf16, one launch"}
    for N in (64, 16384):
        g = torch.Generator(device=dev).manual_seed(N)
        qkv = torch.randn(N, (H + 2 * KVH) * 128, generator=g, device=dev, dtype=torch.bfloat16)
        q = qkv[:, :H * 128].view(N, H, 128)
        k = qkv[:, H * 128:(H + KVH) * 128].view(N, KVH, 128)
        v = qkv[:, (H + KVH) * 128:].view(N, KVH, 128)
        pos = torch.randint(0, 40960, (N,), generator=g, device=dev)
        blocks = max(64, (N + 255) // 256 * 2)
        kc = torch.empty(blocks, 256, KVH, 128, device=dev, dtype=torch.bfloat16)
        vc = torch.empty_like(kc)
        slots = torch.randperm(blocks * 256, generator=g, device=dev)[:N]
        q_out = torch.empty(N, H, 128, device=dev, dtype=torch.bfloat16)

        def call():
            qk_norm_rope_store(q, k, v, pos, cache, qw, kw, 1e-6, kc, vc, slots,
                               return_k=False, q_out=q_out)

        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        timer = EventTimer(torch)
        for _ in range(args.steps):
            s = timer.start()
            call()
            timer.stop(s)
        torch.cuda.synchronize()
        ms = timer.mean_ms()
        out[f"tokens_{N}"] = {"us": round(ms * 1e3, 2),
                              "GBps": round(N * per_token / (ms * 1e-3) / 1e9, 1),
                              "tokens_per_s": round(N / (ms * 1e-3), 1)}
    out["bytes_per_token"] = per_token
    return out


def run_decode_graph(args, torch):
    """A 48-layer decode step's KV work (per layer: append one token per
    sequence and paged decode, one paged_decode_append call) run eagerly and
    as a replayed HIP graph of
    the batch's bucket, with the padded rows aimed at the scratch block.  Two
    sizes: batch 64 x context 4096 (the headline shape, GPU-bound) and
    batch 8 x context 512 (launch-bound).  Shape 32 q / 4 kv heads x 128 bf16,
    page 256."""
    from nanovllm_amd.engine.graph_runner import DecodeGraphRunner
    from nanovllm_amd.kernels.paged_attention import paged_decode_append
    from nanovllm_amd.workloads import build_block_tables, slots_for_last_token
    dev = torch.device("cuda:0")
    L, H, KVH = 48, 32, 4
    out = {"workload": "48-layer decode step KV work (append + paged decode per layer), "
                       "eager vs HIP-graph replay"}
    for bs, ctx in ((64, 4096), (8, 512)):
        nb = bs * ((ctx + 255) // 256)
        g = torch.Generator(device=dev).manual_seed(bs)
        kcs = [torch.randn(nb + 1, 256, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
               for _ in range(L)]
        vcs = [torch.randn(nb + 1, 256, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
               for _ in range(L)]
        lens = [ctx] * bs
        bt = build_block_tables(lens, nb, 256, torch.Generator().manual_seed(bs))
        slots = slots_for_last_token(bt, lens, 256).to(dev)
        bt = bt.to(dev)
        cl = torch.tensor(lens, dtype=torch.int32, device=dev)
        q = torch.randn(L, bs, H, 128, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(L, bs, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(L, bs, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)

        def eager():
            for layer in range(L):
                paged_decode_append(q[layer], k[layer], v[layer], kcs[layer], vcs[layer], slots,
                                    bt, cl, 128 ** -0.5)

        runner = DecodeGraphRunner(kcs, vcs, H, max_bs=bs, max_blocks_per_seq=bt.size(1),
                                   scale=128 ** -0.5, buckets=[bs])
        runner.capture()

        def graph():
            runner.run(q, k, v, slots, cl, bt)

        res = {}
        for name, fn in (("eager", eager), ("graph", graph)):
            for _ in range(max(2, args.warmup // 2)):
                fn()
            torch.cuda.synchronize()
            steps = max(5, args.steps // 5)
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            res[f"{name}_ms_per_step"] = round((time.perf_counter() - t0) * 1e3 / steps, 3)
        out[f"bs{bs}_ctx{ctx}"] = res
        del kcs, vcs, runner
        torch.cuda.empty_cache()
    return out


def run_offload_overlap(args, torch):
    """A 48-layer decode step (batch 64 x context 4096: per layer append one
    token per sequence, then paged decode, through bound Attention layers)
    that also offloads E = 8 blocks of 24 MiB to pinned host slots and
    revives the 8 offloaded one step earlier (the BlockManager's evict /
    revive traffic): blocking moves on the compute stream vs the
    AsyncOffloader (copy streams, per-layer-group fences), against the same
    step without offload traffic."""
    from nanovllm_amd.engine.kv_runner import KVCacheRunner
    from nanovllm_amd.layers.attention import Attention
    from nanovllm_amd.utils.context import reset_context, set_context
    from nanovllm_amd.workloads import build_block_tables, slots_for_last_token
    dev = torch.device("cuda:0")
    L, H, KVH, BS, CTX, E = 48, 32, 4, 64, 4096, 8
    nb = BS * CTX // 256
    lens = [CTX] * BS
    bt = build_block_tables(lens, nb, 256, torch.Generator().manual_seed(1))
    slots = slots_for_last_token(bt, lens, 256).to(dev)
    bt = bt.to(dev)
    cl = torch.tensor(lens, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(L, BS, H, 128, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(L, BS, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(L, BS, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
    put_ids = list(range(nb, nb + E))
    get_ids = list(range(nb + E, nb + 2 * E))
    block_mib = 2 * L * 256 * KVH * 128 * 2 / 2 ** 20
    out = {"workload": (f"48-layer decode step (bs {BS} x {CTX}) + offload of {E} and revival "
                        f"of {E} blocks of {block_mib:.0f} MiB per step"),
           "block_MiB": block_mib}
    modes = (("no_offload", 0, None), ("blocking", 0, None), ("copies_only_blocking", 0, None),
             ("async_dma_g4", 4, "dma"), ("async_kernel_g1", 1, "kernel"),
             ("async_kernel_g8", 8, "kernel"))
    for mode, groups, engine in modes:
        r = KVCacheRunner(L, nb + 2 * E, 256, KVH, 128, kv_offload_host_blocks=3 * E,
                          async_offload_groups=groups, async_copy_engine=engine or "kernel",
                          device=dev)
        r.kv_cache.normal_(generator=g)
        mods = [Attention(H, 128, 128 ** -0.5, KVH) for _ in range(L)]
        r.bind(mods)

        fifo = []   # slots filled one step earlier: this step's revivals

        def step():
            revive, fresh = [], []
            if mode != "no_offload":
                fresh = r.offload_put_many(put_ids)
                if fifo:
                    revive = fifo.pop(0)
                    r.offload_get_many(revive, get_ids)
            if mode != "copies_only_blocking":
                set_context(False, slot_mapping=slots, context_lens=cl, block_tables=bt,
                            max_context_len=CTX)
                for i, m in enumerate(mods):
                    m.forward(q[i], k[i], v[i])
                reset_context()
            r.fence()
            for s_ in revive:
                r.offload_release(s_)
            if fresh:
                fifo.append(fresh)

        for _ in range(3):
            step()
        torch.cuda.synchronize()
        n = max(5, args.steps // 5)
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        torch.cuda.synchronize()
        out[f"{mode}_ms_per_step"] = round((time.perf_counter() - t0) * 1e3 / n, 3)
        del r, mods
        torch.cuda.empty_cache()
    extra = out["blocking_ms_per_step"] - out["no_offload_ms_per_step"]
    out["offload_cost_blocking_ms"] = round(extra, 3)
    for gname, _, engine in modes:
        if engine is None:
            continue
        out[f"offload_cost_{gname}_ms"] = round(
            out[f"{gname}_ms_per_step"] - out["no_offload_ms_per_step"], 3)
    return out


def run_pd_wire(args, torch):
    """PD KV transfer of one request's 16 blocks (48 layers x 256 tokens x 4 kv
    heads x 128 bf16: 12 MiB per side per block, 384 MiB per frame) from one
    pool to another through a socketpair, sender in a thread:
    * channel: TcpKVChannel (gather kernels into pinned staging, sent and
      received without host copies, chunked so the link and the GPU overlap);
    * torch_ops: the same frame moved with the engine's own composition
      (index_select + permute + pinned copy_ + tobytes + sendall; recv +
      frombuffer + copy + index_copy_, nanovllm/pd/kv_channel.py:54-178).
    Plus extract_kv / import_kv alone (device <-> pinned, the PCIe legs)."""
    import socket
    import struct
    import threading

    from nanovllm_amd.pd.kv_channel import (KVBlockBuffer, TcpKVChannel, extract_kv,
                                            import_kv)
    dev = torch.device("cuda:0")
    L, KVH, NB, N = 48, 4, 40, 16
    g = torch.Generator(device=dev).manual_seed(4)
    src = torch.randn(2, L, NB, 256, KVH, 128, generator=g, device=dev, dtype=torch.bfloat16)
    dst = torch.zeros_like(src)
    t_src = list(range(0, 2 * N, 2))
    t_dst = list(range(NB - 1, NB - 1 - N, -1))
    frame_bytes = 2 * N * L * 256 * KVH * 128 * 2
    reps = max(3, args.steps // 10)

    def torch_ops_send(sock, buf):
        idx = torch.tensor(t_src, device=dev, dtype=torch.long)
        buf.k[:N].copy_(src[0].index_select(1, idx).permute(1, 0, 2, 3, 4))
        buf.v[:N].copy_(src[1].index_select(1, idx).permute(1, 0, 2, 3, 4))
        torch.cuda.synchronize()
        kb = buf.k[:N].contiguous().view(torch.int16).numpy().tobytes()
        vb = buf.v[:N].contiguous().view(torch.int16).numpy().tobytes()
        sock.sendall(struct.pack("<III", N, len(kb), len(vb)))
        sock.sendall(kb)
        sock.sendall(vb)

    def torch_ops_recv(sock, buf):
        def exact(n):
            parts = []
            while n:
                c = sock.recv(min(n, 1 << 22))
                parts.append(c)
                n -= len(c)
            return b"".join(parts)
        n, kl, vl = struct.unpack("<III", exact(12))
        kd, vd = exact(kl), exact(vl)
        shape = (n,) + tuple(buf.k.shape[1:])
        buf.k[:n] = torch.frombuffer(bytearray(kd), dtype=torch.int16).view(torch.bfloat16).reshape(shape)
        buf.v[:n] = torch.frombuffer(bytearray(vd), dtype=torch.int16).view(torch.bfloat16).reshape(shape)
        idx = torch.tensor(t_dst, device=dev, dtype=torch.long)
        dst[0].index_copy_(1, idx, buf.k[:n].to(dev).permute(1, 0, 2, 3, 4).contiguous())
        dst[1].index_copy_(1, idx, buf.v[:n].to(dev).permute(1, 0, 2, 3, 4).contiguous())
        torch.cuda.synchronize()

    def timed(send, recv):
        a, b = socket.socketpair()
        for sk in (a, b):
            sk.setsockopt(socket.SOL_SOCKET, socket.SO_SNDBUF, 4 << 20)
            sk.setsockopt(socket.SOL_SOCKET, socket.SO_RCVBUF, 4 << 20)
        times = []
        try:
            for _ in range(reps + 1):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                th = threading.Thread(target=send, args=(a,))
                th.start()
                recv(b)
                th.join()
                times.append(time.perf_counter() - t0)
        finally:
            a.close()
            b.close()
        return statistics.median(times[1:])

    out = {"workload": f"PD transfer of {N} blocks (48 layers, 24 MiB each) over a socketpair",
           "frame_MiB": frame_bytes / 2 ** 20}
    tx_buf = KVBlockBuffer.from_pool(src, N)
    rx_buf = KVBlockBuffer.from_pool(dst, N)
    t = timed(lambda sk: torch_ops_send(sk, tx_buf), lambda sk: torch_ops_recv(sk, rx_buf))
    out["torch_ops_ms"] = round(t * 1e3, 2)
    out["torch_ops_GBps"] = round(frame_bytes / t / 1e9, 2)
    torch_ops_dst = dst.clone()
    dst.zero_()
    for chunk in (2, 4):
        holder = {}

        def send(sk, chunk=chunk):
            if "tx" not in holder or holder["tx"].sock is not sk:
                holder["tx"] = TcpKVChannel(sk, src, N, chunk_blocks=chunk)
            holder["tx"].send_blocks(t_src)

        def recv(sk, chunk=chunk):
            if "rx" not in holder or holder["rx"].sock is not sk:
                holder["rx"] = TcpKVChannel(sk, dst, N, chunk_blocks=chunk)
            holder["rx"].recv_blocks(t_dst)
        t = timed(send, recv)
        out[f"channel_chunk{chunk}_ms"] = round(t * 1e3, 2)
        out[f"channel_chunk{chunk}_GBps"] = round(frame_bytes / t / 1e9, 2)
    out["channel_equals_torch_ops"] = bool(torch.equal(dst.view(torch.int16),
                                                       torch_ops_dst.view(torch.int16)))
    buf = KVBlockBuffer.from_pool(src, N)
    for name, fn in (("extract", lambda: extract_kv(src, t_src, buf)),
                     ("import", lambda: import_kv(dst, t_dst, buf))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / reps
        out[f"{name}_ms"] = round(t * 1e3, 2)
        out[f"{name}_GBps"] = round(frame_bytes / t / 1e9, 2)
    return out


def run_swap(args, torch):
    """Block eviction / offload step at the 48-layer 30B-A3B pool shape: a pool of 8192
    blocks of [2 (K, V), 48 layers, 256, 4 kv heads, 128] bf16 (24 MiB each,
    192 GiB; the 16384-block pool of the workload does not fit one 288 GB GPU,
    and bytes/s do not depend on the pool size), 512 active blocks chosen by a
    seeded permutation; each step copies 25 % of them (128 LRU victims) to a
    pinned host buffer, swaps 128 others back in from it, then compacts 1024
    scattered blocks in HBM."""
    from nanovllm_amd.engine.kv_runner import BlockMover
    dev = torch.device("cuda:0")
    L, kvh, pool_blocks, active, n_swap, n_copy = 48, 4, 8192, 512, 128, 1024
    pool = torch.empty(2, L, pool_blocks, 256, kvh, 128, device=dev, dtype=torch.bfloat16)
    mover = BlockMover(pool)
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    act = perm[:active]
    victims = act[:n_swap]                    # LRU-selected: the oldest quarter
    revived = perm[active:active + n_swap]    # blocks coming back from the host
    src = perm[active + n_swap:active + n_swap + n_copy]
    dst = perm[active + n_swap + n_copy:active + n_swap + 2 * n_copy]
    host_out = torch.empty((n_swap,) + mover.item_shape, dtype=pool.dtype, pin_memory=True)
    host_in = torch.empty((n_swap,) + mover.item_shape, dtype=pool.dtype, pin_memory=True)
    item = mover.item_bytes

    # Each move alone (sequential, one timer each) ...
    def step(t_d2h=None, t_h2d=None, t_cp=None):
        for t, fn in ((t_d2h, lambda: mover.d2h(victims, host_out)),
                      (t_h2d, lambda: mover.h2d(host_in, revived)),
                      (t_cp, lambda: mover.copy(src, dst))):
            s = t.start() if t else None
            fn()
            if t:
                t.stop(s)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    timers = [EventTimer(torch) for _ in range(3)]
    steps = max(3, args.steps // 10)
    for _ in range(steps):
        step(*timers)
    torch.cuda.synchronize()
    d2h, h2d, cp = (t.mean_ms() for t in timers)
    # ... and the step as the runner issues it: d2h and h2d concurrently on the
    # two directions of the link, compaction beside them (BlockMover.swap).
    mover.swap(victims, host_out, revived, host_in, src, dst)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        mover.swap(victims, host_out, revived, host_in, src, dst)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    res = {"workload": (f"offload/compaction step: pool {pool_blocks} x 24 MiB blocks "
                         f"([2, {L}, 256, {kvh}, 128] bf16), {active} active; {n_swap} blocks "
                         f"d2h + {n_swap} h2d (pinned, copy engines) + compaction copy of "
                         f"{n_copy} scattered blocks"),
            "ms_per_step_overlapped": round(wall * 1e3, 3),
            "ms_per_step_sequential": round(d2h + h2d + cp, 3),
            "d2h_ms": round(d2h, 3), "d2h_GBps": round(n_swap * item / (d2h * 1e-3) / 1e9, 1),
            "h2d_ms": round(h2d, 3), "h2d_GBps": round(n_swap * item / (h2d * 1e-3) / 1e9, 1),
            "copy_ms": round(cp, 3),
            "copy_GBps_read_plus_write": round(2 * n_copy * item / (cp * 1e-3) / 1e9, 1),
            "copy_frac_of_8TBps": round(2 * n_copy * item / (cp * 1e-3) / 8e12, 4),
            "step_GBps_moved": round((2 * n_swap + 2 * n_copy) * item / wall / 1e9, 1)}
    if not args.no_cpu_baseline:
        del host_out, host_in
        res["cpu_baseline"] = cpu_swap_baseline(torch, L, kvh)
    return res


def run_copy(args, torch):
    """Calibration: a plain contiguous device copy of known size (the
    block-copy kernel moving 512 x 256 KiB blocks = 128 MiB read + 128 MiB
    written), to scale rocprof's FETCH_SIZE / WRITE_SIZE readings."""
    from nanovllm_amd.engine.kv_runner import BlockMover
    dev = torch.device("cuda:0")
    pool = torch.zeros(1, 1, 1024, 256, 4, 128, device=dev, dtype=torch.bfloat16)
    mover = BlockMover(pool)
    src, dst = list(range(512)), list(range(512, 1024))
    for _ in range(args.warmup):
        mover.copy(src, dst)
    timer = EventTimer(torch)
    for _ in range(args.steps):
        s = timer.start()
        mover.copy(src, dst)
        timer.stop(s)
    torch.cuda.synchronize()
    ms = timer.mean_ms()
    nbytes = 512 * mover.item_bytes
    return {"workload": "calibration copy: 512 contiguous 256 KiB blocks (128 MiB read + 128 MiB "
                        "write) per launch", "read_bytes": nbytes, "write_bytes": nbytes,
            "ms": round(ms, 4), "GBps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def run_block_manager(args):
    """Host bookkeeping of the paged pool (engine/block_manager.py, the
    reference's algorithm on intrusive rings): a decode step of 64 sequences
    at context ~4096 (may_append, then the filled-block hash and the token
    append after the forward), averaged over 256 steps so every sequence
    crosses one block boundary; and admitting then freeing a 4096-token
    prompt (can_allocate, allocate, hashing its 16 blocks, deallocate).
    Host CPU only; the decode attention the step would launch is timed by
    the default workload."""
    import random
    from nanovllm_amd.engine.block_manager import BlockManager
    from nanovllm_amd.engine.sequence import Sequence
    rng = random.Random(7)
    bs = 256
    bm = BlockManager(8192, bs)
    seqs = []
    for _ in range(64):
        seq = Sequence([rng.randrange(151936) for _ in range(4096 - 3)])
        seq.block_size = bs
        bm.allocate(seq, bm.can_allocate(seq))
        seq.num_cached_tokens, seq.num_scheduled_tokens = 0, len(seq)
        bm.hash_blocks(seq)
        seq.is_prefill = False
        seqs.append(seq)
    steps = 256
    t0 = time.perf_counter()
    for _ in range(steps):
        for seq in seqs:
            bm.may_append(seq)
        for seq in seqs:
            seq.num_cached_tokens, seq.num_scheduled_tokens = len(seq) - 1, 1
            bm.hash_blocks(seq)
            seq.append_token(rng.randrange(151936))
    step_us = (time.perf_counter() - t0) / steps * 1e6
    for seq in seqs:
        bm.deallocate(seq)
    prompts = [[rng.randrange(151936) for _ in range(4096)] for _ in range(16)]
    t0 = time.perf_counter()
    for toks in prompts:
        seq = Sequence(toks)
        seq.block_size = bs
        bm.allocate(seq, bm.can_allocate(seq))
        seq.num_cached_tokens, seq.num_scheduled_tokens = 0, len(seq)
        bm.hash_blocks(seq)
        bm.deallocate(seq)
    admit_us = (time.perf_counter() - t0) / len(prompts) * 1e6
    return {"workload": "block-manager host bookkeeping (engine/block_manager.py): decode step "
                        "of 64 sequences at context ~4096; admit + free of a 4096-token prompt",
            "decode_step_us": round(step_us, 1), "prompt_admit_free_us": round(admit_us, 1),
            "host": platform_name()}


def platform_name():
    import platform
    return f"{platform.processor() or platform.machine()}, {os.cpu_count()} CPUs visible"


def main():
    args = parse_args()
    if args.workload == "block-manager":
        print(json.dumps(run_block_manager(args)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
              f"(the paged KV path has no cross-GPU exchange to measure)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    if args.workload in ("decode", "decode-dist", "decode-tp2", "decode-cold", "cfg1", "int8"):
        res = run_decode(args, torch, dist=args.workload == "decode-dist",
                         int8=args.workload == "int8")
    elif args.workload == "p15-grid":
        res = run_p15_grid(args, torch)
    elif args.workload == "int8-chan":
        res = run_int8_chan(args, torch)
    elif args.workload == "prefill-int8":
        res = run_prefill_int8(args, torch)
    elif args.workload == "prefill-scale":
        res = run_prefill_scale(args, torch)
    elif args.workload in MIXES:
        res = run_mixed(args, torch, args.workload)
    elif args.workload == "append":
        res = run_append(args, torch)
    elif args.workload == "copy":
        res = run_copy(args, torch)
    elif args.workload == "rope":
        res = run_rope(args, torch)
    elif args.workload == "decode-graph":
        res = run_decode_graph(args, torch)
    elif args.workload == "offload-overlap":
        res = run_offload_overlap(args, torch)
    elif args.workload == "pd-wire":
        res = run_pd_wire(args, torch)
    else:
        res = run_swap(args, torch)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
