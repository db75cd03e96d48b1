"""KV pool allocation and whole-block byte movement (the runner's KV slices).

Mirrors the parts of nanovllm/engine/model_runner.py that own the KV pool:
  allocate_kv_cache   :400-508   pool [2, L, blocks + 1, page, KVH, D] (the
                                  extra block is the graph-padding scratch
                                  block), per-layer views handed to every
                                  module with k_cache/v_cache
  offload_put/get/release :284-308  byte moves behind the BlockManager's
                                  executor protocol call(name, *args)
and adds the batched forms a swap/compaction step needs (one launch or one
DMA submission for a whole id list).

Differences from the reference, all on the byte path:
  * no device-wide synchronize() before a snapshot (model_runner.py:294):
    every move is ordered on the current stream after the kernels that wrote
    the block, and before any later kernel that overwrites it;
  * the block is copied straight from the pool into the pinned slot by the
    copy engines (one strided 2-D copy per block), without the index_select
    staging tensor.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _native as nat
from ..utils.context import set_context


class BlockMover:
    """Whole-block moves on a pool shaped [P0, P1, blocks, ...] (block axis 2),
    i.e. the engine's [2, L, blocks, page, KVH, D] KV pool or its int8 scale /
    side-pool companions.  A block is P0*P1 planes of block_bytes."""

    def __init__(self, pool: torch.Tensor):
        if pool.dim() < 3:
            raise ValueError("pool must be [P0, P1, blocks, ...]")
        if not pool.is_contiguous():
            raise AssertionError("the KV pool must be contiguous")
        nat.require_device(pool)
        self.pool = pool
        self.planes = pool.size(0) * pool.size(1)
        self.num_blocks = pool.size(2)
        self.item_shape = tuple(pool.shape[:2]) + tuple(pool.shape[3:])
        self.block_bytes = pool[0, 0, 0].numel() * pool.element_size()
        self.plane_stride = self.num_blocks * self.block_bytes
        self.item_bytes = self.planes * self.block_bytes

    # -- helpers ---------------------------------------------------------
    def _dev_ids(self, ids) -> torch.Tensor:
        if isinstance(ids, torch.Tensor):
            t = ids.to(device=self.pool.device, dtype=torch.int32)
        else:
            t = torch.as_tensor(list(ids), dtype=torch.int32).to(self.pool.device, non_blocking=True)
        return t.contiguous()

    def _host_ids(self, ids) -> np.ndarray:
        if isinstance(ids, torch.Tensor):
            ids = ids.tolist()
        arr = np.ascontiguousarray(np.asarray(list(ids), dtype=np.int64))
        if arr.size and (arr.min() < 0 or arr.max() >= self.num_blocks):
            raise IndexError(f"block id out of range [0, {self.num_blocks})")
        return arr

    def _check_items(self, t: torch.Tensor, n: int) -> None:
        if tuple(t.shape) != (n,) + self.item_shape or t.dtype != self.pool.dtype:
            raise ValueError(f"expected [{n}, {self.item_shape}] {self.pool.dtype}, got "
                             f"{tuple(t.shape)} {t.dtype}")
        if not t.is_contiguous():
            raise AssertionError("staging buffer must be contiguous")

    def _stream(self) -> int:
        return nat.stream_of(self.pool)

    # -- kernels ---------------------------------------------------------
    def gather(self, ids, out: torch.Tensor | None = None) -> torch.Tensor:
        """out[i] = pool[:, :, ids[i]] (out on the device or pinned host)."""
        n = len(ids)
        if out is None:
            out = torch.empty((n,) + self.item_shape, dtype=self.pool.dtype,
                              device=self.pool.device)
        self._check_items(out, n)
        if n == 0:
            return out
        dev_ids = self._dev_ids(ids)
        nat.call("kvc_block_gather", self.pool.data_ptr(), self.planes, self.plane_stride,
                 self.block_bytes, dev_ids.data_ptr(), n, out.data_ptr(), self.item_bytes,
                 self.block_bytes, self._stream())
        return out

    def scatter(self, items: torch.Tensor, ids) -> None:
        """pool[:, :, ids[i]] = items[i] (items on the device or pinned host)."""
        n = len(ids)
        self._check_items(items, n)
        if n == 0:
            return
        dev_ids = self._dev_ids(ids)
        nat.call("kvc_block_scatter", items.data_ptr(), self.item_bytes, self.block_bytes,
                 self.planes, self.block_bytes, dev_ids.data_ptr(), n, self.pool.data_ptr(),
                 self.plane_stride, self._stream())

    def copy(self, src_ids, dst_ids) -> None:
        """pool[:, :, dst] = pool[:, :, src] as one simultaneous copy; id lists
        that overlap go through a device staging buffer."""
        src = [int(x) for x in (src_ids.tolist() if isinstance(src_ids, torch.Tensor) else src_ids)]
        dst = [int(x) for x in (dst_ids.tolist() if isinstance(dst_ids, torch.Tensor) else dst_ids)]
        if len(src) != len(dst):
            raise ValueError("src_ids and dst_ids differ in length")
        if not src:
            return
        if len(set(dst)) != len(dst):
            raise ValueError("duplicate destination block")
        if set(src) & set(dst):
            staged = self.gather(src)
            self.scatter(staged, dst)
            return
        s, d = self._dev_ids(src), self._dev_ids(dst)
        nat.call("kvc_block_copy", self.pool.data_ptr(), self.planes, self.plane_stride,
                 self.block_bytes, s.data_ptr(), d.data_ptr(), len(src), self._stream())

    # -- copy engines ----------------------------------------------------
    def d2h(self, ids, host: torch.Tensor) -> None:
        """host[i] = pool[:, :, ids[i]] by DMA (host must be pinned)."""
        ids_np = self._host_ids(ids)
        self._check_items(host, len(ids_np))
        if not host.is_pinned():
            raise ValueError("the host staging buffer must be pinned")
        if len(ids_np) == 0:
            return
        nat.call("kvc_block_d2h", self.pool.data_ptr(), self.planes, self.plane_stride,
                 self.block_bytes, ids_np.ctypes.data, len(ids_np), host.data_ptr(),
                 self.item_bytes, self._stream())

    def h2d(self, host: torch.Tensor, ids) -> None:
        """pool[:, :, ids[i]] = host[i] by DMA (host must be pinned)."""
        ids_np = self._host_ids(ids)
        self._check_items(host, len(ids_np))
        if not host.is_pinned():
            raise ValueError("the host staging buffer must be pinned")
        if len(ids_np) == 0:
            return
        nat.call("kvc_block_h2d", host.data_ptr(), self.item_bytes, self.planes,
                 self.block_bytes, ids_np.ctypes.data, len(ids_np), self.pool.data_ptr(),
                 self.plane_stride, self._stream())


    # -- overlapped offload step ------------------------------------------
    def _side_streams(self):
        if getattr(self, "_sides", None) is None:
            dev = self.pool.device
            # default priority (equal to the current stream's)
            self._sides = (torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev))
        return self._sides

    def swap(self, out_ids, host_out: torch.Tensor, in_ids, host_in: torch.Tensor,
             compact_src=None, compact_dst=None) -> None:
        """One offload step with its byte moves overlapped: host_out[i] =
        pool[:, :, out_ids[i]] (device -> host) and pool[:, :, in_ids[j]] =
        host_in[j] (host -> device) run concurrently on two copy-engine streams
        (the link is full duplex), and the optional compaction copy
        pool[:, :, compact_dst] = pool[:, :, compact_src] runs on the current
        stream beside them.  The four id sets must be pairwise disjoint (the
        moves are unordered with respect to each other); all of them are
        ordered after the work already on the current stream, and the current
        stream waits for them before anything it runs next."""
        outs = [int(x) for x in (out_ids.tolist() if isinstance(out_ids, torch.Tensor) else out_ids)]
        ins = [int(x) for x in (in_ids.tolist() if isinstance(in_ids, torch.Tensor) else in_ids)]
        cs = [] if compact_src is None else [int(x) for x in compact_src]
        cd = [] if compact_dst is None else [int(x) for x in compact_dst]
        sets = [set(outs), set(ins), set(cs), set(cd)]
        total = sum(len(x) for x in sets)
        if total != len(set().union(*sets)) or len(outs) != len(sets[0]) or len(ins) != len(sets[1]):
            raise ValueError("swap: the out, in and compaction id sets must be disjoint")
        cur = torch.cuda.current_stream(self.pool.device)
        s_out, s_in = self._side_streams()
        s_out.wait_stream(cur)
        s_in.wait_stream(cur)
        with torch.cuda.stream(s_out):
            self.d2h(outs, host_out)
        with torch.cuda.stream(s_in):
            self.h2d(host_in, ins)
        if cs:
            self.copy(cs, cd)
        cur.wait_stream(s_out)
        cur.wait_stream(s_in)


class KVCacheRunner:
    """The runner's KV duties for one rank: the pool, its per-layer views, and
    the offload executor protocol the BlockManager drives through call()."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, dtype=torch.bfloat16, device="cuda", kv_int8: str | None = None,
                 kv_offload_host_blocks: int = 0, n_out_max: int = 8,
                 async_offload_groups: int = 0, async_copy_engine: str = "kernel"):
        if kv_offload_host_blocks:
            # nanovllm/config.py:75-78: a block's int8 codes would travel
            # without their scales and side pool
            assert kv_int8 is None, (
                "KV offload requires the bf16 KV cache (int8 carries side-channel scales)")
            assert kv_offload_host_blocks >= 0
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kvcache_blocks = num_blocks
        self.kv_int8 = kv_int8
        # one extra block the BlockManager never sees (graph-padding scratch)
        shape = (2, num_layers, num_blocks + 1, block_size, num_kv_heads, head_dim)
        self.kv_cache = torch.empty(shape, dtype=torch.int8 if kv_int8 else dtype, device=device)
        self.kv_scales = self.kv_dscales = self.kv_side = None
        self.kv_out_idx2d = self.kv_head_n_out = None
        if kv_int8 == "tokhead":
            self.kv_scales = torch.ones(shape[:5], dtype=torch.float32, device=device)
        elif kv_int8 == "chan":
            self.kv_scales = torch.ones(2, num_layers, num_kv_heads, head_dim,
                                        dtype=torch.float32, device=device)
            self.kv_dscales = torch.ones_like(self.kv_scales)
            self.kv_side = torch.zeros(2, num_layers, num_blocks + 1, block_size, num_kv_heads,
                                       n_out_max, dtype=torch.bfloat16, device=device)
            self.kv_out_idx2d = torch.zeros(num_layers, num_kv_heads, n_out_max,
                                            dtype=torch.int32, device=device)
            self.kv_head_n_out = torch.zeros(num_layers, num_kv_heads, dtype=torch.int32,
                                             device=device)
        elif kv_int8 is not None:
            raise ValueError(f"kv_int8 must be None, 'tokhead' or 'chan' (got {kv_int8!r})")
        self.scratch_block_id = num_blocks
        self.scratch_slot = num_blocks * block_size
        self.mover = BlockMover(self.kv_cache)
        self.kv_offload_host_blocks = kv_offload_host_blocks
        self.kv_offloader = None
        # async_offload_groups > 0: offload moves run on copy streams
        # (AsyncOffloader, 8 groups recommended), fenced per layer group by the
        # bound attention layers.
        self.async_offload = async_offload_groups > 0
        self.async_offload_groups = async_offload_groups
        self.async_copy_engine = async_copy_engine
        self.kv_async = None
        self._calib = None     # (amax [L, 2, KVH, D], abs_sum, token counts) while calibrating

    def bind(self, modules) -> int:
        """Hand per-layer views to every module that has k_cache/v_cache
        (model_runner.py:494-508); returns the number of layers bound."""
        layer = 0
        for m in modules:
            if not (hasattr(m, "k_cache") and hasattr(m, "v_cache")):
                continue
            m.k_cache = self.kv_cache[0, layer]
            m.v_cache = self.kv_cache[1, layer]
            if self.kv_int8 == "tokhead":
                m.k_scale = self.kv_scales[0, layer]
                m.v_scale = self.kv_scales[1, layer]
            elif self.kv_int8 == "chan":
                m.k_scale = self.kv_scales[0, layer]
                m.v_scale = self.kv_scales[1, layer]
                m.k_dscale = self.kv_dscales[0, layer]
                m.v_dscale = self.kv_dscales[1, layer]
                m.side_k = self.kv_side[0, layer]
                m.side_v = self.kv_side[1, layer]
                m.out_idx2d = self.kv_out_idx2d[layer]
                m.head_n_out = self.kv_head_n_out[layer]
            m.kv_cache_is_int8 = self.kv_int8 is not None
            m.kv_layer = layer
            m.kv_fence = self._fence_layer if self.async_offload else None
            m.kv_observe = self._observe if self.kv_int8 == "chan" else None
            layer += 1
        return layer

    # -- per-channel int8 calibration (model_runner.py:510-577) ---------------
    def kv_calibrate_begin(self) -> None:
        """Start collecting per-channel |K| / |V| statistics in every bound
        layer's forwards (running max and running sum over all calibration
        tokens, on the device)."""
        if self.kv_int8 != "chan":
            raise ValueError("calibration is for the per-channel int8 pool (kv_int8='chan')")
        _, L, _, _, KVH, D = self.kv_cache.shape
        amax = torch.zeros(L, 2, KVH, D, dtype=torch.float32, device=self.device)
        self._calib = (amax, torch.zeros_like(amax), [0] * L)

    def _observe(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        if self._calib is None:
            return
        from ..kernels.kv_int8 import kv_calib_observe
        amax, abs_sum, counts = self._calib
        KVH, D = self.kv_cache.shape[-2:]
        k3, v3 = k.view(-1, KVH, D), v.view(-1, KVH, D)
        kv_calib_observe(k3, v3, amax[layer], abs_sum[layer])
        counts[layer] += k3.size(0)

    def kv_calibrate_freeze(self) -> dict:
        """Freeze the statistics into store scales (amax / 127), read scales
        (0 at outlier dims), out_idx2d and head_n_out (K/V joint ratio
        amax / mean|x| > 10, at most n_out_max dims per head), on the device;
        returns the reference's summary (outlier dims, scale range)."""
        from ..kernels.kv_int8 import kv_calib_freeze
        if self._calib is None:
            raise RuntimeError("kv_calibrate_freeze without kv_calibrate_begin")
        amax, abs_sum, counts = self._calib
        self._calib = None
        for layer, n in enumerate(counts):
            assert n > 0, "calibration saw no activations"
            kv_calib_freeze(amax[layer], abs_sum[layer], n, self.kv_scales[0, layer],
                            self.kv_scales[1, layer], self.kv_dscales[0, layer],
                            self.kv_dscales[1, layer], self.kv_out_idx2d[layer],
                            self.kv_head_n_out[layer])
        summary = {"outlier_dims": int(self.kv_head_n_out.sum()),
                   "scale_min": float(self.kv_scales.min()),
                   "scale_max": float(self.kv_scales.max())}
        print(f"[kv-int8] mixed-precision scales frozen (bf16 outlier dims: "
              f"{summary['outlier_dims']}, scale range [{summary['scale_min']:.4g}, "
              f"{summary['scale_max']:.4g}])", flush=True)
        return summary

    # -- executor protocol (BlockManager -> runner) ------------------------
    def call(self, method: str, *args):
        return getattr(self, method)(*args)

    def _ensure_offloader(self):
        from .kv_offload import HostBlockPool
        if self.kv_offloader is None:
            self.kv_offloader = HostBlockPool(self.kv_offload_host_blocks,
                                              tuple(self.kv_cache[:, :, 0].shape),
                                              dtype=self.kv_cache.dtype)
            if self.async_offload and self.kv_offloader.buffer is not None:
                from .offload_pipeline import AsyncOffloader
                self.kv_async = AsyncOffloader(self.kv_cache, self.kv_offloader,
                                               self.async_offload_groups, self.async_copy_engine)
        return self.kv_offloader

    def _fence_layer(self, layer: int) -> None:
        if self.kv_async is not None:
            self.kv_async.fence_layer(layer)

    def fence(self) -> None:
        """Order the compute stream after every offload copy issued so far
        (needed before pool writes outside the attention layers)."""
        if self.kv_async is not None:
            self.kv_async.fence()

    def offload_put(self, block_id: int) -> int:
        pool = self._ensure_offloader()
        if not pool.has_room():
            return pool.note_full()
        if self.kv_async is not None:
            return self.kv_async.put(block_id)
        return pool.put_from_pool(self.mover, block_id)

    def offload_get(self, slot: int, block_id: int) -> None:
        pool = self._ensure_offloader()
        if self.kv_async is not None:
            return self.kv_async.get(slot, block_id)
        pool.get_into_pool(self.mover, slot, block_id)

    def offload_release(self, slot: int) -> None:
        self._ensure_offloader().release(slot)

    # -- batched forms ---------------------------------------------------
    def offload_put_many(self, block_ids) -> list[int]:
        pool = self._ensure_offloader()
        if self.kv_async is not None:
            return self.kv_async.put_many(block_ids)
        return pool.put_many_from_pool(self.mover, block_ids)

    def offload_get_many(self, slots, block_ids) -> None:
        pool = self._ensure_offloader()
        if self.kv_async is not None:
            return self.kv_async.get_many(slots, block_ids)
        pool.get_many_into_pool(self.mover, slots, block_ids)

    def compact(self, src_ids, dst_ids) -> None:
        self.fence()
        self.mover.copy(src_ids, dst_ids)

    # -- batch preparation (the Context producer) ----------------------------
    @property
    def device(self) -> torch.device:
        return self.kv_cache.device

    def _h2d(self, values, dtype) -> torch.Tensor:
        return torch.tensor(values, dtype=dtype, pin_memory=True).to(self.device, non_blocking=True)

    def prepare_block_tables(self, seqs) -> torch.Tensor:
        """int32 [len(seqs), max blocks] padded with -1 (model_runner.py:579-583)."""
        width = max(len(seq.block_table) for seq in seqs)
        rows = [seq.block_table + [-1] * (width - len(seq.block_table)) for seq in seqs]
        return self._h2d(rows, torch.int32)

    def prepare_decode(self, seqs):
        """One token per sequence at position len - 1 (model_runner.py:676-699):
        slot = block_table[-1] * block_size + last_block_num_tokens - 1."""
        input_ids = [seq.last_token for seq in seqs]
        positions = [len(seq) - 1 for seq in seqs]
        lens = [len(seq) for seq in seqs]
        slots = [seq.block_table[-1] * self.block_size + seq.last_block_num_tokens - 1
                 for seq in seqs]
        set_context(False, slot_mapping=self._h2d(slots, torch.int32),
                    context_lens=self._h2d(lens, torch.int32),
                    block_tables=self.prepare_block_tables(seqs), max_context_len=max(lens))
        return self._h2d(input_ids, torch.int64), self._h2d(positions, torch.int64)

    def prepare_prefill(self, seqs):
        return self._prepare_rows(seqs, mixed=False)

    def prepare_mixed(self, seqs):
        """Decode rows first, then prefill chunks (model_runner.py:587-674);
        ValueError when the rows are not contiguous decode-first."""
        return self._prepare_rows(seqs, mixed=True)

    def _prepare_rows(self, seqs, mixed: bool):
        bs = self.block_size
        n_dec = 0
        dec_lens: list[int] = []
        if mixed:
            while n_dec < len(seqs) and not seqs[n_dec].is_prefill:
                dec_lens.append(len(seqs[n_dec]))
                n_dec += 1
            if not all(seq.is_prefill for seq in seqs[n_dec:]):
                raise ValueError("mixed batch rows not contiguous decode-first")
        input_ids: list[int] = []
        positions: list[int] = []
        cu_q, cu_k = [0], [0]
        max_q = max_k = 0
        slots: list[int] = []
        for seq in seqs:
            start = seq.num_cached_tokens
            end = start + seq.num_scheduled_tokens
            if seq.is_prefill:
                input_ids.extend(seq[start:end])
                cu_q.append(cu_q[-1] + end - start)
                cu_k.append(cu_k[-1] + end)
                max_q, max_k = max(max_q, end - start), max(max_k, end)
            else:
                assert end - start == 1
                input_ids.append(seq.last_token)
                if not mixed:
                    dec_lens.append(len(seq))
                    cu_q.append(cu_q[-1] + 1)
                    cu_k.append(cu_k[-1] + end)
                    max_q, max_k = max(max_q, 1), max(max_k, end)
            positions.extend(range(start, end))
            if not seq.block_table:
                continue
            # slots of positions start .. end-1 through the block table
            for pos in range(start, end):
                slots.append(seq.block_table[pos // bs] * bs + pos % bs)
        block_tables = None
        if mixed or cu_k[-1] > cu_q[-1]:
            block_tables = self.prepare_block_tables(seqs)
        cu_q_t = self._h2d(cu_q, torch.int32)
        cu_k_t = self._h2d(cu_k, torch.int32)
        slot_t = self._h2d(slots, torch.int32)
        if mixed:
            set_context(True, cu_q_t, cu_k_t, max_q, max_k, slot_t, None, block_tables,
                        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k, is_mixed=True,
                        num_decode_rows=n_dec,
                        decode_context_lens=self._h2d(dec_lens, torch.int32),
                        decode_max_context_len=max(dec_lens) if dec_lens else 0,
                        decode_context_lens_list=dec_lens)
        else:
            set_context(True, cu_q_t, cu_k_t, max_q, max_k, slot_t, None, block_tables,
                        cu_seqlens_q_list=cu_q, cu_seqlens_k_list=cu_k)
        return self._h2d(input_ids, torch.int64), self._h2d(positions, torch.int64)
