"""Asynchronous KV offload: the HostBlockPool's puts and gets on a copy
stream, overlapped with the model's compute and fenced per layer group.

The engine's offload is blocking (nanovllm/engine/model_runner.py:284-305: a
device-wide synchronize, a gather, a pinned copy per put); its asynchronous,
double-buffered form was planned but not built (benchmarks/P30-kv-offload.md
section 1, "async + event double buffering").  Here:

* a put or a get moves each (layer group, K/V side) of its blocks straight
  between the pool and the pinned slots, either with one gather / scatter
  kernel that reads or writes the pinned memory through its device mapping
  (copy_engine="kernel"), or with one strided 2-D DMA per block on the copy
  engines (copy_engine="dma"); puts run on one stream and gets on another
  (the link is full duplex), both of default priority;
* a copy stream first waits for the work already enqueued on the compute
  stream, so a put reads the block's final contents and a get does not
  overwrite a block that earlier kernels still read;
* across the two directions: a get waits for the put that filled its slot
  and for the last put that read any of its destination blocks (the block
  manager evicts block B with a put and revives another prefix into the same
  B at once, so the scatter must not overwrite B while the gather still
  copies it); a put waits for the gets issued before it (one of them may
  still read the slot the put reuses, or still write the block it reads);
* every layer group's copies end in an event.  The compute stream waits for
  a group's events only when it reaches that group: fence_layer(l), called by
  the attention layer before it appends to or reads layer l's planes.  The
  copies of later layer groups overlap the compute of earlier layers;
* within a direction the stream is in order, so a slot released and taken
  again is never written before its previous put has finished.

Choice of engine, measured on a 48-layer decode step (batch 64 x 4096) that
offloads 8 and revives 8 blocks of 24 MiB: the DMA copies carry a large
fixed cost per submission while the compute stream is busy (about 125 us
plus a 150 us gap per 2-D copy, against 65 us for the same 3 MiB when the
GPU is otherwise idle), so finer layer groups make them slower; the kernels
(at most 64 workgroups, PCIe-bound) keep the link at 40-55 GB/s but share
CUs with the persistent decode kernel, which then runs up to 3x longer while
they overlap it.  Kernel copies in 8 layer groups cost 5.1 ms per such step
against 8.5 ms for the blocking moves.

Hazards the caller owns: host-side access to a slot's bytes (HostBlockPool
.get/.view/.put) must follow wait_host(); any device work that writes pool
blocks outside the attention layers (a compaction copy, a scatter) must
follow fence().
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _native as nat
from .kv_offload import HostBlockPool


class AsyncOffloader:
    """Offload executor over one KV pool [2, L, blocks, page, KVH, D] and a
    HostBlockPool of matching slots: put/put_many/get/get_many/release with
    the HostBlockPool's accounting (-1 past its room, KeyError on a slot not
    in use), returning before the bytes move; fence_layer/fence order the
    compute stream after them, wait_host the host.  layer_groups: how many
    contiguous layer ranges get an event of their own (8 measured best)."""

    def __init__(self, kv_cache: torch.Tensor, host_pool: HostBlockPool, layer_groups: int = 8,
                 copy_engine: str = "kernel"):
        if copy_engine not in ("kernel", "dma"):
            raise ValueError(f"copy_engine must be 'kernel' or 'dma' (got {copy_engine!r})")
        self.copy_engine = copy_engine
        if kv_cache.dim() != 6 or not kv_cache.is_contiguous():
            raise AssertionError("kv_cache must be a contiguous [2, L, blocks, page, KVH, D] pool")
        nat.require_device(kv_cache)
        if host_pool.block_shape != tuple(kv_cache[:, :, 0].shape) or \
                host_pool.dtype != kv_cache.dtype:
            raise ValueError(f"host slots {host_pool.block_shape} {host_pool.dtype} do not hold "
                             f"blocks {tuple(kv_cache[:, :, 0].shape)} {kv_cache.dtype}")
        self.kv_cache = kv_cache
        self.host_pool = host_pool
        self.num_layers = kv_cache.size(1)
        self.num_blocks = kv_cache.size(2)
        self.block_bytes = kv_cache[0, 0, 0].numel() * kv_cache.element_size()
        self.item_bytes = 2 * self.num_layers * self.block_bytes
        G = max(1, min(int(layer_groups), self.num_layers))
        edges = [round(i * self.num_layers / G) for i in range(G + 1)]
        self.groups = [(edges[i], edges[i + 1]) for i in range(G)]
        self.group_of_layer = [gi for gi, (a, b) in enumerate(self.groups) for _ in range(a, b)]
        # default priority, like the compute stream
        self.put_stream = torch.cuda.Stream(device=kv_cache.device)
        self.get_stream = torch.cuda.Stream(device=kv_cache.device)
        self._pending: list[list[torch.cuda.Event]] = [[] for _ in self.groups]
        self._slot_put_done: dict[int, torch.cuda.Event] = {}
        # last put event per source block, until a get into that block has
        # been ordered after it (the get stream is in order: later gets need
        # no wait of their own)
        self._block_put_done: dict[int, torch.cuda.Event] = {}
        self._gets_done: torch.cuda.Event | None = None
        # the compute stream is whatever stream is current at each call
        self._cur = lambda: torch.cuda.current_stream(kv_cache.device)

    # -- byte moves --------------------------------------------------------
    def _runs(self, slots, block_ids):
        """(first slot, [block ids]) for each run of consecutive slots."""
        order = sorted(range(len(slots)), key=lambda i: slots[i])
        runs, cur = [], []
        for i in order:
            if cur and slots[i] != slots[cur[-1]] + 1:
                runs.append(cur)
                cur = []
            cur.append(i)
        if cur:
            runs.append(cur)
        return [(slots[r[0]], np.ascontiguousarray([block_ids[i] for i in r], dtype=np.int64))
                for r in runs]

    def _check_ids(self, block_ids) -> None:
        for b in block_ids:
            if not 0 <= b < self.num_blocks:
                raise IndexError(f"block id {b} out of range [0, {self.num_blocks})")

    def _move(self, to_host: bool, slots, block_ids) -> None:
        runs = self._runs(slots, block_ids)
        stream = self.put_stream if to_host else self.get_stream
        if self.copy_engine == "kernel":
            # the kernels read the id lists from device memory: upload them on
            # the copy stream itself (ordered before the launches below)
            with torch.cuda.stream(stream):
                runs = [(first, ids, torch.from_numpy(ids.astype(np.int32)).pin_memory()
                         .to(self.kv_cache.device, non_blocking=True)) for first, ids in runs]
        else:
            runs = [(first, ids, None) for first, ids in runs]
        pool_base = self.kv_cache.data_ptr()
        host_base = self.host_pool.buffer.data_ptr()
        L, bb = self.num_layers, self.block_bytes
        plane_stride = self.num_blocks * bb
        sid = stream.cuda_stream
        stream.wait_stream(self._cur())
        if to_host:
            if self._gets_done is not None:
                stream.wait_event(self._gets_done)
        else:
            waits = {self._slot_put_done.get(s) for s in set(slots)}
            waits |= {self._block_put_done.pop(b, None) for b in set(block_ids)}
            waits.discard(None)
            for ev in waits:
                stream.wait_event(ev)
        ev = None
        for gi, (l0, l1) in enumerate(self.groups):
            for side in (0, 1):
                plane0 = side * L + l0  # the group's first plane, in pool and slot alike
                pool_ptr = pool_base + plane0 * plane_stride
                for first_slot, ids, dev_ids in runs:
                    host_ptr = host_base + first_slot * self.item_bytes + plane0 * bb
                    if dev_ids is not None and to_host:
                        nat.call("kvc_block_gather", pool_ptr, l1 - l0, plane_stride, bb,
                                 dev_ids.data_ptr(), len(ids), host_ptr, self.item_bytes, bb, sid)
                    elif dev_ids is not None:
                        nat.call("kvc_block_scatter", host_ptr, self.item_bytes, bb, l1 - l0, bb,
                                 dev_ids.data_ptr(), len(ids), pool_ptr, plane_stride, sid)
                    elif to_host:
                        nat.call("kvc_block_d2h", pool_ptr, l1 - l0, plane_stride, bb,
                                 ids.ctypes.data, len(ids), host_ptr, self.item_bytes, sid)
                    else:
                        nat.call("kvc_block_h2d", host_ptr, self.item_bytes, l1 - l0, bb,
                                 ids.ctypes.data, len(ids), pool_ptr, plane_stride, sid)
            ev = torch.cuda.Event()
            ev.record(stream)
            self._pending[gi].append(ev)
        if to_host:
            for s in slots:
                self._slot_put_done[s] = ev
            for b in block_ids:
                self._block_put_done[b] = ev
        else:
            self._gets_done = ev

    # -- the offload executor protocol, asynchronous ------------------------
    def put_many(self, block_ids) -> list[int]:
        """Offload blocks to free slots (-1 for each block past the pool's
        room, which moves nothing); returns at once."""
        block_ids = [int(b) for b in block_ids]
        self._check_ids(block_ids)
        slots = self.host_pool.reserve(block_ids)
        live = [(s, b) for s, b in zip(slots, block_ids) if s != -1]
        if live:
            self._move(True, [s for s, _ in live], [b for _, b in live])
        return slots

    def put(self, block_id: int) -> int:
        return self.put_many([block_id])[0]

    def get_many(self, slots, block_ids) -> None:
        """Bring slots back into the named blocks; returns at once (the
        blocks are valid for compute after fence_layer / fence)."""
        slots = [int(s) for s in slots]
        block_ids = [int(b) for b in block_ids]
        if len(slots) != len(block_ids):
            raise ValueError("slots and block_ids differ in length")
        self._check_ids(block_ids)
        self.host_pool.check_in_use(slots)
        if slots:
            self._move(False, slots, block_ids)
        self.host_pool.gets += len(slots)

    def get(self, slot: int, block_id: int) -> None:
        self.get_many([slot], [block_id])

    def release(self, slot: int) -> None:
        self.host_pool.release(slot)
        self._slot_put_done.pop(slot, None)

    # -- ordering ------------------------------------------------------------
    def fence_layer(self, layer: int) -> None:
        """Make the compute stream wait for the copies of `layer`'s group
        (device-side wait; the host does not block).

        The wait is enqueued from Python, so it exists only in eager
        execution: a graph captured over the attention layers would replay
        without it.  Under capture, with copies still pending, this raises
        RuntimeError; a caller that replays graphs calls fence() on the
        compute stream before each replay, outside the graph."""
        pending = self._pending[self.group_of_layer[layer]]
        if pending:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "async KV offload copies are pending while a graph is being captured: "
                    "the per-layer fence would not be replayed; call fence() before the "
                    "capture and before every replay")
            cur = self._cur()
            for ev in pending:
                cur.wait_event(ev)
            pending.clear()

    def fence(self) -> None:
        for layer0, _ in self.groups:
            self.fence_layer(layer0)

    def wait_host(self) -> None:
        """Block the host until every copy issued so far has finished."""
        self.put_stream.synchronize()
        self.get_stream.synchronize()
        for p in self._pending:
            p.clear()  # finished: later compute needs no wait for them
        self._block_put_done.clear()
        self._slot_put_done.clear()

    def in_flight(self) -> bool:
        return any(not ev.query() for p in self._pending for ev in p)
