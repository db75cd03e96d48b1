"""Pinned host slot pool for evicted KV blocks.

Same API and accounting as nanovllm/engine/kv_offload.py:31-126 — put/get/
view/release/has_room/note_full/metrics, LIFO slot reuse, -1 (never an
exception) when the pool is full or disabled, ValueError on a shape mismatch,
KeyError on a slot not in use — plus pool-direct forms that move a block
between the device KV pool and a slot on the copy engines (no staging tensor,
no host synchronisation; ordering is the current stream's).
"""
from __future__ import annotations

import torch


class HostBlockPool:

    def __init__(self, num_slots: int, block_shape, dtype=torch.bfloat16, pin: bool = True):
        if num_slots < 0:
            raise ValueError("num_slots must be >= 0")
        self.num_slots = int(num_slots)
        self.block_shape = tuple(block_shape)
        self.dtype = dtype
        self.pin = pin
        self._buf = None
        if self.num_slots:
            self._buf = torch.empty((self.num_slots, *self.block_shape), dtype=dtype,
                                    device="cpu", pin_memory=pin)
        # LIFO: the most recently released slot is reused first.
        self._free = list(range(self.num_slots - 1, -1, -1))
        self._in_use: dict[int, object] = {}
        self.puts = 0
        self.gets = 0
        self.releases = 0
        self.full_count = 0

    def has_room(self) -> bool:
        return self._buf is not None and bool(self._free)

    def note_full(self) -> int:
        self.full_count += 1
        return -1

    def _take_slot(self):
        if not self.has_room():
            self.full_count += 1
            return -1
        return self._free.pop()

    def put(self, tensor: torch.Tensor, key: object = None) -> int:
        """Copy `tensor` into a free slot; -1 when full or disabled."""
        if self._buf is None or not self._free:
            self.full_count += 1
            return -1
        if tuple(tensor.shape) != self.block_shape:
            raise ValueError(f"block shape mismatch: got {tuple(tensor.shape)}, "
                             f"pool expects {self.block_shape}")
        slot = self._free.pop()
        self._buf[slot].copy_(tensor)
        self._in_use[slot] = key
        self.puts += 1
        return slot

    def get(self, slot: int, out: torch.Tensor):
        """Copy a slot into `out` (bitwise; the slot stays valid)."""
        if slot not in self._in_use:
            raise KeyError(f"slot {slot} is not in use")
        if tuple(out.shape) != self.block_shape:
            raise ValueError(f"out shape mismatch: got {tuple(out.shape)}, "
                             f"pool expects {self.block_shape}")
        out.copy_(self._buf[slot])
        self.gets += 1

    def view(self, slot: int) -> torch.Tensor:
        if slot not in self._in_use:
            raise KeyError(f"slot {slot} is not in use")
        self.gets += 1
        return self._buf[slot]

    def release(self, slot: int):
        if slot not in self._in_use:
            raise KeyError(f"slot {slot} is not in use")
        del self._in_use[slot]
        self._free.append(slot)
        self.releases += 1

    # -- slot reservation for callers that move the bytes themselves ---------
    def reserve(self, keys) -> list[int]:
        """A slot for each key, in order (-1 once the pool is full), counted
        as puts; the caller fills the slots."""
        slots = []
        for key in keys:
            slot = self._take_slot()
            if slot != -1:
                self._in_use[slot] = key
                self.puts += 1
            slots.append(slot)
        return slots

    def check_in_use(self, slots) -> None:
        for s in slots:
            if s not in self._in_use:
                raise KeyError(f"slot {s} is not in use")

    @property
    def buffer(self) -> torch.Tensor | None:
        """The pinned slots [num_slots, *block_shape] (None when disabled)."""
        return self._buf

    # -- pool-direct moves (copy engines) ------------------------------------
    def _check_mover(self, mover) -> None:
        if mover.item_shape != self.block_shape or mover.pool.dtype != self.dtype:
            raise ValueError(f"pool block {mover.item_shape} {mover.pool.dtype} does not match "
                             f"slots {self.block_shape} {self.dtype}")

    def put_from_pool(self, mover, block_id: int, key: object = None) -> int:
        """DMA block `block_id` of the device pool into a free slot; -1 when full."""
        self._check_mover(mover)
        slot = self._take_slot()
        if slot == -1:
            return -1
        mover.d2h([block_id], self._buf[slot:slot + 1])
        self._in_use[slot] = block_id if key is None else key
        self.puts += 1
        return slot

    def put_many_from_pool(self, mover, block_ids) -> list[int]:
        """Batched put: as many blocks as there are free slots move in one
        submission per contiguous slot run; the rest get -1."""
        self._check_mover(mover)
        slots = [self._take_slot() for _ in block_ids]
        pairs = [(s, b) for s, b in zip(slots, block_ids) if s != -1]
        # Contiguous slot runs become one d2h call each (LIFO hands out
        # ascending runs from a fresh pool).
        run: list[tuple[int, int]] = []
        for s, b in pairs + [(None, None)]:
            if run and (s is None or s != run[-1][0] + 1):
                first = run[0][0]
                mover.d2h([x[1] for x in run], self._buf[first:first + len(run)])
                run = []
            if s is not None:
                run.append((s, b))
        for s, b in pairs:
            self._in_use[s] = b
            self.puts += 1
        return slots

    def get_into_pool(self, mover, slot: int, block_id: int) -> None:
        """DMA slot contents into block `block_id` of the device pool."""
        self._check_mover(mover)
        if slot not in self._in_use:
            raise KeyError(f"slot {slot} is not in use")
        mover.h2d(self._buf[slot:slot + 1], [block_id])
        self.gets += 1

    def get_many_into_pool(self, mover, slots, block_ids) -> None:
        self._check_mover(mover)
        for s in slots:
            if s not in self._in_use:
                raise KeyError(f"slot {s} is not in use")
        order = sorted(range(len(slots)), key=lambda i: slots[i])
        run: list[int] = []
        for i in order + [None]:
            if run and (i is None or slots[i] != slots[run[-1]] + 1):
                first = slots[run[0]]
                mover.h2d(self._buf[first:first + len(run)], [block_ids[j] for j in run])
                run = []
            if i is not None:
                run.append(i)
        self.gets += len(slots)

    def metrics(self):
        return {
            "kv_offload_slots_capacity": self.num_slots,
            "kv_offload_slots_in_use": len(self._in_use),
            "kv_offload_puts_total": self.puts,
            "kv_offload_gets_total": self.gets,
            "kv_offload_releases_total": self.releases,
            "kv_offload_full_total": self.full_count,
            "kv_offload_pinned": 1 if self.pin else 0,
        }
