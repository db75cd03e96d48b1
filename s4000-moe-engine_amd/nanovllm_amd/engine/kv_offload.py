"""Pinned host slots for KV blocks evicted from the device pool.

The slot accounting is the engine's HostBlockPool
(nanovllm/engine/kv_offload.py:31-126), which the block manager's host map
and the engine's tests depend on: `num_slots` slots of `block_shape`; the
most recently released slot is handed out first (slot 0 first in a fresh
pool); a put into a full or zero-slot pool returns -1 and counts in
full_count, never raises (checked before the shape); get / view / release of
a slot not in use raise KeyError; a shape mismatch raises ValueError;
metrics() carries the engine's keys.

Here one claim / vacate path serves both ways of filling a slot: `put`
copies a tensor (the engine's form), and the pool-direct forms move a block
between the device pool and its slot on the copy engines (a BlockMover; no
staging tensor, no host synchronisation, ordered on the current stream) —
one 2-D DMA per run of consecutive slots in the batched forms.  `reserve`
hands out slots for a caller that moves the bytes itself (the asynchronous
offloader).
"""
from __future__ import annotations

import operator

import torch

_VACANT = object()   # owner of a slot not in use


class HostBlockPool:

    def __init__(self, num_slots: int, block_shape, dtype=torch.bfloat16, pin: bool = True):
        if num_slots < 0:
            raise ValueError("num_slots must be >= 0")
        self.num_slots = int(num_slots)
        self.block_shape = tuple(block_shape)
        self.dtype = dtype
        self.pin = pin
        # device="cpu" explicitly: pinning needs a host tensor whatever the
        # ambient default device is.
        self._slots = (torch.empty((self.num_slots, *self.block_shape), dtype=dtype,
                                   device="cpu", pin_memory=pin) if self.num_slots else None)
        self._owner = [_VACANT] * self.num_slots     # caller key per slot in use
        self._stack = list(reversed(range(self.num_slots)))   # free slots, top = next
        self._live = 0
        self.puts = self.gets = self.releases = self.full_count = 0

    # -- accounting -------------------------------------------------------
    def has_room(self) -> bool:
        """Whether a put would get a slot (the runner asks before moving bytes)."""
        return self._slots is not None and len(self._stack) > 0

    def note_full(self) -> int:
        """Count a put the caller skipped because the pool had no room."""
        self.full_count += 1
        return -1

    def _claim(self) -> int:
        if not self.has_room():
            return self.note_full()
        return self._stack.pop()

    def _occupy(self, slot: int, key: object) -> None:
        self._owner[slot] = key
        self._live += 1
        self.puts += 1

    def _require(self, slot: int) -> None:
        try:
            i = operator.index(slot)
        except TypeError:
            i = -1
        if not 0 <= i < self.num_slots or self._owner[i] is _VACANT:
            raise KeyError(f"slot {slot} is not in use")

    def _require_shape(self, t: torch.Tensor, what: str) -> None:
        if tuple(t.shape) != self.block_shape:
            raise ValueError(f"{what} shape mismatch: got {tuple(t.shape)}, "
                             f"pool expects {self.block_shape}")

    # -- the engine's interface ---------------------------------------------
    def put(self, tensor: torch.Tensor, key: object = None) -> int:
        """Copy `tensor` into a free slot and return it; -1 when full."""
        if not self.has_room():
            return self.note_full()
        self._require_shape(tensor, "block")
        slot = self._claim()
        self._slots[slot].copy_(tensor)
        self._occupy(slot, key)
        return slot

    def get(self, slot: int, out: torch.Tensor):
        """Copy a slot into `out`, bit for bit; the slot stays in use."""
        self._require(slot)
        self._require_shape(out, "out")
        out.copy_(self._slots[slot])
        self.gets += 1

    def view(self, slot: int) -> torch.Tensor:
        """The pinned slot itself (counted as a get)."""
        self._require(slot)
        self.gets += 1
        return self._slots[slot]

    def release(self, slot: int):
        self._require(slot)
        slot = operator.index(slot)
        self._owner[slot] = _VACANT
        self._live -= 1
        self._stack.append(slot)
        self.releases += 1

    def metrics(self):
        return {
            "kv_offload_slots_capacity": self.num_slots,
            "kv_offload_slots_in_use": self._live,
            "kv_offload_puts_total": self.puts,
            "kv_offload_gets_total": self.gets,
            "kv_offload_releases_total": self.releases,
            "kv_offload_full_total": self.full_count,
            "kv_offload_pinned": int(bool(self.pin)),
        }

    # -- for callers that move the bytes themselves -------------------------
    @property
    def buffer(self) -> torch.Tensor | None:
        """The pinned slots [num_slots, *block_shape] (None with no slots)."""
        return self._slots

    def reserve(self, keys) -> list[int]:
        """A slot per key, in order, counted as puts (-1 for each key past the
        pool's room); the caller fills them."""
        out = []
        for key in keys:
            slot = self._claim()
            if slot != -1:
                self._occupy(slot, key)
            out.append(slot)
        return out

    def check_in_use(self, slots) -> None:
        for s in slots:
            self._require(s)

    # -- pool-direct moves (copy engines) -------------------------------------
    def _check_mover(self, mover) -> None:
        if mover.item_shape != self.block_shape or mover.pool.dtype != self.dtype:
            raise ValueError(f"pool block {mover.item_shape} {mover.pool.dtype} does not match "
                             f"slots {self.block_shape} {self.dtype}")

    @staticmethod
    def _slot_runs(pairs):
        """Group (slot, block) pairs into runs of consecutive slots (one DMA
        submission each): [(first slot, [blocks])]."""
        runs = []
        for slot, block in sorted(pairs):
            if runs and slot == runs[-1][0] + len(runs[-1][1]):
                runs[-1][1].append(block)
            else:
                runs.append((slot, [block]))
        return runs

    def put_from_pool(self, mover, block_id: int, key: object = None) -> int:
        """Move block `block_id` of the device pool into a free slot; -1 when full."""
        return self.put_many_from_pool(mover, [block_id],
                                       keys=None if key is None else [key])[0]

    def put_many_from_pool(self, mover, block_ids, keys=None) -> list[int]:
        """Batched put: blocks while there is room get slots (in order), the
        rest -1; the key of a slot is its block id unless keys are given."""
        self._check_mover(mover)
        block_ids = [int(b) for b in block_ids]
        slots = [self._claim() for _ in block_ids]
        live = [(s, b) for s, b in zip(slots, block_ids) if s != -1]
        for first, blocks in self._slot_runs(live):
            mover.d2h(blocks, self._slots[first:first + len(blocks)])
        for i, (s, b) in enumerate(zip(slots, block_ids)):
            if s != -1:
                self._occupy(s, b if keys is None else keys[i])
        return slots

    def get_into_pool(self, mover, slot: int, block_id: int) -> None:
        """Move a slot's bytes into block `block_id` of the device pool."""
        self.get_many_into_pool(mover, [slot], [block_id])

    def get_many_into_pool(self, mover, slots, block_ids) -> None:
        self._check_mover(mover)
        self.check_in_use(slots)
        for first, blocks in self._slot_runs(zip([int(s) for s in slots],
                                                 [int(b) for b in block_ids])):
            mover.h2d(self._slots[first:first + len(blocks)], blocks)
        self.gets += len(slots)
