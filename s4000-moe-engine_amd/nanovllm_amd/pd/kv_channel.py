"""Block-granular KV export/import between a device pool and pinned staging.

Same API as nanovllm/pd/kv_channel.py:28-82 — KVBlockBuffer (pinned k/v
[n_blocks, L, block_size, kv_heads, head_dim]), extract_kv(kv_cache,
block_table, buf), import_kv(kv_cache, block_table, buf) — with the byte
moves done by libkvc: one gather kernel per pool writes straight into the
pinned buffer (no index_select temporary, no permute copy, no device-wide
synchronise), and one scatter kernel reads it back.  The round trip is a
bitwise copy.  Below them: LocalKVChannel, TcpKVChannel and KVFrameAssembler
with the engine's frame format (kv_channel.py:85-220), sent from and received
into the pinned staging rows without host copies.
"""
from __future__ import annotations

import struct

import torch

from ..engine.kv_runner import BlockMover


class KVBlockBuffer:
    """Pinned staging for n whole blocks: k/v [n_blocks, L, block_size, kv_heads, head_dim]."""

    def __init__(self, n_blocks: int, n_layers: int, block_size: int, kv_heads: int,
                 head_dim: int, dtype=torch.bfloat16):
        shape = (n_blocks, n_layers, block_size, kv_heads, head_dim)
        self.k = torch.empty(shape, dtype=dtype, pin_memory=True)
        self.v = torch.empty(shape, dtype=dtype, pin_memory=True)
        self.n_blocks = n_blocks

    @classmethod
    def from_pool(cls, kv_cache: torch.Tensor, n_blocks: int) -> "KVBlockBuffer":
        _, n_layers, _, block_size, kv_heads, head_dim = kv_cache.shape
        return cls(n_blocks, n_layers, block_size, kv_heads, head_dim, dtype=kv_cache.dtype)

    @property
    def nbytes(self) -> int:
        return self.k.element_size() * self.k.numel() + self.v.element_size() * self.v.numel()


def _movers(kv_cache: torch.Tensor):
    # kv_cache[0:1] / kv_cache[1:2] are the K and V pools as [1, L, blocks, ...].
    return BlockMover(kv_cache[0:1]), BlockMover(kv_cache[1:2])


def _items(t: torch.Tensor, n: int) -> torch.Tensor:
    # [n, L, bs, kvh, d] staging viewed as the mover's [n, 1, L, bs, kvh, d] items
    return t[:n].unsqueeze(1)


def extract_kv(kv_cache: torch.Tensor, block_table: list[int], buf: KVBlockBuffer,
               sync: bool = True) -> None:
    """buf.k[i] / buf.v[i] = the blocks block_table[i] of the K / V pools.

    Like the reference's blocking pinned copy, the call returns with the
    bytes in `buf` (it waits for the current stream); sync=False leaves the
    copy in flight, ordered on the current stream."""
    assert len(block_table) <= buf.n_blocks
    n = len(block_table)
    mk, mv = _movers(kv_cache)
    mk.gather(block_table, out=_items(buf.k, n))
    mv.gather(block_table, out=_items(buf.v, n))
    if sync and n:
        torch.cuda.current_stream(kv_cache.device).synchronize()


def import_kv(kv_cache: torch.Tensor, block_table: list[int], buf: KVBlockBuffer,
              sync: bool = True) -> None:
    """Blocks block_table[i] of the K / V pools = buf.k[i] / buf.v[i].

    Returns once `buf` may be reused by the host (sync=False: the kernels
    may still be reading it)."""
    assert len(block_table) <= buf.n_blocks
    n = len(block_table)
    mk, mv = _movers(kv_cache)
    mk.scatter(_items(buf.k, n), block_table)
    mv.scatter(_items(buf.v, n), block_table)
    if sync and n:
        torch.cuda.current_stream(kv_cache.device).synchronize()


# ---------------------------------------------------------------------------
# Channels and the wire format (nanovllm/pd/kv_channel.py:85-220).
#
# A frame is [n_blocks:u32][k_bytes:u32][v_bytes:u32] (little endian), then
# the K payload, then the V payload.  A payload is the staging rows
# buf.k[:n] / buf.v[:n] ([n, L, block_size, kv_heads, head_dim], C order,
# little-endian elements) byte for byte, so the pinned staging buffer IS the
# payload: it is sent from and received into without a host copy.
# ---------------------------------------------------------------------------

FRAME_HEADER = struct.Struct("<III")


def _byte_view(t: torch.Tensor) -> memoryview:
    """The bytes of a contiguous CPU tensor, shared (no copy)."""
    assert t.is_contiguous() and t.device.type == "cpu"
    return memoryview(t.reshape(-1).view(torch.uint8).numpy()).cast("B")


def payload_bytes(buf: KVBlockBuffer, n: int) -> int:
    """Bytes of one side (K or V) of an n-block frame."""
    return n * buf.k[0].numel() * buf.k.element_size()


class LocalKVChannel:
    """Device -> pinned -> device in one process (kv_channel.py:85-107): the
    copy path a cross-process transfer pays, without the socket."""

    def __init__(self, kv_cache: torch.Tensor):
        self.kv_cache = kv_cache
        self.bytes_moved = 0

    def send(self, block_table: list[int]) -> KVBlockBuffer:
        buf = KVBlockBuffer.from_pool(self.kv_cache, len(block_table))
        extract_kv(self.kv_cache, block_table, buf)
        self.bytes_moved += buf.nbytes
        return buf

    def recv(self, block_table: list[int], buf: KVBlockBuffer) -> None:
        import_kv(self.kv_cache, block_table, buf)
        self.bytes_moved += buf.nbytes


class TcpKVChannel:
    """Block-granular KV over a stream socket (kv_channel.py:120-178), same
    frames, same staging buffer, same blocking semantics: send_blocks returns
    once the frame is handed to the socket, recv_blocks once the blocks are in
    the pool.

    Both directions are pipelined in chunks of `chunk_blocks` blocks:
    * send: every chunk's gather into the pinned buffer is enqueued at once,
      each followed by an event; the host sends chunk i as soon as its event
      completes while the GPU still gathers chunk i+1;
    * recv: bytes land straight in the pinned buffer (recv_into); each whole
      chunk's scatter into the pool is enqueued as soon as it has arrived,
      while the host receives the next one.
    """

    MAGIC_HEADER = FRAME_HEADER

    def __init__(self, sock, kv_cache: torch.Tensor, max_blocks: int, chunk_blocks: int = 4):
        if chunk_blocks < 1:
            raise ValueError("chunk_blocks must be >= 1")
        self.sock = sock
        self.kv_cache = kv_cache
        self.buf = KVBlockBuffer.from_pool(kv_cache, max_blocks)
        self.chunk_blocks = chunk_blocks
        self.bytes_moved = 0

    def _chunks(self, n: int):
        return [(i, min(n, i + self.chunk_blocks)) for i in range(0, n, self.chunk_blocks)]

    def send_blocks(self, block_table: list[int]) -> None:
        n = len(block_table)
        assert n <= self.buf.n_blocks
        side = payload_bytes(self.buf, n)
        header = self.MAGIC_HEADER.pack(n, side, side)  # struct.error past u32, as before
        mk, mv = _movers(self.kv_cache)
        stream = torch.cuda.current_stream(self.kv_cache.device)
        pieces = []
        for mover, staging in ((mk, self.buf.k), (mv, self.buf.v)):
            for a, b in self._chunks(n):
                mover.gather(block_table[a:b], out=_items(staging[a:b], b - a))
                ev = torch.cuda.Event()
                ev.record(stream)
                pieces.append((ev, staging[a:b]))
        # the peer reads non-blocking, but sendall needs a blocking socket
        was_blocking = self.sock.getblocking()
        self.sock.setblocking(True)
        try:
            self.sock.sendall(header)
            for ev, rows in pieces:
                ev.synchronize()
                self.sock.sendall(_byte_view(rows))
        finally:
            self.sock.setblocking(was_blocking)
        self.bytes_moved += 2 * side

    def recv_blocks(self, block_table: list[int]) -> None:
        n = len(block_table)
        header = self._recv_exact(self.MAGIC_HEADER.size)
        n_decl, k_len, v_len = self.MAGIC_HEADER.unpack(header)
        assert n_decl == n, f"block count mismatch {n_decl} != {n}"
        side = payload_bytes(self.buf, n)
        if n > self.buf.n_blocks or k_len != side or v_len != side:
            # drain the frame so the stream stays aligned, then refuse it
            self._recv_exact(k_len)
            self._recv_exact(v_len)
            raise RuntimeError(f"frame of {n} blocks carries {k_len}/{v_len} payload bytes; "
                               f"this pool's {n}-block payload is {side} bytes per side")
        mk, mv = _movers(self.kv_cache)
        for mover, staging in ((mk, self.buf.k), (mv, self.buf.v)):
            for a, b in self._chunks(n):
                self._recv_into(_byte_view(staging[a:b]))
                mover.scatter(_items(staging[a:b], b - a), block_table[a:b])
        if n:
            torch.cuda.current_stream(self.kv_cache.device).synchronize()
        self.bytes_moved += k_len + v_len

    def _recv_into(self, view: memoryview) -> None:
        got, total = 0, len(view)
        while got < total:
            k = self.sock.recv_into(view[got:], min(total - got, 1 << 22))
            if not k:
                raise ConnectionError("peer closed during KV transfer")
            got += k

    def _recv_exact(self, n: int) -> bytes:
        out = bytearray(n)
        self._recv_into(memoryview(out))
        return bytes(out)


class KVFrameAssembler:
    """Incremental reassembly of TcpKVChannel frames from a non-blocking
    socket (kv_channel.py:181-220): feed(chunk) returns the frames completed
    by it as (n_blocks, k_bytes, v_bytes) tuples, in order; a frame with
    empty payloads comes back as (n, b"", b"")."""

    def __init__(self):
        self._buf = bytearray()
        self._header = None

    def feed(self, chunk: bytes):
        self._buf += chunk
        frames = []
        pos = 0
        hdr = FRAME_HEADER.size
        while True:
            if self._header is None:
                if len(self._buf) - pos < hdr:
                    break
                self._header = FRAME_HEADER.unpack_from(self._buf, pos)
                pos += hdr
            n, k_len, v_len = self._header
            if len(self._buf) - pos < k_len + v_len:
                break
            frames.append((n, bytes(self._buf[pos:pos + k_len]),
                           bytes(self._buf[pos + k_len:pos + k_len + v_len])))
            pos += k_len + v_len
            self._header = None
        if pos:
            del self._buf[:pos]
        return frames


def import_frame(kv_cache: torch.Tensor, block_table: list[int], buf: KVBlockBuffer,
                 frame) -> None:
    """Import one assembled frame (n, k_bytes, v_bytes) into the blocks named
    by block_table, through `buf` (the decode side's step after
    KVFrameAssembler.feed, scripts/p15_pd_serve.py:167-176): one host copy of
    each payload into the pinned rows, then the scatter."""
    n, k_bytes, v_bytes = frame
    assert n == len(block_table) and n <= buf.n_blocks
    side = payload_bytes(buf, n)
    if len(k_bytes) != side or len(v_bytes) != side:
        raise RuntimeError(f"frame payloads {len(k_bytes)}/{len(v_bytes)} bytes, expected {side}")
    _byte_view(buf.k[:n])[:] = k_bytes
    _byte_view(buf.v[:n])[:] = v_bytes
    import_kv(kv_cache, block_table, buf)
