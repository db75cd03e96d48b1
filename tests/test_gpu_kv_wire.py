"""PD KV transfer over a stream socket (nanovllm/pd/kv_channel.py:85-220):
the frame TcpKVChannel.send_blocks puts on the wire is the oracle's frame
byte for byte; frames received by recv_blocks, or reassembled by
KVFrameAssembler and imported, land in the peer's blocks bit for bit and
touch no other block.  Sockets are an in-process socketpair; the sender runs
in a thread (sendall blocks until the peer reads)."""
import socket
import struct
import threading

import numpy as np
import pytest
import torch

from nanovllm_amd.pd.kv_channel import (KVBlockBuffer, KVFrameAssembler, LocalKVChannel,
                                        TcpKVChannel, import_frame)
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu
DEV = "cuda"
L, PAGE, KVH = 3, 64, 4


def _pool(blocks, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(2, L, blocks, PAGE, KVH, 128, generator=g).to(torch.bfloat16).to(DEV)


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _send_in_thread(fn):
    err = []

    def run():
        try:
            fn()
        except BaseException as e:  # surfaced by the caller
            err.append(e)
    th = threading.Thread(target=run)
    th.start()
    return th, err


def _read_all(sock, n):
    out = bytearray()
    while len(out) < n:
        chunk = sock.recv(min(n - len(out), 1 << 20))
        assert chunk, "peer closed early"
        out += chunk
    return bytes(out)


@pytest.mark.parametrize("chunk", [1, 3, 16])
def test_send_blocks_writes_the_oracle_frame(chunk):
    pool = _pool(12, seed=chunk)
    table = [9, 0, 4, 11, 4, 7, 2]
    want = ko.kv_frame_ref(_u16(pool), table)
    a, b = socket.socketpair()
    chan = TcpKVChannel(a, pool, max_blocks=8, chunk_blocks=chunk)
    print(f"[wire] send chunk={chunk} n={len(table)}", flush=True)
    th, err = _send_in_thread(lambda: chan.send_blocks(table))
    try:
        got = _read_all(b, len(want))
        th.join(60)
    finally:
        a.close(), b.close()
    assert not th.is_alive() and not err, err
    assert got == want
    assert chan.bytes_moved == len(want) - 12


@pytest.mark.parametrize("chunk", [2, 5])
def test_recv_blocks_round_trip_into_other_blocks(chunk):
    src = _pool(10, seed=11)
    dst = _pool(14, seed=12)
    before = _u16(dst).copy()
    t_src, t_dst = [3, 8, 1, 0, 6], [13, 2, 7, 10, 5]
    a, b = socket.socketpair()
    tx = TcpKVChannel(a, src, max_blocks=8, chunk_blocks=chunk)
    rx = TcpKVChannel(b, dst, max_blocks=8, chunk_blocks=chunk)
    print(f"[wire] round trip chunk={chunk}", flush=True)
    th, err = _send_in_thread(lambda: (tx.send_blocks(t_src), tx.send_blocks([])))
    try:
        rx.recv_blocks(t_dst)
        rx.recv_blocks([])
        th.join(60)
    finally:
        a.close(), b.close()
    assert not th.is_alive() and not err, err
    expect = before.copy()
    expect[:, :, t_dst] = _u16(src)[:, :, t_src]
    assert np.array_equal(_u16(dst), expect)
    assert rx.bytes_moved == tx.bytes_moved


def test_assembled_frames_import_and_a_bad_frame_is_refused():
    src = _pool(10, seed=21)
    dst = _pool(10, seed=22)
    tables = [[1, 2], [9], [0, 3, 5, 7]]
    targets = [[8, 6], [4], [2, 9, 0, 1]]
    stream = b"".join(ko.kv_frame_ref(_u16(src), t) for t in tables)
    asm = KVFrameAssembler()
    frames = []
    for i in range(0, len(stream), 100_003):
        frames += asm.feed(stream[i:i + 100_003])
    assert [f[0] for f in frames] == [2, 1, 4]
    buf = KVBlockBuffer.from_pool(dst, 4)
    before = _u16(dst).copy()
    print("[wire] import assembled frames", flush=True)
    for fr, tgt in zip(frames, targets):
        import_frame(dst, tgt, buf, fr)
    expect = before.copy()
    for t, tgt in zip(tables, targets):
        expect[:, :, tgt] = _u16(src)[:, :, t]
    assert np.array_equal(_u16(dst), expect)
    # A frame whose payload does not fit this pool's block shape is drained
    # and refused; the next frame on the stream still decodes.
    a, b = socket.socketpair()
    try:
        rx = TcpKVChannel(b, dst, max_blocks=4)
        bad = ko.kv_frame_ref(_u16(src)[:, :, :, :PAGE // 2], [1, 2])
        good = ko.kv_frame_ref(_u16(src), [5])
        th, err = _send_in_thread(lambda: a.sendall(bad + good))
        with pytest.raises(RuntimeError):
            rx.recv_blocks([3, 4])
        rx.recv_blocks([6])
        th.join(60)
        assert not th.is_alive() and not err, err
        assert np.array_equal(_u16(dst)[:, :, 6], _u16(src)[:, :, 5])
        # a block count that differs from the table's is an AssertionError
        a.sendall(struct.pack("<III", 1, 0, 0))
        with pytest.raises(AssertionError):
            rx.recv_blocks([1, 2])
    finally:
        a.close(), b.close()


def test_local_channel_round_trip():
    pool = _pool(9, seed=31)
    before = _u16(pool).copy()
    chan = LocalKVChannel(pool)
    print("[wire] local channel", flush=True)
    buf = chan.send([8, 1, 5])
    chan.recv([0, 2, 3], buf)
    expect = before.copy()
    expect[:, :, [0, 2, 3]] = before[:, :, [8, 1, 5]]
    assert np.array_equal(_u16(pool), expect)
    assert chan.bytes_moved == 2 * buf.nbytes


def test_int8_pool_frame_and_round_trip():
    # An int8 code pool travels the same way (the reference's int16 byte view
    # of the staging rows, kv_channel.py:110-112, is just its bytes).
    g = torch.Generator().manual_seed(51)
    src = torch.randint(-127, 128, (2, L, 9, PAGE, KVH, 128), generator=g,
                        dtype=torch.int8).to(DEV)
    dst = torch.zeros_like(src)
    table, target = [8, 3, 0], [1, 2, 7]
    want = ko.kv_frame_ref(src.cpu().numpy(), table)
    a, b = socket.socketpair()
    tx = TcpKVChannel(a, src, max_blocks=4, chunk_blocks=2)
    rx = TcpKVChannel(b, dst, max_blocks=4, chunk_blocks=2)
    print("[wire] int8 pool", flush=True)
    th, err = _send_in_thread(lambda: tx.send_blocks(table))
    try:
        got = _read_all(b, len(want))
        th.join(60)
        assert got == want
        th, err2 = _send_in_thread(lambda: a.sendall(got))
        rx.recv_blocks(target)
        th.join(60)
    finally:
        a.close(), b.close()
    assert not err and not err2
    expect = torch.zeros_like(src).cpu()
    expect[:, :, target] = src.cpu()[:, :, table]
    assert torch.equal(dst.cpu(), expect)
