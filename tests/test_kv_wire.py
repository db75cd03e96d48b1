"""PD wire format (nanovllm/pd/kv_channel.py:110-220) on the CPU: the
oracle's frame pinned by a hand-written frame and by the reference's own
torch composition, and KVFrameAssembler against the oracle's splitter under
every way a byte stream can be cut."""
import random
import struct

import numpy as np
import pytest
import torch

from nanovllm_amd.pd.kv_channel import FRAME_HEADER, KVFrameAssembler
from oracle import kv_oracle as ko


def test_frame_known_answer():
    # pool [2, L=1, blocks=3, page=1, kvh=1, d=2] of u16; table [2, 0]
    pool = np.array([[[[[[0x0100, 0x0302]]], [[[0x0504, 0x0706]]], [[[0x0908, 0x0B0A]]]]],
                     [[[[[0x1110, 0x1312]]], [[[0x1514, 0x1716]]], [[[0x1918, 0x1B1A]]]]]],
                    dtype=np.uint16)
    assert pool.shape == (2, 1, 3, 1, 1, 2)
    want = bytes([2, 0, 0, 0, 8, 0, 0, 0, 8, 0, 0, 0,
                  0x08, 0x09, 0x0A, 0x0B, 0x00, 0x01, 0x02, 0x03,
                  0x18, 0x19, 0x1A, 0x1B, 0x10, 0x11, 0x12, 0x13])
    assert ko.kv_frame_ref(pool, [2, 0]) == want
    assert ko.kv_frame_ref(pool, []) == bytes(12)


def test_frame_matches_reference_torch_composition():
    # extract_kv's index_select + permute, then _tensor_to_bytes' int16 view
    # (kv_channel.py:64-69, :110-112), restated with torch on the CPU.
    g = torch.Generator().manual_seed(3)
    pool = torch.randn(2, 3, 9, 4, 2, 8, generator=g).to(torch.bfloat16)
    table = [7, 1, 4, 4, 0]
    idx = torch.tensor(table, dtype=torch.long)
    k = pool[0].index_select(1, idx).permute(1, 0, 2, 3, 4).contiguous()
    v = pool[1].index_select(1, idx).permute(1, 0, 2, 3, 4).contiguous()
    kb = k.view(torch.int16).numpy().tobytes()
    vb = v.view(torch.int16).numpy().tobytes()
    want = struct.pack("<III", len(table), len(kb), len(vb)) + kb + vb
    assert ko.kv_frame_ref(ko.torch_bf16_bits(pool), table) == want


def test_split_frames_ref_round_trip():
    rng = np.random.default_rng(0)
    pool = rng.integers(0, 1 << 16, size=(2, 2, 6, 2, 1, 4), dtype=np.uint16)
    tables = [[0], [5, 2, 3], [], [1, 1]]
    frames = [ko.kv_frame_ref(pool, t) for t in tables]
    stream = b"".join(frames)
    got, tail = ko.split_frames_ref(stream + frames[1][:20])
    assert tail == frames[1][:20]
    assert [f[0] for f in got] == [len(t) for t in tables]
    for (n, k, v), fr in zip(got, frames):
        assert fr == struct.pack("<III", n, len(k), len(v)) + k + v


@pytest.mark.parametrize("seed", range(6))
def test_assembler_matches_oracle_under_any_cut(seed):
    rnd = random.Random(seed)
    rng = np.random.default_rng(seed)
    pool = rng.integers(0, 1 << 16, size=(2, 3, 10, 4, 2, 8), dtype=np.uint16)
    tables = [[rnd.randrange(10) for _ in range(rnd.randrange(0, 5))] for _ in range(7)]
    stream = b"".join(ko.kv_frame_ref(pool, t) for t in tables)
    stream += struct.pack("<III", 3, 0, 0)            # an empty-payload frame
    stream += ko.kv_frame_ref(pool, [1, 2])[:-5]       # a frame cut short
    want, tail = ko.split_frames_ref(stream)
    asm = KVFrameAssembler()
    got, pos = [], 0
    while pos < len(stream):
        step = rnd.choice([1, 2, 11, 12, 13, 97, 4096, 1 << 20])
        got += asm.feed(stream[pos:pos + step])
        pos += step
    assert got == want
    assert got[-1] == (3, b"", b"")
    # the cut frame completes once its last bytes arrive
    rest = ko.kv_frame_ref(pool, [1, 2])[-5:]
    (n, k, v), = asm.feed(rest)
    assert (n, k, v) == ko.split_frames_ref(ko.kv_frame_ref(pool, [1, 2]))[0][0]
    assert len(tail) > 0


def test_header_is_three_little_endian_u32():
    assert FRAME_HEADER.size == 12
    assert FRAME_HEADER.pack(1, 2, 3) == bytes([1, 0, 0, 0, 2, 0, 0, 0, 3, 0, 0, 0])
    with pytest.raises(struct.error):
        FRAME_HEADER.pack(1, 1 << 32, 0)
