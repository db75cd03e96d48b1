"""CPU checks of the C ABI: the library loads and exports every symbol the
header declares, with matching ctypes signatures, and no device call is made."""
import pathlib
import re

from nanovllm_amd import _native

REPO = pathlib.Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (REPO / "include" / "kvc.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = _declared_symbols()
    for required in ("kvc_store_kv", "kvc_store_int8_tokhead", "kvc_store_int8_chan",
                     "kvc_paged_decode", "kvc_varlen_attention", "kvc_block_gather",
                     "kvc_block_scatter", "kvc_block_copy", "kvc_block_d2h", "kvc_block_h2d"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), f"{name} declared in kvc.h but not exported"


def test_binding_covers_the_header_exactly():
    assert sorted(_native.SIGNATURES) == _declared_symbols()


def test_abi_version_and_error_string():
    lib = _native.load()
    assert lib.kvc_abi_version() == 2
    assert isinstance(lib.kvc_last_error(), bytes)


def _al(x):
    return (x + 255) // 256 * 256


def _tail_region(base, rows, kvs, ms, uh, grid=256, tail_max=8):
    """The dynamic tail hand-out's part of a decode workspace, after the
    stream-K part: taken counts int32 [rows][kvs][ms], tail partials fp32
    [grid][tail_max][uh][128], their log2-sum-exps [grid][tail_max][uh] and
    eight dummy int32 words per workgroup, each 256-byte aligned."""
    stolen = _al(base)
    tail_o = _al(stolen + rows * kvs * ms * 4)
    tail_lse = _al(tail_o + grid * tail_max * uh * 128 * 4)
    dummy = _al(tail_lse + grid * tail_max * uh * 4)
    return stolen, _al(dummy + grid * 8 * 4)


def test_workspace_queries_are_host_only():
    # Pure host arithmetic (no GPU here; the plan assumes 256 CUs).  Paged
    # decode is stream-K: every workgroup takes an equal share (>= 8 tiles of
    # 32 keys) of all rows' tiles, so a row of up to 4096 keys (128 tiles) is
    # split at most 128 / 8 + 1 = 17 ways.  The workspace holds fp32 partials
    # (128 dims + 1 log-sum-exp per row, head and split), 256-byte aligned,
    # then one int32 split count per (row, kv slice), plus 256 bytes; shapes
    # of 4 kv heads per workgroup (32q/4kv: 8 q heads per kv head) add the
    # tail hand-out's region for 32 heads per row unit.
    q = _native.query
    part = 64 * 32 * 17 * 129 * 4
    base = (part + 255) // 256 * 256 + 64 * 4 * 4 + 256
    assert q("kvc_paged_decode_workspace_bytes", 64, 32, 4, 128, 256, 16) == \
        _tail_region(base, 64, 4, 17, 32)[1] == 51808512
    # Splits are capped at 64 however long the rows are.
    part = 4 * 32 * 64 * 129 * 4
    base = (part + 255) // 256 * 256 + 4 * 4 * 4 + 256
    assert q("kvc_paged_decode_workspace_bytes", 4, 32, 4, 128, 256, 1024) == \
        _tail_region(base, 4, 4, 64, 32)[1]
    # 32 kv heads (4 per workgroup, 1 q head each): 32 counts per row and a
    # tail region of 4 heads per row unit.
    part = 8 * 32 * 17 * 129 * 4
    base = (part + 255) // 256 * 256 + 8 * 32 * 4 + 256
    assert q("kvc_paged_decode_workspace_bytes", 8, 32, 32, 128, 256, 16) == \
        _tail_region(base, 8, 32, 17, 4)[1]
    # 16q / 2kv (2 kv heads per workgroup): no tail region; 8 row units on
    # 256 CUs may split 256 / 8 + 1 = 33 ways.
    part = 8 * 16 * 33 * 129 * 4
    assert q("kvc_paged_decode_workspace_bytes", 8, 16, 2, 128, 256, 16) == \
        (part + 255) // 256 * 256 + 8 * 2 * 4 + 256


def test_decode_layout_query():
    import ctypes
    lay = (ctypes.c_int64 * 4)()
    _native.call("kvc_paged_decode_layout", 64, 32, 4, 128, 256, 16, lay)
    part = _al(64 * 32 * 17 * 129 * 4)
    base = part + 64 * 4 * 4 + 256
    assert list(lay) == [part, _tail_region(base, 64, 4, 17, 32)[0], 17, 4]
    _native.call("kvc_paged_decode_layout", 8, 16, 2, 128, 256, 16, lay)
    assert list(lay) == [_al(8 * 16 * 33 * 129 * 4), -1, 33, 2]


def test_bad_arguments_map_to_python_exceptions():
    import pytest
    # head_dim 64 is rejected before any device work (ValueError).
    with pytest.raises(ValueError):
        _native.call("kvc_paged_decode", None, 0, 0, None, None, 0, 256, 4, 64, 0, None, None,
                     None, None, None, None, 0, None, 0, 1, None, 1, 32, 1.0, None, 0, 0, None,
                     0, None)
    with pytest.raises(ValueError):
        _native.call("kvc_block_gather", None, 1, 16, 15, None, 1, None, 16, 16, None)


def test_gather_kv_checks_its_arguments_on_the_host():
    import pytest
    # kvc_gather_kv validates shapes, encodings and pointers before any device
    # work; fake pointers are never dereferenced because a check fails first.

    def gather(head_dim=128, kv_dtype=2, scales=64, side=64, head_n_out=64, n_out_max=4,
               num_prefill=1, total_keys=1, pool=64, max_blocks=1, bt_stride=1):
        _native.call("kvc_gather_kv", pool, pool, 2, 256, 4, head_dim, kv_dtype, scales, scales,
                     side, side, 64, head_n_out, n_out_max, 64, bt_stride, max_blocks, 0,
                     num_prefill, 64, total_keys, None if pool is None else 64, 64, None)

    gather(num_prefill=0)   # nothing to gather: validated, then nothing to do
    gather(total_keys=0)
    with pytest.raises(ValueError, match="head_dim"):
        gather(head_dim=64)
    with pytest.raises(ValueError, match="kv_dtype"):
        gather(kv_dtype=7)
    with pytest.raises(ValueError, match="null pointer"):
        gather(pool=None)
    with pytest.raises(ValueError, match="scales"):
        gather(scales=None)
    with pytest.raises(ValueError, match="n_out_max"):
        gather(n_out_max=9)
    with pytest.raises(ValueError, match="n_out_max"):
        gather(side=None)
    with pytest.raises(ValueError, match="max_blocks_per_seq"):
        gather(max_blocks=2, bt_stride=1)


def test_fresh_rows_with_outlier_dims_are_checked_on_the_host():
    import pytest
    # Fresh rows gathered from a per-channel pool may name its outlier dims;
    # their side width follows the attention's rule (1, 2, 4 or 8), checked
    # before any device work (num_q_tokens 0: nothing runs after the checks).

    def call(out_idx2d=64, n_out_max=4):
        _native.call("kvc_varlen_attention", 64, 4096, 128, 0, 32, None, None, 0, 0, 4, 128,
                     _native.KVC_KV_BF16, None, None, None, None, out_idx2d, 64, n_out_max,
                     64, 512, 128, 64, 512, 128, None, 0, 0, 0, None, 0, None, None, 0, 0,
                     0, 0, 1.0, 64, 4096, 128, None, 0, None)

    call()
    for n in (1, 2, 8):
        call(n_out_max=n)
    for n in (0, 3, 16):
        with pytest.raises(ValueError, match="n_out_max"):
            call(n_out_max=n)
    with pytest.raises(ValueError, match="out_idx2d"):
        call(out_idx2d=None)


def test_side_pool_widths_and_alignment():
    import pytest
    # Per-channel side pools (kv_dtype 2): n_out_max must be 1, 2, 4 or 8 and
    # the pools aligned for one load per row; both are checked on the host
    # before any device work (the pointers are never dereferenced here).

    def decode(n_out_max, side=4096):
        _native.call("kvc_paged_decode", None, 0, 0, None, None, 0, 256, 4, 128, 2, 64, 64,
                     side, side, 64, 64, n_out_max, None, 0, 1, None, 0, 32, 1.0, None, 0, 0,
                     None, 0, None)

    for n in (1, 2, 4, 8):
        decode(n)   # batch 0: validated, then nothing to do
    for n in (0, 3, 5, 6, 7, 9, 16):
        with pytest.raises(ValueError, match="n_out_max"):
            decode(n)
    with pytest.raises(ValueError, match="aligned"):
        decode(4, side=4098)
    decode(1, side=4098)


def test_binding_argument_counts_match_the_header():
    text = re.sub(r"/\*.*?\*/", "", (REPO / "include" / "kvc.h").read_text(), flags=re.S)
    for name, (_, argtypes) in _native.SIGNATURES.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", text)
        assert m, name
        params = m.group(1).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(argtypes), f"{name}: header has {n} parameters, binding {len(argtypes)}"


def test_mixed_split_from_the_work_hints(monkeypatch):
    # Host only (256 CUs without a device).  The decode side's share follows
    # the two sides' CU-time: the split sweep of 60 decode rows U[256,4096]
    # plus four 256-token chunks (prefixes 0/512/2048/8192) was fastest at 96
    # decode CUs, 16 rows plus four 512-token chunks at 24 (146.8 / 139.4 /
    # 140.7 us at 16 / 24 / 32: of the two multiples of 8 around the balance
    # point, 19.1, the larger one, where the decode side is not the slower),
    # and 128 rows plus two 128-token chunks kept getting faster up to the 128
    # measured.
    from nanovllm_amd.kernels.varlen import varlen_decode_cus
    from nanovllm_amd.workloads import uniform_lengths
    monkeypatch.delenv("KVC_MIXED_DECODE_CUS", raising=False)

    def split(n, chunks, hinted=True, **kw):
        dec = uniform_lengths(n, 256, 4096, seed=3)
        cq, ck = [0], [0]
        for p, c in chunks:
            cq.append(cq[-1] + c)
            ck.append(ck[-1] + p + c)
        if not hinted:
            return varlen_decode_cus(n, cq[-1], 32, 4, **kw)
        return varlen_decode_cus(n, cq[-1], 32, 4, dec, cq, ck, **kw)

    cfg3 = [(0, 256), (512, 256), (2048, 256), (8192, 256)]
    assert split(60, cfg3) == 96
    assert split(60, cfg3, hinted=False) == 96  # 3/8 of the CUs without hints
    assert split(16, [(0, 512), (512, 512), (2048, 512), (8192, 512)]) == 24
    assert split(128, [(0, 128), (4096, 128)]) >= 192
    # Tiny sides keep at least 8 CUs each.
    assert split(1, [(0, 4096)] * 4) == 8
    assert split(256, [(0, 1)]) == 248
    # int8 pools and groupings without the 4-head LDS decode run in turn.
    assert split(60, cfg3, kv_dtype=_native.KVC_KV_INT8_TOKHEAD) == 0
    assert _native.query("kvc_varlen_decode_cus", 60, 1024, 16, 2, _native.KVC_KV_BF16,
                         100000, 10 ** 7) == 0
    monkeypatch.setenv("KVC_MIXED_DECODE_CUS", "70")
    assert split(60, cfg3) == 64
    monkeypatch.setenv("KVC_MIXED_DECODE_CUS", "0")
    assert split(60, cfg3) == 0
