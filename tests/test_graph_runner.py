"""Host logic of the capture-safe decode step (CPU): bucket choice, the
scratch-block padding of graph inputs (nanovllm/engine/model_runner.py:
842-869, :1154) and the LM head's last-row selection
(nanovllm/layers/embed_head.py:56-71)."""
import torch

from nanovllm_amd.engine.graph_runner import default_buckets, pad_decode_inputs
from nanovllm_amd.utils.context import Context, last_row_indices


def test_default_buckets_follow_the_engine():
    assert default_buckets(512)[:6] == [1, 2, 4, 8, 16, 32]
    assert default_buckets(512)[-1] == 512 and len(default_buckets(512)) == 4 + 32
    assert default_buckets(8) == [1, 2, 4, 8]
    assert default_buckets(20) == [1, 2, 4, 8, 16]


def test_padding_aims_spare_rows_at_the_scratch_block():
    slot_buf = torch.zeros(8, dtype=torch.int32)
    lens_buf = torch.zeros(8, dtype=torch.int32)
    tables_buf = torch.zeros(8, 6, dtype=torch.int32)
    slots = torch.tensor([5, 300, 77], dtype=torch.int32)
    lens = torch.tensor([6, 45, 300], dtype=torch.int32)
    tables = torch.tensor([[3, -1], [1, -1], [0, 2]], dtype=torch.int32)
    pad_decode_inputs(slots, lens, tables, slot_buf, lens_buf, tables_buf,
                      scratch_slot=9 * 256, scratch_block_id=9)
    assert slot_buf.tolist() == [5, 300, 77] + [9 * 256] * 5
    assert lens_buf.tolist() == [6, 45, 300] + [1] * 5
    assert tables_buf[:3, :2].tolist() == tables.tolist()
    assert (tables_buf[:3, 2:] == 9).all() and (tables_buf[3:] == 9).all()


def test_last_row_indices_mixed_prefill_and_decode():
    cu = torch.tensor([0, 4, 5, 9], dtype=torch.int32)
    mixed = Context(is_prefill=True, is_mixed=True, num_decode_rows=3, cu_seqlens_q=cu)
    assert last_row_indices(mixed).tolist() == [0, 1, 2, 6, 7, 11]
    pre = Context(is_prefill=True, cu_seqlens_q=cu)
    assert last_row_indices(pre).tolist() == [3, 4, 8]
    assert last_row_indices(Context()) is None
