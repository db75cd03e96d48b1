"""Per-step batch metadata read by the attention layer.

Same fields, order and setters as nanovllm/utils/context.py:5-50, so an engine
that builds a Context for its own attention builds one for this attention too.
All cu_seqlens fields are prefill-only in a mixed batch; decode rows carry
their own context lengths (nanovllm/utils/context.py:21-28).  One field is
added at the end: decode_context_lens_list, the decode rows' context lengths
as host ints (the runner's dec_ctx_lens, nanovllm/engine/model_runner.py:
597-602), which lets a mixed call size its CU split without a device read.
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    cu_seqlens_q_list: list | None = None
    cu_seqlens_k_list: list | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    max_context_len: int = 0
    is_mixed: bool = False
    num_decode_rows: int = 0
    decode_context_lens: torch.Tensor | None = None
    decode_max_context_len: int = 0
    decode_context_lens_list: list | None = None


_CURRENT = Context()


def get_context() -> Context:
    return _CURRENT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, max_context_len=0,
                cu_seqlens_q_list=None, cu_seqlens_k_list=None,
                is_mixed=False, num_decode_rows=0,
                decode_context_lens=None, decode_max_context_len=0,
                decode_context_lens_list=None):
    global _CURRENT
    _CURRENT = Context(
        is_prefill=is_prefill,
        cu_seqlens_q=cu_seqlens_q,
        cu_seqlens_k=cu_seqlens_k,
        cu_seqlens_q_list=cu_seqlens_q_list,
        cu_seqlens_k_list=cu_seqlens_k_list,
        max_seqlen_q=max_seqlen_q,
        max_seqlen_k=max_seqlen_k,
        slot_mapping=slot_mapping,
        context_lens=context_lens,
        block_tables=block_tables,
        max_context_len=max_context_len,
        is_mixed=is_mixed,
        num_decode_rows=num_decode_rows,
        decode_context_lens=decode_context_lens,
        decode_max_context_len=decode_max_context_len,
        decode_context_lens_list=decode_context_lens_list,
    )


def reset_context():
    global _CURRENT
    _CURRENT = Context()


def last_row_indices(context: Context, device=None) -> torch.Tensor | None:
    """Rows the LM head samples (nanovllm/layers/embed_head.py:56-71): in a
    mixed batch every decode row [0, n) then each prefill chunk's last row
    (cu_seqlens_q is prefill-relative, so + n); in a prefill batch each
    chunk's last row; None for a decode batch (every row).  Built on the
    device from the context's tensors, with no host read, so it can run
    inside a captured graph."""
    if context.is_mixed:
        n = context.num_decode_rows
        cu = context.cu_seqlens_q
        dec = torch.arange(n, device=cu.device if device is None else device, dtype=torch.long)
        return torch.cat([dec, cu[1:].long() - 1 + n])
    if context.is_prefill:
        return context.cu_seqlens_q[1:].long() - 1
    return None
