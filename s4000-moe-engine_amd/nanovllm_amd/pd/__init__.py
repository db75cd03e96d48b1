"""Block-granular KV export/import and its wire format (nanovllm/pd/)."""
from .kv_channel import (FRAME_HEADER, KVBlockBuffer, KVFrameAssembler, LocalKVChannel,
                         TcpKVChannel, extract_kv, import_frame, import_kv)

__all__ = ["FRAME_HEADER", "KVBlockBuffer", "KVFrameAssembler", "LocalKVChannel",
           "TcpKVChannel", "extract_kv", "import_frame", "import_kv"]
