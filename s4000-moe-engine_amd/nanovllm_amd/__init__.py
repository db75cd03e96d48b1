"""MI355X (gfx950) paged KV-cache hot path with the engine's own Python API.

Module layout mirrors the engine it drops into:
  utils.context        per-step batch metadata (Context, set/get/reset)
  layers.attention     store_kvcache, Attention
  kernels.paged_attention   paged_decode_attention, set_paged_config
  kernels.kv_int8      store_kvcache_int8, dequant_gathered (+ per-token-head)
  kernels.varlen       one-launch mixed decode + chunked-prefill attention
  engine.block_manager BlockManager (prefix cache, LRU, host offload policy)
  engine.kv_offload    HostBlockPool (pinned host slots)
  engine.kv_runner     KV pool allocation, offload byte moves, batch prep
  pd.kv_channel        batched block export/import (KVBlockBuffer)
All compute runs in libkvc.so (hand-written HIP); see _native.
"""
