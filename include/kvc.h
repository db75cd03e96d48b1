/*
 * kvc.h — C ABI of the MI355X (gfx950) paged KV-cache library `libkvc.so`.
 *
 * Every entry point takes raw device pointers, element counts and element
 * strides (never framework types), enqueues its work on `stream` (a
 * hipStream_t; NULL is the legacy default stream), never allocates device
 * memory and never synchronises the host.  Return value: KVC_OK (0) or a
 * negative KVC_ERR_* code; kvc_last_error() then holds a message for the
 * calling thread.  Caller-side ownership: the caller owns every buffer.
 *
 * Layouts (the engine's own, unchanged):
 *   KV pool per layer      [num_blocks, page_size, num_kv_heads, head_dim]
 *                          contiguous; a "slot" is block_id * page_size +
 *                          offset, i.e. the row index of the flat
 *                          [num_blocks * page_size, num_kv_heads * head_dim]
 *                          view.
 *   block_tables           int32 [batch, max_blocks_per_seq], row stride
 *                          bt_stride, padded with -1 (entries past a row's
 *                          context are never read).
 *   context_lens           int32 [batch], read on the device (no host copy).
 *   int8 per-token-head    codes int8 in the pool layout + fp32 scales
 *     scales               [num_blocks, page_size, num_kv_heads].
 *   int8 per-channel       codes int8 in the pool layout, scales fp32
 *     (outlier side pool)  [num_kv_heads, head_dim], side pool bf16
 *                          [num_blocks, page_size, num_kv_heads, n_out_max],
 *                          out_idx2d int32 [num_kv_heads, n_out_max],
 *                          head_n_out int32 [num_kv_heads].
 *   whole-block slabs      a block of a multi-layer pool
 *                          [planes, num_blocks, block_bytes] (planes =
 *                          2 * layers for the engine's [2, L, ...] pool) is
 *                          `planes` rows of block_bytes at plane_stride.
 */
#ifndef KVC_H_
#define KVC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kvc_stream_t; /* hipStream_t */

enum kvc_status {
  KVC_OK = 0,
  KVC_ERR_VALUE = -1,     /* unsupported shape / dtype / argument (ValueError) */
  KVC_ERR_ASSERT = -2,    /* violated layout precondition (AssertionError)     */
  KVC_ERR_RUNTIME = -3,   /* HIP runtime failure (RuntimeError)                */
  KVC_ERR_WORKSPACE = -4, /* workspace missing or too small (ValueError)        */
};

/* KV element encodings accepted by the attention entry points. */
enum kvc_kv_dtype {
  KVC_KV_BF16 = 0,          /* bf16 pool                                       */
  KVC_KV_INT8_TOKHEAD = 1,  /* int8 codes + fp32 scale per (slot, kv_head)     */
  KVC_KV_INT8_CHAN = 2,     /* int8 codes * per-channel read scale + bf16 side */
};

/* Thread-local message for the last failing call on this thread. */
const char* kvc_last_error(void);
/* ABI revision of this header (bumped on any signature change). */
int kvc_abi_version(void);

/* ---------------------------------------------------------------------------
 * KV append.
 * ------------------------------------------------------------------------- */

/* Replaces store_kvcache (nanovllm/layers/attention.py:9-30):
 *   k_cache.view(-1, KVH*D)[slot_mapping] = key.reshape(N, KVH*D), same for V.
 * key/value rows are addressed with their own strides (elements), so a V that
 * is a strided view of a fused qkv projection needs no copy.  A negative slot
 * wraps like a Python index (slot + num_slots); a slot still outside
 * [0, num_slots) is skipped.  elem_bytes: 2 (bf16/fp16) or 4 (fp32).
 * slot_index_bytes: 4 (int32) or 8 (int64). */
int kvc_store_kv(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                 const void* value, int64_t value_stride_n, int64_t value_stride_h,
                 void* k_cache, void* v_cache, int64_t num_slots,
                 const void* slot_mapping, int slot_index_bytes,
                 int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                 int elem_bytes, kvc_stream_t stream);

/* Per-token-per-head int8 quantise-on-append (the P17 layout documented in
 * benchmarks/archive/P17-kv-int8.md:9-11, arithmetic of
 * scripts/archive/p14_int8_kv_probe.py:37-41):
 *   amax = max_d |x[d]| (bf16, exact) -> fp32, clamped to >= 1e-6
 *   s    = amax / 127            (IEEE fp32 division)
 *   code = clamp(rint_half_even(x / s), -127, 127)
 * codes land in k_cache/v_cache [slots, KVH, D] int8 and s in
 * k_scale/v_scale [slots, KVH] fp32.  key/value are bf16. */
int kvc_store_int8_tokhead(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                           const void* value, int64_t value_stride_n, int64_t value_stride_h,
                           int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
                           int64_t num_slots, const void* slot_mapping, int slot_index_bytes,
                           int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                           kvc_stream_t stream);

/* Replaces store_kvcache_int8 (nanovllm/kernels/kv_int8.py:72-93), the
 * per-channel mode with a bf16 outlier side pool:
 *   code = clamp(floor(x / s[h][d] + 0.5), -127, 127)   (IEEE fp32 division)
 *   code = 0 at the head's outlier dims out_idx2d[h][:head_n_out[h]]
 *   side[slot][h][j] = bf16(x[out_idx2d[h][j]]) for j < head_n_out[h].
 * Unlike the reference kernel, V is read with V's own strides. */
int kvc_store_int8_chan(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                        const void* value, int64_t value_stride_n, int64_t value_stride_h,
                        int8_t* k_cache, int8_t* v_cache,
                        const float* k_scale, const float* v_scale,
                        void* side_k, void* side_v, int64_t n_out_max,
                        const int32_t* out_idx2d, const int32_t* head_n_out,
                        int64_t num_slots, const void* slot_mapping, int slot_index_bytes,
                        int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                        kvc_stream_t stream);

/* Calibration statistics of the per-channel encoding: the forward pre-hook
 * of ModelRunner.kv_calibrate_begin (nanovllm/engine/model_runner.py:510-539)
 * run over one observed forward's key/value rows [num_tokens, KVH, 128]
 * (bf16, own element strides):
 *   amax[s][h][d]    = max(amax[s][h][d], max_n |x_s[n][h][d]|)
 *   abs_sum[s][h][d] += bf16(sum_n |x_s[n][h][d]|)    (fp32 add)
 * for s = 0 (key) and 1 (value); amax and abs_sum are fp32 [2, KVH, 128],
 * zeroed by the caller before the first call.  As in the hook, whose
 * `k.abs().sum(dim=0)` torch returns in bf16 (model_runner.py:529-532), each
 * call's sum is rounded to bf16 (nearest, ties to even) before it is added;
 * the sum is formed exactly before that rounding, so it does not depend on
 * the order of the additions.  The caller counts the tokens. */
int kvc_kv_calib_observe(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                         const void* value, int64_t value_stride_n, int64_t value_stride_h,
                         int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                         float* amax, float* abs_sum, kvc_stream_t stream);

/* Freeze of one layer's statistics over `count` observed tokens
 * (ModelRunner.kv_calibrate_freeze, model_runner.py:541-577):
 *   scale  = max(amax / 127, 1e-6)                   -> k_scale / v_scale [KVH, 128]
 *   typ    = max(abs_sum / count, 1e-6)
 *   ratio  = max(amax_k / typ_k, amax_v / typ_v)     (K and V jointly)
 *   outlier dims of head h: its first n_out_max dims, in index order, with
 *   ratio > 10 -> out_idx2d[h][0 .. head_n_out[h]) (entries past head_n_out
 *   are left as they are)
 *   read scales k_dscale / v_dscale = scale, 0 at the outlier dims.
 * KVC_ERR_ASSERT when count is 0 (the reference asserts). */
int kvc_kv_calib_freeze(const float* amax, const float* abs_sum, int64_t count,
                        int64_t num_kv_heads, int64_t head_dim, int64_t n_out_max,
                        float* k_scale, float* v_scale, float* k_dscale, float* v_dscale,
                        int32_t* out_idx2d, int32_t* head_n_out, kvc_stream_t stream);

/* ---------------------------------------------------------------------------
 * Paged decode attention.
 * ------------------------------------------------------------------------- */

/* Bytes of split-K workspace kvc_paged_decode needs for this launch shape
 * (0 when every sequence fits in one split).  max_blocks_per_seq is the
 * block_tables width: the launch is sized from it, never from a host copy of
 * the context lengths, so one captured launch serves every length. */
size_t kvc_paged_decode_workspace_bytes(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                        int64_t head_dim, int64_t page_size,
                                        int64_t max_blocks_per_seq);

/* Diagnostics (no counterpart in the reference): where a stream-K paged
 * decode launch of this shape leaves, in its workspace, the split count of
 * every (row, kv slice) (int32 [batch][kv_slices], low 16 bits) and the
 * number of tail tiles other workgroups took from each piece of it (int32
 * [batch][kv_slices][max_splits], valid for pieces below the split count).
 * layout[0] = byte offset of the split counts, layout[1] = byte offset of
 * the taken counts (-1: this shape has no dynamic tail hand-out), layout[2]
 * = max_splits, layout[3] = kv_slices.  Returns KVC_ERR_VALUE when the
 * launch would not be stream-K.  Reading these after a launch tells how
 * much work the dynamic hand-out moved. */
int kvc_paged_decode_layout(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t page_size, int64_t max_blocks_per_seq,
                            int64_t* layout);

/* Replaces paged_decode_attention / _paged_decode_kernel
 * (nanovllm/kernels/paged_attention.py:73-245):
 *   out[b, h] = softmax(q[b, h] . K[b, :ctx, h // G]^T * scale) . V[b, :ctx, h // G]
 * with G = num_heads / num_kv_heads and ctx = context_lens[b] (device).
 * q/out bf16 [batch, num_heads, head_dim] with the given strides.  head_dim
 * must be 128 and page_size a multiple of 32.  kv_dtype selects the pool
 * encoding; for KVC_KV_INT8_TOKHEAD k_scale/v_scale are the per-slot scales,
 * for KVC_KV_INT8_CHAN they are the [KVH, D] read scales (0 at outlier dims)
 * and side_k/side_v/out_idx2d/head_n_out/n_out_max describe the side pool
 * (side pointers may be NULL when no head has outliers; with head_n_out
 * given, n_out_max must be 1, 2, 4 or 8, the powers of two the reference
 * kernel's tl.arange(0, N_OUT_MAX) admits, and the side pools 4-byte
 * aligned, 2-byte for n_out_max 1; a head's outlier dims are distinct, as
 * the calibration makes them: the reference kernel sums the side logits of
 * a repeated dim and stores its output once, in no defined order).
 * context_lens[b] == 0 yields 0/0 = NaN rows, as the reference kernel does. */
int kvc_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                     int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int kv_dtype,
                     const float* k_scale, const float* v_scale,
                     const void* side_k, const void* side_v, const int32_t* out_idx2d,
                     const int32_t* head_n_out, int64_t n_out_max,
                     const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
                     const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale,
                     void* out, int64_t out_stride_b, int64_t out_stride_h,
                     void* workspace, size_t workspace_bytes, kvc_stream_t stream);

/* The decode step's KV work on a bf16 pool: kvc_store_kv of one new token
 * per row (key/value [batch, num_kv_heads, head_dim] with their own element
 * strides, at slot_mapping[b], with kvc_store_kv's slot rules) followed by
 * kvc_paged_decode over context_lens (which count the new token).  Replaces
 * store_kvcache + paged_decode_attention of the engine's decode step
 * (nanovllm/layers/attention.py:9-30, :239-245;
 * nanovllm/kernels/paged_attention.py:193-245).  Where the decode launch
 * stages 4 kv heads per workgroup and the rows are 16-byte aligned, the
 * store rides in the decode launch itself: the workgroup holding a row's
 * last tile stores the row and uses it straight from the inputs.  That form
 * requires what the engine's decode slots satisfy (model_runner.py:685):
 * slot_mapping[b] is the slot of position context_lens[b] - 1 in row b's
 * block table, and no other row of the call reads that slot.  Otherwise,
 * or for other layouts, the store runs as its own launch first.  Results
 * and pool contents equal the two calls' bit for bit. */
int kvc_paged_decode_append(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* key, int64_t key_stride_n, int64_t key_stride_h,
                            const void* value, int64_t value_stride_n, int64_t value_stride_h,
                            const void* slot_mapping, int slot_index_bytes, void* k_cache,
                            void* v_cache, int64_t num_cache_blocks, int64_t page_size,
                            int64_t num_kv_heads, int64_t head_dim,
                            const int32_t* block_tables, int64_t bt_stride,
                            int64_t max_blocks_per_seq, const int32_t* context_lens,
                            int64_t batch, int64_t num_heads, float scale, void* out,
                            int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                            size_t workspace_bytes, kvc_stream_t stream);

/* The decode step over a per-token-head int8 pool in one call: the new
 * token's K/V rows (bf16, [batch, num_kv_heads, 128], own strides) are
 * quantised as kvc_store_int8_tokhead does (codes and fp32 scales at
 * slot_mapping[b]), then kvc_paged_decode runs over context_lens with that
 * pool.  Replaces the step of the per-token-head mode
 * (scripts/archive/p14_int8_kv_probe.py:37-46: quantise-on-append, then the
 * decode that dequantises on read; nanovllm/kernels/paged_attention.py:
 * 193-245).  Where the decode launch stages 4 kv heads per workgroup and the
 * rows are 16-byte aligned, the quantiser runs inside the decode launch: the
 * workgroup holding a row's last tile quantises and stores the row and uses
 * the codes and scales straight from registers.  That form requires the
 * engine's decode slots (as kvc_paged_decode_append); otherwise the store
 * runs as its own launch first.  Codes, scales and outputs equal the two
 * calls' bit for bit. */
int kvc_paged_decode_append_int8(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void* key, int64_t key_stride_n, int64_t key_stride_h,
                                 const void* value, int64_t value_stride_n,
                                 int64_t value_stride_h, const void* slot_mapping,
                                 int slot_index_bytes, int8_t* k_cache, int8_t* v_cache,
                                 float* k_scale, float* v_scale, int64_t num_cache_blocks,
                                 int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
                                 const int32_t* block_tables, int64_t bt_stride,
                                 int64_t max_blocks_per_seq, const int32_t* context_lens,
                                 int64_t batch, int64_t num_heads, float scale, void* out,
                                 int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                                 size_t workspace_bytes, kvc_stream_t stream);

/* The decode step over a per-channel int8 pool in one call: the new token's
 * K/V rows (bf16, [batch, num_kv_heads, 128], own strides) go to the pool as
 * kvc_store_int8_chan stores them (codes against the store scales k_scale /
 * v_scale [KVH, D], 0 at each head's outlier dims, whose bf16 values go to
 * the side pools at slot_mapping[b]), then kvc_paged_decode runs over
 * context_lens with the read scales k_dscale / v_dscale and the side pools.
 * Replaces the per-channel int8 step of Attention.forward
 * (nanovllm/layers/attention.py:130-177: store_kvcache_int8,
 * nanovllm/kernels/kv_int8.py:29-93, then paged_decode_attention's int8 path,
 * nanovllm/kernels/paged_attention.py:101-172).
 * The store runs as its own launch ahead of the decode (inside the decode's
 * LDS ring the quantiser's registers spilled the tile loop, which cost more
 * than the launch it saves).  Codes, side values and outputs equal the two
 * calls' bit for bit. */
int kvc_paged_decode_append_int8_chan(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, int8_t* k_cache, int8_t* v_cache,
    const float* k_scale, const float* v_scale, const float* k_dscale, const float* v_dscale,
    void* side_k, void* side_v, const int32_t* out_idx2d, const int32_t* head_n_out,
    int64_t n_out_max, int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads,
    int64_t head_dim, const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale, void* out,
    int64_t out_stride_b, int64_t out_stride_h, void* workspace, size_t workspace_bytes,
    kvc_stream_t stream);

/* Bytes of device scratch kvc_paged_decode_append_static holds on each GPU
 * it runs on: 64 MiB, reserved by the first static call on that GPU (the
 * array is a code object of its own, loaded when first used) and held until
 * the process ends; processes that never call it reserve none.  At 32 q / 4 kv heads and pages of 256 that covers
 * batch 32 at any table width, batch 64 with tables of up to 62 pages
 * (15872 tokens), batch 128 up to 30 pages, batch 256 up to 14 pages. */
#define KVC_STATIC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under graph capture that must not allocate, tight serving
 * loops, harnesses that forbid hipMalloc).  kvc_paged_decode_append with the
 * split-K workspace taken from a file-scope device array of
 * KVC_STATIC_SCRATCH_BYTES per GPU (held until the process ends) instead of
 * a caller buffer; same kernels, results and pool contents.  Allocates
 * nothing (no hipMalloc, no library allocation); the caller passes inputs
 * and outputs.  A launch shape whose workspace
 * (kvc_paged_decode_workspace_bytes) exceeds the scratch returns
 * KVC_ERR_WORKSPACE before any device work.  Every call on one GPU shares
 * that GPU's scratch, which keeps the last call's contents: calls that
 * overlap on one GPU (on different streams or from different threads) race
 * and must be ordered by the caller, e.g. on one stream.  The scratch is
 * that of the device `stream` belongs to.  The first call on a device
 * resolves (and loads) its scratch: make it before any graph capture. */
int kvc_paged_decode_append_static(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, void* k_cache, void* v_cache,
    int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
    const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale, void* out,
    int64_t out_stride_b, int64_t out_stride_h, kvc_stream_t stream);

/* Diagnostics, no reference counterpart: with KVC_DECODE_STAMPS=1 in the
 * environment, every stream-K decode launch (up to 4096 workgroups) has each
 * workgroup w record its start and end wall-clock stamps (with
 * KVC_PREFILL_STAMPS=1, every prefill-only stream-K prefill launch); this
 * copies the last recording launch's stamps on the current device to host_out
 * ([2 w] start, [2 w + 1] end, up to max_workgroups workgroups; a blocking
 * copy, so synchronise the launch's stream first) and reports the number of
 * workgroups and the stamp clock's rate in kHz.  KVC_ERR_VALUE when no launch
 * recorded. */
int kvc_decode_stamps(unsigned long long* host_out, int max_workgroups, int* workgroups,
                      int* clock_khz);

/* ---------------------------------------------------------------------------
 * Mixed decode + chunked-prefill attention in one launch.
 * ------------------------------------------------------------------------- */

/* Bytes of workspace kvc_varlen_attention needs.  num_q_tokens counts every
 * query row (decode rows + prefill tokens); max_seqlen_k bounds the prefill
 * key length; max_blocks_per_seq bounds the decode context. */
size_t kvc_varlen_workspace_bytes(int64_t num_q_tokens, int64_t num_heads, int64_t num_kv_heads,
                                  int64_t head_dim, int64_t num_decode_rows, int64_t max_seqlen_k,
                                  int64_t page_size, int64_t max_blocks_per_seq);

/* Number of prefill workgroups kvc_varlen_attention launches for these chunks
 * (cu_q_host/cu_k_host: HOST copies of cu_seqlens_q/k, num_prefill + 1
 * entries each — the engine keeps them as cu_seqlens_q_list/k_list). */
int64_t kvc_varlen_prefill_units(const int32_t* cu_q_host, const int32_t* cu_k_host,
                                 int64_t num_prefill, int64_t num_heads, int64_t num_kv_heads,
                                 int64_t max_seqlen_k);

/* Replaces the mixed / prefill branches of Attention.forward
 * (nanovllm/layers/attention.py:146-173, _forward_decode :215-238 and the
 * per-sequence loop _forward_prefill :179-213) with ONE attention launch plus
 * a split-K merge pass.
 *   rows [0, num_decode_rows): one decode token each, context
 *     decode_context_lens[i] (device), block table row i.
 *   rows num_decode_rows + [cu_seqlens_q[i], cu_seqlens_q[i+1]): prefill
 *     chunk i with sk_i = cu_seqlens_k[i+1] - cu_seqlens_k[i] keys; query r
 *     of the chunk sits at position sk_i - sq_i + r and sees keys j <= that
 *     position (attention.py:210-212).  Keys come from the paged pool through
 *     block table row num_decode_rows + i, or, when block_tables is NULL (no
 *     prefix cache, attention.py:195-199), from the bf16 k_fresh/v_fresh
 *     [tokens, KVH, D] rows cu_seqlens_k[i] .. (then num_decode_rows == 0).
 *     Fresh rows gathered from a per-channel int8 pool (kvc_gather_kv) may
 *     come with that pool's out_idx2d / head_n_out / n_out_max (side pools
 *     unused): the outlier dims' P V and the softmax sums then also take the
 *     rounding residue of the bf16 P operand.
 * cu_seqlens_q/k are int32 device arrays of num_prefill + 1 entries;
 * num_prefill_units comes from kvc_varlen_prefill_units.
 * decode_ctx_tokens and prefill_kq_pairs are host-side hints (0: none) that
 * size the two sides of the one-launch form over a bf16 pool: the sum of the
 * decode rows' context lengths (the runner holds them as ints,
 * nanovllm/engine/model_runner.py:595-674) and the prefill's query-key pairs
 * per head, sum over chunks of sq_i (sk_i - sq_i) + sq_i (sq_i + 1) / 2; see
 * kvc_varlen_decode_cus.  They change the work split, never the result
 * beyond floating-point summation order. */
int kvc_varlen_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                         int64_t num_q_tokens, int64_t num_heads,
                         const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                         int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int kv_dtype,
                         const float* k_scale, const float* v_scale,
                         const void* side_k, const void* side_v, const int32_t* out_idx2d,
                         const int32_t* head_n_out, int64_t n_out_max,
                         const void* k_fresh, int64_t kf_stride_t, int64_t kf_stride_h,
                         const void* v_fresh, int64_t vf_stride_t, int64_t vf_stride_h,
                         const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
                         int64_t num_decode_rows, const int32_t* decode_context_lens,
                         int64_t num_prefill, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int64_t num_prefill_units,
                         int64_t max_seqlen_k, int64_t decode_ctx_tokens,
                         int64_t prefill_kq_pairs, float scale, void* out,
                         int64_t out_stride_t, int64_t out_stride_h, void* workspace,
                         size_t workspace_bytes, kvc_stream_t stream);

/* The step's store and the mixed call together, over a bf16 pool: replaces
 * store_kvcache (nanovllm/layers/attention.py:138-140) followed by the mixed
 * / prefill branches (:146-173).  Row t of key / value ([T, KVH, D] bf16,
 * element strides, 16-byte rows) goes to pool slot slot_mapping[t] (int32 or
 * int64, kvc_store_kv's slot rules) for every query row t; then attention as
 * kvc_varlen_attention (same rows, tables, hints and workspace).  The prefill
 * rows' k/v are stored by one launch ahead of the attention (the prefill
 * reads them back from the pool); the decode rows' k/v are appended inside
 * the decode launch (or the decode side of the one-launch form), as
 * kvc_paged_decode_append does, so a decode row's slot must be position
 * decode_context_lens[i] - 1 of its own table row. */
int kvc_varlen_attention_append(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t num_q_tokens,
    int64_t num_heads, const void* key, int64_t key_stride_t, int64_t key_stride_h,
    const void* value, int64_t value_stride_t, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, void* k_cache, void* v_cache,
    int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
    const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    int64_t num_decode_rows, const int32_t* decode_context_lens, int64_t num_prefill,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_prefill_units,
    int64_t max_seqlen_k, int64_t decode_ctx_tokens, int64_t prefill_kq_pairs, float scale,
    void* out, int64_t out_stride_t, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, kvc_stream_t stream);

/* CUs the decode side of a mixed call's one-launch form gets for these sizes
 * and hints (0: the decode launch and the prefill launch run in turn).  No
 * reference counterpart (the reference runs the two sub-paths in turn,
 * nanovllm/layers/attention.py:146-166).  With both hints the split follows
 * the two sides' CU-time at their measured per-CU rates; without, 3/8 of the
 * CUs; KVC_MIXED_DECODE_CUS overrides.  Host only: reads the device's CU
 * count (256 when no device is visible). */
int kvc_varlen_decode_cus(int64_t num_decode_rows, int64_t num_prefill_tokens, int64_t num_heads,
                          int64_t num_kv_heads, int kv_dtype, int64_t decode_ctx_tokens,
                          int64_t prefill_kq_pairs);

/* ---------------------------------------------------------------------------
 * Dequantise gathered int8 rows (the torch-side read path).
 * ------------------------------------------------------------------------- */

/* Replaces dequant_gathered (nanovllm/kernels/kv_int8.py:96-107):
 *   out[t,h,d] = bf16(fp32(kv[t,h,d]) * dscale[h,d]), then
 *   out[t,h,out_idx2d[h,j]] = side[t,h,j] for j < head_n_out[h].
 * kv int8 [T, KVH, D] contiguous, side bf16 [T, KVH, n_out_max] (may be NULL
 * when no head has outliers), out bf16 [T, KVH, D]. */
int kvc_dequant_chan(const int8_t* kv, const float* dscale, const void* side,
                     const int32_t* out_idx2d, const int32_t* head_n_out, int64_t n_out_max,
                     int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                     void* out, kvc_stream_t stream);

/* Per-token-per-head read path of scripts/archive/p14_int8_kv_probe.py:45-46:
 *   out[t,h,d] = bf16(fp32(code[t,h,d]) * scale[t,h]). */
int kvc_dequant_tokhead(const int8_t* kv, const float* scale, int64_t num_tokens,
                        int64_t num_kv_heads, int64_t head_dim, void* out, kvc_stream_t stream);

/* Replaces _gather_kv (nanovllm/layers/attention.py:33-51), called there per
 * prefill chunk for K and for V, with one launch over every chunk of a step:
 * chunk i's keys 0 .. sk_i - 1 (sk_i = cu_seqlens_k[i+1] - cu_seqlens_k[i]),
 * read through block table row block_table_row0 + i, land at rows
 * cu_seqlens_k[i] .. of out_k / out_v (bf16 [total_keys, KVH, D],
 * contiguous; total_keys = cu_seqlens_k[num_prefill], the host's value).
 * Per-channel int8: bf16(fp32(code) * k_scale[h][d]) (the [KVH, D] read
 * scales), then the head's outlier dims out_idx2d[h][j], j < head_n_out[h],
 * take the side pool's values (a later j wins on a duplicate dim), exactly as
 * _gather_kv; per-token-head int8 (the p14 probe's encoding):
 * bf16(fp32(code) * k_scale[slot][h]); bf16 pools are copied.  A table entry
 * outside the pool reads zeros.  cu_seqlens_k: int32 device array of
 * num_prefill + 1 entries, non-decreasing from 0; n_out_max at most 8. */
int kvc_gather_kv(const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                  int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int kv_dtype,
                  const float* k_scale, const float* v_scale, const void* side_k,
                  const void* side_v, const int32_t* out_idx2d, const int32_t* head_n_out,
                  int64_t n_out_max, const int32_t* block_tables, int64_t bt_stride,
                  int64_t max_blocks_per_seq, int64_t block_table_row0, int64_t num_prefill,
                  const int32_t* cu_seqlens_k, int64_t total_keys, void* out_k, void* out_v,
                  kvc_stream_t stream);

/* ---------------------------------------------------------------------------
 * Whole-block movement (LRU eviction, host offload, compaction).
 * ------------------------------------------------------------------------- */

/* Gather: dst[i][p] = src[p][block_ids[i]] for p < planes, i < n.
 * Replaces the index_select gathers of ModelRunner.offload_put
 * (nanovllm/engine/model_runner.py:284-298) and extract_kv
 * (nanovllm/pd/kv_channel.py:54-69).  block_ids: int32 device array.
 * src plane p, block b starts at src + p*src_plane_stride + b*block_bytes;
 * dst item i, plane p at dst + i*dst_item_stride + p*dst_plane_stride
 * (bytes).  dst may be device memory or pinned host memory. */
int kvc_block_gather(const void* src, int64_t planes, int64_t src_plane_stride,
                     int64_t block_bytes, const int32_t* block_ids, int64_t n,
                     void* dst, int64_t dst_item_stride, int64_t dst_plane_stride,
                     kvc_stream_t stream);

/* Scatter: dst[p][block_ids[i]] = src[i][p].  Replaces the index_copy_ of
 * ModelRunner.offload_get (model_runner.py:300-305) and import_kv
 * (pd/kv_channel.py:72-82).  src may be device or pinned host memory. */
int kvc_block_scatter(const void* src, int64_t src_item_stride, int64_t src_plane_stride,
                      int64_t planes, int64_t block_bytes, const int32_t* block_ids, int64_t n,
                      void* dst, int64_t dst_plane_stride, kvc_stream_t stream);

/* In-HBM copy pool[p][dst_ids[i]] = pool[p][src_ids[i]] (no reference
 * function; the closed form of a compaction step).  The id sets must be
 * disjoint (the caller stages overlapping lists). */
int kvc_block_copy(void* pool, int64_t planes, int64_t plane_stride, int64_t block_bytes,
                   const int32_t* src_ids, const int32_t* dst_ids, int64_t n,
                   kvc_stream_t stream);

/* DMA form of the offload byte moves: one strided 2-D copy per block on the
 * copy engines, block ids read from HOST memory (the block manager's ints).
 * d2h: host_dst + i*host_item_stride <- pool planes of block host_ids[i].
 * h2d: pool planes of block host_ids[i] <- host_src + i*host_item_stride.
 * Each item is `planes` rows of block_bytes (host side packed). */
int kvc_block_d2h(const void* pool, int64_t planes, int64_t plane_stride, int64_t block_bytes,
                  const int64_t* host_ids, int64_t n, void* host_dst, int64_t host_item_stride,
                  kvc_stream_t stream);
int kvc_block_h2d(const void* host_src, int64_t host_item_stride, int64_t planes,
                  int64_t block_bytes, const int64_t* host_ids, int64_t n, void* pool,
                  int64_t plane_stride, kvc_stream_t stream);

/* ---------------------------------------------------------------------------
 * The step that feeds the path: q/k RMSNorm + rotary embedding + KV append.
 * ------------------------------------------------------------------------- */

/* Replaces, in one launch, Qwen3Attention.forward's sequence between the qkv
 * projection and attention (nanovllm/models/qwen3.py:77-86):
 *   q = q_norm(q); k = k_norm(k)                 (nanovllm/layers/layernorm.py:18-26)
 *   q, k = rotary_emb(positions, q, k)           (nanovllm/layers/rotary_embedding.py:7-15,
 *                                                 :38-49, neox halves)
 *   store_kvcache(k, v, k_cache, v_cache, slots) (nanovllm/layers/attention.py:9-30)
 * q/k/v are bf16 [num_tokens, heads, 128] with their own element strides
 * (views of the fused qkv projection need no copy).  Per (token, head):
 *   xf = float(x); r = 1 / sqrt(sum(xf^2) / 128 + eps)   (IEEE sqrt and divide)
 *   y = bf16(bf16(xf * r) * w)                            (skipped when w is NULL)
 *   out = bf16(y1 * c - y2 * s | y2 * c + y1 * s)         (c, s = cos_sin_cache[pos])
 * cos_sin_cache is fp32 [max_position, 128] (cos in 0..63, sin in 64..127),
 * as RotaryEmbedding builds it.  q_out receives the rotated q; k_out (may be
 * NULL) the rotated k.  With k_cache/v_cache non-NULL, the rotated k and the
 * unchanged v are appended at slot_mapping like kvc_store_kv (negative slots
 * wrap, slots outside [0, num_slots) are skipped).  A negative position wraps
 * like a Python index; one still outside the cache yields NaN rows (torch
 * raises IndexError).  position/slot index bytes: 4 or 8. */
int kvc_qk_norm_rope_store(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                           const void* k, int64_t k_stride_t, int64_t k_stride_h,
                           const void* v, int64_t v_stride_t, int64_t v_stride_h,
                           int64_t num_tokens, int64_t num_heads, int64_t num_kv_heads,
                           int64_t head_dim, const void* positions, int position_index_bytes,
                           const void* q_norm_weight, const void* k_norm_weight, float eps,
                           const float* cos_sin_cache, int64_t max_position, void* q_out,
                           int64_t q_out_stride_t, int64_t q_out_stride_h, void* k_out,
                           int64_t k_out_stride_t, int64_t k_out_stride_h, void* k_cache,
                           void* v_cache, int64_t num_slots, const void* slot_mapping,
                           int slot_index_bytes, kvc_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVC_H_ */
