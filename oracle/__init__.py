"""CPU oracle of the paged KV-cache hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (byte and integer work, fp32 attention arithmetic)
and CPU torch (only where it restates the engine's own torch CPU path), of the
reference algorithms this repository's HIP kernels replace.  Each function
cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the results the tests compare against or as the timed
CPU baseline — never as a product code path.  The product (s4000-moe-engine_amd/nanovllm_amd) has no
CPU fallback and raises if libkvc.so is missing.

How each function is pinned (checked in tests/test_oracle.py):
  store_kvcache            closed form (row i of the flat cache equals token
                           row j exactly where slot_mapping[j] == i) and a
                           brute-force loop; negative slots against Python
                           indexing.
  quant_tokhead            known answers: exact half-way ties (half to even),
                           the 1e-6 clamp, the IEEE-divide edge of amax/127,
                           saturation; against Python's round() on the fp32
                           quotient.
  quant_chan / store_int8_chan
                           known answers: half-way ties round up, negative
                           ties toward +inf, outlier dims zeroed, side values
                           exact; the seeded tests/p17_kv_int8.py unit case.
  dequant_*                closed form code * scale with bf16 RNE (checked
                           against torch's bf16 cast).
  calib_stats / calib_fold / calib_freeze
                           the engine hook's own torch statements
                           (model_runner.py:527-533: torch's bf16 sum per
                           forward, fp32 fold) over forwards of different
                           lengths, bit for bit; two dims whose outlier
                           decision flips with the per-forward bf16 rounding;
                           the calibration of tests/p17_kv_int8.py:80-101 on
                           its seeded unit case; known answers at the ratio
                           threshold (10 is not an outlier, the first
                           n_out_max dims in index order win), the 1e-6
                           clamps.
  f64_to_bf16_value        torch's fp32 -> bf16 cast on fp32-exact values
                           (ties, subnormals, overflow) and known answers a
                           double rounding through fp32 would miss.
  paged_decode_ref         float64 torch scaled_dot_product_attention; closed
                           forms (one key -> V row; identical keys -> mean of
                           V); a NaN-poisoned tail never read; the reference
                           tests' page-boundary length matrix.
  prefill_ref / mixed_ref  float64 SDPA with the causal-with-prefix boolean
                           mask; a zero-prefix chunk equals causal SDPA; the
                           mixed result equals decode rows + prefill rows.
  gather_sdpa_decode       equals paged_decode_ref within fp32 rounding.
  block_gather/scatter/copy closed forms (bytes equal), simultaneous-copy
                           semantics of a compaction with overlapping ids.
"""
