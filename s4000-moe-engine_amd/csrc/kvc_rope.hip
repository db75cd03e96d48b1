// Fused q/k RMSNorm + rotary embedding + KV append for gfx950: the step that
// feeds the paged KV path.  One pass over the fused qkv projection replaces
// the engine's four launches per layer (q_norm, k_norm, rotary_emb,
// store_kvcache) and the full-activation round trips between them.
//
// Work unit: a 16-lane group owns one (token, head row).  Rows 0 .. H-1 are
// q heads, H .. H+KVH-1 k heads, H+KVH .. H+2KVH-1 v heads.  In a q/k row
// lane j holds dims 4 j .. 4 j + 3 and 64 + 4 j .. 64 + 4 j + 3, so the
// rotation's pairs (i, i + 64) never leave a lane; the RMS over 128 dims is a
// 16-lane butterfly of DPP moves.
//
// Arithmetic follows the engine's torch ops in their order, each result
// rounded where torch rounds it:
//   RMSNorm (nanovllm/layers/layernorm.py:18-26):
//     xf = float(x); var = sum(xf * xf) / 128; r = 1 / sqrt(var + eps)
//     y = bf16(xf * r); y = bf16(float(y) * float(w))
//   RoPE, neox halves (nanovllm/layers/rotary_embedding.py:7-15, :38-49):
//     x1, x2 = halves of float(y); c, s = cos_sin_cache[pos] halves (fp32)
//     out1 = bf16(x1 * c - x2 * s); out2 = bf16(x2 * c + x1 * s)
// with no contraction into fma (the library is built -ffp-contract=off) and
// an IEEE square root and division.  The only freedom is the order of the
// 128-term sum of squares.
#include "kvc_internal.h"

namespace kvc {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kLanes = 16;
constexpr int kRowsPerBlock = kThreads / kLanes;

struct RopeArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* k;
  int64_t k_st, k_sh;
  const uint16_t* v;
  int64_t v_st, v_sh;
  const void* positions;
  const uint16_t* q_w;  // bf16 [128] or null (no norm)
  const uint16_t* k_w;
  const float* cos_sin;  // fp32 [max_position, 128]: cos in dims 0..63, sin in 64..127
  int64_t max_position;
  float eps;
  uint16_t* q_out;
  int64_t qo_st, qo_sh;
  uint16_t* k_out;  // may be null
  int64_t ko_st, ko_sh;
  uint16_t* k_cache;  // [num_slots, KVH, 128] or null (no append)
  uint16_t* v_cache;
  int64_t num_slots;
  const void* slots;
  int64_t num_tokens;
  int num_heads, num_kv_heads;
};

// bf16 round trip with the hardware round-to-nearest-even conversion
// (v_cvt_pk_bf16_f32): the rounding torch's .to(bfloat16) applies to every
// finite value.
__device__ __forceinline__ float round_bf16(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}

// Sum over a 16-lane row without LDS: the xor-1 and xor-2 partners through
// quad permutes, then the other quad of each half (row_half_mirror) and the
// other half (row_mirror).  After the quad steps every lane of a quad holds
// the same value, so each mirror adds exactly what the xor-4 / xor-8 partner
// of a butterfly would: the same sums, in the same order, as the butterfly.
__device__ __forceinline__ float sum16(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));
  return x;
}

__device__ __forceinline__ void unpack4(const u32x2_t& w, float* x) {
  x[0] = bf16_bits_to_f32(w[0] & 0xffffu);
  x[1] = bf16_bits_to_f32(w[0] >> 16);
  x[2] = bf16_bits_to_f32(w[1] & 0xffffu);
  x[3] = bf16_bits_to_f32(w[1] >> 16);
}

// One workgroup per token: the token's position, slot and row bases are
// wave-uniform (scalar) values, and 16-lane group g takes rows g, g + 16,
// g + 32, ... with every row's loads issued before any is computed.  Lane j
// of a q/k row holds dims 4 j .. 4 j + 3 (x1) and 64 + 4 j .. (x2), so each
// rotation pair sits in one lane; v rows are copied 16 bytes per lane.
constexpr int kMaxRowsPerGroup = 4;  // heads + 2 kv heads <= 64

template <int kPosBytes, int kSlotBytes>
__global__ void __launch_bounds__(kThreads) qk_norm_rope_store_kernel(RopeArgs a) {
  const int j = threadIdx.x & (kLanes - 1);
  const int g = threadIdx.x / kLanes;
  const int64_t n = blockIdx.x;
  const int rows = a.num_heads + 2 * a.num_kv_heads;
  const bool has_cache = a.k_cache != nullptr;
  // Token-uniform values.
  const uint16_t* qn = a.q + n * a.q_st;
  const uint16_t* kn = a.k + n * a.k_st;
  const uint16_t* vn = a.v + n * a.v_st;
  int64_t sl = -1;
  if (has_cache) {
    sl = wrap_slot(uniform(load_index<kSlotBytes>(a.slots, n)), a.num_slots);
    if (sl >= a.num_slots) sl = -1;
  }
  // A negative position wraps like a Python index; one still outside the
  // cache (torch raises IndexError there) reads nothing and yields NaN.
  const int64_t p = wrap_slot(uniform(load_index<kPosBytes>(a.positions, n)), a.max_position);
  const bool pos_ok = p >= 0 && p < a.max_position;

  // Phase 1: every load of this group's rows.
  u32x2_t lo[kMaxRowsPerGroup], hi[kMaxRowsPerGroup];
#pragma unroll
  for (int u = 0; u < kMaxRowsPerGroup; ++u) {
    const int r = g + kRowsPerBlock * u;
    lo[u] = hi[u] = u32x2_t{0u, 0u};
    if (r >= rows) continue;
    const int vrow = r - a.num_heads - a.num_kv_heads;
    if (vrow >= 0) {
      if (sl >= 0) {
        const uint16_t* src = vn + vrow * a.v_sh + 8 * j;
        lo[u] = reinterpret_cast<const u32x2_t*>(src)[0];
        hi[u] = reinterpret_cast<const u32x2_t*>(src)[1];
      }
    } else {
      const uint16_t* src = r < a.num_heads ? qn + r * a.q_sh : kn + (r - a.num_heads) * a.k_sh;
      lo[u] = *reinterpret_cast<const u32x2_t*>(src + 4 * j);
      hi[u] = *reinterpret_cast<const u32x2_t*>(src + kD / 2 + 4 * j);
    }
  }
  const float* cs = a.cos_sin + (pos_ok ? p : 0) * kD + 4 * j;
  const float4 c4 = *reinterpret_cast<const float4*>(cs);
  const float4 s4 = *reinterpret_cast<const float4*>(cs + kD / 2);
  float c[4] = {c4.x, c4.y, c4.z, c4.w};
  float s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = pos_ok ? c[i] : __builtin_nanf("");
    s[i] = pos_ok ? s[i] : __builtin_nanf("");
  }

  // Phase 2: normalise, rotate, store.
#pragma unroll
  for (int u = 0; u < kMaxRowsPerGroup; ++u) {
    const int r = g + kRowsPerBlock * u;
    if (r >= rows) continue;  // whole 16-lane groups skip together
    const int vrow = r - a.num_heads - a.num_kv_heads;
    if (vrow >= 0) {
      // v head: appended as is.
      if (sl >= 0) {
        u32x2_t* dst = reinterpret_cast<u32x2_t*>(a.v_cache + (sl * a.num_kv_heads + vrow) * kD + 8 * j);
        dst[0] = lo[u];
        dst[1] = hi[u];
      }
      continue;
    }
    const bool isq = r < a.num_heads;
    const int h = isq ? r : r - a.num_heads;
    float x1[4], x2[4];
    unpack4(lo[u], x1);
    unpack4(hi[u], x2);
    const uint16_t* w = isq ? a.q_w : a.k_w;
    if (w != nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += x1[i] * x1[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += x2[i] * x2[i];
      ss = sum16(ss);
      const float var = ss / float(kD);
      const float rinv = 1.f / __fsqrt_rn(var + a.eps);
      float w1[4], w2[4];
      unpack4(*reinterpret_cast<const u32x2_t*>(w + 4 * j), w1);
      unpack4(*reinterpret_cast<const u32x2_t*>(w + kD / 2 + 4 * j), w2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x1[i] = round_bf16(round_bf16(x1[i] * rinv) * w1[i]);
        x2[i] = round_bf16(round_bf16(x2[i] * rinv) * w2[i]);
      }
    }
    float y1[4], y2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a1 = x1[i] * c[i];
      const float b1 = x2[i] * s[i];
      y1[i] = a1 - b1;
      const float a2 = x2[i] * c[i];
      const float b2 = x1[i] * s[i];
      y2[i] = a2 + b2;
    }
    const u32x2_t plo = u32x2_t{pack_bf16x2_fast(y1[0], y1[1]), pack_bf16x2_fast(y1[2], y1[3])};
    const u32x2_t phi = u32x2_t{pack_bf16x2_fast(y2[0], y2[1]), pack_bf16x2_fast(y2[2], y2[3])};
    auto put = [&](uint16_t* row) {
      *reinterpret_cast<u32x2_t*>(row + 4 * j) = plo;
      *reinterpret_cast<u32x2_t*>(row + kD / 2 + 4 * j) = phi;
    };
    if (isq) {
      put(a.q_out + n * a.qo_st + h * a.qo_sh);
    } else {
      if (a.k_out != nullptr) put(a.k_out + n * a.ko_st + h * a.ko_sh);
      if (sl >= 0) put(a.k_cache + (sl * a.num_kv_heads + h) * kD);
    }
  }
}

template <int kPosBytes>
void launch_rope(const RopeArgs& a, int slot_bytes, dim3 grid, hipStream_t st) {
  if (slot_bytes == 8) {
    qk_norm_rope_store_kernel<kPosBytes, 8><<<grid, kThreads, 0, st>>>(a);
  } else {
    qk_norm_rope_store_kernel<kPosBytes, 4><<<grid, kThreads, 0, st>>>(a);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_qk_norm_rope_store(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
    int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
    int64_t num_tokens, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
    const void* positions, int position_index_bytes, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const float* cos_sin_cache, int64_t max_position,
    void* q_out, int64_t q_out_stride_t, int64_t q_out_stride_h, void* k_out,
    int64_t k_out_stride_t, int64_t k_out_stride_h, void* k_cache, void* v_cache,
    int64_t num_slots, const void* slot_mapping, int slot_index_bytes, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "qk_norm_rope_store: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(num_tokens >= 0 && num_heads > 0 && num_kv_heads > 0, KVC_ERR_VALUE,
              "qk_norm_rope_store: bad head counts");
  KVC_REQUIRE(position_index_bytes == 4 || position_index_bytes == 8, KVC_ERR_VALUE,
              "qk_norm_rope_store: positions must be int32 or int64");
  if (num_tokens == 0) return KVC_OK;  // empty tensors may carry null pointers
  KVC_REQUIRE(q != nullptr && k != nullptr && q_out != nullptr && positions != nullptr &&
                  cos_sin_cache != nullptr,
              KVC_ERR_VALUE, "qk_norm_rope_store: missing q, k, q_out, positions or cache");
  const bool cache = k_cache != nullptr || v_cache != nullptr;
  if (cache) {
    KVC_REQUIRE(k_cache != nullptr && v_cache != nullptr && v != nullptr &&
                    slot_mapping != nullptr,
                KVC_ERR_VALUE, "qk_norm_rope_store: the append needs v, both caches and slots");
    KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
                "qk_norm_rope_store: slot_mapping must be int32 or int64");
    KVC_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && aligned16(v) &&
                    v_stride_t % 8 == 0 && v_stride_h % 8 == 0,
                KVC_ERR_ASSERT, "qk_norm_rope_store: v rows and caches must be 16-byte aligned");
  }
  KVC_REQUIRE(aligned16(q) && aligned16(k) && aligned16(q_out) && q_stride_t % 8 == 0 &&
                  q_stride_h % 8 == 0 && k_stride_t % 8 == 0 && k_stride_h % 8 == 0 &&
                  q_out_stride_t % 8 == 0 && q_out_stride_h % 8 == 0,
              KVC_ERR_ASSERT, "qk_norm_rope_store: q/k rows must be 16-byte aligned");
  KVC_REQUIRE(k_out == nullptr || (aligned16(k_out) && k_out_stride_t % 8 == 0 &&
                                   k_out_stride_h % 8 == 0),
              KVC_ERR_ASSERT, "qk_norm_rope_store: k_out rows must be 16-byte aligned");
  KVC_REQUIRE((q_norm_weight == nullptr || aligned16(q_norm_weight)) &&
                  (k_norm_weight == nullptr || aligned16(k_norm_weight)) &&
                  aligned16(cos_sin_cache),
              KVC_ERR_ASSERT, "qk_norm_rope_store: weights and cache must be 16-byte aligned");
  RopeArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k = static_cast<const uint16_t*>(k);
  a.k_st = k_stride_t;
  a.k_sh = k_stride_h;
  a.v = static_cast<const uint16_t*>(v);
  a.v_st = v_stride_t;
  a.v_sh = v_stride_h;
  a.positions = positions;
  a.q_w = static_cast<const uint16_t*>(q_norm_weight);
  a.k_w = static_cast<const uint16_t*>(k_norm_weight);
  a.cos_sin = cos_sin_cache;
  a.max_position = max_position;
  a.eps = eps;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.qo_st = q_out_stride_t;
  a.qo_sh = q_out_stride_h;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.ko_st = k_out_stride_t;
  a.ko_sh = k_out_stride_h;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.num_slots = num_slots;
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.num_heads = int(num_heads);
  a.num_kv_heads = int(num_kv_heads);
  KVC_REQUIRE(num_heads + 2 * num_kv_heads <= kRowsPerBlock * kMaxRowsPerGroup, KVC_ERR_VALUE,
              "qk_norm_rope_store: at most %d q + 2 kv heads", kRowsPerBlock * kMaxRowsPerGroup);
  KVC_REQUIRE(num_tokens < (int64_t(1) << 31), KVC_ERR_VALUE, "qk_norm_rope_store: too many tokens");
  const dim3 grid{unsigned(num_tokens)};  // one workgroup per token
  hipStream_t st = as_stream(stream);
  const int sb = cache ? slot_index_bytes : 4;
  if (position_index_bytes == 8) {
    launch_rope<8>(a, sb, grid, st);
  } else {
    launch_rope<4>(a, sb, grid, st);
  }
  return check_launch("qk_norm_rope_store");
}
