// KV append kernels: plain copy through slot_mapping, and the two int8
// quantise-on-append encodings.  All are HBM/launch bound; each thread moves
// whole 16-byte vectors where alignment allows.
#include "kvc_internal.h"

namespace kvc {
namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// Plain append.  Thread (token n, vector v) copies vector v of the token's
// [KVH, D] row for both K and V: source head h = v / vec_per_head, read with
// the tensor's own (stride_n, stride_h); destination is the contiguous cache
// row of slot_mapping[n].
// ---------------------------------------------------------------------------
template <typename Vec, int kIdxBytes>
__global__ void __launch_bounds__(kThreads)
store_kv_kernel(const char* __restrict__ key, int64_t k_sn, int64_t k_sh,
                const char* __restrict__ value, int64_t v_sn, int64_t v_sh,
                char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t num_slots,
                const void* __restrict__ slots, int64_t num_tokens, int vec_per_head,
                int vec_per_token, int64_t row_bytes) {
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t n = gid / vec_per_token;
  if (n >= num_tokens) return;
  const int v = int(gid - n * vec_per_token);
  const int h = v / vec_per_head;
  const int hv = v - h * vec_per_head;
  int64_t slot = wrap_slot(load_index<kIdxBytes>(slots, n), num_slots);
  if (slot < 0 || slot >= num_slots) return;
  const Vec kx = *reinterpret_cast<const Vec*>(key + n * k_sn + h * k_sh + int64_t(hv) * sizeof(Vec));
  const Vec vx = *reinterpret_cast<const Vec*>(value + n * v_sn + h * v_sh + int64_t(hv) * sizeof(Vec));
  const int64_t dst = slot * row_bytes + int64_t(v) * sizeof(Vec);
  *reinterpret_cast<Vec*>(k_cache + dst) = kx;
  *reinterpret_cast<Vec*>(v_cache + dst) = vx;
}

template <int kIdxBytes>
int launch_store_kv(int vec, const char* key, int64_t k_sn, int64_t k_sh, const char* value,
                    int64_t v_sn, int64_t v_sh, char* kc, char* vc, int64_t num_slots,
                    const void* slots, int64_t n, int64_t head_bytes, int64_t kvh,
                    hipStream_t st) {
  const int vec_per_head = int(head_bytes / vec);
  const int vec_per_token = int(vec_per_head * kvh);
  const int64_t total = n * vec_per_token;
  const dim3 grid(unsigned((total + kThreads - 1) / kThreads));
  const int64_t row = head_bytes * kvh;
#define KVC_STORE_CASE(BYTES, TYPE)                                                          \
  case BYTES:                                                                               \
    store_kv_kernel<TYPE, kIdxBytes><<<grid, kThreads, 0, st>>>(                            \
        key, k_sn, k_sh, value, v_sn, v_sh, kc, vc, num_slots, slots, n, vec_per_head,      \
        vec_per_token, row);                                                                \
    break;
  switch (vec) {
    KVC_STORE_CASE(16, u32x4_t)
    KVC_STORE_CASE(8, u32x2_t)
    KVC_STORE_CASE(4, uint32_t)
    KVC_STORE_CASE(2, uint16_t)
    default:
      set_error("store_kv: unsupported vector width %d", vec);
      return KVC_ERR_VALUE;
  }
#undef KVC_STORE_CASE
  return check_launch("store_kv");
}

// Largest power-of-two vector (<= 16 bytes) that divides every address and
// stride the copy kernel forms.
int pick_vec(std::initializer_list<int64_t> quantities) {
  int vec = 16;
  for (int64_t q : quantities) {
    while (vec > 1 && (q % vec) != 0) vec >>= 1;
  }
  return vec;
}

// ---------------------------------------------------------------------------
// int8 append.  A 16-lane group owns one (token, head) row of 128 values:
// lane j holds dims [8j, 8j+8) of K and of V (one 16-byte load each).
// ---------------------------------------------------------------------------
constexpr int kD = 128;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerBlock = kThreads / kLanesPerRow;

template <int kIdxBytes>
__global__ void __launch_bounds__(kThreads)
store_int8_tokhead_kernel(const uint16_t* __restrict__ key, int64_t k_sn, int64_t k_sh,
                          const uint16_t* __restrict__ value, int64_t v_sn, int64_t v_sh,
                          int8_t* __restrict__ k_cache, int8_t* __restrict__ v_cache,
                          float* __restrict__ k_scale, float* __restrict__ v_scale,
                          int64_t num_slots, const void* __restrict__ slots, int64_t num_tokens,
                          int kvh) {
  const int lane16 = threadIdx.x & (kLanesPerRow - 1);
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x / kLanesPerRow);
  const int64_t n = row / kvh;
  const int h = int(row - n * kvh);
  // Whole 16-lane groups share n, so the early exits keep groups intact.
  if (n >= num_tokens) return;
  int64_t slot = wrap_slot(load_index<kIdxBytes>(slots, n), num_slots);
  if (slot < 0 || slot >= num_slots) return;
  const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(key + n * k_sn + h * k_sh + lane16 * 8);
  const u32x4_t vw = *reinterpret_cast<const u32x4_t*>(value + n * v_sn + h * v_sh + lane16 * 8);
  float kx[8], vx[8];
  unpack8(kw, kx);
  unpack8(vw, vx);
  int kc[8], vc[8];
  const float ks = quant_tokhead_row(kx, kc);
  const float vs = quant_tokhead_row(vx, vc);
  const int64_t dst = (slot * kvh + h) * kD + lane16 * 8;
  *reinterpret_cast<u32x2_t*>(k_cache + dst) = u32x2_t{pack_codes4(kc, 0), pack_codes4(kc, 4)};
  *reinterpret_cast<u32x2_t*>(v_cache + dst) = u32x2_t{pack_codes4(vc, 0), pack_codes4(vc, 4)};
  if (lane16 == 0) {
    k_scale[slot * kvh + h] = ks;
    v_scale[slot * kvh + h] = vs;
  }
}

// Per-channel quantisation floor(x / s + 0.5) with outlier dims zeroed and
// their exact bf16 values written to the compacted side row.
template <int kIdxBytes>
__global__ void __launch_bounds__(kThreads)
store_int8_chan_kernel(const uint16_t* __restrict__ key, int64_t k_sn, int64_t k_sh,
                       const uint16_t* __restrict__ value, int64_t v_sn, int64_t v_sh,
                       int8_t* __restrict__ k_cache, int8_t* __restrict__ v_cache,
                       const float* __restrict__ k_scale, const float* __restrict__ v_scale,
                       uint16_t* __restrict__ side_k, uint16_t* __restrict__ side_v, int n_out_max,
                       const int32_t* __restrict__ out_idx2d, const int32_t* __restrict__ head_n_out,
                       int64_t num_slots, const void* __restrict__ slots, int64_t num_tokens,
                       int kvh) {
  const int lane16 = threadIdx.x & (kLanesPerRow - 1);
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x / kLanesPerRow);
  const int64_t n = row / kvh;
  const int h = int(row - n * kvh);
  if (n >= num_tokens) return;
  int64_t slot = wrap_slot(load_index<kIdxBytes>(slots, n), num_slots);
  if (slot < 0 || slot >= num_slots) return;
  const uint16_t* krow = key + n * k_sn + h * k_sh;
  const uint16_t* vrow = value + n * v_sn + h * v_sh;
  const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(krow + lane16 * 8);
  const u32x4_t vw = *reinterpret_cast<const u32x4_t*>(vrow + lane16 * 8);
  float kx[8], vx[8];
  unpack8(kw, kx);
  unpack8(vw, vx);
  const float4* ks4 = reinterpret_cast<const float4*>(k_scale + h * kD + lane16 * 8);
  const float4* vs4 = reinterpret_cast<const float4*>(v_scale + h * kD + lane16 * 8);
  const float4 ks0 = ks4[0], ks1 = ks4[1], vs0 = vs4[0], vs1 = vs4[1];
  const float ks[8] = {ks0.x, ks0.y, ks0.z, ks0.w, ks1.x, ks1.y, ks1.z, ks1.w};
  const float vs[8] = {vs0.x, vs0.y, vs0.z, vs0.w, vs1.x, vs1.y, vs1.z, vs1.w};
  int kc[8], vc[8];
  quant_chan8(kx, ks, kc);
  quant_chan8(vx, vs, vc);
  const int n_out = head_n_out != nullptr ? head_n_out[h] : 0;
  for (int j = 0; j < n_out; ++j) {
    const int d = out_idx2d[h * n_out_max + j];
    const int local = d - lane16 * 8;
    if (local >= 0 && local < 8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i == local) {
          kc[i] = 0;
          vc[i] = 0;
        }
      }
    }
  }
  if (lane16 < n_out) {
    const int d = out_idx2d[h * n_out_max + lane16];
    const int64_t so = (slot * kvh + h) * n_out_max + lane16;
    side_k[so] = krow[d];
    side_v[so] = vrow[d];
  }
  const int64_t dst = (slot * kvh + h) * kD + lane16 * 8;
  *reinterpret_cast<u32x2_t*>(k_cache + dst) = u32x2_t{pack_codes4(kc, 0), pack_codes4(kc, 4)};
  *reinterpret_cast<u32x2_t*>(v_cache + dst) = u32x2_t{pack_codes4(vc, 0), pack_codes4(vc, 4)};
}

// ---------------------------------------------------------------------------
// Dequantise gathered rows (torch-side read path).  Thread = 8 dims.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
dequant_chan_kernel(const int8_t* __restrict__ kv, const float* __restrict__ dscale,
                    const uint16_t* __restrict__ side, const int32_t* __restrict__ out_idx2d,
                    const int32_t* __restrict__ head_n_out, int n_out_max, int64_t rows, int kvh,
                    uint16_t* __restrict__ out) {
  const int lane16 = threadIdx.x & (kLanesPerRow - 1);
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x / kLanesPerRow);
  if (row >= rows) return;
  const int h = int(row % kvh);
  const u32x2_t c = *reinterpret_cast<const u32x2_t*>(kv + row * kD + lane16 * 8);
  const float* ds = dscale + h * kD + lane16 * 8;
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = c[i >> 2];
    e[i] = f32_to_bf16_bits(float(int8_t((word >> ((i & 3) * 8)) & 0xffu)) * ds[i]);
  }
  if (side != nullptr && head_n_out != nullptr) {
    // Outlier dims take the exact side value (a later j wins on duplicates,
    // like the sequential assignment of the torch path).
    const int n_out = head_n_out[h];
    for (int j = 0; j < n_out; ++j) {
      const int local = out_idx2d[h * n_out_max + j] - lane16 * 8;
      if (local >= 0 && local < 8) {
        const uint32_t sv = side[row * n_out_max + j];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (i == local) ? sv : e[i];
      }
    }
  }
  *reinterpret_cast<u32x4_t*>(out + row * kD + lane16 * 8) =
      u32x4_t{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
}

__global__ void __launch_bounds__(kThreads)
dequant_tokhead_kernel(const int8_t* __restrict__ kv, const float* __restrict__ scale,
                       int64_t rows, uint16_t* __restrict__ out) {
  const int lane16 = threadIdx.x & (kLanesPerRow - 1);
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x / kLanesPerRow);
  if (row >= rows) return;
  const float s = scale[row];
  const u32x2_t c = *reinterpret_cast<const u32x2_t*>(kv + row * kD + lane16 * 8);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = c[i >> 1];
    const int sh = (i & 1) * 16;
    o[i] = pack_bf16x2(float(int8_t((word >> sh) & 0xffu)) * s,
                       float(int8_t((word >> (sh + 8)) & 0xffu)) * s);
  }
  *reinterpret_cast<u32x4_t*>(out + row * kD + lane16 * 8) = u32x4_t{o[0], o[1], o[2], o[3]};
}

// ---------------------------------------------------------------------------
// Gather of every prefill chunk's keys out of the paged pool, dequantised to
// bf16 (the prefill's read of an int8 pool).  Block = 32 tokens of one kv
// head (blockIdx.y), so the head's scales and outlier dims are uniform;
// thread = 16 dims of one token's row of K and of V (8 threads a row).  The
// token's chunk is found by a binary search over cu_k (num_prefill + 1
// entries).
// ---------------------------------------------------------------------------
constexpr int kSideMaxStore = 8;  // side slots a gathered row takes (the attention's bound)
constexpr int kGatherLanes = 8;
constexpr int kGatherRows = kThreads / kGatherLanes;
// Token groups a block runs: two for the per-channel pool (its per-head read
// scales and outlier dims are loaded once for both; 14.8 against 19 us on four
// 256-token chunks after prefixes 0 / 512 / 2048 / 8192, 4 kv heads), one
// otherwise (10.3 against 11.7 us per-token-head).
template <int kEnc>
constexpr int gather_iters() { return kEnc == KVC_KV_INT8_CHAN ? 2 : 1; }

// One side-pool row (n_out_max bf16, up to 8) as 16-bit values: one aligned
// load for the power-of-two widths (a row then starts at a multiple of its
// size), else element by element.
__device__ __forceinline__ void load_side_row16(const uint16_t* row, int nom,
                                                uint32_t (&v)[kSideMaxStore]) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (nom == 8) {
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(row);
    w[0] = x[0], w[1] = x[1], w[2] = x[2], w[3] = x[3];
  } else if (nom == 4) {
    const u32x2_t x = *reinterpret_cast<const u32x2_t*>(row);
    w[0] = x[0], w[1] = x[1];
  } else if (nom == 2) {
    w[0] = *reinterpret_cast<const uint32_t*>(row);
  } else {
#pragma unroll
    for (int j = 0; j < kSideMaxStore; ++j)
      if (j < nom) w[j >> 1] |= uint32_t(row[j]) << ((j & 1) * 16);
  }
#pragma unroll
  for (int j = 0; j < kSideMaxStore; ++j) v[j] = (w[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

template <int kEnc>
__global__ void __launch_bounds__(kThreads)
gather_kv_kernel(const char* __restrict__ k_cache, const char* __restrict__ v_cache,
                 int64_t num_slots, int page, int kvh, const float* __restrict__ k_scale,
                 const float* __restrict__ v_scale, const uint16_t* __restrict__ side_k,
                 const uint16_t* __restrict__ side_v, const int32_t* __restrict__ out_idx2d,
                 const int32_t* __restrict__ head_n_out, int n_out_max,
                 const int32_t* __restrict__ block_tables, int64_t bt_stride, int max_blocks,
                 int64_t bt_row0, int num_prefill, const int32_t* __restrict__ cu_k,
                 int64_t tokens, uint16_t* __restrict__ out_k, uint16_t* __restrict__ out_v) {
  const int lane8 = threadIdx.x & (kGatherLanes - 1);
  const int h = int(blockIdx.y);
  // Per-block constants of head h: this thread's 16 read scales of K and V
  // (per-channel), the head's outlier dims relative to this thread's 16.
  float dsk[16], dsv[16];
  int n_out = 0;
  int dims[kSideMaxStore];
  if constexpr (kEnc == KVC_KV_INT8_CHAN) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      dsk[i] = k_scale[h * kD + lane8 * 16 + i];
      dsv[i] = v_scale[h * kD + lane8 * 16 + i];
    }
    if (head_n_out != nullptr) n_out = min(head_n_out[h], n_out_max);
#pragma unroll
    for (int j = 0; j < kSideMaxStore; ++j)
      dims[j] = j < n_out ? out_idx2d[h * n_out_max + j] - lane8 * 16 : -1;
  }
#pragma unroll
  for (int it = 0; it < gather_iters<kEnc>(); ++it) {
    const int64_t t =
        (int64_t(blockIdx.x) * gather_iters<kEnc>() + it) * kGatherRows +
        (threadIdx.x / kGatherLanes);
    if (t >= tokens) break;
    const int64_t row = t * kvh + h;
    // chunk i: the last with cu_k[i] <= t
    int lo = 0, hi = num_prefill - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cu_k[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int64_t key = t - cu_k[lo];
    const int64_t bi = key / page;
    const int64_t blk = bi < max_blocks ? block_tables[(bt_row0 + lo) * bt_stride + bi] : -1;
    const int64_t slot = blk * page + (key - bi * page);
    const bool ok = blk >= 0 && slot < num_slots;  // a bad table entry reads nothing
    const int64_t src = (slot * kvh + h) * kD + lane8 * 16;  // element index
    const int64_t dst = row * kD + lane8 * 16;
    uint32_t sk[kSideMaxStore], sv[kSideMaxStore];
    if constexpr (kEnc == KVC_KV_INT8_CHAN) {
      if (ok && n_out > 0) {
        load_side_row16(side_k + (slot * kvh + h) * n_out_max, n_out_max, sk);
        load_side_row16(side_v + (slot * kvh + h) * n_out_max, n_out_max, sv);
      }
    }
#pragma unroll
    for (int tensor = 0; tensor < 2; ++tensor) {
      const char* cache = tensor == 0 ? k_cache : v_cache;
      uint16_t* out = tensor == 0 ? out_k : out_v;
      u32x4_t o0 = u32x4_t{0u, 0u, 0u, 0u}, o1 = o0;
      if (ok) {
        if constexpr (kEnc == KVC_KV_BF16) {
          o0 = *reinterpret_cast<const u32x4_t*>(cache + src * 2);
          o1 = *reinterpret_cast<const u32x4_t*>(cache + src * 2 + 16);
        } else {
          const u32x4_t c = *reinterpret_cast<const u32x4_t*>(cache + src);
          float sc[16];
          if constexpr (kEnc == KVC_KV_INT8_TOKHEAD) {
            const float s1 = (tensor == 0 ? k_scale : v_scale)[slot * kvh + h];
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[i] = s1;
          } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[i] = tensor == 0 ? dsk[i] : dsv[i];
          }
          uint32_t e[16];
#pragma unroll
          for (int i = 0; i < 16; ++i)
            e[i] = f32_to_bf16_bits(float(int8_t((c[i >> 2] >> ((i & 3) * 8)) & 0xffu)) * sc[i]);
          o0 = u32x4_t{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                       e[6] | (e[7] << 16)};
          o1 = u32x4_t{e[8] | (e[9] << 16), e[10] | (e[11] << 16), e[12] | (e[13] << 16),
                       e[14] | (e[15] << 16)};
        }
      }
      *reinterpret_cast<u32x4_t*>(out + dst) = o0;
      *reinterpret_cast<u32x4_t*>(out + dst + 8) = o1;
      if constexpr (kEnc == KVC_KV_INT8_CHAN) {
        // The head's outlier dims in this thread's 16 take the side values,
        // written over the row just stored (one thread's stores to an address
        // land in order), slot by slot: a later slot wins on a duplicate dim,
        // as the sequential assignment does.
#pragma unroll
        for (int j = 0; j < kSideMaxStore; ++j) {
          if (j < n_out && ok && dims[j] >= 0 && dims[j] < 16)
            out[dst + dims[j]] = uint16_t(tensor == 0 ? sk[j] : sv[j]);
        }
      }
    }
  }
}

int check_int8_args(const void* key, int64_t k_sn, int64_t k_sh, const void* value, int64_t v_sn,
                    int64_t v_sh, int64_t num_tokens, int64_t kvh, int64_t head_dim,
                    int slot_bytes, const char* what) {
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "%s: head_dim must be 128 (got %lld)", what,
              (long long)head_dim);
  KVC_REQUIRE(num_tokens >= 0 && kvh > 0, KVC_ERR_VALUE, "%s: bad token/head count", what);
  KVC_REQUIRE(slot_bytes == 4 || slot_bytes == 8, KVC_ERR_VALUE,
              "%s: slot_mapping must be int32 or int64", what);
  const bool aligned = (reinterpret_cast<uintptr_t>(key) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(value) % 16 == 0) && (k_sn * 2) % 16 == 0 &&
                       (k_sh * 2) % 16 == 0 && (v_sn * 2) % 16 == 0 && (v_sh * 2) % 16 == 0;
  KVC_REQUIRE(aligned, KVC_ERR_ASSERT,
              "%s: key/value rows must be 16-byte aligned (base and strides)", what);
  return KVC_OK;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_store_kv(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                            const void* value, int64_t value_stride_n, int64_t value_stride_h,
                            void* k_cache, void* v_cache, int64_t num_slots,
                            const void* slot_mapping, int slot_index_bytes, int64_t num_tokens,
                            int64_t num_kv_heads, int64_t head_dim, int elem_bytes,
                            kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(elem_bytes == 2 || elem_bytes == 4, KVC_ERR_VALUE,
              "store_kv: element size must be 2 or 4 bytes (got %d)", elem_bytes);
  KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
              "store_kv: slot_mapping must be int32 or int64");
  KVC_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0, KVC_ERR_VALUE,
              "store_kv: bad shape");
  if (num_tokens == 0) return KVC_OK;
  const int64_t eb = elem_bytes;
  const int64_t head_bytes = head_dim * eb;
  const int vec = pick_vec({int64_t(reinterpret_cast<uintptr_t>(key)),
                            int64_t(reinterpret_cast<uintptr_t>(value)),
                            int64_t(reinterpret_cast<uintptr_t>(k_cache)),
                            int64_t(reinterpret_cast<uintptr_t>(v_cache)), key_stride_n * eb,
                            key_stride_h * eb, value_stride_n * eb, value_stride_h * eb,
                            head_bytes});
  KVC_REQUIRE(vec >= 2, KVC_ERR_ASSERT, "store_kv: rows are not 2-byte aligned");
  const char* k = static_cast<const char*>(key);
  const char* v = static_cast<const char*>(value);
  if (slot_index_bytes == 8) {
    return launch_store_kv<8>(vec, k, key_stride_n * eb, key_stride_h * eb, v,
                              value_stride_n * eb, value_stride_h * eb,
                              static_cast<char*>(k_cache), static_cast<char*>(v_cache), num_slots,
                              slot_mapping, num_tokens, head_bytes, num_kv_heads,
                              as_stream(stream));
  }
  return launch_store_kv<4>(vec, k, key_stride_n * eb, key_stride_h * eb, v, value_stride_n * eb,
                            value_stride_h * eb, static_cast<char*>(k_cache),
                            static_cast<char*>(v_cache), num_slots, slot_mapping, num_tokens,
                            head_bytes, num_kv_heads, as_stream(stream));
}

extern "C" int kvc_store_int8_tokhead(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                                      const void* value, int64_t value_stride_n,
                                      int64_t value_stride_h, int8_t* k_cache, int8_t* v_cache,
                                      float* k_scale, float* v_scale, int64_t num_slots,
                                      const void* slot_mapping, int slot_index_bytes,
                                      int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                                      kvc_stream_t stream) {
  clear_error();
  int rc = check_int8_args(key, key_stride_n, key_stride_h, value, value_stride_n,
                           value_stride_h, num_tokens, num_kv_heads, head_dim, slot_index_bytes,
                           "store_int8_tokhead");
  if (rc != KVC_OK) return rc;
  if (num_tokens == 0) return KVC_OK;
  const int64_t rows = num_tokens * num_kv_heads;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const auto* k = static_cast<const uint16_t*>(key);
  const auto* v = static_cast<const uint16_t*>(value);
  if (slot_index_bytes == 8) {
    store_int8_tokhead_kernel<8><<<grid, kThreads, 0, as_stream(stream)>>>(
        k, key_stride_n, key_stride_h, v, value_stride_n, value_stride_h, k_cache, v_cache,
        k_scale, v_scale, num_slots, slot_mapping, num_tokens, int(num_kv_heads));
  } else {
    store_int8_tokhead_kernel<4><<<grid, kThreads, 0, as_stream(stream)>>>(
        k, key_stride_n, key_stride_h, v, value_stride_n, value_stride_h, k_cache, v_cache,
        k_scale, v_scale, num_slots, slot_mapping, num_tokens, int(num_kv_heads));
  }
  return check_launch("store_int8_tokhead");
}

extern "C" int kvc_store_int8_chan(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                                   const void* value, int64_t value_stride_n,
                                   int64_t value_stride_h, int8_t* k_cache, int8_t* v_cache,
                                   const float* k_scale, const float* v_scale, void* side_k,
                                   void* side_v, int64_t n_out_max, const int32_t* out_idx2d,
                                   const int32_t* head_n_out, int64_t num_slots,
                                   const void* slot_mapping, int slot_index_bytes,
                                   int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                                   kvc_stream_t stream) {
  clear_error();
  int rc = check_int8_args(key, key_stride_n, key_stride_h, value, value_stride_n,
                           value_stride_h, num_tokens, num_kv_heads, head_dim, slot_index_bytes,
                           "store_int8_chan");
  if (rc != KVC_OK) return rc;
  KVC_REQUIRE(n_out_max >= 0 && n_out_max <= kLanesPerRow, KVC_ERR_VALUE,
              "store_int8_chan: n_out_max must be in [0, 16] (got %lld)", (long long)n_out_max);
  KVC_REQUIRE(head_n_out == nullptr || (side_k != nullptr && side_v != nullptr &&
                                        out_idx2d != nullptr),
              KVC_ERR_VALUE, "store_int8_chan: outlier dims need side pools and out_idx2d");
  if (num_tokens == 0) return KVC_OK;
  const int64_t rows = num_tokens * num_kv_heads;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const auto* k = static_cast<const uint16_t*>(key);
  const auto* v = static_cast<const uint16_t*>(value);
  auto* sk = static_cast<uint16_t*>(side_k);
  auto* sv = static_cast<uint16_t*>(side_v);
  if (slot_index_bytes == 8) {
    store_int8_chan_kernel<8><<<grid, kThreads, 0, as_stream(stream)>>>(
        k, key_stride_n, key_stride_h, v, value_stride_n, value_stride_h, k_cache, v_cache,
        k_scale, v_scale, sk, sv, int(n_out_max), out_idx2d, head_n_out, num_slots,
        slot_mapping, num_tokens, int(num_kv_heads));
  } else {
    store_int8_chan_kernel<4><<<grid, kThreads, 0, as_stream(stream)>>>(
        k, key_stride_n, key_stride_h, v, value_stride_n, value_stride_h, k_cache, v_cache,
        k_scale, v_scale, sk, sv, int(n_out_max), out_idx2d, head_n_out, num_slots,
        slot_mapping, num_tokens, int(num_kv_heads));
  }
  return check_launch("store_int8_chan");
}

extern "C" int kvc_dequant_chan(const int8_t* kv, const float* dscale, const void* side,
                                const int32_t* out_idx2d, const int32_t* head_n_out,
                                int64_t n_out_max, int64_t num_tokens, int64_t num_kv_heads,
                                int64_t head_dim, void* out, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "dequant_chan: head_dim must be 128");
  KVC_REQUIRE(n_out_max >= 0 && n_out_max <= kLanesPerRow, KVC_ERR_VALUE,
              "dequant_chan: n_out_max must be in [0, 16]");
  const int64_t rows = num_tokens * num_kv_heads;
  if (rows == 0) return KVC_OK;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  dequant_chan_kernel<<<grid, kThreads, 0, as_stream(stream)>>>(
      kv, dscale, static_cast<const uint16_t*>(side), out_idx2d, head_n_out, int(n_out_max), rows,
      int(num_kv_heads), static_cast<uint16_t*>(out));
  return check_launch("dequant_chan");
}

extern "C" int kvc_dequant_tokhead(const int8_t* kv, const float* scale, int64_t num_tokens,
                                   int64_t num_kv_heads, int64_t head_dim, void* out,
                                   kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "dequant_tokhead: head_dim must be 128");
  const int64_t rows = num_tokens * num_kv_heads;
  if (rows == 0) return KVC_OK;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  dequant_tokhead_kernel<<<grid, kThreads, 0, as_stream(stream)>>>(kv, scale, rows,
                                                                   static_cast<uint16_t*>(out));
  return check_launch("dequant_tokhead");
}

extern "C" int kvc_gather_kv(const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                             int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
                             int kv_dtype, const float* k_scale, const float* v_scale,
                             const void* side_k, const void* side_v, const int32_t* out_idx2d,
                             const int32_t* head_n_out, int64_t n_out_max,
                             const int32_t* block_tables, int64_t bt_stride,
                             int64_t max_blocks_per_seq, int64_t block_table_row0,
                             int64_t num_prefill, const int32_t* cu_seqlens_k,
                             int64_t total_keys, void* out_k, void* out_v, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "gather_kv: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(num_kv_heads > 0 && num_kv_heads < 65536 && page_size > 0 && num_cache_blocks >= 0,
              KVC_ERR_VALUE,
              "gather_kv: bad pool geometry");
  KVC_REQUIRE(num_prefill >= 0 && total_keys >= 0 && block_table_row0 >= 0, KVC_ERR_VALUE,
              "gather_kv: bad chunk count / key total / table row");
  KVC_REQUIRE(kv_dtype == KVC_KV_BF16 || kv_dtype == KVC_KV_INT8_TOKHEAD ||
                  kv_dtype == KVC_KV_INT8_CHAN,
              KVC_ERR_VALUE, "gather_kv: unknown kv_dtype %d", kv_dtype);
  if (num_prefill == 0 || total_keys == 0) return KVC_OK;
  KVC_REQUIRE(k_cache && v_cache && block_tables && cu_seqlens_k && out_k && out_v,
              KVC_ERR_VALUE, "gather_kv: null pointer");
  KVC_REQUIRE(kv_dtype == KVC_KV_BF16 || (k_scale && v_scale), KVC_ERR_VALUE,
              "gather_kv: int8 pools need their scales");
  if (kv_dtype == KVC_KV_INT8_CHAN && head_n_out != nullptr) {
    KVC_REQUIRE(side_k && side_v && out_idx2d && n_out_max >= 1 && n_out_max <= kSideMaxStore,
                KVC_ERR_VALUE,
                "gather_kv: head_n_out needs side_k, side_v, out_idx2d and n_out_max in [1, %d]",
                kSideMaxStore);
  }
  KVC_REQUIRE(max_blocks_per_seq > 0 && max_blocks_per_seq <= bt_stride, KVC_ERR_VALUE,
              "gather_kv: max_blocks_per_seq must be in [1, bt_stride]");
  auto launch = [&](auto kern, int iters) {
    const int64_t per_block = int64_t(kGatherRows) * iters;
    const dim3 grid(unsigned((total_keys + per_block - 1) / per_block), unsigned(num_kv_heads));
    kern<<<grid, kThreads, 0, as_stream(stream)>>>(
        static_cast<const char*>(k_cache), static_cast<const char*>(v_cache),
        num_cache_blocks * page_size, int(page_size), int(num_kv_heads), k_scale, v_scale,
        static_cast<const uint16_t*>(side_k), static_cast<const uint16_t*>(side_v), out_idx2d,
        kv_dtype == KVC_KV_INT8_CHAN ? head_n_out : nullptr, int(n_out_max), block_tables,
        bt_stride, int(max_blocks_per_seq), block_table_row0, int(num_prefill), cu_seqlens_k,
        total_keys, static_cast<uint16_t*>(out_k), static_cast<uint16_t*>(out_v));
  };
  if (kv_dtype == KVC_KV_BF16) {
    launch(gather_kv_kernel<KVC_KV_BF16>, gather_iters<KVC_KV_BF16>());
  } else if (kv_dtype == KVC_KV_INT8_TOKHEAD) {
    launch(gather_kv_kernel<KVC_KV_INT8_TOKHEAD>, gather_iters<KVC_KV_INT8_TOKHEAD>());
  } else {
    launch(gather_kv_kernel<KVC_KV_INT8_CHAN>, gather_iters<KVC_KV_INT8_CHAN>());
  }
  return check_launch("gather_kv");
}
