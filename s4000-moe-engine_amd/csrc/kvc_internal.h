// Shared device and host helpers of libkvc (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "kvc.h"

namespace kvc {

// ---------------------------------------------------------------------------
// Host-side error plumbing: every entry point returns a kvc_status and leaves
// a message in a thread-local buffer.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define KVC_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::kvc::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)

// Launch-time error check (configuration errors surface synchronously; no
// host synchronisation is performed).
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return KVC_ERR_RUNTIME;
  }
  return KVC_OK;
}

inline hipStream_t as_stream(kvc_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Zeroed claim words for one paged decode launch on `stream` with `words`
// workgroups (kvc_claims.hip), or null: the launch then uses the static
// partition alone.
unsigned long long* claim_set(hipStream_t stream, int words);
int claim_set_words();

// The device's per-workgroup stamp buffer of the stream-K decode's
// diagnostics (kvc_claims.hip; 2 stamps per workgroup), recording that the
// next launch has `grid` workgroups; null when it cannot be resolved.
unsigned long long* stamp_buffer(int grid);
int stamp_slots();

// The device `stream` runs on (the current device for the NULL stream), for
// kvc_paged_decode_append_static (kvc_scratch.hip).
int stream_device(hipStream_t stream, int* dev);

// Address of device `dev`'s copy of the static scratch array
// (KVC_STATIC_SCRATCH_BYTES, kvc_scratch.hip), resolved once per device.
int scratch_for_device(int dev, void** ptr);

// ---------------------------------------------------------------------------
// Device-side vector types and helpers.
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet), the rounding
// torch uses for .to(torch.bfloat16).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// The same round-to-nearest-even conversion in one instruction
// (v_cvt_pk_bf16_f32); a NaN keeps its NaN-ness but not necessarily its
// payload, so bit-exact byte paths use pack_bf16x2 instead.
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
__device__ __forceinline__ uint32_t pack_bf16x2_fast(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// fp16 pair, round to nearest even (v_cvt_f16_f32), and back.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const _Float16 a = static_cast<_Float16>(lo), b = static_cast<_Float16>(hi);
  return uint32_t(__builtin_bit_cast(uint16_t, a)) | (uint32_t(__builtin_bit_cast(uint16_t, b)) << 16);
}
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return float(__builtin_bit_cast(_Float16, uint16_t(w & 0xffffu)));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16)));
}

// max / sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows),
// with the row-swap permutes instead of LDS-routed shuffles.
__device__ __forceinline__ float rows4_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// v_perm_b32 byte selectors: (lo half of a, lo half of b) and (hi of a, hi of b)
// for perm(b, a, sel) where a supplies bytes 0-3 and b bytes 4-7.
constexpr uint32_t kPermLoLo = 0x05040100u;
constexpr uint32_t kPermHiHi = 0x07060302u;

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ __forceinline__ f32x4_t mfma_bf16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Wave-wide shuffles inside a 64-lane wavefront (ds_swizzle/bpermute).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

template <typename T>
__device__ __forceinline__ T uniform(T v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Entry idx of a table that nothing writes while the kernel runs (block
// tables), read as one scalar load: the address is made wave-uniform and the
// load goes through the constant address space, so it never becomes a vector
// load whose wait would also drain the loads in flight.
__device__ __forceinline__ int table_entry(const int32_t* table, int64_t idx) {
  const uint64_t a = reinterpret_cast<uint64_t>(table + idx);
  // (readfirstlane returns int: each half goes back through uint32_t so the
  // low half is zero-extended, not sign-extended into the high word)
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
  const uint64_t u = (uint64_t(hi) << 32) | uint64_t(lo);
  return *reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(u);
}

// Touch every 64-byte line of the kernel's argument block once, at entry:
// the scalar loads issue together and are waited for once, so the
// parameter reads spread through the kernel hit the scalar cache instead of
// each first touch of a line being its own round trip to memory.
__device__ __forceinline__ void touch_kernel_args(int bytes) {
  const __attribute__((address_space(4))) char* k =
      (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
  int acc = 0;
#pragma unroll
  for (int off = 0; off < 1024; off += 64)
    if (off < bytes) acc ^= *(const __attribute__((address_space(4))) int*)(k + off);
  asm volatile("" ::"s"(acc));
}

// floor(x / d) for 0 <= x < 2^24 with a quotient below 2^21, given rcp, 1 / d
// to within a few ulp (v_rcp_f32): the float estimate is then within one of
// the quotient, and one correction each way makes it exact.  (The compiler's
// general int32 division is some thirty dependent instructions.)
__device__ __forceinline__ int div_small(int x, int d, float rcp) {
  int q = int(float(x) * rcp);
  q += (q + 1) * d <= x ? 1 : 0;
  q -= q * d > x ? 1 : 0;
  return q;
}

// Inclusive prefix sum / running maximum over the 64 lanes of a wave (every
// lane active), by DPP without LDS round trips: row_shr 1, 2, 4, 8 build the
// prefix inside each 16-lane row (lanes shifted in from outside the row read
// 0), then row_bcast:15 carries each row's last lane into the next row (rows
// 1 and 3) and row_bcast:31 carries lane 31 into rows 2 and 3.  The maximum
// form takes non-negative values (0 is its identity here).
__device__ __forceinline__ int wave_scan_add(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}
__device__ __forceinline__ int wave_scan_max_nonneg(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
  return x;
}

// The same scan for max over any ints (lanes without a source read INT_MIN).
__device__ __forceinline__ int wave_scan_max(int x) {
  constexpr int kLow = -2147483647 - 1;
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x111, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x112, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x114, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x118, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x142, 0xa, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(kLow, x, 0x143, 0xc, 0xf, false));
  return x;
}

// Wave-wide sum and max (integers, so any order gives the same result) from
// the DPP scans, read back from lane 63: no LDS round trips.
__device__ __forceinline__ int wave_sum(int v) {
  return __builtin_amdgcn_readlane(wave_scan_add(v), 63);
}

__device__ __forceinline__ int wave_max(int v) {
  return __builtin_amdgcn_readlane(wave_scan_max(v), 63);
}

__device__ __forceinline__ int64_t wrap_slot(int64_t s, int64_t num_slots) {
  return s < 0 ? s + num_slots : s;
}

template <int kIdxBytes>
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i) {
  if constexpr (kIdxBytes == 8) {
    return reinterpret_cast<const int64_t*>(p)[i];
  } else {
    return reinterpret_cast<const int32_t*>(p)[i];
  }
}

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Per-token-head int8 quantisation of one 16-lane group's row (8 dims per
// lane), shared by the store kernel and the decode launch's fused append.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void unpack8(const u32x4_t& w, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
    x[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
  }
}

__device__ __forceinline__ float group16_max(float v) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ uint32_t pack_codes4(const int (&c)[8], int base) {
  return (uint32_t(c[base]) & 0xffu) | ((uint32_t(c[base + 1]) & 0xffu) << 8) |
         ((uint32_t(c[base + 2]) & 0xffu) << 16) | ((uint32_t(c[base + 3]) & 0xffu) << 24);
}

// Per-token-head symmetric quantisation, rounding half to even.
__device__ __forceinline__ float quant_tokhead_row(const float (&x)[8], int (&code)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = group16_max(amax);
  amax = fmaxf(amax, 1e-6f);
  const float s = amax / 127.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q = __builtin_rintf(x[i] / s);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    code[i] = int(q);
  }
  return s;
}

// Per-channel quantisation of 8 dims against their store scales:
// clamp(floor(x / s + 0.5), -127, 127), IEEE division (the store kernel's and
// the decode launch's fused append's arithmetic).
__device__ __forceinline__ int quant_chan1(float x, float s) {
  const float q = floorf(x / s + 0.5f);
  return int(fminf(fmaxf(q, -127.0f), 127.0f));
}

__device__ __forceinline__ void quant_chan8(const float (&x)[8], const float (&s)[8],
                                            int (&code)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) code[i] = quant_chan1(x[i], s[i]);
}


}  // namespace kvc
