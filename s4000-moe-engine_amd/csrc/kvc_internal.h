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

}  // namespace kvc
