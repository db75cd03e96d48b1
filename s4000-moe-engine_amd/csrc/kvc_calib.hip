// Per-channel int8 calibration of the KV pool (the engine's P20 encoding):
// statistics of the K/V rows seen while calibrating, then the freeze into
// store scales, read scales and each kv head's outlier dims.
//
// Statistics are per (K or V, kv head, dim): the running max of |x| and the
// running fp32 sum, over the observed forwards, of each forward's sum of |x|
// rounded to bf16.  The engine's hook sums a bf16 tensor, and torch returns
// that sum as bf16 (nanovllm/engine/model_runner.py:529-532); here the
// forward's sum is formed exactly (fp64: every bf16 term is exact in it while
// the terms of one forward span less than 2^45) and rounded once to bf16
// with round-to-nearest-even, so the result does not depend on the order of
// the additions.  No atomics: one workgroup owns a (side, head).
#include "kvc_internal.h"

namespace kvc {
namespace {

constexpr int kD = 128;
constexpr int kLanes = 8;                 // token lanes per workgroup
constexpr int kObsThreads = kD * kLanes;  // 1024
constexpr float kRatioThreshold = 10.f;

// Round a non-negative finite double to the nearest bf16 (ties to even),
// returned as the fp32 holding that bf16 value.  In the normal range the
// 45 low mantissa bits are rounded off in the double itself (a carry moves
// into the exponent, and past bf16's largest value the result becomes
// infinity on the conversion).  Below 2^-126 the sum is a multiple of 2^-133
// (a sum of bf16 subnormals) and exact in fp32, whose bf16 rounding then is
// the usual add-and-truncate.
__device__ __forceinline__ float round_bf16_rne(double x) {
  if (x < 0x1p-126) {
    const uint32_t b = __float_as_uint(float(x));
    return __uint_as_float((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
  }
  uint64_t b = uint64_t(__double_as_longlong(x));
  b += (uint64_t(1) << 44) - 1 + ((b >> 45) & 1);
  b &= ~((uint64_t(1) << 45) - 1);
  return float(__longlong_as_double(int64_t(b)));
}

// Workgroup (side, head): thread (lane, d) walks tokens lane, lane + 8, ...
// of column d, then lane 0 folds the 8 partials (all sums exact in fp64).
__global__ void __launch_bounds__(kObsThreads)
calib_observe_kernel(const uint16_t* __restrict__ key, int64_t k_sn, int64_t k_sh,
                     const uint16_t* __restrict__ value, int64_t v_sn, int64_t v_sh,
                     int64_t num_tokens, int kvh, float* __restrict__ amax,
                     float* __restrict__ abs_sum) {
  __shared__ float s_max[kLanes][kD];
  __shared__ double s_sum[kLanes][kD];
  const int side = blockIdx.x / kvh;
  const int h = blockIdx.x - side * kvh;
  const int d = threadIdx.x % kD;
  const int lane = threadIdx.x / kD;
  const uint16_t* base = side == 0 ? key + h * k_sh + d : value + h * v_sh + d;
  const int64_t sn = side == 0 ? k_sn : v_sn;
  float mx = 0.f;
  double sum = 0.0;
  int64_t n = lane;
  // four tokens' loads in flight
  for (; n + 3 * kLanes < num_tokens; n += 4 * kLanes) {
    uint32_t b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = base[(n + u * kLanes) * sn];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float a = __uint_as_float((b[u] & 0x7fffu) << 16);
      mx = fmaxf(mx, a);
      sum += double(a);
    }
  }
  for (; n < num_tokens; n += kLanes) {
    const float a = __uint_as_float((uint32_t(base[n * sn]) & 0x7fffu) << 16);
    mx = fmaxf(mx, a);
    sum += double(a);
  }
  s_max[lane][d] = mx;
  s_sum[lane][d] = sum;
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int l = 1; l < kLanes; ++l) {
      mx = fmaxf(mx, s_max[l][d]);
      sum += s_sum[l][d];
    }
    const int64_t i = (int64_t(side) * kvh + h) * kD + d;
    amax[i] = fmaxf(amax[i], mx);
    abs_sum[i] += round_bf16_rne(sum);
  }
}

// Workgroup h, thread d (two waves).  Outlier dims of head h: its first
// n_out_max dims, in index order, whose K/V joint ratio amax / mean|x|
// exceeds 10; their read scales are 0 (the side pool holds them exactly).
__global__ void __launch_bounds__(kD)
calib_freeze_kernel(const float* __restrict__ amax, const float* __restrict__ abs_sum,
                    float count, int kvh, int n_out_max, float* __restrict__ k_scale,
                    float* __restrict__ v_scale, float* __restrict__ k_dscale,
                    float* __restrict__ v_dscale, int32_t* __restrict__ out_idx2d,
                    int32_t* __restrict__ head_n_out) {
  __shared__ int s_wave0;
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  const int64_t ik = int64_t(h) * kD + d;
  const int64_t iv = int64_t(kvh + h) * kD + d;
  const float ak = amax[ik], av = amax[iv];
  const float sk = fmaxf(ak / 127.f, 1e-6f);
  const float sv = fmaxf(av / 127.f, 1e-6f);
  const float tk = fmaxf(abs_sum[ik] / count, 1e-6f);
  const float tv = fmaxf(abs_sum[iv] / count, 1e-6f);
  const float ratio = fmaxf(ak / tk, av / tv);
  const bool flag = ratio > kRatioThreshold;
  const uint64_t bal = __ballot(flag);
  const int lane = d & 63;
  const int below = __popcll(bal & ((uint64_t(1) << lane) - 1));
  if (d == 0) s_wave0 = __popcll(bal);
  __syncthreads();
  const int rank = (d >= 64 ? s_wave0 : 0) + below;
  const bool out = flag && rank < n_out_max;
  if (out) out_idx2d[int64_t(h) * n_out_max + rank] = d;
  k_scale[ik] = sk;
  v_scale[ik] = sv;
  k_dscale[ik] = out ? 0.f : sk;
  v_dscale[ik] = out ? 0.f : sv;
  if (d == 64) head_n_out[h] = min(s_wave0 + __popcll(bal), n_out_max);
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_kv_calib_observe(const void* key, int64_t key_stride_n, int64_t key_stride_h,
                                    const void* value, int64_t value_stride_n,
                                    int64_t value_stride_h, int64_t num_tokens,
                                    int64_t num_kv_heads, int64_t head_dim, float* amax,
                                    float* abs_sum, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "kv_calib_observe: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(num_kv_heads > 0 && num_kv_heads <= 64, KVC_ERR_VALUE,
              "kv_calib_observe: num_kv_heads must be in [1, 64] (got %lld)",
              (long long)num_kv_heads);
  KVC_REQUIRE(num_tokens >= 0, KVC_ERR_VALUE, "kv_calib_observe: negative token count");
  KVC_REQUIRE(amax != nullptr && abs_sum != nullptr, KVC_ERR_VALUE,
              "kv_calib_observe: amax and abs_sum are required");
  if (num_tokens == 0) return KVC_OK;
  KVC_REQUIRE(key != nullptr && value != nullptr, KVC_ERR_VALUE,
              "kv_calib_observe: key and value are required");
  calib_observe_kernel<<<unsigned(2 * num_kv_heads), kObsThreads, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(key), key_stride_n, key_stride_h,
      static_cast<const uint16_t*>(value), value_stride_n, value_stride_h, num_tokens,
      int(num_kv_heads), amax, abs_sum);
  return check_launch("kv_calib_observe");
}

extern "C" int kvc_kv_calib_freeze(const float* amax, const float* abs_sum, int64_t count,
                                   int64_t num_kv_heads, int64_t head_dim, int64_t n_out_max,
                                   float* k_scale, float* v_scale, float* k_dscale,
                                   float* v_dscale, int32_t* out_idx2d, int32_t* head_n_out,
                                   kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "kv_calib_freeze: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(count > 0, KVC_ERR_ASSERT, "kv_calib_freeze: calibration saw no activations");
  KVC_REQUIRE(count < (int64_t(1) << 24), KVC_ERR_VALUE,
              "kv_calib_freeze: %lld tokens exceed the exact fp32 count", (long long)count);
  KVC_REQUIRE(num_kv_heads > 0 && n_out_max >= 0 && n_out_max <= kD, KVC_ERR_VALUE,
              "kv_calib_freeze: bad num_kv_heads / n_out_max");
  KVC_REQUIRE(amax && abs_sum && k_scale && v_scale && k_dscale && v_dscale && head_n_out &&
                  (n_out_max == 0 || out_idx2d),
              KVC_ERR_VALUE, "kv_calib_freeze: every output is required");
  calib_freeze_kernel<<<unsigned(num_kv_heads), kD, 0, as_stream(stream)>>>(
      amax, abs_sum, float(count), int(num_kv_heads), int(n_out_max), k_scale, v_scale,
      k_dscale, v_dscale, out_idx2d, head_n_out);
  return check_launch("kv_calib_freeze");
}
