// Static scratch of kvc_paged_decode_append_static.
//
// The split-K partials and split counts of a decode step without a caller
// workspace live in `scratch`, one array per GPU.  The array sits alone in
// this file so that it is part of a code object of its own: the runtime
// loads a code object, and reserves its device arrays, on a device when
// something in it is first used there (here: the first
// kvc_paged_decode_append_static call on that device resolves the array), so
// a process that never calls the static entry point never holds the
// KVC_STATIC_SCRATCH_BYTES.  Once reserved, a device's copy is held until the
// process ends.  Host code never uses the array's name as an address: the
// first call on a device resolves that device's copy with
// hipGetSymbolAddress (the device current while it does so) and every later
// call passes the cached pointer.
#include <atomic>
#include <mutex>

#include "kvc_internal.h"

static __device__ __align__(256) unsigned char scratch[KVC_STATIC_SCRATCH_BYTES];

namespace kvc {
namespace {
constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;
}  // namespace

int stream_device(hipStream_t stream, int* dev) {
  hipError_t e = hipGetDevice(dev);
  KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "paged_decode_append_static: hipGetDevice: %s",
              hipGetErrorString(e));
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, dev);
    KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME,
                "paged_decode_append_static: hipStreamGetDevice: %s", hipGetErrorString(e));
  }
  KVC_REQUIRE(*dev >= 0 && *dev < kMaxScratchDevices, KVC_ERR_RUNTIME,
              "paged_decode_append_static: device %d out of range", *dev);
  return KVC_OK;
}

int scratch_for_device(int dev, void** ptr) {
  KVC_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, KVC_ERR_RUNTIME,
              "paged_decode_append_static: device %d out of range", dev);
  void* cached = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (cached != nullptr) {
    *ptr = cached;
    return KVC_OK;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  cached = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (cached == nullptr) {
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "paged_decode_append_static: hipGetDevice: %s",
                hipGetErrorString(e));
    if (prev != dev) {
      e = hipSetDevice(dev);
      KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME,
                  "paged_decode_append_static: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t restore = prev != dev ? hipSetDevice(prev) : hipSuccess;
    KVC_REQUIRE(e == hipSuccess && p != nullptr, KVC_ERR_RUNTIME,
                "paged_decode_append_static: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
    KVC_REQUIRE(restore == hipSuccess, KVC_ERR_RUNTIME,
                "paged_decode_append_static: hipSetDevice(%d): %s", prev,
                hipGetErrorString(restore));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
    cached = p;
  }
  *ptr = cached;
  return KVC_OK;
}
}  // namespace kvc
