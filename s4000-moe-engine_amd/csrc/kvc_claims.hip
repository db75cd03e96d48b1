// Claim words of the paged decode's dynamic tail hand-out.
//
// A stream-K decode launch lets workgroups that finish their own share take
// tail tiles of slower shares; every share has one 64-bit claim word that
// must be zero when the launch starts, and the launch's merge kernel zeroes
// the words again when the launch is over.  The words live here, in a
// library array per GPU (zero when the code object loads), cut into sets of
// kClaimWords words:
// * a launch outside graph capture uses its stream's set (one per stream,
//   so launches that run concurrently on different streams never share
//   words, and launches on one stream run one after the other);
// * a launch being captured into a graph gets a set of its own, never given
//   out again (replays of one graph are ordered; different graphs can run
//   concurrently).
// When the sets run out, or the launch has more workgroups than a set has
// words, the launch runs the static partition alone (claim_set returns
// null).  Host code never uses the array's name as an address: each
// device's copy is resolved once with hipGetSymbolAddress (that device
// current) and cached.
#include <mutex>
#include <unordered_map>

#include "kvc_internal.h"

namespace {
constexpr int kClaimSets = 512;
constexpr int kClaimWords = 256;
constexpr int kMaxClaimDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned long long claims[kClaimSets * kClaimWords];

namespace kvc {
namespace {
struct DeviceSets {
  unsigned long long* base = nullptr;
  int next = 0;
  std::unordered_map<hipStream_t, int> by_stream;
};
DeviceSets g_sets[kMaxClaimDevices];
std::mutex g_sets_mu;
}  // namespace

int claim_set_words() { return kClaimWords; }

unsigned long long* claim_set(hipStream_t stream, int words) {
  if (words <= 0 || words > kClaimWords) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  if (stream != nullptr && hipStreamGetDevice(stream, &dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxClaimDevices) return nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_sets_mu);
  DeviceSets& ds = g_sets[dev];
  if (ds.base == nullptr) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return nullptr;
    if (prev != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(claims));
    if (prev != dev && hipSetDevice(prev) != hipSuccess) return nullptr;
    if (e != hipSuccess || p == nullptr) return nullptr;
    ds.base = static_cast<unsigned long long*>(p);
  }
  int set = -1;
  if (cap == hipStreamCaptureStatusActive) {
    set = ds.next < kClaimSets ? ds.next++ : -1;
  } else {
    auto it = ds.by_stream.find(stream);
    if (it != ds.by_stream.end()) {
      set = it->second;
    } else if (ds.next < kClaimSets) {
      set = ds.next++;
      ds.by_stream.emplace(stream, set);
    }
  }
  return set < 0 ? nullptr : ds.base + int64_t(set) * kClaimWords;
}

}  // namespace kvc

// ---------------------------------------------------------------------------
// Per-workgroup wall-clock stamps of a stream-K decode launch (diagnostics,
// KVC_DECODE_STAMPS=1): one buffer per device, overwritten by every launch
// that records; kvc_decode_stamps copies the last one to the host.
// ---------------------------------------------------------------------------
namespace {
constexpr int kStampSlots = 4096;
}  // namespace

static __device__ __align__(256) unsigned long long wg_stamps[2 * kStampSlots];

namespace kvc {
namespace {
unsigned long long* g_stamp_ptr[kMaxClaimDevices];
int g_stamp_grid[kMaxClaimDevices];
std::mutex g_stamp_mu;
}  // namespace

int stamp_slots() { return kStampSlots; }

unsigned long long* stamp_buffer(int grid) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxClaimDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_stamp_mu);
  if (g_stamp_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(wg_stamps)) != hipSuccess || p == nullptr)
      return nullptr;
    g_stamp_ptr[dev] = static_cast<unsigned long long*>(p);
  }
  g_stamp_grid[dev] = grid;
  return g_stamp_ptr[dev];
}
}  // namespace kvc

extern "C" int kvc_decode_stamps(unsigned long long* host_out, int max_workgroups, int* workgroups,
                                 int* clock_khz) {
  kvc::clear_error();
  KVC_REQUIRE(host_out != nullptr && workgroups != nullptr && clock_khz != nullptr, KVC_ERR_VALUE,
              "decode_stamps: output pointers are required");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  KVC_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxClaimDevices, KVC_ERR_RUNTIME,
              "decode_stamps: hipGetDevice: %s", hipGetErrorString(e));
  unsigned long long* src = nullptr;
  int grid = 0;
  {
    std::lock_guard<std::mutex> lock(kvc::g_stamp_mu);
    src = kvc::g_stamp_ptr[dev];
    grid = kvc::g_stamp_grid[dev];
  }
  KVC_REQUIRE(src != nullptr && grid > 0, KVC_ERR_VALUE,
              "decode_stamps: no launch on this device recorded stamps (KVC_DECODE_STAMPS=1)");
  const int n = grid < max_workgroups ? grid : max_workgroups;
  e = hipMemcpy(host_out, src, size_t(n) * 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "decode_stamps: hipMemcpy: %s",
              hipGetErrorString(e));
  int khz = 0;
  e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
  KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "decode_stamps: wall clock rate: %s",
              hipGetErrorString(e));
  *workgroups = n;
  *clock_khz = khz;
  return KVC_OK;
}

