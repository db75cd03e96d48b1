// Whole-block movement for LRU eviction, host offload and compaction.
//
// A block of the engine's pool [2, L, blocks, page, KVH, D] is `planes`
// (= 2L) rows of block_bytes, one per (K|V, layer), plane_stride apart.
// Kernels copy 16-byte vectors, four in flight per thread, one 16 KiB piece
// of one (item, plane) row per workgroup iteration; the block id is resolved
// once per piece.  An in-HBM move launches a workgroup per piece.  A move to
// or from pinned host memory is PCIe-bound: a few workgroups saturate the
// link, so it launches at most KVC_HOST_MOVE_WGS (default 64) workgroups that
// stride over the pieces, and leaves the other CUs to whatever kernels run
// beside it.  The DMA entry points issue one strided 2-D copy per block on
// the copy engines instead.
#include <algorithm>
#include <cstdlib>

#include "kvc_internal.h"

namespace kvc {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int64_t kPiece = int64_t(kThreads) * kUnroll * 16;  // bytes per workgroup

struct MoveArgs {
  const char* src;
  char* dst;
  int64_t planes;
  int64_t block_bytes;
  int64_t pieces;  // per (item, plane) row
  // source row (item i, plane p) = src + p * src_plane + sel(src_ids, i) * src_item
  const int32_t* src_ids;
  int64_t src_plane, src_item;
  // destination row = dst + p * dst_plane + sel(dst_ids, i) * dst_item
  const int32_t* dst_ids;
  int64_t dst_plane, dst_item;
};

__global__ void __launch_bounds__(kThreads) move_blocks_kernel(MoveArgs a, int64_t total) {
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int64_t row = w / a.pieces;
    const int64_t piece = w - row * a.pieces;
    const int64_t item = row / a.planes;
    const int64_t plane = row - item * a.planes;
    const int64_t s_sel = a.src_ids ? int64_t(a.src_ids[item]) : item;
    const int64_t d_sel = a.dst_ids ? int64_t(a.dst_ids[item]) : item;
    const char* s = a.src + plane * a.src_plane + s_sel * a.src_item + piece * kPiece;
    char* d = a.dst + plane * a.dst_plane + d_sel * a.dst_item + piece * kPiece;
    const int64_t limit = a.block_bytes - piece * kPiece;
    u32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = (int64_t(u) * kThreads + threadIdx.x) * 16;
      if (off < limit) v[u] = *reinterpret_cast<const u32x4_t*>(s + off);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = (int64_t(u) * kThreads + threadIdx.x) * 16;
      if (off < limit) *reinterpret_cast<u32x4_t*>(d + off) = v[u];
    }
  }
}

int64_t host_move_workgroups() {
  static const int64_t wgs = [] {
    const char* e = std::getenv("KVC_HOST_MOVE_WGS");
    const long v = e ? std::strtol(e, nullptr, 10) : 0;
    return int64_t(v > 0 ? v : 64);
  }();
  return wgs;
}

int launch_move(const MoveArgs& a, int64_t n, hipStream_t st, const char* what,
                bool host_side = false) {
  if (n == 0 || a.planes == 0 || a.block_bytes == 0) return KVC_OK;
  const int64_t total = n * a.planes * a.pieces;
  const int64_t grid = host_side ? std::min(total, host_move_workgroups()) : total;
  KVC_REQUIRE(grid < (int64_t(1) << 31), KVC_ERR_VALUE, "%s: %lld workgroups exceed one launch",
              what, (long long)grid);
  move_blocks_kernel<<<unsigned(grid), kThreads, 0, st>>>(a, total);
  return check_launch(what);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Address a kernel may dereference for `p`: device memory as is, pinned host
// memory through its device mapping (*is_host set).  Pageable (unregistered)
// host memory is rejected rather than handed to a kernel.
int device_view(const void* p, const void** out, const char* what, bool* is_host) {
  *is_host = false;
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    set_error("%s: buffer %p is not device or pinned host memory", what, p);
    return KVC_ERR_VALUE;
  }
  if (attr.type == hipMemoryTypeUnregistered) {
    set_error("%s: buffer %p is pageable host memory (pin it first)", what, p);
    return KVC_ERR_VALUE;
  }
  if (attr.type == hipMemoryTypeHost) {
    KVC_REQUIRE(attr.devicePointer != nullptr, KVC_ERR_VALUE,
                "%s: pinned buffer %p has no device mapping", what, p);
    *out = static_cast<const char*>(attr.devicePointer) +
           (static_cast<const char*>(p) - static_cast<const char*>(attr.hostPointer));
    *is_host = true;
    return KVC_OK;
  }
  *out = p;
  return KVC_OK;
}

int check_geometry(const void* a, const void* b, int64_t planes, int64_t block_bytes,
                   std::initializer_list<int64_t> strides, int64_t n, const char* what) {
  KVC_REQUIRE(n >= 0 && planes >= 0 && block_bytes >= 0, KVC_ERR_VALUE, "%s: negative size",
              what);
  KVC_REQUIRE(block_bytes % 16 == 0, KVC_ERR_VALUE,
              "%s: block_bytes (%lld) must be a multiple of 16", what, (long long)block_bytes);
  KVC_REQUIRE(aligned16(a) && aligned16(b), KVC_ERR_ASSERT, "%s: buffers must be 16-byte aligned",
              what);
  for (int64_t s : strides)
    KVC_REQUIRE(s % 16 == 0, KVC_ERR_ASSERT, "%s: strides must be multiples of 16 bytes", what);
  return KVC_OK;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_block_gather(const void* src, int64_t planes, int64_t src_plane_stride,
                                int64_t block_bytes, const int32_t* block_ids, int64_t n,
                                void* dst, int64_t dst_item_stride, int64_t dst_plane_stride,
                                kvc_stream_t stream) {
  clear_error();
  int rc = check_geometry(src, dst, planes, block_bytes,
                          {src_plane_stride, dst_item_stride, dst_plane_stride}, n,
                          "block_gather");
  if (rc != KVC_OK) return rc;
  if (n == 0) return KVC_OK;
  const void* dview = nullptr;
  bool host_side = false;
  rc = device_view(dst, &dview, "block_gather", &host_side);
  if (rc != KVC_OK) return rc;
  MoveArgs a{};
  a.src = static_cast<const char*>(src);
  a.dst = static_cast<char*>(const_cast<void*>(dview));
  a.planes = planes;
  a.block_bytes = block_bytes;
  a.pieces = (block_bytes + kPiece - 1) / kPiece;
  a.src_ids = block_ids;
  a.src_plane = src_plane_stride;
  a.src_item = block_bytes;
  a.dst_ids = nullptr;
  a.dst_plane = dst_plane_stride;
  a.dst_item = dst_item_stride;
  return launch_move(a, n, as_stream(stream), "block_gather", host_side);
}

extern "C" int kvc_block_scatter(const void* src, int64_t src_item_stride,
                                 int64_t src_plane_stride, int64_t planes, int64_t block_bytes,
                                 const int32_t* block_ids, int64_t n, void* dst,
                                 int64_t dst_plane_stride, kvc_stream_t stream) {
  clear_error();
  int rc = check_geometry(src, dst, planes, block_bytes,
                          {src_item_stride, src_plane_stride, dst_plane_stride}, n,
                          "block_scatter");
  if (rc != KVC_OK) return rc;
  if (n == 0) return KVC_OK;
  const void* sview = nullptr;
  bool host_side = false;
  rc = device_view(src, &sview, "block_scatter", &host_side);
  if (rc != KVC_OK) return rc;
  MoveArgs a{};
  a.src = static_cast<const char*>(sview);
  a.dst = static_cast<char*>(dst);
  a.planes = planes;
  a.block_bytes = block_bytes;
  a.pieces = (block_bytes + kPiece - 1) / kPiece;
  a.src_ids = nullptr;
  a.src_plane = src_plane_stride;
  a.src_item = src_item_stride;
  a.dst_ids = block_ids;
  a.dst_plane = dst_plane_stride;
  a.dst_item = block_bytes;
  return launch_move(a, n, as_stream(stream), "block_scatter", host_side);
}

extern "C" int kvc_block_copy(void* pool, int64_t planes, int64_t plane_stride,
                              int64_t block_bytes, const int32_t* src_ids, const int32_t* dst_ids,
                              int64_t n, kvc_stream_t stream) {
  clear_error();
  int rc = check_geometry(pool, pool, planes, block_bytes, {plane_stride}, n, "block_copy");
  if (rc != KVC_OK) return rc;
  KVC_REQUIRE(n == 0 || (src_ids != nullptr && dst_ids != nullptr), KVC_ERR_VALUE,
              "block_copy: src_ids and dst_ids are required");
  MoveArgs a{};
  a.src = static_cast<const char*>(pool);
  a.dst = static_cast<char*>(pool);
  a.planes = planes;
  a.block_bytes = block_bytes;
  a.pieces = (block_bytes + kPiece - 1) / kPiece;
  a.src_ids = src_ids;
  a.src_plane = plane_stride;
  a.src_item = block_bytes;
  a.dst_ids = dst_ids;
  a.dst_plane = plane_stride;
  a.dst_item = block_bytes;
  return launch_move(a, n, as_stream(stream), "block_copy");
}

extern "C" int kvc_block_d2h(const void* pool, int64_t planes, int64_t plane_stride,
                             int64_t block_bytes, const int64_t* host_ids, int64_t n,
                             void* host_dst, int64_t host_item_stride, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(n >= 0 && planes >= 0 && block_bytes >= 0, KVC_ERR_VALUE, "block_d2h: bad size");
  hipStream_t st = as_stream(stream);
  for (int64_t i = 0; i < n; ++i) {
    const char* s = static_cast<const char*>(pool) + host_ids[i] * block_bytes;
    char* d = static_cast<char*>(host_dst) + i * host_item_stride;
    hipError_t e = hipMemcpy2DAsync(d, size_t(block_bytes), s, size_t(plane_stride),
                                    size_t(block_bytes), size_t(planes), hipMemcpyDeviceToHost, st);
    KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "block_d2h: hipMemcpy2DAsync failed: %s",
                hipGetErrorString(e));
  }
  return KVC_OK;
}

extern "C" int kvc_block_h2d(const void* host_src, int64_t host_item_stride, int64_t planes,
                             int64_t block_bytes, const int64_t* host_ids, int64_t n, void* pool,
                             int64_t plane_stride, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(n >= 0 && planes >= 0 && block_bytes >= 0, KVC_ERR_VALUE, "block_h2d: bad size");
  hipStream_t st = as_stream(stream);
  for (int64_t i = 0; i < n; ++i) {
    const char* s = static_cast<const char*>(host_src) + i * host_item_stride;
    char* d = static_cast<char*>(pool) + host_ids[i] * block_bytes;
    hipError_t e = hipMemcpy2DAsync(d, size_t(plane_stride), s, size_t(block_bytes),
                                    size_t(block_bytes), size_t(planes), hipMemcpyHostToDevice, st);
    KVC_REQUIRE(e == hipSuccess, KVC_ERR_RUNTIME, "block_h2d: hipMemcpy2DAsync failed: %s",
                hipGetErrorString(e));
  }
  return KVC_OK;
}
