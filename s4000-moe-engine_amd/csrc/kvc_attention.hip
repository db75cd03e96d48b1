// Paged attention for gfx950: split-K paged decode and the single-launch
// mixed decode + chunked-prefill ("varlen") kernel, plus their split-K merge.
//
// Work unit: one wavefront owns a "column block" of 16 attention columns.  A
// column is one (query row, q head) pair; the heads of a column block all
// read the same kv head, so the block is a real GQA contraction and runs on
// MFMA (v_mfma_f32_16x16x32_bf16).  Per 32-key tile a wave computes
//   S^T[key, col] = K[key, :] . Q[col, :]^T            (2 x 4 MFMAs)
// and, after the online softmax,
//   O^T[d, col]  += V^T[d, key] . P^T[key, col]        (8 MFMAs)
// Writing both products transposed puts one column per lane (col = lane % 16)
// in every accumulator, so the running max / sum and the rescale of O are
// lane-local; the max and sum reductions over keys are two xor-shuffles.
// The key order inside the PV contraction is chosen so that the P^T operand
// is exactly the register set the S^T MFMA produced (no data movement), and
// V rows are read as whole 16-byte vectors and transposed in registers with
// v_perm_b32.
//
// Decode (the headline path): a stream-K launch whose workgroups stream 4 kv
// heads at a time through LDS.  Direct-to-LDS buffer loads bring each 32-key
// K/V tile into a two-stage ring (int8 per-token-head pools: a four-stage
// ring), so eight waves keep two tiles in flight with no VGPRs held by the
// loads; each wave then reads its head's rows from LDS.  Other head layouts
// run register segments (K/V straight from HBM into VGPRs, the next tile in
// flight).  Prefill: a stream-K launch over (chunk, kv slice, query tile)
// items whose 32-key tiles stream through a four-stage LDS ring, every tile
// consumed by eight waves of different query columns.  A mixed call over a
// bf16 pool runs both in one launch over a static CU split (decode shares on
// the first workgroups, prefill shares on the rest) and both merges in one
// more launch.
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "kvc_internal.h"

namespace kvc {
namespace {

constexpr int kD = 128;
constexpr int kTile = 32;
constexpr int kWaves = 8;  // two waves per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kSideMax = 8;
constexpr int kPitchBF16 = kD * 2 + 16;  // a bf16 key row in LDS (16 B pad)
constexpr int kPreNCB = 2;  // column blocks per wave in prefill units
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
// Virtual tiles per row of a ragged stream-K decode (see decode_sk_share):
// on 64 rows of U[512,4096], 1 / 2 / 3 / 4 measured 51.6 / 51.4 / 51.1 /
// 51.1 us.
#ifndef KVC_DEC_ROW_COST
#define KVC_DEC_ROW_COST 3
#endif
constexpr int kDecRowCost = KVC_DEC_ROW_COST;
// Tail tiles per share of the dynamic decode hand-out, at most.
constexpr int kDecTailMax = 8;

enum Enc : int { kBF16 = KVC_KV_BF16, kI8Tok = KVC_KV_INT8_TOKHEAD, kI8Chan = KVC_KV_INT8_CHAN };

struct AttnParams {
  // queries / outputs (element strides)
  const uint16_t* q;
  int64_t q_st, q_sh;
  uint16_t* out;
  int64_t o_st, o_sh;
  int num_heads, kvh, group, hs, nslices, tpb;
  int kvs_per_wg;  // decode: kv slices per workgroup (divides 8 and kvh * nslices)
  float scale_log2;
  // paged pool
  const char* k_cache;
  const char* v_cache;
  int page;
  int64_t tok_bytes;  // bytes between consecutive slots
  const float* k_scale;
  const float* v_scale;
  const uint16_t* side_k;
  const uint16_t* side_v;
  const int32_t* out_idx;
  const int32_t* head_n_out;
  int n_out_max;
  const int32_t* block_tables;
  int64_t bt_stride;
  // decode rows
  int n_dec;
  const int32_t* ctx_lens;
  int chunk_tokens;
  int dec_max_chunks;
  int dec_units;
  // prefill chunks
  int n_pre;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int split_tokens;
  int pre_units;
  const uint16_t* kf;
  int64_t kf_st, kf_sh;
  const uint16_t* vf;
  int64_t vf_st, vf_sh;
  // split-K partials: [rows, heads, max_splits, D] fp32 and [rows, heads, max_splits]
  // (the stream-K prefill: fp16 rows in part_o's first half, (lse, scale
  // exponent) pairs in part_ml, in its second half)
  float* part_o;
  float* part_lse;
  float2* part_ml;
  int max_splits;
  int merge_first;  // splits the merge loads before it reads a row's split count
  float xcd_skew;   // stream-K decode: even workgroups take (1 + skew) shares, odd (1 - skew)
  // Stream-K decode (paged decode launches): each workgroup takes an equal
  // share (at least sk_min_share) of the tiles of all rows; sk_nseg[r] gets
  // the number of workgroups that row unit r (= row * groups + group) spans.
  int sk_min_share;
  int* sk_nseg;
  // Diagnostics (null: off): workgroup w of a stream-K decode writes its
  // start and end wall-clock stamps to wg_stamps[2 w], [2 w + 1].
  unsigned long long* wg_stamps;
  // Paged decode with the step's append fused (app_k null: no append): row b
  // of app_k / app_v (element strides) goes to pool slot app_slots[b]
  // (int32 or int64, wrapped like a Python index, skipped when outside
  // [0, app_num_slots)).
  const uint16_t* app_k;
  const uint16_t* app_v;
  int64_t app_k_st, app_k_sh, app_v_st, app_v_sh;
  const void* app_slots;
  int app_slot_bytes;
  int64_t app_num_slots;
};

// Dynamic tail hand-out of a bf16 stream-K decode (the kernels that take it
// are separate instantiations; claims null: none).  Share w's last segment
// ends in up to `tail` tiles that its owner claims one at a time from the
// front while workgroups done with their own shares take them from the back
// (claims[w]: front count | back count << 16 | tail tiles << 32).  A taken
// tile is its own partial, at tail slot (w * kDecTailMax + j) of tail_o /
// tail_lse ([slot][uh heads of the row unit][D]); stolen[row, kv slice,
// piece] counts a piece's taken tiles, and sk_nseg then also carries the
// row's first share (<< 16).
struct StealArgs {
  unsigned long long* claims;
  int* dummy;
  int* stolen;
  float* tail_o;
  float* tail_lse;
  int tail;
  int uh;
  int grid;
  int steal_min;
};

struct LaneId {
  int lane, lm, lg;
};

__device__ __forceinline__ LaneId lane_id() {
  const int lane = threadIdx.x & 63;
  return {lane, lane & 15, lane >> 4};
}

// Key (within a tile) carried by k-slot i of lane group lg: slots 0-3 are the
// S^T rows of the first 16-key half, slots 4-7 those of the second half.
__device__ __forceinline__ int key_of_slot(int lg, int i) {
  return i < 4 ? 4 * lg + i : 12 + 4 * lg + i;
}

// ---------------------------------------------------------------------------
// Per-tile operand registers.
// bf16: k[h][c] = key h*16+lm, dims 32c+8lg..+8;  v[i] = key slot i, dims 8lm..+8
// int8: k[h][w] = key h*16+lm, dims 32lg+16w..+16; v[i] = key slot i, dims 8lm..+8
// ---------------------------------------------------------------------------
template <int kEnc>
struct Tile;

template <>
struct Tile<kBF16> {
  u32x4_t k[2][4];
  u32x4_t v[8];
};

template <>
struct Tile<kI8Tok> {
  u32x4_t k[2][2];
  u32x2_t v[8];
  // Scales: lane l < 32 holds the K scale of key l in sck, lane 32 + l the V
  // scale of key l in scv, the other field 0.  They are only added when the
  // tile is attended: an add at load time would make the prefetch of the
  // next tile wait for its own loads.
  float sck, scv;
};

template <>
struct Tile<kI8Chan> {
  u32x4_t k[2][2];
  u32x2_t v[8];
  // Side-pool rows (decode ring only): lane (lm, lg) with lm < 8 holds the
  // n_out_max bf16 outlier values of key key_of_slot(lg, lm), K in sk and V
  // in sv (dword d = values 2d, 2d + 1; only the first max(1, n_out_max / 2)
  // dwords are used).  Slot i's row is read from lane i of the lane's
  // 16-lane row.
  uint32_t sk[4], sv[4];
};

// kSideN bounds the per-channel side-pool width (n_out_max <= kSideN).
template <int NCB, int kSideN = kSideMax>
struct ColState {
  f32x4_t o[NCB][8];  // O^T: [col block][d chunk jj], row r -> d = 32lg + 8r + jj
  float m[NCB];       // running max (log2 domain), identical on the 4 lanes of a column
  float l[NCB];       // lane-partial softmax sum
  float vb[NCB];      // lane-partial sum of the bf16 P operand (int8 bias correction)
  float sd[NCB][kSideN];  // lane-partial side-pool PV (per-channel int8 only)
};

template <int NCB, int kSideN>
__device__ __forceinline__ void init_state(ColState<NCB, kSideN>& st) {
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) st.o[cb][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    st.m[cb] = -INFINITY;
    st.l[cb] = 0.f;
    st.vb[cb] = 0.f;
#pragma unroll
    for (int j = 0; j < kSideN; ++j) st.sd[cb][j] = 0.f;
  }
}

// ---------------------------------------------------------------------------
// Tile loads from a paged pool in HBM (decode units).  Every load goes
// through a buffer resource covering the tile's 32 key rows.
// ---------------------------------------------------------------------------
// Scales of a tile (per-token-head int8): lane l < 32 loads the K scale of
// key l, lane 32 + l the V scale of key l, for kv head g.  Both loads use
// buffer resources, so out-of-range lanes read 0 and `live` = false costs no
// memory traffic.
__device__ __forceinline__ void load_scales_buf(const float* ksb, const float* vsb, int kvh, int g,
                                                bool live, const LaneId& L, float& sck,
                                                float& scv) {
  const int bytes = live ? kTile * kvh * 4 : 0;
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(ksb), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(vsb), 0, bytes, 0x00020000);
  const int key = L.lane & (kTile - 1);
  const int off = (key * kvh + g) * 4;
  const int big = 0x40000000;  // past num_records: reads 0
  sck = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                      kr, L.lane < kTile ? off : big, 0, 0));
  scv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                      vr, L.lane < kTile ? big : off, 0, 0));
}

// Buffer-resource forms of the tile loads.  A resource covers one tile's key
// rows; a resource with num_records = 0 turns every load into a zero-returning
// no-op with no memory traffic, which lets the prefetch ring issue its loads
// unconditionally (no branch, exact waitcnt bookkeeping) past a wave's range.
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format
// Cache policy of the decode KV reads: non-temporal (gfx94x/gfx950 NT bit).
// Each KV byte is read once per layer per step, so it is streamed past the
// caches instead of evicting the block tables and queries.
constexpr int kStreamCPol = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufWord3);
}

// The same for a base and size that are wave-uniform by construction: taking
// them through readfirstlane puts the resource in scalar registers even where
// the compiler cannot prove the uniformity itself (it would otherwise wrap
// each load in a loop over the distinct resources of the wave's lanes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_rsrc(const void* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  // (readfirstlane returns int: each half goes back through uint32_t so the
  // low half is zero-extended, not sign-extended into the high word)
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
  const uint64_t u = (uint64_t(hi) << 32) | uint64_t(lo);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), 0,
                                           __builtin_amdgcn_readfirstlane(bytes), kBufWord3);
}

struct TileOffsets {
  int k[2];      // K row of key half h for this lane: (16h + lm) * tok + lane part
  int v[8];      // V row of key slot i: key_of_slot(lg, i) * tok + lane part
};

template <int kEnc>
__device__ __forceinline__ TileOffsets tile_offsets(int tok, const LaneId& L) {
  TileOffsets o;
  const int kpart = (kEnc == kBF16) ? L.lg * 16 : L.lg * 32;
  const int vpart = (kEnc == kBF16) ? L.lm * 16 : L.lm * 8;
#pragma unroll
  for (int h = 0; h < 2; ++h) o.k[h] = (h * 16 + L.lm) * tok + kpart;
#pragma unroll
  for (int i = 0; i < 8; ++i) o.v[i] = key_of_slot(L.lg, i) * tok + vpart;
  return o;
}

__device__ __forceinline__ void load_tile_buf(Tile<kBF16>& t, __amdgpu_buffer_rsrc_t kr,
                                              __amdgpu_buffer_rsrc_t vr, const TileOffsets& o) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      t.k[h][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, o.k[h] + c * 64, 0, kStreamCPol));
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    t.v[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(vr, o.v[i], 0, kStreamCPol));
}

template <int kEnc>
__device__ __forceinline__ void load_tile_buf_i8(Tile<kEnc>& t, __amdgpu_buffer_rsrc_t kr,
                                                 __amdgpu_buffer_rsrc_t vr, const TileOffsets& o) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    t.k[h][0] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, o.k[h], 0, kStreamCPol));
    t.k[h][1] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, o.k[h] + 16, 0, kStreamCPol));
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    t.v[i] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(vr, o.v[i], 0, kStreamCPol));
}

// Side-pool rows of a tile (per-channel int8), loaded with the tile so that
// the attend step waits for them with the tile's own loads.  A row is the
// kN = n_out_max bf16 outlier values of one (slot, kv head); kN is 1, 2, 4 or
// 8, so a row is one 2-, 4-, 8- or 16-byte load at a multiple of its size.
// Lane (lm, lg) with lm < 8 loads the row of key key_of_slot(lg, lm); the
// other lanes read past num_records (0, no memory traffic), and so does every
// lane when `live` is false.
template <int kN>
__device__ __forceinline__ void load_side_row(uint32_t (&w)[4], __amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (kN == 8) {
    const u32x4_t v =
        __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kStreamCPol));
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  } else if constexpr (kN == 4) {
    const u32x2_t v =
        __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kStreamCPol));
    w[0] = v[0];
    w[1] = v[1];
  } else if constexpr (kN == 2) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kStreamCPol);
  } else {
    static_assert(kN == 1, "side rows of 1, 2, 4 or 8 values");
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kStreamCPol);
  }
}

template <int kN>
__device__ __forceinline__ void load_side_buf(Tile<kI8Chan>& t, const AttnParams& p,
                                              int64_t slot0, int g, bool live, const LaneId& L) {
  constexpr int kRow = 2 * kN;  // bytes of one (slot, kv head) row
  const int64_t first = (slot0 * p.kvh + g) * kN;
  const int bytes = live ? ((kTile - 1) * p.kvh + 1) * kRow : 0;
  const int off = L.lm < 8 ? key_of_slot(L.lg, L.lm) * p.kvh * kRow : 0x40000000;
  load_side_row<kN>(t.sk, wave_rsrc(live ? p.side_k + first : p.side_k, bytes), off);
  load_side_row<kN>(t.sv, wave_rsrc(live ? p.side_v + first : p.side_v, bytes), off);
}

// Dword d of the row of key slot i: lane i of this lane's 16-lane row holds
// it (DPP row broadcast, no LDS).
__device__ __forceinline__ uint32_t row_lane(uint32_t v, int i) {
#define KVC_ROW_LANE(n) \
  case n:               \
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x150 + n, 0xf, 0xf, false));
  switch (i) {
    KVC_ROW_LANE(0)
    KVC_ROW_LANE(1)
    KVC_ROW_LANE(2)
    KVC_ROW_LANE(3)
    KVC_ROW_LANE(4)
    KVC_ROW_LANE(5)
    KVC_ROW_LANE(6)
    default:
      return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x150 + 7, 0xf, 0xf, false));
  }
#undef KVC_ROW_LANE
}

// The kN values of key slot i's row, as bf16 bit patterns in dwords.
template <int kN>
__device__ __forceinline__ void side_row_of_slot(uint32_t (&w)[4], const uint32_t (&rows)[4],
                                                 int i) {
#pragma unroll
  for (int d = 0; d < 4; ++d) w[d] = (2 * d < kN) ? row_lane(rows[d], i) : 0u;
}

__device__ __forceinline__ float side_value(const uint32_t (&w)[4], int j) {
  return bf16_bits_to_f32((j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xffffu));
}

// ---------------------------------------------------------------------------
// Operand formation.
// ---------------------------------------------------------------------------
// 8 int8 codes -> 8 bf16 of (code + 128), exact (0..255 fit bf16's mantissa).
__device__ __forceinline__ u32x4_t i8x8_biased_bf16(uint32_t w0, uint32_t w1) {
  w0 ^= 0x80808080u;
  w1 ^= 0x80808080u;
  const float f0 = float(w0 & 0xffu), f1 = float((w0 >> 8) & 0xffu);
  const float f2 = float((w0 >> 16) & 0xffu), f3 = float(w0 >> 24);
  const float f4 = float(w1 & 0xffu), f5 = float((w1 >> 8) & 0xffu);
  const float f6 = float((w1 >> 16) & 0xffu), f7 = float(w1 >> 24);
  return u32x4_t{perm(__float_as_uint(f1), __float_as_uint(f0), kPermHiHi),
                 perm(__float_as_uint(f3), __float_as_uint(f2), kPermHiHi),
                 perm(__float_as_uint(f5), __float_as_uint(f4), kPermHiHi),
                 perm(__float_as_uint(f7), __float_as_uint(f6), kPermHiHi)};
}

// K operand for MFMA (key half h, d chunk c).
__device__ __forceinline__ u32x4_t k_operand(const Tile<kBF16>& t, int h, int c) {
  return t.k[h][c];
}
template <int kEnc>
__device__ __forceinline__ u32x4_t k_operand_i8(const Tile<kEnc>& t, int h, int c) {
  const u32x4_t w = t.k[h][c >> 1];
  return (c & 1) ? i8x8_biased_bf16(w[2], w[3]) : i8x8_biased_bf16(w[0], w[1]);
}

// V^T operand for PV MFMA jj: MFMA row m = lm is dim d = 8lm + jj, and the 8
// bf16 of the operand are that dim of the lane's 8 key slots, picked out of
// the row vectors with v_perm_b32.
__device__ __forceinline__ u32x4_t v_operand(const u32x4_t (&v)[8], int jj) {
  const uint32_t sel = (jj & 1) ? kPermHiHi : kPermLoLo;
  const int dw = jj >> 1;
  return u32x4_t{perm(v[1][dw], v[0][dw], sel), perm(v[3][dw], v[2][dw], sel),
                 perm(v[5][dw], v[4][dw], sel), perm(v[7][dw], v[6][dw], sel)};
}

// int8 form: the codes of dim jj for the 8 key slots, as bf16 of (code + 128).
// `w` holds the key rows already XOR-ed with 0x80 (code + 128 as unsigned).
__device__ __forceinline__ u32x4_t v_operand_i8(const uint32_t (&w)[8][2], int jj) {
  const int dw = jj >> 2, sh = (jj & 3) * 8;
  u32x4_t r;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float a = float((w[2 * s][dw] >> sh) & 0xffu);
    const float b = float((w[2 * s + 1][dw] >> sh) & 0xffu);
    r[s] = perm(__float_as_uint(b), __float_as_uint(a), kPermHiHi);
  }
  return r;
}

// ---------------------------------------------------------------------------
// Query side of a column block.
// ---------------------------------------------------------------------------
struct ColInfo {
  int64_t row;  // query row (output row)
  int head;     // q head
  bool valid;
  int klim;     // largest key index the column may attend (inclusive)
};

template <int kEnc, int NCB, int kSideN = kSideMax>
struct QOps {
  u32x4_t op[NCB][4];
  // Per-channel int8 folds the read scale into the query, q' = q * s; q' is
  // carried as a bf16 pair hi + lo (about 16 mantissa bits) because a single
  // bf16 rounding of a large-scale channel moves logits visibly.
  u32x4_t lo[NCB][4];
  float qsum[NCB];           // int8: sum over d of the query operand(s)
  float qout[NCB][kSideN];   // per-channel int8: query at the head's outlier dims
  int n_out;                 // per-channel int8: the kv head's outlier count (wave-uniform)
};

template <int kEnc, int NCB, int kSideN>
__device__ __forceinline__ void build_q(QOps<kEnc, NCB, kSideN>& Q, const AttnParams& p,
                                        const ColInfo (&ci)[NCB], int g, const LaneId& L) {
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const uint16_t* qrow = p.q + ci[cb].row * p.q_st + int64_t(ci[cb].head) * p.q_sh;
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      // bf16 pool: dims 32c + 8lg; int8 pools: dims 32lg + 8c.
      const int d0 = (kEnc == kBF16) ? (32 * c + 8 * L.lg) : (32 * L.lg + 8 * c);
      u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
      if (ci[cb].valid) w = *reinterpret_cast<const u32x4_t*>(qrow + d0);
      if constexpr (kEnc == kI8Chan) {
        // q'[d] = q[d] * s[g][d] in fp32, split as hi = bf16(q'), lo = bf16(q' - hi).
        const float* ds = p.k_scale + g * kD + d0;
        u32x4_t wl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = bf16_bits_to_f32(w[e] & 0xffffu) * ds[2 * e];
          const float b = bf16_bits_to_f32(w[e] >> 16) * ds[2 * e + 1];
          const uint32_t ah = f32_to_bf16_bits(a), bh = f32_to_bf16_bits(b);
          w[e] = ah | (bh << 16);
          wl[e] = pack_bf16x2(a - bf16_bits_to_f32(ah), b - bf16_bits_to_f32(bh));
          part += bf16_bits_to_f32(wl[e] & 0xffffu) + bf16_bits_to_f32(wl[e] >> 16);
        }
        Q.lo[cb][c] = wl;
      }
      if constexpr (kEnc != kBF16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) part += bf16_bits_to_f32(w[e] & 0xffffu) + bf16_bits_to_f32(w[e] >> 16);
      }
      Q.op[cb][c] = w;
    }
    if constexpr (kEnc != kBF16) {
      part += shfl_xor(part, 16);
      part += shfl_xor(part, 32);
      Q.qsum[cb] = part;
    }
    if constexpr (kEnc == kI8Chan) {
      const int n_out = p.head_n_out != nullptr ? uniform(p.head_n_out[g]) : 0;
      Q.n_out = n_out;
#pragma unroll
      for (int j = 0; j < kSideN; ++j) {
        float v = 0.f;
        if (ci[cb].valid && j < n_out) v = bf16_bits_to_f32(qrow[p.out_idx[g * p.n_out_max + j]]);
        Q.qout[cb][j] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// One 32-key tile against NCB column blocks.
//   key0       absolute index of the tile's first key
//   valid_end  keys >= valid_end do not exist (masked; bf16 V rows zeroed so a
//              poisoned tail never reaches 0 * NaN inside the MFMA)
//   slot0      pool slot of the tile's first key (side pool rows)
// kMasked = false is the fast path for tiles whose 32 keys are all visible to
// every valid column (all but the last tile of a decode row).
// Per-channel int8 (the register decode segment): the side-pool rows came
// with the tile (t.sk, t.sv).
// kPLo (bf16 tiles dequantised from a per-channel pool, whose outlier dims
// hold the side pool's values): the PV product of the outlier dims also takes
// the rounding residue of the bf16 P operand, P - bf16(P), so that the large
// side values meet an fp32-accurate P.  plo_v is the tile's V rows in LDS
// (pitch kPitchBF16), plo_dim the outlier dim of side slot lm (lanes
// lm < n_plo); plo[cb] accumulates the residue product, C row j = slot j,
// column = the lane's query column.
// ---------------------------------------------------------------------------
template <int kEnc, int NCB, bool kMasked, bool kSideRegs = false, int kSideN = kSideMax,
          bool kPLo = false>
__device__ __forceinline__ void attend_tile(ColState<NCB, kSideN>& st, const Tile<kEnc>& t,
                                            const QOps<kEnc, NCB, kSideN>& Q,
                                            const ColInfo (&ci)[NCB],
                                            int key0, int valid_end, int64_t slot0,
                                            const AttnParams& p, int g, const LaneId& L,
                                            const char* plo_v = nullptr,
                                            f32x4_t* plo = nullptr, int n_plo = 0,
                                            int plo_dim = 0) {
  static_assert(kEnc != kI8Chan || kSideRegs, "per-channel tiles carry their side rows");
  static_assert(!kPLo || kEnc == kBF16, "the residue product is for bf16 tiles");
  bool kvalid[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) kvalid[i] = !kMasked || (key0 + key_of_slot(L.lg, i) < valid_end);

  // V rows as the PV operands will read them.
  u32x4_t vrow[8];
  uint32_t vq[8][2];
  if constexpr (kEnc == kBF16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vrow[i] = t.v[i];
      if (kMasked && !kvalid[i]) vrow[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vq[i][0] = t.v[i][0] ^ 0x80808080u;
      vq[i][1] = t.v[i][1] ^ 0x80808080u;
    }
  }
  // With several column blocks the V operands are formed once per tile.
  u32x4_t va[NCB > 1 ? 8 : 1];
  if constexpr (NCB > 1) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if constexpr (kEnc == kBF16) {
        va[jj] = v_operand(vrow, jj);
      } else {
        va[jj] = v_operand_i8(vq, jj);
      }
    }
  }

  int n_out = 0;
  if constexpr (kEnc == kI8Chan) n_out = Q.n_out;

  // S^T of every column block first: the K operands die before the softmax,
  // and a later block's MFMAs can run under an earlier block's softmax.
  f32x4_t sacc[NCB][2];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    sacc[cb][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    sacc[cb][1] = sacc[cb][0];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4_t k0, k1;
    if constexpr (kEnc == kBF16) {
      k0 = k_operand(t, 0, c);
      k1 = k_operand(t, 1, c);
    } else {
      k0 = k_operand_i8(t, 0, c);
      k1 = k_operand_i8(t, 1, c);
    }
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      sacc[cb][0] = mfma_bf16(k0, Q.op[cb][c], sacc[cb][0]);
      sacc[cb][1] = mfma_bf16(k1, Q.op[cb][c], sacc[cb][1]);
      if constexpr (kEnc == kI8Chan) {
        sacc[cb][0] = mfma_bf16(k0, Q.lo[cb][c], sacc[cb][0]);
        sacc[cb][1] = mfma_bf16(k1, Q.lo[cb][c], sacc[cb][1]);
      }
    }
  }

  // Residue A operand (kPLo): row j = lm (side slot j, whose value the V
  // tile holds at dim plo_dim), the lane's 8 key slots; rows past n_plo 0.
  u32x4_t plo_op = u32x4_t{0u, 0u, 0u, 0u};
  if constexpr (kPLo) {
    if (n_plo > 0) {
      uint32_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        e[i] = L.lm < n_plo ? *reinterpret_cast<const uint16_t*>(
                                  plo_v + key_of_slot(L.lg, i) * kPitchBF16 + 2 * plo_dim)
                            : 0u;
      plo_op = u32x4_t{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                       e[6] | (e[7] << 16)};
    }
  }
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const f32x4_t s0 = sacc[cb][0], s1 = sacc[cb][1];
    float x[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    if constexpr (kEnc != kBF16) {
      const float bias = 128.f * Q.qsum[cb];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] -= bias;
    }
    if constexpr (kEnc == kI8Tok) {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] *= __shfl(t.sck + t.scv, key_of_slot(L.lg, i), 64);
    }
    if constexpr (kEnc == kI8Chan) {
      if (n_out > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float acc = 0.f;
          uint32_t w[4];
          side_row_of_slot<kSideN>(w, t.sk, i);
#pragma unroll
          for (int j = 0; j < kSideN; ++j)
            if (j < n_out) acc += Q.qout[cb][j] * side_value(w, j);
          x[i] += acc;
        }
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (kMasked) {
        const bool ok = kvalid[i] && (key0 + key_of_slot(L.lg, i) <= ci[cb].klim);
        x[i] = ok ? x[i] * p.scale_log2 : -INFINITY;
      } else {
        x[i] *= p.scale_log2;
      }
      tmax = fmaxf(tmax, x[i]);
    }
    tmax = rows4_max(tmax);
    // Lazy rescale: the accumulators stay relative to a reference max that
    // only moves when some column's max exceeds it by more than kRescaleLog2
    // (then probabilities stay <= 2^kRescaleLog2, exact in the fp32
    // accumulators and within bf16 range); the final normalisation divides by
    // the sum taken against the same reference, so the result is the same
    // softmax.  Rescales become rare after the first tiles.
    float alpha = 1.f;
    if (__builtin_expect(__ballot(tmax > st.m[cb] + kRescaleLog2) != 0, 0)) {
      const float m_new = fmaxf(st.m[cb], tmax);
      const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
      alpha = __builtin_amdgcn_exp2f(st.m[cb] - m_ref);
      st.m[cb] = m_new;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        st.o[cb][jj][0] *= alpha;
        st.o[cb][jj][1] *= alpha;
        st.o[cb][jj][2] *= alpha;
        st.o[cb][jj][3] *= alpha;
      }
      if constexpr (kPLo) {
#pragma unroll
        for (int r = 0; r < 4; ++r) plo[cb][r] *= alpha;
      }
    }
    const float m_use = (st.m[cb] == -INFINITY) ? 0.f : st.m[cb];
    float pr[8], psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
      psum += pr[i];
    }
    st.l[cb] = st.l[cb] * alpha + psum;
    // P^T operand (k-slot order == the S^T register order).
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (kEnc == kI8Tok) {
        const float vsc = __shfl(t.sck + t.scv, kTile + key_of_slot(L.lg, i), 64);
        pv[i] = kvalid[i] ? pr[i] * vsc : 0.f;
      } else {
        pv[i] = pr[i];
      }
    }
    u32x4_t pb;
#pragma unroll
    for (int w = 0; w < 4; ++w) pb[w] = pack_bf16x2_fast(pv[2 * w], pv[2 * w + 1]);
    if constexpr (kPLo) {
      if (n_plo > 0) {
        u32x4_t pl;
#pragma unroll
        for (int w = 0; w < 4; ++w)
          pl[w] = pack_bf16x2_fast(pv[2 * w] - bf16_bits_to_f32(pb[w] & 0xffffu),
                                   pv[2 * w + 1] - bf16_bits_to_f32(pb[w] >> 16));
        plo[cb] = mfma_bf16(plo_op, pl, plo[cb]);
      }
    }
    if constexpr (kEnc != kBF16) {
      float vsum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) vsum += bf16_bits_to_f32(pb[w] & 0xffffu) + bf16_bits_to_f32(pb[w] >> 16);
      st.vb[cb] = st.vb[cb] * alpha + vsum;
    }
    if constexpr (kEnc == kI8Chan) {
      if (n_out > 0) {
#pragma unroll
        for (int j = 0; j < kSideN; ++j) st.sd[cb][j] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          // Every lane of a 16-lane row shares kvalid[i]: the row read stays
          // outside the branch all the same.
          uint32_t w[4];
          side_row_of_slot<kSideN>(w, t.sv, i);
          if (!kvalid[i]) continue;
#pragma unroll
          for (int j = 0; j < kSideN; ++j)
            if (j < n_out) st.sd[cb][j] += pr[i] * side_value(w, j);
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      u32x4_t a;
      if constexpr (NCB > 1) {
        a = va[jj];
      } else if constexpr (kEnc == kBF16) {
        a = v_operand(vrow, jj);
      } else {
        a = v_operand_i8(vq, jj);
      }
      st.o[cb][jj] = mfma_bf16(a, pb, st.o[cb][jj]);
    }
  }
}

// Full tiles take the unmasked path; a tile with a key at or past valid_end,
// or past some valid column's limit, takes the masked one.
template <int kEnc, int NCB, bool kSideRegs = false, int kSideN = kSideMax, bool kPLo = false>
__device__ __forceinline__ void attend(ColState<NCB, kSideN>& st, const Tile<kEnc>& t,
                                       const QOps<kEnc, NCB, kSideN>& Q, const ColInfo (&ci)[NCB],
                                       int key0, int valid_end, int min_klim, int64_t slot0,
                                       const AttnParams& p, int g, const LaneId& L,
                                       const char* plo_v = nullptr, f32x4_t* plo = nullptr,
                                       int n_plo = 0, int plo_dim = 0) {
  if (key0 + kTile <= valid_end && key0 + kTile - 1 <= min_klim) {
    attend_tile<kEnc, NCB, false, kSideRegs, kSideN, kPLo>(st, t, Q, ci, key0, valid_end, slot0,
                                                           p, g, L, plo_v, plo, n_plo, plo_dim);
  } else {
    attend_tile<kEnc, NCB, true, kSideRegs, kSideN, kPLo>(st, t, Q, ci, key0, valid_end, slot0,
                                                          p, g, L, plo_v, plo, n_plo, plo_dim);
  }
}

// ---------------------------------------------------------------------------
// Epilogue helpers.  A wave dumps one column block (unnormalised O, final
// max and sum) into LDS: obuf[col][d] fp32, ml[col] = (m, l).
// ---------------------------------------------------------------------------
struct WaveOut {
  float o[16][kD];
  float m[16];
  float l[16];
};

template <int kEnc, int NCB, int kSideN>
__device__ __forceinline__ void dump_block(WaveOut& wo, const ColState<NCB, kSideN>& st, int cb,
                                           const AttnParams& p, int g, const LaneId& L) {
  float l = st.l[cb];
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  float bias = 0.f;
  if constexpr (kEnc != kBF16) {
    float vb = st.vb[cb];
    vb += shfl_xor(vb, 16);
    vb += shfl_xor(vb, 32);
    bias = 128.f * vb;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d0 = 32 * L.lg + 8 * r;
    float v[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) v[jj] = st.o[cb][jj][r] - bias;
    if constexpr (kEnc == kI8Chan) {
      const float* vs = p.v_scale + g * kD + d0;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) v[jj] *= vs[jj];
    }
    float4* dst = reinterpret_cast<float4*>(&wo.o[L.lm][d0]);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  if (L.lg == 0) {
    wo.m[L.lm] = st.m[cb];
    wo.l[L.lm] = l;
  }
  if constexpr (kEnc == kI8Chan) {
    const int n_out = p.head_n_out != nullptr ? p.head_n_out[g] : 0;
    float sd[kSideN];
#pragma unroll
    for (int j = 0; j < kSideN; ++j) {
      float s = st.sd[cb][j];
      s += shfl_xor(s, 16);
      s += shfl_xor(s, 32);
      sd[j] = s;
    }
    // The main path left exactly 0 at the outlier dims (read scale 0 there);
    // the exact side contribution takes their place.
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (L.lg == 0) {
#pragma unroll
      for (int j = 0; j < kSideN; ++j)
        if (j < n_out) wo.o[L.lm][p.out_idx[g * p.n_out_max + j]] = sd[j];
    }
  }
}

__device__ __forceinline__ void store_final(const AttnParams& p, int64_t row, int head, int d0,
                                            const float (&v)[8], float inv_l) {
  uint16_t* dst = p.out + row * p.o_st + int64_t(head) * p.o_sh + d0;
  *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{
      pack_bf16x2_fast(v[0] * inv_l, v[1] * inv_l), pack_bf16x2_fast(v[2] * inv_l, v[3] * inv_l),
      pack_bf16x2_fast(v[4] * inv_l, v[5] * inv_l), pack_bf16x2_fast(v[6] * inv_l, v[7] * inv_l)};
}

__device__ __forceinline__ void store_partial(const AttnParams& p, int64_t row, int head, int split,
                                              int d0, const float (&v)[8], float m, float l) {
  const int64_t base = (row * p.num_heads + head) * p.max_splits + split;
  const float inv_l = l > 0.f ? 1.f / l : 0.f;
  float4* dst = reinterpret_cast<float4*>(p.part_o + base * kD + d0);
  dst[0] = make_float4(v[0] * inv_l, v[1] * inv_l, v[2] * inv_l, v[3] * inv_l);
  dst[1] = make_float4(v[4] * inv_l, v[5] * inv_l, v[6] * inv_l, v[7] * inv_l);
  if (d0 == 0) p.part_lse[base] = l > 0.f ? m + __log2f(l) : -INFINITY;
}

constexpr int kDecodeSmem = kWaves * int(sizeof(WaveOut));
constexpr int kTileBytesBF16 = kTile * kPitchBF16;
// Two buffers of (K tile, V tile) in bf16 (an int8 pool's tiles are
// dequantised on their way in), then the per-channel read scales (1 KiB).
constexpr int kPrefillStage = 2 * kTileBytesBF16;
constexpr int kPrefillSmem = 2 * kPrefillStage + 2 * kD * 4;
constexpr int kSmemBytes = kDecodeSmem > kPrefillSmem ? kDecodeSmem : kPrefillSmem;

// ---------------------------------------------------------------------------
// Decode segment: 32-key tiles [t0, t1) of row b's context for a group of kv
// slices.  A kv slice is one kv head (or a 16-head slice of a group wider
// than 16 q heads).  The workgroup covers p.kvs_per_wg slices: wave w serves
// slice w % kvs_per_wg and takes every streams-th tile of the segment
// (streams = 8 / kvs_per_wg).  With the engine's layout a token row holds
// every kv head contiguously ([page, KVH, D]), so the waves of one workgroup
// read whole token rows (KVH x 256 B) together instead of 256-byte slivers at
// a KVH x 256-byte stride; the streaming read rate of the first pattern is
// measured ~13 % higher on MI355X.  Waves of the same slice merge through
// LDS; the result is the final output row (split < 0) or split-K partial
// `split`.  Ends with a barrier, so LDS can be reused right after.
// ---------------------------------------------------------------------------
template <int kEnc>
__device__ __forceinline__ void decode_segment(const AttnParams& p, char* smem, const int32_t* bt, int b, int kvg,
                               int ctx, int t0, int t1, int split) {
  b = uniform(b);
  // The kv group too: it sets every tile's buffer resource, which must sit in
  // scalar registers (a resource the compiler cannot prove uniform becomes a
  // loop over lanes around each load).
  kvg = uniform(kvg);
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));  // wave-uniform (scalar) index
  const int per = p.kvs_per_wg;
  const int streams = kWaves / per;
  const int local = wave % per;   // slice within the workgroup
  const int stream = wave / per;  // tile stream of that slice
  const int kvs = kvg * per + local;
  const int g = kvs / p.nslices;
  const int s = kvs - g * p.nslices;
  const int hs = min(p.hs, p.group - s * p.hs);
  // The segment bounds are wave-uniform whatever path computed them; keeping
  // them (and the key index below) scalar keeps the block-table lookups on
  // the scalar unit, off the vector-memory counter that the tile prefetch
  // ring waits on.
  ctx = uniform(ctx);
  t0 = uniform(t0);
  t1 = uniform(t1);
  const int ntiles = t1 > t0 ? t1 - t0 : 0;
  const int c0 = t0 * kTile;
  // Tiles are dealt round-robin over the streams: at any moment the
  // workgroup reads `streams` consecutive tiles of every slice, one
  // contiguous stretch of the page.
  const int my_tiles = ntiles > stream ? (ntiles - stream + streams - 1) / streams : 0;

  ColInfo ci[1];
  ci[0].row = b;
  ci[0].head = g * p.group + s * p.hs + L.lm;
  ci[0].valid = L.lm < hs;
  ci[0].klim = ctx - 1;

  const int64_t head_off = int64_t(g) * ((kEnc == kBF16) ? kD * 2 : kD);
  const int tok = int(p.tok_bytes);
  const int span = kTile * tok;
  const TileOffsets off = tile_offsets<kEnc>(tok, L);
  // j-th tile of this wave -> segment-relative tile index
  auto tile_of = [&](int j) { return stream + j * streams; };
  auto tile_slot0 = [&](int tix) -> int64_t {
    const int key0 = uniform(c0 + tix * kTile);
    const int blk = table_entry(bt, key0 / p.page);
    return int64_t(blk) * p.page + (key0 % p.page);
  };
  WaveOut* wo = reinterpret_cast<WaveOut*>(smem);
  // The tile loop, for a side-pool width of kN values (per-channel int8: the
  // pool's n_out_max, which sizes the side loads and the side state; 1 for
  // the other encodings, which have no side pool).
  auto run = [&](auto side_width) {
    constexpr int kN = decltype(side_width)::value;
    QOps<kEnc, 1, kN> Q;
    build_q<kEnc, 1>(Q, p, ci, g, L);
    ColState<1, kN> st;
    init_state(st);
    // live == false turns the tile's loads into no-ops (num_records = 0).
    auto load = [&](Tile<kEnc>& t, int64_t slot0, bool live) {
      const char* kb = p.k_cache + slot0 * p.tok_bytes + head_off;
      const char* vb = p.v_cache + slot0 * p.tok_bytes + head_off;
      const int nrec = live ? span : 0;
      if constexpr (kEnc == kBF16) {
        load_tile_buf(t, wave_rsrc(kb, nrec), wave_rsrc(vb, nrec), off);
      } else {
        load_tile_buf_i8<kEnc>(t, wave_rsrc(kb, nrec), wave_rsrc(vb, nrec), off);
      }
      if constexpr (kEnc == kI8Tok) {
        load_scales_buf(p.k_scale + slot0 * p.kvh, p.v_scale + slot0 * p.kvh, p.kvh, g, live, L,
                        t.sck, t.scv);
      }
      if constexpr (kEnc == kI8Chan) load_side_buf<kN>(t, p, slot0, g, live && Q.n_out > 0, L);
    };

    if (my_tiles > 0) {
      // Ring of kRing tile buffers: tile j is computed from buffer j % kRing
      // while the next kRing - 1 tiles are in flight; the buffer is refilled
      // with tile j + kRing right after.
      constexpr int kRing = 2;
      Tile<kEnc> ring[kRing];
      int64_t slot[kRing];
#pragma unroll
      for (int r = 0; r < kRing; ++r) {
        slot[r] = tile_slot0(tile_of(min(r, my_tiles - 1)));
        load(ring[r], slot[r], r < my_tiles);
      }
      for (int j0 = 0; j0 < my_tiles; j0 += kRing) {
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
          const int j = j0 + r;
          if (j < my_tiles)
            attend<kEnc, 1, kEnc == kI8Chan>(st, ring[r], Q, ci, c0 + tile_of(j) * kTile, ctx,
                                             ctx - 1, slot[r], p, g, L);
          const int nxt = j + kRing;
          slot[r] = tile_slot0(tile_of(min(nxt, my_tiles - 1)));
          load(ring[r], slot[r], nxt < my_tiles);
        }
      }
    }
    dump_block<kEnc, 1>(wo[wave], st, 0, p, g, L);
  };
  if constexpr (kEnc == kI8Chan) {
    switch (p.n_out_max) {
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      case 4: run(std::integral_constant<int, 4>{}); break;
      default: run(std::integral_constant<int, 8>{}); break;
    }
  } else {
    run(std::integral_constant<int, 1>{});
  }
  __syncthreads();
  // Merge the streams of every slice: 16 threads per (slice, column), each
  // owning 8 dims; 32 columns per pass over the workgroup.
  const int ncols = per * 16;
  for (int cidx = threadIdx.x >> 4; cidx < ncols; cidx += kThreads / 16) {
    const int sl = cidx >> 4;   // slice within the workgroup
    const int col = cidx & 15;  // q head within the slice
    const int kvs_c = kvg * per + sl;
    const int g_c = kvs_c / p.nslices;
    const int s_c = kvs_c - g_c * p.nslices;
    const int hs_c = min(p.hs, p.group - s_c * p.hs);
    if (col >= hs_c) continue;
    const int d0 = (threadIdx.x & 15) * 8;
    float m = -INFINITY;
    for (int w = sl; w < kWaves; w += per) m = fmaxf(m, wo[w].m[col]);
    const float m_use = (m == -INFINITY) ? 0.f : m;
    float l = 0.f, v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int w = sl; w < kWaves; w += per) {
      const float e = __builtin_amdgcn_exp2f(wo[w].m[col] - m_use);
      l += e * wo[w].l[col];
      const float4 a = *reinterpret_cast<const float4*>(&wo[w].o[col][d0]);
      const float4 c = *reinterpret_cast<const float4*>(&wo[w].o[col][d0 + 4]);
      v[0] += e * a.x; v[1] += e * a.y; v[2] += e * a.z; v[3] += e * a.w;
      v[4] += e * c.x; v[5] += e * c.y; v[6] += e * c.z; v[7] += e * c.w;
    }
    const int head = g_c * p.group + s_c * p.hs + col;
    if (split < 0) {
      store_final(p, b, head, d0, v, 1.f / l);
    } else {
      store_partial(p, b, head, split, d0, v, m, l);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// LDS-staged decode segment (bf16 pool, a group of 4 kv heads = 1 KiB of each
// token row).  Each 32-key tile is brought into LDS as whole token rows — one
// 1 KiB direct-to-LDS load per row, 64 rows (K and V) spread over the 8 waves
// — double-buffered, rows padded to 1040 B so the operand reads are free of
// bank conflicts.  Streaming whole contiguous rows is measurably faster than
// per-head register loads (~7.2 vs ~6.85 TB/s on MI355X).  Wave w serves kv
// head w % 4 and dim half w / 4: both halves compute the full S^T tile and
// softmax (identical), each accumulates O^T for its 64 dims (dims
// 8m + 4h .. 8m + 4h + 3 of the PV MFMA rows), so no cross-wave merge.
// ---------------------------------------------------------------------------
constexpr int kLdsPitch = 1024 + 16;
constexpr int kLdsTensor = kTile * kLdsPitch;
constexpr int kLdsStage = 2 * kLdsTensor;
// Query block of the LDS path: [4 kv heads][16 columns][256 B], the 16-byte
// chunks of row (h, c) stored at chunk index ^ c so that 16 columns reading
// the same dims hit 16 different bank groups.
constexpr int kLdsQ = 4 * 16 * 256;

// V^T operand of PV MFMA jj (0..3 within the wave's half) from half rows:
// v[i] holds dims 8lm + 4h .. +3 of key slot i.
__device__ __forceinline__ u32x4_t v_operand_half(const u32x2_t (&v)[8], int jj) {
  const uint32_t sel = (jj & 1) ? kPermHiHi : kPermLoLo;
  const int dw = jj >> 1;
  return u32x4_t{perm(v[1][dw], v[0][dw], sel), perm(v[3][dw], v[2][dw], sel),
                 perm(v[5][dw], v[4][dw], sel), perm(v[7][dw], v[6][dw], sel)};
}

// One 16-byte-per-lane load straight into LDS: lane i's 16 bytes from
// rsrc + voff land at LDS address lds + 16 i.  Issued through inline asm so
// the compiler's wait-count pass does not treat it as a pending LDS write
// (it would then drain every load in flight before each barrier and LDS read,
// serialising the prefetch); the caller waits with explicit vmcnt counts.
// M0 carries the LDS address and is restored afterwards.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4_t raw_rsrc(const void* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{int(__builtin_amdgcn_readfirstlane(uint32_t(a))),
                 int(__builtin_amdgcn_readfirstlane(uint32_t(a >> 32) & 0xffffu)),
                 int(__builtin_amdgcn_readfirstlane(uint32_t(bytes))), kBufWord3};
}

__device__ __forceinline__ void dma_to_lds(const i32x4_t& rsrc, int voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "buffer_load_dwordx4 %1, %3, 0 offen nt lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(lds), "s"(rsrc)
      : "memory");
}

// The same load with the default cache policy, for data that other
// workgroups read again soon (prefill keys and queries).
__device__ __forceinline__ void dma_to_lds_cached(const i32x4_t& rsrc, int voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(lds), "s"(rsrc)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p)));
}

// s_waitcnt immediate for lgkmcnt(0) alone (vmcnt 63 and expcnt 7 do not wait).
constexpr int kWaitLgkm0 = 0xC07F;

// Workgroup barrier over LDS only: this wave's LDS accesses are complete and
// every wave has arrived.  (__syncthreads would also wait for the epilogue's
// global stores, and with them for every direct-to-LDS load in flight.)  The
// wait and the barrier are builtins, so the compiler's wait-count model knows
// the LDS queue is empty after it; the empty asm statements keep memory
// accesses from moving across it.
__device__ __forceinline__ void pf_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Scalar loads (block-table entries, chunk bounds) are waited for right where
// they are issued: while one is pending the compiler's wait-count model must
// treat the LDS counter as out of order and waits for every LDS read before
// the first use of any, which serialises the K and V operand reads with the
// MFMAs.  With the queue drained here its LDS waits stay partial.
__device__ __forceinline__ void smem_drain() { __builtin_amdgcn_s_waitcnt(kWaitLgkm0); }

// Scores are kept relative to mu (the running max m, or 0 while m is -inf):
// x' = x - mu comes out of one FMA and feeds exp2 directly.  The rescale test
// is lane-local (x' > thr, thr = kRescaleLog2 once m is finite, -inf before),
// so the column max across the four lane groups is only formed on the rare
// rescale path, which also carries its own copy of the P V part (the common
// path's accumulators then flow straight into its MFMAs).
struct HalfState {
  f32x4_t o[4];  // O^T rows of PV MFMA jj (local 0..3): dim 32lg + 8r + 4h + jj
  float m;       // running reference max of x (log2 units), -inf before any key
  float mu;      // m, or 0 while m is -inf
  float thr;     // rescale threshold on x'
  float l;       // lane-partial sum of exp2(x') over the lane's key slots
};

__device__ __forceinline__ void init_half(HalfState& st) {
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) st.o[jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.mu = 0.f;
  st.thr = -INFINITY;
  st.l = 0.f;
}

__device__ __forceinline__ void half_pv(HalfState& st, const float (&x)[8],
                                        const u32x2_t (&vrow)[8]) {
  float pr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pr[i] = __builtin_amdgcn_exp2f(x[i]);
  st.l += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
  u32x4_t pb;
#pragma unroll
  for (int w = 0; w < 4; ++w) pb[w] = pack_bf16x2_fast(pr[2 * w], pr[2 * w + 1]);
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) st.o[jj] = mfma_bf16(v_operand_half(vrow, jj), pb, st.o[jj]);
}

template <bool kMasked>
__device__ __forceinline__ void attend_tile_half(HalfState& st, const u32x4_t (&k)[2][4],
                                                 const u32x2_t (&vh)[8],
                                                 const QOps<kBF16, 1>& Q, int key0,
                                                 int valid_end, int klim, float scale_log2,
                                                 const LaneId& L) {
  bool kvalid[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) kvalid[i] = !kMasked || (key0 + key_of_slot(L.lg, i) < valid_end);
  u32x2_t vrow[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    vrow[i] = vh[i];
    if (kMasked && !kvalid[i]) vrow[i] = u32x2_t{0u, 0u};
  }
  f32x4_t s0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    s0 = mfma_bf16(k[0][c], Q.op[0][c], s0);
    s1 = mfma_bf16(k[1][c], Q.op[0][c], s1);
  }
  const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  float x[8];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float v = fmaf(sv[i], scale_log2, -st.mu);
    if constexpr (kMasked) {
      const bool ok = kvalid[i] && (key0 + key_of_slot(L.lg, i) <= klim);
      x[i] = ok ? v : -INFINITY;
    } else {
      x[i] = v;
    }
    tmax = fmaxf(tmax, x[i]);
  }
  if (__builtin_expect(__ballot(tmax > st.thr) != 0, 0)) {
    const float m_new = fmaxf(st.m, rows4_max(tmax + st.mu));
    const float mu_new = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m - mu_new);
    const float shift = st.mu - mu_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] += shift;
    st.m = m_new;
    st.mu = mu_new;
    st.thr = (m_new == -INFINITY) ? -INFINITY : kRescaleLog2;
    st.l *= alpha;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      st.o[jj][0] *= alpha;
      st.o[jj][1] *= alpha;
      st.o[jj][2] *= alpha;
      st.o[jj][3] *= alpha;
    }
    half_pv(st, x, vrow);
  } else {
    half_pv(st, x, vrow);
  }
}

// The fused append's 16 bytes of lane `lane` of row b's new K and V, for kv
// heads 4 kvg .. 4 kvg + 3: head 4 kvg + lane / 16, dims 8 (lane % 16) .. +7,
// i.e. the bytes the lane's DMA slot covers in a token row of the pool.
template <int kHeads = 4>
__device__ __forceinline__ void append_load(const AttnParams& p, int b, int kvg, int lane,
                                            u32x4_t& kn, u32x4_t& vn) {
  const int head = kvg * kHeads + (lane >> 4);
  const int d = (lane & 15) * 8;
  kn = *reinterpret_cast<const u32x4_t*>(p.app_k + int64_t(b) * p.app_k_st +
                                         int64_t(head) * p.app_k_sh + d);
  vn = *reinterpret_cast<const u32x4_t*>(p.app_v + int64_t(b) * p.app_v_st +
                                         int64_t(head) * p.app_v_sh + d);
}

// Stores them at row b's slot (store_kvcache's rules for the slot).
template <int kHeads = 4>
__device__ __forceinline__ void append_store(const AttnParams& p, int b, int kvg, int lane,
                                             const u32x4_t& kn, const u32x4_t& vn) {
  const int64_t raw = p.app_slot_bytes == 8 ? load_index<8>(p.app_slots, b)
                                            : load_index<4>(p.app_slots, b);
  const int64_t slot = wrap_slot(raw, p.app_num_slots);
  if (slot < 0 || slot >= p.app_num_slots) return;
  const int64_t off = slot * p.tok_bytes + int64_t(kvg) * (kHeads * 256) + lane * 16;
  *reinterpret_cast<u32x4_t*>(const_cast<char*>(p.k_cache) + off) = kn;
  *reinterpret_cast<u32x4_t*>(const_cast<char*>(p.v_cache) + off) = vn;
}

// One segment of a decode share: tiles t0 .. t1 of row b's kv group kvg,
// written as a split partial when split >= 0.  (Block-table rows are formed
// from the kernel argument where they are read, so the compiler keeps those
// reads scalar.)  With the dynamic tail hand-out:
// * tail > 0 (the owner's last segment): its last `tail` tiles are claimed
//   one at a time from the front of the share's claim word and the segment
//   ends early at the first tile another workgroup took;
// * tslot >= 0 (a taken tile of another share): one tile, written to that
//   tail slot.
struct DecSeg {
  int b, kvg, ctx, t0, t1, split;
  int tail, tslot;
};

// Claim-word fields (see StealArgs::claims).
__device__ __forceinline__ int claim_front(unsigned long long o) { return int(o & 0xffffu); }
__device__ __forceinline__ int claim_back(unsigned long long o) { return int((o >> 16) & 0xffffu); }
__device__ __forceinline__ int claim_tiles(unsigned long long o) { return int((o >> 32) & 0xffffu); }

// One claim on a share's word (lane 0 of a wave): `inc` 1 takes the next tile
// from the front, 1 << 16 the next from the back; the returned word before
// the add decides (valid iff front + back < tiles).  Eight ordinary stores to
// the workgroup's dummy words follow, so the compiler's wait-count model sees
// the atomic eight memory operations deep: any wait it inserts before the
// result is used is then at most vmcnt(8), which in hardware never waits for
// the tile loads issued after these stores (eight per wave per tile).
__device__ __forceinline__ unsigned long long claim_word(unsigned long long* word,
                                                         unsigned long long inc, int* dummy) {
  const unsigned long long old =
      __hip_atomic_fetch_add(word, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __hip_atomic_store(dummy + i, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  asm volatile("" ::: "memory");
  return old;
}

// `next(nx)` names the share's next segment (false: none); it is asked
// after this segment's first loads are issued, so its reads overlap them.
// Returns whether a next segment was found (its first loads are then in
// flight: call it with `pre`).  s_claim: one LDS int, the verdict of the
// owner's pending tail claim for every wave; w: this workgroup's share.
template <bool kSteal = false, typename NextFn>
__device__ __forceinline__ bool decode_segment_lds(const AttnParams& p, char* stage0, char* stage1,
                                                   char* qlds,
                                                   const int32_t* __restrict__ block_tables,
                                                   const DecSeg& sg, bool pre, NextFn&& next,
                                                   DecSeg& nx, const StealArgs& sa, int* s_claim,
                                                   int w) {
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));
  const int gl = wave & 3;   // kv head within the group
  const int hf = wave >> 2;  // dim half
  const int b = uniform(sg.b);
  const int kvg = uniform(sg.kvg);
  const int ctx = uniform(sg.ctx);
  const int t0 = uniform(sg.t0);
  const int t1 = uniform(sg.t1);
  const int split = uniform(sg.split);
  const int tail = kSteal ? uniform(sg.tail) : 0;
  const int tslot = kSteal ? uniform(sg.tslot) : -1;
  const int g = kvg * 4 + gl;
  const int nstatic = t1 > t0 ? t1 - t0 : 0;
  int ntiles = nstatic;  // shrinks when another workgroup takes tail tiles
  const int ft = nstatic - tail;  // first tail tile (tail <= nstatic - 4)
  const int c0 = t0 * kTile;
  // Fused append: the segment holding the row's last tile stores the new
  // token's K/V rows, and the wave whose DMA brings that token's row into
  // the last tile's stage overwrites it there with the same bytes (so the
  // tile never depends on when the pool store lands).  When the owner's
  // last tile is taken, the taker does both.
  const bool app = p.app_k != nullptr && nstatic > 0 && t1 == (ctx + kTile - 1) / kTile;
  const int app_row = (ctx - 1) & (kTile - 1);
  const bool app_wave = app && wave == (app_row & 7);
  u32x4_t app_kn, app_vn;

  QOps<kBF16, 1> Q;
  HalfState st;
  init_half(st);
  bool has_next = false;

  // The owner's claims (lane 0 of wave 0): the claim for tile x is issued
  // right after the DMA of tile x - 2 (step x - 4) and decided in step
  // x - 2, before tile x's DMA, so like a tile it has two steps to return
  // (loads complete in issue order: a claim issued ahead of a tile's DMA
  // would have to return one step later, and an agent-scope atomic under
  // full load takes longer).  After a step that issued a claim, wave 0's
  // tile wait leaves that claim and its eight dummy stores outstanding too
  // (vmcnt(17)).  claimed: the last tile whose claim went out.
  unsigned long long cret[2] = {0, 0};  // claims in flight, by tile parity
  int claimed = ft - 1;
  int claim_step = -2;                  // the step that issued the last claim
  unsigned long long* const cword = tail > 0 ? sa.claims + w : nullptr;
  int* const cdummy = sa.dummy + int64_t(w) * 8;

  const int tok = int(p.tok_bytes);
  // Wave w loads rows w, w + 8, w + 16, w + 24 of K and of V of the tile at
  // key0 of a segment's row (b_) and kv group (kvg_).
  auto issue_tile = [&](int b_, int kvg_, int key0, char* base) {
    const int blk = table_entry(block_tables, int64_t(b_) * p.bt_stride + key0 / p.page);
    const int64_t slot0 = int64_t(blk) * p.page + (key0 % p.page);
    const int64_t grp_off = int64_t(kvg_) * 1024;
    const i32x4_t kr = raw_rsrc(p.k_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
    const i32x4_t vr = raw_rsrc(p.v_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
    const uint32_t lb = lds_addr(base);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = wave + 8 * q;
      dma_to_lds(kr, row * tok + L.lane * 16, lb + row * kLdsPitch);
      dma_to_lds(vr, row * tok + L.lane * 16, lb + kLdsTensor + row * kLdsPitch);
    }
  };
  auto issue = [&](int tix, char* base) {
    issue_tile(b, kvg, uniform(c0 + tix * kTile), base);
  };
  // The query rides the same DMA ahead of a segment's first two tiles: wave
  // w brings columns 8 (w >> 2) .. + 7 of kv head w & 3 (columns past the
  // head count repeat the last head; their results are never stored).
  auto issue_q = [&](int b_, int kvg_) {
    const int g_ = kvg_ * 4 + gl;
    const i32x4_t qr =
        raw_rsrc(p.q + int64_t(b_) * p.q_st, int(int64_t(p.num_heads) * p.q_sh * 2));
    const uint32_t lb = lds_addr(qlds);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int col = 8 * hf + 4 * s + (L.lane >> 4);
      const int head = g_ * p.group + min(col, p.hs - 1);
      const int chunk = (L.lane & 15) ^ col;
      dma_to_lds(qr, int(int64_t(head) * p.q_sh * 2) + chunk * 16,
                 lb + (gl * 16 + 8 * hf + 4 * s) * 256);
    }
  };

  // Tile j lives in stage j & 1.  A stage is read into registers as soon as
  // its tile has landed and is refilled with tile j + 2 before tile j is
  // computed, so two tiles stay in flight under the arithmetic.  The loop is
  // unrolled by two so every access names its stage statically.  At the
  // last tile both stages and the query block are free: the next segment's
  // query and first two tiles are issued there (its `pre`), so its start
  // does not wait out a full load latency.  Barriers cover LDS only: the
  // epilogue's global stores must not hold back the loads in flight.
  u32x4_t k[2][4];
  u32x2_t vh[8];
  auto read_stage = [&](const char* kb) {
    const char* vb = kb + kLdsTensor;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const char* row = kb + (h * 16 + L.lm) * kLdsPitch + gl * 256 + L.lg * 16;
#pragma unroll
      for (int c = 0; c < 4; ++c) k[h][c] = *reinterpret_cast<const u32x4_t*>(row + c * 64);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vh[i] = *reinterpret_cast<const u32x2_t*>(vb + key_of_slot(L.lg, i) * kLdsPitch + gl * 256 +
                                                L.lm * 16 + hf * 8);
  };
  auto compute = [&](int j) {
    const int key0 = c0 + j * kTile;
    if (key0 + kTile <= ctx) {
      attend_tile_half<false>(st, k, vh, Q, key0, ctx, ctx - 1, p.scale_log2, L);
    } else {
      attend_tile_half<true>(st, k, vh, Q, key0, ctx, ctx - 1, p.scale_log2, L);
    }
  };
  // One step: tile j is in `stage`; tile j + 1 (if any) is already in flight.
  auto step = [&](int j, char* stage) {
    if (j + 1 < ntiles) {
      if (kSteal && wave == 0 && claim_step == j - 1) {
        __builtin_amdgcn_s_waitcnt(0x4F71);  // vmcnt(17): tile j + 1, a claim, 8 stores
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): this wave's loads of tile j
      }
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    // The claim for tile j + 2 went out in step j - 2: it is done.
    const bool pend = tail > 0 && j + 2 >= ft && j + 2 <= claimed && j + 2 < ntiles;
    if (pend && wave == 0 && L.lane == 0) {
      const unsigned long long c = cret[j & 1];
      *s_claim = claim_front(c) + claim_back(c) < claim_tiles(c) ? 1 : 0;
    }
    if (app_wave && j == nstatic - 1) {
      // this wave's DMA of the row has landed (vmcnt(0) above); the pool
      // store is issued after the segment's last tile
      *reinterpret_cast<u32x4_t*>(stage + app_row * kLdsPitch + L.lane * 16) = app_kn;
      *reinterpret_cast<u32x4_t*>(stage + kLdsTensor + app_row * kLdsPitch + L.lane * 16) = app_vn;
    }
    pf_barrier();
    if (pend && uniform(*s_claim) == 0) ntiles = j + 2;
    read_stage(stage);
    pf_barrier();  // every wave holds the stage in registers (and the verdict)
    if (j + 2 < ntiles) {
      issue(j + 2, stage);
      if (tail > 0 && j + 4 >= ft && j + 4 < nstatic) {
        if (wave == 0 && L.lane == 0) cret[j & 1] = claim_word(cword, 1ull, cdummy);
        claimed = j + 4;
        claim_step = j;
      }
    }
    if (has_next && j == ntiles - 1) {
      const int nb = uniform(nx.b);
      const int nkvg = uniform(nx.kvg);
      const int nc0 = uniform(nx.t0) * kTile;
      issue_q(nb, nkvg);
      issue_tile(nb, nkvg, nc0, stage0);
      if (uniform(nx.t1) - uniform(nx.t0) > 1) issue_tile(nb, nkvg, nc0 + kTile, stage1);
    }
    compute(j);
  };
  if (ntiles > 0) {
    if (!pre) {
      issue_q(b, kvg);
      issue(0, stage0);
      if (ntiles > 1) issue(1, stage1);
    }
    has_next = next(nx);
    // Issued after the segment's first DMAs (and, with `pre`, after the
    // previous segment's output stores): the waits below count only the
    // youngest loads as outstanding, so they can only wait longer, never
    // less, than they name.
    if (app_wave) append_load(p, b, kvg, L.lane, app_kn, app_vn);
    if (ntiles > 1) {
      __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16): this wave's query loads
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    }
    pf_barrier();
    {
      const char* row = qlds + (gl * 16 + L.lm) * 256;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        Q.op[0][c] = *reinterpret_cast<const u32x4_t*>(row + (((4 * c + L.lg) ^ L.lm) * 16));
    }
    // The first tail tile is at least 4: its claim goes out in step 0,
    // after tile 2's DMA.
    for (int j0 = 0; j0 < ntiles; j0 += 2) {
      step(j0, stage0);
      if (j0 + 1 < ntiles) step(j0 + 1, stage1);
    }
  }

  if (app_wave && ntiles == nstatic) append_store(p, b, kvg, L.lane, app_kn, app_vn);
  // Tiles of the owner's tail that other workgroups took: they are pieces of
  // their own, so this row is split even when the share held all of it.
  const int taken = tail > 0 ? nstatic - ntiles : 0;
  const int piece = split < 0 ? 0 : split;
  const int out_split = split < 0 && taken > 0 ? 0 : split;
  if (kSteal && tslot < 0 && wave == 0 && L.lane < 4)
    sa.stolen[(int64_t(b) * (p.kvh * p.nslices) + kvg * 4 + L.lane) * p.max_splits + piece] =
        taken;
  // Epilogue: lane (lm, lg) holds, for r = 0..3, dims 32lg + 8r + 4hf .. +3
  // of column lm; l is lane-partial over the key slots.
  const float l = rows4_sum(st.l);
  if (L.lm < p.hs) {
    const int head = g * p.group + L.lm;
    const float inv_l = 1.f / l;
    if (out_split < 0 && tslot < 0) {
      uint16_t* dst = p.out + int64_t(b) * p.o_st + int64_t(head) * p.o_sh;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = 32 * L.lg + 8 * r + 4 * hf;
        *reinterpret_cast<u32x2_t*>(dst + d0) =
            u32x2_t{pack_bf16x2_fast(st.o[0][r] * inv_l, st.o[1][r] * inv_l),
                    pack_bf16x2_fast(st.o[2][r] * inv_l, st.o[3][r] * inv_l)};
      }
    } else {
      float* po;
      float* pl;
      if (tslot >= 0) {
        const int64_t base = int64_t(tslot) * sa.uh + gl * p.group + L.lm;
        po = sa.tail_o + base * kD;
        pl = sa.tail_lse + base;
      } else {
        const int64_t base = (int64_t(b) * p.num_heads + head) * p.max_splits + out_split;
        po = p.part_o + base * kD;
        pl = p.part_lse + base;
      }
      const float il = l > 0.f ? inv_l : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = 32 * L.lg + 8 * r + 4 * hf;
        *reinterpret_cast<float4*>(po + d0) =
            make_float4(st.o[0][r] * il, st.o[1][r] * il, st.o[2][r] * il, st.o[3][r] * il);
      }
      if (L.lg == 0 && hf == 0) *pl = l > 0.f ? st.m + __log2f(l) : -INFINITY;
    }
  }
  if (!has_next) {
    // nothing in flight for a next segment: drain and realign the waves
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  return has_next;
}

// The LDS-staged segment for 2 kv heads per workgroup (bf16; the 16q/2kv
// shard of a 2-way tensor-parallel rank): a token row is 512 B, so one
// 66.5 KB stage holds 64 keys (two 32-key tiles) of K and V and a step
// attends both.  Wave w serves kv head w & 1, dim half (w >> 1) & 1 and tile
// w >> 2 of the step: per step every wave does exactly the work of the 4-head
// segment (one head, one dim half, one 32-key tile) and issues the same 8
// loads, so the wait counts are unchanged.  A direct-to-LDS load brings two
// consecutive token rows (64 lanes x 16 B), stored as a pair at the 1040-byte
// pitch.  A step's second tile past the segment loads nothing (a zero-length
// buffer) and is not attended.  The two tiles' softmax states of a (head, dim
// half) merge through LDS once, in the epilogue.
constexpr int kLdsQ2 = 2 * 16 * 256;            // query block: [2 heads][16 columns][256 B]
constexpr int kLds2Merge = 4 * 18 * 64 * 4;     // tile-1 waves' states: 16 O, m, l per lane
constexpr int kLdsSmem2 = kLdsQ2 + kLds2Merge;
static_assert(2 * kLdsStage + kLdsSmem2 <= 160 * 1024, "one workgroup per CU");

template <typename NextFn>
__device__ __forceinline__ bool decode_segment_lds2(const AttnParams& p, char* stage0,
                                                    char* stage1, char* smem2,
                                                    const int32_t* __restrict__ block_tables,
                                                    const DecSeg& sg, bool pre, NextFn&& next,
                                                    DecSeg& nx) {
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));
  const int gl = wave & 1;         // kv head within the pair
  const int hf = (wave >> 1) & 1;  // dim half
  const int kt = wave >> 2;        // tile of the step
  char* const qlds = smem2;
  float* const mlds = reinterpret_cast<float*>(smem2 + kLdsQ2);
  const int b = uniform(sg.b);
  const int kvg = uniform(sg.kvg);
  const int ctx = uniform(sg.ctx);
  const int t0 = uniform(sg.t0);
  const int t1 = uniform(sg.t1);
  const int split = uniform(sg.split);
  const int g = kvg * 2 + gl;
  const int ntiles = t1 > t0 ? t1 - t0 : 0;
  const int nsteps = (ntiles + 1) >> 1;
  const int c0 = t0 * kTile;
  // Fused append: the row's last tile is tile ntiles - 1 of this segment; its
  // new token is stage row app_r of step app_step, brought by the lanes
  // 32 (app_r & 1) .. + 31 of wave (app_r >> 1) & 7.
  const bool app = p.app_k != nullptr && ntiles > 0 && t1 == (ctx + kTile - 1) / kTile;
  const int app_r = ((ntiles - 1) & 1) * kTile + ((ctx - 1) & (kTile - 1));
  const int app_step = (ntiles - 1) >> 1;
  const bool app_wave = app && wave == ((app_r >> 1) & 7);
  const bool app_lane = app_wave && (L.lane >> 5) == (app_r & 1);
  u32x4_t app_kn, app_vn;

  QOps<kBF16, 1> Q;
  HalfState st;
  init_half(st);
  bool has_next = false;

  const int tok = int(p.tok_bytes);
  // Tile `key0` of a segment's row (b_) and kv pair (kvg_) as half `half` of
  // a stage: wave w loads row pairs w and w + 8 of it, K and V.
  auto issue_tile = [&](int b_, int kvg_, int key0, int half, bool live, char* base) {
    i32x4_t kr, vr;
    if (live) {
      const int blk = table_entry(block_tables, int64_t(b_) * p.bt_stride + key0 / p.page);
      const int64_t slot0 = int64_t(blk) * p.page + (key0 % p.page);
      const int64_t grp_off = int64_t(kvg_) * 512;
      kr = raw_rsrc(p.k_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
      vr = raw_rsrc(p.v_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
    } else {
      kr = raw_rsrc(p.k_cache, 0);
      vr = kr;
    }
    const uint32_t lb = lds_addr(base);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pr = wave + 8 * q;  // row pair within the tile
      const uint32_t dst = lb + (half * 16 + pr) * kLdsPitch;
      dma_to_lds(kr, 2 * pr * tok + L.lane * 16, dst);
      dma_to_lds(vr, 2 * pr * tok + L.lane * 16, dst + kLdsTensor);
    }
  };
  // Step s of a segment starting at tile key c0_ with nt_ tiles.
  auto issue_step = [&](int b_, int kvg_, int c0_, int nt_, int s_, char* base) {
    issue_tile(b_, kvg_, uniform(c0_ + 2 * s_ * kTile), 0, true, base);
    issue_tile(b_, kvg_, uniform(c0_ + (2 * s_ + 1) * kTile), 1, 2 * s_ + 1 < nt_, base);
  };
  // The query rides the same DMA ahead of a segment's first two steps: wave w
  // brings columns 8 ((w >> 1) & 1) .. + 7 of kv head w & 1 (the waves of
  // both tiles bring the same bytes to the same place).
  auto issue_q = [&](int b_, int kvg_) {
    const int g_ = kvg_ * 2 + gl;
    const i32x4_t qr =
        raw_rsrc(p.q + int64_t(b_) * p.q_st, int(int64_t(p.num_heads) * p.q_sh * 2));
    const uint32_t lb = lds_addr(qlds);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int col = 8 * hf + 4 * s + (L.lane >> 4);
      const int head = g_ * p.group + min(col, p.hs - 1);
      const int chunk = (L.lane & 15) ^ col;
      dma_to_lds(qr, int(int64_t(head) * p.q_sh * 2) + chunk * 16,
                 lb + (gl * 16 + 8 * hf + 4 * s) * 256);
    }
  };

  u32x4_t k[2][4];
  u32x2_t vh[8];
  // Key j of this wave's tile: stage row kt * 32 + j, pair (row >> 1).
  auto row_addr = [&](const char* tb, int j) {
    const int r = kt * kTile + j;
    return tb + (r >> 1) * kLdsPitch + (r & 1) * 512 + gl * 256;
  };
  auto read_stage = [&](const char* kb) {
    const char* vb = kb + kLdsTensor;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const char* row = row_addr(kb, h * 16 + L.lm) + L.lg * 16;
#pragma unroll
      for (int c = 0; c < 4; ++c) k[h][c] = *reinterpret_cast<const u32x4_t*>(row + c * 64);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vh[i] = *reinterpret_cast<const u32x2_t*>(row_addr(vb, key_of_slot(L.lg, i)) + L.lm * 16 +
                                                hf * 8);
  };
  auto compute = [&](int s) {
    const int tx = 2 * s + kt;
    if (tx >= ntiles) return;  // the step's second tile past the segment
    const int key0 = c0 + tx * kTile;
    if (key0 + kTile <= ctx) {
      attend_tile_half<false>(st, k, vh, Q, key0, ctx, ctx - 1, p.scale_log2, L);
    } else {
      attend_tile_half<true>(st, k, vh, Q, key0, ctx, ctx - 1, p.scale_log2, L);
    }
  };
  auto step = [&](int s, char* stage) {
    if (s + 1 < nsteps) {
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): this wave's loads of step s
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    if (app_lane && s == app_step) {
      char* row = stage + (app_r >> 1) * kLdsPitch + (app_r & 1) * 512 + (L.lane & 31) * 16;
      *reinterpret_cast<u32x4_t*>(row) = app_kn;
      *reinterpret_cast<u32x4_t*>(row + kLdsTensor) = app_vn;
    }
    pf_barrier();
    read_stage(stage);
    pf_barrier();  // every wave holds the stage in registers
    if (s + 2 < nsteps) issue_step(b, kvg, c0, ntiles, s + 2, stage);
    if (has_next && s == nsteps - 1) {
      const int nb = uniform(nx.b);
      const int nkvg = uniform(nx.kvg);
      const int nc0 = uniform(nx.t0) * kTile;
      const int nnt = uniform(nx.t1) - uniform(nx.t0);
      issue_q(nb, nkvg);
      issue_step(nb, nkvg, nc0, nnt, 0, stage0);
      if (nnt > 2) issue_step(nb, nkvg, nc0, nnt, 1, stage1);
    }
    compute(s);
  };
  if (ntiles > 0) {
    if (!pre) {
      issue_q(b, kvg);
      issue_step(b, kvg, c0, ntiles, 0, stage0);
      if (nsteps > 1) issue_step(b, kvg, c0, ntiles, 1, stage1);
    }
    has_next = next(nx);
    if (app_lane) append_load<2>(p, b, kvg, L.lane & 31, app_kn, app_vn);
    if (nsteps > 1) {
      __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16): this wave's query loads
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    }
    pf_barrier();
    {
      const char* row = qlds + (gl * 16 + L.lm) * 256;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        Q.op[0][c] = *reinterpret_cast<const u32x4_t*>(row + (((4 * c + L.lg) ^ L.lm) * 16));
    }
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
      step(s0, stage0);
      if (s0 + 1 < nsteps) step(s0 + 1, stage1);
    }
  }

  if (app_lane) append_store<2>(p, b, kvg, L.lane & 31, app_kn, app_vn);
  // The tile-1 waves hand their state to the tile-0 waves of the same (head,
  // dim half): [pair (gl, hf)][16 O values, m, l][lane].
  float* mb = mlds + (gl * 2 + hf) * 18 * 64 + L.lane;
  if (kt == 1) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) mb[(jj * 4 + r) * 64] = st.o[jj][r];
    mb[16 * 64] = st.m;
    mb[17 * 64] = st.l;
  }
  pf_barrier();
  if (kt == 0) {
    const float mo = mb[16 * 64];
    if (mo != -INFINITY) {
      const float lo = mb[17 * 64];
      if (st.m == -INFINITY) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int r = 0; r < 4; ++r) st.o[jj][r] = mb[(jj * 4 + r) * 64];
        st.l = lo;
        st.m = mo;
      } else {
        const float mn = fmaxf(st.m, mo);
        const float a = __builtin_amdgcn_exp2f(st.m - mn);
        const float c = __builtin_amdgcn_exp2f(mo - mn);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int r = 0; r < 4; ++r) st.o[jj][r] = st.o[jj][r] * a + mb[(jj * 4 + r) * 64] * c;
        st.l = st.l * a + lo * c;
        st.m = mn;
      }
    }
    // Epilogue: lane (lm, lg) holds, for r = 0..3, dims 32lg + 8r + 4hf .. +3
    // of column lm; l is lane-partial over the key slots.
    const float l = rows4_sum(st.l);
    if (L.lm < p.hs) {
      const int head = g * p.group + L.lm;
      const float inv_l = 1.f / l;
      if (split < 0) {
        uint16_t* dst = p.out + int64_t(b) * p.o_st + int64_t(head) * p.o_sh;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d0 = 32 * L.lg + 8 * r + 4 * hf;
          *reinterpret_cast<u32x2_t*>(dst + d0) =
              u32x2_t{pack_bf16x2_fast(st.o[0][r] * inv_l, st.o[1][r] * inv_l),
                      pack_bf16x2_fast(st.o[2][r] * inv_l, st.o[3][r] * inv_l)};
        }
      } else {
        const int64_t base = (int64_t(b) * p.num_heads + head) * p.max_splits + split;
        const float il = l > 0.f ? inv_l : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d0 = 32 * L.lg + 8 * r + 4 * hf;
          *reinterpret_cast<float4*>(p.part_o + base * kD + d0) =
              make_float4(st.o[0][r] * il, st.o[1][r] * il, st.o[2][r] * il, st.o[3][r] * il);
        }
        if (L.lg == 0 && hf == 0) p.part_lse[base] = l > 0.f ? st.m + __log2f(l) : -INFINITY;
      }
    }
  }
  if (!has_next) {
    // nothing in flight for a next segment: drain and realign the waves
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  return has_next;
}

// The query against int8 key codes, as two int8 terms per dim: q ~= scale
// (hi + lo / 254) with |hi|, |lo| <= 127, so q . k = scale (hi . k + lo . k /
// 254) comes out of integer MFMAs with the codes used as stored (the error is
// at most max|q| / 64516 per dim, below bf16's own rounding of q).  Lane
// (lm, lg) holds dims 64 c + 16 lg .. +16 of column lm.
typedef int i32x4v_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
struct QueryI8 {
  i32x4v_t hi[2], lo[2];
  float scale;
};

__device__ __forceinline__ i32x4v_t mfma_i8(const u32x4_t& a, const i32x4v_t& b,
                                            const i32x4v_t& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4v_t, a), b, c, 0, 0, 0);
}

// 16x16 output, 16-deep bf16 product: lane (lm, lg) supplies row / column lm
// and k = 4 lg .. +3 of each operand.
__device__ __forceinline__ f32x4_t mfma_bf16_k16(const u32x2_t& a, const u32x2_t& b,
                                                 const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                   __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
}

// q[32] = dims 64 c + 16 lg + e (c = 0, 1; e < 16) of the lane's column.
__device__ __forceinline__ QueryI8 quantise_query(const float (&q)[32]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(q[i]));
  amax = rows4_max(amax);
  QueryI8 Q;
  Q.scale = amax * (1.f / 127.f);
  const float inv = amax > 0.f ? 127.f / amax : 0.f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t hw = 0u, lw = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = q[16 * c + 4 * w + e] * inv;
        const float h = __builtin_rintf(t);
        const float l = __builtin_rintf((t - h) * 254.f);
        hw |= (uint32_t(int(h)) & 0xffu) << (8 * e);
        lw |= (uint32_t(int(l)) & 0xffu) << (8 * e);
      }
      Q.hi[c][w] = int(hw);
      Q.lo[c][w] = int(lw);
    }
  }
  return Q;
}

// One wave's half of an int8 tile: keys 16 kh + 4 lg + i (i < 4) of the
// lane's S^T column, every dim of the output (o[jj][i] = dim 32 lg + 8 i + jj).
// Scores are kept relative to mu (the running max m, or 0 while m is -inf):
// x' = x - mu comes out of one FMA and feeds exp2 directly.  The rescale test
// is lane-local (x' > thr, thr = kRescaleLog2 once m is finite, -inf
// before), so the column max across the four lane groups is only formed on
// the rare rescale path.
struct KeyHalfState {
  f32x4_t o[8];
  f32x4_t vb;  // every row: the column's sum of the bf16 P operand (the +128 bias of V)
  float m;     // running reference max of x (log2 units), -inf before any key
  float mu;    // m, or 0 while m is -inf
  float thr;   // rescale threshold on x'
  float l;     // lane-partial sum of exp2(x') over the lane's keys
};

__device__ __forceinline__ void init_key_half(KeyHalfState& st) {
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) st.o[jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  st.vb = f32x4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.mu = 0.f;
  st.thr = -INFINITY;
  st.l = 0.f;
}

// exp2 of the shifted scores, the P operand and the PV products of one key
// half (the part after any rescale).
template <bool kMasked>
__device__ __forceinline__ void key_half_pv_i8(KeyHalfState& st, const float (&x)[4],
                                               const bool (&kvalid)[4], const u32x2_t (&vr)[4],
                                               const float (&vsc)[4], u32x2_t& pb) {
  float pr[4], pv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pr[i] = __builtin_amdgcn_exp2f(x[i]);
    pv[i] = kvalid[i] ? pr[i] * vsc[i] : 0.f;
  }
  st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
  pb = u32x2_t{pack_bf16x2_fast(pv[0], pv[1]), pack_bf16x2_fast(pv[2], pv[3])};
  // Column sums of the P operand as rounded, from a ones operand: the
  // +128 bias of V comes off exactly at the end.
  st.vb = mfma_bf16_k16(u32x2_t{0x3f803f80u, 0x3f803f80u}, pb, st.vb);
  // V^T operand of dims 8 lm + jj: byte jj of the lane's 4 key rows, as
  // bf16 of (code + 128).
  u32x2_t vq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vq[i] = vr[i] ^ 0x80808080u;
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int dw = jj >> 2, sh = (jj & 3) * 8;
    const float a0 = float((vq[0][dw] >> sh) & 0xffu), a1 = float((vq[1][dw] >> sh) & 0xffu);
    const float a2 = float((vq[2][dw] >> sh) & 0xffu), a3 = float((vq[3][dw] >> sh) & 0xffu);
    const u32x2_t va = {perm(__float_as_uint(a1), __float_as_uint(a0), kPermHiHi),
                        perm(__float_as_uint(a3), __float_as_uint(a2), kPermHiHi)};
    st.o[jj] = mfma_bf16_k16(va, pb, st.o[jj]);
  }
}

template <bool kMasked>
__device__ __forceinline__ void attend_key_half_i8(KeyHalfState& st, const u32x4_t (&kc)[2],
                                                   const u32x2_t (&vr)[4], const float (&ksc)[4],
                                                   const float (&vsc)[4], const QueryI8& Q,
                                                   int key0, int valid_end, int klim,
                                                   float scale_log2, const LaneId& L) {
  bool kvalid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kvalid[i] = !kMasked || (key0 + 4 * L.lg + i < valid_end);
  i32x4v_t h = {0, 0, 0, 0}, lo = h;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    h = mfma_i8(kc[c], Q.hi[c], h);
    lo = mfma_i8(kc[c], Q.lo[c], lo);
  }
  // q . k = scale (254 hi.k + lo.k) / 254; |hi.k| <= 128 * 128 * 127 < 2^23,
  // so 254 hi.k + lo.k is one exact 24-bit multiply-add.
  const float qs = Q.scale * scale_log2 * (1.f / 254.f);
  float x[4];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = fmaf(float(__mul24(h[i], 254) + lo[i]), qs * ksc[i], -st.mu);
    if constexpr (kMasked) {
      const bool ok = kvalid[i] && (key0 + 4 * L.lg + i <= klim);
      x[i] = ok ? v : -INFINITY;
    } else {
      x[i] = v;
    }
    tmax = fmaxf(tmax, x[i]);
  }
  // The rescale path carries its own copy of the PV part, so the common
  // path's accumulators flow straight into its MFMAs (no merge of two
  // versions of o ahead of them).
  if (__builtin_expect(__ballot(tmax > st.thr) != 0, 0)) {
    const float m_new = fmaxf(st.m, rows4_max(tmax + st.mu));
    const float mu_new = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m - mu_new);
    const float shift = st.mu - mu_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] += shift;
    st.m = m_new;
    st.mu = mu_new;
    st.thr = (m_new == -INFINITY) ? -INFINITY : kRescaleLog2;
    st.l *= alpha;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      st.o[jj][0] *= alpha;
      st.o[jj][1] *= alpha;
      st.o[jj][2] *= alpha;
      st.o[jj][3] *= alpha;
    }
    st.vb[0] *= alpha;
    st.vb[1] *= alpha;
    st.vb[2] *= alpha;
    st.vb[3] *= alpha;
    u32x2_t pb;
    key_half_pv_i8<kMasked>(st, x, kvalid, vr, vsc, pb);
  } else {
    u32x2_t pb;
    key_half_pv_i8<kMasked>(st, x, kvalid, vr, vsc, pb);
  }
}

// Per-channel int8 on the LDS ring: the query q' = q * s_k (the read scales
// folded in, as the register segment does) rides the same int8 hi / lo
// MFMAs.  The side pool's outlier dims come in through two 16-deep bf16
// MFMAs per key half, with the outlier index j as the inner dimension:
//   K side  S[key][col] += sum_j side_k[key][j] q[col][out_idx[j]]
//   V side  O[j][col]   += sum_key side_v[key][j] P[key][col]
// Lane (lm, lg) holds j = 4 lg .. + 3 of each operand.
struct ChanSide {
  u32x2_t qop;     // K side B operand: bf16 q[col lm][out_idx[j]], 0 past the head's count
  u32x2_t kmask;   // K side A operand mask: j past the head's count reads as 0
  f32x4_t sd;      // V side accumulator: j = 4 lg + r of column lm
  int n_out;       // the kv head's outlier count (wave-uniform)
};

// K side A operand: key row r of the staged tile, this wave's head gl,
// values j = 4 lg .. + 3 (side block layout [key][4 heads][kN] bf16).
template <int kN>
__device__ __forceinline__ u32x2_t side_k_operand(const char* side, int r, int gl,
                                                  const LaneId& L) {
  const char* a = side + r * (8 * kN) + gl * (2 * kN) + 8 * L.lg;
  if constexpr (kN == 8) {
    return L.lg < 2 ? *reinterpret_cast<const u32x2_t*>(a) : u32x2_t{0u, 0u};
  } else if constexpr (kN == 4) {
    return L.lg == 0 ? *reinterpret_cast<const u32x2_t*>(a) : u32x2_t{0u, 0u};
  } else {
    static_assert(kN == 2, "LDS side blocks of 2, 4 or 8 values");
    return u32x2_t{L.lg == 0 ? *reinterpret_cast<const uint32_t*>(a) : 0u, 0u};
  }
}

// V side A operand: row j = lm, keys r0 .. r0 + 3 (r0 = the lane's first key
// row), bf16 side_v[key][j]; rows past the head's count and invalid keys 0.
template <int kN, bool kMasked>
__device__ __forceinline__ u32x2_t side_v_operand(const char* side, int r0, int gl, int n_out,
                                                  const bool (&kvalid)[4], const LaneId& L) {
  uint32_t e[4] = {0u, 0u, 0u, 0u};
  if (L.lm < kN && L.lm < n_out) {
    const char* a = side + r0 * (8 * kN) + gl * (2 * kN) + 2 * L.lm;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = *reinterpret_cast<const uint16_t*>(a + i * (8 * kN));
      e[i] = (!kMasked || kvalid[i]) ? v : 0u;
    }
  }
  return u32x2_t{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
}

// One wave's key half of a per-channel tile (attend_key_half_i8 with no
// per-key scales and the side terms).  `side` is the tile's side block (K
// rows, then V rows kSideSlot bytes on).
template <bool kMasked, int kN, int kSideSlot>
__device__ __forceinline__ void attend_key_half_chan(KeyHalfState& st, ChanSide& cs,
                                                     const u32x4_t (&kc)[2],
                                                     const u32x2_t (&vr)[4], const char* side,
                                                     const QueryI8& Q, int key0, int valid_end,
                                                     int klim, float scale_log2, int gl,
                                                     const LaneId& L) {
  bool kvalid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kvalid[i] = !kMasked || (key0 + 4 * L.lg + i < valid_end);
  const int rh = key0 & 31;  // the key half's first row in the tile
  u32x2_t ka = side_k_operand<kN>(side, rh + L.lm, gl, L);
  ka[0] &= cs.kmask[0];
  ka[1] &= cs.kmask[1];
  const u32x2_t va = side_v_operand<kN, kMasked>(side + kSideSlot, rh + 4 * L.lg, gl, cs.n_out,
                                                 kvalid, L);
  i32x4v_t h = {0, 0, 0, 0}, lo = h;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    h = mfma_i8(kc[c], Q.hi[c], h);
    lo = mfma_i8(kc[c], Q.lo[c], lo);
  }
  const f32x4_t sdot = mfma_bf16_k16(ka, cs.qop, f32x4_t{0.f, 0.f, 0.f, 0.f});
  const float qs = Q.scale * scale_log2 * (1.f / 254.f);
  float x[4];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = fmaf(float(__mul24(h[i], 254) + lo[i]), qs, fmaf(sdot[i], scale_log2, -st.mu));
    if constexpr (kMasked) {
      const bool ok = kvalid[i] && (key0 + 4 * L.lg + i <= klim);
      x[i] = ok ? v : -INFINITY;
    } else {
      x[i] = v;
    }
    tmax = fmaxf(tmax, x[i]);
  }
  const float ones[4] = {1.f, 1.f, 1.f, 1.f};
  u32x2_t pb;
  if (__builtin_expect(__ballot(tmax > st.thr) != 0, 0)) {
    const float m_new = fmaxf(st.m, rows4_max(tmax + st.mu));
    const float mu_new = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m - mu_new);
    const float shift = st.mu - mu_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] += shift;
    st.m = m_new;
    st.mu = mu_new;
    st.thr = (m_new == -INFINITY) ? -INFINITY : kRescaleLog2;
    st.l *= alpha;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      st.o[jj][0] *= alpha;
      st.o[jj][1] *= alpha;
      st.o[jj][2] *= alpha;
      st.o[jj][3] *= alpha;
    }
    st.vb[0] *= alpha;
    st.vb[1] *= alpha;
    st.vb[2] *= alpha;
    st.vb[3] *= alpha;
    cs.sd[0] *= alpha;
    cs.sd[1] *= alpha;
    cs.sd[2] *= alpha;
    cs.sd[3] *= alpha;
    key_half_pv_i8<kMasked>(st, x, kvalid, vr, ones, pb);
  } else {
    key_half_pv_i8<kMasked>(st, x, kvalid, vr, ones, pb);
  }
  cs.sd = mfma_bf16_k16(va, pb, cs.sd);
}

// ---------------------------------------------------------------------------
// LDS-staged decode segment, per-token-head int8 pool, a group of 4 kv heads
// (512 B of each token row).  A ring of four stages holds 32-key tiles: K
// codes [32][512] and V codes [32][512], unpadded, the 16-byte chunk c of row
// r stored at chunk c ^ (r & 15) so that the rows a read touches fall on
// different banks; then the tile's K and V scales (16 B per token: the
// group's 4 heads).  Every wave issues exactly five 1 KiB DMA loads per tile
// (two of K, two of V, and the K scales on wave 0, the V scales on wave 1, a
// zero-length load into a dummy block on the others), so one vmcnt count
// covers every wave.  A stage is read into registers as soon as its tile
// lands and refilled four tiles ahead, so up to four tiles are in flight
// under the arithmetic.  Wave w serves kv head w & 3 and keys 16 (w >> 2) ..
// +15 of every tile; the two key halves of a head merge through LDS at the
// end.
// ---------------------------------------------------------------------------
constexpr int kI8Rows = kTile * 512;
constexpr int kI8Stage = 2 * kI8Rows + 2 * 1024;
constexpr int kI8Ring = 4;
// + the dummy block, + the fused append's new K and V rows (1 KiB each)
constexpr int kLdsI8 = kI8Ring * kI8Stage + 1024 + 2048;
constexpr int kI8LoadsPerTile = 5;
constexpr int kI8MergePitch = kD + 4;  // floats per (head, column) row of the merge block
static_assert(4 * 16 * kI8MergePitch * 4 + 4 * 16 * 8 <= kI8Stage, "merge block fits a stage");

// The ring's layout in LDS.  Per-token-head: kI8Ring stages of (K rows, V
// rows, K and V scale blocks), the dummy block, the fused append's rows.
// Per-channel (side width kN = 2, 4 or 8): stages of K and V rows only, a
// ring of side blocks one slot deeper ([K side][V side], kSideSlot bytes
// each: 32 keys x 4 heads x kN bf16, at least the 1 KiB one load writes),
// the dummy block and the group's K read scales (2 KiB); kN = 8 runs three
// stages, so that the ring and the query block fit 160 KiB.
template <int kEnc, int kN>
struct I8LdsLayout {
  static constexpr int kRing = kI8Ring;
  static constexpr int kStage = kI8Stage;
  static constexpr int kSideSlot = 1024;
  static constexpr int kSide = 0;
  static constexpr int kDummy = kI8Ring * kI8Stage;
  static constexpr int kScales = 0;
  static constexpr int kBytes = kLdsI8;
};
template <int kN>
struct I8LdsLayout<kI8Chan, kN> {
  static_assert(kN == 2 || kN == 4 || kN == 8, "LDS side blocks of 2, 4 or 8 values");
  static constexpr int kRing = kN == 8 ? 3 : 4;
  static constexpr int kStage = 2 * kI8Rows;
  static constexpr int kSideSlot = kN * 256 > 1024 ? kN * 256 : 1024;
  static constexpr int kSide = kRing * kStage;
  static constexpr int kDummy = kSide + (kRing + 1) * 2 * kSideSlot;
  static constexpr int kScales = kDummy + 1024;
  static constexpr int kBytes = kScales + 2048;
};
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int kLdsChan = cmax(I8LdsLayout<kI8Chan, 2>::kBytes,
                              cmax(I8LdsLayout<kI8Chan, 4>::kBytes, I8LdsLayout<kI8Chan, 8>::kBytes));
static_assert(4 * 16 * kI8MergePitch * 4 + 4 * 16 * (2 + 16) * 4 <= I8LdsLayout<kI8Chan, 8>::kSide,
              "per-channel merge block fits the stages");

constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// Wait until at most `tiles` tiles' loads of this wave are outstanding (the
// immediate is static, so the count is switched over).
__device__ __forceinline__ void wait_tiles_left(int tiles) {
  switch (tiles) {
    case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kI8LoadsPerTile)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kI8LoadsPerTile)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kI8LoadsPerTile)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * kI8LoadsPerTile)); break;
  }
}

// The fused int8 append of a row with no context (its NaN-row owner): one
// lane quantises and stores the group's 4 heads of the new K and V rows with
// the arithmetic of quant_tokhead_row (amax over the 128 dims, scale
// max(amax, 1e-6) / 127, codes rint(x / scale) clamped to +-127).
__device__ void append_i8_row_lane(const AttnParams& p, int b, int kvg) {
  const int64_t raw = p.app_slot_bytes == 8 ? load_index<8>(p.app_slots, b)
                                            : load_index<4>(p.app_slots, b);
  const int64_t slot = wrap_slot(raw, p.app_num_slots);
  if (slot < 0 || slot >= p.app_num_slots) return;
  for (int side = 0; side < 2; ++side) {
    for (int hh = 0; hh < 4; ++hh) {
      const int head = kvg * 4 + hh;
      const uint16_t* src = side == 0 ? p.app_k + int64_t(b) * p.app_k_st + head * p.app_k_sh
                                      : p.app_v + int64_t(b) * p.app_v_st + head * p.app_v_sh;
      float amax = 0.f;
      for (int d = 0; d < kD; ++d) amax = fmaxf(amax, fabsf(bf16_bits_to_f32(src[d])));
      const float s = fmaxf(amax, 1e-6f) / 127.0f;
      int8_t* dst = const_cast<int8_t*>(reinterpret_cast<const int8_t*>(
                        side == 0 ? p.k_cache : p.v_cache)) +
                    slot * p.tok_bytes + head * kD;
      for (int d = 0; d < kD; ++d) {
        const float q = fminf(fmaxf(__builtin_rintf(bf16_bits_to_f32(src[d]) / s), -127.0f),
                              127.0f);
        dst[d] = int8_t(int(q));
      }
      const_cast<float*>(side == 0 ? p.k_scale : p.v_scale)[slot * p.kvh + head] = s;
    }
  }
}

template <int kEnc, int kN>
__device__ void decode_segment_lds_i8(const AttnParams& p, char* ring, char* qlds,
                                      const int32_t* bt, int b, int kvg, int ctx, int t0, int t1,
                                      int split) {
  constexpr bool kChan = kEnc == kI8Chan;
  using Lay = I8LdsLayout<kEnc, kN>;
  constexpr int kRingN = Lay::kRing;
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));
  const int gl = wave & 3;   // kv head within the group
  const int kh = wave >> 2;  // key half of every tile
  const int g = kvg * 4 + gl;
  b = uniform(b);
  ctx = uniform(ctx);
  t0 = uniform(t0);
  t1 = uniform(t1);
  const int ntiles = t1 > t0 ? t1 - t0 : 0;
  const int c0 = t0 * kTile;
  // Fused append (per-token-head quantise-on-append): the segment holding
  // the row's last tile quantises the new token's K and V rows of the group's
  // 4 heads exactly as store_int8_tokhead_kernel does and stores codes and
  // scales to the pool.  The rows come into LDS by DMA ahead of the query
  // (waves 0 and 1), so they have landed with it and the quantiser runs
  // under the first tiles' loads.  The last tile's stage is patched before
  // any wave reads it: the wave whose DMA brought the token's code rows
  // (pair app_r >> 1) overwrites them, wave 0 the token's K scales, wave 1
  // its V scales, each after its own wait for that tile and before the
  // barrier.  (The pool store may land before or after that tile's DMA
  // reads the slot: the bytes are the same.)
  const bool app = p.app_k != nullptr && ntiles > 0 && t1 == (ctx + kTile - 1) / kTile;
  const int app_r = (ctx - 1) & (kTile - 1);
  const bool app_codes = app && wave == ((app_r >> 1) & 7);
  const bool app_ks = app && wave == 0;
  const bool app_vs = app && wave == 1;
  const bool app_any = app_codes || app_ks || app_vs;
  char* const app_rows = ring + Lay::kDummy + 1024;  // [K row 1 KiB][V row 1 KiB]
  u32x2_t app_kc{0u, 0u}, app_vc{0u, 0u};
  float app_ksc = 0.f, app_vsc = 0.f;

  QueryI8 Q;
  KeyHalfState st;
  init_key_half(st);
  ChanSide cs;
  if constexpr (kChan) {
    cs.sd = f32x4_t{0.f, 0.f, 0.f, 0.f};
    cs.n_out = p.head_n_out != nullptr ? min(table_entry(p.head_n_out, g), kN) : 0;
  }

  const int tok = int(p.tok_bytes);
  const int64_t grp_off = int64_t(kvg) * 512;
  const int sc_tok = p.kvh * 4;  // bytes of scales per token
  const uint32_t dummy = lds_addr(ring + Lay::kDummy);
  auto stage_of = [&](int j) { return ring + (unsigned(j) % kRingN) * Lay::kStage; };
  // (per-channel) the side block of tile j, one ring slot deeper than the
  // stages: it is read while its tile is computed, after the stage itself
  // has been handed to the DMA of a later tile.
  auto side_of = [&](int j) {
    return ring + Lay::kSide + (unsigned(j) % (kRingN + 1)) * (2 * Lay::kSideSlot);
  };
  // Wave w brings rows 2n, 2n + 1 (n = w, w + 8) of K and of V, then one
  // scale block (per-token-head), one 1 KiB piece of the side rows
  // (per-channel) or the dummy load.
  auto issue = [&](int tix) {
    char* base = stage_of(tix);
    const int key0 = uniform(c0 + tix * kTile);
    const int blk = table_entry(bt, key0 / p.page);
    const int64_t slot0 = int64_t(blk) * p.page + (key0 % p.page);
    const i32x4_t kr = raw_rsrc(p.k_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
    const i32x4_t vr = raw_rsrc(p.v_cache + slot0 * p.tok_bytes + grp_off, kTile * tok);
    const uint32_t lb = lds_addr(base);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int n = wave + 8 * m;
      const int row = 2 * n + (L.lane >> 5);
      const int chunk = (L.lane & 31) ^ (row & 15);
      const int voff = row * tok + chunk * 16;
      dma_to_lds(kr, voff, lb + n * 1024);
      dma_to_lds(vr, voff, lb + kI8Rows + n * 1024);
    }
    if constexpr (kChan) {
      // Side rows of the tile's 32 keys for the group's 4 heads: 8 kN bytes
      // per key at a stride of kvh * kN * 2 bytes, kN / 2 lanes of 16 bytes
      // each per key; kN = 8 takes two 1 KiB pieces per side (waves 0-3),
      // smaller widths one (waves 0 and 1; lanes past the 32 keys read 0).
      constexpr int kPieces = kN == 8 ? 2 : 1;
      constexpr int kLanesPerKey = kN / 2;
      if (wave < 2 * kPieces) {
        const int sidew = wave / kPieces;  // 0: K, 1: V
        const int piece = wave - sidew * kPieces;
        // (the rows of all 4 heads: whether this wave's own head has
        // outliers does not matter)
        const bool has = p.head_n_out != nullptr;
        // (the pool is picked arithmetically: a select between the two
        // parameter fields compiles to an indexed read of a private copy)
        const uint64_t kb = reinterpret_cast<uint64_t>(p.side_k);
        const uint64_t side_base = kb + (reinterpret_cast<uint64_t>(p.side_v) - kb) * uint64_t(sidew);
        const uint16_t* sp = !has ? reinterpret_cast<const uint16_t*>(p.k_scale)
                                  : reinterpret_cast<const uint16_t*>(side_base) +
                                        (slot0 * p.kvh + kvg * 4) * kN;
        const int stride = p.kvh * kN * 2;
        const int nrec = has ? (kTile - 1) * stride + 8 * kN : 0;
        const int key = piece * (64 / kLanesPerKey) + L.lane / kLanesPerKey;
        const int soff = key < kTile ? key * stride + (L.lane % kLanesPerKey) * 16 : 0x40000000;
        dma_to_lds(raw_rsrc(sp, nrec), soff,
                   lds_addr(side_of(tix)) + sidew * Lay::kSideSlot + piece * 1024);
      } else {
        dma_to_lds(raw_rsrc(p.k_scale, 0), 0, dummy);
      }
    } else if (wave < 2) {
      const float* sp = (wave == 0 ? p.k_scale : p.v_scale) + slot0 * p.kvh;
      const i32x4_t sr = raw_rsrc(sp, kTile * sc_tok);
      const int soff = L.lane < kTile ? L.lane * sc_tok + kvg * 16 : 0x40000000;
      dma_to_lds(sr, soff, lb + 2 * kI8Rows + wave * 1024);
    } else {
      dma_to_lds(raw_rsrc(p.k_scale, 0), 0, dummy);
    }
  };
  // The query rides the same DMA ahead of the first tiles: wave w brings
  // columns 8 (w >> 2) .. + 7 of kv head w & 3 (columns past the head count
  // repeat the last head; their results are never stored), 16-byte chunk c
  // of column col at chunk c ^ col.
  auto issue_q = [&]() {
    const i32x4_t qr =
        raw_rsrc(p.q + int64_t(b) * p.q_st, int(int64_t(p.num_heads) * p.q_sh * 2));
    const uint32_t lb = lds_addr(qlds);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int col = 8 * kh + 4 * s + (L.lane >> 4);
      const int head = g * p.group + min(col, p.hs - 1);
      const int chunk = (L.lane & 15) ^ col;
      dma_to_lds(qr, int(int64_t(head) * p.q_sh * 2) + chunk * 16,
                 lb + (gl * 16 + 8 * kh + 4 * s) * 256);
    }
    if constexpr (kChan) {
      // The group's read scales s_k [4 heads][128] fp32 (2 KiB): waves 0
      // and 1 bring one half each, the others a dummy load, so every wave
      // issues three loads here.
      if (wave < 2) {
        dma_to_lds(raw_rsrc(p.k_scale + (kvg * 4 + 2 * wave) * kD, 1024), L.lane * 16,
                   lds_addr(ring + Lay::kScales) + wave * 1024);
      } else {
        dma_to_lds(raw_rsrc(p.k_scale, 0), 0, dummy);
      }
    }
  };

  // Quantise the new rows (from LDS, after the barrier that follows their
  // DMA) and store them to the pool; the codes and scales stay in registers
  // for the patch.
  auto quantise_append = [&]() {
    if (!app_any) return;
    float kx[8], vx[8];
    unpack8(*reinterpret_cast<const u32x4_t*>(app_rows + L.lane * 16), kx);
    unpack8(*reinterpret_cast<const u32x4_t*>(app_rows + 1024 + L.lane * 16), vx);
    int kc[8], vc[8];
    app_ksc = quant_tokhead_row(kx, kc);
    app_vsc = quant_tokhead_row(vx, vc);
    app_kc = u32x2_t{pack_codes4(kc, 0), pack_codes4(kc, 4)};
    app_vc = u32x2_t{pack_codes4(vc, 0), pack_codes4(vc, 4)};
    if (app_codes) {
      // the pool, at row b's slot (store_kvcache's rules for the slot)
      const int64_t raw = p.app_slot_bytes == 8 ? load_index<8>(p.app_slots, b)
                                                : load_index<4>(p.app_slots, b);
      const int64_t slot = wrap_slot(raw, p.app_num_slots);
      if (slot >= 0 && slot < p.app_num_slots) {
        const int h = L.lane >> 4;
        const int64_t dst = slot * p.tok_bytes + grp_off + h * kD + (L.lane & 15) * 8;
        *reinterpret_cast<u32x2_t*>(const_cast<char*>(p.k_cache) + dst) = app_kc;
        *reinterpret_cast<u32x2_t*>(const_cast<char*>(p.v_cache) + dst) = app_vc;
        if ((L.lane & 15) == 0) {
          const_cast<float*>(p.k_scale)[slot * p.kvh + kvg * 4 + h] = app_ksc;
          const_cast<float*>(p.v_scale)[slot * p.kvh + kvg * 4 + h] = app_vsc;
        }
      }
    }
  };
  // The patch of the last tile's stage (after this wave's wait for it).
  auto patch_append = [&]() {
    if (!app_any) return;
    char* base = stage_of(ntiles - 1);
    const int h = L.lane >> 4;
    if (app_codes) {
      // lane l holds dims 8 (l & 15) .. + 7 of head l >> 4: half (l & 1) of
      // 16-byte chunk 8 h + (l & 15) / 2, stored at chunk ^ (row & 15)
      const int chunk = (8 * h + ((L.lane & 15) >> 1)) ^ (app_r & 15);
      const int off = app_r * 512 + chunk * 16 + 8 * (L.lane & 1);
      *reinterpret_cast<u32x2_t*>(base + off) = app_kc;
      *reinterpret_cast<u32x2_t*>(base + kI8Rows + off) = app_vc;
    }
    if ((L.lane & 15) == 0) {
      char* sb = base + 2 * kI8Rows + app_r * 16 + h * 4;
      if (app_ks) *reinterpret_cast<float*>(sb) = app_ksc;
      if (app_vs) *reinterpret_cast<float*>(sb + 1024) = app_vsc;
    }
  };

  // One tile's operands of this wave, read from its stage.
  struct Regs {
    u32x4_t kc[2];
    u32x2_t vr[4];
    float ksc[4], vsc[4];
  };
  auto read_stage = [&](const char* base, Regs& r) {
    const int krow = 16 * kh + L.lm;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int chunk = (8 * gl + 4 * c + L.lg) ^ (krow & 15);
      r.kc[c] = *reinterpret_cast<const u32x4_t*>(base + krow * 512 + chunk * 16);
    }
    const char* vb = base + kI8Rows;
    const char* sb = base + 2 * kI8Rows;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * kh + 4 * L.lg + i;
      const int chunk = (8 * gl + (L.lm >> 1)) ^ (row & 15);
      r.vr[i] = *reinterpret_cast<const u32x2_t*>(vb + row * 512 + chunk * 16 + 8 * (L.lm & 1));
      if constexpr (!kChan) {
        r.ksc[i] = *reinterpret_cast<const float*>(sb + row * 16 + gl * 4);
        r.vsc[i] = *reinterpret_cast<const float*>(sb + 1024 + row * 16 + gl * 4);
      }
    }
  };
  auto compute = [&](int j, const Regs& r) {
    const int key0 = c0 + j * kTile;
    const int hkey0 = key0 + 16 * kh;
    if constexpr (kChan) {
      if (key0 + kTile <= ctx) {
        attend_key_half_chan<false, kN, Lay::kSideSlot>(st, cs, r.kc, r.vr, side_of(j), Q, hkey0,
                                                        ctx, ctx - 1, p.scale_log2, gl, L);
      } else {
        attend_key_half_chan<true, kN, Lay::kSideSlot>(st, cs, r.kc, r.vr, side_of(j), Q, hkey0,
                                                       ctx, ctx - 1, p.scale_log2, gl, L);
      }
    } else if (key0 + kTile <= ctx) {
      attend_key_half_i8<false>(st, r.kc, r.vr, r.ksc, r.vsc, Q, hkey0, ctx, ctx - 1,
                                p.scale_log2, L);
    } else {
      attend_key_half_i8<true>(st, r.kc, r.vr, r.ksc, r.vsc, Q, hkey0, ctx, ctx - 1,
                               p.scale_log2, L);
    }
  };
  // Step j: tile j is in registers `cur`; once tile j + 1 has landed (one
  // barrier, which also retires every wave's reads of stage j), stage j is
  // refilled with tile j + 4, tile j + 1 is read into `nxt`, and tile j is
  // computed while those reads are in flight.
  auto step = [&](int j, const Regs& cur, Regs& nxt) {
    if (j + 1 < ntiles) wait_tiles_left(min(ntiles - 2 - j, kRingN - 2));
    if (j + 2 == ntiles) patch_append();  // the last tile has landed (vmcnt(0) above)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): `cur` has arrived
    __syncthreads();
    if (j + kRingN < ntiles) issue(j + kRingN);
    if (j + 1 < ntiles) read_stage(stage_of(j + 1), nxt);
    compute(j, cur);
  };

  if (ntiles > 0) {
    if (app && wave < 2) {
      // The new K (wave 0) or V (wave 1) row of the group's 4 heads: lane l
      // brings dims 8 (l & 15) .. + 7 of head l >> 4.  Issued first, so the
      // query wait below covers it.
      const uint16_t* src = wave == 0 ? p.app_k + int64_t(b) * p.app_k_st + kvg * 4 * p.app_k_sh
                                      : p.app_v + int64_t(b) * p.app_v_st + kvg * 4 * p.app_v_sh;
      const int64_t sh = wave == 0 ? p.app_k_sh : p.app_v_sh;
      const i32x4_t ar = raw_rsrc(src, int((3 * sh + kD) * 2));
      dma_to_lds(ar, int(((L.lane >> 4) * sh + (L.lane & 15) * 8) * 2),
                 lds_addr(app_rows + wave * 1024));
    }
    issue_q();
    const int first = min(ntiles, kRingN);
    for (int j = 0; j < first; ++j) issue(j);
    wait_tiles_left(first);  // the query loads (and the new rows), issued first, have landed
    __syncthreads();
    if constexpr (!kChan) quantise_append();
    {
      const char* row = qlds + (gl * 16 + L.lm) * 256;
      float qf[32];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const u32x4_t w =
              *reinterpret_cast<const u32x4_t*>(row + (((8 * c + 2 * L.lg + e) ^ L.lm) * 16));
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            qf[16 * c + 8 * e + 2 * k] = bf16_bits_to_f32(w[k] & 0xffffu);
            qf[16 * c + 8 * e + 2 * k + 1] = bf16_bits_to_f32(w[k] >> 16);
          }
        }
      }
      if constexpr (kChan) {
        // q' = q * s_k: dims 64 c + 16 lg + 8 e + m of the lane's column.
        const float* sc = reinterpret_cast<const float*>(ring + Lay::kScales) + gl * kD;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float* s8 = sc + 64 * c + 16 * L.lg + 8 * e;
            const float4 s0 = *reinterpret_cast<const float4*>(s8);
            const float4 s1 = *reinterpret_cast<const float4*>(s8 + 4);
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int m = 0; m < 8; ++m) qf[16 * c + 8 * e + m] *= sv[m];
          }
        }
        // The K side's B operand: the column's query at the head's outlier
        // dims j = 4 lg .. + 3 (unscaled: the side pool holds the keys' own
        // values there), and the mask of the j below the head's count.
        uint32_t qv[4] = {0u, 0u, 0u, 0u}, km[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < kN; ++j) {
          if (j < cs.n_out) {
            const int d = table_entry(p.out_idx, int64_t(g) * p.n_out_max + j);
            const uint32_t v =
                *reinterpret_cast<const uint16_t*>(row + (((d >> 3) ^ L.lm) * 16) + (d & 7) * 2);
            if ((j >> 2) == L.lg) {
              qv[j & 3] = v;
              km[j & 3] = 0xffffu;
            }
          }
        }
        cs.qop = u32x2_t{qv[0] | (qv[1] << 16), qv[2] | (qv[3] << 16)};
        cs.kmask = u32x2_t{km[0] | (km[1] << 16), km[2] | (km[3] << 16)};
      }
      Q = quantise_query(qf);
    }
    Regs ra, rb;
    // Tile 0 lands (tiles 1 .. min(3, ntiles - 1) may still be in flight).
    wait_tiles_left(min(ntiles - 1, kRingN - 1));
    if (ntiles == 1) patch_append();  // vmcnt(0) above
    __syncthreads();
    read_stage(stage_of(0), ra);
    for (int j = 0; j < ntiles; j += 2) {
      step(j, ra, rb);
      if (j + 1 < ntiles) step(j + 1, rb, ra);
    }
  }

  // Epilogue: each wave's o has the +128 V bias removed, then the key-half-1
  // waves hand (o, m, l) to the key-half-0 waves through the first stage,
  // which write the merged rows.  Lane (lm, lg) holds dims 32 lg + 8 i + jj.
  const float l = rows4_sum(st.l);
  const float bias = 128.f * st.vb[0];
  float* mo = reinterpret_cast<float*>(ring);
  float* mml = mo + 4 * 16 * kI8MergePitch;
  // per-channel: both key halves' side sums, [kh][head][column][8]
  float* msd = mml + 4 * 16 * 2;
  float* orow = mo + (gl * 16 + L.lm) * kI8MergePitch + 32 * L.lg;
  __syncthreads();
  if constexpr (kChan) {
    if (4 * L.lg < kN) {
      float* d = msd + ((kh * 4 + gl) * 16 + L.lm) * 8 + 4 * L.lg;
      *reinterpret_cast<float4*>(d) = make_float4(cs.sd[0], cs.sd[1], cs.sd[2], cs.sd[3]);
    }
  }
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      reinterpret_cast<float4*>(orow + 8 * i)[0] =
          make_float4(st.o[0][i] - bias, st.o[1][i] - bias, st.o[2][i] - bias, st.o[3][i] - bias);
      reinterpret_cast<float4*>(orow + 8 * i)[1] =
          make_float4(st.o[4][i] - bias, st.o[5][i] - bias, st.o[6][i] - bias, st.o[7][i] - bias);
    }
    if (L.lg == 0) {
      mml[(gl * 16 + L.lm) * 2] = st.m;
      mml[(gl * 16 + L.lm) * 2 + 1] = l;
    }
  }
  __syncthreads();
  if (kh == 0 && L.lm < p.hs) {
    const float m1 = mml[(gl * 16 + L.lm) * 2], l1 = mml[(gl * 16 + L.lm) * 2 + 1];
    const float mm = fmaxf(st.m, m1);
    const float mref = mm == -INFINITY ? 0.f : mm;
    const float a0 = __builtin_amdgcn_exp2f(st.m - mref), a1 = __builtin_amdgcn_exp2f(m1 - mref);
    const float lt = a0 * l + a1 * l1;
    const int head = g * p.group + L.lm;
    float v[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 u0 = reinterpret_cast<const float4*>(orow + 8 * i)[0];
      const float4 u1 = reinterpret_cast<const float4*>(orow + 8 * i)[1];
      const float o1[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) v[i][jj] = a0 * (st.o[jj][i] - bias) + a1 * o1[jj];
    }
    if constexpr (kChan) {
      // V's read scales (0 at the outlier dims), then the side pool's exact
      // values in the outlier dims' place.
      const float* vs = p.v_scale + int64_t(g) * kD + 32 * L.lg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 s0 = reinterpret_cast<const float4*>(vs + 8 * i)[0];
        const float4 s1 = reinterpret_cast<const float4*>(vs + 8 * i)[1];
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) v[i][jj] *= sv[jj];
      }
#pragma unroll
      for (int j = 0; j < kN; ++j) {
        if (j < cs.n_out) {
          const float sdt = a0 * msd[(gl * 16 + L.lm) * 8 + j] +
                            a1 * msd[((4 + gl) * 16 + L.lm) * 8 + j];
          const int d = table_entry(p.out_idx, int64_t(g) * p.n_out_max + j);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
              if (32 * L.lg + 8 * i + jj == d) v[i][jj] = sdt;
          }
        }
      }
    }
    if (split < 0) {
      const float inv = 1.f / lt;
      uint16_t* dst = p.out + int64_t(b) * p.o_st + int64_t(head) * p.o_sh + 32 * L.lg;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x4_t*>(dst + 8 * i) =
            u32x4_t{pack_bf16x2_fast(v[i][0] * inv, v[i][1] * inv),
                    pack_bf16x2_fast(v[i][2] * inv, v[i][3] * inv),
                    pack_bf16x2_fast(v[i][4] * inv, v[i][5] * inv),
                    pack_bf16x2_fast(v[i][6] * inv, v[i][7] * inv)};
    } else {
      const int64_t base = (int64_t(b) * p.num_heads + head) * p.max_splits + split;
      const float il = lt > 0.f ? 1.f / lt : 0.f;
      float* dst = p.part_o + base * kD + 32 * L.lg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        reinterpret_cast<float4*>(dst + 8 * i)[0] =
            make_float4(v[i][0] * il, v[i][1] * il, v[i][2] * il, v[i][3] * il);
        reinterpret_cast<float4*>(dst + 8 * i)[1] =
            make_float4(v[i][4] * il, v[i][5] * il, v[i][6] * il, v[i][7] * il);
      }
      if (L.lg == 0) p.part_lse[base] = lt > 0.f ? mref + __log2f(lt) : -INFINITY;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Fixed-chunk decode unit (the mixed varlen launch): chunk `chunk` of row b,
// p.chunk_tokens keys per chunk.
// bt_base is the launch's block-table argument (declared __restrict__ by the
// kernel, so its reads stay scalar loads).
template <int kEnc>
__device__ void decode_unit(const AttnParams& p, char* smem, const int32_t* bt_base, int b,
                            int kvg, int chunk) {
  const int ctx = p.ctx_lens[b];
  const int nch = ctx > 0 ? (ctx + p.chunk_tokens - 1) / p.chunk_tokens : 1;
  if (chunk >= nch) return;  // uniform over the workgroup
  const int chunk_tiles = p.chunk_tokens / kTile;
  const int ntiles = (ctx + kTile - 1) / kTile;
  const int t0 = chunk * chunk_tiles;
  decode_segment<kEnc>(p, smem, bt_base + int64_t(b) * p.bt_stride, b, kvg, ctx, t0,
                       min(t0 + chunk_tiles, ntiles), nch == 1 ? -1 : chunk);
}

// ---------------------------------------------------------------------------
// Prefill epilogue of column block cb (bf16 and per-token-head int8 keys):
// lane (lm, lg) holds dims 32 lg + 8 r + jj (r < 4, jj < 8) of column lm,
// four runs of 8 contiguous dims stored straight from registers, either as
// the final bf16 row (split < 0) or as split-K partial `split`.  `ok` is the
// lane's column validity; every lane must call (the sum is a wave reduction).
// ---------------------------------------------------------------------------
template <int kEnc, int NCB>
__device__ __forceinline__ void store_prefill_block(const AttnParams& p, const ColState<NCB>& st,
                                                    int cb, int64_t row, int head, bool ok,
                                                    int split, const LaneId& L) {
  float l = st.l[cb];
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  float bias = 0.f;
  if constexpr (kEnc != kBF16) {
    float vb = st.vb[cb];
    vb += shfl_xor(vb, 16);
    vb += shfl_xor(vb, 32);
    bias = 128.f * vb;
  }
  if (!ok) return;
  if (split < 0) {
    const float inv = 1.f / l;
    uint16_t* dst = p.out + row * p.o_st + int64_t(head) * p.o_sh + 32 * L.lg;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) v[jj] = (st.o[cb][jj][r] - bias) * inv;
      *reinterpret_cast<u32x4_t*>(dst + 8 * r) =
          u32x4_t{pack_bf16x2_fast(v[0], v[1]), pack_bf16x2_fast(v[2], v[3]),
                  pack_bf16x2_fast(v[4], v[5]), pack_bf16x2_fast(v[6], v[7])};
    }
  } else {
    const int64_t base = (row * p.num_heads + head) * p.max_splits + split;
    const float il = l > 0.f ? 1.f / l : 0.f;
    float* dst = p.part_o + base * kD + 32 * L.lg;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) v[jj] = (st.o[cb][jj][r] - bias) * il;
      reinterpret_cast<float4*>(dst + 8 * r)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(dst + 8 * r)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (L.lg == 0) p.part_lse[base] = l > 0.f ? st.m[cb] + __log2f(l) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Prefill segment: key tiles [t0, t1) of item (chunk i, query tile qt, kv
// slice kvs); the tiles stop at the last key any query of the tile sees.  The
// workgroup covers kWaves waves x kPreNCB column blocks; K/V tiles go through
// LDS.  split < 0: the segment is the whole item and writes final rows;
// otherwise it writes split-K partials at slot `split`.
// ---------------------------------------------------------------------------
template <int kEnc, bool kFresh, bool kPLo = (kEnc == kI8Chan)>
__device__ void prefill_segment(const AttnParams& p, char* smem, const int32_t* bt_base, int i,
                                int qt, int kvs, int t0, int t1, int split) {
  // An int8 pool's tiles are dequantised to bf16 as they are committed to
  // LDS (the reference's prefill reads the pool through dequant_gathered,
  // nanovllm/kernels/kv_int8.py:96-107, then attends in bf16), so the
  // attention itself is the bf16 path (kCmp) whatever the pool encoding.
  constexpr int kCmp = kBF16;
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));  // wave-uniform (scalar) index
  const int g = kvs / p.nslices;
  const int s = kvs - g * p.nslices;
  const int hs = min(p.hs, p.group - s * p.hs);
  const int cq0 = p.cu_q[i];
  const int sq = p.cu_q[i + 1] - cq0;
  const int ck0 = p.cu_k[i];
  const int sk = p.cu_k[i + 1] - ck0;
  const int prefix = sk - sq;
  const int qtile_tokens = kWaves * kPreNCB * p.tpb;
  const int q0 = qt * qtile_tokens;

  ColInfo ci[kPreNCB];
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
    const int tq = q0 + (wave * kPreNCB + cb) * p.tpb + L.lm / p.hs;
    const int hh = L.lm % p.hs;
    const bool ok = (L.lm < p.tpb * p.hs) && hh < hs && tq < sq;
    ci[cb].row = int64_t(p.n_dec) + cq0 + (ok ? tq : 0);
    ci[cb].head = g * p.group + s * p.hs + hh;
    ci[cb].valid = ok;
    ci[cb].klim = ok ? prefix + tq : -1;
  }
  QOps<kCmp, kPreNCB> Q;
  build_q<kCmp, kPreNCB>(Q, p, ci, g, L);
  ColState<kPreNCB> st;
  init_state(st);
  // Smallest key limit over the wave's valid columns: tiles entirely below it
  // need no causal mask.
  int min_klim = 0x7fffffff;
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb)
    if (ci[cb].valid) min_klim = min(min_klim, ci[cb].klim);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) min_klim = min(min_klim, __shfl_xor(min_klim, m, 64));

  // Key range of the segment, cut at the last key any column of the tile sees.
  const int last_q = min(q0 + qtile_tokens, sq) - 1;
  const int k_begin = uniform(t0 * kTile);
  const int k_end = uniform(min(t1 * kTile, min(sk, prefix + last_q + 1)));
  const int ntiles = k_end > k_begin ? (k_end - k_begin + kTile - 1) / kTile : 0;

  const int32_t* bt = kFresh ? nullptr : bt_base + int64_t(p.n_dec + i) * p.bt_stride;
  constexpr int kPitch = kPitchBF16;  // the stage holds bf16 rows
  constexpr int kRowBytes = (kEnc == kBF16) ? kD * 2 : kD;  // a pool row
  constexpr int kVecPerRow = kRowBytes / 16;
  static_assert(kEnc != kI8Chan || kVecPerRow >= kSideMax, "a key's chunk lanes hold its side row");
  constexpr int kVecPerTile = kTile * kVecPerRow;  // per tensor
  constexpr int kLoadsPerThread = (2 * kVecPerTile + kThreads - 1) / kThreads;
  const int64_t head_off = int64_t(g) * kRowBytes;

  auto stage_ptr = [&](int buf) { return smem + buf * kPrefillStage; };
  auto tile_slot0 = [&](int tix) -> int64_t {
    const int key0 = k_begin + tix * kTile;
    if constexpr (kFresh) {
      return int64_t(ck0) + key0;
    } else {
      const int blk = uniform(bt[key0 / p.page]);
      return int64_t(blk) * p.page + (key0 % p.page);
    }
  };
  // Cooperative global -> register fetch of one tile (16 B per element) into
  // register set `set`; two sets keep two tiles in flight.
  u32x4_t pre[2][kLoadsPerThread];
  // int8 pools: the element's dequantisation scale (per-token-head) or one
  // side value of its key (per-channel)
  float pre_sc[2][kLoadsPerThread];
  uint32_t pre_sd[2][kLoadsPerThread];
  // live = false (int8 pools): issue the loads all the same, out of range
  // (no traffic, 0), so that every iteration has the same loads in flight
  // and the commit's waits count only the loads it needs.
  auto fetch = [&](int set, int64_t slot0, int key0, bool live) {
#pragma unroll
    for (int e = 0; e < kLoadsPerThread; ++e) {
      const int idx = e * kThreads + threadIdx.x;
      pre[set][e] = u32x4_t{0u, 0u, 0u, 0u};
      if constexpr (kEnc == kI8Tok) pre_sc[set][e] = 0.f;
      if constexpr (kEnc != kBF16) {
        // int8 pools: one buffer load and no branch (a key past the chunk
        // reads 0).  Under a branch the code unpacking of the commit would
        // be folded into the branch, and the load's wait with it.
        const int tensor = idx / kVecPerTile;  // wave-uniform
        const int rem = idx - tensor * kVecPerTile;
        const int key = rem / kVecPerRow;
        const int vec = rem - key * kVecPerRow;
        const uintptr_t kc = reinterpret_cast<uintptr_t>(p.k_cache);
        const uintptr_t vc = reinterpret_cast<uintptr_t>(p.v_cache);
        const char* base = reinterpret_cast<const char*>(kc + (vc - kc) * uintptr_t(tensor != 0)) +
                           slot0 * p.tok_bytes + head_off;
        const __amdgpu_buffer_rsrc_t rs = wave_rsrc(base, int((kTile - 1) * p.tok_bytes) + kRowBytes);
        const bool ok = live && idx < 2 * kVecPerTile && key0 + key < sk;
        pre[set][e] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         rs, ok ? int(key * p.tok_bytes) + vec * 16 : 0x40000000, 0, 0));
        if constexpr (kEnc == kI8Tok) {
          const uintptr_t ksc = reinterpret_cast<uintptr_t>(p.k_scale);
          const uintptr_t vsc = reinterpret_cast<uintptr_t>(p.v_scale);
          const float* sbase = reinterpret_cast<const float*>(ksc + (vsc - ksc) * uintptr_t(tensor != 0)) +
                               slot0 * p.kvh + g;
          const __amdgpu_buffer_rsrc_t ss = wave_rsrc(sbase, ((kTile - 1) * p.kvh + 1) * 4);
          pre_sc[set][e] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(ss, ok ? key * p.kvh * 4 : 0x40000000, 0, 0));
        }
      } else if (idx < 2 * kVecPerTile) {
        const int tensor = idx / kVecPerTile;
        const int rem = idx - tensor * kVecPerTile;
        const int key = rem / kVecPerRow;
        const int vec = rem - key * kVecPerRow;
        if (key0 + key < sk) {
          if constexpr (kFresh) {
            const uint16_t* src = tensor == 0 ? p.kf + (slot0 + key) * p.kf_st + int64_t(g) * p.kf_sh
                                              : p.vf + (slot0 + key) * p.vf_st + int64_t(g) * p.vf_sh;
            pre[set][e] = reinterpret_cast<const u32x4_t*>(src)[vec];
          } else {
            const char* src = (tensor == 0 ? p.k_cache : p.v_cache) + (slot0 + key) * p.tok_bytes +
                              head_off;
            pre[set][e] = reinterpret_cast<const u32x4_t*>(src)[vec];
          }
        }
      }
      if constexpr (kEnc == kI8Chan) {
        // The dword holding one side value of the element's key (K rows for
        // tensor 0, V rows for tensor 1, the tensor being wave-uniform): the
        // lane of chunk v holds slot v's, so the 8 lanes of a key hold its
        // row (n_out_max <= 8 slots).  Whole aligned dwords (a 16-bit load
        // result would be widened by a copy that waits for it); slots past
        // n_out_max and keys past the chunk read 0 (no traffic).
        const int tensor = idx / kVecPerTile;
        const int key = (idx - tensor * kVecPerTile) / kVecPerRow;
        const int slot = idx & (kVecPerRow - 1);
        const int nom = p.n_out_max;
        const bool has = live && p.head_n_out != nullptr && idx < 2 * kVecPerTile && key0 + key < sk;
        const uintptr_t ks = reinterpret_cast<uintptr_t>(p.side_k);
        const uintptr_t vs = reinterpret_cast<uintptr_t>(p.side_v);
        const uint16_t* sbase = reinterpret_cast<const uint16_t*>(ks + (vs - ks) * uintptr_t(tensor != 0));
        // all heads of the tile's 32 slots (a tile lies in one block)
        const __amdgpu_buffer_rsrc_t rs = wave_rsrc(sbase + slot0 * p.kvh * nom, kTile * p.kvh * nom * 2);
        const int el = (key * p.kvh + g) * nom + slot;
        pre_sd[set][e] = __builtin_amdgcn_raw_buffer_load_b32(rs, has && slot < nom ? (2 * el) & ~3 : 0x40000000, 0, 0);
      }
    }
  };
  // (per-channel) the read scales of kv head g, K then V, in LDS after the
  // two stages: filled once per segment, read at every commit.
  float* const sc_lds = reinterpret_cast<float*>(smem + 2 * kPrefillStage);
  if constexpr (kEnc == kI8Chan) {
    if (threadIdx.x < 2 * kD)
      sc_lds[threadIdx.x] = (threadIdx.x < kD ? p.k_scale : p.v_scale)[g * kD + (threadIdx.x & (kD - 1))];
    __syncthreads();
  }
  const int n_out = (kPLo && p.head_n_out != nullptr)
                        ? min(table_entry(p.head_n_out, g), int(p.n_out_max))
                        : 0;
  // (per-channel) the slots whose outlier dims fall in this lane's 16-dim
  // chunk of a key row (the chunk is the same in every tile): bit j of
  // hit_mask, the dim within the chunk in bits 4j .. 4j + 3 of hit_pos.
  uint32_t hit_mask = 0, hit_pos = 0;
  if constexpr (kEnc == kI8Chan) {
    static_assert(kLoadsPerThread == 1, "one 16-code chunk per lane");
    const int vec = (threadIdx.x % kVecPerTile) % kVecPerRow;
    for (int j = 0; j < n_out; ++j) {
      const int d = table_entry(p.out_idx, int64_t(g) * p.n_out_max + j);
      if ((d >> 4) == vec) {
        hit_mask |= 1u << j;
        hit_pos |= uint32_t(d & 15) << (4 * j);
      }
    }
  }
  // (per-channel) the outlier dim of side slot lm, for the residue product
  const int plo_dim =
      (kPLo && L.lm < n_out) ? (p.out_idx[int64_t(g) * p.n_out_max + L.lm] & (kD - 1)) : 0;
  f32x4_t plo[kPreNCB];
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) plo[cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto commit = [&](int set, int buf) {
    char* st_base = stage_ptr(buf);
#pragma unroll
    for (int e = 0; e < kLoadsPerThread; ++e) {
      const int idx = e * kThreads + threadIdx.x;
      if (idx < 2 * kVecPerTile) {
        const int tensor = idx / kVecPerTile;
        const int rem = idx - tensor * kVecPerTile;
        const int key = rem / kVecPerRow;
        const int vec = rem - key * kVecPerRow;
        if constexpr (kEnc == kBF16) {
          char* dst = st_base + tensor * kTileBytesBF16 + key * kPitch + vec * 16;
          *reinterpret_cast<u32x4_t*>(dst) = pre[set][e];
        } else {
          // 16 codes, dims 16 vec .. + 15, to bf16 exactly as the dequant
          // kernels round them: bf16(float(code) * scale), nearest-even.
          const u32x4_t c = pre[set][e];
          uint32_t o[8];
          if constexpr (kEnc == kI8Tok) {
            const float sc = pre_sc[set][e];
#pragma unroll
            for (int w2 = 0; w2 < 8; ++w2) {
              const uint32_t word = c[w2 >> 1];
              const int sh = (w2 & 1) * 16;
              o[w2] = pack_bf16x2_fast(float(int8_t((word >> sh) & 0xffu)) * sc,
                                       float(int8_t((word >> (sh + 8)) & 0xffu)) * sc);
            }
          } else {
            const float* ds = sc_lds + tensor * kD + vec * 16;
#pragma unroll
            for (int w2 = 0; w2 < 8; ++w2) {
              const uint32_t word = c[w2 >> 1];
              const int sh = (w2 & 1) * 16;
              o[w2] = pack_bf16x2_fast(float(int8_t((word >> sh) & 0xffu)) * ds[2 * w2],
                                       float(int8_t((word >> (sh + 8)) & 0xffu)) * ds[2 * w2 + 1]);
            }
          }
          char* dst = st_base + tensor * kTileBytesBF16 + key * kPitch + vec * 32;
          *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{o[0], o[1], o[2], o[3]};
          *reinterpret_cast<u32x4_t*>(dst + 16) = u32x4_t{o[4], o[5], o[6], o[7]};
          if constexpr (kEnc == kI8Chan) {
            // The head's outlier dims take the side row's exact values: the
            // lane that wrote the chunk rewrites them (one lane's LDS writes
            // land in order), slot by slot, so that a later slot wins on a
            // duplicate dim, like dequant_chan.
            if (n_out > 0) {
              const int kl = L.lane & ~7;  // lane of the key's chunk 0 (slot 0)
              const int hsel = ((key * p.kvh + g) * p.n_out_max) & 1;  // slot 0's half
              uint32_t w[kSideMax];
#pragma unroll
              for (int j = 0; j < kSideMax; ++j) w[j] = __shfl(pre_sd[set][e], kl + j, 64);
#pragma unroll
              for (int j = 0; j < kSideMax; ++j) {
                if ((hit_mask >> j) & 1u) {
                  const uint16_t sv = uint16_t(((hsel + j) & 1) ? (w[j] >> 16) : (w[j] & 0xffffu));
                  *reinterpret_cast<uint16_t*>(dst + 2 * ((hit_pos >> (4 * j)) & 15u)) = sv;
                }
              }
            }
          }
        }
      }
    }
  };
  // LDS -> operand registers, same lane mapping as the HBM loads.
  auto read_tile = [&](Tile<kCmp>& t, int buf) {
    const char* kb = stage_ptr(buf);
    const char* vb = kb + kTileBytesBF16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const char* row = kb + (h * 16 + L.lm) * kPitch + L.lg * 16;
#pragma unroll
      for (int c = 0; c < 4; ++c) t.k[h][c] = *reinterpret_cast<const u32x4_t*>(row + c * 64);
    }
#pragma unroll
    for (int ii = 0; ii < 8; ++ii)
      t.v[ii] = *reinterpret_cast<const u32x4_t*>(vb + key_of_slot(L.lg, ii) * kPitch + L.lm * 16);
  };

  if (ntiles > 0) {
    // Tile j sits in register set j & 1 while in flight, then in LDS stage
    // j & 1.  Iteration j issues tile j + 2's loads, attends tile j from LDS
    // and commits tile j + 1 (loaded during iteration j - 1): two tiles of
    // compute cover each tile's global latency.
    int64_t slots[3];
    slots[0] = tile_slot0(0);
    fetch(0, slots[0], k_begin, true);
    commit(0, 0);
    slots[1] = 0;
    if (ntiles > 1) {
      slots[1] = tile_slot0(1);
      fetch(1, slots[1], k_begin + kTile, true);
    }
    __syncthreads();
    for (int j0 = 0; j0 < ntiles; j0 += 2) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int tix = j0 + r;
        if (tix < ntiles) {
          slots[2] = 0;
          const bool more = tix + 2 < ntiles;
          if (more) slots[2] = tile_slot0(tix + 2);
          if constexpr (kEnc != kBF16) {
            fetch(r, slots[2], k_begin + (tix + 2) * kTile, more);
          } else if (more) {
            fetch(r, slots[2], k_begin + (tix + 2) * kTile, true);
          }
          Tile<kCmp> t;
          read_tile(t, r);
          attend<kCmp, kPreNCB, false, kSideMax, kPLo>(
              st, t, Q, ci, k_begin + tix * kTile, sk, min_klim, kFresh ? -1 : slots[0], p, g, L,
              stage_ptr(r) + kTileBytesBF16, plo, n_out, plo_dim);
          if (tix + 1 < ntiles) commit(1 - r, 1 - r);
          __syncthreads();
          slots[0] = slots[1];
          slots[1] = slots[2];
        }
      }
    }
  }

  // Epilogue: each wave finalises its own columns (no cross-wave merge).
  {
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
      const int col = L.lm;
      const int tq = q0 + (wave * kPreNCB + cb) * p.tpb + col / p.hs;
      const int hh = col % p.hs;
      if constexpr (kPLo) {
        // The residue product of side slot j (C row j: lane lm + 16 (j >> 2),
        // element j & 3) joins O at the slot's dim d (lane group d >> 5,
        // chunk d & 7, row (d >> 3) & 3).  A dim listed twice took the later
        // slot's value, so only that slot's residue counts.
        for (int j = 0; j < n_out; ++j) {
          const int d = table_entry(p.out_idx, int64_t(g) * p.n_out_max + j);
          bool later = false;
          for (int j2 = j + 1; j2 < n_out; ++j2)
            later |= table_entry(p.out_idx, int64_t(g) * p.n_out_max + j2) == d;
          if (later) continue;
          const int e = j & 3;
          const f32x4_t c = plo[cb];
          const float mine = e == 0 ? c[0] : e == 1 ? c[1] : e == 2 ? c[2] : c[3];
          const float val = __shfl(mine, L.lm + 16 * (j >> 2), 64);
          if (L.lg == (d >> 5)) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (jj == (d & 7) && r == ((d >> 3) & 3)) st.o[cb][jj][r] += val;
          }
        }
      }
      store_prefill_block<kCmp, kPreNCB>(p, st, cb, int64_t(p.n_dec) + cq0 + tq,
                                         g * p.group + s * p.hs + hh,
                                         col < p.tpb * p.hs && hh < hs && tq < sq, split, L);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Kernels.
// ---------------------------------------------------------------------------
// Decode unit u -> (row b, kv-slice group, chunk); the slice group is the
// fastest index, then the chunk, so the units of one row are adjacent.
__device__ __forceinline__ void decode_unit_of(const AttnParams& p, int u, int& b, int& kvg,
                                               int& chunk) {
  const int groups = (p.kvh * p.nslices) / p.kvs_per_wg;
  const int units_per_row = groups * p.dec_max_chunks;
  b = u / units_per_row;
  const int rem = u - b * units_per_row;
  chunk = rem / groups;
  kvg = rem - chunk * groups;
}

template <int kEnc>
__global__ void __launch_bounds__(kThreads) paged_decode_kernel(AttnParams p) {
  __shared__ __align__(16) char smem[kDecodeSmem];
  int b, kvg, chunk;
  decode_unit_of(p, blockIdx.x, b, kvg, chunk);
  decode_unit<kEnc>(p, smem, p.block_tables, b, kvg, chunk);
}

// ---------------------------------------------------------------------------
// Stream-K paged decode.  The rows' 32-key tiles, concatenated in row-unit
// order (row unit r = row * groups + slice group), are cut into gridDim.x
// equal shares of S = max(sk_min_share, ceil(W / gridDim.x),
// ceil(Tmax / (max_splits - 1))) tiles, W = total tiles, Tmax = longest row;
// workgroup w attends the tiles [w S, (w + 1) S).  A share may span several
// rows (one segment each) and a row may span several shares: every share
// costs the same whatever the context lengths, and a row spans at most
// ceil(T / S) + 1 <= max_splits workgroups.  Rows inside one share are
// written final; the others as partials, merged by merge_kernel with
// sk_nseg[r] splits.  Zero-length rows (no tiles) get NaN, the reference's
// 0 / 0, from the workgroup whose share holds their start.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int ctx_tiles(int ctx) { return ctx > 0 ? (ctx + kTile - 1) / kTile : 0; }

// Split count of every kv slice of slice group kvg of row b (sk_nseg is
// [rows, kv slices]).
__device__ __forceinline__ void set_nseg(const AttnParams& p, int b, int kvg, int nseg) {
  const int per = p.kvs_per_wg;
  for (int j = 0; j < per; ++j) p.sk_nseg[int64_t(b) * (p.kvh * p.nslices) + kvg * per + j] = nseg;
}

// NaN output rows for every head of slice group kvg of row b.
__device__ void write_nan_rows(const AttnParams& p, int b, int kvg) {
  const int per = p.kvs_per_wg;
  for (int sl = 0; sl < per; ++sl) {
    const int kvs = kvg * per + sl;
    const int g = kvs / p.nslices;
    const int s = kvs - g * p.nslices;
    const int hs = min(p.hs, p.group - s * p.hs);
    for (int col = 0; col < hs; ++col) {
      uint16_t* dst = p.out + int64_t(b) * p.o_st + int64_t(g * p.group + s * p.hs + col) * p.o_sh;
      for (int d = 0; d < kD; d += 8)
        *reinterpret_cast<u32x4_t*>(dst + d) =
            u32x4_t{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
    }
  }
}

// block_tables and ctx_lens come as restrict-qualified kernel arguments:
// the kernel's stores (split counts, outputs, partials) provably never touch
// them, so their wave-uniform reads stay scalar loads inside the segment
// loop.  Every wave computes the partition itself from one read of the
// context lengths (lane l sums the tiles of a contiguous run of row units, a wave
// scan by shuffles gives the prefix), so no workgroup barrier stands between
// the launch and the first KV load.  Wave 0 also records each row's split
// count (from the share holding its first tile) and writes NaN rows for
// empty contexts.
// One workgroup's share (share w of `grid`) of a stream-K decode launch.
// kLds: 4 kv heads per workgroup staged through LDS, bf16
// (decode_segment_lds: two stages in smem and smem1) or per-token-head int8
// (decode_segment_lds_i8: a four-stage ring in smem); smem2 holds the query.
template <int kEnc, bool kLds, bool kSteal = false, int kHeads = 4>
__device__ __forceinline__ void decode_sk_share(const AttnParams& p,
                                                const int32_t* __restrict__ block_tables,
                                                const int32_t* __restrict__ ctx_lens, int w,
                                                int grid, char* smem, char* smem1, char* smem2,
                                                const StealArgs& sa) {
  constexpr bool kBfLds = kLds && kEnc == kBF16;
  constexpr bool kI8Lds = kLds && (kEnc == kI8Tok || kEnc == kI8Chan);
  static_assert(!kLds || kBfLds || kI8Lds, "no LDS-staged form for this encoding");
  const unsigned long long t_start =
      p.wg_stamps != nullptr ? __builtin_amdgcn_s_memrealtime() : 0ull;
  // kvs_per_wg divides 8 (a power of two)
  const int groups = (p.kvh * p.nslices) >> __builtin_ctz(unsigned(p.kvs_per_wg));
  const float rgroups = __builtin_amdgcn_rcpf(float(groups));
  auto row_of = [&](int r) { return div_small(r, groups, rgroups); };
  const int R = p.n_dec * groups;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(int(threadIdx.x >> 6));
  const int per_lane = (R + 63) / 64;
  const int r0 = min(R, lane * per_lane);
  const int r1 = min(R, r0 + per_lane);
  // The first kCached context lengths of the lane's run stay in registers for
  // the second pass (one round trip to memory for batches up to 256 x groups).
  constexpr int kCached = 4;
  int cl[kCached];
#pragma unroll
  for (int i = 0; i < kCached; ++i) cl[i] = r0 + i < r1 ? ctx_lens[row_of(r0 + i)] : 0;
  auto ctx_of = [&](int r) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < kCached; ++i) c = (r == r0 + i) ? cl[i] : c;
    return r - r0 < kCached ? c : ctx_lens[row_of(r)];
  };
  int mine = 0, tmax = 0, rows = 0;
  for (int r = r0; r < r1; ++r) {
    const int t = ctx_tiles(ctx_of(r));
    mine += t;
    tmax = max(tmax, t);
    rows += t > 0;
  }
  // Wave prefix sums of the lanes' tiles and non-empty rows, and the
  // longest row (DPP scans; lane 63 holds the totals).
  const int tiles_incl = wave_scan_add(mine);
  const int rows_incl = wave_scan_add(rows);
  const int tsum = __builtin_amdgcn_readlane(tiles_incl, 63);
  const int rsum = __builtin_amdgcn_readlane(rows_incl, 63);
  const int Tmax = __builtin_amdgcn_readlane(wave_scan_max_nonneg(tmax), 63);
  // Rows of unequal length: each non-empty row also carries kDecRowCost
  // virtual tiles (a share that starts a second row pays the ring's restart:
  // its drain, query and first tiles), so such shares get fewer real tiles.
  // Equal rows keep shares aligned to rows and carry none.
  const int row_cost = tsum == Tmax * rsum ? 0 : kDecRowCost;
  mine += row_cost * rows;
  const int incl = tiles_incl + row_cost * rows_incl;
  const int W = tsum + row_cost * rsum;
  const int excl = incl - mine;
  int S = max(p.sk_min_share, (W + grid - 1) / grid);
  const int need = p.max_splits > 1 ? (Tmax + p.max_splits - 2) / (p.max_splits - 1) : 1;
  S = max(S, need);
  // XCD-aware shares: workgroup v runs on XCD v mod 8, and the odd XCDs
  // stream measurably slower, so even shares take S + d tiles and odd ones
  // S - d (d <= S / 4, and S - d still meets the split bound).
  int d = int(p.xcd_skew * float(S) + 0.5f);
  d = max(0, min(d, min(S / 4, S - max(need, 1))));
  auto share_start = [&](int v) { return v * S + ((v & 1) ? d : 0); };
  const float rS = __builtin_amdgcn_rcpf(float(S));
  auto share_of = [&](int x) {
    int v = div_small(x, S, rS);
    if ((v & 1) && x - v * S < d) --v;
    return v;
  };
  const int start = share_start(w);
  const int end = min(W, share_start(w + 1));
  // The row unit holding tile `start` opens this share.
  int found_r = R, found_p = 0, found_c = 0;
  {
    int P = excl;
    for (int r = r0; r < r1; ++r) {
      const int c = ctx_of(r);
      const int t = ctx_tiles(c);
      const int span = t > 0 ? t + row_cost : 0;  // real tiles at [P + row_cost, P + span)
      if (t > 0 && P <= start && start < P + span) {
        found_r = r;
        found_p = P;
        found_c = c;
      }
      if (wave == 0) {
        if (t == 0) {
          const int owner = W > 0 ? share_of(min(P, W - 1)) : 0;
          if (owner == w) {
            const int rb = row_of(r), rg = r - rb * groups;
            write_nan_rows(p, rb, rg);
            set_nseg(p, rb, rg, 0);
            if constexpr (kI8Lds && kEnc == kI8Tok) {
              if (p.app_k != nullptr) append_i8_row_lane(p, rb, rg);
            }
            if constexpr (kBfLds) {
              if (p.app_k != nullptr) {
                // one lane holds this row unit here: it stores all its chunks
                for (int c = 0; c < 16 * kHeads; ++c) {
                  u32x4_t kn, vn;
                  append_load<kHeads>(p, rb, rg, c, kn, vn);
                  append_store<kHeads>(p, rb, rg, c, kn, vn);
                }
              }
            }
          }
        } else if (share_of(P + row_cost) == w) {
          const int rb = row_of(r);
          const int nseg = share_of(P + row_cost + t - 1) - share_of(P + row_cost) + 1;
          // with the tail hand-out the merge also needs the row's first share
          set_nseg(p, rb, r - rb * groups, kSteal ? nseg | (w << 16) : nseg);
        }
      }
      P += span;
    }
  }
  const unsigned long long hit = __ballot(found_r < R);
  const int src = uniform(hit ? __ffsll(hit) - 1 : 0);
  int r = __builtin_amdgcn_readlane(found_r, src);
  int P = __builtin_amdgcn_readlane(found_p, src);
  int ctx = __builtin_amdgcn_readlane(found_c, src);
  // The last segment of share v (every lane of the wave takes part): its row
  // unit, context, tiles [t0, t1) of the row and tail length.  The dynamic
  // hand-out puts share v's tail there: min(tail, len - 4) tiles, so the
  // owner keeps at least four (its first claim goes out in step 0).
  struct TailGeo {
    int r, ctx, t0, t1, n;
  };
  auto last_seg = [&](int v) -> TailGeo {
    const int sv = share_start(v);
    const int ev = min(W, share_start(v + 1));
    int hr = -1, hp = 0, hc = 0, ht = 0;
    int Q = excl;
    for (int rr = r0; rr < r1; ++rr) {
      const int c = ctx_of(rr);
      const int t = ctx_tiles(c);
      if (t > 0) {
        const int Pr = Q + row_cost;
        if (Pr < ev && Pr + t > sv) {
          hr = rr;
          hp = Pr;
          hc = c;
          ht = t;
        }
        Q += t + row_cost;
      }
    }
    const unsigned long long m = __ballot(hr >= 0);
    TailGeo tg{-1, 0, 0, 0, 0};
    if (m != 0) {
      const int src = uniform(63 - __clzll(m));  // the last row with tiles in the share
      tg.r = __builtin_amdgcn_readlane(hr, src);
      tg.ctx = __builtin_amdgcn_readlane(hc, src);
      const int Pr = __builtin_amdgcn_readlane(hp, src);
      const int t = __builtin_amdgcn_readlane(ht, src);
      tg.t0 = max(sv, Pr) - Pr;
      tg.t1 = min(ev, Pr + t) - Pr;
      const int len = tg.t1 - tg.t0;
      tg.n = len >= 5 ? min(sa.tail, len - 4) : 0;
    }
    return tg;
  };
  // The share's own tail; its owner announces the tail length in its claim
  // word (a word still 0 offers nothing to take).
  TailGeo own{-1, 0, 0, 0, 0};
  if constexpr (kBfLds && kSteal) {
    {
      own = last_seg(w);
      if (own.n > 0 && wave == 0 && lane == 0)
        __hip_atomic_fetch_add(sa.claims + w, (unsigned long long)(own.n) << 32,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // The share's segments in order: each row unit with real tiles in
  // [start, end).
  auto next_seg = [&](DecSeg& sg) -> bool {
    while (r < R && P < end) {
      const int b = uniform(row_of(r));
      const int t = ctx_tiles(ctx);
      const int Pr = P + row_cost;  // the row's first real tile
      bool hit = false;
      if (t > 0 && Pr < end) {
        const int first_share = share_of(Pr);
        const int nseg = share_of(Pr + t - 1) - first_share + 1;
        sg = DecSeg{b, r - b * groups, ctx, max(start, Pr) - Pr, min(end, Pr + t) - Pr,
                    nseg == 1 ? -1 : w - first_share, r == own.r ? own.n : 0, -1};
        hit = true;
      }
      P += t > 0 ? t + row_cost : 0;
      ++r;
      if (r < R && P < end) ctx = table_entry(ctx_lens, row_of(r));
      if (hit) return true;
    }
    return false;
  };
  if constexpr (kBfLds && kHeads == 2) {
    DecSeg cur, nxt;
    bool have = next_seg(cur);
    bool pre = false;
    while (have) {
      have = decode_segment_lds2(p, smem, smem1, smem2, block_tables, cur, pre, next_seg, nxt);
      pre = have;
      cur = nxt;
    }
  } else if constexpr (kBfLds) {
    __shared__ int s_steal[12];  // [0]: owner claim verdict; [1..]: a taken tile
    // Each segment finds the next one (after issuing its own first loads)
    // and issues that one's first loads under its own last tile.
    DecSeg cur, nxt;
    bool have = next_seg(cur);
    bool pre = false;
    while (have) {
      have = decode_segment_lds<kSteal>(p, smem, smem1, smem2, block_tables, cur, pre, next_seg,
                                        nxt, sa, s_steal, w);
      pre = have;
      cur = nxt;
    }
    if constexpr (kSteal) {
      // Own share done: take single tail tiles from the back of other shares,
      // the one with the most left first (then the nearest after this one).
      // A taken tile is its own partial (tail slot v * kDecTailMax + j).  The
      // claims are wave 0's; the others read the result from LDS.  Every
      // failed claim leaves that share's word at or past its tail, so no
      // share is tried twice and the loop ends.
      int tv = -1, tleft = 0;
      int* const dummy = sa.dummy + int64_t(w) * 8;
      auto thief_next = [&](DecSeg& nx) -> bool {
        if (wave == 0) {
          int got = 0;
          DecSeg out{0, 0, 0, 0, 0, -1, 0, -1};
          for (int tries = 0; tries <= grid && got == 0; ++tries) {
            if (tleft <= 0) {
              int best = 0;
              for (int v0 = 0; v0 < grid; v0 += 64) {
                const int v = v0 + lane;
                if (v < grid && v != w) {
                  const unsigned long long o = __hip_atomic_load(
                      sa.claims + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                  const int rem = claim_tiles(o) - claim_front(o) - claim_back(o);
                  const int dist = (v - w - 1 + grid) % grid;
                  if (rem >= sa.steal_min) best = max(best, (rem << 9) | (511 - dist));
                }
              }
              best = wave_max(best);
              if (best == 0) break;
              tv = (w + 1 + (511 - (best & 511))) % grid;
              tleft = 1;
            }
            unsigned long long o = 0;
            if (lane == 0) o = claim_word(sa.claims + tv, 1ull << 16, dummy);
            const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(o))));
            const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(o >> 32))));
            o = (uint64_t(hi) << 32) | lo;
            const int f = claim_front(o), bk = claim_back(o), n = claim_tiles(o);
            // The word's tail length must be the one the partition gives that
            // share (it always is while every launch's merge resets the words),
            // so a taken tile is always one of the share's tail tiles.
            const TailGeo tg = last_seg(tv);
            if (f + bk < n && n == tg.n) {
              tleft = n - f - bk - 1 >= sa.steal_min ? 1 : 0;
              const int rb = uniform(row_of(tg.r));
              out = DecSeg{rb, tg.r - rb * groups, tg.ctx, tg.t1 - 1 - bk, tg.t1 - bk, -1, 0,
                           tv * kDecTailMax + bk};
              got = 1;
            } else {
              tleft = 0;
            }
          }
          if (lane == 0) {
            s_steal[1] = got;
            s_steal[2] = out.b;
            s_steal[3] = out.kvg;
            s_steal[4] = out.ctx;
            s_steal[5] = out.t0;
            s_steal[6] = out.t1;
            s_steal[7] = out.tslot;
          }
        }
        pf_barrier();
        const int got = uniform(s_steal[1]);
        if (got) {
          nx = DecSeg{uniform(s_steal[2]), uniform(s_steal[3]), uniform(s_steal[4]),
                      uniform(s_steal[5]), uniform(s_steal[6]), -1, 0, uniform(s_steal[7])};
        }
        return got != 0;
      };
      have = thief_next(cur);
      pre = false;
      while (have) {
        have = decode_segment_lds<kSteal>(p, smem, smem1, smem2, block_tables, cur, pre,
                                          thief_next, nxt, sa, s_steal, w);
        pre = have;
        cur = nxt;
      }
    }
  } else {
    DecSeg sg;
    while (next_seg(sg)) {
      if constexpr (kI8Lds && kEnc == kI8Chan) {
        const int32_t* bt = block_tables + int64_t(sg.b) * p.bt_stride;
        switch (p.n_out_max) {
          case 2:
            decode_segment_lds_i8<kI8Chan, 2>(p, smem, smem2, bt, sg.b, sg.kvg, sg.ctx, sg.t0,
                                              sg.t1, sg.split);
            break;
          case 8:
            decode_segment_lds_i8<kI8Chan, 8>(p, smem, smem2, bt, sg.b, sg.kvg, sg.ctx, sg.t0,
                                              sg.t1, sg.split);
            break;
          default:  // 4, or no side pool
            decode_segment_lds_i8<kI8Chan, 4>(p, smem, smem2, bt, sg.b, sg.kvg, sg.ctx, sg.t0,
                                              sg.t1, sg.split);
            break;
        }
      } else if constexpr (kI8Lds) {
        decode_segment_lds_i8<kI8Tok, 0>(p, smem, smem2,
                                         block_tables + int64_t(sg.b) * p.bt_stride, sg.b,
                                         sg.kvg, sg.ctx, sg.t0, sg.t1, sg.split);
      } else {
        decode_segment<kEnc>(p, smem, block_tables + int64_t(sg.b) * p.bt_stride, sg.b, sg.kvg,
                             sg.ctx, sg.t0, sg.t1, sg.split);
      }
    }
  }
  if (p.wg_stamps != nullptr) {
    __syncthreads();  // every wave has issued its last stores
    if (threadIdx.x == 0) {
      p.wg_stamps[2 * w] = t_start;
      p.wg_stamps[2 * w + 1] = __builtin_amdgcn_s_memrealtime();
    }
  }
}

template <int kEnc, bool kLds>
__global__ void __launch_bounds__(kThreads)
paged_decode_sk_kernel(AttnParams p, const int32_t* __restrict__ block_tables,
                       const int32_t* __restrict__ ctx_lens) {
  constexpr bool kBfLds = kLds && kEnc == kBF16;
  constexpr bool kI8Lds = kLds && kEnc == kI8Tok;
  constexpr bool kChLds = kLds && kEnc == kI8Chan;
  __shared__ __align__(16) char
      smem[kBfLds ? kLdsStage : (kI8Lds ? kLdsI8 : (kChLds ? kLdsChan : kDecodeSmem))];
  __shared__ __align__(16) char smem1[kBfLds ? kLdsStage : 16];
  __shared__ __align__(16) char smem2[kLds ? kLdsQ : 16];
  touch_kernel_args(int(sizeof(AttnParams) + 2 * sizeof(void*)));
  decode_sk_share<kEnc, kLds>(p, block_tables, ctx_lens, int(blockIdx.x), int(gridDim.x), smem,
                              smem1, smem2, StealArgs{});
}

// The bf16 LDS decode with 2 kv heads per workgroup.
__global__ void __launch_bounds__(kThreads)
paged_decode_sk2_kernel(AttnParams p, const int32_t* __restrict__ block_tables,
                        const int32_t* __restrict__ ctx_lens) {
  __shared__ __align__(16) char smem[kLdsStage];
  __shared__ __align__(16) char smem1[kLdsStage];
  __shared__ __align__(16) char smem2[kLdsSmem2];
  touch_kernel_args(int(sizeof(AttnParams) + 2 * sizeof(void*)));
  decode_sk_share<kBF16, true, false, 2>(p, block_tables, ctx_lens, int(blockIdx.x),
                                         int(gridDim.x), smem, smem1, smem2, StealArgs{});
}

// The bf16 LDS decode with the dynamic tail hand-out.
__global__ void __launch_bounds__(kThreads)
paged_decode_steal_kernel(AttnParams p, const int32_t* __restrict__ block_tables,
                          const int32_t* __restrict__ ctx_lens, StealArgs sa) {
  __shared__ __align__(16) char smem[kLdsStage];
  __shared__ __align__(16) char smem1[kLdsStage];
  __shared__ __align__(16) char smem2[kLdsQ];
  touch_kernel_args(int(sizeof(AttnParams) + 2 * sizeof(void*) + sizeof(StealArgs)));
  decode_sk_share<kBF16, true, true>(p, block_tables, ctx_lens, int(blockIdx.x), int(gridDim.x),
                                     smem, smem1, smem2, sa);
}

// Geometry of prefill chunk i: its query rows, key rows, the keys before its
// first query (prefix) and its query tiles of qtile tokens.
struct ChunkGeo {
  int sq, sk, prefix, ntq;
};

__device__ __forceinline__ ChunkGeo chunk_geo(const int32_t* cu_q, const int32_t* cu_k, int i,
                                              int qtile) {
  ChunkGeo c;
  c.sq = cu_q[i + 1] - cu_q[i];
  c.sk = cu_k[i + 1] - cu_k[i];
  c.prefix = c.sk - c.sq;
  c.ntq = (c.sq > 0 && c.sk > 0) ? (c.sq + qtile - 1) / qtile : 0;
  return c;
}

// Key tiles of query tile qt: its last query sees keys [0, prefix + last + 1).
__device__ __forceinline__ int qtile_tiles(const ChunkGeo& c, int qtile, int qt) {
  const int keys = qt + 1 < c.ntq ? c.prefix + (qt + 1) * qtile : c.sk;
  return (keys + kTile - 1) / kTile;
}

// Key tiles of query tiles [0, q), q <= ntq.  Every tile but the last sees
// prefix + 16 tpb u keys (u = 1, 2, ...; a query tile is 16 tpb tokens), so
// its tile count is floor(tpb u / 2) + floor((prefix + 31 + 16 (tpb u mod 2))
// / 32): a quadratic in u plus one of two constants, by the parity of tpb u.
static_assert(kWaves * kPreNCB == 16, "query tiles are 16 tpb tokens");
__device__ __forceinline__ int64_t qtile_cum(const ChunkGeo& c, int tpb, int q) {
  if (q <= 0) return 0;
  const int64_t n = min(q, c.ntq - 1);
  const int64_t B = int64_t(c.prefix) + kTile - 1;
  const int64_t c0 = B >> 5, c1 = (B + 16) >> 5;
  const int64_t nodd = (tpb & 1) ? (n + 1) >> 1 : 0;
  int64_t s = ((int64_t(tpb) * n * (n + 1) >> 1) - nodd) / 2 + nodd * c1 + (n - nodd) * c0;
  if (q == c.ntq) s += (c.sk + kTile - 1) / kTile;
  return s;
}

// Locate prefill unit u: chunk i, query tile, kv slice, split (query tile
// fastest so that units sharing K/V are adjacent).
__device__ __forceinline__ bool find_prefill_unit(const AttnParams& p, int u, int& i, int& qt,
                                                  int& kvs, int& split) {
  const int qtile_tokens = kWaves * kPreNCB * p.tpb;
  const int kvslices = p.kvh * p.nslices;
  for (i = 0; i < p.n_pre; ++i) {
    const int sq = p.cu_q[i + 1] - p.cu_q[i];
    const int sk = p.cu_k[i + 1] - p.cu_k[i];
    if (sq <= 0 || sk <= 0) continue;
    const int ntq = (sq + qtile_tokens - 1) / qtile_tokens;
    const int ns = max(1, (sk + p.split_tokens - 1) / p.split_tokens);
    const int units = ntq * kvslices * ns;
    if (u < units) {
      qt = u % ntq;
      const int r = u / ntq;
      kvs = r % kvslices;
      split = r / kvslices;
      return true;
    }
    u -= units;
  }
  return false;
}

// One workgroup per prefill unit (chunk, query tile, kv slice, key split):
// the launch under KVC_PREFILL_SK=0, and for a paged int8 pool passed to
// kvc_varlen_attention directly (its stage dequantises the tiles; the faster
// route gathers the keys first, kvc_gather_kv, and runs the stream-K
// prefill over them).
template <int kEnc, bool kFresh, bool kPLo = (kEnc == kI8Chan)>
__global__ void __launch_bounds__(kThreads)
varlen_kernel(AttnParams p, const int32_t* __restrict__ block_tables) {
  __shared__ __align__(16) char smem[kSmemBytes];
  const int u = blockIdx.x;
  if (u >= p.pre_units) return;
  int i, qt, kvs, split;
  if (!find_prefill_unit(p, u, i, qt, kvs, split)) return;
  const int sk = p.cu_k[i + 1] - p.cu_k[i];
  const int nsplit = max(1, (sk + p.split_tokens - 1) / p.split_tokens);
  const int per = p.split_tokens / kTile;
  prefill_segment<kEnc, kFresh, kPLo>(p, smem, block_tables, i, qt, kvs, split * per,
                                      (split + 1) * per, nsplit == 1 ? -1 : split);
}

// ---------------------------------------------------------------------------
// Stream-K prefill launch over bf16 keys (a paged bf16 pool, or fresh rows:
// the step's k/v when there is no prefix cache, or an int8 pool's keys
// gathered by kvc_gather_kv).  Items are (chunk i, kv slice,
// query tile), query tile fastest; each is a run of 32-key tiles that stops
// at the last key its queries see.  The concatenated tiles (plus a fixed cost
// per item) are cut into one equal share per workgroup, so chunks of any
// length mix spread evenly over the CUs, and a workgroup streams its share
// with no break at item boundaries.  Items spanning several shares write
// split-K partials; the share holding an item's first tile records the split
// count of its rows for the merge.
//
// K rows in LDS are 256 bytes padded to 272 (17 chunks of 16 bytes): 16 rows
// read at one column offset touch 16 different bank groups, and every operand
// read is a per-lane base plus an immediate.  A 64-lane direct-to-LDS load
// fills 64 consecutive chunks, so lane l of load k fetches whichever chunk
// belongs at slot 64 k + l (pad slots and rows past the tile read 0).
// ---------------------------------------------------------------------------
constexpr int kPfRowSlots = 17;
constexpr int kPfPitch = kPfRowSlots * 16;                          // 272
constexpr int kPfLoadsPerTensor = (kTile * kPfRowSlots + 63) / 64;  // 9
constexpr int kPfTensor = kPfLoadsPerTensor * 1024;
constexpr int kPfStage = 2 * kPfTensor;  // K then V
constexpr int kPfTileLoads = (2 * kPfLoadsPerTensor + kWaves - 1) / kWaves;  // per wave: 3
constexpr int kPfMinShare = 4;
constexpr int kOob = 0x40000000;  // a buffer offset past every resource: reads 0, no traffic
static_assert(kPfTileLoads == 3, "wait counts below assume three tile loads per wave");

struct PfItem {
  int i, kvs, qt;  // chunk, kv slice, query tile
  int g, s;        // kv head and slice within its group: kvs = g * nslices + s
  int P;           // weighted position of the item's span (item cost + T long)
  int T;           // tiles of the item
  int cq0, ck0;    // chunk's first query row / key row (prefill-relative)
  ChunkGeo geo;
};

__device__ __forceinline__ void pf_load_chunk(PfItem& it, const int32_t* cu_q, const int32_t* cu_k,
                                              int qtile) {
  it.geo = chunk_geo(cu_q, cu_k, it.i, qtile);
  it.cq0 = cu_q[it.i];
  it.ck0 = cu_k[it.i];
}



// One 32-key tile of the stream-K prefill against the wave's kPreNCB column
// blocks (bf16 keys).  Differences from attend_tile, each removing VALU work:
//  * V^T operands come straight from LDS through transposing reads
//    (ds_read_b64_tr_b16: lane j of a 16-lane group receives element j % 4 of
//    the 8-byte rows addressed by lanes j / 4 + 4 k, k = 0..3), so PV MFMA jj
//    row m is dim 16 jj + m and the O^T accumulators hold, in lane (lm, lg),
//    dims 16 jj + 4 lg + r (r < 4) of column lm;
//  * the scale folds into the exponent (one fma per logit; the max is taken
//    on raw logits, the scale being positive);
//  * the column sums of P come from one more MFMA against an all-ones
//    operand (every row of the result is the sum, of the same bf16 P that
//    weights V), not from lane adds and a final reduction.
constexpr int kPfVRowSlots = 18;              // V rows padded to 288 B: tr reads conflict-free
constexpr int kPfPitchV = kPfVRowSlots * 16;  // 288
constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;

struct PfState {
  f32x4_t o[kPreNCB][8];  // O^T of PV MFMA jj (dims 16 jj + 4 lg + r)
  f32x4_t l[kPreNCB];     // column sums of P (all four rows equal)
  float m[kPreNCB];       // reference max (log2 domain), identical on the column's lanes
};

__device__ __forceinline__ void pf_init(PfState& st) {
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) st.o[cb][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    st.l[cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    st.m[cb] = -INFINITY;
  }
}

typedef short s16x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2_t lds_read_tr16(const char* p) {
  const s16x4v_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4v_t*)(
          (__attribute__((address_space(3))) char*)(p)));
  return __builtin_bit_cast(u32x2_t, r);
}

// S^T, the online softmax and P of one tile.  k: K operands as in
// Tile<kBF16>; klim[cb]: the lane's column key limit (-1 for an invalid
// column); pb[cb]: P^T of column block cb (bf16), the PV operand.
// kPLo: also pl[cb] = bf16(P - pb), the rounding residue of the operand, and
// the residue accumulators plo[cb] follow a move of the reference max.
template <bool kMasked, bool kPLo = false>
__device__ __forceinline__ void pf_score(PfState& st, const u32x4_t (&k)[2][4],
                                         const QOps<kBF16, kPreNCB>& Q,
                                         const int (&klim)[kPreNCB], int key0, int valid_end,
                                         float scale_log2, const LaneId& L,
                                         u32x4_t (&pb)[kPreNCB], f32x4_t* plo = nullptr,
                                         u32x4_t* pl = nullptr) {
  static_assert(kPreNCB == 2, "the schedule below pairs two column blocks");
  // S^T of column block 0, then of block 1 (block 0's max runs under block
  // 1's MFMAs).
  f32x4_t sacc[kPreNCB][2];
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
    sacc[cb][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    sacc[cb][1] = sacc[cb][0];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sacc[cb][0] = mfma_bf16(k[0][c], Q.op[cb][c], sacc[cb][0]);
      sacc[cb][1] = mfma_bf16(k[1][c], Q.op[cb][c], sacc[cb][1]);
    }
  }
  float x[kPreNCB][8];
  float tmax[kPreNCB];
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[cb][i] = sacc[cb][0][i];
      x[cb][4 + i] = sacc[cb][1][i];
    }
    if constexpr (kMasked) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int key = key0 + key_of_slot(L.lg, i);
        x[cb][i] = (key < valid_end && key <= klim[cb]) ? x[cb][i] : -INFINITY;
      }
    }
    float t = fmaxf(fmaxf(x[cb][0], x[cb][1]), x[cb][2]);
    t = fmaxf(fmaxf(t, x[cb][3]), x[cb][4]);
    t = fmaxf(fmaxf(t, x[cb][5]), x[cb][6]);
    t = fmaxf(t, x[cb][7]);
    tmax[cb] = rows4_max(t) * scale_log2;
  }
  // One rare branch for both blocks: rescale whichever moved its max by more
  // than the threshold.
  if (__builtin_expect(__ballot(tmax[0] > st.m[0] + kRescaleLog2 ||
                                tmax[1] > st.m[1] + kRescaleLog2) != 0, 0)) {
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
      if (__ballot(tmax[cb] > st.m[cb] + kRescaleLog2) == 0) continue;
      const float m_new = fmaxf(st.m[cb], tmax[cb]);
      const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(st.m[cb] - m_ref);
      st.m[cb] = m_new;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
        for (int r = 0; r < 4; ++r) st.o[cb][jj][r] *= alpha;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) st.l[cb][r] *= alpha;
      if constexpr (kPLo) {
#pragma unroll
        for (int r = 0; r < 4; ++r) plo[cb][r] *= alpha;
      }
    }
  }
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
    const float neg_m = (st.m[cb] == -INFINITY) ? 0.f : -st.m[cb];
    float pr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[cb][i], scale_log2, neg_m));
#pragma unroll
    for (int w = 0; w < 4; ++w) pb[cb][w] = pack_bf16x2_fast(pr[2 * w], pr[2 * w + 1]);
    if constexpr (kPLo) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pl[cb][w] = pack_bf16x2_fast(pr[2 * w] - bf16_bits_to_f32(pb[cb][w] & 0xffffu),
                                     pr[2 * w + 1] - bf16_bits_to_f32(pb[cb][w] >> 16));
    }
  }
}

// The fast loop's form of pf_score (unmasked tiles, reference max already
// set by the segment's first tile): P against the current reference max
// first, and the overflow test (a logit more than 2^kRescaleLog2 above the
// reference, i.e. a P above 2^kRescaleLog2) on the exp2 results, which as
// arithmetic results need no canonicalising max (MFMA results do).  The rare
// branch recomputes S^T (the logits are not kept live across the test),
// moves the reference and redoes P exactly as pf_score does.
template <bool kPLo = false>
__device__ __forceinline__ void pf_score_fast(PfState& st, const u32x4_t (&k)[2][4],
                                              const QOps<kBF16, kPreNCB>& Q, float scale_log2,
                                              u32x4_t (&pb)[kPreNCB], f32x4_t* plo = nullptr,
                                              u32x4_t* pl = nullptr) {
  auto qk = [&](f32x4_t (&sacc)[kPreNCB][2]) {
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
      sacc[cb][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      sacc[cb][1] = sacc[cb][0];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sacc[cb][0] = mfma_bf16(k[0][c], Q.op[cb][c], sacc[cb][0]);
        sacc[cb][1] = mfma_bf16(k[1][c], Q.op[cb][c], sacc[cb][1]);
      }
    }
  };
  auto exp_all = [&](const f32x4_t (&sacc)[kPreNCB][2], float (&pr)[kPreNCB][8]) {
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
      const float neg_m = (st.m[cb] == -INFINITY) ? 0.f : -st.m[cb];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[cb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[cb][0][i], scale_log2, neg_m));
        pr[cb][4 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[cb][1][i], scale_log2, neg_m));
      }
    }
  };
  float pr[kPreNCB][8];
  {
    f32x4_t sacc[kPreNCB][2];
    qk(sacc);
    exp_all(sacc, pr);
  }
  constexpr float kRescaleP = float(1 << int(kRescaleLog2));
  bool over = false;
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
    const float pm = fmaxf(fmaxf(fmaxf(pr[cb][0], pr[cb][1]), fmaxf(pr[cb][2], pr[cb][3])),
                           fmaxf(fmaxf(pr[cb][4], pr[cb][5]), fmaxf(pr[cb][6], pr[cb][7])));
    over |= pm > kRescaleP;
  }
  if (__builtin_expect(__ballot(over) != 0, 0)) {
    f32x4_t sacc[kPreNCB][2];
    qk(sacc);
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
      float t = fmaxf(fmaxf(sacc[cb][0][0], sacc[cb][0][1]), sacc[cb][0][2]);
      t = fmaxf(fmaxf(t, sacc[cb][0][3]), sacc[cb][1][0]);
      t = fmaxf(fmaxf(t, sacc[cb][1][1]), sacc[cb][1][2]);
      t = fmaxf(t, sacc[cb][1][3]);
      const float tmax = rows4_max(t) * scale_log2;
      if (__ballot(tmax > st.m[cb] + kRescaleLog2) == 0) continue;
      const float m_new = fmaxf(st.m[cb], tmax);
      const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(st.m[cb] - m_ref);
      st.m[cb] = m_new;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
        for (int r = 0; r < 4; ++r) st.o[cb][jj][r] *= alpha;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) st.l[cb][r] *= alpha;
      if constexpr (kPLo) {
#pragma unroll
        for (int r = 0; r < 4; ++r) plo[cb][r] *= alpha;
      }
    }
    exp_all(sacc, pr);
  }
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
#pragma unroll
    for (int w = 0; w < 4; ++w) pb[cb][w] = pack_bf16x2_fast(pr[cb][2 * w], pr[cb][2 * w + 1]);
    if constexpr (kPLo) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pl[cb][w] = pack_bf16x2_fast(pr[cb][2 * w] - bf16_bits_to_f32(pb[cb][w] & 0xffffu),
                                     pr[cb][2 * w + 1] - bf16_bits_to_f32(pb[cb][w] >> 16));
    }
  }
}

// O^T += V^T P^T and the column sums of P.  va[jj]: V^T operand of PV MFMA jj.
__device__ __forceinline__ void pf_pv(PfState& st, const u32x4_t (&va)[8],
                                      const u32x4_t (&pb)[kPreNCB]) {
  const u32x4_t ones = u32x4_t{kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
#pragma unroll
  for (int cb = 0; cb < kPreNCB; ++cb) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) st.o[cb][jj] = mfma_bf16(va[jj], pb[cb], st.o[cb][jj]);
    st.l[cb] = mfma_bf16(ones, pb[cb], st.l[cb]);
  }
}

// ---------------------------------------------------------------------------
// Stream-K prefill over bf16 keys (prefill_sk2_kernel), with a lean tile
// loop:
//  * each wave stages its own 32 query columns in a private LDS region by
//    direct-to-LDS loads and reads them back after its own vmcnt wait, so a
//    query reload needs no workgroup barrier.  The next segment's query is
//    loaded as soon as the current one is in registers;
//  * every vector memory operation a wave issues is counted (tile loads,
//    query loads and the epilogue stores, which are buffer stores issued
//    unconditionally with out-of-range offsets for the lanes that do not
//    write): vector memory operations complete in issue order, so a wait for
//    tile j is vmcnt(operations issued after tile j) exactly, and an epilogue
//    never holds the next tile's wait;
//  * the steady state waits with one immediate.
// ---------------------------------------------------------------------------
constexpr int kP2Stages = 4;
constexpr int kP2QSlots = kPreNCB * 16 * kPfRowSlots;       // 32 columns x 17 slots
constexpr int kP2QLoads = (kP2QSlots + 63) / 64;            // 9 per wave
constexpr int kP2QRegion = kP2QLoads * 1024;
constexpr int kP2QOff = kP2Stages * kPfStage;
constexpr int kP2DummyOff = kP2QOff + kWaves * kP2QRegion;
constexpr int kP2Smem = kP2DummyOff + 1024;
constexpr int kP2StoresFinal = kPreNCB * 4;   // bf16 rows: 4 x 16 B a lane per column block
constexpr int kP2StoresPart = kPreNCB * 5;    // fp16 partials: 4 x 16 B + (lse, exponent)
constexpr int kP2Steady = kPfTileLoads * (kP2Stages - 2);   // loads after the next tile's
static_assert(kP2Smem <= 160 * 1024, "one workgroup per CU");
static_assert(kPfTileLoads * (kP2Stages - 1) + kP2QLoads + kP2StoresPart + 1 <= 47,
              "every pending count is below the clamp of vm_wait");

template <int N>
__device__ __forceinline__ void vm_wait_const() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <int LO, int HI>
__device__ __forceinline__ void vm_wait_range(int n) {
  if constexpr (LO == HI) {
    vm_wait_const<LO>();
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID) {
      vm_wait_range<LO, MID>(n);
    } else {
      vm_wait_range<MID + 1, HI>(n);
    }
  }
}

// Wait until at most n of this wave's vector memory operations are pending
// (n >= 0 and wave-uniform; values above 47 wait for 47, more than needed,
// which is safe).
__device__ __forceinline__ void vm_wait(int n) { vm_wait_range<0, 47>(uniform(n)); }

// Chunk geometry of the first 64 chunks, kept in LDS by the stream-K prefill
// launch (sq, sk, first query row, first key row): an item change then costs
// an LDS read instead of a chain of scalar loads.
__device__ __forceinline__ void p2_load_chunk(PfItem& it, const int4* ctab, const int32_t* cu_q,
                                              const int32_t* cu_k, int qtile) {
  if (it.i < 64) {
    const int4 e = ctab[it.i];
    it.geo.sq = uniform(e.x);
    it.geo.sk = uniform(e.y);
    it.geo.prefix = it.geo.sk - it.geo.sq;
    it.geo.ntq = (it.geo.sq > 0 && it.geo.sk > 0) ? (it.geo.sq + qtile - 1) / qtile : 0;
    it.cq0 = uniform(e.z);
    it.ck0 = uniform(e.w);
  } else {
    pf_load_chunk(it, cu_q, cu_k, qtile);
  }
}

// Virtual tiles per item in the partition of prefill_sk2_kernel: an item
// change (its query, its epilogue, the first step of the next segment, the
// general steps of its masked tiles) costs several tiles' time; 6 balanced
// the shares best on mixed chunk lengths (3, 5, 6 and 8 measured).
#ifndef KVC_P2_ITEM_COST
#define KVC_P2_ITEM_COST 6
#endif
constexpr int kP2ItemCost = KVC_P2_ITEM_COST;

// Weighted tiles of query tiles [0, q) of chunk c.
__device__ __forceinline__ int p2_qcum(const ChunkGeo& c, int tpb, int q) {
  return int(qtile_cum(c, tpb, q)) + kP2ItemCost * q;
}

// The item after `it` (T = 0 past the last one), chunks read from the table.
__device__ __forceinline__ void p2_next_item(PfItem& it, const int4* ctab, const int32_t* cu_q,
                                             const int32_t* cu_k, int n_pre, int kvs_total,
                                             int nslices, int qtile) {
  it.P += kP2ItemCost + it.T;
  if (++it.qt == it.geo.ntq) {
    it.qt = 0;
    ++it.kvs;
    if (++it.s == nslices) {
      it.s = 0;
      ++it.g;
    }
    if (it.kvs == kvs_total) {
      it.kvs = it.g = it.s = 0;
      do {
        ++it.i;
        if (it.i < n_pre) p2_load_chunk(it, ctab, cu_q, cu_k, qtile);
      } while (it.i < n_pre && it.geo.ntq == 0);
    }
  }
  it.T = it.i < n_pre ? qtile_tiles(it.geo, qtile, it.qt) : 0;
}

// One workgroup's share (workgroup v of G) of a stream-K prefill launch;
// lds holds the ring, the query regions and the dummy block (kP2Smem bytes),
// ctab the first 64 chunks' geometry.
// kPLo (fresh rows gathered from a per-channel int8 pool, p.head_n_out set):
// the outlier dims' PV and the column sums also take the rounding residue of
// the bf16 P operand (one MFMA per column block and tile: rows j < n_plo read
// the V stage at slot j's dim, row 15 is ones), added in at the segment end.
template <bool kFresh, bool kPLo = false>
__device__ __forceinline__ void prefill_sk2_share(const AttnParams& p,
                                                  const int32_t* __restrict__ cu_q,
                                                  const int32_t* __restrict__ cu_k,
                                                  const int32_t* __restrict__ block_tables,
                                                  const int v, const int G, char* lds,
                                                  int4* ctab) {
  const unsigned long long t_start =
      p.wg_stamps != nullptr ? __builtin_amdgcn_s_memrealtime() : 0ull;
  auto stamp = [&]() {  // diagnostics: this workgroup's start and end
    if (p.wg_stamps != nullptr && threadIdx.x == 0) {
      p.wg_stamps[2 * v] = t_start;
      p.wg_stamps[2 * v + 1] = __builtin_amdgcn_s_memrealtime();
    }
  };
  const LaneId L = lane_id();
  const int wave = uniform(int(threadIdx.x >> 6));
  const int kvs_total = p.kvh * p.nslices;
  const int qtile = kWaves * kPreNCB * p.tpb;
  // Consecutive shares run on one XCD (workgroup v is placed on XCD v mod 8).
  const int w = (G % 8 == 0) ? (v % 8) * (G / 8) + v / 8 : v;

  // Weighted total W and the longest item; shares of S.
  int W = 0, Tmax = 0;
  int t_first = 0;
  int cq_first = 0, ck_first = 0;
  ChunkGeo g_first{0, 0, 0, 0};
  for (int c0 = 0; c0 < p.n_pre; c0 += 64) {
    const int ci = c0 + L.lane;
    int t = 0, tm = 0;
    if (ci < p.n_pre) {
      const ChunkGeo c = chunk_geo(cu_q, cu_k, ci, qtile);
      if (c.ntq > 0) {
        tm = (c.sk + kTile - 1) / kTile;
        t = kvs_total * p2_qcum(c, p.tpb, c.ntq);
      }
      if (c0 == 0) {
        g_first = c;
        cq_first = cu_q[ci];
        ck_first = cu_k[ci];
        ctab[L.lane] = int4{c.sq, c.sk, cq_first, ck_first};  // every wave writes the same
      }
    }
    if (c0 == 0) t_first = t;
    W += wave_sum(t);
    Tmax = max(Tmax, wave_max(tm));
  }
  W = uniform(W);
  Tmax = uniform(Tmax);
  int S = max(p.sk_min_share, (W + G - 1) / G);
  if (p.max_splits > 1) S = max(S, (Tmax + kP2ItemCost + p.max_splits - 2) / (p.max_splits - 1));
  S = uniform(S);
  if (int64_t(w) * S >= W) {
    stamp();
    return;
  }
  const int start = w * S;
  const int end = min(W, start + S);

  // The item whose weighted span holds `start`.
  PfItem it;
  {
    int base = 0, ci = -1, P = 0;
    for (int c0 = 0; c0 < p.n_pre && ci < 0; c0 += 64) {
      int t = t_first;
      if (c0 > 0) {
        t = 0;
        if (c0 + L.lane < p.n_pre) {
          const ChunkGeo c = chunk_geo(cu_q, cu_k, c0 + L.lane, qtile);
          if (c.ntq > 0) t = kvs_total * p2_qcum(c, p.tpb, c.ntq);
        }
      }
      const int inc = wave_scan_add(t);
      const int total = uniform(__builtin_amdgcn_readlane(inc, 63));
      if (start < base + total) {
        const unsigned long long hit =
            __ballot(t > 0 && base + inc - t <= start && start < base + inc);
        const int src = __ffsll(hit) - 1;
        ci = uniform(c0 + src);
        P = uniform(base + __builtin_amdgcn_readlane(inc - t, src));
        if (c0 == 0) {
          it.geo.sq = uniform(__builtin_amdgcn_readlane(g_first.sq, src));
          it.geo.sk = uniform(__builtin_amdgcn_readlane(g_first.sk, src));
          it.geo.prefix = it.geo.sk - it.geo.sq;
          it.geo.ntq = uniform(__builtin_amdgcn_readlane(g_first.ntq, src));
          it.cq0 = uniform(__builtin_amdgcn_readlane(cq_first, src));
          it.ck0 = uniform(__builtin_amdgcn_readlane(ck_first, src));
        }
      }
      base += total;
    }
    it.i = ci;
    if (ci >= 64) pf_load_chunk(it, cu_q, cu_k, qtile);
    const int per_kvs = p2_qcum(it.geo, p.tpb, it.geo.ntq);
    int off = start - P;
    it.kvs = uniform(off / per_kvs);
    off -= it.kvs * per_kvs;
    int lo = 0, hi = it.geo.ntq - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p2_qcum(it.geo, p.tpb, mid) <= off) lo = mid; else hi = mid - 1;
    }
    it.qt = uniform(lo);
    it.g = uniform(it.kvs / p.nslices);
    it.s = it.kvs - it.g * p.nslices;
    it.P = uniform(P + it.kvs * per_kvs + p2_qcum(it.geo, p.tpb, it.qt));
    it.T = qtile_tiles(it.geo, qtile, it.qt);
  }
  int ct = max(0, start - it.P - kP2ItemCost);  // consumer's tile in `it`

  // Tile loads: wave w issues loads w, w + 8, w + 16 of the 18 per tile (9 of
  // K, 9 of V; the six past 18 are zero loads into a dummy block).
  const uint32_t lds0 = lds_addr(lds);
  int boff[kPfTileLoads];
#pragma unroll
  for (int jj = 0; jj < kPfTileLoads; ++jj) {
    const int k = wave + kWaves * jj;
    const int sl = (k % kPfLoadsPerTensor) * 64 + L.lane;
    const int slots = k < kPfLoadsPerTensor ? kPfRowSlots : kPfVRowSlots;
    const int row = sl / slots;
    const int ch = sl - row * slots;
    int rs;
    if constexpr (kFresh) {
      rs = int((k >= kPfLoadsPerTensor ? p.vf_st : p.kf_st) * 2);
    } else {
      rs = int(p.tok_bytes);
    }
    const bool ok = k < 2 * kPfLoadsPerTensor && row < kTile && ch < 16;
    boff[jj] = ok ? row * rs + ch * 16 : kOob;
  }
  static_assert(kWaves == 8 && kPfLoadsPerTensor == 9 && kPfTileLoads == 3,
                "the load pattern below");
  const bool w0 = wave == 0;
  const bool w01 = wave < 2;
  const uint32_t dst0 = uint32_t(wave) * 1024;
  const uint32_t dst1 = w0 ? 8 * 1024 : kPfTensor + uint32_t(wave - 1) * 1024;
  const uint32_t dst2 = kPfTensor + uint32_t(7 + wave) * 1024;

  // Producer cursor: the item and tile whose loads are issued next, running
  // ahead of the consumer (it, ct) by the ring depth.
  PfItem pi = it;
  int pt = ct;
  int pblk = 0, poff = 0, pblk_val = 0, pnext_val = 0, plast = 0;
  int64_t pbt = 0;
  auto table_setup = [&]() {
    if constexpr (!kFresh) {
      pbt = int64_t(p.n_dec + pi.i) * p.bt_stride;
      const int key0 = pt * kTile;
      pblk = uniform(key0 / p.page);
      poff = uniform(key0 - pblk * p.page);
      plast = uniform((pi.geo.sk - 1) / p.page);
      pblk_val = block_tables[pbt + pblk];
      pnext_val = block_tables[pbt + min(pblk + 1, plast)];
    }
  };
  table_setup();
  int issued = 0;  // vector memory operations this wave has issued
  auto produce = [&](int stage) {
    const int nvalid = min(kTile, pi.geo.sk - pt * kTile);
    int hk, hv;
    const char* kb;
    const char* vb;
    int kbytes, vbytes;
    if constexpr (kFresh) {
      hk = int(pi.g * p.kf_sh * 2);
      hv = int(pi.g * p.vf_sh * 2);
      const int64_t r0 = int64_t(pi.ck0) + pt * kTile;
      kb = reinterpret_cast<const char*>(p.kf + r0 * p.kf_st);
      vb = reinterpret_cast<const char*>(p.vf + r0 * p.vf_st);
      kbytes = int(nvalid * p.kf_st * 2);
      vbytes = int(nvalid * p.vf_st * 2);
    } else {
      hk = hv = pi.g * kD * 2;
      const int64_t slot0 = int64_t(pblk_val) * p.page + poff;
      kb = p.k_cache + slot0 * p.tok_bytes;
      vb = p.v_cache + slot0 * p.tok_bytes;
      kbytes = vbytes = nvalid * int(p.tok_bytes);
    }
    const i32x4_t rk = raw_rsrc(kb, kbytes);
    const i32x4_t rv = raw_rsrc(vb, vbytes);
    const uint32_t sb = lds0 + stage * kPfStage;
    dma_to_lds_cached(rk, boff[0] + hk, sb + dst0);
    dma_to_lds_cached(w0 ? rk : rv, boff[1] + (w0 ? hk : hv), sb + dst1);
    dma_to_lds_cached(rv, boff[2] + hv, w01 ? sb + dst2 : lds0 + kP2DummyOff);
    issued += kPfTileLoads;
    if (++pt == pi.T) {
      p2_next_item(pi, ctab, cu_q, cu_k, p.n_pre, kvs_total, p.nslices, qtile);
      pt = 0;
      if (pi.P + kP2ItemCost < end) table_setup();
    } else if constexpr (!kFresh) {
      poff += kTile;
      if (poff == p.page) {
        poff = 0;
        ++pblk;
        pblk_val = pnext_val;
        pnext_val = block_tables[pbt + min(pblk + 1, plast)];
      }
    }
  };
  auto prod_live = [&]() { return pi.P + kP2ItemCost + pt < end; };

  // This wave's query columns of item x into its LDS region: column c
  // (0..31: block c / 16, lane c % 16) at slots 17 c .. 17 c + 15; columns
  // past the chunk or the slice read 0.
  const uint32_t qreg = lds0 + kP2QOff + uint32_t(wave) * kP2QRegion;
  const char* qreg_p = lds + kP2QOff + wave * kP2QRegion;
  const float inv_hs = 1.f / float(p.hs);
  auto issue_q = [&](const PfItem& x) {
    const int hs = min(p.hs, p.group - x.s * p.hs);
    const int q0 = x.qt * qtile + wave * kPreNCB * p.tpb;  // this wave's first query row
    const int rows = max(0, min(kPreNCB * p.tpb, x.geo.sq - q0));
    const uint16_t* qb = p.q + (int64_t(p.n_dec) + x.cq0 + q0) * p.q_st;
    const i32x4_t rq = raw_rsrc(qb, int(rows * p.q_st * 2));
    const int hbase = x.g * p.group + x.s * p.hs;
#pragma unroll
    for (int k = 0; k < kP2QLoads; ++k) {
      const int sl = k * 64 + L.lane;
      const int col = sl / kPfRowSlots;
      const int ch = sl - col * kPfRowSlots;
      const int lm = col & 15;
      const int tdiv = int((float(lm) + 0.5f) * inv_hs);  // lm / hs (lm < 16)
      const int hh = lm - tdiv * p.hs;
      const int tq = (col >> 4) * p.tpb + tdiv;  // row past q0
      const bool ok = col < 32 && ch < 16 && lm < p.tpb * p.hs && hh < hs && tq < rows;
      const int off =
          ok ? int((int64_t(tq) * p.q_st + int64_t(hbase + hh) * p.q_sh) * 2) + ch * 16 : kOob;
      dma_to_lds_cached(rq, off, qreg + k * 1024);
    }
    issued += kP2QLoads;
  };

  // Prologue: this wave's first query, then the first kP2Stages - 1 tiles.
  // tmk[k]: `issued` right after the loads of tile j + k, j being the tile
  // the next step attends; q_mark: right after the latest query loads.
  issue_q(it);
  int q_mark = issued;
  int q_for = it.P;  // item (by its span start) whose query is in the region
  int tmk[kP2Stages - 1];
#pragma unroll
  for (int k = 0; k < kP2Stages - 1; ++k) {
    if (prod_live()) produce(k);
    tmk[k] = issued;
  }

  QOps<kBF16, kPreNCB> Q;
  // The query of the item in the region into registers (once its loads have
  // landed), and the query of the item after `it` into the region (once the
  // region's reads are back).
  auto read_q = [&]() {
    vm_wait(issued - q_mark);
#pragma unroll
    for (int cb = 0; cb < kPreNCB; ++cb) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        Q.op[cb][c] = *reinterpret_cast<const u32x4_t*>(qreg_p + (cb * 16 + L.lm) * kPfPitch +
                                                        c * 64 + L.lg * 16);
    }
  };
  auto issue_next_q = [&]() {
    const int nP = it.P + kP2ItemCost + it.T;  // span start of the item after `it`
    if (nP + kP2ItemCost < end) {
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      PfItem nx = it;
      p2_next_item(nx, ctab, cu_q, cu_k, p.n_pre, kvs_total, p.nslices, qtile);
      issue_q(nx);
      q_mark = issued;
      q_for = nP;
    }
  };
  read_q();
  issue_next_q();

  PfState st;
  f32x4_t plo[kPreNCB];
  u32x4_t pl[kPreNCB];
  int n_plo = 0, plo_dim = 0;  // (kPLo) the item's slots, the dim of slot lm
  // (kPLo) residue operand rows: lanes lm < n_plo keep the V values, lane
  // row 15 is ones, the rest 0
  const uint32_t plo_one = L.lm == 15 ? kOnesBf16x2 : 0u;
  uint32_t plo_keep = 0u;
  int klim[kPreNCB];
  int min_klim = 0, split = -1, nrows = 0;
  int stage = 0;  // stage of the tile the next step attends
  bool first = true;
  __amdgpu_buffer_rsrc_t ro = tile_rsrc(p.out, 0);
  __amdgpu_buffer_rsrc_t rl = tile_rsrc(p.out, 0);

  // K operands (lane (lm, lg): key lm, + 16 for the second half, dims
  // 32 c + 8 lg .. + 7) and V^T operands (transposing reads: PV MFMA jj row m
  // is dim 16 jj + m) of the tile in stage stg.
  auto read_k = [&](int stg, u32x4_t (&kop)[2][4]) {
    const char* kb = lds + stg * kPfStage + L.lm * kPfPitch + L.lg * 16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kop[h][c] = *reinterpret_cast<const u32x4_t*>(kb + h * 16 * kPfPitch + c * 64);
    }
  };
  auto read_v = [&](int stg, u32x4_t (&va)[8]) {
    const char* vb =
        lds + stg * kPfStage + kPfTensor + (4 * L.lg + (L.lm >> 2)) * kPfPitchV + (L.lm & 3) * 8;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const u32x2_t lo = lds_read_tr16(vb + jj * 32);
      const u32x2_t hi = lds_read_tr16(vb + 16 * kPfPitchV + jj * 32);
      va[jj] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
    }
  };

  // (kPLo) the residue product of the tile in stage stg (branch-free, so
  // that its LDS reads schedule with the tile's own).
  auto residue = [&](int stg) {
    if constexpr (kPLo) {
      const char* vb = lds + stg * kPfStage + kPfTensor + 2 * plo_dim;
      uint32_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        e[i] = *reinterpret_cast<const uint16_t*>(vb + key_of_slot(L.lg, i) * kPfPitchV);
      u32x4_t op;
#pragma unroll
      for (int w = 0; w < 4; ++w) op[w] = ((e[2 * w] | (e[2 * w + 1] << 16)) & plo_keep) | plo_one;
#pragma unroll
      for (int cb = 0; cb < kPreNCB; ++cb) plo[cb] = mfma_bf16(op, pl[cb], plo[cb]);
    }
  };

  // Fast producer step: a full tile inside the producer's item.  Its K/V
  // addresses advance by one tile per step (kcur, vcur include the kv head's
  // offset); a page boundary reloads them from the prefetched table entry.
  const char* kcur = nullptr;
  const char* vcur = nullptr;
  int64_t kstep = 0, vstep = 0;
  auto fast_setup = [&]() {
    if constexpr (kFresh) {
      const int64_t r0 = int64_t(pi.ck0) + pt * kTile;
      kcur = reinterpret_cast<const char*>(p.kf + r0 * p.kf_st + pi.g * p.kf_sh);
      vcur = reinterpret_cast<const char*>(p.vf + r0 * p.vf_st + pi.g * p.vf_sh);
      kstep = int64_t(kTile) * p.kf_st * 2;
      vstep = int64_t(kTile) * p.vf_st * 2;
    } else {
      const int64_t off = (int64_t(pblk_val) * p.page + poff) * p.tok_bytes + pi.g * kD * 2;
      kcur = p.k_cache + off;
      vcur = p.v_cache + off;
      kstep = vstep = int64_t(kTile) * p.tok_bytes;
    }
  };
  auto produce_fast = [&](int stg) {
    const i32x4_t rk = raw_rsrc(kcur, int(kstep));
    const i32x4_t rv = raw_rsrc(vcur, int(vstep));
    const uint32_t sb = lds0 + stg * kPfStage;
    dma_to_lds_cached(rk, boff[0], sb + dst0);
    dma_to_lds_cached(w0 ? rk : rv, boff[1], sb + dst1);
    dma_to_lds_cached(rv, boff[2], w01 ? sb + dst2 : lds0 + kP2DummyOff);
    issued += kPfTileLoads;
    ++pt;
    kcur += kstep;
    vcur += vstep;
    if constexpr (!kFresh) {
      poff += kTile;
      if (poff == p.page) {
        poff = 0;
        ++pblk;
        pblk_val = pnext_val;
        pnext_val = block_tables[pbt + min(pblk + 1, plast)];
        const int64_t off = int64_t(pblk_val) * p.page * p.tok_bytes + pi.g * kD * 2;
        kcur = p.k_cache + off;
        vcur = p.v_cache + off;
      }
    }
  };

  // Top of a step: the tile it attends has landed for every wave and every
  // wave is done with the previous tile's stage, which then receives the tile
  // kP2Stages - 1 ahead.
  auto step_top = [&](bool fast) {
    const int n = issued - tmk[0];
    if (n == kP2Steady) {
      vm_wait_const<kP2Steady>();
    } else {
      vm_wait(n);
    }
    pf_barrier();
    const int free_stage = stage == 0 ? kP2Stages - 1 : stage - 1;
    if (fast) {
      produce_fast(free_stage);
    } else if (prod_live()) {
      produce(free_stage);
    }
#pragma unroll
    for (int k = 0; k + 1 < kP2Stages - 1; ++k) tmk[k] = tmk[k + 1];
    tmk[kP2Stages - 2] = issued;
  };

  // Fast steps available from the current state: consumer tiles ct, ct + 1,
  // ... that are unmasked and not the last of their segment; producer steps
  // inside its item and the share.
  auto run_length = [&]() {
    const int mk = uniform(min_klim);
    const int unmasked = min(it.geo.sk >> 5, mk >= kTile - 1 ? ((mk - (kTile - 1)) >> 5) + 1 : 0);
    const int r1 = min(min(it.T - 1, unmasked), end - 1 - (it.P + kP2ItemCost)) - ct;
    const int r2 = min(pi.T - 1 - pt, end - (pi.P + kP2ItemCost + pt));
    return uniform(max(0, min(r1, r2)));
  };

  while (it.P + kP2ItemCost + ct < end) {
    if (!first && ct != 0) {
      const int R = run_length();
      if (R > 0) {
        fast_setup();
        for (int r = 0; r < R; ++r) {
          step_top(true);
          u32x4_t pb[kPreNCB];
          {
            u32x4_t kop[2][4];
            read_k(stage, kop);
            pf_score_fast<kPLo>(st, kop, Q, p.scale_log2, pb, plo, pl);
          }
          u32x4_t va[8];
          read_v(stage, va);
          pf_pv(st, va, pb);
          residue(stage);
          ++ct;
          stage = stage == kP2Stages - 1 ? 0 : stage + 1;
        }
      }
    }
    // General step.
    const bool seg_start = first || ct == 0;
    const bool seg_end = ct + 1 == it.T || it.P + kP2ItemCost + ct + 1 >= end;
    first = false;
    step_top(false);
    const int q0 = it.qt * qtile;
    if (seg_start) {
      const int hs = min(p.hs, p.group - it.s * p.hs);
      const int prefix = it.geo.sk - it.geo.sq;
#pragma unroll
      for (int cb = 0; cb < kPreNCB; ++cb) {
        const int tq = q0 + (wave * kPreNCB + cb) * p.tpb + L.lm / p.hs;
        const int hh = L.lm % p.hs;
        const bool ok = (L.lm < p.tpb * p.hs) && hh < hs && tq < it.geo.sq;
        klim[cb] = ok ? prefix + tq : -1;
      }
      // The wave's smallest key limit is lane 0's first column's (the wave's
      // first query row); when that column does not exist, no column does.
      {
        const int k0 = __shfl(klim[0], 0, 64);
        min_klim = k0 >= 0 ? k0 : 0x7fffffff;
      }
      pf_init(st);
      if constexpr (kPLo) {
#pragma unroll
        for (int cb = 0; cb < kPreNCB; ++cb) plo[cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        n_plo = p.head_n_out != nullptr ? min(table_entry(p.head_n_out, it.g), p.n_out_max) : 0;
        int dsel = 0;
#pragma unroll
        for (int j = 0; j < kSideMax; ++j) {
          if (j < n_plo) {
            const int d = table_entry(p.out_idx, int64_t(it.g) * p.n_out_max + j) & (kD - 1);
            dsel = L.lm == j ? d : dsel;
          }
        }
        plo_dim = dsel;
        plo_keep = L.lm < n_plo ? 0xffffffffu : 0u;
      }
      const int f = (it.P + kP2ItemCost) / S;
      const int nseg = (it.P + kP2ItemCost + it.T - 1) / S - f + 1;
      split = nseg == 1 ? -1 : w - f;
      nrows = min(qtile, it.geo.sq - q0);
      const int64_t row0 = int64_t(p.n_dec) + it.cq0 + q0;
      if (split < 0) {
        ro = tile_rsrc(p.out + row0 * p.o_st, int(int64_t(nrows) * p.o_st * 2));
      } else {
        const int64_t per_row = int64_t(p.num_heads) * p.max_splits;
        ro = tile_rsrc(reinterpret_cast<const uint16_t*>(p.part_o) + row0 * per_row * kD,
                       int(nrows * per_row * kD * 2));
        rl = tile_rsrc(p.part_ml + row0 * per_row, int(nrows * per_row * 8));
      }
      if (f == w && p.sk_nseg != nullptr && 64 * wave < nrows) {
        // Split counts of the item's rows (one per row and kv slice).
        const __amdgpu_buffer_rsrc_t rn =
            tile_rsrc(p.sk_nseg + row0 * kvs_total, int(nrows * kvs_total * 4));
        const int t = int(threadIdx.x);
        const int off = t < nrows ? (t * kvs_total + it.kvs) * 4 : kOob;
        __builtin_amdgcn_raw_buffer_store_b32(uint32_t(nseg), rn, off, 0, 0);
        ++issued;
      }
    }
    const int key0 = ct * kTile;
    u32x4_t pb[kPreNCB];
    {
      u32x4_t kop[2][4];
      read_k(stage, kop);
      if (key0 + kTile <= it.geo.sk && key0 + kTile - 1 <= min_klim) {
        pf_score<false, kPLo>(st, kop, Q, klim, key0, it.geo.sk, p.scale_log2, L, pb, plo, pl);
      } else {
        pf_score<true, kPLo>(st, kop, Q, klim, key0, it.geo.sk, p.scale_log2, L, pb, plo, pl);
      }
    }
    {
      u32x4_t va[8];
      read_v(stage, va);
      pf_pv(st, va, pb);
      residue(stage);
    }
    stage = stage == kP2Stages - 1 ? 0 : stage + 1;
    // Segment end: every lane's dims (16 jj + 4 lg .. + 3 of its column), as
    // unconditional buffer stores (lanes of columns that do not exist store
    // out of range).  bf16 rows: lanes lg and lg ^ 1 swap halves first
    // (v_permlane16_swap), so each lane stores 16 contiguous bytes and each
    // row gets 64-byte pieces.
    const bool next_in = ct + 1 == it.T && it.P + 2 * kP2ItemCost + it.T < end;
    if (next_in) {
      // The next item's query into registers (the query registers are dead
      // after this tile's S^T) and the one after into the region, ahead of the
      // stores, so those loads do not queue behind them.
      const PfItem cur = it;
      p2_next_item(it, ctab, cu_q, cu_k, p.n_pre, kvs_total, p.nslices, qtile);
      if (q_for != it.P) {  // defensive: its query is normally issued one item ahead
        issue_q(it);
        q_mark = issued;
        q_for = it.P;
      }
      read_q();
      issue_next_q();
      it = cur;
    }
    if (seg_end) {
      const int hs = min(p.hs, p.group - it.s * p.hs);
      const int hbase = it.g * p.group + it.s * p.hs;
      float lres[kPreNCB] = {};
      if constexpr (kPLo) {
        {
          // Residue row j (lane lm + 16 (j >> 2), element j & 3) joins O at
          // slot j's dim d (lane group (d >> 2) & 3, chunk d >> 4, row d & 3;
          // a dim listed twice took the later slot's value, so only that
          // slot's residue counts); row 15 joins the column sum.
#pragma unroll
          for (int cb = 0; cb < kPreNCB; ++cb) {
            lres[cb] = __shfl(plo[cb][3], L.lm + 48, 64);
            for (int j = 0; j < n_plo; ++j) {
              const int d = table_entry(p.out_idx, int64_t(it.g) * p.n_out_max + j) & (kD - 1);
              bool later = false;
              for (int j2 = j + 1; j2 < n_plo; ++j2)
                later |= (table_entry(p.out_idx, int64_t(it.g) * p.n_out_max + j2) & (kD - 1)) == d;
              if (later) continue;
              const int e = j & 3;
              const f32x4_t c = plo[cb];
              const float mine = e == 0 ? c[0] : e == 1 ? c[1] : e == 2 ? c[2] : c[3];
              const float val = __shfl(mine, L.lm + 16 * (j >> 2), 64);
              if (L.lg == ((d >> 2) & 3)) {
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                  for (int r = 0; r < 4; ++r)
                    if (jj == (d >> 4) && r == (d & 3)) st.o[cb][jj][r] += val;
              }
            }
          }
        }
      }
#pragma unroll
      for (int cb = 0; cb < kPreNCB; ++cb) {
        const int tr = (wave * kPreNCB + cb) * p.tpb + L.lm / p.hs;  // row in the query tile
        const int hh = L.lm % p.hs;
        const bool ok = (L.lm < p.tpb * p.hs) && hh < hs && tr < nrows;
        const float l = st.l[cb][0] + lres[cb];
        if (split < 0) {
          const float inv = 1.f / l;
          // Even rows of lanes (lg even) keep jj = 2t, odd rows jj = 2t + 1.
          const int base = ok ? int((int64_t(tr) * p.o_st + int64_t(hbase + hh) * p.o_sh) * 2) +
                                    32 * (L.lg & 1) + 16 * (L.lg >> 1)
                              : kOob;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t a0 = pack_bf16x2_fast(st.o[cb][2 * t][0] * inv, st.o[cb][2 * t][1] * inv);
            const uint32_t a1 = pack_bf16x2_fast(st.o[cb][2 * t][2] * inv, st.o[cb][2 * t][3] * inv);
            const uint32_t b0 =
                pack_bf16x2_fast(st.o[cb][2 * t + 1][0] * inv, st.o[cb][2 * t + 1][1] * inv);
            const uint32_t b1 =
                pack_bf16x2_fast(st.o[cb][2 * t + 1][2] * inv, st.o[cb][2 * t + 1][3] * inv);
            const auto x0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
            const auto x1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
            // Lane lg even: its own 4 dims then lane lg + 1's (jj = 2t); lane lg
            // odd: lane lg - 1's 4 dims then its own (jj = 2t + 1).
            const u32x4_t val = u32x4_t{x0[0], x1[0], x0[1], x1[1]};
            __builtin_amdgcn_raw_buffer_store_b128(val, ro, base + 64 * t, 0, 0);
          }
        } else {
          // Normalised partial row in fp16 (half the bytes of fp32 both
          // ways), scaled by 2^-ex: ex = 0 unless the row's largest |value|
          // reaches 2^15, then the smallest that keeps it below; the merge
          // takes ex from the (lse, ex) pair.  Same lane swap and 16-byte
          // pieces as the bf16 rows.
          const int idx = (tr * p.num_heads + hbase + hh) * p.max_splits + split;
          const float il = l > 0.f ? 1.f / l : 0.f;
          float amax = 0.f;
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) amax = fmaxf(amax, fabsf(st.o[cb][jj][r]));
          amax = rows4_max(amax) * il;
          const int ex = amax >= 32768.f ? ((__float_as_int(amax) >> 23) & 0xff) - 127 - 14 : 0;
          const float sc = ldexpf(il, -ex);
          const int base = ok ? idx * (kD * 2) + 32 * (L.lg & 1) + 16 * (L.lg >> 1) : kOob;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t a0 = pack_f16x2(st.o[cb][2 * t][0] * sc, st.o[cb][2 * t][1] * sc);
            const uint32_t a1 = pack_f16x2(st.o[cb][2 * t][2] * sc, st.o[cb][2 * t][3] * sc);
            const uint32_t b0 = pack_f16x2(st.o[cb][2 * t + 1][0] * sc, st.o[cb][2 * t + 1][1] * sc);
            const uint32_t b1 = pack_f16x2(st.o[cb][2 * t + 1][2] * sc, st.o[cb][2 * t + 1][3] * sc);
            const auto x0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
            const auto x1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
            const u32x4_t val = u32x4_t{x0[0], x1[0], x0[1], x1[1]};
            __builtin_amdgcn_raw_buffer_store_b128(val, ro, base + 64 * t, 0, 0);
          }
          const float lse = l > 0.f ? st.m[cb] + __log2f(l) : -INFINITY;
          __builtin_amdgcn_raw_buffer_store_b64(
              u32x2_t{__float_as_uint(lse), __float_as_uint(float(ex))}, rl,
              (ok && L.lg == 0) ? idx * 8 : kOob, 0, 0);
        }
      }
      issued += split < 0 ? kP2StoresFinal : kP2StoresPart;
    }
    if (++ct == it.T) {
      // The next item, if one of its real tiles is in this share.
      if (it.P + 2 * kP2ItemCost + it.T >= end) break;
      p2_next_item(it, ctab, cu_q, cu_k, p.n_pre, kvs_total, p.nslices, qtile);
      ct = 0;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (p.wg_stamps != nullptr) {
    __syncthreads();  // every wave has issued its last stores
    stamp();
  }

}

template <bool kFresh, bool kPLo = false>
__global__ void __launch_bounds__(kThreads)
prefill_sk2_kernel(AttnParams p, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                   const int32_t* __restrict__ block_tables) {
  __shared__ __align__(16) char lds[kP2Smem];
  __shared__ int4 ctab[64];
  touch_kernel_args(int(sizeof(AttnParams) + 3 * sizeof(void*)));
  prefill_sk2_share<kFresh, kPLo>(p, cu_q, cu_k, block_tables, int(blockIdx.x), int(gridDim.x), lds,
                            ctab);
}

// A mixed call's decode rows and prefill rows in one launch over a static
// CU split: workgroups [0, dec_wgs) run the stream-K decode over dec_wgs
// shares (bf16 pool, LDS-staged), the others the stream-K prefill over the
// rest.  dec_wgs is a multiple of 8, so both sides keep their XCD placement
// (workgroup b runs on XCD b mod 8).  Each side plans, and is merged, as its
// own launch would be.
constexpr int kMixSplitLds = 2 * kLdsStage + kLdsQ;
static_assert(kMixSplitLds >= kP2Smem + 64 * int(sizeof(int4)), "one LDS block serves both sides");
__global__ void __launch_bounds__(kThreads)
mixed_split_kernel(AttnParams pd, AttnParams pp, int dec_wgs) {
  __shared__ __align__(16) char lds[kMixSplitLds];
  touch_kernel_args(int(2 * sizeof(AttnParams) + sizeof(int)));
  const int b = int(blockIdx.x);
  if (b < dec_wgs) {
    decode_sk_share<kBF16, true>(pd, pd.block_tables, pd.ctx_lens, b, dec_wgs, lds,
                                 lds + kLdsStage, lds + 2 * kLdsStage, StealArgs{});
  } else {
    prefill_sk2_share<false>(pp, pp.cu_q, pp.cu_k, pp.block_tables, b - dec_wgs,
                             int(gridDim.x) - dec_wgs, lds,
                             reinterpret_cast<int4*>(lds + kP2Smem));
  }
}

// Split-K merge: one wave per (query row, head), lane l owning dims 2l and
// 2l + 1.  The splits are taken 16 at a time with every load of a batch in
// flight together (log-sum-exps are wave-uniform), so a row split 16 ways
// costs one memory round trip.  Rows that were not split were finalised by
// the attention kernel and are skipped.
constexpr int kMergeWaves = 4;
constexpr int kMergeBatch = 16;
// Block `block` of the split merge of a decode launch (merge_kernel).
template <bool kSteal = false>
__device__ __forceinline__ void merge_rows(const AttnParams& p, int num_rows, int64_t block,
                                           const StealArgs& sa = StealArgs{}) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = block * kMergeWaves + (threadIdx.x >> 6);
  const int64_t row = wv / p.num_heads;
  if (row >= num_rows) return;
  const int head = int(wv - row * p.num_heads);
  int nsplit;
  int first_share = 0;
  int taken = 0;  // lane k: tiles other workgroups took from piece k (tail hand-out)
  if (p.sk_nseg != nullptr) {
    // Stream-K: the split count of the head's kv slice in this row.
    const int g = head / p.group;
    const int kvs = g * p.nslices + (head - g * p.group) / p.hs;
    const int64_t unit = row * (p.kvh * p.nslices) + kvs;
    nsplit = p.sk_nseg[unit];
    if constexpr (kSteal) {
      if (lane < p.max_splits) taken = sa.stolen[unit * p.max_splits + lane];
      first_share = nsplit >> 16;
      nsplit &= 0xffff;
    }
  } else if (row < p.n_dec) {
    const int ctx = p.ctx_lens[row];
    nsplit = ctx > 0 ? (ctx + p.chunk_tokens - 1) / p.chunk_tokens : 1;
  } else {
    // Prefill row -> its chunk (cu_q is prefill-relative and nondecreasing):
    // i = #{j in 1 .. n_pre - 1 : cu_q[j] <= r}, counted 64 entries per load.
    const int r = int(row - p.n_dec);
    int i = 0;
    for (int j0 = 1; j0 < p.n_pre; j0 += 64) {
      const int j = j0 + lane;
      i += __popcll(__ballot(j < p.n_pre && p.cu_q[j] <= r));
    }
    i = uniform(i);
    const int sk = p.cu_k[i + 1] - p.cu_k[i];
    nsplit = max(1, (sk + p.split_tokens - 1) / p.split_tokens);
  }
  const int64_t base = (row * p.num_heads + head) * p.max_splits;
  // The first p.merge_first slots are loaded before the split count is known
  // (slots past it hold stale values, are inside the workspace and are masked
  // below), so a row with that many splits costs one memory round trip.
  float lse[kMergeBatch];
  float2 o[kMergeBatch];
  auto load_batch = [&](int s0, int cnt) {
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (k < cnt) {
        lse[k] = p.part_lse[base + s0 + k];
        o[k] = *reinterpret_cast<const float2*>(p.part_o + (base + s0 + k) * kD + 2 * lane);
      }
    }
  };
  const int first = min(p.merge_first, p.max_splits);
  load_batch(0, first);
  nsplit = uniform(nsplit);
  const unsigned long long taken_mask = __ballot(lane < nsplit && taken > 0);
  if (nsplit <= 1 && taken_mask == 0) return;
  float m = -INFINITY, l = 0.f, acc0 = 0.f, acc1 = 0.f;
  int s0 = 0, cnt = min(first, nsplit);
  while (true) {
    float bm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k)
      if (k < cnt) bm = fmaxf(bm, lse[k]);
    const float m_new = fmaxf(m, bm);
    if (m_new != -INFINITY) {  // else every split so far is empty
      const float a = __builtin_amdgcn_exp2f(m - m_new);
      l *= a;
      acc0 *= a;
      acc1 *= a;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        if (k < cnt) {
          const float w = __builtin_amdgcn_exp2f(lse[k] - m_new);
          l += w;
          acc0 += w * o[k].x;
          acc1 += w * o[k].y;
        }
      }
      m = m_new;
    }
    s0 += cnt;
    if (s0 >= nsplit) break;
    cnt = min(kMergeBatch, nsplit - s0);
    load_batch(s0, cnt);
  }
  // Tiles taken from piece k's tail: tail slots (first_share + k) *
  // kDecTailMax + j, j < taken[k], of this head within its row unit.
  if (kSteal && taken_mask != 0) {
    const int g = head / p.group;
    const int hu = head - (g & ~3) * p.group;  // 4 kv heads per row unit
    unsigned long long mask = taken_mask;
    while (mask != 0) {
      const int k = uniform(int(__ffsll(mask)) - 1);
      mask &= mask - 1;
      const int c = min(kDecTailMax, uniform(__builtin_amdgcn_readlane(taken, k)));
      const int64_t slot0 = int64_t(first_share + k) * kDecTailMax;
      float tl[kDecTailMax];
      float2 to[kDecTailMax];
#pragma unroll
      for (int j = 0; j < kDecTailMax; ++j) {
        if (j < c) {
          const int64_t base = (slot0 + j) * sa.uh + hu;
          tl[j] = sa.tail_lse[base];
          to[j] = *reinterpret_cast<const float2*>(sa.tail_o + base * kD + 2 * lane);
        }
      }
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < kDecTailMax; ++j)
        if (j < c) bm = fmaxf(bm, tl[j]);
      const float m_new = fmaxf(m, bm);
      if (m_new != -INFINITY) {
        const float a = __builtin_amdgcn_exp2f(m - m_new);
        l *= a;
        acc0 *= a;
        acc1 *= a;
#pragma unroll
        for (int j = 0; j < kDecTailMax; ++j) {
          if (j < c) {
            const float wgt = __builtin_amdgcn_exp2f(tl[j] - m_new);
            l += wgt;
            acc0 += wgt * to[j].x;
            acc1 += wgt * to[j].y;
          }
        }
        m = m_new;
      }
    }
  }
  const float inv = 1.f / l;
  uint16_t* dst = p.out + row * p.o_st + int64_t(head) * p.o_sh + 2 * lane;
  *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2_fast(acc0 * inv, acc1 * inv);
}

__global__ void __launch_bounds__(64 * kMergeWaves) merge_kernel(AttnParams p, int num_rows) {
  touch_kernel_args(int(sizeof(AttnParams) + sizeof(int)));
  merge_rows(p, num_rows, blockIdx.x);
}

// The merge of a decode launch with the dynamic tail hand-out: the taken
// tiles' partials too.  The decode launch is over, so its claim words go
// back to zero here for the next launch that uses this claim set.
__global__ void __launch_bounds__(64 * kMergeWaves)
merge_steal_kernel(AttnParams p, int num_rows, StealArgs sa) {
  touch_kernel_args(int(sizeof(AttnParams) + sizeof(int) + sizeof(StealArgs)));
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < sa.grid; i += 64 * kMergeWaves) sa.claims[i] = 0;
  }
  merge_rows<true>(p, num_rows, blockIdx.x, sa);
}

void launch_merge(const AttnParams& p, int64_t rows, hipStream_t st) {
  const int64_t waves = rows * p.num_heads;
  merge_kernel<<<unsigned((waves + kMergeWaves - 1) / kMergeWaves), 64 * kMergeWaves, 0, st>>>(
      p, int(rows));
}

void launch_merge_steal(const AttnParams& p, int64_t rows, const StealArgs& sa, hipStream_t st) {
  const int64_t waves = rows * p.num_heads;
  merge_steal_kernel<<<unsigned((waves + kMergeWaves - 1) / kMergeWaves), 64 * kMergeWaves, 0,
                       st>>>(p, int(rows), sa);
}

// Split-K merge of a stream-K prefill launch: one wave per (query row, kv
// slice).  The wave reads the slice's split count once; lane l then owns
// head l / 8 of the slice (eight heads per pass) and dims 32 q + 4 (l % 8)
// .. + 3 (q < 4: each load instruction reads 64 contiguous bytes of a head's
// fp16 partial row; with fp32 rows, 128 bytes were 0.8 us faster than 16
// contiguous dims per lane on the merge of 60 decode rows + four 256-token
// chunks after prefixes 0 / 512 / 2048 / 8192), so a whole slice's partials
// are in flight together and a row costs two memory round trips (the count,
// then the partials) whatever its head count.
constexpr int kSliceBatch = 4;  // splits per load batch (124 VGPRs: every wave resident)
// Block `block` of the split merge of a stream-K prefill launch
// (merge_slices_kernel).
__device__ __forceinline__ void merge_slice_rows(const AttnParams& p, int num_rows,
                                                 const uint16_t* __restrict__ part_h,
                                                 const float2* __restrict__ part_ml,
                                                 const int* __restrict__ nseg_arr,
                                                 int64_t block) {
  const int lane = threadIdx.x & 63;
  const int e = lane >> 3;   // head within the pass
  const int sub = lane & 7;  // 16-dim chunk
  const int kvs_total = p.kvh * p.nslices;
  const int64_t wv = block * kMergeWaves + (threadIdx.x >> 6);
  const int64_t row = wv / kvs_total;
  if (row >= num_rows) return;
  const int kvs = int(wv - row * kvs_total);
  const int nsplit = uniform(nseg_arr[row * kvs_total + kvs]);
  if (nsplit <= 1) return;
  const int g = kvs / p.nslices;
  const int s = kvs - g * p.nslices;
  const int h0 = g * p.group + s * p.hs;
  const int hs = min(p.hs, p.group - s * p.hs);
  for (int hb = 0; hb < hs; hb += 8) {
    const int hh = min(hb + e, hs - 1);  // lanes past the slice repeat its last head
    const int64_t base = (row * p.num_heads + h0 + hh) * p.max_splits;
    float m = -INFINITY, l = 0.f;
    float acc[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) acc[d] = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += kSliceBatch) {
      const int cnt = min(kSliceBatch, nsplit - s0);
      float lse[kSliceBatch], esc[kSliceBatch];
      float4 o[kSliceBatch][4];
#pragma unroll
      for (int k = 0; k < kSliceBatch; ++k) {
        if (k < cnt) {
          const float2 ml = part_ml[base + s0 + k];
          lse[k] = ml.x;
          esc[k] = ml.y;
          // lane sub: dims 32 q + 4 sub .. + 3 (fp16), so each load of a
          // wave reads 64 contiguous bytes per head
          const u32x2_t* src = reinterpret_cast<const u32x2_t*>(part_h + (base + s0 + k) * kD) + sub;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u32x2_t h = src[8 * q];
            o[k][q] = float4{f16_lo(h[0]), f16_hi(h[0]), f16_lo(h[1]), f16_hi(h[1])};
          }
        }
      }
      float bm = -INFINITY;
#pragma unroll
      for (int k = 0; k < kSliceBatch; ++k)
        if (k < cnt) bm = fmaxf(bm, lse[k]);
      const float m_new = fmaxf(m, bm);
      if (m_new != -INFINITY) {  // else every split so far is empty
        const float a = __builtin_amdgcn_exp2f(m - m_new);
        l *= a;
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[d] *= a;
#pragma unroll
        for (int k = 0; k < kSliceBatch; ++k) {
          if (k < cnt) {
            const float wgt = __builtin_amdgcn_exp2f(lse[k] - m_new);
            l += wgt;
            const float wo = ldexpf(wgt, int(esc[k]));  // the row's fp16 scale
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc[4 * q + 0] += wo * o[k][q].x;
              acc[4 * q + 1] += wo * o[k][q].y;
              acc[4 * q + 2] += wo * o[k][q].z;
              acc[4 * q + 3] += wo * o[k][q].w;
            }
          }
        }
        m = m_new;
      }
    }
    if (hb + e < hs) {
      const float inv = 1.f / l;
      uint16_t* dst = p.out + row * p.o_st + int64_t(h0 + hb + e) * p.o_sh + 4 * sub;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        *reinterpret_cast<u32x2_t*>(dst + 32 * q) =
            u32x2_t{pack_bf16x2_fast(acc[4 * q + 0] * inv, acc[4 * q + 1] * inv),
                    pack_bf16x2_fast(acc[4 * q + 2] * inv, acc[4 * q + 3] * inv)};
      }
    }
  }
}

__global__ void __launch_bounds__(64 * kMergeWaves)
merge_slices_kernel(AttnParams p, int num_rows, const uint16_t* __restrict__ part_h,
                    const float2* __restrict__ part_ml, const int* __restrict__ nseg_arr) {
  touch_kernel_args(int(sizeof(AttnParams) + 4 * sizeof(void*)));
  merge_slice_rows(p, num_rows, part_h, part_ml, nseg_arr, blockIdx.x);
}

// Both merges of a mixed call's split launch in one launch: blocks
// [0, dec_blocks) merge the decode rows' splits, the others the prefill
// rows' splits.
__global__ void __launch_bounds__(64 * kMergeWaves)
merge_mixed_kernel(AttnParams pd, AttnParams pp, int dec_rows, int dec_blocks, int pre_rows) {
  touch_kernel_args(int(2 * sizeof(AttnParams) + 3 * sizeof(int)));
  const int64_t b = blockIdx.x;
  if (b < dec_blocks) {
    merge_rows(pd, dec_rows, b);
  } else {
    merge_slice_rows(pp, pre_rows, reinterpret_cast<const uint16_t*>(pp.part_o), pp.part_ml,
                     pp.sk_nseg, b - dec_blocks);
  }
}

void launch_merge_slices(const AttnParams& p, int64_t rows, hipStream_t st) {
  const int64_t waves = rows * p.kvh * p.nslices;
  merge_slices_kernel<<<unsigned((waves + kMergeWaves - 1) / kMergeWaves), 64 * kMergeWaves, 0,
                        st>>>(p, int(rows), reinterpret_cast<const uint16_t*>(p.part_o),
                              p.part_ml, p.sk_nseg);
}

// ---------------------------------------------------------------------------
// Host-side launch planning.
// ---------------------------------------------------------------------------
int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  return atoi(v);
}

float env_float(const char* name, float fallback) {
  const char* v = getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  return float(atof(v));
}

// Share skew of the stream-K decode between even and odd workgroups (XCDs):
// with the 4-kv-head LDS segment the odd XCDs stream the same share ~8-14 %
// slower (per-workgroup stamps, KVC_DECODE_STAMPS; 4.4-7.4 us later median
// ends at batch 64 x 4096 without skew), so they take 4 % less of a bf16
// decode (0.04-0.06 measured alike).  The 2-kv-head segment shows no such gap
// (odd XCDs 1.4-1.6 us later without skew, 1.5 us earlier with 0.04) and
// runs without skew.  The per-token-head int8 segment's odd XCDs end 4.5-5 us
// later at batch 16 x 32768 without skew; 0.03 brings that to 1 us (kernel
// 92.6 us against 93.1-94.4 us).
constexpr float kXcdSkew = 0.04f;
constexpr float kXcdSkewI8 = 0.03f;

// Workgroups of a stream-K launch: one per CU, or the CUs this thread's
// current launch may occupy (a mixed call running its decode and prefill
// launches side by side gives each a share of the CUs; LDS keeps their
// workgroups on separate CUs).
thread_local int tl_launch_cus = 0;
struct LaunchCus {
  int saved;
  explicit LaunchCus(int n) : saved(tl_launch_cus) { tl_launch_cus = n; }
  ~LaunchCus() { tl_launch_cus = saved; }
};

// A stream-K launch recorded instead of launched: while tl_record is set,
// the paged decode entry point (bf16 pool, LDS-staged, no append) and the
// prefill-only entry point (stream-K launch over cached bf16 keys) validate,
// plan and fill their parameters as usual, store them here and return
// without launching the kernel or its merge.  A mixed call then runs both in
// one mixed_split_kernel launch.  An entry point that cannot take this form
// launches as usual and leaves `taken` false.
struct SkRecord {
  bool taken = false;
  AttnParams p{};
  int grid = 0;
  int64_t rows = 0;  // rows its merge covers
};
thread_local SkRecord* tl_record = nullptr;
struct RecordInto {
  SkRecord* saved;
  explicit RecordInto(SkRecord* r) : saved(tl_record) { tl_record = r; }
  ~RecordInto() { tl_record = saved; }
};
int device_cus();
int launch_cus() { return tl_launch_cus > 0 ? tl_launch_cus : device_cus(); }

// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Kv slices per decode workgroup: the largest of 4, 2, 1 that divides the
// slice count, so the eight waves split evenly over slices and tile streams
// (4 slices of one head each are a 1 KiB slice of a token row: the LDS
// segments stream those; 2 are a 512 B row of a 2-kv-head shard).
int plan_kvs_per_wg(int64_t kvslices) {
  int per = 4;
  while (per > 1 && kvslices % per != 0) per >>= 1;
  return per;
}

// Keys per decode chunk.  The plan aims at one workgroup per CU: the
// (rows x slice groups) units are split into just enough chunks to reach the
// CU count (a workgroup keeps its eight waves busy with two tiles in flight
// each, which saturates HBM with one workgroup per CU).  KVC_DECODE_CHUNK
// overrides it (a multiple of 32).
int plan_decode_chunk(int64_t rows, int64_t groups, int64_t max_ctx) {
  const int forced = env_int("KVC_DECODE_CHUNK", 0);
  if (forced > 0) return forced;
  const int64_t units = rows * groups;
  const int64_t cus = device_cus();
  int64_t nch = units >= cus ? 1 : (cus + units - 1) / units;
  int64_t ch = (max_ctx + nch - 1) / nch;
  ch = ((ch + 127) / 128) * 128;
  return int(ch < 128 ? 128 : ch);
}

// Stream-K plan of a paged decode launch: one workgroup per CU, shares of
// at least kSkMinShare tiles, at most max_splits workgroups per row (bounded
// so the partials stay within kSkMaxPartialBytes).  KVC_DECODE_STREAMK=0
// selects the fixed-chunk partition instead.
constexpr int kSkMinShare = 8;
// The device-side share floor (tiles): small batches spread over every CU.
constexpr int kSkMinShareDev = 2;
constexpr int64_t kSkMaxPartialBytes = int64_t(256) << 20;

struct SkPlan {
  bool on;
  int grid;
  int max_splits;
};

SkPlan plan_stream_k(int64_t rows, int64_t heads, int64_t max_ctx, int64_t units) {
  SkPlan sp{env_int("KVC_DECODE_STREAMK", 1) != 0, launch_cus(), 2};
  const int64_t max_tiles = (max_ctx + kTile - 1) / kTile;
  int64_t ms = (max_tiles + kSkMinShare - 1) / kSkMinShare + 1;
  // A batch with fewer row units than CUs lets each unit split over about
  // CUs / units workgroups (every CU then streams a few tiles); larger
  // batches keep the 8-tile bound.
  if (units > 0 && units < sp.grid) ms = std::max<int64_t>(ms, (sp.grid + units - 1) / units + 1);
  const int64_t per_split = rows * heads * (kD + 1) * int64_t(sizeof(float));
  const int64_t cap = per_split > 0 ? kSkMaxPartialBytes / per_split : 64;
  ms = ms > 64 ? 64 : ms;
  ms = ms > cap ? cap : ms;
  sp.max_splits = int(ms < 2 ? 2 : ms);
  return sp;
}

// Workspace of a stream-K launch: the partials, then one int32 split count
// per (row, kv slice) (256-byte aligned).
size_t sk_partial_part(int64_t rows, int64_t heads, int max_splits) {
  const size_t part = size_t(rows) * size_t(heads) * size_t(max_splits) * (kD + 1) * sizeof(float);
  return (part + 255) / 256 * 256;
}
size_t sk_workspace_bytes(int64_t rows, int64_t heads, int64_t kv_slices, int max_splits) {
  return sk_partial_part(rows, heads, max_splits) + size_t(rows) * size_t(kv_slices) * sizeof(int) +
         256;
}

// Workspace of a stream-K paged decode whose shape can take the dynamic tail
// hand-out (4 kv heads of one slice per workgroup): after the stream-K part,
// the taken-tile counts per (row, kv slice, piece), the tail partials of
// every share ([share][kDecTailMax][uh heads][D] fp32 and the matching
// log2-sum-exps) and eight dummy words per workgroup.
struct StealLayout {
  size_t stolen, tail_o, tail_lse, dummy, total;
};
StealLayout steal_layout(size_t base, int64_t rows, int64_t kv_slices, int max_splits, int grid,
                         int uh) {
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  StealLayout L;
  L.stolen = al(base);
  L.tail_o = al(L.stolen + size_t(rows) * size_t(kv_slices) * size_t(max_splits) * sizeof(int));
  L.tail_lse = al(L.tail_o + size_t(grid) * kDecTailMax * size_t(uh) * kD * sizeof(float));
  L.dummy = al(L.tail_lse + size_t(grid) * kDecTailMax * size_t(uh) * sizeof(float));
  L.total = al(L.dummy + size_t(grid) * 8 * sizeof(int));
  return L;
}

// Keys per prefill split: an eighth of the longest key range, at least 512
// (the long chunk of a mixed batch then fills the CUs with its splits).
int plan_prefill_split(int64_t max_seqlen_k) {
  const int forced = env_int("KVC_PREFILL_SPLIT", 0);
  if (forced > 0) return (forced + kTile - 1) / kTile * kTile;
  int64_t ks = (max_seqlen_k + 7) / 8;
  ks = ((ks + kTile - 1) / kTile) * kTile;
  return int(ks < 512 ? 512 : ks);
}

struct HeadPlan {
  int group, hs, nslices, tpb;
  int kvs_per_wg;  // decode slices per workgroup
  int groups;      // decode slice groups: kvh * nslices / kvs_per_wg
};

// Shapes whose bf16 stream-K decode runs LDS-staged segments of 4 kv heads
// (one slice each): the ones that can take the dynamic tail hand-out.
bool steal_shape(const HeadPlan& hp) { return hp.kvs_per_wg == 4 && hp.nslices == 1; }
// Default tail tiles per share, and the fewest tiles a share must have left
// in its tail for another workgroup to take one.
constexpr int kDecTailDefault = 6;
constexpr int kStealMinDefault = 2;

HeadPlan plan_heads(int64_t num_heads, int64_t kvh) {
  HeadPlan h;
  h.group = int(num_heads / kvh);
  h.hs = h.group < 16 ? h.group : 16;
  h.nslices = (h.group + h.hs - 1) / h.hs;
  h.tpb = 16 / h.hs;
  h.kvs_per_wg = plan_kvs_per_wg(kvh * h.nslices);
  h.groups = int(kvh * h.nslices / h.kvs_per_wg);
  return h;
}

size_t partial_bytes(int64_t rows, int64_t heads, int64_t splits) {
  if (splits <= 1) return 0;
  return size_t(rows) * size_t(heads) * size_t(splits) * (kD + 1) * sizeof(float) + 256;
}

void set_partials(AttnParams& p, void* ws, int64_t rows) {
  if (p.max_splits <= 1 || ws == nullptr) {
    p.part_o = nullptr;
    p.part_lse = nullptr;
    p.part_ml = nullptr;
    return;
  }
  p.part_o = static_cast<float*>(ws);
  p.part_lse = p.part_o + size_t(rows) * p.num_heads * p.max_splits * kD;
  // (stream-K prefill) pairs after the fp16 rows, inside part_o's span
  p.part_ml = reinterpret_cast<float2*>(reinterpret_cast<char*>(ws) +
                                        size_t(rows) * p.num_heads * p.max_splits * kD * 2);
}

int check_kv_args(int kv_dtype, const float* k_scale, const float* v_scale, const void* side_k,
                  const void* side_v, const int32_t* out_idx2d, const int32_t* head_n_out,
                  int64_t n_out_max, const char* what) {
  KVC_REQUIRE(kv_dtype == KVC_KV_BF16 || kv_dtype == KVC_KV_INT8_TOKHEAD ||
                  kv_dtype == KVC_KV_INT8_CHAN,
              KVC_ERR_VALUE, "%s: unknown kv_dtype %d", what, kv_dtype);
  if (kv_dtype != KVC_KV_BF16) {
    KVC_REQUIRE(k_scale != nullptr && v_scale != nullptr, KVC_ERR_VALUE,
                "%s: int8 KV needs k_scale and v_scale", what);
  }
  if (kv_dtype == KVC_KV_INT8_CHAN && head_n_out != nullptr) {
    KVC_REQUIRE(side_k != nullptr && side_v != nullptr && out_idx2d != nullptr, KVC_ERR_VALUE,
                "%s: outlier dims need side pools and out_idx2d", what);
    // A power of two, as the reference kernel's tl.arange(0, N_OUT_MAX)
    // requires (nanovllm/kernels/paged_attention.py:107): a side row is then
    // one aligned 2-, 4-, 8- or 16-byte load.
    KVC_REQUIRE(n_out_max >= 1 && n_out_max <= kSideMax && (n_out_max & (n_out_max - 1)) == 0,
                KVC_ERR_VALUE, "%s: n_out_max must be 1, 2, 4 or 8 (got %lld)", what,
                (long long)n_out_max);
    const uintptr_t row_align = uintptr_t(n_out_max >= 2 ? 4 : 2);
    KVC_REQUIRE(reinterpret_cast<uintptr_t>(side_k) % row_align == 0 &&
                    reinterpret_cast<uintptr_t>(side_v) % row_align == 0,
                KVC_ERR_VALUE, "%s: side pools must be %d-byte aligned", what, int(row_align));
  }
  return KVC_OK;
}

void fill_kv(AttnParams& p, const void* k_cache, const void* v_cache, int64_t page, int64_t kvh,
             int kv_dtype, const float* k_scale, const float* v_scale, const void* side_k,
             const void* side_v, const int32_t* out_idx2d, const int32_t* head_n_out,
             int64_t n_out_max) {
  p.k_cache = static_cast<const char*>(k_cache);
  p.v_cache = static_cast<const char*>(v_cache);
  p.page = int(page);
  p.kvh = int(kvh);
  p.tok_bytes = kvh * kD * (kv_dtype == KVC_KV_BF16 ? 2 : 1);
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  const bool side = kv_dtype == KVC_KV_INT8_CHAN && head_n_out != nullptr;
  p.side_k = side ? static_cast<const uint16_t*>(side_k) : nullptr;
  p.side_v = side ? static_cast<const uint16_t*>(side_v) : nullptr;
  p.out_idx = side ? out_idx2d : nullptr;
  p.head_n_out = side ? head_n_out : nullptr;
  p.n_out_max = side ? int(n_out_max) : 0;
}

template <int kEnc>
void launch_decode_enc(const AttnParams& p, int grid, hipStream_t st) {
  paged_decode_kernel<kEnc><<<grid, kThreads, 0, st>>>(p);
}




// A varlen call with decode rows over a paged pool runs them as a paged decode
// (stream-K) and the prefill rows as a stream-K prefill: in one launch over a
// CU split where both sides allow it (mixed_split_kernel), else one launch
// after the other on the same stream.  (One combined launch of decode and
// prefill units, and one stream-K launch over both, both measured slower on
// every mix.)
bool split_mixed(int64_t num_decode_rows, int64_t page_size) {
  return num_decode_rows > 0 && page_size > 0;
}

// Per-CU rates of the two sides of a mixed launch, measured on MI355X with
// the other side idle and each side held to n workgroups (n = 16 .. 192; the
// time of a side fits c + work / n there): the LDS-staged decode streams
// about 41 GB/s of bf16 K/V per CU, the stream-K prefill about 4.3 TFLOP/s
// per CU.
constexpr double kMixDecodeBytesPerCuUs = 41.0e3;
constexpr double kMixPrefillFlopsPerCuUs = 4.3e6;

// Workgroups (= CUs) the decode side of a mixed call's split launch gets
// (mixed_split_kernel: decode rows on that many CUs, prefill rows on the rest
// at once; 0: the decode launch, then the prefill launch).  The split form
// needs both sides in their stream-K forms: a bf16 pool with 4 kv heads per
// decode workgroup (LDS-staged) and the stream-K prefill.
// With the host's hints (the decode rows' total context in tokens, and the
// prefill's query-key pairs per head: sum over chunks of
// sq (sk - sq) + sq (sq + 1) / 2), the CUs split in proportion to the two
// sides' CU-time at the rates above, so that both end together (at a
// multiple of 8, at least 8 on each side: of the two around the balance
// point, the one whose slower side ends sooner).  Without hints the decode side
// gets 3/8 of the CUs, the balance of 60 decode rows of U[256,4096] and four
// 256-token chunks.  KVC_MIXED_DECODE_CUS overrides both (rounded down to a
// multiple of 8; 0: the two launches one after the other).
int mixed_decode_cus(int64_t num_decode_rows, int64_t num_prefill_tokens, int kv_dtype,
                     int64_t num_heads, int64_t num_kv_heads, int64_t decode_ctx_tokens,
                     int64_t prefill_kq_pairs) {
  if (num_decode_rows <= 0 || num_prefill_tokens <= 0) return 0;
  if (kv_dtype != KVC_KV_BF16 || env_int("KVC_DECODE_STREAMK", 1) == 0 ||
      env_int("KVC_DECODE_LDS", 1) == 0 || env_int("KVC_PREFILL_SK", 1) == 0)
    return 0;
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  if (hp.kvs_per_wg != 4 || hp.nslices != 1) return 0;
  const int total = device_cus();
  if (total < 16 || total % 8 != 0) return 0;
  int n = env_int("KVC_MIXED_DECODE_CUS", -1);
  if (n < 0) {
    if (decode_ctx_tokens > 0 && prefill_kq_pairs > 0) {
      const double dec = double(decode_ctx_tokens) * double(num_kv_heads) * (2.0 * kD * 2.0) /
                         kMixDecodeBytesPerCuUs;
      const double pre =
          4.0 * kD * double(num_heads) * double(prefill_kq_pairs) / kMixPrefillFlopsPerCuUs;
      // The two multiples of 8 around the balance point; of them, the one
      // whose slower side ends sooner (a side's time falls as 1 / its CUs,
      // so the nearer multiple is not always the better one).
      const double nf = double(total) * dec / (dec + pre);
      const int lo = std::min(std::max(int(nf / 8.0) * 8, 8), total - 8);
      const int hi = std::min(lo + 8, total - 8);
      auto slower = [&](int m) { return std::max(dec / m, pre / (total - m)); };
      n = slower(hi) < slower(lo) ? hi : lo;
    } else {
      n = total * 3 / 8;
    }
  }
  n = n / 8 * 8;
  return (n >= 8 && n <= total - 8) ? n : 0;
}

// Prefill-only launches over bf16 keys run as one stream-K launch
// (prefill_sk2_kernel) unless KVC_PREFILL_SK=0 selects one workgroup per
// prefill unit.  The workspace query cannot see the key encoding or the
// query strides, so it sizes for both; the launch also needs every chunk's
// query rows below 2 GiB (one buffer resource).
bool prefill_stream_k(int64_t num_decode_rows) {
  return num_decode_rows == 0 && env_int("KVC_PREFILL_SK", 1) != 0;
}

// Split cap of a stream-K prefill launch: an item of T tiles spans at most
// ceil(T / S) + 1 shares; the cap is 64 and the partials' byte bound.
SkPlan plan_prefill_sk(int64_t num_q_tokens, int64_t num_heads, int64_t max_seqlen_k) {
  SkPlan sp{true, launch_cus(), 2};
  int64_t ms = (max_seqlen_k + kTile - 1) / kTile / kPfMinShare + 2;
  const int64_t per_split = num_q_tokens * num_heads * (kD + 1) * int64_t(sizeof(float));
  const int64_t cap = per_split > 0 ? kSkMaxPartialBytes / per_split : 64;
  ms = std::min<int64_t>(std::min<int64_t>(ms, 64), cap);
  sp.max_splits = int(ms < 2 ? 2 : ms);
  return sp;
}

void launch_prefill_sk(const AttnParams& p, int grid, bool fresh, hipStream_t st) {
  if (fresh) {
    if (p.head_n_out != nullptr) {
      prefill_sk2_kernel<true, true><<<grid, kThreads, 0, st>>>(p, p.cu_q, p.cu_k, p.block_tables);
    } else {
      prefill_sk2_kernel<true><<<grid, kThreads, 0, st>>>(p, p.cu_q, p.cu_k, p.block_tables);
    }
  } else {
    prefill_sk2_kernel<false><<<grid, kThreads, 0, st>>>(p, p.cu_q, p.cu_k, p.block_tables);
  }
}

template <int kEnc>
void launch_varlen_enc(const AttnParams& p, int grid, bool fresh, hipStream_t st) {
  if (fresh) {
    // Fresh rows gathered from a per-channel pool carry its outlier dims.
    if constexpr (kEnc == kBF16) {
      if (p.head_n_out != nullptr) {
        varlen_kernel<kBF16, true, true><<<grid, kThreads, 0, st>>>(p, p.block_tables);
      } else {
        varlen_kernel<kBF16, true><<<grid, kThreads, 0, st>>>(p, p.block_tables);
      }
    }
  } else {
    varlen_kernel<kEnc, false><<<grid, kThreads, 0, st>>>(p, p.block_tables);
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" size_t kvc_paged_decode_workspace_bytes(int64_t batch, int64_t num_heads,
                                                   int64_t num_kv_heads, int64_t head_dim,
                                                   int64_t page_size,
                                                   int64_t max_blocks_per_seq) {
  if (batch <= 0 || num_kv_heads <= 0 || head_dim != kD) return 0;
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  const int64_t max_ctx = max_blocks_per_seq * page_size;
  const SkPlan sp = plan_stream_k(batch, num_heads, max_ctx, batch * hp.groups);
  if (sp.on) {
    const size_t base = sk_workspace_bytes(batch, num_heads, num_kv_heads * hp.nslices,
                                           sp.max_splits);
    if (!steal_shape(hp)) return base;
    return steal_layout(base, batch, num_kv_heads * hp.nslices, sp.max_splits, sp.grid,
                        hp.kvs_per_wg * hp.hs)
        .total;
  }
  const int ch = plan_decode_chunk(batch, hp.groups, max_ctx);
  const int64_t splits = max_ctx > 0 ? (max_ctx + ch - 1) / ch : 1;
  return partial_bytes(batch, num_heads, splits);
}

extern "C" int kvc_paged_decode_layout(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                       int64_t head_dim, int64_t page_size,
                                       int64_t max_blocks_per_seq, int64_t* layout) {
  clear_error();
  KVC_REQUIRE(layout != nullptr, KVC_ERR_VALUE, "paged_decode_layout: layout is required");
  KVC_REQUIRE(batch > 0 && num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0 &&
                  head_dim == kD && page_size > 0 && max_blocks_per_seq > 0,
              KVC_ERR_VALUE, "paged_decode_layout: bad launch shape");
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  const SkPlan sp =
      plan_stream_k(batch, num_heads, max_blocks_per_seq * page_size, batch * hp.groups);
  KVC_REQUIRE(sp.on, KVC_ERR_VALUE, "paged_decode_layout: the launch is not stream-K");
  const int64_t kv_slices = num_kv_heads * hp.nslices;
  const size_t base = sk_workspace_bytes(batch, num_heads, kv_slices, sp.max_splits);
  layout[0] = int64_t(sk_partial_part(batch, num_heads, sp.max_splits));
  layout[1] = steal_shape(hp) ? int64_t(steal_layout(base, batch, kv_slices, sp.max_splits,
                                                     sp.grid, hp.kvs_per_wg * hp.hs)
                                            .stolen)
                              : -1;
  layout[2] = sp.max_splits;
  layout[3] = kv_slices;
  return KVC_OK;
}

namespace {
// The step's append to fuse into a paged decode launch (key null: none).
struct DecodeAppend {
  const void* key;
  int64_t key_stride_n, key_stride_h;
  const void* value;
  int64_t value_stride_n, value_stride_h;
  const void* slot_mapping;
  int slot_index_bytes;
  // per-channel int8: the store scales [KVH, D] (the decode reads with its
  // own read scales)
  const float* store_k_scale = nullptr;
  const float* store_v_scale = nullptr;
};

// The side pool arguments of a per-channel int8 decode.
struct SidePool {
  const void* side_k;
  const void* side_v;
  const int32_t* out_idx2d;
  const int32_t* head_n_out;
  int64_t n_out_max;
};

// The step's append as its own launch (before a decode launch that cannot
// take it in): store_kvcache, or the int8 quantisers.
int store_append(const DecodeAppend& app, const void* k_cache, const void* v_cache,
                 const float* k_scale, const float* v_scale, const SidePool& side,
                 int64_t num_slots, int64_t batch, int64_t num_kv_heads, int kv_dtype,
                 kvc_stream_t stream) {
  if (kv_dtype == KVC_KV_INT8_CHAN) {
    return kvc_store_int8_chan(app.key, app.key_stride_n, app.key_stride_h, app.value,
                               app.value_stride_n, app.value_stride_h,
                               static_cast<int8_t*>(const_cast<void*>(k_cache)),
                               static_cast<int8_t*>(const_cast<void*>(v_cache)),
                               app.store_k_scale, app.store_v_scale,
                               const_cast<void*>(side.side_k), const_cast<void*>(side.side_v),
                               side.n_out_max, side.out_idx2d, side.head_n_out, num_slots,
                               app.slot_mapping, app.slot_index_bytes, batch, num_kv_heads, kD,
                               stream);
  }
  if (kv_dtype == KVC_KV_INT8_TOKHEAD) {
    return kvc_store_int8_tokhead(app.key, app.key_stride_n, app.key_stride_h, app.value,
                                  app.value_stride_n, app.value_stride_h,
                                  static_cast<int8_t*>(const_cast<void*>(k_cache)),
                                  static_cast<int8_t*>(const_cast<void*>(v_cache)),
                                  const_cast<float*>(k_scale), const_cast<float*>(v_scale),
                                  num_slots, app.slot_mapping, app.slot_index_bytes, batch,
                                  num_kv_heads, kD, stream);
  }
  return kvc_store_kv(app.key, app.key_stride_n, app.key_stride_h, app.value,
                      app.value_stride_n, app.value_stride_h, const_cast<void*>(k_cache),
                      const_cast<void*>(v_cache), num_slots, app.slot_mapping,
                      app.slot_index_bytes, batch, num_kv_heads, kD, 2, stream);
}

int paged_decode_impl(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                      const void* v_cache, int64_t num_cache_blocks, int64_t page_size,
                      int64_t num_kv_heads, int64_t head_dim, int kv_dtype, const float* k_scale,
                      const float* v_scale, const void* side_k, const void* side_v,
                      const int32_t* out_idx2d, const int32_t* head_n_out, int64_t n_out_max,
                      const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
                      const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale,
                      void* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                      size_t workspace_bytes, const DecodeAppend& app, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "paged_decode: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(page_size > 0 && page_size % kTile == 0, KVC_ERR_VALUE,
              "paged_decode: page_size must be a positive multiple of 32 (got %lld)",
              (long long)page_size);
  KVC_REQUIRE(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0, KVC_ERR_VALUE,
              "paged_decode: num_heads (%lld) must be a multiple of num_kv_heads (%lld)",
              (long long)num_heads, (long long)num_kv_heads);
  KVC_REQUIRE(num_cache_blocks >= 0, KVC_ERR_VALUE, "paged_decode: bad num_cache_blocks");
  int rc = check_kv_args(kv_dtype, k_scale, v_scale, side_k, side_v, out_idx2d, head_n_out,
                         n_out_max, "paged_decode");
  if (rc != KVC_OK) return rc;
  KVC_REQUIRE((q_stride_b % 8) == 0 && (q_stride_h % 8) == 0 && (out_stride_b % 8) == 0 &&
                  (out_stride_h % 8) == 0 && (reinterpret_cast<uintptr_t>(q) % 16) == 0 &&
                  (reinterpret_cast<uintptr_t>(out) % 16) == 0,
              KVC_ERR_ASSERT, "paged_decode: q/out rows must be 16-byte aligned");
  if (batch == 0) return KVC_OK;
  KVC_REQUIRE(max_blocks_per_seq > 0, KVC_ERR_VALUE, "paged_decode: empty block_tables");

  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  AttnParams p{};
  p.merge_first = 0;  // most rows of these launches are not split
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_stride_b;
  p.q_sh = q_stride_h;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = out_stride_b;
  p.o_sh = out_stride_h;
  p.num_heads = int(num_heads);
  p.group = hp.group;
  p.hs = hp.hs;
  p.nslices = hp.nslices;
  p.tpb = hp.tpb;
  p.kvs_per_wg = hp.kvs_per_wg;
  p.scale_log2 = scale * kLog2e;
  fill_kv(p, k_cache, v_cache, page_size, num_kv_heads, kv_dtype, k_scale, v_scale, side_k, side_v,
          out_idx2d, head_n_out, n_out_max);
  p.block_tables = block_tables;
  p.bt_stride = bt_stride;
  p.n_dec = int(batch);
  p.ctx_lens = context_lens;
  const int64_t max_ctx = max_blocks_per_seq * page_size;
  p.kvs_per_wg = hp.kvs_per_wg;
  hipStream_t st = as_stream(stream);
  const SkPlan sp = plan_stream_k(batch, num_heads, max_ctx, batch * hp.groups);
  if (sp.on) {
    p.max_splits = sp.max_splits;
    p.sk_min_share = std::max(1, env_int("KVC_SK_MIN_SHARE", kSkMinShareDev));
    // The per-channel int8 segment runs without skew (not measured).
    {
      const float dflt = kv_dtype == KVC_KV_BF16 ? (hp.kvs_per_wg == 4 ? kXcdSkew : 0.f)
                         : kv_dtype == KVC_KV_INT8_TOKHEAD ? kXcdSkewI8
                                                           : 0.f;
      p.xcd_skew = std::min(0.25f, std::max(0.f, env_float("KVC_XCD_SKEW", dflt)));
    }
    // Equal rows split into grid / units shares (+1 where a share boundary
    // falls inside a row); longer rows of a ragged batch load the rest later.
    const int64_t units = batch * hp.groups;
    p.merge_first = int(std::min<int64_t>(kMergeBatch, (sp.grid + units - 1) / units + 1));
    const int64_t kv_slices = num_kv_heads * hp.nslices;
    const size_t base = sk_workspace_bytes(batch, num_heads, kv_slices, sp.max_splits);
    const StealLayout sl =
        steal_layout(base, batch, kv_slices, sp.max_splits, sp.grid, hp.kvs_per_wg * hp.hs);
    const size_t need = steal_shape(hp) ? sl.total : base;
    KVC_REQUIRE(workspace != nullptr && workspace_bytes >= need, KVC_ERR_WORKSPACE,
                "paged_decode: workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
    set_partials(p, workspace, batch);
    p.sk_nseg = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                       sk_partial_part(batch, num_heads, p.max_splits));
    p.chunk_tokens = kTile;
    // LDS-staged bf16 segments: 4 kv heads per workgroup (1 KiB token-row
    // slices) or 2 (512 B rows, two tiles per stage).
    // (A 2-head load brings two whole token rows, so that form needs rows of
    // exactly 2 kv heads.)
    const bool lds_bf16 = kv_dtype == KVC_KV_BF16 && hp.nslices == 1 &&
                          (hp.kvs_per_wg == 4 || (hp.kvs_per_wg == 2 && num_kv_heads == 2)) &&
                          env_int("KVC_DECODE_LDS", 1) != 0;
    const bool lds4 = lds_bf16 && hp.kvs_per_wg == 4;
    if (app.key != nullptr) {
      // The LDS segments take the append in (16-byte chunks of the kv group's
      // token-row slice: bf16 rows, or the per-token-head int8 quantiser's
      // input); any other form gets the store launch first.
      const bool lds_i8 = kv_dtype == KVC_KV_INT8_TOKHEAD && hp.kvs_per_wg == 4 &&
                          hp.nslices == 1 && env_int("KVC_DECODE_LDS", 1) != 0;
      const bool fuse = (lds_bf16 || lds_i8) && (reinterpret_cast<uintptr_t>(app.key) % 16) == 0 &&
                        (reinterpret_cast<uintptr_t>(app.value) % 16) == 0 &&
                        app.key_stride_n % 8 == 0 && app.key_stride_h % 8 == 0 &&
                        app.value_stride_n % 8 == 0 && app.value_stride_h % 8 == 0;
      if (fuse) {
        p.app_k = static_cast<const uint16_t*>(app.key);
        p.app_v = static_cast<const uint16_t*>(app.value);
        p.app_k_st = app.key_stride_n;
        p.app_k_sh = app.key_stride_h;
        p.app_v_st = app.value_stride_n;
        p.app_v_sh = app.value_stride_h;
        p.app_slots = app.slot_mapping;
        p.app_slot_bytes = app.slot_index_bytes;
        p.app_num_slots = num_cache_blocks * page_size;
      } else {
        rc = store_append(app, k_cache, v_cache, k_scale, v_scale,
                          SidePool{side_k, side_v, out_idx2d, head_n_out, n_out_max},
                          num_cache_blocks * page_size,
                          batch, num_kv_heads, kv_dtype, stream);
        if (rc != KVC_OK) return rc;
      }
    }
    // Per-workgroup stamps for diagnostics (KVC_DECODE_STAMPS=1; the buffer
    // holds up to kvc::stamp_slots() workgroups; kvc_decode_stamps reads it).
    if (env_int("KVC_DECODE_STAMPS", 0) != 0 && sp.grid <= stamp_slots())
      p.wg_stamps = stamp_buffer(sp.grid);
    // (mixed_split_kernel's decode side is this launch's kernel, the append
    // included.)
    if (tl_record != nullptr && lds4) {
      tl_record->taken = true;
      tl_record->p = p;
      tl_record->grid = sp.grid;
      tl_record->rows = batch;
      return KVC_OK;
    }
    // The dynamic tail hand-out (bf16 LDS segments): a zeroed claim set for
    // this launch, the tail partials and counts in the workspace.
    StealArgs sa{};
    const int tail = std::min(kDecTailMax, std::max(0, env_int("KVC_DECODE_TAIL", kDecTailDefault)));
    if (lds4 && steal_shape(hp) && tail > 0 && env_int("KVC_DECODE_STEAL", 0) != 0) {
      unsigned long long* claims = claim_set(st, sp.grid);
      if (claims != nullptr) {
        char* ws = static_cast<char*>(workspace);
        sa.claims = claims;
        sa.stolen = reinterpret_cast<int*>(ws + sl.stolen);
        sa.tail_o = reinterpret_cast<float*>(ws + sl.tail_o);
        sa.tail_lse = reinterpret_cast<float*>(ws + sl.tail_lse);
        sa.dummy = reinterpret_cast<int*>(ws + sl.dummy);
        sa.tail = tail;
        sa.uh = hp.kvs_per_wg * hp.hs;
        sa.grid = sp.grid;
        sa.steal_min = std::max(1, env_int("KVC_STEAL_MIN", kStealMinDefault));
      }
    }
    if (sa.claims != nullptr) {
      paged_decode_steal_kernel<<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens, sa);
      rc = check_launch("paged_decode");
      if (rc != KVC_OK) return rc;
      launch_merge_steal(p, batch, sa, st);
      return check_launch("paged_decode merge");
    }
    switch (kv_dtype) {
      case KVC_KV_BF16:
        if (lds4) {
          paged_decode_sk_kernel<kBF16, true>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        } else if (lds_bf16) {
          paged_decode_sk2_kernel<<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        } else {
          paged_decode_sk_kernel<kBF16, false>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        }
        break;
      case KVC_KV_INT8_TOKHEAD:
        if (hp.kvs_per_wg == 4 && hp.nslices == 1 && env_int("KVC_DECODE_LDS", 1) != 0) {
          paged_decode_sk_kernel<kI8Tok, true>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        } else {
          paged_decode_sk_kernel<kI8Tok, false>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        }
        break;
      default:
        // The LDS ring takes side widths of 2, 4 or 8 (16-byte loads of whole
        // side rows); width 1 runs the register segment.
        if (hp.kvs_per_wg == 4 && hp.nslices == 1 && env_int("KVC_DECODE_LDS", 1) != 0 &&
            (head_n_out == nullptr || n_out_max >= 2)) {
          paged_decode_sk_kernel<kI8Chan, true>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        } else {
          paged_decode_sk_kernel<kI8Chan, false>
              <<<sp.grid, kThreads, 0, st>>>(p, block_tables, context_lens);
        }
        break;
    }
    rc = check_launch("paged_decode");
    if (rc != KVC_OK) return rc;
    launch_merge(p, batch, st);
    return check_launch("paged_decode merge");
  }
  if (app.key != nullptr) {
    rc = store_append(app, k_cache, v_cache, k_scale, v_scale,
                      SidePool{side_k, side_v, out_idx2d, head_n_out, n_out_max},
                      num_cache_blocks * page_size,
                      batch, num_kv_heads, kv_dtype, stream);
    if (rc != KVC_OK) return rc;
  }
  p.chunk_tokens = plan_decode_chunk(batch, hp.groups, max_ctx);
  KVC_REQUIRE(p.chunk_tokens % kTile == 0, KVC_ERR_VALUE,
              "paged_decode: decode chunk must be a multiple of 32");
  p.dec_max_chunks = int((max_ctx + p.chunk_tokens - 1) / p.chunk_tokens);
  p.max_splits = p.dec_max_chunks;
  const size_t need = partial_bytes(batch, num_heads, p.max_splits);
  KVC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), KVC_ERR_WORKSPACE,
              "paged_decode: workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
  set_partials(p, workspace, batch);
  const int64_t units = batch * hp.groups * p.dec_max_chunks;
  KVC_REQUIRE(units < (int64_t(1) << 31), KVC_ERR_VALUE, "paged_decode: launch too large");
  p.dec_units = int(units);
  switch (kv_dtype) {
    case KVC_KV_BF16: launch_decode_enc<kBF16>(p, int(units), st); break;
    case KVC_KV_INT8_TOKHEAD: launch_decode_enc<kI8Tok>(p, int(units), st); break;
    default: launch_decode_enc<kI8Chan>(p, int(units), st); break;
  }
  rc = check_launch("paged_decode");
  if (rc != KVC_OK) return rc;
  if (p.max_splits > 1) {
    launch_merge(p, batch, st);
    rc = check_launch("paged_decode merge");
  }
  return rc;
}
}  // namespace

extern "C" int kvc_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache,
                                int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads,
                                int64_t head_dim, int kv_dtype, const float* k_scale,
                                const float* v_scale, const void* side_k, const void* side_v,
                                const int32_t* out_idx2d, const int32_t* head_n_out,
                                int64_t n_out_max, const int32_t* block_tables, int64_t bt_stride,
                                int64_t max_blocks_per_seq, const int32_t* context_lens,
                                int64_t batch, int64_t num_heads, float scale, void* out,
                                int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                                size_t workspace_bytes, kvc_stream_t stream) {
  return paged_decode_impl(q, q_stride_b, q_stride_h, k_cache, v_cache, num_cache_blocks,
                           page_size, num_kv_heads, head_dim, kv_dtype, k_scale, v_scale, side_k,
                           side_v, out_idx2d, head_n_out, n_out_max, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, batch, num_heads, scale, out,
                           out_stride_b, out_stride_h, workspace, workspace_bytes,
                           DecodeAppend{}, stream);
}

extern "C" int kvc_paged_decode_append(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, void* k_cache, void* v_cache,
    int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
    const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale, void* out,
    int64_t out_stride_b, int64_t out_stride_h, void* workspace, size_t workspace_bytes,
    kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(key != nullptr && value != nullptr && slot_mapping != nullptr, KVC_ERR_VALUE,
              "paged_decode_append: key, value and slot_mapping are required");
  KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
              "paged_decode_append: slot_mapping must be int32 or int64");
  const DecodeAppend app{key, key_stride_n, key_stride_h, value, value_stride_n, value_stride_h,
                         slot_mapping, slot_index_bytes};
  return paged_decode_impl(q, q_stride_b, q_stride_h, k_cache, v_cache, num_cache_blocks,
                           page_size, num_kv_heads, head_dim, KVC_KV_BF16, nullptr, nullptr,
                           nullptr, nullptr, nullptr, nullptr, 0, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, batch, num_heads, scale, out,
                           out_stride_b, out_stride_h, workspace, workspace_bytes, app, stream);
}

extern "C" int kvc_paged_decode_append_int8(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, int8_t* k_cache, int8_t* v_cache,
    float* k_scale, float* v_scale, int64_t num_cache_blocks, int64_t page_size,
    int64_t num_kv_heads, int64_t head_dim, const int32_t* block_tables, int64_t bt_stride,
    int64_t max_blocks_per_seq, const int32_t* context_lens, int64_t batch, int64_t num_heads,
    float scale, void* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(key != nullptr && value != nullptr && slot_mapping != nullptr, KVC_ERR_VALUE,
              "paged_decode_append_int8: key, value and slot_mapping are required");
  KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
              "paged_decode_append_int8: slot_mapping must be int32 or int64");
  const DecodeAppend app{key, key_stride_n, key_stride_h, value, value_stride_n, value_stride_h,
                         slot_mapping, slot_index_bytes};
  return paged_decode_impl(q, q_stride_b, q_stride_h, k_cache, v_cache, num_cache_blocks,
                           page_size, num_kv_heads, head_dim, KVC_KV_INT8_TOKHEAD, k_scale,
                           v_scale, nullptr, nullptr, nullptr, nullptr, 0, block_tables,
                           bt_stride, max_blocks_per_seq, context_lens, batch, num_heads, scale,
                           out, out_stride_b, out_stride_h, workspace, workspace_bytes, app,
                           stream);
}

extern "C" int kvc_paged_decode_append_int8_chan(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, int8_t* k_cache, int8_t* v_cache,
    const float* k_scale, const float* v_scale, const float* k_dscale, const float* v_dscale,
    void* side_k, void* side_v, const int32_t* out_idx2d, const int32_t* head_n_out,
    int64_t n_out_max, int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads,
    int64_t head_dim, const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale, void* out,
    int64_t out_stride_b, int64_t out_stride_h, void* workspace, size_t workspace_bytes,
    kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(key != nullptr && value != nullptr && slot_mapping != nullptr, KVC_ERR_VALUE,
              "paged_decode_append_int8_chan: key, value and slot_mapping are required");
  KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
              "paged_decode_append_int8_chan: slot_mapping must be int32 or int64");
  KVC_REQUIRE(k_scale != nullptr && v_scale != nullptr, KVC_ERR_VALUE,
              "paged_decode_append_int8_chan: the store scales are required");
  DecodeAppend app{key, key_stride_n, key_stride_h, value, value_stride_n, value_stride_h,
                   slot_mapping, slot_index_bytes};
  app.store_k_scale = k_scale;
  app.store_v_scale = v_scale;
  return paged_decode_impl(q, q_stride_b, q_stride_h, k_cache, v_cache, num_cache_blocks,
                           page_size, num_kv_heads, head_dim, KVC_KV_INT8_CHAN, k_dscale,
                           v_dscale, side_k, side_v, out_idx2d, head_n_out, n_out_max,
                           block_tables, bt_stride, max_blocks_per_seq, context_lens, batch,
                           num_heads, scale, out, out_stride_b, out_stride_h, workspace,
                           workspace_bytes, app, stream);
}

// The decode step without a caller workspace: the split-K partials and split
// counts live in the library's static scratch array of the stream's device
// (kvc_scratch.hip).  The array needs no clearing: each launch writes every
// split count and partial its merge reads.
extern "C" int kvc_paged_decode_append_static(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* key, int64_t key_stride_n,
    int64_t key_stride_h, const void* value, int64_t value_stride_n, int64_t value_stride_h,
    const void* slot_mapping, int slot_index_bytes, void* k_cache, void* v_cache,
    int64_t num_cache_blocks, int64_t page_size, int64_t num_kv_heads, int64_t head_dim,
    const int32_t* block_tables, int64_t bt_stride, int64_t max_blocks_per_seq,
    const int32_t* context_lens, int64_t batch, int64_t num_heads, float scale, void* out,
    int64_t out_stride_b, int64_t out_stride_h, kvc_stream_t stream) {
  clear_error();
  const size_t need = kvc_paged_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim,
                                                       page_size, max_blocks_per_seq);
  KVC_REQUIRE(need <= size_t(KVC_STATIC_SCRATCH_BYTES), KVC_ERR_WORKSPACE,
              "paged_decode_append_static: this launch needs %zu bytes of split-K scratch; the "
              "static scratch holds %zu (batch %lld, %lld heads, %lld-block tables): use "
              "kvc_paged_decode_append with a workspace",
              need, size_t(KVC_STATIC_SCRATCH_BYTES), (long long)batch, (long long)num_heads,
              (long long)max_blocks_per_seq);
  if (batch == 0) {
    return kvc_paged_decode_append(q, q_stride_b, q_stride_h, key, key_stride_n, key_stride_h,
                                   value, value_stride_n, value_stride_h, slot_mapping,
                                   slot_index_bytes, k_cache, v_cache, num_cache_blocks,
                                   page_size, num_kv_heads, head_dim, block_tables, bt_stride,
                                   max_blocks_per_seq, context_lens, batch, num_heads, scale, out,
                                   out_stride_b, out_stride_h, nullptr, 0, stream);
  }
  int dev = 0;
  int rc = stream_device(as_stream(stream), &dev);
  if (rc != KVC_OK) return rc;
  void* ws = nullptr;
  rc = scratch_for_device(dev, &ws);
  if (rc != KVC_OK) return rc;
  return kvc_paged_decode_append(q, q_stride_b, q_stride_h, key, key_stride_n, key_stride_h,
                                 value, value_stride_n, value_stride_h, slot_mapping,
                                 slot_index_bytes, k_cache, v_cache, num_cache_blocks, page_size,
                                 num_kv_heads, head_dim, block_tables, bt_stride,
                                 max_blocks_per_seq, context_lens, batch, num_heads, scale, out,
                                 out_stride_b, out_stride_h, ws, size_t(KVC_STATIC_SCRATCH_BYTES),
                                 stream);
}

extern "C" size_t kvc_varlen_workspace_bytes(int64_t num_q_tokens, int64_t num_heads,
                                             int64_t num_kv_heads, int64_t head_dim,
                                             int64_t num_decode_rows, int64_t max_seqlen_k,
                                             int64_t page_size, int64_t max_blocks_per_seq) {
  if (num_q_tokens <= 0 || num_kv_heads <= 0 || head_dim != kD) return 0;
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  if (split_mixed(num_decode_rows, page_size)) {
    // Decode rows through the paged decode launch, then the prefill rows.
    const size_t dec = kvc_paged_decode_workspace_bytes(num_decode_rows, num_heads, num_kv_heads,
                                                        head_dim, page_size, max_blocks_per_seq);
    const size_t pre = kvc_varlen_workspace_bytes(num_q_tokens - num_decode_rows, num_heads,
                                                  num_kv_heads, head_dim, 0, max_seqlen_k,
                                                  page_size, max_blocks_per_seq);
    return (dec + 255) / 256 * 256 + pre;
  }
  // Prefill rows only (decode rows without a paged pool are refused).
  int64_t splits = 1;
  if (max_seqlen_k > 0) {
    const int ks = plan_prefill_split(max_seqlen_k);
    const int64_t ps = (max_seqlen_k + ks - 1) / ks;
    splits = ps > splits ? ps : splits;
  }
  const size_t units = partial_bytes(num_q_tokens, num_heads, splits);
  if (prefill_stream_k(num_decode_rows)) {
    const SkPlan sp = plan_prefill_sk(num_q_tokens, num_heads, max_seqlen_k);
    const size_t sk =
        sk_workspace_bytes(num_q_tokens, num_heads, num_kv_heads * hp.nslices, sp.max_splits);
    return sk > units ? sk : units;
  }
  return units;
}

namespace {
// kvc_varlen_attention with the decode rows' append (app.key null: none; rows
// [0, num_decode_rows) of app's key / value / slot_mapping) and the split
// hints of mixed_decode_cus.
int varlen_impl(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t num_q_tokens,
    int64_t num_heads, const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
    int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int kv_dtype,
    const float* k_scale, const float* v_scale, const void* side_k, const void* side_v,
    const int32_t* out_idx2d, const int32_t* head_n_out, int64_t n_out_max, const void* k_fresh,
    int64_t kf_stride_t, int64_t kf_stride_h, const void* v_fresh, int64_t vf_stride_t,
    int64_t vf_stride_h, const int32_t* block_tables, int64_t bt_stride,
    int64_t max_blocks_per_seq, int64_t num_decode_rows, const int32_t* decode_context_lens,
    int64_t num_prefill, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    int64_t num_prefill_units, int64_t max_seqlen_k, int64_t decode_ctx_tokens,
    int64_t prefill_kq_pairs, float scale, void* out, int64_t out_stride_t, int64_t out_stride_h,
    void* workspace, size_t workspace_bytes, const DecodeAppend& app, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(head_dim == kD, KVC_ERR_VALUE, "varlen_attention: head_dim must be 128 (got %lld)",
              (long long)head_dim);
  KVC_REQUIRE(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0, KVC_ERR_VALUE,
              "varlen_attention: num_heads must be a multiple of num_kv_heads");
  const bool fresh = block_tables == nullptr;
  if (!fresh) {
    KVC_REQUIRE(page_size > 0 && page_size % kTile == 0, KVC_ERR_VALUE,
                "varlen_attention: page_size must be a positive multiple of 32");
    KVC_REQUIRE(max_blocks_per_seq > 0, KVC_ERR_VALUE, "varlen_attention: empty block_tables");
  } else {
    KVC_REQUIRE(num_decode_rows == 0, KVC_ERR_VALUE,
                "varlen_attention: decode rows need block_tables");
    KVC_REQUIRE(k_fresh != nullptr && v_fresh != nullptr, KVC_ERR_VALUE,
                "varlen_attention: without block_tables keys come from k_fresh/v_fresh");
    KVC_REQUIRE((kf_stride_t % 8) == 0 && (kf_stride_h % 8) == 0 && (vf_stride_t % 8) == 0 &&
                    (vf_stride_h % 8) == 0 && (reinterpret_cast<uintptr_t>(k_fresh) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(v_fresh) % 16) == 0,
                KVC_ERR_ASSERT, "varlen_attention: k/v rows must be 16-byte aligned");
  }
  int rc = check_kv_args(fresh ? KVC_KV_BF16 : kv_dtype, k_scale, v_scale, side_k, side_v,
                         out_idx2d, head_n_out, n_out_max, "varlen_attention");
  if (rc != KVC_OK) return rc;
  // Fresh rows gathered from a per-channel pool (kvc_gather_kv) name its
  // outlier dims through out_idx2d / head_n_out (side pools unused).
  const bool fresh_outliers = fresh && head_n_out != nullptr;
  if (fresh_outliers) {
    KVC_REQUIRE(out_idx2d != nullptr, KVC_ERR_VALUE,
                "varlen_attention: head_n_out needs out_idx2d");
    KVC_REQUIRE(n_out_max >= 1 && n_out_max <= kSideMax && (n_out_max & (n_out_max - 1)) == 0,
                KVC_ERR_VALUE, "varlen_attention: n_out_max must be 1, 2, 4 or 8 (got %lld)",
                (long long)n_out_max);
  }
  KVC_REQUIRE((q_stride_t % 8) == 0 && (q_stride_h % 8) == 0 && (out_stride_t % 8) == 0 &&
                  (out_stride_h % 8) == 0 && (reinterpret_cast<uintptr_t>(q) % 16) == 0 &&
                  (reinterpret_cast<uintptr_t>(out) % 16) == 0,
              KVC_ERR_ASSERT, "varlen_attention: q/out rows must be 16-byte aligned");
  KVC_REQUIRE(num_prefill == 0 || (cu_seqlens_q != nullptr && cu_seqlens_k != nullptr),
              KVC_ERR_VALUE, "varlen_attention: prefill chunks need cu_seqlens_q/k");
  (void)num_cache_blocks;
  if (num_q_tokens == 0) return KVC_OK;

  if (!fresh && split_mixed(num_decode_rows, page_size)) {
    KVC_REQUIRE(decode_context_lens != nullptr, KVC_ERR_VALUE,
                "varlen_attention: decode rows need decode_context_lens");
    KVC_REQUIRE(num_q_tokens >= num_decode_rows, KVC_ERR_VALUE,
                "varlen_attention: fewer query rows than decode rows");
    const size_t dec_ws = kvc_paged_decode_workspace_bytes(num_decode_rows, num_heads,
                                                           num_kv_heads, head_dim, page_size,
                                                           max_blocks_per_seq);
    const size_t dec_span = (dec_ws + 255) / 256 * 256;
    const size_t pre_ws = kvc_varlen_workspace_bytes(num_q_tokens - num_decode_rows, num_heads,
                                                     num_kv_heads, head_dim, 0, max_seqlen_k,
                                                     page_size, max_blocks_per_seq);
    KVC_REQUIRE((dec_span + pre_ws == 0) ||
                    (workspace != nullptr && workspace_bytes >= dec_span + pre_ws),
                KVC_ERR_WORKSPACE, "varlen_attention: workspace of %zu bytes needed (got %zu)",
                dec_span + pre_ws, workspace_bytes);
    char* ws = static_cast<char*>(workspace);
    const int64_t nd = num_decode_rows;
    const int dec_cus = mixed_decode_cus(nd, num_q_tokens - nd, kv_dtype, num_heads, num_kv_heads,
                                         decode_ctx_tokens, prefill_kq_pairs);
    if (dec_cus > 0) {
      // One launch over a static CU split (mixed_split_kernel): the decode
      // rows planned for dec_cus workgroups, the prefill rows for the rest,
      // each recorded by its own entry point, then both merges.
      hipStream_t main_st = as_stream(stream);
      SkRecord rd, rp;
      {
        LaunchCus cus(dec_cus);
        RecordInto rec(&rd);
        rc = paged_decode_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_cache_blocks,
                               page_size, num_kv_heads, head_dim, kv_dtype, k_scale, v_scale,
                               side_k, side_v, out_idx2d, head_n_out, n_out_max, block_tables,
                               bt_stride, max_blocks_per_seq, decode_context_lens, nd, num_heads,
                               scale, out, out_stride_t, out_stride_h, dec_ws ? ws : nullptr,
                               dec_ws, app, stream);
      }
      if (rc != KVC_OK) return rc;
      {
        LaunchCus cus(device_cus() - dec_cus);
        RecordInto rec(&rp);
        rc = varlen_impl(
            static_cast<const uint16_t*>(q) + nd * q_stride_t, q_stride_t, q_stride_h,
            num_q_tokens - nd, num_heads, k_cache, v_cache, num_cache_blocks, page_size,
            num_kv_heads, head_dim, kv_dtype, k_scale, v_scale, side_k, side_v, out_idx2d,
            head_n_out, n_out_max, nullptr, 0, 0, nullptr, 0, 0, block_tables + nd * bt_stride,
            bt_stride, max_blocks_per_seq, 0, nullptr, num_prefill, cu_seqlens_q, cu_seqlens_k,
            num_prefill_units, max_seqlen_k, 0, 0, scale,
            static_cast<uint16_t*>(out) + nd * out_stride_t, out_stride_t, out_stride_h,
            pre_ws ? ws + dec_span : nullptr, pre_ws, DecodeAppend{}, stream);
      }
      if (rc != KVC_OK) return rc;
      if (rd.taken && rp.taken) {
        mixed_split_kernel<<<rd.grid + rp.grid, kThreads, 0, main_st>>>(rd.p, rp.p, rd.grid);
        rc = check_launch("varlen_attention");
        if (rc != KVC_OK) return rc;
      } else if (rd.taken) {
        paged_decode_sk_kernel<kBF16, true>
            <<<rd.grid, kThreads, 0, main_st>>>(rd.p, rd.p.block_tables, rd.p.ctx_lens);
        rc = check_launch("varlen_attention decode");
        if (rc != KVC_OK) return rc;
      } else if (rp.taken) {
        launch_prefill_sk(rp.p, rp.grid, false, main_st);
        rc = check_launch("varlen_attention prefill");
        if (rc != KVC_OK) return rc;
      }
      if (rd.taken && rp.taken) {
        const int64_t dec_blocks = (rd.rows * rd.p.num_heads + kMergeWaves - 1) / kMergeWaves;
        const int64_t pre_blocks =
            (rp.rows * rp.p.kvh * rp.p.nslices + kMergeWaves - 1) / kMergeWaves;
        merge_mixed_kernel<<<unsigned(dec_blocks + pre_blocks), 64 * kMergeWaves, 0, main_st>>>(
            rd.p, rp.p, int(rd.rows), int(dec_blocks), int(rp.rows));
      } else {
        if (rd.taken) launch_merge(rd.p, rd.rows, main_st);
        if (rp.taken) launch_merge_slices(rp.p, rp.rows, main_st);
      }
      return check_launch("varlen_attention merge");
    }
    rc = paged_decode_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_cache_blocks,
                           page_size, num_kv_heads, head_dim, kv_dtype, k_scale, v_scale, side_k,
                           side_v, out_idx2d, head_n_out, n_out_max, block_tables, bt_stride,
                           max_blocks_per_seq, decode_context_lens, num_decode_rows, num_heads,
                           scale, out, out_stride_t, out_stride_h, dec_ws ? ws : nullptr, dec_ws,
                           app, stream);
    if (rc != KVC_OK || num_q_tokens == num_decode_rows) return rc;
    return varlen_impl(
        static_cast<const uint16_t*>(q) + nd * q_stride_t, q_stride_t, q_stride_h,
        num_q_tokens - nd, num_heads, k_cache, v_cache, num_cache_blocks, page_size,
        num_kv_heads, head_dim, kv_dtype, k_scale, v_scale, side_k, side_v, out_idx2d,
        head_n_out, n_out_max, nullptr, 0, 0, nullptr, 0, 0, block_tables + nd * bt_stride,
        bt_stride, max_blocks_per_seq, 0, nullptr, num_prefill, cu_seqlens_q, cu_seqlens_k,
        num_prefill_units, max_seqlen_k, 0, 0, scale,
        static_cast<uint16_t*>(out) + nd * out_stride_t, out_stride_t, out_stride_h,
        pre_ws ? ws + dec_span : nullptr, pre_ws, DecodeAppend{}, stream);
  }

  // Prefill rows only from here: decode rows went to the paged decode above
  // (with block tables the page size is positive; without, decode rows are
  // refused).
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  AttnParams p{};
  p.merge_first = 0;  // most rows of these launches are not split
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_stride_t;
  p.q_sh = q_stride_h;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = out_stride_t;
  p.o_sh = out_stride_h;
  p.num_heads = int(num_heads);
  p.group = hp.group;
  p.hs = hp.hs;
  p.nslices = hp.nslices;
  p.tpb = hp.tpb;
  p.kvs_per_wg = hp.kvs_per_wg;
  p.scale_log2 = scale * kLog2e;
  fill_kv(p, k_cache, v_cache, page_size, num_kv_heads, fresh ? KVC_KV_BF16 : kv_dtype, k_scale,
          v_scale, side_k, side_v, out_idx2d, head_n_out, n_out_max);
  if (fresh_outliers) {
    p.out_idx = out_idx2d;
    p.head_n_out = head_n_out;
    p.n_out_max = int(n_out_max);
  }
  p.block_tables = block_tables;
  p.bt_stride = bt_stride;
  p.n_dec = 0;
  int64_t max_splits = 1;
  p.chunk_tokens = kTile;
  p.dec_max_chunks = 0;
  p.n_pre = int(num_prefill);
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.split_tokens = plan_prefill_split(max_seqlen_k);
  if (max_seqlen_k > 0) {
    const int64_t ps = (max_seqlen_k + p.split_tokens - 1) / p.split_tokens;
    max_splits = ps > max_splits ? ps : max_splits;
  }
  p.kf = static_cast<const uint16_t*>(k_fresh);
  p.kf_st = kf_stride_t;
  p.kf_sh = kf_stride_h;
  p.vf = static_cast<const uint16_t*>(v_fresh);
  p.vf_st = vf_stride_t;
  p.vf_sh = vf_stride_h;
  if (prefill_stream_k(num_decode_rows) && (fresh || kv_dtype == KVC_KV_BF16) &&
      num_q_tokens * q_stride_t * 2 < (int64_t(1) << 31)) {
    // Prefill rows only, bf16 keys: one workgroup per CU over the
    // concatenated tiles of every item (prefill_sk2_kernel), then the merge.
    const int64_t kv_slices = num_kv_heads * hp.nslices;
    const int64_t qtile = int64_t(kWaves) * kPreNCB * hp.tpb;
    const int64_t bound =
        kv_slices * (num_q_tokens / qtile + num_prefill + 1) * ((max_seqlen_k + kTile - 1) / kTile);
    KVC_REQUIRE(bound < (int64_t(1) << 30), KVC_ERR_VALUE, "varlen_attention: launch too large");
    const SkPlan sp = plan_prefill_sk(num_q_tokens, num_heads, max_seqlen_k);
    p.max_splits = sp.max_splits;
    p.sk_min_share = kPfMinShare;
    p.merge_first = 0;
    const size_t need = sk_workspace_bytes(num_q_tokens, num_heads, kv_slices, sp.max_splits);
    KVC_REQUIRE(workspace != nullptr && workspace_bytes >= need, KVC_ERR_WORKSPACE,
                "varlen_attention: workspace of %zu bytes needed (got %zu)", need,
                workspace_bytes);
    set_partials(p, workspace, num_q_tokens);
    p.sk_nseg = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                       sk_partial_part(num_q_tokens, num_heads, p.max_splits));
    hipStream_t st = as_stream(stream);
    if (num_prefill > 0 && tl_record != nullptr && !fresh) {
      tl_record->taken = true;
      tl_record->p = p;
      tl_record->grid = sp.grid;
      tl_record->rows = num_q_tokens;
      return KVC_OK;
    }
    if (num_prefill > 0) {
      // Per-workgroup stamps for diagnostics (KVC_PREFILL_STAMPS=1), read
      // back through kvc_decode_stamps.
      if (env_int("KVC_PREFILL_STAMPS", 0) != 0 && sp.grid <= stamp_slots())
        p.wg_stamps = stamp_buffer(sp.grid);
      launch_prefill_sk(p, sp.grid, fresh, st);
      rc = check_launch("varlen_attention");
      if (rc != KVC_OK) return rc;
      launch_merge_slices(p, num_q_tokens, st);
      rc = check_launch("varlen_attention merge");
    }
    return rc;
  }
  p.max_splits = int(max_splits);
  const size_t need = partial_bytes(num_q_tokens, num_heads, max_splits);
  KVC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), KVC_ERR_WORKSPACE,
              "varlen_attention: workspace of %zu bytes needed (got %zu)", need,
              workspace_bytes);
  set_partials(p, workspace, num_q_tokens);
  KVC_REQUIRE(num_prefill_units < (int64_t(1) << 31) && num_prefill_units >= 0, KVC_ERR_VALUE,
              "varlen_attention: launch too large");
  p.dec_units = 0;
  p.pre_units = int(num_prefill_units);
  const int grid = int(num_prefill_units);
  hipStream_t st = as_stream(stream);
  if (grid > 0) {
    switch (fresh ? KVC_KV_BF16 : kv_dtype) {
      case KVC_KV_BF16: launch_varlen_enc<kBF16>(p, grid, fresh, st); break;
      case KVC_KV_INT8_TOKHEAD: launch_varlen_enc<kI8Tok>(p, grid, false, st); break;
      default: launch_varlen_enc<kI8Chan>(p, grid, false, st); break;
    }
    rc = check_launch("varlen_attention");
    if (rc != KVC_OK) return rc;
  }
  if (p.max_splits > 1) {
    launch_merge(p, num_q_tokens, st);
    rc = check_launch("varlen_attention merge");
  }
  return rc;
}

}  // namespace

extern "C" int kvc_varlen_attention(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t num_q_tokens,
    int64_t num_heads, const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
    int64_t page_size, int64_t num_kv_heads, int64_t head_dim, int kv_dtype,
    const float* k_scale, const float* v_scale, const void* side_k, const void* side_v,
    const int32_t* out_idx2d, const int32_t* head_n_out, int64_t n_out_max, const void* k_fresh,
    int64_t kf_stride_t, int64_t kf_stride_h, const void* v_fresh, int64_t vf_stride_t,
    int64_t vf_stride_h, const int32_t* block_tables, int64_t bt_stride,
    int64_t max_blocks_per_seq, int64_t num_decode_rows, const int32_t* decode_context_lens,
    int64_t num_prefill, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    int64_t num_prefill_units, int64_t max_seqlen_k, int64_t decode_ctx_tokens,
    int64_t prefill_kq_pairs, float scale, void* out, int64_t out_stride_t, int64_t out_stride_h,
    void* workspace, size_t workspace_bytes, kvc_stream_t stream) {
  return varlen_impl(q, q_stride_t, q_stride_h, num_q_tokens, num_heads, k_cache, v_cache,
                     num_cache_blocks, page_size, num_kv_heads, head_dim, kv_dtype, k_scale,
                     v_scale, side_k, side_v, out_idx2d, head_n_out, n_out_max, k_fresh,
                     kf_stride_t, kf_stride_h, v_fresh, vf_stride_t, vf_stride_h, block_tables,
                     bt_stride, max_blocks_per_seq, num_decode_rows, decode_context_lens,
                     num_prefill, cu_seqlens_q, cu_seqlens_k, num_prefill_units, max_seqlen_k,
                     decode_ctx_tokens, prefill_kq_pairs, scale, out, out_stride_t, out_stride_h,
                     workspace, workspace_bytes, DecodeAppend{}, stream);
}

// The step's store and the mixed call together (bf16 pool): the prefill rows'
// k/v go to their slots first (one store launch: the prefill attention reads
// them back from the pool), then the call runs as kvc_varlen_attention with
// the decode rows' k/v appended inside the decode launch (or the decode side
// of the split launch), as kvc_paged_decode_append does.
extern "C" int kvc_varlen_attention_append(
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
    size_t workspace_bytes, kvc_stream_t stream) {
  clear_error();
  KVC_REQUIRE(key != nullptr && value != nullptr && slot_mapping != nullptr, KVC_ERR_VALUE,
              "varlen_attention_append: key, value and slot_mapping are required");
  KVC_REQUIRE(slot_index_bytes == 4 || slot_index_bytes == 8, KVC_ERR_VALUE,
              "varlen_attention_append: slot_mapping must be int32 or int64");
  KVC_REQUIRE(block_tables != nullptr && k_cache != nullptr && v_cache != nullptr, KVC_ERR_VALUE,
              "varlen_attention_append: a paged pool and block_tables are required");
  KVC_REQUIRE(num_decode_rows >= 0 && num_decode_rows <= num_q_tokens, KVC_ERR_VALUE,
              "varlen_attention_append: fewer query rows than decode rows");
  KVC_REQUIRE(page_size > 0 && num_cache_blocks >= 0, KVC_ERR_VALUE,
              "varlen_attention_append: bad pool shape");
  const int64_t nd = num_decode_rows;
  if (num_q_tokens > nd) {
    const int rc = kvc_store_kv(
        static_cast<const uint16_t*>(key) + nd * key_stride_t, key_stride_t, key_stride_h,
        static_cast<const uint16_t*>(value) + nd * value_stride_t, value_stride_t,
        value_stride_h, k_cache, v_cache, num_cache_blocks * page_size,
        static_cast<const char*>(slot_mapping) + nd * slot_index_bytes, slot_index_bytes,
        num_q_tokens - nd, num_kv_heads, head_dim, 2, stream);
    if (rc != KVC_OK) return rc;
  }
  const DecodeAppend app{key, key_stride_t, key_stride_h, value, value_stride_t, value_stride_h,
                         slot_mapping, slot_index_bytes};
  return varlen_impl(q, q_stride_t, q_stride_h, num_q_tokens, num_heads, k_cache, v_cache,
                     num_cache_blocks, page_size, num_kv_heads, head_dim, KVC_KV_BF16, nullptr,
                     nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, 0, nullptr, 0,
                     0, block_tables, bt_stride, max_blocks_per_seq, num_decode_rows,
                     decode_context_lens, num_prefill, cu_seqlens_q, cu_seqlens_k,
                     num_prefill_units, max_seqlen_k, decode_ctx_tokens, prefill_kq_pairs, scale,
                     out, out_stride_t, out_stride_h, workspace, workspace_bytes,
                     nd > 0 ? app : DecodeAppend{}, stream);
}

// Decode CUs of a mixed call's split launch for these sizes and hints (0: the
// decode launch, then the prefill launch).
extern "C" int kvc_varlen_decode_cus(int64_t num_decode_rows, int64_t num_prefill_tokens,
                                     int64_t num_heads, int64_t num_kv_heads, int kv_dtype,
                                     int64_t decode_ctx_tokens, int64_t prefill_kq_pairs) {
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0) return 0;
  return mixed_decode_cus(num_decode_rows, num_prefill_tokens, kv_dtype, num_heads, num_kv_heads,
                          decode_ctx_tokens, prefill_kq_pairs);
}

// Number of prefill workgroups for the given chunk lengths (host arrays of
// num_prefill + 1 cumulative offsets), matching the kernel's unit order.
extern "C" int64_t kvc_varlen_prefill_units(const int32_t* cu_q_host, const int32_t* cu_k_host,
                                            int64_t num_prefill, int64_t num_heads,
                                            int64_t num_kv_heads, int64_t max_seqlen_k) {
  if (num_prefill <= 0 || num_kv_heads <= 0) return 0;
  const HeadPlan hp = plan_heads(num_heads, num_kv_heads);
  const int ks = plan_prefill_split(max_seqlen_k);
  const int qtile_tokens = kWaves * kPreNCB * hp.tpb;
  int64_t units = 0;
  for (int64_t i = 0; i < num_prefill; ++i) {
    const int64_t sq = cu_q_host[i + 1] - cu_q_host[i];
    const int64_t sk = cu_k_host[i + 1] - cu_k_host[i];
    if (sq <= 0 || sk <= 0) continue;
    const int64_t ntq = (sq + qtile_tokens - 1) / qtile_tokens;
    const int64_t ns = (sk + ks - 1) / ks;
    units += ntq * num_kv_heads * hp.nslices * (ns < 1 ? 1 : ns);
  }
  return units;
}
