// Prefill / verify grouped path: token-sorted grouped GEMMs on bf16 MFMA.
//
// Reference path: StreamingSwitchGLU._one_pass/_issue
// (models/flashnext/expert_cache.py:1743-1810) sorts the flattened
// (token, slot) rows by expert (build_plan :750-760 and mlx-vlm _gather_sort),
// runs gather_qmm(transpose=True, group 32, bits 4) for gate and up, the
// SwiGLU activation, gather_qmm for down, unsorts, and combines the slots in
// bf16 (models/flashnext/adaptive_topk.py:274-277).
//
// Here:
//   1. count / plan / scatter: a counting sort of the rows by route key (pool
//      slot or expert id; the shared expert is one more key over all tokens)
//      and a tile list of (route word, first sorted row, rows <= 128), in one
//      block up to 16,384 rows and 12,288 keys, else in four kernels;
//   2. gate/up GEMM: a persistent grid of 8-wave blocks (one per CU) walks
//      (tile, 128 features) items.  Each wave streams 32 weight rows (waves
//      0-3 gate, 4-7 up) straight into registers, dequantizes them to bf16
//      MFMA operands there, and multiplies them with the tile's token rows,
//      staged 128 inputs per stage in LDS, on v_mfma_f32_32x32x16_bf16
//      (fp32 accumulate); the epilogue rounds gate and up to bf16 and writes
//      act = swiglu(g, u) in sorted row order;
//   3. down GEMM: per (tile, 256 features) the same scheme over act, the
//      bf16 outputs are scattered back to y[token, slot] (or the shared
//      expert's row);
//   4. combine: out = bf16 generic combine of y with the scores + the gated
//      shared expert.
// Weights are dequantized as bf16(fma(q, s, b)) (one float32 rounding, then
// bf16); every output row is computed independently of its position in a
// tile, so the result does not depend on the order rows land in a tile.
#include <mutex>

#include "mq_internal.h"
#include "mq_select.h"

namespace mq {
namespace {

constexpr uint32_t kTileRows = 128;  // sorted rows (tokens) per tile: four 32-row slabs
constexpr uint32_t kKS = 128;        // inputs per pipeline stage
constexpr uint32_t kGemmWaves = 8;                      // waves per GEMM block (one block per CU)
constexpr uint32_t kGemmThreads = 64 * kGemmWaves;
constexpr uint32_t kWRows = kGemmWaves * 32;            // weight rows per block: 32 per wave
constexpr uint32_t kGateUpFeatures = kWRows / 2;        // per gate/up block: 128 gate + 128 up rows
constexpr uint32_t kDownFeatures = kWRows;              // per down block
constexpr uint32_t kXParts = kGemmThreads / kTileRows;  // threads per activation row of a stage
constexpr uint32_t kXChunks = kKS / 8 / kXParts;        // 16-byte chunks per thread and stage
constexpr uint32_t kSharedWord = 0xfffffffeu;  // tile word of the shared expert group
constexpr uint32_t kDeadWord = 0xffffffffu;    // tile word of rows with invalid route words
constexpr int kPlanThreads = 1024;

// GEMM modes: gate/up (two projections of the token rows, SwiGLU epilogue),
// down (one projection of the sorted act rows, output scattered to y) and
// gather (one projection of caller rows picked through a row map, output
// scattered back to the caller's row order).
constexpr int kModeGateUp = 0;
constexpr int kModeDown = 1;
constexpr int kModeGather = 2;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t2 __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

struct GroupTile {
  uint32_t word;   // route word of the group (kSharedWord / kDeadWord for the extra groups)
  uint32_t start;  // first sorted row
  uint32_t count;  // rows in this tile (1..kTileRows)
  uint32_t pad;
};

// Route keys: pool slots [0, slots), plain ids [slots, slots + ids), then the
// shared group and the dead group.
struct KeySpace {
  uint32_t slots;  // pool slots addressable by slot words
  uint32_t ids;    // plain expert ids
  __host__ __device__ uint32_t shared_key() const { return slots + ids; }
  __host__ __device__ uint32_t dead_key() const { return slots + ids + 1u; }
  __host__ __device__ uint32_t size() const { return slots + ids + 2u; }
};

__device__ __forceinline__ uint32_t key_of(uint32_t word, const KeySpace &ks) {
  if (word & MQ_SLOT_BIT) {
    const uint32_t slot = word & 0x7fffffffu;
    return slot < ks.slots ? slot : ks.dead_key();
  }
  return word < ks.ids ? ks.slots + word : ks.dead_key();
}

__device__ __forceinline__ uint32_t word_of(uint32_t key, const KeySpace &ks) {
  if (key < ks.slots) return MQ_SLOT_BIT | key;
  if (key < ks.slots + ks.ids) return key - ks.slots;
  return key == ks.shared_key() ? kSharedWord : kDeadWord;
}

// Workspace layout (byte offsets, 256-aligned).
struct Layout {
  uint64_t counts, cursor, row_key, order, tiles, n_tiles, act, y_shared, total;
  uint32_t rows, max_tiles;
};

inline uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

Layout make_layout(uint32_t tokens, uint32_t slots, uint32_t hidden, uint32_t inter, uint32_t route_keys,
                   bool shared) {
  Layout l{};
  const uint64_t keys = uint64_t(route_keys) + 2u;
  l.rows = tokens * slots + (shared ? tokens : 0u);
  l.max_tiles = static_cast<uint32_t>((l.rows + kTileRows - 1) / kTileRows + std::min<uint64_t>(l.rows, keys));
  uint64_t off = 0;
  l.counts = off;   off = align256(off + keys * 4);
  l.cursor = off;   off = align256(off + keys * 4);
  l.row_key = off;  off = align256(off + uint64_t(l.rows) * 4);
  l.order = off;    off = align256(off + uint64_t(l.rows) * 4);
  l.tiles = off;    off = align256(off + uint64_t(l.max_tiles) * sizeof(GroupTile));
  l.n_tiles = off;  off = align256(off + 4);
  l.act = off;      off = align256(off + uint64_t(l.rows) * inter * 2);
  l.y_shared = off; off = align256(off + (shared ? uint64_t(tokens) * hidden * 2 : 0));
  l.total = off;
  return l;
}

// Workspace of the gather entry point: the sort arrays and the row map.
struct GatherLayout {
  uint64_t counts, cursor, row_key, order, tiles, n_tiles, xmap, total;
  uint32_t max_tiles;
};

GatherLayout make_gather_layout(uint32_t rows, uint32_t route_keys) {
  GatherLayout l{};
  const uint64_t keys = uint64_t(route_keys) + 2u;
  l.max_tiles = static_cast<uint32_t>((rows + kTileRows - 1) / kTileRows + std::min<uint64_t>(rows, keys));
  uint64_t off = 0;
  l.counts = off;   off = align256(off + keys * 4);
  l.cursor = off;   off = align256(off + keys * 4);
  l.row_key = off;  off = align256(off + uint64_t(rows) * 4);
  l.order = off;    off = align256(off + uint64_t(rows) * 4);
  l.tiles = off;    off = align256(off + uint64_t(l.max_tiles) * sizeof(GroupTile));
  l.n_tiles = off;  off = align256(off + 4);
  l.xmap = off;     off = align256(off + uint64_t(rows) * 4);
  l.total = off;
  return l;
}

// ------------------------------------------------------------------ sort
__global__ void grouped_zero_kernel(uint32_t *p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// counter[key] += 1 for every lane with `active`, with one atomic per
// distinct key in the wave, all issued together (hot experts would otherwise
// serialize thousands of atomics on one address, and one atomic per loop trip
// would serialize their latencies).  With WANT_SLOT, returns the lane's slot:
// the counter's previous value plus the number of lower lanes with its key.
template <bool WANT_SLOT>
__device__ __forceinline__ uint32_t wave_aggregated_increment(uint32_t *counter, uint32_t key, bool active) {
  const int lane = threadIdx.x & 63;
  uint64_t pending = __ballot(active);
  int my_leader = lane;
  uint32_t my_rank = 0u, my_count = 0u;
  while (pending != 0ull) {  // wave-uniform; one trip per distinct key
    const int leader = __builtin_ctzll(pending);
    const uint32_t lkey = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), leader));
    const uint64_t same = __ballot(active && key == lkey) & pending;
    if ((same >> lane) & 1ull) {
      my_leader = leader;
      my_rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(same >> 32),
                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(same), 0u));
    }
    if (lane == leader) my_count = static_cast<uint32_t>(__popcll(same));
    pending &= ~same;
  }
  if constexpr (!WANT_SLOT) {
    if (my_count != 0u) atomicAdd(&counter[key], my_count);
    return 0u;
  } else {
    uint32_t base = 0u;
    if (my_count != 0u) base = atomicAdd(&counter[key], my_count);
    base = static_cast<uint32_t>(__shfl(static_cast<int>(base), my_leader, 64));
    return base + my_rank;
  }
}

__global__ void grouped_count_kernel(const uint32_t *__restrict__ routes, uint32_t routed_rows, uint32_t rows,
                                     KeySpace ks, uint32_t *__restrict__ counts, uint32_t *__restrict__ row_key,
                                     unsigned int *__restrict__ err) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = r < rows;  // no early return: the whole wave takes part in the aggregation
  const uint32_t key = !active ? 0u : (r < routed_rows ? key_of(routes[r], ks) : ks.shared_key());
  if (active) {
    if (key == ks.dead_key()) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);
    row_key[r] = key;
  }
  wave_aggregated_increment<false>(counts, key, active);
}

// One block: exclusive scans of the rows and tiles per key, the scatter
// cursors, and the tile list.  Each thread owns a contiguous run of keys and
// reads each key's count before it writes that key's cursor, so `counts` and
// `cursor` may be the same array (the single-block sort keeps both in LDS).
__device__ __forceinline__ void plan_keys(const uint32_t *counts, uint32_t *cursor, GroupTile *__restrict__ tiles,
                                          uint32_t *__restrict__ n_tiles, KeySpace ks, uint32_t *s_rows,
                                          uint32_t *s_tiles) {
  const uint32_t keys = ks.size();
  const uint32_t per = (keys + kPlanThreads - 1) / kPlanThreads;
  const uint32_t lo = min(threadIdx.x * per, keys), hi = min(lo + per, keys);
  uint32_t rows = 0, ntile = 0;
  for (uint32_t k = lo; k < hi; ++k) {
    const uint32_t c = counts[k];
    rows += c;
    ntile += (c + kTileRows - 1) / kTileRows;
  }
  s_rows[threadIdx.x] = rows;
  s_tiles[threadIdx.x] = ntile;
  __syncthreads();
  // Hillis-Steele inclusive scans.
  for (uint32_t d = 1; d < kPlanThreads; d <<= 1) {
    const uint32_t a = threadIdx.x >= d ? s_rows[threadIdx.x - d] : 0u;
    const uint32_t b = threadIdx.x >= d ? s_tiles[threadIdx.x - d] : 0u;
    __syncthreads();
    s_rows[threadIdx.x] += a;
    s_tiles[threadIdx.x] += b;
    __syncthreads();
  }
  uint32_t row_off = s_rows[threadIdx.x] - rows;
  uint32_t tile_off = s_tiles[threadIdx.x] - ntile;
  for (uint32_t k = lo; k < hi; ++k) {
    const uint32_t c = counts[k];
    cursor[k] = row_off;
    const uint32_t word = word_of(k, ks);
    for (uint32_t first = 0; first < c; first += kTileRows) {
      GroupTile t;
      t.word = word;
      t.start = row_off + first;
      t.count = min(kTileRows, c - first);
      t.pad = 0u;
      tiles[tile_off++] = t;
    }
    row_off += c;
  }
  if (threadIdx.x == kPlanThreads - 1) *n_tiles = s_tiles[kPlanThreads - 1];
}

__global__ __launch_bounds__(kPlanThreads) void grouped_plan_kernel(const uint32_t *__restrict__ counts,
                                                                     uint32_t *__restrict__ cursor,
                                                                     GroupTile *__restrict__ tiles,
                                                                     uint32_t *__restrict__ n_tiles, KeySpace ks) {
  __shared__ uint32_t s_rows[kPlanThreads], s_tiles[kPlanThreads];
  plan_keys(counts, cursor, tiles, n_tiles, ks, s_rows, s_tiles);
}

// The whole sort in one block when the rows fit in registers (KPT <= 16 keys
// per thread, two 16-bit keys per register) and the key histogram in LDS:
// count into the LDS histogram, scan it in place into the cursors and the
// tile list, then scatter through LDS atomics.  One launch instead of four (zero, count, plan, scatter), which is
// most of the sort's cost at verify and small-prefill row counts; at 40,960
// rows one CU is slower (31.6 us) than the four kernels (23.5 us).
constexpr uint32_t kSingleSortKeys = 12288;  // 48 KB of dynamic LDS beside the 8 KB of scan scratch

template <int KPT>
__global__ __launch_bounds__(kPlanThreads) void grouped_sort_single_kernel(
    const uint32_t *__restrict__ routes, uint32_t routed_rows, uint32_t rows, KeySpace ks,
    uint32_t *__restrict__ order, GroupTile *__restrict__ tiles, uint32_t *__restrict__ n_tiles,
    unsigned int *__restrict__ err) {
  constexpr int kBatch = KPT < 16 ? KPT : 16;  // route loads in flight per thread
  static_assert(KPT % kBatch == 0 && kBatch % 2 == 0 && kSingleSortKeys <= 65536u, "16-bit keys");
  extern __shared__ uint32_t hist[];
  __shared__ uint32_t s_rows[kPlanThreads], s_tiles[kPlanThreads];
  const uint32_t nk = ks.size();
  for (uint32_t i = threadIdx.x; i < nk; i += kPlanThreads) hist[i] = 0u;
  uint32_t kp[KPT / 2];  // row (j * 1024 + tid)'s key in bits 16 (j & 1) .. +15 of kp[j / 2]
  bool bad = false;
  __syncthreads();  // the histogram is zero
#pragma unroll
  for (int b = 0; b < KPT; b += kBatch) {
    uint32_t w[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const uint32_t r = static_cast<uint32_t>(b + i) * kPlanThreads + threadIdx.x;
      w[i] = r < routed_rows ? routes[r] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const uint32_t r = static_cast<uint32_t>(b + i) * kPlanThreads + threadIdx.x;
      const uint32_t key = r < rows ? (r < routed_rows ? key_of(w[i], ks) : ks.shared_key()) : 0u;
      bad |= r < rows && key == ks.dead_key();
      if (r < rows) atomicAdd(&hist[key], 1u);
      if (i & 1) kp[(b + i) / 2] |= key << 16;
      else kp[(b + i) / 2] = key;
    }
  }
  if (__ballot(bad) != 0ull && (threadIdx.x & 63) == 0) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);
  __syncthreads();
  plan_keys(hist, hist, tiles, n_tiles, ks, s_rows, s_tiles);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const uint32_t r = static_cast<uint32_t>(j) * kPlanThreads + threadIdx.x;
    if (r < rows) order[atomicAdd(&hist[(kp[j / 2] >> (16 * (j & 1))) & 0xffffu], 1u)] = r;
  }
}

__global__ void grouped_scatter_kernel(const uint32_t *__restrict__ row_key, uint32_t rows,
                                       uint32_t *__restrict__ cursor, uint32_t *__restrict__ order) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = r < rows;
  const uint32_t key = active ? row_key[r] : 0u;
  const uint32_t pos = wave_aggregated_increment<true>(cursor, key, active);
  if (active) order[pos] = r;
}

// Block-histogram variants for key spaces that fit in LDS (kLdsKeys).  Each
// block takes kSortRows consecutive rows and counts them in an LDS histogram
// first, so a hot expert costs one global atomic per block instead of one
// per wave (Zipf-skewed prefill routes put thousands of rows on one key, and
// same-address global atomics serialize).
constexpr uint32_t kSortThreads = 256;
constexpr uint32_t kSortPerThread = 8;
constexpr uint32_t kSortRows = kSortThreads * kSortPerThread;
constexpr uint32_t kLdsKeys = 16384;  // 64 KB of dynamic LDS

__global__ __launch_bounds__(kSortThreads) void grouped_count_lds_kernel(
    const uint32_t *__restrict__ routes, uint32_t routed_rows, uint32_t rows, KeySpace ks,
    uint32_t *__restrict__ counts, uint32_t *__restrict__ row_key, unsigned int *__restrict__ err) {
  extern __shared__ uint32_t hist[];
  const uint32_t nk = ks.size();
  for (uint32_t i = threadIdx.x; i < nk; i += kSortThreads) hist[i] = 0u;
  __syncthreads();
  const uint32_t base = blockIdx.x * kSortRows;
  bool bad = false;
#pragma unroll
  for (uint32_t j = 0; j < kSortPerThread; ++j) {
    const uint32_t r = base + j * kSortThreads + threadIdx.x;
    if (r < rows) {
      const uint32_t key = r < routed_rows ? key_of(routes[r], ks) : ks.shared_key();
      bad |= key == ks.dead_key();
      row_key[r] = key;
      atomicAdd(&hist[key], 1u);
    }
  }
  if (__ballot(bad) != 0ull && (threadIdx.x & 63) == 0) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < nk; i += kSortThreads) {
    const uint32_t c = hist[i];
    if (c != 0u) atomicAdd(&counts[i], c);
  }
}

// Scatter: each row's position is its key's cursor, advanced once per block
// by the block's count of that key, plus the row's rank among the block's
// rows of that key (the LDS atomic's return value).
__global__ __launch_bounds__(kSortThreads) void grouped_scatter_lds_kernel(const uint32_t *__restrict__ row_key,
                                                                          uint32_t rows, KeySpace ks,
                                                                          uint32_t *__restrict__ cursor,
                                                                          uint32_t *__restrict__ order) {
  extern __shared__ uint32_t hist[];
  const uint32_t nk = ks.size();
  for (uint32_t i = threadIdx.x; i < nk; i += kSortThreads) hist[i] = 0u;
  __syncthreads();
  const uint32_t base = blockIdx.x * kSortRows;
  uint32_t key[kSortPerThread], rank[kSortPerThread];
#pragma unroll
  for (uint32_t j = 0; j < kSortPerThread; ++j) {
    const uint32_t r = base + j * kSortThreads + threadIdx.x;
    key[j] = r < rows ? row_key[r] : 0u;
    rank[j] = r < rows ? atomicAdd(&hist[key[j]], 1u) : 0u;
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < nk; i += kSortThreads) {
    const uint32_t c = hist[i];
    if (c != 0u) hist[i] = atomicAdd(&cursor[i], c);
  }
  __syncthreads();
#pragma unroll
  for (uint32_t j = 0; j < kSortPerThread; ++j) {
    const uint32_t r = base + j * kSortThreads + threadIdx.x;
    if (r < rows) order[hist[key[j]] + rank[j]] = r;
  }
}

// Gather row map: xmap[i] = x row of sorted row i (~0u, with a flag, when the
// caller's row index is past the end of x).
__global__ void gather_map_kernel(const uint32_t *__restrict__ order, const uint32_t *__restrict__ x_rows,
                                  uint32_t rows, uint32_t x_count, uint32_t *__restrict__ xmap,
                                  unsigned int *__restrict__ err) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows) return;
  const uint32_t r = x_rows[order[i]];
  const bool bad = r >= x_count;
  xmap[i] = bad ? ~0u : r;
  if (bad) raise_flag(err, MQ_DEVFLAG_BAD_ROW);
}

// ------------------------------------------------------------------ GEMM
template <int B>
__device__ __forceinline__ float ubyte_to_f32(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2_t2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// K order inside a stage.  MFMA k-slots can be assigned to inputs in any
// order as long as both operands agree.  Lane l (fragment row or tile row
// l%32, half h = l/32) supplies, at k16-step j of a stage, the eight inputs
// k0 + 32 h + 8 j .. +7 for j < 4 and k0 + 64 + 32 h + 8 (j - 4) .. +7 for
// j >= 4.  A lane's packed weights are then two 16-byte pieces (words 4h ..
// 4h+3 and 8+4h .. 8+4h+3 of the row's 64-byte stage), loaded straight into
// registers with no LDS, and lanes l and l + 32 read adjacent pieces, so
// each load instruction reads 32 contiguous bytes of each of the wave's 32
// rows.  The activation fragments follow the same order.

// Activation tile in LDS: 128 rows x 128 bf16, rows padded by one 16-byte
// chunk (272 bytes), so the 32 rows of a slab read at one chunk column fall
// on different banks while every read address is a per-lane base plus an
// immediate offset.
constexpr uint32_t kXRow = kKS + 8;  // bf16 per padded LDS row
__device__ __forceinline__ uint32_t xs_off(uint32_t row, uint32_t chunk) { return row * kXRow + chunk * 8u; }

// Dequantize one packed word (8 consecutive inputs) to bf16(fma(q, s, b)) in
// MFMA operand order.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0f0f0f0fu;         // inputs 0, 2, 4, 6 (one per byte)
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // inputs 1, 3, 5, 7
  const uint4 v = make_uint4(pack_bf16(fmaf(ubyte_to_f32<0>(lo), s, b), fmaf(ubyte_to_f32<0>(hi), s, b)),
                             pack_bf16(fmaf(ubyte_to_f32<1>(lo), s, b), fmaf(ubyte_to_f32<1>(hi), s, b)),
                             pack_bf16(fmaf(ubyte_to_f32<2>(lo), s, b), fmaf(ubyte_to_f32<2>(hi), s, b)),
                             pack_bf16(fmaf(ubyte_to_f32<3>(lo), s, b), fmaf(ubyte_to_f32<3>(hi), s, b)));
  return __builtin_bit_cast(bf16x8_t, v);
}

constexpr uint32_t kXTile = kTileRows * kXRow;  // bf16 per LDS activation tile

// One lane's weights for one stage: 64 inputs of its weight row as 8 packed
// words (two 16-byte loads) and the scales and biases of their groups as bf16
// pairs (words 0-3 use the low half, words 4-7 the high half).
struct WStage {
  uint4 w[2];
  uint32_t s, b;
};

// The weight row a lane streams for one work item: the wave's projection
// descriptors (wave-uniform, so the loads need no per-lane descriptor) and
// the lane's row.
struct WRow {
  ExpertRsrc e;
  uint32_t row;
  bool ok;
};

// Byte offset of a lane's first weight piece of a stage: lanes l and l + 32
// (halves 0 and 1) read adjacent 16-byte pieces, so each of the two load
// instructions reads 32 contiguous bytes of each of the wave's 32 rows.
__device__ __forceinline__ uint32_t wstage_off(const WRow &wr, uint32_t K, uint32_t stage, uint32_t half) {
  return wr.ok ? wr.row * (K / 2u) + stage * (kKS / 2u) + 16u * half : kOutOfRange;
}

// Group scales and biases of a lane's words, as bf16 pairs: the low half for
// w[0], the high half for w[1].  Group 32: groups half and half + 2 of the
// stage's four; group 64: groups 0 and 1.
template <int G>
__device__ __forceinline__ void load_groups(uint32_t &s, uint32_t &b, const WRow &wr, uint32_t K, uint32_t stage,
                                            uint32_t half) {
  const uint32_t g0 = wr.row * (K / G) + stage * (kKS / G);
  if constexpr (G == 32) {  // the stage's four groups in one 8-byte load, then (g[half], g[half + 2])
    const uint32_t o = wr.ok ? g0 * 2u : kOutOfRange;
    const u32x2_t sv = __builtin_amdgcn_raw_buffer_load_b64(wr.e.s, static_cast<int>(o), 0, 0);
    const u32x2_t bv = __builtin_amdgcn_raw_buffer_load_b64(wr.e.b, static_cast<int>(o), 0, 0);
    const uint32_t sel = half ? 0x07060302u : 0x05040100u;
    s = __builtin_amdgcn_perm(sv.y, sv.x, sel);
    b = __builtin_amdgcn_perm(bv.y, bv.x, sel);
  } else {
    const uint32_t o = wr.ok ? g0 * 2u : kOutOfRange;
    s = buf_load4(wr.e.s, o);
    b = buf_load4(wr.e.b, o);
  }
}

template <int G, bool GROUPS = true>
__device__ __forceinline__ void load_wstage(WStage &r, const WRow &wr, uint32_t K, uint32_t stage, uint32_t half) {
  const uint32_t off_w = wstage_off(wr, K, stage, half);
  r.w[0] = buf_load16(wr.e.w, off_w);
  r.w[1] = buf_load16(wr.e.w, off_w + 32u);
  if constexpr (GROUPS) load_groups<G>(r.s, r.b, wr, K, stage, half);
}

// Group windows: when the stage count allows, the scales and biases are
// fetched W = 2 or 4 stages at a time.  Lane (row, half) loads the groups of
// stages stage0 + half * W / 2 .. + W / 2 - 1 of its row, so one load
// instruction per array covers W stages of the wave's 32 rows in 8 W
// contiguous bytes each (group 32; 4 W with group 64), and v_permlane32_swap
// then hands each half the other half's stages.  Small scattered loads are
// what limits the stream here: every row's scales sit in their own cache
// line, and per-stage 8-byte loads spend as many L1 tag lookups and miss
// slots as the weights themselves.
template <int G, int W>
struct GroupWindow {
  static constexpr int kWords = W * (kKS / G) / 4;  // 32-bit words per lane and array
  uint32_t s[kWords], b[kWords];                     // as loaded: this half's stages
};

template <int G, int W>
__device__ __forceinline__ void load_window(GroupWindow<G, W> &r, const WRow &wr, uint32_t K, uint32_t stage0,
                                            uint32_t half) {
  constexpr int kWords = GroupWindow<G, W>::kWords;
  const uint32_t g0 = wr.row * (K / G) + (stage0 + half * (W / 2)) * (kKS / G);
  const int o = static_cast<int>(wr.ok ? g0 * 2u : kOutOfRange);
  if constexpr (kWords == 4) {
    const u32x4_t sv = __builtin_amdgcn_raw_buffer_load_b128(wr.e.s, o, 0, 0);
    const u32x4_t bv = __builtin_amdgcn_raw_buffer_load_b128(wr.e.b, o, 0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      r.s[q] = sv[q];
      r.b[q] = bv[q];
    }
  } else if constexpr (kWords == 2) {
    const u32x2_t sv = __builtin_amdgcn_raw_buffer_load_b64(wr.e.s, o, 0, 0);
    const u32x2_t bv = __builtin_amdgcn_raw_buffer_load_b64(wr.e.b, o, 0, 0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      r.s[q] = sv[q];
      r.b[q] = bv[q];
    }
  } else {
    r.s[0] = buf_load4(wr.e.s, static_cast<uint32_t>(o));
    r.b[0] = buf_load4(wr.e.b, static_cast<uint32_t>(o));
  }
}

// The lane's (scale, bias) bf16 pairs for stages stage0 .. stage0 + W - 1
// from an arrived window (the pair layout of load_groups).
template <int G, int W>
__device__ __forceinline__ void open_window(const GroupWindow<G, W> &r, uint32_t half, uint32_t (&sp)[W],
                                            uint32_t (&bp)[W]) {
  constexpr int kWords = GroupWindow<G, W>::kWords;
  // v_permlane32_swap(x, x): the first result holds lanes 0-31's value in
  // both halves (the window's first W / 2 stages), the second lanes 32-63's.
  uint32_t sw[2][kWords], bw[2][kWords];
#pragma unroll
  for (int q = 0; q < kWords; ++q) {
    const auto sx = __builtin_amdgcn_permlane32_swap(r.s[q], r.s[q], false, false);
    const auto bx = __builtin_amdgcn_permlane32_swap(r.b[q], r.b[q], false, false);
    sw[0][q] = sx[0];
    sw[1][q] = sx[1];
    bw[0][q] = bx[0];
    bw[1][q] = bx[1];
  }
  constexpr int kPerStage = kKS / G / 2;  // words per stage: 2 (group 32) or 1 (group 64)
#pragma unroll
  for (int st = 0; st < W; ++st) {
    const int h = st / (W / 2), w0 = (st % (W / 2)) * kPerStage;
    if constexpr (G == 32) {
      const uint32_t sel = half ? 0x07060302u : 0x05040100u;  // groups (half, half + 2) of the stage's four
      sp[st] = __builtin_amdgcn_perm(sw[h][w0 + 1], sw[h][w0], sel);
      bp[st] = __builtin_amdgcn_perm(bw[h][w0 + 1], bw[h][w0], sel);
    } else {
      sp[st] = sw[h][w0];
      bp[st] = bw[h][w0];
    }
  }
}

// A thread's share of the activation tile of one stage: kXChunks 16-byte
// chunks (32 inputs) of tile row tid / kXParts, part tid % kXParts.
struct XStage {
  uint4 x[kXChunks];
};

__device__ __forceinline__ void load_xstage(XStage &r, __amdgpu_buffer_rsrc_t xr, uint32_t src, uint32_t K,
                                            uint32_t stage, uint32_t xpart) {
  const uint32_t off = src != ~0u ? (src * K + stage * kKS + 8u * kXChunks * xpart) * 2u : kOutOfRange;
#pragma unroll
  for (uint32_t j = 0; j < kXChunks; ++j) r.x[j] = buf_load16(xr, off + 16u * j);
}

__device__ __forceinline__ void store_xstage(uint16_t *xb, const XStage &r, uint32_t xrow, uint32_t xpart) {
#pragma unroll
  for (uint32_t j = 0; j < kXChunks; ++j)
    *reinterpret_cast<uint4 *>(xb + xs_off(xrow, kXChunks * xpart + j)) = r.x[j];
}

// The B operand of slab t at k16 step j: tile row 32 t + lane%32, eight
// inputs at 32 h + 8 j (+ 32 for j >= 4) of the stage (`xl` is the lane's
// base in the LDS activation tile, at input 32 h).
__device__ __forceinline__ bf16x8_t b_frag(const uint16_t *xl, int t, int j) {
  return *reinterpret_cast<const bf16x8_t *>(xl + 32u * t * kXRow + 8u * j + (j >= 4 ? 32u : 0u));
}

// One k16 step: C[32 weight rows x 32 tile rows] += A . B for the NSLAB
// active slabs (the tile's rows, 32 per slab).  The B fragments of step j
// were read during step j - 1; each slab's register is refilled with step
// j + 1 as soon as its MFMA has issued, so an LDS read has a whole step
// (the next A dequantization and the other slabs' MFMAs) to land instead of
// stalling the MFMA that follows it.  The slab count is a template argument
// so that no branch splits the MFMA stream.
template <int NSLAB>
__device__ __forceinline__ void mma_step(f32x16_t (&acc)[4], bf16x8_t (&bq)[4], const uint16_t *xl,
                                         const bf16x8_t &a, int j) {
#pragma unroll
  for (int t = 0; t < NSLAB; ++t) {
    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq[t], acc[t], 0, 0, 0);
    if (j < 7) bq[t] = b_frag(xl, t, j + 1);
  }
}

// A stage of MFMAs from ring slot `w`, refilling the slot for the load
// cursor's stage as soon as each part of it has been consumed (scales and
// biases first, then the first and second four words), so that a slot's
// registers are never live twice.
template <int G, int NSLAB, bool GROUPS>
__device__ __forceinline__ void stage_mma(f32x16_t (&acc)[4], const uint16_t *xl, WStage &w, const WRow &lw,
                                          uint32_t K, uint32_t ls, uint32_t half, uint32_t sp, uint32_t bp) {
  const float s0 = __uint_as_float(sp << 16), b0 = __uint_as_float(bp << 16);
  const float s1 = __uint_as_float(sp & 0xffff0000u), b1 = __uint_as_float(bp & 0xffff0000u);
  const uint32_t off_w = wstage_off(lw, K, ls, half);
  if constexpr (GROUPS) load_groups<G>(w.s, w.b, lw, K, ls, half);
  // Software pipeline over the eight k16 steps: the A operand of step j+1 is
  // dequantized while the MFMAs of step j run; a scheduling barrier per step
  // keeps the compiler from hoisting further ahead (which only adds live
  // registers: the other wave on the SIMD covers the LDS latency).
  bf16x8_t bq[4];
#pragma unroll
  for (int t = 0; t < NSLAB; ++t) bq[t] = b_frag(xl, t, 0);
  bf16x8_t a = dequant_word(w.w[0].x, s0, b0);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bf16x8_t an = a;
    if (j < 7) {
      const int k = j + 1;
      const uint4 &q = w.w[k >> 2];
      const uint32_t word = (k & 3) == 0 ? q.x : (k & 3) == 1 ? q.y : (k & 3) == 2 ? q.z : q.w;
      an = dequant_word(word, k < 4 ? s0 : s1, k < 4 ? b0 : b1);
    }
    if (j == 3) w.w[0] = buf_load16(lw.e.w, off_w);  // words 0-3 consumed
    if (j == 7) w.w[1] = buf_load16(lw.e.w, off_w + 32u);
    mma_step<NSLAB>(acc, bq, xl, a, j);
    a = an;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// C-tile register r of lane l holds weight row 8*(r/4) + 4*(l/32) + r%4 of the
// 32-row fragment and tile row l%32 of the 32-row slab.
__device__ __forceinline__ uint32_t c_row(int r, int lane) { return 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3); }

// XCD-aware persistent schedule.  Workgroups are dispatched round-robin over
// the 8 XCDs (block b runs on XCD b % 8) and each XCD has its own L2.  Tile t
// is owned by XCD t % 8, and the XCD's blocks walk its (tile, feature block)
// items in order, so the feature blocks of one tile run at the same time on
// one XCD and read the tile's activation rows through one L2.  The grid is a
// multiple of 8 blocks.
struct XcdItems {
  uint32_t xcd, first, stride, count, nb_count;
  __device__ __forceinline__ XcdItems(uint32_t n_tiles, uint32_t nb) : nb_count(nb) {
    xcd = blockIdx.x & 7u;
    first = blockIdx.x >> 3;
    stride = gridDim.x >> 3;
    const uint32_t tiles_here = n_tiles > xcd ? (n_tiles - xcd + 7u) / 8u : 0u;
    count = tiles_here * nb;
  }
  __device__ __forceinline__ uint32_t tile(uint32_t j) const { return xcd + 8u * (j / nb_count); }
};

struct GemmParams {
  const uint16_t *x;     // gate/up: token activations [tokens, K]; down: act [rows, K] in sorted order;
                         // gather: the caller's rows [x_count, K]
  uint32_t x_bytes;
  const uint32_t *xmap;  // gather: x row of each sorted row (~0u: none)
  uint32_t xmap_bytes;
  MqProjection w0, w1;   // gate/up: gate, up; down: down (w1 unused)
  MqProjection s0, s1;   // the shared expert's matching projections (dense, expert 0) or unused
  const GroupTile *tiles;
  uint32_t tiles_bytes;
  const uint32_t *n_tiles;
  const uint32_t *order;
  uint32_t order_bytes;
  uint16_t *out;         // gate/up: act [rows, N] sorted; down: y [routed_rows, N]; gather: [rows, N]
  uint16_t *out_shared;  // down: the shared expert's output [tokens, N] or null
  uint32_t slots, routed_rows, K, N, dense_count;
  unsigned int *err;
};

// A work item of the block's sequence, as fetched ahead of use.  The fields
// loaded from memory stay in vector registers and are made uniform only where
// used, so that issuing the fetch never waits for it.
struct Item {
  uint32_t j;       // index in the XCD's item list (uniform)
  uint4 tile;       // GroupTile: word, start, count (all zero past the end)
  uint32_t xraw;    // gate/up: `order` entry of this thread's tile row; gather: its x row
  uint32_t dst[4];  // down, gather: `order` entries of this lane's tile rows in the four slabs
};

__device__ __forceinline__ void fetch_tile(Item &m, uint32_t j, const XcdItems &it, __amdgpu_buffer_rsrc_t tr) {
  m.j = j;
  m.tile = buf_load16(tr, j < it.count ? it.tile(j) * 16u : kOutOfRange);
}

// Second fetch step, once the tile record has arrived: the sorted-row entries
// (`orr`: order, `xmr`: the gather row map).
template <int MODE>
__device__ __forceinline__ void fetch_rows(Item &m, __amdgpu_buffer_rsrc_t orr, __amdgpu_buffer_rsrc_t xmr, int tid) {
  const uint32_t start = m.tile.y, count = m.tile.z;
  if constexpr (MODE != kModeGateUp) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t i = 32u * t + (static_cast<uint32_t>(tid) & 31u);
      m.dst[t] = buf_load4(orr, i < count ? (start + i) * 4u : kOutOfRange);
    }
  }
  if constexpr (MODE != kModeDown) {
    const uint32_t i = static_cast<uint32_t>(tid) / kXParts;
    m.xraw = buf_load4(MODE == kModeGather ? xmr : orr, i < count ? (start + i) * 4u : kOutOfRange);
  }
}

// This thread's activation row for the item's X loads (~0u: none).
template <int MODE>
__device__ __forceinline__ uint32_t x_source(const Item &m, const GemmParams &p, int tid) {
  const uint32_t i = static_cast<uint32_t>(tid) / kXParts;
  if (i >= m.tile.z) return ~0u;
  if constexpr (MODE == kModeDown) return m.tile.y + i;
  else if constexpr (MODE == kModeGather) return m.xraw;
  else return m.xraw < p.routed_rows ? m.xraw / p.slots : m.xraw - p.routed_rows;
}

// The lane's weight row of an item.  Gate/up: waves 0-3 stream gate rows and
// waves 4-7 the up rows of the same 128 features; down and gather: wave w
// streams rows 32 w .. +31 of the item's 256 output features.
template <int MODE, int G>
__device__ __forceinline__ WRow weight_row(const Item &m, const GemmParams &p, const XcdItems &it,
                                           uint32_t nb_count, uint32_t wave, int lane) {
  const bool valid = m.j < it.count;
  const uint32_t word = uniform(m.tile.x);
  const uint32_t nb = m.j % nb_count;
  const bool shared = word == kSharedWord;
  ExpertPtrs e;
  uint32_t row;
  if constexpr (MODE != kModeGateUp) {
    if (shared) e = expert_ptrs(p.s0, 0u, p.N, p.K, G, 1u);
    else e = expert_ptrs(p.w0, word, p.N, p.K, G, p.dense_count);
    row = nb * kDownFeatures + 32u * wave + (static_cast<uint32_t>(lane) & 31u);
  } else {
    if (wave < kGemmWaves / 2) {
      if (shared) e = expert_ptrs(p.s0, 0u, p.N, p.K, G, 1u);
      else e = expert_ptrs(p.w0, word, p.N, p.K, G, p.dense_count);
    } else {
      if (shared) e = expert_ptrs(p.s1, 0u, p.N, p.K, G, 1u);
      else e = expert_ptrs(p.w1, word, p.N, p.K, G, p.dense_count);
    }
    row = nb * kGateUpFeatures + 32u * (wave % (kGemmWaves / 2)) + (static_cast<uint32_t>(lane) & 31u);
  }
  if (valid && !e.ok && word != kDeadWord && lane == 0) raise_flag(p.err, MQ_DEVFLAG_BAD_ROUTE);
  WRow r;
  r.e = expert_rsrc(e, p.N, p.K, G);
  r.row = row;
  r.ok = valid && e.ok && row < p.N;
  return r;
}

// Gate/up epilogue: act = swiglu(bf16(g), bf16(u)) in sorted row order.  Lane
// l of gate wave f and lane l of up wave 4+f hold the same (row, feature)
// cells, in four runs q of 4 consecutive features.  Gate waves compute runs
// 0-1 and up waves runs 2-3, each handing the other its bf16 values of the
// runs the other computes through LDS (the tile buffer just consumed), so all
// eight waves share the SwiGLU sequence.  The sigmoid comes from a per-block
// LDS table of the sequence's |g|-only part, filled once per launch (about 15
// VALU instructions per cell instead of about 50 for the whole sequence).
constexpr uint32_t kExchange = 4u * 4u * 64u * 4u;  // bf16 per gate/up wave pair: 4 slabs x 16 values x 64 lanes
static_assert(kExchange * (kGemmWaves / 2) <= kXTile, "gate/up exchange must fit in one activation tile");

__device__ __forceinline__ uint32_t ex_off(int t, int i, int lane) {  // run i (0, 1) of slab t, lane `lane`
  return ((2u * t + i) * 64u + lane) * 4u;
}

template <bool UP>
__device__ __forceinline__ void gateup_epilogue_half(const f32x16_t (&acc)[4], uint16_t *ex, const Item &m,
                                                     const GemmParams &p, uint32_t nb, uint32_t fw, int lane,
                                                     const bool (&slab)[4], const uint32_t *sig_tab) {
  constexpr int kRun = UP ? 2 : 0;   // first run this wave computes
  constexpr int kGive = UP ? 0 : 2;  // first run this wave hands over
  uint16_t *give = ex + (UP ? kExchange / 2 : 0u);
  const uint16_t *take = ex + (UP ? 0u : kExchange / 2);
#pragma unroll
  for (int t = 0; t < 4; ++t)
    if (slab[t])
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int q = kGive + i;
        const uint32_t lo = f32_to_bf16(acc[t][4 * q]) | (static_cast<uint32_t>(f32_to_bf16(acc[t][4 * q + 1])) << 16);
        const uint32_t hi =
            f32_to_bf16(acc[t][4 * q + 2]) | (static_cast<uint32_t>(f32_to_bf16(acc[t][4 * q + 3])) << 16);
        *reinterpret_cast<uint2 *>(give + ex_off(t, i, lane)) = make_uint2(lo, hi);
      }
  __syncthreads();
  const uint32_t start = uniform(m.tile.y), count = uniform(m.tile.z);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t trow = 32u * t + (static_cast<uint32_t>(lane) & 31u);
    if (!slab[t] || trow >= count) continue;
    uint16_t *dst = p.out + static_cast<uint64_t>(start + trow) * p.N;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = kRun + i;
      const uint32_t feat = nb * kGateUpFeatures + 32u * fw + c_row(4 * q, lane);
      const uint2 o = *reinterpret_cast<const uint2 *>(take + ex_off(t, i, lane));
      const uint32_t oo[2] = {o.x, o.y};
      float gv[4], uv[4], v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float own = round_bf16(acc[t][4 * q + e]);
        const float other = __uint_as_float((e & 1) ? (oo[e >> 1] & 0xffff0000u) : (oo[e >> 1] << 16));
        gv[e] = UP ? other : own;
        uv[e] = UP ? own : other;
      }
      swiglu_bf16_tab_n<4>(gv, uv, v, sig_tab);
      if (feat < p.N) *reinterpret_cast<uint2 *>(dst + feat) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    }
  }
}

__device__ __forceinline__ void gateup_epilogue(const f32x16_t (&acc)[4], uint16_t *xb, const Item &m,
                                                const GemmParams &p, uint32_t nb, uint32_t wave, int lane,
                                                const bool (&slab)[4], const uint32_t *sig_tab) {
  const uint32_t fw = wave % (kGemmWaves / 2);
  __syncthreads();  // every wave is done reading the tile in xb
  if (wave >= kGemmWaves / 2) gateup_epilogue_half<true>(acc, xb + fw * kExchange, m, p, nb, fw, lane, slab, sig_tab);
  else gateup_epilogue_half<false>(acc, xb + fw * kExchange, m, p, nb, fw, lane, slab, sig_tab);
}

// Down and gather epilogue: the bf16 outputs go back to the row's `order`
// entry: y[token, slot] (or the shared expert's row), or the gather row.
__device__ __forceinline__ void down_epilogue(const f32x16_t (&acc)[4], const Item &m, const GemmParams &p,
                                              uint32_t nb, uint32_t wave, int lane, const bool (&slab)[4]) {
  const uint32_t count = uniform(m.tile.z);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t trow = 32u * t + (static_cast<uint32_t>(lane) & 31u);
    if (!slab[t] || trow >= count) continue;
    const uint32_t r = m.dst[t];
    uint16_t *dst = r < p.routed_rows ? p.out + static_cast<uint64_t>(r) * p.N
                                      : p.out_shared + static_cast<uint64_t>(r - p.routed_rows) * p.N;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t feat = nb * kDownFeatures + 32u * wave + c_row(4 * q, lane);
      if (feat < p.N)
        *reinterpret_cast<uint2 *>(dst + feat) =
            make_uint2(pack_bf16(acc[t][4 * q], acc[t][4 * q + 1]), pack_bf16(acc[t][4 * q + 2], acc[t][4 * q + 3]));
    }
  }
}

// Pipeline state carried across stages and items: the weight ring, the load
// cursor (row and stage, NS stages ahead of compute), and the activation
// registers of the next stage with their source rows.
template <int MODE, int NS, int G, int W>
struct Pipe {
  // W stages per group window (W = 2 or 4, NS == 2, W divides the stage
  // count); W = 1: the groups ride in the ring slots.  The stage loop is
  // unrolled by U = max(NS, W) stages, so every window starts at u = 0.
  static constexpr bool kWindow = W > 1;
  static constexpr int U = NS > W ? NS : W;
  WStage ring[NS];
  GroupWindow<G, kWindow ? W : 2> win;  // the next window, loaded W - NS stages before it opens
  uint32_t wsp[kWindow ? W : 1], wbp[kWindow ? W : 1];  // the open window's pairs
  WRow lw;
  uint32_t ls;
  XStage xv;
  uint32_t xsrc, xsrc_next;

  // All stages of one item with NSLAB active slabs.  NS divides S, so ring
  // slot u always holds stage s0 + u and the item ends with an unrolled trip.
  template <int NSLAB>
  __device__ __forceinline__ void run(f32x16_t (&acc)[4], uint16_t *xs, const Item &n, const Item &n2,
                                      const GemmParams &p, const XcdItems &it, uint32_t nb_count, uint32_t wave,
                                      int lane, int tid, uint32_t S, __amdgpu_buffer_rsrc_t xr) {
    const uint32_t half = static_cast<uint32_t>(lane) >> 5;
    const uint32_t xrow = static_cast<uint32_t>(tid) / kXParts, xpart = static_cast<uint32_t>(tid) % kXParts;
    const uint32_t xl_off = (static_cast<uint32_t>(lane) & 31u) * kXRow + 32u * half;
    for (uint32_t s0 = 0; s0 < S; s0 += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t s = s0 + u;
        uint16_t *xb = xs + (s & 1u) * kXTile;
        if (xrow < 32u * NSLAB) store_xstage(xb, xv, xrow, xpart);  // rows past the active slabs are never read
        __syncthreads();
        const bool last = u == U - 1 && s + 1u == S;
        if (last) xsrc_next = x_source<MODE>(n, p, tid);
        load_xstage(xv, xr, last ? xsrc_next : xsrc, p.K, last ? 0u : s + 1u, xpart);
        if constexpr (kWindow) {
          if (u == 0) open_window<G, W>(win, half, wsp, wbp);  // stages s .. s + W - 1
          // The load cursor (NS stages ahead) reaches the next window's first stage.
          if (u == W - NS) load_window<G, W>(win, lw, p.K, ls, half);
          stage_mma<G, NSLAB, false>(acc, xb + xl_off, ring[u % NS], lw, p.K, ls, half, wsp[u], wbp[u]);
        } else {
          stage_mma<G, NSLAB, true>(acc, xb + xl_off, ring[u % NS], lw, p.K, ls, half, ring[u % NS].s,
                                    ring[u % NS].b);
        }
        if (++ls == S) {
          // The load cursor finished an item.  With NS == S it was already
          // in the next item n, and this is compute's last stage of c.
          ls = 0;
          lw = weight_row<MODE, G>(last ? n2 : n, p, it, nb_count, wave, lane);
        }
      }
    }
  }
};

// The grouped GEMM, persistent over the block's work items (tile, feature
// block).  Per stage of kKS inputs: the activations loaded one stage earlier
// go to one of two LDS tiles (one barrier per stage), the next stage's
// activations and the weights NS stages ahead are issued, and the stage's
// weights (loaded NS stages earlier into ring slot u) are dequantized and fed
// to the MFMAs.  The stage sequence runs on across items: the weight loads of
// the next item start while the current one finishes (NS <= stages per item,
// so the load cursor is at most one item ahead), and tile records and sorted
// rows are fetched two items ahead.
template <int MODE, int NS, int G, int W>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(GemmParams p) {
  __shared__ __align__(16) uint16_t xs[2 * kXTile];
  __shared__ uint32_t sig_tab[MODE == kModeGateUp ? kSigTabEntries : 1u];  // gate/up: the SwiGLU sigmoid table
  constexpr uint32_t kFeat = MODE == kModeGateUp ? kGateUpFeatures : kDownFeatures;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t half = static_cast<uint32_t>(lane) >> 5;
  const uint32_t xpart = static_cast<uint32_t>(tid) % kXParts;
  const uint32_t S = p.K / kKS;
  const uint32_t nb_count = (p.N + kFeat - 1) / kFeat;
  const XcdItems it(*p.n_tiles, nb_count);
  if (it.first >= it.count) return;  // uniform: no work for this block
  const __amdgpu_buffer_rsrc_t tr = make_rsrc(p.tiles, p.tiles_bytes);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(p.order, p.order_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t xmr = make_rsrc(p.xmap, MODE == kModeGather ? p.xmap_bytes : 0u);

  Item c, n, n2;  // the compute item and the next two
  fetch_tile(c, it.first, it, tr);
  fetch_tile(n, it.first + it.stride, it, tr);
  fetch_tile(n2, it.first + 2u * it.stride, it, tr);
  fetch_rows<MODE>(c, orr, xmr, tid);
  fetch_rows<MODE>(n, orr, xmr, tid);

  // Load cursor: NS stages ahead of the compute cursor.
  Pipe<MODE, NS, G, W> pp;
  pp.lw = weight_row<MODE, G>(c, p, it, nb_count, wave, lane);
  pp.ls = 0;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if constexpr (Pipe<MODE, NS, G, W>::kWindow) {
      if (u == 0) load_window<G>(pp.win, pp.lw, p.K, pp.ls, half);
      load_wstage<G, false>(pp.ring[u], pp.lw, p.K, pp.ls, half);
    } else {
      load_wstage<G>(pp.ring[u], pp.lw, p.K, pp.ls, half);
    }
    if (++pp.ls == S) {
      pp.ls = 0;
      pp.lw = weight_row<MODE, G>(n, p, it, nb_count, wave, lane);
    }
  }
  pp.xsrc = x_source<MODE>(c, p, tid);
  pp.xsrc_next = ~0u;
  load_xstage(pp.xv, xr, pp.xsrc, p.K, 0u, xpart);
  // While the first loads are in flight.  The stage loop's barriers order
  // these LDS writes before the first epilogue reads them.
  if constexpr (MODE == kModeGateUp) fill_sig_tab(sig_tab, static_cast<uint32_t>(tid), kGemmThreads);

  f32x16_t acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  bool slab[4];
  uint32_t count = uniform(c.tile.z);
#pragma unroll
  for (int t = 0; t < 4; ++t) slab[t] = 32u * t < count;
  uint32_t nb = c.j % nb_count;
  for (;;) {
    switch ((count + 31u) / 32u) {  // active slabs (uniform)
      case 0:
      case 1: pp.template run<1>(acc, xs, n, n2, p, it, nb_count, wave, lane, tid, S, xr); break;
      case 2: pp.template run<2>(acc, xs, n, n2, p, it, nb_count, wave, lane, tid, S, xr); break;
      case 3: pp.template run<3>(acc, xs, n, n2, p, it, nb_count, wave, lane, tid, S, xr); break;
      default: pp.template run<4>(acc, xs, n, n2, p, it, nb_count, wave, lane, tid, S, xr); break;
    }
    // Every item starts on LDS tile 0; its last stage used tile (S - 1) & 1.
    if constexpr (MODE != kModeGateUp) down_epilogue(acc, c, p, nb, wave, lane, slab);
    else gateup_epilogue(acc, xs + ((S - 1u) & 1u) * kXTile, c, p, nb, wave, lane, slab, sig_tab);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
    c = n;
    n = n2;
    fetch_tile(n2, c.j + 2u * it.stride, it, tr);
    fetch_rows<MODE>(n, orr, xmr, tid);
    pp.xsrc = pp.xsrc_next;
    if (c.j >= it.count) break;  // uniform
    count = uniform(c.tile.z);
#pragma unroll
    for (int t = 0; t < 4; ++t) slab[t] = 32u * t < count;
    nb = c.j % nb_count;
    if (S & 1u) __syncthreads();  // odd S: tile 0 is reused back to back across the item boundary
  }
}

// ------------------------------------------------------------------ combine
// out[t] = bf16(bf16(sum_s bf16(y[t,s] * score[t,s])) + bf16(sg[t] * shared[t])):
// products rounded to bf16, the slot sum accumulated in float32 in slot order
// and rounded once (adaptive_topk.py:274-277 in MLX bf16 arithmetic).
__global__ void grouped_combine_kernel(const uint16_t *__restrict__ y, const uint16_t *__restrict__ scores,
                                       const uint16_t *__restrict__ shared, const uint16_t *__restrict__ shared_gate,
                                       uint16_t *__restrict__ out, uint32_t tokens, uint32_t slots, uint32_t hidden) {
  const uint32_t per_token = hidden / 8u;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * per_token) return;
  const uint32_t t = i / per_token, n0 = (i % per_token) * 8u;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (uint32_t s = 0; s < slots; ++s) {
    const float sc = bf16_to_f32(scores[static_cast<uint64_t>(t) * slots + s]);
    const uint4 v = *reinterpret_cast<const uint4 *>(y + (static_cast<uint64_t>(t) * slots + s) * hidden + n0);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float yv = bf16_to_f32(static_cast<uint16_t>(u[e >> 1] >> (16 * (e & 1))));
      acc[e] = __fadd_rn(acc[e], round_bf16(__fmul_rn(yv, sc)));
    }
  }
  uint32_t o[4];
  float sg = 0.0f;
  uint4 sh = make_uint4(0u, 0u, 0u, 0u);
  if (shared != nullptr) {
    sg = bf16_to_f32(shared_gate[t]);
    sh = *reinterpret_cast<const uint4 *>(shared + static_cast<uint64_t>(t) * hidden + n0);
  }
  const uint32_t su[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = 2 * q + h;
      float total = round_bf16(acc[e]);
      if (shared != nullptr) {
        const float comp = round_bf16(__fmul_rn(sg, bf16_to_f32(static_cast<uint16_t>(su[q] >> (16 * h)))));
        total = __fadd_rn(total, comp);
      }
      v[h] = total;
    }
    o[q] = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  }
  *reinterpret_cast<uint4 *>(out + static_cast<uint64_t>(t) * hidden + n0) = make_uint4(o[0], o[1], o[2], o[3]);
}

int device_flags_grouped(unsigned int **flags, hipStream_t stream) {
  DeviceWorkspace *ws = nullptr;
  const int rc = workspace(&ws, stream);
  if (rc) return rc;
  *flags = ws->flags;
  return MQ_OK;
}

int validate_proj_grouped(const MqProjection &p, const char *name) {
  if (p.pool == nullptr && p.stream_pack == nullptr && (p.weight == nullptr || p.scales == nullptr || p.biases == nullptr))
    return fail(MQ_ERR_INVALID, "%s projection needs dense arrays, a pool or a stream pack", name);
  if ((p.pool != nullptr || p.stream_pack != nullptr) && p.pool_stride == 0)
    return fail(MQ_ERR_INVALID, "%s projection record stride is zero", name);
  return MQ_OK;
}

// Weight stages in flight: a divisor of the stages per item, so the ring
// slot of a stage is fixed and the load cursor stays within one item of the
// compute cursor.  Two stages ahead keep the kernel within 256 registers per
// lane with the B-fragment read-ahead (four stages spill; measured on the
// 4096-token chunk: 4 stages 918-928 us, 2 stages 897-909 us per call).
template <int MODE, int NS, int W>
int launch_gemm_ns(const GemmParams &p, uint32_t group, uint32_t grid, hipStream_t s) {
  if (group == 32)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, NS, 32, W>), dim3(grid), dim3(kGemmThreads), 0, s, p);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, NS, 64, W>), dim3(grid), dim3(kGemmThreads), 0, s, p);
  return check_launch(MODE == kModeGateUp ? "grouped_gemm_kernel (gate/up)"
                      : MODE == kModeDown ? "grouped_gemm_kernel (down)"
                                          : "grouped_gemm_kernel (gather)");
}

template <int MODE>
int launch_gemm(const GemmParams &p, uint32_t group, uint32_t grid, hipStream_t s) {
  const uint32_t stages = p.K / kKS;
  if (stages % 4 == 0) return launch_gemm_ns<MODE, 2, 4>(p, group, grid, s);
  if (stages % 2 == 0) return launch_gemm_ns<MODE, 2, 2>(p, group, grid, s);
  if (stages % 3 == 0) return launch_gemm_ns<MODE, 3, 1>(p, group, grid, s);
  return launch_gemm_ns<MODE, 1, 1>(p, group, grid, s);
}

KeySpace key_space(const MqGroupedArgs &a) {
  KeySpace ks;
  ks.slots = a.gate.pool != nullptr ? a.gate.pool_slots : 0u;
  ks.ids = a.gate.stream_pack != nullptr ? a.gate.stream_records : (a.gate.weight != nullptr ? a.expert_count : 0u);
  return ks;
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" uint64_t mq_grouped_workspace_size(uint32_t tokens, uint32_t slots, uint32_t hidden, uint32_t inter,
                                              uint32_t route_keys, int shared) {
  return make_layout(tokens, slots, hidden, inter, route_keys, shared != 0).total;
}

namespace mq {
namespace {

// Argument checks shared by both entry points; fills the key space and layout.
int grouped_validate(const MqGroupedArgs &a, KeySpace *ks_out, Layout *l_out) {
  if (a.x == nullptr || a.routes == nullptr || a.y == nullptr)
    return fail(MQ_ERR_INVALID, "x, routes and y are required");
  if (a.tokens == 0 || a.slots == 0 || a.slots > 64) return fail(MQ_ERR_INVALID, "tokens must be positive and slots 1..64");
  if (a.group_size != 32 && a.group_size != 64) return fail(MQ_ERR_INVALID, "group_size must be 32 or 64");
  if (a.hidden % kKS || a.inter % kKS)
    return fail(MQ_ERR_UNSUPPORTED, "grouped path needs hidden and inter multiples of %u (got %u, %u)", kKS,
                a.hidden, a.inter);
  if (a.hidden > MQ_MAX_WIDTH || a.inter > MQ_MAX_WIDTH) return fail(MQ_ERR_INVALID, "width out of bounds");
  int rc;
  if ((rc = validate_proj_grouped(a.gate, "gate")) || (rc = validate_proj_grouped(a.up, "up")) ||
      (rc = validate_proj_grouped(a.down, "down")))
    return rc;
  const bool shared_expert = a.shared_expert != nullptr;
  if (shared_expert)
    for (int i = 0; i < 3; ++i)
      if ((rc = validate_proj_grouped(a.shared_expert[i], "shared"))) return rc;
  if (shared_expert && a.shared != nullptr) return fail(MQ_ERR_INVALID, "give shared or shared_expert, not both");
  if ((shared_expert || a.shared != nullptr) && a.shared_gate == nullptr)
    return fail(MQ_ERR_INVALID, "shared_gate is required with a shared expert");
  if (a.out != nullptr && a.scores == nullptr) return fail(MQ_ERR_INVALID, "scores are required to combine into out");
  const KeySpace ks = key_space(a);
  const Layout l = make_layout(a.tokens, a.slots, a.hidden, a.inter, ks.slots + ks.ids, shared_expert);
  if (static_cast<uint64_t>(a.tokens) * a.hidden * 2u >= (1ull << 31) ||
      static_cast<uint64_t>(l.rows) * a.inter * 2u >= (1ull << 31))
    return fail(MQ_ERR_UNSUPPORTED, "activation buffers must stay below 2 GiB");
  *ks_out = ks;
  *l_out = l;
  return MQ_OK;
}

struct SortBufs {
  uint32_t *counts, *cursor, *row_key, *order;
  GroupTile *tiles;
  uint32_t *n_tiles;
};

// Counting sort of `rows` rows by route key (rows past routed_rows belong to
// the shared group): `order` lists the row indices grouped by key, `tiles`
// the (word, start, count) tiles.  One block when the rows and keys fit,
// else zero / count / plan / scatter.
int sort_rows(const uint32_t *routes, uint32_t routed_rows, uint32_t rows, const KeySpace &ks, const SortBufs &b,
              unsigned int *err, hipStream_t s) {
  int rc;
  if (ks.size() <= kSingleSortKeys && rows <= 16u * kPlanThreads) {
    const uint32_t kpt = ceil_div(rows, kPlanThreads);
    const uint32_t hist_bytes = ks.size() * 4u;
    if (kpt <= 4)
      hipLaunchKernelGGL(grouped_sort_single_kernel<4>, dim3(1), dim3(kPlanThreads), hist_bytes, s, routes,
                         routed_rows, rows, ks, b.order, b.tiles, b.n_tiles, err);
    else
      hipLaunchKernelGGL(grouped_sort_single_kernel<16>, dim3(1), dim3(kPlanThreads), hist_bytes, s, routes,
                         routed_rows, rows, ks, b.order, b.tiles, b.n_tiles, err);
    return check_launch("grouped_sort_single_kernel");
  }
  hipLaunchKernelGGL(grouped_zero_kernel, dim3(ceil_div(ks.size(), 256)), dim3(256), 0, s, b.counts, ks.size());
  if ((rc = check_launch("grouped_zero_kernel"))) return rc;
  const bool lds_sort = ks.size() <= kLdsKeys;
  const uint32_t hist_bytes = ks.size() * 4u;
  if (lds_sort)
    hipLaunchKernelGGL(grouped_count_lds_kernel, dim3(ceil_div(rows, kSortRows)), dim3(kSortThreads), hist_bytes, s,
                       routes, routed_rows, rows, ks, b.counts, b.row_key, err);
  else
    hipLaunchKernelGGL(grouped_count_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0, s, routes, routed_rows, rows,
                       ks, b.counts, b.row_key, err);
  if ((rc = check_launch("grouped_count_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, b.counts, b.cursor, b.tiles, b.n_tiles,
                     ks);
  if ((rc = check_launch("grouped_plan_kernel"))) return rc;
  if (lds_sort)
    hipLaunchKernelGGL(grouped_scatter_lds_kernel, dim3(ceil_div(rows, kSortRows)), dim3(kSortThreads), hist_bytes, s,
                       b.row_key, rows, ks, b.cursor, b.order);
  else
    hipLaunchKernelGGL(grouped_scatter_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0, s, b.row_key, rows, b.cursor,
                       b.order);
  return check_launch("grouped_scatter_kernel");
}

// GEMM grid bound: one 8-wave block per CU, a multiple of 8 (XCD-aware item
// schedule).
int gemm_blocks(uint32_t *resident) {
  int device = 0, cus = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  MQ_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  *resident = std::max(8u, (static_cast<uint32_t>(cus > 0 ? cus : 256) / 8u) * 8u);
  return MQ_OK;
}

// The whole grouped call with its scratch at `ws` (at least the layout's bytes).
int grouped_call(const MqGroupedArgs &a, uint8_t *ws, uint64_t ws_bytes, hipStream_t s) {
  KeySpace ks;
  Layout l;
  int rc = grouped_validate(a, &ks, &l);
  if (rc) return rc;
  if (ws == nullptr || ws_bytes < l.total)
    return fail(MQ_ERR_INVALID, "workspace needs %llu bytes (got %llu)", static_cast<unsigned long long>(l.total),
                static_cast<unsigned long long>(ws_bytes));
  const bool shared_expert = a.shared_expert != nullptr;
  unsigned int *err = nullptr;
  if ((rc = device_flags_grouped(&err, s))) return rc;

  uint32_t *order = reinterpret_cast<uint32_t *>(ws + l.order);
  GroupTile *tiles = reinterpret_cast<GroupTile *>(ws + l.tiles);
  uint32_t *n_tiles = reinterpret_cast<uint32_t *>(ws + l.n_tiles);
  uint16_t *act = reinterpret_cast<uint16_t *>(ws + l.act);
  uint16_t *y_shared = shared_expert ? reinterpret_cast<uint16_t *>(ws + l.y_shared) : nullptr;
  const uint32_t routed_rows = a.tokens * a.slots;
  const SortBufs sb{reinterpret_cast<uint32_t *>(ws + l.counts), reinterpret_cast<uint32_t *>(ws + l.cursor),
                    reinterpret_cast<uint32_t *>(ws + l.row_key), order, tiles, n_tiles};
  if ((rc = sort_rows(a.routes, routed_rows, l.rows, ks, sb, err, s))) return rc;

  uint32_t resident = 0;
  if ((rc = gemm_blocks(&resident))) return rc;
  GemmParams gp{};
  gp.x = a.x;
  gp.x_bytes = a.tokens * a.hidden * 2u;
  gp.w0 = a.gate;
  gp.w1 = a.up;
  if (shared_expert) {
    gp.s0 = a.shared_expert[0];
    gp.s1 = a.shared_expert[1];
  }
  gp.tiles = tiles;
  gp.tiles_bytes = l.max_tiles * static_cast<uint32_t>(sizeof(GroupTile));
  gp.n_tiles = n_tiles;
  gp.order = order;
  gp.order_bytes = l.rows * 4u;
  gp.out = act;
  gp.slots = a.slots;
  gp.routed_rows = routed_rows;
  gp.K = a.hidden;
  gp.N = a.inter;
  gp.dense_count = a.expert_count;
  gp.err = err;
  const uint32_t gu_items = l.max_tiles * ceil_div(a.inter, kGateUpFeatures);
  if ((rc = launch_gemm<kModeGateUp>(gp, a.group_size, std::min(ceil_div(gu_items, 8) * 8u, resident), s))) return rc;

  GemmParams dp = gp;
  dp.x = act;
  dp.x_bytes = l.rows * a.inter * 2u;
  dp.w0 = a.down;
  dp.w1 = MqProjection{};
  dp.s0 = shared_expert ? a.shared_expert[2] : MqProjection{};
  dp.s1 = MqProjection{};
  dp.out = a.y;
  dp.out_shared = y_shared;
  dp.K = a.inter;
  dp.N = a.hidden;
  const uint32_t dn_items = l.max_tiles * ceil_div(a.hidden, kDownFeatures);
  if ((rc = launch_gemm<kModeDown>(dp, a.group_size, std::min(ceil_div(dn_items, 8) * 8u, resident), s))) return rc;

  if (a.out != nullptr) {
    const uint16_t *shared_vec = shared_expert ? y_shared : a.shared;
    const uint32_t n = a.tokens * (a.hidden / 8u);
    hipLaunchKernelGGL(grouped_combine_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, s, a.y, a.scores, shared_vec,
                       a.shared_gate, a.out, a.tokens, a.slots, a.hidden);
    if ((rc = check_launch("grouped_combine_kernel"))) return rc;
  }
  return MQ_OK;
}

// Scratch of mq_moe_grouped_static: one copy per device, held until the
// process ends.  Host code never uses the array's name as an address: the
// device address of the current device's copy is resolved once per device
// with hipGetSymbolAddress and kept in g_static_scratch.
constexpr uint64_t kStaticScratchBytes = MQ_GROUPED_STATIC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

int static_scratch(uint8_t **out) {
  static std::mutex mu;
  static uint8_t *per_device[64];
  int device = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  if (device < 0 || device >= 64) return fail(MQ_ERR_DEVICE, "device ordinal %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (per_device[device] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    per_device[device] = static_cast<uint8_t *>(ptr);
  }
  *out = per_device[device];
  return MQ_OK;
}

}  // namespace
}  // namespace mq

extern "C" uint64_t mq_gather_qmm_workspace_size(uint32_t rows, uint32_t route_keys) {
  return make_gather_layout(rows, route_keys).total;
}

extern "C" int mq_gather_qmm(const MqGatherArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqGatherArgs &a = *args;
  if (a.x == nullptr || a.routes == nullptr || a.out == nullptr) return fail(MQ_ERR_INVALID, "x, routes and out are required");
  if (a.group_size != 32 && a.group_size != 64) return fail(MQ_ERR_INVALID, "group_size must be 32 or 64");
  if (a.in_width == 0 || a.in_width % kKS)
    return fail(MQ_ERR_UNSUPPORTED, "gather_qmm needs in_width a positive multiple of %u (got %u)", kKS, a.in_width);
  if (a.out_width == 0 || a.out_width % 4u)
    return fail(MQ_ERR_UNSUPPORTED, "gather_qmm needs out_width a positive multiple of 4 (got %u)", a.out_width);
  if (a.in_width > MQ_MAX_WIDTH || a.out_width > MQ_MAX_WIDTH) return fail(MQ_ERR_INVALID, "width out of bounds");
  if (a.x_rows == nullptr && a.x_count < a.rows)
    return fail(MQ_ERR_INVALID, "without x_rows, x must hold every row (x_count %u < rows %u)", a.x_count, a.rows);
  if (static_cast<uint64_t>(a.x_count) * a.in_width * 2u >= (1ull << 31) || a.rows >= (1u << 28))
    return fail(MQ_ERR_UNSUPPORTED, "x must stay below 2 GiB and rows below 2^28");
  int rc;
  if ((rc = validate_proj_grouped(a.w, "w"))) return rc;
  if (a.rows == 0) return MQ_OK;
  KeySpace ks;
  ks.slots = a.w.pool != nullptr ? a.w.pool_slots : 0u;
  ks.ids = a.w.stream_pack != nullptr ? a.w.stream_records : (a.w.weight != nullptr ? a.expert_count : 0u);
  const GatherLayout l = make_gather_layout(a.rows, ks.slots + ks.ids);
  if (a.workspace == nullptr || a.workspace_bytes < l.total)
    return fail(MQ_ERR_INVALID, "workspace needs %llu bytes (got %llu)", static_cast<unsigned long long>(l.total),
                static_cast<unsigned long long>(a.workspace_bytes));
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned int *err = nullptr;
  if ((rc = device_flags_grouped(&err, s))) return rc;
  uint8_t *ws = static_cast<uint8_t *>(a.workspace);
  uint32_t *order = reinterpret_cast<uint32_t *>(ws + l.order);
  GroupTile *tiles = reinterpret_cast<GroupTile *>(ws + l.tiles);
  uint32_t *n_tiles = reinterpret_cast<uint32_t *>(ws + l.n_tiles);
  const SortBufs sb{reinterpret_cast<uint32_t *>(ws + l.counts), reinterpret_cast<uint32_t *>(ws + l.cursor),
                    reinterpret_cast<uint32_t *>(ws + l.row_key), order, tiles, n_tiles};
  if ((rc = sort_rows(a.routes, a.rows, a.rows, ks, sb, err, s))) return rc;
  const uint32_t *xmap = order;  // without x_rows, sorted row i reads x row order[i]
  if (a.x_rows != nullptr) {
    uint32_t *m = reinterpret_cast<uint32_t *>(ws + l.xmap);
    hipLaunchKernelGGL(gather_map_kernel, dim3(ceil_div(a.rows, 256)), dim3(256), 0, s, order, a.x_rows, a.rows,
                       a.x_count, m, err);
    if ((rc = check_launch("gather_map_kernel"))) return rc;
    xmap = m;
  }
  uint32_t resident = 0;
  if ((rc = gemm_blocks(&resident))) return rc;
  GemmParams gp{};
  gp.x = a.x;
  gp.x_bytes = a.x_count * a.in_width * 2u;
  gp.xmap = xmap;
  gp.xmap_bytes = a.rows * 4u;
  gp.w0 = a.w;
  gp.tiles = tiles;
  gp.tiles_bytes = l.max_tiles * static_cast<uint32_t>(sizeof(GroupTile));
  gp.n_tiles = n_tiles;
  gp.order = order;
  gp.order_bytes = a.rows * 4u;
  gp.out = a.out;
  gp.slots = 1u;
  gp.routed_rows = a.rows;
  gp.K = a.in_width;
  gp.N = a.out_width;
  gp.dense_count = a.expert_count;
  gp.err = err;
  const uint32_t items = l.max_tiles * ceil_div(a.out_width, kDownFeatures);
  return launch_gemm<kModeGather>(gp, a.group_size, std::min(ceil_div(items, 8) * 8u, resident), s);
}

extern "C" int mq_moe_grouped(const MqGroupedArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  return grouped_call(*args, static_cast<uint8_t *>(args->workspace), args->workspace_bytes,
                      static_cast<hipStream_t>(stream));
}

extern "C" int mq_moe_grouped_static(const MqGroupedArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqGroupedArgs &a = *args;
  KeySpace ks;
  Layout l;
  int rc = grouped_validate(a, &ks, &l);
  if (rc) return rc;
  if (l.total > kStaticScratchBytes)
    return fail(MQ_ERR_INVALID,
                "mq_moe_grouped_static: this call needs %llu bytes of scratch, above the static maximum of %llu "
                "(MQ_GROUPED_STATIC_SCRATCH_BYTES); use mq_moe_grouped with a workspace",
                static_cast<unsigned long long>(l.total), static_cast<unsigned long long>(kStaticScratchBytes));
  uint8_t *scratch_ptr = nullptr;
  if ((rc = static_scratch(&scratch_ptr))) return rc;
  return grouped_call(a, scratch_ptr, kStaticScratchBytes, static_cast<hipStream_t>(stream));
}
