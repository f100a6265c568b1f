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
//      and a tile list of (route word, first sorted row, rows <= 128);
//   2. gate/up GEMM: per (tile, 64 features) a 256-thread block stages the
//      tile's token rows of x and the 128 weight rows (64 gate + 64 up
//      features) dequantized to bf16 in LDS, 64 inputs per stage, and runs
//      v_mfma_f32_32x32x16_bf16 (fp32 accumulate); the epilogue rounds gate
//      and up to bf16 and writes act = swiglu(g, u) in sorted row order;
//   3. down GEMM: per (tile, 128 features) the same scheme over act, the
//      bf16 outputs are scattered back to y[token, slot] (or the shared
//      expert's row);
//   4. combine: out = bf16 generic combine of y with the scores + the gated
//      shared expert.
// Weights are dequantized as bf16(fma(q, s, b)) (one float32 rounding, then
// bf16); every output row is computed independently of its position in a
// tile, so the result does not depend on the order rows land in a tile.
#include "mq_internal.h"
#include "mq_select.h"

namespace mq {
namespace {

constexpr uint32_t kTileRows = 128;  // sorted rows (tokens) per tile: four 32-row slabs
constexpr uint32_t kKS = 128;        // inputs per pipeline stage
constexpr uint32_t kFrags = 1;       // 32-row weight fragments per wave
constexpr uint32_t kWRows = 4 * kFrags * 32;  // weight rows per block (256)
constexpr uint32_t kGateUpFeatures = kWRows / 2;  // per gate/up block: 128 gate + 128 up rows
constexpr uint32_t kDownFeatures = kWRows;        // per down block
constexpr uint32_t kSharedWord = 0xfffffffeu;  // tile word of the shared expert group
constexpr uint32_t kDeadWord = 0xffffffffu;    // tile word of rows with invalid route words
constexpr int kPlanThreads = 1024;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t2 __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

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
// cursors, and the tile list.  Each thread owns a contiguous run of keys.
__global__ __launch_bounds__(kPlanThreads) void grouped_plan_kernel(const uint32_t *__restrict__ counts,
                                                                     uint32_t *__restrict__ cursor,
                                                                     GroupTile *__restrict__ tiles,
                                                                     uint32_t *__restrict__ n_tiles, KeySpace ks) {
  __shared__ uint32_t s_rows[kPlanThreads], s_tiles[kPlanThreads];
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

__global__ void grouped_scatter_kernel(const uint32_t *__restrict__ row_key, uint32_t rows,
                                       uint32_t *__restrict__ cursor, uint32_t *__restrict__ order) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = r < rows;
  const uint32_t key = active ? row_key[r] : 0u;
  const uint32_t pos = wave_aggregated_increment<true>(cursor, key, active);
  if (active) order[pos] = r;
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
// k0 + 64 h + 8 j .. +7: each lane then owns 64 consecutive inputs of its
// row per stage, i.e. 32 contiguous bytes of packed weights (two 16-byte
// loads straight into registers, no LDS), and the same 128 contiguous bytes
// of its activation row.

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

// One lane's weight fragment rows: descriptor (uniform across the wave) and
// global row (feature), with validity.
struct WFrag {
  ExpertRsrc e;
  uint32_t feature;
  bool ok;
};

// A lane's packed weights for one stage and fragment: 64 inputs = 8 words
// (two 16-byte loads) and the scale/bias of each of their groups (one for
// group 64, two for group 32).
struct WRegs {
  uint4 w[kFrags][2];
  uint16_t s[kFrags][2], b[kFrags][2];
};

__device__ __forceinline__ void load_w(WRegs &r, const WFrag (&wf)[kFrags], uint32_t K, uint32_t group,
                                       uint32_t kbase) {
#pragma unroll
  for (uint32_t f = 0; f < kFrags; ++f)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t k = kbase + 32u * h;
      const uint32_t off_w = wf[f].ok ? wf[f].feature * (K / 2u) + k / 2u : kOutOfRange;
      const uint32_t off_g = wf[f].ok ? (wf[f].feature * (K / group) + k / group) * 2u : kOutOfRange;
      r.w[f][h] = buf_load16(wf[f].e.w, off_w);
      r.s[f][h] = buf_load2(wf[f].e.s, off_g);
      r.b[f][h] = buf_load2(wf[f].e.b, off_g);
    }
}

// A thread's share of the activation tile of one stage: 64 inputs (128 bytes)
// of tile row t/2, half t%2 of the stage.
struct XRegs {
  uint4 x[8];
};

__device__ __forceinline__ void load_x(XRegs &r, __amdgpu_buffer_rsrc_t xr, bool ok, uint32_t src, uint32_t K,
                                       uint32_t kbase) {
  const uint32_t off = ok ? (src * K + kbase) * 2u : kOutOfRange;
#pragma unroll
  for (int j = 0; j < 8; ++j) r.x[j] = buf_load16(xr, off + 16u * j);
}

// The grouped GEMM core of one work item: C[256 weight rows x 128 tile rows]
// over K inputs.  Wave w owns weight rows [64 w, +64) as kFrags fragments
// (weights dequantized from registers) x 4 slabs of 32 tile rows (activations
// from LDS); fp32 accumulators.
struct GemmCore {
  f32x16_t acc[kFrags][4];
};

// One pipeline stage: publish this stage's activations (loaded last stage)
// to LDS, issue the next stage's loads (weights into `wn`), then run the
// stage's MFMAs with the weights in `wc` dequantized per k16 step.
__device__ __forceinline__ void gemm_stage(GemmCore &c, uint16_t *xs, const uint16_t *xs_lane, const WRegs &wc,
                                           WRegs &wn, XRegs &x, const WFrag (&wf)[kFrags], uint32_t K,
                                           uint32_t group, __amdgpu_buffer_rsrc_t xr, bool x_ok, uint32_t xsrc,
                                           uint32_t s, uint32_t stages, uint32_t xrow, uint32_t xhalf, uint32_t half,
                                           const bool (&slab)[4]) {
  __syncthreads();  // every wave is done reading the previous activation tile
#pragma unroll
  for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4 *>(xs + xs_off(xrow, 8u * xhalf + j)) = x.x[j];
  __syncthreads();
  if (s + 1 < stages) {
    load_w(wn, wf, K, group, (s + 1) * kKS + 64u * half);
    load_x(x, xr, x_ok, xsrc, K, (s + 1) * kKS + 64u * xhalf);
  }
  float sf[kFrags][2], bf[kFrags][2];
#pragma unroll
  for (uint32_t f = 0; f < kFrags; ++f)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sf[f][h] = bf16_to_f32(wc.s[f][h]);
      bf[f][h] = bf16_to_f32(wc.b[f][h]);
    }
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // k16 steps: inputs k0 + 64 half + 8 j
    bf16x8_t b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) b[t] = *reinterpret_cast<const bf16x8_t *>(xs_lane + 32u * t * kXRow + 8u * j);
#pragma unroll
    for (uint32_t f = 0; f < kFrags; ++f) {
      const uint4 &q = wc.w[f][j >> 2];
      const uint32_t word = (j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w;
      const bf16x8_t a = dequant_word(word, sf[f][j >> 2], bf[f][j >> 2]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (slab[t]) c.acc[f][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[t], c.acc[f][t], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void gemm_core(GemmCore &c, uint16_t *xs, const WFrag (&wf)[kFrags], uint32_t K,
                                          uint32_t group, __amdgpu_buffer_rsrc_t xr, bool x_ok, uint32_t xsrc,
                                          uint32_t count) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t half = static_cast<uint32_t>(lane) >> 5;
  const uint32_t xrow = static_cast<uint32_t>(tid) >> 1, xhalf = static_cast<uint32_t>(tid) & 1u;
#pragma unroll
  for (uint32_t f = 0; f < kFrags; ++f)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) c.acc[f][j][r] = 0.0f;
  bool slab[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) slab[j] = 32u * j < count;
  const uint32_t stages = K / kKS;
  WRegs w0, w1;
  XRegs x;
  load_w(w0, wf, K, group, 64u * half);
  load_x(x, xr, x_ok, xsrc, K, 64u * xhalf);
  const uint16_t *xs_lane = xs + (lane & 31) * kXRow + 64u * half;
  // Two stages per trip so the weight registers alternate without copies.
  for (uint32_t s = 0; s < stages; s += 2) {
    gemm_stage(c, xs, xs_lane, w0, w1, x, wf, K, group, xr, x_ok, xsrc, s, stages, xrow, xhalf, half, slab);
    if (s + 1 < stages)
      gemm_stage(c, xs, xs_lane, w1, w0, x, wf, K, group, xr, x_ok, xsrc, s + 1, stages, xrow, xhalf, half, slab);
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

struct GateUpParams {
  const uint16_t *x;
  uint32_t tokens;
  MqProjection gate, up;
  MqProjection sgate, sup;  // shared expert (dense, expert 0) or unused
  const GroupTile *tiles;
  const uint32_t *n_tiles;
  const uint32_t *order;
  uint16_t *act;  // [rows, inter] sorted order
  uint32_t slots, routed_rows, hidden, inter, group, dense_count;
  unsigned int *err;
};

// Fragment F (0..7) of a gate/up block holds gate features 16 F .. +15 in
// its rows 0-15 and the matching up features in rows 16-31, so a lane's C
// registers r and r+8 are gate and up of the same feature.
__global__ __launch_bounds__(256, 2) void grouped_gateup_kernel(GateUpParams p) {
  __shared__ __align__(16) uint16_t xs[kTileRows * kXRow];
  __shared__ uint32_t row_src[kTileRows];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t nb_count = (p.inter + kGateUpFeatures - 1) / kGateUpFeatures;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.tokens * p.hidden * 2u);
  const XcdItems it(*p.n_tiles, nb_count);
  for (uint32_t j = it.first; j < it.count; j += it.stride) {
    const uint32_t nb = j % nb_count;
    const GroupTile tile = p.tiles[it.tile(j)];
    __syncthreads();  // the previous item is done with row_src
    if (tid < static_cast<int>(kTileRows)) {
      uint32_t src = ~0u;
      if (static_cast<uint32_t>(tid) < tile.count) {
        const uint32_t r = p.order[tile.start + tid];
        src = r < p.routed_rows ? r / p.slots : r - p.routed_rows;
      }
      row_src[tid] = src;
    }
    ExpertPtrs eg, eu;
    if (tile.word == kSharedWord) {
      eg = expert_ptrs(p.sgate, 0u, p.inter, p.hidden, p.group, 1u);
      eu = expert_ptrs(p.sup, 0u, p.inter, p.hidden, p.group, 1u);
    } else {
      eg = expert_ptrs(p.gate, tile.word, p.inter, p.hidden, p.group, p.dense_count);
      eu = expert_ptrs(p.up, tile.word, p.inter, p.hidden, p.group, p.dense_count);
    }
    if ((!eg.ok || !eu.ok) && tid == 0 && tile.word != kDeadWord) raise_flag(p.err, MQ_DEVFLAG_BAD_ROUTE);
    __syncthreads();
    // Lane rows: fragment row (lane % 32) < 16 is a gate row, else an up row.
    const bool up_half = (lane & 31) >= 16;
    const ExpertRsrc rg = expert_rsrc(eg, p.inter, p.hidden, p.group);
    const ExpertRsrc ru = expert_rsrc(eu, p.inter, p.hidden, p.group);
    WFrag wf[kFrags];
#pragma unroll
    for (uint32_t f = 0; f < kFrags; ++f) {
      const uint32_t frag = wave * kFrags + f;
      const uint32_t feature = nb * kGateUpFeatures + 16u * frag + (lane & 15);
      wf[f] = {up_half ? ru : rg, feature, feature < p.inter};
    }
    const uint32_t xsrc = row_src[static_cast<uint32_t>(tid) >> 1];
    GemmCore c;
    gemm_core(c, xs, wf, p.hidden, p.group, xr, xsrc != ~0u, xsrc, tile.count);
    // Epilogue: act = swiglu(bf16(g), bf16(u)) in sorted row order.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t trow = 32u * t + (lane & 31);
      if (trow >= tile.count) continue;
      uint16_t *dst = p.act + static_cast<uint64_t>(tile.start + trow) * p.inter;
#pragma unroll
      for (uint32_t f = 0; f < kFrags; ++f) {
        const uint32_t frag = wave * kFrags + f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint32_t feat = nb * kGateUpFeatures + 16u * frag + c_row(r, lane);
          if (feat >= p.inter) continue;
          const float g = round_bf16(c.acc[f][t][r]);
          const float u = round_bf16(c.acc[f][t][r + 8]);
          dst[feat] = f32_to_bf16(swiglu_bf16(g, u));
        }
      }
    }
  }
}

struct DownParams {
  const uint16_t *act;
  uint32_t rows;
  MqProjection down, sdown;
  const GroupTile *tiles;
  const uint32_t *n_tiles;
  const uint32_t *order;
  uint16_t *y;         // [routed_rows, hidden]
  uint16_t *y_shared;  // [tokens, hidden] or null
  uint32_t routed_rows, hidden, inter, group, dense_count;
};

// Fragment F (0..7) of a down block holds features 32 F .. +31.
__global__ __launch_bounds__(256, 2) void grouped_down_kernel(DownParams p) {
  __shared__ __align__(16) uint16_t xs[kTileRows * kXRow];
  __shared__ uint32_t row_dst[kTileRows];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t nb_count = (p.hidden + kDownFeatures - 1) / kDownFeatures;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.act, p.rows * p.inter * 2u);
  const XcdItems it(*p.n_tiles, nb_count);
  for (uint32_t j = it.first; j < it.count; j += it.stride) {
    const uint32_t nb = j % nb_count;
    const GroupTile tile = p.tiles[it.tile(j)];
    __syncthreads();  // the previous item's epilogue is done with row_dst
    if (tid < static_cast<int>(kTileRows))
      row_dst[tid] = static_cast<uint32_t>(tid) < tile.count ? p.order[tile.start + tid] : ~0u;
    const ExpertPtrs ed = tile.word == kSharedWord
                              ? expert_ptrs(p.sdown, 0u, p.hidden, p.inter, p.group, 1u)
                              : expert_ptrs(p.down, tile.word, p.hidden, p.inter, p.group, p.dense_count);
    __syncthreads();
    const ExpertRsrc e = expert_rsrc(ed, p.hidden, p.inter, p.group);
    WFrag wf[kFrags];
#pragma unroll
    for (uint32_t f = 0; f < kFrags; ++f) {
      const uint32_t feature = nb * kDownFeatures + 32u * (wave * kFrags + f) + (lane & 31);
      wf[f] = {e, feature, feature < p.hidden};
    }
    const uint32_t xrow = static_cast<uint32_t>(tid) >> 1;
    GemmCore c;
    gemm_core(c, xs, wf, p.inter, p.group, xr, xrow < tile.count, tile.start + xrow, tile.count);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t trow = 32u * t + (lane & 31);
      if (trow >= tile.count) continue;
      const uint32_t r = row_dst[trow];
      uint16_t *dst = r < p.routed_rows ? p.y + static_cast<uint64_t>(r) * p.hidden
                                        : p.y_shared + static_cast<uint64_t>(r - p.routed_rows) * p.hidden;
#pragma unroll
      for (uint32_t f = 0; f < kFrags; ++f)
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // four runs of 4 consecutive features
          const uint32_t feat = nb * kDownFeatures + 32u * (wave * kFrags + f) + c_row(4 * q, lane);
          if (feat >= p.hidden) continue;
          const uint32_t lo = pack_bf16(c.acc[f][t][4 * q], c.acc[f][t][4 * q + 1]);
          const uint32_t hi = pack_bf16(c.acc[f][t][4 * q + 2], c.acc[f][t][4 * q + 3]);
          *reinterpret_cast<uint2 *>(dst + feat) = make_uint2(lo, hi);
        }
    }
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

extern "C" int mq_moe_grouped(const MqGroupedArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqGroupedArgs &a = *args;
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
  if (a.workspace == nullptr || a.workspace_bytes < l.total)
    return fail(MQ_ERR_INVALID, "workspace needs %llu bytes (got %llu)", static_cast<unsigned long long>(l.total),
                static_cast<unsigned long long>(a.workspace_bytes));
  if (static_cast<uint64_t>(a.tokens) * a.hidden * 2u >= (1ull << 31) ||
      static_cast<uint64_t>(l.rows) * a.inter * 2u >= (1ull << 31))
    return fail(MQ_ERR_UNSUPPORTED, "activation buffers must stay below 2 GiB");
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned int *err = nullptr;
  if ((rc = device_flags_grouped(&err, s))) return rc;

  uint8_t *ws = static_cast<uint8_t *>(a.workspace);
  uint32_t *counts = reinterpret_cast<uint32_t *>(ws + l.counts);
  uint32_t *cursor = reinterpret_cast<uint32_t *>(ws + l.cursor);
  uint32_t *row_key = reinterpret_cast<uint32_t *>(ws + l.row_key);
  uint32_t *order = reinterpret_cast<uint32_t *>(ws + l.order);
  GroupTile *tiles = reinterpret_cast<GroupTile *>(ws + l.tiles);
  uint32_t *n_tiles = reinterpret_cast<uint32_t *>(ws + l.n_tiles);
  uint16_t *act = reinterpret_cast<uint16_t *>(ws + l.act);
  uint16_t *y_shared = shared_expert ? reinterpret_cast<uint16_t *>(ws + l.y_shared) : nullptr;
  const uint32_t routed_rows = a.tokens * a.slots;

  hipLaunchKernelGGL(grouped_zero_kernel, dim3(ceil_div(ks.size(), 256)), dim3(256), 0, s, counts, ks.size());
  if ((rc = check_launch("grouped_zero_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_count_kernel, dim3(ceil_div(l.rows, 256)), dim3(256), 0, s, a.routes, routed_rows,
                     l.rows, ks, counts, row_key, err);
  if ((rc = check_launch("grouped_count_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, counts, cursor, tiles, n_tiles, ks);
  if ((rc = check_launch("grouped_plan_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_scatter_kernel, dim3(ceil_div(l.rows, 256)), dim3(256), 0, s, row_key, l.rows, cursor,
                     order);
  if ((rc = check_launch("grouped_scatter_kernel"))) return rc;

  int device = 0, cus = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  MQ_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  // One 256-thread block per CU, a multiple of 8 (XCD-aware item schedule).
  const uint32_t resident = std::max(8u, (static_cast<uint32_t>(cus > 0 ? cus : 256) * 2u / 8u) * 8u);

  GateUpParams gp{};
  gp.x = a.x;
  gp.tokens = a.tokens;
  gp.gate = a.gate;
  gp.up = a.up;
  if (shared_expert) {
    gp.sgate = a.shared_expert[0];
    gp.sup = a.shared_expert[1];
  }
  gp.tiles = tiles;
  gp.n_tiles = n_tiles;
  gp.order = order;
  gp.act = act;
  gp.slots = a.slots;
  gp.routed_rows = routed_rows;
  gp.hidden = a.hidden;
  gp.inter = a.inter;
  gp.group = a.group_size;
  gp.dense_count = a.expert_count;
  gp.err = err;
  const uint32_t gu_items = l.max_tiles * ceil_div(a.inter, kGateUpFeatures);
  hipLaunchKernelGGL(grouped_gateup_kernel, dim3(std::min(ceil_div(gu_items, 8) * 8u, resident)), dim3(256), 0, s, gp);
  if ((rc = check_launch("grouped_gateup_kernel"))) return rc;

  DownParams dp{};
  dp.act = act;
  dp.rows = l.rows;
  dp.down = a.down;
  if (shared_expert) dp.sdown = a.shared_expert[2];
  dp.tiles = tiles;
  dp.n_tiles = n_tiles;
  dp.order = order;
  dp.y = a.y;
  dp.y_shared = y_shared;
  dp.routed_rows = routed_rows;
  dp.hidden = a.hidden;
  dp.inter = a.inter;
  dp.group = a.group_size;
  dp.dense_count = a.expert_count;
  const uint32_t dn_items = l.max_tiles * ceil_div(a.hidden, kDownFeatures);
  hipLaunchKernelGGL(grouped_down_kernel, dim3(std::min(ceil_div(dn_items, 8) * 8u, resident)), dim3(256), 0, s, dp);
  if ((rc = check_launch("grouped_down_kernel"))) return rc;

  if (a.out != nullptr) {
    const uint16_t *shared_vec = shared_expert ? y_shared : a.shared;
    const uint32_t n = a.tokens * (a.hidden / 8u);
    hipLaunchKernelGGL(grouped_combine_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, s, a.y, a.scores, shared_vec,
                       a.shared_gate, a.out, a.tokens, a.slots, a.hidden);
    if ((rc = check_launch("grouped_combine_kernel"))) return rc;
  }
  return MQ_OK;
}
