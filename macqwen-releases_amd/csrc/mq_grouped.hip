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

constexpr uint32_t kTileRows = 128;  // sorted rows (tokens) per tile
constexpr uint32_t kBK = 64;         // inputs per pipeline stage
constexpr uint32_t kLdsK = kBK + 8;  // padded LDS row (bf16), keeps 16-byte reads conflict-free
constexpr uint32_t kGateUpFeatures = 64;  // per gate/up block: 64 gate + 64 up weight rows
constexpr uint32_t kDownFeatures = 128;   // per down block
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

__global__ void grouped_count_kernel(const uint32_t *__restrict__ routes, uint32_t routed_rows, uint32_t rows,
                                     KeySpace ks, uint32_t *__restrict__ counts, uint32_t *__restrict__ row_key,
                                     unsigned int *__restrict__ err) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const uint32_t key = r < routed_rows ? key_of(routes[r], ks) : ks.shared_key();
  if (key == ks.dead_key()) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);
  row_key[r] = key;
  atomicAdd(&counts[key], 1u);
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
  if (r >= rows) return;
  const uint32_t pos = atomicAdd(&cursor[row_key[r]], 1u);
  order[pos] = r;
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

// One thread's share of one pipeline stage: 32 consecutive inputs (one
// 16-byte packed weight load, its group's scale and bias) of one weight row,
// and 32 consecutive inputs (four 16-byte loads) of one activation row.
struct StageRegs {
  uint4 w;
  uint16_t s, b;
  uint4 x[4];
};

__device__ __forceinline__ void stage_load(StageRegs &r, const ExpertRsrc &e, bool w_ok, uint32_t feature,
                                           uint32_t K, uint32_t group, uint32_t k0,
                                           __amdgpu_buffer_rsrc_t xr, bool x_ok, uint32_t xsrc) {
  const uint32_t off_w = w_ok ? feature * (K / 2u) + k0 / 2u : kOutOfRange;
  const uint32_t off_g = w_ok ? (feature * (K / group) + k0 / group) * 2u : kOutOfRange;
  r.w = buf_load16<kNonTemporal>(e.w, off_w);
  r.s = buf_load2(e.s, off_g);
  r.b = buf_load2(e.b, off_g);
  const uint32_t off_x = x_ok ? (xsrc * K + k0) * 2u : kOutOfRange;
#pragma unroll
  for (int j = 0; j < 4; ++j) r.x[j] = buf_load16(xr, off_x + 16u * j);
}

// Dequantize the weight part to bf16(fma(q, s, b)) and write both parts to LDS.
__device__ __forceinline__ void stage_store(const StageRegs &r, uint16_t *ws_row, uint16_t *xs_row) {
  const float s = bf16_to_f32(r.s), b = bf16_to_f32(r.b);
  const uint32_t words[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
  uint32_t pk[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // Nibble e of word j is input 8j+e; even nibbles sit in the low halves of
    // the bytes of `lo`, odd ones in `hi`.
    const uint32_t lo = words[j] & 0x0f0f0f0fu;
    const uint32_t hi = (words[j] >> 4) & 0x0f0f0f0fu;
    pk[4 * j + 0] = pack_bf16(fmaf(ubyte_to_f32<0>(lo), s, b), fmaf(ubyte_to_f32<0>(hi), s, b));
    pk[4 * j + 1] = pack_bf16(fmaf(ubyte_to_f32<1>(lo), s, b), fmaf(ubyte_to_f32<1>(hi), s, b));
    pk[4 * j + 2] = pack_bf16(fmaf(ubyte_to_f32<2>(lo), s, b), fmaf(ubyte_to_f32<2>(hi), s, b));
    pk[4 * j + 3] = pack_bf16(fmaf(ubyte_to_f32<3>(lo), s, b), fmaf(ubyte_to_f32<3>(hi), s, b));
  }
  uint4 *wd = reinterpret_cast<uint4 *>(ws_row);
#pragma unroll
  for (int j = 0; j < 4; ++j) wd[j] = make_uint4(pk[4 * j], pk[4 * j + 1], pk[4 * j + 2], pk[4 * j + 3]);
  uint4 *xd = reinterpret_cast<uint4 *>(xs_row);
#pragma unroll
  for (int j = 0; j < 4; ++j) xd[j] = r.x[j];
}

// The grouped GEMM core of one work item: C[128 weight rows x 128 rows] over
// K inputs.  Wave (wr, wt) owns weight rows [64 wr, +64) and tile rows
// [64 wt, +64) as 2 x 2 MFMA 32x32 tiles.  Thread t stages weight row t/2 and
// tile row t/2, inputs 32 (t%2) .. +32 of every stage.
struct GemmCore {
  f32x16_t acc[2][2];
};

// `w_lds_row`: the LDS weight row this thread stages (its descriptor `e` must
// be the same for all lanes of a wave).
__device__ __forceinline__ void gemm_core(GemmCore &c, uint16_t *ws, uint16_t *xs, const ExpertRsrc &e, bool w_ok,
                                          uint32_t feature, uint32_t w_lds_row, uint32_t K, uint32_t group,
                                          __amdgpu_buffer_rsrc_t xr, bool x_ok, uint32_t xsrc, uint32_t count) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t wr = wave & 1u, wt = wave >> 1;
  const uint32_t half = tid & 1;
  uint16_t *ws_row = ws + w_lds_row * kLdsK + half * 32u;
  uint16_t *xs_row = xs + (tid >> 1) * kLdsK + half * 32u;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) c.acc[i][j][r] = 0.0f;
  const bool tok_frag[2] = {wt * 64u < count, wt * 64u + 32u < count};
  const uint32_t stages = K / kBK;
  StageRegs st;
  stage_load(st, e, w_ok, feature, K, group, half * 32u, xr, x_ok, xsrc);
  for (uint32_t s = 0; s < stages; ++s) {
    __syncthreads();  // every wave is done reading the previous stage
    stage_store(st, ws_row, xs_row);
    __syncthreads();
    if (s + 1 < stages) stage_load(st, e, w_ok, feature, K, group, (s + 1) * kBK + half * 32u, xr, x_ok, xsrc);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t kcol = kk * 16u + (lane >> 5) * 8u;
      bf16x8_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t *>(ws + (wr * 64u + i * 32u + (lane & 31)) * kLdsK + kcol);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t *>(xs + (wt * 64u + j * 32u + (lane & 31)) * kLdsK + kcol);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (!tok_frag[j]) continue;  // wave-uniform: no rows in this 32-row slab
#pragma unroll
        for (int i = 0; i < 2; ++i) c.acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], c.acc[i][j], 0, 0, 0);
      }
    }
  }
}

// C-tile register r of lane l holds weight row 8*(r/4) + 4*(l/32) + r%4 of the
// 32-row fragment and tile row l%32 of the 32-row slab.
__device__ __forceinline__ uint32_t c_row(int r, int lane) { return 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3); }

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

// LDS weight row w (0..127) of a gate/up block: fragment w/32 holds gate
// features 16*(w/32) + (w%32) for w%32 < 16 and the matching up features for
// the rest, so a lane's C registers r and r+8 are gate and up of the same
// feature.
__global__ __launch_bounds__(256, 2) void grouped_gateup_kernel(GateUpParams p) {
  __shared__ __align__(16) uint16_t ws[128 * kLdsK];
  __shared__ __align__(16) uint16_t xs[kTileRows * kLdsK];
  __shared__ uint32_t row_src[kTileRows];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t wr = wave & 1u, wt = wave >> 1;
  const uint32_t nb_count = p.inter / kGateUpFeatures;
  const uint32_t total = *p.n_tiles * nb_count;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.tokens * p.hidden * 2u);
  for (uint32_t item = blockIdx.x; item < total; item += gridDim.x) {
    const uint32_t nb = item % nb_count;
    const GroupTile tile = p.tiles[item / nb_count];
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
    // Waves 0-1 stage the gate rows, waves 2-3 the up rows (one descriptor per wave).
    const bool is_up = wave >= 2u;
    const uint32_t f = (static_cast<uint32_t>(tid) & 127u) >> 1;  // feature within the block
    const uint32_t feature = nb * kGateUpFeatures + f;
    const uint32_t w_lds_row = 32u * (f >> 4) + (is_up ? 16u : 0u) + (f & 15u);
    const ExpertRsrc e = is_up ? expert_rsrc(eu, p.inter, p.hidden, p.group) : expert_rsrc(eg, p.inter, p.hidden, p.group);
    const uint32_t xsrc = row_src[static_cast<uint32_t>(tid) >> 1];
    GemmCore c;
    gemm_core(c, ws, xs, e, feature < p.inter, feature, w_lds_row, p.hidden, p.group, xr, xsrc != ~0u, xsrc,
              tile.count);
    // Epilogue: act = swiglu(bf16(g), bf16(u)) in sorted row order.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t trow = wt * 64u + j * 32u + (lane & 31);
      if (trow >= tile.count) continue;
      uint16_t *dst = p.act + static_cast<uint64_t>(tile.start + trow) * p.inter + nb * kGateUpFeatures;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t frag = wr * 2u + i;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const float g = round_bf16(c.acc[i][j][r]);
          const float u = round_bf16(c.acc[i][j][r + 8]);
          dst[16u * frag + c_row(r, lane)] = f32_to_bf16(swiglu_bf16(g, u));
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

__global__ __launch_bounds__(256, 2) void grouped_down_kernel(DownParams p) {
  __shared__ __align__(16) uint16_t ws[128 * kLdsK];
  __shared__ __align__(16) uint16_t xs[kTileRows * kLdsK];
  __shared__ uint32_t row_dst[kTileRows];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = wave_id();
  const uint32_t wr = wave & 1u, wt = wave >> 1;
  const uint32_t nb_count = p.hidden / kDownFeatures;
  const uint32_t total = *p.n_tiles * nb_count;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.act, p.rows * p.inter * 2u);
  for (uint32_t item = blockIdx.x; item < total; item += gridDim.x) {
    const uint32_t nb = item % nb_count;
    const GroupTile tile = p.tiles[item / nb_count];
    __syncthreads();  // the previous item's epilogue is done with row_dst
    if (tid < static_cast<int>(kTileRows))
      row_dst[tid] = static_cast<uint32_t>(tid) < tile.count ? p.order[tile.start + tid] : ~0u;
    const ExpertPtrs ed = tile.word == kSharedWord
                              ? expert_ptrs(p.sdown, 0u, p.hidden, p.inter, p.group, 1u)
                              : expert_ptrs(p.down, tile.word, p.hidden, p.inter, p.group, p.dense_count);
    __syncthreads();
    const uint32_t w = static_cast<uint32_t>(tid) >> 1;
    const uint32_t feature = nb * kDownFeatures + w;
    const ExpertRsrc e = expert_rsrc(ed, p.hidden, p.inter, p.group);
    const bool x_ok = w < tile.count;
    GemmCore c;
    gemm_core(c, ws, xs, e, feature < p.hidden, feature, w, p.inter, p.group, xr, x_ok, tile.start + w, tile.count);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t trow = wt * 64u + j * 32u + (lane & 31);
      if (trow >= tile.count) continue;
      const uint32_t r = row_dst[trow];
      uint16_t *dst = r < p.routed_rows ? p.y + static_cast<uint64_t>(r) * p.hidden
                                        : p.y_shared + static_cast<uint64_t>(r - p.routed_rows) * p.hidden;
      dst += nb * kDownFeatures + wr * 64u;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // four runs of 4 consecutive features
          const uint32_t f0 = 32u * i + c_row(4 * q, lane);
          const uint32_t lo = pack_bf16(c.acc[i][j][4 * q], c.acc[i][j][4 * q + 1]);
          const uint32_t hi = pack_bf16(c.acc[i][j][4 * q + 2], c.acc[i][j][4 * q + 3]);
          *reinterpret_cast<uint2 *>(dst + f0) = make_uint2(lo, hi);
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
  if (a.hidden % kBK || a.inter % kBK || a.hidden % kDownFeatures || a.inter % kGateUpFeatures)
    return fail(MQ_ERR_UNSUPPORTED, "grouped path needs hidden %% 128 == 0 and inter %% 64 == 0 (got %u, %u)",
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
  const uint32_t resident = static_cast<uint32_t>(cus > 0 ? cus : 256) * 2u;

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
  const uint32_t gu_items = l.max_tiles * (a.inter / kGateUpFeatures);
  hipLaunchKernelGGL(grouped_gateup_kernel, dim3(std::min(gu_items, resident)), dim3(256), 0, s, gp);
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
  const uint32_t dn_items = l.max_tiles * (a.hidden / kDownFeatures);
  hipLaunchKernelGGL(grouped_down_kernel, dim3(std::min(dn_items, resident)), dim3(256), 0, s, dp);
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
