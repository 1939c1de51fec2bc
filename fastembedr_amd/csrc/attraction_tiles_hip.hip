// Tiled attraction of the t-SNE gradient loop on gfx950 (CDNA4): P regrouped
// by (row block, column tile) into padded runs (layout at fehip::Tiles),
// built on the device from the CSR, and the kernel that sums the attractive
// forces over it.
//
// The sum is the reference's attraction, src/tsne_neighbors.cpp:985-1012
// (sum_j p_ij q_ij (y_i - y_j) per row, q_ij = 1 / (1 + |y_i - y_j|^2)), the
// same sum as the row-parallel k_attract, taken in another order.
//
// A workgroup owns one block of ROWS rows; for each of its column tiles it
// stages the COLS positions y_j of that tile in LDS, so the neighbour
// gathers read LDS instead of L2 (ROWS x COLS = 1024 x 4096 or 2048 x 2048,
// Tiles::rows and cols).  Each lane takes kTileRun
// consecutive entries of the run; entries of one row are adjacent, so a lane
// sums them in registers, and rows that run across lanes are merged by a
// segmented scan over the wave before one LDS add per row part.
//
// Build (launch_tile_build), all on the device and allocation-free:
//   k_tile_keys, radix sort    entries by (row block, column tile), stable,
//                              so each run's entries are in row order
//   k_tile_heads, scan, k_tile_meta
//                              runs: first run per row block, column tile,
//                              first entry, count
//   scan                       slots per entry (itself and its bridges) ->
//                              slot offsets
//   k_tile_sizes, scan         padded run sizes -> padded run begins
//   k_tile_scatter             entries and bridges to their padded places
//   k_tile_bases               each slot group's base row into its values

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>

#include "device_common.h"
#include "tsne_device.h"

namespace fehip {
namespace {

// Slot format (kTileRun = 8 slots per lane group, a group starting at a
// multiple of 8): the 16-bit word of a slot is (local column << 3) | step,
// so that word & 0x7ff8 is the column's LDS byte offset, and step (3 bits)
// is the slot's row minus the previous slot's row in the group (0 for a
// group's first slot).  p is stored as its IEEE-754 bits; P is a
// normalised joint distribution built from validated distances, so every
// value lies in [0, 1] and bits 30 and 31 of its pattern are zero.  Those
// bits of slots 0..5 of a group hold the group's base row (the local row of
// its first slot, 10 or 11 bits), 2 bits per slot.  Steps above 7 are made of
// bridge slots (p = 0) 7 rows apart (0.003 % more slots than 15-row bridges
// at config 2's late layout, 0.03 % at config 4's); a run's padding repeats its last slot
// with step 0 and p = 0.  Bridges and padding add nothing.
static_assert(kTileRun == 8, "a lane reads its group as one 16-byte vector of words and two of values");
constexpr int kBaseSlots = 6;  // slots whose spare value bits carry the base row
static_assert(kTileRows <= 1 << (2 * kBaseSlots) && kTileRowsWide <= 1 << (2 * kBaseSlots),
              "a group's base row fits the spare bits of its first kBaseSlots values");
static_assert(kTileCols <= 4096 && kTileColsWide <= 4096, "a local column fits 12 bits of a slot word");
constexpr int kStepMax = 7;
constexpr unsigned int kColMask = 0x7ff8u;  // a slot word's column byte offset
constexpr unsigned int kValueMask = 0x3fffffffu;

constexpr int kBuildThreads = 256;

__device__ __forceinline__ long long grid_first() {
  return static_cast<long long>(blockIdx.x) * kBuildThreads + threadIdx.x;
}
__device__ __forceinline__ long long grid_stride() { return static_cast<long long>(gridDim.x) * kBuildThreads; }

// Sort payload of one entry: p's bits, local row, local column.
__device__ __forceinline__ unsigned long long tile_payload(float p, unsigned int local_row, unsigned int local_col) {
  return (static_cast<unsigned long long>(__float_as_uint(p)) << 32) | (local_row << 16) | local_col;
}
__device__ __forceinline__ int payload_row(unsigned long long w) { return static_cast<int>((w >> 16) & 0xffffu); }
__device__ __forceinline__ int payload_col(unsigned long long w) { return static_cast<int>(w & 0xffffu); }

// Bridge slots needed before an entry whose row is `gap` rows past the
// previous entry of its run.
__device__ __forceinline__ int bridges_for(int gap) { return gap > 0 ? (gap - 1) / kStepMax : 0; }

template <int L>
__global__ __launch_bounds__(kBuildThreads) void k_tile_keys(const int* __restrict__ row_ptr,
                                                             const int* __restrict__ col,
                                                             const float* __restrict__ val, int n, int col_bits,
                                                             int rows_log2, int cols_log2,
                                                             unsigned int* __restrict__ key,
                                                             unsigned long long* __restrict__ pay) {
  constexpr int RPB = kBuildThreads / L;
  const int lane = threadIdx.x & (L - 1);
  for (int i = static_cast<int>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / L; i < n;
       i += static_cast<int>(gridDim.x) * RPB) {
    const unsigned int rb = static_cast<unsigned int>(i) >> rows_log2;
    const unsigned int lr = static_cast<unsigned int>(i) & ((1u << rows_log2) - 1u);
    const int e1 = row_ptr[i + 1];
    for (int e = row_ptr[i] + lane; e < e1; e += L) {
      const int j = col[e];
      key[e] = (rb << col_bits) | (static_cast<unsigned int>(j) >> cols_log2);
      pay[e] = tile_payload(val[e], lr, static_cast<unsigned int>(j) & ((1u << cols_log2) - 1u));
    }
  }
}

// Run heads (first entry of each (row block, column tile)) and the slots each
// entry takes: itself and its bridges.
__global__ __launch_bounds__(kBuildThreads) void k_tile_heads(const unsigned int* __restrict__ key,
                                                              const unsigned long long* __restrict__ pay,
                                                              long long nnz, int* __restrict__ heads,
                                                              int* __restrict__ slots) {
  for (long long p = grid_first(); p < nnz; p += grid_stride()) {
    const bool head = p == 0 || key[p] != key[p - 1];
    heads[p] = head ? 1 : 0;
    slots[p] = 1 + (head ? 0 : bridges_for(payload_row(pay[p]) - payload_row(pay[p - 1])));
  }
}

// Run records from the sorted keys: column tile, first entry, the first run
// of each row block, and the count (to *tile_count).
__global__ __launch_bounds__(kBuildThreads) void k_tile_meta(const unsigned int* __restrict__ key,
                                                             const int* __restrict__ heads,
                                                             const int* __restrict__ pos, long long nnz, int col_bits,
                                                             int row_blocks, int* __restrict__ tile_ptr,
                                                             int* __restrict__ tile_cb, int* __restrict__ ubeg,
                                                             int* __restrict__ tile_count) {
  for (long long p = grid_first(); p < nnz; p += grid_stride()) {
    const unsigned int k = key[p];
    const int cur = static_cast<int>(k >> col_bits);
    if (heads[p]) {
      const int t = pos[p];
      tile_cb[t] = static_cast<int>(k & ((1u << col_bits) - 1u));
      ubeg[t] = static_cast<int>(p);
      // this is the first run of every row block in (previous run's block, cur]
      const int prev = p == 0 ? -1 : static_cast<int>(key[p - 1] >> col_bits);
      for (int rb = prev + 1; rb <= cur; ++rb) tile_ptr[rb] = t;
    }
    if (p == nnz - 1) {
      const int total = pos[p] + heads[p];
      ubeg[total] = static_cast<int>(nnz);
      *tile_count = total;
      for (int rb = cur + 1; rb <= row_blocks; ++rb) tile_ptr[rb] = total;
    }
  }
}

// Slot offset of entry u (entries and bridges before it), u <= nnz.
__device__ __forceinline__ int slot_of(const int* __restrict__ sbeg, const int* __restrict__ slots, long long nnz,
                                       int u) {
  return u < nnz ? sbeg[u] : sbeg[nnz - 1] + slots[nnz - 1];
}

// Padded run sizes (multiples of kTileRun), zero past the last run.
__global__ __launch_bounds__(kBuildThreads) void k_tile_sizes(const int* __restrict__ ubeg,
                                                              const int* __restrict__ tile_count, long long tiles,
                                                              const int* __restrict__ sbeg,
                                                              const int* __restrict__ slots, long long nnz,
                                                              int* __restrict__ psize) {
  const int total = *tile_count;
  for (long long t = grid_first(); t < tiles; t += grid_stride()) {
    int v = 0;
    if (t < total) {
      const int len = slot_of(sbeg, slots, nnz, ubeg[t + 1]) - slot_of(sbeg, slots, nnz, ubeg[t]);
      v = (len + kTileRun - 1) / kTileRun * kTileRun;
    }
    psize[t] = v;
  }
}

// One slot: its word (step 0 at a group start) and p; the row of a group's
// first slot goes to base_row, merged into the values by k_tile_bases.
__device__ __forceinline__ void put_slot(long long q, int col, int row, int step, unsigned int p_bits,
                                         unsigned short* __restrict__ ent, float* __restrict__ val,
                                         unsigned short* __restrict__ base_row) {
  const bool first = (q & (kTileRun - 1)) == 0;
  ent[q] = static_cast<unsigned short>((col << 3) | (first ? 0 : step));
  val[q] = __uint_as_float(p_bits);
  if (first) base_row[q / kTileRun] = static_cast<unsigned short>(row);
}

// Entries and their bridges to their padded places; the last entry of each
// run also fills the run's padding.
__global__ __launch_bounds__(kBuildThreads) void k_tile_scatter(const unsigned long long* __restrict__ pay,
                                                                const int* __restrict__ heads,
                                                                const int* __restrict__ pos,
                                                                const int* __restrict__ ubeg,
                                                                const int* __restrict__ sbeg,
                                                                const int* __restrict__ tile_beg, long long nnz,
                                                                unsigned short* __restrict__ ent,
                                                                float* __restrict__ val,
                                                                unsigned short* __restrict__ base_row) {
  for (long long p = grid_first(); p < nnz; p += grid_stride()) {
    const int t = pos[p] + heads[p] - 1;
    const long long s0 = tile_beg[t] + (sbeg[p] - sbeg[ubeg[t]]);  // p's first slot (its first bridge)
    const unsigned long long w = pay[p];
    const int row = payload_row(w);
    const int col = payload_col(w);
    const int prev = heads[p] ? row : payload_row(pay[p - 1]);
    const int nb = bridges_for(row - prev);
    for (int m = 0; m < nb; ++m) {
      put_slot(s0 + m, col, prev + (m + 1) * kStepMax, kStepMax, 0u, ent, val, base_row);
    }
    const long long q = s0 + nb;
    put_slot(q, col, row, row - prev - nb * kStepMax, static_cast<unsigned int>(w >> 32), ent, val, base_row);
    if (p == nnz - 1 || heads[p + 1]) {
      for (long long r = q + 1; r < tile_beg[t + 1]; ++r) put_slot(r, col, row, 0, 0u, ent, val, base_row);
    }
  }
}

// Each group's base row into bits 30-31 of its first kBaseSlots values.
__global__ __launch_bounds__(kBuildThreads) void k_tile_bases(const unsigned short* __restrict__ base_row,
                                                              const int* __restrict__ tile_beg,
                                                              const int* __restrict__ tile_count,
                                                              float* __restrict__ val) {
  const long long groups = tile_beg[*tile_count] / kTileRun;
  for (long long g = grid_first(); g < groups; g += grid_stride()) {
    const unsigned int b = base_row[g];
#pragma unroll
    for (int q = 0; q < kBaseSlots; ++q) {
      float& v = val[g * kTileRun + q];
      v = __uint_as_float(__float_as_uint(v) | (((b >> (2 * q)) & 3u) << 30));
    }
  }
}

__global__ __launch_bounds__(kBuildThreads) void k_tile_empty(int* __restrict__ tile_ptr, int* __restrict__ tile_beg,
                                                              int* __restrict__ tile_count, int row_blocks) {
  for (int rb = threadIdx.x; rb <= row_blocks; rb += kBuildThreads) tile_ptr[rb] = 0;
  if (threadIdx.x == 0) {
    tile_beg[0] = 0;
    *tile_count = 0;
  }
}

// ---- the attraction ----------------------------------------------------------

template <typename T>
__device__ __forceinline__ T& lds_at(T* base, unsigned int byte_offset) {
  return *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + byte_offset);
}

// p_ij q_ij (y_i - y_j) without the exaggeration (applied once per row when
// the accumulators are written), q_ij = 1 / (1 + |y_i - y_j|^2) taken with
// the hardware reciprocal (v_rcp_f32, within 1 ulp; the argument is >= 1).
__device__ __forceinline__ float2 attract_term(float2 yi, float2 yj, float p) {
  const float dx = yi.x - yj.x;
  const float dy = yi.y - yj.y;
  const float c = p * __builtin_amdgcn_rcpf(fmaf(dx, dx, fmaf(dy, dy, 1.0f)));
  return make_float2(c * dx, c * dy);
}

// Whole-wave shifts by one lane (gfx9 DPP); a lane whose source lies outside
// the wave reads 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}
constexpr int kDppWaveShl1 = 0x130;  // lane l reads lane l + 1
constexpr int kDppWaveShr1 = 0x138;  // lane l reads lane l - 1

// Inclusive segmented scan of (x, y) over the wave (Hillis-Steele: row
// shifts 1, 2, 4, 8, then row broadcasts 15 and 31).  `take` is 0 on a lane
// that starts a segment and 1 elsewhere; at each step a lane adds the
// partial sums the step reaches, times its take, and its take becomes the
// minimum of the two (0 once its window holds a segment start).  Each step
// is one DPP multiply-add per value and one DPP minimum: bound_ctrl is off,
// so a lane whose source lies outside its row (or the rows a broadcast
// writes) is not written and keeps its partial and its take.  gfx9 needs two
// wait states between a VALU write of a VGPR and a DPP read of it: every
// DPP source here was written three instructions earlier, and the s_nop 1
// at each end covers the code around the block.  Needs the whole wave
// active.
__device__ __forceinline__ void seg_scan(float& x, float& y, float take) {
  asm volatile(
      "s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
      "v_min_f32_dpp %2, %2, %2 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
      "v_min_f32_dpp %2, %2, %2 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
      "v_min_f32_dpp %2, %2, %2 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_shr:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_shr:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_min_f32_dpp %2, %2, %2 row_shr:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "v_min_f32_dpp %2, %2, %2 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %0, %2 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %1, %2 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(x), "+v"(y), "+v"(take));
}

// A lane's kTileRun entries of one round of a run [e0, e1).  Lanes past the
// run's end take its last group instead (in bounds, rows in order) and are
// told to add nothing; as a lane's entries start at a fixed stride, the
// active lanes are a prefix of each wave.
struct TileGroup {
  uint4 w;  // 8 slot words, two per component (low half first)
  float4 p0, p1;
};

template <int NT>
__device__ __forceinline__ TileGroup load_tile_group(const unsigned short* __restrict__ ent,
                                                     const float* __restrict__ val, int e0, int e1, int round,
                                                     int tid) {
  const int e_lane = e0 + (round * NT + tid) * kTileRun;
  const int e = e_lane < e1 ? e_lane : e1 - kTileRun;
  TileGroup g;
  g.w = *reinterpret_cast<const uint4*>(ent + e);
  g.p0 = *reinterpret_cast<const float4*>(val + e);
  g.p1 = *reinterpret_cast<const float4*>(val + e + 4);
  return g;
}

// One step of a block's walk over its runs: round `round` of tile t, whose
// run is [e0, e1) (a positive multiple of kTileRun entries).  Block-uniform.
struct TileStep {
  int t, round, e0, e1;
};

template <int NT>
__device__ __forceinline__ TileStep next_tile_step(TileStep s, const int* __restrict__ tile_beg, int t1) {
  if (s.e0 + (s.round + 1) * NT * kTileRun < s.e1) {
    ++s.round;
    return s;
  }
  ++s.t;
  s.round = 0;
  s.e0 = s.e1;
  if (s.t < t1) s.e1 = tile_beg[s.t + 1];
  return s;
}

// The positions of column tile `cb` to LDS, between barriers (the first
// waits for the previous tile's readers).  Each lane issues all its loads
// before its first write; slots past the tile's last column repeat it.
template <int NT, int COLS>
struct TileColumns {
  static_assert(COLS % NT == 0, "whole column slots per lane");
  static constexpr int kPer = COLS / NT;
  float2 v[kPer];
  // the lane's positions of column tile cb (loads only)
  __device__ __forceinline__ void load(const float2* __restrict__ y_cur, int cb, int n, int tid) {
    const int base = cb * COLS;
    const int last = min(COLS, n - base) - 1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = y_cur[base + min(tid + i * NT, last)];
  }
  // to LDS, between barriers (the first waits for the previous tile's readers)
  __device__ __forceinline__ void store(float2* ys, int tid) const {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) ys[tid + i * NT] = v[i];
    __syncthreads();
  }
};

template <int NT, int COLS>
__device__ __forceinline__ void stage_tile_columns(float2* ys, const float2* __restrict__ y_cur, int cb, int n,
                                                   int tid) {
  TileColumns<NT, COLS> c;
  c.load(y_cur, cb, n, tid);
  c.store(ys, tid);
}

// Adds (x, y) to the accumulator at row byte offset k: by a plain read and
// write when no other wave can add to that row before the next barrier
// (`own`; a wave adds to a row at most once per group), else atomically.
__device__ __forceinline__ void acc_add(float2* acc, unsigned int k, float x, float y, bool own) {
  if (own) {
    float2 v = lds_at(acc, k);
    v.x += x;
    v.y += y;
    lds_at(acc, k) = v;
  } else {
    atomicAdd(&lds_at(acc, k).x, x);
    atomicAdd(&lds_at(acc, k).y, y);
  }
}

// Sum one lane group; a step that is not `live` adds nothing.  A lane's
// entries hold one or more rows (in order); it sums each row's part in
// registers.  Rows that begin and end inside the group go straight to the
// row's LDS accumulator.  The last row's part, which may run on into the
// next lanes, is summed over the wave by an inclusive segmented scan (DPP)
// and added by the lane that ends the chain; the first row's part, when a
// later row follows it in the group, ends the chain of lane l - 1 when it
// continues it, and the lane adds the two together.  So a wave issues one
// LDS add pair for the first rows and one for the chains, plus one per slot
// position where some lane completes a row wholly inside its group (an LDS
// float atomic costs far more than its few active lanes suggest: adding the
// first rows at each break instead took the kernel from 1.64 to 2.01 ms at
// config 4's ~7 entries per row and run, and from 0.230 to 0.245 ms beside
// the repulsion at config 2).
template <int NT, int ROWS>
__device__ __forceinline__ void sum_tile_group(const TileGroup& g, const TileStep& s, bool live, int tid, float2* yr,
                                               float2* ys, float2* acc) {
  const unsigned int wp[4] = {g.w.x, g.w.y, g.w.z, g.w.w};
  const unsigned int pb[kTileRun] = {__float_as_uint(g.p0.x), __float_as_uint(g.p0.y), __float_as_uint(g.p0.z),
                                     __float_as_uint(g.p0.w), __float_as_uint(g.p1.x), __float_as_uint(g.p1.y),
                                     __float_as_uint(g.p1.z), __float_as_uint(g.p1.w)};
  // Row byte offsets (8 bytes per LDS position): the base row from the spare
  // value bits (slot 0's step is 0), masked to the block, then the steps.
  // A group whose last row lies past the block (which a layout built here
  // never holds) adds nothing; its reads stay inside the workgroup's LDS
  // (rows < ROWS + 49).
  static_assert(ROWS <= 1 << (2 * kBaseSlots), "the base row fits its spare bits");
  unsigned int kr[kTileRun];
  unsigned int r8 = 0;
#pragma unroll
  for (int q = 0; q < kBaseSlots; ++q) r8 |= (pb[q] >> 30) << (2 * q + 3);
  r8 &= (ROWS - 1u) << 3;
  kr[0] = r8;
#pragma unroll
  for (int q = 1; q < kTileRun; ++q) {
    const unsigned int step = ((q & 1) ? wp[q / 2] >> 16 : wp[q / 2]) & 7u;
    r8 += step << 3;
    kr[q] = r8;
  }
  const bool active = live && s.e0 + (s.round * NT + tid) * kTileRun < s.e1 && r8 < ROWS * 8u;
  const unsigned int kf = kr[0];
  const unsigned int kl = kr[kTileRun - 1];
  float tx = 0.0f, ty = 0.0f;  // the current row's part
  float hx = 0.0f, hy = 0.0f;  // the first row's part, once a later row follows it
#pragma unroll
  for (int q = 0; q < kTileRun; ++q) {
    const unsigned int kc = ((q & 1) ? wp[q / 2] >> 16 : wp[q / 2]) & kColMask;
    // only the first kBaseSlots slots carry base-row bits
    const float p = __uint_as_float(q < kBaseSlots ? pb[q] & kValueMask : pb[q]);
    const float2 c = attract_term(lds_at(yr, kr[q]), lds_at(ys, kc), p);
    if (q == 0) {
      tx = c.x;
      ty = c.y;
      continue;
    }
    const bool brk = kr[q] != kr[q - 1];   // the previous row's part is complete
    const bool first = kr[q - 1] == kf;    // ... and it is the group's first row's
    if (brk && !first && active) acc_add(acc, kr[q - 1], tx, ty, true);  // a row wholly inside the group
    hx = brk && first ? tx : hx;
    hy = brk && first ? ty : hy;
    tx = (brk ? 0.0f : tx) + c.x;
    ty = (brk ? 0.0f : ty) + c.y;
  }
  // Chains over lanes: the first row continues lane l - 1's last when they
  // are the same row (active lanes are a prefix of the wave, so lane l - 1
  // is active too); a lane holding one row that continues lane l - 1's
  // extends the chain, any other lane starts one with its last row's part.
  const bool split = kf != kl;
  const int prev_kl = dpp_i<kDppWaveShr1, 0xf>(static_cast<int>(kl) + 1) - 1;  // -1 on lane 0
  const bool cont = active && static_cast<int>(kf) == prev_kl;
  seg_scan(tx, ty, cont && !split ? 1.0f : 0.0f);
  const float px = __int_as_float(dpp_i<kDppWaveShr1, 0xf>(__float_as_int(tx)));  // lane l - 1's chain
  const float py = __int_as_float(dpp_i<kDppWaveShr1, 0xf>(__float_as_int(ty)));
  const int next_cont = dpp_i<kDppWaveShl1, 0xf>(cont ? 1 : 0);  // 0 on lane 63
  // Only the wave's first and last rows can be shared with other waves
  // (rounds and row parts are contiguous slot ranges in row order).
  const unsigned int wave_first = __builtin_amdgcn_readfirstlane(kf);
  const unsigned int wave_last = __builtin_amdgcn_readlane(kl, 63);
  if (active && !next_cont) {  // the lane ends its last row's chain
    acc_add(acc, kl, tx, ty, kl != wave_first && kl != wave_last);
  }
  if (active && split) {  // the first row's part, with the chain it ends
    acc_add(acc, kf, cont ? hx + px : hx, cont ? hy + py : hy, kf != wave_first);
  }
}

// The row block rb's attraction (XCD-aware: block b runs on XCD b % xcds and
// each XCD takes one contiguous range of row blocks, whose column tiles then
// stay in its L2).  The block's steps (run, round) go through a ring of D
// register buffers: a buffer is refilled with the step D ahead as soon as it
// has been summed, so each wave keeps D - 1 groups of slots in flight while
// it sums one.  Every load is unconditional and the steps past the last
// repeat it and add nothing, so the compiler's wait counts leave the
// prefetch in flight; every wave runs the same steps (DPP needs whole
// waves).  Starts and ends with LDS free for the next row block (every
// thread passes a barrier between its last LDS access and the end).
// PREF: a step that opens a column tile other than the block's first finds
// the tile's positions already in registers, loaded before the step ahead of
// it was summed, so that the switch waits only for its two barriers (4
// positions per lane with 2048-column tiles: 8 VGPRs).
template <int NT, int D, int ROWS, int COLS, bool PREF>
__device__ __forceinline__ void attract_row_block(int rb, const unsigned short* __restrict__ ent,
                                                  const float* __restrict__ val, const int* __restrict__ tile_ptr,
                                                  const int* __restrict__ tile_cb, const int* __restrict__ tile_beg,
                                                  const float2* __restrict__ y_cur, float2* __restrict__ attr,
                                                  float exaggeration, int n, float2* ys, float2* yr, float2* acc) {
  const int tid = static_cast<int>(threadIdx.x);
  const int r0 = rb * ROWS;
  const int rows = min(ROWS, n - r0);
  for (int r = tid; r < ROWS; r += NT) {
    acc[r] = make_float2(0.0f, 0.0f);
    yr[r] = r < rows ? y_cur[r0 + r] : make_float2(0.0f, 0.0f);
  }
  const int t0 = tile_ptr[rb];
  const int t1 = tile_ptr[rb + 1];
  int steps = 0;
  for (int t = t0; t < t1; ++t) steps += (tile_beg[t + 1] - tile_beg[t] + NT * kTileRun - 1) / (NT * kTileRun);
  if (steps > 0) {
    TileStep st[D];
    TileGroup g[D];
    st[0] = TileStep{t0, 0, tile_beg[t0], tile_beg[t0 + 1]};
#pragma unroll
    for (int d = 1; d < D; ++d) st[d] = d < steps ? next_tile_step<NT>(st[d - 1], tile_beg, t1) : st[d - 1];
#pragma unroll
    for (int d = 0; d < D; ++d) g[d] = load_tile_group<NT>(ent, val, st[d].e0, st[d].e1, st[d].round, tid);
    TileColumns<NT, COLS> next;  // PREF: the positions of the tile that the next step opens
    for (int k = 0; k < steps; k += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const bool live = k + d < steps;
        if (live && st[d].round == 0) {
          if (PREF && k + d > 0) {
            next.store(ys, tid);
          } else {
            stage_tile_columns<NT, COLS>(ys, y_cur, tile_cb[st[d].t], n, tid);
          }
        }
        // the buffer after d holds step k + d + 1 (refilled earlier when d + 1 == D)
        if (PREF && k + d + 1 < steps && st[(d + 1) % D].round == 0) {
          next.load(y_cur, tile_cb[st[(d + 1) % D].t], n, tid);
        }
        sum_tile_group<NT, ROWS>(g[d], st[d], live, tid, yr, ys, acc);
        // refill with step k + d + D, whose predecessor is the newest buffer
        const TileStep newest = st[(d + D - 1) % D];
        st[d] = k + d + D < steps ? next_tile_step<NT>(newest, tile_beg, t1) : newest;
        g[d] = load_tile_group<NT>(ent, val, st[d].e0, st[d].e1, st[d].round, tid);
      }
    }
  }
  __syncthreads();
  for (int r = tid; r < rows; r += NT) attr[r0 + r] = make_float2(exaggeration * acc[r].x, exaggeration * acc[r].y);
  __syncthreads();
}

// Workgroups take the row blocks of their XCD's range: a primary launch's
// first the one at their slot (slots = workgroups per XCD), then, like every
// workgroup of a helper launch, the next unclaimed one from the XCD's counter
// work[xcd] (claims count from `slots`).  With one slot per row block this is
// one row block per workgroup; with fewer, the kernel leaves LDS and wave
// slots free for kernels that run beside it, and the dynamic claims balance
// the row blocks' unequal work.  A helper launch, enqueued later on another
// stream once the kernels beside the primary are done, takes over the row
// blocks still unclaimed.  The last workgroup of the pair (`total` workgroups
// between them) resets work[] (its xcds + 1 counters start and end each
// launch or pair at zero).  Launch bounds: MINB is HIP's minimum of waves
// per SIMD (3 leaves the D-deep prefetch ring up to 168 VGPRs; the 48 KB of
// LDS hold the kernel at 3 workgroups, 6 waves per SIMD, in any case).
// HELPER: a helper launch (its own symbol, so that profiles tell the two
// launches of a pair apart).  ROWS x COLS: the tile shape.
template <int NT, int D, int MINB, bool HELPER, int ROWS, int COLS>
__global__ __launch_bounds__(NT, MINB) void k_attract_tiles_seg(
    const unsigned short* __restrict__ ent, const float* __restrict__ val, const int* __restrict__ tile_ptr,
    const int* __restrict__ tile_cb, const int* __restrict__ tile_beg, const float2* __restrict__ y_cur,
    float2* __restrict__ attr, float exaggeration, int n, int row_blocks, int xcds, unsigned int* __restrict__ work,
    int slots, unsigned int total) {
  __shared__ float2 ys[COLS];
  __shared__ float2 yr[ROWS];
  __shared__ float2 acc[ROWS];
  // the claimed row block is passed through the first word of the column
  // tile, which is free between row blocks (no LDS beyond the three arrays:
  // 48 KB exactly, so that three workgroups leave a CU 16 KB for the
  // transforms that run beside them)
  int& claimed = *reinterpret_cast<int*>(ys);
  const int xcd = static_cast<int>(blockIdx.x) % xcds;
  const int per_xcd = (row_blocks + xcds - 1) / xcds;
  const int first = xcd * per_xcd;
  const int end = min(row_blocks, first + per_xcd);
  int slot = static_cast<int>(blockIdx.x) / xcds;
  if (HELPER) {
    if (threadIdx.x == 0) claimed = slots + static_cast<int>(atomicAdd(&work[xcd], 1u));
    __syncthreads();
    slot = claimed;
    __syncthreads();
  }
  while (first + slot < end) {
    attract_row_block<NT, D, ROWS, COLS, (COLS / NT <= 4)>(first + slot, ent, val, tile_ptr, tile_cb, tile_beg, y_cur, attr,
                                         exaggeration, n, ys, yr, acc);
    if (threadIdx.x == 0) claimed = slots + static_cast<int>(atomicAdd(&work[xcd], 1u));
    __syncthreads();
    slot = claimed;
    __syncthreads();  // every thread has read `claimed` before it is written again
  }
  if (threadIdx.x == 0 && atomicAdd(&work[xcds], 1u) == total - 1u) {
    // every other workgroup (of both launches) has made its last claim
    for (int x = 0; x <= xcds; ++x) atomicExch(&work[x], 0u);
  }
}

int bits_for(long long count) {  // bits needed to hold values 0 .. count - 1
  int b = 0;
  while (b < 62 && (1ll << b) < count) ++b;
  return b;
}

unsigned int build_blocks(long long items) {
  return static_cast<unsigned int>(
      std::max<long long>(1, std::min<long long>((items + kBuildThreads - 1) / kBuildThreads, 65536)));
}

}  // namespace

void tiles_shape(int n, long long nnz, Tiles& t, int wide) {
  t.n = n;
  t.nnz = nnz;
  const bool w = wide == 2 || (wide == 0 && n >= kTileWideFrom);
  t.rows = w ? kTileRowsWide : kTileRows;
  t.cols = w ? kTileColsWide : kTileCols;
  t.row_blocks = (n + t.rows - 1) / t.rows;
  t.col_tiles = (n + t.cols - 1) / t.cols;
  t.col_bits = bits_for(t.col_tiles);
  t.key_bits = t.col_bits + bits_for(t.row_blocks);
  t.max_tiles = std::min<long long>(nnz, static_cast<long long>(t.row_blocks) * t.col_tiles);
  // a run's rows rise by at most rows - 1, so it holds at most
  // (rows - 1) / kStepMax bridges, and at most kTileRun - 1 padding slots
  t.padded = nnz + ((t.rows - 1) / kStepMax + kTileRun - 1) * t.max_tiles;
}

hipError_t tiles_temp_bytes(const Tiles& t, std::size_t& bytes) {
  std::size_t sort_b = 0, scan_b = 0, scan_t = 0;
  const std::size_t count = static_cast<std::size_t>(std::max<long long>(t.nnz, 1));
  hipError_t e = rocprim::radix_sort_pairs(nullptr, sort_b, static_cast<const unsigned int*>(nullptr),
                                           static_cast<unsigned int*>(nullptr),
                                           static_cast<const unsigned long long*>(nullptr),
                                           static_cast<unsigned long long*>(nullptr), count, 0u,
                                           static_cast<unsigned int>(std::max(t.key_bits, 1)));
  if (e != hipSuccess) return e;
  e = rocprim::exclusive_scan(nullptr, scan_b, static_cast<const int*>(nullptr), static_cast<int*>(nullptr), 0,
                              count, rocprim::plus<int>());
  if (e != hipSuccess) return e;
  e = rocprim::exclusive_scan(nullptr, scan_t, static_cast<const int*>(nullptr), static_cast<int*>(nullptr), 0,
                              static_cast<std::size_t>(t.max_tiles) + 1, rocprim::plus<int>());
  bytes = std::max(sort_b, std::max(scan_b, scan_t));
  return e;
}

hipError_t launch_tile_build(const Csr& p, Tiles& t, hipStream_t stream) {
  if (t.key_bits > 32) return hipErrorInvalidValue;  // row blocks x column tiles beyond a 32-bit key
  if (t.nnz == 0) {
    k_tile_empty<<<1, kBuildThreads, 0, stream>>>(t.tile_ptr, t.tile_beg, t.tile_count, t.row_blocks);
    return hipGetLastError();
  }
  const std::size_t count = static_cast<std::size_t>(t.nnz);
  // after the sort the key and payload inputs are dead: the run heads, their
  // scan and each entry's slot count reuse them; after k_tile_meta the sorted
  // keys are dead and the scan of the slot counts takes their place
  int* heads = reinterpret_cast<int*>(t.key_in);
  int* pos = reinterpret_cast<int*>(t.pay_in);
  int* slot_count = reinterpret_cast<int*>(t.pay_in) + t.nnz;
  int* sbeg = reinterpret_cast<int*>(t.key_out);
  const unsigned int eb = build_blocks(t.nnz);
  if (t.rows != (t.rows & -t.rows) || t.cols != (t.cols & -t.cols)) return hipErrorInvalidValue;
  k_tile_keys<32><<<std::min((p.n + 7) / 8, 65536), kBuildThreads, 0, stream>>>(
      p.row_ptr, p.col, p.val, p.n, t.col_bits, bits_for(t.rows), bits_for(t.cols), t.key_in, t.pay_in);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  std::size_t tb = t.temp_bytes;
  // stable: entries of one (row block, column tile) keep their CSR (row) order
  e = rocprim::radix_sort_pairs(t.temp, tb, t.key_in, t.key_out, t.pay_in, t.pay_out, count, 0u,
                                static_cast<unsigned int>(std::max(t.key_bits, 1)), stream);
  if (e != hipSuccess) return e;
  k_tile_heads<<<eb, kBuildThreads, 0, stream>>>(t.key_out, t.pay_out, t.nnz, heads, slot_count);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  tb = t.temp_bytes;
  e = rocprim::exclusive_scan(t.temp, tb, heads, pos, 0, count, rocprim::plus<int>(), stream);
  if (e != hipSuccess) return e;
  k_tile_meta<<<eb, kBuildThreads, 0, stream>>>(t.key_out, heads, pos, t.nnz, t.col_bits, t.row_blocks, t.tile_ptr,
                                                t.tile_cb, t.ubeg, t.tile_count);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  tb = t.temp_bytes;
  e = rocprim::exclusive_scan(t.temp, tb, slot_count, sbeg, 0, count, rocprim::plus<int>(), stream);
  if (e != hipSuccess) return e;
  const long long slots = t.max_tiles + 1;
  k_tile_sizes<<<build_blocks(slots), kBuildThreads, 0, stream>>>(t.ubeg, t.tile_count, slots, sbeg, slot_count,
                                                                  t.nnz, t.psize);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  tb = t.temp_bytes;
  e = rocprim::exclusive_scan(t.temp, tb, t.psize, t.tile_beg, 0, static_cast<std::size_t>(slots),
                              rocprim::plus<int>(), stream);
  if (e != hipSuccess) return e;
  k_tile_scatter<<<eb, kBuildThreads, 0, stream>>>(t.pay_out, heads, pos, t.ubeg, sbeg, t.tile_beg, t.nnz, t.ent,
                                                   t.val, t.base_row);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_tile_bases<<<build_blocks(t.padded / kTileRun + 1), kBuildThreads, 0, stream>>>(t.base_row, t.tile_beg,
                                                                                    t.tile_count, t.val);
  return hipGetLastError();
}

namespace {

// Workgroups per XCD of a primary launch.
int primary_slots(const Tiles& t, int xcds, int slots_per_xcd) {
  const int per_xcd = (t.row_blocks + xcds - 1) / xcds;
  return std::max(1, slots_per_xcd > 0 ? std::min(slots_per_xcd, per_xcd) : per_xcd);
}

template <int ROWS, int COLS>
hipError_t attract_launch_shape(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration, int xcds,
                                int blocks, int slots, int helper, unsigned int total, hipStream_t stream,
                                hipEvent_t done) {
  constexpr int NT = kTileThreads;
  // a ring of 2 groups (one in flight while one is summed); deeper rings
  // measured no faster at config 2, and the LDS allows 3 workgroups per CU
  if (helper) {
    k_attract_tiles_seg<NT, 2, 3, true, ROWS, COLS><<<blocks, NT, 0, stream>>>(
        t.ent, t.val, t.tile_ptr, t.tile_cb, t.tile_beg, y_cur, attr, exaggeration, t.n, t.row_blocks, xcds, t.work,
        slots, total);
  } else if (done != nullptr) {
    hipExtLaunchKernelGGL(k_attract_tiles_seg<NT, 2, 3, false, ROWS, COLS>, dim3(blocks), dim3(NT), 0, stream,
                          nullptr, done, 0, t.ent, t.val, t.tile_ptr, t.tile_cb, t.tile_beg, y_cur, attr,
                          exaggeration, t.n, t.row_blocks, xcds, t.work, slots, total);
  } else {
    k_attract_tiles_seg<NT, 2, 3, false, ROWS, COLS><<<blocks, NT, 0, stream>>>(
        t.ent, t.val, t.tile_ptr, t.tile_cb, t.tile_beg, y_cur, attr, exaggeration, t.n, t.row_blocks, xcds, t.work,
        slots, total);
  }
  return hipGetLastError();
}

hipError_t attract_launch(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration, int xcds, int blocks,
                          int slots, int helper, unsigned int total, hipStream_t stream, hipEvent_t done) {
  if (t.rows == kTileRows && t.cols == kTileCols) {
    return attract_launch_shape<kTileRows, kTileCols>(t, y_cur, attr, exaggeration, xcds, blocks, slots, helper,
                                                      total, stream, done);
  }
  if (t.rows == kTileRowsWide && t.cols == kTileColsWide) {
    return attract_launch_shape<kTileRowsWide, kTileColsWide>(t, y_cur, attr, exaggeration, xcds, blocks, slots,
                                                              helper, total, stream, done);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attract_tiled(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration, int xcds,
                                int slots_per_xcd, int helper_per_xcd, hipStream_t stream, hipEvent_t done) {
  if (t.work == nullptr || xcds < 1 || xcds > kTileMaxXcds || helper_per_xcd < 0) return hipErrorInvalidValue;
  const int slots = primary_slots(t, xcds, slots_per_xcd);
  const unsigned int total = static_cast<unsigned int>((slots + helper_per_xcd) * xcds);
  return attract_launch(t, y_cur, attr, exaggeration, xcds, slots * xcds, slots, 0, total, stream, done);
}

hipError_t launch_attract_tiled_helper(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration,
                                       int xcds, int slots_per_xcd, int helper_per_xcd, hipStream_t stream) {
  if (t.work == nullptr || xcds < 1 || xcds > kTileMaxXcds || helper_per_xcd < 1) return hipErrorInvalidValue;
  const int slots = primary_slots(t, xcds, slots_per_xcd);
  const unsigned int total = static_cast<unsigned int>((slots + helper_per_xcd) * xcds);
  return attract_launch(t, y_cur, attr, exaggeration, xcds, helper_per_xcd * xcds, slots, 1, total, stream, nullptr);
}

}  // namespace fehip
