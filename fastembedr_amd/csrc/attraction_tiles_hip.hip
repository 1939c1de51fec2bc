// Tiled attraction of the t-SNE gradient loop on gfx950 (CDNA4): P regrouped
// by (row block, column tile) into padded runs (layout at fehip::Tiles),
// built on the device from the CSR, and the kernel that sums the attractive
// forces over it.
//
// The sum is the reference's attraction, src/tsne_neighbors.cpp:985-1012
// (sum_j p_ij q_ij (y_i - y_j) per row, q_ij = 1 / (1 + |y_i - y_j|^2)), the
// same sum as the row-parallel k_attract, taken in another order.
//
// A workgroup owns one block of kTileRows rows; for each of its column tiles
// it stages the kTileCols positions y_j of that tile in LDS, so the
// neighbour gathers read LDS instead of L2.  Each lane takes kTileRun
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
//   k_tile_sizes, scan         padded run sizes -> padded run begins
//   k_tile_scatter             entries to their padded places

#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>

#include "device_common.h"
#include "tsne_device.h"

namespace fehip {
namespace {

// An entry word holds two byte offsets into the LDS position arrays (8 bytes
// per position): the row's in its high half, the column's in its low half,
// so the kernel addresses LDS with no shifts.  A run's padding repeats the
// run's last entry word with p = 0 and so adds nothing.
static_assert(kTileRun == 8, "a lane reads its run group as two 16-byte vectors per array");
static_assert(kTileRows * 8 <= 0x10000 && kTileCols * 8 <= 0x10000, "entry offsets are 16-bit byte offsets");

constexpr int kBuildThreads = 256;

__device__ __forceinline__ long long grid_first() {
  return static_cast<long long>(blockIdx.x) * kBuildThreads + threadIdx.x;
}
__device__ __forceinline__ long long grid_stride() { return static_cast<long long>(gridDim.x) * kBuildThreads; }

__device__ __forceinline__ unsigned int tile_word(unsigned int local_row, unsigned int local_col) {
  return ((local_row * 8u) << 16) | (local_col * 8u);
}

template <int L>
__global__ __launch_bounds__(kBuildThreads) void k_tile_keys(const int* __restrict__ row_ptr,
                                                             const int* __restrict__ col,
                                                             const float* __restrict__ val, int n, int col_bits,
                                                             unsigned int* __restrict__ key,
                                                             unsigned long long* __restrict__ pay) {
  constexpr int RPB = kBuildThreads / L;
  const int lane = threadIdx.x & (L - 1);
  for (int i = static_cast<int>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / L; i < n;
       i += static_cast<int>(gridDim.x) * RPB) {
    const unsigned int rb = static_cast<unsigned int>(i / kTileRows);
    const unsigned int lr = static_cast<unsigned int>(i % kTileRows);
    const int e1 = row_ptr[i + 1];
    for (int e = row_ptr[i] + lane; e < e1; e += L) {
      const int j = col[e];
      key[e] = (rb << col_bits) | static_cast<unsigned int>(j / kTileCols);
      pay[e] = (static_cast<unsigned long long>(__float_as_uint(val[e])) << 32) |
               static_cast<unsigned long long>(tile_word(lr, static_cast<unsigned int>(j % kTileCols)));
    }
  }
}

__global__ __launch_bounds__(kBuildThreads) void k_tile_heads(const unsigned int* __restrict__ key, long long nnz,
                                                              int* __restrict__ heads) {
  for (long long p = grid_first(); p < nnz; p += grid_stride()) heads[p] = (p == 0 || key[p] != key[p - 1]) ? 1 : 0;
}

// Run records from the sorted keys: column tile, first entry (before
// padding), the first run of each row block, and the count (to *tile_count).
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

// Padded run sizes (multiples of kTileRun), zero past the last run.
__global__ __launch_bounds__(kBuildThreads) void k_tile_sizes(const int* __restrict__ ubeg,
                                                              const int* __restrict__ tile_count, long long slots,
                                                              int* __restrict__ psize) {
  const int total = *tile_count;
  for (long long t = grid_first(); t < slots; t += grid_stride()) {
    int v = 0;
    if (t < total) {
      const int len = ubeg[t + 1] - ubeg[t];
      v = (len + kTileRun - 1) / kTileRun * kTileRun;
    }
    psize[t] = v;
  }
}

// Entries to their padded places; the last entry of each run fills the
// run's padding with copies of its own word and p = 0.
__global__ __launch_bounds__(kBuildThreads) void k_tile_scatter(const unsigned long long* __restrict__ pay,
                                                                const int* __restrict__ heads,
                                                                const int* __restrict__ pos,
                                                                const int* __restrict__ ubeg,
                                                                const int* __restrict__ tile_beg, long long nnz,
                                                                unsigned int* __restrict__ ent,
                                                                float* __restrict__ val) {
  for (long long p = grid_first(); p < nnz; p += grid_stride()) {
    const int t = pos[p] + heads[p] - 1;
    const int u0 = ubeg[t];
    const int b0 = tile_beg[t];
    const unsigned long long w = pay[p];
    const long long q = b0 + (p - u0);
    ent[q] = static_cast<unsigned int>(w);
    val[q] = __uint_as_float(static_cast<unsigned int>(w >> 32));
    const int u1 = ubeg[t + 1];
    if (p == u1 - 1) {
      for (int r = b0 + (u1 - u0); r < tile_beg[t + 1]; ++r) {
        ent[r] = static_cast<unsigned int>(w);
        val[r] = 0.0f;
      }
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

// Wave-level helpers (gfx9 DPP: row shifts within 16-lane rows, row
// broadcasts 15 / 31, whole-wave shifts by one lane).  Lanes whose source
// lies outside the row / wave read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}
constexpr int kDppRowShr = 0x110;    // + shift (1..15)
constexpr int kDppWaveShl1 = 0x130;  // lane l reads lane l + 1
constexpr int kDppWaveShr1 = 0x138;  // lane l reads lane l - 1
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

// One step of an inclusive segmented scan: (x, y) combined with the value
// CTRL's shift below.  `stop` holds the bits of 1.0f once the lane's window
// reaches back to a segment start (a lane whose value takes nothing from
// below), else 0; a source outside the row / wave reads (0, 0, 0), the
// identity of the step.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void seg_step(float& x, float& y, unsigned int& stop) {
  const float take = 1.0f - __uint_as_float(stop);
  x = fmaf(dpp_f<CTRL, ROW_MASK>(x), take, x);
  y = fmaf(dpp_f<CTRL, ROW_MASK>(y), take, y);
  stop = max(stop, static_cast<unsigned int>(dpp_i<CTRL, ROW_MASK>(static_cast<int>(stop))));
}

// A lane's kTileRun entries of one round of a run [e0, e1).  Lanes past the
// run's end take its last group instead (in bounds, rows in order) and are
// told to add nothing; as a lane's entries start at a fixed stride, the
// active lanes are a prefix of each wave.
struct TileGroup {
  uint4 w0, w1;
  float4 p0, p1;
};

template <int NT>
__device__ __forceinline__ TileGroup load_tile_group(const unsigned int* __restrict__ ent,
                                                     const float* __restrict__ val, int e0, int e1, int round,
                                                     int tid) {
  const int e_lane = e0 + (round * NT + tid) * kTileRun;
  const int e = e_lane < e1 ? e_lane : e1 - kTileRun;
  TileGroup g;
  g.w0 = *reinterpret_cast<const uint4*>(ent + e);
  g.w1 = *reinterpret_cast<const uint4*>(ent + e + 4);
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
template <int NT>
__device__ __forceinline__ void stage_tile_columns(float2* ys, const float2* __restrict__ y_cur, int cb, int n,
                                                   int tid) {
  constexpr int kPer = kTileCols / NT;
  static_assert(kTileCols % NT == 0, "whole column slots per lane");
  const int base = cb * kTileCols;
  const int last = min(kTileCols, n - base) - 1;
  float2 v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) v[i] = y_cur[base + min(tid + i * NT, last)];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer; ++i) ys[tid + i * NT] = v[i];
  __syncthreads();
}

// Sum one lane group; a step that is not `live` adds nothing.  A lane's
// entries hold one or more rows (in order); it sums each row's part in
// registers and adds every part but the last (which its group completes)
// straight to the row's LDS accumulator.  The last part, which may run on
// into the next lanes, is summed over the wave by an inclusive segmented
// scan (DPP), and only the lane that ends the row adds it.
template <int NT>
__device__ __forceinline__ void sum_tile_group(const TileGroup& g, const TileStep& s, bool live, int tid, float2* yr,
                                               float2* ys, float2* acc) {
  const bool active = live && s.e0 + (s.round * NT + tid) * kTileRun < s.e1;
  const unsigned int w[kTileRun] = {g.w0.x, g.w0.y, g.w0.z, g.w0.w, g.w1.x, g.w1.y, g.w1.z, g.w1.w};
  const float p[kTileRun] = {g.p0.x, g.p0.y, g.p0.z, g.p0.w, g.p1.x, g.p1.y, g.p1.z, g.p1.w};
  float tx = 0.0f, ty = 0.0f;  // the current row's part
#pragma unroll
  for (int q = 0; q < kTileRun; ++q) {
    const unsigned int kr = w[q] >> 16;
    const float2 c = attract_term(lds_at(yr, kr), lds_at(ys, w[q] & 0xffffu), p[q]);
    const bool brk = q > 0 && kr != (w[q > 0 ? q - 1 : 0] >> 16);  // the previous row's part is complete
    if (brk && active) {
      atomicAdd(&lds_at(acc, w[q > 0 ? q - 1 : 0] >> 16).x, tx);
      atomicAdd(&lds_at(acc, w[q > 0 ? q - 1 : 0] >> 16).y, ty);
    }
    tx = (brk ? 0.0f : tx) + c.x;
    ty = (brk ? 0.0f : ty) + c.y;
  }
  // The last row's part continues lane l - 1's when the whole group is that
  // one row; the scan sums each such chain into its last lane.
  const int kf = static_cast<int>(w[0] >> 16);
  const int kl = static_cast<int>(w[kTileRun - 1] >> 16);
  const int prev_kl = dpp_i<kDppWaveShr1, 0xf>(kl + 1) - 1;  // -1 on lane 0
  const bool start = !active || kf != kl || kf != prev_kl;
  unsigned int stop = start ? __float_as_uint(1.0f) : 0u;
  seg_step<kDppRowShr + 1, 0xf>(tx, ty, stop);
  seg_step<kDppRowShr + 2, 0xf>(tx, ty, stop);
  seg_step<kDppRowShr + 4, 0xf>(tx, ty, stop);
  seg_step<kDppRowShr + 8, 0xf>(tx, ty, stop);
  seg_step<kDppRowBcast15, 0xa>(tx, ty, stop);
  seg_step<kDppRowBcast31, 0xc>(tx, ty, stop);
  const int next_joins = dpp_i<kDppWaveShl1, 0xf>(start ? 0 : 1);  // 0 on lane 63
  if (active && !next_joins) {
    atomicAdd(&lds_at(acc, static_cast<unsigned int>(kl)).x, tx);
    atomicAdd(&lds_at(acc, static_cast<unsigned int>(kl)).y, ty);
  }
}

// The row block rb's attraction (XCD-aware: block b runs on XCD b % xcds and
// each XCD takes one contiguous range of row blocks, whose column tiles then
// stay in its L2).  The block's steps (run, round) are processed two at a
// time from two register buffers: the next step's loads are issued before
// the current one is summed, so each wave keeps two groups of entries in
// flight.  Every load is unconditional and an odd last step is paired with
// a step that adds nothing (it repeats the last one), so the compiler's wait
// counts leave the prefetch in flight; every wave runs the same steps (DPP
// needs whole waves).  Starts and ends with LDS free for the next row block
// (every thread passes a barrier between its last LDS access and the end).
template <int NT>
__device__ __forceinline__ void attract_row_block(int rb, const unsigned int* __restrict__ ent,
                                                  const float* __restrict__ val, const int* __restrict__ tile_ptr,
                                                  const int* __restrict__ tile_cb, const int* __restrict__ tile_beg,
                                                  const float2* __restrict__ y_cur, float2* __restrict__ attr,
                                                  float exaggeration, int n, float2* ys, float2* yr, float2* acc) {
  const int tid = static_cast<int>(threadIdx.x);
  const int r0 = rb * kTileRows;
  const int rows = min(kTileRows, n - r0);
  for (int r = tid; r < kTileRows; r += NT) {
    acc[r] = make_float2(0.0f, 0.0f);
    yr[r] = r < rows ? y_cur[r0 + r] : make_float2(0.0f, 0.0f);
  }
  const int t0 = tile_ptr[rb];
  const int t1 = tile_ptr[rb + 1];
  int steps = 0;
  for (int t = t0; t < t1; ++t) steps += (tile_beg[t + 1] - tile_beg[t] + NT * kTileRun - 1) / (NT * kTileRun);
  if (steps > 0) {
    TileStep sa{t0, 0, tile_beg[t0], tile_beg[t0 + 1]};
    TileGroup ga = load_tile_group<NT>(ent, val, sa.e0, sa.e1, sa.round, tid);
    for (int k = 0; k < steps; k += 2) {
      const bool b_live = k + 1 < steps;
      const TileStep sb = b_live ? next_tile_step<NT>(sa, tile_beg, t1) : sa;
      const TileGroup gb = load_tile_group<NT>(ent, val, sb.e0, sb.e1, sb.round, tid);
      if (sa.round == 0) stage_tile_columns<NT>(ys, y_cur, tile_cb[sa.t], n, tid);
      sum_tile_group<NT>(ga, sa, true, tid, yr, ys, acc);
      const TileStep sc = k + 2 < steps ? next_tile_step<NT>(sb, tile_beg, t1) : sb;
      ga = load_tile_group<NT>(ent, val, sc.e0, sc.e1, sc.round, tid);
      if (b_live && sb.round == 0) stage_tile_columns<NT>(ys, y_cur, tile_cb[sb.t], n, tid);
      sum_tile_group<NT>(gb, sb, b_live, tid, yr, ys, acc);
      sa = sc;
    }
  }
  __syncthreads();
  for (int r = tid; r < rows; r += NT) attr[r0 + r] = make_float2(exaggeration * acc[r].x, exaggeration * acc[r].y);
  __syncthreads();
}

// Workgroups take the row blocks of their XCD's range: first the one at their
// slot, then the next unclaimed one from the XCD's counter work[xcd] (claims
// count from the number of slots).  With one slot per row block this is one
// row block per workgroup; with fewer, the kernel leaves LDS and wave slots
// free for kernels that run beside it, and the dynamic claims balance the
// row blocks' unequal work.  The last workgroup to finish resets work[] (its
// xcds + 1 counters start and end each launch at zero).  Launch bounds:
// 2048 / NT blocks per CU, 8 waves per SIMD, as many as the LDS allows.
template <int NT>
__global__ __launch_bounds__(NT, 2048 / NT) void k_attract_tiles_seg(
    const unsigned int* __restrict__ ent, const float* __restrict__ val, const int* __restrict__ tile_ptr,
    const int* __restrict__ tile_cb, const int* __restrict__ tile_beg, const float2* __restrict__ y_cur,
    float2* __restrict__ attr, float exaggeration, int n, int row_blocks, int xcds, unsigned int* __restrict__ work) {
  __shared__ float2 ys[kTileCols];
  __shared__ float2 yr[kTileRows];
  __shared__ float2 acc[kTileRows];
  __shared__ int claimed;
  const int xcd = static_cast<int>(blockIdx.x) % xcds;
  const int slots = static_cast<int>(gridDim.x) / xcds;  // the grid is a whole number of slots per XCD
  const int per_xcd = (row_blocks + xcds - 1) / xcds;
  const int first = xcd * per_xcd;
  const int end = min(row_blocks, first + per_xcd);
  int slot = static_cast<int>(blockIdx.x) / xcds;
  while (first + slot < end) {
    attract_row_block<NT>(first + slot, ent, val, tile_ptr, tile_cb, tile_beg, y_cur, attr, exaggeration, n, ys, yr,
                          acc);
    if (threadIdx.x == 0) claimed = slots + static_cast<int>(atomicAdd(&work[xcd], 1u));
    __syncthreads();
    slot = claimed;
    __syncthreads();  // every thread has read `claimed` before it is written again
  }
  if (threadIdx.x == 0 && atomicAdd(&work[xcds], 1u) == gridDim.x - 1) {
    // every other workgroup has made its last claim
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

void tiles_shape(int n, long long nnz, Tiles& t) {
  t.n = n;
  t.nnz = nnz;
  t.row_blocks = (n + kTileRows - 1) / kTileRows;
  t.col_tiles = (n + kTileCols - 1) / kTileCols;
  t.col_bits = bits_for(t.col_tiles);
  t.key_bits = t.col_bits + bits_for(t.row_blocks);
  t.max_tiles = std::min<long long>(nnz, static_cast<long long>(t.row_blocks) * t.col_tiles);
  t.padded = nnz + (kTileRun - 1) * t.max_tiles;
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
  // after the sort the key and payload inputs are dead: the run heads and
  // their scan reuse them
  int* heads = reinterpret_cast<int*>(t.key_in);
  int* pos = reinterpret_cast<int*>(t.pay_in);
  const unsigned int eb = build_blocks(t.nnz);
  k_tile_keys<32><<<std::min((p.n + 7) / 8, 65536), kBuildThreads, 0, stream>>>(p.row_ptr, p.col, p.val, p.n,
                                                                               t.col_bits, t.key_in, t.pay_in);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  std::size_t tb = t.temp_bytes;
  // stable: entries of one (row block, column tile) keep their CSR (row) order
  e = rocprim::radix_sort_pairs(t.temp, tb, t.key_in, t.key_out, t.pay_in, t.pay_out, count, 0u,
                                static_cast<unsigned int>(std::max(t.key_bits, 1)), stream);
  if (e != hipSuccess) return e;
  k_tile_heads<<<eb, kBuildThreads, 0, stream>>>(t.key_out, t.nnz, heads);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  tb = t.temp_bytes;
  e = rocprim::exclusive_scan(t.temp, tb, heads, pos, 0, count, rocprim::plus<int>(), stream);
  if (e != hipSuccess) return e;
  k_tile_meta<<<eb, kBuildThreads, 0, stream>>>(t.key_out, heads, pos, t.nnz, t.col_bits, t.row_blocks, t.tile_ptr,
                                                t.tile_cb, t.ubeg, t.tile_count);
  const long long slots = t.max_tiles + 1;
  k_tile_sizes<<<build_blocks(slots), kBuildThreads, 0, stream>>>(t.ubeg, t.tile_count, slots, t.psize);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  tb = t.temp_bytes;
  e = rocprim::exclusive_scan(t.temp, tb, t.psize, t.tile_beg, 0, static_cast<std::size_t>(slots),
                              rocprim::plus<int>(), stream);
  if (e != hipSuccess) return e;
  k_tile_scatter<<<eb, kBuildThreads, 0, stream>>>(t.pay_out, heads, pos, t.ubeg, t.tile_beg, t.nnz, t.ent, t.val);
  return hipGetLastError();
}

hipError_t launch_attract_tiled(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration, int threads,
                                int xcds, int slots_per_xcd, hipStream_t stream) {
  if (t.work == nullptr || xcds < 1 || xcds > kTileMaxXcds) return hipErrorInvalidValue;
  const int per_xcd = (t.row_blocks + xcds - 1) / xcds;
  const int slots = slots_per_xcd > 0 ? std::min(slots_per_xcd, per_xcd) : per_xcd;
  const int blocks = std::max(slots, 1) * xcds;
#define FEHIP_TILED(NT_)                                                                                        \
  k_attract_tiles_seg<NT_><<<blocks, NT_, 0, stream>>>(t.ent, t.val, t.tile_ptr, t.tile_cb, t.tile_beg, y_cur, \
                                                       attr, exaggeration, t.n, t.row_blocks, xcds, t.work);
  switch (threads) {
    case 256:
      FEHIP_TILED(256)
      break;
    case 512:
      FEHIP_TILED(512)
      break;
    case 1024:
      FEHIP_TILED(1024)
      break;
    default:
      return hipErrorInvalidValue;
  }
#undef FEHIP_TILED
  return hipGetLastError();
}

}  // namespace fehip
