// FIt-SNE interpolation grid on gfx950 (CDNA4).
//
// An extension of the reference path.  The reference's native backends
// approximate the repulsion on a bilinear node lattice
// (src/tsne_neighbors.cpp:1089-1182 of tkcaccia/fastEmbedR and its CUDA and
// Metal ports); the benchmark configurations of this build ask for the
// interpolation grid of FIt-SNE (Linderman et al., Nat. Methods 16, 243
// (2019)) with 3 interpolation points per interval and at least 50
// intervals.  The layout's bounding square is cut into boxes about one unit
// wide; each box holds 3 x 3 nodes of its own (spacing h, uniform across
// boxes); every point is spread onto its box's nodes with Lagrange weights
// L_a, the node charges are convolved with kernels between nodes, and the
// potentials are interpolated back with the same weights (in k_update).
//
// FIt-SNE writes the repulsion of point i as (y_i phi0 - phi1) / Z with
// phi_t = K (x) c_t, K = 1 / (1 + d^2)^2, charges c_0 = sum_j L_b(y_j) and
// c_1 = sum_j L_b(y_j) y_j, and Z from a fourth charge |y_j|^2.  In fp32 the
// difference y_i phi0 - phi1 cancels: |y| reaches hundreds while the result
// is set by neighbours about a unit away.  This file evaluates the same
// approximation (the same nodes, weights and kernel, equal in exact
// arithmetic) in a form without cancellation.  With node positions y_a,
// per-node moments relative to the node,
//   m0_b = sum_j L_b(y_j),  m1_b = sum_j L_b(y_j) (y_j - y_b),
//   m2_b = sum_j L_b(y_j) |y_j - y_b|^2,
// and splitting y_i - y_j = (y_i - y_a) + (y_a - y_b) - (y_j - y_b):
//   y_i phi0 - phi1 = sum_a L_a(y_i) [(y_i - y_a) phi0(a) + xi(a)],
//   xi  = Kv (x) m0 - K (x) m1,  Kv(a - b) = K(a - b) (y_a - y_b),
//   Z + n = sum_a m0 (K1 (x) m0) + 2 sum_a m2 phi0 + 4 sum_a m1 . (Kv (x) m0)
//           - 2 sum_a m1 . (K (x) m1),   K1 = 1 / (1 + d^2),
// using K (1 + |y_a - y_b|^2) = K1 and the symmetry of the double sum.  Every
// term is local (|y_i - y_a| and |y_j - y_b| are within a box) or a
// well-conditioned convolution.  The three sums that involve convolutions of
// transformed charges are taken in the spectral domain (Parseval), the
// fourth with the potentials.  Distances are in units of h inside the
// kernels and charges; the factors of h are applied at the end.
//
// Per iteration, after the statistics have set the geometry on the device:
//   k_lg_bin_count, k_bin_plan, k_lg_bin_scatter
//                         points into tiles of T x T boxes and work items of
//                         at most 2048 points of one tile
//   k_lg_spread           per work item: points ordered by box in LDS; one
//                         wave per box sums its points' 9 nodes x 4 moments
//                         in registers and DPP adds across the wave, and
//                         stores the box's nodes in the item's LDS window;
//                         the window goes straight to the charge planes when
//                         the item is its tile's only one, else to scratch
//   k_lg_gather           sums the scratch windows of multi-item tiles in a
//                         fixed order (no float atomics in global memory), a
//                         workgroup per tile; every node is written, so
//                         nothing is cleared
//   k_lg_kernel_rows/cols spectra of K, K1 (real, even) and Kv (imaginary,
//                         odd in its own axis), a quadrant each, two real
//                         sequences per complex transform
//   k_lg_charge_rows      m0 + i m1x and m1y per complex row transform, half
//                         spectra kept
//   k_lg_conv_cols        forward column transforms, spectral products for
//                         phi0, xi_x, xi_y and the spectral sums of Z, inverse
//                         column transforms, in one pass
//   k_lg_inverse_rows     inverse row transforms, potentials per node and the
//                         m2 phi0 sum
//   k_lg_finalize_z       Z and its reciprocal
// Row transforms read and write contiguous rows; the column passes read
// their columns straight from the row-major row spectra and write the
// potential spectra back row-major (no transposes), with their blocks mapped
// to columns XCD by XCD (col_block) so that the blocks sharing a cache line
// of adjacent columns share one XCD's L2.  Twiddles are staged in LDS.
//
// The FFT length f is 2^a or 3 * 2^a with f >= 2 m (m nodes per axis, read
// on the device); the host picks it from a bound on m.  Rows and columns of
// the padded grid that are known to be zero are skipped.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>

#include "device_common.h"
#include "tsne_device.h"

namespace fehip {
namespace {

constexpr int kLgThreads = 256;
// partial-sum slots: three per convolution-pass block, then one per row block
constexpr int kLgMaxSpecBlocks = kLgMaxColBlocks;
constexpr int kLgRun = kChunk / kLgThreads;  // points per lane in k_lg_spread
constexpr int kLgBoxesPerTile = kLgMaxTile * kLgMaxTile;
static_assert(kLgBoxesPerTile == kLgThreads, "one box of the largest tile per thread in the box scan");
static_assert(kLgRun * kLgThreads == kChunk, "a work item is one run per lane");

__device__ __forceinline__ int lg_tile_of(const LgPoint& b, int tile, int ta) {
  return (b.by / tile) * ta + b.bx / tile;
}

__global__ __launch_bounds__(kLgThreads) void k_lg_bin_count(const float2* __restrict__ y_stored,
                                                             float2* __restrict__ y_cur, const DeviceScalars* sc,
                                                             int* __restrict__ tile_count, int n) {
#pragma clang fp contract(off)
  chain_priority();
  __shared__ int hist[kMaxTiles];
  const DeviceScalars s = *sc;
  const int ta = s.lg_tiles_axis;
  const int tiles = ta * ta;
  for (int t = threadIdx.x; t < tiles; t += kLgThreads) hist[t] = 0;
  __syncthreads();
  for (int i = blockIdx.x * kLgThreads + threadIdx.x; i < n; i += gridDim.x * kLgThreads) {
    const float2 r = y_stored[i];
    const float px = r.x - s.shift_x;
    const float py = r.y - s.shift_y;
    y_cur[i] = make_float2(px, py);
    atomicAdd(&hist[lg_tile_of(lg_locate(px, py, s), s.lg_tile, ta)], 1);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < tiles; t += kLgThreads) {
    if (hist[t] != 0) atomicAdd(tile_count + t, hist[t]);
  }
}

constexpr int kLgScatterPerThread = 4;

// The workgroup's tile histogram lives in dynamic LDS of tiles_cap ints,
// tiles_cap the most tiles the FFT length allows, and is overwritten in
// place by the tiles' reserved base offsets (each point keeps its rank in
// registers), so that several workgroups fit on a CU beside the attraction.
// More tiles than tiles_cap (which the host's FFT-length bound excludes)
// raise kErrInterpGrid.
__global__ __launch_bounds__(kLgThreads) void k_lg_bin_scatter(const float2* __restrict__ y_cur,
                                                               DeviceScalars* sc,
                                                               int* __restrict__ tile_cursor,
                                                               float2* __restrict__ binned, int n, int tiles_cap) {
  chain_priority();
  extern __shared__ int hist[];  // counts, then base offsets
  const DeviceScalars s = *sc;
  const int ta = s.lg_tiles_axis;
  const int tiles = ta * ta;
  if (tiles > tiles_cap) {  // uniform over the grid
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(&sc->error_flags, kErrInterpGrid);
    return;
  }
  constexpr int kBatch = kLgThreads * kLgScatterPerThread;
  for (int b0 = blockIdx.x * kBatch; b0 < n; b0 += gridDim.x * kBatch) {
    for (int t = threadIdx.x; t < tiles; t += kLgThreads) hist[t] = 0;
    __syncthreads();
    float2 v[kLgScatterPerThread];
    int tile[kLgScatterPerThread], rank[kLgScatterPerThread];
#pragma unroll
    for (int q = 0; q < kLgScatterPerThread; ++q) {
      const int i = b0 + q * kLgThreads + threadIdx.x;
      tile[q] = -1;
      if (i < n) {
        v[q] = y_cur[i];
        tile[q] = lg_tile_of(lg_locate(v[q].x, v[q].y, s), s.lg_tile, ta);
        rank[q] = atomicAdd(&hist[tile[q]], 1);
      }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < tiles; t += kLgThreads) {
      const int c = hist[t];
      if (c != 0) hist[t] = atomicAdd(tile_cursor + t, c);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kLgScatterPerThread; ++q) {
      if (tile[q] >= 0) binned[hist[tile[q]] + rank[q]] = v[q];
    }
    __syncthreads();
  }
}

// One point's contributions to its box's 9 nodes x 4 moments, added to a.
// Offsets from the nodes in units of h: node c of a box sits at (c + 1/2) h
// from the box's corner, the point at 3 u h.
__device__ __forceinline__ void lg_accumulate(const LgPoint& b, float (&a)[4 * kLgOrder * kLgOrder]) {
#pragma clang fp contract(off)
  float wx[kLgOrder], wy[kLgOrder];
  lg_weights3(b.ux, wx);
  lg_weights3(b.uy, wy);
  const float tx3 = 3.0f * b.ux;
  const float ty3 = 3.0f * b.uy;
#pragma unroll
  for (int r = 0; r < kLgOrder; ++r) {
    const float oy = ty3 - (static_cast<float>(r) + 0.5f);
#pragma unroll
    for (int c = 0; c < kLgOrder; ++c) {
      const float ox = tx3 - (static_cast<float>(c) + 0.5f);
      const float w = wy[r] * wx[c];
      float* d = a + (r * kLgOrder + c) * 4;
      d[0] += w;
      d[1] += w * ox;
      d[2] += w * oy;
      d[3] += w * (ox * ox + oy * oy);
    }
  }
}

// v + (v of the lane the DPP control `ctrl` names), 0 from lanes outside
// row_mask or without a source.
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ float lg_dpp_add(float v) {
  const int src = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, BOUND_ZERO);
  return v + __int_as_float(src);
}

// Sum over the 64 lanes of a wave into lane 63, in VALU cross-lane adds: a
// prefix sum within each row of 16 lanes (row_shr 1, 2, 4, 8) leaves each
// row's sum in its lane 15; row_bcast 15 adds row 0's into row 1 and row 2's
// into row 3, row_bcast 31 adds lane 31 (rows 0 + 1) into row 3.  The order
// is fixed, so the charges do not depend on scheduling.
__device__ __forceinline__ void lg_wave_sum(float (&a)[4 * kLgOrder * kLgOrder]) {
#pragma unroll
  for (int e = 0; e < 4 * kLgOrder * kLgOrder; ++e) {
    float t = a[e];
    t = lg_dpp_add<0x111, 0xf, true>(t);   // row_shr:1
    t = lg_dpp_add<0x112, 0xf, true>(t);   // row_shr:2
    t = lg_dpp_add<0x114, 0xf, true>(t);   // row_shr:4
    t = lg_dpp_add<0x118, 0xf, true>(t);   // row_shr:8
    t = lg_dpp_add<0x142, 0xa, false>(t);  // row_bcast:15 into rows 1 and 3
    t = lg_dpp_add<0x143, 0xc, false>(t);  // row_bcast:31 into rows 2 and 3
    a[e] = t;
  }
}

// Writes one box's 9 nodes x 4 moments into the window of win x win nodes
// (box = local index in a tile of win / 3 boxes per axis).  Every node
// belongs to exactly one box, so plain stores suffice.
__device__ __forceinline__ void lg_store_box(float* acc, int box, int tile, int win,
                                             const float (&a)[4 * kLgOrder * kLgOrder]) {
  const int lbx = box % tile;
  const int lby = box / tile;
  const int wn = win * win;
  const int node0 = (lby * kLgOrder) * win + lbx * kLgOrder;
#pragma unroll
  for (int r = 0; r < kLgOrder; ++r) {
#pragma unroll
    for (int c = 0; c < kLgOrder; ++c) {
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t * wn + node0 + r * win + c] = a[(r * kLgOrder + c) * 4 + t];
    }
  }
}

// The window `acc` is dynamic LDS of acc_cap floats, sized by the host for
// the largest tile its FFT length allows (a 48 x 48 x 4 window is 36 KB, the
// late-phase 6 x 6 x 4 one 576 bytes), so that small tiles leave LDS for more
// workgroups per CU.  A window that would not fit raises kErrInterpGrid.
//
// Per work item (<= kChunk points of one tile): the points are ordered by box
// in LDS (counting sort), then each box is reduced by one wave: lanes take the
// box's points with stride 64 and sum their 9 x 4 contributions in
// registers, DPP adds carry the 64 lanes into one, and the box's nodes are
// stored.
// A tile of one box (the early, compact layouts) splits the box's points over
// the workgroup's waves and adds their sums in wave order.  Every order is
// fixed, so the charges do not depend on scheduling.
constexpr int kLgWaves = kLgThreads / 64;

__global__ __launch_bounds__(kLgThreads) void k_lg_spread(const float2* __restrict__ binned,
                                                          const int4* __restrict__ items,
                                                          const int* __restrict__ tile_item0, DeviceScalars* sc,
                                                          float* __restrict__ charge, float* __restrict__ windows,
                                                          int acc_cap) {
#pragma clang fp contract(off)
  chain_priority();
  extern __shared__ float acc[];  // [charge][node of the window], acc_cap floats
  __shared__ int box_start[kLgBoxesPerTile];
  __shared__ int part[kLgThreads];
  __shared__ float2 sorted[kChunk];
  __shared__ float wave_part[kLgWaves][4 * kLgOrder * kLgOrder];
  __shared__ int wave_total[kLgWaves];
  if (static_cast<int>(blockIdx.x) >= sc->num_items) return;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const DeviceScalars s = *sc;
  const int4 it = items[blockIdx.x];
  const int tile = s.lg_tile;
  const int win = tile * kLgOrder;
  const int wvals = 4 * win * win;
  if (wvals > acc_cap) {  // uniform over the grid: no workgroup touches LDS beyond acc_cap
    if (threadIdx.x == 0) atomicOr(&sc->error_flags, kErrInterpGrid);
    return;
  }
  const int ta = s.lg_tiles_axis;
  const int tx = it.x % ta, ty = it.x / ta;
  const int bx0 = tx * tile, by0 = ty * tile;
  const int nbox = tile * tile;
  box_start[threadIdx.x] = 0;
  __syncthreads();
  const int count = it.z - it.y;  // <= kChunk
  // counting sort of the item's points by box
  float2 v[kLgRun];
  int box[kLgRun], rank[kLgRun];
#pragma unroll
  for (int q = 0; q < kLgRun; ++q) {
    const int p = q * kLgThreads + static_cast<int>(threadIdx.x);
    box[q] = -1;
    if (p < count) {
      v[q] = binned[it.y + p];
      const LgPoint b = lg_locate(v[q].x, v[q].y, s);
      box[q] = (b.by - by0) * tile + (b.bx - bx0);
      rank[q] = atomicAdd(&box_start[box[q]], 1);
    }
  }
  __syncthreads();
  {  // scan of the box counts: shuffles within each wave, wave sums through LDS
    const int t = threadIdx.x;
    const int c = box_start[t];
    int inc = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int x = __shfl_up(inc, off, 64);
      if (lane >= off) inc += x;
    }
    if (lane == 63) wave_total[wave] = inc;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kLgWaves; ++w) inc += w < wave ? wave_total[w] : 0;
    part[t] = inc;               // inclusive end
    box_start[t] = inc - c;      // exclusive start
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kLgRun; ++q) {
    if (box[q] >= 0) sorted[box_start[box[q]] + rank[q]] = v[q];
  }
  __syncthreads();
  float a[4 * kLgOrder * kLgOrder];
  if (nbox == 1) {
    // one box: the waves take interleaved stretches of 64 points
#pragma unroll
    for (int e = 0; e < 4 * kLgOrder * kLgOrder; ++e) a[e] = 0.0f;
    for (int p = wave * 64 + lane; p < count; p += kLgThreads) lg_accumulate(lg_locate(sorted[p].x, sorted[p].y, s), a);
    lg_wave_sum(a);
    if (lane == 63) {
#pragma unroll
      for (int e = 0; e < 4 * kLgOrder * kLgOrder; ++e) wave_part[wave][e] = a[e];
    }
    __syncthreads();
    if (threadIdx.x < 4 * kLgOrder * kLgOrder) {
      const int e = threadIdx.x;
      float t = wave_part[0][e];
#pragma unroll
      for (int w = 1; w < kLgWaves; ++w) t += wave_part[w][e];
      wave_part[0][e] = t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int e = 0; e < 4 * kLgOrder * kLgOrder; ++e) a[e] = wave_part[0][e];
      lg_store_box(acc, 0, tile, win, a);
    }
  } else {
    for (int b = wave; b < nbox; b += kLgWaves) {
      const int b0 = box_start[b];
      const int b1 = part[b];
#pragma unroll
      for (int e = 0; e < 4 * kLgOrder * kLgOrder; ++e) a[e] = 0.0f;
      for (int p = b0 + lane; p < b1; p += 64) lg_accumulate(lg_locate(sorted[p].x, sorted[p].y, s), a);
      // uniform over the wave: the sum lands in lane 63; with at most one
      // point, lane 0 already holds it (zeros for an empty box)
      const bool many = b1 - b0 > 1;
      if (many) lg_wave_sum(a);
      if (lane == (many ? 63 : 0)) lg_store_box(acc, b, tile, win, a);
    }
  }
  __syncthreads();
  const bool sole = tile_item0[it.x + 1] - tile_item0[it.x] == 1;
  if (sole) {
    const int m = s.lg_nodes;
    const int mm = m * m;
    const int wn = win * win;
    for (int e = threadIdx.x; e < wvals; e += kLgThreads) {
      const int ch = e / wn;
      const int node = e - ch * wn;
      const int gy = ty * win + node / win;
      const int gx = tx * win + node % win;
      if (gx < m && gy < m) charge[ch * mm + gy * m + gx] = acc[e];
    }
  } else {
    float* w = windows + static_cast<std::size_t>(blockIdx.x) * kLgWinVals;
    for (int e = threadIdx.x; e < wvals; e += kLgThreads) w[e] = acc[e];
  }
}

// Every node of every plane; nodes of single-item tiles were written by the
// spread itself, nodes of empty tiles get zero.  One workgroup per tile: G
// threads share each window value, thread g summing the tile's items
// i0 + g, i0 + g + G, ..., and the G partial sums are added in the order
// g = 0 .. G - 1, so the result does not depend on scheduling.  A dense box
// early in the optimisation (hundreds of items in one tile) is then summed by
// the whole workgroup, not by one thread per node.
__global__ __launch_bounds__(kLgThreads) void k_lg_gather(const int* __restrict__ tile_item0,
                                                          const float* __restrict__ windows, const DeviceScalars* sc,
                                                          float* __restrict__ charge) {
  chain_priority();
  __shared__ float part[kLgThreads];
  const int m = sc->lg_nodes;
  const int ta = sc->lg_tiles_axis;
  const int win = sc->lg_tile * kLgOrder;
  const int wn = win * win;
  const int wvals = 4 * wn;
  const int mm = m * m;
  const int per = wvals < kLgThreads ? wvals : kLgThreads;  // values per pass
  const int groups = kLgThreads / per;                      // threads per value
  const int g = static_cast<int>(threadIdx.x) / per;
  const int v = static_cast<int>(threadIdx.x) - g * per;
  for (int t = blockIdx.x; t < ta * ta; t += gridDim.x) {
    const int i0 = tile_item0[t];
    const int i1 = tile_item0[t + 1];
    if (i1 - i0 == 1) continue;  // uniform over the workgroup
    const int tx = t % ta, ty = t / ta;
    for (int e0 = 0; e0 < wvals; e0 += per) {
      const int e = e0 + v;
      float acc = 0.0f;
      if (g < groups && e < wvals) {
        const float* src = windows + e;
        int i = i0 + g;
        for (; i + 3 * groups < i1; i += 4 * groups) {
          const float a0 = src[static_cast<std::size_t>(i) * kLgWinVals];
          const float a1 = src[static_cast<std::size_t>(i + groups) * kLgWinVals];
          const float a2 = src[static_cast<std::size_t>(i + 2 * groups) * kLgWinVals];
          const float a3 = src[static_cast<std::size_t>(i + 3 * groups) * kLgWinVals];
          acc += a0;
          acc += a1;
          acc += a2;
          acc += a3;
        }
        for (; i < i1; i += groups) acc += src[static_cast<std::size_t>(i) * kLgWinVals];
      }
      __syncthreads();
      part[threadIdx.x] = acc;
      __syncthreads();
      if (g == 0 && e < wvals) {
        float sum = part[v];
        for (int q = 1; q < groups; ++q) sum += part[q * per + v];
        const int ch = e / wn;
        const int node = e - ch * wn;
        const int gy = ty * win + node / win;
        const int gx = tx * win + node % win;
        if (gx < m && gy < m) charge[ch * mm + gy * m + gx] = sum;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Convolution.  Launch shapes per FFT length F: sequences of length F per
// block so that small transforms still fill a workgroup.
// ---------------------------------------------------------------------------

// Column block of launch block b when `blocks` column blocks are spread over
// col_launch(blocks) launch blocks: the blocks of XCD x (b % kLgColXcds,
// the hardware's round-robin placement) take the x-th contiguous range, so
// the columns of one cache line are read and written through one L2.  -1: a
// padding block with no columns.
__device__ __forceinline__ int col_block(int b, int blocks) {
  const int per = (blocks + kLgColXcds - 1) / kLgColXcds;
  const int c = (b % kLgColXcds) * per + b / kLgColXcds;
  return c < blocks ? c : -1;
}
constexpr int col_launch(int blocks) { return (blocks + kLgColXcds - 1) / kLgColXcds * kLgColXcds; }
template <int F>
struct LgShape {
  static constexpr int G = F / 2;
  static constexpr int H = F / 2 + 1;
  static constexpr int NT = F >= 2048 ? 512 : 256;
  static constexpr int KR = F >= 1024 ? 1 : 1024 / F;  // kernel rows / columns per block (two sequences each)
  static constexpr int CR = F >= 1024 ? 1 : 1024 / F;  // charge / inverse rows per block (two sequences each)
  static constexpr int CC = F >= 512 ? 1 : 512 / F;    // columns of the convolution pass (three sequences each)
};

// K = 1 / (1 + r^2)^2 and K1 = 1 / (1 + r^2) at node offset (dx, dy), r = h |d|.
__device__ __forceinline__ void lg_kernels(int dx, int dy, float h, float& k, float& k1) {
#pragma clang fp contract(off)
  const float ox = static_cast<float>(dx) * h;
  const float oy = static_cast<float>(dy) * h;
  k1 = 1.0f / (1.0f + (ox * ox + oy * oy));
  k = k1 * k1;
}

// Row transforms of the four kernels on rows y in [0, min(m, F/2 + 1)) of the
// wrapped grid (|dx| < m, zero beyond): A = K + i K1 (both real and even in
// dx, so the spectra are the real and imaginary parts) and B = Kx + Ky with
// Kx = K dx (odd in dx: spectrum i Bx) and Ky = K y (even in dx: spectrum By),
// so Re B^ = By and Im B^ = Bx.  Kept for kx in [0, F/2] as two float2
// planes, (K^r, K1^r) and (Bx, By), row-major with row stride F/2 + 1.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_kernel_rows(const DeviceScalars* sc,
                                                                   const float2* __restrict__ tw,
                                                                   float2* __restrict__ k_rows) {
  chain_priority();
  using S = LgShape<F>;
  constexpr int HH = S::H * S::H;
  __shared__ float2 lds[2 * S::KR * F];
  __shared__ float2 tws[F];
  const int m = sc->lg_nodes;
  const float h = sc->lg_node_h;
  const int row0 = blockIdx.x * S::KR;
  if (row0 >= m) return;  // rows >= m are zero and never read
  stage_twiddles<F, S::NT>(tws, tw);
  for (int e = threadIdx.x; e < S::KR * F; e += S::NT) {
    const int r = e / F;
    const int x = e - r * F;
    const int y = row0 + r;
    const int dx = x < S::G ? x : x - F;
    const int adx = dx < 0 ? -dx : dx;
    float k = 0.0f, k1 = 0.0f;
    if (adx < m && y < m) lg_kernels(dx, y, h, k, k1);
    lds[(2 * r) * F + x] = make_float2(k, k1);
    lds[(2 * r + 1) * F + x] = make_float2(k * static_cast<float>(dx) + k * static_cast<float>(y), 0.0f);
  }
  __syncthreads();
  fft_lds<F, 2 * S::KR, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KR * S::H; e += S::NT) {
    const int r = e / S::H;
    const int kx = e - r * S::H;
    const int y = row0 + r;
    if (y >= S::H || y >= m) continue;
    const float2 a = lds[(2 * r) * F + kx];
    const float2 b = lds[(2 * r + 1) * F + kx];
    const int at = y * S::H + kx;
    k_rows[at] = a;
    k_rows[HH + at] = make_float2(b.y, b.x);
  }
}

// Column transforms of the row spectra, read down the columns of the
// row-major rows (row stride F/2 + 1, rows y < min(m, F/2 + 1) valid):
// P = K^r + i K1^r (even in y) gives K^ and K1^ (real); Q = Bx + By, with Bx
// even and By odd in y, gives Cx + i Cy where the kernel spectra of Kx and Ky
// are i Cx and i Cy.  Kept for ky in [0, F/2], kx-major: planes (K^, K1^)
// and (Cx, Cy); Cx is even in ky, Cy odd.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_kernel_cols(const DeviceScalars* sc,
                                                                   const float2* __restrict__ k_rows,
                                                                   const float2* __restrict__ tw,
                                                                   float2* __restrict__ k_hat) {
  chain_priority();
  using S = LgShape<F>;
  constexpr int HH = S::H * S::H;
  __shared__ float2 lds[2 * S::KR * F];
  __shared__ float2 tws[F];
  const int m = sc->lg_nodes;
  const int cb = col_block(static_cast<int>(blockIdx.x), (S::H + S::KR - 1) / S::KR);
  if (cb < 0) return;  // whole block
  const int col0 = cb * S::KR;
  stage_twiddles<F, S::NT>(tws, tw);
  for (int e = threadIdx.x; e < S::KR * F; e += S::NT) {
    const int c = e / F;
    const int y = e - c * F;
    const int kx = col0 + c;
    const bool up = y <= S::G;
    const int ys = up ? y : F - y;
    float2 p = make_float2(0.0f, 0.0f), q = p;
    if (ys < m && kx < S::H) {
      const int at = ys * S::H + kx;
      p = k_rows[at];
      const float2 b = k_rows[HH + at];  // (Bx, By)
      q = make_float2(b.x + (up ? b.y : -b.y), 0.0f);
    }
    lds[(2 * c) * F + y] = p;
    lds[(2 * c + 1) * F + y] = q;
  }
  __syncthreads();
  fft_lds<F, 2 * S::KR, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KR * S::H; e += S::NT) {
    const int c = e / S::H;
    const int ky = e - c * S::H;
    const int kx = col0 + c;
    if (kx >= S::H) continue;
    const int at = kx * S::H + ky;
    k_hat[at] = lds[(2 * c) * F + ky];
    k_hat[HH + at] = lds[(2 * c + 1) * F + ky];
  }
}

// Row transforms of the charge planes: A = m0 + i m1x and B = m1y per row
// y < m (zero-padded to F); A is separated with the Hermitian mirror,
// X[k] = (A[k] + conj A[-k]) / 2 and Y[k] = (A[k] - conj A[-k]) / 2i; B is
// the spectrum of a real row already.  Kept for kx in [0, F/2], row-major
// (row stride F/2 + 1), planes plane_stride apart.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_charge_rows(const DeviceScalars* sc,
                                                                   const float* __restrict__ charge,
                                                                   const float2* __restrict__ tw,
                                                                   float2* __restrict__ rows, long long plane) {
  chain_priority();
  using S = LgShape<F>;
  __shared__ float2 lds[2 * S::CR * F];
  __shared__ float2 tws[F];
  const int m = sc->lg_nodes;
  const int mm = m * m;
  const int row0 = blockIdx.x * S::CR;
  if (row0 >= m) return;
  stage_twiddles<F, S::NT>(tws, tw);
  for (int e = threadIdx.x; e < S::CR * F; e += S::NT) {
    const int r = e / F;
    const int x = e - r * F;
    const int y = row0 + r;
    float2 a = make_float2(0.0f, 0.0f), b = a;
    if (y < m && x < m) {
      const int at = y * m + x;
      a = make_float2(charge[at], charge[mm + at]);
      b = make_float2(charge[2 * mm + at], 0.0f);
    }
    lds[(2 * r) * F + x] = a;
    lds[(2 * r + 1) * F + x] = b;
  }
  __syncthreads();
  fft_lds<F, 2 * S::CR, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::CR * S::H; e += S::NT) {
    const int r = e / S::H;
    const int kx = e - r * S::H;
    const int y = row0 + r;
    if (y >= m) continue;
    const int mk = kx == 0 ? 0 : F - kx;
    const float2 a = lds[(2 * r) * F + kx];
    const float2 am = conjf2(lds[(2 * r) * F + mk]);
    const float2 sa = cadd(a, am), da = csub(a, am);
    const int at = y * S::H + kx;
    rows[at] = cscale(sa, 0.5f);
    rows[plane + at] = make_float2(0.5f * da.y, -0.5f * da.x);
    rows[2 * plane + at] = lds[(2 * r + 1) * F + kx];
  }
}

// Column pass down the columns of the row-major charge spectra (row stride
// F/2 + 1, rows y < m valid): for each column kx, forward transforms of M0,
// M1x, M1y (rows >= m are the zero padding), then per ky
//   Phi0 = M0 K^,  Xi_x = i Cx M0 - K^ M1x,  Xi_y = i Cy M0 - K^ M1y,
// the spectral sums of Z (weight 2 for 0 < kx < F/2, whose mirror column is
// not stored; 1/F^2 applied later)
//   s1 = |M0|^2 K1^,  s3 = Re(conj(M1) . i C M0),  s4 = |M1|^2 K^,
// inverse transforms, rows y < m written back row-major.  A padding block
// (col_block) writes zero partial sums.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_conv_cols(const DeviceScalars* sc,
                                                                 const float2* __restrict__ rows_in,
                                                                 const float2* __restrict__ k_hat,
                                                                 const float2* __restrict__ tw,
                                                                 float2* __restrict__ rows_out, long long plane,
                                                                 double* __restrict__ zpart) {
  chain_priority();
  using S = LgShape<F>;
  constexpr int C = S::CC;
  constexpr int HH = S::H * S::H;
  __shared__ float2 lds[3 * C * F];
  __shared__ float2 tws[F];
  const int m = sc->lg_nodes;
  const int cb = col_block(static_cast<int>(blockIdx.x), (S::H + C - 1) / C);
  if (cb < 0) {  // whole block
    if (threadIdx.x == 0) {
      zpart[3 * blockIdx.x] = 0.0;
      zpart[3 * blockIdx.x + 1] = 0.0;
      zpart[3 * blockIdx.x + 2] = 0.0;
    }
    return;
  }
  const int col0 = cb * C;
  stage_twiddles<F, S::NT>(tws, tw);
  for (int e = threadIdx.x; e < C * F; e += S::NT) {
    const int c = e / F;
    const int y = e - c * F;
    const int kx = col0 + c;
    const bool live = y < m && kx < S::H;
    const long long at = static_cast<long long>(y) * S::H + kx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
      lds[(ch * C + c) * F + y] = live ? rows_in[ch * plane + at] : make_float2(0.0f, 0.0f);
    }
  }
  __syncthreads();
  fft_lds<F, 3 * C, S::NT, false, 1>(lds, tws);
  double s1 = 0.0, s3 = 0.0, s4 = 0.0;
  for (int e = threadIdx.x; e < C * F; e += S::NT) {
    const int c = e / F;
    const int ky = e - c * F;
    const int kx = col0 + c;
    if (kx >= S::H) continue;
    const bool up = ky <= S::G;
    const int at = kx * S::H + (up ? ky : F - ky);
    const float2 kk2 = k_hat[at];       // (K^, K1^)
    const float2 cc = k_hat[HH + at];   // (Cx, Cy)
    const float kk = kk2.x;
    const float k1 = kk2.y;
    const float cx = cc.x;
    const float cy = up ? cc.y : -cc.y;
    float2& v0 = lds[(0 * C + c) * F + ky];
    float2& v1 = lds[(1 * C + c) * F + ky];
    float2& v2 = lds[(2 * C + c) * F + ky];
    const float2 m0 = v0, mx = v1, my = v2;
    const float2 im0 = mul_i(m0);  // i M0
    const double wk = (kx == 0 || kx == S::G) ? 1.0 : 2.0;
    const double a0 = static_cast<double>(m0.x) * m0.x + static_cast<double>(m0.y) * m0.y;
    const double ax = static_cast<double>(mx.x) * mx.x + static_cast<double>(mx.y) * mx.y;
    const double ay = static_cast<double>(my.x) * my.x + static_cast<double>(my.y) * my.y;
    // Re(conj(M1x) i M0) cx + Re(conj(M1y) i M0) cy
    const double rx = static_cast<double>(mx.x) * im0.x + static_cast<double>(mx.y) * im0.y;
    const double ry = static_cast<double>(my.x) * im0.x + static_cast<double>(my.y) * im0.y;
    s1 += wk * a0 * k1;
    s3 += wk * (rx * cx + ry * cy);
    s4 += wk * (ax + ay) * kk;
    v0 = cscale(m0, kk);
    v1 = csub(cscale(im0, cx), cscale(mx, kk));
    v2 = csub(cscale(im0, cy), cscale(my, kk));
  }
  __syncthreads();
  fft_lds<F, 3 * C, S::NT, true, 1>(lds, tws);
  for (int e = threadIdx.x; e < C * S::G; e += S::NT) {
    const int c = e / S::G;
    const int y = e - c * S::G;
    const int kx = col0 + c;
    if (y >= m || kx >= S::H) continue;
    const long long at = static_cast<long long>(y) * S::H + kx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) rows_out[ch * plane + at] = lds[(ch * C + c) * F + y];
  }
  s1 = block_sum<S::NT>(s1);
  s3 = block_sum<S::NT>(s3);
  s4 = block_sum<S::NT>(s4);
  if (threadIdx.x == 0) {
    zpart[3 * blockIdx.x] = s1;
    zpart[3 * blockIdx.x + 1] = s3;
    zpart[3 * blockIdx.x + 2] = s4;
  }
}

// Inverse row pass on the row-major potential spectra: U = Phi0 + i Xi_x and
// V = Xi_y (spectra of real rows, upper half rebuilt from conjugates);
// potentials for x < m scaled by 1/F^2 and stored per node as (phi0, xi_x,
// xi_y, 0); per-block sums of m2 phi0 in fp64.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_inverse_rows(const DeviceScalars* sc,
                                                                    const float2* __restrict__ rows, long long plane,
                                                                    const float* __restrict__ charge,
                                                                    const float2* __restrict__ tw,
                                                                    float4* __restrict__ field,
                                                                    double* __restrict__ partial) {
  chain_priority();
  using S = LgShape<F>;
  __shared__ float2 lds[2 * S::CR * F];
  __shared__ float2 tws[F];
  const int m = sc->lg_nodes;
  const int mm = m * m;
  const int row0 = blockIdx.x * S::CR;
  double acc = 0.0;
  if (row0 < m) {  // uniform over the block
    stage_twiddles<F, S::NT>(tws, tw);
    for (int e = threadIdx.x; e < S::CR * F; e += S::NT) {
      const int r = e / F;
      const int kx = e - r * F;
      const int y = row0 + r;
      float2 u = make_float2(0.0f, 0.0f), v = u;
      if (y < m) {
        const bool low = kx <= S::G;
        const int at = y * S::H + (low ? kx : F - kx);
        float2 a = rows[at], b = rows[plane + at], c = rows[2 * plane + at];
        if (!low) {
          a = conjf2(a);
          b = conjf2(b);
          c = conjf2(c);
        }
        u = cadd(a, mul_i(b));
        v = c;
      }
      lds[(2 * r) * F + kx] = u;
      lds[(2 * r + 1) * F + kx] = v;
    }
    __syncthreads();
    fft_lds<F, 2 * S::CR, S::NT, true, 1>(lds, tws);
    const float scale = 1.0f / (static_cast<float>(F) * static_cast<float>(F));
    for (int e = threadIdx.x; e < S::CR * S::G; e += S::NT) {
      const int r = e / S::G;
      const int x = e - r * S::G;
      const int y = row0 + r;
      if (y >= m || x >= m) continue;
      const float2 u = cscale(lds[(2 * r) * F + x], scale);
      const float vx = lds[(2 * r + 1) * F + x].x * scale;
      const int at = y * m + x;
      field[at] = make_float4(u.x, u.y, vx, 0.0f);
      acc += static_cast<double>(charge[3 * mm + at]) * static_cast<double>(u.x);
    }
  }
  acc = block_sum<S::NT>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = acc;
}

// Z = s1 / F^2 + h^2 (2 sum m2 phi0 + (4 s3 - 2 s4) / F^2) - n and its fp32
// reciprocal (floor FLT_MIN, as the bilinear grid's normaliser); flags a
// node count that the FFT length could not hold.
__global__ __launch_bounds__(256) void k_lg_finalize_z(const double* __restrict__ spec_part, int spec_blocks,
                                                       const double* __restrict__ row_part, int row_blocks, int n,
                                                       int fft_len, DeviceScalars* sc) {
  chain_priority();
  double s1 = 0.0, s3 = 0.0, s4 = 0.0, t2 = 0.0;
  for (int b = threadIdx.x; b < spec_blocks; b += 256) {
    s1 += spec_part[3 * b];
    s3 += spec_part[3 * b + 1];
    s4 += spec_part[3 * b + 2];
  }
  for (int b = threadIdx.x; b < row_blocks; b += 256) t2 += row_part[b];
  s1 = block_sum<256>(s1);
  s3 = block_sum<256>(s3);
  s4 = block_sum<256>(s4);
  t2 = block_sum<256>(t2);
  if (threadIdx.x == 0) {
    const double inv_f2 = 1.0 / (static_cast<double>(fft_len) * static_cast<double>(fft_len));
    const double h = sc->lg_node_h;
    const double total = s1 * inv_f2 + h * h * (2.0 * t2 + (4.0 * s3 - 2.0 * s4) * inv_f2);
    sc->sum_q = total;
    const double z = total - static_cast<double>(n);
    sc->inv_sum_q = static_cast<float>(1.0 / (z > static_cast<double>(FLT_MIN) ? z : static_cast<double>(FLT_MIN)));
    if (2 * sc->lg_nodes > fft_len) sc->error_flags |= kErrInterpGrid;
  }
}

// Buffers of one FFT length.  Spectra planes are G * H float2 (G = F/2,
// H = F/2 + 1) apart: A holds the charge row spectra, B the potential row
// spectra.  The kernel row spectra and the kernel spectrum have a buffer
// each (H * H float2 planes).
template <int F>
hipError_t lg_fft_launch(int which, InterpBuffers& ib, DeviceScalars* sc, const float2* tw, int n,
                         hipStream_t stream) {
  using S = LgShape<F>;
  const int kblocks = (S::H + S::KR - 1) / S::KR;
  const int rblocks = (S::G + S::CR - 1) / S::CR;
  const int cblocks = col_launch((S::H + S::CC - 1) / S::CC);
  const long long plane = static_cast<long long>(S::G) * S::H;
  double* spec_part = ib.z_partial;
  double* row_part = ib.z_partial + 3 * kLgMaxSpecBlocks;
  static_assert(col_launch((S::H + S::CC - 1) / S::CC) <= kLgMaxSpecBlocks, "a partial-sum slot per column block");
  switch (which) {
    case 0:
      k_lg_kernel_rows<F><<<kblocks, S::NT, 0, stream>>>(sc, tw, ib.k_rows);
      break;
    case 2:
      k_lg_kernel_cols<F><<<col_launch(kblocks), S::NT, 0, stream>>>(sc, ib.k_rows, tw, ib.k_cols);
      break;
    case 3:
      k_lg_charge_rows<F><<<rblocks, S::NT, 0, stream>>>(sc, ib.charge, tw, ib.spec_a, plane);
      break;
    case 5:
      k_lg_conv_cols<F><<<cblocks, S::NT, 0, stream>>>(sc, ib.spec_a, ib.k_cols, tw, ib.spec_b, plane, spec_part);
      break;
    case 7:
      k_lg_inverse_rows<F><<<rblocks, S::NT, 0, stream>>>(sc, ib.spec_b, plane, ib.charge, tw, ib.field, row_part);
      k_lg_finalize_z<<<1, 256, 0, stream>>>(spec_part, cblocks, row_part, rblocks, n, F, sc);
      break;

    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_interp_bin_count(const float2* y_stored, float2* y_cur, const DeviceScalars* sc,
                                   InterpBuffers& ib, int n, hipStream_t stream) {
  const int needed = (n + kLgThreads - 1) / kLgThreads;
  const int blocks = std::max(1, std::min(needed, 1024));
  k_lg_bin_count<<<blocks, kLgThreads, 0, stream>>>(y_stored, y_cur, sc, ib.tile_count, n);
  return hipGetLastError();
}

// Boxes per axis of a grid of at most fft_len / 2 nodes per axis.
int lg_boxes_bound(int fft_len) { return std::max(1, std::min(fft_len / 2, kLgMaxNodes) / kLgOrder); }

// The most tiles per axis any such grid is cut into (lg_tile_for, as the
// statistics apply it on the device).
int lg_tiles_axis_bound(int fft_len) {
  int most = 1;
  for (int nb = 1; nb <= lg_boxes_bound(fft_len); ++nb) most = std::max(most, (nb + lg_tile_for(nb) - 1) / lg_tile_for(nb));
  return most;
}

hipError_t launch_interp_bin_scatter(const float2* y_cur, DeviceScalars* sc, InterpBuffers& ib, int n, int fft_len,
                                     hipStream_t stream) {
  constexpr int kBatch = kLgThreads * kLgScatterPerThread;
  const int needed = (n + kBatch - 1) / kBatch;
  const int blocks = std::max(1, std::min(needed, 1024));
  const int ta = lg_tiles_axis_bound(fft_len);
  const int tiles_cap = ta * ta;
  k_lg_bin_scatter<<<blocks, kLgThreads, tiles_cap * sizeof(int), stream>>>(y_cur, sc, ib.tile_cursor, ib.binned, n,
                                                                           tiles_cap);
  return hipGetLastError();
}

// The largest tile a grid of at most fft_len / 2 nodes per axis can use (the
// tile grows with the box count).
int lg_tile_bound(int fft_len) { return lg_tile_for(lg_boxes_bound(fft_len)); }

hipError_t launch_interp_spread(DeviceScalars* sc, InterpBuffers& ib, int n, int fft_len, hipStream_t stream) {
  const int win = lg_tile_bound(fft_len) * kLgOrder;
  const int acc_cap = 4 * win * win;
  k_lg_spread<<<lg_max_items(n), kLgThreads, static_cast<std::size_t>(acc_cap) * sizeof(float), stream>>>(
      ib.binned, ib.items, ib.tile_item0, sc, ib.charge, ib.windows, acc_cap);
  return hipGetLastError();
}

hipError_t launch_interp_gather(const DeviceScalars* sc, InterpBuffers& ib, hipStream_t stream) {
  k_lg_gather<<<kLgMaxTilesAxis * kLgMaxTilesAxis, kLgThreads, 0, stream>>>(ib.tile_item0, ib.windows, sc, ib.charge);
  return hipGetLastError();
}

hipError_t launch_interp_fft(int which, int fft_len, InterpBuffers& ib, DeviceScalars* sc, const float2* tw, int n,
                             hipStream_t stream) {
  switch (fft_len) {
    case 64: return lg_fft_launch<64>(which, ib, sc, tw, n, stream);
    case 96: return lg_fft_launch<96>(which, ib, sc, tw, n, stream);
    case 128: return lg_fft_launch<128>(which, ib, sc, tw, n, stream);
    case 192: return lg_fft_launch<192>(which, ib, sc, tw, n, stream);
    case 256: return lg_fft_launch<256>(which, ib, sc, tw, n, stream);
    case 384: return lg_fft_launch<384>(which, ib, sc, tw, n, stream);
    case 512: return lg_fft_launch<512>(which, ib, sc, tw, n, stream);
    case 768: return lg_fft_launch<768>(which, ib, sc, tw, n, stream);
    case 1024: return lg_fft_launch<1024>(which, ib, sc, tw, n, stream);
    case 1536: return lg_fft_launch<1536>(which, ib, sc, tw, n, stream);
    case 2048: return lg_fft_launch<2048>(which, ib, sc, tw, n, stream);
    case 3072: return lg_fft_launch<3072>(which, ib, sc, tw, n, stream);
    case 4096: return lg_fft_launch<4096>(which, ib, sc, tw, n, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fehip
