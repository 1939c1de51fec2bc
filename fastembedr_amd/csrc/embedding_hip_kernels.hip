// gfx950 (CDNA4) kernels of the openTSNE-style t-SNE gradient loop.
//
// Wave64 throughout.  Nothing here uses MFMA: the loop is HBM/L2-bound
// (CSR streaming, grid FFTs) and its arithmetic is fp32 vector work.
//
// Kernel map (reference semantics in src/tsne_neighbors.cpp of
// tkcaccia/fastEmbedR):
//   k_row_search        per-row fp32 perplexity bisection (:488-538) and the
//                       directed edges of both orientations (:566-579)
//   sort + k_mark_heads + scan + k_compact
//                       duplicate merge in fp64 and symmetric CSR (:581-648)
//   k_stats             bounding box + fp64 mean -> grid geometry
//                       (:1089-1110, :1200-1211)
//   k_spread            bilinear charge spreading (:1111-1148)
//   k_kernel_rows/cols  spectrum of the Cauchy kernel and its square (:860-897)
//   k_charge_rows, k_conv_cols, k_inverse_rows
//                       zero-padded 2-D convolution (:899-941) with
//                       real-input packing, pruned rows and fused products;
//                       sum of q (:1150-1163) as a grid dot product
//   k_attract<mode>     CSR attraction (:985-1012) + bilinear read-back
//                       (:1165-1180) + gains/momentum/clip update (:1217-1256)
//                       + statistics for the next iteration's centring
//   k_exact_rep, k_kl_rows
//                       exact O(n^2) terms for checking (:1014-1074, :958-983,
//                       :1258-1285)

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <cfloat>
#include <algorithm>
#include <cmath>

#include "device_common.h"
#include "tsne_device.h"

namespace fehip {
namespace {

// Grid-wide reductions write one partial per block and are finished by a
// separate single-block kernel.  (A "last block done" finish would need a
// device-scope release fence in every block, which on multi-XCD parts writes
// back the L2 each time.)

// Grid geometry from the bounding box and mean of the stored layout
// (src/tsne_neighbors.cpp:1089-1110 and :1200-1211).  Subtracting a constant
// is monotone under rounding, so the box of the centred layout is the centred
// box of the stored one.  fp32, no contraction, same operation order.
__device__ void set_geometry(DeviceScalars* sc, const BlockStats& t, int n, int g, bool center) {
#pragma clang fp contract(off)
  const double mx = t.sum_x / static_cast<double>(n);
  const double my = t.sum_y / static_cast<double>(n);
  const float sx = center ? static_cast<float>(mx) : 0.0f;
  const float sy = center ? static_cast<float>(my) : 0.0f;
  const float mnx = t.min_x - sx, mxx = t.max_x - sx;
  const float mny = t.min_y - sy, mxy = t.max_y - sy;
  const float cx = 0.5f * (mnx + mxx);
  const float cy = 0.5f * (mny + mxy);
  const float ex = mxx - mnx, ey = mxy - mny;
  float span = (ex < ey) ? ey : ex;
  if (!isfinite(span) || span <= 0.0f) span = 1.0f;
  const float half = 0.55f * span + 1.0e-3f;
  const float h = (2.0f * half) / static_cast<float>(g - 1);
  sc->shift_x = sx;
  sc->shift_y = sy;
  sc->lo_x = cx - half;
  sc->lo_y = cy - half;
  sc->h = h;
  sc->inv_h = 1.0f / h;
  sc->mean_x = mx;
  sc->mean_y = my;
  sc->min_x = mnx;
  sc->max_x = mxx;
  sc->min_y = mny;
  sc->max_y = mxy;
  if (sc->lg_order > 0) {
    // FIt-SNE interpolation grid: one square over both axes from the
    // smallest to the largest centred coordinate, max(min_intervals,
    // ceil(span / ints_per_unit)) boxes per axis, capped at kLgMaxNodes nodes.
    const float lo = (mnx < mny) ? mnx : mny;
    const float hi = (mxx > mxy) ? mxx : mxy;
    double lspan = static_cast<double>(hi) - static_cast<double>(lo);
    if (!(lspan > 0.0) || !isfinite(lspan)) lspan = 1.0;
    const double want = ceil(lspan / static_cast<double>(sc->lg_ints_per_unit));
    double boxes = want > static_cast<double>(sc->lg_min_intervals) ? want : static_cast<double>(sc->lg_min_intervals);
    const double cap = static_cast<double>(kLgMaxNodes / sc->lg_order);
    if (!(boxes <= cap)) boxes = cap;
    const int nb = static_cast<int>(boxes);
    const double w = lspan / static_cast<double>(nb);
    sc->lg_lo = lo;
    sc->lg_box_w = static_cast<float>(w);
    sc->lg_box_wd = w;
    sc->lg_inv_box_wd = 1.0 / w;
    sc->lg_node_h = static_cast<float>(w / static_cast<double>(sc->lg_order));
    sc->lg_boxes = nb;
    sc->lg_nodes = nb * sc->lg_order;
  }
}

template <int NT>
__device__ void publish_stats(BlockStats local, BlockStats* partial) {
  BlockStats s = block_stats<NT>(local);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

// Reduces the per-block statistics in a fixed order (deterministic) and sets
// the grid geometry.  With box_out (a ring of kBoxRing slots in pinned,
// coherent host memory) the interpolation grid's box count, tagged with the
// sequence number sc->ring_seq, is also stored in slot ring_seq % kBoxRing
// (one 64-bit store) and the counter advanced, so the host learns it by
// reading host memory: no device-to-host copy and no event.  The slot is
// chosen on the device so that a replayed graph of the iteration writes the
// next slot each time.
__global__ __launch_bounds__(256) void k_finalize_stats(const BlockStats* __restrict__ partial, int blocks,
                                                        DeviceScalars* sc, int n, int g, int center,
                                                        unsigned long long* box_out) {
  chain_priority();
  BlockStats acc = stats_identity();
  for (int b = threadIdx.x; b < blocks; b += 256) combine(acc, partial[b]);
  acc = block_stats<256>(acc);
  if (threadIdx.x == 0) {
    set_geometry(sc, acc, n, g, center != 0);
    if (box_out != nullptr) {
      const unsigned int seq = sc->ring_seq;
      const unsigned long long tagged =
          (static_cast<unsigned long long>(seq) << 32) | static_cast<unsigned int>(sc->lg_boxes);
      __hip_atomic_store(box_out + (seq & (kBoxRing - 1)), tagged, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      sc->ring_seq = seq + 1u;
    }
  }
}

// ---------------------------------------------------------------------------
// P construction
// ---------------------------------------------------------------------------
constexpr int kSearchThreads = 64;

// One thread per row; the row's squared distances are staged in LDS as
// [column][thread] (conflict-free).  Input is column-major, so both the
// distance and the index reads are coalesced across the wave.  The search is
// the reference's fp32 algorithm in the same operation order; the two loops
// of the reference (mass, then entropy) are fused, which does not change
// either accumulation order.
template <typename DT>
__global__ __launch_bounds__(kSearchThreads) void k_row_search(const int* __restrict__ idx_cm,
                                                               const DT* __restrict__ dist_cm, int n, int k,
                                                               int offset, float log_perp,
                                                               float* __restrict__ p_cond,
                                                               std::uint64_t* __restrict__ keys,
                                                               float* __restrict__ vals, int key_bits,
                                                               double* __restrict__ mass_partial,
                                                               DeviceScalars* sc) {
#pragma clang fp contract(off)
  extern __shared__ float sq[];
  const int t = threadIdx.x;
  const int i = blockIdx.x * kSearchThreads + t;
  const bool active = i < n;
  unsigned int bad = 0u;
  if (active) {
    for (int j = 0; j < k; ++j) {
      const float d = static_cast<float>(dist_cm[static_cast<std::size_t>(j) * n + i]);
      if (!isfinite(d) || d < 0.0f) bad |= kErrDistance;
      sq[j * kSearchThreads + t] = d * d;
    }
  }
  double mass_sum = 0.0;
  unsigned long long self = 0ull;
  if (active) {
    float beta = 1.0f;
    float lo = -FLT_MAX;
    float hi = FLT_MAX;
    float mass = FLT_MIN;
    float beta_eval = beta;
    bool done = false;
    for (int step = 0; !done && step < 200; ++step) {
      beta_eval = beta;
      mass = FLT_MIN;
      float ent = 0.0f;
      for (int j = 0; j < k; ++j) {
        const float s = sq[j * kSearchThreads + t];
        const float w = expf(-beta * s);
        mass += w;
        ent += beta * (s * w);
      }
      ent = ent / mass + logf(mass);
      const float gap = ent - log_perp;
      if (fabsf(gap) < 1e-5f) {
        done = true;
      } else if (gap > 0.0f) {
        lo = beta;
        beta = (hi == FLT_MAX || hi == -FLT_MAX) ? beta * 2.0f : (beta + hi) * 0.5f;
      } else {
        hi = beta;
        beta = (lo == -FLT_MAX || lo == FLT_MAX) ? beta * 0.5f : (beta + lo) * 0.5f;
      }
    }
    const float inv = 1.0f / mass;
    const std::uint64_t sentinel = (key_bits >= 32) ? ~0ull : ((1ull << (2 * key_bits)) - 1ull);
    for (int j = 0; j < k; ++j) {
      const std::size_t e = static_cast<std::size_t>(j) * n + i;
      const float p = expf(-beta_eval * sq[j * kSearchThreads + t]) * inv;
      p_cond[e] = p;
      const int nb = idx_cm[e] - offset;
      if (nb < 0 || nb >= n) bad |= kErrIndex;
      if (nb == i || nb < 0 || nb >= n) {
        keys[2 * e] = sentinel;
        keys[2 * e + 1] = sentinel;
        vals[2 * e] = 0.0f;
        vals[2 * e + 1] = 0.0f;
        ++self;
      } else {
        keys[2 * e] = (static_cast<std::uint64_t>(i) << key_bits) | static_cast<std::uint64_t>(nb);
        keys[2 * e + 1] = (static_cast<std::uint64_t>(nb) << key_bits) | static_cast<std::uint64_t>(i);
        vals[2 * e] = p;
        vals[2 * e + 1] = p;
        mass_sum += static_cast<double>(p);
      }
    }
  }
  mass_sum = wave_sum(mass_sum);
  if (t == 0) {
    mass_partial[blockIdx.x] = mass_sum;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) self += __shfl_xor(self, off, kWave);
  unsigned int bad_all = bad;
  for (int off = kWave / 2; off > 0; off >>= 1) bad_all |= __shfl_xor(bad_all, off, kWave);
  if (t == 0) {
    if (self) atomicAdd(&sc->self_edges, self);
    if (bad_all) atomicOr(&sc->error_flags, bad_all);
  }
}

__global__ __launch_bounds__(256) void k_finalize_mass(const double* __restrict__ partial, int blocks,
                                                       DeviceScalars* sc) {
  double acc = 0.0;
  for (int b = threadIdx.x; b < blocks; b += 256) acc += partial[b];
  acc = block_sum<256>(acc);
  if (threadIdx.x == 0) sc->total_mass = acc;
}

__global__ __launch_bounds__(256) void k_mark_heads(const std::uint64_t* __restrict__ keys, std::size_t count,
                                                    int* __restrict__ heads) {
  const std::size_t e = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= count) return;
  heads[e] = (e == 0 || keys[e] != keys[e - 1]) ? 1 : 0;
}

// One thread per run head: fp64 sum of the run (the reference sums the
// duplicates of a key in fp64, src/tsne_neighbors.cpp:590-597), scaled by
// float(0.5 / total_mass) after narrowing (:632-637).  Row pointers are filled
// at each row change; the last entry closes the remaining rows.
__global__ __launch_bounds__(256) void k_compact(const std::uint64_t* __restrict__ keys,
                                                 const float* __restrict__ vals, const int* __restrict__ heads,
                                                 const int* __restrict__ pos, std::size_t count, int key_bits,
                                                 int n, const DeviceScalars* sc, int* __restrict__ row_ptr,
                                                 int* __restrict__ col, float* __restrict__ val) {
  const std::size_t e = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= count) return;
  const std::uint64_t mask = (1ull << key_bits) - 1ull;
  const std::uint64_t key = keys[e];
  const int row = static_cast<int>(key >> key_bits);
  if (heads[e]) {
    const int u = pos[e];
    double s = 0.0;
    for (std::size_t f = e; f < count && keys[f] == key; ++f) s += static_cast<double>(vals[f]);
    const float norm = static_cast<float>(0.5 / sc->total_mass);
    col[u] = static_cast<int>(key & mask);
    val[u] = static_cast<float>(s) * norm;
    const int prev_row = (e == 0) ? -1 : static_cast<int>(keys[e - 1] >> key_bits);
    for (int r = prev_row + 1; r <= row; ++r) row_ptr[r] = u;
  }
  if (e == count - 1) {
    const int nnz = pos[e] + heads[e];
    for (int r = row + 1; r <= n; ++r) row_ptr[r] = nnz;
  }
}

// ---------------------------------------------------------------------------
// Layout statistics, spreading, centring
// ---------------------------------------------------------------------------
constexpr int kPointThreads = 256;

__global__ __launch_bounds__(kPointThreads) void k_stats(const float2* __restrict__ y, int n, int g, int center,
                                                         BlockStats* __restrict__ partial, DeviceScalars* sc) {
  BlockStats s = stats_identity();
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) {
    const float2 v = y[i];
    s.min_x = fminf(s.min_x, v.x);
    s.max_x = fmaxf(s.max_x, v.x);
    s.min_y = fminf(s.min_y, v.y);
    s.max_y = fmaxf(s.max_y, v.y);
    s.sum_x += static_cast<double>(v.x);
    s.sum_y += static_cast<double>(v.y);
  }
  publish_stats<kPointThreads>(s, partial);
}

// Bilinear weights of one point, exactly as the reference computes them
// (src/tsne_neighbors.cpp:1116-1133).
struct Bilinear {
  int x0, y0;
  float tx, ty;
};

__device__ __forceinline__ Bilinear locate(float px, float py, const DeviceScalars& s, int g) {
#pragma clang fp contract(off)
  const float top = static_cast<float>(g - 1);
  const float ux = fmaxf(0.0f, fminf(top, (px - s.lo_x) * s.inv_h));
  const float uy = fmaxf(0.0f, fminf(top, (py - s.lo_y) * s.inv_h));
  Bilinear b;
  b.x0 = max(0, min(g - 2, static_cast<int>(floorf(ux))));
  b.y0 = max(0, min(g - 2, static_cast<int>(floorf(uy))));
  b.tx = ux - static_cast<float>(b.x0);
  b.ty = uy - static_cast<float>(b.y0);
  return b;
}

// ---------------------------------------------------------------------------
// Tile-binned spreading.  Points are counted per tile of kTile x kTile cells
// (LDS histogram, one global atomic per block and tile), the counts are
// scanned into tile ranges and work items of at most kChunk points, points
// are scattered into tile order (LDS ranks, one global atomic per batch and
// tile), and each work item accumulates its points' bilinear charges into a
// (kTile + 1)^2 node window in LDS before adding the window to the grid.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int tile_of(const Bilinear& b, int ta) { return (b.y0 / kTile) * ta + b.x0 / kTile; }

__global__ __launch_bounds__(kPointThreads) void k_bin_count(const float2* __restrict__ y_stored,
                                                             float2* __restrict__ y_cur, const DeviceScalars* sc,
                                                             int* __restrict__ tile_count, int n, int g, int ta) {
#pragma clang fp contract(off)
  chain_priority();
  __shared__ int hist[kMaxTiles];
  const int tiles = ta * ta;
  for (int t = threadIdx.x; t < tiles; t += kPointThreads) hist[t] = 0;
  __syncthreads();
  const DeviceScalars s = *sc;
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) {
    const float2 r = y_stored[i];
    const float px = r.x - s.shift_x;
    const float py = r.y - s.shift_y;
    y_cur[i] = make_float2(px, py);
    atomicAdd(&hist[tile_of(locate(px, py, s, g), ta)], 1);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < tiles; t += kPointThreads) {
    if (hist[t] != 0) atomicAdd(tile_count + t, hist[t]);
  }
}

// The plan's scans run in one block of kPlanThreads threads, kPlanPer
// consecutive tiles per thread.  A block of 4 waves finds room on a CU beside
// the attraction sooner than a block of 16 would.
constexpr int kPlanThreads = 256;
constexpr int kPlanPer = kMaxTiles / kPlanThreads;
static_assert(kPlanPer * kPlanThreads == kMaxTiles, "whole entries per thread");

// Each tile's first point (tile_cursor, for the scatter's reservations) and
// work items of <= kChunk points, from the tile counts (which it clears for
// the next iteration).
__global__ __launch_bounds__(kPlanThreads) void k_bin_plan(int* __restrict__ tile_count,
                                                           int* __restrict__ tile_cursor, int4* __restrict__ items,
                                                           DeviceScalars* sc, int tiles) {
  chain_priority();
  __shared__ int part[2 * kPlanThreads / kWave];
  int cnt[kPlanPer], start[kPlanPer], chunks[kPlanPer], base[kPlanPer];
  for (int q = 0; q < kPlanPer; ++q) {
    const int t = threadIdx.x * kPlanPer + q;
    cnt[q] = t < tiles ? tile_count[t] : 0;
    if (t < tiles) tile_count[t] = 0;  // ready for the next iteration's count
    start[q] = cnt[q];
    chunks[q] = (cnt[q] + kChunk - 1) / kChunk;
    base[q] = chunks[q];
  }
  int total_points = 0, total_items = 0;
  block_exclusive_scan2<kPlanPer, kPlanThreads>(start, base, part, total_points, total_items);
  (void)total_points;
  for (int q = 0; q < kPlanPer; ++q) {
    const int t = threadIdx.x * kPlanPer + q;
    if (t >= tiles) continue;
    tile_cursor[t] = start[q];
    for (int c = 0; c < chunks[q]; ++c) {
      const int b = start[q] + c * kChunk;
      const int e = min(start[q] + cnt[q], b + kChunk);
      items[base[q] + c] = make_int4(t, b, e, 0);
    }
  }
  if (threadIdx.x == 0) sc->num_items = total_items;
}

constexpr int kScatterPerThread = 4;

__global__ __launch_bounds__(kPointThreads) void k_bin_scatter(const float2* __restrict__ y_cur,
                                                               const DeviceScalars* sc,
                                                               int* __restrict__ tile_cursor,
                                                               float2* __restrict__ binned, int n, int g, int ta) {
  chain_priority();
  __shared__ int hist[kMaxTiles];
  __shared__ int base[kMaxTiles];
  const int tiles = ta * ta;
  const DeviceScalars s = *sc;
  constexpr int kBatch = kPointThreads * kScatterPerThread;
  for (int b0 = blockIdx.x * kBatch; b0 < n; b0 += gridDim.x * kBatch) {
    for (int t = threadIdx.x; t < tiles; t += kPointThreads) hist[t] = 0;
    __syncthreads();
    float2 v[kScatterPerThread];
    int tile[kScatterPerThread], rank[kScatterPerThread];
#pragma unroll
    for (int q = 0; q < kScatterPerThread; ++q) {
      const int i = b0 + q * kPointThreads + threadIdx.x;
      tile[q] = -1;
      if (i < n) {
        v[q] = y_cur[i];
        tile[q] = tile_of(locate(v[q].x, v[q].y, s, g), ta);
        rank[q] = atomicAdd(&hist[tile[q]], 1);
      }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < tiles; t += kPointThreads) {
      const int c = hist[t];
      if (c != 0) base[t] = atomicAdd(tile_cursor + t, c);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kScatterPerThread; ++q) {
      if (tile[q] >= 0) binned[base[tile[q]] + rank[q]] = v[q];
    }
    __syncthreads();
  }
}

// One work item (<= kChunk points of one tile).  The points are first
// ordered by cell inside the tile (LDS counting sort over the kTile^2 cells),
// then each lane walks kSpreadRun consecutive points of that order: points of
// one cell share their four nodes, so a lane sums their 12 charges in
// registers and adds them to the LDS window once per cell it meets instead of
// once per point.  Dense cells, where many points pile onto the same nodes,
// are what made per-point LDS atomics serialise.
constexpr int kSpreadRun = kChunk / kPointThreads;
static_assert(kSpreadRun * kPointThreads == kChunk, "a work item is one run per lane");

__global__ __launch_bounds__(kPointThreads) void k_spread_tiles(const float2* __restrict__ binned,
                                                                const int4* __restrict__ items,
                                                                const DeviceScalars* sc, float* __restrict__ mass,
                                                                float* __restrict__ mass_x,
                                                                float* __restrict__ mass_y, int g, int ta) {
#pragma clang fp contract(off)
  chain_priority();
  constexpr int W = kTile + 1;
  constexpr int kCells = kTile * kTile;
  __shared__ float acc[3 * W * W];
  __shared__ int cell_start[kCells];
  __shared__ float2 sorted[kChunk];
  if (static_cast<int>(blockIdx.x) >= sc->num_items) return;
  const int4 it = items[blockIdx.x];
  const int tx = it.x % ta, ty = it.x / ta;
  const int x_base = tx * kTile, y_base = ty * kTile;
  for (int e = threadIdx.x; e < 3 * W * W; e += kPointThreads) acc[e] = 0.0f;
  for (int e = threadIdx.x; e < kCells; e += kPointThreads) cell_start[e] = 0;
  __syncthreads();
  const DeviceScalars s = *sc;
  const int count = it.z - it.y;  // <= kChunk
  // counting sort by cell: counts and ranks
  float2 v[kSpreadRun];
  int cell[kSpreadRun], rank[kSpreadRun];
#pragma unroll
  for (int q = 0; q < kSpreadRun; ++q) {
    const int p = q * kPointThreads + static_cast<int>(threadIdx.x);
    cell[q] = -1;
    if (p < count) {
      v[q] = binned[it.y + p];
      const Bilinear b = locate(v[q].x, v[q].y, s, g);
      cell[q] = (b.y0 - y_base) * kTile + (b.x0 - x_base);
      rank[q] = atomicAdd(&cell_start[cell[q]], 1);
    }
  }
  __syncthreads();
  // exclusive scan of the kCells counts (one per thread)
  static_assert(kCells == kPointThreads, "one cell per thread in the scan");
  {
    const int t = threadIdx.x;
    const int c = cell_start[t];
    int incl = c;
    __shared__ int part[kPointThreads];
    part[t] = incl;
    __syncthreads();
    for (int off = 1; off < kPointThreads; off <<= 1) {
      const int add = t >= off ? part[t - off] : 0;
      __syncthreads();
      part[t] += add;
      __syncthreads();
    }
    cell_start[t] = part[t] - c;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kSpreadRun; ++q) {
    if (cell[q] >= 0) sorted[cell_start[cell[q]] + rank[q]] = v[q];
  }
  __syncthreads();
  // each lane: kSpreadRun consecutive points of the cell order
  float c[12];
  int cur = -1;
#pragma unroll
  for (int m = 0; m < 12; ++m) c[m] = 0.0f;
  const int p0 = static_cast<int>(threadIdx.x) * kSpreadRun;
#pragma unroll
  for (int q = 0; q < kSpreadRun; ++q) {
    const int p = p0 + q;
    if (p >= count) break;
    const float2 u = sorted[p];
    const Bilinear b = locate(u.x, u.y, s, g);
    const int node = (b.y0 - y_base) * W + (b.x0 - x_base);
    if (node != cur) {
      if (cur >= 0) {
#pragma unroll
        for (int m = 0; m < 3; ++m) {
          float* a = acc + m * W * W + cur;
          atomicAdd(a, c[4 * m + 0]);
          atomicAdd(a + 1, c[4 * m + 1]);
          atomicAdd(a + W, c[4 * m + 2]);
          atomicAdd(a + W + 1, c[4 * m + 3]);
        }
      }
      cur = node;
#pragma unroll
      for (int m = 0; m < 12; ++m) c[m] = 0.0f;
    }
    const float w00 = (1.0f - b.tx) * (1.0f - b.ty);
    const float w10 = b.tx * (1.0f - b.ty);
    const float w01 = (1.0f - b.tx) * b.ty;
    const float w11 = b.tx * b.ty;
    c[0] += w00;
    c[1] += w10;
    c[2] += w01;
    c[3] += w11;
    c[4] += w00 * u.x;
    c[5] += w10 * u.x;
    c[6] += w01 * u.x;
    c[7] += w11 * u.x;
    c[8] += w00 * u.y;
    c[9] += w10 * u.y;
    c[10] += w01 * u.y;
    c[11] += w11 * u.y;
  }
  if (cur >= 0) {
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      float* a = acc + m * W * W + cur;
      atomicAdd(a, c[4 * m + 0]);
      atomicAdd(a + 1, c[4 * m + 1]);
      atomicAdd(a + W, c[4 * m + 2]);
      atomicAdd(a + W + 1, c[4 * m + 3]);
    }
  }
  __syncthreads();
  float* grids[3] = {mass, mass_x, mass_y};
  for (int e = threadIdx.x; e < 3 * W * W; e += kPointThreads) {
    const float val = acc[e];
    if (val == 0.0f) continue;
    const int m = e / (W * W);
    const int node = e - m * W * W;
    const int gx = x_base + node % W;
    const int gy = y_base + node / W;
    if (gx < g && gy < g) atomicAdd(grids[m] + gy * g + gx, val);
  }
}

__global__ __launch_bounds__(kPointThreads) void k_commit(float2* __restrict__ y, const DeviceScalars* sc, int n) {
  const float sx = sc->shift_x, sy = sc->shift_y;
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) {
    const float2 v = y[i];
    y[i] = make_float2(v.x - sx, v.y - sy);
  }
}

// Row transforms of the kernel quadrant.  Row y in [0, F/2] of the wrapped
// (F x F) kernel holds K1 = 1 / (1 + h^2 (dx^2 + dy^2)) and K2 = K1^2 at
// |dx|, |dy| <= G - 1 (src/tsne_neighbors.cpp:878-897), packed as K1 + i K2.
// Both are real and even, so the transform of the packed row is R1 + i R2
// with R1, R2 real and even in kx: only kx in [0, F/2] is kept.
template <int F>
__global__ __launch_bounds__(256) void k_kernel_rows(const DeviceScalars* sc, const float2* __restrict__ tw,
                                                     float2* __restrict__ k_rows) {
  chain_priority();
  using S = Shape<F>;
  __shared__ float2 lds[S::KROWS * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  stage_twiddles<F, S::NT>(tws, tw);
  const float h = sc->h;
  const int row0 = blockIdx.x * S::KROWS;
  for (int e = threadIdx.x; e < S::KROWS * F; e += S::NT) {
    const int r = e / F;
    const int x = e - r * F;
    const int y = row0 + r;
    float2 v = make_float2(0.0f, 0.0f);
    if (y < S::G && x != S::G) {
      const int dx = x < S::G ? x : x - F;
      const float ox = static_cast<float>(dx) * h;
      const float oy = static_cast<float>(y) * h;
      const float q = 1.0f / (1.0f + (ox * ox + oy * oy));
      v = make_float2(q, q * q);
    }
    lds[fft_at<F>(r, x)] = v;
  }
  __syncthreads();
  fft_lds<F, S::KROWS, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KROWS * S::H; e += S::NT) {
    const int r = e / S::H;
    const int kx = e - r * S::H;
    const int y = row0 + r;
    if (y < S::H) k_rows[y * S::H + kx] = lds[fft_at<F>(r, kx)];
  }
}

// Column transforms of the kernel: column kx of the row transforms is even
// in y, so it is rebuilt from rows [0, F/2]; the output is (K1^, K2^) for
// ky in [0, F/2].
template <int F>
__global__ __launch_bounds__(256) void k_kernel_cols(const float2* __restrict__ k_rows,
                                                     const float2* __restrict__ tw, float2* __restrict__ k_hat) {
  chain_priority();
  using S = Shape<F>;
  __shared__ float2 lds[S::KROWS * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  stage_twiddles<F, S::NT>(tws, tw);
  const int col0 = blockIdx.x * S::KROWS;
  for (int e = threadIdx.x; e < S::KROWS * F; e += S::NT) {
    const int y = e / S::KROWS;
    const int c = e - y * S::KROWS;
    const int kx = col0 + c;
    const int ys = y <= F / 2 ? y : F - y;
    lds[fft_at<F>(c, y)] = kx < S::H ? k_rows[ys * S::H + kx] : make_float2(0.0f, 0.0f);
  }
  __syncthreads();
  fft_lds<F, S::KROWS, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KROWS * S::H; e += S::NT) {
    const int ky = e / S::KROWS;
    const int c = e - ky * S::KROWS;
    const int kx = col0 + c;
    if (kx < S::H) k_hat[ky * S::H + kx] = lds[fft_at<F>(c, ky)];
  }
}

// Row transforms of the charges.  Row y < G of A = mass_x + i mass_y and of
// B = mass (zero-padded to F) is transformed; the real-input spectra are
// separated with the Hermitian mirror, Mx[k] = (A[k] + conj A[-k]) / 2 and
// My[k] = (A[k] - conj A[-k]) / 2i, and only kx in [0, F/2] is stored.  The
// packed pair shares one scale (|coordinate| x mass): packing mass with
// mass_x instead would give mass's spectrum the rounding error of one |x|
// times larger.
template <int F>
__global__ __launch_bounds__(256) void k_charge_rows(const float* __restrict__ mass,
                                                     const float* __restrict__ mass_x,
                                                     const float* __restrict__ mass_y,
                                                     const float2* __restrict__ tw, float2* __restrict__ m_rows,
                                                     float2* __restrict__ mx_rows, float2* __restrict__ my_rows) {
  chain_priority();
  using S = Shape<F>;
  __shared__ float2 lds[2 * S::CROWS * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  stage_twiddles<F, S::NT>(tws, tw);
  const int row0 = blockIdx.x * S::CROWS;
  for (int e = threadIdx.x; e < S::CROWS * F; e += S::NT) {
    const int r = e / F;
    const int x = e - r * F;
    const int y = row0 + r;
    float2 a = make_float2(0.0f, 0.0f), b = make_float2(0.0f, 0.0f);
    if (x < S::G && y < S::G) {
      const int at = y * S::G + x;
      a = make_float2(mass_x[at], mass_y[at]);
      b = make_float2(mass[at], 0.0f);
    }
    lds[fft_at<F>(2 * r, x)] = a;
    lds[fft_at<F>(2 * r + 1, x)] = b;
  }
  __syncthreads();
  fft_lds<F, 2 * S::CROWS, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::CROWS * S::H; e += S::NT) {
    const int r = e / S::H;
    const int kx = e - r * S::H;
    const int y = row0 + r;
    if (y >= S::G) continue;
    const float2 a = lds[fft_at<F>(2 * r, kx)];
    const float2 b = conjf2(lds[fft_at<F>(2 * r, ((F - kx) & (F - 1)))]);
    const float2 sum = cadd(a, b);
    const float2 dif = csub(a, b);
    m_rows[y * S::H + kx] = lds[fft_at<F>(2 * r + 1, kx)];
    mx_rows[y * S::H + kx] = cscale(sum, 0.5f);
    my_rows[y * S::H + kx] = make_float2(0.5f * dif.y, -0.5f * dif.x);
  }
}

// Column pass with the spectral products fused between the forward and
// inverse transforms.  For each stored column kx: forward transforms of the
// three charge columns (rows >= G are the zero padding), products with the
// real kernel spectra, inverse transforms of the four potentials, and only
// rows y < G are written (the rest of the padded result is never read).
//   X  = M  K1^ -> q      V1 = M  K2^ -> q2
//   V2 = Mx K2^ -> xq2    Y  = My K2^ -> yq2
template <int F>
__global__ __launch_bounds__(256) void k_conv_cols(const float2* __restrict__ m_rows,
                                                   const float2* __restrict__ mx_rows,
                                                   const float2* __restrict__ my_rows,
                                                   const float2* __restrict__ k_hat,
                                                   const float2* __restrict__ tw, float2* __restrict__ x_rows,
                                                   float2* __restrict__ v1_rows, float2* __restrict__ v2_rows,
                                                   float2* __restrict__ y_rows) {
  chain_priority();
  using S = Shape<F>;
  constexpr int C = S::CCOLS;
  __shared__ float2 lds[4 * C * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  stage_twiddles<F, S::NT>(tws, tw);
  const int col0 = blockIdx.x * C;
  for (int e = threadIdx.x; e < C * F; e += S::NT) {
    const int y = e / C;
    const int c = e - y * C;
    const int kx = col0 + c;
    float2 a = make_float2(0.0f, 0.0f), b = a, d = a;
    if (y < S::G && kx < S::H) {
      const int at = y * S::H + kx;
      a = m_rows[at];
      b = mx_rows[at];
      d = my_rows[at];
    }
    lds[fft_at<F>(0 * C + c, y)] = a;
    lds[fft_at<F>(1 * C + c, y)] = b;
    lds[fft_at<F>(2 * C + c, y)] = d;
  }
  __syncthreads();
  fft_lds<F, 3 * C, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < C * F; e += S::NT) {
    const int ky = e / C;
    const int c = e - ky * C;
    const int kx = col0 + c;
    const int ks = ky <= F / 2 ? ky : F - ky;
    const float2 kk = kx < S::H ? k_hat[ks * S::H + kx] : make_float2(0.0f, 0.0f);
    const float2 m = lds[fft_at<F>(0 * C + c, ky)];
    const float2 mx = lds[fft_at<F>(1 * C + c, ky)];
    const float2 my = lds[fft_at<F>(2 * C + c, ky)];
    lds[fft_at<F>(0 * C + c, ky)] = cscale(m, kk.x);
    lds[fft_at<F>(3 * C + c, ky)] = cscale(m, kk.y);
    lds[fft_at<F>(1 * C + c, ky)] = cscale(mx, kk.y);
    lds[fft_at<F>(2 * C + c, ky)] = cscale(my, kk.y);
  }
  __syncthreads();
  fft_lds<F, 4 * C, S::NT, true, 1>(lds, tws);
  for (int e = threadIdx.x; e < C * S::G; e += S::NT) {
    const int y = e / C;
    const int c = e - y * C;
    const int kx = col0 + c;
    if (kx >= S::H) continue;
    const int at = y * S::H + kx;
    x_rows[at] = lds[fft_at<F>(0 * C + c, y)];
    v2_rows[at] = lds[fft_at<F>(1 * C + c, y)];
    y_rows[at] = lds[fft_at<F>(2 * C + c, y)];
    v1_rows[at] = lds[fft_at<F>(3 * C + c, y)];
  }
}

// Inverse row pass.  The potential rows are spectra of real rows stored for
// kx <= F/2; two of them are packed per transform, U = X + i V1 (q, q2) and
// V = V2 + i Y (xq2, yq2), with the upper half rebuilt from conjugates.  A
// packed transform's rounding error in either part scales with the larger of
// the two, so each pair has a common scale: q2 is never paired with xq2
// (|x| times larger), whose error the read-back y q2 - xq2 would multiply by
// |y| again.  Outputs for x < G are scaled by 1/F^2 and stored as (q2, xq2,
// yq2, q) per node.  The sum
// over points of the bilinear read of q equals sum over nodes of mass * q,
// because read-back and spreading use the same weights; it is accumulated
// here in fp64, and the charge grids are cleared for the next iteration.
template <int F>
__global__ __launch_bounds__(256) void k_inverse_rows(const float2* __restrict__ x_rows,
                                                      const float2* __restrict__ v1_rows,
                                                      const float2* __restrict__ v2_rows,
                                                      const float2* __restrict__ y_rows,
                                                      const float2* __restrict__ tw, float* __restrict__ mass,
                                                      float* __restrict__ mass_x, float* __restrict__ mass_y,
                                                      float4* __restrict__ field, double* __restrict__ partial,
                                                      int n, DeviceScalars* sc) {
  chain_priority();
  using S = Shape<F>;
  __shared__ float2 lds[2 * S::CROWS * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  stage_twiddles<F, S::NT>(tws, tw);
  const int row0 = blockIdx.x * S::CROWS;
  for (int e = threadIdx.x; e < S::CROWS * F; e += S::NT) {
    const int r = e / F;
    const int kx = e - r * F;
    const int y = row0 + r;
    float2 u = make_float2(0.0f, 0.0f), v = u;
    if (y < S::G) {
      const bool low = kx <= F / 2;
      const int at = y * S::H + (low ? kx : F - kx);
      float2 X = x_rows[at], Y = y_rows[at], V1 = v1_rows[at], V2 = v2_rows[at];
      if (!low) {
        X = conjf2(X);
        Y = conjf2(Y);
        V1 = conjf2(V1);
        V2 = conjf2(V2);
      }
      u = cadd(X, mul_i(V1));
      v = cadd(V2, mul_i(Y));
    }
    lds[fft_at<F>(2 * r, kx)] = u;
    lds[fft_at<F>(2 * r + 1, kx)] = v;
  }
  __syncthreads();
  fft_lds<F, 2 * S::CROWS, S::NT, true, 1>(lds, tws);
  const float scale = 1.0f / (static_cast<float>(F) * static_cast<float>(F));
  double acc = 0.0;
  for (int e = threadIdx.x; e < S::CROWS * S::G; e += S::NT) {
    const int r = e / S::G;
    const int x = e - r * S::G;
    const int y = row0 + r;
    if (y >= S::G) continue;
    const float2 u = cscale(lds[fft_at<F>(2 * r, x)], scale);
    const float2 v = cscale(lds[fft_at<F>(2 * r + 1, x)], scale);
    const int at = y * S::G + x;
    field[at] = make_float4(u.y, v.x, v.y, u.x);
    acc += static_cast<double>(mass[at]) * static_cast<double>(u.x);
    mass[at] = 0.0f;
    mass_x[at] = 0.0f;
    mass_y[at] = 0.0f;
  }
  acc = block_sum<S::NT>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = acc;
}

// sum_q and its fp32 reciprocal normaliser (src/tsne_neighbors.cpp:1160-1163).
__global__ __launch_bounds__(256) void k_finalize_sumq(const double* __restrict__ partial, int blocks, int n,
                                                       DeviceScalars* sc) {
  chain_priority();
  double tot = 0.0;
  for (int b = threadIdx.x; b < blocks; b += 256) tot += partial[b];
  tot = block_sum<256>(tot);
  if (threadIdx.x == 0) {
    sc->sum_q = tot;
    const double z = tot - static_cast<double>(n);
    sc->inv_sum_q = static_cast<float>(1.0 / (z > static_cast<double>(FLT_MIN) ? z : static_cast<double>(FLT_MIN)));
  }
}

// ---------------------------------------------------------------------------
// Attraction + read-back + update
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sign0(float v) { return v == 0.0f ? 0.0f : (v < 0.0f ? -1.0f : 1.0f); }

// Bilinear read of one field component (src/tsne_neighbors.cpp:760-781).
__device__ __forceinline__ float blend(float v00, float v10, float v01, float v11, float tx, float ty) {
#pragma clang fp contract(off)
  return (1.0f - tx) * (1.0f - ty) * v00 + tx * (1.0f - ty) * v10 + (1.0f - tx) * ty * v01 + tx * ty * v11;
}

// Attraction, one CSR row per L lanes: col/val streamed in L-wide coalesced
// segments, kUnroll gathers of y_j in flight per lane, a shuffle reduction
// per row, and the row sum written out (src/tsne_neighbors.cpp:985-1012).
// Only this loop is in the kernel, so it keeps few registers and a high
// occupancy, which is what hides the gather latency.
//
// XCD-aware row mapping: workgroups are dispatched round-robin over the
// XCDs, so block b runs on XCD b % xcds.  Each XCD is given one contiguous
// range of row groups; with points numbered cluster-contiguously, the y_j
// that an XCD gathers then stay within about 1/xcds of y and hit its own L2.
constexpr int kUnroll = 8;

template <int L>
__global__ __launch_bounds__(256) void k_attract(const int* __restrict__ row_ptr, const int* __restrict__ col,
                                                 const float* __restrict__ val, const float2* __restrict__ y_cur,
                                                 float2* __restrict__ attr, float exaggeration, int n, int xcds) {
  constexpr int RPB = 256 / L;
  const int lane = threadIdx.x & (L - 1);
  const int groups = (n + RPB - 1) / RPB;
  const int xcd = static_cast<int>(blockIdx.x) % xcds;
  const int blocks_per_xcd = static_cast<int>(gridDim.x) / xcds;
  const int per_xcd = (groups + xcds - 1) / xcds;
  const int g_end = min(groups, (xcd + 1) * per_xcd);
  for (int grp = xcd * per_xcd + static_cast<int>(blockIdx.x) / xcds; grp < g_end; grp += blocks_per_xcd) {
    const int i = grp * RPB + threadIdx.x / L;
    float ax = 0.0f, ay = 0.0f;
    if (i < n) {
      const float2 yi = y_cur[i];
      const int e1 = row_ptr[i + 1];
      // Out-of-row slots point at row i itself with p = 0: no contribution.
      for (int e = row_ptr[i] + lane; e < e1; e += kUnroll * L) {
        int j[kUnroll];
        float p[kUnroll];
#pragma unroll
        for (int q = 0; q < kUnroll; ++q) {
          const int eq = e + q * L;
          const bool ok = eq < e1;
          j[q] = ok ? col[eq] : i;
          p[q] = ok ? val[eq] : 0.0f;
        }
        float2 yj[kUnroll];
#pragma unroll
        for (int q = 0; q < kUnroll; ++q) yj[q] = y_cur[j[q]];
#pragma unroll
        for (int q = 0; q < kUnroll; ++q) {
          const float dx = yi.x - yj[q].x;
          const float dy = yi.y - yj[q].y;
          const float qq = 1.0f / (1.0f + (dx * dx + dy * dy));
          const float c = exaggeration * p[q] * qq;
          ax += c * dx;
          ay += c * dy;
        }
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) {
      ax += __shfl_xor(ax, off, L);
      ay += __shfl_xor(ay, off, L);
    }
    if (lane == 0 && i < n) attr[i] = make_float2(ax, ay);
  }
}

// Point-parallel second half of an iteration: the grid repulsion read back
// at the point (src/tsne_neighbors.cpp:1165-1180) or an exact one, plus the
// attraction, gives the gradient; then the gains/momentum/step-clip update
// (src/tsne_neighbors.cpp:1217-1256), and the bounding box and fp64 mean of
// the new layout for the next iteration's centring and grid.  With the
// bilinear grid y_cur is the centred copy the binning wrote; with the
// interpolation grid it is the stored layout, centred here (the shift of the
// current geometry), and y_out may be the same buffer (each point is read
// before it is written, by the same thread).  At least 5 waves per SIMD (the
// second launch bound): 89 VGPRs instead of 105 with the interpolation
// grid's nine node fields per point in flight, no spills (6 waves spill).
template <int MODE, bool LG>
__global__ __launch_bounds__(kPointThreads, 5) void k_update(const float2* y_cur,
                                                          const float2* __restrict__ attr,
                                                          float2* y_out, float2* __restrict__ update,
                                                          float2* __restrict__ gains, float2* __restrict__ grad_out,
                                                          const float2* __restrict__ exact_rep,
                                                          const float4* __restrict__ field, int g, UpdateParams up,
                                                          BlockStats* __restrict__ partial, DeviceScalars* sc,
                                                          int n) {
#pragma clang fp contract(off)
  chain_priority();
  const DeviceScalars s = *sc;
  BlockStats st = stats_identity();
  const float inv_exact = (MODE == kModeGradientExact)
                              ? static_cast<float>(1.0 / (s.exact_z > static_cast<double>(FLT_MIN)
                                                              ? s.exact_z
                                                              : static_cast<double>(FLT_MIN)))
                              : 0.0f;
  // the gradient of a point at yi (centred for the interpolation grid) with
  // attraction a
  auto gradient_at = [&](int i, float2 yi, float2 a) {
    float gx, gy;
    if (MODE == kModeGradientExact) {
      const float2 r = exact_rep[i];
      gx = r.x * inv_exact;
      gy = r.y * inv_exact;
    } else if (LG) {
      // Interpolation-grid read-back: the 3 x 3 nodes of the point's box with
      // the spreading's Lagrange weights.  Per node the field holds (phi0,
      // xi_x, xi_y); the repulsion is -h sum_a L_a [o_a phi0 + xi] / Z with
      // o_a the point's offset from node a in units of h.
      const LgPoint b = lg_locate(yi.x, yi.y, s);
      float wx[kLgOrder], wy[kLgOrder];
      lg_weights3(b.ux, wx);
      lg_weights3(b.uy, wy);
      const int m = s.lg_nodes;
      const float4* f0 = field + (b.by * kLgOrder) * m + b.bx * kLgOrder;
      const float tx = 3.0f * b.ux;
      const float ty = 3.0f * b.uy;
      float fx = 0.0f, fy = 0.0f;
#pragma unroll
      for (int a = 0; a < kLgOrder; ++a) {
        const float oy = ty - (static_cast<float>(a) + 0.5f);
#pragma unroll
        for (int c = 0; c < kLgOrder; ++c) {
          const float ox = tx - (static_cast<float>(c) + 0.5f);
          const float w = wy[a] * wx[c];
          const float4 f = f0[a * m + c];
          fx += w * (ox * f.x + f.y);
          fy += w * (oy * f.x + f.z);
        }
      }
      const float scale = s.lg_node_h * s.inv_sum_q;
      gx = -fx * scale;
      gy = -fy * scale;
    } else {
      const Bilinear b = locate(yi.x, yi.y, s, g);
      const int a00 = b.y0 * g + b.x0;
      const float4 f00 = field[a00];
      const float4 f10 = field[a00 + 1];
      const float4 f01 = field[a00 + g];
      const float4 f11 = field[a00 + g + 1];
      const float q2 = blend(f00.x, f10.x, f01.x, f11.x, b.tx, b.ty);
      const float xq2 = blend(f00.y, f10.y, f01.y, f11.y, b.tx, b.ty);
      const float yq2 = blend(f00.z, f10.z, f01.z, f11.z, b.tx, b.ty);
      gx = -(yi.x * q2 - xq2) * s.inv_sum_q;
      gy = -(yi.y * q2 - yq2) * s.inv_sum_q;
    }
    gx += a.x;
    gy += a.y;
    return make_float2(gx, gy);
  };
  // the update of point i from its gradient, gains and update
  auto apply = [&](int i, float2 yi, float gx, float gy, float2 gn, float2 u) {
    if (MODE != kModeUpdate) {
      grad_out[i] = make_float2(gx, gy);
      return;
    }
    if (sign0(u.x) != sign0(gx)) {
      gn.x += 0.2f;
    } else {
      gn.x = gn.x * 0.8f + up.min_gain;
    }
    if (gn.x < up.min_gain) gn.x = up.min_gain;
    u.x = up.momentum * u.x - up.learning_rate * gn.x * gx;
    float norm_sq = 0.0f;
    norm_sq += u.x * u.x;
    if (sign0(u.y) != sign0(gy)) {
      gn.y += 0.2f;
    } else {
      gn.y = gn.y * 0.8f + up.min_gain;
    }
    if (gn.y < up.min_gain) gn.y = up.min_gain;
    u.y = up.momentum * u.y - up.learning_rate * gn.y * gy;
    norm_sq += u.y * u.y;
    float scale = 1.0f;
    if (up.clip && norm_sq > up.max_step_norm * up.max_step_norm) {
      scale = up.max_step_norm / sqrtf(fmaxf(norm_sq, FLT_MIN));
    }
    u.x *= scale;
    u.y *= scale;
    const float2 yn = make_float2(yi.x + u.x, yi.y + u.y);
    gains[i] = gn;
    update[i] = u;
    y_out[i] = yn;
    st.min_x = fminf(st.min_x, yn.x);
    st.max_x = fmaxf(st.max_x, yn.x);
    st.min_y = fminf(st.min_y, yn.y);
    st.max_y = fmaxf(st.max_y, yn.y);
    st.sum_x += static_cast<double>(yn.x);
    st.sum_y += static_cast<double>(yn.y);
  };
  // Two points per thread and pass: every load of both (the interpolation
  // grid's nine node fields included) is issued before either is stored,
  // so their latencies overlap (y_out may be y_cur: each point reads its own
  // entries before they are written)
  const int stride = static_cast<int>(gridDim.x) * kPointThreads;
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += 2 * stride) {
    const int j = i + stride < n ? i + stride : i;
    float2 yi = y_cur[i];
    float2 yj = y_cur[j];
    if (LG && MODE != kModeGradientExact) {
      yi = make_float2(yi.x - s.shift_x, yi.y - s.shift_y);
      yj = make_float2(yj.x - s.shift_x, yj.y - s.shift_y);
    }
    const float2 ai = attr[i];
    const float2 aj = attr[j];
    float2 gni = make_float2(0.0f, 0.0f), ui = gni, gnj = gni, uj = gni;
    if (MODE == kModeUpdate) {
      gni = gains[i];
      ui = update[i];
      gnj = gains[j];
      uj = update[j];
    }
    const float2 gi = gradient_at(i, yi, ai);
    const float2 gj = gradient_at(j, yj, aj);
    apply(i, yi, gi.x, gi.y, gni, ui);
    if (j != i) apply(j, yj, gj.x, gj.y, gnj, uj);
  }
  if (MODE == kModeUpdate) publish_stats<kPointThreads>(st, partial);
}

// ---------------------------------------------------------------------------
// Exact O(n^2) terms
// ---------------------------------------------------------------------------
// rep_i = -sum_{j != i} q_ij^2 (y_i - y_j) with q in fp32, and the normaliser
// sum_{i != j} q_ij in fp64 (src/tsne_neighbors.cpp:1024-1048).
__global__ __launch_bounds__(256) void k_exact_rep(const float2* __restrict__ y, int n, float2* __restrict__ rep,
                                                   double* __restrict__ partial, DeviceScalars* sc) {
  __shared__ float2 tile[256];
  const int i = blockIdx.x * 256 + threadIdx.x;
  const float2 yi = i < n ? y[i] : make_float2(0.0f, 0.0f);
  float rx = 0.0f, ry = 0.0f;
  double z = 0.0;
  for (int b0 = 0; b0 < n; b0 += 256) {
    const int j = b0 + threadIdx.x;
    tile[threadIdx.x] = j < n ? y[j] : make_float2(0.0f, 0.0f);
    __syncthreads();
    const int lim = min(256, n - b0);
    if (i < n) {
      for (int t = 0; t < lim; ++t) {
        if (b0 + t == i) continue;
        const float2 yj = tile[t];
        const float dx = yi.x - yj.x;
        const float dy = yi.y - yj.y;
        const float q = 1.0f / (1.0f + (dx * dx + dy * dy));
        z += static_cast<double>(q);
        const float c = -(q * q);
        rx += c * dx;
        ry += c * dy;
      }
    }
    __syncthreads();
  }
  if (i < n) rep[i] = make_float2(rx, ry);
  z = block_sum<256>(z);
  if (threadIdx.x == 0) partial[blockIdx.x] = z;
}

__global__ __launch_bounds__(256) void k_finalize_exact(const double* __restrict__ partial, int blocks,
                                                        DeviceScalars* sc) {
  double tot = 0.0;
  for (int b = threadIdx.x; b < blocks; b += 256) tot += partial[b];
  tot = block_sum<256>(tot);
  if (threadIdx.x == 0) sc->exact_z = tot;
}

// sum_{i != j} 1 / (1 + |y_i - y_j|^2) with the squared distance in fp32 and
// the reciprocal in fp64, as the KL's normaliser (src/tsne_neighbors.cpp:958-983).
__global__ __launch_bounds__(256) void k_exact_z_double(const float2* __restrict__ y, int n,
                                                        double* __restrict__ partial) {
  __shared__ float2 tile[256];
  const int i = blockIdx.x * 256 + threadIdx.x;
  const float2 yi = i < n ? y[i] : make_float2(0.0f, 0.0f);
  double z = 0.0;
  for (int b0 = 0; b0 < n; b0 += 256) {
    const int j = b0 + threadIdx.x;
    tile[threadIdx.x] = j < n ? y[j] : make_float2(0.0f, 0.0f);
    __syncthreads();
    const int lim = min(256, n - b0);
    if (i < n) {
      for (int t = 0; t < lim; ++t) {
        if (b0 + t == i) continue;
        const float2 yj = tile[t];
        float r2 = 0.0f;
        const float dx = yi.x - yj.x;
        r2 += dx * dx;
        const float dy = yi.y - yj.y;
        r2 += dy * dy;
        z += 1.0 / (1.0 + static_cast<double>(r2));
      }
    }
    __syncthreads();
  }
  z = block_sum<256>(z);
  if (threadIdx.x == 0) partial[blockIdx.x] = z;
}

// Per-row KL terms (src/tsne_neighbors.cpp:1258-1285): each row's sum in
// fp64, written to row_out when given, and the rows' block partial sums.
__global__ __launch_bounds__(256) void k_kl_rows(const int* __restrict__ row_ptr, const int* __restrict__ col,
                                                 const float* __restrict__ val, const float2* __restrict__ y,
                                                 int n, double sum_q, double* __restrict__ partial,
                                                 double* __restrict__ row_out) {
  double acc = 0.0;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float2 yi = y[i];
    double row = 0.0;
    for (int e = row_ptr[i]; e < row_ptr[i + 1]; ++e) {
      const float2 yj = y[col[e]];
      float r2 = 0.0f;
      const float dx = yi.x - yj.x;
      r2 += dx * dx;
      const float dy = yi.y - yj.y;
      r2 += dy * dy;
      const double p = static_cast<double>(val[e]);
      const double q = (1.0 / (1.0 + static_cast<double>(r2))) / sum_q;
      row += p * log((p + 1e-9) / (q + 1e-9));
    }
    if (row_out != nullptr) row_out[i] = row;
    acc += row;
  }
  acc = block_sum<256>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = acc;
}

// ---------------------------------------------------------------------------
// Locality renumbering
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned int spread_bits16(unsigned int v) {
  v &= 0xffffu;
  v = (v | (v << 8)) & 0x00ff00ffu;
  v = (v | (v << 4)) & 0x0f0f0f0fu;
  v = (v | (v << 2)) & 0x33333333u;
  v = (v | (v << 1)) & 0x55555555u;
  return v;
}

// Sort key of each point: its connected component in the high 32 bits (so
// components are numbered contiguously), then the 32-bit Morton code of its
// position on a 65536^2 lattice over the bounding box of the layout (stored
// values minus the pending centring shift).
__global__ __launch_bounds__(kPointThreads) void k_morton_keys(const float2* __restrict__ y, const DeviceScalars* sc,
                                                               int n, const int* __restrict__ component,
                                                               const int* __restrict__ perm,
                                                               unsigned long long* __restrict__ keys,
                                                               int* __restrict__ idx) {
  const DeviceScalars s = *sc;
  const float sx = fmaxf(s.max_x - s.min_x, 1e-30f);
  const float sy = fmaxf(s.max_y - s.min_y, 1e-30f);
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) {
    const float2 v = y[i];
    const float ux = fminf(fmaxf((v.x - s.shift_x - s.min_x) / sx, 0.0f), 1.0f);
    const float uy = fminf(fmaxf((v.y - s.shift_y - s.min_y) / sy, 0.0f), 1.0f);
    const unsigned int qx = static_cast<unsigned int>(ux * 65535.0f);
    const unsigned int qy = static_cast<unsigned int>(uy * 65535.0f);
    const unsigned long long comp = static_cast<unsigned long long>(component[perm[i]]);
    keys[i] = (comp << 32) | (spread_bits16(qx) | (spread_bits16(qy) << 1));
    idx[i] = i;
  }
}

// Estimated number of (row block, column tile) runs that P would have in a
// candidate numbering, counted on the 1024 x 4096 shape whichever shape the
// session's tiles have (a proxy for locality, compared between two
// numberings): every step-th block of kTileRows new rows is taken,
// the distinct column tiles of its entries are marked in an LDS bitmap
// (`words` 32-bit words) and counted.  order maps new -> old rows and map old
// -> new columns; null pointers stand for the identity (the current
// numbering).  One wave per row, 16 waves per workgroup; a lane marks a tile
// only when it differs from the last one it marked (a row's columns mostly
// fall in a few tiles, and the bitmap's few words took every lane's LDS
// atomic in turn: 0.7 ms per estimate at 1M points).
constexpr int kEstimateThreads = 1024;
__global__ __launch_bounds__(kEstimateThreads) void k_tile_estimate(const int* __restrict__ row_ptr,
                                                                    const int* __restrict__ col,
                                                                    const int* __restrict__ order,
                                                                    const int* __restrict__ map, int n, int step,
                                                                    int words, unsigned long long* __restrict__ out) {
  extern __shared__ unsigned int bits[];
  __shared__ unsigned int block_count;
  const int r0 = static_cast<int>(blockIdx.x) * step * kTileRows;
  if (r0 >= n) return;  // whole block
  for (int w = threadIdx.x; w < words; w += kEstimateThreads) bits[w] = 0u;
  if (threadIdx.x == 0) block_count = 0u;
  __syncthreads();
  const int r1 = min(n, r0 + kTileRows);
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  int last = -1;
  for (int q = r0 + wave; q < r1; q += kEstimateThreads / kWave) {
    const int i = order != nullptr ? order[q] : q;
    const int e1 = row_ptr[i + 1];
    for (int e = row_ptr[i] + lane; e < e1; e += kWave) {
      const int j = map != nullptr ? map[col[e]] : col[e];
      const int t = j / kTileCols;
      if (t != last) {
        atomicOr(&bits[t >> 5], 1u << (t & 31));
        last = t;
      }
    }
  }
  __syncthreads();
  unsigned int c = 0u;
  for (int w = threadIdx.x; w < words; w += kEstimateThreads) c += static_cast<unsigned int>(__popc(bits[w]));
  if (c != 0u) atomicAdd(&block_count, c);
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(out, static_cast<unsigned long long>(block_count));
}

__global__ __launch_bounds__(kPointThreads) void k_label_init(int* __restrict__ label, int n) {
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) label[i] = i;
}

// One min-label propagation sweep (a wave per row) followed in the same pass
// by pointer jumping.  Labels only decrease and always name a member of the
// same component, so concurrent reads of partly updated labels are safe.
__global__ __launch_bounds__(256) void k_label_step(const int* __restrict__ row_ptr, const int* __restrict__ col,
                                                    int* label, int* changed, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int i = (blockIdx.x * 256 + threadIdx.x) / kWave; i < n; i += gridDim.x * (256 / kWave)) {
    int m = label[i];
    for (int e = row_ptr[i] + lane; e < row_ptr[i + 1]; e += kWave) m = min(m, label[col[e]]);
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off, kWave));
    if (lane == 0) {
      m = min(m, label[m]);
      if (m < label[i]) {
        label[i] = m;
        *changed = 1;
      }
    }
  }
}

__global__ __launch_bounds__(kPointThreads) void k_apply_order(const int* __restrict__ order, int n,
                                                               const int* __restrict__ perm_old,
                                                               int* __restrict__ perm_new, int* __restrict__ map,
                                                               const float2* __restrict__ y_old,
                                                               float2* __restrict__ y_new,
                                                               const float2* __restrict__ u_old,
                                                               float2* __restrict__ u_new,
                                                               const float2* __restrict__ g_old,
                                                               float2* __restrict__ g_new,
                                                               const int* __restrict__ rp_old, int* __restrict__ len) {
  for (int q = blockIdx.x * kPointThreads + threadIdx.x; q <= n; q += gridDim.x * kPointThreads) {
    if (q == n) {
      len[n] = 0;
      continue;
    }
    const int r = order[q];
    perm_new[q] = perm_old[r];
    map[r] = q;
    y_new[q] = y_old[r];
    u_new[q] = u_old[r];
    g_new[q] = g_old[r];
    len[q] = rp_old[r + 1] - rp_old[r];
  }
}

// One wave per new row; columns are renamed to the new numbering.
__global__ __launch_bounds__(256) void k_copy_rows(const int* __restrict__ order, const int* __restrict__ map,
                                                   const int* __restrict__ rp_old, const int* __restrict__ col_old,
                                                   const float* __restrict__ val_old, const int* __restrict__ rp_new,
                                                   int* __restrict__ col_new, float* __restrict__ val_new, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int q = (blockIdx.x * 256 + threadIdx.x) / kWave; q < n; q += gridDim.x * (256 / kWave)) {
    const int r = order[q];
    const int b = rp_old[r];
    const int len = rp_old[r + 1] - b;
    const int d = rp_new[q];
    for (int t = lane; t < len; t += kWave) {
      col_new[d + t] = map[col_old[b + t]];
      val_new[d + t] = val_old[b + t];
    }
  }
}

__global__ __launch_bounds__(kPointThreads) void k_invert(const int* __restrict__ perm, int* __restrict__ inv, int n) {
  for (int q = blockIdx.x * kPointThreads + threadIdx.x; q < n; q += gridDim.x * kPointThreads) inv[perm[q]] = q;
}

__global__ __launch_bounds__(kPointThreads) void k_gather2(const float2* __restrict__ src,
                                                           const int* __restrict__ idx, float2* __restrict__ dst,
                                                           int n) {
  for (int i = blockIdx.x * kPointThreads + threadIdx.x; i < n; i += gridDim.x * kPointThreads) dst[i] = src[idx[i]];
}

template <int F>
hipError_t grid_fft_launch(int which, GridBuffers& gb, const DeviceScalars* sc_const, DeviceScalars* sc,
                           const float2* tw, int n, hipStream_t stream) {
  using S = Shape<F>;
  switch (which) {
    case 0:
      k_kernel_rows<F><<<(S::H + S::KROWS - 1) / S::KROWS, S::NT, 0, stream>>>(sc_const, tw, gb.k_rows);
      break;
    case 1:
      k_kernel_cols<F><<<(S::H + S::KROWS - 1) / S::KROWS, S::NT, 0, stream>>>(gb.k_rows, tw, gb.k_hat);
      break;
    case 2:
      k_charge_rows<F><<<(S::G + S::CROWS - 1) / S::CROWS, S::NT, 0, stream>>>(
          gb.mass, gb.mass_x, gb.mass_y, tw, gb.m_rows, gb.mx_rows, gb.my_rows);
      break;
    case 3:
      k_conv_cols<F><<<(S::H + S::CCOLS - 1) / S::CCOLS, S::NT, 0, stream>>>(
          gb.m_rows, gb.mx_rows, gb.my_rows, gb.k_hat, tw, gb.x_rows, gb.v1_rows, gb.v2_rows, gb.y_rows);
      break;
    case 4:
      k_inverse_rows<F><<<(S::G + S::CROWS - 1) / S::CROWS, S::NT, 0, stream>>>(
          gb.x_rows, gb.v1_rows, gb.v2_rows, gb.y_rows, tw, gb.mass, gb.mass_x, gb.mass_y, gb.field,
          gb.sumq_partial, n, sc);
      k_finalize_sumq<<<1, 256, 0, stream>>>(gb.sumq_partial, (S::G + S::CROWS - 1) / S::CROWS, n, sc);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t grid_fft_dispatch(int which, GridBuffers& gb, DeviceScalars* sc, const float2* tw, int n,
                             hipStream_t stream) {
  switch (2 * gb.g) {
    case 64: return grid_fft_launch<64>(which, gb, sc, sc, tw, n, stream);
    case 128: return grid_fft_launch<128>(which, gb, sc, sc, tw, n, stream);
    case 256: return grid_fft_launch<256>(which, gb, sc, sc, tw, n, stream);
    case 512: return grid_fft_launch<512>(which, gb, sc, sc, tw, n, stream);
    case 1024: return grid_fft_launch<1024>(which, gb, sc, sc, tw, n, stream);
    case 2048: return grid_fft_launch<2048>(which, gb, sc, sc, tw, n, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int L>
hipError_t attract_launch(const Csr& p, const float2* y_cur, float2* attr, float exaggeration, int xcds,
                          hipStream_t stream) {
  constexpr int RPB = 256 / L;
  const int needed = (p.n + RPB - 1) / RPB;
  // a whole number of blocks per XCD
  const int blocks = std::max(xcds, (std::min(needed, 4096) / xcds) * xcds);
  k_attract<L><<<blocks, 256, 0, stream>>>(p.row_ptr, p.col, p.val, y_cur, attr, exaggeration, p.n, xcds);
  return hipGetLastError();
}

template <int MODE>
hipError_t update_launch(const float2* y_cur, const float2* attr, float2* y_out, float2* update, float2* gains,
                         float2* grad_out, const float2* exact_rep, const GridBuffers& gb, const UpdateParams& up,
                         BlockStats* partial, DeviceScalars* sc, int n, hipStream_t stream,
                         const float4* interp_field, hipEvent_t done) {
  const int blocks = reduce_blocks_for(n);
  if (interp_field != nullptr && MODE != kModeGradientExact) {
    if (done != nullptr) {
      hipExtLaunchKernelGGL(k_update<MODE, true>, dim3(blocks), dim3(kPointThreads), 0, stream, nullptr, done, 0,
                            y_cur, attr, y_out, update, gains, grad_out, exact_rep, interp_field, gb.g, up, partial,
                            sc, n);
    } else {
      k_update<MODE, true><<<blocks, kPointThreads, 0, stream>>>(y_cur, attr, y_out, update, gains, grad_out,
                                                                 exact_rep, interp_field, gb.g, up, partial, sc, n);
    }
  } else if (done != nullptr) {
    hipExtLaunchKernelGGL(k_update<MODE, false>, dim3(blocks), dim3(kPointThreads), 0, stream, nullptr, done, 0,
                          y_cur, attr, y_out, update, gains, grad_out, exact_rep, gb.field, gb.g, up, partial, sc,
                          n);
  } else {
    k_update<MODE, false><<<blocks, kPointThreads, 0, stream>>>(y_cur, attr, y_out, update, gains, grad_out,
                                                                exact_rep, gb.field, gb.g, up, partial, sc, n);
  }
  return hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
hipError_t launch_row_search(const int* idx_cm, const void* dist_cm, bool dist_is_double, int n, int k,
                             int index_offset, float log_perplexity, float* p_cond, std::uint64_t* keys,
                             float* vals, int key_bits, double* mass_partial, int mass_blocks, DeviceScalars* sc,
                             hipStream_t stream) {
  const std::size_t lds = static_cast<std::size_t>(k) * kSearchThreads * sizeof(float);
  if (dist_is_double) {
    k_row_search<double><<<mass_blocks, kSearchThreads, lds, stream>>>(
        idx_cm, static_cast<const double*>(dist_cm), n, k, index_offset, log_perplexity, p_cond, keys, vals,
        key_bits, mass_partial, sc);
  } else {
    k_row_search<float><<<mass_blocks, kSearchThreads, lds, stream>>>(
        idx_cm, static_cast<const float*>(dist_cm), n, k, index_offset, log_perplexity, p_cond, keys, vals,
        key_bits, mass_partial, sc);
  }
  return hipGetLastError();
}

hipError_t launch_finalize_mass(const double* mass_partial, int blocks, DeviceScalars* sc, hipStream_t stream) {
  k_finalize_mass<<<1, 256, 0, stream>>>(mass_partial, blocks, sc);
  return hipGetLastError();
}

hipError_t sort_edges(void* temp, std::size_t& temp_bytes, const std::uint64_t* keys_in, std::uint64_t* keys_out,
                      const float* vals_in, float* vals_out, std::size_t count, int end_bit, hipStream_t stream) {
  return rocprim::radix_sort_pairs(temp, temp_bytes, keys_in, keys_out, vals_in, vals_out, count, 0u,
                                   static_cast<unsigned int>(end_bit), stream);
}

hipError_t launch_mark_heads(const std::uint64_t* keys, std::size_t count, int* heads, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const unsigned int blocks = static_cast<unsigned int>((count + 255) / 256);
  k_mark_heads<<<blocks, 256, 0, stream>>>(keys, count, heads);
  return hipGetLastError();
}

hipError_t scan_heads(void* temp, std::size_t& temp_bytes, const int* heads, int* pos, std::size_t count,
                      hipStream_t stream) {
  return rocprim::exclusive_scan(temp, temp_bytes, heads, pos, 0, count, rocprim::plus<int>(), stream);
}

hipError_t launch_compact(const std::uint64_t* keys, const float* vals, const int* heads, const int* pos,
                          std::size_t count, int key_bits, int n, const DeviceScalars* sc, int* row_ptr, int* col,
                          float* val, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const unsigned int blocks = static_cast<unsigned int>((count + 255) / 256);
  k_compact<<<blocks, 256, 0, stream>>>(keys, vals, heads, pos, count, key_bits, n, sc, row_ptr, col, val);
  return hipGetLastError();
}

int reduce_blocks_for(int n) {
  const int needed = (n + kPointThreads - 1) / kPointThreads;
  return needed < 1 ? 1 : (needed < 2048 ? needed : 2048);
}

hipError_t launch_stats(const float2* y, int n, int g, int center, BlockStats* partial, DeviceScalars* sc,
                        hipStream_t stream) {
  const int blocks = reduce_blocks_for(n);
  k_stats<<<blocks, kPointThreads, 0, stream>>>(y, n, g, center, partial, sc);
  k_finalize_stats<<<1, 256, 0, stream>>>(partial, blocks, sc, n, g, center, nullptr);
  return hipGetLastError();
}

hipError_t launch_finalize_stats(const BlockStats* partial, int n, int g, DeviceScalars* sc,
                                 unsigned long long* box_out, hipStream_t stream) {
  k_finalize_stats<<<1, 256, 0, stream>>>(partial, reduce_blocks_for(n), sc, n, g, 1, box_out);
  return hipGetLastError();
}

hipError_t launch_bin_count(const float2* y_stored, float2* y_cur, const DeviceScalars* sc, GridBuffers& gb, int n,
                            hipStream_t stream) {
  const int ta = tiles_per_axis(gb.g);
  const int blocks = std::min(reduce_blocks_for(n), 1024);
  k_bin_count<<<blocks, kPointThreads, 0, stream>>>(y_stored, y_cur, sc, gb.tile_count, n, gb.g, ta);
  return hipGetLastError();
}

hipError_t launch_bin_plan(GridBuffers& gb, DeviceScalars* sc, hipStream_t stream) {
  const int ta = tiles_per_axis(gb.g);
  k_bin_plan<<<1, kPlanThreads, 0, stream>>>(gb.tile_count, gb.tile_cursor, gb.items, sc, ta * ta);
  return hipGetLastError();
}

hipError_t launch_bin_scatter(const float2* y_cur, const DeviceScalars* sc, GridBuffers& gb, int n,
                              hipStream_t stream) {
  const int ta = tiles_per_axis(gb.g);
  constexpr int kBatch = kPointThreads * kScatterPerThread;
  const int needed = (n + kBatch - 1) / kBatch;
  const int blocks = std::max(1, std::min(needed, 1024));
  k_bin_scatter<<<blocks, kPointThreads, 0, stream>>>(y_cur, sc, gb.tile_cursor, gb.binned, n, gb.g, ta);
  return hipGetLastError();
}

hipError_t launch_spread_tiles(const DeviceScalars* sc, GridBuffers& gb, int n, hipStream_t stream) {
  const int ta = tiles_per_axis(gb.g);
  k_spread_tiles<<<max_spread_items(n, gb.g), kPointThreads, 0, stream>>>(gb.binned, gb.items, sc, gb.mass,
                                                                          gb.mass_x, gb.mass_y, gb.g, ta);
  return hipGetLastError();
}

hipError_t launch_kernel_rows(GridBuffers& gb, const DeviceScalars* sc, const float2* tw, hipStream_t stream) {
  return grid_fft_dispatch(0, gb, const_cast<DeviceScalars*>(sc), tw, 0, stream);
}
hipError_t launch_kernel_cols(GridBuffers& gb, const float2* tw, hipStream_t stream) {
  return grid_fft_dispatch(1, gb, nullptr, tw, 0, stream);
}
hipError_t launch_charge_rows(GridBuffers& gb, const float2* tw, hipStream_t stream) {
  return grid_fft_dispatch(2, gb, nullptr, tw, 0, stream);
}
hipError_t launch_conv_cols(GridBuffers& gb, const float2* tw, hipStream_t stream) {
  return grid_fft_dispatch(3, gb, nullptr, tw, 0, stream);
}
hipError_t launch_inverse_rows(GridBuffers& gb, const float2* tw, int n, DeviceScalars* sc, hipStream_t stream) {
  return grid_fft_dispatch(4, gb, sc, tw, n, stream);
}

hipError_t launch_attract(const Csr& p, const float2* y_cur, float2* attr, float exaggeration, int lanes_per_row,
                          int xcds, hipStream_t stream) {
  switch (lanes_per_row) {
    case 8: return attract_launch<8>(p, y_cur, attr, exaggeration, xcds, stream);
    case 16: return attract_launch<16>(p, y_cur, attr, exaggeration, xcds, stream);
    case 32: return attract_launch<32>(p, y_cur, attr, exaggeration, xcds, stream);
    case 64: return attract_launch<64>(p, y_cur, attr, exaggeration, xcds, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_update(int mode, const float2* y_cur, const float2* attr, float2* y_out, float2* update,
                         float2* gains, float2* grad_out, const float2* exact_rep, const GridBuffers& gb,
                         const UpdateParams& up, BlockStats* partial, DeviceScalars* sc, int n, hipStream_t stream,
                         const float4* interp_field, hipEvent_t done) {
  switch (mode) {
    case kModeUpdate:
      return update_launch<kModeUpdate>(y_cur, attr, y_out, update, gains, grad_out, exact_rep, gb, up, partial, sc,
                                        n, stream, interp_field, done);
    case kModeGradientGrid:
      return update_launch<kModeGradientGrid>(y_cur, attr, y_out, update, gains, grad_out, exact_rep, gb, up,
                                              partial, sc, n, stream, interp_field, done);
    case kModeGradientExact:
      return update_launch<kModeGradientExact>(y_cur, attr, y_out, update, gains, grad_out, exact_rep, gb, up,
                                               partial, sc, n, stream, nullptr, done);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_commit(float2* y, const DeviceScalars* sc, int n, hipStream_t stream) {
  k_commit<<<reduce_blocks_for(n), kPointThreads, 0, stream>>>(y, sc, n);
  return hipGetLastError();
}

hipError_t renumber_temp_bytes(int n, std::size_t& bytes) {
  std::size_t sort_b = 0, scan_b = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, sort_b, static_cast<const unsigned long long*>(nullptr),
                                           static_cast<unsigned long long*>(nullptr),
                                           static_cast<const int*>(nullptr), static_cast<int*>(nullptr),
                                           static_cast<std::size_t>(n), 0u, 64u);
  if (e != hipSuccess) return e;
  e = rocprim::exclusive_scan(nullptr, scan_b, static_cast<const int*>(nullptr), static_cast<int*>(nullptr), 0,
                              static_cast<std::size_t>(n) + 1, rocprim::plus<int>());
  bytes = std::max(sort_b, scan_b);
  return e;
}

hipError_t launch_morton_keys(const float2* y, const DeviceScalars* sc, int n, Renumber& r, hipStream_t stream) {
  k_morton_keys<<<reduce_blocks_for(n), kPointThreads, 0, stream>>>(y, sc, n, r.component, r.perm, r.keys_in,
                                                                    r.idx_in);
  return hipGetLastError();
}

hipError_t sort_morton(Renumber& r, int n, hipStream_t stream) {
  std::size_t tb = r.temp_bytes;
  return rocprim::radix_sort_pairs(r.temp, tb, r.keys_in, r.keys_out, r.idx_in, r.order,
                                   static_cast<std::size_t>(n), 0u, static_cast<unsigned int>(r.key_bits),
                                   stream);
}

hipError_t launch_label_init(int* label, int n, hipStream_t stream) {
  k_label_init<<<reduce_blocks_for(n), kPointThreads, 0, stream>>>(label, n);
  return hipGetLastError();
}

hipError_t launch_label_step(const Csr& p, int* label, int* changed, hipStream_t stream) {
  const int blocks = std::max(1, std::min((p.n + 3) / 4, 8192));
  k_label_step<<<blocks, 256, 0, stream>>>(p.row_ptr, p.col, label, changed, p.n);
  return hipGetLastError();
}

hipError_t launch_apply_order(const Renumber& r, int n, const int* perm_old, int* perm_new, const float2* y_old,
                              float2* y_new, const float2* u_old, float2* u_new, const float2* g_old, float2* g_new,
                              const int* rp_old, hipStream_t stream) {
  k_apply_order<<<reduce_blocks_for(n + 1), kPointThreads, 0, stream>>>(r.order, n, perm_old, perm_new, r.map,
                                                                        y_old, y_new, u_old, u_new, g_old, g_new,
                                                                        rp_old, r.len);
  return hipGetLastError();
}

hipError_t scan_row_lengths(Renumber& r, int n, int* rp_new, hipStream_t stream) {
  std::size_t tb = r.temp_bytes;
  return rocprim::exclusive_scan(r.temp, tb, r.len, rp_new, 0, static_cast<std::size_t>(n) + 1,
                                 rocprim::plus<int>(), stream);
}

hipError_t launch_copy_rows(const Renumber& r, int n, const Csr& src, Csr& dst, hipStream_t stream) {
  const int blocks = std::max(1, std::min((n + 3) / 4, 8192));
  k_copy_rows<<<blocks, 256, 0, stream>>>(r.order, r.map, src.row_ptr, src.col, src.val, dst.row_ptr, dst.col,
                                          dst.val, n);
  return hipGetLastError();
}

hipError_t launch_tile_estimate(const Csr& p, const int* order, const int* map, int step,
                                unsigned long long* out, hipStream_t stream) {
  const int tiles = (p.n + kTileCols - 1) / kTileCols;
  const int words = (tiles + 31) / 32;
  const int row_blocks = (p.n + kTileRows - 1) / kTileRows;
  const int blocks = (row_blocks + step - 1) / step;
  const std::size_t lds = static_cast<std::size_t>(words) * sizeof(unsigned int);
  if (lds > 60 * 1024) return hipErrorInvalidValue;
  k_tile_estimate<<<blocks, kEstimateThreads, lds, stream>>>(p.row_ptr, p.col, order, map, p.n, step, words, out);
  return hipGetLastError();
}

hipError_t launch_invert(const int* perm, int* inv, int n, hipStream_t stream) {
  k_invert<<<reduce_blocks_for(n), kPointThreads, 0, stream>>>(perm, inv, n);
  return hipGetLastError();
}

hipError_t launch_gather2(const float2* src, const int* idx, float2* dst, int n, hipStream_t stream) {
  k_gather2<<<reduce_blocks_for(n), kPointThreads, 0, stream>>>(src, idx, dst, n);
  return hipGetLastError();
}

int exact_blocks_for(int n) { return (n + 255) / 256; }

hipError_t launch_exact_repulsion(const float2* y, int n, float2* rep, double* z_partial, DeviceScalars* sc,
                                  hipStream_t stream) {
  k_exact_rep<<<exact_blocks_for(n), 256, 0, stream>>>(y, n, rep, z_partial, sc);
  k_finalize_exact<<<1, 256, 0, stream>>>(z_partial, exact_blocks_for(n), sc);
  return hipGetLastError();
}

hipError_t launch_exact_z_double(const float2* y, int n, double* z_partial, hipStream_t stream) {
  k_exact_z_double<<<exact_blocks_for(n), 256, 0, stream>>>(y, n, z_partial);
  return hipGetLastError();
}

hipError_t launch_kl_rows(const Csr& p, const float2* y, double sum_q, double* partial, int blocks,
                          hipStream_t stream, double* row_out) {
  k_kl_rows<<<blocks, 256, 0, stream>>>(p.row_ptr, p.col, p.val, y, p.n, sum_q, partial, row_out);
  return hipGetLastError();
}

}  // namespace fehip
