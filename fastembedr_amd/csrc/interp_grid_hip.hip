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
//   k_lg_order_keys + radix sort
//                         every few iterations: the spread order, points
//                         sorted by the Morton code of their position
//   k_lg_spread           per workgroup, 1024 consecutive points of the
//                         spread order: each point centred and located, its
//                         21 power sums (below) summed over the runs of one
//                         box among a wave's 64 consecutive points (DPP
//                         segmented scan), each run's sums added into the
//                         box's slot of an LDS table keyed by box, each
//                         occupied slot stored to the next entry of its box
//   k_lg_kernel_rows/cols spectra of K, K1 (real, even) and Kv (imaginary,
//                         odd in its own axis), a quadrant each, two real
//                         sequences per complex transform
//   k_lg_box_chunks       every box's entries summed in chunks of 32, each
//                         chunk's sum stored over its first entry
//   k_lg_charge_rows      one workgroup per node row: the chunk sums (and
//                         the rare straggler sums) of each box of its box
//                         row summed, combined into the row's node moments
//                         (m2 stored), then m0 + i m1x and m1y per complex
//                         row transform, half spectra kept
//   k_lg_conv_cols        forward column transforms, spectral products for
//                         phi0, xi_x, xi_y and the spectral sums of Z, inverse
//                         column transforms, in one pass; clears the box
//                         counts and straggler sums for the next spread
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

#include <rocprim/device/device_radix_sort.hpp>

#include "device_common.h"
#include "tsne_device.h"

namespace fehip {
namespace {

constexpr int kLgThreads = 256;
// partial-sum slots: three per convolution-pass block, then one per row block
constexpr int kLgMaxSpecBlocks = kLgMaxColBlocks;

// Node moments of a box as polynomials.  With v = u - 1/2 a point's offset
// from the box centre (in box widths, |v| <= 1/2), node c sits at
// v_c = (c - 1) / 3 and the order-3 Lagrange weight of node c is the degree-2
// polynomial L_c(v); the point's offset from node c in units of the node
// spacing h is 3 (v - v_c).  So every node moment is a fixed combination of
// power sums of the box's points,
//   m0(r, c)  = sum_ij A_r[i] A_c[j] S_ij,   m1x(r, c) = sum_ij A_r[i] B_c[j] S_ij,
//   m1y(r, c) = sum_ij B_r[i] A_c[j] S_ij,
//   m2(r, c)  = sum_ij (A_r[i] D_c[j] + D_r[i] A_c[j]) S_ij,
// with S_ij = sum over points vy^i vx^j, A_c = L_c, B_c = L_c 3 (v - v_c),
// D_c = L_c 9 (v - v_c)^2 (r is the node row, along y).  The spread sums
// the 21 power sums that occur (i <= 2 with j <= 4, i in {3, 4} with
// j <= 2) instead of 36 node moments; the gather combines them.  In v the
// coefficients are small (|A| <= 9, |B| <= 27, |D| <= 81 at |v|^k <= 2^-k),
// so the combination loses a few ulps at most.
constexpr int kLgSums = 21;
__host__ __device__ constexpr int lg_sum_index(int i, int j) { return i <= 2 ? i * 5 + j : 15 + (i - 3) * 3 + j; }
__host__ __device__ constexpr bool lg_sum_exists(int i, int j) { return (i <= 2 && j <= 4) || (i <= 4 && j <= 2); }

struct LgPoly {
  double k[5];  // coefficients of v^0 .. v^4
};
constexpr double lg_node_v(int c) { return (c - 1) / 3.0; }
constexpr LgPoly lg_poly_lin(LgPoly p, double a, double b) {  // p(v) (a v + b)
  LgPoly q{};
  for (int i = 0; i < 5; ++i) {
    q.k[i] += b * p.k[i];
    if (i + 1 < 5) q.k[i + 1] += a * p.k[i];
  }
  return q;
}
// kind 0: A_c = L_c, 1: B_c = L_c 3 (v - v_c), 2: D_c = L_c 9 (v - v_c)^2
constexpr LgPoly lg_node_poly(int kind, int c) {
  LgPoly p{{1.0, 0.0, 0.0, 0.0, 0.0}};
  for (int d = 0; d < kLgOrder; ++d) {
    if (d != c) p = lg_poly_lin(p, 1.0 / (lg_node_v(c) - lg_node_v(d)), -lg_node_v(d) / (lg_node_v(c) - lg_node_v(d)));
  }
  for (int t = 0; t < kind; ++t) p = lg_poly_lin(p, 3.0, -3.0 * lg_node_v(c));
  return p;
}
struct LgPolyTable {
  float k[3][kLgOrder][5];
};
constexpr LgPolyTable lg_poly_table() {
  LgPolyTable t{};
  for (int kind = 0; kind < 3; ++kind)
    for (int c = 0; c < kLgOrder; ++c)
      for (int i = 0; i < 5; ++i) t.k[kind][c][i] = static_cast<float>(lg_node_poly(kind, c).k[i]);
  return t;
}
static_assert(lg_poly_table().k[0][1][0] == 1.0f && lg_poly_table().k[0][1][2] == -9.0f &&
                  lg_poly_table().k[0][0][1] == -1.5f && lg_poly_table().k[0][2][2] == 4.5f &&
                  lg_poly_table().k[2][1][4] == -81.0f && lg_poly_table().k[1][0][3] == 13.5f,
              "Lagrange weights on the nodes (c - 1) / 3: L_0 = 4.5 v^2 - 1.5 v, L_1 = 1 - 9 v^2");

// kLgCoef.k[r][c][t][s]: the coefficient of power sum s in moment t (m0, m1x,
// m1y, m2) of node (r, c), from the polynomials above (exact in fp32: the
// products of 1.5, 3, 4.5, 9, 13.5, 27, 40.5 and 81).
struct LgCoefTable {
  float k[kLgOrder][kLgOrder][4][kLgSums];
};
constexpr LgCoefTable lg_coef_table() {
  LgCoefTable t{};
  for (int r = 0; r < kLgOrder; ++r)
    for (int c = 0; c < kLgOrder; ++c)
      for (int mo = 0; mo < 4; ++mo)
        for (int i = 0; i < 5; ++i)
          for (int j = 0; j < 5; ++j) {
            if (!lg_sum_exists(i, j)) continue;
            // (y polynomial, x polynomial) kinds: m0 (A, A), m1x (A, B),
            // m1y (B, A), m2 (A, D) + (D, A)
            const int ky = mo == 2 ? 1 : 0, kx = mo == 1 ? 1 : (mo == 3 ? 2 : 0);
            double v = lg_node_poly(ky, r).k[i] * lg_node_poly(kx, c).k[j];
            if (mo == 3) v += lg_node_poly(2, r).k[i] * lg_node_poly(0, c).k[j];
            t.k[r][c][mo][lg_sum_index(i, j)] = static_cast<float>(v);
          }
  return t;
}
__constant__ LgCoefTable kLgCoef = lg_coef_table();

// The 21 power sums one point contributes.
__device__ __forceinline__ void lg_power_sums(const LgPoint& b, float (&s)[kLgSums]) {
#pragma clang fp contract(off)
  const float vx = b.ux - 0.5f;
  const float vy = b.uy - 0.5f;
  float px[5], py[5];
  px[0] = 1.0f;
  px[1] = vx;
  px[2] = vx * vx;
  px[3] = px[2] * vx;
  px[4] = px[2] * px[2];
  py[0] = 1.0f;
  py[1] = vy;
  py[2] = vy * vy;
  py[3] = py[2] * vy;
  py[4] = py[2] * py[2];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      if (lg_sum_exists(i, j)) s[lg_sum_index(i, j)] = i == 0 ? px[j] : (j == 0 ? py[i] : py[i] * px[j]);
    }
  }
}

// gfx9 DPP controls: whole-wave shifts by one lane.
constexpr int kDppWaveShl1 = 0x130;  // lane l reads lane l + 1
constexpr int kDppWaveShr1 = 0x138;  // lane l reads lane l - 1

// Inclusive segmented scan (Hillis-Steele) of the 21 sums over the wave: row
// shifts 1, 2, 4, 8, then row broadcasts 15 (into rows 1 and 3) and 31 (into
// rows 2 and 3).  `take` is 0 on a lane that starts a run and 1 elsewhere;
// at each step a lane adds the partial sums the step reaches, times its take
// (one DPP multiply-add per value: the sum is an fp32 add, take being 0 or
// 1), and its take becomes the minimum of the two (0 once its window holds a
// run start).  bound_ctrl is off, so a lane whose source lies outside its row
// (or the rows a broadcast writes) is not written and keeps its partial sum
// and its take.  gfx9 needs two wait states between a VALU write of a VGPR
// and a DPP read of it: every DPP source here was written at least 21
// instructions earlier, and the s_nop 1 at each end covers the code around
// the block.  Needs the whole wave active.
#define LG_FMAC(i, CTRL) "v_fmac_f32_dpp %" #i ", %" #i ", %21 " CTRL "\n\t"
#define LG_SCAN_STEP(CTRL)                                                                                          \
  LG_FMAC(0, CTRL) LG_FMAC(1, CTRL) LG_FMAC(2, CTRL) LG_FMAC(3, CTRL) LG_FMAC(4, CTRL) LG_FMAC(5, CTRL)           \
  LG_FMAC(6, CTRL) LG_FMAC(7, CTRL) LG_FMAC(8, CTRL) LG_FMAC(9, CTRL) LG_FMAC(10, CTRL) LG_FMAC(11, CTRL)         \
  LG_FMAC(12, CTRL) LG_FMAC(13, CTRL) LG_FMAC(14, CTRL) LG_FMAC(15, CTRL) LG_FMAC(16, CTRL) LG_FMAC(17, CTRL)     \
  LG_FMAC(18, CTRL) LG_FMAC(19, CTRL) LG_FMAC(20, CTRL) "v_min_f32_dpp %21, %21, %21 " CTRL "\n\t"
static_assert(kLgSums == 21, "the scan block names 21 sums");

__device__ __forceinline__ void lg_seg_scan(float (&a)[kLgSums], float& take) {
  asm volatile("s_nop 1\n\t"
               LG_SCAN_STEP("row_shr:1 row_mask:0xf bank_mask:0xf")
               LG_SCAN_STEP("row_shr:2 row_mask:0xf bank_mask:0xf")
               LG_SCAN_STEP("row_shr:4 row_mask:0xf bank_mask:0xf")
               LG_SCAN_STEP("row_shr:8 row_mask:0xf bank_mask:0xf")
               LG_SCAN_STEP("row_bcast:15 row_mask:0xa bank_mask:0xf")
               LG_SCAN_STEP("row_bcast:31 row_mask:0xc bank_mask:0xf")
               "s_nop 1"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]),
                 "+v"(a[7]), "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]),
                 "+v"(a[14]), "+v"(a[15]), "+v"(a[16]), "+v"(a[17]), "+v"(a[18]), "+v"(a[19]), "+v"(a[20]),
                 "+v"(take));
}
#undef LG_SCAN_STEP
#undef LG_FMAC

// Spread order: points sorted by the Morton code of their position on a
// lattice of kLgOrderSub x kLgOrderSub cells per box, so that points of one
// box are contiguous when the order is made and stay in long runs while the
// layout drifts.  Keys use kLgOrderBits bits per axis.
constexpr int kLgOrderSub = 4;
constexpr int kLgOrderBits = 12;
static_assert(kLgOrderSub * (kLgMaxNodes / kLgOrder) <= (1 << kLgOrderBits), "lattice cells fit the key");

__device__ __forceinline__ unsigned int lg_interleave12(unsigned int v) {
  v &= 0xfffu;
  v = (v | (v << 8)) & 0x00ff00ffu;
  v = (v | (v << 4)) & 0x0f0f0f0fu;
  v = (v | (v << 2)) & 0x33333333u;
  v = (v | (v << 1)) & 0x55555555u;
  return v;
}

__global__ __launch_bounds__(kLgThreads) void k_lg_order_keys(const float2* __restrict__ y_stored,
                                                              const DeviceScalars* sc, unsigned int* __restrict__ keys,
                                                              int* __restrict__ idx, int n) {
#pragma clang fp contract(off)
  const DeviceScalars s = *sc;
  const double lo = static_cast<double>(s.lg_lo);
  const double scale = static_cast<double>(kLgOrderSub) / s.lg_box_wd;
  const int cells = kLgOrderSub * s.lg_boxes;
  for (int i = blockIdx.x * kLgThreads + threadIdx.x; i < n; i += gridDim.x * kLgThreads) {
    const float2 r = y_stored[i];
    const double rx = (static_cast<double>(r.x - s.shift_x) - lo) * scale;
    const double ry = (static_cast<double>(r.y - s.shift_y) - lo) * scale;
    const int qx = max(0, min(cells - 1, static_cast<int>(floor(rx))));
    const int qy = max(0, min(cells - 1, static_cast<int>(floor(ry))));
    keys[i] = lg_interleave12(static_cast<unsigned int>(qx)) | (lg_interleave12(static_cast<unsigned int>(qy)) << 1);
    idx[i] = i;
  }
}

// Per iteration, two kernels.  k_lg_spread: each workgroup takes kLgChunk
// consecutive points of the spread order (`order`, working indices sorted by
// position), so that its points fall into few boxes, and sums them in LDS,
// in a table of 2^TB slots keyed by box (open addressing; 256, or 64 where
// the host expects dense boxes: 6 KB instead of 22 KB of LDS, so that a CU
// that holds attraction workgroups still fits several spread workgroups).
// Each lane fetches its points' positions for all steps first; then every
// point is centred and located, its 21 power sums (above) are summed with those of the
// other points of its box among the wave's 64 consecutive points (an
// inclusive segmented scan over runs of one box, lg_seg_scan), and the last
// lane of each run finds its box's slot (atomicCAS on the slot's key) and adds
// the run's sums into it (LDS float atomics).  Each occupied slot then takes
// the next of its box's entries (an integer atomic on the box's count; K
// entries per box, K = min(kLgMaxPerBox, kLgEntryPool / boxes), so that few
// boxes get many) and stores its sums there with plain stores.  Each box's
// entries are then summed in chunks (k_lg_box_chunks), and the charge row
// transform (k_lg_charge_rows, one workgroup per node row) sums each box's
// chunks and combines them into the nodes' moments.  Float
// atomics in global memory (they resolve beyond the XCDs' L2s and cost far
// more than the LDS path) are left for the rare exceptions, which go to a
// straggler array of power sums per box that the row transform adds (only
// for boxes flagged in their count word; the convolution pass clears the
// counts and those sums): a run whose chunk
// already fills its table (more than 2^TB boxes in kLgChunk points) and a
// box with more than K contributing workgroups.  Any permutation gives
// the same charges up to the order of the fp32 adds; a spatial one keeps runs
// long and tables sparse.  A grid the FFT length cannot hold (2 m > fft_len,
// excluded by the host's bound) raises kErrInterpGrid; the spread and the
// row transform then write nothing.
constexpr int kLgSteps = 4;                        // 64-point steps per wave
constexpr int kLgChunk = kLgThreads * kLgSteps;    // points per workgroup
static_assert(kLgChunk == kLgSpreadChunk, "the host sizes the spread's scratch by kLgSpreadChunk");
static_assert(kLgSums == kLgSumsPerBox, "the host sizes the sums by kLgSumsPerBox");
// A box's count word: the slots listed (low bits) and a flag set when
// straggler sums were added for the box (the row transform reads them and
// the convolution pass clears them only then).
constexpr int kLgStraggled = 1 << 30;
constexpr int kLgCountMask = kLgStraggled - 1;

// Entries per box at nb boxes per axis (the spread and the gather agree).
__device__ __forceinline__ int lg_entries_per_box(int nb) {
  return max(1, min(kLgMaxPerBox, static_cast<int>(kLgEntryPool / (static_cast<long long>(nb) * nb))));
}

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
// Groups a wave's points by box before the scan: a stable partition of the
// lanes by key (boxes in order of first appearance, past-the-end lanes
// last), the point's key and position in its box moved to its new lane by a
// forward permute.  Once the grid has drifted from the lattice the spread
// order was made on, the points of two or three boxes alternate in the
// order (a Z-curve crosses a box's shifted edges many times): ~10 runs per
// 64 points instead of ~2, and every run end costs 21 LDS float atomics,
// which took ~60 % of the kernel.  Grouped, a wave step has one run per box.
// With more than kLgGroupMax boxes in a step (sparse regions, where runs are
// short anyway) the order is kept.  Needs the whole wave active.
constexpr int kLgGroupMax = 8;
__device__ __forceinline__ void lg_group_by_box(int& key, float& ux, float& uy) {
  unsigned long long pending = __ballot(key >= 0);
  int base = 0;
  int dst = -1;
  for (int g = 0; g < kLgGroupMax && pending != 0; ++g) {
    const int leader = __ffsll(static_cast<long long>(pending)) - 1;
    const int k = __builtin_amdgcn_readlane(key, leader);
    const unsigned long long m = __ballot(key == k);
    const int below = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(m >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(m), 0u)));
    if (key == k) dst = base + below;
    base += __popcll(m);
    pending &= ~m;
  }
  if (pending != 0) return;  // too many boxes: keep the order
  const unsigned long long rest = __ballot(key < 0);
  const int below = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(rest >> 32),
                                                               __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(rest), 0u)));
  if (key < 0) dst = base + below;
  key = __builtin_amdgcn_ds_permute(dst * 4, key);
  ux = __int_as_float(__builtin_amdgcn_ds_permute(dst * 4, __float_as_int(ux)));
  uy = __int_as_float(__builtin_amdgcn_ds_permute(dst * 4, __float_as_int(uy)));
}

template <int TB>
__global__ __launch_bounds__(kLgThreads) void k_lg_spread(const float2* __restrict__ y_stored,
                                                          const int* __restrict__ order, DeviceScalars* sc, int n,
                                                          int max_nodes, float* __restrict__ entries,
                                                          int* __restrict__ box_count, float* __restrict__ straggler) {
#pragma clang fp contract(off)
  constexpr int kSlots = 1 << TB;
  static_assert(kSlots <= kLgThreads, "one table slot per thread in the flush");
  chain_priority();
  __shared__ int tkey[kSlots];              // box of each slot, -1: free
  __shared__ int tdst[kSlots];              // the slot's entry, -1: none
  __shared__ float tval[kSlots * kLgSums];  // the slots' sums
  const DeviceScalars s = *sc;
  const int m = s.lg_nodes;
  if (m > max_nodes) {  // uniform over the grid
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(&sc->error_flags, kErrInterpGrid);
    return;
  }
  const int nb = s.lg_boxes;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  // a wave's steps are consecutive points of the order; the chunks of one
  // XCD are one contiguous range of the order (col_block), a compact region
  // of the layout, so the cache lines of y that its points share are fetched
  // into that XCD's L2 once (round-robin chunks fetched each line into
  // several L2s: 75 MB read per spread at config 2)
  const int chunks = (n + kLgChunk - 1) / kLgChunk;
  const int chunk = col_block(static_cast<int>(blockIdx.x), chunks);
  const long long base = chunk < 0 ? static_cast<long long>(n)
                                   : static_cast<long long>(chunk) * kLgChunk + static_cast<long long>(wave) * kLgSteps * 64;
  // every step's position is fetched before the table is cleared, so the
  // gathers of all steps are in flight together
  float2 r[kLgSteps];
  {
    int src[kLgSteps];
#pragma unroll
    for (int k = 0; k < kLgSteps; ++k) {
      const long long i = base + k * 64 + lane;
      src[k] = i < n ? (order != nullptr ? order[i] : static_cast<int>(i)) : -1;
    }
#pragma unroll
    for (int k = 0; k < kLgSteps; ++k) r[k] = src[k] >= 0 ? y_stored[src[k]] : make_float2(0.0f, 0.0f);
  }
  if (threadIdx.x < kSlots) tkey[threadIdx.x] = -1;
  for (int e = threadIdx.x; e < kSlots * kLgSums; e += kLgThreads) tval[e] = 0.0f;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kLgSteps; ++k) {
    const long long i = base + k * 64 + lane;
    LgPoint b{0, 0, 0.0f, 0.0f};
    int key = -1;  // past the end: a run of its own, never added
    if (i < n) {
      b = lg_locate(r[k].x - s.shift_x, r[k].y - s.shift_y, s);
      key = b.by * nb + b.bx;
    }
    lg_group_by_box(key, b.ux, b.uy);
    float a[kLgSums];
    if (key >= 0) {
      lg_power_sums(b, a);
    } else {
#pragma unroll
      for (int e = 0; e < kLgSums; ++e) a[e] = 0.0f;
    }
    const int prev = __builtin_amdgcn_update_dpp(0, key, kDppWaveShr1, 0xf, 0xf, true);
    const int next = __builtin_amdgcn_update_dpp(0, key, kDppWaveShl1, 0xf, 0xf, true);
    float take = (lane == 0 || prev != key) ? 0.0f : 1.0f;
    lg_seg_scan(a, take);
    if (key >= 0 && (lane == 63 || next != key)) {  // the last lane of its run
      unsigned int h = (static_cast<unsigned int>(key) * 2654435761u) >> (32 - TB);
      int slot = -1;
      for (int probe = 0; probe < kSlots; ++probe) {
        const int old = atomicCAS(&tkey[h], -1, key);
        if (old == -1 || old == key) {
          slot = static_cast<int>(h);
          break;
        }
        h = (h + 1u) & (kSlots - 1);
      }
      if (slot >= 0) {
        float* dst = tval + slot * kLgSums;
#pragma unroll
        for (int e = 0; e < kLgSums; ++e) atomicAdd(dst + e, a[e]);
      } else {
#pragma unroll
        for (int e = 0; e < kLgSums; ++e) {
          unsafeAtomicAdd(straggler + static_cast<std::size_t>(key) * kLgSums + e, a[e]);
        }
        atomicOr(box_count + key, kLgStraggled);
      }
    }
  }
  __syncthreads();
  // occupied slots: each takes an entry of its box (beyond K: added as
  // stragglers), then the sums are stored, slot by slot
  const int t = threadIdx.x;
  if (t < kSlots) {
    const int gb = tkey[t];
    int dst = -1;
    if (gb >= 0) {
      const int per = lg_entries_per_box(nb);
      const int k = atomicAdd(box_count + gb, 1) & kLgCountMask;
      if (k < per) {
        dst = gb * per + k;
      } else {
#pragma unroll
        for (int e = 0; e < kLgSums; ++e) {
          unsafeAtomicAdd(straggler + static_cast<std::size_t>(gb) * kLgSums + e, tval[t * kLgSums + e]);
        }
        atomicOr(box_count + gb, kLgStraggled);
      }
    }
    tdst[t] = dst;
  }
  __syncthreads();
  for (int q = threadIdx.x; q < kSlots * kLgSums; q += kLgThreads) {
    const int slot = q / kLgSums;
    const int d = tdst[slot];
    if (d >= 0) entries[static_cast<std::size_t>(d) * kLgSums + (q - slot * kLgSums)] = tval[q];
  }
}

// ---------------------------------------------------------------------------
// Convolution.  Launch shapes per FFT length F: sequences of length F per
// block so that small transforms still fill a workgroup.
// ---------------------------------------------------------------------------

template <int F>
struct LgShape {
  static constexpr int G = F / 2;
  static constexpr int H = F / 2 + 1;
  static constexpr int NT = F >= 2048 ? 512 : 256;
  // kernel rows, convolution columns and inverse rows: 1024 threads from
  // F = 3072, where one workgroup's LDS fills most of a CU (sequential, 1M
  // points: conv 191 -> 175 us at 3072, 290 -> 276 at 4096; the charge rows,
  // whose box sums scale badly with the threads, went 91 -> 209 us)
  static constexpr int NTW = F >= 3072 ? 1024 : NT;
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
__global__ __launch_bounds__(LgShape<F>::NTW) void k_lg_kernel_rows(const DeviceScalars* sc,
                                                                   const float2* __restrict__ tw,
                                                                   float2* __restrict__ k_rows) {
  chain_priority();
  using S = LgShape<F>;
  constexpr int HH = S::H * S::H;
  __shared__ float2 lds[2 * S::KR * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  const int m = sc->lg_nodes;
  const float h = sc->lg_node_h;
  const int row0 = blockIdx.x * S::KR;
  if (row0 >= m) return;  // rows >= m are zero and never read
  stage_twiddles<F, S::NTW>(tws, tw);
  for (int e = threadIdx.x; e < S::KR * F; e += S::NTW) {
    const int r = e / F;
    const int x = e - r * F;
    const int y = row0 + r;
    const int dx = x < S::G ? x : x - F;
    const int adx = dx < 0 ? -dx : dx;
    float k = 0.0f, k1 = 0.0f;
    if (adx < m && y < m) lg_kernels(dx, y, h, k, k1);
    lds[fft_at<F>(2 * r, x)] = make_float2(k, k1);
    lds[fft_at<F>(2 * r + 1, x)] = make_float2(k * static_cast<float>(dx) + k * static_cast<float>(y), 0.0f);
  }
  __syncthreads();
  fft_lds<F, 2 * S::KR, S::NTW, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KR * S::H; e += S::NTW) {
    const int r = e / S::H;
    const int kx = e - r * S::H;
    const int y = row0 + r;
    if (y >= S::H || y >= m) continue;
    const float2 a = lds[fft_at<F>(2 * r, kx)];
    const float2 b = lds[fft_at<F>(2 * r + 1, kx)];
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
  __shared__ float2 lds[2 * S::KR * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
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
    lds[fft_at<F>(2 * c, y)] = p;
    lds[fft_at<F>(2 * c + 1, y)] = q;
  }
  __syncthreads();
  fft_lds<F, 2 * S::KR, S::NT, false, 1>(lds, tws);
  for (int e = threadIdx.x; e < S::KR * S::H; e += S::NT) {
    const int c = e / S::H;
    const int ky = e - c * S::H;
    const int kx = col0 + c;
    if (kx >= S::H) continue;
    const int at = kx * S::H + ky;
    k_hat[at] = lds[fft_at<F>(2 * c, ky)];
    k_hat[HH + at] = lds[fft_at<F>(2 * c + 1, ky)];
  }
}

// The boxes' entries summed in chunks of kLgEntryChunk, once: one thread
// per (box, chunk, sum) writes its chunk's sum over the chunk's first entry
// (the only location it reads that another thread could read is its own),
// so that the row transform reads one partial per chunk; dense boxes (early
// in the optimisation, the 50 x 50 grid's crowded boxes) spread over as many
// threads as they have chunks.  A grid flagged by the spread is skipped.
constexpr int kLgEntryChunk = 32;
__global__ __launch_bounds__(256) void k_lg_box_chunks(const DeviceScalars* sc, int max_nodes, float* entries,
                                                       const int* __restrict__ box_count) {
  chain_priority();
  if (sc->lg_nodes > max_nodes) return;
  const int nb = sc->lg_boxes;
  const int per = lg_entries_per_box(nb);
  const int maxc = (per + kLgEntryChunk - 1) / kLgEntryChunk;
  const long long items = static_cast<long long>(nb) * nb * maxc * kLgSums;
  for (long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; t < items;
       t += static_cast<long long>(gridDim.x) * 256) {
    const int e = static_cast<int>(t % kLgSums);
    const long long rest = t / kLgSums;
    const int c = static_cast<int>(rest % maxc);
    const int b = static_cast<int>(rest / maxc);
    const int k0 = c * kLgEntryChunk;
    const int k1 = min(min(box_count[b] & kLgCountMask, per), k0 + kLgEntryChunk);
    if (k0 >= k1) continue;
    float* src = entries + (static_cast<std::size_t>(b) * per + k0) * kLgSums + e;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int k = 0;
    const int len = k1 - k0;
    for (; k + 4 <= len; k += 4) {
      s0 += src[static_cast<std::size_t>(k) * kLgSums];
      s1 += src[static_cast<std::size_t>(k + 1) * kLgSums];
      s2 += src[static_cast<std::size_t>(k + 2) * kLgSums];
      s3 += src[static_cast<std::size_t>(k + 3) * kLgSums];
    }
    for (; k < len; ++k) s0 += src[static_cast<std::size_t>(k) * kLgSums];
    src[0] = (s0 + s1) + (s2 + s3);
  }
}

// Row transforms of the charges, one workgroup per row of boxes (by < nb):
// the row's boxes' chunk sums (k_lg_box_chunks) and, when flagged, straggler
// sums are summed into each box's 21 power
// sums, which give the node moments of the box row's kLgOrder node rows
// (kLgCoef); m2 goes to its plane for the inverse pass, and A = m0 + i m1x
// and B = m1y per node row (zero-padded to F) are transformed, one node row
// at a time.  A is separated with the Hermitian mirror, X[k] = (A[k] + conj
// A[-k]) / 2 and Y[k] = (A[k] - conj A[-k]) / 2i; B is the spectrum of a real
// row already.  Kept for kx in [0, F/2], row-major (row stride F/2 + 1),
// planes `plane` apart.  Each box is read by exactly one workgroup, so its
// count and stragglers are cleared here for the next iteration's spread.
template <int F>
__global__ __launch_bounds__(LgShape<F>::NT) void k_lg_charge_rows(const DeviceScalars* sc, int max_nodes,
                                                                   const float* __restrict__ entries,
                                                                   int* __restrict__ box_count,
                                                                   float* __restrict__ straggler,
                                                                   float* __restrict__ m2,
                                                                   const float2* __restrict__ tw,
                                                                   float2* __restrict__ rows, long long plane) {
#pragma clang fp contract(off)
  chain_priority();
  using S = LgShape<F>;
  // one node row per workgroup (blockIdx.y): three workgroups per row of
  // boxes, each summing the row's boxes itself, so that the few, long
  // workgroups of one per box row do not trail beside the attraction; the
  // box counts and straggler sums are cleared by the convolution pass, once
  // all three have read them
  constexpr int RG = 1;
  constexpr int NB = F / 2 / kLgOrder;          // boxes per axis this length holds
  __shared__ float2 lds[2 * RG * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  // the box sums share the transform's buffer: the node moments are taken
  // to registers before the buffer is written (15.4 KB of LDS at F = 768,
  // so that a workgroup fits a CU beside three attraction workgroups)
  static_assert(NB * kLgSums * sizeof(float) <= sizeof(lds), "box sums fit the transform buffer");
  float* ps = reinterpret_cast<float*>(lds);
  const int m = sc->lg_nodes;
  if (m > max_nodes) return;  // flagged by the spread
  const int nb = sc->lg_boxes;
  const int by = blockIdx.x;
  if (by >= nb) return;
  stage_twiddles<F, S::NT>(tws, tw);
  const int per = lg_entries_per_box(nb);
  // each box's sums: its straggler sums (when flagged) as the starting
  // values, then its chunks' sums in chunk order
  for (int q = threadIdx.x; q < nb * kLgSums; q += S::NT) {
    const int bx = q / kLgSums;
    const int e = q - bx * kLgSums;
    const int b = by * nb + bx;
    const int word = box_count[b];
    float acc = (word & kLgStraggled) != 0 ? straggler[static_cast<std::size_t>(b) * kLgSums + e] : 0.0f;
    const int chunks = (min(word & kLgCountMask, per) + kLgEntryChunk - 1) / kLgEntryChunk;
    const float* src = entries + static_cast<std::size_t>(b) * per * kLgSums + e;
    for (int c = 0; c < chunks; ++c) acc += src[static_cast<std::size_t>(c) * kLgEntryChunk * kLgSums];
    ps[q] = acc;
  }
  __syncthreads();
  {
    const int r0 = blockIdx.y;
    constexpr int PER = (RG * F + S::NT - 1) / S::NT;  // node moments per thread
    float2 av[PER], bv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = threadIdx.x + i * S::NT;
      const int rr = e / F;
      const int x = e - rr * F;
      const int r = r0 + rr;
      float2 a = make_float2(0.0f, 0.0f), b = a;
      if (e < RG * F && x < m) {
        const int bx = x / kLgOrder;
        const int c = x - bx * kLgOrder;
        const float* p = ps + bx * kLgSums;
        const float* k = kLgCoef.k[r][c][0];
        float v0 = 0.0f, v1 = 0.0f, v2 = 0.0f, v3 = 0.0f;
#pragma unroll
        for (int q = 0; q < kLgSums; ++q) {
          const float pq = p[q];
          v0 += k[q] * pq;
          v1 += k[kLgSums + q] * pq;
          v2 += k[2 * kLgSums + q] * pq;
          v3 += k[3 * kLgSums + q] * pq;
        }
        a = make_float2(v0, v1);
        b = make_float2(v2, 0.0f);
        m2[(by * kLgOrder + r) * m + x] = v3;
      }
      av[i] = a;
      bv[i] = b;
    }
    __syncthreads();  // every box sum read: the buffer takes the rows
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = threadIdx.x + i * S::NT;
      if (e < RG * F) {
        const int rr = e / F;
        const int x = e - rr * F;
        lds[fft_at<F>(2 * rr, x)] = av[i];
        lds[fft_at<F>(2 * rr + 1, x)] = bv[i];
      }
    }
    __syncthreads();
    fft_lds<F, 2 * RG, S::NT, false, 1>(lds, tws);
    for (int e = threadIdx.x; e < RG * S::H; e += S::NT) {
      const int rr = e / S::H;
      const int kx = e - rr * S::H;
      const int y = by * kLgOrder + r0 + rr;  // < m
      const int mk = kx == 0 ? 0 : F - kx;
      const float2 a = lds[fft_at<F>(2 * rr, kx)];
      const float2 am = conjf2(lds[fft_at<F>(2 * rr, mk)]);
      const float2 sa = cadd(a, am), da = csub(a, am);
      const int at = y * S::H + kx;
      rows[at] = cscale(sa, 0.5f);
      rows[plane + at] = make_float2(0.5f * da.y, -0.5f * da.x);
      rows[2 * plane + at] = lds[fft_at<F>(2 * rr + 1, kx)];
    }
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
__global__ __launch_bounds__(LgShape<F>::NTW) void k_lg_conv_cols(const DeviceScalars* sc,
                                                                 const float2* __restrict__ rows_in,
                                                                 const float2* __restrict__ k_hat,
                                                                 const float2* __restrict__ tw,
                                                                 float2* __restrict__ rows_out, long long plane,
                                                                 double* __restrict__ zpart,
                                                                 int* __restrict__ box_count,
                                                                 float* __restrict__ straggler) {
  chain_priority();
  using S = LgShape<F>;
  constexpr int C = S::CC;
  constexpr int HH = S::H * S::H;
  __shared__ float2 lds[3 * C * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  const int m = sc->lg_nodes;
  {
    // the spread's box counts and straggler sums, read by every charge-row
    // workgroup of the box, start the next spread at zero
    const int boxes = sc->lg_boxes * sc->lg_boxes;
    for (int b = static_cast<int>(blockIdx.x * S::NTW + threadIdx.x); b < boxes;
         b += static_cast<int>(gridDim.x * S::NTW)) {
      if ((box_count[b] & kLgStraggled) != 0) {
#pragma unroll
        for (int e = 0; e < kLgSums; ++e) straggler[static_cast<std::size_t>(b) * kLgSums + e] = 0.0f;
      }
      box_count[b] = 0;
    }
  }
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
  stage_twiddles<F, S::NTW>(tws, tw);
  for (int e = threadIdx.x; e < C * F; e += S::NTW) {
    const int c = e / F;
    const int y = e - c * F;
    const int kx = col0 + c;
    const bool live = y < m && kx < S::H;
    const long long at = static_cast<long long>(y) * S::H + kx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
      lds[fft_at<F>(ch * C + c, y)] = live ? rows_in[ch * plane + at] : make_float2(0.0f, 0.0f);
    }
  }
  __syncthreads();
  fft_lds<F, 3 * C, S::NTW, false, 1>(lds, tws);
  double s1 = 0.0, s3 = 0.0, s4 = 0.0;
  for (int e = threadIdx.x; e < C * F; e += S::NTW) {
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
    float2& v0 = lds[fft_at<F>(0 * C + c, ky)];
    float2& v1 = lds[fft_at<F>(1 * C + c, ky)];
    float2& v2 = lds[fft_at<F>(2 * C + c, ky)];
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
  fft_lds<F, 3 * C, S::NTW, true, 1>(lds, tws);
  for (int e = threadIdx.x; e < C * S::G; e += S::NTW) {
    const int c = e / S::G;
    const int y = e - c * S::G;
    const int kx = col0 + c;
    if (y >= m || kx >= S::H) continue;
    const long long at = static_cast<long long>(y) * S::H + kx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) rows_out[ch * plane + at] = lds[fft_at<F>(ch * C + c, y)];
  }
  s1 = block_sum<S::NTW>(s1);
  s3 = block_sum<S::NTW>(s3);
  s4 = block_sum<S::NTW>(s4);
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
__global__ __launch_bounds__(LgShape<F>::NTW) void k_lg_inverse_rows(const DeviceScalars* sc,
                                                                    const float2* __restrict__ rows, long long plane,
                                                                    const float* __restrict__ m2,
                                                                    const float2* __restrict__ tw,
                                                                    float4* __restrict__ field,
                                                                    double* __restrict__ partial) {
  chain_priority();
  using S = LgShape<F>;
  __shared__ float2 lds[2 * S::CR * FftPad<F>::kStride];
  __shared__ float2 tws[F / 2];
  const int m = sc->lg_nodes;
  const int row0 = blockIdx.x * S::CR;
  double acc = 0.0;
  if (row0 < m) {  // uniform over the block
    stage_twiddles<F, S::NTW>(tws, tw);
    for (int e = threadIdx.x; e < S::CR * F; e += S::NTW) {
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
      lds[fft_at<F>(2 * r, kx)] = u;
      lds[fft_at<F>(2 * r + 1, kx)] = v;
    }
    __syncthreads();
    fft_lds<F, 2 * S::CR, S::NTW, true, 1>(lds, tws);
    const float scale = 1.0f / (static_cast<float>(F) * static_cast<float>(F));
    for (int e = threadIdx.x; e < S::CR * S::G; e += S::NTW) {
      const int r = e / S::G;
      const int x = e - r * S::G;
      const int y = row0 + r;
      if (y >= m || x >= m) continue;
      const float2 u = cscale(lds[fft_at<F>(2 * r, x)], scale);
      const float vx = lds[fft_at<F>(2 * r + 1, x)].x * scale;
      const int at = y * m + x;
      field[at] = make_float4(u.x, u.y, vx, 0.0f);
      acc += static_cast<double>(m2[at]) * static_cast<double>(u.x);
    }
  }
  acc = block_sum<S::NTW>(acc);
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

// Boxes per axis of a grid of at most fft_len / 2 nodes per axis.
int lg_boxes_bound(int fft_len) { return std::max(1, std::min(fft_len / 2, kLgMaxNodes) / kLgOrder); }

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
      k_lg_kernel_rows<F><<<kblocks, S::NTW, 0, stream>>>(sc, tw, ib.k_rows);
      break;
    case 2:
      k_lg_kernel_cols<F><<<col_launch(kblocks), S::NT, 0, stream>>>(sc, ib.k_rows, tw, ib.k_cols);
      break;
    case 3: {
      // every (box, chunk, sum) item of the largest grid this length holds
      const int nbb = lg_boxes_bound(F);
      const long long per_max = std::max(1LL, std::min<long long>(kLgMaxPerBox, kLgEntryPool / (static_cast<long long>(nbb) * nbb)));
      const long long items = static_cast<long long>(nbb) * nbb * ((per_max + kLgEntryChunk - 1) / kLgEntryChunk) * kLgSums;
      const unsigned int cblocks_sum = static_cast<unsigned int>(std::min<long long>((items + 255) / 256, 8192));
      k_lg_box_chunks<<<cblocks_sum, 256, 0, stream>>>(sc, nbb * kLgOrder, ib.entries, ib.box_count);
      k_lg_charge_rows<F><<<dim3(F / 2 / kLgOrder, kLgOrder), S::NT, 0, stream>>>(sc, lg_boxes_bound(F) * kLgOrder, ib.entries,
                                                                  ib.box_count, ib.straggler, ib.m2, tw, ib.spec_a,
                                                                  plane);
      break;
    }
    case 5:
      k_lg_conv_cols<F><<<cblocks, S::NTW, 0, stream>>>(sc, ib.spec_a, ib.k_cols, tw, ib.spec_b, plane, spec_part,
                                                         ib.box_count, ib.straggler);
      break;
    case 7:
      k_lg_inverse_rows<F><<<rblocks, S::NTW, 0, stream>>>(sc, ib.spec_b, plane, ib.m2, tw, ib.field, row_part);
      k_lg_finalize_z<<<1, 256, 0, stream>>>(spec_part, cblocks, row_part, rblocks, n, F, sc);
      break;

    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_interp_spread(const float2* y_stored, const int* order, DeviceScalars* sc, InterpBuffers& ib, int n,
                                int fft_len, int table_bits, hipStream_t stream) {
  const int max_nodes = lg_boxes_bound(fft_len) * kLgOrder;
  const int blocks = col_launch(lg_spread_blocks(n));
  if (table_bits == kLgSmallTableBits) {
    k_lg_spread<kLgSmallTableBits><<<blocks, kLgThreads, 0, stream>>>(y_stored, order, sc, n, max_nodes, ib.entries,
                                                                      ib.box_count, ib.straggler);
  } else if (table_bits == kLgTableBits) {
    k_lg_spread<kLgTableBits><<<blocks, kLgThreads, 0, stream>>>(y_stored, order, sc, n, max_nodes, ib.entries,
                                                                 ib.box_count, ib.straggler);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The order's sort: rocPRIM picks a block sort and ~10 merge passes up to
// 2^20 items by default (about 0.23 ms at 1M points on MI355X); a merge-sort
// limit of 0 makes it use the onesweep radix sort at every size.
using LgOrderSortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                     rocprim::default_config, 0>;

hipError_t interp_order_temp_bytes(int n, std::size_t& bytes) {
  bytes = 0;
  return rocprim::radix_sort_pairs<LgOrderSortConfig>(nullptr, bytes, static_cast<const unsigned int*>(nullptr),
                                   static_cast<unsigned int*>(nullptr), static_cast<const int*>(nullptr),
                                   static_cast<int*>(nullptr), static_cast<std::size_t>(n), 0u,
                                   static_cast<unsigned int>(2 * kLgOrderBits));
}

hipError_t launch_interp_order(const float2* y_stored, const DeviceScalars* sc, InterpBuffers& ib, int n, int fft_len,
                               hipStream_t stream) {
  const int blocks = std::max(1, std::min((n + kLgThreads - 1) / kLgThreads, 4096));
  k_lg_order_keys<<<blocks, kLgThreads, 0, stream>>>(y_stored, sc, ib.order_keys, ib.order_idx, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the keys' bits: the lattice of the largest grid this FFT length holds
  // (a grid beyond it raises kErrInterpGrid in the spread, whatever the order)
  int axis_bits = 1;
  while ((1 << axis_bits) < kLgOrderSub * lg_boxes_bound(fft_len)) ++axis_bits;
  std::size_t bytes = ib.order_temp_bytes;
  return rocprim::radix_sort_pairs<LgOrderSortConfig>(ib.order_temp, bytes, ib.order_keys, ib.order_keys + n,
                                                      ib.order_idx, ib.order, static_cast<std::size_t>(n), 0u,
                                                      static_cast<unsigned int>(2 * axis_bits), stream);
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
