// Internal interface between the host orchestration (embedding_hip_session.cpp)
// and the gfx950 kernels (embedding_hip_kernels.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <string>

namespace fehip {

// Thread-local message behind fastembedr_hip_embedding_last_error().
void set_last_error(const std::string& msg);
void clear_last_error();

// Per-session scalars that the kernels read and write on the device, so that
// an iteration never waits for the host.  Written by the single-block
// finalize kernels of the reductions (stats -> geometry, inverse rows -> sum
// of q, exact repulsion -> its normaliser).
struct alignas(16) DeviceScalars {
  float shift_x, shift_y;   // subtracted from the stored layout to centre it
  float lo_x, lo_y;         // grid origin in centred coordinates
  float h, inv_h;           // node spacing and its reciprocal
  float inv_sum_q;          // 1 / max(sum_q - n, FLT_MIN), fp32
  float pad0;
  double sum_q;             // sum over nodes of mass * q (self terms included)
  double mean_x, mean_y;    // fp64 mean of the stored layout
  float min_x, max_x, min_y, max_y;  // bounding box of the centred layout
  double exact_z;           // exact-repulsion normaliser (pairs i != j)
  double total_mass;        // sum of directed p_{j|i} over non-self columns
  unsigned int error_flags;  // bit 0: index out of range, bit 1: bad distance
  unsigned int pad2;
  unsigned long long self_edges;
  int num_items;             // spread work items of the current iteration
  unsigned int ring_seq;     // updates that wrote the host's box-count ring so far
  // FIt-SNE interpolation grid.  The host sets the specification (lg_order
  // 0 = unused); the statistics finalize sets the geometry of the current
  // layout: the square [lg_lo, lg_lo + lg_boxes * lg_box_w]^2 of centred
  // coordinates, lg_order nodes per box and axis at spacing lg_node_h.
  int lg_order, lg_min_intervals;
  float lg_ints_per_unit;
  float lg_lo, lg_box_w, lg_node_h;
  int lg_boxes, lg_nodes;
  double lg_box_wd;            // box width in fp64: points are located in fp64
  double lg_inv_box_wd;        // its correctly rounded reciprocal (lg_locate)
};

struct BlockStats {
  float min_x, max_x, min_y, max_y;
  double sum_x, sum_y;
};

constexpr int kMaxReduceBlocks = 4096;
// Slots of the pinned ring through which the update's statistics kernel hands
// the interpolation grid's box count to the host (a power of two).  Each slot
// holds (sequence number << 32) | box count, so the host can tell which
// update wrote it without an event.
constexpr int kBoxRing = 8;
// Twiddle table: e^{-2 pi i m / 4096} for m < 4096, then e^{-2 pi i m / 3072}
// for m < 3072; a transform of length F = 2^a (3 * 2^a) <= 4096 takes every
// (4096 / F)-th entry of the first part (every (3072 / F)-th of the second).
constexpr int kTwiddlePow2 = 4096;
constexpr int kTwiddlePow3 = 3072;
constexpr int kTwiddleLen = kTwiddlePow2 + kTwiddlePow3;
constexpr int kMaxGrid = 1024;        // nodes per axis (FFT length 2048)

// Spreading is binned by tiles of kTile x kTile cells; each work item is at
// most kChunk points of one tile, accumulated in LDS ((kTile + 1)^2 nodes).
constexpr int kTile = 16;
constexpr int kChunk = 2048;
constexpr int kMaxTilesPerAxis = (kMaxGrid - 2) / kTile + 1;  // 64
constexpr int kMaxTiles = kMaxTilesPerAxis * kMaxTilesPerAxis;
inline int tiles_per_axis(int g) { return (g - 2) / kTile + 1; }
inline int max_spread_items(int n, int g) {
  return (n + kChunk - 1) / kChunk + tiles_per_axis(g) * tiles_per_axis(g);
}

enum ErrorBits : unsigned int { kErrIndex = 1u, kErrDistance = 2u, kErrInterpGrid = 4u };

// FIt-SNE interpolation grid: order-3 nodes, at most kLgMaxNodes nodes per
// axis (FFT length <= 4096).
constexpr int kLgOrder = 3;
constexpr int kLgMaxNodes = 2048;
constexpr int kLgMaxFft = 2 * kLgMaxNodes;
constexpr int kLgMaxBoxes = kLgMaxNodes / kLgOrder;  // per axis
// Spreading: a workgroup sums kLgSpreadChunk points of the spread order into
// an LDS table of 2^table_bits slots keyed by box (kLgTableBits, or
// kLgSmallTableBits where the points are dense enough that a chunk touches
// few boxes); each box takes the sums of up to K = min(kLgMaxPerBox,
// kLgEntryPool / boxes) workgroups.
constexpr int kLgSpreadChunk = 1024;
constexpr int kLgTableBits = 8;
constexpr int kLgSmallTableBits = 6;
constexpr int kLgTable = 1 << kLgTableBits;
// A pool of 2^21 entries (176 MB) shared by the boxes: early in the
// optimisation a few boxes of the 50 x 50 minimum grid hold hundreds of
// workgroups' points, and entries beyond K fall back to float atomics on the
// box's straggler row, all on the same 21 addresses (with K capped at 64 the
// spread took 170 us instead of 15 in the first 50 iterations of config 2).
constexpr int kLgMaxPerBox = 1024;
constexpr long long kLgEntryPool = 1LL << 21;
constexpr int kLgSumsPerBox = 21;  // power sums of a box's points (the node moments' ingredients)
inline int lg_spread_blocks(int n) { return std::max(1, (n + kLgSpreadChunk - 1) / kLgSpreadChunk); }
// Column passes of the interpolation grid map their blocks to columns XCD by
// XCD (block b on XCD b % kLgColXcds takes the next column of that XCD's
// contiguous range), so their launches are rounded up to a multiple of it.
constexpr int kLgColXcds = 8;
constexpr int kLgMaxColBlocks = (kLgMaxFft / 2 + 1 + kLgColXcds - 1) / kLgColXcds * kLgColXcds;
// three spectral sums per column-pass block, one per row block (<= f/2)
constexpr int kLgZPartials = 3 * kLgMaxColBlocks + kLgMaxFft / 2;

enum KernelId : int {
  kKStats = 0,
  kKBinCount,
  kKBinPlan,
  kKBinScatter,
  kKSpread,
  kKKernelRows,
  kKKernelCols,
  kKChargeRows,
  kKConvCols,
  kKInverseRows,
  kKAttract,
  kKUpdate,
  kKCommit,
  kKRenumber,
  kKTileBuild,
  kKLgOrder,
  kKLgSpread,
  kKLgKernelRows,
  kKLgKernelCols,
  kKLgChargeRows,
  kKLgConvCols,
  kKLgInverseRows,
  kKFinalize,
  // not a kernel: the repulsion step's span, from its first kernel to its
  // last, run in sequence (timed only when it is the one id timed)
  kKRepulsion,
  kKernelCount
};

// Buffers of one grid configuration (g nodes per axis, f = 2g, hh = g + 1).
struct GridBuffers {
  int g = 0;
  float* mass = nullptr;     // g*g, zero between iterations
  float* mass_x = nullptr;
  float* mass_y = nullptr;
  float4* field = nullptr;   // g*g of (q2, xq2, yq2, q)
  float2* k_rows = nullptr;  // hh*hh: row transforms of the kernel quadrant
  float2* k_hat = nullptr;   // hh*hh: (K1^, K2^) quadrant
  float2* m_rows = nullptr;  // g*hh each: half-spectrum rows of the charges
  float2* mx_rows = nullptr;
  float2* my_rows = nullptr;
  float2* x_rows = nullptr;  // g*hh each: half-spectrum rows of the potentials
  float2* v1_rows = nullptr;
  float2* v2_rows = nullptr;
  float2* y_rows = nullptr;
  double* sumq_partial = nullptr;  // kMaxReduceBlocks
  // spreading bins
  int* tile_count = nullptr;   // kMaxTiles, zero between iterations
  int* tile_cursor = nullptr;  // kMaxTiles
  int4* items = nullptr;       // max_spread_items(n, g): (tile, begin, end, -)
  float2* binned = nullptr;    // n centred points in tile order
};

// Buffers of the FIt-SNE interpolation grid, sized for the largest grid
// (kLgMaxNodes nodes per axis, FFT length kLgMaxFft).  At run time the node
// count m and the FFT length f vary; planes use row stride m, spectra row
// stride f / 2 + 1.
struct InterpBuffers {
  float* m2 = nullptr;         // m*m: node moments m2 (squared offsets in units of h), for the inverse pass
  float4* field = nullptr;     // m*m potentials (phi0, xi_x, xi_y, 0)
  float2* k_rows = nullptr;    // 2 planes of (G+1)^2: kernel row spectra ((K^r, K1^r), (Bx, By)), row-major
  float2* k_cols = nullptr;    // 2 planes of (G+1)^2: the kernel spectrum quadrant ((K^, K1^), (Cx, Cy)),
                               // kx-major
  float2* spec_a = nullptr;    // 3 planes of G*(G+1): charge row spectra, row-major
  float2* spec_b = nullptr;    // 3 planes of G*(G+1): potential row spectra, row-major
  double* z_partial = nullptr; // kLgZPartials: sums of the normaliser per block
  float* entries = nullptr;    // kLgEntryPool x kLgSumsPerBox: workgroups' sums per box (K per box)
  int* box_count = nullptr;    // boxes of the largest grid: entries taken per box, zero between iterations
  float* straggler = nullptr;  // boxes x kLgSumsPerBox: atomic exceptions, zero between iterations
  int* order = nullptr;        // n: spread order (working indices sorted by position)
  unsigned int* order_keys = nullptr;  // 2n: Morton keys, sorted keys
  int* order_idx = nullptr;    // n: 0 .. n-1 (the sort's payload)
  void* order_temp = nullptr;  // radix sort scratch
  std::size_t order_temp_bytes = 0;
};

struct Csr {
  int n = 0;
  long long nnz = 0;
  int* row_ptr = nullptr;
  int* col = nullptr;
  float* val = nullptr;
};

// ---- P construction -------------------------------------------------------
// Row search + directed edge emission (both orientations); self edges get the
// sentinel key and are counted.  `dist_is_double` selects the input type.
hipError_t launch_row_search(const int* idx_cm, const void* dist_cm, bool dist_is_double, int n, int k,
                             int index_offset, float log_perplexity, float* p_cond, std::uint64_t* keys,
                             float* vals, int key_bits, double* mass_partial, int mass_blocks,
                             DeviceScalars* sc, hipStream_t stream);
hipError_t launch_finalize_mass(const double* mass_partial, int blocks, DeviceScalars* sc, hipStream_t stream);
hipError_t sort_edges(void* temp, std::size_t& temp_bytes, const std::uint64_t* keys_in, std::uint64_t* keys_out,
                      const float* vals_in, float* vals_out, std::size_t count, int end_bit, hipStream_t stream);
hipError_t launch_mark_heads(const std::uint64_t* keys, std::size_t count, int* heads, hipStream_t stream);
hipError_t scan_heads(void* temp, std::size_t& temp_bytes, const int* heads, int* pos, std::size_t count,
                      hipStream_t stream);
hipError_t launch_compact(const std::uint64_t* keys, const float* vals, const int* heads, const int* pos,
                          std::size_t count, int key_bits, int n, const DeviceScalars* sc, int* row_ptr, int* col,
                          float* val, hipStream_t stream);

// ---- iteration ------------------------------------------------------------
int reduce_blocks_for(int n);
hipError_t launch_stats(const float2* y, int n, int g, int center, BlockStats* partial, DeviceScalars* sc,
                        hipStream_t stream);
// Spreading in four launches: centre + count points per tile, plan (scan and
// work items), scatter into tile order, per-item LDS accumulation.
hipError_t launch_bin_count(const float2* y_stored, float2* y_cur, const DeviceScalars* sc, GridBuffers& gb, int n,
                            hipStream_t stream);
hipError_t launch_bin_plan(GridBuffers& gb, DeviceScalars* sc, hipStream_t stream);
hipError_t launch_bin_scatter(const float2* y_cur, const DeviceScalars* sc, GridBuffers& gb, int n,
                              hipStream_t stream);
hipError_t launch_spread_tiles(const DeviceScalars* sc, GridBuffers& gb, int n, hipStream_t stream);
hipError_t launch_kernel_rows(GridBuffers& gb, const DeviceScalars* sc, const float2* tw, hipStream_t stream);
hipError_t launch_kernel_cols(GridBuffers& gb, const float2* tw, hipStream_t stream);
hipError_t launch_charge_rows(GridBuffers& gb, const float2* tw, hipStream_t stream);
hipError_t launch_conv_cols(GridBuffers& gb, const float2* tw, hipStream_t stream);
hipError_t launch_inverse_rows(GridBuffers& gb, const float2* tw, int n, DeviceScalars* sc, hipStream_t stream);

// ---- FIt-SNE interpolation grid ---------------------------------------------
// Spreading and the zero-padded convolution at FFT length fft_len (2^a or
// 3 * 2^a in [64, kLgMaxFft] with fft_len >= 2 * lg_nodes); the node count
// itself is read on the device.  The spread reads the stored layout in
// `order` (working indices; nullptr: the working order itself) and adds the node moments to the charge planes, which must be
// zero (they are after allocation and after every convolution).  table_bits:
// kLgTableBits or kLgSmallTableBits (any value gives the same charges up to
// the order of the fp32 adds; the small table keeps more workgroups resident
// beside other kernels).
hipError_t launch_interp_spread(const float2* y_stored, const int* order, DeviceScalars* sc, InterpBuffers& ib, int n,
                                int fft_len, int table_bits, hipStream_t stream);
// The spread order of the current layout (needs this iteration's geometry):
// working indices sorted by position.  Any permutation is correct; a spatial
// one keeps the spread's runs long.
hipError_t interp_order_temp_bytes(int n, std::size_t& bytes);
hipError_t launch_interp_order(const float2* y_stored, const DeviceScalars* sc, InterpBuffers& ib, int n, int fft_len,
                               hipStream_t stream);
// which: 0 kernel rows, 2 kernel cols, 3 charge rows, 5 conv cols, 7 inverse
// rows (+ normaliser); other values are invalid
hipError_t launch_interp_fft(int which, int fft_len, InterpBuffers& ib, DeviceScalars* sc, const float2* tw, int n,
                             hipStream_t stream);

enum AttractMode : int { kModeUpdate = 0, kModeGradientGrid = 1, kModeGradientExact = 2 };
struct UpdateParams {
  float exaggeration;
  float momentum;
  float learning_rate;
  float min_gain;
  float max_step_norm;
  int clip;
};
// Row sums of the attractive term into attr (n float2).
hipError_t launch_attract(const Csr& p, const float2* y_cur, float2* attr, float exaggeration, int lanes_per_row,
                          int xcds, hipStream_t stream);
// Repulsion read-back + attr -> gradient; kModeUpdate applies the update and
// writes per-block statistics of the new layout to `partial` (finished by
// launch_finalize_stats), the gradient modes write grad_out.  interp_field !=
// nullptr reads the FIt-SNE interpolation grid instead of the bilinear one
// (kModeUpdate and kModeGradientGrid).  done != nullptr is an event that the
// launch itself completes (the kernel's own completion, no marker behind it).
hipError_t launch_update(int mode, const float2* y_cur, const float2* attr, float2* y_out, float2* update,
                         float2* gains, float2* grad_out, const float2* exact_rep, const GridBuffers& gb,
                         const UpdateParams& up, BlockStats* partial, DeviceScalars* sc, int n, hipStream_t stream,
                         const float4* interp_field = nullptr, hipEvent_t done = nullptr);
// The next iteration's centring and grid geometry from kModeUpdate's
// statistics (one workgroup).  With box_out != nullptr (device pointer of a
// ring of kBoxRing slots in pinned coherent host memory) the interpolation
// grid's box count is also stored there, tagged with DeviceScalars::ring_seq.
hipError_t launch_finalize_stats(const BlockStats* partial, int n, int g, DeviceScalars* sc,
                                 unsigned long long* box_out, hipStream_t stream);
hipError_t launch_commit(float2* y, const DeviceScalars* sc, int n, hipStream_t stream);

// ---- locality renumbering ---------------------------------------------------
// Points are renumbered by the Morton order of the current layout so that
// CSR neighbours sit close in memory.  `order[q]` is the old working index of
// new index q; perm maps working -> original indices.
struct Renumber {
  // key = (connected component of the point << 32) | Morton code of its position
  unsigned long long* keys_in = nullptr;
  unsigned long long* keys_out = nullptr;
  const int* component = nullptr;  // per point, caller's numbering
  const int* perm = nullptr;       // current working -> caller's index
  int key_bits = 64;
  int* idx_in = nullptr;
  int* order = nullptr;
  int* map = nullptr;   // old working index -> new working index
  int* len = nullptr;   // n + 1 row lengths, then the new row pointers
  void* temp = nullptr;
  std::size_t temp_bytes = 0;
};
hipError_t renumber_temp_bytes(int n, std::size_t& bytes);
hipError_t launch_morton_keys(const float2* y, const DeviceScalars* sc, int n, Renumber& r, hipStream_t stream);
hipError_t sort_morton(Renumber& r, int n, hipStream_t stream);
hipError_t launch_apply_order(const Renumber& r, int n, const int* perm_old, int* perm_new, const float2* y_old,
                              float2* y_new, const float2* u_old, float2* u_new, const float2* g_old, float2* g_new,
                              const int* rp_old, hipStream_t stream);
hipError_t scan_row_lengths(Renumber& r, int n, int* rp_new, hipStream_t stream);
hipError_t launch_copy_rows(const Renumber& r, int n, const Csr& src, Csr& dst, hipStream_t stream);
hipError_t launch_invert(const int* perm, int* inv, int n, hipStream_t stream);
// Adds to *out the distinct column tiles of every step-th row block of P in
// the numbering given by order (new -> old rows) and map (old -> new
// columns); null for the identity.  An estimate of the tile count / step.
hipError_t launch_tile_estimate(const Csr& p, const int* order, const int* map, int step,
                                unsigned long long* out, hipStream_t stream);
// Connected components of the P graph by min-label propagation with pointer
// jumping; label[i] ends as the smallest index of i's component.
hipError_t launch_label_init(int* label, int n, hipStream_t stream);
hipError_t launch_label_step(const Csr& p, int* label, int* changed, hipStream_t stream);
hipError_t launch_gather2(const float2* src, const int* idx, float2* dst, int n, hipStream_t stream);

// ---- tiled attraction ---------------------------------------------------------
// P regrouped for the attraction: rows in blocks of kTileRows, columns in
// tiles of kTileCols.  The entries of one (row block, column tile) pair form
// one contiguous run ("tile") of slots, in row order: a 16-bit word (local
// column, row step from the previous slot of its group of kTileRun) and the
// value, whose two spare top bits carry the group's base row (slot format at
// attraction_tiles_hip.hip).  A row block's tiles are tile_ptr[rb] ..
// tile_ptr[rb + 1]; tile t covers slots tile_beg[t] .. tile_beg[t + 1] and
// column tile tile_cb[t].  Every run starts at a multiple of kTileRun slots
// and is padded to one with slots of value 0.
// Two shapes, chosen per session (tiles_shape): 2048 rows x 2048 columns
// from kTileWideFrom points, 1024 x 4096 below (more row blocks for small
// n).  Both take 48 KB of LDS and hold about the same slots per run; a
// square tile stages half the positions per visit, few enough (4 per lane)
// that the kernel loads the next tile's into registers before the switch.
constexpr int kTileRows = 1024;
constexpr int kTileCols = 4096;
constexpr int kTileRowsWide = 2048;
constexpr int kTileColsWide = 2048;
constexpr int kTileWideFrom = 1 << 19;  // points from which tiles_shape picks the wide shape (>= 256 row blocks)
constexpr int kTileRun = 8;
constexpr int kTileMaxXcds = 16;
constexpr int kTileThreads = 512;

struct Tiles {
  int n = 0;
  long long nnz = 0;
  int rows = kTileRows;  // rows per row block: kTileRows or kTileRowsWide
  int cols = kTileCols;  // columns per column tile: kTileCols or kTileColsWide
  int row_blocks = 0;
  int col_tiles = 0;
  int col_bits = 0;   // bits of the column-tile part of the sort key
  int key_bits = 0;   // col_bits + bits of the row-block part
  long long max_tiles = 0;
  long long padded = 0;          // capacity of ent / val: entries + bridges + padding at most
  unsigned short* ent = nullptr; // padded
  float* val = nullptr;          // padded; 0 in the padding
  int* tile_ptr = nullptr;       // row_blocks + 1
  int* tile_cb = nullptr;        // max_tiles + 1
  int* tile_beg = nullptr;       // max_tiles + 1 (padded begins; multiples of kTileRun)
  int* ubeg = nullptr;           // max_tiles + 1 (begins before padding)
  int* psize = nullptr;          // max_tiles + 1 (padded sizes)
  int* tile_count = nullptr;     // 1
  unsigned short* base_row = nullptr;  // padded / kTileRun + 1 (build scratch)
  unsigned int* work = nullptr;  // kTileMaxXcds + 1 claim counters of the attraction; zero between launches
  // build scratch, nnz each; after the sort the inputs hold the run heads
  // (key_in) and their scan (pay_in)
  unsigned int* key_in = nullptr;
  unsigned int* key_out = nullptr;
  unsigned long long* pay_in = nullptr;
  unsigned long long* pay_out = nullptr;
  void* temp = nullptr;
  std::size_t temp_bytes = 0;
};
// The tile shape for n points (wide: 0 = by n, 1 = 1024 x 4096, 2 = 2048 x
// 2048) and the capacities that follow from it.
void tiles_shape(int n, long long nnz, Tiles& t, int wide = 0);
hipError_t tiles_temp_bytes(const Tiles& t, std::size_t& bytes);
// Rebuilds t from the CSR (same numbering), all on `stream`.
hipError_t launch_tile_build(const Csr& p, Tiles& t, hipStream_t stream);
// Workgroups of kTileThreads.  slots_per_xcd: workgroups per XCD (<= 0: one
// per row block); with fewer, each claims row blocks of its XCD's range until
// none is left.  helper_per_xcd > 0: a helper launch of that many workgroups
// per XCD (launch_attract_tiled_helper, same arguments, enqueued later on
// another stream) shares the claims and must follow.  t.work must be zero
// (it is after a launch or a launch and its helper); xcds <= kTileMaxXcds.
// done != nullptr: an event that the launch itself completes.
hipError_t launch_attract_tiled(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration, int xcds,
                                int slots_per_xcd, int helper_per_xcd, hipStream_t stream, hipEvent_t done = nullptr);
hipError_t launch_attract_tiled_helper(const Tiles& t, const float2* y_cur, float2* attr, float exaggeration,
                                       int xcds, int slots_per_xcd, int helper_per_xcd, hipStream_t stream);

// ---- exact O(n^2) terms (gradient check and KL) ----------------------------
hipError_t launch_exact_repulsion(const float2* y, int n, float2* rep, double* z_partial, DeviceScalars* sc,
                                  hipStream_t stream);
hipError_t launch_exact_z_double(const float2* y, int n, double* z_partial, hipStream_t stream);
int exact_blocks_for(int n);
// row_out (n doubles, may be null) receives each row's KL term.
hipError_t launch_kl_rows(const Csr& p, const float2* y, double sum_q, double* partial, int blocks,
                          hipStream_t stream, double* row_out = nullptr);

}  // namespace fehip
