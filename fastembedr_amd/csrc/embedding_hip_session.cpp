// Host orchestration and C ABI of the gfx950 openTSNE-style t-SNE backend.
//
// One session = one device arena holding P (CSR), the optimiser state and the
// grid work buffers, plus one HIP stream at default priority.  Every
// iteration is enqueued without a host round trip: the kernels exchange the
// grid geometry and the repulsion normaliser through DeviceScalars.
//
// Error convention (src/embedding_cuda_kernels.cpp:55-72, 3753-3755 of the
// reference): entry points return 0 / 1, and a thread-local message is kept
// for fastembedr_hip_embedding_last_error().

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cfloat>
#include <cstddef>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "fastembedr_hip.h"
#include "knn_device.h"
#include "metrics_device.h"
#include "tsne_device.h"

using fehip::BlockStats;
using fehip::Csr;
using fehip::DeviceScalars;
using fehip::GridBuffers;

namespace {

thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

bool hip_ok(hipError_t code, const char* where) {
  if (code == hipSuccess) return true;
  set_error(std::string(where) + ": " + hipGetErrorString(code));
  return false;
}

std::size_t align_up(std::size_t v, std::size_t a = 256) { return (v + a - 1) & ~(a - 1); }

int env_int(const char* name, int fallback) {
  const char* raw = std::getenv(name);
  if (raw == nullptr || raw[0] == '\0') return fallback;
  char* end = nullptr;
  const long v = std::strtol(raw, &end, 10);
  if (end == raw || v <= 0 || v > std::numeric_limits<int>::max()) return fallback;
  return static_cast<int>(v);
}

// The reference CPU backend's grid policy (src/tsne_neighbors.cpp:392-398).
int policy_grid_size(int n) {
  const int fallback = n >= 50000 ? 256 : (n >= 10000 ? 128 : 64);
  const int requested = env_int("FASTEMBEDR_TSNE_FFT_GRID", fallback);
  int g = 32;
  while (g < requested && g < 512) g <<= 1;
  return std::max(32, std::min(512, g));
}

int resolve_grid_size(int n, int requested) {
  if (requested <= 0) return policy_grid_size(n);
  int g = 32;
  while (g < requested && g < fehip::kMaxGrid) g <<= 1;
  return g;
}

// Carves 256-byte aligned buffers out of one hipMalloc.
struct Arena {
  char* base = nullptr;
  std::size_t size = 0;
  std::size_t used = 0;
  bool init(std::size_t bytes, const char* what) {
    size = bytes;
    used = 0;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes), what)) return false;
    base = static_cast<char*>(p);
    return true;
  }
  template <typename T>
  T* take(std::size_t count) {
    const std::size_t bytes = align_up(count * sizeof(T));
    if (used + bytes > size) return nullptr;
    T* p = reinterpret_cast<T*>(base + used);
    used += bytes;
    return p;
  }
  void release() {
    if (base != nullptr) (void)hipFree(base);
    base = nullptr;
    size = used = 0;
  }
};

// FASTEMBEDR_HIP_GRAPH_CAPTURE: unset, empty, 0, false, FALSE, no, NO = off;
// anything else = on.  The reference's FASTEMBEDR_CUDA_GRAPH_CAPTURE switch
// (src/embedding_cuda_kernels.cpp:170-178) parses the same off values but is
// on when unset; here eager launches are the default, being faster than
// replays at every configuration measured on MI355X (whole 750-iteration
// schedule, interpolation grid: config 0 8721 against 8037 it/s, config 1
// 8105 against 7410, config 2 3416 against 3389).
bool graph_capture_enabled() {
  const char* env = std::getenv("FASTEMBEDR_HIP_GRAPH_CAPTURE");
  if (env == nullptr || env[0] == '\0') return false;
  for (const char* off : {"0", "false", "FALSE", "no", "NO"}) {
    if (std::strcmp(env, off) == 0) return false;
  }
  return true;
}

bool memory_preflight(std::size_t bytes, const char* where) {
  std::size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return true;
  const std::size_t reserve = free_b / 20;
  if (bytes > free_b - reserve) {
    set_error(std::string(where) + ": device memory request exceeds available memory; required " +
              std::to_string(bytes) + " bytes, free " + std::to_string(free_b) + " bytes");
    return false;
  }
  return true;
}

}  // namespace

struct fastembedr_hip_tsne {
  int n = 0;
  int k = 0;
  int lanes = 16;
  int xcds = 1;              // XCDs of the device (blocks are dispatched round-robin over them)
  hipStream_t stream = nullptr;
  // Side streams of run(): the attraction depends only on the stored layout
  // and the kernel spectrum only on the grid geometry, so they run beside the
  // binning, spreading and convolution of the repulsion chain, which waits
  // for the spectrum (an event) before the convolution; the attraction and
  // the chain share `stream` and side_attr (see `home`).  All streams have
  // the default priority.
  hipStream_t side_attr = nullptr;
  hipStream_t side_kern = nullptr;
  hipEvent_t ev_layout = nullptr; // stored layout written (the previous update's stream)
  hipEvent_t ev_ready = nullptr;  // grid geometry set (the chain's stream)
  hipEvent_t ev_attr = nullptr;   // attraction done, or (update on main) the chain done
  hipEvent_t ev_kern = nullptr;   // kernel spectrum done (side_kern)
  hipEvent_t ev_home = nullptr;   // the latest update done (settle)
  // The stream that holds the latest update: the next attraction follows it
  // there without a wait.  With update_on_chain an overlapped iteration runs
  // its update on the chain's stream (after the chain, waiting for the
  // attraction's event), so the two streams trade roles every iteration;
  // without it (the default) the update follows the attraction and `home`
  // stays put.  settle() hands the state back to `stream` for everything
  // else.
  hipStream_t home = nullptr;
  // ev_layout already marks the end of the latest update, the last work on
  // `home` (the update's launch completes it itself, so that no marker
  // stands between the update and the attraction behind it); cleared by
  // settle() and by every iteration's start.
  bool layout_at_tail = false;
  // FASTEMBEDR_HIP_UPDATE_ON_CHAIN=1: the update on the chain's stream, after
  // waiting for the attraction's event (the streams then trade roles every
  // iteration); 0, the default: the update right behind the attraction on its
  // stream, after waiting for the chain's event.  A wait for an event that
  // another stream has yet to signal cost ~18 us here, one for an event
  // already signalled ~6 us; the chain ends ~30 us before the attraction at
  // config 2, so the attraction's stream carries the update (whole schedule
  // 4104-4115 against 4080-4083 it/s, config 4 even).
  bool update_on_chain = false;
  bool mark_layout = true;  // FASTEMBEDR_HIP_MARK_LAYOUT=0: a marker after the update instead
  Arena arena;
  Arena work_arena;         // working-order CSR copies, permutations, state double buffers
  Arena tile_arena;         // tiled P for the attraction and its build scratch
  DeviceScalars* sc = nullptr;
  Csr p;                    // P in the caller's numbering (columns ascending)
  Csr pw[2];                // P in the working numbering (after renumbering)
  int wi = -1;              // current working copy; -1: working numbering == caller's
  float* p_cond = nullptr;
  // Optimiser state in the working numbering, double-buffered for renumbering.
  float2* ys[2] = {nullptr, nullptr};   // stored layout (raw between iterations)
  float2* us[2] = {nullptr, nullptr};   // update
  float2* gs[2] = {nullptr, nullptr};   // gains
  int si = 0;
  int* perm[2] = {nullptr, nullptr};    // working index -> caller's index
  int pi = 0;
  int* inv_perm = nullptr;              // caller's index -> working index
  fehip::Renumber rn;
  int reorder_period = 25;
  int reorder_gap = 0;       // 0: check at the next iteration
  int renumber_count = 0;    // orders applied
  int renumber_rejected = 0; // candidate orders not better than the current one
  unsigned long long* tile_est = nullptr;  // 2 device counters for the tile estimates
  long long last_tile_estimate[2] = {0, 0};
  int since_reorder = 0;
  int label_sweeps = 0;
  float2* y_b = nullptr;    // centred layout of the current iteration (also scratch)
  float2* grad = nullptr;
  // Attraction over tiled P (kernel k_attract_tiles_seg) unless disabled; the
  // tiles follow the working numbering and are rebuilt after it changes.
  bool attract_tiled = true;
  // Workgroups per CU of the attraction when it runs beside the repulsion
  // kernels, possibly fractional: fewer than the 3 its LDS allows leave room
  // on every CU for the latency-bound repulsion chain, whose waves also take
  // issue priority (chain_priority).  Set by FASTEMBEDR_HIP_ATTRACT_SHARED_PER_CU,
  // else (attract_share_auto) after each tile build from the tiled P's mean
  // run length, which sets the attraction's cost per entry against the
  // chain's per point.  Bilinear grid: 2 at 16K slots per run or more, 2.5 at
  // 8K or fewer, linear between (config 2, runs of 25k slots, late window:
  // 2 3906 / 3877 it/s, 2.5 3735 / 3764).  Interpolation grid: 2 at 24K
  // slots per run or more, 3 at 8K or fewer, linear between (config 2,
  // late window: 1.5 3719, 1.75 3710 / 3722, 2 3811 / 3837 / 3823,
  // 2.25 3773 / 3774, 2.5 3743; config 4, runs of 7.4k slots: 2.75 895 / 899,
  // 3 919 / 916 / 918).  Alone it takes one workgroup per row block.
  double attract_shared_per_cu = 2.0;
  bool attract_share_auto = true;
  double attract_share_base = 2.0;     // bilinear grid, from the last tile build
  double attract_share_base_lg = 2.5;  // interpolation grid, same
  double attract_share() const {
    if (!attract_share_auto) return attract_shared_per_cu;
    return repulsion == FASTEMBEDR_HIP_REPULSION_LAGRANGE ? attract_share_base_lg : attract_share_base;
  }
  // Workgroups per CU of the helper launch that joins the attraction on the
  // main stream once the repulsion chain is done, taking over the row blocks
  // still unclaimed (FASTEMBEDR_HIP_ATTRACT_HELPER_PER_CU; 0: none).  The
  // pair adapts to the balance of the two: a short chain leaves the helper
  // most of the attraction, a long one leaves it nothing.
  double attract_helper_per_cu = 1.0;
  // The attraction on the stream of the previous update and the repulsion
  // chain on the other one of `stream` and side_attr (the default;
  // FASTEMBEDR_HIP_ATTRACT_MAIN=0: the attraction on side_attr with a helper
  // launch on the main stream after the chain, which runs on `stream`); the
  // attraction then takes attract_share() workgroups per CU and no helper
  // (3270 against 3205 it/s in the late window at config 2, 3409 against
  // 3340 over the whole schedule).
  bool attract_main = true;
  int helper_pending = 0;            // helper workgroups per XCD still to launch this iteration
  int helper_slots = 0;              // the primary's workgroups per XCD
  bool helper_span_open = false;     // the attraction's timed span ends after the helper
  std::size_t helper_span = 0;
  int cus = 0;  // compute units of the device
  fehip::Tiles tiles;
  int tiles_for = -2;       // value of wi the tiles were built for; -2: none
  // Repulsion used by run(): the bilinear grid (reference) or the FIt-SNE
  // interpolation grid.  The interpolation buffers are allocated on first use.
  int repulsion = FASTEMBEDR_HIP_REPULSION_GRID;
  int lg_min_intervals = 50;
  float lg_ints_per_unit = 1.0f;
  bool lg_ready = false;
  Arena lg_arena;
  fehip::InterpBuffers ib;
  int lg_last_fft = 0;       // FFT length of the last interpolation-grid iteration
  // The spread's LDS table: the small one (fehip::kLgSmallTableBits) when
  // the latest known box count leaves at least lg_dense_points points per
  // box on average, so that a chunk of the spread order touches few boxes
  // (FASTEMBEDR_HIP_SPREAD_DENSE: that threshold; 0 keeps the large table).
  int lg_table_bits = fehip::kLgTableBits;
  double lg_dense_points = 32.0;
  // The spread's point order (working indices sorted by position) is made
  // again every lg_order_period interpolation-grid iterations, on first use
  // and after a renumbering (stale), and for every gradient probe.  Any
  // permutation gives the same charges (up to the order of fp32 adds); a
  // spatial one keeps the spread's runs long.  lg_order_due asks the next
  // gradient pieces to make it before the spread.  Config 2, whole schedule:
  // 4118 / 4156 / 4140 it/s at periods 32 / 64 / 128 (a refresh costs ~0.2 ms
  // beside the attraction; the spread slows as the order ages, less since it
  // groups each wave's points by box; at periods 16 / 32 / 48 before that,
  // 3664 / 3690 / 3677); the working order itself (period 0,
  // FASTEMBEDR_HIP_LG_ORDER_PERIOD) is far from spatial late in the run
  // (spread 109 us instead of 36 before the grouping).
  int lg_order_period = 64;
  // Attraction tile shape (fehip::tiles_shape): 0 by point count, 1 the
  // 1024 x 4096 tiles, 2 the 2048 x 2048 ones (FASTEMBEDR_HIP_TILE_SHAPE).
  int tile_shape = 0;
  bool lg_order_stale = true;
  bool lg_order_due = false;
  int lg_order_age = 0;
  // Box counts of recent iterations: a pinned coherent ring that the
  // update's statistics kernel writes, slot DeviceScalars::ring_seq % kLgRing
  // = (ring_seq << 32) | boxes, before it advances ring_seq.  The host reads
  // it directly (no event per iteration).
  static constexpr int kLgRing = fehip::kBoxRing;
  unsigned long long* lg_ring = nullptr;
  unsigned long long* lg_ring_dev = nullptr;  // the ring's device address

  // Replayed iterations (FASTEMBEDR_HIP_GRAPH_CAPTURE, off by default): one
  // iteration's launches (gradient pieces + update) on the main stream alone
  // are captured into a graph keyed by everything the launches bake in, and
  // replayed with one hipGraphLaunch.  A key is captured the second time it
  // is met (a one-off FFT length is not worth an instantiation); renumbering,
  // the attraction's tile build and timed runs stay eager.  The captured
  // iteration is single-stream: on ROCm 7 a graph with parallel branches,
  // once launched, keeps the allocations its side-branch kernels read from
  // being returned by hipFree until the next device-wide synchronisation
  // (4.7 GB per session at config 2, piling up over sessions), which a
  // single-stream graph does not.
  struct IterGraph {
    std::array<std::uint32_t, 15> key{};
    hipGraphExec_t exec = nullptr;
    int seen = 0;
    unsigned long long last_use = 0;
  };
  static constexpr std::size_t kMaxGraphs = 8;
  bool graph_capture = false;
  std::vector<IterGraph> graphs;
  unsigned long long graph_clock = 0;
  long long graph_launches = 0;
  int graph_captures = 0;

  bool renumbered() const { return wi >= 0; }
  const Csr& work_p() const { return wi < 0 ? p : pw[wi]; }
  float2* y_a() const { return ys[si]; }
  float2* update() const { return us[si]; }
  float2* gains() const { return gs[si]; }
  float2* exact_rep = nullptr;
  float2* attr = nullptr;   // attractive term per row (working numbering)
  float2* tw = nullptr;
  BlockStats* partial = nullptr;
  double* dpartial = nullptr;
  int dpartial_len = 0;
  GridBuffers gb;
  double p_build_ms = 0.0;
  bool timing = false;
  int timed_only = -1;      // >= 0: time only this kernel id (others run without events)
  int timing_every = 1;     // with timed_only: time it on every timing_every-th iteration
  long long timing_iter = 0;  // iterations run since timing was enabled
  std::vector<hipEvent_t> events;
  std::vector<int> event_kernel;
  long long launches[fehip::kKernelCount] = {};
  double total_ms[fehip::kKernelCount] = {};

  ~fastembedr_hip_tsne() {
    if (stream != nullptr) (void)hipStreamSynchronize(stream);
    for (IterGraph& g : graphs) {
      if (g.exec != nullptr) (void)hipGraphExecDestroy(g.exec);
    }
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    if (lg_ring != nullptr) (void)hipHostFree(lg_ring);
    lg_arena.release();
    for (hipStream_t st : {side_attr, side_kern}) {
      if (st != nullptr) (void)hipStreamSynchronize(st);
    }
    for (hipEvent_t e : {ev_layout, ev_ready, ev_attr, ev_kern, ev_home}) {
      if (e != nullptr) (void)hipEventDestroy(e);
    }
    tile_arena.release();
    work_arena.release();
    arena.release();
    for (hipStream_t st : {stream, side_attr, side_kern}) {
      if (st != nullptr) (void)hipStreamDestroy(st);
    }
  }

  bool records(int kernel_id) const {
    return timing && (timed_only < 0 || (timed_only == kernel_id && timing_iter % timing_every == 0));
  }

  // Opens a timed span of kernel_id with an event on stream `on`; *slot names
  // it for span_end (the end may be recorded on another stream).
  bool span_begin(int kernel_id, hipStream_t on, std::size_t* slot) {
    *slot = event_kernel.size();
    while (events.size() < 2 * (*slot + 1)) {
      hipEvent_t e;
      if (!hip_ok(hipEventCreate(&e), "hipEventCreate")) return false;
      events.push_back(e);
    }
    event_kernel.push_back(kernel_id);
    return hip_ok(hipEventRecord(events[2 * *slot], on), "hipEventRecord");
  }
  bool span_end(std::size_t slot, hipStream_t on) {
    return hip_ok(hipEventRecord(events[2 * slot + 1], on), "hipEventRecord");
  }

  // Enqueues one kernel, bracketed by events on stream `on` (the main stream
  // by default) when timing is on.
  template <typename Launch>
  bool timed(int kernel_id, const char* what, Launch&& launch, hipStream_t on = nullptr) {
    if (on == nullptr) on = stream;
    std::size_t slot = 0;
    const bool record = records(kernel_id);
    if (record && !span_begin(kernel_id, on, &slot)) return false;
    if (!hip_ok(launch(), what)) return false;
    return !record || span_end(slot, on);
  }

  bool sync_all() {
    for (hipStream_t st : {stream, side_attr, side_kern}) {
      if (st != nullptr && !hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize")) return false;
    }
    return true;
  }

  bool harvest_timing() {
    if (!timing || event_kernel.empty()) return true;
    if (!sync_all()) return false;
    for (std::size_t s = 0; s < event_kernel.size(); ++s) {
      float ms = 0.0f;
      if (!hip_ok(hipEventElapsedTime(&ms, events[2 * s], events[2 * s + 1]), "hipEventElapsedTime")) return false;
      launches[event_kernel[s]] += 1;
      total_ms[event_kernel[s]] += ms;
    }
    event_kernel.clear();
    return true;
  }
};

namespace {

const char* kKernelNames[fehip::kKernelCount] = {
    "stats", "bin_count", "bin_plan", "bin_scatter", "spread", "kernel_rows", "kernel_cols", "charge_rows",
    "conv_cols", "inverse_rows", "attract", "update", "commit", "renumber", "tile_build",
    "interp_order", "interp_spread",
    "interp_kernel_rows", "interp_kernel_cols", "interp_charge_rows", "interp_conv_cols", "interp_inverse_rows",
    "finalize_stats", "repulsion"};

int key_bits_for(int n) {
  int b = 1;
  while ((1LL << b) <= static_cast<long long>(n)) ++b;
  return b;
}

bool upload_twiddles(fastembedr_hip_tsne* s) {
  std::vector<float2> host(fehip::kTwiddleLen);
  for (int m = 0; m < fehip::kTwiddleLen; ++m) {
    const bool pow2 = m < fehip::kTwiddlePow2;
    const double ang = -2.0 * M_PI * static_cast<double>(pow2 ? m : m - fehip::kTwiddlePow2) /
                       static_cast<double>(pow2 ? fehip::kTwiddlePow2 : fehip::kTwiddlePow3);
    host[m] = make_float2(static_cast<float>(std::cos(ang)), static_cast<float>(std::sin(ang)));
  }
  // Synchronous: `host` is released when this function returns.
  return hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(twiddles)") &&
         hip_ok(hipMemcpy(s->tw, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice),
                "hipMemcpy(twiddles)");
}

// Working-numbering buffers: two CSR copies, permutations, the second half of
// the state double buffers and the renumbering scratch.  perm starts as the
// identity, so until the first renumbering the working numbering is the
// caller's.
bool alloc_working_buffers(fastembedr_hip_tsne* s) {
  const int n = s->n;
  const std::size_t nnz = static_cast<std::size_t>(s->p.nnz);
  std::size_t temp = 0;
  if (!hip_ok(fehip::renumber_temp_bytes(n, temp), "renumber size query")) return false;
  const std::size_t nn = static_cast<std::size_t>(n);
  const std::size_t bytes = 2 * (align_up((nn + 1) * 4) + align_up(nnz * 4) + align_up(nnz * 4)) +
                            3 * align_up(nn * 4) + 3 * align_up(nn * sizeof(float2)) + 2 * align_up(nn * 8) +
                            4 * align_up(nn * 4) + align_up((nn + 1) * 4) + align_up(temp) + 3 * 256 + 4096;
  if (!memory_preflight(bytes, "HIP openTSNE working buffers") ||
      !s->work_arena.init(bytes, "hipMalloc(HIP openTSNE working buffers)")) {
    return false;
  }
  Arena& a = s->work_arena;
  for (int w = 0; w < 2; ++w) {
    s->pw[w].n = n;
    s->pw[w].nnz = s->p.nnz;
    s->pw[w].row_ptr = a.take<int>(nn + 1);
    s->pw[w].col = a.take<int>(nnz);
    s->pw[w].val = a.take<float>(nnz);
  }
  s->perm[0] = a.take<int>(nn);
  s->perm[1] = a.take<int>(nn);
  s->inv_perm = a.take<int>(nn);
  s->ys[1] = a.take<float2>(nn);
  s->us[1] = a.take<float2>(nn);
  s->gs[1] = a.take<float2>(nn);
  s->rn.keys_in = a.take<unsigned long long>(nn);
  s->rn.keys_out = a.take<unsigned long long>(nn);
  s->rn.idx_in = a.take<int>(nn);
  s->rn.order = a.take<int>(nn);
  s->rn.map = a.take<int>(nn);
  s->rn.len = a.take<int>(nn + 1);
  int* component = a.take<int>(nn);
  int* changed = a.take<int>(1);
  s->tile_est = a.take<unsigned long long>(2);
  s->rn.component = component;
  s->rn.temp = a.take<char>(temp);
  s->rn.temp_bytes = temp;
  if (s->rn.temp == nullptr || changed == nullptr || s->tile_est == nullptr) {
    set_error("internal: working buffers do not fit their arena");
    return false;
  }
  std::vector<int> iota(nn);
  for (int i = 0; i < n; ++i) iota[static_cast<std::size_t>(i)] = i;
  if (!hip_ok(hipMemcpy(s->perm[0], iota.data(), nn * 4, hipMemcpyHostToDevice), "perm init") ||
      !hip_ok(hipMemcpy(s->inv_perm, iota.data(), nn * 4, hipMemcpyHostToDevice), "perm init")) {
    return false;
  }
  // Connected components of P (fixed for the session): renumbering keeps
  // each component contiguous.  Sort keys use 32 + bits(n) bits.
  if (!hip_ok(fehip::launch_label_init(component, n, s->stream), "label init")) return false;
  int flag = 1;
  for (int sweep = 0; flag != 0 && sweep < 256; ++sweep) {
    flag = 0;
    if (!hip_ok(hipMemsetAsync(changed, 0, sizeof(int), s->stream), "label flag") ||
        !hip_ok(fehip::launch_label_step(s->p, component, changed, s->stream), "label step") ||
        !hip_ok(hipMemcpyAsync(&flag, changed, sizeof(int), hipMemcpyDeviceToHost, s->stream), "label flag") ||
        !hip_ok(hipStreamSynchronize(s->stream), "label sync")) {
      return false;
    }
    s->label_sweeps = sweep + 1;
  }
  int bits = 1;
  while ((1LL << bits) <= static_cast<long long>(n)) ++bits;
  s->rn.key_bits = 32 + bits;
  return true;
}

// Tiled P and its build scratch (see fehip::Tiles).  The sort scratch is
// sized for the whole of P and kept for the session, so rebuilding after a
// renumbering allocates nothing.
bool alloc_tiles(fastembedr_hip_tsne* s) {
  fehip::Tiles& t = s->tiles;
  fehip::tiles_shape(s->n, s->p.nnz, t, s->tile_shape);
  if (t.key_bits > 32 || t.padded > static_cast<long long>(std::numeric_limits<int>::max())) {
    s->attract_tiled = false;  // beyond a 32-bit sort key or int offsets: row-parallel attraction
    return true;
  }
  std::size_t temp = 0;
  if (!hip_ok(fehip::tiles_temp_bytes(t, temp), "tile build size query")) return false;
  const std::size_t nnz = static_cast<std::size_t>(std::max<long long>(t.nnz, 1));
  const std::size_t padded = static_cast<std::size_t>(std::max<long long>(t.padded, 1));
  const std::size_t slots = static_cast<std::size_t>(t.max_tiles) + 1;
  const std::size_t bytes = align_up(padded * 2) + align_up(padded * 4) + align_up((padded / 8 + 1) * 2) +
                            2 * align_up(nnz * 4) + 2 * align_up(nnz * 8) +
                            align_up((static_cast<std::size_t>(t.row_blocks) + 1) * 4) + 4 * align_up(slots * 4) +
                            align_up(4) + align_up((fehip::kTileMaxXcds + 1) * 4) + align_up(temp) + 4096;
  if (!memory_preflight(bytes, "HIP openTSNE attraction tiles") ||
      !s->tile_arena.init(bytes, "hipMalloc(HIP openTSNE attraction tiles)")) {
    return false;
  }
  Arena& a = s->tile_arena;
  t.ent = a.take<unsigned short>(padded);
  t.val = a.take<float>(padded);
  t.key_in = a.take<unsigned int>(nnz);
  t.key_out = a.take<unsigned int>(nnz);
  t.pay_in = a.take<unsigned long long>(nnz);
  t.pay_out = a.take<unsigned long long>(nnz);
  t.tile_ptr = a.take<int>(static_cast<std::size_t>(t.row_blocks) + 1);
  t.tile_cb = a.take<int>(slots);
  t.tile_beg = a.take<int>(slots);
  t.ubeg = a.take<int>(slots);
  t.psize = a.take<int>(slots);
  t.tile_count = a.take<int>(1);
  t.work = a.take<unsigned int>(fehip::kTileMaxXcds + 1);
  t.base_row = a.take<unsigned short>(padded / 8 + 1);
  t.temp = a.take<char>(std::max<std::size_t>(temp, 1));
  t.temp_bytes = temp;
  if (t.temp == nullptr) {
    set_error("internal: attraction tiles do not fit their arena");
    return false;
  }
  return hip_ok(hipMemsetAsync(t.work, 0, (fehip::kTileMaxXcds + 1) * sizeof(unsigned int), s->stream),
                "hipMemset(attraction claims)");
}

// Builds the attraction's tiles for the current working numbering on stream
// st, unless they are built already.
bool ensure_tiles(fastembedr_hip_tsne* s, hipStream_t st) {
  if (!s->attract_tiled || s->tiles_for == s->wi) return true;
  if (!s->timed(
          fehip::kKTileBuild, "tile build", [&] { return fehip::launch_tile_build(s->work_p(), s->tiles, st); }, st)) {
    return false;
  }
  s->tiles_for = s->wi;
  if (!s->attract_share_auto) return true;
  // the attraction's share beside the chain from the mean run length (a
  // synchronous read, once per build)
  int count = 0, total = 0;
  if (!hip_ok(hipMemcpyAsync(&count, s->tiles.tile_count, sizeof(int), hipMemcpyDeviceToHost, st), "tile count") ||
      !hip_ok(hipStreamSynchronize(st), "tile count") ||
      !hip_ok(hipMemcpyAsync(&total, s->tiles.tile_beg + count, sizeof(int), hipMemcpyDeviceToHost, st),
              "tile slots") ||
      !hip_ok(hipStreamSynchronize(st), "tile slots")) {
    return false;
  }
  const double run = count > 0 ? static_cast<double>(total) / count : 0.0;
  s->attract_share_base = std::clamp(2.5 - (run - 8192.0) / 16384.0, 2.0, 2.5);
  s->attract_share_base_lg = std::clamp(3.0 - (run - 8192.0) / 16384.0, 2.0, 3.0);
  return true;
}

// Workgroups per XCD for `per_cu` workgroups per CU (at least one).
int per_xcd_for(const fastembedr_hip_tsne* s, double per_cu) {
  return std::max(1, static_cast<int>(std::lround(per_cu * std::max(1, s->cus / s->xcds))));
}

// Attractive term of every row into s->attr at the centred layout y_cur, on
// stream st (the main stream when null); `shared`: other kernels run beside
// it, and (tiled attraction) a helper launch follows on the main stream
// (enqueue_attract_helper) once they are done.
// done (optional): recorded on st right after the kernel, ahead of the
// timing event that closes its span, so that a stream waiting for it does
// not wait behind that event as well.
bool enqueue_attract(fastembedr_hip_tsne* s, const float2* y_cur, float exaggeration, hipStream_t st = nullptr,
                     bool shared = false, hipEvent_t done = nullptr) {
  if (st == nullptr) st = s->stream;
  auto then_done = [&](hipError_t e) { return e == hipSuccess && done != nullptr ? hipEventRecord(done, st) : e; };
  s->helper_pending = 0;
  s->helper_span_open = false;
  if (!s->attract_tiled) {
    return s->timed(
        fehip::kKAttract, "attract launch",
        [&] {
          return then_done(fehip::launch_attract(s->work_p(), y_cur, s->attr, exaggeration, s->lanes, s->xcds, st));
        },
        st);
  }
  if (!ensure_tiles(s, st)) return false;  // may set attract_share_base
  const double per_cu = s->attract_share();
  const bool share = shared && s->cus > 0 && per_cu > 0.0;
  const int slots = share ? per_xcd_for(s, per_cu) : 0;
  const int helper =
      share && !s->attract_main && s->attract_helper_per_cu > 0.0 ? per_xcd_for(s, s->attract_helper_per_cu) : 0;
  if (helper == 0) {
    // the launch completes `done` itself (no marker behind the kernel)
    return s->timed(
        fehip::kKAttract, "attract launch",
        [&] {
          return s->mark_layout
                     ? fehip::launch_attract_tiled(s->tiles, y_cur, s->attr, exaggeration, s->xcds, slots, 0, st, done)
                     : then_done(
                           fehip::launch_attract_tiled(s->tiles, y_cur, s->attr, exaggeration, s->xcds, slots, 0, st));
        },
        st);
  }
  // the timed span runs from the primary's start to the point where the
  // main stream has both (see enqueue_attract_helper)
  if (s->records(fehip::kKAttract) && !s->span_begin(fehip::kKAttract, st, &s->helper_span)) return false;
  s->helper_span_open = s->records(fehip::kKAttract);
  s->helper_pending = helper;
  s->helper_slots = slots;
  return hip_ok(fehip::launch_attract_tiled(s->tiles, y_cur, s->attr, exaggeration, s->xcds, slots, helper, st),
                "attract launch");
}

// The helper launch of a shared tiled attraction, on the main stream, then
// the main stream's wait for the primary (event done_attr on its stream).
bool enqueue_attract_helper(fastembedr_hip_tsne* s, const float2* y_cur, float exaggeration, hipEvent_t done_attr) {
  if (s->helper_pending > 0 &&
      !hip_ok(fehip::launch_attract_tiled_helper(s->tiles, y_cur, s->attr, exaggeration, s->xcds, s->helper_slots,
                                                 s->helper_pending, s->stream),
              "attract helper launch")) {
    return false;
  }
  s->helper_pending = 0;
  if (!hip_ok(hipStreamWaitEvent(s->stream, done_attr, 0), "hipStreamWaitEvent(main, attraction)")) return false;
  if (s->helper_span_open) {
    s->helper_span_open = false;
    return s->span_end(s->helper_span, s->stream);
  }
  return true;
}

// The spread's table for a layout of about `boxes` boxes per axis.
void set_spread_table(fastembedr_hip_tsne* s, int boxes) {
  const double per_box = static_cast<double>(s->n) / std::max(1.0, static_cast<double>(boxes) * boxes);
  s->lg_table_bits =
      s->lg_dense_points > 0.0 && per_box >= s->lg_dense_points ? fehip::kLgSmallTableBits : fehip::kLgTableBits;
}

// FFT length for an interpolation grid of `nodes` nodes per axis: the
// smallest 2^a or 3 * 2^a >= 2 * nodes (a zero-padded linear convolution;
// the transforms take radix 3 once), at least 64, at most kLgMaxFft.
int interp_fft_len(int nodes) {
  int f = 64;
  while (f < 2 * nodes && f < fehip::kLgMaxFft) f = (f & (f - 1)) == 0 ? f / 2 * 3 : f / 3 * 4;
  return f;
}

// Interpolation-grid buffers (sized for the largest grid) and the pinned ring
// of box counts; allocated once per session.
bool ensure_interp(fastembedr_hip_tsne* s) {
  if (s->lg_ready) return true;
  const std::size_t n = static_cast<std::size_t>(s->n);
  const std::size_t mn = fehip::kLgMaxNodes;
  const std::size_t gmax = fehip::kLgMaxFft / 2;
  const std::size_t hmax = gmax + 1;
  std::size_t sort_bytes = 0;
  if (!hip_ok(fehip::interp_order_temp_bytes(s->n, sort_bytes), "interp order size query")) return false;
  constexpr std::size_t kSums = fehip::kLgSumsPerBox;
  const std::size_t boxes = static_cast<std::size_t>(fehip::kLgMaxBoxes) * fehip::kLgMaxBoxes;
  const std::size_t bytes = align_up(mn * mn * sizeof(float)) + align_up(mn * mn * sizeof(float4)) +
                            2 * align_up(2 * hmax * hmax * sizeof(float2)) +
                            2 * align_up(3 * gmax * hmax * sizeof(float2)) +
                            align_up(fehip::kLgZPartials * sizeof(double)) + 2 * align_up(n * sizeof(int)) +
                            align_up(2 * n * sizeof(unsigned int)) + align_up(sort_bytes) +
                            align_up(static_cast<std::size_t>(fehip::kLgEntryPool) * kSums * sizeof(float)) +
                            align_up(boxes * sizeof(int)) + align_up(boxes * kSums * sizeof(float)) + 4096;
  if (!memory_preflight(bytes, "HIP openTSNE interpolation grid") ||
      !s->lg_arena.init(bytes, "hipMalloc(HIP openTSNE interpolation grid)")) {
    return false;
  }
  Arena& a = s->lg_arena;
  fehip::InterpBuffers& ib = s->ib;
  ib.m2 = a.take<float>(mn * mn);
  ib.field = a.take<float4>(mn * mn);
  ib.k_rows = a.take<float2>(2 * hmax * hmax);
  ib.k_cols = a.take<float2>(2 * hmax * hmax);
  ib.spec_a = a.take<float2>(3 * gmax * hmax);
  ib.spec_b = a.take<float2>(3 * gmax * hmax);
  ib.z_partial = a.take<double>(fehip::kLgZPartials);
  ib.order = a.take<int>(n);
  ib.order_idx = a.take<int>(n);
  ib.order_keys = a.take<unsigned int>(2 * n);
  ib.order_temp = a.take<unsigned char>(std::max<std::size_t>(sort_bytes, 1));
  ib.order_temp_bytes = sort_bytes;
  ib.entries = a.take<float>(static_cast<std::size_t>(fehip::kLgEntryPool) * kSums);
  ib.box_count = a.take<int>(boxes);
  ib.straggler = a.take<float>(boxes * kSums);
  s->lg_order_stale = true;
  if (ib.straggler == nullptr) {
    set_error("internal: interpolation grid buffers do not fit their arena");
    return false;
  }
  // the box counts and the straggler planes are zero between iterations
  // (each gather clears what it read)
  if (!hip_ok(hipMemsetAsync(ib.box_count, 0, boxes * sizeof(int), s->stream), "hipMemset(interpolation boxes)") ||
      !hip_ok(hipMemsetAsync(ib.straggler, 0, boxes * kSums * sizeof(float), s->stream),
              "hipMemset(interpolation stragglers)") ||
      !hip_ok(hipHostMalloc(reinterpret_cast<void**>(&s->lg_ring),
                            fastembedr_hip_tsne::kLgRing * sizeof(unsigned long long),
                            hipHostMallocMapped | hipHostMallocCoherent),
              "hipHostMalloc(box ring)") ||
      !hip_ok(hipHostGetDevicePointer(reinterpret_cast<void**>(&s->lg_ring_dev), s->lg_ring, 0),
              "hipHostGetDevicePointer(box ring)")) {
    return false;
  }
  // no sequence number the device writes before 2^32 updates
  for (int r = 0; r < fastembedr_hip_tsne::kLgRing; ++r) __atomic_store_n(s->lg_ring + r, ~0ull, __ATOMIC_RELEASE);
  s->lg_ready = true;
  return true;
}

// Writes the interpolation-grid specification into DeviceScalars, so that the
// statistics finalize computes its geometry (order 0 switches it off).
bool write_interp_spec(fastembedr_hip_tsne* s, int order) {
  struct Spec {
    int order, min_intervals;
    float ints_per_unit;
  } spec{order, s->lg_min_intervals, s->lg_ints_per_unit};
  static_assert(offsetof(DeviceScalars, lg_min_intervals) == offsetof(DeviceScalars, lg_order) + 4 &&
                    offsetof(DeviceScalars, lg_ints_per_unit) == offsetof(DeviceScalars, lg_order) + 8,
                "specification fields are contiguous");
  char* dst = reinterpret_cast<char*>(s->sc) + offsetof(DeviceScalars, lg_order);
  return hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(interp spec)") &&
         hip_ok(hipMemcpy(dst, &spec, sizeof(spec), hipMemcpyHostToDevice), "hipMemcpy(interp spec)");
}

// One iteration's gradient pieces.  With the bilinear grid the centred
// layout goes to y_b (the interpolation grid's spread and update centre the
// stored layout themselves, the spread reading it in its spatial order); the
// attraction of the layout goes to attr; the repulsion fields (bilinear grid or
// interpolation grid at FFT length fft_len) to the grid buffers.  With
// `finalize` the previous update's statistics are finished first (the grid
// geometry of this iteration; with the interpolation grid the box count also
// goes to the host's ring).  With `overlap` the attraction and the kernel
// spectrum run on the side streams and the main stream waits for them (before
// the convolution and before whatever follows this call); without it
// everything runs on the main stream.
// Hands the latest update back to the main stream (`stream` waits for
// `home`), for work that is enqueued there.
bool settle(fastembedr_hip_tsne* s) {
  s->layout_at_tail = false;
  if (s->home == s->stream) return true;
  if (!hip_ok(hipEventRecord(s->ev_home, s->home), "hipEventRecord(home)") ||
      !hip_ok(hipStreamWaitEvent(s->stream, s->ev_home, 0), "hipStreamWaitEvent(home)")) {
    return false;
  }
  s->home = s->stream;
  return true;
}

bool enqueue_gradient_pieces(fastembedr_hip_tsne* s, bool lg, int fft_len, float exaggeration, bool overlap,
                             bool finalize = false) {
  const int n = s->n;
  fehip::InterpBuffers& ib = s->ib;
  // The attraction's stream: the one that holds the latest update (the other
  // of the pair runs the chain); everything else starts from `stream`.
  if (!(overlap && s->attract_main) && !settle(s)) return false;
  const bool layout_marked = overlap && s->layout_at_tail;
  s->layout_at_tail = false;
  hipStream_t main = s->home;
  hipStream_t other = main == s->stream ? s->side_attr : s->stream;
  // Two arrangements of an overlapped iteration.  Attraction first
  // (attract_main, the default): the attraction runs on the stream of the
  // previous update, right behind it, and the chain on the other stream,
  // which then carries the update (update_on_chain) or hands it back.
  // Attraction beside (attract_main off): the attraction runs on side_attr
  // from the top of the iteration, the chain on `stream`, and a helper
  // launch joins the attraction once the chain is done.
  const bool swap = overlap && s->attract_main;
  hipStream_t sa = overlap && !swap ? other : main;  // attraction
  hipStream_t chain = swap ? other : main;           // repulsion chain
  hipStream_t sk = overlap ? s->side_kern : main;
  if (lg) s->lg_last_fft = fft_len;
  // The attraction needs only differences y_i - y_j, so it reads the stored
  // layout (no centring) and starts at once, beside the statistics' finish
  // and the whole repulsion chain.
  if (overlap && !swap &&
      ((!layout_marked && !hip_ok(hipEventRecord(s->ev_layout, main), "hipEventRecord(layout)")) ||
       !hip_ok(hipStreamWaitEvent(sa, s->ev_layout, 0), "hipStreamWaitEvent(attraction)"))) {
    return false;
  }
  if (!swap && (!enqueue_attract(s, s->y_a(), exaggeration, sa, overlap) ||
                (overlap && !hip_ok(hipEventRecord(s->ev_attr, sa), "hipEventRecord(attraction)")))) {
    return false;
  }
  // With the attraction on the main stream, the statistics' finish heads the
  // chain's stream, so the attraction starts right after the previous update
  // (config 2, late window: 3298 -> 3392 it/s).
  const bool fin_chain = swap;
  hipStream_t fin = fin_chain ? chain : main;
  if (fin_chain && ((!layout_marked && !hip_ok(hipEventRecord(s->ev_layout, main), "hipEventRecord(layout)")) ||
               !hip_ok(hipStreamWaitEvent(chain, s->ev_layout, 0), "hipStreamWaitEvent(chain)"))) {
    return false;
  }
  if (finalize && !s->timed(
                      fehip::kKFinalize, "finalize launch",
                      [&] {
                        return fehip::launch_finalize_stats(s->partial, n, s->gb.g, s->sc,
                                                            lg ? s->lg_ring_dev : nullptr, fin);
                      },
                      fin)) {
    return false;
  }
  // The kernel spectrum needs only the node spacing of the geometry.
  if (overlap && (!hip_ok(hipEventRecord(s->ev_ready, fin), "hipEventRecord(ready)") ||
                  !hip_ok(hipStreamWaitEvent(sk, s->ev_ready, 0), "hipStreamWaitEvent(kernel)") ||
                  (swap && !fin_chain && !hip_ok(hipStreamWaitEvent(chain, s->ev_ready, 0), "hipStreamWaitEvent(chain)")))) {
    return false;
  }
  if (swap && !enqueue_attract(s, s->y_a(), exaggeration, main, true, s->update_on_chain ? s->ev_attr : nullptr)) {
    return false;
  }
  // Run in sequence (no overlap), the repulsion step's kernels are
  // contiguous on the main stream from the kernel spectrum to the
  // potentials: with the step the one id timed, two events bracket them all.
  std::size_t rep_slot = 0;
  const bool rep_span = !overlap && s->timed_only == fehip::kKRepulsion && s->records(fehip::kKRepulsion);
  if (rep_span && !s->span_begin(fehip::kKRepulsion, main, &rep_slot)) return false;
  if (lg) {
    static constexpr int kIds[2] = {fehip::kKLgKernelRows, fehip::kKLgKernelCols};
    static constexpr int kSteps[2] = {0, 2};
    for (int q = 0; q < 2; ++q) {
      if (!s->timed(
              kIds[q], "interpolation-grid kernel launch",
              [&] { return fehip::launch_interp_fft(kSteps[q], fft_len, ib, s->sc, s->tw, n, sk); }, sk)) {
        return false;
      }
    }
  } else if (!s->timed(
                 fehip::kKKernelRows, "kernel_rows launch",
                 [&] { return fehip::launch_kernel_rows(s->gb, s->sc, s->tw, sk); }, sk) ||
             !s->timed(
                 fehip::kKKernelCols, "kernel_cols launch",
                 [&] { return fehip::launch_kernel_cols(s->gb, s->tw, sk); }, sk)) {
    return false;
  }
  if (overlap && !hip_ok(hipEventRecord(s->ev_kern, sk), "hipEventRecord(kernel)")) return false;
  // chain: centre + count (the interpolation grid's spread centres the
  // layout itself)
  if (!lg && !s->timed(
                 fehip::kKBinCount, "bin_count launch",
                 [&] { return fehip::launch_bin_count(s->y_a(), s->y_b, s->sc, s->gb, n, chain); }, chain)) {
    return false;
  }
  // chain: bins, spread, charge transforms
  bool ok;
  if (lg) {
    if (s->lg_order_due) {
      // the spread order of this iteration's layout (any order is correct;
      // a spatial one keeps the spread's runs of one box long)
      if (!s->timed(
              fehip::kKLgOrder, "interp order launch",
              [&] { return fehip::launch_interp_order(s->y_a(), s->sc, ib, n, fft_len, chain); }, chain)) {
        return false;
      }
      s->lg_order_due = false;
      s->lg_order_stale = false;
      s->lg_order_age = 0;
    }
    ok = s->timed(
             fehip::kKLgSpread, "interp spread launch",
             [&] {
               return fehip::launch_interp_spread(s->y_a(), s->lg_order_period > 0 ? ib.order : nullptr, s->sc, ib,
                                                  n, fft_len, s->lg_table_bits, chain);
             },
             chain) &&
         s->timed(
             fehip::kKLgChargeRows, "interp charge_rows launch",
             [&] { return fehip::launch_interp_fft(3, fft_len, ib, s->sc, s->tw, n, chain); }, chain);
  } else {
    ok = s->timed(
             fehip::kKBinPlan, "bin_plan launch", [&] { return fehip::launch_bin_plan(s->gb, s->sc, chain); },
             chain) &&
         s->timed(
             fehip::kKBinScatter, "bin_scatter launch",
             [&] { return fehip::launch_bin_scatter(s->y_b, s->sc, s->gb, n, chain); }, chain) &&
         s->timed(
             fehip::kKSpread, "spread launch", [&] { return fehip::launch_spread_tiles(s->sc, s->gb, n, chain); },
             chain) &&
         s->timed(
             fehip::kKChargeRows, "charge_rows launch",
             [&] { return fehip::launch_charge_rows(s->gb, s->tw, chain); }, chain);
  }
  if (!ok) return false;
  if (overlap && !hip_ok(hipStreamWaitEvent(chain, s->ev_kern, 0), "hipStreamWaitEvent(chain, kernel)")) {
    return false;
  }
  // chain: convolution and potentials
  if (lg) {
    ok = s->timed(
             fehip::kKLgConvCols, "interp conv_cols launch",
             [&] { return fehip::launch_interp_fft(5, fft_len, ib, s->sc, s->tw, n, chain); }, chain) &&
         s->timed(
             fehip::kKLgInverseRows, "interp inverse_rows launch",
             [&] { return fehip::launch_interp_fft(7, fft_len, ib, s->sc, s->tw, n, chain); }, chain);
  } else {
    ok = s->timed(
             fehip::kKConvCols, "conv_cols launch", [&] { return fehip::launch_conv_cols(s->gb, s->tw, chain); },
             chain) &&
         s->timed(
             fehip::kKInverseRows, "inverse_rows launch",
             [&] { return fehip::launch_inverse_rows(s->gb, s->tw, n, s->sc, chain); }, chain);
  }
  if (!ok || (rep_span && !s->span_end(rep_slot, main))) return false;
  if (swap) {
    if (s->update_on_chain) {
      // the chain's stream waits for the attraction (ev_attr, recorded right
      // after it) and carries the update
      if (!hip_ok(hipStreamWaitEvent(chain, s->ev_attr, 0), "hipStreamWaitEvent(chain, attraction)")) return false;
      s->home = chain;
      return true;
    }
    // the attraction's stream waits for the chain and carries the update
    return hip_ok(hipEventRecord(s->ev_attr, chain), "hipEventRecord(chain)") &&
           hip_ok(hipStreamWaitEvent(main, s->ev_attr, 0), "hipStreamWaitEvent(main, chain)");
  }
  return !overlap || enqueue_attract_helper(s, s->y_a(), exaggeration, s->ev_attr);
}

// One optimisation iteration: the previous update's statistics finished
// (`finalize`, see enqueue_gradient_pieces), the gradient pieces and the
// update.  The update's own statistics are finished by the next iteration or
// by the caller, so that the next attraction can start beside that finish.
bool enqueue_iteration(fastembedr_hip_tsne* s, bool lg, int fft_len, const fehip::UpdateParams& up, bool overlap,
                       bool finalize) {
  // An overlapped iteration's update completes ev_layout itself: the next
  // iteration's chain waits for it, and its attraction follows the update on
  // the same stream with no marker between them.
  const bool mark = overlap && s->mark_layout;
  if (!enqueue_gradient_pieces(s, lg, fft_len, up.exaggeration, overlap, finalize) ||
      !s->timed(
          fehip::kKUpdate, "update launch",
          [&] {
            // the interpolation grid's update centres the stored layout itself
            return fehip::launch_update(fehip::kModeUpdate, lg ? s->y_a() : s->y_b, s->attr, s->y_a(), s->update(),
                                        s->gains(), nullptr, nullptr, s->gb, up, s->partial, s->sc, s->n, s->home,
                                        lg ? s->ib.field : nullptr, mark ? s->ev_layout : nullptr);
          },
          s->home)) {
    return false;
  }
  s->layout_at_tail = mark;
  return true;
}

// Captures enqueue_iteration() on the main stream alone (no side branches,
// whose kernels' allocations a launched graph would hold past hipFree) into an
// executable graph (nothing runs).
bool capture_iteration(fastembedr_hip_tsne* s, bool lg, int fft_len, const fehip::UpdateParams& up, bool finalize,
                       hipGraphExec_t* exec) {
  if (!hip_ok(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture")) {
    return false;
  }
  const bool enqueued = enqueue_iteration(s, lg, fft_len, up, false, finalize);
  hipGraph_t graph = nullptr;
  const hipError_t ended = hipStreamEndCapture(s->stream, &graph);
  bool ok = enqueued && hip_ok(ended, "hipStreamEndCapture") && graph != nullptr;
  if (ok) ok = hip_ok(hipGraphInstantiate(exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  if (graph != nullptr) (void)hipGraphDestroy(graph);
  return ok;
}

// Enqueues one iteration as a replayed graph when its key has a captured one,
// captures it the second time the key is met, and runs it eagerly otherwise.
bool enqueue_iteration_graphed(fastembedr_hip_tsne* s, bool lg, int fft_len, const fehip::UpdateParams& up,
                               bool finalize) {
  using IterGraph = fastembedr_hip_tsne::IterGraph;
  // Graph nodes keep the streams' order but not the tile build's host-side
  // bookkeeping: build the tiles eagerly first.
  if (!settle(s) || !ensure_tiles(s, s->stream)) return false;
  auto bits = [](float v) {
    std::uint32_t u;
    std::memcpy(&u, &v, sizeof(u));
    return u;
  };
  const std::array<std::uint32_t, 15> key = {static_cast<std::uint32_t>(lg),
                                             static_cast<std::uint32_t>(finalize),
                                             static_cast<std::uint32_t>(fft_len),
                                             static_cast<std::uint32_t>(s->lg_table_bits),
                                             static_cast<std::uint32_t>(s->si),
                                             static_cast<std::uint32_t>(s->wi),
                                             static_cast<std::uint32_t>(s->attract_tiled),
                                             static_cast<std::uint32_t>(std::lround(1000.0 * s->attract_share())),
                                             static_cast<std::uint32_t>(std::lround(1000.0 * s->attract_helper_per_cu)),
                                             bits(up.exaggeration),
                                             bits(up.momentum),
                                             bits(up.learning_rate),
                                             bits(up.min_gain),
                                             bits(up.max_step_norm),
                                             static_cast<std::uint32_t>(up.clip)};
  ++s->graph_clock;
  IterGraph* g = nullptr;
  for (IterGraph& c : s->graphs) {
    if (c.key == key) g = &c;
  }
  if (g == nullptr) {
    if (s->graphs.size() >= fastembedr_hip_tsne::kMaxGraphs) {
      auto lru = std::min_element(s->graphs.begin(), s->graphs.end(),
                                  [](const IterGraph& a, const IterGraph& b) { return a.last_use < b.last_use; });
      if (lru->exec != nullptr) {
        // an executable graph may still be in flight: drain before destroying it
        if (!s->sync_all() || !hip_ok(hipGraphExecDestroy(lru->exec), "hipGraphExecDestroy")) return false;
      }
      s->graphs.erase(lru);
    }
    s->graphs.push_back(IterGraph{});
    g = &s->graphs.back();
    g->key = key;
  }
  g->last_use = s->graph_clock;
  // An iteration that makes the spread order runs eagerly (it counts as a
  // sight of its key): the radix sort's library launches stay out of
  // captured graphs.
  if (lg && s->lg_order_due) {
    ++g->seen;
    return enqueue_iteration(s, lg, fft_len, up, true, finalize);
  }
  if (g->exec == nullptr && ++g->seen >= 2) {
    if (!capture_iteration(s, lg, fft_len, up, finalize, &g->exec)) {
      // A capture the runtime refuses leaves the session on eager launches.
      if (g->exec != nullptr) (void)hipGraphExecDestroy(g->exec);
      g->exec = nullptr;
      (void)hipGetLastError();
      s->graph_capture = false;
      g_last_error.clear();
    } else {
      ++s->graph_captures;
    }
  }
  if (g->exec == nullptr) return enqueue_iteration(s, lg, fft_len, up, true, finalize);
  ++s->graph_launches;
  return hip_ok(hipGraphLaunch(g->exec, s->stream), "hipGraphLaunch");
}

// Current interpolation geometry and the device's ring counter, read
// synchronously.
bool read_interp_boxes(fastembedr_hip_tsne* s, int* boxes, unsigned int* ring_seq) {
  return hip_ok(hipMemcpyAsync(boxes, &s->sc->lg_boxes, sizeof(int), hipMemcpyDeviceToHost, s->stream),
                "hipMemcpy(boxes)") &&
         hip_ok(hipMemcpyAsync(ring_seq, &s->sc->ring_seq, sizeof(int), hipMemcpyDeviceToHost, s->stream),
                "hipMemcpy(ring counter)") &&
         hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(boxes)");
}

// Waits until the ring slot of sequence number `seq` holds it and returns its
// box count.  The update that writes it is enqueued on the main stream: if
// that stream has drained and the slot still lacks the number, the write
// never happened (an error, not a wait).
bool wait_ring(fastembedr_hip_tsne* s, unsigned int seq, int* boxes) {
  const unsigned long long* slot = s->lg_ring + (seq & (fastembedr_hip_tsne::kLgRing - 1));
  for (unsigned int spin = 1;; ++spin) {
    const unsigned long long v = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
    if (static_cast<unsigned int>(v >> 32) == seq) {
      *boxes = static_cast<int>(v & 0xffffffffull);
      return true;
    }
    if (spin % 64 == 0) {
      const hipError_t q = hipStreamQuery(s->home);  // holds the latest update, after everything before it
      if (q == hipSuccess) {
        const unsigned long long again = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
        if (static_cast<unsigned int>(again >> 32) == seq) continue;
        set_error("internal: the interpolation grid's box count was not handed over");
        return false;
      }
      if (q != hipErrorNotReady) return hip_ok(q, "hipStreamQuery(box ring)");
    }
    std::this_thread::yield();
  }
}

// Device error flags raised during iterations (so far only the interpolation
// grid's FFT-length check, which the host's bound should never trip).
bool check_iteration_flags(fastembedr_hip_tsne* s) {
  if (!s->lg_ready) return true;
  unsigned int flags = 0;
  if (!hip_ok(hipMemcpyAsync(&flags, &s->sc->error_flags, sizeof(flags), hipMemcpyDeviceToHost, s->stream),
              "hipMemcpy(flags)") ||
      !hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(flags)")) {
    return false;
  }
  if (flags & fehip::kErrInterpGrid) {
    set_error("internal: interpolation grid outgrew the FFT length chosen for it");
    return false;
  }
  return true;
}

// Renumbers points by the Morton order of the current layout: permutes the
// state, rebuilds the working CSR in the new numbering and updates the
// permutations.  Needs the bounding box and pending shift in DeviceScalars
// (set by the stats kernel or by the previous update).  Stream-ordered, no
// host synchronisation.
hipError_t enqueue_renumber(fastembedr_hip_tsne* s) {
  const int n = s->n;
  const int next = s->wi < 0 ? 0 : 1 - s->wi;
  const Csr& src = s->work_p();
  Csr& dst = s->pw[next];
  s->rn.perm = s->perm[s->pi];
  hipError_t e = fehip::launch_morton_keys(s->ys[s->si], s->sc, n, s->rn, s->stream);
  if (e == hipSuccess) e = fehip::sort_morton(s->rn, n, s->stream);
  if (e != hipSuccess) return e;
  // The layout is a proxy for P's locality that can be poor (early in the
  // optimisation points pass through one another), so the candidate order is
  // kept only if it gives fewer attraction tiles than the current one, by a
  // sampled estimate.  A host round trip, at renumbering points only.
  if (s->renumbered() || s->tiles_for != -2) {
    const int row_blocks = (n + fehip::kTileRows - 1) / fehip::kTileRows;
    const int step = std::max(1, std::min(64, row_blocks / 128));
    unsigned long long est[2] = {0ull, 0ull};
    e = hipMemsetAsync(s->tile_est, 0, 2 * sizeof(unsigned long long), s->stream);
    if (e == hipSuccess) e = fehip::launch_invert(s->rn.order, s->rn.map, n, s->stream);
    if (e == hipSuccess) e = fehip::launch_tile_estimate(src, nullptr, nullptr, step, s->tile_est, s->stream);
    if (e == hipSuccess) e = fehip::launch_tile_estimate(src, s->rn.order, s->rn.map, step, s->tile_est + 1, s->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(est, s->tile_est, sizeof(est), hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return e;
    s->last_tile_estimate[0] = static_cast<long long>(est[0]) * step;
    s->last_tile_estimate[1] = static_cast<long long>(est[1]) * step;
    if (!(static_cast<double>(est[1]) < 0.95 * static_cast<double>(est[0]))) {
      ++s->renumber_rejected;
      s->since_reorder = 0;
      return hipSuccess;  // keep the current numbering
    }
  }
  if (e == hipSuccess)
    e = fehip::launch_apply_order(s->rn, n, s->perm[s->pi], s->perm[1 - s->pi], s->ys[s->si], s->ys[1 - s->si],
                                  s->us[s->si], s->us[1 - s->si], s->gs[s->si], s->gs[1 - s->si], src.row_ptr,
                                  s->stream);
  if (e == hipSuccess) e = fehip::scan_row_lengths(s->rn, n, dst.row_ptr, s->stream);
  if (e == hipSuccess) e = fehip::launch_copy_rows(s->rn, n, src, dst, s->stream);
  if (e == hipSuccess) e = fehip::launch_invert(s->perm[1 - s->pi], s->inv_perm, n, s->stream);
  if (e != hipSuccess) return e;
  s->wi = next;
  s->si = 1 - s->si;
  s->pi = 1 - s->pi;
  s->since_reorder = 0;
  ++s->renumber_count;
  s->lg_order_stale = true;  // the spread order holds working indices
  return hipSuccess;
}

// Iterations until the next renumbering check after one at gap `gap` (0: the
// first, before the first iteration), for period P: checks at iterations 0,
// P and 16P, then at gaps that double (P = 25: 0, 25, 400, 1150, ...).  The
// check at P repairs an initial order that says little about P's locality (a
// random initialisation); the one at 16P comes after the early exaggeration,
// once the clusters have formed.  Every check drains the queue for its
// estimate and an accepted one rebuilds the tiles (~2-7 ms at 1M points,
// ~35 ms at 4M), so the old schedule 0, 25, 75, 175, 375 cost config 2's whole
// schedule 3826 against 3926 it/s with checks at 0 and 400 only; config 4,
// which needs a renumbering after its clusters form (its PCA order leaves the
// attraction at 1.30 instead of 0.96 ms), 731-754 against 763.
int next_reorder_gap(int gap, int period) {
  if (gap == 0) return period;
  if (gap == period) return 15 * period;
  return 2 * gap;
}

// Host (caller's numbering) -> working numbering, through y_b as staging.
bool upload_permuted(fastembedr_hip_tsne* s, const float* host, float2* dst) {
  const std::size_t bytes = static_cast<std::size_t>(s->n) * sizeof(float2);
  if (!s->renumbered()) {
    return hip_ok(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, s->stream), "state upload");
  }
  return hip_ok(hipMemcpyAsync(s->y_b, host, bytes, hipMemcpyHostToDevice, s->stream), "state upload") &&
         hip_ok(fehip::launch_gather2(s->y_b, s->perm[s->pi], dst, s->n, s->stream), "permute launch") &&
         hip_ok(hipStreamSynchronize(s->stream), "state upload sync");
}

// Working numbering -> host (caller's numbering), through y_b as staging.
bool download_permuted(fastembedr_hip_tsne* s, const float2* src, float* host) {
  const std::size_t bytes = static_cast<std::size_t>(s->n) * sizeof(float2);
  if (!s->renumbered()) {
    return hip_ok(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, s->stream), "state download") &&
           hip_ok(hipStreamSynchronize(s->stream), "state download sync");
  }
  return hip_ok(fehip::launch_gather2(src, s->inv_perm, s->y_b, s->n, s->stream), "permute launch") &&
         hip_ok(hipMemcpyAsync(host, s->y_b, bytes, hipMemcpyDeviceToHost, s->stream), "state download") &&
         hip_ok(hipStreamSynchronize(s->stream), "state download sync");
}

// Builds P from KNN (src/tsne_neighbors.cpp:540-648 semantics) and allocates
// the iteration buffers.
int create_session(const int* indices, const void* distances, bool dist_double, int n, int k, float perplexity,
                   int index_offset, int on_device, int grid_size, fastembedr_hip_tsne** out) {
  g_last_error.clear();
  *out = nullptr;
  if (indices == nullptr || distances == nullptr) {
    set_error("null HIP openTSNE input pointer");
    return 1;
  }
  if (n < 2 || k < 1) {
    set_error("KNN input must have at least two rows and one neighbor column.");
    return 1;
  }
  if (k > 256) {
    // Same cap as the reference CUDA backend (src/embedding_cuda_impl.cpp:384);
    // the search stages k x 64 squared distances in LDS (64 KB at k = 256).
    set_error("HIP openTSNE FFT-grid currently supports at most 256 neighbors.");
    return 1;
  }
  if (!(perplexity > 0.0f) || !std::isfinite(perplexity)) {
    set_error("perplexity must be positive");
    return 1;
  }
  if (index_offset != 0 && index_offset != 1) {
    set_error("index_offset must be 0 or 1");
    return 1;
  }
  int dev_count = 0;
  if (!hip_ok(hipGetDeviceCount(&dev_count), "hipGetDeviceCount")) return 1;
  if (dev_count < 1) {
    set_error("No HIP device is available.");
    return 1;
  }

  auto* s = new fastembedr_hip_tsne();
  s->n = n;
  s->k = k;
  const int g = resolve_grid_size(n, grid_size);
  // (device-scope or no system fence on these events measured no faster:
  // 3646 / 3578 it/s against 3671 at config 2)
  const unsigned ev_flags = hipEventDisableTiming;
  if (!hip_ok(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate") ||
      !hip_ok(hipStreamCreateWithFlags(&s->side_attr, hipStreamNonBlocking), "hipStreamCreate") ||
      !hip_ok(hipStreamCreateWithFlags(&s->side_kern, hipStreamNonBlocking), "hipStreamCreate") ||
      !hip_ok(hipEventCreateWithFlags(&s->ev_layout, ev_flags), "hipEventCreate") ||
      !hip_ok(hipEventCreateWithFlags(&s->ev_ready, ev_flags), "hipEventCreate") ||
      !hip_ok(hipEventCreateWithFlags(&s->ev_attr, ev_flags), "hipEventCreate") ||
      !hip_ok(hipEventCreateWithFlags(&s->ev_kern, ev_flags), "hipEventCreate") ||
      !hip_ok(hipEventCreateWithFlags(&s->ev_home, ev_flags), "hipEventCreate")) {
    delete s;
    return 1;
  }
  s->home = s->stream;
  hipEvent_t t0, t1;
  (void)hipEventCreate(&t0);
  (void)hipEventCreate(&t1);

  const std::size_t nk = static_cast<std::size_t>(n) * k;
  const std::size_t edges = 2 * nk;
  const int key_bits = key_bits_for(n);
  const int search_blocks = (n + 63) / 64;

  // Scratch for the construction of P (released before returning).
  Arena scratch;
  std::size_t sort_temp = 0, scan_temp = 0;
  if (!hip_ok(fehip::sort_edges(nullptr, sort_temp, nullptr, nullptr, nullptr, nullptr, edges, 2 * key_bits,
                                s->stream),
              "radix_sort_pairs(size query)") ||
      !hip_ok(fehip::scan_heads(nullptr, scan_temp, nullptr, nullptr, edges, s->stream), "exclusive_scan(size query)")) {
    delete s;
    return 1;
  }
  const std::size_t in_bytes = on_device ? 0 : align_up(nk * sizeof(int)) + align_up(nk * (dist_double ? 8 : 4));
  const std::size_t scratch_bytes = in_bytes + 2 * align_up(edges * 8) + 2 * align_up(edges * 4) +
                                    2 * align_up(edges * 4) + align_up(std::max(sort_temp, scan_temp)) +
                                    align_up(search_blocks * sizeof(double)) + 4096;
  // Persistent part: everything except CSR col/val (added once nnz is known).
  const int dpart = std::max(fehip::kMaxReduceBlocks, fehip::exact_blocks_for(n));
  const std::size_t gg = static_cast<std::size_t>(g) * g;
  const std::size_t hh = static_cast<std::size_t>(g + 1);
  const std::size_t persistent_fixed =
      align_up(sizeof(DeviceScalars)) + align_up(nk * 4) + align_up((n + 1) * sizeof(int)) +
      7 * align_up(static_cast<std::size_t>(n) * sizeof(float2)) + align_up(fehip::kTwiddleLen * sizeof(float2)) +
      align_up(fehip::kMaxReduceBlocks * sizeof(BlockStats)) + align_up(dpart * sizeof(double)) +
      3 * align_up(gg * 4) + align_up(gg * sizeof(float4)) + 2 * align_up(hh * hh * sizeof(float2)) +
      7 * align_up(g * hh * sizeof(float2)) + align_up(fehip::kMaxReduceBlocks * sizeof(double)) +
      2 * align_up(fehip::kMaxTiles * sizeof(int)) +
      align_up(static_cast<std::size_t>(fehip::max_spread_items(n, g)) * sizeof(int4)) +
      align_up(static_cast<std::size_t>(n) * sizeof(float2)) + 4096;
  if (!memory_preflight(scratch_bytes + persistent_fixed + edges * 8, "HIP openTSNE allocation preflight") ||
      !scratch.init(scratch_bytes, "hipMalloc(P construction scratch)")) {
    delete s;
    return 1;
  }

  const int* d_idx = indices;
  const void* d_dist = distances;
  if (!on_device) {
    int* di = scratch.take<int>(nk);
    char* dd = scratch.take<char>(nk * (dist_double ? 8 : 4));
    if (!hip_ok(hipMemcpyAsync(di, indices, nk * sizeof(int), hipMemcpyHostToDevice, s->stream),
                "hipMemcpy(indices H2D)") ||
        !hip_ok(hipMemcpyAsync(dd, distances, nk * (dist_double ? 8 : 4), hipMemcpyHostToDevice, s->stream),
                "hipMemcpy(distances H2D)")) {
      scratch.release();
      delete s;
      return 1;
    }
    d_idx = di;
    d_dist = dd;
  }
  auto* keys_a = scratch.take<std::uint64_t>(edges);
  auto* keys_b = scratch.take<std::uint64_t>(edges);
  auto* vals_a = scratch.take<float>(edges);
  auto* vals_b = scratch.take<float>(edges);
  auto* heads = scratch.take<int>(edges);
  auto* pos = scratch.take<int>(edges);
  void* temp = scratch.take<char>(std::max(sort_temp, scan_temp));
  auto* mass_partial = scratch.take<double>(search_blocks);

  // Persistent buffers (P values and columns are added after nnz is known).
  std::size_t csr_bytes_guess = 2 * align_up(edges * 4);
  if (!s->arena.init(persistent_fixed + csr_bytes_guess, "hipMalloc(HIP openTSNE arena)")) {
    scratch.release();
    delete s;
    return 1;
  }
  s->sc = s->arena.take<DeviceScalars>(1);
  s->p_cond = s->arena.take<float>(nk);
  s->p.row_ptr = s->arena.take<int>(n + 1);
  s->ys[0] = s->arena.take<float2>(n);
  s->y_b = s->arena.take<float2>(n);
  s->us[0] = s->arena.take<float2>(n);
  s->gs[0] = s->arena.take<float2>(n);
  s->grad = s->arena.take<float2>(n);
  s->exact_rep = s->arena.take<float2>(n);
  s->attr = s->arena.take<float2>(n);
  s->tw = s->arena.take<float2>(fehip::kTwiddleLen);
  s->partial = s->arena.take<BlockStats>(fehip::kMaxReduceBlocks);
  s->dpartial = s->arena.take<double>(dpart);
  s->dpartial_len = dpart;
  s->gb.g = g;
  s->gb.mass = s->arena.take<float>(gg);
  s->gb.mass_x = s->arena.take<float>(gg);
  s->gb.mass_y = s->arena.take<float>(gg);
  s->gb.field = s->arena.take<float4>(gg);
  s->gb.k_rows = s->arena.take<float2>(hh * hh);
  s->gb.k_hat = s->arena.take<float2>(hh * hh);
  s->gb.m_rows = s->arena.take<float2>(g * hh);
  s->gb.mx_rows = s->arena.take<float2>(g * hh);
  s->gb.my_rows = s->arena.take<float2>(g * hh);
  s->gb.x_rows = s->arena.take<float2>(g * hh);
  s->gb.v1_rows = s->arena.take<float2>(g * hh);
  s->gb.v2_rows = s->arena.take<float2>(g * hh);
  s->gb.y_rows = s->arena.take<float2>(g * hh);
  s->gb.sumq_partial = s->arena.take<double>(fehip::kMaxReduceBlocks);
  s->gb.tile_count = s->arena.take<int>(fehip::kMaxTiles);
  s->gb.tile_cursor = s->arena.take<int>(fehip::kMaxTiles);
  s->gb.items = s->arena.take<int4>(fehip::max_spread_items(n, g));
  s->gb.binned = s->arena.take<float2>(n);

  auto fail = [&](void) {
    scratch.release();
    delete s;
    return 1;
  };
  if (!hip_ok(hipMemsetAsync(s->sc, 0, sizeof(DeviceScalars), s->stream), "hipMemset(scalars)") ||
      !hip_ok(hipMemsetAsync(s->gb.mass, 0, gg * 4, s->stream), "hipMemset(grid)") ||
      !hip_ok(hipMemsetAsync(s->gb.mass_x, 0, gg * 4, s->stream), "hipMemset(grid)") ||
      !hip_ok(hipMemsetAsync(s->gb.mass_y, 0, gg * 4, s->stream), "hipMemset(grid)") ||
      !hip_ok(hipMemsetAsync(s->gb.tile_count, 0, fehip::kMaxTiles * sizeof(int), s->stream), "hipMemset(tiles)") ||
      !upload_twiddles(s)) {
    return fail();
  }

  (void)hipEventRecord(t0, s->stream);
  const float log_perp = static_cast<float>(std::log(static_cast<double>(perplexity)));
  if (!hip_ok(fehip::launch_row_search(d_idx, d_dist, dist_double, n, k, index_offset, log_perp, s->p_cond, keys_a,
                                       vals_a, key_bits, mass_partial, search_blocks, s->sc, s->stream),
              "row_search launch") ||
      !hip_ok(fehip::launch_finalize_mass(mass_partial, search_blocks, s->sc, s->stream), "finalize_mass launch")) {
    return fail();
  }
  DeviceScalars host_sc;
  if (!hip_ok(hipMemcpyAsync(&host_sc, s->sc, sizeof(DeviceScalars), hipMemcpyDeviceToHost, s->stream),
              "hipMemcpy(scalars D2H)") ||
      !hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(row search)")) {
    return fail();
  }
  if (host_sc.error_flags & fehip::kErrIndex) {
    set_error("KNN indices are out of range.");
    return fail();
  }
  if (host_sc.error_flags & fehip::kErrDistance) {
    set_error("KNN distances must be finite and non-negative.");
    return fail();
  }
  const std::size_t valid = edges - 2 * static_cast<std::size_t>(host_sc.self_edges);
  if (valid == 0) {
    set_error("KNN graph produced no non-self t-SNE edges.");
    return fail();
  }
  if (!std::isfinite(host_sc.total_mass) || host_sc.total_mass <= 0.0) {
    set_error("t-SNE probability normalization failed.");
    return fail();
  }
  std::size_t tb = sort_temp;
  if (!hip_ok(fehip::sort_edges(temp, tb, keys_a, keys_b, vals_a, vals_b, edges, 2 * key_bits, s->stream),
              "radix_sort_pairs") ||
      !hip_ok(fehip::launch_mark_heads(keys_b, valid, heads, s->stream), "mark_heads launch")) {
    return fail();
  }
  tb = 0;
  if (!hip_ok(fehip::scan_heads(nullptr, tb, heads, pos, valid, s->stream), "exclusive_scan(size query)")) {
    return fail();
  }
  if (tb > std::max(sort_temp, scan_temp)) {
    set_error("internal: scan scratch larger than reserved");
    return fail();
  }
  if (!hip_ok(fehip::scan_heads(temp, tb, heads, pos, valid, s->stream), "exclusive_scan")) return fail();
  int last_pos = 0, last_head = 0;
  if (!hip_ok(hipMemcpyAsync(&last_pos, pos + (valid - 1), sizeof(int), hipMemcpyDeviceToHost, s->stream),
              "hipMemcpy(nnz)") ||
      !hip_ok(hipMemcpyAsync(&last_head, heads + (valid - 1), sizeof(int), hipMemcpyDeviceToHost, s->stream),
              "hipMemcpy(nnz)") ||
      !hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(scan)")) {
    return fail();
  }
  const long long nnz = static_cast<long long>(last_pos) + last_head;
  s->p.n = n;
  s->p.nnz = nnz;
  s->p.col = s->arena.take<int>(static_cast<std::size_t>(nnz));
  s->p.val = s->arena.take<float>(static_cast<std::size_t>(nnz));
  if (s->p.col == nullptr || s->p.val == nullptr) {
    set_error("internal: CSR does not fit the arena");
    return fail();
  }
  if (!hip_ok(fehip::launch_compact(keys_b, vals_b, heads, pos, valid, key_bits, n, s->sc, s->p.row_ptr, s->p.col,
                                    s->p.val, s->stream),
              "compact launch")) {
    return fail();
  }
  (void)hipEventRecord(t1, s->stream);
  if (!hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(P build)")) return fail();
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, t0, t1);
  s->p_build_ms = ms;
  (void)hipEventDestroy(t0);
  (void)hipEventDestroy(t1);
  scratch.release();

  // Lanes per CSR row: enough to cover the mean row in a few passes.
  const double mean_row = static_cast<double>(nnz) / n;
  int lanes = mean_row > 96.0 ? 32 : (mean_row > 24.0 ? 16 : 8);
  lanes = env_int("FASTEMBEDR_HIP_ATTRACT_LANES", lanes);
  if (lanes != 8 && lanes != 16 && lanes != 32 && lanes != 64) lanes = 16;
  s->lanes = lanes;
  // Renumbering checks: before the first iteration, after this many, after
  // 16 times as many, then at gaps that double (next_reorder_gap).
  s->reorder_period = env_int("FASTEMBEDR_HIP_RENUMBER_PERIOD", 25);
  if (const char* off = std::getenv("FASTEMBEDR_HIP_RENUMBER_PERIOD")) {
    if (std::strcmp(off, "0") == 0) s->reorder_period = 0;
  }
  // CDNA3/CDNA4 parts (gfx94x, gfx95x) dispatch workgroups round-robin over 8 XCDs.
  {
    int dev = 0;
    hipDeviceProp_t prop;
    s->xcds = 1;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
        (std::strncmp(prop.gcnArchName, "gfx94", 5) == 0 || std::strncmp(prop.gcnArchName, "gfx95", 5) == 0)) {
      s->xcds = 8;
    }
    s->xcds = std::max(1, std::min(fehip::kTileMaxXcds, env_int("FASTEMBEDR_HIP_XCDS", s->xcds)));
    if (hipDeviceGetAttribute(&s->cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) s->cus = 0;
  }
  // Attraction: tiled unless FASTEMBEDR_HIP_ATTRACT_TILED=0 (row-parallel).
  if (const char* tiled = std::getenv("FASTEMBEDR_HIP_ATTRACT_TILED")) {
    if (std::strcmp(tiled, "0") == 0) s->attract_tiled = false;
  }

  for (auto [name, knob] : {std::pair<const char*, double*>{"FASTEMBEDR_HIP_ATTRACT_SHARED_PER_CU",
                                                             &s->attract_shared_per_cu},
                            {"FASTEMBEDR_HIP_ATTRACT_HELPER_PER_CU", &s->attract_helper_per_cu}}) {
    if (const char* v = std::getenv(name)) {
      char* end = nullptr;
      const double d = std::strtod(v, &end);
      if (end != v && std::isfinite(d) && d >= 0.0) {
        *knob = d;
        if (knob == &s->attract_shared_per_cu) s->attract_share_auto = false;
      }
    }
  }
  if (const char* v = std::getenv("FASTEMBEDR_HIP_ATTRACT_MAIN")) s->attract_main = std::strcmp(v, "0") != 0;
  if (const char* v = std::getenv("FASTEMBEDR_HIP_UPDATE_ON_CHAIN")) s->update_on_chain = std::strcmp(v, "0") != 0;
  if (const char* v = std::getenv("FASTEMBEDR_HIP_MARK_LAYOUT")) s->mark_layout = std::strcmp(v, "0") != 0;
  if (const char* v = std::getenv("FASTEMBEDR_HIP_LG_ORDER_PERIOD")) s->lg_order_period = std::max(0, std::atoi(v));
  s->tile_shape = std::max(0, std::min(2, env_int("FASTEMBEDR_HIP_TILE_SHAPE", 0)));
  if (const char* v = std::getenv("FASTEMBEDR_HIP_SPREAD_DENSE")) {
    char* end = nullptr;
    const double d = std::strtod(v, &end);
    if (end != v && std::isfinite(d) && d >= 0.0) s->lg_dense_points = d;
  }
  s->graph_capture = graph_capture_enabled();
  if (!alloc_working_buffers(s) || (s->attract_tiled && !alloc_tiles(s))) {
    delete s;
    return 1;
  }
  *out = s;
  return 0;
}

bool valid_state_args(const fastembedr_hip_tsne* s) {
  if (s == nullptr) {
    set_error("null HIP openTSNE session");
    return false;
  }
  return true;
}

std::vector<float> random_init(int n, unsigned int seed) {
  // src/tsne_neighbors.cpp:1693-1700: mt19937(seed), normal_distribution<float>(0, 1e-4).
  std::vector<float> y(2 * static_cast<std::size_t>(n));
  std::mt19937 rng(seed);
  std::normal_distribution<float> normal(0.0f, 1.0e-4f);
  for (float& v : y) v = normal(rng);
  return y;
}

template <typename DT>
int one_shot(const int* indices, const DT* distances, const float* init, int has_init, int n, int k,
             int n_components, float perplexity, int early_exaggeration_iter, int n_iter, float early_exaggeration,
             float exaggeration, float learning_rate, int learning_rate_auto, float initial_momentum,
             float final_momentum, float min_gain, float max_step_norm, unsigned int seed, int index_offset,
             float* out, int on_device) {
  g_last_error.clear();
  if (indices == nullptr || distances == nullptr || out == nullptr || (has_init && init == nullptr)) {
    set_error("null HIP openTSNE input pointer");
    return 1;
  }
  if (n < 2 || k < 1 || n_components != 2 || !(perplexity > 0.0f) || early_exaggeration_iter < 0 || n_iter < 0 ||
      early_exaggeration_iter + n_iter < 1 || !(early_exaggeration > 0.0f) || !(exaggeration > 0.0f) ||
      (!learning_rate_auto && !(learning_rate > 0.0f)) || initial_momentum < 0.0f || final_momentum < 0.0f ||
      !(min_gain > 0.0f)) {
    set_error("invalid HIP openTSNE FFT-grid dimensions or parameters");
    return 1;
  }
  if (static_cast<double>(n - 1) < 3.0 * static_cast<double>(perplexity)) {
    set_error("perplexity is too large for the number of samples.");
    return 1;
  }
  fastembedr_hip_tsne* s = nullptr;
  if (create_session(indices, distances, sizeof(DT) == 8, n, k, perplexity, index_offset, on_device, 0, &s) != 0) {
    return 1;
  }
  std::vector<float> y0;
  if (has_init) {
    y0.assign(init, init + 2 * static_cast<std::size_t>(n));
  } else {
    y0 = random_init(n, seed);
  }
  int rc = fastembedr_hip_tsne_set_state(s, y0.data(), nullptr, nullptr);
  if (rc == 0) rc = fastembedr_hip_tsne_center(s);
  const auto phase_lr = [&](float ex) {
    // fp32 n / exaggeration, as the reference computes it (src/embedding_cuda_kernels.cpp:5908-5913)
    return learning_rate_auto ? static_cast<float>(n) / ex : learning_rate;
  };
  if (rc == 0 && early_exaggeration_iter > 0) {
    rc = fastembedr_hip_tsne_run(s, early_exaggeration_iter, early_exaggeration, initial_momentum,
                                 phase_lr(early_exaggeration), min_gain, max_step_norm);
  }
  if (rc == 0 && n_iter > 0) {
    rc = fastembedr_hip_tsne_run(s, n_iter, exaggeration, final_momentum, phase_lr(exaggeration), min_gain,
                                 max_step_norm);
  }
  if (rc == 0) rc = fastembedr_hip_tsne_get_state(s, out, nullptr, nullptr);
  const std::string msg = g_last_error;
  fastembedr_hip_tsne_destroy(s);
  if (rc != 0) g_last_error = msg;
  return rc;
}

}  // namespace

namespace fehip {
void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }
}  // namespace fehip

extern "C" {

const char* fastembedr_hip_embedding_last_error(void) { return g_last_error.c_str(); }

bool fastembedr_hip_available(void) {
  int count = 0;
  const hipError_t code = hipGetDeviceCount(&count);
  if (code != hipSuccess) {
    set_error(std::string("hipGetDeviceCount: ") + hipGetErrorString(code));
    return false;
  }
  if (count < 1) return false;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return false;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

int fastembedr_hip_opentsne_fft_from_knn_float(const int* indices, const float* distances, const float* init,
                                               int has_init, int n, int k, int n_components, float perplexity,
                                               int early_exaggeration_iter, int n_iter, float early_exaggeration,
                                               float exaggeration, float learning_rate, int learning_rate_auto,
                                               float initial_momentum, float final_momentum, float min_gain,
                                               float max_step_norm, unsigned int seed, int index_offset,
                                               float* out) {
  return one_shot<float>(indices, distances, init, has_init, n, k, n_components, perplexity,
                         early_exaggeration_iter, n_iter, early_exaggeration, exaggeration, learning_rate,
                         learning_rate_auto, initial_momentum, final_momentum, min_gain, max_step_norm, seed,
                         index_offset, out, 0);
}

int fastembedr_hip_opentsne_fft_from_knn(const int* indices, const double* distances, const float* init,
                                         int has_init, int n, int k, int n_components, float perplexity,
                                         int early_exaggeration_iter, int n_iter, float early_exaggeration,
                                         float exaggeration, float learning_rate, int learning_rate_auto,
                                         float initial_momentum, float final_momentum, float min_gain,
                                         float max_step_norm, unsigned int seed, int index_offset, float* out) {
  return one_shot<double>(indices, distances, init, has_init, n, k, n_components, perplexity,
                          early_exaggeration_iter, n_iter, early_exaggeration, exaggeration, learning_rate,
                          learning_rate_auto, initial_momentum, final_momentum, min_gain, max_step_norm, seed,
                          index_offset, out, 0);
}

int fastembedr_hip_opentsne_fft_from_device_knn_float(const int* indices, const float* distances,
                                                      const float* init, int has_init, int n, int k,
                                                      int n_components, float perplexity,
                                                      int early_exaggeration_iter, int n_iter,
                                                      float early_exaggeration, float exaggeration,
                                                      float learning_rate, int learning_rate_auto,
                                                      float initial_momentum, float final_momentum, float min_gain,
                                                      float max_step_norm, unsigned int seed, int index_offset,
                                                      float* out) {
  return one_shot<float>(indices, distances, init, has_init, n, k, n_components, perplexity,
                         early_exaggeration_iter, n_iter, early_exaggeration, exaggeration, learning_rate,
                         learning_rate_auto, initial_momentum, final_momentum, min_gain, max_step_norm, seed,
                         index_offset, out, 1);
}

int fastembedr_hip_tsne_create(const int* indices, const float* distances, int n, int k, float perplexity,
                               int index_offset, int inputs_on_device, int grid_size,
                               fastembedr_hip_tsne** out_session) {
  if (out_session == nullptr) {
    set_error("null session output pointer");
    return 1;
  }
  return create_session(indices, distances, false, n, k, perplexity, index_offset, inputs_on_device, grid_size,
                        out_session);
}

void fastembedr_hip_tsne_destroy(fastembedr_hip_tsne* session) { delete session; }

int fastembedr_hip_tsne_p_nnz(const fastembedr_hip_tsne* s, long long* nnz) {
  if (!valid_state_args(s) || nnz == nullptr) return 1;
  *nnz = s->p.nnz;
  return 0;
}

int fastembedr_hip_tsne_copy_p(const fastembedr_hip_tsne* s, int* row_ptr, int* col, float* val) {
  if (!valid_state_args(s)) return 1;
  if (row_ptr != nullptr &&
      !hip_ok(hipMemcpy(row_ptr, s->p.row_ptr, (s->n + 1) * sizeof(int), hipMemcpyDeviceToHost), "copy row_ptr"))
    return 1;
  if (col != nullptr &&
      !hip_ok(hipMemcpy(col, s->p.col, static_cast<std::size_t>(s->p.nnz) * sizeof(int), hipMemcpyDeviceToHost),
              "copy col"))
    return 1;
  if (val != nullptr &&
      !hip_ok(hipMemcpy(val, s->p.val, static_cast<std::size_t>(s->p.nnz) * sizeof(float), hipMemcpyDeviceToHost),
              "copy val"))
    return 1;
  return 0;
}

int fastembedr_hip_tsne_copy_conditional_p(const fastembedr_hip_tsne* s, float* p_cond) {
  if (!valid_state_args(s) || p_cond == nullptr) return 1;
  return hip_ok(hipMemcpy(p_cond, s->p_cond, static_cast<std::size_t>(s->n) * s->k * sizeof(float),
                          hipMemcpyDeviceToHost),
                "copy conditional P")
             ? 0
             : 1;
}

int fastembedr_hip_tsne_grid_size(const fastembedr_hip_tsne* s, int* grid_size) {
  if (!valid_state_args(s) || grid_size == nullptr) return 1;
  *grid_size = s->gb.g;
  return 0;
}

int fastembedr_hip_tsne_set_state(fastembedr_hip_tsne* s, const float* y, const float* update, const float* gains) {
  if (!valid_state_args(s) || y == nullptr) {
    if (y == nullptr) set_error("null layout pointer");
    return 1;
  }
  const std::size_t bytes = static_cast<std::size_t>(s->n) * sizeof(float2);
  std::vector<float> fill;
  // a new layout: renumbering checks start again (at the next iteration,
  // then after gaps that double)
  s->since_reorder = 0;
  s->reorder_gap = 0;
  if (!upload_permuted(s, y, s->y_a())) return 1;
  if (update != nullptr) {
    if (!upload_permuted(s, update, s->update())) return 1;
  } else if (!hip_ok(hipMemsetAsync(s->update(), 0, bytes, s->stream), "set_state update")) {
    return 1;
  }
  if (gains != nullptr) {
    if (!upload_permuted(s, gains, s->gains())) return 1;
  } else {
    fill.assign(2 * static_cast<std::size_t>(s->n), 1.0f);
    if (!hip_ok(hipMemcpyAsync(s->gains(), fill.data(), bytes, hipMemcpyHostToDevice, s->stream), "set_state gains"))
      return 1;
  }
  return hip_ok(hipStreamSynchronize(s->stream), "set_state sync") ? 0 : 1;
}

int fastembedr_hip_tsne_get_state(fastembedr_hip_tsne* s, float* y, float* update, float* gains) {
  if (!valid_state_args(s) || !check_iteration_flags(s)) return 1;
  if (y != nullptr && !download_permuted(s, s->y_a(), y)) return 1;
  if (update != nullptr && !download_permuted(s, s->update(), update)) return 1;
  if (gains != nullptr && !download_permuted(s, s->gains(), gains)) return 1;
  return 0;
}

int fastembedr_hip_tsne_gradient(fastembedr_hip_tsne* s, float exaggeration, int repulsion, float* grad_out) {
  if (!valid_state_args(s) || grad_out == nullptr) return 1;
  g_last_error.clear();
  fehip::UpdateParams up{exaggeration, 0.0f, 0.0f, 0.0f, 0.0f, 0};
  const bool was_timing = s->timing;
  s->timing = false;
  bool ok = true;
  if (repulsion == FASTEMBEDR_HIP_REPULSION_EXACT) {
    ok = hip_ok(fehip::launch_exact_repulsion(s->y_a(), s->n, s->exact_rep, s->dpartial, s->sc, s->stream),
                "exact repulsion launch") &&
         enqueue_attract(s, s->y_a(), exaggeration) &&
         hip_ok(fehip::launch_update(fehip::kModeGradientExact, s->y_a(), s->attr, nullptr, nullptr, nullptr, s->grad,
                                     s->exact_rep, s->gb, up, s->partial, s->sc, s->n, s->stream),
                "update launch");
  } else if (repulsion == FASTEMBEDR_HIP_REPULSION_LAGRANGE) {
    int boxes = 0;
    unsigned int ring_seq = 0;
    s->lg_order_due = true;  // a probe's layout may be any: order it
    ok = ensure_interp(s) && write_interp_spec(s, fehip::kLgOrder) &&
         hip_ok(fehip::launch_stats(s->y_a(), s->n, s->gb.g, 0, s->partial, s->sc, s->stream), "stats launch") &&
         read_interp_boxes(s, &boxes, &ring_seq) && (set_spread_table(s, boxes), true) &&
         enqueue_gradient_pieces(s, true, interp_fft_len(std::min(boxes * fehip::kLgOrder, fehip::kLgMaxNodes)),
                                 exaggeration, false) &&
         hip_ok(fehip::launch_update(fehip::kModeGradientGrid, s->y_a(), s->attr, nullptr, nullptr, nullptr, s->grad,
                                     nullptr, s->gb, up, s->partial, s->sc, s->n, s->stream, s->ib.field),
                "update launch") &&
         check_iteration_flags(s);
  } else if (repulsion == FASTEMBEDR_HIP_REPULSION_GRID) {
    ok = hip_ok(fehip::launch_stats(s->y_a(), s->n, s->gb.g, 0, s->partial, s->sc, s->stream), "stats launch") &&
         enqueue_gradient_pieces(s, false, 0, exaggeration, false) &&
         hip_ok(fehip::launch_update(fehip::kModeGradientGrid, s->y_b, s->attr, nullptr, nullptr, nullptr, s->grad,
                                     nullptr, s->gb, up, s->partial, s->sc, s->n, s->stream),
                "update launch");
  } else {
    set_error("unsupported repulsion mode");
    ok = false;
  }
  s->timing = was_timing;
  if (!ok) return 1;
  return download_permuted(s, s->grad, grad_out) ? 0 : 1;
}

int fastembedr_hip_tsne_center(fastembedr_hip_tsne* s) {
  if (!valid_state_args(s)) return 1;
  if (!hip_ok(fehip::launch_stats(s->y_a(), s->n, s->gb.g, 1, s->partial, s->sc, s->stream), "stats launch") ||
      !hip_ok(fehip::launch_commit(s->y_a(), s->sc, s->n, s->stream), "commit launch")) {
    return 1;
  }
  return 0;
}

int fastembedr_hip_tsne_run(fastembedr_hip_tsne* s, int n_iter, float exaggeration, float momentum,
                            float learning_rate, float min_gain, float max_step_norm) {
  if (!valid_state_args(s)) return 1;
  g_last_error.clear();
  if (n_iter < 0) {
    set_error("n_iter must be non-negative");
    return 1;
  }
  if (n_iter == 0) return 0;
  // every return leaves the latest update on the main stream
  struct SettleOnExit {
    fastembedr_hip_tsne* s;
    ~SettleOnExit() { (void)settle(s); }
  } settle_on_exit{s};
  fehip::UpdateParams up;
  up.exaggeration = exaggeration;
  up.momentum = momentum;
  up.learning_rate = learning_rate;
  up.min_gain = min_gain;
  up.max_step_norm = max_step_norm;
  up.clip = (std::isfinite(max_step_norm) && max_step_norm > 0.0f) ? 1 : 0;
  const int n = s->n;
  if (!s->timed(fehip::kKStats, "stats launch",
                [&] { return fehip::launch_stats(s->y_a(), n, s->gb.g, 0, s->partial, s->sc, s->stream); })) {
    return 1;
  }
  // Interpolation grid: the FFT length must hold 2 * nodes, and the node
  // count is set on the device each iteration.  The host learns the box
  // count of earlier iterations through a pinned ring and bounds the current
  // one.  With the step clip every update u_i has |u_i| <= s = max_step_norm,
  // and so has their mean; a centred coordinate moves by u_i - mean(u).  The
  // span runs from the smallest to the largest centred coordinate over both
  // axes: two extremes on one axis separate by at most 2 s per iteration
  // (the mean cancels), extremes on different axes by at most
  // 2 s + |mean_x - mean_y| <= (2 + sqrt 2) s.  With boxes = ceil(span /
  // ints_in_interval) >= span / ints_in_interval, a growth of at most d
  // adds at most ceil(d / ints_in_interval) boxes.  The host runs at most
  // kMaxLag iterations ahead of what it knows (none without the clip).  One
  // iteration keeps the margin small enough for the FFT length to follow the
  // grid (at 1M points late in the schedule: 108 boxes known, 126 allowed,
  // length 768; three iterations would allow 160 and take 1024), and the
  // queue still holds the iteration in flight while the host waits.
  const bool lg = s->repulsion == FASTEMBEDR_HIP_REPULSION_LAGRANGE;
  constexpr int kRing = fastembedr_hip_tsne::kLgRing;
  constexpr int kMaxLag = 1;
  static_assert(kMaxLag + 2 <= kRing, "ring slots outlive the lag");
  const int allowed_lag = up.clip ? kMaxLag : 0;
  const double growth =
      up.clip ? (2.0 + std::sqrt(2.0)) * (static_cast<double>(max_step_norm) * 1.0001 + 1e-3) /
                    static_cast<double>(s->lg_ints_per_unit)
              : 0.0;
  int known_boxes = 0;
  int known_it = 0;
  unsigned int ring_base = 0;  // iteration it's update writes sequence number ring_base + it
  if (lg && !read_interp_boxes(s, &known_boxes, &ring_base)) return 1;
  // Each update's statistics are finished (k_finalize_stats) at the top of
  // the next iteration, beside the start of its attraction, or after the
  // loop; `pending` says that the previous update's are not finished yet.
  bool pending = false;
  auto finish_pending = [&](unsigned long long* ring) {
    pending = false;
    return settle(s) && s->timed(fehip::kKFinalize, "finalize launch", [&] {
      return fehip::launch_finalize_stats(s->partial, n, s->gb.g, s->sc, ring, s->stream);
    });
  };
  for (int it = 0; it < n_iter; ++it) {
    // Renumber before the first iteration ever run and then on the schedule
    // of next_reorder_gap; the bounding box and pending shift it needs are in
    // DeviceScalars (stats kernel above, or the previous update's finished
    // statistics).
    if (s->reorder_period > 0 && s->since_reorder >= s->reorder_gap) {
      if (pending && !finish_pending(lg ? s->lg_ring_dev : nullptr)) return 1;
      if (!settle(s) || !s->timed(fehip::kKRenumber, "renumber", [&] { return enqueue_renumber(s); })) return 1;
      s->reorder_gap = next_reorder_gap(s->reorder_gap, s->reorder_period);
    }
    ++s->since_reorder;
    int fft_len = 0;
    if (lg) {
      // the newest geometry handed over: the statistics of iteration d's
      // update (sequence number ring_base + d) set iteration d + 1's
      for (int r = 0; r < kRing; ++r) {
        const unsigned long long v = __atomic_load_n(s->lg_ring + r, __ATOMIC_ACQUIRE);
        const unsigned int d = static_cast<unsigned int>(v >> 32) - ring_base;
        if (d < static_cast<unsigned int>(it) && static_cast<int>(d) + 1 > known_it) {
          known_it = static_cast<int>(d) + 1;
          known_boxes = static_cast<int>(v & 0xffffffffull);
        }
      }
      if (it - known_it > allowed_lag) {
        const int target = it - allowed_lag;  // set by the statistics of iteration target - 1 < it
        // (without the step clip that is this iteration's own geometry: finish it first)
        if (target == it && pending && !finish_pending(s->lg_ring_dev)) return 1;
        if (!wait_ring(s, ring_base + static_cast<unsigned int>(target - 1), &known_boxes)) return 1;
        known_it = target;
      }
      const long long bound =
          static_cast<long long>(known_boxes) + static_cast<long long>(std::ceil(growth * (it - known_it)));
      const int nodes = static_cast<int>(std::min<long long>(bound * fehip::kLgOrder, fehip::kLgMaxNodes));
      fft_len = interp_fft_len(nodes);
      set_spread_table(s, known_boxes);
    }
    if (lg) {
      s->lg_order_due = s->lg_order_period > 0 && (s->lg_order_stale || s->lg_order_age >= s->lg_order_period);
    }
    // Timing every kernel (mode 1) or the repulsion step's span runs the
    // pieces in sequence, so that each duration is the kernel's (the step's)
    // alone; timed runs are never replayed graphs.
    const bool overlap = !(s->timing && (s->timed_only < 0 || s->timed_only == fehip::kKRepulsion));
    const bool ok = s->graph_capture && !s->timing ? enqueue_iteration_graphed(s, lg, fft_len, up, pending)
                                                   : enqueue_iteration(s, lg, fft_len, up, overlap, pending);
    if (!ok) return 1;
    pending = true;
    if (lg) ++s->lg_order_age;  // iterations spread since the order was made
    ++s->timing_iter;
  }
  // the last update's statistics (no box count is needed from them)
  if (pending && !finish_pending(nullptr)) return 1;
  if (!settle(s)) return 1;
  if (!s->timed(fehip::kKCommit, "commit launch",
                [&] { return fehip::launch_commit(s->y_a(), s->sc, n, s->stream); })) {
    return 1;
  }
  return s->harvest_timing() ? 0 : 1;
}

int fastembedr_hip_tsne_sync(fastembedr_hip_tsne* s) {
  if (!valid_state_args(s)) return 1;
  return s->sync_all() && check_iteration_flags(s) ? 0 : 1;
}

int fastembedr_hip_tsne_set_repulsion(fastembedr_hip_tsne* s, int repulsion, int n_interpolation_points,
                                      int min_num_intervals, float ints_in_interval) {
  if (!valid_state_args(s)) return 1;
  g_last_error.clear();
  if (repulsion == FASTEMBEDR_HIP_REPULSION_GRID) {
    s->repulsion = repulsion;
    return 0;
  }
  if (repulsion != FASTEMBEDR_HIP_REPULSION_LAGRANGE) {
    set_error("run() supports the bilinear grid and the FIt-SNE interpolation grid only");
    return 1;
  }
  if (n_interpolation_points != fehip::kLgOrder) {
    set_error("the HIP interpolation grid supports 3 interpolation points per interval");
    return 1;
  }
  if (min_num_intervals < 1 || !(ints_in_interval > 0.0f) || !std::isfinite(ints_in_interval)) {
    set_error("min_num_intervals must be >= 1 and ints_in_interval positive and finite");
    return 1;
  }
  s->lg_min_intervals = min_num_intervals;
  s->lg_ints_per_unit = ints_in_interval;
  if (!ensure_interp(s) || !write_interp_spec(s, fehip::kLgOrder)) return 1;
  s->repulsion = repulsion;
  return 0;
}

int fastembedr_hip_tsne_attraction_info(fastembedr_hip_tsne* s, long long* tiles, int* renumbers) {
  if (!valid_state_args(s)) return 1;
  if (tiles != nullptr) {
    int count = -1;
    if (s->attract_tiled && s->tiles_for != -2) {
      if (!s->sync_all() ||
          !hip_ok(hipMemcpy(&count, s->tiles.tile_count, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(tiles)")) {
        return 1;
      }
    }
    *tiles = count;
  }
  if (renumbers != nullptr) *renumbers = s->renumber_count;
  return 0;
}

int fastembedr_hip_tsne_attraction_slots(fastembedr_hip_tsne* s, long long* slots) {
  if (!valid_state_args(s)) return 1;
  if (slots == nullptr) {
    set_error("null pointer");
    return 1;
  }
  *slots = -1;
  if (s->attract_tiled && s->tiles_for != -2) {
    int count = 0, total = 0;
    if (!s->sync_all() ||
        !hip_ok(hipMemcpy(&count, s->tiles.tile_count, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(tiles)") ||
        !hip_ok(hipMemcpy(&total, s->tiles.tile_beg + count, sizeof(int), hipMemcpyDeviceToHost),
                "hipMemcpy(slots)")) {
      return 1;
    }
    *slots = total;
  }
  return 0;
}

int fastembedr_hip_tsne_graph_info(fastembedr_hip_tsne* s, long long* launches, int* captures, int* enabled) {
  if (!valid_state_args(s)) return 1;
  if (launches != nullptr) *launches = s->graph_launches;
  if (captures != nullptr) *captures = s->graph_captures;
  if (enabled != nullptr) *enabled = s->graph_capture ? 1 : 0;
  return 0;
}

int fastembedr_hip_tsne_interp_info(fastembedr_hip_tsne* s, int* boxes, int* nodes, int* fft_len, float* box_width,
                                    double* z) {
  if (!valid_state_args(s)) return 1;
  DeviceScalars h;
  if (!hip_ok(hipMemcpyAsync(&h, s->sc, sizeof(h), hipMemcpyDeviceToHost, s->stream), "hipMemcpy(scalars)") ||
      !hip_ok(hipStreamSynchronize(s->stream), "hipStreamSynchronize(scalars)")) {
    return 1;
  }
  if (boxes != nullptr) *boxes = h.lg_boxes;
  if (nodes != nullptr) *nodes = h.lg_nodes;
  if (fft_len != nullptr) *fft_len = s->lg_last_fft;
  if (box_width != nullptr) *box_width = h.lg_box_w;
  if (z != nullptr) *z = h.sum_q - static_cast<double>(s->n);
  return 0;
}

int fastembedr_hip_tsne_kl(fastembedr_hip_tsne* s, double* kl) { return fastembedr_hip_tsne_kl_rows(s, kl, nullptr); }

int fastembedr_hip_tsne_kl_rows(fastembedr_hip_tsne* s, double* kl, double* row_costs) {
  if (!valid_state_args(s) || kl == nullptr) return 1;
  const int zb = fehip::exact_blocks_for(s->n);
  std::vector<double> part(static_cast<std::size_t>(std::max(zb, 1024)));
  if (!hip_ok(fehip::launch_exact_z_double(s->y_a(), s->n, s->dpartial, s->stream), "exact_z launch") ||
      !hip_ok(hipMemcpyAsync(part.data(), s->dpartial, zb * sizeof(double), hipMemcpyDeviceToHost, s->stream),
              "copy z partials") ||
      !hip_ok(hipStreamSynchronize(s->stream), "kl sync")) {
    return 1;
  }
  double z = 0.0;
  for (int b = 0; b < zb; ++b) z += part[b];
  const double sum_q = static_cast<double>(static_cast<float>(std::max(z, static_cast<double>(FLT_MIN))));
  const int kb = 1024;
  // Row terms go to the gradient buffer (n 8-byte values, unused between
  // iterations) and are returned through the permuted download, which moves
  // 8-byte elements.
  double* rows_dev = row_costs != nullptr ? reinterpret_cast<double*>(s->grad) : nullptr;
  static_assert(sizeof(double) == sizeof(float2), "a row term fits one float2 slot");
  if (!hip_ok(fehip::launch_kl_rows(s->work_p(), s->y_a(), sum_q, s->dpartial, kb, s->stream, rows_dev),
              "kl launch") ||
      !hip_ok(hipMemcpyAsync(part.data(), s->dpartial, kb * sizeof(double), hipMemcpyDeviceToHost, s->stream),
              "copy kl partials") ||
      !hip_ok(hipStreamSynchronize(s->stream), "kl sync")) {
    return 1;
  }
  double total = 0.0;
  for (int b = 0; b < kb; ++b) total += part[b];
  *kl = total;
  if (row_costs != nullptr &&
      !download_permuted(s, reinterpret_cast<const float2*>(rows_dev), reinterpret_cast<float*>(row_costs))) {
    return 1;
  }
  return 0;
}

int fastembedr_hip_tsne_set_timing(fastembedr_hip_tsne* s, int enabled) {
  if (!valid_state_args(s)) return 1;
  if (!s->harvest_timing()) return 1;
  s->timing = enabled != 0;
  s->timed_only = enabled >= 2 ? (enabled - 2) & 0xffff : -1;
  s->timing_every = enabled >= 2 ? std::max(1, enabled >> 16) : 1;
  s->timing_iter = 0;
  if (enabled) {
    std::fill(std::begin(s->launches), std::end(s->launches), 0LL);
    std::fill(std::begin(s->total_ms), std::end(s->total_ms), 0.0);
  }
  return 0;
}

int fastembedr_hip_tsne_timing_stats(fastembedr_hip_tsne* s, int max_kernels, long long* launches,
                                     double* total_ms) {
  if (!valid_state_args(s)) return 1;
  if (!s->harvest_timing()) return 1;
  const int m = std::min(max_kernels, static_cast<int>(fehip::kKernelCount));
  for (int i = 0; i < m; ++i) {
    if (launches != nullptr) launches[i] = s->launches[i];
    if (total_ms != nullptr) total_ms[i] = s->total_ms[i];
  }
  return 0;
}

const char* fastembedr_hip_tsne_kernel_name(int kernel_id) {
  if (kernel_id < 0 || kernel_id >= fehip::kKernelCount) return "";
  return kKernelNames[kernel_id];
}

int fastembedr_hip_tsne_kernel_count(void) { return fehip::kKernelCount; }

int fastembedr_hip_random_init(int n, unsigned int seed, float* out) {
  if (n < 1 || out == nullptr) {
    set_error("invalid random_init arguments");
    return 1;
  }
  const std::vector<float> y = random_init(n, seed);
  std::copy(y.begin(), y.end(), out);
  return 0;
}

int fastembedr_hip_tsne_p_build_ms(const fastembedr_hip_tsne* s, double* ms) {
  if (!valid_state_args(s) || ms == nullptr) return 1;
  *ms = s->p_build_ms;
  return 0;
}

static_assert(FASTEMBEDR_HIP_KNN_EUCLIDEAN == fehip::kKnnEuclidean && FASTEMBEDR_HIP_KNN_COSINE == fehip::kKnnCosine &&
                  FASTEMBEDR_HIP_KNN_CORRELATION == fehip::kKnnCorrelation,
              "metric codes of the C ABI and the search agree");

int fastembedr_hip_knn_exact_metric(const float* x, int n, int d, int x_col_major, int k, int exclude_self,
                                    int metric, int x_on_device, int* indices, float* distances,
                                    int output_on_device, long long* stats) {
  g_last_error.clear();
  std::string err;
  if (fehip::knn_exact_run(x, n, d, x_col_major, k, exclude_self, metric, x_on_device, indices, distances,
                           output_on_device, stats, err) != 0) {
    set_error("fastembedr_hip_knn_exact: " + err);
    return 1;
  }
  return 0;
}

int fastembedr_hip_knn_exact(const float* x, int n, int d, int x_col_major, int k, int exclude_self, int x_on_device,
                             int* indices, float* distances, int output_on_device, long long* stats) {
  return fastembedr_hip_knn_exact_metric(x, n, d, x_col_major, k, exclude_self, FASTEMBEDR_HIP_KNN_EUCLIDEAN,
                                         x_on_device, indices, distances, output_on_device, stats);
}

int fastembedr_hip_structure_metrics(const double* high, int n, int p_high, const double* low, int p_low,
                                     const int* requested_k, int nk, double* out) {
  g_last_error.clear();
  std::string err;
  if (fehip::structure_metrics_run(high, n, p_high, low, p_low, requested_k, nk, out, err) != 0) {
    set_error("fastembedr_hip_structure_metrics: " + err);
    return 1;
  }
  return 0;
}

int fastembedr_hip_knn_query_metric(const float* reference, int n_reference, const float* query, int n_query,
                                    int d, int col_major, int k, int metric, int inputs_on_device, int* indices,
                                    float* distances, int output_on_device, long long* stats) {
  g_last_error.clear();
  std::string err;
  if (fehip::knn_query_run(reference, n_reference, query, n_query, d, col_major, k, metric, inputs_on_device,
                           indices, distances, output_on_device, stats, err) != 0) {
    set_error("fastembedr_hip_knn_query: " + err);
    return 1;
  }
  return 0;
}

int fastembedr_hip_knn_query(const float* reference, int n_reference, const float* query, int n_query, int d,
                             int col_major, int k, int inputs_on_device, int* indices, float* distances,
                             int output_on_device, long long* stats) {
  return fastembedr_hip_knn_query_metric(reference, n_reference, query, n_query, d, col_major, k,
                                         FASTEMBEDR_HIP_KNN_EUCLIDEAN, inputs_on_device, indices, distances,
                                         output_on_device, stats);
}

}  // extern "C"
