// CPU oracle for the openTSNE-style t-SNE gradient loop.
//
// TEST INFRASTRUCTURE ONLY.  This file is a restatement, in independent C++17,
// of the reference package's CPU path (src/tsne_neighbors.cpp of
// tkcaccia/fastEmbedR).  It exists so that tests/, bench.py's cpu_baseline leg
// and __graft_entry__.smoke() have a checker for the HIP backend.  No product
// code may link, load or call it; the HIP library never falls back to it.
//
// Every function cites the reference lines whose semantics it restates.  The
// arithmetic is kept in the same precision and operation order as the
// reference (fp32 where it is fp32, fp64 accumulators where it uses fp64), and
// the file is compiled with -ffp-contract=off so that no multiply-add is fused,
// matching an x86-64 build of the reference without -mfma.
//
// Pinning (what checks this restatement independently of itself) lives in
// tests/test_oracle_*.py: row entropy / row sums and a float64 bisection for
// the perplexity search, a scipy.sparse closed form for the symmetrisation,
// numpy.fft for the grid convolution, the O(n^2) closed form for the exact
// gradient and KL, and elementwise closed forms for the update.
//
// Extensions that the reference does not have (marked "extension" below):
//   * an explicit grid size up to 4096 (the reference clamps to [32, 512]);
//   * the FIt-SNE order-p Lagrange interpolation grid ("lagrange" repulsion),
//     restating Linderman et al., Nat. Methods 16, 243 (2019); this function is
//     pinned against the exact O(n^2) gradient only.

#include <algorithm>
#include <array>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <complex>
#include <condition_variable>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <numeric>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_error;

// ---------------------------------------------------------------------------
// Worker pool.  Same static partition as the reference's ParallelExecutor
// (src/tsne_neighbors.cpp:127-172,176-205): chunk = ceil(n / threads), worker t
// owns [t*chunk, min(n, (t+1)*chunk)); thread 0 is the caller.  The partition
// matters because per-chunk fp64 partial sums are combined in worker order.
// ---------------------------------------------------------------------------
class Pool {
 public:
  static Pool& get() {
    static Pool pool;
    return pool;
  }

  void run(int n, int threads, const std::function<void(int, int, int)>& fn) {
    const int active = std::max(1, std::min(threads, std::max(1, n)));
    if (active <= 1 || n < 2) {
      fn(0, n, 0);
      return;
    }
    std::lock_guard<std::mutex> call_lock(call_mutex_);
    ensure(active - 1);
    const int chunk = (n + active - 1) / active;
    {
      std::lock_guard<std::mutex> lock(mutex_);
      task_ = &fn;
      n_ = n;
      chunk_ = chunk;
      active_ = active;
      done_ = 0;
      ++generation_;
    }
    cv_start_.notify_all();
    fn(0, std::min(n, chunk), 0);
    std::unique_lock<std::mutex> lock(mutex_);
    cv_done_.wait(lock, [&] { return done_ == static_cast<int>(workers_.size()); });
    task_ = nullptr;
  }

  ~Pool() {
    {
      std::lock_guard<std::mutex> lock(mutex_);
      stop_ = true;
      ++generation_;
    }
    cv_start_.notify_all();
    for (auto& w : workers_) w.join();
  }

 private:
  void ensure(int n_workers) {
    while (static_cast<int>(workers_.size()) < n_workers) {
      // A new worker must not run the generation that is already published.
      const int id = static_cast<int>(workers_.size()) + 1;
      std::uint64_t seen;
      {
        std::lock_guard<std::mutex> lock(mutex_);
        seen = generation_;
      }
      workers_.emplace_back([this, id, seen] { loop(id, seen); });
    }
  }

  void loop(int id, std::uint64_t seen) {
    for (;;) {
      const std::function<void(int, int, int)>* task = nullptr;
      int begin = 0, end = 0;
      {
        std::unique_lock<std::mutex> lock(mutex_);
        cv_start_.wait(lock, [&] { return stop_ || generation_ != seen; });
        if (stop_) return;
        seen = generation_;
        task = task_;
        if (id < active_) {
          begin = id * chunk_;
          end = std::min(n_, begin + chunk_);
        }
      }
      if (task != nullptr && begin < end) (*task)(begin, end, id);
      {
        std::lock_guard<std::mutex> lock(mutex_);
        ++done_;
        if (done_ == static_cast<int>(workers_.size())) cv_done_.notify_one();
      }
    }
  }

  std::mutex call_mutex_;
  std::mutex mutex_;
  std::condition_variable cv_start_, cv_done_;
  std::vector<std::thread> workers_;
  const std::function<void(int, int, int)>* task_ = nullptr;
  std::uint64_t generation_ = 0;
  int n_ = 0, chunk_ = 0, active_ = 1, done_ = 0;
  bool stop_ = false;
};

template <typename F>
void parallel_for(int n, int threads, F&& body) {
  std::function<void(int, int, int)> fn = [&](int b, int e, int t) { body(b, e, t); };
  Pool::get().run(n, threads, fn);
}

// ---------------------------------------------------------------------------
// Symmetric sparse P (src/tsne_neighbors.cpp:32-54, 488-648)
// ---------------------------------------------------------------------------
struct CsrP {
  int n = 0;
  std::vector<int> row_ptr;
  std::vector<int> col;
  std::vector<float> val;
};

// 1-based iff every index lies in [1, n] (src/tsne_neighbors.cpp:79-90).
int detect_index_base(const int* idx_cm, int n, int k) {
  int lo = std::numeric_limits<int>::max();
  int hi = std::numeric_limits<int>::min();
  const std::size_t total = static_cast<std::size_t>(n) * k;
  for (std::size_t e = 0; e < total; ++e) {
    lo = std::min(lo, idx_cm[e]);
    hi = std::max(hi, idx_cm[e]);
  }
  return (lo >= 1 && hi <= n) ? 1 : 0;
}

// Per-row fp32 bisection on beta (src/tsne_neighbors.cpp:488-538).
// `d` is one row of k distances; writes the normalised conditional p_{j|i}.
// Returns the number of search steps taken; *beta_out receives the final beta.
int row_search_fp32(const float* d, int k, double perplexity, float* p, float* beta_out) {
  std::fill(p, p + k, 0.0f);
  const float target = static_cast<float>(std::log(perplexity));
  float beta = 1.0f;
  float lo = -FLT_MAX;
  float hi = FLT_MAX;
  float mass = FLT_MIN;
  bool done = false;
  int steps = 0;
  while (!done && steps < 200) {
    mass = FLT_MIN;
    for (int j = 0; j < k; ++j) {
      const float sq = d[j] * d[j];
      const float w = std::exp(-beta * sq);
      p[j] = w;
      mass += w;
    }
    float h = 0.0f;
    for (int j = 0; j < k; ++j) h += beta * (d[j] * d[j] * p[j]);
    h = h / mass + std::log(mass);
    const float gap = h - target;
    ++steps;
    if (std::fabs(gap) < 1e-5f) {
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
  for (int j = 0; j < k; ++j) p[j] *= inv;
  if (beta_out != nullptr) *beta_out = beta;
  return steps;
}

struct KeyedValue {
  std::uint64_t key;
  float value;
};

// Edges in ascending key order, the order the reference's std::sort of the
// whole array gives (src/tsne_neighbors.cpp:593-596): a counting pass places
// them by the row part of the key (key >> 32), then each row's run is sorted
// on its own, rows in parallel.  Equal keys are summed afterwards, so their
// relative order only matters at fp64 rounding when three or more coincide.
void sort_edges(std::vector<KeyedValue>& edges, int n, int threads) {
  std::vector<std::size_t> start(static_cast<std::size_t>(n) + 1, 0);
  for (const KeyedValue& e : edges) ++start[static_cast<std::size_t>(e.key >> 32) + 1];
  for (int i = 0; i < n; ++i) start[static_cast<std::size_t>(i) + 1] += start[static_cast<std::size_t>(i)];
  std::vector<KeyedValue> out(edges.size());
  {
    std::vector<std::size_t> cursor(start.begin(), start.end() - 1);
    for (const KeyedValue& e : edges) out[cursor[static_cast<std::size_t>(e.key >> 32)]++] = e;
  }
  std::vector<KeyedValue>().swap(edges);
  parallel_for(n, threads, [&](int b, int e, int) {
    for (int i = b; i < e; ++i) {
      std::sort(out.begin() + static_cast<std::ptrdiff_t>(start[static_cast<std::size_t>(i)]),
                out.begin() + static_cast<std::ptrdiff_t>(start[static_cast<std::size_t>(i) + 1]),
                [](const KeyedValue& x, const KeyedValue& y) { return x.key < y.key; });
    }
  });
  edges.swap(out);
}

// Directed KNN edges -> symmetric CSR (src/tsne_neighbors.cpp:540-648).
// Inputs are R-ordered (column-major n x k); the reference copies distances to
// row-major first (src/tsne_neighbors.cpp:327-352), which is what `dist_rm` is.
bool build_symmetric_p(const int* idx_cm, const float* dist_cm, int n, int k,
                       double perplexity, int threads, CsrP& out) {
  const int base = detect_index_base(idx_cm, n, k);
  std::vector<float> dist_rm(static_cast<std::size_t>(n) * k);
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < k; ++j)
      dist_rm[static_cast<std::size_t>(i) * k + j] = dist_cm[static_cast<std::size_t>(j) * n + i];
  for (int i = 0; i < n; ++i) {
    for (int j = 0; j < k; ++j) {
      const int nb = idx_cm[static_cast<std::size_t>(j) * n + i] - base;
      if (nb < 0 || nb >= n) {
        g_error = "KNN indices are out of range.";
        return false;
      }
      const float dv = dist_rm[static_cast<std::size_t>(i) * k + j];
      if (!std::isfinite(dv) || dv < 0.0f) {
        g_error = "KNN distances must be finite and non-negative.";
        return false;
      }
    }
  }

  const int t_count = std::max(1, threads);
  std::vector<std::vector<KeyedValue>> per_thread(static_cast<std::size_t>(t_count));
  parallel_for(n, t_count, [&](int b, int e, int t) {
    std::vector<float> p(static_cast<std::size_t>(k));
    auto& bucket = per_thread[static_cast<std::size_t>(t)];
    bucket.reserve(static_cast<std::size_t>(e - b) * k);
    for (int i = b; i < e; ++i) {
      row_search_fp32(dist_rm.data() + static_cast<std::size_t>(i) * k, k, perplexity, p.data(), nullptr);
      for (int j = 0; j < k; ++j) {
        const int nb = idx_cm[static_cast<std::size_t>(j) * n + i] - base;
        if (nb == i) continue;  // self column: searched over, then dropped
        const std::uint32_t a = static_cast<std::uint32_t>(std::min(i, nb));
        const std::uint32_t c = static_cast<std::uint32_t>(std::max(i, nb));
        bucket.push_back({(static_cast<std::uint64_t>(a) << 32) | c, p[static_cast<std::size_t>(j)]});
      }
    }
  });
  std::vector<KeyedValue> edges;
  {
    std::size_t total = 0;
    for (auto& b : per_thread) total += b.size();
    edges.reserve(total);
    for (auto& b : per_thread) {
      edges.insert(edges.end(), b.begin(), b.end());
      std::vector<KeyedValue>().swap(b);
    }
  }
  if (edges.empty()) {
    g_error = "KNN graph produced no non-self t-SNE edges.";
    return false;
  }
  sort_edges(edges, n, t_count);

  out.n = n;
  out.row_ptr.assign(static_cast<std::size_t>(n) + 1, 0);
  std::size_t unique = 0;
  double mass = 0.0;
  for (std::size_t r = 0; r < edges.size();) {
    const std::uint64_t key = edges[r].key;
    double s = 0.0;
    for (; r < edges.size() && edges[r].key == key; ++r) s += static_cast<double>(edges[r].value);
    edges[unique++] = {key, static_cast<float>(s)};
    mass += s;
    out.row_ptr[static_cast<std::size_t>(key >> 32) + 1] += 1;
    out.row_ptr[static_cast<std::size_t>(key & 0xffffffffu) + 1] += 1;
  }
  edges.resize(unique);
  if (!std::isfinite(mass) || mass <= 0.0) {
    g_error = "t-SNE probability normalization failed.";
    return false;
  }
  for (int i = 0; i < n; ++i) out.row_ptr[i + 1] += out.row_ptr[i];
  out.col.assign(static_cast<std::size_t>(out.row_ptr[n]), 0);
  out.val.assign(out.col.size(), 0.0f);
  std::vector<int> cursor(out.row_ptr.begin(), out.row_ptr.end() - 1);
  const float scale = static_cast<float>(0.5 / mass);
  for (const KeyedValue& e : edges) {
    const int a = static_cast<int>(e.key >> 32);
    const int c = static_cast<int>(e.key & 0xffffffffu);
    const float v = e.value * scale;
    int at = cursor[a]++;
    out.col[at] = c;
    out.val[at] = v;
    at = cursor[c]++;
    out.col[at] = a;
    out.val[at] = v;
  }
  return true;
}

// ---------------------------------------------------------------------------
// FFT-grid repulsion (src/tsne_neighbors.cpp:392-398, 650-942, 1076-1182)
// ---------------------------------------------------------------------------
using cf = std::complex<float>;

// Grid-size policy (src/tsne_neighbors.cpp:392-398): 64/128/256 nodes per axis
// below 10k / below 50k / from 50k points, overridable by
// FASTEMBEDR_TSNE_FFT_GRID, rounded up to a power of two in [32, 512].
int policy_grid_size(int n) {
  const int fallback = n >= 50000 ? 256 : (n >= 10000 ? 128 : 64);
  int requested = fallback;
  if (const char* raw = std::getenv("FASTEMBEDR_TSNE_FFT_GRID")) {
    char* end = nullptr;
    const long v = std::strtol(raw, &end, 10);
    if (raw[0] != '\0' && end != raw && v > 0 && v <= std::numeric_limits<int>::max())
      requested = static_cast<int>(v);
  }
  int g = 32;
  while (g < requested && g < 512) g <<= 1;
  return std::max(32, std::min(512, g));
}

// extension: explicit sizes are honoured as powers of two in [4, 4096].
int resolve_grid_size(int n, int requested) {
  if (requested <= 0) return policy_grid_size(n);
  int g = 4;
  while (g < requested && g < 4096) g <<= 1;
  return g;
}

// The bilinear grid's pieces are templates on the arithmetic type, as the
// reference's are (FftGridWorkspaceT<T>, fft_1d_t, fft_2d_t,
// bilinear_grid_value_t, src/tsne_neighbors.cpp:650-942): T = float is the
// reference's path; T = double evaluates the same algorithm in fp64, the
// yardstick that separates either fp32 side's rounding from the other's.
template <typename T>
struct Radix2PlanT {
  using C = std::complex<T>;
  int size = 0;
  std::vector<int> rev;
  std::vector<C> up;    // e^{+2 pi i / len}, used by the transform the reference calls forward
  std::vector<C> down;  // e^{-2 pi i / len}
  void build(int f) {
    if (size == f) return;
    size = f;
    int bits = 0;
    for (int v = f; v > 1; v >>= 1) ++bits;
    rev.assign(static_cast<std::size_t>(f), 0);
    for (int i = 0; i < f; ++i) {
      unsigned r = 0, v = static_cast<unsigned>(i);
      for (int b = 0; b < bits; ++b) {
        r = (r << 1) | (v & 1u);
        v >>= 1;
      }
      rev[static_cast<std::size_t>(i)] = static_cast<int>(r);
    }
    up.clear();
    down.clear();
    for (int len = 2; len <= f; len <<= 1) {
      const T ang = static_cast<T>(6.283185307179586476925286766559) / static_cast<T>(len);
      up.emplace_back(std::cos(ang), std::sin(ang));
      down.emplace_back(std::cos(-ang), std::sin(-ang));
    }
  }
};

// Iterative radix-2 decimation-in-time with bit reversal and a per-stage
// twiddle recurrence w *= root (src/tsne_neighbors.cpp:697-729).  The
// reference's "forward" transform uses the +i exponent; the convolution below
// only needs forward/inverse to be mutually inverse.
template <typename T>
void fft_radix2(std::complex<T>* a, int f, bool inverse, const Radix2PlanT<T>& plan) {
  using C = std::complex<T>;
  for (int i = 1; i < f; ++i) {
    const int j = plan.rev[static_cast<std::size_t>(i)];
    if (i < j) std::swap(a[i], a[j]);
  }
  const std::vector<C>& roots = inverse ? plan.down : plan.up;
  int stage = 0;
  for (int len = 2; len <= f; len <<= 1, ++stage) {
    const C root = roots[static_cast<std::size_t>(stage)];
    const int half = len >> 1;
    for (int s = 0; s < f; s += len) {
      C w(T(1), T(0));
      for (int j = 0; j < half; ++j) {
        const C u = a[s + j];
        const C v = a[s + j + half] * w;
        a[s + j] = u + v;
        a[s + j + half] = u - v;
        w *= root;
      }
    }
  }
  if (inverse) {
    const T sc = T(1) / static_cast<T>(f);
    for (int i = 0; i < f; ++i) a[i] *= sc;
  }
}

// Rows, then columns through a per-thread scratch column
// (src/tsne_neighbors.cpp:731-758).
template <typename T>
void fft_2d(std::vector<std::complex<T>>& grid, int f, bool inverse, int threads, const Radix2PlanT<T>& plan,
            std::vector<std::complex<T>>& scratch) {
  parallel_for(f, threads, [&](int b, int e, int) {
    for (int r = b; r < e; ++r) fft_radix2<T>(grid.data() + static_cast<std::size_t>(r) * f, f, inverse, plan);
  });
  if (static_cast<int>(scratch.size()) < f * std::max(1, threads))
    scratch.assign(static_cast<std::size_t>(f) * std::max(1, threads), std::complex<T>());
  parallel_for(f, threads, [&](int b, int e, int t) {
    std::complex<T>* column = scratch.data() + static_cast<std::size_t>(t) * f;
    for (int c = b; c < e; ++c) {
      for (int r = 0; r < f; ++r) column[r] = grid[static_cast<std::size_t>(r) * f + c];
      fft_radix2<T>(column, f, inverse, plan);
      for (int r = 0; r < f; ++r) grid[static_cast<std::size_t>(r) * f + c] = column[r];
    }
  });
}

// Bilinear read of a g x g grid at fractional node coordinates
// (src/tsne_neighbors.cpp:760-781).
template <typename T>
T bilinear(const std::vector<T>& grid, int g, T gx, T gy) {
  const T cx = std::max(T(0), std::min(static_cast<T>(g - 1), gx));
  const T cy = std::max(T(0), std::min(static_cast<T>(g - 1), gy));
  const int x0 = std::max(0, std::min(g - 2, static_cast<int>(std::floor(cx))));
  const int y0 = std::max(0, std::min(g - 2, static_cast<int>(std::floor(cy))));
  const T tx = cx - static_cast<T>(x0);
  const T ty = cy - static_cast<T>(y0);
  const T v00 = grid[static_cast<std::size_t>(y0) * g + x0];
  const T v10 = grid[static_cast<std::size_t>(y0) * g + x0 + 1];
  const T v01 = grid[static_cast<std::size_t>(y0 + 1) * g + x0];
  const T v11 = grid[static_cast<std::size_t>(y0 + 1) * g + x0 + 1];
  return (T(1) - tx) * (T(1) - ty) * v00 + tx * (T(1) - ty) * v10 +
         (T(1) - tx) * ty * v01 + tx * ty * v11;
}

template <typename T>
struct GridScratchT {
  int g = 0;
  Radix2PlanT<T> plan;
  std::vector<T> mass, mass_x, mass_y, gx, gy, q, q2, xq2, yq2;
  std::vector<std::complex<T>> f_mass, f_mx, f_my, k1, k2, work, column;
};
using GridScratch = GridScratchT<float>;

// Zero-padded circular convolution of the three charge grids with the Cauchy
// kernel and its square (src/tsne_neighbors.cpp:842-942).
template <typename T>
void grid_convolve(GridScratchT<T>& ws, T spacing, int threads) {
  using C = std::complex<T>;
  const int g = ws.g;
  const int f = 2 * g;
  const std::size_t ff = static_cast<std::size_t>(f) * f;
  ws.plan.build(f);
  auto pad = [&](const std::vector<T>& src, std::vector<C>& dst) {
    dst.assign(ff, C(T(0), T(0)));
    for (int r = 0; r < g; ++r)
      for (int c = 0; c < g; ++c)
        dst[static_cast<std::size_t>(r) * f + c] = C(src[static_cast<std::size_t>(r) * g + c], T(0));
  };
  pad(ws.mass, ws.f_mass);
  pad(ws.mass_x, ws.f_mx);
  pad(ws.mass_y, ws.f_my);
  ws.k1.assign(ff, C(T(0), T(0)));
  ws.k2.assign(ff, C(T(0), T(0)));
  for (int dy = -(g - 1); dy <= g - 1; ++dy) {
    const int row = dy < 0 ? dy + f : dy;
    const T oy = static_cast<T>(dy) * spacing;
    for (int dx = -(g - 1); dx <= g - 1; ++dx) {
      const int colx = dx < 0 ? dx + f : dx;
      const T ox = static_cast<T>(dx) * spacing;
      const T r2 = ox * ox + oy * oy;
      const T qv = T(1) / (T(1) + r2);
      const std::size_t at = static_cast<std::size_t>(row) * f + colx;
      ws.k1[at] = C(qv, T(0));
      ws.k2[at] = C(qv * qv, T(0));
    }
  }
  fft_2d<T>(ws.f_mass, f, false, threads, ws.plan, ws.column);
  fft_2d<T>(ws.f_mx, f, false, threads, ws.plan, ws.column);
  fft_2d<T>(ws.f_my, f, false, threads, ws.plan, ws.column);
  fft_2d<T>(ws.k1, f, false, threads, ws.plan, ws.column);
  fft_2d<T>(ws.k2, f, false, threads, ws.plan, ws.column);
  auto conv = [&](const std::vector<C>& a, const std::vector<C>& b, std::vector<T>& out) {
    ws.work.resize(ff);
    parallel_for(static_cast<int>(ff), threads, [&](int lo, int hi, int) {
      for (int i = lo; i < hi; ++i) ws.work[static_cast<std::size_t>(i)] = a[static_cast<std::size_t>(i)] * b[static_cast<std::size_t>(i)];
    });
    fft_2d<T>(ws.work, f, true, threads, ws.plan, ws.column);
    out.assign(static_cast<std::size_t>(g) * g, T(0));
    for (int r = 0; r < g; ++r)
      for (int c = 0; c < g; ++c)
        out[static_cast<std::size_t>(r) * g + c] = ws.work[static_cast<std::size_t>(r) * f + c].real();
  };
  conv(ws.f_mass, ws.k1, ws.q);
  conv(ws.f_mass, ws.k2, ws.q2);
  conv(ws.f_mx, ws.k2, ws.xq2);
  conv(ws.f_my, ws.k2, ws.yq2);
}

// Attractive term over the CSR rows (src/tsne_neighbors.cpp:985-1012);
// openTSNE convention, no factor 4.
template <typename T>
void add_attraction(const CsrP& p, const float* y, int n, T ex, int threads, T* grad) {
  parallel_for(n, threads, [&](int b, int e, int) {
    for (int i = b; i < e; ++i) {
      for (int at = p.row_ptr[i]; at < p.row_ptr[i + 1]; ++at) {
        const int j = p.col[static_cast<std::size_t>(at)];
        const T dx = static_cast<T>(y[2 * i]) - static_cast<T>(y[2 * j]);
        const T dy = static_cast<T>(y[2 * i + 1]) - static_cast<T>(y[2 * j + 1]);
        T r2 = T(0);
        r2 += dx * dx;
        r2 += dy * dy;
        const T qv = T(1) / (T(1) + r2);
        const T c = ex * static_cast<T>(p.val[static_cast<std::size_t>(at)]) * qv;
        grad[2 * i] += c * dx;
        grad[2 * i + 1] += c * dy;
      }
    }
  });
}

// Bilinear FFT-grid gradient (src/tsne_neighbors.cpp:1076-1182).  Geometry:
// square box of side 1.1 * span + 2e-3 centred on the bounding box, g nodes
// per axis; bilinear spread of (1, x, y) charges; convolution; bilinear read
// back; normalisation by sum(q) - n; attraction added last.  The layout y is
// fp32 (the optimiser's state) for either T.
template <typename T>
void gradient_grid(const CsrP& p, const float* y, int n, T ex, int g, int threads,
                   GridScratchT<T>& ws, T* grad, T* geometry_out) {
  std::fill(grad, grad + 2 * static_cast<std::size_t>(n), T(0));
  T min_x = y[0], max_x = y[0], min_y = y[1], max_y = y[1];
  for (int i = 1; i < n; ++i) {
    min_x = std::min(min_x, static_cast<T>(y[2 * i]));
    max_x = std::max(max_x, static_cast<T>(y[2 * i]));
    min_y = std::min(min_y, static_cast<T>(y[2 * i + 1]));
    max_y = std::max(max_y, static_cast<T>(y[2 * i + 1]));
  }
  const T cx = T(0.5) * (min_x + max_x);
  const T cy = T(0.5) * (min_y + max_y);
  T span = std::max(max_x - min_x, max_y - min_y);
  if (!std::isfinite(span) || span <= T(0)) span = T(1);
  const T half = static_cast<T>(0.55) * span + static_cast<T>(1.0e-3);
  const T lo_x = cx - half;
  const T lo_y = cy - half;
  const T h = (T(2) * half) / static_cast<T>(g - 1);
  const T inv_h = T(1) / h;
  if (geometry_out != nullptr) {
    geometry_out[0] = lo_x;
    geometry_out[1] = lo_y;
    geometry_out[2] = h;
    geometry_out[3] = inv_h;
  }

  ws.g = g;
  const std::size_t gg = static_cast<std::size_t>(g) * g;
  ws.mass.assign(gg, T(0));
  ws.mass_x.assign(gg, T(0));
  ws.mass_y.assign(gg, T(0));
  ws.gx.assign(static_cast<std::size_t>(n), T(0));
  ws.gy.assign(static_cast<std::size_t>(n), T(0));
  for (int i = 0; i < n; ++i) {  // sequential on purpose, as in the reference
    const T px = y[2 * i];
    const T py = y[2 * i + 1];
    const T ux = std::max(T(0), std::min(static_cast<T>(g - 1), (px - lo_x) * inv_h));
    const T uy = std::max(T(0), std::min(static_cast<T>(g - 1), (py - lo_y) * inv_h));
    const int x0 = std::max(0, std::min(g - 2, static_cast<int>(std::floor(ux))));
    const int y0 = std::max(0, std::min(g - 2, static_cast<int>(std::floor(uy))));
    const T tx = ux - static_cast<T>(x0);
    const T ty = uy - static_cast<T>(y0);
    ws.gx[static_cast<std::size_t>(i)] = ux;
    ws.gy[static_cast<std::size_t>(i)] = uy;
    const T w00 = (T(1) - tx) * (T(1) - ty);
    const T w10 = tx * (T(1) - ty);
    const T w01 = (T(1) - tx) * ty;
    const T w11 = tx * ty;
    const std::size_t a00 = static_cast<std::size_t>(y0) * g + x0;
    const std::size_t a10 = a00 + 1;
    const std::size_t a01 = a00 + g;
    const std::size_t a11 = a01 + 1;
    ws.mass[a00] += w00;
    ws.mass[a10] += w10;
    ws.mass[a01] += w01;
    ws.mass[a11] += w11;
    ws.mass_x[a00] += w00 * px;
    ws.mass_x[a10] += w10 * px;
    ws.mass_x[a01] += w01 * px;
    ws.mass_x[a11] += w11 * px;
    ws.mass_y[a00] += w00 * py;
    ws.mass_y[a10] += w10 * py;
    ws.mass_y[a01] += w01 * py;
    ws.mass_y[a11] += w11 * py;
  }

  grid_convolve<T>(ws, h, threads);

  const int t_count = std::max(1, threads);
  std::vector<double> partial(static_cast<std::size_t>(t_count), 0.0);
  parallel_for(n, t_count, [&](int b, int e, int t) {
    double acc = 0.0;
    for (int i = b; i < e; ++i)
      acc += static_cast<double>(bilinear<T>(ws.q, g, ws.gx[static_cast<std::size_t>(i)], ws.gy[static_cast<std::size_t>(i)]));
    partial[static_cast<std::size_t>(t)] = acc;
  });
  const double total = std::accumulate(partial.begin(), partial.end(), 0.0);
  const T inv_z = static_cast<T>(1.0 / std::max(total - static_cast<double>(n), static_cast<double>(FLT_MIN)));

  parallel_for(n, t_count, [&](int b, int e, int) {
    for (int i = b; i < e; ++i) {
      const T ux = ws.gx[static_cast<std::size_t>(i)];
      const T uy = ws.gy[static_cast<std::size_t>(i)];
      const T a = bilinear<T>(ws.q2, g, ux, uy);
      const T bx = bilinear<T>(ws.xq2, g, ux, uy);
      const T by = bilinear<T>(ws.yq2, g, ux, uy);
      grad[2 * i] = -(static_cast<T>(y[2 * i]) * a - bx) * inv_z;
      grad[2 * i + 1] = -(static_cast<T>(y[2 * i + 1]) * a - by) * inv_z;
    }
  });
  add_attraction<T>(p, y, n, ex, t_count, grad);
}

// Exact O(n^2) repulsion with a strided pair partition
// (src/tsne_neighbors.cpp:1014-1074).
void gradient_exact(const CsrP& p, const float* y, int n, float ex, int threads, float* grad) {
  const int t_count = std::max(1, threads);
  std::fill(grad, grad + 2 * static_cast<std::size_t>(n), 0.0f);
  std::vector<std::vector<float>> local(static_cast<std::size_t>(t_count),
                                        std::vector<float>(2 * static_cast<std::size_t>(n), 0.0f));
  std::vector<double> zpart(static_cast<std::size_t>(t_count), 0.0);
  auto worker = [&](int t) {
    std::vector<float>& g = local[static_cast<std::size_t>(t)];
    double z = 0.0;
    for (int i = t; i < n - 1; i += t_count) {
      for (int j = i + 1; j < n; ++j) {
        float r2 = 0.0f;
        const float ddx = y[2 * i] - y[2 * j];
        r2 += ddx * ddx;
        const float ddy = y[2 * i + 1] - y[2 * j + 1];
        r2 += ddy * ddy;
        const float qv = 1.0f / (1.0f + r2);
        z += 2.0 * static_cast<double>(qv);
        const float c = -(qv * qv);
        const float sx = c * (y[2 * i] - y[2 * j]);
        g[2 * i] += sx;
        g[2 * j] -= sx;
        const float sy = c * (y[2 * i + 1] - y[2 * j + 1]);
        g[2 * i + 1] += sy;
        g[2 * j + 1] -= sy;
      }
    }
    zpart[static_cast<std::size_t>(t)] = z;
  };
  if (t_count == 1) {
    worker(0);
  } else {
    std::vector<std::thread> pool;
    for (int t = 1; t < t_count; ++t) pool.emplace_back(worker, t);
    worker(0);
    for (auto& th : pool) th.join();
  }
  const float inv_z = static_cast<float>(
      1.0 / std::max(std::accumulate(zpart.begin(), zpart.end(), 0.0), static_cast<double>(FLT_MIN)));
  const int total = 2 * n;
  parallel_for(total, t_count, [&](int b, int e, int) {
    for (int idx = b; idx < e; ++idx) {
      float v = 0.0f;
      for (int t = 0; t < t_count; ++t) v += local[static_cast<std::size_t>(t)][static_cast<std::size_t>(idx)];
      grad[idx] = v * inv_z;
    }
  });
  add_attraction(p, y, n, ex, t_count, grad);
}

// ---------------------------------------------------------------------------
// extension: FIt-SNE interpolation grid (Linderman et al., Nat. Methods 16,
// 243 (2019), Algorithm 1, in its two-dimensional form).
//
// Geometry: one square region [lo, lo + span]^2 with lo the smallest and
// lo + span the largest coordinate over both axes; n_boxes per axis =
// max(min_intervals, ceil(span / ints_per_unit)), capped so that the node
// count stays <= kLagrangeMaxNodes (the FFT length 2 * nodes <= 4096); box
// width w = span / n_boxes.  Each box holds `order` equispaced nodes per
// axis at (j + 1/2) w / order, so nodes are private to their box.
// Charges (1, x, y, x^2 + y^2) are spread with order-p Lagrange weights; one
// kernel, the squared Cauchy kernel 1 / (1 + d^2)^2 between nodes, is
// convolved with all four; the potentials are interpolated back with the
// same weights and combined as
//   Z   = sum_i [(1 + |y_i|^2) phi0 - 2 (x_i phi1 + y_i phi2) + phi3] - n
//   F_i = (y_i phi0 - (phi1, phi2)) / Z.
// Everything after the geometry is fp64, so this is an accurate check for
// the fp32 device version.  The convolution is a zero-padded fp64 FFT of
// power-of-two length f >= 2 * nodes (any f >= 2 * nodes - 1 gives the same
// linear convolution); `direct` replaces it by the O(nodes^4) node sum.
// ---------------------------------------------------------------------------
constexpr int kLagrangeMaxNodes = 2048;

struct LagrangeGeometry {
  int boxes = 0;
  int order = 3;
  int nodes = 0;  // boxes * order per axis
  double lo = 0.0;
  double box_w = 0.0;
  double node_h = 0.0;
};

LagrangeGeometry lagrange_geometry(const float* y, int n, int order, int min_intervals, float ints_per_unit) {
  float mnf = y[0], mxf = y[0];
  for (std::size_t e = 0; e < 2 * static_cast<std::size_t>(n); ++e) {
    mnf = std::min(mnf, y[e]);
    mxf = std::max(mxf, y[e]);
  }
  double span = static_cast<double>(mxf) - static_cast<double>(mnf);
  if (!(span > 0.0) || !std::isfinite(span)) span = 1.0;
  long long boxes = static_cast<long long>(std::ceil(span / static_cast<double>(ints_per_unit)));
  boxes = std::max<long long>(boxes, min_intervals);
  boxes = std::min<long long>(boxes, kLagrangeMaxNodes / order);
  LagrangeGeometry g;
  g.order = order;
  g.boxes = static_cast<int>(boxes);
  g.nodes = g.boxes * order;
  g.lo = static_cast<double>(mnf);
  g.box_w = span / static_cast<double>(g.boxes);
  g.node_h = g.box_w / order;
  return g;
}

// Lagrange basis on the nodes (j + 1/2) / order of the unit box, at u.
void lagrange_weights(double u, int order, double* w) {
  for (int j = 0; j < order; ++j) {
    const double tj = (j + 0.5) / order;
    double num = 1.0, den = 1.0;
    for (int l = 0; l < order; ++l) {
      if (l == j) continue;
      const double tl = (l + 0.5) / order;
      num *= (u - tl);
      den *= (tj - tl);
    }
    w[j] = num / den;
  }
}

void lagrange_locate(const LagrangeGeometry& g, double v, int& box, double& u) {
  const double rel = (v - g.lo) / g.box_w;
  box = std::min(g.boxes - 1, std::max(0, static_cast<int>(std::floor(rel))));
  u = rel - box;
}

// In-place iterative radix-2 FFT of length f (a power of two), fp64, with
// twiddles tw[k] = e^{-2 pi i k / f} (conjugated for the inverse).
void fft_pow2(std::complex<double>* a, int f, bool inv, const std::vector<std::complex<double>>& tw) {
  for (int i = 1, j = 0; i < f; ++i) {
    int bit = f >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) std::swap(a[i], a[j]);
  }
  for (int len = 2; len <= f; len <<= 1) {
    const int stride = f / len;
    for (int i = 0; i < f; i += len) {
      for (int k = 0; k < len / 2; ++k) {
        const std::complex<double> w = inv ? std::conj(tw[static_cast<std::size_t>(k) * stride])
                                           : tw[static_cast<std::size_t>(k) * stride];
        const std::complex<double> u = a[i + k];
        const std::complex<double> v = a[i + k + len / 2] * w;
        a[i + k] = u + v;
        a[i + k + len / 2] = u - v;
      }
    }
  }
}

void fft2_pow2(std::vector<std::complex<double>>& a, int f, bool inv, int threads) {
  std::vector<std::complex<double>> tw(static_cast<std::size_t>(f / 2));
  for (int k = 0; k < f / 2; ++k) tw[static_cast<std::size_t>(k)] = std::polar(1.0, -2.0 * M_PI * k / f);
  parallel_for(f, threads, [&](int b, int e, int) {
    for (int r = b; r < e; ++r) fft_pow2(&a[static_cast<std::size_t>(r) * f], f, inv, tw);
  });
  parallel_for(f, threads, [&](int b, int e, int) {
    std::vector<std::complex<double>> col(static_cast<std::size_t>(f));
    for (int c = b; c < e; ++c) {
      for (int r = 0; r < f; ++r) col[static_cast<std::size_t>(r)] = a[static_cast<std::size_t>(r) * f + c];
      fft_pow2(col.data(), f, inv, tw);
      for (int r = 0; r < f; ++r) a[static_cast<std::size_t>(r) * f + c] = col[static_cast<std::size_t>(r)];
    }
  });
  if (inv) {
    const double s = 1.0 / (static_cast<double>(f) * f);
    for (auto& v : a) v *= s;
  }
}

// Potentials phi_t at every node (nodes x nodes x 4, row-major by y then x).
std::vector<double> lagrange_potentials(const std::vector<double>& charge, const LagrangeGeometry& g, bool direct,
                                        int threads) {
  const int m = g.nodes;
  const double h2 = g.node_h * g.node_h;
  auto kern = [&](int dx, int dy) {
    const double q = 1.0 / (1.0 + h2 * (static_cast<double>(dx) * dx + static_cast<double>(dy) * dy));
    return q * q;
  };
  std::vector<double> phi(static_cast<std::size_t>(m) * m * 4, 0.0);
  if (direct) {
    for (int ay = 0; ay < m; ++ay)
      for (int ax = 0; ax < m; ++ax) {
        double acc[4] = {0, 0, 0, 0};
        for (int by = 0; by < m; ++by)
          for (int bx = 0; bx < m; ++bx) {
            const double k = kern(ax - bx, ay - by);
            const double* c = &charge[(static_cast<std::size_t>(by) * m + bx) * 4];
            for (int t = 0; t < 4; ++t) acc[t] += k * c[t];
          }
        for (int t = 0; t < 4; ++t) phi[(static_cast<std::size_t>(ay) * m + ax) * 4 + t] = acc[t];
      }
    return phi;
  }
  int f = 1;
  while (f < 2 * m) f <<= 1;
  std::vector<std::complex<double>> kh(static_cast<std::size_t>(f) * f, 0.0);
  for (int r = 0; r < f; ++r) {
    const int dy = r < f / 2 ? r : r - f;
    if (std::abs(dy) >= m) continue;
    for (int c = 0; c < f; ++c) {
      const int dx = c < f / 2 ? c : c - f;
      if (std::abs(dx) >= m) continue;
      kh[static_cast<std::size_t>(r) * f + c] = kern(dx, dy);
    }
  }
  fft2_pow2(kh, f, false, threads);
  std::vector<std::complex<double>> buf(static_cast<std::size_t>(f) * f);
  for (int t = 0; t < 4; t += 2) {
    // two real charge grids per complex transform: conv(a + ib) = conv(a) + i conv(b)
    std::fill(buf.begin(), buf.end(), std::complex<double>(0.0, 0.0));
    for (int r = 0; r < m; ++r)
      for (int c = 0; c < m; ++c) {
        const double* ch = &charge[(static_cast<std::size_t>(r) * m + c) * 4];
        buf[static_cast<std::size_t>(r) * f + c] = std::complex<double>(ch[t], ch[t + 1]);
      }
    fft2_pow2(buf, f, false, threads);
    for (std::size_t e = 0; e < buf.size(); ++e) buf[e] *= kh[e];
    fft2_pow2(buf, f, true, threads);
    for (int r = 0; r < m; ++r)
      for (int c = 0; c < m; ++c) {
        const std::complex<double> v = buf[static_cast<std::size_t>(r) * f + c];
        phi[(static_cast<std::size_t>(r) * m + c) * 4 + t] = v.real();
        phi[(static_cast<std::size_t>(r) * m + c) * 4 + t + 1] = v.imag();
      }
  }
  return phi;
}

void gradient_lagrange(const CsrP& p, const float* y, int n, float ex, int order, int min_intervals,
                       float ints_per_unit, int threads, float* grad, LagrangeGeometry* geo_out,
                       bool direct = false, double* z_out = nullptr) {
  const LagrangeGeometry g = lagrange_geometry(y, n, order, min_intervals, ints_per_unit);
  if (geo_out != nullptr) *geo_out = g;
  const int m = g.nodes;
  std::vector<double> charge(static_cast<std::size_t>(m) * m * 4, 0.0);
  std::vector<double> wx(static_cast<std::size_t>(order)), wy(static_cast<std::size_t>(order));
  for (int i = 0; i < n; ++i) {
    const double px = y[2 * i], py = y[2 * i + 1];
    int bx, by;
    double ux, uy;
    lagrange_locate(g, px, bx, ux);
    lagrange_locate(g, py, by, uy);
    lagrange_weights(ux, order, wx.data());
    lagrange_weights(uy, order, wy.data());
    const double c[4] = {1.0, px, py, px * px + py * py};
    for (int a = 0; a < order; ++a)
      for (int b = 0; b < order; ++b) {
        const std::size_t node = static_cast<std::size_t>(by * order + a) * m + (bx * order + b);
        const double w = wy[static_cast<std::size_t>(a)] * wx[static_cast<std::size_t>(b)];
        for (int t = 0; t < 4; ++t) charge[node * 4 + t] += w * c[t];
      }
  }
  const std::vector<double> phi = lagrange_potentials(charge, g, direct, threads);
  std::vector<double> pot(static_cast<std::size_t>(n) * 4, 0.0);
  double z = 0.0;
  for (int i = 0; i < n; ++i) {
    const double px = y[2 * i], py = y[2 * i + 1];
    int bx, by;
    double ux, uy;
    lagrange_locate(g, px, bx, ux);
    lagrange_locate(g, py, by, uy);
    lagrange_weights(ux, order, wx.data());
    lagrange_weights(uy, order, wy.data());
    double ph[4] = {0, 0, 0, 0};
    for (int a = 0; a < order; ++a)
      for (int b = 0; b < order; ++b) {
        const std::size_t node = static_cast<std::size_t>(by * order + a) * m + (bx * order + b);
        const double w = wy[static_cast<std::size_t>(a)] * wx[static_cast<std::size_t>(b)];
        for (int t = 0; t < 4; ++t) ph[t] += w * phi[node * 4 + t];
      }
    for (int t = 0; t < 4; ++t) pot[static_cast<std::size_t>(i) * 4 + t] = ph[t];
    z += (1.0 + px * px + py * py) * ph[0] - 2.0 * (px * ph[1] + py * ph[2]) + ph[3];
  }
  z -= n;
  if (z_out != nullptr) *z_out = z;
  const double inv_z = 1.0 / std::max(z, static_cast<double>(FLT_MIN));
  for (int i = 0; i < n; ++i) {
    const double* ph = &pot[static_cast<std::size_t>(i) * 4];
    grad[2 * i] = static_cast<float>(-(y[2 * i] * ph[0] - ph[1]) * inv_z);
    grad[2 * i + 1] = static_cast<float>(-(y[2 * i + 1] * ph[0] - ph[2]) * inv_z);
  }
  add_attraction(p, y, n, ex, threads, grad);
}

// ---------------------------------------------------------------------------
// Optimiser (src/tsne_neighbors.cpp:1200-1256)
// ---------------------------------------------------------------------------
void zero_mean(float* y, int n) {
  double sx = 0.0, sy = 0.0;
  for (int i = 0; i < n; ++i) {
    sx += y[2 * i];
    sy += y[2 * i + 1];
  }
  sx /= static_cast<double>(n);
  sy /= static_cast<double>(n);
  const float fx = static_cast<float>(sx), fy = static_cast<float>(sy);
  for (int i = 0; i < n; ++i) {
    y[2 * i] -= fx;
    y[2 * i + 1] -= fy;
  }
}

inline float sgn0(float v) { return v == 0.0f ? 0.0f : (v < 0.0f ? -1.0f : 1.0f); }

void apply_update(float* y, float* upd, float* gains, const float* grad, int n, float lr, float mom,
                  float min_gain, float max_step, int threads) {
  const bool clip = std::isfinite(max_step) && max_step > 0.0f;
  const float max_sq = max_step * max_step;
  parallel_for(n, threads, [&](int b, int e, int) {
    for (int i = b; i < e; ++i) {
      float norm_sq = 0.0f;
      for (int d = 0; d < 2; ++d) {
        const int at = 2 * i + d;
        if (sgn0(upd[at]) != sgn0(grad[at])) {
          gains[at] += 0.2f;
        } else {
          gains[at] = gains[at] * 0.8f + min_gain;
        }
        if (gains[at] < min_gain) gains[at] = min_gain;
        upd[at] = mom * upd[at] - lr * gains[at] * grad[at];
        norm_sq += upd[at] * upd[at];
      }
      float s = 1.0f;
      if (clip && norm_sq > max_sq) s = max_step / std::sqrt(std::max(norm_sq, FLT_MIN));
      for (int d = 0; d < 2; ++d) {
        const int at = 2 * i + d;
        upd[at] *= s;
        y[at] += upd[at];
      }
    }
  });
}

// Exact KL(P || Q) over the CSR support (src/tsne_neighbors.cpp:958-983,
// 1258-1285); sum_q is rounded to fp32 as in the reference.
double kl_divergence(const CsrP& p, const float* y, int n, int threads, double* row_costs) {
  const int t_count = std::max(1, threads);
  std::vector<double> zpart(static_cast<std::size_t>(t_count), 0.0);
  auto worker = [&](int t) {
    double z = 0.0;
    for (int i = t; i < n - 1; i += t_count) {
      for (int j = i + 1; j < n; ++j) {
        float r2 = 0.0f;
        const float ddx = y[2 * i] - y[2 * j];
        r2 += ddx * ddx;
        const float ddy = y[2 * i + 1] - y[2 * j + 1];
        r2 += ddy * ddy;
        z += 2.0 / (1.0 + static_cast<double>(r2));
      }
    }
    zpart[static_cast<std::size_t>(t)] = z;
  };
  if (t_count == 1) {
    worker(0);
  } else {
    std::vector<std::thread> pool;
    for (int t = 1; t < t_count; ++t) pool.emplace_back(worker, t);
    worker(0);
    for (auto& th : pool) th.join();
  }
  const double sum_q = static_cast<double>(static_cast<float>(
      std::max(std::accumulate(zpart.begin(), zpart.end(), 0.0), static_cast<double>(FLT_MIN))));
  std::vector<double> part(static_cast<std::size_t>(t_count), 0.0);
  parallel_for(n, t_count, [&](int b, int e, int t) {
    double acc = 0.0;
    for (int i = b; i < e; ++i) {
      double row = 0.0;
      for (int at = p.row_ptr[i]; at < p.row_ptr[i + 1]; ++at) {
        const int j = p.col[static_cast<std::size_t>(at)];
        const double pij = static_cast<double>(p.val[static_cast<std::size_t>(at)]);
        float r2 = 0.0f;
        const float ddx = y[2 * i] - y[2 * j];
        r2 += ddx * ddx;
        const float ddy = y[2 * i + 1] - y[2 * j + 1];
        r2 += ddy * ddy;
        const double qij = (1.0 / (1.0 + static_cast<double>(r2))) / sum_q;
        row += pij * std::log((pij + 1e-9) / (qij + 1e-9));
      }
      if (row_costs != nullptr) row_costs[i] = row;
      acc += row;
    }
    part[static_cast<std::size_t>(t)] = acc;
  });
  return std::accumulate(part.begin(), part.end(), 0.0);
}

enum Repulsion { kGrid = 0, kExact = 1, kLagrange = 2 };

struct GradientConfig {
  int method = kGrid;
  int grid_size = 0;         // bilinear grid: 0 = reference policy
  int lagrange_order = 3;    // FIt-SNE: interpolation points per interval
  int min_intervals = 50;    // FIt-SNE: minimum intervals per axis
  float ints_per_unit = 1.0f;
};

void gradient(const CsrP& p, const float* y, int n, float ex, const GradientConfig& cfg, int threads,
              GridScratch& ws, float* grad) {
  if (cfg.method == kExact) {
    gradient_exact(p, y, n, ex, threads, grad);
  } else if (cfg.method == kLagrange) {
    gradient_lagrange(p, y, n, ex, cfg.lagrange_order, cfg.min_intervals, cfg.ints_per_unit, threads, grad,
                      nullptr);
  } else {
    gradient_grid<float>(p, y, n, ex, resolve_grid_size(n, cfg.grid_size), threads, ws, grad, nullptr);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI used by tests/ and bench.py (via ctypes).
// ---------------------------------------------------------------------------
extern "C" {

const char* tsne_oracle_last_error() { return g_error.c_str(); }

int tsne_oracle_policy_grid_size(int n) { return policy_grid_size(n); }

// Row search only; distances column-major n x k; p column-major n x k.
int tsne_oracle_conditional_p(const float* dist_cm, int n, int k, double perplexity, float* p_cm,
                              float* beta, int* steps) {
  std::vector<float> row(static_cast<std::size_t>(k)), pr(static_cast<std::size_t>(k));
  for (int i = 0; i < n; ++i) {
    for (int j = 0; j < k; ++j) row[static_cast<std::size_t>(j)] = dist_cm[static_cast<std::size_t>(j) * n + i];
    float b = 0.0f;
    const int s = row_search_fp32(row.data(), k, perplexity, pr.data(), &b);
    for (int j = 0; j < k; ++j) p_cm[static_cast<std::size_t>(j) * n + i] = pr[static_cast<std::size_t>(j)];
    if (beta != nullptr) beta[i] = b;
    if (steps != nullptr) steps[i] = s;
  }
  return 0;
}

void* tsne_oracle_build_p(const int* idx_cm, const float* dist_cm, int n, int k, double perplexity,
                          int threads) {
  g_error.clear();
  if (n < 2 || k < 1 || idx_cm == nullptr || dist_cm == nullptr) {
    g_error = "KNN input must have at least two rows and one neighbor column.";
    return nullptr;
  }
  auto* p = new CsrP();
  if (!build_symmetric_p(idx_cm, dist_cm, n, k, perplexity, threads, *p)) {
    delete p;
    return nullptr;
  }
  return p;
}

void* tsne_oracle_wrap_p(const int* row_ptr, const int* col, const float* val, int n) {
  auto* p = new CsrP();
  p->n = n;
  p->row_ptr.assign(row_ptr, row_ptr + n + 1);
  p->col.assign(col, col + row_ptr[n]);
  p->val.assign(val, val + row_ptr[n]);
  return p;
}

long long tsne_oracle_p_nnz(void* h) { return static_cast<CsrP*>(h)->row_ptr.back(); }

void tsne_oracle_p_copy(void* h, int* row_ptr, int* col, float* val) {
  const CsrP* p = static_cast<CsrP*>(h);
  std::copy(p->row_ptr.begin(), p->row_ptr.end(), row_ptr);
  std::copy(p->col.begin(), p->col.end(), col);
  std::copy(p->val.begin(), p->val.end(), val);
}

void tsne_oracle_p_free(void* h) { delete static_cast<CsrP*>(h); }

// method: 0 bilinear FFT grid (reference), 1 exact, 2 FIt-SNE Lagrange grid.
int tsne_oracle_gradient(void* h, const float* y, int n, float exaggeration, int method, int grid_size,
                         int lagrange_order, int min_intervals, int threads, float* grad) {
  g_error.clear();
  const CsrP& p = *static_cast<CsrP*>(h);
  if (p.n != n) {
    g_error = "P has a different number of rows";
    return 1;
  }
  GradientConfig cfg;
  cfg.method = method;
  cfg.grid_size = grid_size;
  cfg.lagrange_order = lagrange_order > 0 ? lagrange_order : 3;
  cfg.min_intervals = min_intervals > 0 ? min_intervals : 50;
  GridScratch ws;
  gradient(p, y, n, exaggeration, cfg, threads, ws, grad);
  return 0;
}

// The bilinear FFT-grid gradient of tsne_oracle_gradient (method 0) with
// every step in fp64 (extension): the same algorithm, spread, recurrence
// twiddles and read-back, with fp64 arithmetic; y is the fp32 layout.
int tsne_oracle_gradient_grid_f64(void* h, const float* y, int n, float exaggeration, int grid_size, int threads,
                                  double* grad) {
  g_error.clear();
  const CsrP& p = *static_cast<CsrP*>(h);
  if (p.n != n) {
    g_error = "P has a different number of rows";
    return 1;
  }
  GridScratchT<double> ws;
  gradient_grid<double>(p, y, n, static_cast<double>(exaggeration), resolve_grid_size(n, grid_size), threads, ws,
                        grad, nullptr);
  return 0;
}

// FIt-SNE interpolation-grid gradient (extension) with its geometry
// (boxes, nodes, lo, box width) and normaliser Z; direct != 0 convolves by
// the O(nodes^4) node sum instead of the FFT.
int tsne_oracle_lagrange_gradient(void* h, const float* y, int n, float exaggeration, int order, int min_intervals,
                                  float ints_per_unit, int direct, int threads, float* grad, double* geometry,
                                  double* z) {
  g_error.clear();
  const CsrP& p = *static_cast<CsrP*>(h);
  if (p.n != n || order < 1 || min_intervals < 1 || !(ints_per_unit > 0.0f)) {
    g_error = "invalid Lagrange gradient arguments";
    return 1;
  }
  LagrangeGeometry g;
  gradient_lagrange(p, y, n, exaggeration, order, min_intervals, ints_per_unit, threads, grad, &g, direct != 0, z);
  if (geometry != nullptr) {
    geometry[0] = g.boxes;
    geometry[1] = g.nodes;
    geometry[2] = g.lo;
    geometry[3] = g.box_w;
  }
  return 0;
}

// Lagrange basis values of the given order at u (extension; for the pins).
void tsne_oracle_lagrange_weights(double u, int order, double* w) { lagrange_weights(u, order, w); }

// Grid geometry (lower_x, lower_y, spacing, 1/spacing) and the four
// convolved grids (q, q2, xq2, yq2; each g*g row-major) for one y.
int tsne_oracle_grid_fields(void* h, const float* y, int n, int grid_size, int threads, float* geometry,
                            float* fields) {
  const CsrP& p = *static_cast<CsrP*>(h);
  const int g = resolve_grid_size(n, grid_size);
  GridScratch ws;
  std::vector<float> grad(2 * static_cast<std::size_t>(n));
  gradient_grid<float>(p, y, n, 1.0f, g, threads, ws, grad.data(), geometry);
  const std::size_t gg = static_cast<std::size_t>(g) * g;
  if (fields != nullptr) {
    std::copy(ws.q.begin(), ws.q.end(), fields);
    std::copy(ws.q2.begin(), ws.q2.end(), fields + gg);
    std::copy(ws.xq2.begin(), ws.xq2.end(), fields + 2 * gg);
    std::copy(ws.yq2.begin(), ws.yq2.end(), fields + 3 * gg);
  }
  return g;
}

void tsne_oracle_update(float* y, float* update, float* gains, const float* grad, int n, float lr,
                        float momentum, float min_gain, float max_step_norm, int threads) {
  apply_update(y, update, gains, grad, n, lr, momentum, min_gain, max_step_norm, threads);
}

void tsne_oracle_zero_mean(float* y, int n) { zero_mean(y, n); }

double tsne_oracle_kl(void* h, const float* y, int n, int threads, double* row_costs) {
  return kl_divergence(*static_cast<CsrP*>(h), y, n, threads, row_costs);
}

// Two-phase optimiser (src/tsne_neighbors.cpp:1702-1814): y holds the
// initialisation on entry (centred here, as the reference does) and the final
// layout on exit.  record_costs != 0 stores the KL every 50 iterations and at
// the last one into costs/cost_iters (capacity ceil(total/50)).  The KL-based
// early stop is omitted: the package's R layer always disables it
// (R/tsne_affinity_dispatch.R:311, auto_kld_stop is FALSE from
// src/tsne_neighbors.cpp:1596).
int tsne_oracle_optimize(void* h, float* y, int n, int early_iter, int n_iter, double early_ex,
                         double ex, double learning_rate, int learning_rate_auto, double m0, double m1,
                         double min_gain, double max_step_norm, int method, int grid_size, int threads,
                         int record_costs, double* costs, int* cost_iters) {
  g_error.clear();
  const CsrP& p = *static_cast<CsrP*>(h);
  if (p.n != n) {
    g_error = "P has a different number of rows";
    return -1;
  }
  GradientConfig cfg;
  cfg.method = method;
  cfg.grid_size = grid_size;
  GridScratch ws;
  zero_mean(y, n);
  std::vector<float> grad(2 * static_cast<std::size_t>(n), 0.0f);
  std::vector<float> upd(2 * static_cast<std::size_t>(n), 0.0f);
  std::vector<float> gains(2 * static_cast<std::size_t>(n), 1.0f);
  const int total = early_iter + n_iter;
  int recorded = 0;
  int done = 0;
  auto phase = [&](int iters, double phase_ex, double mom) {
    const float lr = static_cast<float>(learning_rate_auto ? static_cast<double>(n) / std::max(phase_ex, DBL_MIN)
                                                           : learning_rate);
    const float exf = static_cast<float>(phase_ex);
    const float mf = static_cast<float>(mom);
    const float mg = static_cast<float>(min_gain);
    const float ms = std::isfinite(max_step_norm) ? static_cast<float>(max_step_norm)
                                                  : std::numeric_limits<float>::quiet_NaN();
    for (int it = 0; it < iters; ++it) {
      gradient(p, y, n, exf, cfg, threads, ws, grad.data());
      apply_update(y, upd.data(), gains.data(), grad.data(), n, lr, mf, mg, ms, threads);
      zero_mean(y, n);
      ++done;
      if (record_costs && (done % 50 == 0 || done == total)) {
        costs[recorded] = kl_divergence(p, y, n, threads, nullptr);
        cost_iters[recorded] = done;
        ++recorded;
      }
    }
  };
  phase(early_iter, early_ex, m0);
  phase(n_iter, ex, m1);
  return recorded;
}

// Random initialisation used when no Y_init is supplied
// (src/tsne_neighbors.cpp:1693-1700): mt19937(seed) feeding
// normal_distribution<float>(0, 1e-4), row-major interleaved.
void tsne_oracle_random_init(float* y, int n, unsigned int seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> normal(0.0f, 1.0e-4f);
  for (std::size_t i = 0; i < 2 * static_cast<std::size_t>(n); ++i) y[i] = normal(rng);
}

}  // extern "C"
