// Fixed-reference t-SNE transform on gfx950: new query points are placed
// against a frozen reference layout, each query independently.
//
// Semantics follow the reference CPU path transform_tsne_cpp
// (src/tsne_neighbors.cpp:1859-2109 of tkcaccia/fastEmbedR), two-dimensional
// layouts only, in fp64 with the reference's operation order and no fused
// multiply-add:
//   * conditional probabilities per query by bisection on beta
//     (compute_row_probabilities_flat, :437-486);
//   * median / weighted initialisation from the neighbours' reference
//     positions (initialize_tsne_transform, :1304-1372); the random
//     initialisation (per-query mt19937 + normal_distribution<double>) is
//     drawn on the host with the same standard-library generators;
//   * per iteration and query: repulsion over every reference point (exact)
//     or over n_negatives reference points drawn with xorshift32 /
//     multiply-shift from a per-query, per-iteration hashed state, normalised
//     by the query's own sum of q; attraction exaggeration * p * q * d
//     (compute_tsne_transform_gradient_2d_flat, :1472-1568); then the
//     gradient-norm clip, gains, momentum and step-norm clip (:2040-2075).
//
// One thread owns one query and walks its samples in the reference's order,
// so every sum is formed exactly as the CPU forms it: the two sampling passes
// regenerate the same indices instead of storing them.  The reference layout
// (16 bytes per point, 1.1 MB at 70K points) stays in L2.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "fastembedr_hip.h"
#include "tsne_device.h"

namespace fehip {
namespace {

constexpr int kQueryThreads = 256;

__host__ __device__ inline std::uint32_t hash32(std::uint32_t v) {  // mix_uint32 (:56-63)
  v ^= v >> 16u;
  v *= 0x7feb352du;
  v ^= v >> 15u;
  v *= 0x846ca68bu;
  v ^= v >> 16u;
  return v == 0u ? 0x6d2b79f5u : v;
}

__device__ inline int draw_index(std::uint32_t& s, int n) {  // xorshift32 + multiply-shift (:65-77)
  s ^= s << 13u;
  s ^= s >> 17u;
  s ^= s << 5u;
  return static_cast<int>((static_cast<std::uint64_t>(s) * static_cast<std::uint64_t>(n)) >> 32u);
}

__device__ inline double sign0(double v) { return v == 0.0 ? 0.0 : (v < 0.0 ? -1.0 : 1.0); }

__global__ __launch_bounds__(kQueryThreads) void k_transform_p(const double* __restrict__ dist_cm, int nq, int k,
                                                               double perplexity, double* __restrict__ p_cm) {
#pragma clang fp contract(off)
  const int i = static_cast<int>(blockIdx.x) * kQueryThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  const double target = log(perplexity);
  double beta = 1.0, lo = -DBL_MAX, hi = DBL_MAX;
  double used = beta, sum = DBL_MIN;
  bool done = false;
  for (int it = 0; !done && it < 200; ++it) {
    used = beta;
    sum = DBL_MIN;
    double h = 0.0;
    // The reference stores p_j in one pass and forms the entropy sum in a
    // second; both sums run in j order, as here.
    for (int j = 0; j < k; ++j) {
      const double d = dist_cm[static_cast<std::size_t>(j) * nq + i];
      sum += exp(-beta * (d * d));
    }
    for (int j = 0; j < k; ++j) {
      const double d = dist_cm[static_cast<std::size_t>(j) * nq + i];
      h += beta * (d * d * exp(-beta * (d * d)));
    }
    h = h / sum + log(sum);
    const double diff = h - target;
    if (fabs(diff) < 1e-5) {
      done = true;
    } else if (diff > 0.0) {
      lo = beta;
      beta = (hi == DBL_MAX || hi == -DBL_MAX) ? beta * 2.0 : (beta + hi) / 2.0;
    } else {
      hi = beta;
      beta = (lo == -DBL_MAX || lo == DBL_MAX) ? beta / 2.0 : (beta + lo) / 2.0;
    }
  }
  const double inv = 1.0 / sum;
  for (int j = 0; j < k; ++j) {
    const double d = dist_cm[static_cast<std::size_t>(j) * nq + i];
    p_cm[static_cast<std::size_t>(j) * nq + i] = exp(-used * (d * d)) * inv;
  }
}

// Value at sorted position `rank` of the k neighbour coordinates (component c).
__device__ double coordinate_at_rank(const double2* __restrict__ ref, const int* __restrict__ idx_cm, int nq, int k,
                                     int offset, int i, int c, int rank) {
  for (int a = 0; a < k; ++a) {
    const double2 ra = ref[idx_cm[static_cast<std::size_t>(a) * nq + i] - offset];
    const double va = c == 0 ? ra.x : ra.y;
    int less = 0, leq = 0;
    for (int b = 0; b < k; ++b) {
      const double2 rb = ref[idx_cm[static_cast<std::size_t>(b) * nq + i] - offset];
      const double vb = c == 0 ? rb.x : rb.y;
      less += vb < va ? 1 : 0;
      leq += vb <= va ? 1 : 0;
    }
    if (less <= rank && rank < leq) return va;
  }
  return 0.0;  // not reached for finite coordinates
}

__global__ __launch_bounds__(kQueryThreads) void k_transform_init(const double2* __restrict__ ref,
                                                                  const int* __restrict__ idx_cm,
                                                                  const double* __restrict__ dist_cm, int nq, int k,
                                                                  int offset, int weighted, double2* __restrict__ y) {
#pragma clang fp contract(off)
  const int i = static_cast<int>(blockIdx.x) * kQueryThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  double out[2];
  for (int c = 0; c < 2; ++c) {
    if (weighted) {
      double num = 0.0, den = DBL_MIN;
      for (int j = 0; j < k; ++j) {
        const std::size_t e = static_cast<std::size_t>(j) * nq + i;
        const double2 r = ref[idx_cm[e] - offset];
        const double w = 1.0 / (fmax(0.0, dist_cm[e]) + 1e-6);
        num += w * (c == 0 ? r.x : r.y);
        den += w;
      }
      out[c] = num / den;
    } else {
      const int mid = k / 2;
      double m = coordinate_at_rank(ref, idx_cm, nq, k, offset, i, c, mid);
      if ((k & 1) == 0) m = 0.5 * (m + coordinate_at_rank(ref, idx_cm, nq, k, offset, i, c, mid - 1));
      out[c] = m;
    }
  }
  y[i] = make_double2(out[0], out[1]);
}

// Repulsion term of one query: sum over the samples of -(q^2 / sum_q) d.
template <bool EXACT>
__device__ inline double2 repulsion(const double2* __restrict__ ref, int n_ref, int samples, std::uint32_t state,
                                    double yx, double yy) {
#pragma clang fp contract(off)
  double sum_q = DBL_MIN;
  std::uint32_t s = state;
#pragma unroll 4
  for (int m = 0; m < samples; ++m) {
    const int r = EXACT ? m : draw_index(s, n_ref);
    const double2 p = ref[r];
    const double dx = yx - p.x;
    const double dy = yy - p.y;
    sum_q += 1.0 / (1.0 + dx * dx + dy * dy);
  }
  const double inv = 1.0 / sum_q;
  double gx = 0.0, gy = 0.0;
  s = state;
#pragma unroll 4
  for (int m = 0; m < samples; ++m) {
    const int r = EXACT ? m : draw_index(s, n_ref);
    const double2 p = ref[r];
    const double dx = yx - p.x;
    const double dy = yy - p.y;
    const double q = 1.0 / (1.0 + dx * dx + dy * dy);
    const double c = -(q * q) * inv;
    gx += c * dx;
    gy += c * dy;
  }
  return make_double2(gx, gy);
}

struct StepParams {
  double exaggeration, momentum, learning_rate, max_grad, max_step;
  int samples;      // n_reference (exact) or n_negatives (sampled)
  int iter_seed;
};

// One iteration for every query; GRAD_ONLY writes the gradient and leaves
// the state alone.
template <bool EXACT, bool GRAD_ONLY>
__global__ __launch_bounds__(kQueryThreads) void k_transform_step(const double2* __restrict__ ref, int n_ref,
                                                                  const int* __restrict__ idx_cm,
                                                                  const double* __restrict__ p_cm, int nq, int k,
                                                                  int offset, StepParams sp, double2* __restrict__ y,
                                                                  double2* __restrict__ upd,
                                                                  double2* __restrict__ gains,
                                                                  double2* __restrict__ grad_out) {
#pragma clang fp contract(off)
  const int i = static_cast<int>(blockIdx.x) * kQueryThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  const double2 yi = y[i];
  const std::uint32_t state =
      hash32(static_cast<std::uint32_t>(sp.iter_seed) ^ (static_cast<std::uint32_t>(i + 1) * 0x9e3779b9u));
  const double2 rep = repulsion<EXACT>(ref, n_ref, sp.samples, state, yi.x, yi.y);
  double gx = rep.x, gy = rep.y;
  for (int j = 0; j < k; ++j) {
    const std::size_t e = static_cast<std::size_t>(j) * nq + i;
    const double2 p = ref[idx_cm[e] - offset];
    const double dx = yi.x - p.x;
    const double dy = yi.y - p.y;
    const double q = 1.0 / (1.0 + dx * dx + dy * dy);
    const double c = sp.exaggeration * p_cm[e] * q;
    gx += c * dx;
    gy += c * dy;
  }
  if (GRAD_ONLY) {
    grad_out[i] = make_double2(gx, gy);
    return;
  }
  const double gn = gx * gx + gy * gy;
  if (gn > sp.max_grad * sp.max_grad) {
    const double s = sp.max_grad / (sqrt(gn) + 1e-12);
    gx *= s;
    gy *= s;
  }
  double2 u = upd[i];
  double2 w = gains[i];
  w.x = sign0(u.x) != sign0(gx) ? w.x + 0.2 : w.x * 0.8 + 0.01;
  if (w.x < 0.01) w.x = 0.01;
  u.x = sp.momentum * u.x - sp.learning_rate * w.x * gx;
  w.y = sign0(u.y) != sign0(gy) ? w.y + 0.2 : w.y * 0.8 + 0.01;
  if (w.y < 0.01) w.y = 0.01;
  u.y = sp.momentum * u.y - sp.learning_rate * w.y * gy;
  const double sn = u.x * u.x + u.y * u.y;
  if (sn > sp.max_step * sp.max_step) {
    const double s = sp.max_step / (sqrt(sn) + 1e-12);
    u.x *= s;
    u.y *= s;
  }
  upd[i] = u;
  gains[i] = w;
  y[i] = make_double2(yi.x + u.x, yi.y + u.y);
}

__global__ __launch_bounds__(kQueryThreads) void k_transform_reset(double2* __restrict__ upd,
                                                                   double2* __restrict__ gains, int nq) {
  const int i = static_cast<int>(blockIdx.x) * kQueryThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  upd[i] = make_double2(0.0, 0.0);
  gains[i] = make_double2(1.0, 1.0);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
bool ok(hipError_t e, const char* where) {
  if (e == hipSuccess) return true;
  set_last_error(std::string(where) + ": " + hipGetErrorString(e));
  return false;
}

int query_blocks(int nq) { return (nq + kQueryThreads - 1) / kQueryThreads; }

// (seed or 5489) + 65537 (iter + 1) with wrap-around (:2009).
int iteration_seed(int seed, int iter) {
  const std::uint32_t base = seed == INT_MIN ? 5489u : static_cast<std::uint32_t>(seed);
  return static_cast<int>(base + 65537u * static_cast<std::uint32_t>(iter + 1));
}

// 1 when every index is in [1, n_ref] (:1290-1302), else 0.
int reference_offset(const int* idx_cm, std::size_t count, int n_ref) {
  int lo = INT_MAX, hi = INT_MIN;
  for (std::size_t c = 0; c < count; ++c) {
    lo = std::min(lo, idx_cm[c]);
    hi = std::max(hi, idx_cm[c]);
  }
  return (lo >= 1 && hi <= n_ref) ? 1 : 0;
}

// Device buffers of one call, carved from a single allocation.
struct TransformBuffers {
  void* base = nullptr;
  double2* ref = nullptr;
  int* idx = nullptr;
  double* dist = nullptr;
  double* p = nullptr;
  double2* y = nullptr;
  double2* upd = nullptr;
  double2* gains = nullptr;
  double2* grad = nullptr;
  hipStream_t stream = nullptr;
  ~TransformBuffers() {
    if (stream != nullptr) (void)hipStreamSynchronize(stream);
    if (base != nullptr) (void)hipFree(base);
    if (stream != nullptr) (void)hipStreamDestroy(stream);
  }
  bool init(int n_ref, int nq, int k) {
    const auto up = [](std::size_t b) { return (b + 255) & ~static_cast<std::size_t>(255); };
    const std::size_t nk = static_cast<std::size_t>(nq) * k;
    const std::size_t sizes[] = {up(sizeof(double2) * n_ref), up(sizeof(int) * nk), up(sizeof(double) * nk),
                                 up(sizeof(double) * nk), 4 * up(sizeof(double2) * nq)};
    std::size_t total = 0;
    for (std::size_t s : sizes) total += s;
    if (!ok(hipStreamCreate(&stream), "hipStreamCreate(transform)") ||
        !ok(hipMalloc(&base, total), "hipMalloc(transform buffers)")) {
      return false;
    }
    char* c = static_cast<char*>(base);
    ref = reinterpret_cast<double2*>(c);
    c += sizes[0];
    idx = reinterpret_cast<int*>(c);
    c += sizes[1];
    dist = reinterpret_cast<double*>(c);
    c += sizes[2];
    p = reinterpret_cast<double*>(c);
    c += sizes[3];
    const std::size_t yb = up(sizeof(double2) * nq);
    y = reinterpret_cast<double2*>(c);
    upd = reinterpret_cast<double2*>(c + yb);
    gains = reinterpret_cast<double2*>(c + 2 * yb);
    grad = reinterpret_cast<double2*>(c + 3 * yb);
    return true;
  }
};

std::vector<double> rows_of(const double* cm, int n) {  // n x 2 column-major -> interleaved
  std::vector<double> r(2 * static_cast<std::size_t>(n));
  for (int i = 0; i < n; ++i) {
    r[2 * static_cast<std::size_t>(i)] = cm[i];
    r[2 * static_cast<std::size_t>(i) + 1] = cm[static_cast<std::size_t>(n) + i];
  }
  return r;
}

bool upload(TransformBuffers& b, const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq,
            int k) {
  const std::vector<double> ref = rows_of(ref_cm, n_ref);
  const std::size_t nk = static_cast<std::size_t>(nq) * k;
  // Synchronous copies: the staging vector dies with this function.
  return ok(hipMemcpy(b.ref, ref.data(), ref.size() * sizeof(double), hipMemcpyHostToDevice), "reference upload") &&
         ok(hipMemcpy(b.idx, idx_cm, nk * sizeof(int), hipMemcpyHostToDevice), "index upload") &&
         ok(hipMemcpy(b.dist, dist_cm, nk * sizeof(double), hipMemcpyHostToDevice), "distance upload");
}

template <bool GRAD_ONLY>
hipError_t launch_step(bool exact, const TransformBuffers& b, int n_ref, int nq, int k, int offset,
                       const StepParams& sp) {
  const int blocks = query_blocks(nq);
  if (exact) {
    k_transform_step<true, GRAD_ONLY><<<blocks, kQueryThreads, 0, b.stream>>>(
        b.ref, n_ref, b.idx, b.p, nq, k, offset, sp, b.y, b.upd, b.gains, b.grad);
  } else {
    k_transform_step<false, GRAD_ONLY><<<blocks, kQueryThreads, 0, b.stream>>>(
        b.ref, n_ref, b.idx, b.p, nq, k, offset, sp, b.y, b.upd, b.gains, b.grad);
  }
  return hipGetLastError();
}

// The reference's argument checks (:1880-1921); returns false with the message set.
bool check_inputs(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq, int k,
                  double perplexity, int offset) {
  if (ref_cm == nullptr || idx_cm == nullptr || dist_cm == nullptr) {
    set_last_error("reference_layout, indices and distances must not be NULL.");
    return false;
  }
  if (n_ref < 1) {
    set_last_error("`reference_layout` must be a non-empty matrix.");
    return false;
  }
  if (nq < 1 || k < 1) {
    set_last_error("KNN input must have at least one query row and one neighbor column.");
    return false;
  }
  if (!(perplexity > 0.0)) {
    set_last_error("`perplexity` must be positive.");
    return false;
  }
  const std::size_t nk = static_cast<std::size_t>(nq) * k;
  for (std::size_t c = 0; c < nk; ++c) {
    const int r = idx_cm[c] - offset;
    if (r < 0 || r >= n_ref) {
      set_last_error("KNN indices are out of range for `reference_layout`.");
      return false;
    }
    if (!std::isfinite(dist_cm[c]) || dist_cm[c] < 0.0) {
      set_last_error("KNN distances must be finite and non-negative.");
      return false;
    }
  }
  for (int i = 0; i < 2 * n_ref; ++i) {
    if (!std::isfinite(ref_cm[i])) {
      set_last_error("`reference_layout` must be finite.");
      return false;
    }
  }
  return true;
}

// Scalar arguments of a transform run (:1880-1929); on success
// the clip norms, the negative count and the repulsion mode are resolved in
// place.
struct RunArgs {
  int n_reference, n_iter, early_iter;
  double learning_rate, early_exaggeration, exaggeration, initial_momentum, final_momentum, max_grad, max_step;
  int n_negatives, exact_threshold, initialization;
  bool exact = false;
};

bool check_run_args(RunArgs& a) {
  if (a.n_iter < 0 || a.early_iter < 0) {
    set_last_error("iteration counts must be non-negative.");
    return false;
  }
  if (a.n_iter + a.early_iter < 1) {
    set_last_error("at least one transform iteration is required.");
    return false;
  }
  if (!(a.learning_rate > 0.0)) {
    set_last_error("`learning_rate` must be positive.");
    return false;
  }
  if (!(a.early_exaggeration > 0.0) || !(a.exaggeration > 0.0)) {
    set_last_error("exaggeration values must be positive.");
    return false;
  }
  if (a.initial_momentum < 0.0 || a.final_momentum < 0.0) {
    set_last_error("momentum values must be non-negative.");
    return false;
  }
  if (a.n_negatives < 1) {
    set_last_error("`n_negatives` must be positive.");
    return false;
  }
  if (a.initialization < 0 || a.initialization > 2) {
    set_last_error("`initialization` must be 'median', 'weighted', or 'random'.");
    return false;
  }
  if (a.exact_threshold < 1) a.exact_threshold = 1;
  if (!(a.max_grad > 0.0) || !std::isfinite(a.max_grad)) a.max_grad = DBL_MAX;
  if (!(a.max_step > 0.0) || !std::isfinite(a.max_step)) a.max_step = DBL_MAX;
  if (a.n_negatives > a.n_reference) a.n_negatives = a.n_reference;
  a.exact = a.n_reference <= a.exact_threshold || a.n_negatives >= a.n_reference;
  return true;
}

}  // namespace
}  // namespace fehip

extern "C" {

int fastembedr_hip_transform_tsne(const double* reference_layout, int n_reference, const int* indices,
                                  const double* distances, int n_query, int k, const double* y_init,
                                  int initialization, double perplexity, int n_iter, int early_exaggeration_iter,
                                  double learning_rate, double early_exaggeration, double exaggeration,
                                  double initial_momentum, double final_momentum, double max_grad_norm,
                                  double max_step_norm, int n_negatives, int exact_repulsion_threshold, int seed,
                                  double* out, int* repulsion_exact) {
  using namespace fehip;
  clear_last_error();
  if (out == nullptr || n_reference < 1 || n_query < 1 || k < 1 || reference_layout == nullptr ||
      indices == nullptr || distances == nullptr) {
    set_last_error("invalid transform arguments (NULL pointer or empty input).");
    return 1;
  }
  const int offset = reference_offset(indices, static_cast<std::size_t>(n_query) * k, n_reference);
  if (!check_inputs(reference_layout, n_reference, indices, distances, n_query, k, perplexity, offset)) return 1;
  RunArgs ra{n_reference, n_iter, early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
             initial_momentum, final_momentum, max_grad_norm, max_step_norm, n_negatives, exact_repulsion_threshold,
             initialization};
  if (!check_run_args(ra)) return 1;
  max_grad_norm = ra.max_grad;
  max_step_norm = ra.max_step;
  n_negatives = ra.n_negatives;
  const bool exact = ra.exact;

  TransformBuffers b;
  if (!b.init(n_reference, n_query, k) ||
      !upload(b, reference_layout, n_reference, indices, distances, n_query, k)) {
    return 1;
  }
  const int blocks = query_blocks(n_query);
  k_transform_p<<<blocks, kQueryThreads, 0, b.stream>>>(b.dist, n_query, k, perplexity, b.p);
  if (!ok(hipGetLastError(), "transform P launch")) return 1;
  std::vector<double> y_host;
  if (y_init != nullptr) {
    y_host = rows_of(y_init, n_query);
  } else if (initialization == 2) {
    // Per-query mt19937 seeded through mix_uint32, then two draws of
    // normal_distribution<double>(0, 1e-4) (:1317-1335).
    y_host.resize(2 * static_cast<std::size_t>(n_query));
    const unsigned int s = seed == INT_MIN ? 5489u : static_cast<unsigned int>(seed);
    for (int i = 0; i < n_query; ++i) {
      std::normal_distribution<double> normal(0.0, 1.0e-4);
      std::mt19937 rng(hash32(s ^ (static_cast<std::uint32_t>(i + 1) * 0x9e3779b9u)));
      y_host[2 * static_cast<std::size_t>(i)] = normal(rng);
      y_host[2 * static_cast<std::size_t>(i) + 1] = normal(rng);
    }
  }
  if (!y_host.empty()) {
    if (!ok(hipMemcpyAsync(b.y, y_host.data(), y_host.size() * sizeof(double), hipMemcpyHostToDevice, b.stream),
            "initial layout upload")) {
      return 1;
    }
  } else {
    k_transform_init<<<blocks, kQueryThreads, 0, b.stream>>>(b.ref, b.idx, b.dist, n_query, k, offset,
                                                            initialization == 1 ? 1 : 0, b.y);
    if (!ok(hipGetLastError(), "transform init launch")) return 1;
  }
  k_transform_reset<<<blocks, kQueryThreads, 0, b.stream>>>(b.upd, b.gains, n_query);
  if (!ok(hipGetLastError(), "transform reset launch")) return 1;
  const int total = early_exaggeration_iter + n_iter;
  for (int it = 0; it < total; ++it) {
    const bool early = it < early_exaggeration_iter;
    StepParams sp{early ? early_exaggeration : exaggeration, early ? initial_momentum : final_momentum,
                  learning_rate, max_grad_norm, max_step_norm, exact ? n_reference : n_negatives,
                  iteration_seed(seed, it)};
    if (!ok(launch_step<false>(exact, b, n_reference, n_query, k, offset, sp), "transform step launch")) return 1;
  }
  std::vector<double> y(2 * static_cast<std::size_t>(n_query));
  if (!ok(hipMemcpyAsync(y.data(), b.y, y.size() * sizeof(double), hipMemcpyDeviceToHost, b.stream),
          "layout download") ||
      !ok(hipStreamSynchronize(b.stream), "transform sync")) {
    return 1;
  }
  for (int i = 0; i < n_query; ++i) {
    out[i] = y[2 * static_cast<std::size_t>(i)];
    out[static_cast<std::size_t>(n_query) + i] = y[2 * static_cast<std::size_t>(i) + 1];
  }
  if (repulsion_exact != nullptr) *repulsion_exact = exact ? 1 : 0;
  return 0;
}

int fastembedr_hip_transform_probe(const double* reference_layout, int n_reference, const int* indices,
                                   const double* distances, int n_query, int k, double perplexity,
                                   const double* y, double exaggeration, int n_negatives,
                                   int exact_repulsion_threshold, int iter_seed, int initialization,
                                   double* p_out, double* grad_out, double* init_out) {
  using namespace fehip;
  clear_last_error();
  if (n_reference < 1 || n_query < 1 || k < 1 || reference_layout == nullptr || indices == nullptr ||
      distances == nullptr) {
    set_last_error("invalid transform arguments (NULL pointer or empty input).");
    return 1;
  }
  const int offset = reference_offset(indices, static_cast<std::size_t>(n_query) * k, n_reference);
  if (!check_inputs(reference_layout, n_reference, indices, distances, n_query, k, perplexity, offset)) return 1;
  if (n_negatives < 1 || initialization < 0 || initialization > 1) {
    set_last_error("invalid transform probe arguments.");
    return 1;
  }
  if (exact_repulsion_threshold < 1) exact_repulsion_threshold = 1;
  if (n_negatives > n_reference) n_negatives = n_reference;
  const bool exact = n_reference <= exact_repulsion_threshold || n_negatives >= n_reference;
  TransformBuffers b;
  if (!b.init(n_reference, n_query, k) ||
      !upload(b, reference_layout, n_reference, indices, distances, n_query, k)) {
    return 1;
  }
  const int blocks = query_blocks(n_query);
  const std::size_t nk = static_cast<std::size_t>(n_query) * k;
  k_transform_p<<<blocks, kQueryThreads, 0, b.stream>>>(b.dist, n_query, k, perplexity, b.p);
  if (!ok(hipGetLastError(), "transform P launch")) return 1;
  std::vector<double> host(std::max(nk, 2 * static_cast<std::size_t>(n_query)));
  if (init_out != nullptr) {
    k_transform_init<<<blocks, kQueryThreads, 0, b.stream>>>(b.ref, b.idx, b.dist, n_query, k, offset,
                                                            initialization, b.y);
    if (!ok(hipGetLastError(), "transform init launch") ||
        !ok(hipMemcpyAsync(host.data(), b.y, 2 * static_cast<std::size_t>(n_query) * sizeof(double),
                           hipMemcpyDeviceToHost, b.stream),
            "init download") ||
        !ok(hipStreamSynchronize(b.stream), "transform sync")) {
      return 1;
    }
    std::copy(host.begin(), host.begin() + 2 * static_cast<std::size_t>(n_query), init_out);
  }
  if (p_out != nullptr) {  // p_out: n_query x k row-major, as the reference stores it
    if (!ok(hipMemcpyAsync(host.data(), b.p, nk * sizeof(double), hipMemcpyDeviceToHost, b.stream), "P download") ||
        !ok(hipStreamSynchronize(b.stream), "transform sync")) {
      return 1;
    }
    for (int i = 0; i < n_query; ++i)
      for (int j = 0; j < k; ++j)
        p_out[static_cast<std::size_t>(i) * k + j] = host[static_cast<std::size_t>(j) * n_query + i];
  }
  if (grad_out != nullptr && y != nullptr) {  // y, grad_out: n_query x 2 row-major
    StepParams sp{exaggeration, 0.0, 0.0, 0.0, 0.0, exact ? n_reference : n_negatives, iter_seed};
    if (!ok(hipMemcpyAsync(b.y, y, 2 * static_cast<std::size_t>(n_query) * sizeof(double), hipMemcpyHostToDevice,
                           b.stream),
            "state upload") ||
        !ok(launch_step<true>(exact, b, n_reference, n_query, k, offset, sp), "transform gradient launch") ||
        !ok(hipMemcpyAsync(grad_out, b.grad, 2 * static_cast<std::size_t>(n_query) * sizeof(double),
                           hipMemcpyDeviceToHost, b.stream),
            "gradient download") ||
        !ok(hipStreamSynchronize(b.stream), "transform sync")) {
      return 1;
    }
  }
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free transform (fastembedr_hip_transform_tsne_noalloc)
//
// The same kernels and operation order as fastembedr_hip_transform_tsne, with
// the caller's arrays in device memory and the per-call work buffers in one
// static device array instead of a hipMalloc:
//   [0, 256)            NaHeader: validation flags and the index range
//   reference           n_reference double2 (the layout, interleaved)
//   p                   n_query * k fp64 conditional probabilities
//   y, update, gains    n_query double2 each
// Each GPU holds its own copy of the array for the life of the process; its
// device address is looked up once per device (hipGetSymbolAddress) and only
// that address is handed to kernels.  Every call on one GPU uses the same
// array, so calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
namespace fehip {
namespace {

constexpr int kNaMaxReference = 1 << 18;
constexpr int kNaMaxQuery = 1 << 17;
constexpr long long kNaMaxEntries = 1LL << 22;
constexpr std::size_t kNaReferenceOffset = 256;
constexpr std::size_t kNaPOffset = kNaReferenceOffset + sizeof(double2) * kNaMaxReference;
constexpr std::size_t kNaStateOffset = kNaPOffset + sizeof(double) * static_cast<std::size_t>(kNaMaxEntries);
constexpr std::size_t kNaStateStride = sizeof(double2) * kNaMaxQuery;
constexpr std::size_t kNaScratchBytes = kNaStateOffset + 3 * kNaStateStride;
constexpr int kNaMaxDevices = 64;

struct NaHeader {
  unsigned int flags;  // kNaBadDistance | kNaBadReference
  int idx_min;
  int idx_max;
  int pad;
};
static_assert(sizeof(NaHeader) <= kNaReferenceOffset, "the header fits its slot");
constexpr unsigned int kNaBadDistance = 1u;
constexpr unsigned int kNaBadReference = 2u;

}  // namespace
}  // namespace fehip

static __device__ __align__(256) unsigned char transform_scratch[fehip::kNaScratchBytes];

namespace fehip {
namespace {

__global__ void k_na_clear(NaHeader* h) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    h->flags = 0u;
    h->idx_min = INT_MAX;
    h->idx_max = INT_MIN;
  }
}

// Index range and distance checks of check_inputs, as a reduction: the host
// derives the index offset and the range error from the smallest and largest
// index.
__global__ __launch_bounds__(256) void k_na_check_knn(const int* __restrict__ idx_cm,
                                                      const double* __restrict__ dist_cm, long long count,
                                                      NaHeader* h) {
  int lo = INT_MAX, hi = INT_MIN;
  unsigned int bad = 0u;
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  for (long long c = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; c < count; c += stride) {
    const int v = idx_cm[c];
    lo = v < lo ? v : lo;
    hi = v > hi ? v : hi;
    const double d = dist_cm[c];
    if (!isfinite(d) || d < 0.0) bad = 1u;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const int olo = __shfl_xor(lo, off);
    const int ohi = __shfl_xor(hi, off);
    lo = olo < lo ? olo : lo;
    hi = ohi > hi ? ohi : hi;
    bad |= static_cast<unsigned int>(__shfl_xor(static_cast<int>(bad), off));
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMin(&h->idx_min, lo);
    atomicMax(&h->idx_max, hi);
    if (bad != 0u) atomicOr(&h->flags, kNaBadDistance);
  }
}

// n x 2 column-major reference layout -> interleaved, with the finiteness check.
__global__ __launch_bounds__(256) void k_na_load_reference(const double* __restrict__ ref_cm, int n_ref,
                                                           double2* __restrict__ ref, NaHeader* h) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i >= n_ref) return;
  const double x = ref_cm[i];
  const double y = ref_cm[static_cast<std::size_t>(n_ref) + i];
  if (!isfinite(x) || !isfinite(y)) atomicOr(&h->flags, kNaBadReference);
  ref[i] = make_double2(x, y);
}

__global__ __launch_bounds__(256) void k_na_load_layout(const double* __restrict__ cm, int n,
                                                        double2* __restrict__ rows) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i < n) rows[i] = make_double2(cm[i], cm[static_cast<std::size_t>(n) + i]);
}

__global__ __launch_bounds__(256) void k_na_store_layout(const double2* __restrict__ rows, int n,
                                                         double* __restrict__ cm) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i >= n) return;
  const double2 v = rows[i];
  cm[i] = v.x;
  cm[static_cast<std::size_t>(n) + i] = v.y;
}

std::mutex g_na_mutex;
char* g_na_scratch[kNaMaxDevices] = {};

// Device address of transform_scratch on the current device, looked up on
// the first call there.
bool na_scratch(char** out) {
  int dev = 0;
  if (!ok(hipGetDevice(&dev), "hipGetDevice")) return false;
  if (dev < 0 || dev >= kNaMaxDevices) {
    set_last_error("allocation-free transform: device ordinal " + std::to_string(dev) + " is beyond " +
                   std::to_string(kNaMaxDevices));
    return false;
  }
  std::lock_guard<std::mutex> lock(g_na_mutex);
  if (g_na_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (!ok(hipGetSymbolAddress(&p, HIP_SYMBOL(transform_scratch)), "hipGetSymbolAddress(transform scratch)")) {
      return false;
    }
    g_na_scratch[dev] = static_cast<char*>(p);
  }
  *out = g_na_scratch[dev];
  return true;
}

}  // namespace
}  // namespace fehip

extern "C" {

int fastembedr_hip_transform_tsne_noalloc(const double* reference_layout, int n_reference, const int* indices,
                                          const double* distances, int n_query, int k, const double* y_init,
                                          int initialization, double perplexity, int n_iter,
                                          int early_exaggeration_iter, double learning_rate,
                                          double early_exaggeration, double exaggeration, double initial_momentum,
                                          double final_momentum, double max_grad_norm, double max_step_norm,
                                          int n_negatives, int exact_repulsion_threshold, int seed, double* out,
                                          int* repulsion_exact) {
  using namespace fehip;
  clear_last_error();
  if (out == nullptr || n_reference < 1 || n_query < 1 || k < 1 || reference_layout == nullptr ||
      indices == nullptr || distances == nullptr) {
    set_last_error("invalid transform arguments (NULL pointer or empty input).");
    return 1;
  }
  const long long entries = static_cast<long long>(n_query) * k;
  if (n_reference > kNaMaxReference || n_query > kNaMaxQuery || entries > kNaMaxEntries) {
    set_last_error("allocation-free transform: input exceeds its static work buffer (n_reference <= " +
                   std::to_string(kNaMaxReference) + ", n_query <= " + std::to_string(kNaMaxQuery) +
                   ", n_query * k <= " + std::to_string(kNaMaxEntries) + "); use fastembedr_hip_transform_tsne");
    return 1;
  }
  if (!(perplexity > 0.0)) {
    set_last_error("`perplexity` must be positive.");
    return 1;
  }
  RunArgs ra{n_reference, n_iter, early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
             initial_momentum, final_momentum, max_grad_norm, max_step_norm, n_negatives, exact_repulsion_threshold,
             initialization};
  if (!check_run_args(ra)) return 1;
  if (initialization == 2 && y_init == nullptr) {
    set_last_error("allocation-free transform: the random initialisation is drawn on the host; pass y_init");
    return 1;
  }
  char* base = nullptr;
  if (!na_scratch(&base)) return 1;
  NaHeader* hdr = reinterpret_cast<NaHeader*>(base);
  double2* ref = reinterpret_cast<double2*>(base + kNaReferenceOffset);
  double* p = reinterpret_cast<double*>(base + kNaPOffset);
  double2* y = reinterpret_cast<double2*>(base + kNaStateOffset);
  double2* upd = reinterpret_cast<double2*>(base + kNaStateOffset + kNaStateStride);
  double2* gains = reinterpret_cast<double2*>(base + kNaStateOffset + 2 * kNaStateStride);
  hipStream_t st = nullptr;  // the null stream: no stream is created

  const int check_blocks = static_cast<int>(std::min<long long>((entries + 255) / 256, 2048));
  k_na_clear<<<1, 64, 0, st>>>(hdr);
  k_na_check_knn<<<check_blocks, 256, 0, st>>>(indices, distances, entries, hdr);
  k_na_load_reference<<<(n_reference + 255) / 256, 256, 0, st>>>(reference_layout, n_reference, ref, hdr);
  NaHeader h{};
  if (!ok(hipGetLastError(), "transform check launch") ||
      !ok(hipMemcpyAsync(&h, hdr, sizeof(h), hipMemcpyDeviceToHost, st), "transform check download") ||
      !ok(hipStreamSynchronize(st), "transform check sync")) {
    return 1;
  }
  // 1-based iff every index is in [1, n_reference] (:1290-1302), then every
  // index must name a reference row.
  const int offset = (h.idx_min >= 1 && h.idx_max <= n_reference) ? 1 : 0;
  if (static_cast<long long>(h.idx_min) - offset < 0 ||
      static_cast<long long>(h.idx_max) - offset >= static_cast<long long>(n_reference)) {
    set_last_error("KNN indices are out of range for `reference_layout`.");
    return 1;
  }
  if ((h.flags & kNaBadDistance) != 0u) {
    set_last_error("KNN distances must be finite and non-negative.");
    return 1;
  }
  if ((h.flags & kNaBadReference) != 0u) {
    set_last_error("`reference_layout` must be finite.");
    return 1;
  }

  const int blocks = query_blocks(n_query);
  k_transform_p<<<blocks, kQueryThreads, 0, st>>>(distances, n_query, k, perplexity, p);
  if (y_init != nullptr) {
    k_na_load_layout<<<(n_query + 255) / 256, 256, 0, st>>>(y_init, n_query, y);
  } else {
    k_transform_init<<<blocks, kQueryThreads, 0, st>>>(ref, indices, distances, n_query, k, offset,
                                                      initialization == 1 ? 1 : 0, y);
  }
  k_transform_reset<<<blocks, kQueryThreads, 0, st>>>(upd, gains, n_query);
  if (!ok(hipGetLastError(), "transform setup launch")) return 1;
  const int total = early_exaggeration_iter + n_iter;
  for (int it = 0; it < total; ++it) {
    const bool early = it < early_exaggeration_iter;
    const StepParams sp{early ? early_exaggeration : exaggeration, early ? initial_momentum : final_momentum,
                        learning_rate, ra.max_grad, ra.max_step, ra.exact ? n_reference : ra.n_negatives,
                        iteration_seed(seed, it)};
    if (ra.exact) {
      k_transform_step<true, false><<<blocks, kQueryThreads, 0, st>>>(ref, n_reference, indices, p, n_query, k,
                                                                      offset, sp, y, upd, gains, nullptr);
    } else {
      k_transform_step<false, false><<<blocks, kQueryThreads, 0, st>>>(ref, n_reference, indices, p, n_query, k,
                                                                       offset, sp, y, upd, gains, nullptr);
    }
    if (!ok(hipGetLastError(), "transform step launch")) return 1;
  }
  k_na_store_layout<<<(n_query + 255) / 256, 256, 0, st>>>(y, n_query, out);
  if (!ok(hipGetLastError(), "transform store launch") || !ok(hipStreamSynchronize(st), "transform sync")) return 1;
  if (repulsion_exact != nullptr) *repulsion_exact = ra.exact ? 1 : 0;
  return 0;
}

}  // extern "C"
