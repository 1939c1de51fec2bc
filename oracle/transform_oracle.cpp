// CPU oracle for the fixed-reference t-SNE transform.
//
// TEST INFRASTRUCTURE ONLY.  An independent C++17 restatement of the
// reference package's transform_tsne_cpp (src/tsne_neighbors.cpp:1859-2109 of
// tkcaccia/fastEmbedR) for two-dimensional layouts, so that tests/ and
// bench.py's cpu_baseline leg have a checker for the HIP transform.  No
// product code links or loads it.
//
// Semantics restated (all fp64, no fused multiply-add: -ffp-contract=off):
//   * per-query conditional probabilities by bisection on beta
//     (compute_row_probabilities_flat, :437-486);
//   * initialisation: median / weighted / random (initialize_tsne_transform,
//     :1304-1372), with the per-query mt19937 seeded through mix_uint32
//     (:56-63) and normal_distribution<double>(0, 1e-4);
//   * gradient: exact repulsion over every reference point when
//     n_reference <= exact_repulsion_threshold or n_negatives >= n_reference,
//     otherwise n_negatives reference points drawn with xorshift32 /
//     multiply-shift (uniform_index, :65-77) from a per-query, per-iteration
//     state; normalised by the query's own sum of q; attraction
//     exaggeration * p * q * d (compute_tsne_transform_gradient_2d_flat,
//     :1472-1568);
//   * update: gradient-norm clip, gains (+0.2 / *0.8 + 0.01, floor 0.01,
//     fp64 sign with sign(0) = 0), momentum, step-norm clip, y += update
//     (:2040-2075).
// Queries are independent, so the result does not depend on the thread
// count or on the reference's batching (tests/testthat/test-transform-tsne.R
// asserts both at tolerance 0).

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_error;

std::uint32_t hash32(std::uint32_t v) {  // mix_uint32 (:56-63)
  v ^= v >> 16u;
  v *= 0x7feb352du;
  v ^= v >> 15u;
  v *= 0x846ca68bu;
  v ^= v >> 16u;
  return v == 0u ? 0x6d2b79f5u : v;
}

std::uint32_t xorshift(std::uint32_t& s) {  // Marsaglia (13, 17, 5) (:65-70)
  s ^= s << 13u;
  s ^= s >> 17u;
  s ^= s << 5u;
  return s;
}

int draw_index(std::uint32_t& s, int n) {  // multiply-shift to [0, n) (:72-77)
  return static_cast<int>((static_cast<std::uint64_t>(xorshift(s)) * static_cast<std::uint64_t>(n)) >> 32u);
}

std::uint32_t query_state(int seed, int query) {
  return hash32(static_cast<std::uint32_t>(seed) ^ (static_cast<std::uint32_t>(query + 1) * 0x9e3779b9u));
}

double sign0(double v) { return v == 0.0 ? 0.0 : (v < 0.0 ? -1.0 : 1.0); }

template <typename F>
void for_queries(int n, int threads, F&& body) {
  threads = std::max(1, std::min(threads, n));
  if (threads == 1) {
    body(0, n);
    return;
  }
  std::vector<std::thread> pool;
  const int chunk = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const int b = t * chunk, e = std::min(n, b + chunk);
    if (b < e) pool.emplace_back([&body, b, e] { body(b, e); });
  }
  for (auto& th : pool) th.join();
}

// Bisection on beta for one query row of distances (column-major input).
void row_p(const double* dist_cm, int nq, int k, int i, double perplexity, double* p) {
  double beta = 1.0, lo = -DBL_MAX, hi = DBL_MAX;
  double sum = DBL_MIN;
  const double target = std::log(perplexity);
  bool done = false;
  for (int it = 0; !done && it < 200; ++it) {
    sum = DBL_MIN;
    for (int j = 0; j < k; ++j) {
      const double d = dist_cm[static_cast<std::size_t>(j) * nq + i];
      p[j] = std::exp(-beta * (d * d));
      sum += p[j];
    }
    double h = 0.0;
    for (int j = 0; j < k; ++j) {
      const double d = dist_cm[static_cast<std::size_t>(j) * nq + i];
      h += beta * (d * d * p[j]);
    }
    h = h / sum + std::log(sum);
    const double diff = h - target;
    if (std::abs(diff) < 1e-5) {
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
  for (int j = 0; j < k; ++j) p[j] *= inv;
}

struct Problem {
  const double* ref = nullptr;  // n_ref x 2 row-major (x0, y0, x1, y1, ...)
  int n_ref = 0;
  const int* idx_cm = nullptr;  // nq x k column-major
  int nq = 0, k = 0, offset = 0;
  const double* p = nullptr;    // nq x k row-major
};

void gradient_2d(const Problem& pr, const double* y, double ex, int n_neg, bool exact, int seed, int threads,
                 double* grad) {
  for_queries(pr.nq, threads, [&](int b, int e) {
    std::vector<double> qv(static_cast<std::size_t>(exact ? pr.n_ref : n_neg));
    std::vector<int> pick(static_cast<std::size_t>(n_neg));
    for (int i = b; i < e; ++i) {
      const double yx = y[2 * static_cast<std::size_t>(i)];
      const double yy = y[2 * static_cast<std::size_t>(i) + 1];
      double gx = 0.0, gy = 0.0, sum_q = DBL_MIN;
      std::uint32_t st = query_state(seed, i);
      const int m_count = exact ? pr.n_ref : n_neg;
      for (int m = 0; m < m_count; ++m) {
        const int r = exact ? m : draw_index(st, pr.n_ref);
        if (!exact) pick[static_cast<std::size_t>(m)] = r;
        const double dx = yx - pr.ref[2 * static_cast<std::size_t>(r)];
        const double dy = yy - pr.ref[2 * static_cast<std::size_t>(r) + 1];
        const double q = 1.0 / (1.0 + dx * dx + dy * dy);
        qv[static_cast<std::size_t>(m)] = q;
        sum_q += q;
      }
      const double inv = 1.0 / sum_q;
      for (int m = 0; m < m_count; ++m) {
        const int r = exact ? m : pick[static_cast<std::size_t>(m)];
        const double q = qv[static_cast<std::size_t>(m)];
        const double c = -(q * q) * inv;
        gx += c * (yx - pr.ref[2 * static_cast<std::size_t>(r)]);
        gy += c * (yy - pr.ref[2 * static_cast<std::size_t>(r) + 1]);
      }
      for (int j = 0; j < pr.k; ++j) {
        const int r = pr.idx_cm[static_cast<std::size_t>(j) * pr.nq + i] - pr.offset;
        const double dx = yx - pr.ref[2 * static_cast<std::size_t>(r)];
        const double dy = yy - pr.ref[2 * static_cast<std::size_t>(r) + 1];
        const double q = 1.0 / (1.0 + dx * dx + dy * dy);
        const double c = ex * pr.p[static_cast<std::size_t>(i) * pr.k + j] * q;
        gx += c * dx;
        gy += c * dy;
      }
      grad[2 * static_cast<std::size_t>(i)] = gx;
      grad[2 * static_cast<std::size_t>(i) + 1] = gy;
    }
  });
}

void update_2d(double* y, double* upd, double* gains, double* grad, int nq, double lr, double mom,
               double max_grad, double max_step, int threads) {
  for_queries(nq, threads, [&](int b, int e) {
    for (int i = b; i < e; ++i) {
      double* g = grad + 2 * static_cast<std::size_t>(i);
      double* u = upd + 2 * static_cast<std::size_t>(i);
      double* w = gains + 2 * static_cast<std::size_t>(i);
      const double gn = g[0] * g[0] + g[1] * g[1];
      if (gn > max_grad * max_grad) {
        const double s = max_grad / (std::sqrt(gn) + 1e-12);
        g[0] *= s;
        g[1] *= s;
      }
      for (int d = 0; d < 2; ++d) {
        if (sign0(u[d]) != sign0(g[d])) {
          w[d] += 0.2;
        } else {
          w[d] = w[d] * 0.8 + 0.01;
        }
        if (w[d] < 0.01) w[d] = 0.01;
        u[d] = mom * u[d] - lr * w[d] * g[d];
      }
      const double sn = u[0] * u[0] + u[1] * u[1];
      if (sn > max_step * max_step) {
        const double s = max_step / (std::sqrt(sn) + 1e-12);
        u[0] *= s;
        u[1] *= s;
      }
      y[2 * static_cast<std::size_t>(i)] += u[0];
      y[2 * static_cast<std::size_t>(i) + 1] += u[1];
    }
  });
}

// init: 0 median, 1 weighted, 2 random.  y is nq x 2 row-major.
void initialise(const Problem& pr, const double* dist_cm, int mode, int seed, int threads, double* y) {
  if (mode == 2) {
    const unsigned int s = seed == INT_MIN ? 5489u : static_cast<unsigned int>(seed);
    for_queries(pr.nq, threads, [&](int b, int e) {
      std::normal_distribution<double> normal(0.0, 1.0e-4);
      for (int i = b; i < e; ++i) {
        std::mt19937 rng(hash32(s ^ (static_cast<std::uint32_t>(i + 1) * 0x9e3779b9u)));
        y[2 * static_cast<std::size_t>(i)] = normal(rng);
        y[2 * static_cast<std::size_t>(i) + 1] = normal(rng);
      }
    });
    return;
  }
  for_queries(pr.nq, threads, [&](int b, int e) {
    std::vector<double> vals(static_cast<std::size_t>(pr.k));
    for (int i = b; i < e; ++i) {
      for (int d = 0; d < 2; ++d) {
        double out;
        if (mode == 1) {
          double num = 0.0, den = DBL_MIN;
          for (int j = 0; j < pr.k; ++j) {
            const std::size_t c = static_cast<std::size_t>(j) * pr.nq + i;
            const int r = pr.idx_cm[c] - pr.offset;
            const double w = 1.0 / (std::max(0.0, dist_cm[c]) + 1e-6);
            num += w * pr.ref[2 * static_cast<std::size_t>(r) + d];
            den += w;
          }
          out = num / den;
        } else {
          for (int j = 0; j < pr.k; ++j) {
            const int r = pr.idx_cm[static_cast<std::size_t>(j) * pr.nq + i] - pr.offset;
            vals[static_cast<std::size_t>(j)] = pr.ref[2 * static_cast<std::size_t>(r) + d];
          }
          std::sort(vals.begin(), vals.end());
          const int mid = pr.k / 2;
          out = vals[static_cast<std::size_t>(mid)];
          if ((pr.k & 1) == 0) out = 0.5 * (out + vals[static_cast<std::size_t>(mid - 1)]);
        }
        y[2 * static_cast<std::size_t>(i) + d] = out;
      }
    }
  });
}

std::vector<double> ref_rows(const double* ref_cm, int n_ref) {
  std::vector<double> r(2 * static_cast<std::size_t>(n_ref));
  for (int i = 0; i < n_ref; ++i) {
    r[2 * static_cast<std::size_t>(i)] = ref_cm[i];
    r[2 * static_cast<std::size_t>(i) + 1] = ref_cm[static_cast<std::size_t>(n_ref) + i];
  }
  return r;
}

int iteration_seed(int seed, int iter) {  // (seed or 5489) + 65537 (iter + 1), wrapping
  const std::uint32_t base = seed == INT_MIN ? 5489u : static_cast<std::uint32_t>(seed);
  return static_cast<int>(base + 65537u * static_cast<std::uint32_t>(iter + 1));
}

// ---------------------------------------------------------------------------
// Reference-grid repulsion (no counterpart in the reference: the benchmark's
// config 3, "the reference's grid charges are precomputed once, and only the
// query points move").  The fixed reference's repulsion fields
//   Z(y) = sum_j q(y - r_j),   F(y) = sum_j q(y - r_j)^2 (y - r_j),
//   q(d) = 1 / (1 + |d|^2)
// are summed directly at the nodes of a FIt-SNE-style interpolation grid once,
// and each query's repulsion is -F(y) / Z(y) with both fields interpolated
// from the 3 x 3 nodes of its box (order-3 Lagrange).  The exact mode's
// repulsion is the same quotient with exact sums (plus DBL_MIN in Z), so the
// grid mode converges to it as the boxes shrink.  A query outside the grid
// takes the exact sums.
// ---------------------------------------------------------------------------
constexpr int kGridOrder = 3;
constexpr int kGridMaxNodes = 2048;

struct GridGeo {
  double lo = 0.0, w = 1.0, h = 1.0 / 3.0;
  int nb = 1, m = 3;
};

// One square over both axes around the reference and the queries' start,
// widened on each side by max(1, 5 % of the span); max(min_intervals,
// ceil(span / ints_in_interval)) boxes per axis, at most kGridMaxNodes nodes.
GridGeo grid_geometry(const double* ref, int n_ref, const double* y, int nq, int min_intervals, double ints) {
  double lo = DBL_MAX, hi = -DBL_MAX;
  for (std::size_t c = 0; c < 2 * static_cast<std::size_t>(n_ref); ++c) {
    lo = std::min(lo, ref[c]);
    hi = std::max(hi, ref[c]);
  }
  for (std::size_t c = 0; c < 2 * static_cast<std::size_t>(nq); ++c) {
    if (!std::isfinite(y[c])) continue;
    lo = std::min(lo, y[c]);
    hi = std::max(hi, y[c]);
  }
  double span = hi - lo;
  if (!(span > 0.0) || !std::isfinite(span)) span = 1.0;
  const double margin = std::max(1.0, 0.05 * span);
  GridGeo g;
  g.lo = lo - margin;
  span += 2.0 * margin;
  double boxes = std::max(static_cast<double>(min_intervals), std::ceil(span / ints));
  boxes = std::min(boxes, static_cast<double>(kGridMaxNodes / kGridOrder));
  g.nb = static_cast<int>(boxes);
  g.w = span / static_cast<double>(g.nb);
  g.h = g.w / static_cast<double>(kGridOrder);
  g.m = g.nb * kGridOrder;
  return g;
}

// Node fields (Z, Fx, Fy) per node, node (a, b) at
// (lo + (a + 1/2) h, lo + (b + 1/2) h), stored at 3 (b m + a); sums over the
// reference in index order.
void grid_fields(const GridGeo& g, const double* ref, int n_ref, int threads, double* field) {
  const int nodes = g.m * g.m;
  for_queries(nodes, threads, [&](int b, int e) {
    for (int v = b; v < e; ++v) {
      const double nx = g.lo + (static_cast<double>(v % g.m) + 0.5) * g.h;
      const double ny = g.lo + (static_cast<double>(v / g.m) + 0.5) * g.h;
      double z = 0.0, fx = 0.0, fy = 0.0;
      for (int j = 0; j < n_ref; ++j) {
        const double dx = nx - ref[2 * static_cast<std::size_t>(j)];
        const double dy = ny - ref[2 * static_cast<std::size_t>(j) + 1];
        const double q = 1.0 / (1.0 + dx * dx + dy * dy);
        const double q2 = q * q;
        z += q;
        fx += q2 * dx;
        fy += q2 * dy;
      }
      field[3 * static_cast<std::size_t>(v)] = z;
      field[3 * static_cast<std::size_t>(v) + 1] = fx;
      field[3 * static_cast<std::size_t>(v) + 2] = fy;
    }
  });
}

// Lagrange basis on the nodes 1/6, 1/2, 5/6 of a box, at t in [0, 1).
void grid_weights(double t, double* w) {
  const double a = t - 1.0 / 6.0;
  const double b = t - 0.5;
  const double c = t - 5.0 / 6.0;
  w[0] = 4.5 * (b * c);
  w[1] = -9.0 * (a * c);
  w[2] = 4.5 * (a * b);
}

// Repulsion of a query at (yx, yy) from the grid; false when the query is
// outside the grid (or the interpolated Z is not positive).
bool grid_repulsion(const GridGeo& g, const double* field, double yx, double yy, double* gx, double* gy) {
  const double ux = (yx - g.lo) / g.w;
  const double uy = (yy - g.lo) / g.w;
  const double fx0 = std::floor(ux);
  const double fy0 = std::floor(uy);
  if (!(fx0 >= 0.0 && fx0 < static_cast<double>(g.nb) && fy0 >= 0.0 && fy0 < static_cast<double>(g.nb))) return false;
  const int bx = static_cast<int>(fx0);
  const int by = static_cast<int>(fy0);
  double wx[3], wy[3];
  grid_weights(ux - fx0, wx);
  grid_weights(uy - fy0, wy);
  double z = 0.0, fx = 0.0, fy = 0.0;
  for (int sb = 0; sb < kGridOrder; ++sb) {
    const std::size_t row = static_cast<std::size_t>(by * kGridOrder + sb) * g.m;
    for (int sa = 0; sa < kGridOrder; ++sa) {
      const double wgt = wx[sa] * wy[sb];
      const double* f = field + 3 * (row + static_cast<std::size_t>(bx * kGridOrder + sa));
      z += wgt * f[0];
      fx += wgt * f[1];
      fy += wgt * f[2];
    }
  }
  if (!(z > 0.0)) return false;
  const double inv = 1.0 / z;
  *gx = -fx * inv;
  *gy = -fy * inv;
  return true;
}

// The exact mode's repulsion of one query (every reference point).
void exact_repulsion(const double* ref, int n_ref, double yx, double yy, double* gx, double* gy) {
  double sum_q = DBL_MIN;
  for (int j = 0; j < n_ref; ++j) {
    const double dx = yx - ref[2 * static_cast<std::size_t>(j)];
    const double dy = yy - ref[2 * static_cast<std::size_t>(j) + 1];
    sum_q += 1.0 / (1.0 + dx * dx + dy * dy);
  }
  const double inv = 1.0 / sum_q;
  double ax = 0.0, ay = 0.0;
  for (int j = 0; j < n_ref; ++j) {
    const double dx = yx - ref[2 * static_cast<std::size_t>(j)];
    const double dy = yy - ref[2 * static_cast<std::size_t>(j) + 1];
    const double q = 1.0 / (1.0 + dx * dx + dy * dy);
    const double c = -(q * q) * inv;
    ax += c * dx;
    ay += c * dy;
  }
  *gx = ax;
  *gy = ay;
}

// Gradient of every query with the grid repulsion; returns the number of
// queries that took the exact sums.
long long grid_gradient(const Problem& pr, const GridGeo& g, const double* field, const double* y, double ex,
                        int threads, double* grad) {
  std::vector<long long> outside(static_cast<std::size_t>(std::max(1, threads)), 0);
  std::atomic<int> slot{0};
  for_queries(pr.nq, threads, [&](int b, int e) {
    const int my = slot.fetch_add(1);
    long long miss = 0;
    for (int i = b; i < e; ++i) {
      const double yx = y[2 * static_cast<std::size_t>(i)];
      const double yy = y[2 * static_cast<std::size_t>(i) + 1];
      double gx = 0.0, gy = 0.0;
      if (!grid_repulsion(g, field, yx, yy, &gx, &gy)) {
        exact_repulsion(pr.ref, pr.n_ref, yx, yy, &gx, &gy);
        ++miss;
      }
      for (int j = 0; j < pr.k; ++j) {
        const int r = pr.idx_cm[static_cast<std::size_t>(j) * pr.nq + i] - pr.offset;
        const double dx = yx - pr.ref[2 * static_cast<std::size_t>(r)];
        const double dy = yy - pr.ref[2 * static_cast<std::size_t>(r) + 1];
        const double q = 1.0 / (1.0 + dx * dx + dy * dy);
        const double c = ex * pr.p[static_cast<std::size_t>(i) * pr.k + j] * q;
        gx += c * dx;
        gy += c * dy;
      }
      grad[2 * static_cast<std::size_t>(i)] = gx;
      grad[2 * static_cast<std::size_t>(i) + 1] = gy;
    }
    outside[static_cast<std::size_t>(my) % outside.size()] += miss;
  });
  long long total = 0;
  for (long long v : outside) total += v;
  return total;
}

}  // namespace

extern "C" {

const char* transform_oracle_last_error() { return g_error.c_str(); }

// 1 when every index is in [1, n_ref] (src/tsne_neighbors.cpp:1290-1302), else 0.
int transform_oracle_offset(const int* idx_cm, int nq, int k, int n_ref) {
  int lo = INT_MAX, hi = INT_MIN;
  for (std::size_t c = 0; c < static_cast<std::size_t>(nq) * k; ++c) {
    lo = std::min(lo, idx_cm[c]);
    hi = std::max(hi, idx_cm[c]);
  }
  return (lo >= 1 && hi <= n_ref) ? 1 : 0;
}

// Conditional probabilities, nq x k row-major.
void transform_oracle_conditional_p(const double* dist_cm, int nq, int k, double perplexity, int threads,
                                    double* p_rm) {
  for_queries(nq, threads, [&](int b, int e) {
    for (int i = b; i < e; ++i) row_p(dist_cm, nq, k, i, perplexity, p_rm + static_cast<std::size_t>(i) * k);
  });
}

// Initial query layout (nq x 2 row-major); mode 0 median, 1 weighted, 2 random.
void transform_oracle_init(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq, int k,
                           int mode, int seed, int threads, double* y_rm) {
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  Problem pr{ref.data(), n_ref, idx_cm, nq, k, transform_oracle_offset(idx_cm, nq, k, n_ref), nullptr};
  initialise(pr, dist_cm, mode, seed, threads, y_rm);
}

// One gradient (nq x 2 row-major) at y_rm for the given iteration seed.
void transform_oracle_gradient(const double* ref_cm, int n_ref, const int* idx_cm, const double* p_rm, int nq, int k,
                               const double* y_rm, double exaggeration, int n_negatives, int exact_threshold,
                               int iter_seed, int threads, double* grad_rm) {
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  Problem pr{ref.data(), n_ref, idx_cm, nq, k, transform_oracle_offset(idx_cm, nq, k, n_ref), p_rm};
  const int neg = std::min(n_negatives, n_ref);
  const bool exact = n_ref <= std::max(1, exact_threshold) || neg >= n_ref;
  gradient_2d(pr, y_rm, exaggeration, neg, exact, iter_seed, threads, grad_rm);
}

// One update step in place (nq x 2 row-major arrays); grad is clipped in place.
void transform_oracle_update(double* y, double* upd, double* gains, double* grad, int nq, double lr, double mom,
                             double max_grad_norm, double max_step_norm) {
  if (!(max_grad_norm > 0.0) || !std::isfinite(max_grad_norm)) max_grad_norm = DBL_MAX;
  if (!(max_step_norm > 0.0) || !std::isfinite(max_step_norm)) max_step_norm = DBL_MAX;
  update_2d(y, upd, gains, grad, nq, lr, mom, max_grad_norm, max_step_norm, 1);
}

// Whole transform.  out_cm: nq x 2 column-major (R's layout).  init_cm may be
// NULL (then `initialization` applies).  Returns -1 on invalid input, else
// 1 when the repulsion was exact and 0 when sampled.
int transform_oracle_run(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq, int k,
                         const double* init_cm, int initialization, double perplexity, int n_iter, int early_iter,
                         double lr, double early_ex, double ex, double mom0, double mom1, double max_grad_norm,
                         double max_step_norm, int n_negatives, int exact_threshold, int seed, int threads,
                         double* out_cm) {
  if (n_ref < 1 || nq < 1 || k < 1 || !(perplexity > 0.0) || n_iter < 0 || early_iter < 0 ||
      n_iter + early_iter < 1 || !(lr > 0.0) || !(early_ex > 0.0) || !(ex > 0.0) || mom0 < 0.0 || mom1 < 0.0 ||
      n_negatives < 1) {
    g_error = "invalid transform arguments";
    return -1;
  }
  if (exact_threshold < 1) exact_threshold = 1;
  if (!(max_grad_norm > 0.0) || !std::isfinite(max_grad_norm)) max_grad_norm = DBL_MAX;
  if (!(max_step_norm > 0.0) || !std::isfinite(max_step_norm)) max_step_norm = DBL_MAX;
  const int offset = transform_oracle_offset(idx_cm, nq, k, n_ref);
  for (std::size_t c = 0; c < static_cast<std::size_t>(nq) * k; ++c) {
    const int r = idx_cm[c] - offset;
    if (r < 0 || r >= n_ref) {
      g_error = "KNN indices are out of range for `reference_layout`.";
      return -1;
    }
    if (!std::isfinite(dist_cm[c]) || dist_cm[c] < 0.0) {
      g_error = "KNN distances must be finite and non-negative.";
      return -1;
    }
  }
  const int neg = std::min(n_negatives, n_ref);
  const bool exact = n_ref <= exact_threshold || neg >= n_ref;
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  std::vector<double> p(static_cast<std::size_t>(nq) * k);
  transform_oracle_conditional_p(dist_cm, nq, k, perplexity, threads, p.data());
  Problem pr{ref.data(), n_ref, idx_cm, nq, k, offset, p.data()};
  const std::size_t m = 2 * static_cast<std::size_t>(nq);
  std::vector<double> y(m), upd(m, 0.0), gains(m, 1.0), grad(m, 0.0);
  if (init_cm != nullptr) {
    for (int i = 0; i < nq; ++i) {
      y[2 * static_cast<std::size_t>(i)] = init_cm[i];
      y[2 * static_cast<std::size_t>(i) + 1] = init_cm[static_cast<std::size_t>(nq) + i];
    }
  } else {
    initialise(pr, dist_cm, initialization, seed, threads, y.data());
  }
  const int total = early_iter + n_iter;
  for (int it = 0; it < total; ++it) {
    const bool early = it < early_iter;
    gradient_2d(pr, y.data(), early ? early_ex : ex, neg, exact, iteration_seed(seed, it), threads, grad.data());
    update_2d(y.data(), upd.data(), gains.data(), grad.data(), nq, lr, early ? mom0 : mom1, max_grad_norm,
              max_step_norm, threads);
  }
  for (int i = 0; i < nq; ++i) {
    out_cm[i] = y[2 * static_cast<std::size_t>(i)];
    out_cm[static_cast<std::size_t>(nq) + i] = y[2 * static_cast<std::size_t>(i) + 1];
  }
  return exact ? 1 : 0;
}

// Geometry of the reference grid around ref_cm (n_ref x 2 column-major) and
// y_rm (nq x 2 row-major): geo = (lo, box width, boxes, nodes per axis).
// field (may be NULL): nodes x nodes x (Z, Fx, Fy).
int transform_oracle_grid_fields(const double* ref_cm, int n_ref, const double* y_rm, int nq, int min_intervals,
                                 double ints_in_interval, int threads, double* geo, double* field) {
  if (n_ref < 1 || min_intervals < 1 || !(ints_in_interval > 0.0)) {
    g_error = "invalid grid arguments";
    return -1;
  }
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  const GridGeo g = grid_geometry(ref.data(), n_ref, y_rm, nq, min_intervals, ints_in_interval);
  geo[0] = g.lo;
  geo[1] = g.w;
  geo[2] = g.nb;
  geo[3] = g.m;
  if (field != nullptr) grid_fields(g, ref.data(), n_ref, threads, field);
  return 0;
}

// One gradient at y_rm with the grid repulsion, the grid's geometry taken
// from the reference and geo_rm (n_geo x 2 row-major: the layout the grid was
// built for); returns the number of queries that took the exact sums, or -1.
long long transform_oracle_grid_gradient(const double* ref_cm, int n_ref, const int* idx_cm, const double* p_rm,
                                         int nq, int k, const double* y_rm, const double* geo_rm, int n_geo,
                                         double exaggeration, int min_intervals, double ints_in_interval,
                                         int threads, double* grad_rm) {
  if (n_ref < 1 || nq < 1 || k < 1 || min_intervals < 1 || !(ints_in_interval > 0.0)) {
    g_error = "invalid grid arguments";
    return -1;
  }
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  const GridGeo g = grid_geometry(ref.data(), n_ref, geo_rm, n_geo, min_intervals, ints_in_interval);
  std::vector<double> field(3 * static_cast<std::size_t>(g.m) * g.m);
  grid_fields(g, ref.data(), n_ref, threads, field.data());
  Problem pr{ref.data(), n_ref, idx_cm, nq, k, transform_oracle_offset(idx_cm, nq, k, n_ref), p_rm};
  return grid_gradient(pr, g, field.data(), y_rm, exaggeration, threads, grad_rm);
}

// Whole transform with the grid repulsion; the other arguments as
// transform_oracle_run.  stats (may be NULL): boxes per axis, nodes per axis,
// query-iterations that took the exact sums.  Returns 0, or -1.
int transform_oracle_grid_run(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq,
                              int k, const double* init_cm, int initialization, double perplexity, int n_iter,
                              int early_iter, double lr, double early_ex, double ex, double mom0, double mom1,
                              double max_grad_norm, double max_step_norm, int seed, int min_intervals,
                              double ints_in_interval, int threads, double* out_cm, long long* stats) {
  if (n_ref < 1 || nq < 1 || k < 1 || !(perplexity > 0.0) || n_iter < 0 || early_iter < 0 ||
      n_iter + early_iter < 1 || !(lr > 0.0) || !(early_ex > 0.0) || !(ex > 0.0) || mom0 < 0.0 || mom1 < 0.0 ||
      min_intervals < 1 || !(ints_in_interval > 0.0)) {
    g_error = "invalid transform arguments";
    return -1;
  }
  if (!(max_grad_norm > 0.0) || !std::isfinite(max_grad_norm)) max_grad_norm = DBL_MAX;
  if (!(max_step_norm > 0.0) || !std::isfinite(max_step_norm)) max_step_norm = DBL_MAX;
  const int offset = transform_oracle_offset(idx_cm, nq, k, n_ref);
  for (std::size_t c = 0; c < static_cast<std::size_t>(nq) * k; ++c) {
    const int r = idx_cm[c] - offset;
    if (r < 0 || r >= n_ref || !std::isfinite(dist_cm[c]) || dist_cm[c] < 0.0) {
      g_error = "invalid KNN input";
      return -1;
    }
  }
  const std::vector<double> ref = ref_rows(ref_cm, n_ref);
  std::vector<double> p(static_cast<std::size_t>(nq) * k);
  transform_oracle_conditional_p(dist_cm, nq, k, perplexity, threads, p.data());
  Problem pr{ref.data(), n_ref, idx_cm, nq, k, offset, p.data()};
  const std::size_t m2 = 2 * static_cast<std::size_t>(nq);
  std::vector<double> y(m2), upd(m2, 0.0), gains(m2, 1.0), grad(m2, 0.0);
  if (init_cm != nullptr) {
    for (int i = 0; i < nq; ++i) {
      y[2 * static_cast<std::size_t>(i)] = init_cm[i];
      y[2 * static_cast<std::size_t>(i) + 1] = init_cm[static_cast<std::size_t>(nq) + i];
    }
  } else {
    initialise(pr, dist_cm, initialization, seed, threads, y.data());
  }
  const GridGeo g = grid_geometry(ref.data(), n_ref, y.data(), nq, min_intervals, ints_in_interval);
  std::vector<double> field(3 * static_cast<std::size_t>(g.m) * g.m);
  grid_fields(g, ref.data(), n_ref, threads, field.data());
  long long outside = 0;
  const int total = early_iter + n_iter;
  for (int it = 0; it < total; ++it) {
    const bool early = it < early_iter;
    outside += grid_gradient(pr, g, field.data(), y.data(), early ? early_ex : ex, threads, grad.data());
    update_2d(y.data(), upd.data(), gains.data(), grad.data(), nq, lr, early ? mom0 : mom1, max_grad_norm,
              max_step_norm, threads);
  }
  for (int i = 0; i < nq; ++i) {
    out_cm[i] = y[2 * static_cast<std::size_t>(i)];
    out_cm[static_cast<std::size_t>(nq) + i] = y[2 * static_cast<std::size_t>(i) + 1];
  }
  if (stats != nullptr) {
    stats[0] = g.nb;
    stats[1] = g.m;
    stats[2] = outside;
  }
  return 0;
}

int transform_oracle_iteration_seed(int seed, int iter) { return iteration_seed(seed, iter); }

unsigned int transform_oracle_hash32(unsigned int v) { return hash32(v); }

// The first `count` outputs of xorshift32 from `state`.
void transform_oracle_xorshift(unsigned int state, int count, unsigned int* out) {
  std::uint32_t s = state;
  for (int i = 0; i < count; ++i) out[i] = xorshift(s);
}

}  // extern "C"
