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
// regenerate the same indices instead of storing them.  With the reference
// fixed, a query's iterations depend only on its own state, so one launch runs
// the whole schedule with each query's layout, update and gains in registers
// (k_transform_run).  The reference layout (16 bytes per point, 1.1 MB at 70K
// points) stays in L2.
//
// A third repulsion, with no counterpart in the reference, precomputes the
// reference's repulsion fields on an interpolation grid once per call and
// interpolates them at each query (fastembedr_hip_transform_tsne_grid).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <random>
#include <string>
#include <type_traits>
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

// Median initialisation (the default) with L lanes per query (k <= L <= 64,
// L divides the wave): lane a holds neighbour a's coordinates, counts the
// neighbours below and at them with k shuffles, and the value at rank r is
// that of a lane with less <= r < leq, as in coordinate_at_rank.
template <int L>
__global__ __launch_bounds__(kQueryThreads) void k_transform_init_lanes(const double2* __restrict__ ref,
                                                                        const int* __restrict__ idx_cm, int nq,
                                                                        int k, int offset,
                                                                        double2* __restrict__ y) {
#pragma clang fp contract(off)
  static_assert(L >= 2 && L <= 64 && (64 % L) == 0, "groups tile the wave");
  const long long t = static_cast<long long>(blockIdx.x) * kQueryThreads + threadIdx.x;
  const int i = static_cast<int>(t / L);
  const int lane = static_cast<int>(t % L);
  const bool mine = i < nq && lane < k;
  double vx = 0.0, vy = 0.0;
  if (mine) {
    const double2 r = ref[idx_cm[static_cast<std::size_t>(lane) * nq + i] - offset];
    vx = r.x;
    vy = r.y;
  }
  int lx = 0, ex = 0, ly = 0, ey = 0;  // neighbours below / at or below, per component
  for (int b = 0; b < k; ++b) {        // every lane of the wave takes part (k is uniform)
    const double bx = __shfl(vx, b, L);
    const double by = __shfl(vy, b, L);
    lx += bx < vx ? 1 : 0;
    ex += bx <= vx ? 1 : 0;
    ly += by < vy ? 1 : 0;
    ey += by <= vy ? 1 : 0;
  }
  const int base = static_cast<int>(threadIdx.x & 63) & ~(L - 1);
  const unsigned long long group = ~0ull >> (64 - L);
  auto at_rank = [&](double v, int less, int leq, int r) {
    const unsigned long long hit = (__ballot(mine && less <= r && r < leq) >> base) & group;
    return __shfl(v, hit != 0ull ? __ffsll(static_cast<long long>(hit)) - 1 : 0, L);
  };
  const int mid = k / 2;
  double mx = at_rank(vx, lx, ex, mid);
  double my = at_rank(vy, ly, ey, mid);
  if ((k & 1) == 0) {
    mx = 0.5 * (mx + at_rank(vx, lx, ex, mid - 1));
    my = 0.5 * (my + at_rank(vy, ly, ey, mid - 1));
  }
  if (i < nq && lane == 0) y[i] = make_double2(mx, my);
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

// ---- reference grid (no counterpart in the reference) ---------------------
// The fixed reference's repulsion fields Z(y) = sum_j q(y - r_j) and
// F(y) = sum_j q(y - r_j)^2 (y - r_j) are summed directly at the nodes of an
// interpolation grid once per call (k_grid_fields); a query's repulsion is
// then -F / Z with both fields interpolated (order 3, Lagrange) from the
// 3 x 3 nodes of its box.  The grid is one square of nb x nb boxes of width
// w from lo on both axes, 3 nodes per box and axis at 1/6, 1/2 and 5/6 of the
// box, m = 3 nb nodes per axis, node (a, b) at (lo + (a + 1/2) h,
// lo + (b + 1/2) h) with h = w / 3.  A query outside the square (or whose
// interpolated Z is not positive) takes the exact sums over every reference
// point.
constexpr int kGridOrder = 3;
constexpr int kGridMaxNodes = 2048;

struct GridGeo {
  double lo, w, h;
  int nb, m;
};

__device__ inline void grid_weights(double t, double* w) {
#pragma clang fp contract(off)
  const double a = t - 1.0 / 6.0;
  const double b = t - 0.5;
  const double c = t - 5.0 / 6.0;
  w[0] = 4.5 * (b * c);
  w[1] = -9.0 * (a * c);
  w[2] = 4.5 * (a * b);
}

// field: m * m double4 of (Z, Fx, Fy, 0), node (a, b) at b * m + a.
__device__ inline bool grid_repulsion(const double4* __restrict__ field, const GridGeo& g, double yx, double yy,
                                      double* gx, double* gy) {
#pragma clang fp contract(off)
  const double ux = (yx - g.lo) / g.w;
  const double uy = (yy - g.lo) / g.w;
  const double fx0 = floor(ux);
  const double fy0 = floor(uy);
  if (!(fx0 >= 0.0 && fx0 < static_cast<double>(g.nb) && fy0 >= 0.0 && fy0 < static_cast<double>(g.nb))) {
    return false;
  }
  const int bx = static_cast<int>(fx0);
  const int by = static_cast<int>(fy0);
  double wx[3], wy[3];
  grid_weights(ux - fx0, wx);
  grid_weights(uy - fy0, wy);
  double z = 0.0, fx = 0.0, fy = 0.0;
#pragma unroll
  for (int sb = 0; sb < kGridOrder; ++sb) {
    const std::size_t row = static_cast<std::size_t>(by * kGridOrder + sb) * static_cast<std::size_t>(g.m);
#pragma unroll
    for (int sa = 0; sa < kGridOrder; ++sa) {
      const double wgt = wx[sa] * wy[sb];
      const double4 f = field[row + static_cast<std::size_t>(bx * kGridOrder + sa)];
      z += wgt * f.x;
      fx += wgt * f.y;
      fy += wgt * f.z;
    }
  }
  if (!(z > 0.0)) return false;
  const double inv = 1.0 / z;
  *gx = -fx * inv;
  *gy = -fy * inv;
  return true;
}

// Node fields.  Each thread sums kFieldRows nodes of one column of the grid
// over one chunk of the reference, staged through LDS in tiles and summed in
// index order.  When the nodes alone would leave SIMDs idle (config 3: 552^2
// nodes, 1,191 waves of 4-node threads for 1,024 SIMDs) the reference is cut
// into chunks: one grid row of workgroups per chunk writes partial sums, and
// k_grid_fields_sum adds them in chunk order.  The four nodes of a thread
// share dx and 1 + dx^2 and one reciprocal (recip4).
constexpr int kFieldThreads = 256;
constexpr int kFieldRows = 4;
static_assert(kFieldRows % 4 == 0, "recip4 takes the rows four at a time");
constexpr int kFieldWavesTarget = 16 * 1024;  // ~16 waves per SIMD
constexpr int kFieldMinChunk = 4 * kFieldThreads;

// 1 / d for d >= 1: the hardware estimate (relative error below 2^-24 on
// MI355X) and two Newton-Raphson steps r <- r + r (1 - d r), each squaring
// the relative error; a probe over 2^22 log-uniform d in [1, 2^40) matched
// the correctly rounded quotient in every case.  About a quarter of the
// instructions of the IEEE division sequence, which the attraction sums of
// the reference-grid run take 8 times per lane and iteration.
__device__ __forceinline__ double recip_ge1(double d) {
  double r = __builtin_amdgcn_rcp(d);
  r = fma(r, fma(-d, r, 1.0), r);
  return fma(r, fma(-d, r, 1.0), r);
}

// q_k = 1 / d_k for four values d_k >= 1 with one reciprocal: r = 1 / p,
// p = d0 d1 d2 d3, from the hardware estimate and two Newton-Raphson steps
// r <- r + r (1 - p r) (each squares the relative error), then
// 1 / d0 = r d1 d2 d3 and so on.  A few units in the last place of the
// correctly rounded quotient; p stays finite for every d_k below 1e76.
__device__ inline void recip4(const double* d, double* q) {
  const double p01 = d[0] * d[1];
  const double p23 = d[2] * d[3];
  const double p = p01 * p23;
  double r = __builtin_amdgcn_rcp(p);
  r = fma(r, fma(-p, r, 1.0), r);
  r = fma(r, fma(-p, r, 1.0), r);
  const double i01 = r * p23;
  const double i23 = r * p01;
  q[0] = i01 * d[1];
  q[1] = i01 * d[0];
  q[2] = i23 * d[3];
  q[3] = i23 * d[2];
}

// Threads take (column, strip of kFieldRows rows) units, columns fastest;
// blockIdx.y is the reference chunk [y * chunk, (y + 1) * chunk).  With
// partial == nullptr (one chunk) the fields go straight to `field`, else to
// partial[(chunk * 3 + t) * m^2 + node], t = Z, Fx, Fy.
__global__ __launch_bounds__(kFieldThreads) void k_grid_fields(const double2* __restrict__ ref, int n_ref, int chunk,
                                                               GridGeo g, double4* __restrict__ field,
                                                               double* __restrict__ partial) {
  __shared__ double2 tile[kFieldThreads];
  const int m = g.m;
  const long long strips = (m + kFieldRows - 1) / kFieldRows;
  const long long units = static_cast<long long>(m) * strips;
  const long long u = static_cast<long long>(blockIdx.x) * kFieldThreads + threadIdx.x;
  const int col = static_cast<int>(u % m);
  const int strip = static_cast<int>(u / m);
  const double nx = g.lo + (static_cast<double>(col) + 0.5) * g.h;
  double ny[kFieldRows];
#pragma unroll
  for (int k = 0; k < kFieldRows; ++k) ny[k] = g.lo + (static_cast<double>(strip * kFieldRows + k) + 0.5) * g.h;
  double z[kFieldRows], fx[kFieldRows], fy[kFieldRows];
#pragma unroll
  for (int k = 0; k < kFieldRows; ++k) z[k] = fx[k] = fy[k] = 0.0;
  const int j0 = static_cast<int>(blockIdx.y) * chunk;
  const int j1 = min(n_ref, j0 + chunk);
  for (int base = j0; base < j1; base += kFieldThreads) {
    const int j = base + static_cast<int>(threadIdx.x);
    __syncthreads();
    if (j < j1) tile[threadIdx.x] = ref[j];
    __syncthreads();
    const int count = min(kFieldThreads, j1 - base);
    for (int t = 0; t < count; ++t) {
      const double2 r = tile[t];
      const double dx = nx - r.x;
      const double d1 = fma(dx, dx, 1.0);
      double dy[kFieldRows], d[kFieldRows], q[kFieldRows];
#pragma unroll
      for (int k = 0; k < kFieldRows; ++k) {
        dy[k] = ny[k] - r.y;
        d[k] = fma(dy[k], dy[k], d1);
      }
#pragma unroll
      for (int k = 0; k < kFieldRows; k += 4) recip4(d + k, q + k);
#pragma unroll
      for (int k = 0; k < kFieldRows; ++k) {
        const double q2 = q[k] * q[k];
        z[k] += q[k];
        fx[k] = fma(q2, dx, fx[k]);
        fy[k] = fma(q2, dy[k], fy[k]);
      }
    }
  }
  if (u >= units) return;
  const std::size_t nodes = static_cast<std::size_t>(m) * static_cast<std::size_t>(m);
#pragma unroll
  for (int k = 0; k < kFieldRows; ++k) {
    const int row = strip * kFieldRows + k;
    if (row >= m) break;
    const std::size_t v = static_cast<std::size_t>(row) * static_cast<std::size_t>(m) + static_cast<std::size_t>(col);
    if (partial == nullptr) {
      field[v] = make_double4(z[k], fx[k], fy[k], 0.0);
    } else {
      double* out = partial + static_cast<std::size_t>(blockIdx.y) * 3 * nodes + v;
      out[0] = z[k];
      out[nodes] = fx[k];
      out[2 * nodes] = fy[k];
    }
  }
}

// The chunks' partial sums added in chunk order.
__global__ __launch_bounds__(kFieldThreads) void k_grid_fields_sum(const double* __restrict__ partial, int chunks,
                                                                   long long nodes, double4* __restrict__ field) {
  const long long v = static_cast<long long>(blockIdx.x) * kFieldThreads + threadIdx.x;
  if (v >= nodes) return;
  double z = 0.0, fx = 0.0, fy = 0.0;
  for (int c = 0; c < chunks; ++c) {
    const double* in = partial + static_cast<std::size_t>(c) * 3 * static_cast<std::size_t>(nodes) + v;
    z += in[0];
    fx += in[nodes];
    fy += in[2 * nodes];
  }
  field[v] = make_double4(z, fx, fy, 0.0);
}

// Reference chunks of the node fields at m nodes per axis (1: no partial
// sums) and the chunk length (a multiple of the tile).
struct FieldSplit {
  int chunks, chunk;
};
FieldSplit field_split(int m, int n_ref) {
  const long long strips = (m + kFieldRows - 1) / kFieldRows;
  const long long waves = (static_cast<long long>(m) * strips + 63) / 64;
  long long c = (kFieldWavesTarget + waves - 1) / waves;
  c = std::max(1LL, std::min({c, 64LL, static_cast<long long>(n_ref) / kFieldMinChunk}));
  int chunk = static_cast<int>((n_ref + c - 1) / c);
  chunk = (chunk + kFieldThreads - 1) / kFieldThreads * kFieldThreads;
  return FieldSplit{static_cast<int>((n_ref + chunk - 1) / chunk), chunk};
}

// ---- one query's iteration ----------------------------------------------------
enum RepulsionMode : int { kSampled = 0, kExact = 1, kGrid = 2 };

// Attraction exaggeration * p * q * d over the query's neighbours, added to (gx, gy).
__device__ inline void attraction(const double2* __restrict__ ref, const int* __restrict__ idx_cm,
                                  const double* __restrict__ p_cm, int nq, int k, int offset, int i, double ex,
                                  double yx, double yy, double& gx, double& gy) {
#pragma clang fp contract(off)
  for (int j = 0; j < k; ++j) {
    const std::size_t e = static_cast<std::size_t>(j) * nq + i;
    const double2 p = ref[idx_cm[e] - offset];
    const double dx = yx - p.x;
    const double dy = yy - p.y;
    const double q = 1.0 / (1.0 + dx * dx + dy * dy);
    const double c = ex * p_cm[e] * q;
    gx += c * dx;
    gy += c * dy;
  }
}

// Gradient-norm clip, gains, momentum, step-norm clip and y += update (:2040-2075).
__device__ inline void update_query(double gx, double gy, double momentum, double learning_rate, double max_grad,
                                    double max_step, double2& y, double2& u, double2& w) {
#pragma clang fp contract(off)
  const double gn = gx * gx + gy * gy;
  if (gn > max_grad * max_grad) {
    const double s = max_grad / (sqrt(gn) + 1e-12);
    gx *= s;
    gy *= s;
  }
  w.x = sign0(u.x) != sign0(gx) ? w.x + 0.2 : w.x * 0.8 + 0.01;
  if (w.x < 0.01) w.x = 0.01;
  u.x = momentum * u.x - learning_rate * w.x * gx;
  w.y = sign0(u.y) != sign0(gy) ? w.y + 0.2 : w.y * 0.8 + 0.01;
  if (w.y < 0.01) w.y = 0.01;
  u.y = momentum * u.y - learning_rate * w.y * gy;
  const double sn = u.x * u.x + u.y * u.y;
  if (sn > max_step * max_step) {
    const double s = max_step / (sqrt(sn) + 1e-12);
    u.x *= s;
    u.y *= s;
  }
  y = make_double2(y.x + u.x, y.y + u.y);
}

// The repulsion of query i in the given mode; returns false when a grid query
// took the exact sums.
template <int MODE>
__device__ inline bool query_repulsion(const double2* __restrict__ ref, int n_ref, int samples, std::uint32_t state,
                                       const double4* __restrict__ field, const GridGeo& g, double yx, double yy,
                                       double& gx, double& gy) {
  if (MODE == kGrid) {
    if (grid_repulsion(field, g, yx, yy, &gx, &gy)) return true;
    const double2 r = repulsion<true>(ref, n_ref, n_ref, 0u, yx, yy);
    gx = r.x;
    gy = r.y;
    return false;
  }
  const double2 r = repulsion<MODE == kExact>(ref, n_ref, samples, state, yx, yy);
  gx = r.x;
  gy = r.y;
  return true;
}

__device__ inline std::uint32_t query_state(std::uint32_t iter_seed, int i) {
  return hash32(iter_seed ^ (static_cast<std::uint32_t>(i + 1) * 0x9e3779b9u));
}

struct StepParams {
  double exaggeration, momentum, learning_rate, max_grad, max_step;
  int samples;      // n_reference (exact) or n_negatives (sampled)
  int iter_seed;
};

// One gradient for every query (parity probes): grad_out, state untouched.
template <int MODE>
__global__ __launch_bounds__(kQueryThreads) void k_transform_gradient(
    const double2* __restrict__ ref, int n_ref, const int* __restrict__ idx_cm, const double* __restrict__ p_cm,
    int nq, int k, int offset, StepParams sp, const double4* __restrict__ field, GridGeo g,
    const double2* __restrict__ y, double2* __restrict__ grad_out, unsigned long long* __restrict__ exact_count) {
  const int i = static_cast<int>(blockIdx.x) * kQueryThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  const double2 yi = y[i];
  double gx = 0.0, gy = 0.0;
  if (!query_repulsion<MODE>(ref, n_ref, sp.samples, query_state(static_cast<std::uint32_t>(sp.iter_seed), i), field,
                             g, yi.x, yi.y, gx, gy)) {
    atomicAdd(exact_count, 1ull);
  }
  attraction(ref, idx_cm, p_cm, nq, k, offset, i, sp.exaggeration, yi.x, yi.y, gx, gy);
  grad_out[i] = make_double2(gx, gy);
}

// The whole schedule of the reference's transform loop (:1985-2080) for one
// query per thread.  With the reference fixed, a query's iterations depend on
// nothing but its own state, so running them back to back in registers gives
// exactly the iteration-by-iteration result; y holds the initial layout on
// entry and the final one on exit.
struct RunSchedule {
  double early_exaggeration, exaggeration, initial_momentum, final_momentum, learning_rate, max_grad, max_step;
  int early_iter, total, samples;
  unsigned int seed_base;  // (seed or 5489): iteration it uses seed_base + 65537 (it + 1) (:2009)
};

constexpr int kRunThreads = 64;  // small blocks spread the queries evenly over the CUs

template <int MODE>
__global__ __launch_bounds__(kRunThreads) void k_transform_run(
    const double2* __restrict__ ref, int n_ref, const int* __restrict__ idx_cm, const double* __restrict__ p_cm,
    int nq, int k, int offset, RunSchedule rs, const double4* __restrict__ field, GridGeo g,
    double2* __restrict__ y, unsigned long long* __restrict__ exact_count) {
  const int i = static_cast<int>(blockIdx.x) * kRunThreads + static_cast<int>(threadIdx.x);
  if (i >= nq) return;
  double2 yi = y[i];
  double2 u = make_double2(0.0, 0.0);
  double2 w = make_double2(1.0, 1.0);
  unsigned long long exact_evals = 0;
  for (int it = 0; it < rs.total; ++it) {
    const bool early = it < rs.early_iter;
    const std::uint32_t iter_seed = rs.seed_base + 65537u * static_cast<std::uint32_t>(it + 1);
    double gx = 0.0, gy = 0.0;
    if (!query_repulsion<MODE>(ref, n_ref, rs.samples, query_state(iter_seed, i), field, g, yi.x, yi.y, gx, gy)) {
      ++exact_evals;
    }
    attraction(ref, idx_cm, p_cm, nq, k, offset, i, early ? rs.early_exaggeration : rs.exaggeration, yi.x, yi.y, gx,
               gy);
    update_query(gx, gy, early ? rs.initial_momentum : rs.final_momentum, rs.learning_rate, rs.max_grad,
                 rs.max_step, yi, u, w);
  }
  y[i] = yi;
  if (exact_evals != 0ull) atomicAdd(exact_count, exact_evals);
}

// Grid mode with L lanes per query (L a power of two dividing the wave): the
// query's neighbours are dealt round-robin to its lanes, which load their
// reference positions and p once, keep them in registers for the whole
// schedule, and sum their part of the attraction; the parts are added by a
// butterfly over the group (the same value in every lane).  The grid
// repulsion's 9 nodes are split over the lanes the same way; the update is
// computed by every lane of the group from the same inputs, so the lanes
// keep identical states (the rare exact sums of a query outside the grid are
// taken by the whole wave and handed to the group's lanes).  L lanes per query put
// L times as many waves in flight as k_transform_run, which waits on the
// neighbours' positions every iteration.  The attraction is summed in
// another order than the reference's (per lane, then across lanes).
constexpr int kLaneThreads = 256;

template <int L>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int off = 1; off < L; off <<= 1) v += __shfl_xor(v, off, L);
  return v;
}

// grid_repulsion with the 3 x 3 nodes dealt to the group's L lanes (node
// a = lane, lane + L, ...) and their weighted fields added by group_sum.
template <int L>
__device__ inline bool grid_repulsion_lanes(const double4* __restrict__ field, const GridGeo& g, double yx, double yy,
                                            int lane, double* gx, double* gy) {
#pragma clang fp contract(off)
  const double ux = (yx - g.lo) / g.w;
  const double uy = (yy - g.lo) / g.w;
  const double fx0 = floor(ux);
  const double fy0 = floor(uy);
  if (!(fx0 >= 0.0 && fx0 < static_cast<double>(g.nb) && fy0 >= 0.0 && fy0 < static_cast<double>(g.nb))) {
    return false;
  }
  const int bx = static_cast<int>(fx0);
  const int by = static_cast<int>(fy0);
  double wx[3], wy[3];
  grid_weights(ux - fx0, wx);
  grid_weights(uy - fy0, wy);
  double z = 0.0, fx = 0.0, fy = 0.0;
#pragma unroll
  for (int a0 = 0; a0 < kGridOrder * kGridOrder; a0 += L) {
    const int a = a0 + lane;
    if (a < kGridOrder * kGridOrder) {
      const int sb = a / kGridOrder;
      const int sa = a - sb * kGridOrder;
      const double wgt = wx[sa] * wy[sb];
      const double4 f = field[static_cast<std::size_t>(by * kGridOrder + sb) * static_cast<std::size_t>(g.m) +
                              static_cast<std::size_t>(bx * kGridOrder + sa)];
      z += wgt * f.x;
      fx += wgt * f.y;
      fy += wgt * f.z;
    }
  }
  z = group_sum<L>(z);
  fx = group_sum<L>(fx);
  fy = group_sum<L>(fy);
  if (!(z > 0.0)) return false;
  const double inv = 1.0 / z;
  *gx = -fx * inv;
  *gy = -fy * inv;
  return true;
}

template <int L, int MAXJ>
__global__ __launch_bounds__(kLaneThreads) void k_transform_grid_lanes(
    const double2* __restrict__ ref, int n_ref, const int* __restrict__ idx_cm, const double* __restrict__ p_cm,
    int nq, int k, int offset, RunSchedule rs, const double4* __restrict__ field, GridGeo g,
    double2* __restrict__ y, unsigned long long* __restrict__ exact_count) {
#pragma clang fp contract(off)
  static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "a power-of-two group within the wave");
  const int gid = static_cast<int>(blockIdx.x) * kLaneThreads + static_cast<int>(threadIdx.x);
  const int i = gid / L;
  const int lane = gid & (L - 1);
  // every lane of a group takes part in the shuffles: a group past the last
  // query repeats the last one and writes nothing
  const int qi = i < nq ? i : nq - 1;
  double px[MAXJ], py[MAXJ], pj[MAXJ];
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = lane + jj * L;
    px[jj] = 0.0;
    py[jj] = 0.0;
    pj[jj] = 0.0;
    if (j < k) {
      const std::size_t e = static_cast<std::size_t>(j) * nq + qi;
      const double2 r = ref[idx_cm[e] - offset];
      px[jj] = r.x;
      py[jj] = r.y;
      pj[jj] = p_cm[e];
    }
  }
  double2 yi = y[qi];
  double2 u = make_double2(0.0, 0.0);
  double2 w = make_double2(1.0, 1.0);
  unsigned long long exact_evals = 0;
  for (int it = 0; it < rs.total; ++it) {
    const bool early = it < rs.early_iter;
    double gx = 0.0, gy = 0.0;
    const bool on_grid = grid_repulsion_lanes<L>(field, g, yi.x, yi.y, lane, &gx, &gy);
    // Outside the grid: the exact sums over every reference point (rare),
    // one such query at a time by the whole wave (its 64 lanes stride over
    // the references, in one pass: Z = DBL_MIN + sum q and sum q^2 d, then
    // -sum q^2 d / Z), so that a query off the grid does not hold its wave
    // for n_ref steps per lane.  The group's lanes take the same values.
    // Groups past the last query (their results are never stored) take no
    // part, so that they add no wave-wide passes of their own.
    unsigned long long off = __ballot(!on_grid && i < nq);  // uniform over the wave
    while (off != 0ull) {
      const int src = __ffsll(static_cast<long long>(off)) - 1;
      const double qx = __shfl(yi.x, src, 64);
      const double qy = __shfl(yi.y, src, 64);
      const int lane64 = static_cast<int>(threadIdx.x) & 63;
      double sq = 0.0, sx = 0.0, sy = 0.0;
      for (int m = lane64; m < n_ref; m += 64) {
        const double2 pr = ref[m];
        const double dx = qx - pr.x;
        const double dy = qy - pr.y;
        const double q = 1.0 / (1.0 + dx * dx + dy * dy);
        const double q2 = q * q;
        sq += q;
        sx += q2 * dx;
        sy += q2 * dy;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        sq += __shfl_xor(sq, o, 64);
        sx += __shfl_xor(sx, o, 64);
        sy += __shfl_xor(sy, o, 64);
      }
      const int first = src & ~(L - 1);
      if ((lane64 & ~(L - 1)) == first) {
        const double inv = 1.0 / (DBL_MIN + sq);
        gx = -sx * inv;
        gy = -sy * inv;
        ++exact_evals;
      }
      off &= ~((L == 64 ? ~0ull : ((1ull << L) - 1ull)) << first);
    }
    const double ex = early ? rs.early_exaggeration : rs.exaggeration;
    double ax = 0.0, ay = 0.0;
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) {
      if (lane + jj * L < k) {
        const double dx = yi.x - px[jj];
        const double dy = yi.y - py[jj];
        const double q = recip_ge1(1.0 + dx * dx + dy * dy);
        const double c = ex * pj[jj] * q;
        ax += c * dx;
        ay += c * dy;
      }
    }
    gx += group_sum<L>(ax);
    gy += group_sum<L>(ay);
    update_query(gx, gy, early ? rs.initial_momentum : rs.final_momentum, rs.learning_rate, rs.max_grad,
                 rs.max_step, yi, u, w);
  }
  if (i < nq && lane == 0) {
    y[i] = yi;
    if (exact_evals != 0ull) atomicAdd(exact_count, exact_evals);
  }
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

// The queries' initialisation (weighted: the inverse-distance mean, else the
// median): the lane kernel for medians of up to 64 neighbours.
hipError_t launch_init(const double2* ref, const int* idx, const double* dist, int nq, int k, int offset,
                       bool weighted, double2* y, hipStream_t st) {
  const auto lanes = [&](auto tag) {
    constexpr int L = decltype(tag)::value;
    const long long threads = static_cast<long long>(nq) * L;
    k_transform_init_lanes<L><<<static_cast<unsigned int>((threads + kQueryThreads - 1) / kQueryThreads),
                                kQueryThreads, 0, st>>>(ref, idx, nq, k, offset, y);
  };
  if (weighted || k > 64) {
    k_transform_init<<<query_blocks(nq), kQueryThreads, 0, st>>>(ref, idx, dist, nq, k, offset, weighted ? 1 : 0,
                                                                 y);
  } else if (k <= 8) {
    lanes(std::integral_constant<int, 8>{});
  } else if (k <= 16) {
    lanes(std::integral_constant<int, 16>{});
  } else if (k <= 32) {
    lanes(std::integral_constant<int, 32>{});
  } else {
    lanes(std::integral_constant<int, 64>{});
  }
  return hipGetLastError();
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

// Validation of the KNN input on the device (check_inputs' index and
// distance checks as one reduction), for the calls whose arrays are on the
// device already: the allocating calls after their upload, and the
// allocation-free call.
struct NaHeader {
  unsigned int flags;  // kNaBadReference
  int idx_min;
  int idx_max;
  int pad;
  unsigned long long exact_evals;  // the run kernel's counter (unused by the sampled and exact modes)
  // First failing entry (column-major position) of each kind, or ULLONG_MAX:
  // an index outside [0, n_ref) and outside [1, n_ref] (the two offsets the
  // host may settle on), and a distance that is not finite and >= 0.  The
  // host reports whichever comes first, as check_inputs' sequential scan does.
  unsigned long long first_bad_index[2];
  unsigned long long first_bad_distance;
};
constexpr unsigned int kNaBadReference = 2u;

__global__ void k_na_clear(NaHeader* h) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    h->flags = 0u;
    h->idx_min = INT_MAX;
    h->idx_max = INT_MIN;
    h->exact_evals = 0ull;
    h->first_bad_index[0] = ULLONG_MAX;
    h->first_bad_index[1] = ULLONG_MAX;
    h->first_bad_distance = ULLONG_MAX;
  }
}

// Index range and distance checks of check_inputs, as a reduction: the host
// derives the index offset from the smallest and largest index, and the error
// from the first failing entry of each kind.
__device__ inline unsigned long long wave_min_u64(unsigned long long v) {
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off);
    v = o < v ? o : v;
  }
  return v;
}

__global__ __launch_bounds__(256) void k_na_check_knn(const int* __restrict__ idx_cm,
                                                      const double* __restrict__ dist_cm, long long count,
                                                      int n_ref, NaHeader* h) {
  int lo = INT_MAX, hi = INT_MIN;
  unsigned long long bad0 = ULLONG_MAX, bad1 = ULLONG_MAX, badd = ULLONG_MAX;
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  // a thread's entries ascend, so its first failure of each kind is its least
  for (long long c = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; c < count; c += stride) {
    const int v = idx_cm[c];
    lo = v < lo ? v : lo;
    hi = v > hi ? v : hi;
    const unsigned long long at = static_cast<unsigned long long>(c);
    if ((v < 0 || v >= n_ref) && bad0 == ULLONG_MAX) bad0 = at;
    if ((v < 1 || v > n_ref) && bad1 == ULLONG_MAX) bad1 = at;
    const double d = dist_cm[c];
    if ((!isfinite(d) || d < 0.0) && badd == ULLONG_MAX) badd = at;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const int olo = __shfl_xor(lo, off);
    const int ohi = __shfl_xor(hi, off);
    lo = olo < lo ? olo : lo;
    hi = ohi > hi ? ohi : hi;
  }
  bad0 = wave_min_u64(bad0);
  bad1 = wave_min_u64(bad1);
  badd = wave_min_u64(badd);
  // the block's four waves, then one set of atomics per block (thousands of
  // atomics on the header's few words serialise: 194 us at 3M entries)
  __shared__ int wlo[4], whi[4];
  __shared__ unsigned long long wb[3][4];
  const int w = static_cast<int>(threadIdx.x) >> 6;
  if ((threadIdx.x & 63) == 0) {
    wlo[w] = lo;
    whi[w] = hi;
    wb[0][w] = bad0;
    wb[1][w] = bad1;
    wb[2][w] = badd;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int v = 1; v < 4; ++v) {
      lo = wlo[v] < lo ? wlo[v] : lo;
      hi = whi[v] > hi ? whi[v] : hi;
      bad0 = wb[0][v] < bad0 ? wb[0][v] : bad0;
      bad1 = wb[1][v] < bad1 ? wb[1][v] : bad1;
      badd = wb[2][v] < badd ? wb[2][v] : badd;
    }
    atomicMin(&h->idx_min, lo);
    atomicMax(&h->idx_max, hi);
    if (bad0 != ULLONG_MAX) atomicMin(&h->first_bad_index[0], bad0);
    if (bad1 != ULLONG_MAX) atomicMin(&h->first_bad_index[1], bad1);
    if (badd != ULLONG_MAX) atomicMin(&h->first_bad_distance, badd);
  }
}

// check_inputs' KNN result from a header filled by k_na_check_knn: the index
// offset (1-based iff every index is in [1, n_ref], :1290-1302), or -1 after
// setting the error of the earlier failing entry, as check_inputs' sequential
// scan reports it (then the reference's finiteness, which it checks last).
int knn_offset_from(const NaHeader& h, int n_ref) {
  const int offset = (h.idx_min >= 1 && h.idx_max <= n_ref) ? 1 : 0;
  const unsigned long long bad_index = h.first_bad_index[offset];
  if (bad_index != ULLONG_MAX && bad_index <= h.first_bad_distance) {
    set_last_error("KNN indices are out of range for `reference_layout`.");
    return -1;
  }
  if (h.first_bad_distance != ULLONG_MAX) {
    set_last_error("KNN distances must be finite and non-negative.");
    return -1;
  }
  return offset;
}

// Workgroups of the KNN check: at least 16 entries per thread, at most 512.
int knn_check_blocks(long long entries) {
  return static_cast<int>(std::max<long long>(1, std::min<long long>((entries + 4095) / 4096, 512)));
}

// Device buffers of one call, carved from a single allocation; the grid
// mode's node fields are a second allocation once the grid size is known.
struct TransformBuffers {
  void* base = nullptr;
  void* field_base = nullptr;
  double2* ref = nullptr;
  int* idx = nullptr;
  double* dist = nullptr;
  double* p = nullptr;
  double2* y = nullptr;
  double2* grad = nullptr;
  unsigned long long* counter = nullptr;
  NaHeader* hdr = nullptr;  // the KNN checks' result
  double4* field = nullptr;
  hipStream_t stream = nullptr;
  hipStream_t side = nullptr;     // P beside the node fields (grid mode)
  hipEvent_t side_done = nullptr;
  ~TransformBuffers() {
    if (side != nullptr) (void)hipStreamSynchronize(side);
    if (stream != nullptr) (void)hipStreamSynchronize(stream);
    if (side_done != nullptr) (void)hipEventDestroy(side_done);
    if (side != nullptr) (void)hipStreamDestroy(side);
    if (field_base != nullptr) (void)hipFree(field_base);
    if (base != nullptr) (void)hipFree(base);
    if (stream != nullptr) (void)hipStreamDestroy(stream);
  }
  bool init_side() {
    return ok(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "hipStreamCreate(transform side)") &&
           ok(hipEventCreateWithFlags(&side_done, hipEventDisableTiming), "hipEventCreate(transform side)");
  }
  bool init(int n_ref, int nq, int k) {
    const auto up = [](std::size_t b) { return (b + 255) & ~static_cast<std::size_t>(255); };
    const std::size_t nk = static_cast<std::size_t>(nq) * k;
    const std::size_t yb = up(sizeof(double2) * nq);
    const std::size_t sizes[] = {up(sizeof(double2) * n_ref), up(sizeof(int) * nk), up(sizeof(double) * nk),
                                 up(sizeof(double) * nk), 2 * yb, 256, up(sizeof(NaHeader))};
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
    y = reinterpret_cast<double2*>(c);
    grad = reinterpret_cast<double2*>(c + yb);
    c += sizes[4];
    counter = reinterpret_cast<unsigned long long*>(c);
    c += sizes[5];
    hdr = reinterpret_cast<NaHeader*>(c);
    return true;
  }
  double* field_partial = nullptr;  // the node fields' partial sums per reference chunk (null: one chunk)
  bool init_field(int m, int chunks) {
    const std::size_t nodes = static_cast<std::size_t>(m) * static_cast<std::size_t>(m);
    const std::size_t bytes = sizeof(double4) * nodes;
    const std::size_t extra = chunks > 1 ? sizeof(double) * 3 * nodes * static_cast<std::size_t>(chunks) : 0;
    if (!ok(hipMalloc(&field_base, bytes + extra), "hipMalloc(reference grid)")) return false;
    field = static_cast<double4*>(field_base);
    field_partial = chunks > 1 ? reinterpret_cast<double*>(static_cast<char*>(field_base) + bytes) : nullptr;
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

// The grid around the reference rows and the queries' layout (interleaved
// rows): one square over both axes, widened on each side by max(1, 5 % of
// the span), max(min_intervals, ceil(span / ints_in_interval)) boxes per axis
// and at most kGridMaxNodes nodes.
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
  GridGeo g{};
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

// The node fields into b.field (b.init_field(g.m, field_split(g.m, n_ref).chunks) first).
hipError_t launch_grid_fields(const double2* ref, int n_ref, const GridGeo& g, const TransformBuffers& b,
                              hipStream_t st) {
  const FieldSplit fs = field_split(g.m, n_ref);
  const long long strips = (g.m + kFieldRows - 1) / kFieldRows;
  const long long units = static_cast<long long>(g.m) * strips;
  const dim3 grid(static_cast<unsigned int>((units + kFieldThreads - 1) / kFieldThreads),
                  static_cast<unsigned int>(fs.chunks));
  double* partial = fs.chunks > 1 ? b.field_partial : nullptr;
  if (fs.chunks > 1 && partial == nullptr) return hipErrorInvalidValue;
  k_grid_fields<<<grid, kFieldThreads, 0, st>>>(ref, n_ref, fs.chunk, g, b.field, partial);
  if (fs.chunks == 1) return hipGetLastError();
  const long long nodes = static_cast<long long>(g.m) * g.m;
  k_grid_fields_sum<<<static_cast<unsigned int>((nodes + kFieldThreads - 1) / kFieldThreads), kFieldThreads, 0, st>>>(
      partial, fs.chunks, nodes, b.field);
  return hipGetLastError();
}

hipError_t launch_run(int mode, const double2* ref, int n_ref, const int* idx, const double* p, int nq, int k,
                      int offset, const RunSchedule& rs, const double4* field, const GridGeo& g, double2* y,
                      unsigned long long* counter, hipStream_t st) {
  const int blocks = (nq + kRunThreads - 1) / kRunThreads;
  if (mode == kGrid && k <= 256 && nq > 0) {
    // lanes per query: 4 up to 32 neighbours (8 per lane), then groups with
    // up to 8 per lane (config 3, k = 30: 4 lanes 158k it/s, 8 lanes 119k,
    // 16 lanes 74k, one thread per query 43k)
    const auto lanes = [&](auto tag_l, auto tag_j) {
      constexpr int L = decltype(tag_l)::value;
      constexpr int J = decltype(tag_j)::value;
      const long long threads = static_cast<long long>(nq) * L;
      const int lb = static_cast<int>((threads + kLaneThreads - 1) / kLaneThreads);
      k_transform_grid_lanes<L, J><<<lb, kLaneThreads, 0, st>>>(ref, n_ref, idx, p, nq, k, offset, rs, field, g, y,
                                                                counter);
    };
    using I8 = std::integral_constant<int, 8>;
    if (k <= 32) {
      lanes(std::integral_constant<int, 4>{}, I8{});
    } else if (k <= 64) {
      lanes(I8{}, I8{});
    } else if (k <= 128) {
      lanes(std::integral_constant<int, 16>{}, I8{});
    } else {
      lanes(std::integral_constant<int, 32>{}, I8{});
    }
  } else if (mode == kGrid) {
    k_transform_run<kGrid><<<blocks, kRunThreads, 0, st>>>(ref, n_ref, idx, p, nq, k, offset, rs, field, g, y,
                                                          counter);
  } else if (mode == kExact) {
    k_transform_run<kExact><<<blocks, kRunThreads, 0, st>>>(ref, n_ref, idx, p, nq, k, offset, rs, field, g, y,
                                                           counter);
  } else {
    k_transform_run<kSampled><<<blocks, kRunThreads, 0, st>>>(ref, n_ref, idx, p, nq, k, offset, rs, field, g, y,
                                                             counter);
  }
  return hipGetLastError();
}

hipError_t launch_gradient(int mode, const TransformBuffers& b, int n_ref, int nq, int k, int offset,
                           const StepParams& sp, const GridGeo& g) {
  const int blocks = query_blocks(nq);
  if (mode == kGrid) {
    k_transform_gradient<kGrid><<<blocks, kQueryThreads, 0, b.stream>>>(b.ref, n_ref, b.idx, b.p, nq, k, offset, sp,
                                                                        b.field, g, b.y, b.grad, b.counter);
  } else if (mode == kExact) {
    k_transform_gradient<kExact><<<blocks, kQueryThreads, 0, b.stream>>>(b.ref, n_ref, b.idx, b.p, nq, k, offset,
                                                                         sp, b.field, g, b.y, b.grad, b.counter);
  } else {
    k_transform_gradient<kSampled><<<blocks, kQueryThreads, 0, b.stream>>>(b.ref, n_ref, b.idx, b.p, nq, k, offset,
                                                                           sp, b.field, g, b.y, b.grad, b.counter);
  }
  return hipGetLastError();
}

// The reference's argument checks (:1880-1921); returns false with the message set.
// check_inputs in three parts: the scalar arguments, the KNN entries in
// order (index range, distance finite and >= 0; the first failing entry
// names the error) and the reference's finiteness.
bool check_scalars(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq, int k,
                   double perplexity) {
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
  return true;
}

bool check_reference_finite(const double* ref_cm, int n_ref) {
  for (int i = 0; i < 2 * n_ref; ++i) {
    if (!std::isfinite(ref_cm[i])) {
      set_last_error("`reference_layout` must be finite.");
      return false;
    }
  }
  return true;
}

bool check_inputs(const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm, int nq, int k,
                  double perplexity, int offset) {
  if (!check_scalars(ref_cm, n_ref, idx_cm, dist_cm, nq, k, perplexity)) return false;
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
  return check_reference_finite(ref_cm, n_ref);
}

// check_inputs' checks in its order with the KNN entries checked on the
// device after the upload (one pass instead of a host scan of every entry):
// the scalars, buffers and upload, the KNN entries, the reference's
// finiteness.  Returns the index offset, or -1 after setting the error.
int upload_checked(TransformBuffers& b, const double* ref_cm, int n_ref, const int* idx_cm, const double* dist_cm,
                   int nq, int k, double perplexity) {
  if (!check_scalars(ref_cm, n_ref, idx_cm, dist_cm, nq, k, perplexity) || !b.init(n_ref, nq, k) ||
      !upload(b, ref_cm, n_ref, idx_cm, dist_cm, nq, k)) {
    return -1;
  }
  const long long entries = static_cast<long long>(nq) * k;
  k_na_clear<<<1, 64, 0, b.stream>>>(b.hdr);
  k_na_check_knn<<<knn_check_blocks(entries), 256, 0, b.stream>>>(b.idx, b.dist, entries, n_ref, b.hdr);
  NaHeader h{};
  if (!ok(hipGetLastError(), "transform check launch") ||
      !ok(hipMemcpyAsync(&h, b.hdr, sizeof(h), hipMemcpyDeviceToHost, b.stream), "transform check download") ||
      !ok(hipStreamSynchronize(b.stream), "transform check sync")) {
    return -1;
  }
  const int offset = knn_offset_from(h, n_ref);
  if (offset < 0 || !check_reference_finite(ref_cm, n_ref)) return -1;
  return offset;
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

RunSchedule make_schedule(const RunArgs& ra, int seed) {
  RunSchedule rs{};
  rs.early_exaggeration = ra.early_exaggeration;
  rs.exaggeration = ra.exaggeration;
  rs.initial_momentum = ra.initial_momentum;
  rs.final_momentum = ra.final_momentum;
  rs.learning_rate = ra.learning_rate;
  rs.max_grad = ra.max_grad;
  rs.max_step = ra.max_step;
  rs.early_iter = ra.early_iter;
  rs.total = ra.early_iter + ra.n_iter;
  rs.samples = ra.exact ? ra.n_reference : ra.n_negatives;
  rs.seed_base = seed == INT_MIN ? 5489u : static_cast<unsigned int>(seed);
  return rs;
}

// Conditional P of every query, then its starting layout in b.y: y_init
// (n x 2 column-major), the random draw (per-query mt19937 seeded through
// mix_uint32, two normal_distribution<double>(0, 1e-4) draws, :1317-1335) or
// the median / weighted initialisation on the device.
// The queries' P (on p_stream, b.stream when null) and initial layout.
bool prepare_queries(TransformBuffers& b, int n_query, int k, int offset, double perplexity, const double* y_init,
                     int initialization, int seed, hipStream_t p_stream = nullptr) {
  const int blocks = query_blocks(n_query);
  k_transform_p<<<blocks, kQueryThreads, 0, p_stream != nullptr ? p_stream : b.stream>>>(b.dist, n_query, k,
                                                                                        perplexity, b.p);
  if (!ok(hipGetLastError(), "transform P launch")) return false;
  std::vector<double> y_host;
  if (y_init != nullptr) {
    y_host = rows_of(y_init, n_query);
  } else if (initialization == 2) {
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
    // synchronous: the staging vector dies with this function
    return ok(hipMemcpyAsync(b.y, y_host.data(), y_host.size() * sizeof(double), hipMemcpyHostToDevice, b.stream),
              "initial layout upload") &&
           ok(hipStreamSynchronize(b.stream), "transform sync");
  }
  return ok(launch_init(b.ref, b.idx, b.dist, n_query, k, offset, initialization == 1, b.y, b.stream),
            "transform init launch");
}

// b.y -> out, n x 2 column-major; waits for the stream.
bool download_layout(TransformBuffers& b, int n_query, double* out) {
  std::vector<double> y(2 * static_cast<std::size_t>(n_query));
  if (!ok(hipMemcpyAsync(y.data(), b.y, y.size() * sizeof(double), hipMemcpyDeviceToHost, b.stream),
          "layout download") ||
      !ok(hipStreamSynchronize(b.stream), "transform sync")) {
    return false;
  }
  for (int i = 0; i < n_query; ++i) {
    out[i] = y[2 * static_cast<std::size_t>(i)];
    out[static_cast<std::size_t>(n_query) + i] = y[2 * static_cast<std::size_t>(i) + 1];
  }
  return true;
}

bool check_grid_settings(int n_interpolation_points, int min_num_intervals, double ints_in_interval) {
  if (n_interpolation_points != kGridOrder) {
    set_last_error("the reference grid supports 3 interpolation points per interval");
    return false;
  }
  if (min_num_intervals < 1 || !(ints_in_interval > 0.0) || !std::isfinite(ints_in_interval)) {
    set_last_error("min_num_intervals must be >= 1 and ints_in_interval positive and finite");
    return false;
  }
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
  TransformBuffers b;
  const int offset =
      upload_checked(b, reference_layout, n_reference, indices, distances, n_query, k, perplexity);
  if (offset < 0) return 1;
  RunArgs ra{n_reference, n_iter, early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
             initial_momentum, final_momentum, max_grad_norm, max_step_norm, n_negatives, exact_repulsion_threshold,
             initialization};
  if (!check_run_args(ra) || !prepare_queries(b, n_query, k, offset, perplexity, y_init, initialization, seed)) {
    return 1;
  }
  const GridGeo none{};
  if (!ok(launch_run(ra.exact ? kExact : kSampled, b.ref, n_reference, b.idx, b.p, n_query, k, offset,
                     make_schedule(ra, seed), nullptr, none, b.y, b.counter, b.stream),
          "transform run launch") ||
      !download_layout(b, n_query, out)) {
    return 1;
  }
  if (repulsion_exact != nullptr) *repulsion_exact = ra.exact ? 1 : 0;
  return 0;
}

int fastembedr_hip_transform_tsne_grid(const double* reference_layout, int n_reference, const int* indices,
                                       const double* distances, int n_query, int k, const double* y_init,
                                       int initialization, double perplexity, int n_iter,
                                       int early_exaggeration_iter, double learning_rate, double early_exaggeration,
                                       double exaggeration, double initial_momentum, double final_momentum,
                                       double max_grad_norm, double max_step_norm, int seed,
                                       int n_interpolation_points, int min_num_intervals, double ints_in_interval,
                                       double* out, long long* stats) {
  using namespace fehip;
  clear_last_error();
  if (out == nullptr || n_reference < 1 || n_query < 1 || k < 1 || reference_layout == nullptr ||
      indices == nullptr || distances == nullptr) {
    set_last_error("invalid transform arguments (NULL pointer or empty input).");
    return 1;
  }
  if (!check_grid_settings(n_interpolation_points, min_num_intervals, ints_in_interval)) return 1;
  TransformBuffers b;
  const int offset =
      upload_checked(b, reference_layout, n_reference, indices, distances, n_query, k, perplexity);
  if (offset < 0) return 1;
  RunArgs ra{n_reference, n_iter, early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
             initial_momentum, final_momentum, max_grad_norm, max_step_norm, 1, 1, initialization};
  // P on a side stream, beside the initialisation and the node fields; the
  // run waits for it
  if (!check_run_args(ra) || !b.init_side() ||
      !prepare_queries(b, n_query, k, offset, perplexity, y_init, initialization, seed, b.side) ||
      !ok(hipEventRecord(b.side_done, b.side), "hipEventRecord(transform P)")) {
    return 1;
  }
  // The grid covers the reference and the queries' start; its geometry is
  // set on the host from both.
  std::vector<double> y0(2 * static_cast<std::size_t>(n_query));
  if (!ok(hipMemcpyAsync(y0.data(), b.y, y0.size() * sizeof(double), hipMemcpyDeviceToHost, b.stream),
          "initial layout download") ||
      !ok(hipStreamSynchronize(b.stream), "transform sync")) {
    return 1;
  }
  const std::vector<double> ref = rows_of(reference_layout, n_reference);
  const GridGeo g = grid_geometry(ref.data(), n_reference, y0.data(), n_query, min_num_intervals, ints_in_interval);
  unsigned long long exact_evals = 0;
  if (!b.init_field(g.m, field_split(g.m, n_reference).chunks) ||
      !ok(launch_grid_fields(b.ref, n_reference, g, b, b.stream), "grid fields launch") ||
      !ok(hipMemsetAsync(b.counter, 0, sizeof(unsigned long long), b.stream), "counter clear") ||
      !ok(hipStreamWaitEvent(b.stream, b.side_done, 0), "hipStreamWaitEvent(transform P)") ||
      !ok(launch_run(kGrid, b.ref, n_reference, b.idx, b.p, n_query, k, offset, make_schedule(ra, seed), b.field, g,
                     b.y, b.counter, b.stream),
          "transform run launch") ||
      !ok(hipMemcpyAsync(&exact_evals, b.counter, sizeof(exact_evals), hipMemcpyDeviceToHost, b.stream),
          "counter download") ||
      !download_layout(b, n_query, out)) {
    return 1;
  }
  if (stats != nullptr) {
    stats[0] = g.nb;
    stats[1] = g.m;
    stats[2] = static_cast<long long>(exact_evals);
  }
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
    if (!ok(launch_init(b.ref, b.idx, b.dist, n_query, k, offset, initialization != 0, b.y, b.stream),
            "transform init launch") ||
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
    const StepParams sp{exaggeration, 0.0, 0.0, 0.0, 0.0, exact ? n_reference : n_negatives, iter_seed};
    const GridGeo none{};
    if (!ok(hipMemcpyAsync(b.y, y, 2 * static_cast<std::size_t>(n_query) * sizeof(double), hipMemcpyHostToDevice,
                           b.stream),
            "state upload") ||
        !ok(launch_gradient(exact ? kExact : kSampled, b, n_reference, n_query, k, offset, sp, none),
            "transform gradient launch") ||
        !ok(hipMemcpyAsync(grad_out, b.grad, 2 * static_cast<std::size_t>(n_query) * sizeof(double),
                           hipMemcpyDeviceToHost, b.stream),
            "gradient download") ||
        !ok(hipStreamSynchronize(b.stream), "transform sync")) {
      return 1;
    }
  }
  return 0;
}

int fastembedr_hip_transform_grid_probe(const double* reference_layout, int n_reference, const int* indices,
                                        const double* distances, int n_query, int k, double perplexity,
                                        const double* y, const double* geometry_y, int n_geometry,
                                        double exaggeration, int n_interpolation_points, int min_num_intervals,
                                        double ints_in_interval, double* grad_out, long long* stats) {
  using namespace fehip;
  clear_last_error();
  if (n_reference < 1 || n_query < 1 || k < 1 || reference_layout == nullptr || indices == nullptr ||
      distances == nullptr || y == nullptr || grad_out == nullptr || (geometry_y == nullptr && n_geometry != 0) ||
      n_geometry < 0) {
    set_last_error("invalid transform probe arguments.");
    return 1;
  }
  if (!check_grid_settings(n_interpolation_points, min_num_intervals, ints_in_interval)) return 1;
  const int offset = reference_offset(indices, static_cast<std::size_t>(n_query) * k, n_reference);
  if (!check_inputs(reference_layout, n_reference, indices, distances, n_query, k, perplexity, offset)) return 1;
  TransformBuffers b;
  if (!b.init(n_reference, n_query, k) ||
      !upload(b, reference_layout, n_reference, indices, distances, n_query, k)) {
    return 1;
  }
  const std::vector<double> ref = rows_of(reference_layout, n_reference);
  const GridGeo g = grid_geometry(ref.data(), n_reference, geometry_y != nullptr ? geometry_y : y,
                                  geometry_y != nullptr ? n_geometry : n_query, min_num_intervals, ints_in_interval);
  const StepParams sp{exaggeration, 0.0, 0.0, 0.0, 0.0, n_reference, 0};
  unsigned long long exact_evals = 0;
  k_transform_p<<<query_blocks(n_query), kQueryThreads, 0, b.stream>>>(b.dist, n_query, k, perplexity, b.p);
  if (!ok(hipGetLastError(), "transform P launch") || !b.init_field(g.m, field_split(g.m, n_reference).chunks) ||
      !ok(launch_grid_fields(b.ref, n_reference, g, b, b.stream), "grid fields launch") ||
      !ok(hipMemsetAsync(b.counter, 0, sizeof(unsigned long long), b.stream), "counter clear") ||
      !ok(hipMemcpyAsync(b.y, y, 2 * static_cast<std::size_t>(n_query) * sizeof(double), hipMemcpyHostToDevice,
                         b.stream),
          "state upload") ||
      !ok(launch_gradient(kGrid, b, n_reference, n_query, k, offset, sp, g), "transform gradient launch") ||
      !ok(hipMemcpyAsync(grad_out, b.grad, 2 * static_cast<std::size_t>(n_query) * sizeof(double),
                         hipMemcpyDeviceToHost, b.stream),
          "gradient download") ||
      !ok(hipMemcpyAsync(&exact_evals, b.counter, sizeof(exact_evals), hipMemcpyDeviceToHost, b.stream),
          "counter download") ||
      !ok(hipStreamSynchronize(b.stream), "transform sync")) {
    return 1;
  }
  if (stats != nullptr) {
    stats[0] = g.nb;
    stats[1] = g.m;
    stats[2] = static_cast<long long>(exact_evals);
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
//   [0, 256)            NaHeader: validation flags, the index range and the
//                       run's exact-evaluation counter
//   reference           n_reference double2 (the layout, interleaved)
//   p                   n_query * k fp64 conditional probabilities
//   y                   n_query double2 (update and gains live in registers)
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
constexpr std::size_t kNaScratchBytes = kNaStateOffset + sizeof(double2) * kNaMaxQuery;
constexpr int kNaMaxDevices = 64;

static_assert(sizeof(NaHeader) <= kNaReferenceOffset, "the header fits its slot");

}  // namespace
}  // namespace fehip

static __device__ __align__(256) unsigned char transform_scratch[fehip::kNaScratchBytes];

namespace fehip {
namespace {

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
  hipStream_t st = nullptr;  // the null stream: no stream is created

  k_na_clear<<<1, 64, 0, st>>>(hdr);
  k_na_check_knn<<<knn_check_blocks(entries), 256, 0, st>>>(indices, distances, entries, n_reference, hdr);
  k_na_load_reference<<<(n_reference + 255) / 256, 256, 0, st>>>(reference_layout, n_reference, ref, hdr);
  NaHeader h{};
  if (!ok(hipGetLastError(), "transform check launch") ||
      !ok(hipMemcpyAsync(&h, hdr, sizeof(h), hipMemcpyDeviceToHost, st), "transform check download") ||
      !ok(hipStreamSynchronize(st), "transform check sync")) {
    return 1;
  }
  const int offset = knn_offset_from(h, n_reference);
  if (offset < 0) return 1;
  if ((h.flags & kNaBadReference) != 0u) {
    set_last_error("`reference_layout` must be finite.");
    return 1;
  }

  const int blocks = query_blocks(n_query);
  k_transform_p<<<blocks, kQueryThreads, 0, st>>>(distances, n_query, k, perplexity, p);
  if (y_init != nullptr) {
    k_na_load_layout<<<(n_query + 255) / 256, 256, 0, st>>>(y_init, n_query, y);
  } else {
    const hipError_t e = launch_init(ref, indices, distances, n_query, k, offset, initialization == 1, y, st);
    if (!ok(e, "transform init launch")) return 1;
  }
  if (!ok(hipGetLastError(), "transform setup launch")) return 1;
  const GridGeo none{};
  if (!ok(launch_run(ra.exact ? kExact : kSampled, ref, n_reference, indices, p, n_query, k, offset,
                     make_schedule(ra, seed), nullptr, none, y, &hdr->exact_evals, st),
          "transform run launch")) {
    return 1;
  }
  k_na_store_layout<<<(n_query + 255) / 256, 256, 0, st>>>(y, n_query, out);
  if (!ok(hipGetLastError(), "transform store launch") || !ok(hipStreamSynchronize(st), "transform sync")) return 1;
  if (repulsion_exact != nullptr) *repulsion_exact = ra.exact ? 1 : 0;
  return 0;
}

}  // extern "C"
