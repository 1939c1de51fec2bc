// Exact k-nearest neighbours (Euclidean) on gfx950 (CDNA4), producing the
// device-resident KNN contract of the reference's GPU route
// (src/native_knn_cuda_impl.cpp:427-466: column-major query-by-k, 1-based
// int32 indices, float32 distances, self excluded on request).  The
// reference's exact route is a third-party brute force (cuVS / FAISS GPU,
// src/native_knn_cuda_impl.cpp:549, :704) finished by
// src/embedding_cuda_kernels.cpp:1412-1464 (k + 1 searched, self dropped,
// sqrt of the squared L2 distance); its tests define exact KNN as a dense
// squared-distance matrix ordered per row, ties by index
// (tests/testthat/helper-knn.R:5-38).
//
// Three steps, all on the device:
//  1. prep: column means in fp64; a centred fp32 copy xc of the data whose
//     rows are padded with zeros to a pitch P = round_up(d, 4) + 2 (so that a
//     64-row tile is one contiguous block and 8-byte LDS reads down a column
//     of the tile hit distinct banks: P / 2 is odd); squared norms of the
//     centred rows (+inf for the rows that pad the last tile) and their
//     maximum.
//  2. scan (k_knn_scan, MFMA-bound): a wave owns 32 queries, whose
//     coordinates sit in its registers as MFMA A operands; a workgroup of 4
//     waves streams every reference through LDS in tiles of 64 rows.
//     v_mfma_f32_32x32x2f32 gives 32 x 32 dot products per step; each lane
//     reads a float2 of its reference column per two steps (dimensions
//     4m + 2h and 4m + 2h + 1 for half h, so both halves of the wave cover
//     the four dimensions of chunk m).  Per (query, reference) the scan
//     keeps s = |r|^2 - 2 q.r, which orders references as |q - r|^2 does.
//     Each query keeps a threshold t (the kp-th smallest s seen, +inf until
//     kp were seen) and a candidate buffer of B entries in global memory;
//     slots come from ballots (a wave owns its rows), and when a buffer
//     could overflow in the next tile the wave sorts it (bitonic across its
//     64 lanes) and keeps the kp best.  The host picks B >= 2 kp + 64, so
//     compactions are rare once t has settled.
//  3. finalize (k_knn_finalize): per query, the candidates' squared
//     distances are recomputed from the input rows in fp64, the query itself
//     is dropped on request, and the rest are sorted by (d2, index); the
//     first k are written.  The result is certified when no rejected
//     reference can beat the k-th: each had s >= t, and s + |q|^2 is within
//     eps = (D + 12) 2^-23 (|q|^2 + max |r|^2) of its exact squared distance
//     (D = round_up(d, 4); fp32 rounding of the centred rows, their norms and
//     D-term MFMA dot products), so t + |q|^2 - eps > d2_k suffices.
//     Uncertified queries are listed for a rerun with twice the candidates.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <string>
#include <vector>

#include "device_common.h"
#include "knn_device.h"

namespace fehip {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKnnThreads = 256;  // 4 waves
constexpr int kKnnWaves = kKnnThreads / kWave;
constexpr int kKnnWaveQueries = 32;
constexpr int kKnnQueryBlock = kKnnWaves * kKnnWaveQueries;  // 128
constexpr int kKnnRefTile = 64;                               // two 32-column MFMA blocks
constexpr int kPrepThreads = 256;

// Row pitch of xc for d dimensions: a multiple of 4 plus 2.
__host__ __device__ constexpr int knn_pitch(int d) { return (d + 3) / 4 * 4 + 2; }
// float2 copies per thread that stage one 64 x P tile (P <= 4 MAXM + 2).
__host__ __device__ constexpr int knn_tile_pairs(int maxm) { return (4 * maxm + 2 + 7) / 8; }
// xc is read up to this many floats past its last tile (whole staging copies
// and the last query row's A loads)
constexpr int kKnnOverRead = knn_tile_pairs(32) * 2 * kKnnThreads + 256;

// ---- 1. prep --------------------------------------------------------------------

// partial[b * d + c] = sum over rows [b * rows_per, (b + 1) * rows_per) of x[., c] in fp64.
__global__ __launch_bounds__(kPrepThreads) void k_knn_col_partials(const float* __restrict__ x, int n, int d,
                                                                    Strides st, int rows_per,
                                                                    double* __restrict__ partial) {
  const int r0 = static_cast<int>(blockIdx.x) * rows_per;
  const int r1 = min(n, r0 + rows_per);
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    double s = 0.0;
    for (int r = r0; r < r1; ++r) s += static_cast<double>(x[st.at(r, c)]);
    partial[static_cast<long long>(blockIdx.x) * d + c] = s;
  }
}

__global__ __launch_bounds__(kPrepThreads) void k_knn_col_means(const double* __restrict__ partial, int blocks, int d,
                                                                 int n, double* __restrict__ mean) {
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    double s = 0.0;
    for (int b = 0; b < blocks; ++b) s += partial[static_cast<long long>(b) * d + c];
    mean[c] = s / static_cast<double>(n);
  }
}

// One row per thread: xc row = fl32(x - mean), zero from column d to P - 1;
// the squared norm of the stored fp32 row, summed in fp64; the norms'
// maximum (bits of a non-negative float compare as unsigned); rows holding a
// NaN or an infinity (or whose centred norm overflows fp32) are counted in
// bad_rows.  Rows n to n_pad - 1 (the rest of the last 64-row tile) are zero
// with norm +inf, so that no query ever accepts them.
__global__ __launch_bounds__(kPrepThreads) void k_knn_center(const float* __restrict__ x, int n, int n_pad, int d,
                                                              Strides st, int P, const double* __restrict__ mean,
                                                              float* __restrict__ xc,
                                                              float* __restrict__ nrm,
                                                              unsigned int* __restrict__ nrm_max_bits,
                                                              int* __restrict__ bad_rows) {
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  float local = 0.0f;
  if (r < n) {
    double s = 0.0;
    for (int c = 0; c < P; ++c) {
      const float v = c < d ? static_cast<float>(static_cast<double>(x[st.at(r, c)]) - mean[c]) : 0.0f;
      xc[static_cast<long long>(r) * P + c] = v;
      s += static_cast<double>(v) * static_cast<double>(v);
    }
    local = static_cast<float>(s);
    if (!isfinite(local)) {  // NaN/inf input, or a norm beyond fp32
      atomicAdd(bad_rows, 1);
      local = 0.0f;
    }
    nrm[r] = local;
  } else if (r < n_pad) {
    for (int c = 0; c < P; ++c) xc[static_cast<long long>(r) * P + c] = 0.0f;
    nrm[r] = INFINITY;
  }
  // wave maximum, then one atomic per wave
  for (int off = kWave / 2; off > 0; off >>= 1) local = fmaxf(local, __shfl_xor(local, off));
  if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(nrm_max_bits, __float_as_uint(local));
}

// ---- cosine and correlation ------------------------------------------------------
// The reference searches these metrics as Euclidean distances between rows
// normalised to unit length, centred first for correlation
// (src/native_knn_common.h:50-67, 119-120), and reports half the squared
// distance, 1 - cos (:122-128; src/embedding_cuda_kernels.cpp:1441-1442).
// One row per thread, in the reference's operation order: row mean as a
// sequential fp64 sum / d, fl32(x - mean), sequential fp64 sum of the
// squares of the stored values, inverse norm fl32(1 / sqrt(sum)), and each
// value times it in fp32; a row whose sum of squares is 0 stays as it is.
// Output row-major n x d.
__global__ __launch_bounds__(kPrepThreads) void k_knn_normalize_rows(const float* __restrict__ x, int n, int d,
                                                                    Strides st, int center,
                                                                    float* __restrict__ out) {
#pragma clang fp contract(off)
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  if (r >= n) return;
  double mean = 0.0;
  if (center) {
    for (int j = 0; j < d; ++j) mean += static_cast<double>(x[st.at(r, j)]);
    mean /= static_cast<double>(d);
  }
  float* row = out + static_cast<long long>(r) * d;
  double sq = 0.0;
  for (int j = 0; j < d; ++j) {
    const float v = static_cast<float>(static_cast<double>(x[st.at(r, j)]) - mean);
    row[j] = v;
    sq += static_cast<double>(v) * static_cast<double>(v);
  }
  if (sq <= 0.0) return;
  const float inv = static_cast<float>(1.0 / sqrt(sq));
  for (int j = 0; j < d; ++j) row[j] = row[j] * inv;
}

// ---- projection of wide rows -----------------------------------------------------
// Rows wider than kKnnMaxDim are scanned in a kKnnMaxDim-dimensional
// subspace.  With Q (d x kKnnMaxDim) of orthonormal columns,
// |Q^T (x - y)| <= |x - y| for every pair: distances between projected rows
// bound the true ones from below.  The scan, its screening and its
// certificate then work on the projected rows (the certificate with a
// margin for their fp32 rounding), and the final ranking is computed from
// the input rows in fp64, so the result is the exact KNN whatever Q is.  A Q
// spanning the data's leading principal directions keeps the bound tight
// (few candidates, few reruns): it comes from block power iterations on the
// covariance of a sample of rows.

constexpr int kProjDim = kKnnMaxDim;
// Certificate margin for projected rows, in units of 2^-23 (|q|^2 + max |r|^2):
// rounding the fp64 projections to fp32 moves each by at most 2^-24 of its
// length, which changes a squared distance by at most 2^-22 (|q|^2 + |r|^2);
// the rest covers the fp64 projection and the basis' departure from exact
// orthonormality (both below 1e-12 relative).
constexpr int kProjSlack = 5;
constexpr int kCovTile = 32;
constexpr int kCovRows = 64;  // sample rows staged per step
constexpr int kProjRows = 64;
constexpr int kProjChunk = 32;

// One 32 x 32 tile (bi, bj), bi <= bj, of the covariance of the centred
// sample rows s * stride (s < m), fp64, mirrored into the lower tile.  Each
// thread owns a 2 x 2 block of the tile.
__global__ __launch_bounds__(256) void k_knn_cov(const float* __restrict__ x, Strides st, int d,
                                                 const double* __restrict__ mean, int m, long long stride,
                                                 double* __restrict__ cov) {
  const int bi = static_cast<int>(blockIdx.y), bj = static_cast<int>(blockIdx.x);
  if (bj < bi) return;  // whole block
  __shared__ double a[kCovRows][kCovTile + 1];
  __shared__ double b[kCovRows][kCovTile + 1];
  const int tid = static_cast<int>(threadIdx.x);
  const int ti = tid / 16, tj = tid % 16;
  double acc00 = 0.0, acc01 = 0.0, acc10 = 0.0, acc11 = 0.0;
  for (int s0 = 0; s0 < m; s0 += kCovRows) {
    for (int e = tid; e < kCovRows * kCovTile; e += 256) {
      const int r = e / kCovTile, c = e % kCovTile;
      const int s = s0 + r;
      const int ca = bi * kCovTile + c, cb = bj * kCovTile + c;
      const long long row = static_cast<long long>(s) * stride;
      a[r][c] = s < m && ca < d ? static_cast<double>(x[st.at(row, ca)]) - mean[ca] : 0.0;
      b[r][c] = s < m && cb < d ? static_cast<double>(x[st.at(row, cb)]) - mean[cb] : 0.0;
    }
    __syncthreads();
    for (int r = 0; r < kCovRows; ++r) {
      const double a0 = a[r][2 * ti], a1 = a[r][2 * ti + 1];
      const double b0 = b[r][2 * tj], b1 = b[r][2 * tj + 1];
      acc00 = fma(a0, b0, acc00);
      acc01 = fma(a0, b1, acc01);
      acc10 = fma(a1, b0, acc10);
      acc11 = fma(a1, b1, acc11);
    }
    __syncthreads();
  }
  const double v[2][2] = {{acc00, acc01}, {acc10, acc11}};
  for (int u = 0; u < 2; ++u) {
    for (int w = 0; w < 2; ++w) {
      const int i = bi * kCovTile + 2 * ti + u, j = bj * kCovTile + 2 * tj + w;
      if (i < d && j < d) {
        cov[static_cast<long long>(i) * d + j] = v[u][w];
        cov[static_cast<long long>(j) * d + i] = v[u][w];
      }
    }
  }
}

// y = cov q (d x d times d x kProjDim, row-major, fp64).  One block per row
// of y, one thread per column.
__global__ __launch_bounds__(kProjDim) void k_knn_cov_times(const double* __restrict__ cov,
                                                            const double* __restrict__ q, int d,
                                                            double* __restrict__ y) {
  const long long i = blockIdx.x;
  const int j = static_cast<int>(threadIdx.x);
  double s = 0.0;
  for (int c = 0; c < d; ++c) s = fma(cov[i * d + c], q[static_cast<long long>(c) * kProjDim + j], s);
  y[i * kProjDim + j] = s;
}

// Projected rows: xc row = fl32(Q^T (x - mean)) (fp64 sums), zero in
// columns kProjDim .. P - 1, with norms, their maximum and the count of
// non-finite rows exactly as k_knn_center.  A block takes 64 rows; dims are
// staged 32 at a time (the centred rows and the rows of Q); four threads
// share a row, 32 outputs each.
__global__ __launch_bounds__(256) void k_knn_project(const float* __restrict__ x, int n, int n_pad, int d,
                                                     Strides st, int P, const double* __restrict__ mean,
                                                     const double* __restrict__ q, float* __restrict__ xc,
                                                     float* __restrict__ nrm, unsigned int* __restrict__ nrm_max_bits,
                                                     int* __restrict__ bad_rows) {
  __shared__ double xs[kProjRows][kProjChunk + 1];
  __shared__ double qs[kProjChunk][kProjDim];
  const int tid = static_cast<int>(threadIdx.x);
  const int r0 = static_cast<int>(blockIdx.x) * kProjRows;
  const int lr = tid / 4;
  const int c0 = (tid % 4) * (kProjDim / 4);
  double acc[kProjDim / 4];
#pragma unroll
  for (int j = 0; j < kProjDim / 4; ++j) acc[j] = 0.0;
  for (int k0 = 0; k0 < d; k0 += kProjChunk) {
    for (int e = tid; e < kProjRows * kProjChunk; e += 256) {
      const int rr = e / kProjChunk, cc = e % kProjChunk;
      const int r = r0 + rr, c = k0 + cc;
      xs[rr][cc] = r < n && c < d ? static_cast<double>(x[st.at(r, c)]) - mean[c] : 0.0;
    }
    for (int e = tid; e < kProjChunk * kProjDim; e += 256) {
      const int cc = e / kProjDim, j = e % kProjDim;
      qs[cc][j] = k0 + cc < d ? q[static_cast<long long>(k0 + cc) * kProjDim + j] : 0.0;
    }
    __syncthreads();
    for (int cc = 0; cc < kProjChunk; ++cc) {
      const double v = xs[lr][cc];
#pragma unroll
      for (int j = 0; j < kProjDim / 4; ++j) acc[j] = fma(v, qs[cc][c0 + j], acc[j]);
    }
    __syncthreads();
  }
  const int r = r0 + lr;
  double s = 0.0;
  if (r < n) {
#pragma unroll
    for (int j = 0; j < kProjDim / 4; ++j) {
      const float v = static_cast<float>(acc[j]);
      xc[static_cast<long long>(r) * P + c0 + j] = v;
      s += static_cast<double>(v) * static_cast<double>(v);
    }
  } else if (r < n_pad) {
    for (int j = 0; j < kProjDim / 4; ++j) xc[static_cast<long long>(r) * P + c0 + j] = 0.0f;
  }
  if (r < n_pad && tid % 4 == 0) {
    for (int c = kProjDim; c < P; ++c) xc[static_cast<long long>(r) * P + c] = 0.0f;
  }
  // the row's four threads are adjacent lanes
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  float local = 0.0f;
  if (tid % 4 == 0) {
    if (r < n) {
      local = static_cast<float>(s);
      if (!isfinite(local)) {  // NaN/inf input, or a norm beyond fp32
        atomicAdd(bad_rows, 1);
        local = 0.0f;
      }
      nrm[r] = local;
    } else if (r < n_pad) {
      nrm[r] = INFINITY;
    }
  }
  for (int off = kWave / 2; off > 0; off >>= 1) local = fmaxf(local, __shfl_xor(local, off));
  if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(nrm_max_bits, __float_as_uint(local));
}

// ---- locality order ----------------------------------------------------------------
// The scan visits every reference for every query, so its result does not
// depend on the row order; its cost does, through the number of candidates
// a query accepts before its threshold settles.  Rows are therefore put in
// an order where near rows are near each other: each row goes to the cell of
// its nearest pivot (C rows spread evenly over the input), and cells are laid
// out one after another.  A block of queries then starts its scan at its own
// cell.

// Nearest pivot (pivot j = reference row j * stride) of every row of xc, by
// |p|^2 - 2 x.p in fp32 (only the order matters here, not exactness).  One row per thread, in
// registers (MAXP >= P, zero padded); pivots staged 32 at a time in LDS.
template <int MAXP>
__global__ __launch_bounds__(kPrepThreads) void k_knn_assign(const float* __restrict__ xc, int n,
                                                              const float* __restrict__ pivot_rows,
                                                              const float* __restrict__ pivot_norms, int P, int C,
                                                              int stride, int* __restrict__ cell) {
  constexpr int kPiv = 32;
  __shared__ float4 piv[kPiv * (MAXP / 4)];
  __shared__ float pn[kPiv];
  const int tid = static_cast<int>(threadIdx.x);
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + tid;
  float x[MAXP];
#pragma unroll
  for (int c = 0; c < MAXP; ++c) x[c] = (r < n && c < P) ? xc[static_cast<long long>(r) * P + c] : 0.0f;
  float best = INFINITY;
  int best_j = 0;
  for (int j0 = 0; j0 < C; j0 += kPiv) {
    __syncthreads();
    float* const pf = reinterpret_cast<float*>(piv);
    for (int e = tid; e < kPiv * MAXP; e += kPrepThreads) {
      const int j = e / MAXP, c = e % MAXP;
      pf[e] = (j0 + j < C && c < P) ? pivot_rows[static_cast<long long>(j0 + j) * stride * P + c] : 0.0f;
    }
    if (tid < kPiv) pn[tid] = j0 + tid < C ? pivot_norms[static_cast<long long>(j0 + tid) * stride] : INFINITY;
    __syncthreads();
    for (int j = 0; j < kPiv; ++j) {
      float dot = 0.0f;
#pragma unroll
      for (int c4 = 0; c4 < MAXP / 4; ++c4) {
        const float4 v = piv[j * (MAXP / 4) + c4];
        dot = fmaf(x[4 * c4], v.x, dot);
        dot = fmaf(x[4 * c4 + 1], v.y, dot);
        dot = fmaf(x[4 * c4 + 2], v.z, dot);
        dot = fmaf(x[4 * c4 + 3], v.w, dot);
      }
      const float sj = fmaf(-2.0f, dot, pn[j]);
      if (sj < best) {
        best = sj;
        best_j = j0 + j;
      }
    }
  }
  if (r < n) cell[r] = best_j;
}

__global__ __launch_bounds__(kPrepThreads) void k_knn_cell_count(const int* __restrict__ cell, int n,
                                                                  int* __restrict__ count) {
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  if (r < n) atomicAdd(&count[cell[r]], 1);
}

// Cell layout in scan order: cell j occupies positions pad_off[j] ..
// pad_off[j + 1] - 1, its count rounded up to whole 64-row tiles (so that no
// tile mixes cells); real_off[j] is the number of real rows before it.
// pad_off[C] is the number of scan positions.  C is at most a few thousand:
// one thread.
__global__ void k_knn_cell_offsets(const int* __restrict__ count, int C, int* __restrict__ pad_off,
                                   int* __restrict__ real_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int pad = 0, real = 0;
  for (int j = 0; j < C; ++j) {
    const int v = count[j];
    pad_off[j] = pad;
    real_off[j] = real;
    pad += (v + kKnnRefTile - 1) / kKnnRefTile * kKnnRefTile;
    real += v;
  }
  pad_off[C] = pad;
}

// perm[position] = row (positions of a cell's real rows in arrival order;
// the rest of its last tile keeps perm = -1), and qpos[i] = position of the
// i-th real row in scan order.
__global__ __launch_bounds__(kPrepThreads) void k_knn_cell_scatter(const int* __restrict__ cell, int n,
                                                                    int* __restrict__ cursor,
                                                                    const int* __restrict__ pad_off,
                                                                    const int* __restrict__ real_off,
                                                                    int* __restrict__ perm, int* __restrict__ qpos) {
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  if (r >= n) return;
  const int c = cell[r];
  const int i = atomicAdd(&cursor[c], 1);
  perm[pad_off[c] + i] = r;
  qpos[real_off[c] + i] = pad_off[c] + i;
}

// Queries of a query set in cell order (order[i] = query id), and each
// query's home tile: the first tile of its cell among the references.
__global__ __launch_bounds__(kPrepThreads) void k_knn_query_scatter(const int* __restrict__ cell, int n,
                                                                     int* __restrict__ cursor,
                                                                     const int* __restrict__ real_off,
                                                                     const int* __restrict__ ref_pad_off,
                                                                     int* __restrict__ order,
                                                                     int* __restrict__ home) {
  const int q = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  if (q >= n) return;
  const int c = cell[q];
  order[real_off[c] + atomicAdd(&cursor[c], 1)] = q;
  home[q] = ref_pad_off[c] / kKnnRefTile;
}

// Rows of xc and their norms in scan order; padding positions (perm -1) get
// a zero row and norm +inf, which no query accepts.  One float2 per thread.
__global__ __launch_bounds__(kPrepThreads) void k_knn_permute(const float* __restrict__ xc,
                                                               const float* __restrict__ nrm,
                                                               const int* __restrict__ perm, int n_scan, int P,
                                                               float* __restrict__ xs, float* __restrict__ ns) {
  const long long e = static_cast<long long>(blockIdx.x) * kPrepThreads + threadIdx.x;
  const int half = P / 2;
  if (e >= static_cast<long long>(n_scan) * half) return;
  const int i = static_cast<int>(e / half), c2 = static_cast<int>(e % half);
  const int src = perm[i];
  reinterpret_cast<float2*>(xs)[e] =
      src >= 0 ? reinterpret_cast<const float2*>(xc)[static_cast<long long>(src) * half + c2] : make_float2(0.0f, 0.0f);
  if (c2 == 0) ns[i] = src >= 0 ? nrm[src] : INFINITY;
}

// Bounding sphere of every 64-row tile of the scan-order rows: centre c =
// mean of the tile's real rows (norm < +inf; fp64 sums, stored fp32, pitch
// P), |c|^2 of the stored centre, and a radius >= max |r - c| over the real
// rows (fp64 from the stored fp32 values, rounded up).  Tiles without real
// rows (past the last, up to a whole group of 64) get a zero centre and
// radius -inf, which bounds every distance at +inf.  One 64-thread block per
// tile.
__global__ __launch_bounds__(kKnnRefTile) void k_knn_tile_bounds(const float* __restrict__ xs,
                                                                 const float* __restrict__ ns, int n_scan, int P,
                                                                 float* __restrict__ centre,
                                                                 float* __restrict__ cnorm,
                                                                 float* __restrict__ radius) {
  __shared__ float cen[kKnnMaxDim + 8];
  __shared__ double part[kKnnRefTile];
  __shared__ int real[kKnnRefTile];
  const int t = static_cast<int>(blockIdx.x);
  const int tid = static_cast<int>(threadIdx.x);
  const int r0 = t * kKnnRefTile;
  const bool mine = r0 + tid < n_scan && ns[r0 + tid] < INFINITY;  // a real row
  real[tid] = mine ? 1 : 0;
  __syncthreads();
  int rows = 0;
  for (int i = 0; i < kKnnRefTile; ++i) rows += real[i];
  for (int c = tid; c < P; c += kKnnRefTile) {
    double s = 0.0;
    for (int i = 0; i < kKnnRefTile; ++i)
      if (real[i]) s += static_cast<double>(xs[static_cast<long long>(r0 + i) * P + c]);
    const float v = rows > 0 ? static_cast<float>(s / rows) : 0.0f;
    cen[c] = v;
    centre[static_cast<long long>(t) * P + c] = v;
  }
  __syncthreads();
  double d2 = 0.0;
  if (mine) {
    for (int c = 0; c < P; ++c) {
      const double diff = static_cast<double>(xs[static_cast<long long>(r0 + tid) * P + c]) - cen[c];
      d2 = fma(diff, diff, d2);
    }
  }
  part[tid] = d2;
  __syncthreads();
  if (tid == 0) {
    double m = 0.0, cc = 0.0;
    for (int i = 0; i < kKnnRefTile; ++i) m = fmax(m, part[i]);
    for (int c = 0; c < P; ++c) cc = fma(static_cast<double>(cen[c]), static_cast<double>(cen[c]), cc);
    cnorm[t] = static_cast<float>(cc);
    radius[t] = rows > 0 ? __double2float_ru(sqrt(m) * (1.0 + 0x1.0p-40)) : -INFINITY;
  }
}

// ---- sorting inside one wave ------------------------------------------------------
// PER keys per lane; element E = j * 64 + lane (j = register).  Ascending
// bitonic sort of the 64 * PER keys.

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int mask) {
  const int lo = __shfl_xor(static_cast<int>(v & 0xffffffffull), mask);
  const int hi = __shfl_xor(static_cast<int>(v >> 32), mask);
  return (static_cast<unsigned long long>(static_cast<unsigned int>(hi)) << 32) | static_cast<unsigned int>(lo);
}

// The stage loops stay rolled (size and distance are wave-uniform); only
// the per-register work is unrolled, with the in-lane distance a template
// argument so that registers are never indexed at run time.
template <int PER, int JD>
__device__ __forceinline__ void inlane_step_u64(unsigned long long (&key)[PER], int lane, int size) {
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((j & JD) == 0) {
      const bool asc = ((j * kWave + lane) & size) == 0;
      const unsigned long long a = key[j], b = key[j | JD];
      const bool swap = asc ? (a > b) : (a < b);
      key[j] = swap ? b : a;
      key[j | JD] = swap ? a : b;
    }
  }
}

template <int PER>
__device__ __forceinline__ void wave_sort_u64(unsigned long long (&key)[PER], int lane) {
  constexpr int N = PER * kWave;
  for (int size = 2; size <= N; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      if (dist >= kWave) {
        switch (dist / kWave) {
          case 1: if constexpr (PER > 1) inlane_step_u64<PER, 1>(key, lane, size); break;
          case 2: if constexpr (PER > 2) inlane_step_u64<PER, 2>(key, lane, size); break;
          case 4: if constexpr (PER > 4) inlane_step_u64<PER, 4>(key, lane, size); break;
          case 8: if constexpr (PER > 8) inlane_step_u64<PER, 8>(key, lane, size); break;
          default: break;
        }
      } else {
        const bool lower = (lane & dist) == 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const unsigned long long other = shfl_xor_u64(key[j], dist);
          const bool keep_min = lower == (((j * kWave + lane) & size) == 0);
          key[j] = keep_min ? (other < key[j] ? other : key[j]) : (other > key[j] ? other : key[j]);
        }
      }
    }
  }
}

// (d2, index) pairs in fp64 / int: same network, lexicographic order.
template <int PER, int JD>
__device__ __forceinline__ void inlane_step_pairs(double (&d2)[PER], int (&id)[PER], int lane, int size) {
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((j & JD) == 0) {
      const bool asc = ((j * kWave + lane) & size) == 0;
      const double a = d2[j], b = d2[j | JD];
      const int ia = id[j], ib = id[j | JD];
      const bool a_gt = a > b || (a == b && ia > ib);
      const bool swap = asc ? a_gt : !a_gt;
      d2[j] = swap ? b : a;
      d2[j | JD] = swap ? a : b;
      id[j] = swap ? ib : ia;
      id[j | JD] = swap ? ia : ib;
    }
  }
}

template <int PER>
__device__ __forceinline__ void wave_sort_pairs(double (&d2)[PER], int (&id)[PER], int lane) {
  constexpr int N = PER * kWave;
  for (int size = 2; size <= N; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      if (dist >= kWave) {
        switch (dist / kWave) {
          case 1: if constexpr (PER > 1) inlane_step_pairs<PER, 1>(d2, id, lane, size); break;
          case 2: if constexpr (PER > 2) inlane_step_pairs<PER, 2>(d2, id, lane, size); break;
          case 4: if constexpr (PER > 4) inlane_step_pairs<PER, 4>(d2, id, lane, size); break;
          case 8: if constexpr (PER > 8) inlane_step_pairs<PER, 8>(d2, id, lane, size); break;
          default: break;
        }
      } else {
        const bool lower = (lane & dist) == 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const double od = __shfl_xor(d2[j], dist);
          const int oi = __shfl_xor(id[j], dist);
          const bool keep_min = lower == (((j * kWave + lane) & size) == 0);
          const bool other_less = od < d2[j] || (od == d2[j] && oi < id[j]);
          const bool take = keep_min ? other_less : !other_less;
          d2[j] = take ? od : d2[j];
          id[j] = take ? oi : id[j];
        }
      }
    }
  }
}

// ---- 2. scan ----------------------------------------------------------------------

// Order-preserving bits of a float (no NaN): a < b iff key(a) < key(b) as
// unsigned integers, negatives included.
__device__ __forceinline__ unsigned int ordered_bits(float f) {
  const unsigned int u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(unsigned int o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ unsigned long long cand_key(uint2 c) {
  return (static_cast<unsigned long long>(c.x) << 32) | c.y;
}

// Sorts the row's buffer of (ordered s bits, index) entries and keeps its kp
// best (in order at its front); returns the new count, and the new
// threshold (the kp-th s) through thr when kp were seen.
template <int B>
__device__ __noinline__ int compact_row(uint2* __restrict__ row_buf, int cnt, int kp, int lane, float* thr) {
  constexpr int PER = B / kWave;
  // The entries were stored by other lanes of this wave: wait until those
  // stores are done (the CU's L1 is shared by the workgroup).
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  unsigned long long key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    key[j] = e < cnt ? cand_key(row_buf[e]) : ~0ull;
  }
  wave_sort_u64<PER>(key, lane);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    if (e < kp && e < cnt)
      row_buf[e] = make_uint2(static_cast<unsigned int>(key[j] >> 32), static_cast<unsigned int>(key[j]));
  }
  if (cnt >= kp) {
    // element kp - 1 sits in lane (kp - 1) % 64, register (kp - 1) / 64
    unsigned int bits = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (j == (kp - 1) / kWave) bits = static_cast<unsigned int>(key[j] >> 32);
    bits = __shfl(static_cast<int>(bits), (kp - 1) % kWave);
    *thr = from_ordered_bits(bits);
  }
  return min(cnt, kp);
}

// Query list position p -> point index.
__device__ __forceinline__ int query_id(const int* __restrict__ qlist, int q_offset, int p) {
  return qlist != nullptr ? qlist[p] : q_offset + p;
}

// Per wave row state in LDS: threshold, count and squared norm of each of its
// 32 queries.
struct alignas(16) WaveRows {
  float thr[kKnnWaves][kKnnWaveQueries];
  int cnt[kKnnWaves][kKnnWaveQueries];
  float nq[kKnnWaves][kKnnWaveQueries];  // |q|^2
};

// The dot products of a tile: per chunk m of 4 dimensions, one float2 LDS
// read of the lane's query (dims 4m + 2h, 4m + 2h + 1) and one per block of
// 32 references (reference c32, the same dims), then four MFMA steps.  The
// next chunk's operands are read while the current chunk's steps run (the
// read one chunk past the last stays inside the LDS rows and is not used);
// the first chunk starts both accumulators from zero.
__device__ __forceinline__ void knn_chunk_mfma(float2 a, float2 b0, float2 b1, v16f& acc0, v16f& acc1) {
  acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0.x, acc0, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b1.x, acc1, 0, 0, 0);
  acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b0.y, acc0, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1.y, acc1, 0, 0, 0);
}

__device__ __forceinline__ void knn_tile_dots(int chunks, const float* qa, const float* col0, const float* col1,
                                              v16f& acc0, v16f& acc1) {
  const float2* const q2 = reinterpret_cast<const float2*>(qa);
  const float2* const c0 = reinterpret_cast<const float2*>(col0);
  const float2* const c1 = reinterpret_cast<const float2*>(col1);
  float2 xa = q2[0], x0 = c0[0], x1 = c1[0];
  float2 ya = q2[2], y0 = c0[2], y1 = c1[2];
  const v16f zero = {0};
  acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.x, x0.x, zero, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.x, x1.x, zero, 0, 0, 0);
  acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.y, x0.y, acc0, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.y, x1.y, acc1, 0, 0, 0);
  for (int m = 1; m < chunks; m += 2) {
    // chunk m is in y; read chunk m + 1 into x
    xa = q2[2 * m + 2];
    x0 = c0[2 * m + 2];
    x1 = c1[2 * m + 2];
    knn_chunk_mfma(ya, y0, y1, acc0, acc1);
    if (m + 1 >= chunks) break;
    // chunk m + 1 is in x; read chunk m + 2 into y
    ya = q2[2 * m + 4];
    y0 = c0[2 * m + 4];
    y1 = c1[2 * m + 4];
    knn_chunk_mfma(xa, x0, x1, acc0, acc1);
  }
}

// One 64-row block's staging copy for one thread: float2 number tid + 256 s
// (s < pairs = ceil(P / 8)) of the block's contiguous 64 x P rows (the last
// copy reads past the block's end, into the next rows or the array's tail
// allowance, and is never used), and one auxiliary float per row: aux0[row]
// for tid < 64, aux1[row] for 64 <= tid < 128.  Reference tiles carry their
// norms (aux0); a group's tile centres carry |c|^2 (aux0) and radii (aux1).
template <int MAXM>
struct TileRegs {
  float2 v[knn_tile_pairs(MAXM)];
  float aux;
};

template <int MAXM>
__device__ __forceinline__ void knn_load_tile(TileRegs<MAXM>& r, const float* __restrict__ rows,
                                              const float* __restrict__ aux0, const float* __restrict__ aux1, int t,
                                              int P, int pairs, int tid) {
  const float2* const src = reinterpret_cast<const float2*>(rows + static_cast<long long>(t) * kKnnRefTile * P);
#pragma unroll
  for (int s = 0; s < knn_tile_pairs(MAXM); ++s)
    if (s < pairs) r.v[s] = src[tid + s * kKnnThreads];
  if (tid < kKnnRefTile)
    r.aux = aux0[t * kKnnRefTile + tid];
  else if (tid < 2 * kKnnRefTile && aux1 != nullptr)
    r.aux = aux1[t * kKnnRefTile + tid - kKnnRefTile];
}

// LDS of a scan block, in floats: the staged 64 rows (pairs * 512), aux0
// (64), aux1 (64), then the 128 query rows (pitch P) and 4 floats for the
// read one chunk past the last row.
__host__ __device__ constexpr int knn_lds_aux(int P) { return (P + 7) / 8 * 2 * kKnnThreads; }
__host__ __device__ constexpr int knn_lds_queries(int P) { return knn_lds_aux(P) + 2 * kKnnRefTile; }
__host__ __device__ constexpr int knn_scan_lds_floats(int P) { return knn_lds_queries(P) + kKnnQueryBlock * P + 4; }

template <int MAXM>
__device__ __forceinline__ void knn_store_tile(const TileRegs<MAXM>& r, float* dst, int P, int pairs, int tid) {
  float2* const d2 = reinterpret_cast<float2*>(dst);
#pragma unroll
  for (int s = 0; s < knn_tile_pairs(MAXM); ++s)
    if (s < pairs) d2[tid + s * kKnnThreads] = r.v[s];
  if (tid < 2 * kKnnRefTile) dst[knn_lds_aux(P) + tid] = r.aux;
}

// Lower bound of |q - r|^2 over a ball (centre c, radius rad): (|q - c| -
// rad)^2 when positive, with |q - c|^2 = |q|^2 + |c|^2 - 2 q.c computed in
// fp32 and lowered by its rounding bound eps (|q|^2 + |c|^2), the square root
// and square shaded down by 2^-20.  A ball of radius -inf (padding) bounds
// at +inf.
__device__ __forceinline__ float knn_ball_bound(float nq, float nc, float rad, float qc, float eps) {
  const float d2 = nq + nc - 2.0f * qc - eps * (nq + nc);
  const float gap = sqrtf(fmaxf(d2, 0.0f)) - rad;
  return gap > 0.0f ? gap * gap * (1.0f - 0x1.0p-20f) : 0.0f;
}

// Occupancy: 3 workgroups per CU (3 waves per SIMD) for up to 64 dimensions,
// 2 above (their LDS, 70 KB at 128 dimensions, allows no more).
template <int MAXM>
constexpr int knn_scan_blocks_per_cu() {
  return MAXM <= 16 ? 3 : 2;
}

// Reference tiles and their groups: tiles of 64 rows, groups of 64 tiles;
// the centres of a group's tiles are staged like a tile and screened with
// the same MFMA steps.
struct TileGroups {
  const float* centre;  // 64 * groups rows of pitch P (zero past the last tile)
  const float* cnorm;   // |c|^2 per tile
  const float* radius;  // per tile (-inf past the last tile)
};

template <int B, int MAXM>
__global__ __launch_bounds__(kKnnThreads, knn_scan_blocks_per_cu<MAXM>()) void k_knn_scan(
    const float* __restrict__ xc, const float* __restrict__ nrm, TileGroups tg, const float* __restrict__ xq,
    const float* __restrict__ nrm_q, const int* __restrict__ home, const int* __restrict__ qlist, int q_offset, int nq,
    int n, int P, int chunks, int kp, float eps_lb, uint2* __restrict__ buf, float* __restrict__ thr_out,
    int* __restrict__ cnt_out, unsigned long long* __restrict__ work) {
  const int pairs = (P + 7) / 8;
  const int aux_at = knn_lds_aux(P);
  extern __shared__ float smem[];
  float* const rt = smem;                       // the staged rows, then aux0 and aux1
  float* const qa = smem + knn_lds_queries(P);  // the block's 128 query rows, pitch P
  __shared__ WaveRows rs;
  __shared__ unsigned long long wave_need[kKnnWaves];
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid & (kWave - 1);
  const int h = lane >> 5;
  const int c32 = lane & 31;
  const int p0 = static_cast<int>(blockIdx.x) * kKnnQueryBlock;  // first list position of the block

  // the wave's 32 query rows to LDS (zero rows past the list's end)
  const int p_lane = p0 + wave * kKnnWaveQueries + c32;
  const int q_lane = p_lane < nq ? query_id(qlist, q_offset, p_lane) : -1;
  for (int r = 0; r < kKnnWaveQueries; ++r) {
    const int q = __shfl(q_lane, r);
    const float2* const src = reinterpret_cast<const float2*>(xq + static_cast<long long>(q >= 0 ? q : 0) * P);
    float2* const dst = reinterpret_cast<float2*>(qa + (wave * kKnnWaveQueries + r) * P);
    for (int e = lane; e < P / 2; e += kWave) dst[e] = q >= 0 ? src[e] : make_float2(0.0f, 0.0f);
  }
  if (lane < kKnnWaveQueries) {
    rs.thr[wave][lane] = q_lane >= 0 ? INFINITY : -INFINITY;  // -inf: no row, accepts nothing
    rs.cnt[wave][lane] = 0;
    rs.nq[wave][lane] = q_lane >= 0 ? nrm_q[q_lane] : 0.0f;
  }

  // Groups of 64 tiles are visited from the group holding the block's first
  // query's home tile (its own position among the references, or the first
  // tile of its cell for a separate query set: rows are in locality order, so
  // the nearest references come first and the thresholds settle early),
  // wrapping around.  Per group: stage its
  // tile centres, and find per wave the tiles that can hold a candidate of
  // one of its queries: a reference r of a tile with centre c and radius rad
  // has |q - r| >= |q - c| - rad, and only tiles whose bound is below
  // t + |q|^2 for some query (s = |r|^2 - 2 q.r < t) are staged.  Skipped
  // references count as rejected: their squared distance is at least the
  // query's threshold, as the certificate requires.  The next 64-row block
  // (tile or group centres) is loaded into registers while one is used.
  const int tiles = (n + kKnnRefTile - 1) / kKnnRefTile;
  const int groups = (tiles + kKnnRefTile - 1) / kKnnRefTile;
  const int q_first = query_id(qlist, q_offset, p0);
  const int t0 = __builtin_amdgcn_readfirstlane(home != nullptr ? home[q_first] : q_first / kKnnRefTile);
  const int g0 = t0 / kKnnRefTile;
  const float* const qrow = qa + (wave * kKnnWaveQueries + c32) * P + 2 * h;
  uint2* const wave_buf = buf + static_cast<long long>(p0 + wave * kKnnWaveQueries) * B;
  unsigned int staged = 0, computed = 0;  // tiles staged by the block, tiles computed by the wave
  TileRegs<MAXM> pre;
  knn_load_tile<MAXM>(pre, tg.centre, tg.cnorm, tg.radius, g0, P, pairs, tid);
  for (int gi = 0; gi < groups; ++gi) {
    const int g = g0 + gi < groups ? g0 + gi : g0 + gi - groups;
    __syncthreads();  // every wave is done with the rows in LDS
    knn_store_tile<MAXM>(pre, rt, P, pairs, tid);
    __syncthreads();
    unsigned long long need;  // bit j: tile 64 g + j can hold a candidate of this wave's queries
    {
      v16f acc0, acc1;
      knn_tile_dots(chunks, qrow, rt + c32 * P + 2 * h, rt + (32 + c32) * P + 2 * h, acc0, acc1);
      const float nc0 = rt[aux_at + c32], nc1 = rt[aux_at + 32 + c32];
      const float rd0 = rt[aux_at + kKnnRefTile + c32], rd1 = rt[aux_at + kKnnRefTile + 32 + c32];
      bool need0 = false, need1 = false;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int row0 = 8 * g4 + 4 * h;
        const float4 thr4 = *reinterpret_cast<const float4*>(&rs.thr[wave][row0]);
        const float4 nq4 = *reinterpret_cast<const float4*>(&rs.nq[wave][row0]);
        const float thr_a[4] = {thr4.x, thr4.y, thr4.z, thr4.w};
        const float nq_a[4] = {nq4.x, nq4.y, nq4.z, nq4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float lim = thr_a[u] + nq_a[u];
          need0 |= knn_ball_bound(nq_a[u], nc0, rd0, acc0[4 * g4 + u], eps_lb) < lim;
          need1 |= knn_ball_bound(nq_a[u], nc1, rd1, acc1[4 * g4 + u], eps_lb) < lim;
        }
      }
      const unsigned long long b0 = __ballot(need0), b1 = __ballot(need1);
      need = ((b0 | (b0 >> 32)) & 0xffffffffull) | (((b1 | (b1 >> 32)) & 0xffffffffull) << 32);
    }
    if (lane == 0) wave_need[wave] = need;
    __syncthreads();
    // Tiles are taken in order from `rot` (the block's own tile in the first
    // group, so that the thresholds start from the nearest references), as
    // bits of the mask rotated right by rot.
    const int rot = gi == 0 ? t0 - g * kKnnRefTile : 0;
    auto rotr = [](unsigned long long v, int r) { return r == 0 ? v : (v >> r) | (v << (kKnnRefTile - r)); };
    unsigned long long todo = rotr(wave_need[0] | wave_need[1] | wave_need[2] | wave_need[3], rot);
    need = rotr(need, rot);
    int cur = -1;  // tile index within the group, rotated
    if (todo != 0ull) {
      cur = __ffsll(static_cast<long long>(todo)) - 1;
      todo &= todo - 1ull;
      knn_load_tile<MAXM>(pre, xc, nrm, nullptr, g * kKnnRefTile + ((cur + rot) & (kKnnRefTile - 1)), P, pairs,
                          tid);
    } else if (gi + 1 < groups) {
      const int gn = g + 1 < groups ? g + 1 : 0;
      knn_load_tile<MAXM>(pre, tg.centre, tg.cnorm, tg.radius, gn, P, pairs, tid);
    }
    while (cur >= 0) {
      __syncthreads();  // every wave is done with the rows in LDS
      knn_store_tile<MAXM>(pre, rt, P, pairs, tid);
      __syncthreads();
      int next = -1;
      if (todo != 0ull) {
        next = __ffsll(static_cast<long long>(todo)) - 1;
        todo &= todo - 1ull;
        knn_load_tile<MAXM>(pre, xc, nrm, nullptr, g * kKnnRefTile + ((next + rot) & (kKnnRefTile - 1)), P, pairs,
                            tid);
      } else if (gi + 1 < groups) {
        const int gn = g + 1 < groups ? g + 1 : 0;
        knn_load_tile<MAXM>(pre, tg.centre, tg.cnorm, tg.radius, gn, P, pairs, tid);
      }
      ++staged;
      if ((need >> cur) & 1ull) {
        ++computed;
        v16f acc0, acc1;
        knn_tile_dots(chunks, qrow, rt + c32 * P + 2 * h, rt + (32 + c32) * P + 2 * h, acc0, acc1);
        // filter: s = |r|^2 - 2 q.r below the row's threshold goes to the
        // row's buffer.  Output i of this lane is row 8 (i / 4) + 4 h + i % 4
        // of the wave's 32, reference c32 of the 32-reference block.
        const float nr0 = rt[aux_at + c32];
        const float nr1 = rt[aux_at + 32 + c32];
        const unsigned int col0 =
            static_cast<unsigned int>((g * kKnnRefTile + ((cur + rot) & (kKnnRefTile - 1))) * kKnnRefTile + c32);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int row0 = 8 * g4 + 4 * h;
          const float4 thr4 = *reinterpret_cast<const float4*>(&rs.thr[wave][row0]);
          const float thr_a[4] = {thr4.x, thr4.y, thr4.z, thr4.w};
          float sv[8];
          unsigned long long m[8];
          unsigned long long any = 0ull;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            sv[2 * u] = fmaf(-2.0f, acc0[4 * g4 + u], nr0);
            sv[2 * u + 1] = fmaf(-2.0f, acc1[4 * g4 + u], nr1);
            m[2 * u] = __ballot(sv[2 * u] < thr_a[u]);
            m[2 * u + 1] = __ballot(sv[2 * u + 1] < thr_a[u]);
            any |= m[2 * u] | m[2 * u + 1];
          }
          if (any != 0ull) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              if (m[j] != 0ull) {
                const int row = row0 + j / 2;
                const unsigned int half =
                    h ? static_cast<unsigned int>(m[j] >> 32) : static_cast<unsigned int>(m[j]);
                const int base = rs.cnt[wave][row];
                if (sv[j] < thr_a[j / 2])
                  wave_buf[static_cast<long long>(row) * B + base + __popc(half & ((1u << c32) - 1u))] =
                      make_uint2(ordered_bits(sv[j]), col0 + (j & 1) * 32u);
                if (c32 == 0) rs.cnt[wave][row] = base + __popc(half);
              }
            }
          }
        }
        // rows that could overflow in the next tile: sort, keep kp
        unsigned long long full = __ballot(lane < kKnnWaveQueries && rs.cnt[wave][c32] > B - kKnnRefTile);
        while (full != 0ull) {
          const int r = __ffsll(static_cast<long long>(full)) - 1;
          full &= full - 1ull;
          float thr = rs.thr[wave][r];
          const int c = compact_row<B>(wave_buf + static_cast<long long>(r) * B, rs.cnt[wave][r], kp, lane, &thr);
          if (lane == 0) {
            rs.cnt[wave][r] = c;
            rs.thr[wave][r] = thr;
          }
        }
      }
      cur = next;
    }
  }
  // final: keep kp per row; the threshold is what a rejected reference beat
  for (int r = 0; r < kKnnWaveQueries; ++r) {
    const int p = p0 + wave * kKnnWaveQueries + r;
    if (p >= nq) break;  // wave-uniform
    float thr = rs.thr[wave][r];
    int c = rs.cnt[wave][r];
    if (c > kp) c = compact_row<B>(wave_buf + static_cast<long long>(r) * B, c, kp, lane, &thr);
    if (lane == 0) {
      thr_out[p] = thr;
      cnt_out[p] = c;
    }
  }
  if (lane == 0) {
    if (wave == 0) atomicAdd(&work[0], static_cast<unsigned long long>(staged));
    atomicAdd(&work[1], static_cast<unsigned long long>(computed));
  }
}

// ---- 3. finalize -------------------------------------------------------------------

// One wave per query: exact squared distances of the candidates from the
// input rows (fp64); the query itself is dropped when exclude_self; the rest
// are sorted by (d2, index) and the first k written as 1-based indices and
// float distances, column-major (neighbour j of query i at j * n_out + i).
// Queries are ids in the scan's query set (qperm maps them to query input
// rows, identity when null); candidates are reference positions in scan
// order (rperm maps them to reference input rows).  Uncertified queries are
// appended to retry.
template <int B>
__global__ __launch_bounds__(kKnnThreads) void k_knn_finalize(
    const float* __restrict__ xq_in, Strides stq, const float* __restrict__ xr_in, Strides str, int n_out, int d,
    const int* __restrict__ qperm, const int* __restrict__ rperm, const int* __restrict__ qlist, int q_offset,
    int nq, const uint2* __restrict__ buf, const float* __restrict__ thr_in, const int* __restrict__ cnt_in,
    const float* __restrict__ nrm_q, const unsigned int* __restrict__ nrm_max_bits, float eps_unit, int k,
    int exclude_self, int half_squared, int* __restrict__ idx_out, float* __restrict__ dist_out,
    int* __restrict__ retry, int* __restrict__ retry_count, int* __restrict__ short_rows) {
  constexpr int PER = B / kWave;
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int p = static_cast<int>(blockIdx.x) * kKnnWaves + static_cast<int>(threadIdx.x) / kWave;
  if (p >= nq) return;  // whole wave
  const int qid = query_id(qlist, q_offset, p);
  const int q = qperm != nullptr ? qperm[qid] : qid;
  const int c = cnt_in[p];
  const uint2* cand = buf + static_cast<long long>(p) * B;
  double dd[PER];
  int id[PER];
  bool self_here = false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    dd[j] = INFINITY;
    id[j] = 0x7fffffff;
    if (e < c) {
      const int r = rperm[cand[e].y];
      if (exclude_self && r == q) {
        self_here = true;  // sorts last
      } else {
        double s = 0.0;
        for (int t = 0; t < d; ++t) {
          const double diff = static_cast<double>(xq_in[stq.at(q, t)]) - static_cast<double>(xr_in[str.at(r, t)]);
          s = fma(diff, diff, s);
        }
        dd[j] = s;
        id[j] = r;
      }
    }
  }
  const int valid = c - (__ballot(self_here) != 0ull ? 1 : 0);
  wave_sort_pairs<PER>(dd, id, lane);
  double d2k = 0.0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    if (e < k && e < valid) {
      idx_out[static_cast<long long>(e) * n_out + q] = id[j] + 1;
      dist_out[static_cast<long long>(e) * n_out + q] = static_cast<float>(half_squared ? 0.5 * dd[j] : sqrt(dd[j]));
    }
    if (j == (k - 1) / kWave) d2k = dd[j];
  }
  d2k = __shfl(d2k, (k - 1) % kWave);
  if (lane == 0) {
    if (valid < k) {
      atomicAdd(short_rows, 1);
    } else {
      const float thr = thr_in[p];
      if (thr < INFINITY) {
        const double nq_d = static_cast<double>(nrm_q[qid]);
        const double eps = static_cast<double>(eps_unit) *
                           (nq_d + static_cast<double>(__uint_as_float(*nrm_max_bits)));
        if (!(static_cast<double>(thr) + nq_d - eps > d2k)) retry[atomicAdd(retry_count, 1)] = qid;
      }
    }
  }
}

// ---- full pass for the rows no candidate set certifies -------------------------------
// A row whose k-th neighbour has more than the largest candidate set of
// references within fp32 resolution of it (a zero row under cosine is
// equidistant from every other row), or whose projection bounds its
// distances too loosely, is ranked by a full pass over the references:
// squared distances in fp64 exactly as k_knn_finalize forms them, and the
// (d2, index) pairs below the running k-th kept in an LDS buffer, sorted and
// cut to k whenever the next 256 could overflow it.  Exact by construction
// (nothing below the k-th is ever dropped).  One workgroup per row.
constexpr int kBruteBuf = 2048;

__device__ void brute_sort(double* key, int* ids, int count) {
  for (int e = count + static_cast<int>(threadIdx.x); e < kBruteBuf; e += kKnnThreads) {
    key[e] = INFINITY;
    ids[e] = INT_MAX;
  }
  __syncthreads();
  for (int size = 2; size <= kBruteBuf; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      for (int e = threadIdx.x; e < kBruteBuf / 2; e += kKnnThreads) {
        const int lo = 2 * e - (e & (dist - 1));
        const int hi = lo + dist;
        const bool asc = (lo & size) == 0;
        const double ka = key[lo], kb = key[hi];
        const int ia = ids[lo], ib = ids[hi];
        const bool a_gt = ka > kb || (ka == kb && ia > ib);
        if (a_gt == asc) {
          key[lo] = kb;
          key[hi] = ka;
          ids[lo] = ib;
          ids[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kKnnThreads) void k_knn_brute(const int* __restrict__ list,
                                                           const float* __restrict__ xq_in, Strides stq,
                                                           const float* __restrict__ xr_in, Strides str, int n_ref,
                                                           int d, const int* __restrict__ qperm, int k,
                                                           int exclude_self, int half_squared, int n_out,
                                                           int* __restrict__ idx_out, float* __restrict__ dist_out) {
  __shared__ double key[kBruteBuf];
  __shared__ int ids[kBruteBuf];
  __shared__ int count;
  __shared__ double tau_d;
  __shared__ int tau_i;
  const int tid = static_cast<int>(threadIdx.x);
  const int qid = list[blockIdx.x];
  const int q = qperm != nullptr ? qperm[qid] : qid;
  if (tid == 0) {
    count = 0;
    tau_d = INFINITY;
    tau_i = INT_MAX;
  }
  __syncthreads();
  for (int j0 = 0; j0 < n_ref; j0 += kKnnThreads) {
    const int r = j0 + tid;
    if (r < n_ref && !(exclude_self && r == q)) {
      double s = 0.0;
      for (int t = 0; t < d; ++t) {
        const double diff = static_cast<double>(xq_in[stq.at(q, t)]) - static_cast<double>(xr_in[str.at(r, t)]);
        s = fma(diff, diff, s);
      }
      if (s < tau_d || (s == tau_d && r < tau_i)) {
        const int slot = atomicAdd(&count, 1);
        key[slot] = s;
        ids[slot] = r;
      }
    }
    __syncthreads();
    if (count > kBruteBuf - kKnnThreads) {  // block-uniform
      brute_sort(key, ids, count);
      if (tid == 0) {
        count = k;
        tau_d = key[k - 1];
        tau_i = ids[k - 1];
      }
    }
    __syncthreads();
  }
  const int c = count;
  brute_sort(key, ids, c);
  for (int e = tid; e < k && e < c; e += kKnnThreads) {
    idx_out[static_cast<long long>(e) * n_out + q] = ids[e] + 1;
    dist_out[static_cast<long long>(e) * n_out + q] = static_cast<float>(half_squared ? 0.5 * key[e] : sqrt(key[e]));
  }
}

// Rows times references times dimensions up to which the rows left
// uncertified by the largest candidate set go through k_knn_brute (about a
// second); beyond it the call fails rather than run for minutes.
constexpr double kBruteBudget = 2e11;

// Everything one scan + finalize pass over a list of queries needs.
struct KnnPass {
  const float* xq_in;  // query input rows (strides stq)
  Strides stq;
  const float* xr_in;  // reference input rows (strides str)
  Strides str;
  const int* qperm;    // query id -> query input row (null: identity)
  const int* rperm;    // reference scan position -> reference input row
  const float* xr;     // centred references in scan order, pitch P, cells padded to whole tiles
  const float* nrm_r;  // their squared norms (+inf on padding)
  TileGroups tg;       // bounding spheres of their 64-row tiles
  const float* xq;     // centred queries by query id, pitch P
  const float* nrm_q;  // their squared norms
  const int* home;     // query id -> home tile (null: id / 64, the query is a reference position)
  const unsigned int* nrm_max_bits;
  int n_out;   // rows of the output (queries)
  int n_scan;  // reference scan positions
  int d, P, chunks, k, exclude_self;
  int proj_slack;  // certificate margin for projected rows, in units of 2^-23 (|q|^2 + max |r|^2)
  int half_squared;  // distances written as d^2 / 2 (cosine, correlation) instead of d
  uint2* buf;  // candidate buffers, nq x B
  float* thr;
  int* cnt;
  int* idx_out;
  float* dist_out;
  int* retry;        // uncertified query ids
  int* retry_count;  // counters[0]
  int* short_rows;   // counters[1]
  unsigned long long* work;  // [0] tiles staged (per block), [1] tiles computed (per wave)
};

template <int B, int MAXM>
hipError_t launch_scan(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq, hipStream_t stream) {
  const std::size_t lds = static_cast<std::size_t>(knn_scan_lds_floats(a.P)) * sizeof(float);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_knn_scan<B, MAXM>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (e != hipSuccess) return e;
  const int blocks = (nq + kKnnQueryBlock - 1) / kKnnQueryBlock;
  const float eps_lb = static_cast<float>(4 * a.chunks + 8) * 0x1.0p-23f;
  k_knn_scan<B, MAXM><<<blocks, kKnnThreads, lds, stream>>>(a.xr, a.nrm_r, a.tg, a.xq, a.nrm_q, a.home, qlist,
                                                            q_offset, nq, a.n_scan, a.P, a.chunks, kp, eps_lb, a.buf,
                                                            a.thr, a.cnt, a.work);
  return hipGetLastError();
}

template <int B>
hipError_t launch_scan_finalize(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq,
                                hipStream_t stream) {
  static_assert(kKnnMaxDim <= 4 * 32, "at most 32 chunks of 4 dimensions");
  hipError_t e = a.chunks <= 16 ? launch_scan<B, 16>(a, kp, qlist, q_offset, nq, stream)
                                : launch_scan<B, 32>(a, kp, qlist, q_offset, nq, stream);
  if (e != hipSuccess) return e;
  const float eps_unit = static_cast<float>(4 * a.chunks + 12 + a.proj_slack) * 0x1.0p-23f;
  k_knn_finalize<B><<<(nq + kKnnWaves - 1) / kKnnWaves, kKnnThreads, 0, stream>>>(
      a.xq_in, a.stq, a.xr_in, a.str, a.n_out, a.d, a.qperm, a.rperm, qlist, q_offset, nq, a.buf, a.thr, a.cnt,
      a.nrm_q, a.nrm_max_bits, eps_unit, a.k, a.exclude_self, a.half_squared, a.idx_out, a.dist_out, a.retry,
      a.retry_count,
      a.short_rows);
  return hipGetLastError();
}

// Candidates per query: k plus a margin of max(32, k / 2) (plus the query
// itself, which the scan does not skip) on the first pass, doubled for every
// rerun, at most kKnnMaxCand.
constexpr int kKnnMaxCand = 1024 - 2 * kKnnRefTile;  // 896

// Smallest buffer with room for kp entries plus at least kp new ones (and a
// tile's 64) between compactions; 1024 for the largest kp.
int buffer_for(int kp) {
  for (int B = 128; B <= 1024; B <<= 1)
    if (B - kKnnRefTile >= 2 * kp) return B;
  return 1024;
}

hipError_t launch_pass(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq, hipStream_t stream) {
#define FEHIP_KNN_PASS(B_) \
  case B_:                 \
    return launch_scan_finalize<B_>(a, kp, qlist, q_offset, nq, stream);
  switch (buffer_for(kp)) {
    FEHIP_KNN_PASS(128)
    FEHIP_KNN_PASS(256)
    FEHIP_KNN_PASS(512)
    FEHIP_KNN_PASS(1024)
    default:
      return hipErrorInvalidValue;
  }
#undef FEHIP_KNN_PASS
}

template <typename T>
struct DevBuf {
  T* p = nullptr;
  hipError_t alloc(std::size_t count) {
    return hipMalloc(reinterpret_cast<void**>(&p), std::max<std::size_t>(count, 1) * sizeof(T));
  }
  ~DevBuf() {
    if (p != nullptr) (void)hipFree(p);
  }
};

// A matrix handed to the KNN entry points.
struct KnnSet {
  const float* x;
  int n;
  int col_major;
  int on_device;
};

// Uniform 64-bit stream (SplitMix64) and standard normals from it
// (Box-Muller), for the power iterations' fixed start.
struct ProjRng {
  std::uint64_t s;
  std::uint64_t next() {
    std::uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double uniform() { return (static_cast<double>(next() >> 11) + 0.5) * 0x1.0p-53; }
  double normal() { return std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()); }
};

// Orthonormal columns for the d x kProjDim row-major matrix y (modified
// Gram-Schmidt, two passes, fp64).  A column left without a direction of its
// own (the data's rank below kProjDim) is redrawn at random.
void proj_orthonormalize(std::vector<double>& y, int d, ProjRng& rng) {
  constexpr int m = kProjDim;
  for (int j = 0; j < m; ++j) {
    for (;;) {
      double before = 0.0;
      for (int i = 0; i < d; ++i) before += y[static_cast<std::size_t>(i) * m + j] * y[static_cast<std::size_t>(i) * m + j];
      for (int pass = 0; pass < 2; ++pass) {
        for (int k = 0; k < j; ++k) {
          double dot = 0.0;
          for (int i = 0; i < d; ++i) dot += y[static_cast<std::size_t>(i) * m + k] * y[static_cast<std::size_t>(i) * m + j];
          for (int i = 0; i < d; ++i) y[static_cast<std::size_t>(i) * m + j] -= dot * y[static_cast<std::size_t>(i) * m + k];
        }
      }
      double after = 0.0;
      for (int i = 0; i < d; ++i) after += y[static_cast<std::size_t>(i) * m + j] * y[static_cast<std::size_t>(i) * m + j];
      if (after > 1e-20 * before && after > 0.0 && std::isfinite(after)) {
        const double inv = 1.0 / std::sqrt(after);
        for (int i = 0; i < d; ++i) y[static_cast<std::size_t>(i) * m + j] *= inv;
        break;
      }
      for (int i = 0; i < d; ++i) y[static_cast<std::size_t>(i) * m + j] = rng.normal();
    }
  }
}

// Q (d x kProjDim, orthonormal columns, on the device) spanning the leading
// principal directions of the rows of x: covariance of up to kProjSample
// evenly spaced rows, then kProjIters block power iterations from a fixed
// random start, each followed by an orthonormalisation on the host.
constexpr int kProjSample = 32768;
constexpr int kProjIters = 4;

hipError_t knn_projection_basis(const float* x, Strides st, int n, int d, const double* mean, double* q_dev,
                                hipStream_t stream) {
  const int m = std::min(n, kProjSample);
  const long long stride = std::max(1, n / m);
  DevBuf<double> cov, y_dev;
  hipError_t e;
  if ((e = cov.alloc(static_cast<std::size_t>(d) * d)) != hipSuccess ||
      (e = y_dev.alloc(static_cast<std::size_t>(d) * kProjDim)) != hipSuccess)
    return e;
  const int tiles = (d + kCovTile - 1) / kCovTile;
  k_knn_cov<<<dim3(tiles, tiles), 256, 0, stream>>>(x, st, d, mean, m, stride, cov.p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  std::vector<double> q(static_cast<std::size_t>(d) * kProjDim);
  ProjRng rng{0x6b6e6e70726f6aull};
  for (double& v : q) v = rng.normal();
  proj_orthonormalize(q, d, rng);
  const std::size_t bytes = q.size() * sizeof(double);
  for (int it = 0; it < kProjIters; ++it) {
    if ((e = hipMemcpyAsync(q_dev, q.data(), bytes, hipMemcpyHostToDevice, stream)) != hipSuccess) return e;
    k_knn_cov_times<<<d, kProjDim, 0, stream>>>(cov.p, q_dev, d, y_dev.p);
    if ((e = hipGetLastError()) != hipSuccess ||
        (e = hipMemcpyAsync(q.data(), y_dev.p, bytes, hipMemcpyDeviceToHost, stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return e;
    proj_orthonormalize(q, d, rng);
  }
  if ((e = hipMemcpyAsync(q_dev, q.data(), bytes, hipMemcpyHostToDevice, stream)) != hipSuccess) return e;
  return hipStreamSynchronize(stream);
}

// The whole search: references `ref`, queries `query` (null: the references
// themselves, self excluded on request).
int knn_run(const KnnSet& ref, const KnnSet* query, int d, int k, int exclude_self, int metric, int* idx_out_in,
            float* dist_out_in, int output_on_device, long long* stats, std::string& err) {
  auto fail = [&](const std::string& what, hipError_t e) {
    err = what + ": " + hipGetErrorString(e);
    return 1;
  };
  const bool self = query == nullptr;
  const int n = ref.n;
  const int n_out = self ? n : query->n;
  const bool project = d > kKnnMaxDim;         // scan a kProjDim-dimensional projection
  const int ds = project ? kProjDim : d;       // scanned dimensions
  const int P = knn_pitch(ds);
  const int chunks = (ds + 3) / 4;
  const int n_pad = (n + kKnnRefTile - 1) / kKnnRefTile * kKnnRefTile;  // whole reference tiles
  hipStream_t stream = nullptr;
  hipError_t e;
  DevBuf<float> xr_dev, xq_dev, xc, nrm, xcq, nrmq, dist_dev;
  DevBuf<double> partial, mean, basis;
  DevBuf<unsigned int> nrm_max;
  DevBuf<int> idx_dev, retry, counters;
  auto upload = [&](const KnnSet& set, DevBuf<float>& dev, const float*& out) -> hipError_t {
    out = set.x;
    if (set.on_device) return hipSuccess;
    const std::size_t bytes = static_cast<std::size_t>(set.n) * d * sizeof(float);
    hipError_t r = dev.alloc(static_cast<std::size_t>(set.n) * d);
    if (r == hipSuccess) r = hipMemcpy(dev.p, set.x, bytes, hipMemcpyHostToDevice);
    out = dev.p;
    return r;
  };
  const float* xr = nullptr;
  const float* xq = nullptr;
  if ((e = upload(ref, xr_dev, xr)) != hipSuccess) return fail("KNN reference upload", e);
  if (!self && (e = upload(*query, xq_dev, xq)) != hipSuccess) return fail("KNN query upload", e);
  // cosine / correlation: the search runs on the normalised rows (row-major)
  DevBuf<float> xr_unit, xq_unit;
  bool ref_col_major = ref.col_major != 0;
  bool query_col_major = !self && query->col_major != 0;
  if (metric != kKnnEuclidean) {
    const int center = metric == kKnnCorrelation ? 1 : 0;
    if ((e = xr_unit.alloc(static_cast<std::size_t>(n) * d)) != hipSuccess ||
        (!self && (e = xq_unit.alloc(static_cast<std::size_t>(n_out) * d)) != hipSuccess))
      return fail("hipMalloc(KNN normalised rows)", e);
    k_knn_normalize_rows<<<(n + kPrepThreads - 1) / kPrepThreads, kPrepThreads, 0, stream>>>(
        xr, n, d, ref_col_major ? Strides{1, n} : Strides{d, 1}, center, xr_unit.p);
    xr = xr_unit.p;
    ref_col_major = false;
    if (!self) {
      k_knn_normalize_rows<<<(n_out + kPrepThreads - 1) / kPrepThreads, kPrepThreads, 0, stream>>>(
          xq, n_out, d, query_col_major ? Strides{1, n_out} : Strides{d, 1}, center, xq_unit.p);
      xq = xq_unit.p;
      query_col_major = false;
    }
    if ((e = hipGetLastError()) != hipSuccess) return fail("KNN normalisation launch", e);
  }
  int* idx_out = idx_out_in;
  float* dist_out = dist_out_in;
  if (!output_on_device) {
    if ((e = idx_dev.alloc(static_cast<std::size_t>(n_out) * k)) != hipSuccess)
      return fail("hipMalloc(KNN indices)", e);
    if ((e = dist_dev.alloc(static_cast<std::size_t>(n_out) * k)) != hipSuccess)
      return fail("hipMalloc(KNN distances)", e);
    idx_out = idx_dev.p;
    dist_out = dist_dev.p;
  }
  const int rows_per = 4096;
  const int pblocks = (n + rows_per - 1) / rows_per;
  if ((e = xc.alloc(static_cast<std::size_t>(n_pad) * P + kKnnOverRead)) != hipSuccess ||
      (e = nrm.alloc(n_pad)) != hipSuccess ||
      (e = partial.alloc(static_cast<std::size_t>(pblocks) * d)) != hipSuccess || (e = mean.alloc(d)) != hipSuccess ||
      (e = nrm_max.alloc(2)) != hipSuccess || (e = retry.alloc(n_out)) != hipSuccess ||
      (e = counters.alloc(3)) != hipSuccess)
    return fail("hipMalloc(KNN scratch)", e);
  if (!self && ((e = xcq.alloc(static_cast<std::size_t>(n_out) * P + kKnnOverRead)) != hipSuccess ||
                (e = nrmq.alloc(n_out)) != hipSuccess))
    return fail("hipMalloc(KNN query scratch)", e);
  // counters: [0] uncertified rows, [1] rows with fewer than k candidates,
  // [2] rows with non-finite values; nrm_max: [0] references, [1] queries
  if ((e = hipMemsetAsync(counters.p, 0, 3 * sizeof(int), stream)) != hipSuccess ||
      (e = hipMemsetAsync(nrm_max.p, 0, 2 * sizeof(unsigned int), stream)) != hipSuccess ||
      (e = hipMemsetAsync(xc.p + static_cast<std::size_t>(n_pad) * P, 0, kKnnOverRead * sizeof(float), stream)) !=
          hipSuccess)
    return fail("hipMemset", e);
  const Strides str = ref_col_major ? Strides{1, n} : Strides{d, 1};
  const Strides stq = self ? str : (query_col_major ? Strides{1, n_out} : Strides{d, 1});
  // both sets are centred on the references' column means (and projected
  // on the references' leading directions when wider than kKnnMaxDim)
  k_knn_col_partials<<<pblocks, kPrepThreads, 0, stream>>>(xr, n, d, str, rows_per, partial.p);
  k_knn_col_means<<<1, kPrepThreads, 0, stream>>>(partial.p, pblocks, d, n, mean.p);
  if (project) {
    if ((e = basis.alloc(static_cast<std::size_t>(d) * kProjDim)) != hipSuccess) return fail("hipMalloc(KNN basis)", e);
    if ((e = knn_projection_basis(xr, str, n, d, mean.p, basis.p, stream)) != hipSuccess)
      return fail("KNN projection basis", e);
    k_knn_project<<<(n_pad + kProjRows - 1) / kProjRows, 256, 0, stream>>>(xr, n, n_pad, d, str, P, mean.p, basis.p,
                                                                          xc.p, nrm.p, nrm_max.p, counters.p + 2);
  } else {
    k_knn_center<<<(n_pad + kPrepThreads - 1) / kPrepThreads, kPrepThreads, 0, stream>>>(
        xr, n, n_pad, d, str, P, mean.p, xc.p, nrm.p, nrm_max.p, counters.p + 2);
  }
  if (!self) {
    if ((e = hipMemsetAsync(xcq.p + static_cast<std::size_t>(n_out) * P, 0, kKnnOverRead * sizeof(float), stream)) !=
        hipSuccess)
      return fail("hipMemset", e);
    if (project) {
      k_knn_project<<<(n_out + kProjRows - 1) / kProjRows, 256, 0, stream>>>(
          xq, n_out, n_out, d, stq, P, mean.p, basis.p, xcq.p, nrmq.p, nrm_max.p + 1, counters.p + 2);
    } else {
      k_knn_center<<<(n_out + kPrepThreads - 1) / kPrepThreads, kPrepThreads, 0, stream>>>(
          xq, n_out, n_out, d, stq, P, mean.p, xcq.p, nrmq.p, nrm_max.p + 1, counters.p + 2);
    }
  }
  if ((e = hipGetLastError()) != hipSuccess) return fail("KNN prep launch", e);
  {
    int bad = 0;
    if ((e = hipMemcpyAsync(&bad, counters.p + 2, sizeof(int), hipMemcpyDeviceToHost, stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return fail("KNN prep", e);
    if (bad != 0) {
      err = "exact KNN input has " + std::to_string(bad) +
            " rows with non-finite values (or a centred squared norm beyond the fp32 range)";
      return 1;
    }
  }

  // Locality order: each reference goes to the cell of its nearest pivot;
  // cells are laid out one after another, each padded to whole 64-row tiles.
  // Separate queries are ordered by the same cells.
  const int C = std::max(1, std::min(1024, n / 256));
  const int stride = n / C;
  const int scan_max = n_pad + C * kKnnRefTile;  // bound on the scan positions
  DevBuf<int> cell, cursor, pad_off, real_off, perm, qpos, qcell, qreal_off, qpad_off, qorder, qhome;
  DevBuf<float> xs, ns;
  if ((e = cell.alloc(n)) != hipSuccess || (e = cursor.alloc(C)) != hipSuccess ||
      (e = pad_off.alloc(C + 1)) != hipSuccess || (e = real_off.alloc(C)) != hipSuccess ||
      (e = perm.alloc(scan_max)) != hipSuccess || (e = qpos.alloc(n)) != hipSuccess ||
      (e = xs.alloc(static_cast<std::size_t>(scan_max) * P + kKnnOverRead)) != hipSuccess ||
      (e = ns.alloc(scan_max)) != hipSuccess)
    return fail("hipMalloc(KNN order)", e);
  if (!self && ((e = qcell.alloc(n_out)) != hipSuccess || (e = qreal_off.alloc(C)) != hipSuccess ||
                (e = qpad_off.alloc(C + 1)) != hipSuccess || (e = qorder.alloc(n_out)) != hipSuccess ||
                (e = qhome.alloc(n_out)) != hipSuccess))
    return fail("hipMalloc(KNN query order)", e);
  int n_scan = 0;
  {
    const int rb = (n + kPrepThreads - 1) / kPrepThreads;
    if ((e = hipMemsetAsync(cursor.p, 0, C * sizeof(int), stream)) != hipSuccess ||
        (e = hipMemsetAsync(perm.p, 0xff, scan_max * sizeof(int), stream)) != hipSuccess)
      return fail("hipMemset", e);
    if (P <= 68)
      k_knn_assign<68><<<rb, kPrepThreads, 0, stream>>>(xc.p, n, xc.p, nrm.p, P, C, stride, cell.p);
    else
      k_knn_assign<132><<<rb, kPrepThreads, 0, stream>>>(xc.p, n, xc.p, nrm.p, P, C, stride, cell.p);
    k_knn_cell_count<<<rb, kPrepThreads, 0, stream>>>(cell.p, n, cursor.p);
    k_knn_cell_offsets<<<1, 64, 0, stream>>>(cursor.p, C, pad_off.p, real_off.p);
    if ((e = hipGetLastError()) != hipSuccess ||
        (e = hipMemsetAsync(cursor.p, 0, C * sizeof(int), stream)) != hipSuccess)
      return fail("KNN order launch", e);
    k_knn_cell_scatter<<<rb, kPrepThreads, 0, stream>>>(cell.p, n, cursor.p, pad_off.p, real_off.p, perm.p, qpos.p);
    if (!self) {
      const int qb = (n_out + kPrepThreads - 1) / kPrepThreads;
      if ((e = hipMemsetAsync(cursor.p, 0, C * sizeof(int), stream)) != hipSuccess) return fail("hipMemset", e);
      if (P <= 68)
        k_knn_assign<68><<<qb, kPrepThreads, 0, stream>>>(xcq.p, n_out, xc.p, nrm.p, P, C, stride, qcell.p);
      else
        k_knn_assign<132><<<qb, kPrepThreads, 0, stream>>>(xcq.p, n_out, xc.p, nrm.p, P, C, stride, qcell.p);
      k_knn_cell_count<<<qb, kPrepThreads, 0, stream>>>(qcell.p, n_out, cursor.p);
      k_knn_cell_offsets<<<1, 64, 0, stream>>>(cursor.p, C, qpad_off.p, qreal_off.p);
      if ((e = hipGetLastError()) != hipSuccess ||
          (e = hipMemsetAsync(cursor.p, 0, C * sizeof(int), stream)) != hipSuccess)
        return fail("KNN query order launch", e);
      k_knn_query_scatter<<<qb, kPrepThreads, 0, stream>>>(qcell.p, n_out, cursor.p, qreal_off.p, pad_off.p,
                                                            qorder.p, qhome.p);
    }
    if ((e = hipMemcpyAsync(&n_scan, pad_off.p + C, sizeof(int), hipMemcpyDeviceToHost, stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return fail("KNN order", e);
    if (n_scan < n || n_scan > scan_max || n_scan % kKnnRefTile != 0) {
      err = "exact KNN: inconsistent cell layout";
      return 1;
    }
    const long long pairs = static_cast<long long>(n_scan) * (P / 2);
    k_knn_permute<<<static_cast<unsigned int>((pairs + kPrepThreads - 1) / kPrepThreads), kPrepThreads, 0, stream>>>(
        xc.p, nrm.p, perm.p, n_scan, P, xs.p, ns.p);
    if ((e = hipGetLastError()) != hipSuccess ||
        (e = hipMemsetAsync(xs.p + static_cast<std::size_t>(n_scan) * P, 0, kKnnOverRead * sizeof(float), stream)) !=
            hipSuccess)
      return fail("KNN order launch", e);
  }
  // tile bounding spheres, for whole groups of 64 tiles
  const int tiles = n_scan / kKnnRefTile;
  const int tiles_pad = (tiles + kKnnRefTile - 1) / kKnnRefTile * kKnnRefTile;
  DevBuf<float> tcentre, tcnorm, tradius;
  if ((e = tcentre.alloc(static_cast<std::size_t>(tiles_pad) * P + kKnnOverRead)) != hipSuccess ||
      (e = tcnorm.alloc(tiles_pad)) != hipSuccess || (e = tradius.alloc(tiles_pad)) != hipSuccess)
    return fail("hipMalloc(KNN tile bounds)", e);
  if ((e = hipMemsetAsync(tcentre.p + static_cast<std::size_t>(tiles_pad) * P, 0, kKnnOverRead * sizeof(float),
                          stream)) != hipSuccess)
    return fail("hipMemset", e);
  k_knn_tile_bounds<<<tiles_pad, kKnnRefTile, 0, stream>>>(xs.p, ns.p, n_scan, P, tcentre.p, tcnorm.p, tradius.p);
  if ((e = hipGetLastError()) != hipSuccess) return fail("KNN tile bounds launch", e);

  // Candidate buffers: B entries per query of a launch, at most
  // kKnnCandEntries in all; a pass launches as many queries at once as they
  // allow (one launch for the whole input up to millions of rows, so that
  // the grid is many rounds of workgroups deep).
  // (projected rows: the bound is looser by the spread outside the
  // projection, so the first pass starts with twice the margin)
  int kp = std::min(kKnnMaxCand, k + (project ? 2 : 1) * std::max(32, k / 2) + (self ? 1 : 0));
  const std::size_t entries = std::min<std::size_t>(
      kKnnCandEntries, static_cast<std::size_t>(n_out) * static_cast<std::size_t>(buffer_for(kp)));
  auto batch_for = [&](int kp_) {
    return static_cast<int>(std::min<std::size_t>(static_cast<std::size_t>(n_out), entries / buffer_for(kp_)));
  };
  DevBuf<uint2> buf;
  DevBuf<float> thr;
  DevBuf<int> cnt;
  if ((e = buf.alloc(entries)) != hipSuccess || (e = thr.alloc(n_out)) != hipSuccess ||
      (e = cnt.alloc(n_out)) != hipSuccess)
    return fail("hipMalloc(KNN candidates)", e);
  DevBuf<unsigned long long> work;
  if ((e = work.alloc(2)) != hipSuccess) return fail("hipMalloc(KNN work)", e);
  if ((e = hipMemsetAsync(work.p, 0, 2 * sizeof(unsigned long long), stream)) != hipSuccess)
    return fail("hipMemset", e);
  KnnPass pass{};
  pass.xq_in = self ? xr : xq;
  pass.stq = stq;
  pass.xr_in = xr;
  pass.str = str;
  pass.qperm = self ? perm.p : nullptr;
  pass.rperm = perm.p;
  pass.xr = xs.p;
  pass.nrm_r = ns.p;
  pass.tg = TileGroups{tcentre.p, tcnorm.p, tradius.p};
  pass.xq = self ? xs.p : xcq.p;
  pass.nrm_q = self ? ns.p : nrmq.p;
  pass.home = self ? nullptr : qhome.p;
  pass.nrm_max_bits = nrm_max.p;
  pass.n_out = n_out;
  pass.n_scan = n_scan;
  pass.d = d;
  pass.P = P;
  pass.chunks = chunks;
  pass.proj_slack = project ? kProjSlack : 0;
  pass.half_squared = metric != kKnnEuclidean ? 1 : 0;
  pass.k = k;
  pass.exclude_self = self ? exclude_self : 0;
  pass.buf = buf.p;
  pass.thr = thr.p;
  pass.cnt = cnt.p;
  pass.idx_out = idx_out;
  pass.dist_out = dist_out;
  pass.retry = retry.p;
  pass.retry_count = counters.p;
  pass.short_rows = counters.p + 1;
  pass.work = work.p;
  const int* main_list = self ? qpos.p : qorder.p;
  for (int q0 = 0, batch = batch_for(kp); q0 < n_out; q0 += batch) {
    const int nq = std::min(batch, n_out - q0);
    if ((e = launch_pass(pass, kp, main_list + q0, 0, nq, stream)) != hipSuccess) return fail("KNN scan launch", e);
  }
  int host_counts[2] = {0, 0};
  long long retried = 0;
  int passes = 1;
  for (;;) {
    if ((e = hipMemcpyAsync(host_counts, counters.p, sizeof(host_counts), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return fail("KNN pass", e);
    if (host_counts[1] != 0) {
      err = "exact KNN found fewer candidates than k for " + std::to_string(host_counts[1]) + " rows";
      return 1;
    }
    if (host_counts[0] == 0) break;
    if (kp == kKnnMaxCand) {
      const int nr = host_counts[0];
      if (static_cast<double>(nr) * n * d <= kBruteBudget) {
        // the rest by a full pass each
        k_knn_brute<<<nr, kKnnThreads, 0, stream>>>(retry.p, pass.xq_in, pass.stq, pass.xr_in, pass.str, n, d,
                                                     pass.qperm, k, pass.exclude_self, pass.half_squared, n_out,
                                                     idx_out, dist_out);
        if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(stream)) != hipSuccess)
          return fail("KNN full pass", e);
        retried += nr;
        ++passes;
        break;
      }
      if (project) {
        err = "exact KNN could not certify " + std::to_string(nr) + " rows of " + std::to_string(d) +
              " dimensions: their projection on " + std::to_string(kProjDim) +
              " leading directions, which the search scans, keeps too little of their spread to bound the k-th "
              "neighbour within " +
              std::to_string(kKnnMaxCand) + " candidates (nearly isotropic data), and a full pass over " +
              std::to_string(n) + " references for each would exceed the time budget; reduce the dimension first";
      } else {
        err = "exact KNN could not certify " + std::to_string(nr) + " rows: more than " +
              std::to_string(kKnnMaxCand) + " points lie within fp32 resolution of their k-th neighbour distance, "
              "and a full pass for each would exceed the time budget";
      }
      return 1;
    }
    // rerun the uncertified rows with twice the candidates
    retried += host_counts[0];
    ++passes;
    kp = std::min(kKnnMaxCand, 2 * kp);
    DevBuf<int> list;
    const int nr = host_counts[0];
    if ((e = list.alloc(nr)) != hipSuccess) return fail("hipMalloc(KNN retry)", e);
    if ((e = hipMemcpyAsync(list.p, retry.p, nr * sizeof(int), hipMemcpyDeviceToDevice, stream)) != hipSuccess ||
        (e = hipMemsetAsync(counters.p, 0, 2 * sizeof(int), stream)) != hipSuccess)
      return fail("KNN retry setup", e);
    for (int q0 = 0, batch = batch_for(kp); q0 < nr; q0 += batch) {
      const int nq = std::min(batch, nr - q0);
      if ((e = launch_pass(pass, kp, list.p + q0, 0, nq, stream)) != hipSuccess) return fail("KNN retry launch", e);
    }
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return fail("KNN retry", e);
  }
  if (!output_on_device) {
    if ((e = hipMemcpy(idx_out_in, idx_out, static_cast<std::size_t>(n_out) * k * sizeof(int),
                       hipMemcpyDeviceToHost)) != hipSuccess ||
        (e = hipMemcpy(dist_out_in, dist_out, static_cast<std::size_t>(n_out) * k * sizeof(float),
                       hipMemcpyDeviceToHost)) != hipSuccess)
      return fail("hipMemcpy(KNN output)", e);
  } else if ((e = hipStreamSynchronize(stream)) != hipSuccess) {
    return fail("KNN sync", e);
  }
  if (stats != nullptr) {
    unsigned long long w[2] = {0, 0};
    if ((e = hipMemcpy(w, work.p, sizeof(w), hipMemcpyDeviceToHost)) != hipSuccess) return fail("KNN stats", e);
    stats[0] = retried;
    stats[1] = passes;
    stats[2] = kp;
    stats[3] = static_cast<long long>(w[0]);
    stats[4] = static_cast<long long>(w[1]);
  }
  return 0;
}

bool knn_common_checks(const float* x, int n, int d, int k, int metric, const void* idx, const void* dist,
                       std::string& err) {
  if (x == nullptr || idx == nullptr || dist == nullptr) {
    err = "null KNN pointer";
    return false;
  }
  if (metric != kKnnEuclidean && metric != kKnnCosine && metric != kKnnCorrelation) {
    err = "Native HIP KNN does not support this metric (euclidean, cosine or correlation)";
    return false;
  }
  if (n < 1 || d < 1 || k < 1) {
    err = "invalid KNN dimensions (need n >= 1, d >= 1, k >= 1)";
    return false;
  }
  if (d > kKnnMaxInputDim) {
    err = "exact KNN supports up to " + std::to_string(kKnnMaxInputDim) + " dimensions";
    return false;
  }
  if (k > kKnnMaxK) {
    err = "exact KNN supports k up to " + std::to_string(kKnnMaxK);
    return false;
  }
  if (n > INT_MAX - (1 << 17)) {
    err = "exact KNN supports fewer than 2^31 - 2^17 rows";
    return false;
  }
  return true;
}

}  // namespace

int knn_exact_run(const float* x_in, int n, int d, int x_col_major, int k, int exclude_self, int metric,
                  int input_on_device, int* idx_out_in, float* dist_out_in, int output_on_device, long long* stats,
                  std::string& err) {
  if (!knn_common_checks(x_in, n, d, k, metric, idx_out_in, dist_out_in, err)) return 1;
  if (n < 2) {
    err = "invalid KNN dimensions (need n >= 2, d >= 1, k >= 1)";
    return 1;
  }
  if (k > n - (exclude_self ? 1 : 0)) {
    err = "k exceeds the number of " + std::string(exclude_self ? "non-self " : "") + "neighbors";
    return 1;
  }
  const KnnSet ref{x_in, n, x_col_major, input_on_device};
  return knn_run(ref, nullptr, d, k, exclude_self, metric, idx_out_in, dist_out_in, output_on_device, stats, err);
}

int knn_query_run(const float* ref_in, int n_ref, const float* query_in, int n_query, int d, int col_major, int k,
                  int metric, int input_on_device, int* idx_out, float* dist_out, int output_on_device,
                  long long* stats, std::string& err) {
  if (!knn_common_checks(ref_in, n_ref, d, k, metric, idx_out, dist_out, err)) return 1;
  if (query_in == nullptr) {
    err = "null KNN pointer";
    return 1;
  }
  if (n_query < 1 || n_query > INT_MAX - (1 << 17)) {
    err = "invalid query count";
    return 1;
  }
  if (k > n_ref) {
    err = "k exceeds the number of reference rows";
    return 1;
  }
  const KnnSet ref{ref_in, n_ref, col_major, input_on_device};
  const KnnSet query{query_in, n_query, col_major, input_on_device};
  return knn_run(ref, &query, d, k, 0, metric, idx_out, dist_out, output_on_device, stats, err);
}

}  // namespace fehip
