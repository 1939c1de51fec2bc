// Exact rank-based structure metrics of an embedding on gfx950: the
// reference's exact_structure_metrics_cpp (src/embedding_utils.cpp:1582-1752)
// on the device.  For a sample of n <= 5000 rows of the high-dimensional data
// and of the layout (both column-major fp64, R's matrix order), every row is
// ranked against all others in both spaces by squared distance, ties by
// index; for each requested k the k nearest in each space give
//   shared      #(low neighbours with high rank <= k)
//   trust       sum over low neighbours of (high rank - k) when > k
//   continuity  sum over high neighbours of (low rank - k) when > k
//   rank error  sum over the low neighbours at position r of |high rank - r|
// and trustworthiness = 1 - 2 trust / (n k (2n - 3k - 1)) (clamped to [0, 1]),
// continuity likewise, knn preservation = shared / (n k), mean neighbour rank
// error = rank error / (n k).
//
// One workgroup per row: its squared distances in each space are formed in
// fp64 with the reference's operation order (a sequential sum over columns of
// the rounded squares, no fused multiply-add), so they are bit-identical to
// the reference's; the (d2, index) pairs are sorted in LDS (bitonic), ranks
// scattered to LDS, and the row's integer-valued sums written.  The host adds
// the rows' sums (exact: integers below 2^53) and applies the formulas.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "metrics_device.h"

namespace fehip {
namespace {

constexpr int kMetThreads = 256;

// Squared distance between rows i and j of a column-major n x p matrix, in
// the reference's order: d2 = ((0 + a0^2) + a1^2) + ..., each square rounded.
__device__ __forceinline__ double row_d2(const double* __restrict__ x, int n, int p, int i, int j) {
  double d2 = 0.0;
  for (int c = 0; c < p; ++c) {
    const long long off = static_cast<long long>(c) * n;
    const double delta = __dsub_rn(x[off + i], x[off + j]);
    d2 = __dadd_rn(d2, __dmul_rn(delta, delta));
  }
  return d2;
}

// Ascending bitonic sort of m (a power of two) (key, index) pairs in LDS,
// lexicographic; every thread of the block takes part.
__device__ void lds_sort_pairs(double* key, int* idx, int m) {
  for (int size = 2; size <= m; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      for (int e = threadIdx.x; e < m / 2; e += kMetThreads) {
        const int lo = 2 * e - (e & (dist - 1));  // element whose partner is lo + dist
        const int hi = lo + dist;
        const bool asc = (lo & size) == 0;
        const double ka = key[lo], kb = key[hi];
        const int ia = idx[lo], ib = idx[hi];
        const bool a_gt = ka > kb || (ka == kb && ia > ib);
        if (a_gt == asc) {
          key[lo] = kb;
          key[hi] = ka;
          idx[lo] = ib;
          idx[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
}

// Fills the (d2, j) pairs of row i in one space (j != i; padding +inf with
// index INT_MAX), sorts them and writes rank[j] = position + 1.
__device__ void rank_row(const double* __restrict__ x, int n, int p, int i, int m, double* key, int* idx, int* rank) {
  for (int e = threadIdx.x; e < m; e += kMetThreads) {
    if (e < n - 1) {
      const int j = e < i ? e : e + 1;
      key[e] = row_d2(x, n, p, i, j);
      idx[e] = j;
    } else {
      key[e] = INFINITY;
      idx[e] = 0x7fffffff;
    }
  }
  __syncthreads();
  lds_sort_pairs(key, idx, m);
  for (int r = threadIdx.x; r < n - 1; r += kMetThreads) rank[idx[r]] = r + 1;
  __syncthreads();
}

// Dynamic LDS: key[m] (fp64), idx[m], high_rank[n], low_rank[n], high_order[kmax].
// Row sums: sums[(i * nk + q) * 4 + {0: shared, 1: trust, 2: continuity, 3: rank error}].
__global__ __launch_bounds__(kMetThreads) void k_structure_rows(const double* __restrict__ high, int p_high,
                                                                const double* __restrict__ low, int p_low, int n,
                                                                int m, const int* __restrict__ ks, int nk, int kmax,
                                                                double* __restrict__ sums) {
  extern __shared__ double lds[];
  double* const key = lds;
  int* const idx = reinterpret_cast<int*>(key + m);
  int* const high_rank = idx + m;
  int* const low_rank = high_rank + n;
  int* const high_order = low_rank + n;
  __shared__ double part[4][kMetThreads / 64];
  const int i = static_cast<int>(blockIdx.x);
  const int tid = static_cast<int>(threadIdx.x);

  rank_row(high, n, p_high, i, m, key, idx, high_rank);
  for (int r = tid; r < kmax; r += kMetThreads) high_order[r] = idx[r];
  __syncthreads();
  rank_row(low, n, p_low, i, m, key, idx, low_rank);  // idx[r] is now the low order

  for (int q = 0; q < nk; ++q) {
    const int k = ks[q];
    double shared = 0.0, trust = 0.0, cont = 0.0, rerr = 0.0;
    for (int r = tid; r < k; r += kMetThreads) {
      const int low_nb = idx[r];
      const int high_nb = high_order[r];
      const int in_high = high_rank[low_nb];
      const int in_low = low_rank[high_nb];
      if (in_high <= k) shared += 1.0;
      if (in_high > k) trust += in_high - k;
      if (in_low > k) cont += in_low - k;
      rerr += abs(in_high - (r + 1));
    }
    // integer-valued partial sums: exact in any order
    for (int off = 32; off > 0; off >>= 1) {
      shared += __shfl_xor(shared, off);
      trust += __shfl_xor(trust, off);
      cont += __shfl_xor(cont, off);
      rerr += __shfl_xor(rerr, off);
    }
    if ((tid & 63) == 0) {
      part[0][tid / 64] = shared;
      part[1][tid / 64] = trust;
      part[2][tid / 64] = cont;
      part[3][tid / 64] = rerr;
    }
    __syncthreads();
    if (tid < 4) {
      double s = 0.0;
      for (int w = 0; w < kMetThreads / 64; ++w) s += part[tid][w];
      sums[(static_cast<long long>(i) * nk + q) * 4 + tid] = s;
    }
    __syncthreads();
  }
}

template <typename T>
struct MetBuf {
  T* p = nullptr;
  hipError_t alloc(std::size_t count) {
    return hipMalloc(reinterpret_cast<void**>(&p), std::max<std::size_t>(count, 1) * sizeof(T));
  }
  ~MetBuf() {
    if (p != nullptr) (void)hipFree(p);
  }
};

}  // namespace

int structure_metrics_run(const double* high, int n, int p_high, const double* low, int p_low, const int* ks,
                          int nk, double* out, std::string& err) {
  if (high == nullptr || low == nullptr || ks == nullptr || out == nullptr) {
    err = "null pointer";
    return 1;
  }
  if (n < 3) {
    err = "at least three observations are required";
    return 1;
  }
  if (p_high < 1 || p_low < 1) {
    err = "input matrices must have columns";
    return 1;
  }
  if (n > kMetMaxRows) {
    err = "exact rank metrics support at most 5000 sampled observations";
    return 1;
  }
  if (nk < 1) {
    err = "requested_k must not be empty";
    return 1;
  }
  int kmax = 0;
  for (int q = 0; q < nk; ++q) {
    const int k = ks[q];
    if (k < 1 || k >= n || 2 * n - 3 * k - 1 <= 0) {
      err = "each k must satisfy 1 <= k < (2 * n - 1) / 3";
      return 1;
    }
    kmax = std::max(kmax, k);
  }
  int m = 1;
  while (m < n - 1) m <<= 1;
  const std::size_t lds = static_cast<std::size_t>(m) * (sizeof(double) + sizeof(int)) +
                          static_cast<std::size_t>(2 * n + kmax) * sizeof(int);
  hipError_t e;
  auto fail = [&](const char* what) {
    err = std::string(what) + ": " + hipGetErrorString(e);
    return 1;
  };
  MetBuf<double> dh, dl, dsums;
  MetBuf<int> dks;
  const std::size_t sh = static_cast<std::size_t>(n) * p_high, sl = static_cast<std::size_t>(n) * p_low;
  if ((e = dh.alloc(sh)) != hipSuccess || (e = dl.alloc(sl)) != hipSuccess || (e = dks.alloc(nk)) != hipSuccess ||
      (e = dsums.alloc(static_cast<std::size_t>(n) * nk * 4)) != hipSuccess)
    return fail("hipMalloc(structure metrics)");
  if ((e = hipMemcpy(dh.p, high, sh * sizeof(double), hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(dl.p, low, sl * sizeof(double), hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(dks.p, ks, nk * sizeof(int), hipMemcpyHostToDevice)) != hipSuccess)
    return fail("hipMemcpy(structure metrics)");
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_structure_rows),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds))) != hipSuccess)
    return fail("structure metrics LDS");
  k_structure_rows<<<n, kMetThreads, lds, nullptr>>>(dh.p, p_high, dl.p, p_low, n, m, dks.p, nk, kmax, dsums.p);
  if ((e = hipGetLastError()) != hipSuccess) return fail("structure metrics launch");
  std::vector<double> sums(static_cast<std::size_t>(n) * nk * 4);
  if ((e = hipMemcpy(sums.data(), dsums.p, sums.size() * sizeof(double), hipMemcpyDeviceToHost)) != hipSuccess)
    return fail("hipMemcpy(structure metrics)");
  for (int q = 0; q < nk; ++q) {
    double shared = 0.0, trust = 0.0, cont = 0.0, rerr = 0.0;
    for (int i = 0; i < n; ++i) {
      const double* s = sums.data() + (static_cast<std::size_t>(i) * nk + q) * 4;
      shared += s[0];
      trust += s[1];
      cont += s[2];
      rerr += s[3];
    }
    const double k = static_cast<double>(ks[q]);
    const double normalizer = 2.0 / (static_cast<double>(n) * k * (2.0 * n - 3.0 * k - 1.0));
    // out is nk x 4, column-major (R's NumericMatrix(nk, 4))
    out[q] = std::max(0.0, std::min(1.0, 1.0 - normalizer * trust));
    out[nk + q] = std::max(0.0, std::min(1.0, 1.0 - normalizer * cont));
    out[2 * nk + q] = shared / (static_cast<double>(n) * k);
    out[3 * nk + q] = rerr / (static_cast<double>(n) * k);
  }
  return 0;
}

}  // namespace fehip
