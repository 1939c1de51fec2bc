// Exact KNN on the device (knn_hip.hip): limits and the host entry that the
// C ABI (fastembedr_hip_knn_exact) wraps.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace fehip {

constexpr int kKnnMaxDim = 128;    // scanned dimensions: centred rows and a query block stay in LDS
constexpr int kKnnMaxInputDim = 16384;  // wider rows are scanned in a kKnnMaxDim-dimensional projection
constexpr int kKnnMaxK = 256;      // the reference's native GPU KNN limit (kMaxNativeCudaK)
constexpr long long kKnnCandEntries = 1ll << 28;  // candidate buffer entries of a scan launch (2 GiB)

// Element (row, col) of an n x d matrix at row * row_stride + col * col_stride.
struct Strides {
  long long row_stride, col_stride;
  __host__ __device__ long long at(long long r, long long c) const { return r * row_stride + c * col_stride; }
};

// k nearest neighbours of every row of x (n x d fp32; row-major, or
// column-major when x_col_major; on the device when input_on_device), by
// Euclidean distance, self excluded when exclude_self.  Writes n x k
// column-major (neighbour j of row i at j * n + i) 1-based indices and fp32
// distances, ascending by (distance, index), to the device or the host.
// stats (nullable, 5): rows rerun with a larger candidate set, passes, the
// last pass's candidates per query, 64-row reference tiles staged (summed
// over blocks of 128 queries) and tiles computed (summed over waves of 32
// queries) after pruning.  Returns 0, or 1 with err set.
// metric: kKnnEuclidean, or kKnnCosine / kKnnCorrelation (rows normalised,
// centred first for correlation, and distances written as 1 - cos).
constexpr int kKnnEuclidean = 0;
constexpr int kKnnCosine = 1;
constexpr int kKnnCorrelation = 2;
int knn_exact_run(const float* x, int n, int d, int x_col_major, int k, int exclude_self, int metric,
                  int input_on_device, int* indices, float* distances, int output_on_device, long long* stats,
                  std::string& err);

// k nearest references of every query row: ref (n_ref x d) and query
// (n_query x d), both fp32 in the same layout (column-major when col_major)
// and residency; k <= n_ref.  Writes n_query x k column-major 1-based
// reference indices and fp32 distances; stats as above.
int knn_query_run(const float* ref, int n_ref, const float* query, int n_query, int d, int col_major, int k,
                  int metric, int input_on_device, int* indices, float* distances, int output_on_device,
                  long long* stats, std::string& err);

}  // namespace fehip
