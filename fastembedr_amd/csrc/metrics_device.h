// Exact rank-based structure metrics on the device (metrics_hip.hip): the
// host entry that the C ABI (fastembedr_hip_structure_metrics) wraps.
#pragma once

#include <string>

namespace fehip {

constexpr int kMetMaxRows = 5000;  // the reference's limit (exact_structure_metrics_cpp)

// high: n x p_high, low: n x p_low, both column-major fp64 (host); ks: nk
// requested k; out: nk x 4 column-major (trustworthiness, continuity, knn
// preservation, mean neighbour rank error).  Returns 0, or 1 with err set.
int structure_metrics_run(const double* high, int n, int p_high, const double* low, int p_low, const int* ks,
                          int nk, double* out, std::string& err);

}  // namespace fehip
