// HIP (MI355X, gfx950) implementation behind embedding_hip_bridge.cpp: R
// objects in, the C ABI of fastembedr_hip.h called, R lists out.  Compiled by
// R's C++ compiler when configure.hip finds hipcc; embedding_hip_stub.cpp
// replaces it otherwise.
//
// It mirrors the CUDA implementation's openTSNE entry points
// (src/embedding_cuda_impl.cpp:2088-2218, 2242-2484): the same argument
// checks, layouts and result fields, with HIP labels.  Unlike them it honours
// record_costs as the CPU driver does (src/tsne_neighbors.cpp:1757-1771,
// 1816-1823): the exact KL after every 50th iteration and after the last
// one, and each row's KL term at the end.  Runs that record costs go through
// the session ABI; the others through the one-shot call that replaces
// fastembedr_cuda_opentsne_fft_from_knn_float.

#include <Rcpp.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cctype>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "fastembedr_hip.h"

using Rcpp::CharacterVector;
using Rcpp::IntegerMatrix;
using Rcpp::IntegerVector;
using Rcpp::List;
using Rcpp::Named;
using Rcpp::NumericMatrix;
using Rcpp::NumericVector;

namespace {

constexpr int kMaxHipNeighbors = 256;

std::string lower(std::string s) {
  std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return static_cast<char>(std::tolower(c)); });
  return s;
}

void check_fft_method(const std::string& method) {
  const std::string m = lower(method);
  if (!(m == "fft" || m == "fitsne" || m == "fit_sne" || m == "interpolation" || m == "auto")) {
    Rcpp::stop("HIP openTSNE supports `negative_gradient_method = \"fft\"` only.");
  }
}

bool is_float32(SEXP x) { return Rf_isS4(x) && Rcpp::S4(x).is("float32"); }

// Column-major fp32 values of an n x k matrix: the float::float32 payload (the
// bit patterns of fp32 values held as integers), or a double matrix narrowed
// as the CPU path narrows it on copy (src/tsne_neighbors.cpp:327-352).
std::vector<float> matrix_f32(SEXP x, R_xlen_t count, const char* what) {
  std::vector<float> out(static_cast<std::size_t>(count));
  if (is_float32(x)) {
    SEXP payload = Rcpp::S4(x).slot("Data");
    if (TYPEOF(payload) != INTSXP || Rf_xlength(payload) != count) Rcpp::stop("%s has incompatible dimensions.", what);
    static_assert(sizeof(int) == sizeof(float), "float32 payload uses 32-bit storage");
    std::memcpy(out.data(), INTEGER(payload), out.size() * sizeof(float));
  } else if (Rf_isReal(x) && Rf_xlength(x) == count) {
    const double* v = REAL(x);
    for (R_xlen_t i = 0; i < count; ++i) out[static_cast<std::size_t>(i)] = static_cast<float>(v[i]);
  } else {
    Rcpp::stop("%s must be a numeric or float32 matrix with matching dimensions.", what);
  }
  return out;
}

// Rows and columns of a numeric or float32 matrix.
void matrix_dims(SEXP x, int& nrow, int& ncol) {
  SEXP m = is_float32(x) ? static_cast<SEXP>(Rcpp::S4(x).slot("Data")) : x;
  if (!Rf_isMatrix(m)) Rcpp::stop("`data` must be a matrix.");
  nrow = Rf_nrows(m);
  ncol = Rf_ncols(m);
}

// 1 when every index is in [1, n] (src/tsne_neighbors.cpp:79-90), else 0.
int knn_index_offset(const IntegerMatrix& idx) {
  const int n = idx.nrow();
  for (int v : idx) {
    if (v < 1 || v > n) return 0;
  }
  return 1;
}

std::vector<float> init_rows(const NumericMatrix& y) {  // n x 2 -> interleaved fp32
  const int n = y.nrow();
  std::vector<float> out(2 * static_cast<std::size_t>(n));
  for (int i = 0; i < n; ++i) {
    out[2 * static_cast<std::size_t>(i)] = static_cast<float>(y(i, 0));
    out[2 * static_cast<std::size_t>(i) + 1] = static_cast<float>(y(i, 1));
  }
  return out;
}

struct OptArgs {
  int n_components;
  double perplexity;
  int early_iter, n_iter;
  double early_exaggeration, exaggeration, learning_rate;
  bool learning_rate_auto;
  double initial_momentum, final_momentum, min_gain, max_step_norm;
  int seed;
};

void check_opt_args(const OptArgs& a, int n, int k, bool init, const NumericMatrix& y_init) {
  if (a.n_components != 2) Rcpp::stop("HIP openTSNE FFT-grid currently supports exactly two output components.");
  if (init && (y_init.nrow() != n || y_init.ncol() != 2)) {
    Rcpp::stop("HIP openTSNE FFT-grid requires a two-dimensional initialization.");
  }
  if (k < 1 || k > kMaxHipNeighbors) {
    Rcpp::stop("HIP openTSNE FFT-grid supports between 1 and %d neighbors.", kMaxHipNeighbors);
  }
  if (a.perplexity <= 0.0) Rcpp::stop("perplexity must be positive");
  // The CPU driver's rule (src/tsne_neighbors.cpp:1652), checked here so that
  // the one-shot route and the cost-recording session route refuse alike.
  if (static_cast<double>(n - 1) < 3.0 * a.perplexity) {
    Rcpp::stop("perplexity is too large for the number of samples.");
  }
  if (a.early_iter < 0 || a.n_iter < 0 || a.early_iter + a.n_iter < 1) {
    Rcpp::stop("HIP openTSNE FFT-grid requires at least one optimization iteration.");
  }
  if (a.early_exaggeration <= 0.0 || a.exaggeration <= 0.0) {
    Rcpp::stop("HIP openTSNE FFT-grid exaggeration values must be positive.");
  }
  if (a.learning_rate <= 0.0 && !a.learning_rate_auto) Rcpp::stop("HIP openTSNE FFT-grid learning rate must be positive.");
  if (a.initial_momentum < 0.0 || a.final_momentum < 0.0) {
    Rcpp::stop("HIP openTSNE FFT-grid momentum values must be non-negative.");
  }
  if (a.min_gain <= 0.0) Rcpp::stop("HIP openTSNE FFT-grid min_gain must be positive.");
  if (!fastembedr_hip_available()) Rcpp::stop("No gfx950 HIP device is available.");
}

// A phase's learning rate: fp32 n / exaggeration when automatic, as the
// one-shot entry points compute it.
float phase_learning_rate(const OptArgs& a, int n, double exaggeration) {
  return a.learning_rate_auto ? static_cast<float>(n) / static_cast<float>(exaggeration)
                              : static_cast<float>(a.learning_rate);
}

struct CostRecord {
  std::vector<double> itercosts;
  std::vector<int> iterations;
  std::vector<double> row_costs;
};

// The two phases through the session ABI with the CPU driver's cost
// recording.  init == nullptr draws the CPU driver's initialisation
// (mt19937(seed), normal(0, 1e-4)), as the one-shot calls do.
void optimize_recording_costs(const int* indices, const float* distances, bool on_device, int n, int k,
                              int index_offset, const OptArgs& a, const float* init, float* out, CostRecord& rec) {
  fastembedr_hip_tsne* s = nullptr;
  auto fail = [&](const char* what) {
    const std::string msg = fastembedr_hip_embedding_last_error();
    if (s != nullptr) fastembedr_hip_tsne_destroy(s);
    Rcpp::stop("HIP openTSNE FFT-grid failed (%s): %s", what, msg.c_str());
  };
  if (fastembedr_hip_tsne_create(indices, distances, n, k, static_cast<float>(a.perplexity), index_offset,
                                 on_device ? 1 : 0, 0, &s) != 0) {
    fail("P construction");
  }
  std::vector<float> drawn;
  if (init == nullptr) {
    drawn.resize(2 * static_cast<std::size_t>(n));
    if (fastembedr_hip_random_init(n, static_cast<unsigned int>(a.seed), drawn.data()) != 0) fail("initialisation");
    init = drawn.data();
  }
  if (fastembedr_hip_tsne_set_state(s, init, nullptr, nullptr) != 0 || fastembedr_hip_tsne_center(s) != 0) {
    fail("initial state");
  }
  const float step = std::isfinite(a.max_step_norm) ? static_cast<float>(a.max_step_norm)
                                                    : std::numeric_limits<float>::quiet_NaN();
  const int total = a.early_iter + a.n_iter;
  int done = 0;
  const struct {
    int count;
    double exaggeration, momentum;
  } phases[2] = {{a.early_iter, a.early_exaggeration, a.initial_momentum},
                 {a.n_iter, a.exaggeration, a.final_momentum}};
  for (const auto& ph : phases) {
    const float lr = phase_learning_rate(a, n, ph.exaggeration);
    int left = ph.count;
    while (left > 0) {
      const int chunk = std::min(left, 50 - done % 50);
      if (fastembedr_hip_tsne_run(s, chunk, static_cast<float>(ph.exaggeration), static_cast<float>(ph.momentum), lr,
                                  static_cast<float>(a.min_gain), step) != 0) {
        fail("iterations");
      }
      done += chunk;
      left -= chunk;
      if (done % 50 == 0 || done == total) {
        double kl = 0.0;
        if (fastembedr_hip_tsne_kl(s, &kl) != 0) fail("KL");
        rec.itercosts.push_back(kl);
        rec.iterations.push_back(done);
      }
    }
  }
  rec.row_costs.assign(static_cast<std::size_t>(n), 0.0);
  double kl = 0.0;
  if (fastembedr_hip_tsne_kl_rows(s, &kl, rec.row_costs.data()) != 0) fail("KL");
  if (fastembedr_hip_tsne_get_state(s, out, nullptr, nullptr) != 0) fail("layout download");
  fastembedr_hip_tsne_destroy(s);
}

NumericMatrix layout_matrix(const std::vector<float>& out, int n) {
  NumericMatrix y(n, 2);
  for (int i = 0; i < n; ++i) {
    y(i, 0) = static_cast<double>(out[2 * static_cast<std::size_t>(i)]);
    y(i, 1) = static_cast<double>(out[2 * static_cast<std::size_t>(i) + 1]);
  }
  return y;
}

List opentsne_result(const std::vector<float>& out, int n, const OptArgs& a, bool record_costs,
                     const CostRecord& rec, bool device_knn, const char* initialization) {
  const double lr_early = a.learning_rate_auto ? static_cast<double>(phase_learning_rate(a, n, a.early_exaggeration))
                                               : a.learning_rate;
  const double lr_normal = a.learning_rate_auto ? static_cast<double>(phase_learning_rate(a, n, a.exaggeration))
                                                : a.learning_rate;
  List res = List::create(
      Named("Y") = layout_matrix(out, n),
      Named("costs") = record_costs ? NumericVector(rec.row_costs.begin(), rec.row_costs.end()) : NumericVector(0),
      Named("itercosts") = NumericVector(rec.itercosts.begin(), rec.itercosts.end()),
      Named("itercost_iterations") = IntegerVector(rec.iterations.begin(), rec.iterations.end()),
      Named("optimizer") = device_knn ? "opentsne_fitsne_fft_grid_native_hip_gpu_knn"
                                      : "opentsne_fitsne_fft_grid_native_hip",
      Named("repulsion") = "fft_grid_hip",
      Named("probabilities") = device_knn ? "symmetric_sparse_knn_hip_float32_gpu_resident"
                                          : "symmetric_sparse_knn_hip_float32",
      Named("precision") = "float32", Named("n_negatives") = NA_INTEGER, Named("n_threads") = NA_INTEGER,
      Named("learning_rate_early") = lr_early, Named("learning_rate_normal") = lr_normal,
      Named("early_exaggeration_iter_actual") = a.early_iter, Named("n_iter_actual") = a.n_iter,
      Named("max_iter_actual") = a.early_iter + a.n_iter);
  res["auto_kld_stop"] = false;
  res["auto_stop_reason"] = "hip_fft_no_host_kld_monitor";
  res["auto_iter_end"] = NA_REAL;
  res["initialization"] = initialization;
  res["knn_residency"] = device_knn ? "hip_device" : "host";
  return res;
}

const void* device_address(SEXP ptr, const char* name) {
  if (TYPEOF(ptr) != EXTPTRSXP) Rcpp::stop("%s must be an external pointer", name);
  void* address = R_ExternalPtrAddr(ptr);
  if (address == nullptr) Rcpp::stop("%s points to a released HIP allocation", name);
  return address;
}

// ---- native KNN results -----------------------------------------------------
// A device-resident result owns two hipMalloc buffers (n x k int32 indices and
// fp32 distances, column-major); the R object holds them through external
// pointers whose owner releases them when collected.
struct HipKnnHandle {
  int* indices = nullptr;
  float* distances = nullptr;
  int n = 0;
  int k = 0;
  int device = 0;
};

void hip_knn_finalizer(SEXP owner) {
  auto* h = static_cast<HipKnnHandle*>(R_ExternalPtrAddr(owner));
  if (h == nullptr) return;
  (void)hipFree(h->indices);
  (void)hipFree(h->distances);
  delete h;
  R_ClearExternalPtr(owner);
}

int knn_metric_code(const std::string& metric) {
  const std::string m = lower(metric);
  if (m == "euclidean" || m == "l2") return FASTEMBEDR_HIP_KNN_EUCLIDEAN;
  if (m == "cosine") return FASTEMBEDR_HIP_KNN_COSINE;
  if (m == "correlation") return FASTEMBEDR_HIP_KNN_CORRELATION;
  Rcpp::stop("HIP native KNN supports metric = \"euclidean\", \"cosine\" or \"correlation\".");
}

List knn_metadata(int n, int k, int n_reference, const std::string& metric, double target_recall, bool exclude_self) {
  int device = 0;
  (void)hipGetDevice(&device);
  List out = List::create(Named("n_query") = n, Named("n") = n, Named("k") = k, Named("index_base") = 1,
                          Named("indices_type") = "int32", Named("distance_type") = "float32",
                          Named("layout") = "column_major_query_by_k", Named("metric") = lower(metric),
                          Named("backend_used") = "native_hip_exact_mfma_l2", Named("method") = "exact",
                          Named("accelerator") = "hip");
  out["gpu_provider"] = "fastEmbedR_native_hip";
  out["device"] = device;
  out["exact"] = true;
  out["exclude_self"] = exclude_self;
  out["n_reference"] = n_reference;
  out["target_recall"] = target_recall;
  out["tuning"] = "exact";
  return out;
}

// Runs the exact search (self when query is R_NilValue) and returns the
// result on the device (keep_gpu) or on the host.
List run_native_knn(SEXP data, SEXP query, int k, const std::string& metric, double target_recall, bool keep_gpu) {
  if (!fastembedr_hip_available()) Rcpp::stop("No gfx950 HIP device is available for native KNN.");
  const bool self = query == R_NilValue;
  int n_ref = 0, d = 0;
  matrix_dims(data, n_ref, d);
  int nq = n_ref, dq = d;
  if (!self) matrix_dims(query, nq, dq);
  if (dq != d) Rcpp::stop("`query` must have the same number of columns as `data`.");
  const int max_k = std::min(kMaxHipNeighbors, self ? n_ref - 1 : n_ref);
  if (k < 1 || k > max_k) Rcpp::stop("`k` must be between 1 and %d.", max_k);
  const int code = knn_metric_code(metric);
  const std::vector<float> x = matrix_f32(data, static_cast<R_xlen_t>(n_ref) * d, "`data`");
  std::vector<float> q;
  if (!self) q = matrix_f32(query, static_cast<R_xlen_t>(nq) * d, "`query`");
  const std::size_t count = static_cast<std::size_t>(nq) * k;
  long long stats[5] = {0, 0, 0, 0, 0};
  if (keep_gpu) {
    auto* h = new HipKnnHandle();
    h->n = nq;
    h->k = k;
    (void)hipGetDevice(&h->device);
    if (hipMalloc(reinterpret_cast<void**>(&h->indices), count * sizeof(int)) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&h->distances), count * sizeof(float)) != hipSuccess) {
      (void)hipFree(h->indices);
      (void)hipFree(h->distances);
      delete h;
      Rcpp::stop("HIP native KNN: device allocation of the result failed.");
    }
    const int rc = self ? fastembedr_hip_knn_exact_metric(x.data(), n_ref, d, 1, k, 1, code, 0, h->indices,
                                                          h->distances, 1, stats)
                        : fastembedr_hip_knn_query_metric(x.data(), n_ref, q.data(), nq, d, 1, k, code, 0,
                                                          h->indices, h->distances, 1, stats);
    if (rc != 0) {
      const std::string msg = fastembedr_hip_embedding_last_error();
      (void)hipFree(h->indices);
      (void)hipFree(h->distances);
      delete h;
      Rcpp::stop("Native HIP KNN failed: %s", msg.c_str());
    }
    SEXP owner = PROTECT(R_MakeExternalPtr(h, R_NilValue, R_NilValue));
    R_RegisterCFinalizerEx(owner, hip_knn_finalizer, TRUE);
    SEXP indices_ptr = PROTECT(R_MakeExternalPtr(h->indices, R_NilValue, owner));
    SEXP distances_ptr = PROTECT(R_MakeExternalPtr(h->distances, R_NilValue, owner));
    List out = knn_metadata(nq, k, n_ref, metric, target_recall, self);
    out["handle"] = owner;
    out["indices_ptr"] = indices_ptr;
    out["distances_ptr"] = distances_ptr;
    out["indices_residency"] = "hip_device";
    out["distance_residency"] = "hip_device";
    out["result_residency"] = "hip";
    UNPROTECT(3);
    return out;
  }
  IntegerMatrix idx(nq, k);
  std::vector<float> dist(count);
  const int rc = self ? fastembedr_hip_knn_exact_metric(x.data(), n_ref, d, 1, k, 1, code, 0, idx.begin(),
                                                        dist.data(), 0, stats)
                      : fastembedr_hip_knn_query_metric(x.data(), n_ref, q.data(), nq, d, 1, k, code, 0,
                                                        idx.begin(), dist.data(), 0, stats);
  if (rc != 0) Rcpp::stop("Native HIP KNN failed: %s", fastembedr_hip_embedding_last_error());
  NumericMatrix dd(nq, k);
  for (std::size_t c = 0; c < count; ++c) dd[c] = static_cast<double>(dist[c]);
  List out = knn_metadata(nq, k, n_ref, metric, target_recall, self);
  out["indices"] = idx;
  out["distances"] = dd;
  out["result_residency"] = "host";
  return out;
}

}  // namespace

bool embedding_hip_available_impl() { return fastembedr_hip_available(); }

List knn_tsne_opentsne_hip_float_impl(IntegerMatrix indices, SEXP distances, NumericMatrix y_init, bool init,
                                      int n_components, double perplexity, int early_exaggeration_iter,
                                      int n_iter, double early_exaggeration, double exaggeration,
                                      double learning_rate, bool learning_rate_auto, double initial_momentum,
                                      double final_momentum, double min_gain, double max_step_norm,
                                      std::string negative_gradient_method, int seed, bool record_costs) {
  check_fft_method(negative_gradient_method);
  const int n = indices.nrow();
  const int k = indices.ncol();
  const OptArgs a{n_components, perplexity, early_exaggeration_iter, n_iter, early_exaggeration, exaggeration,
                  learning_rate, learning_rate_auto, initial_momentum, final_momentum, min_gain, max_step_norm,
                  seed};
  check_opt_args(a, n, k, init, y_init);
  const std::vector<float> dist = matrix_f32(distances, static_cast<R_xlen_t>(n) * k, "KNN `distances`");
  std::vector<float> y0 = init ? init_rows(y_init) : std::vector<float>(2 * static_cast<std::size_t>(n), 0.0f);
  std::vector<float> out(2 * static_cast<std::size_t>(n));
  const int offset = knn_index_offset(indices);
  CostRecord rec;
  if (record_costs) {
    optimize_recording_costs(indices.begin(), dist.data(), false, n, k, offset, a, init ? y0.data() : nullptr,
                             out.data(), rec);
  } else {
    const int rc = fastembedr_hip_opentsne_fft_from_knn_float(
        indices.begin(), dist.data(), y0.data(), init ? 1 : 0, n, k, n_components, static_cast<float>(perplexity),
        early_exaggeration_iter, n_iter, static_cast<float>(early_exaggeration), static_cast<float>(exaggeration),
        static_cast<float>(learning_rate), learning_rate_auto ? 1 : 0, static_cast<float>(initial_momentum),
        static_cast<float>(final_momentum), static_cast<float>(min_gain), static_cast<float>(max_step_norm),
        static_cast<unsigned int>(seed), offset, out.data());
    if (rc != 0) Rcpp::stop("HIP openTSNE FFT-grid failed: %s", fastembedr_hip_embedding_last_error());
  }
  return opentsne_result(out, n, a, record_costs, rec, false, init ? "host_supplied" : "random_normal_mt19937");
}

List knn_tsne_opentsne_hip_gpu_impl(SEXP gpu_knn, int requested_k, NumericMatrix y_init, bool init,
                                    SEXP pca_init_data, int n_components, double perplexity,
                                    int early_exaggeration_iter, int n_iter, double early_exaggeration,
                                    double exaggeration, double learning_rate, bool learning_rate_auto,
                                    double initial_momentum, double final_momentum, double min_gain,
                                    double max_step_norm, std::string negative_gradient_method, int seed,
                                    bool record_costs) {
  if (!Rf_isNewList(gpu_knn)) Rcpp::stop("HIP GPU-resident openTSNE requires a GPU KNN list contract.");
  List src(gpu_knn);
  check_fft_method(negative_gradient_method);
  if (!src.containsElementNamed("indices_ptr") || !src.containsElementNamed("distances_ptr")) {
    Rcpp::stop("GPU KNN object is missing HIP KNN device pointers.");
  }
  if (src.containsElementNamed("result_residency") && Rcpp::as<std::string>(src["result_residency"]) != "hip") {
    Rcpp::stop("HIP GPU-resident openTSNE requires a KNN result resident on the HIP device.");
  }
  if (src.containsElementNamed("distance_type") && Rcpp::as<std::string>(src["distance_type"]) != "float32") {
    Rcpp::stop("HIP GPU-resident openTSNE requires float32 KNN distances.");
  }
  if (src.containsElementNamed("layout") && Rcpp::as<std::string>(src["layout"]) != "column_major_query_by_k") {
    Rcpp::stop("Unsupported GPU KNN layout for HIP openTSNE.");
  }
  if (src.containsElementNamed("exclude_self") && !Rcpp::as<bool>(src["exclude_self"])) {
    Rcpp::stop("HIP GPU-resident openTSNE requires non-self KNN. "
               "Create the GPU KNN with `exclude_self = TRUE` or use the host KNN path.");
  }
  if (!init && pca_init_data != R_NilValue) {
    Rcpp::stop("HIP openTSNE takes its initialisation as `Y_init`; device PCA initialisation is not part of the "
               "HIP backend.");
  }
  const int n = src.containsElementNamed("n_query") ? Rcpp::as<int>(src["n_query"]) : Rcpp::as<int>(src["n"]);
  const int available_k = Rcpp::as<int>(src["k"]);
  const int k = requested_k > 0 ? requested_k : available_k;
  if (k < 1 || k > available_k) Rcpp::stop("Requested GPU KNN width exceeds the GPU KNN object width.");
  const OptArgs a{n_components, perplexity, early_exaggeration_iter, n_iter, early_exaggeration, exaggeration,
                  learning_rate, learning_rate_auto, initial_momentum, final_momentum, min_gain, max_step_norm,
                  seed};
  check_opt_args(a, n, k, init, y_init);
  // The first k columns of a column-major n x K buffer are its first n * k
  // elements, so a narrower request reads a prefix of the buffers.
  const int* dev_idx = static_cast<const int*>(device_address(src["indices_ptr"], "indices_ptr"));
  const float* dev_dist = static_cast<const float*>(device_address(src["distances_ptr"], "distances_ptr"));
  const int offset = src.containsElementNamed("index_base") ? Rcpp::as<int>(src["index_base"]) : 1;
  std::vector<float> y0 = init ? init_rows(y_init) : std::vector<float>(2 * static_cast<std::size_t>(n), 0.0f);
  std::vector<float> out(2 * static_cast<std::size_t>(n));
  CostRecord rec;
  if (record_costs) {
    optimize_recording_costs(dev_idx, dev_dist, true, n, k, offset, a, init ? y0.data() : nullptr, out.data(), rec);
  } else {
    const int rc = fastembedr_hip_opentsne_fft_from_device_knn_float(
        dev_idx, dev_dist, y0.data(), init ? 1 : 0, n, k, n_components, static_cast<float>(perplexity),
        early_exaggeration_iter, n_iter, static_cast<float>(early_exaggeration), static_cast<float>(exaggeration),
        static_cast<float>(learning_rate), learning_rate_auto ? 1 : 0, static_cast<float>(initial_momentum),
        static_cast<float>(final_momentum), static_cast<float>(min_gain), static_cast<float>(max_step_norm),
        static_cast<unsigned int>(seed), offset, out.data());
    if (rc != 0) Rcpp::stop("HIP openTSNE FFT-grid failed: %s", fastembedr_hip_embedding_last_error());
  }
  return opentsne_result(out, n, a, record_costs, rec, true, init ? "host_supplied" : "random_normal_mt19937");
}

List transform_tsne_hip_impl(NumericMatrix reference_layout, IntegerMatrix indices, NumericMatrix distances,
                             NumericMatrix y_init, bool init, std::string initialization, double perplexity,
                             int n_iter, int early_exaggeration_iter, double learning_rate,
                             double early_exaggeration, double exaggeration, double initial_momentum,
                             double final_momentum, double max_grad_norm, double max_step_norm, int n_negatives,
                             int exact_repulsion_threshold, int /*n_threads*/, int seed, bool /*verbose*/) {
  if (reference_layout.ncol() != 2) {
    Rcpp::stop("HIP t-SNE transform currently supports only two-dimensional reference layouts.");
  }
  if (indices.nrow() != distances.nrow() || indices.ncol() != distances.ncol()) {
    Rcpp::stop("KNN `indices` and `distances` must have the same dimensions.");
  }
  const std::string init_name = lower(initialization);
  const int init_code = init_name == "median" ? 0 : (init_name == "weighted" ? 1 : (init_name == "random" ? 2 : -1));
  if (init_code < 0) Rcpp::stop("`initialization` must be 'median', 'weighted', or 'random'.");
  const int n_query = indices.nrow();
  if (init && (y_init.nrow() != n_query || y_init.ncol() != 2)) {
    Rcpp::stop("`Y_init` must have one row per query and the same columns as `reference_layout`.");
  }
  if (!fastembedr_hip_available()) Rcpp::stop("No gfx950 HIP device is available.");
  NumericMatrix layout(n_query, 2);
  int exact = 0;
  // R matrices are column-major, the ABI's layout; seed NA_integer_ is INT_MIN.
  const int rc = fastembedr_hip_transform_tsne(
      reference_layout.begin(), reference_layout.nrow(), indices.begin(), distances.begin(), n_query,
      indices.ncol(), init ? y_init.begin() : nullptr, init_code, perplexity, n_iter, early_exaggeration_iter,
      learning_rate, early_exaggeration, exaggeration, initial_momentum, final_momentum, max_grad_norm,
      max_step_norm, n_negatives, exact_repulsion_threshold, seed, layout.begin(), &exact);
  if (rc != 0) Rcpp::stop("HIP t-SNE transform failed: %s", fastembedr_hip_embedding_last_error());
  List res = List::create(Named("Y") = layout, Named("optimizer") = "opentsne_style_fixed_reference_transform",
                          Named("initialization") = init_name,
                          Named("repulsion") = exact ? "exact_reference" : "sampled_reference",
                          Named("affinities") = "precomputed_query_conditional",
                          Named("affinity_storage") = "flat_row_major_double",
                          Named("transform_batch_size") = n_query, Named("transform_batches") = 1,
                          Named("n_negatives") = std::min(n_negatives, reference_layout.nrow()),
                          Named("n_threads") = NA_INTEGER);
  res["backend"] = "hip";
  return res;
}

List native_hip_knn_impl(SEXP data, int k, std::string /*method*/, std::string metric, double target_recall,
                         bool keep_gpu) {
  // Every method runs the exact, certified search (recall 1 meets any target).
  return run_native_knn(data, R_NilValue, k, metric, target_recall, keep_gpu);
}

List native_hip_query_knn_impl(SEXP data, SEXP query, int k, std::string /*method*/, std::string metric,
                               double target_recall, bool keep_gpu) {
  if (query == R_NilValue) Rcpp::stop("`query` must be a matrix.");
  return run_native_knn(data, query, k, metric, target_recall, keep_gpu);
}

List native_hip_knn_to_host_impl(SEXP knn) {
  if (!Rf_isNewList(knn)) Rcpp::stop("`knn` must be a native KNN result.");
  List src(knn);
  if (!src.containsElementNamed("indices_ptr")) return src;  // already on the host
  const int n = src.containsElementNamed("n_query") ? Rcpp::as<int>(src["n_query"]) : Rcpp::as<int>(src["n"]);
  const int k = Rcpp::as<int>(src["k"]);
  const std::size_t count = static_cast<std::size_t>(n) * k;
  IntegerMatrix idx(n, k);
  std::vector<float> dist(count);
  if (hipMemcpy(idx.begin(), device_address(src["indices_ptr"], "indices_ptr"), count * sizeof(int),
                hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(dist.data(), device_address(src["distances_ptr"], "distances_ptr"), count * sizeof(float),
                hipMemcpyDeviceToHost) != hipSuccess) {
    Rcpp::stop("HIP native KNN: copying the result to the host failed.");
  }
  NumericMatrix dd(n, k);
  for (std::size_t c = 0; c < count; ++c) dd[c] = static_cast<double>(dist[c]);
  List out = Rcpp::clone(src);
  out["indices"] = idx;
  out["distances"] = dd;
  out["indices_ptr"] = R_NilValue;
  out["distances_ptr"] = R_NilValue;
  out["handle"] = R_NilValue;
  out["indices_residency"] = "host";
  out["distance_residency"] = "host";
  out["result_residency"] = "host";
  return out;
}

NumericMatrix exact_structure_metrics_hip_impl(NumericMatrix high, NumericMatrix low, IntegerVector requested_k) {
  const int n = high.nrow();
  if (low.nrow() != n) Rcpp::stop("`high` and `low` must have the same number of rows.");
  if (!fastembedr_hip_available()) Rcpp::stop("No gfx950 HIP device is available.");
  const int nk = requested_k.size();
  NumericMatrix out(nk, 4);
  if (fastembedr_hip_structure_metrics(high.begin(), n, high.ncol(), low.begin(), low.ncol(), requested_k.begin(),
                                       nk, out.begin()) != 0) {
    Rcpp::stop("HIP structure metrics failed: %s", fastembedr_hip_embedding_last_error());
  }
  Rcpp::colnames(out) =
      CharacterVector::create("trustworthiness", "continuity", "knn_preservation", "mean_neighbor_rank_error");
  return out;
}
