// Stand-in for embedding_hip_impl.cpp when fastEmbedR is built without HIP
// (configure.hip found no hipcc, or FASTEMBEDR_USE_HIP=0), as
// src/embedding_cuda_stub.cpp stands in for the CUDA implementation
// (:9-11, 108-173): the backend reports itself unavailable, and every entry
// point stops with a message.  Nothing falls back to the CPU.

#include <Rcpp.h>

#include <string>

using Rcpp::IntegerMatrix;
using Rcpp::IntegerVector;
using Rcpp::List;
using Rcpp::NumericMatrix;

namespace {

[[noreturn]] void hip_unavailable(const char* what) {
  Rcpp::stop("HIP %s is available only when the package is built with HIP (hipcc, gfx950) support. "
             "No CPU fallback is used for HIP-labelled runs.",
             what);
}

}  // namespace

bool embedding_hip_available_impl() { return false; }

List knn_tsne_opentsne_hip_float_impl(IntegerMatrix, SEXP, NumericMatrix, bool, int, double, int, int, double,
                                      double, double, bool, double, double, double, double, std::string, int,
                                      bool) {
  hip_unavailable("openTSNE FFT-grid");
}

List knn_tsne_opentsne_hip_gpu_impl(SEXP, int, NumericMatrix, bool, SEXP, int, double, int, int, double, double,
                                    double, bool, double, double, double, double, std::string, int, bool) {
  hip_unavailable("GPU-resident openTSNE FFT-grid");
}

List transform_tsne_hip_impl(NumericMatrix, IntegerMatrix, NumericMatrix, NumericMatrix, bool, std::string, double,
                             int, int, double, double, double, double, double, double, double, int, int, int, int,
                             bool) {
  hip_unavailable("t-SNE transform");
}

List native_hip_knn_impl(SEXP, int, std::string, std::string, double, bool) { hip_unavailable("native KNN"); }

List native_hip_query_knn_impl(SEXP, SEXP, int, std::string, std::string, double, bool) {
  hip_unavailable("native query KNN");
}

List native_hip_knn_to_host_impl(SEXP) { hip_unavailable("native KNN"); }

NumericMatrix exact_structure_metrics_hip_impl(NumericMatrix, NumericMatrix, IntegerVector) {
  hip_unavailable("structure metrics");
}
