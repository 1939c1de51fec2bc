// Rcpp exports of fastEmbedR's HIP (MI355X, gfx950) backend.
//
// Compiled in every build.  The implementations behind these forwarders are
// in embedding_hip_impl.cpp when configure finds hipcc (configure.hip), and
// in embedding_hip_stub.cpp otherwise, exactly as the CUDA bridge forwards to
// embedding_cuda_impl.cpp or embedding_cuda_stub.cpp
// (src/embedding_cuda_bridge.cpp:208-211, 450-536).  Argument lists and
// meanings are those of the CUDA and CPU exports they stand beside:
//   knn_tsne_opentsne_hip_float_cpp  <- knn_tsne_opentsne_cuda_float_cpp
//   knn_tsne_opentsne_hip_gpu_cpp    <- knn_tsne_opentsne_cuda_gpu_cpp
//   transform_tsne_hip_cpp           <- transform_tsne_cpp (src/tsne_neighbors.cpp:1859-1880)
//   native_hip_knn_cpp, native_hip_query_knn_cpp, native_hip_knn_to_host_cpp
//                                    <- native_cuda_knn_cpp, ..._query_..., ..._to_host_cpp
//                                       (src/native_knn_bridge.cpp:102-129)
//   exact_structure_metrics_hip_cpp  <- exact_structure_metrics_cpp
//                                       (src/embedding_utils.cpp:1582-1585)

#include <Rcpp.h>

#include <string>

using Rcpp::IntegerMatrix;
using Rcpp::IntegerVector;
using Rcpp::List;
using Rcpp::NumericMatrix;

bool embedding_hip_available_impl();
List knn_tsne_opentsne_hip_float_impl(IntegerMatrix indices, SEXP distances, NumericMatrix y_init, bool init,
                                      int n_components, double perplexity, int early_exaggeration_iter,
                                      int n_iter, double early_exaggeration, double exaggeration,
                                      double learning_rate, bool learning_rate_auto, double initial_momentum,
                                      double final_momentum, double min_gain, double max_step_norm,
                                      std::string negative_gradient_method, int seed, bool record_costs);
List knn_tsne_opentsne_hip_gpu_impl(SEXP gpu_knn, int requested_k, NumericMatrix y_init, bool init,
                                    SEXP pca_init_data, int n_components, double perplexity,
                                    int early_exaggeration_iter, int n_iter, double early_exaggeration,
                                    double exaggeration, double learning_rate, bool learning_rate_auto,
                                    double initial_momentum, double final_momentum, double min_gain,
                                    double max_step_norm, std::string negative_gradient_method, int seed,
                                    bool record_costs);
List transform_tsne_hip_impl(NumericMatrix reference_layout, IntegerMatrix indices, NumericMatrix distances,
                             NumericMatrix y_init, bool init, std::string initialization, double perplexity,
                             int n_iter, int early_exaggeration_iter, double learning_rate,
                             double early_exaggeration, double exaggeration, double initial_momentum,
                             double final_momentum, double max_grad_norm, double max_step_norm, int n_negatives,
                             int exact_repulsion_threshold, int n_threads, int seed, bool verbose);
List native_hip_knn_impl(SEXP data, int k, std::string method, std::string metric, double target_recall,
                         bool keep_gpu);
List native_hip_query_knn_impl(SEXP data, SEXP query, int k, std::string method, std::string metric,
                               double target_recall, bool keep_gpu);
List native_hip_knn_to_host_impl(SEXP knn);
NumericMatrix exact_structure_metrics_hip_impl(NumericMatrix high, NumericMatrix low, IntegerVector requested_k);

// [[Rcpp::export]]
bool embedding_hip_available_cpp() { return embedding_hip_available_impl(); }

// [[Rcpp::export]]
List knn_tsne_opentsne_hip_float_cpp(IntegerMatrix indices, SEXP distances, NumericMatrix y_init, bool init,
                                     int n_components, double perplexity, int early_exaggeration_iter,
                                     int n_iter, double early_exaggeration, double exaggeration,
                                     double learning_rate, bool learning_rate_auto, double initial_momentum,
                                     double final_momentum, double min_gain, double max_step_norm,
                                     std::string negative_gradient_method, int seed, bool record_costs) {
  return knn_tsne_opentsne_hip_float_impl(indices, distances, y_init, init, n_components, perplexity,
                                          early_exaggeration_iter, n_iter, early_exaggeration, exaggeration,
                                          learning_rate, learning_rate_auto, initial_momentum, final_momentum,
                                          min_gain, max_step_norm, negative_gradient_method, seed, record_costs);
}

// [[Rcpp::export]]
List knn_tsne_opentsne_hip_gpu_cpp(SEXP gpu_knn, int requested_k, NumericMatrix y_init, bool init,
                                   SEXP pca_init_data, int n_components, double perplexity,
                                   int early_exaggeration_iter, int n_iter, double early_exaggeration,
                                   double exaggeration, double learning_rate, bool learning_rate_auto,
                                   double initial_momentum, double final_momentum, double min_gain,
                                   double max_step_norm, std::string negative_gradient_method, int seed,
                                   bool record_costs) {
  return knn_tsne_opentsne_hip_gpu_impl(gpu_knn, requested_k, y_init, init, pca_init_data, n_components,
                                        perplexity, early_exaggeration_iter, n_iter, early_exaggeration,
                                        exaggeration, learning_rate, learning_rate_auto, initial_momentum,
                                        final_momentum, min_gain, max_step_norm, negative_gradient_method, seed,
                                        record_costs);
}

// [[Rcpp::export]]
List transform_tsne_hip_cpp(NumericMatrix reference_layout, IntegerMatrix indices, NumericMatrix distances,
                            NumericMatrix y_init, bool init, std::string initialization, double perplexity,
                            int n_iter, int early_exaggeration_iter, double learning_rate,
                            double early_exaggeration, double exaggeration, double initial_momentum,
                            double final_momentum, double max_grad_norm, double max_step_norm, int n_negatives,
                            int exact_repulsion_threshold, int n_threads, int seed, bool verbose) {
  return transform_tsne_hip_impl(reference_layout, indices, distances, y_init, init, initialization, perplexity,
                                 n_iter, early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
                                 initial_momentum, final_momentum, max_grad_norm, max_step_norm, n_negatives,
                                 exact_repulsion_threshold, n_threads, seed, verbose);
}

// [[Rcpp::export]]
List native_hip_knn_cpp(SEXP data, int k, std::string method = "auto", std::string metric = "euclidean",
                        double target_recall = 0.99, bool keep_gpu = true) {
  return native_hip_knn_impl(data, k, method, metric, target_recall, keep_gpu);
}

// [[Rcpp::export]]
List native_hip_query_knn_cpp(SEXP data, SEXP query, int k, std::string method = "auto",
                              std::string metric = "euclidean", double target_recall = 0.99,
                              bool keep_gpu = true) {
  return native_hip_query_knn_impl(data, query, k, method, metric, target_recall, keep_gpu);
}

// [[Rcpp::export]]
List native_hip_knn_to_host_cpp(SEXP knn) { return native_hip_knn_to_host_impl(knn); }

// [[Rcpp::export]]
NumericMatrix exact_structure_metrics_hip_cpp(NumericMatrix high, NumericMatrix low, IntegerVector requested_k) {
  return exact_structure_metrics_hip_impl(high, low, requested_k);
}
