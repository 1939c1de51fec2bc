# HIP (AMD MI355X, gfx950) backend of fastEmbedR's openTSNE path.
#
# These helpers are what the package's existing switch points call for
# backend = "hip"; each switch point gains one branch, shipped as unified
# diffs against the package's files in integration/r/patches/:
#   embedding_backend_choices()          (R/backend_info.R:102-104)  adds "hip"
#   backend_info()                       (R/backend_info.R:2-41)     rbind(hip_backend_info_row())
#   fast_knn_opentsne_materialized()     (R/tsne_affinity_dispatch.R:65-88)
#                                        optimizer_backend <- require_hip_opentsne()
#                                        (R/tsne_affinity_dispatch.R:122-132)
#                                        negative_gradient_method <- hip_negative_gradient_method(...)
#                                        (R/tsne_affinity_dispatch.R:219-315)
#                                        out <- run_hip_opentsne(...)
#   transform_tsne()                     (R/transform_tsne.R:231-254) run_hip_transform(...)
#   evaluate_embedding()                 (R/evaluate_embedding.R:483-500) hip_structure_metrics(...)
# A HIP-labelled run never falls back to the CPU: when the backend is missing
# it stops with a message, as the CUDA and Metal branches do.

hip_opentsne_native_available <- function() {
  exists("knn_tsne_opentsne_hip_float_cpp", envir = asNamespace("fastEmbedR"), inherits = FALSE) &&
    backend_flag(embedding_hip_available_cpp)
}

require_hip_opentsne <- function() {
  if (!hip_opentsne_native_available()) {
    stop(
      "Native HIP openTSNE optimizer was requested, but it is not available in this build. ",
      "No CPU fallback is used for HIP-labelled runs.",
      call. = FALSE
    )
  }
  "hip"
}

# The HIP backend runs the FFT-grid repulsion for every method string that
# names it; "auto" resolves to "fft" at every n, as on CUDA
# (R/tsne_affinity_dispatch.R:127-130).
hip_negative_gradient_method <- function(negative_gradient_method) {
  if (identical(negative_gradient_method, "auto")) "fft" else negative_gradient_method
}

# The optimizer call of fast_knn_opentsne_materialized() for the HIP backend.
# `args`, `ex` and `lr` are the lists that function builds for the CUDA call
# (Y_init, init, n_components, perplexity, momentum, final_momentum; early,
# normal; value, auto).  gpu_knn is a device-resident KNN result of
# native_hip_knn_cpp(keep_gpu = TRUE).
run_hip_opentsne <- function(indices,
                             distances,
                             args,
                             early_exaggeration_iter,
                             n_iter,
                             ex,
                             lr,
                             min_gain,
                             max_step_norm,
                             negative_gradient_method,
                             seed,
                             record_costs,
                             gpu_knn = NULL,
                             k = NULL) {
  if (!is.null(gpu_knn)) {
    if (!identical(gpu_knn$result_residency, "hip")) {
      stop("backend = \"hip\" needs a KNN result resident on the HIP device ",
           "(native_hip_knn_cpp(keep_gpu = TRUE)) or a host KNN.", call. = FALSE)
    }
    return(knn_tsne_opentsne_hip_gpu_cpp(
      gpu_knn, as.integer(k), args$Y_init, args$init, NULL, args$n_components, args$perplexity,
      as.integer(early_exaggeration_iter), as.integer(n_iter), ex$early, ex$normal, lr$value, lr$auto,
      args$momentum, args$final_momentum, min_gain, max_step_norm, negative_gradient_method,
      as.integer(seed), isTRUE(record_costs)
    ))
  }
  knn_tsne_opentsne_hip_float_cpp(
    indices, distances, args$Y_init, args$init, args$n_components, args$perplexity,
    as.integer(early_exaggeration_iter), as.integer(n_iter), ex$early, ex$normal, lr$value, lr$auto,
    args$momentum, args$final_momentum, min_gain, max_step_norm, negative_gradient_method,
    as.integer(seed), isTRUE(record_costs)
  )
}

# transform_tsne(backend = "hip"): the transform_tsne_cpp arguments
# (src/tsne_neighbors.cpp:1859-1880), computed on the device in fp64 with the
# CPU path's operation order.
run_hip_transform <- function(reference_layout,
                              indices,
                              distances,
                              y_init,
                              init,
                              initialization,
                              perplexity,
                              n_iter,
                              early_exaggeration_iter,
                              learning_rate,
                              early_exaggeration,
                              exaggeration,
                              initial_momentum,
                              final_momentum,
                              max_grad_norm,
                              max_step_norm,
                              n_negatives,
                              exact_repulsion_threshold,
                              seed) {
  if (!backend_flag(embedding_hip_available_cpp)) {
    stop("Native HIP t-SNE transform was requested, but it is not available in this build. ",
         "No CPU fallback is used for HIP-labelled runs.", call. = FALSE)
  }
  if (ncol(reference_layout) != 2L) {
    stop("HIP t-SNE transform currently supports only two-dimensional reference layouts.", call. = FALSE)
  }
  transform_tsne_hip_cpp(
    reference_layout, indices, distances, y_init, init, initialization, perplexity, as.integer(n_iter),
    as.integer(early_exaggeration_iter), as.numeric(learning_rate), as.numeric(early_exaggeration),
    as.numeric(exaggeration), as.numeric(initial_momentum), as.numeric(final_momentum),
    as.numeric(max_grad_norm), as.numeric(max_step_norm), as.integer(n_negatives),
    as.integer(exact_repulsion_threshold), 1L, as.integer(seed), FALSE
  )
}

# exact_structure_metrics_cpp() on the device, for evaluate_embedding()'s
# sampled rows (3 <= n <= 5000).  Same columns and values.
hip_structure_metrics <- function(high, low, requested_k) {
  exact_structure_metrics_hip_cpp(as.matrix(high), as.matrix(low), as.integer(requested_k))
}

# One row of backend_info() for the HIP backend.
hip_backend_info_row <- function() {
  hip_embedding <- backend_flag(embedding_hip_available_cpp)
  data.frame(
    backend = "hip",
    available = hip_embedding,
    knn_available = hip_embedding,
    embedding_available = hip_embedding,
    clustering_available = FALSE,
    explicit_backend = "hip",
    device = if (hip_embedding) "AMD Instinct MI355X (gfx950)" else NA_character_,
    runtime = R.version$platform,
    note = if (hip_embedding) {
      "Package-native HIP openTSNE (FFT grid), exact KNN, transform and structure metrics are available."
    } else {
      "The HIP backend is unavailable in this build (no hipcc or no gfx950 device)."
    },
    stringsAsFactors = FALSE
  )
}
