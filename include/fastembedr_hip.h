/*
 * fastembedr_hip.h -- C ABI of the MI355X (gfx950) openTSNE-style t-SNE backend.
 *
 * Plain pointers and sizes only.  Every entry point returns 0 on success and
 * 1 on failure (the reference's convention); the failure message is then
 * available from fastembedr_hip_embedding_last_error() on the same thread.
 *
 * Layouts (identical to the reference's CUDA ABI):
 *   indices, distances : n x k, column-major (element (i, j) at j * n + i),
 *                        R matrix order; index_offset is 0 or 1.
 *   init, out, y       : n x 2 row-major interleaved (x0, y0, x1, y1, ...).
 *
 * Numerics follow the reference's CPU backend (src/tsne_neighbors.cpp):
 * fp32 perplexity search, symmetric CSR P normalised by the total directed
 * mass, the bilinear FFT grid with the CPU grid-size policy (honouring
 * FASTEMBEDR_TSNE_FFT_GRID), the sign(0) == 0 gains rule and per-iteration
 * centring.  Differences from that backend are limited to fp32 summation
 * order (parallel reductions and float atomics).
 */
#ifndef FASTEMBEDR_HIP_H
#define FASTEMBEDR_HIP_H

#include <stdbool.h>

#if defined(__GNUC__)
#define FASTEMBEDR_HIP_API __attribute__((visibility("default")))
#else
#define FASTEMBEDR_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces fastembedr_cuda_embedding_last_error()
 * (src/embedding_cuda_kernels.cpp:3753-3755). */
FASTEMBEDR_HIP_API const char* fastembedr_hip_embedding_last_error(void);

/* Replaces fastembedr_cuda_available() (src/embedding_cuda_kernels.cpp:3757-3765):
 * true when a HIP device is present and it is a gfx950 part. */
FASTEMBEDR_HIP_API bool fastembedr_hip_available(void);

/* Replaces fastembedr_cuda_opentsne_fft_from_knn_float
 * (src/embedding_cuda_kernels.cpp:6039-6066; declared in
 * src/embedding_cuda_impl.cpp:79-183).  Same 21 parameters, same meaning:
 * host KNN (float32 distances), optional host init (has_init != 0), two-phase
 * optimisation, final layout copied to host `out`.  has_init == 0 draws the
 * reference CPU backend's initialisation: mt19937(seed) feeding
 * normal_distribution<float>(0, 1e-4) (src/tsne_neighbors.cpp:1693-1700).
 * learning_rate_auto != 0 uses n / exaggeration per phase.  max_step_norm
 * that is not finite or <= 0 disables the per-point step clip. */
FASTEMBEDR_HIP_API int fastembedr_hip_opentsne_fft_from_knn_float(
    const int* indices, const float* distances, const float* init, int has_init,
    int n, int k, int n_components, float perplexity,
    int early_exaggeration_iter, int n_iter,
    float early_exaggeration, float exaggeration,
    float learning_rate, int learning_rate_auto,
    float initial_momentum, float final_momentum,
    float min_gain, float max_step_norm,
    unsigned int seed, int index_offset, float* out);

/* Replaces fastembedr_cuda_opentsne_fft_from_knn (double distances)
 * (src/embedding_cuda_kernels.cpp:6010-6037).  Distances are narrowed to fp32
 * on the device, as the reference CPU path narrows them on copy
 * (src/tsne_neighbors.cpp:342-350). */
FASTEMBEDR_HIP_API int fastembedr_hip_opentsne_fft_from_knn(
    const int* indices, const double* distances, const float* init, int has_init,
    int n, int k, int n_components, float perplexity,
    int early_exaggeration_iter, int n_iter,
    float early_exaggeration, float exaggeration,
    float learning_rate, int learning_rate_auto,
    float initial_momentum, float final_momentum,
    float min_gain, float max_step_norm,
    unsigned int seed, int index_offset, float* out);

/* Replaces fastembedr_cuda_opentsne_fft_from_device_knn_float
 * (src/embedding_cuda_kernels.cpp:6068-6094): indices and distances are
 * device pointers (borrowed, column-major n x k); init and out stay on the
 * host, as in the reference. */
FASTEMBEDR_HIP_API int fastembedr_hip_opentsne_fft_from_device_knn_float(
    const int* indices, const float* distances, const float* init, int has_init,
    int n, int k, int n_components, float perplexity,
    int early_exaggeration_iter, int n_iter,
    float early_exaggeration, float exaggeration,
    float learning_rate, int learning_rate_auto,
    float initial_momentum, float final_momentum,
    float min_gain, float max_step_norm,
    unsigned int seed, int index_offset, float* out);

/* ------------------------------------------------------------------------
 * Session ABI.  No counterpart in the reference: the reference exposes only
 * the one-shot calls above.  These entry points split the same work into
 * P construction, per-iteration steps and state transfer so that parity can
 * be checked per stage (P, one gradient, one update) and throughput can be
 * timed with inputs already resident in HBM.  The one-shot calls above are
 * implemented on top of them.
 * ---------------------------------------------------------------------- */
typedef struct fastembedr_hip_tsne fastembedr_hip_tsne;

/* Repulsion modes. */
#define FASTEMBEDR_HIP_REPULSION_GRID 0     /* bilinear FFT grid (reference) */
#define FASTEMBEDR_HIP_REPULSION_EXACT 1    /* O(n^2) pairwise (checking only) */
#define FASTEMBEDR_HIP_REPULSION_LAGRANGE 2 /* FIt-SNE order-p Lagrange grid */

/* Builds P on the device from KNN (host or device pointers, column-major).
 * grid_size == 0 selects the reference CPU policy (64/128/256 by n,
 * FASTEMBEDR_TSNE_FFT_GRID override, clamped to [32, 512]); an explicit grid
 * size is rounded up to a power of two in [32, 1024].  1 <= k <= 256. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_create(const int* indices, const float* distances,
                               int n, int k, float perplexity, int index_offset,
                               int inputs_on_device, int grid_size,
                               fastembedr_hip_tsne** out_session);

FASTEMBEDR_HIP_API void fastembedr_hip_tsne_destroy(fastembedr_hip_tsne* session);

/* Number of stored entries of the symmetric CSR P (both triangles). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_p_nnz(const fastembedr_hip_tsne* session, long long* nnz);

/* Copies P to host arrays of sizes n + 1, nnz, nnz. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_copy_p(const fastembedr_hip_tsne* session,
                               int* row_ptr, int* col, float* val);

/* Conditional p_{j|i} from the perplexity search, column-major n x k (host). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_copy_conditional_p(const fastembedr_hip_tsne* session,
                                           float* p_cond);

/* Grid nodes per axis used by the bilinear repulsion. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_grid_size(const fastembedr_hip_tsne* session, int* grid_size);

/* Sets the optimiser state from host arrays (n x 2 each).  update and gains
 * may be NULL: they are then reset to 0 and 1 (the reference's start state). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_set_state(fastembedr_hip_tsne* session, const float* y,
                                  const float* update, const float* gains);

/* Copies the optimiser state to host arrays; any pointer may be NULL. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_get_state(fastembedr_hip_tsne* session, float* y,
                                  float* update, float* gains);

/* Gradient at the current y without changing the state (no centring):
 * the reference's compute_gradient_fft_grid_f (src/tsne_neighbors.cpp:1076-1182)
 * or, for REPULSION_EXACT, compute_gradient_pair_symmetric_f (:1014-1074). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_gradient(fastembedr_hip_tsne* session, float exaggeration,
                                 int repulsion, float* grad_out);

/* Centres y (the reference's zero_mean_f, src/tsne_neighbors.cpp:1200-1211). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_center(fastembedr_hip_tsne* session);

/* Runs n_iter iterations of gradient + update + centring with fixed phase
 * parameters (src/tsne_neighbors.cpp:1749-1802).  Asynchronous with respect
 * to the host; fastembedr_hip_tsne_sync() waits. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_run(fastembedr_hip_tsne* session, int n_iter,
                            float exaggeration, float momentum, float learning_rate,
                            float min_gain, float max_step_norm);

FASTEMBEDR_HIP_API int fastembedr_hip_tsne_sync(fastembedr_hip_tsne* session);

/* Selects the repulsion that run() uses: FASTEMBEDR_HIP_REPULSION_GRID (the
 * reference's bilinear grid, the default) or FASTEMBEDR_HIP_REPULSION_LAGRANGE,
 * the FIt-SNE interpolation grid (Linderman et al. 2019), which the reference
 * names in its method strings ("fitsne", "interpolation",
 * src/tsne_neighbors.cpp:368) but computes with the bilinear grid.  Its
 * settings follow openTSNE's names: n_interpolation_points per box and axis
 * (3 is supported), min_num_intervals boxes per axis at least, one box per
 * ints_in_interval units of the layout's span.  The node count is capped at
 * 2048 per axis (FFT length 4096); beyond it boxes widen.  gradient() with
 * FASTEMBEDR_HIP_REPULSION_LAGRANGE uses the settings given here (defaults 3,
 * 50, 1).  No counterpart in the reference's ABI. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_set_repulsion(fastembedr_hip_tsne* session, int repulsion,
                                      int n_interpolation_points, int min_num_intervals,
                                      float ints_in_interval);

/* Geometry of the FIt-SNE interpolation grid at the current layout (boxes and
 * nodes per axis, box width), the FFT length of its last iteration and the
 * normaliser Z = sum_{i != j} q_ij of the last repulsion evaluated (either
 * grid).  Any pointer may be NULL. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_interp_info(fastembedr_hip_tsne* session, int* boxes, int* nodes,
                                    int* fft_len, float* box_width, double* z);

/* Replayed iterations of run(): how many iterations ran as a replayed graph,
 * how many graphs were captured, and whether capture is on.  Capture follows
 * FASTEMBEDR_HIP_GRAPH_CAPTURE at session creation: off when unset, empty or
 * 0/false/FALSE/no/NO, on otherwise (the reference's
 * FASTEMBEDR_CUDA_GRAPH_CAPTURE, src/embedding_cuda_kernels.cpp:170-178,
 * takes the same off values but is on when unset; eager launches measured
 * faster on MI355X).  Timed runs never replay.  Any pointer may be NULL.  No
 * counterpart in the reference's ABI. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_graph_info(fastembedr_hip_tsne* session, long long* launches,
                                   int* captures, int* enabled);

/* Locality of the attraction's tiled P: the number of (row block, column
 * tile) runs of the current working numbering (-1 before the first build,
 * or when the row-parallel attraction is used) and the number of
 * renumberings so far.  No counterpart in the reference. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_attraction_info(fastembedr_hip_tsne* session, long long* tiles,
                                        int* renumbers);

/* Size of the attraction's tiled P in the current working numbering: slots
 * (entries, bridge slots between entries more than 7 rows apart, and the
 * padding of each run to a multiple of 8), -1 when there is none (as for
 * attraction_info).  No counterpart in the reference. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_attraction_slots(fastembedr_hip_tsne* session, long long* slots);

/* Exact KL(P || Q) at the current y (src/tsne_neighbors.cpp:1258-1285), with
 * the O(n^2) normalisation computed on the device in fp64. */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_kl(fastembedr_hip_tsne* session, double* kl);

/* The same KL and, when row_costs is not NULL, each row's term (n doubles,
 * caller's numbering): the per-row costs the reference's CPU driver returns
 * as `costs` when costs are recorded (src/tsne_neighbors.cpp:1258-1285,
 * 1816-1823). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_kl_rows(fastembedr_hip_tsne* session, double* kl, double* row_costs);

/* Per-kernel timing.  While enabled, run() records HIP events around every
 * kernel (enabled == 1), or around the kernel with id (enabled - 2) & 0xffff
 * only (enabled >= 2), so that the other launches run without event
 * overhead, on every iteration or, with enabled >> 16 = E > 1, on every E-th
 * iteration (the events' markers delay the launch behind them); events go on
 * the stream the kernel runs on.  run() normally runs the
 * attraction and the repulsion kernel spectrum on side streams beside the
 * rest of the iteration; with every kernel timed it runs them in sequence,
 * so that each duration is the kernel's alone.  The id named "repulsion" is
 * no kernel: timed alone, it runs the iteration in sequence and brackets the
 * repulsion step's kernels (kernel spectrum to potentials) with one pair of
 * events, the step's duration without per-kernel event overhead.  stats
 * returns, per kernel id,
 * the number of launches timed and their summed duration in milliseconds.
 * Kernel ids and names: fastembedr_hip_tsne_kernel_name(). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_set_timing(fastembedr_hip_tsne* session, int enabled);
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_timing_stats(fastembedr_hip_tsne* session, int max_kernels,
                                     long long* launches, double* total_ms);
FASTEMBEDR_HIP_API const char* fastembedr_hip_tsne_kernel_name(int kernel_id);
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_kernel_count(void);

/* Host-side helper with no ABI counterpart in the reference: writes the
 * initialisation that the one-shot calls use when has_init == 0, i.e. the
 * reference CPU driver's mt19937(seed) + normal_distribution<float>(0, 1e-4)
 * draw (src/tsne_neighbors.cpp:1693-1700), n x 2 row-major, so that session
 * users start from the same layout. */
FASTEMBEDR_HIP_API int fastembedr_hip_random_init(int n, unsigned int seed, float* out);

/* ------------------------------------------------------------------------
 * Fixed-reference transform.  Replaces the computation of the reference's
 * transform_tsne_cpp (src/tsne_neighbors.cpp:1859-2109; R entry
 * transform_tsne(), R/transform_tsne.R:57-315) for two-dimensional layouts.
 * The reference has no GPU counterpart (R/transform_tsne.R:231-254 names a
 * transform_tsne_cuda_cpp that src/ does not define), so the arguments are
 * those of transform_tsne_cpp, with R's matrix layouts:
 *   reference_layout : n_reference x 2, column-major, fp64
 *   indices          : n_query x k, column-major, 0- or 1-based (1-based iff
 *                      every index is in [1, n_reference])
 *   distances        : n_query x k, column-major, fp64
 *   y_init, out      : n_query x 2, column-major, fp64; y_init may be NULL
 *   initialization   : 0 median, 1 weighted, 2 random
 *   seed             : INT_MIN stands for R's NA (then 5489)
 * max_grad_norm / max_step_norm that are not finite or <= 0 disable the clip;
 * n_negatives is capped at n_reference; the repulsion is exact when
 * n_reference <= exact_repulsion_threshold or n_negatives >= n_reference,
 * and *repulsion_exact (may be NULL) reports which was used.  All arithmetic
 * is fp64 in the reference's order. */
FASTEMBEDR_HIP_API int fastembedr_hip_transform_tsne(
    const double* reference_layout, int n_reference,
    const int* indices, const double* distances, int n_query, int k,
    const double* y_init, int initialization, double perplexity,
    int n_iter, int early_exaggeration_iter, double learning_rate,
    double early_exaggeration, double exaggeration,
    double initial_momentum, double final_momentum,
    double max_grad_norm, double max_step_norm,
    int n_negatives, int exact_repulsion_threshold, int seed,
    double* out, int* repulsion_exact);

/* Parity probe for the transform, no counterpart in the reference: the
 * conditional probabilities (p_out, n_query x k row-major, as the reference
 * stores them), the median (0) or weighted (1) initialisation (init_out,
 * n_query x 2 row-major) and one gradient at y (grad_out, n_query x 2
 * row-major) for the given per-iteration seed.  Any output may be NULL. */
FASTEMBEDR_HIP_API int fastembedr_hip_transform_probe(
    const double* reference_layout, int n_reference,
    const int* indices, const double* distances, int n_query, int k,
    double perplexity, const double* y, double exaggeration,
    int n_negatives, int exact_repulsion_threshold, int iter_seed,
    int initialization, double* p_out, double* grad_out, double* init_out);

/* Fixed-reference transform with the reference's repulsion precomputed on an
 * interpolation grid (the benchmark's config 3: the reference's grid charges
 * are precomputed once and only the query points move).  No counterpart in
 * the reference, whose transform repulsion is exact or sampled
 * (src/tsne_neighbors.cpp:1472-1568).  The reference's repulsion fields
 * Z(y) = sum_j q(y - r_j) and F(y) = sum_j q(y - r_j)^2 (y - r_j),
 * q(d) = 1 / (1 + |d|^2), are summed directly at the nodes of a grid over the
 * reference and the queries' start (one square, widened by max(1, 5 % of the
 * span) on each side; max(min_num_intervals, ceil(span / ints_in_interval))
 * boxes per axis, n_interpolation_points = 3 nodes per box and axis, at most
 * 2048 nodes per axis), once per call; each query's repulsion is -F / Z with
 * both interpolated (order-3 Lagrange) from its box's 3 x 3 nodes, or the
 * exact sums over every reference point when the query is outside the grid.
 * Attraction, clips, gains and momentum are those of
 * fastembedr_hip_transform_tsne, whose other arguments these are (seed only
 * seeds the random initialisation).  stats (may be NULL, 3 values): boxes per
 * axis, nodes per axis, query-iterations that took the exact sums.  The
 * node sums cost nodes^2 x n_reference kernel evaluations. */
FASTEMBEDR_HIP_API int fastembedr_hip_transform_tsne_grid(
    const double* reference_layout, int n_reference,
    const int* indices, const double* distances, int n_query, int k,
    const double* y_init, int initialization, double perplexity,
    int n_iter, int early_exaggeration_iter, double learning_rate,
    double early_exaggeration, double exaggeration,
    double initial_momentum, double final_momentum,
    double max_grad_norm, double max_step_norm, int seed,
    int n_interpolation_points, int min_num_intervals, double ints_in_interval,
    double* out, long long* stats);

/* Parity probe of the grid transform, no counterpart in the reference: one
 * gradient (grad_out, n_query x 2 row-major) at y (row-major), with the grid
 * built around the reference and geometry_y (n_geometry x 2 row-major; NULL
 * with n_geometry 0: y itself).  stats as above. */
FASTEMBEDR_HIP_API int fastembedr_hip_transform_grid_probe(
    const double* reference_layout, int n_reference,
    const int* indices, const double* distances, int n_query, int k, double perplexity,
    const double* y, const double* geometry_y, int n_geometry, double exaggeration,
    int n_interpolation_points, int min_num_intervals, double ints_in_interval,
    double* grad_out, long long* stats);

/* Allocation-free variant of fastembedr_hip_transform_tsne.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory
 * (serving loops that place batches of new points against a fixed map,
 * harnesses that forbid hipMalloc).  It cannot be recorded into a HIP graph:
 * it launches on the null stream and waits for the device twice (to read the
 * input checks' result, and at the end).  Same arguments, meaning, checks,
 * error messages (for an input with several faults, the one that comes first
 * in column-major entry order, as in the allocating call) and result as
 * fastembedr_hip_transform_tsne (the same kernels in the same order), except:
 *   - reference_layout, indices, distances, y_init and out are DEVICE
 *     pointers, in the same layouts;
 *   - initialization 2 (random, drawn on the host) needs y_init;
 *   - n_reference <= 262144, n_query <= 131072 and n_query * k <= 4194304;
 *     larger inputs are refused with a message.
 * The work buffers (conditional P, layout, the reference in the kernels'
 * layout, flags) live in one static device array of 40 MB per GPU,
 * held until the process ends; the call makes no hipMalloc/hipFree and
 * creates no stream.  It runs on the null stream and returns when done.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * race. */
FASTEMBEDR_HIP_API int fastembedr_hip_transform_tsne_noalloc(
    const double* reference_layout, int n_reference,
    const int* indices, const double* distances, int n_query, int k,
    const double* y_init, int initialization, double perplexity,
    int n_iter, int early_exaggeration_iter, double learning_rate,
    double early_exaggeration, double exaggeration,
    double initial_momentum, double final_momentum,
    double max_grad_norm, double max_step_norm,
    int n_negatives, int exact_repulsion_threshold, int seed,
    double* out, int* repulsion_exact);

/* Wall time of the P construction in milliseconds (device events). */
FASTEMBEDR_HIP_API int fastembedr_hip_tsne_p_build_ms(const fastembedr_hip_tsne* session, double* ms);

/* Exact k-nearest neighbours by Euclidean distance, the exact route of the
 * reference's native GPU KNN (native_cuda_knn_cpp(data, k, method = "exact"),
 * src/native_knn_bridge.cpp:102-112 -> native_cuda_knn_impl,
 * src/native_knn_cuda_impl.cpp:511-704, finished by
 * src/embedding_cuda_kernels.cpp:1412-1464) and of its result contract
 * (src/native_knn_cuda_impl.cpp:427-466: layout "column_major_query_by_k",
 * index_base 1, int32 indices, float32 distances, exclude_self).
 *   x            n x d float32: row-major, or column-major (an R matrix) when
 *                x_col_major; device memory when x_on_device
 *   k            1 .. min(256, n - 1) with exclude_self (n without)
 *   d            1 .. 16384; rows wider than 128 are scanned in their
 *                projection on 128 leading principal directions (a lower
 *                bound of every distance) and ranked exactly in full width
 *   indices      n x k column-major (neighbour j of row i at j * n + i),
 *                1-based; device memory when output_on_device
 *   distances    same layout, sqrt of the squared distance
 * Neighbours are ordered by (distance, index), as an ordered dense distance
 * matrix (tests/testthat/helper-knn.R:5-38) orders them.  stats (may be NULL,
 * 5 values): rows rerun with a larger candidate set, passes, the last pass's
 * candidates per query, 64-row reference tiles staged (summed over blocks of
 * 128 queries) and tiles computed (summed over waves of 32 queries) after
 * pruning.  Returns 0, or 1 with fastembedr_hip_embedding_last_error() set. */
FASTEMBEDR_HIP_API int fastembedr_hip_knn_exact(const float* x, int n, int d, int x_col_major, int k,
                                                int exclude_self, int x_on_device, int* indices, float* distances,
                                                int output_on_device, long long* stats);

/* Exact query-to-reference k-nearest neighbours by Euclidean distance, the
 * exact route of the reference's native GPU query KNN
 * (native_cuda_query_knn_cpp(data, query, k, method = "exact"),
 * src/native_knn_bridge.cpp:115-124 -> native_cuda_query_knn_impl,
 * src/native_knn_cuda_impl.cpp:871-; finished by
 * finalize_cuvs_query_knn_kernel, src/embedding_cuda_kernels.cpp:1466-1503:
 * column-major n_query x k, 1-based reference indices, sqrt of the squared
 * distance; the caller, R/native_knn.R:333-416, requires
 * 1 <= k <= nrow(reference)).
 *   reference    n_reference x d float32, query n_query x d float32, both
 *                row-major or both column-major (col_major); both in device
 *                memory when inputs_on_device
 *   k            1 .. min(256, n_reference);  d  1 .. 16384 (as above)
 *   indices      n_query x k column-major, 1-based rows of reference; device
 *                memory when output_on_device
 *   distances    same layout
 * Neighbours are ordered by (distance, index).  stats as for
 * fastembedr_hip_knn_exact.  Returns 0, or 1 with the last error set. */
FASTEMBEDR_HIP_API int fastembedr_hip_knn_query(const float* reference, int n_reference, const float* query,
                                                int n_query, int d, int col_major, int k, int inputs_on_device,
                                                int* indices, float* distances, int output_on_device,
                                                long long* stats);

/* The same two searches with the reference's other exact metrics
 * (native_cuda_knn_cpp / native_cuda_query_knn_cpp with metric = "cosine" or
 * "correlation", src/native_knn_cuda_impl.cpp:514-560, 875-886): rows are
 * normalised to unit length, centred first for correlation, in the
 * reference's operation order (src/native_knn_common.h:50-67), searched by
 * Euclidean distance, and reported as half the squared distance, 1 - cos
 * (src/native_knn_common.h:119-128; src/embedding_cuda_kernels.cpp:1441-1442).
 * metric: one of the FASTEMBEDR_HIP_KNN_* codes; "inner_product" (CUDA-only
 * in the reference) is refused.  Other arguments as above. */
#define FASTEMBEDR_HIP_KNN_EUCLIDEAN 0
#define FASTEMBEDR_HIP_KNN_COSINE 1
#define FASTEMBEDR_HIP_KNN_CORRELATION 2
FASTEMBEDR_HIP_API int fastembedr_hip_knn_exact_metric(const float* x, int n, int d, int x_col_major, int k,
                                                       int exclude_self, int metric, int x_on_device, int* indices,
                                                       float* distances, int output_on_device, long long* stats);
FASTEMBEDR_HIP_API int fastembedr_hip_knn_query_metric(const float* reference, int n_reference, const float* query,
                                                       int n_query, int d, int col_major, int k, int metric,
                                                       int inputs_on_device, int* indices, float* distances,
                                                       int output_on_device, long long* stats);

/* Replaces exact_structure_metrics_cpp (src/embedding_utils.cpp:1582-1752),
 * which R's evaluate_embedding() calls on a row sample
 * (R/evaluate_embedding.R:483-500): trustworthiness, continuity, k-NN
 * preservation and mean neighbour rank error of a layout against the
 * high-dimensional rows, from full per-row rankings in both spaces (squared
 * Euclidean distance, ties by index).
 *   high         n x p_high fp64, column-major (host)
 *   low          n x p_low fp64, column-major (host)
 *   requested_k  nk values, each 1 <= k < (2n - 1) / 3
 *   out          nk x 4 fp64, column-major: trustworthiness, continuity,
 *                knn_preservation, mean_neighbor_rank_error
 * 3 <= n <= 5000 (the reference's limit).  The distances are formed in the
 * reference's operation order, so the ranks, and the metrics, are identical
 * to the reference's.  Returns 0, or 1 with the last error set. */
FASTEMBEDR_HIP_API int fastembedr_hip_structure_metrics(const double* high, int n, int p_high, const double* low,
                                                        int p_low, const int* requested_k, int nk, double* out);

#ifdef __cplusplus
}
#endif

#endif /* FASTEMBEDR_HIP_H */
