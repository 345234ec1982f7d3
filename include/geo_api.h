/*
 * geo_api.h — C ABI of libgeoembodied_hip.so, the gfx950 (MI355X) implementation of
 * GeoEmbodied's point-cloud geometry kernels: farthest-point sampling, KNN, radius graph,
 * CSR build and segment reduce (sum / mean / max, forward and backward).
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers unless the comment says "host".
 *   - The caller allocates every output and workspace; the library never allocates or frees
 *     device memory.  Workspace sizes come from the matching *_workspace_bytes() function.
 *     (geo_csr_build_noalloc uses a fixed device array of the library instead.)
 *   - All work is enqueued asynchronously on `stream` (a hipStream_t passed as void*; NULL is
 *     the legacy default stream).  No entry point synchronises the host.
 *   - Return value: GEO_OK (0) or a GEO_ERR_* code.  geo_last_error() returns a message for the
 *     last failure on the calling thread (thread-local; valid until the next failing call).
 *   - No mutable global state (except the fixed scratch of geo_csr_build_noalloc): entry
 *     points are re-entrant and thread-safe.
 *   - Index tensors: int64 where the reference's Python API exposes int64, int32 for the CSR
 *     arrays (the reference's CSR is int32 as well).
 *
 * Each entry point names the reference interface it replaces (paths relative to the reference
 * repository root).
 */
#ifndef GEO_API_H
#define GEO_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEO_OK 0
#define GEO_ERR_INVALID 1   /* bad argument (shape, size, range, alignment) */
#define GEO_ERR_HIP 2       /* a HIP runtime call or kernel launch failed */
#define GEO_ERR_WORKSPACE 3 /* workspace pointer NULL or smaller than required */
#define GEO_ERR_UNSUPPORTED 4

/* dtype codes for segment reduce */
#define GEO_F32 0
#define GEO_BF16 1
#define GEO_F64 2

/* reduction codes for segment reduce */
#define GEO_REDUCE_SUM 0
#define GEO_REDUCE_MEAN 1
#define GEO_REDUCE_MAX 2

/* ---------------------------------------------------------------- library --- */

/* Message of the last failing call on this thread ("" if none). */
const char* geo_last_error(void);
/* Build identification: target arch, compiler, flags. */
const char* geo_build_info(void);
/* ABI version, bumped on any signature or argument-meaning change (2: the SE3 CG table is a
 * device array; segment softmax takes zero_tail). */
int geo_abi_version(void);

/* -------------------------------------------------------------------- FPS --- */
/*
 * Replaces fps_cuda (geoembodied/csrc/fps_kernel.cu:160-209, bound at :216-229, dispatched from
 * geoembodied/csrc/__init__.py:566-597).  Semantics follow the CPU path
 * _fps_iterative_fallback (geoembodied/csrc/__init__.py:600-654): per cloud b with
 * n = ptr[b+1]-ptr[b] and k = clamp(k_per_batch[b], 0, n): k == 0 -> nothing; k == n ->
 * ptr[b] + arange(n); otherwise start at ptr[b] and repeatedly take the lowest index attaining
 * the max over points of min squared distance to the selected set.  Squared distance is
 * (fl(dx*dx) + fl(dy*dy)) + fl(dz*dz) in fp32 without contraction.
 *
 * Two phases, because the caller allocates the output:
 *   geo_fps_prepare writes out_ptr[0..B] (exclusive offsets of the clamped k) and
 *   info[0] = total samples, info[1] = largest cloud size, info[2] = 0 or, when ptr is not a
 *   valid non-decreasing offset array inside [0, N_total], the 1-based index of the first bad
 *   entry.  The caller copies info to the host (the one host sync of the op), allocates
 *   out_idx[info[0]] and calls geo_fps with max_cloud = info[1].
 */
int geo_fps_prepare(const int64_t* ptr, const int64_t* k_per_batch, int64_t B, int64_t N_total,
                    int64_t* out_ptr, int64_t* info, void* stream);
/* geo_fps_prepare with k_per_batch[b] = k for every cloud: the ptr path of the public op
 * (geoembodied/functional/fps.py:84-118, `k_per_batch = sizes.clamp(max=num_samples)` at
 * :108-109) without the two elementwise launches that form that array.  info_host (may be
 * NULL) is pinned host memory of 3 int64 (hipHostMalloc'd, e.g. a torch pin_memory tensor) that
 * also receives info, so the host can read it after an event recorded behind this launch
 * instead of copying it behind later work on the stream. */
int geo_fps_prepare_uniform(const int64_t* ptr, int64_t k, int64_t B, int64_t N_total,
                            int64_t* out_ptr, int64_t* info, int64_t* info_host, void* stream);
/* geo_fps for clouds of at most max_cloud_guess points, launched before the host has read
 * info: the kernel reads info (device copy) and does nothing when ptr was invalid or the
 * largest cloud exceeds the variant's capacity, which is returned in *capacity (0 = nothing
 * launched, as for guesses above 8192 points).  The caller then checks info[1] <= *capacity
 * and otherwise calls geo_fps.  Replaces the same kernel call as geo_fps. */
int geo_fps_guarded(const float* pos, int64_t N_total, const int64_t* ptr, const int64_t* out_ptr,
                    int64_t B, int64_t max_cloud_guess, int64_t* out_idx, const int64_t* info,
                    int64_t* capacity, void* stream);
size_t geo_fps_workspace_bytes(int64_t B, int64_t N_total, int64_t max_cloud);
int geo_fps(const float* pos, int64_t N_total, const int64_t* ptr, const int64_t* out_ptr,
            int64_t B, int64_t max_cloud, int64_t* out_idx, void* workspace,
            size_t workspace_bytes, void* stream);

/* -------------------------------------------------------------------- KNN --- */
/*
 * Replaces knn_cuda / knn_self_cuda (geoembodied/csrc/knn_kernel.cu:200-308, bound at
 * :315-327, dispatched from geoembodied/csrc/__init__.py:376-432).  Semantics follow
 * _knn_bruteforce (geoembodied/csrc/__init__.py:435-492) with a total order on ties: for each
 * query of cloud b, out_idx/out_dist[q, 0..k) are the first k sources of cloud b (global
 * indices) sorted ascending by the key (d, j), d = squared distance with dx = q.x - s.x.
 * Rows with fewer than k sources are padded with -1 / 1e30f.  ptr_q and ptr_s both have B+1
 * entries.  query may alias source (knn_self).
 */
size_t geo_knn_workspace_bytes(int64_t Nq, int64_t Ns, int64_t B, int64_t k);
int geo_knn(const float* query, int64_t Nq, const float* source, int64_t Ns,
            const int64_t* ptr_q, const int64_t* ptr_s, int64_t B, int64_t k,
            int64_t* out_idx, float* out_dist, void* workspace, size_t workspace_bytes,
            void* stream);

/* ----------------------------------------------------------- radius graph --- */
/*
 * Replaces radius_graph_cuda and radius_graph_cuda_batched
 * (geoembodied/csrc/radius_graph_kernel.cu:253-467, bound at :474-490, dispatched from
 * geoembodied/csrc/__init__.py:130-186 and geoembodied/functional/radius_graph.py:19-105).
 * Semantics follow the CPU path _radius_graph_batched/_single
 * (geoembodied/functional/radius_graph.py:204-335) with exact distances: edge j -> i exists iff
 * i and j are in the same cloud, both unmasked, (loop or i != j) and d(i,j) < r2, keeping per
 * target i the first K = max_num_neighbors sources by key (d, j).  r2 is the fp32 threshold the
 * caller computed as fl32(fl64(r) * fl64(r)) and r_cell = r (the grid cell edge is derived from
 * it).
 *
 * Cloud membership: batch[i] (values outside [0, B) are treated as masked) when batch != NULL,
 * otherwise contiguous chunks of points_per_cloud points (B * points_per_cloud == N).
 * mask may be NULL (all valid); nonzero bytes mark valid points.
 *
 * Two phases sharing one workspace:
 *   geo_radius_count builds the per-cloud uniform grid, counts (and, when N * max_num_neighbors
 *   fits the workspace bound, collects) the in-radius sources of every target and writes
 *   row_ptr[0..N] (CSR offsets of the edges grouped by target, row_ptr[N] = E).  The caller
 *   reads E (the one host sync), allocates row_out[E], col_out[E] and calls geo_radius_emit
 *   with the same arguments and workspace.  Output order: targets ascending, sources ascending
 *   within a target.
 */
size_t geo_radius_workspace_bytes(int64_t N, int64_t B, int64_t max_num_neighbors);
int geo_radius_count(const float* x, int64_t N, const int64_t* batch, int64_t B,
                     int64_t points_per_cloud, const uint8_t* mask, float r2, float r_cell,
                     int64_t max_num_neighbors, int loop, int64_t* row_ptr, void* workspace,
                     size_t workspace_bytes, void* stream);
int geo_radius_emit(const float* x, int64_t N, const int64_t* batch, int64_t B,
                    int64_t points_per_cloud, const uint8_t* mask, float r2, float r_cell,
                    int64_t max_num_neighbors, int loop, const int64_t* row_ptr,
                    int64_t* row_out, int64_t* col_out, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * The same two phases with the radius read from device memory (`radius`: one float64), so a
 * radius computed on the GPU (geo_knn_radius_stat) needs no host round trip: the threshold is
 * fl32(radius * radius) with the product in float64 — what the host computes for a Python
 * float — and radius <= 0 or NaN gives no edges.  Replaces the .item() of the adaptive radius
 * (geoembodied/nn/modules/multi_scale_se3_net.py:99-124) feeding radius_graph.
 */
int geo_radius_count_dev(const float* x, int64_t N, const int64_t* batch, int64_t B,
                         int64_t points_per_cloud, const uint8_t* mask, const double* radius,
                         int64_t max_num_neighbors, int loop, int64_t* row_ptr, void* workspace,
                         size_t workspace_bytes, void* stream);
int geo_radius_emit_dev(const float* x, int64_t N, const int64_t* batch, int64_t B,
                        int64_t points_per_cloud, const uint8_t* mask, const double* radius,
                        int64_t max_num_neighbors, int loop, const int64_t* row_ptr,
                        int64_t* row_out, int64_t* col_out, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * The two phases without a host wait between them.  geo_radius_count_async is geo_radius_count
 * (or geo_radius_count_dev when radius_dev is not NULL) that also writes E into edges_host[0]
 * (two int64 of mapped pinned host memory: hipHostMalloc'd, e.g. a pin_memory tensor).  The
 * caller records an event, calls geo_radius_emit[_dev] at once with outputs of the bound size
 * N * max_num_neighbors, waits for the event and reads E: the first E entries of the outputs are
 * the graph (geo_radius_copy_edges moves them into exact-sized arrays if wanted).  The same sync
 * as the reference's (geoembodied/csrc/__init__.py:130-186), taken off the GPU's critical path.
 *
 * Clouds given as contiguous chunks of points_per_cloud <= 4096 points take a one-workgroup-per-
 * cloud front end.  With batch != NULL and points_per_cloud > 0, batch is expected to be that
 * chunk layout (batch[i] = i / points_per_cloud: the sorted equal-size batches the reference's
 * GPU path assumes, geoembodied/functional/radius_graph.py:70-85); the front end checks it and
 * edges_host[1] receives the number of clouds where it does not hold, in which case the results
 * are invalid and the caller repeats both phases with points_per_cloud = 0 (the general path).
 * Otherwise edges_host[1] is 0.  (geo_radius_count / _dev ignore points_per_cloud when batch is
 * given.)
 */
int geo_radius_count_async(const float* x, int64_t N, const int64_t* batch, int64_t B,
                           int64_t points_per_cloud, const uint8_t* mask, float r2, float r_cell,
                           const double* radius_dev, int64_t max_num_neighbors, int loop,
                           int64_t* row_ptr, int64_t* edges_host, void* workspace,
                           size_t workspace_bytes, void* stream);
int geo_radius_copy_edges(const int64_t* src_row, const int64_t* src_col, int64_t E,
                          int64_t* row_out, int64_t* col_out, void* stream);

/* ---------------------------------------------------- adaptive radius statistic --- */
/*
 * Device-side statistic of column `col` of a KNN distance matrix dist [N, k] (fp32 squared
 * distances), written as one float64 to `out` (device):
 *   mode 0: multiplier * mean of sqrt(clamp(d, 1e-8, 1e20)) with the mean rounded to fp32
 *           (geoembodied/nn/modules/multi_scale_se3_net.py:118-123, without the .item());
 *   mode 1: multiplier * sqrt(lower median of max(d, 1e-12)), NaN if any d is NaN
 *           (geoembodied/nn/modules/equivariant_skip_fusion.py:243-248, without the .item()).
 */
size_t geo_knn_radius_stat_workspace_bytes(int64_t N);
int geo_knn_radius_stat(const float* dist, int64_t N, int64_t k, int64_t col, int mode,
                        double multiplier, double* out, void* workspace, size_t workspace_bytes,
                        void* stream);

/* -------------------------------------------------------------- CSR build --- */
/*
 * Replaces sort_and_build_csr (geoembodied/csrc/segment_reduce_kernel.cu:100-169, bound at
 * :217-221, dispatched from geoembodied/csrc/__init__.py:261-277 and
 * geoembodied/functional/segment_reduce.py:41-109).  Stable sort of col[E] (int64 targets)
 * by target: col_sorted[e] = col[perm[e]], perm ascending within each target.  node_start /
 * node_end[N] are the CSR ranges (empty targets get start == end).  Targets outside [0, N)
 * sort after every valid target and belong to no segment.
 */
size_t geo_csr_workspace_bytes(int64_t E, int64_t N);
int geo_csr_build(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted,
                  int32_t* perm, int32_t* node_start, int32_t* node_end, void* workspace,
                  size_t workspace_bytes, void* stream);
/* geo_csr_build without a workspace argument and without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The radix-sort scratch is a fixed
 * 9 MiB device array inside the library's code object: every GPU on which the library
 * is loaded holds one copy from the load until the process ends, whether or not this entry
 * point is ever called; E is
 * limited to 2^20 = 1,048,576 edges (larger E returns GEO_ERR_INVALID: use geo_csr_build).  The
 * scratch of a GPU is shared by every call on it, so calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.  `stream` must belong to
 * the current device.  Same outputs as geo_csr_build, bit for bit. */
int geo_csr_build_noalloc(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted,
                          int32_t* perm, int32_t* node_start, int32_t* node_end, void* stream);
/* The same four arrays for edges already grouped by target with int64 offsets row_ptr[N+1]
 * (the radius graph's CSR output): perm = identity, col_sorted = int32(col), node_start =
 * row_ptr[:-1], node_end = row_ptr[1:].  Replaces the casts and arange SpatialGraph.build
 * performs on the radius graph's output (geoembodied/nn/modules/spatial_graph.py:126-153). */
int geo_csr_from_row_ptr(const int64_t* row_ptr, int64_t N, const int64_t* col, int64_t E,
                         int32_t* col_sorted, int32_t* perm, int32_t* node_start,
                         int32_t* node_end, void* stream);

/* --------------------------------------------------------- segment reduce --- */
/*
 * Forward.  Replaces segment_reduce_sum (geoembodied/csrc/segment_reduce_kernel.cu:176-210,
 * bound at :222-228, dispatched from geoembodied/csrc/__init__.py:280-302 and the custom op
 * geoembodied/functional/segment_reduce.py:223-238) and adds mean and max, whose semantics
 * follow global_mean_pool (geoembodied/nn/modules/se3_net.py:226-270: sum / max(count, 1)) and
 * scatter_reduce 'amax' with include_self=False on zeros
 * (geoembodied/nn/modules/invariant_attention.py:212-219: empty segment -> 0).
 *
 *   out[s, c] = reduce over e in [node_start[s], node_end[s]) of msg[perm[e], c]
 *
 * msg is [E, C] row-major of `dtype`; perm may be NULL (identity).  Sum and mean accumulate in
 * fp32 (fp64 for GEO_F64) and round once to dtype.  For GEO_REDUCE_MAX, arg[S, C] (int32) is
 * required and receives the sorted position e of the lowest-position maximum when it is
 * unique, -1 for an empty segment and -(tie count) when tie_mode == 0 and the maximum is
 * attained more than once (tie_mode == 1 always stores the lowest position).
 */
int geo_segment_reduce_fwd(int reduce, int dtype, const void* msg, const int32_t* perm,
                           const int32_t* node_start, const int32_t* node_end, int64_t E,
                           int64_t S, int64_t C, void* out, int32_t* arg, int tie_mode,
                           void* stream);

/*
 * Backward.  Replaces the autograd backward of the reference custom op
 * (geoembodied/functional/segment_reduce.py:259-270: grad_msg[perm[e]] = grad_out[col_sorted[e]])
 * and adds mean (grad / max(count, 1)) and max.  Max routes grad_out[s, c] to the recorded
 * argmax; with tie_mode 0 and -(count) recorded it splits grad_out[s, c] evenly over every
 * position whose msg value equals out[s, c] (PyTorch scatter_reduce 'amax' semantics), which
 * needs msg and out; otherwise msg and out may be NULL.  Every row of grad_msg is written.
 */
int geo_segment_reduce_bwd(int reduce, int dtype, const void* grad_out, const void* msg,
                           const void* out, const int32_t* arg, const int32_t* col_sorted,
                           const int32_t* perm, const int32_t* node_start,
                           const int32_t* node_end, int64_t E, int64_t S, int64_t C,
                           void* grad_msg, void* stream);

/* -------------------------------------------------------- segment softmax --- */
/*
 * Replaces _sparse_softmax (geoembodied/nn/modules/invariant_attention.py:202-230: scatter
 * 'amax' per target, exp(score - max), scatter_add, divide by the sum clamped at 1e-8) with one
 * kernel over the CSR of the targets.  scores and out are [E, H] row-major of `dtype` (GEO_F32
 * or GEO_F64); row perm[e] (e in [node_start[s], node_end[s])) belongs to segment s; perm may be
 * NULL (identity).  NaN scores make their segment NaN, as in the reference.  Rows that belong
 * to no segment are not written, except with zero_tail != 0, which states that the node ranges
 * are ascending and contiguous from position 0 (node_start[0] = 0, node_start[s+1] =
 * node_end[s]: the CSR geo_csr_build and the radius graph produce) and writes 0 to the rows
 * perm[e] of the positions e in [node_end[S-1], E) (edges whose target is outside [0, S)), so
 * every row of out is written without a separate fill.
 */
int geo_segment_softmax_fwd(int dtype, const void* scores, const int32_t* perm,
                            const int32_t* node_start, const int32_t* node_end, int64_t E,
                            int64_t S, int64_t H, int zero_tail, void* out, void* stream);
/*
 * Backward of the above (the gradient autograd forms for the reference's op sequence, whose
 * max-shift term cancels analytically): grad_scores[e] = out[e] * (grad_out[e] - sum over the
 * segment of grad_out * out).  zero_tail as in the forward (the tail rows' gradient is 0).
 */
int geo_segment_softmax_bwd(int dtype, const void* grad_out, const void* out,
                            const int32_t* perm, const int32_t* node_start,
                            const int32_t* node_end, int64_t E, int64_t S, int64_t H,
                            int zero_tail, void* grad_scores, void* stream);

/* --------------------------------------------------- neighbourhood gather-sum --- */
/*
 * Fused weighted gather-sum over fixed-width neighbourhoods, replacing the gather + broadcast +
 * sum over an [N_out, K, C] temporary of the interpolation, pooling and skip-fusion layers
 * (geoembodied/nn/modules/equivariant_interp.py:95-125, equivariant_pool.py:412-471,
 * equivariant_skip_fusion.py:304-320):
 *
 *   out[n, :] = sum_k w[n, k] * feat[idx[n, k], :]
 *
 * feat [N_src, C], w [N_out, K] and out [N_out, C] of `dtype` (accumulation in fp32, fp64 for
 * GEO_F64); idx [N_out, K] int64 as KNN returns it: entries outside [0, N_src) (the -1 padding)
 * contribute nothing, so a row without neighbours is 0.  K <= 32.
 */
int geo_gather_weighted_sum(int dtype, const void* feat, int64_t N_src, int64_t C,
                            const int64_t* idx, const void* w, int64_t N_out, int64_t K,
                            void* out, void* stream);
/*
 * Backward.  grad_w[n, k] = <grad_out[n], feat[idx[n, k]]> (0 for padding) when grad_w is
 * non-NULL; grad_feat[j] = sum over the (n, k) with idx[n, k] = j of w[n, k] * grad_out[n] when
 * grad_feat is non-NULL, which needs the CSR of idx over the sources: geo_csr_build of the
 * flattened idx with N = N_src (perm, node_start, node_end).  Every row of each requested
 * gradient is written.
 */
int geo_gather_weighted_sum_bwd(int dtype, const void* grad_out, const void* feat, const void* w,
                                const int64_t* idx, int64_t N_src, int64_t C, int64_t N_out,
                                int64_t K, const int32_t* perm, const int32_t* node_start,
                                const int32_t* node_end, void* grad_feat, void* grad_w,
                                void* stream);
/*
 * Inverse-distance weights of the interpolation layer (equivariant_interp.py:95-99): for each
 * row, v_k = 1 / sqrt(max(dist[n, k], 1e-4)) where idx[n, k] >= 0 (else 0), w = v / max(sum v,
 * 1e-8).  dist and w are fp32 [N_out, K]; K <= 32.
 */
int geo_idw_weights(const int64_t* idx, const float* dist, int64_t N_out, int64_t K, float* w,
                    void* stream);
/*
 * The interpolation layer's whole forward (equivariant_interp.py:95-125) in one launch: the IDW
 * weights of geo_idw_weights, written to w_out (fp32 [N_out, K], for the backward), and the
 * gather-sum of geo_gather_weighted_sum with those weights rounded to `dtype`, bitwise equal
 * to the two calls in turn.
 */
int geo_idw_interpolate(int dtype, const void* feat, int64_t N_src, int64_t C,
                        const int64_t* idx, const float* dist, int64_t N_out, int64_t K,
                        void* out, float* w_out, void* stream);

/* ----------------------------------------------- spatial-graph edge epilogue --- */
/*
 * The per-edge geometry SpatialGraph.build computes after the radius graph
 * (geoembodied/nn/modules/spatial_graph.py:126-153: compute_edge_vectors,
 * geoembodied/functional/radius_graph.py:336-358, then spherical_harmonics,
 * geoembodied/kernels/triton_sph_harm.py:61-198) in one pass per edge:
 *   diff = pos[col] - pos[row], dist[e] = max(|diff|, 1e-8), direction[e] = diff / dist[e],
 *   Y[e] = real spherical harmonics of direction up to max_l <= 2 ((max_l+1)^2 values, order
 *   Y_0^0 | Y_1^{-1,0,1} | Y_2^{-2..2}, orthonormal on the sphere; Y may be NULL).
 * Edges whose endpoints lie outside [0, N) get the geometry of point 0 to itself.
 */
int geo_edge_geometry(const float* pos, int64_t N, const int64_t* row, const int64_t* col,
                      int64_t E, int max_l, float* direction, float* dist, float* Y, void* stream);
/*
 * Gradient of the loss with respect to diff from the gradients of direction, dist and Y (any
 * of them NULL = zero): through the spherical harmonics, then the normalisation (constant
 * dist where the 1e-8 clamp is active).  The caller adds grad_diff to pos[col] and subtracts it
 * from pos[row] (segment sums over the two CSRs).
 */
int geo_edge_geometry_bwd(const float* direction, const float* dist, const float* grad_direction,
                          const float* grad_dist, const float* grad_Y, int64_t E, int max_l,
                          float* grad_diff, void* stream);
/*
 * spherical_harmonics(xyz, max_l, normalize) of geoembodied/kernels/triton_sph_harm.py:322-372:
 * Y [N, (max_l+1)^2] of the rows of xyz [N, 3], normalised first (xyz / max(|xyz|, 1e-8)) when
 * `normalize`; `unit` [N, 3] and `norm` [N] (may be NULL) receive the normalised vectors and
 * clamped norms for the backward.  The backward (not normalised) writes d loss / d xyz from
 * grad_Y; the normalised backward is geo_edge_geometry_bwd with direction = unit, dist = norm.
 */
int geo_spherical_harmonics(const float* xyz, int64_t N, int max_l, int normalize, float* Y,
                            float* unit, float* norm, void* stream);
int geo_spherical_harmonics_bwd(const float* xyz, const float* grad_Y, int64_t N, int max_l,
                                float* grad_xyz, void* stream);
/*
 * Per-node average degree of its cloud (spatial_graph.py:137-152): from the CSR row pointer
 * row_ptr[N+1], integer degree sums and node counts per cloud, avg = sum / max(count, 1) in fp32,
 * clamped below at 1.  Clouds by batch[N] (values outside [0, B) give 1), or contiguous chunks
 * of points_per_cloud when batch is NULL.  out is fp32 [N].
 */
size_t geo_graph_avg_degree_workspace_bytes(int64_t B);
int geo_graph_avg_degree(const int64_t* row_ptr, int64_t N, const int64_t* batch, int64_t B,
                         int64_t points_per_cloud, float* out, void* workspace,
                         size_t workspace_bytes, void* stream);
/* SpatialGraph.build after the radius graph (geoembodied/nn/modules/spatial_graph.py:126-153)
 * in one call: geo_csr_from_row_ptr, geo_edge_geometry and geo_graph_avg_degree on the same
 * stream (workspace: geo_graph_avg_degree_workspace_bytes(B)). */
int geo_spatial_graph_epilogue(const float* pos, int64_t N, const int64_t* row, const int64_t* col,
                               const int64_t* row_ptr, int64_t E, int max_l, const int64_t* batch,
                               int64_t B, int64_t points_per_cloud, float* direction, float* dist,
                               float* Y, int32_t* col_sorted, int32_t* perm, int32_t* node_start,
                               int32_t* node_end, float* avg_degree, void* workspace,
                               size_t workspace_bytes, void* stream);
/* The same epilogue for a radius graph whose edge count the host does not know yet (the same
 * reference lines): launched on the stream right behind geo_radius_emit, it reads
 * E = row_ptr[N] on the device, so it runs while the host waits for E.  row, col and the edge
 * outputs (direction [cap, 3], dist [cap], Y [cap, (max_l+1)^2], col_sorted, perm [cap]) hold
 * cap >= E rows, of which the first E are read and written; node_start, node_end, avg_degree
 * are [N].  The clouds are contiguous runs of points_per_cloud points (N a multiple of it); the
 * average degree of a cloud is its edge count over points_per_cloud, at least 1. */
int geo_spatial_graph_epilogue_dev(const float* pos, int64_t N, const int64_t* row,
                                   const int64_t* col, const int64_t* row_ptr, int64_t cap,
                                   int max_l, int64_t points_per_cloud, float* direction,
                                   float* dist, float* Y, int32_t* col_sorted, int32_t* perm,
                                   int32_t* node_start, int32_t* node_end, float* avg_degree,
                                   void* stream);

/* ------------------------------------------ SE(3) message passing (fused aggregate) --- */
/*
 * The message computation and aggregation of SE3Conv.forward
 * (geoembodied/nn/modules/se3_conv.py:61-235 `_compute_messages`, :482-566), reordered: each of
 * the nine tensor-product paths is r_p(e) * W_p * x_p(e) with W_p shared by all edges, so the
 * r-weighted source features are summed per target node first and the weights applied per node.
 *
 * geo_se3_aggregate_fwd: for each target n (edges p in [node_start[n], node_end[n]) of the CSR,
 * edge perm[p], source row[edge]) writes the per-node sums (rows zero-padded to Ks / Kv / Kt):
 *   Xs[n]    = [A0 (Cs) | A3 (Cv) | A8 (Ct)]
 *   Xv[n][k] = [A1_k (Cs) | A2_k (Cv) | A4_k (Cv)]       k = x, y, z
 *   Xt[n][m] = [A5_m (Cs) | A6_m (Ct) | A7_m (Cv)]       m = 0..4
 * with A0 = sum r0 y0 s, A1_k = sum r1 d_k s, A2_k = sum r2 y0 v_k, A3 = sum r3 (d . v),
 * A4 = sum r4 (d x v), A5_m = sum r5 y2_m s, A6_m = sum r6 y0 t_m,
 * A7_m = sum r7 sum_ij d_i v_j cg[i][j][m], A8 = sum r8 |t|^2.  s [N, Cs], v [N, Cv, 3],
 * t [N, Ct, 5] fp32; dir [E, 3]; Y [E, ysh] (y0 = Y[:, 0], y2 = Y[:, 4:9]); R [E, P];
 * path_cols[9] (host array) = column of R of each path or -1 when the path is off (the
 * reference's runtime path numbering); cg[45] (device array, e.g. the module's cg_11_2 buffer;
 * may be NULL when path 7 is off) = CG(1,1->2) in Cartesian order [3][3][5].  Xs / Xv / Xt may
 * be NULL.
 */
int geo_se3_aggregate_fwd(const float* s, const float* v, const float* t, int64_t N, int32_t Cs,
                          int32_t Cv, int32_t Ct, const int64_t* row, const int32_t* perm,
                          const int32_t* node_start, const int32_t* node_end, int64_t E,
                          const float* dir, const float* Y, int32_t ysh, const float* R, int32_t P,
                          const int32_t* path_cols, const float* cg, float* Xs, int32_t Ks,
                          float* Xv, int32_t Kv, float* Xt, int32_t Kt, void* stream);
/*
 * The forward of one SE3Conv layer from the radial weights on (se3_conv.py:482-566) in one
 * launch: the per-node sums of geo_se3_aggregate_fwd for a tile of 16 target nodes are kept in
 * LDS and multiplied there by the packed weights (fp32 MFMA) with the epilogue of geo_se3_gemm:
 *   s_out[n][o]    = e(n, sum_k Xs[n][k] Ws[o][k]) + bias[o]      o < Os
 *   v_out[n][o][k] = e(n, sum_j Xv[n][k][j] Wv[o][j])             o < Ov, k < 3
 *   t_out[n][o][m] = e(n, sum_j Xt[n][m][j] Wt[o][j])             o < Ot, m < 5
 * with e(n, x) = x / avg[n] (avg may be NULL), 0 where mask[n] == 0 (mask may be NULL; bias may
 * be NULL).  Ws / Wv / Wt: the packed weight blocks of geo_se3_pack_weights (kinds 0-2), 16-byte
 * aligned, at least 16 * ceil(O / 16) rows of Ks / Kv / Kt floats (multiples of 16, at least
 * Cs+Cv+Ct / Cs+2Cv / Cs+Ct+Cv).  A kind with O = 0 is skipped (its pointers may be NULL).
 * Xs / Xv / Xt, when not NULL (16-byte aligned), also receive the aggregate rows in
 * geo_se3_aggregate_fwd's layout (the weight gradients need them).  Other arguments as geo_se3_aggregate_fwd.  The tile must
 * fit 64 KiB of LDS: geo_se3_fwd_fused_lds_bytes returns its size, or 0 when it does not fit
 * (then run geo_se3_aggregate_fwd and geo_se3_gemm).  No reference counterpart as one call: it
 * replaces the message tensor, segment_reduce and output mixing of se3_conv.py:486-566.
 */
size_t geo_se3_fwd_fused_lds_bytes(int32_t Os, int32_t Ov, int32_t Ot, int32_t Ks, int32_t Kv,
                                   int32_t Kt);
int geo_se3_fwd_fused(const float* s, const float* v, const float* t, int64_t N, int32_t Cs,
                      int32_t Cv, int32_t Ct, const int64_t* row, const int32_t* perm,
                      const int32_t* node_start, const int32_t* node_end, int64_t E,
                      const float* dir, const float* Y, int32_t ysh, const float* R, int32_t P,
                      const int32_t* path_cols, const float* cg, const float* Ws, int32_t Ws_rows,
                      const float* Wv, int32_t Wv_rows, const float* Wt, int32_t Wt_rows,
                      int32_t Os, int32_t Ov, int32_t Ot, int32_t Ks, int32_t Kv, int32_t Kt,
                      const float* avg, const float* bias, const uint8_t* mask, float* s_out,
                      float* v_out, float* t_out, float* Xs, float* Xv, float* Xt, void* stream);
/*
 * fp32 MFMA GEMM with the SE3Conv output epilogue (se3_conv.py:547-566): for r < M, o < O,
 *   v = sum_k A[r, k] B[o, k];  v = v / avg[n] (avg may be NULL);  v += bias[o] (may be NULL);
 *   v = 0 where mask[n] == 0 (mask may be NULL);  out[n * out_stride + o * G + g] = v,
 * with n = r / G, g = r % G.  A [M, K] and B [B_rows, K] row-major, 16-byte aligned, K a multiple
 * of 16; B_rows >= O rounded up to the launch's column tile (16, 32 or 64; zero rows past O).
 */
int geo_se3_gemm(const float* A, int64_t M, int32_t K, const float* B, int32_t B_rows, int32_t O,
                 int32_t G, float* out, int64_t out_stride, const float* avg, const float* bias,
                 const uint8_t* mask, void* stream);
/*
 * Backward helpers.  geo_se3_grad_prep: out[n][g][o] (rows of Opad, zero padded) =
 * grad[n][o][g] / avg[n], zero where mask[n] == 0.
 * geo_se3_bwd_edge: per-edge gradients of R (dR [E, P], only the active paths' columns are
 * written), of the direction (ddir [E, 3]) and of Y (dY [E, ysh]: columns 0 and 4..8) from the
 * per-node gradient rows gX (same layouts as Xs / Xv / Xt) and the source features; each may be
 * NULL.  geo_se3_bwd_src: for each source m over the CSR of the sources (col = target of each
 * edge), sums of the prepared output gradients gs [N, OsP], gv [N][3][OvP], gt [N][5][OtP]:
 *   Zs[m] = [Z0 (Os) | Z1 (Ov) | Z5 (Ot)], Zv[m][k] = [Z2_k (Ov) | Z3_k (Os) | Z4_k (Ov) | Z7_k (Ot)],
 *   Zt[m][j] = Z6_j (Ot), Z8[m] (Os)
 * (Z0 = sum r0 y0 gs, Z1 = sum r1 d . gv, Z5 = sum r5 y2 . gt, Z2_k = sum r2 y0 gv_k,
 * Z3_k = sum r3 d_k gs, Z4 = sum r4 gv x d, Z7_j = sum r7 sum_im d_i cg[i][j][m] gt_m,
 * Z6_j = sum r6 y0 gt_j, Z8 = sum r8 gs), from which the feature gradients are GEMMs with the
 * transposed weights.
 */
/*
 * Weight gradients as one long reduction: out[o * ldo + k] = sum_{r < M} A[r * lda + o] *
 * B[r * ldb + k] for o < O, k < K (fp32 MFMA, rows split over the grid, one partial per
 * workgroup in the workspace, partials added in a fixed order).
 */
size_t geo_se3_gemm_tn_workspace_bytes(int64_t M, int32_t O, int32_t K);
int geo_se3_gemm_tn(const float* A, int64_t M, int32_t lda, int32_t O, const float* B, int32_t ldb,
                    int32_t K, float* out, int32_t ldo, void* workspace, size_t workspace_bytes,
                    void* stream);
/*
 * The same product written in column ranges: part j < nsplit (1 to 3) holds columns
 * [cols[j], cols[j + 1]) (cols[0] = 0, cols[nsplit] = K, ascending) as its own row-major
 * O x (cols[j + 1] - cols[j]) matrix at outs[j] (NULL: not written), so that the weight gradients
 * of the paths that share one product land in separate tensors.  Host arrays cols, outs;
 * workspace as for geo_se3_gemm_tn.
 */
int geo_se3_gemm_tn_split(const float* A, int64_t M, int32_t lda, int32_t O, const float* B,
                          int32_t ldb, int32_t K, int32_t nsplit, const int32_t* cols,
                          float* const* outs, void* workspace, size_t workspace_bytes,
                          void* stream);
/*
 * Bias gradient: out[o] = sum of g[n * O + o] over the rows n with mask[n] != 0 (every row when
 * mask is NULL), g row-major [N, O]; rows summed in a fixed order (per-workgroup partials in the
 * workspace, added in workgroup order), so results are reproducible bit for bit.
 */
size_t geo_se3_colsum_workspace_bytes(int64_t N, int32_t O);
int geo_se3_colsum(const float* g, int64_t N, int32_t O, const uint8_t* mask, float* out,
                   void* workspace, size_t workspace_bytes, void* stream);
/*
 * Zero-padded weight blocks for geo_se3_gemm, built in one launch from the nine path weights
 * W[p] ([out][in] row-major fp32 device pointers, NULL for absent paths; path order w_ss, w_sv,
 * w_vv_scalar, w_vs, w_vv_cross, w_st2, w_t2t2, w_vt2, w_t2s).  Output j is a rows[j] x cols[j]
 * block of kind kinds[j]: 0 [W0|W3|W8], 1 [W1|W2|W4], 2 [W5|W6|W7] (rows = outputs), 3-5 their
 * transposes, 6 [W0^T|W1^T|W5^T], 7 [W2^T|W3^T|W4^T|W7^T], 8 W6^T, 9 W8^T (rows = inputs);
 * entries outside the real block are 0.  Host arrays W, out, rows, cols, kinds; nout <= 10.
 */
int geo_se3_pack_weights(const float* const* W, int32_t Cs, int32_t Cv, int32_t Ct, int32_t Os,
                         int32_t Ov, int32_t Ot, int32_t nout, float* const* out,
                         const int32_t* rows, const int32_t* cols, const int32_t* kinds,
                         void* stream);
int geo_se3_grad_prep(const float* grad, int64_t N, int32_t O, int32_t G, int32_t Opad,
                      const float* avg, const uint8_t* mask, float* out, void* stream);
int geo_se3_bwd_edge(const float* s, const float* v, const float* t, int64_t N, int32_t Cs,
                     int32_t Cv, int32_t Ct, const int64_t* row, const int32_t* perm,
                     const int32_t* node_start, const int32_t* node_end, int64_t E,
                     const float* dir, const float* Y, int32_t ysh, const float* R, int32_t P,
                     const int32_t* path_cols, const float* cg, const float* gXs, int32_t Ks,
                     const float* gXv, int32_t Kv, const float* gXt, int32_t Kt, float* dR,
                     float* ddir, float* dY, void* stream);
/*
 * geo_se3_bwd_edge with gX formed on the chip, for layers without type-2 paths (Cs <= 64 and a
 * multiple of 4, Cv <= 16): each workgroup stages its 16 targets' prepared output-gradient rows
 * Gs ([N][OsP]) and Gv ([N][3][OvP]) (OsP, OvP multiples of 16; either NULL) in LDS, multiplies
 * them there by the packed transposed weights WsT ([WsT_rows >= Ks][OsP], pack kind 3) and WvT
 * ([..][OvP], kind 4), 16-byte aligned -- gXs = Gs WsT^T, gXv = Gv WvT^T, bit for bit as the
 * GEMMs of the two-step path -- and walks the targets' edges with those rows.  Returns
 * GEO_ERR_UNSUPPORTED, having done nothing, for layers it does not cover: the caller then forms
 * gX with geo_se3_gemm and calls geo_se3_bwd_edge.
 */
int geo_se3_bwd_edge_fused(const float* s, const float* v, int64_t N, int32_t Cs, int32_t Cv,
                           const int64_t* row, const int32_t* perm, const int32_t* node_start,
                           const int32_t* node_end, int64_t E, const float* dir, const float* Y,
                           int32_t ysh, const float* R, int32_t P, const int32_t* path_cols,
                           const float* cg, const float* Gs, int32_t OsP, const float* Gv,
                           int32_t OvP, const float* WsT, int32_t WsT_rows, const float* WvT,
                           int32_t WvT_rows, int32_t Ks, int32_t Kv, float* dR, float* ddir,
                           float* dY, void* stream);
int geo_se3_bwd_src(const float* gs, int32_t Os, int32_t OsP, const float* gv, int32_t Ov,
                    int32_t OvP, const float* gt, int32_t Ot, int32_t OtP, int64_t N,
                    const int64_t* col, const int32_t* perm, const int32_t* node_start,
                    const int32_t* node_end, int64_t E, const float* dir, const float* Y,
                    int32_t ysh, const float* R, int32_t P, const int32_t* path_cols,
                    const float* cg, float* Zs, int32_t KZs, float* Zv, int32_t KZv, float* Zt,
                    int32_t KZt, float* Z8, int32_t KZ8, void* stream);
/*
 * geo_se3_bwd_src and the feature-gradient GEMMs in one launch, for layers without type-2 paths:
 * each workgroup keeps its 16 sources' Zs / Zv rows (row lengths KZs, KZv, multiples of 16) in LDS
 * and multiplies them there by the packed transposed weights Bs ([Bs_rows >= 16 ceil(Cs / 16)]
 * [KZs], pack kind 6) and Bv ([..][KZv], kind 7), 16-byte aligned:
 *   ds [N, Cs] = Zs Bs^T,  dv [N, Cv, 3] = Zv Bv^T  (either may be NULL).
 * Returns GEO_ERR_UNSUPPORTED, having done nothing, for layers the row kernel does not cover
 * (type-2 paths, Os > 64, Ov > 16, arrays of 2 GiB or more, tiles beyond 64 KB of LDS): the
 * caller then uses geo_se3_bwd_src and the GEMMs.
 */
int geo_se3_bwd_src_fused(const float* gs, int32_t Os, int32_t OsP, const float* gv, int32_t Ov,
                          int32_t OvP, int64_t N, const int64_t* col, const int32_t* perm,
                          const int32_t* node_start, const int32_t* node_end, int64_t E,
                          const float* dir, const float* Y, int32_t ysh, const float* R, int32_t P,
                          const int32_t* path_cols, const float* cg, int32_t KZs, int32_t KZv,
                          const float* Bs, int32_t Bs_rows, int32_t Cs, float* ds, const float* Bv,
                          int32_t Bv_rows, int32_t Cv, float* dv, void* stream);

/*
 * Radial basis MLP of SE3Conv (geoembodied/nn/modules/se3_conv.py:238-282), per edge length d:
 *   x_i = sin(freqs[i] d) / max(d, 1e-8) * max(0.5 (1 + cos((pi d) / cutoff)), 0)   (i < NB)
 *   R[e][p] = b2[p] + sum_j W2[p][j] silu(b1[j] + sum_i W1[j][i] x_i)          (j < H, p < P)
 * fp32, any layer sizes with NB + H <= 12288 and 2 NB + 2 H + P <= 12288 (matrix-core kernels
 * for NB <= 16, H <= 64, P <= 16, LDS-tiled kernels beyond); W1 [H][NB], W2 [P][H] row-major.
 * The backward writes d loss / d dist (d_dist, may be NULL) and the weight gradients (each may
 * be NULL; written, not accumulated) from dR [E, P]; its workspace holds per-block partial sums.
 */
int geo_radial_mlp_fwd(const float* dist, int64_t E, const float* freqs, int32_t NB, float cutoff,
                       const float* W1, const float* b1, int32_t H, const float* W2, const float* b2,
                       int32_t P, float* R, void* stream);
size_t geo_radial_mlp_bwd_workspace_bytes(int64_t E, int32_t NB, int32_t H, int32_t P);
int geo_radial_mlp_bwd(const float* dist, int64_t E, const float* freqs, int32_t NB, float cutoff,
                       const float* W1, const float* b1, int32_t H, const float* W2, const float* b2,
                       int32_t P, const float* dR, float* d_dist, float* dW1, float* db1, float* dW2,
                       float* db2, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GEO_API_H */
