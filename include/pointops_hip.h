/*
 * C ABI of libpointops_hip.so: MI355X (gfx950) kernels for the
 * neighbourhood-search hot path of mps_pointops.
 *
 * Conventions (every entry point):
 *   - All pointers are DEVICE pointers to contiguous row-major arrays owned by
 *     the caller.  The library never allocates device memory, frees or
 *     synchronises; scratch and workspace buffers are passed in (their size
 *     comes from the matching *_bytes query).  The one exception to "holds no
 *     state" is pointops_fps_query_pipeline_f32, which keeps two events per
 *     host thread and device to order its two streams.
 *   - Sizes are int64_t element counts; float arithmetic is IEEE binary32
 *     (binary64 for the *_f64 entries) with no contraction and no fast-math.
 *   - Work is enqueued on `stream`; the return value is hipSuccess or the
 *     error of the launch.  Argument errors return hipErrorInvalidValue
 *     before anything is enqueued.
 *
 * Each entry point replaces one `lib.<kernel>(...)` enqueue of the reference
 * (/root/reference/mps_pointops), cited below as file:line.
 */
#ifndef POINTOPS_HIP_H
#define POINTOPS_HIP_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header (bumped on any signature change). */
int pointops_abi_version(void);

/* Non-zero when `device` is a gfx950 agent this library was built for. */
int pointops_device_supported(int device);

/* ------------------------------------------------------------------ FPS */

/* Dense batched farthest point sampling.  Replaces ops.py:137-140
 * (`_library("fps").furthest_point_sample`, kernels/fps.metal:19-107).
 * xyz (B,N,3) f32 -> out (B,npoint) int64; ties go to the smaller index; once
 * every point is taken the rest repeat the first maximum (index 0).
 * `scratch` must hold pointops_fps_dense_scratch_bytes(B, N) bytes (0 means
 * it may be NULL: the running distances then live on chip). */
size_t pointops_fps_dense_scratch_bytes(int64_t B, int64_t N);
hipError_t pointops_fps_dense(const float *xyz, int64_t *out, void *scratch, int64_t B,
                              int64_t N, int64_t npoint, int64_t start_idx,
                              int32_t skip_near_origin, hipStream_t stream);

/* Large single-cloud FPS (B = 1, 1 <= N <= 2^32 - 1): one persistent
 * cooperative launch over all CUs exchanging per-wave candidates every few
 * steps.  Up to 2^21 points the cloud lives in registers; above, each
 * exchange streams it from HBM with the running distances in the workspace.
 * Replaces the 2*(npoint-1) dispatch loop of ops.py:119-136
 * (kernels/fps_multigroup.metal:10-133).  `workspace` must hold
 * pointops_fps_large_workspace_bytes(N, npoint) bytes (4 bytes per point
 * more above 2^21 points) and be zero-filled by the caller before every
 * call; afterwards its first 32-bit word is non-zero if the kernel gave up
 * waiting for a workgroup (then every output slot not written holds -1). */
size_t pointops_fps_large_workspace_bytes(int64_t N, int64_t npoint);
hipError_t pointops_fps_large(const float *xyz, int64_t *out, void *workspace, int64_t N,
                              int64_t npoint, int64_t start_idx, int32_t skip_near_origin,
                              hipStream_t stream);

/* pointops_fps_large without a workspace argument: allocates nothing.  No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a 640 KiB array in the library's
 * device memory, one per GPU, held until the process ends; each call clears
 * it with a fill kernel on `stream` before the launch.  Limit: 1 <= N <=
 * 2^21 points (the clouds that fit in registers), else hipErrorInvalidValue
 * before anything is enqueued.  Calls that overlap on one GPU (several
 * streams or host threads) share the array and race: serialise them.  A give-up
 * of the kernel shows as -1 in every output slot it did not write. */
hipError_t pointops_fps_large_noalloc(const float *xyz, int64_t *out, int64_t N, int64_t npoint,
                                      int64_t start_idx, int32_t skip_near_origin,
                                      hipStream_t stream);

/* Ragged FPS (torch_cluster layout).  Replaces _flat_fps_mps.py:86-95
 * (kernels/fps_flat.metal:7-96).  Cloud b is x[ptr[b]:ptr[b+1]]; its samples
 * go to out[out_ptr[b]:out_ptr[b+1]] as global indices starting from the
 * local index starts[b].  `max_len` is max_b(ptr[b+1]-ptr[b]); `scratch` must
 * hold pointops_fps_flat_scratch_bytes(total_n, max_len) bytes. */
size_t pointops_fps_flat_scratch_bytes(int64_t total_n, int64_t max_len);
hipError_t pointops_fps_flat(const float *x, const int64_t *ptr, const int64_t *out_ptr,
                             const int64_t *starts, int64_t *out, void *scratch,
                             int64_t batch, int64_t total_n, int64_t max_len,
                             hipStream_t stream);

/* ------------------------------------------------------------------ kNN */

/* Dense exact kNN, D = 3.  Replaces ops.py:195-199 (kernels/knn.metal:32-140).
 * query (B,M,3), ref (B,N,3) -> dist (B,M,K) Euclidean, idx (B,M,K) int64,
 * sorted by (fl32 squared distance, index).  NaN distances never match;
 * unfilled slots are (inf, 4294967295).  1 <= K <= 256. */
hipError_t pointops_knn3(const float *query, const float *ref, float *dist, int64_t *idx,
                         int64_t B, int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* The same search (identical results) over a uniform grid, for large clouds
 * and 1 <= K <= 32: the references and queries are counting-sorted by cell
 * into `workspace` (pointops_knn3_grid_workspace_bytes(B, M, N) bytes, no
 * initialisation needed; B <= 65535) and each query scans the box of cells
 * around it, grown face by face until no unscanned reference can be nearer
 * than its K-th neighbour; queries still unfinished after a few faces are
 * finished inside the call by a scan that skips chunks of the sorted
 * references whose bounding box is too far.  Replaces ops.py:195-199
 * (kernels/knn.metal:32-140), like pointops_knn3. */
size_t pointops_knn3_grid_workspace_bytes(int64_t B, int64_t M, int64_t N);
hipError_t pointops_knn3_grid(const float *query, const float *ref, float *dist, int64_t *idx,
                              void *workspace, int64_t B, int64_t M, int64_t N, int64_t K,
                              hipStream_t stream);
/* Nearest reference per query over the same grid (K = 1; the search of
 * pointops_chamfer_nearest_f32 with norm 2 for clouds without lengths):
 * dist2 (B,M) the squared distance fl32((dx^2 + dy^2) + dz^2), idx (B,M)
 * the smallest index attaining it, identical to the linear scan, for
 * finite coordinates.  Queries whose nearest reference lies more than a few
 * cells away are finished inside the call by a linear scan over their
 * cloud.  `workspace`: pointops_knn3_grid_workspace_bytes(B, M, N); N >= 1,
 * B <= 65535.
 * Accelerates chamfer.py:122-158 for large clouds. */
hipError_t pointops_nearest3_grid(const float *query, const float *ref, float *dist2,
                                  int64_t *idx, void *workspace, int64_t B, int64_t M, int64_t N,
                                  hipStream_t stream);

/* The same search (identical results) for clouds of 1 <= N <= 8192
 * references, M <= 16384 queries and 1 <= K <= 32, faster: one workgroup per
 * cloud counting-sorts the references by Morton cell into `workspace`
 * (pointops_knn3_windowed_workspace_bytes(B, M, N) bytes, no initialisation
 * needed), and each query starts from a limit taken from the references
 * around its own cell in that order, so that only references at least that
 * near are buffered and merged.  Replaces ops.py:195-199
 * (kernels/knn.metal:32-140), like pointops_knn3. */
size_t pointops_knn3_windowed_workspace_bytes(int64_t B, int64_t M, int64_t N);
hipError_t pointops_knn3_windowed(const float *query, const float *ref, float *dist, int64_t *idx,
                                  void *workspace, int64_t B, int64_t M, int64_t N, int64_t K,
                                  hipStream_t stream);

/* Dense exact kNN in D dimensions (sequential per-dimension accumulation).
 * Replaces ops.py:200-204 (kernels/feature_knn.metal:133-164).  Non-finite
 * queries and non-finite distances never match; unfilled slots are (inf, -1). */
hipError_t pointops_knn_feat(const float *query, const float *ref, float *dist, int64_t *idx,
                             int64_t B, int64_t M, int64_t N, int64_t D, int64_t K,
                             hipStream_t stream);

/* Flat (ragged) kNN, global x indices padded with -1, (Q,K).  Replaces
 * _flat_search_mps.py:96-107 (kernels/flat_search.metal:44-154 for D = 3,
 * kernels/feature_knn.metal:166-199 otherwise).  y (Q,D) queries, x (Nx,D)
 * references, ptr_y/ptr_x (batch+1,) segment offsets. */
hipError_t pointops_knn_flat(const float *y, const float *x, const int64_t *ptr_y,
                             const int64_t *ptr_x, int64_t *out, int64_t Q, int64_t batch,
                             int64_t D, int64_t K, hipStream_t stream);

/* ----------------------------------------------------------- ball query */

/* Dense first-K ball query (PyTorch3D convention).  Replaces
 * _ball_query_mps.py:139-162 (kernels/ball_query.metal:126-166).  The first K
 * points j in input order with fl32((dx^2+dy^2)+dz^2) < radius_sq; empty
 * slots are (idx -1, dist2 0).  Queries at or beyond query_lengths[b] are
 * padding; only points below point_lengths[b] are scanned (either lengths
 * pointer may be NULL: every query / point is valid).  The _f16 entry takes
 * IEEE half coordinates (uint16 bit patterns) widened exactly. */
hipError_t pointops_ball_query_f32(const float *queries, const float *points,
                                   const int64_t *query_lengths, const int64_t *point_lengths,
                                   int64_t *idx, float *dist2, int64_t B, int64_t Q, int64_t P,
                                   int64_t K, float radius_sq, hipStream_t stream);
hipError_t pointops_ball_query_f16(const uint16_t *queries, const uint16_t *points,
                                   const int64_t *query_lengths, const int64_t *point_lengths,
                                   int64_t *idx, float *dist2, int64_t B, int64_t Q, int64_t P,
                                   int64_t K, float radius_sq, hipStream_t stream);
/* Ball queries of nball (<= 8) radii around the same queries in one scan
 * per kBqMulti = 4 radii: each radius r's (idx[r], dist2[r]) of shape
 * (B,Q,ks[r]) equals pointops_ball_query_f32(queries, points, NULL, NULL,
 * idx[r], dist2[r], B, Q, P, ks[r], radii_sq[r]) bit for bit (first ks[r]
 * hits in index order, d < radius_sq, -1 / 0 padding); a radius with
 * ks[r] == 0 writes nothing.  Each pair's distance is computed once for all
 * radii, and a scan stops when every radius has its hits.  The arrays
 * radii_sq, ks, idx and dist2 are host arrays of nball entries; B <= 65535.
 * A multi-scale-grouping layer asks several radii around one set of centres
 * (the config-2 workload: r = 0.1, 0.2, 0.4 with K = 16, 32, 128): this
 * replaces its per-radius ops.ball_query calls (ops.py:208-227, one
 * _ball_query_mps.py:139-162 call each). */
hipError_t pointops_ball_query_multi_f32(const float *queries, const float *points, int64_t nball,
                                         const float *radii_sq, const int64_t *ks,
                                         int64_t *const *idx, float *const *dist2, int64_t B,
                                         int64_t Q, int64_t P, hipStream_t stream);
/* The same float32 query without lengths in pointnet2_ops' form: int32
 * indices only, (B,Q,K), slots past the hits repeating the query's first hit
 * and all 0 for a query without one.  Replaces compat.py:76-85 (the ball
 * query, its -1 -> first-neighbour padding and int32 conversion) in one
 * launch; B <= 65535. */
hipError_t pointops_ball_query_pn2_f32(const float *queries, const float *points, int32_t *idx,
                                       int64_t B, int64_t Q, int64_t P, int64_t K, float radius_sq,
                                       hipStream_t stream);
/* The same query (identical results) over the uniform grid of
 * pointops_knn3_grid, for large clouds without lengths, 1 <= K <= 64, P >= 1:
 * each query scans the cells that cover its ball and keeps its K smallest
 * indices.  `workspace`: pointops_ball_query_grid_workspace_bytes(B, Q, P)
 * bytes, no initialisation needed; B <= 65535.  Replaces
 * _ball_query_mps.py:139-162 for that case. */
size_t pointops_ball_query_grid_workspace_bytes(int64_t B, int64_t Q, int64_t P);
hipError_t pointops_ball_query_grid_f32(const float *queries, const float *points, int64_t *idx,
                                        float *dist2, void *workspace, int64_t B, int64_t Q,
                                        int64_t P, int64_t K, float radius_sq, hipStream_t stream);
/* The ball query of pointops_ball_query_f32 without lengths (identical
 * results), choosing on the device between the grid search above and the
 * index-order scan: from the grid build's bounding boxes it estimates the
 * points per ball, lambda = P (4/3) pi r^3 / V (V the smallest per-cloud box
 * volume, each side at least 2r), and takes the grid when lambda <
 * sqrt(P K / 6.4); the other search's launches return at once.  No host
 * synchronisation, so the call can be captured in a HIP graph.  After the
 * call the first int32 of `workspace` holds the choice (1 grid, 0 index
 * order).  `workspace`: pointops_ball_query_auto_workspace_bytes(B, Q, P)
 * bytes, no initialisation needed; 1 <= K <= 64, B <= 65535.  Replaces
 * _ball_query_mps.py:139-162 for that case. */
size_t pointops_ball_query_auto_workspace_bytes(int64_t B, int64_t Q, int64_t P);
hipError_t pointops_ball_query_auto_f32(const float *queries, const float *points, int64_t *idx,
                                        float *dist2, void *workspace, int64_t B, int64_t Q,
                                        int64_t P, int64_t K, float radius_sq, hipStream_t stream);

/* Backward of the dense ball query: the gradients of dist2 (B,Q,K) with
 * respect to queries (B,Q,3) and points (B,P,3), float32, from the forward's
 * idx.  Replaces _ball_query_mps.py:168-203 (gather, masking and scatter_add
 * in PyTorch).  A slot with idx in [0, P) contributes c = (2 g) (q - p) per
 * axis; padded slots contribute nothing.  grad_queries[b,q] = the row's c
 * summed as ((s0 + s1) + s2) + s3, s_l the sum in order of the slots
 * k = l (mod 4); grad_points[b,j] = -(the c of the slots holding j),
 * summed in row order within 8 contiguous row segments, then over the
 * segments in order: the same bits on every run.  Either gradient pointer
 * may be NULL (not computed); every element of a non-NULL one is written.
 * `workspace`: pointops_ball_query_backward_workspace_bytes(B, Q) bytes (per
 * row its smallest and largest index), no initialisation needed.  The _f16
 * entry takes IEEE half coordinates (uint16 bit patterns), widened exactly;
 * the gradients stay float32. */
size_t pointops_ball_query_backward_workspace_bytes(int64_t B, int64_t Q);
hipError_t pointops_ball_query_backward_f32(const float *queries, const float *points,
                                            const int64_t *idx, const float *grad_dist2,
                                            float *grad_queries, float *grad_points,
                                            void *workspace, int64_t B, int64_t Q, int64_t P,
                                            int64_t K, hipStream_t stream);
hipError_t pointops_ball_query_backward_f16(const uint16_t *queries, const uint16_t *points,
                                            const int64_t *idx, const float *grad_dist2,
                                            float *grad_queries, float *grad_points,
                                            void *workspace, int64_t B, int64_t Q, int64_t P,
                                            int64_t K, hipStream_t stream);

/* Flat radius search (torch_cluster convention): first K global x indices
 * with squared distance < radius_sq, padded with -1, (Q,K); optional
 * exclusion of x index == y index before the cap.  Replaces
 * _flat_search_mps.py:134-146 (kernels/flat_search.metal:229-275). */
hipError_t pointops_radius_flat_f32(const float *y, const float *x, const int64_t *ptr_y,
                                    const int64_t *ptr_x, int64_t *out, int64_t Q,
                                    int64_t batch, int64_t K, float radius_sq,
                                    int32_t ignore_same_index, hipStream_t stream);
hipError_t pointops_radius_flat_f16(const uint16_t *y, const uint16_t *x, const int64_t *ptr_y,
                                    const int64_t *ptr_x, int64_t *out, int64_t Q,
                                    int64_t batch, int64_t K, float radius_sq,
                                    int32_t ignore_same_index, hipStream_t stream);

/* ------------------------------------------------- PointNet++ propagation */

/* Three nearest known points per unknown point (stable index order on equal
 * squared distance, NaN last).  Replaces pointnet2.py:94-99
 * (kernels/pointnet2.metal:8-50).  unknown (B,N,3), known (B,M,3), M >= 3 ->
 * dist (B,N,3) Euclidean, idx (B,N,3) int32. */
hipError_t pointops_three_nn(const float *unknown, const float *known, float *dist,
                             int32_t *idx, int64_t B, int64_t N, int64_t M, hipStream_t stream);

/* out[b,c,n] = (f[b,c,i0]*w0 + f[b,c,i1]*w1) + f[b,c,i2]*w2.  Replaces
 * pointnet2.py:156-162 (kernels/pointnet2.metal:52-71).  features (B,C,M),
 * idx (B,N,3) int32 in [0,M), weights (B,N,3) -> out (B,C,N). */
hipError_t pointops_three_interpolate(const float *features, const int32_t *idx,
                                      const float *weights, float *out, int64_t B, int64_t C,
                                      int64_t M, int64_t N, hipStream_t stream);

/* grad_features[b,c,i_t] += grad_out[b,c,n] * w[b,n,t].  For M <= 1024 and
 * N <= 6826 each element is summed in (n, t) order, the order of a
 * sequential loop (deterministic); otherwise by float atomics, whose order,
 * hence the last bits, is not deterministic.  The caller zero-fills
 * grad_features.  Replaces pointnet2.py:179-186
 * (kernels/pointnet2.metal:85-103). */
hipError_t pointops_three_interpolate_backward(const float *grad_out, const int32_t *idx,
                                               const float *weights, float *grad_features,
                                               int64_t B, int64_t C, int64_t M, int64_t N,
                                               hipStream_t stream);
/* The same gradient in a fixed order (deterministic), for M <= 4096 known
 * points and N <= 4096 unknowns with N % 4 == 0 (grad_out 16-byte aligned),
 * without atomics.  A known point's terms fl32(grad_out * w) are taken in
 * (n, t) order; with M <= 1024 the batch's entries sorted by (known index,
 * n, t) are cut into pieces at every 12th position, each piece summed from
 * +0 in order and a point's pieces added in order (every lane of the kernel
 * sums 12 entries however long the lists are); with more known points the
 * terms are added one by one.  A CSR of the entries by known index is built in
 * `workspace` (256-byte aligned,
 * pointops_three_interpolate_backward_workspace_bytes(B, M, N) bytes, no
 * initialisation needed), then every element of grad_features is written
 * once (it need not be zero-filled).  Indices outside [0, M) contribute
 * nothing.  Replaces pointnet2.py:179-186 (kernels/pointnet2.metal:85-103). */
size_t pointops_three_interpolate_backward_workspace_bytes(int64_t B, int64_t M, int64_t N);
hipError_t pointops_three_interpolate_backward_csr(const float *grad_out, const int32_t *idx,
                                                   const float *weights, float *grad_features,
                                                   void *workspace, int64_t B, int64_t C,
                                                   int64_t M, int64_t N, hipStream_t stream);
/* The two halves of pointops_three_interpolate_backward_csr, so that the CSR
 * can be built when the forward runs (the indices and weights are known
 * then) and the backward only gathers: _csr_build writes the CSR of
 * (idx, weights) into `workspace` (as above); _backward_from_csr reads it
 * and writes grad_features, the same bits as the combined call.  The
 * workspace must hold a CSR built with the same B, M and N on the same
 * stream (or one ordered before it).  Same limits as the combined call.
 * Replace the same reference code (pointnet2.py:179-186). */
hipError_t pointops_three_interpolate_csr_build(const int32_t *idx, const float *weights,
                                               void *workspace, int64_t B, int64_t M, int64_t N,
                                               hipStream_t stream);
hipError_t pointops_three_interpolate_backward_from_csr(const float *grad_out,
                                                        const void *workspace,
                                                        float *grad_features, int64_t B,
                                                        int64_t C, int64_t M, int64_t N,
                                                        hipStream_t stream);

/* --------------------------------------------------- PointNet++ grouping */

/* out[b,c,p] = features[b,c,idx[b,p]]: features (B,C,N), idx (B,P) int32
 * (idx_bits 32) or int64 (64) in [0,N) -> out (B,C,P).  With P = npoint it is
 * gather_operation, with P = npoint*nsample (idx (B,npoint,nsample) read
 * flat) grouping_operation; both replace compat.py:62-73 (torch.gather along
 * the point axis).  Indices outside [0,N) are clamped (callers check them). */
hipError_t pointops_group_points(const float *features, const void *idx, int idx_bits, float *out,
                                 int64_t B, int64_t C, int64_t N, int64_t P, hipStream_t stream);

/* The gradient of that gather (compat.py:62-73, torch.gather's scatter-add):
 * grad_features[b,c,n] = the float sum of grad_out[b,c,p] over the p with
 * idx[b,p] = n; 0 for a point never gathered; every element is written.
 * For a point gathered at most 256 times the sum is deterministic: with
 * P <= 32768 and N <= 4096 the batch's entries sorted by (n, p) are cut
 * into pieces at every 32nd position, each piece is summed from +0 in
 * increasing p and a point's pieces are added in order (so that every lane
 * of the kernel sums 32 entries however long the lists are); otherwise
 * the terms are added in increasing p.  A point gathered more often sums
 * in an unspecified order.  grad_out channel c of batch b starts
 * at grad_out + b*grad_batch_stride + c*P (grad_batch_stride >= C*P, so a
 * channel slice of a larger tensor can be passed).  `workspace` holds
 * pointops_group_points_backward_workspace_bytes(B, C, N, P) bytes (the
 * inverse index and a transposed copy of grad_out; no initialisation
 * needed). */
size_t pointops_group_points_backward_workspace_bytes(int64_t B, int64_t C, int64_t N, int64_t P);
hipError_t pointops_group_points_backward(const float *grad_out, int64_t grad_batch_stride,
                                          const void *idx, int idx_bits, float *grad_features,
                                          void *workspace, int64_t B, int64_t C, int64_t N,
                                          int64_t P, hipStream_t stream);

/* Fused set-abstraction grouping (tests/test_pointnet2_e2e.py:36-45, the
 * QueryAndGroup step after compat.ball_query): out (B,3+C,M,S) with
 * channels 0-2 = xyz[b,idx[b,m,s],a] - centres[b,m,a] and channels 3.. =
 * features[b,c,idx[b,m,s]].  xyz (B,N,3), centres (B,M,3), features (B,C,N)
 * (may be NULL when C = 0), idx (B,M,S) int32/int64 in [0,N).  Replaces the
 * two grouping_operation calls, the subtraction and the concatenation of
 * that layer. */
hipError_t pointops_group_points_rel(const float *xyz, const float *centres, const float *features,
                                     const void *idx, int idx_bits, float *out, int64_t B,
                                     int64_t C, int64_t N, int64_t M, int64_t S,
                                     hipStream_t stream);

/* -------------------------------------------------------------- Chamfer */

/* Nearest reference per query (K = 1), first minimum index on ties, under
 * squared L2 (norm 2) or L1 (norm 1) in D dimensions.  Replaces
 * chamfer.py:136-157 (kernels/chamfer_nn.metal:13-226).  Rows at or beyond
 * query_lengths[b] and rows of an empty reference cloud are (0, -1). */
hipError_t pointops_chamfer_nearest_f32(const float *query, const float *ref,
                                        const int64_t *query_lengths,
                                        const int64_t *ref_lengths, float *dist, int64_t *idx,
                                        int64_t B, int64_t Q, int64_t R, int64_t D,
                                        int32_t norm, hipStream_t stream);
hipError_t pointops_chamfer_nearest_f64(const double *query, const double *ref,
                                        const int64_t *query_lengths,
                                        const int64_t *ref_lengths, double *dist, int64_t *idx,
                                        int64_t B, int64_t Q, int64_t R, int64_t D,
                                        int32_t norm, hipStream_t stream);

/* Chamfer backward for selected pairs.  norm 2: gq = (q - ref[idx]) * (2 g);
 * norm 1: gq = (q > ref[idx] ? 1 : -1) * g; grad_ref[idx] -= gq (float
 * atomics).  Rows with idx < 0 get 0.  The caller zero-fills grad_ref.
 * Replaces the PyTorch gather/scatter_add_ of chamfer.py:227-294. */
hipError_t pointops_chamfer_backward_f32(const float *query, const float *ref,
                                         const int64_t *idx, const float *grad_dist,
                                         float *grad_query, float *grad_ref, int64_t B,
                                         int64_t Q, int64_t R, int64_t D, int32_t norm,
                                         hipStream_t stream);
hipError_t pointops_chamfer_backward_f64(const double *query, const double *ref,
                                         const int64_t *idx, const double *grad_dist,
                                         double *grad_query, double *grad_ref, int64_t B,
                                         int64_t Q, int64_t R, int64_t D, int32_t norm,
                                         hipStream_t stream);

/* A set-abstraction front end in one call, with the queries overlapped with
 * sampling: furthest_point_sample (ops.py:53-141; dense, 1 <= npoint <= N <=
 * 8192, B <= 65535), the centres gathered from the samples (the caller's
 * xyz.gather of the reference's tests/test_pointnet2_e2e.py:36-45), then for
 * every centre `nball` first-K ball queries (ops.py:208-227; radius_sq[r] as
 * pointops_ball_query_f32 takes it, ball_k[r] slots, no lengths) and an
 * exact kNN of knn_k <= 32 neighbours (ops.py:144-205; Euclidean distances),
 * each output (B, npoint, K) as the separate entry points write it, bit for
 * bit.  FPS runs on `fps_stream` and publishes its progress every `chunk`
 * samples; the ball queries of each chunk of centres run on `query_stream` as
 * soon as every cloud has sampled it, and kNN once after the last chunk
 * (`workspace` sized for all npoint centres).  The caller orders fps_stream
 * after the producer of xyz; the call orders query_stream after its own
 * clear of the workspace's progress words and of `status` (a kernel on
 * fps_stream, then an event), and fps_stream after its last query (an
 * event), so work queued on fps_stream afterwards sees every output.  Two
 * events per host thread and device are created on first use and kept.
 * `workspace` (pointops_fps_query_pipeline_workspace_bytes bytes, no
 * initialisation needed) and `status` (one word) belong to one call until
 * fps_stream has passed it: calls that overlap need distinct ones.  FPS
 * stores each centre in the workspace before publishing it and a gate (one
 * wave per cloud) copies the chunk's centres out.  A gate wave reads its
 * cloud's progress word at most 2^24 times (or POINTOPS_PIPELINE_SPIN_LIMIT
 * times, read per call; 0 makes it give up at once).  A wave that gives up,
 * and every wave of a later gate, sets `status` non-zero and writes NaN
 * centres for its cloud's chunk, whose queries then return the results for
 * a NaN query (ball query (0, -1), kNN (inf, 2^32 - 1)); the samples stay
 * exact.  No counterpart in the
 * reference, which runs these steps one after another. */
size_t pointops_fps_query_pipeline_workspace_bytes(int64_t B, int64_t N, int64_t npoint,
                                                   int64_t chunk);
hipError_t pointops_fps_query_pipeline_f32(
    const float *xyz, int64_t *samples, float *centres, int64_t nball, const float *radii_sq,
    const int64_t *ball_k, int64_t *const *ball_idx, float *const *ball_dist2, int64_t knn_k,
    float *knn_dist, int64_t *knn_idx, void *workspace, uint32_t *status, int64_t B, int64_t N,
    int64_t npoint, int64_t start_idx, int32_t skip_near_origin, int64_t chunk,
    hipStream_t fps_stream, hipStream_t query_stream);

#ifdef __cplusplus
}
#endif

#endif /* POINTOPS_HIP_H */
