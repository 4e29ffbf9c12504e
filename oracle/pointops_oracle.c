/*
 * CPU restatement of the reference's neighbourhood-search arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package links, loads or
 * calls this file: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * Build: gcc -O2 -std=c11 -fPIC -shared -ffp-contract=off -fno-fast-math
 *        -fopenmp (see oracle/Makefile).  Every float operation below is one
 * IEEE binary32 operation rounded to nearest-even, in the order written,
 * because contraction is off and there is no fast-math: that is exactly the
 * rounding sequence of the reference's separately rounded tensor ops.
 *
 * Reference files are cited relative to /root/reference/mps_pointops/.
 * Parity pinning of each function is listed in the oracle/oracle.py header.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define PAD_UINT32_AS_I64 4294967295LL

/* ((dx*dx + dy*dy) + dz*dz) with d = a - b: reference.py:21-24 (_sqdist). */
static inline float sqdist3(const float *a, const float *b) {
    float dx = a[0] - b[0];
    float dy = a[1] - b[1];
    float dz = a[2] - b[2];
    float d = dx * dx;
    d = d + dy * dy;
    d = d + dz * dz;
    return d;
}

/* torch.minimum semantics (propagates NaN). */
static inline float torch_minimum(float a, float b) {
    if (isnan(a) || isnan(b)) return NAN;
    return a < b ? a : b;
}

/* (d, i) strictly before (e, j): smaller distance, then smaller index.
 * kernels/knn.metal:27-30 (`before`). NaN is never before anything. */
static inline int before(float d, int64_t i, float e, int64_t j) {
    return d < e || (d == e && i < j);
}

/* ------------------------------------------------------------------ FPS */

/*
 * reference.py:27-58 (furthest_point_sample).  For each cloud:
 *   min_d2 = +inf; skipped points (mag < fl32(1e-3), reference.py:46-50) = -inf
 *   farthest = start
 *   for i: idx[i] = farthest
 *          min_d2 = minimum(min_d2, sqdist(xyz, xyz[farthest]))
 *          farthest = argmax(min_d2)   (first maximum; NaN counts as maximum,
 *                                       like torch.argmax)
 * `min_d2` is caller-provided scratch of N floats per thread team.
 */
static void fps_one(const float *p, int64_t N, int64_t npoint, int64_t start,
                    int skip, int64_t *out) {
    float *md = (float *)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
    const float zero[3] = {0.f, 0.f, 0.f};
    const float thr = 1e-3f; /* torch.tensor(1e-3, dtype=float32) */
    for (int64_t j = 0; j < N; ++j) {
        md[j] = INFINITY;
        if (skip && sqdist3(p + 3 * j, zero) < thr) md[j] = -INFINITY;
    }
    int64_t far = start;
    for (int64_t i = 0; i < npoint; ++i) {
        out[i] = far;
        const float *c = p + 3 * far;
        int64_t best = 0;
        float bv = 0.f;
        int have = 0, best_nan = 0;
        for (int64_t j = 0; j < N; ++j) {
            float m = torch_minimum(md[j], sqdist3(p + 3 * j, c));
            md[j] = m;
            if (best_nan) continue;
            if (isnan(m)) { best = j; best_nan = 1; continue; }
            if (!have || m > bv) { bv = m; best = j; have = 1; }
        }
        far = best;
    }
    free(md);
}

/* Parallel variant for one large cloud: the per-step argmax is reduced
 * over thread-local first maxima, then the lowest index among equal maxima. */
static void fps_one_parallel(const float *p, int64_t N, int64_t npoint,
                             int64_t start, int skip, int64_t *out) {
#ifdef _OPENMP
    float *md = (float *)malloc(sizeof(float) * (size_t)N);
    const float zero[3] = {0.f, 0.f, 0.f};
    const float thr = 1e-3f;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < N; ++j) {
        md[j] = INFINITY;
        if (skip && sqdist3(p + 3 * j, zero) < thr) md[j] = -INFINITY;
    }
    int nt = omp_get_max_threads();
    float *tv = (float *)malloc(sizeof(float) * nt);
    int64_t *ti = (int64_t *)malloc(sizeof(int64_t) * nt);
    int *tn = (int *)malloc(sizeof(int) * nt);
    int64_t far = start;
    for (int64_t i = 0; i < npoint; ++i) {
        out[i] = far;
        const float c[3] = {p[3 * far], p[3 * far + 1], p[3 * far + 2]};
#pragma omp parallel
        {
            int t = omp_get_thread_num();
            int T = omp_get_num_threads();
            int64_t lo = N * t / T, hi = N * (t + 1) / T;
            float bv = 0.f;
            int64_t bi = -1;
            int isn = 0;
            for (int64_t j = lo; j < hi; ++j) {
                float m = torch_minimum(md[j], sqdist3(p + 3 * j, c));
                md[j] = m;
                if (isn) continue;
                if (isnan(m)) { bi = j; isn = 1; continue; }
                if (bi < 0 || m > bv) { bv = m; bi = j; }
            }
            tv[t] = bv; ti[t] = bi; tn[t] = isn;
            if (t == 0) {
                for (int u = T; u < nt; ++u) ti[u] = -1;
            }
        }
        /* Threads own increasing index ranges, so the first thread that
         * holds the overall maximum (or the first NaN) owns the first index. */
        int64_t best = 0;
        float bv = 0.f;
        int have = 0;
        for (int u = 0; u < nt; ++u) {
            if (ti[u] < 0) continue;
            if (tn[u]) { best = ti[u]; break; }
            if (!have || tv[u] > bv) { bv = tv[u]; best = ti[u]; have = 1; }
        }
        far = best;
    }
    free(tv); free(ti); free(tn); free(md);
#else
    fps_one(p, N, npoint, start, skip, out);
#endif
}

void oracle_fps(const float *xyz, int64_t B, int64_t N, int64_t npoint,
                int64_t start, int skip, int64_t *out) {
    if (B == 1 && N >= (1 << 16)) {
        fps_one_parallel(xyz, N, npoint, start, skip, out);
        return;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t b = 0; b < B; ++b)
        fps_one(xyz + 3 * N * b, N, npoint, start, skip, out + npoint * b);
}

/*
 * Ragged FPS with torch_cluster's layout: cloud b is x[ptr[b]:ptr[b+1]],
 * its samples go to out[out_ptr[b]:out_ptr[b+1]] as GLOBAL indices, starting
 * at the LOCAL index starts[b].  flat.py:209-217 runs reference.py's FPS per
 * segment (no near-origin skip); kernels/fps_flat.metal:7-96 is the same rule.
 */
void oracle_fps_flat(const float *x, const int64_t *ptr, const int64_t *out_ptr,
                     const int64_t *starts, int64_t batch, int64_t *out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t b = 0; b < batch; ++b) {
        int64_t lo = ptr[b], n = ptr[b + 1] - ptr[b];
        int64_t olo = out_ptr[b], cnt = out_ptr[b + 1] - out_ptr[b];
        if (cnt <= 0) continue;
        fps_one(x + 3 * lo, n, cnt, starts[b], 0, out + olo);
        for (int64_t i = 0; i < cnt; ++i) out[olo + i] += lo;
    }
}

/* ------------------------------------------------------------------ kNN */

/* Insert (d, j) into the sorted (by `before`) list of length k if it beats
 * the last entry.  The result is the k smallest keys seen. */
static inline void topk_insert(float *ld, int64_t *li, int64_t k, float d, int64_t j) {
    if (!before(d, j, ld[k - 1], li[k - 1])) return;
    int64_t s = k - 1;
    while (s > 0 && before(d, j, ld[s - 1], li[s - 1])) {
        ld[s] = ld[s - 1];
        li[s] = li[s - 1];
        --s;
    }
    ld[s] = d;
    li[s] = j;
}

/*
 * Dense 3-D exact kNN with the reference kernel's semantics
 * (kernels/knn.metal:32-140, ops.py:144-205; exact oracle tests/test_knn.py:15-23):
 * key (fl32 ((dx^2+dy^2)+dz^2) with d = ref - query, index); the k smallest
 * keys ascending; a NaN distance is never a candidate; unfilled slots keep
 * (inf, 2^32-1).  dist = sqrt(d2).
 */
void oracle_knn3(const float *query, const float *ref, int64_t B, int64_t M,
                 int64_t N, int64_t K, float *dist, int64_t *idx) {
    if (K <= 0) return;
#pragma omp parallel
    {
        float *ld = (float *)malloc(sizeof(float) * K);
        int64_t *li = (int64_t *)malloc(sizeof(int64_t) * K);
#pragma omp for schedule(dynamic, 16)
        for (int64_t bq = 0; bq < B * M; ++bq) {
            int64_t b = bq / M;
            const float *q = query + 3 * bq;
            const float *r = ref + 3 * N * b;
            for (int64_t s = 0; s < K; ++s) { ld[s] = INFINITY; li[s] = PAD_UINT32_AS_I64; }
            for (int64_t j = 0; j < N; ++j) {
                float d = sqdist3(r + 3 * j, q);
                if (isnan(d)) continue;
                topk_insert(ld, li, K, d, j);
            }
            for (int64_t s = 0; s < K; ++s) {
                dist[bq * K + s] = sqrtf(ld[s]);
                idx[bq * K + s] = li[s];
            }
        }
        free(ld); free(li);
    }
}

/* Sequential D-dim squared L2: s = d0^2; s = s + dt^2 for t = 1..D-1 with
 * dt = ref - query (kernels/feature_knn.metal:82-90, docs/feature-knn.md). */
static inline float sqdist_nd(const float *r, const float *q, int64_t D) {
    float first = r[0] - q[0];
    float s = first * first;
    for (int64_t t = 1; t < D; ++t) {
        float delta = r[t] - q[t];
        float term = delta * delta;
        s = s + term;
    }
    return s;
}

static int all_finite(const float *v, int64_t n) {
    for (int64_t t = 0; t < n; ++t)
        if (!isfinite(v[t])) return 0;
    return 1;
}

/*
 * Dense D-dim exact kNN (ops.py:200-204 -> kernels/feature_knn.metal:133-164;
 * oracle tests/test_feature_knn.py:16-35): non-finite queries and non-finite
 * distances never match; unfilled slots are (inf, -1).
 */
void oracle_knn_feat(const float *query, const float *ref, int64_t B, int64_t M,
                     int64_t N, int64_t D, int64_t K, float *dist, int64_t *idx) {
    if (K <= 0) return;
#pragma omp parallel
    {
        float *ld = (float *)malloc(sizeof(float) * K);
        int64_t *li = (int64_t *)malloc(sizeof(int64_t) * K);
#pragma omp for schedule(dynamic, 16)
        for (int64_t bq = 0; bq < B * M; ++bq) {
            int64_t b = bq / M;
            const float *q = query + D * bq;
            const float *r = ref + D * N * b;
            for (int64_t s = 0; s < K; ++s) { ld[s] = INFINITY; li[s] = -1; }
            if (all_finite(q, D)) {
                for (int64_t j = 0; j < N; ++j) {
                    float d = sqdist_nd(r + D * j, q, D);
                    if (!isfinite(d)) continue;
                    topk_insert(ld, li, K, d, j);
                }
            }
            for (int64_t s = 0; s < K; ++s) {
                dist[bq * K + s] = sqrtf(ld[s]);
                idx[bq * K + s] = li[s];
            }
        }
        free(ld); free(li);
    }
}

/* Segment of a flat query by ptr (first b with ptr[b+1] > q). */
static inline int64_t segment_of(const int64_t *ptr, int64_t batch, int64_t q) {
    int64_t lo = 0, hi = batch;
    while (lo < hi) {
        int64_t mid = lo + (hi - lo) / 2;
        if (ptr[mid + 1] <= q) lo = mid + 1; else hi = mid;
    }
    return lo;
}

/*
 * Flat (torch_cluster) kNN indices, (Q, K) global indices padded with -1:
 * flat.py:264-288 (_reference_search, stable argsort of finite d2, D-dim
 * accumulation flat.py:256-261 with d = refs - query) and
 * kernels/flat_search.metal:140-250 / kernels/feature_knn.metal:166-199.
 * A non-finite query has no neighbours.
 */
void oracle_knn_flat(const float *y, const float *x, const int64_t *ptr_y,
                     const int64_t *ptr_x, int64_t Q, int64_t batch, int64_t D,
                     int64_t K, int64_t *out) {
    if (K <= 0) return;
#pragma omp parallel
    {
        float *ld = (float *)malloc(sizeof(float) * K);
        int64_t *li = (int64_t *)malloc(sizeof(int64_t) * K);
#pragma omp for schedule(dynamic, 16)
        for (int64_t q = 0; q < Q; ++q) {
            int64_t b = segment_of(ptr_y, batch, q);
            int64_t lo = ptr_x[b], n = ptr_x[b + 1] - lo;
            for (int64_t s = 0; s < K; ++s) { ld[s] = INFINITY; li[s] = -1; }
            const float *qp = y + D * q;
            if (all_finite(qp, D)) {
                for (int64_t j = 0; j < n; ++j) {
                    float d = sqdist_nd(x + D * (lo + j), qp, D);
                    if (!isfinite(d)) continue;
                    topk_insert(ld, li, K, d, j);
                }
            }
            for (int64_t s = 0; s < K; ++s)
                out[q * K + s] = li[s] < 0 ? -1 : lo + li[s];
        }
        free(ld); free(li);
    }
}

/* ------------------------------------------------------------ ball query */

/*
 * Dense first-K ball query, reference.py:83-121: hits are the first K points
 * j (input order) with fl32((dx^2+dy^2)+dz^2) < r2 (strict), d = query - ref,
 * r2 = fl32(fl32(r) * fl32(r)) (_ball_query_mps.py:87-119).  Empty slots are
 * (d2 0, idx -1).  Lengths follow _ball_query_mps.py:73-84 / the native
 * kernel (kernels/ball_query.metal:64-75): queries at or beyond
 * query_lengths[b] are all padding, only points below point_lengths[b] are
 * scanned.  NaN never satisfies `<`, so non-finite coordinates never match.
 */
void oracle_ball_query(const float *q, const float *p, const int64_t *qlen,
                       const int64_t *plen, int64_t B, int64_t Q, int64_t P,
                       int64_t K, float r2, float *dist2, int64_t *idx) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t bq = 0; bq < B * Q; ++bq) {
        int64_t b = bq / Q, qi = bq % Q;
        int64_t found = 0;
        float *od = dist2 + bq * K;
        int64_t *oi = idx + bq * K;
        if (qi < qlen[b]) {
            int64_t n = plen[b] < P ? plen[b] : P;
            const float *qp = q + 3 * bq;
            const float *pp = p + 3 * P * b;
            for (int64_t j = 0; j < n && found < K; ++j) {
                float d = sqdist3(qp, pp + 3 * j);
                if (d < r2) {
                    od[found] = d;
                    oi[found] = j;
                    ++found;
                }
            }
        }
        for (int64_t s = found; s < K; ++s) { od[s] = 0.f; oi[s] = -1; }
    }
}

/*
 * Flat radius search (torch_cluster convention), (Q, K) global indices padded
 * with -1: flat.py:264-288 (_reference_search with radius; d = refs - query),
 * threshold r2 = fl32(r*r computed in double) (_flat_search_mps.py:66-76),
 * optional exclusion of j == q before the cap (kernels/flat_search.metal:196-199),
 * r == 0 returns no neighbours (_flat_search_mps.py:130-132).
 */
void oracle_radius_flat(const float *y, const float *x, const int64_t *ptr_y,
                        const int64_t *ptr_x, int64_t Q, int64_t batch,
                        int64_t K, float r2, int ignore_same_index,
                        int64_t *out) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t q = 0; q < Q; ++q) {
        int64_t b = segment_of(ptr_y, batch, q);
        int64_t lo = ptr_x[b], hi = ptr_x[b + 1];
        int64_t found = 0;
        const float *qp = y + 3 * q;
        if (r2 > 0.f) {
            for (int64_t j = lo; j < hi && found < K; ++j) {
                if (ignore_same_index && j == q) continue;
                float d = sqdist3(x + 3 * j, qp);
                if (d < r2) out[q * K + found++] = j;
            }
        }
        for (int64_t s = found; s < K; ++s) out[q * K + s] = -1;
    }
}

/* ------------------------------------------------------- PointNet++ prop */

/* Total order for three_nn: stable argsort of d2 (pointnet2.py:54-72) puts
 * NaN after every number; ties keep input order. */
static inline int tn_before(float d, int64_t i, float e, int64_t j) {
    int dn = isnan(d), en = isnan(e);
    if (dn != en) return en;          /* number before NaN */
    if (!dn && d != e) return d < e;
    return i < j;
}

/*
 * three_nn: the three smallest keys of d2 = ((dx^2)+dy^2)+dz^2, d = unknown -
 * known, under stable argsort (pointnet2.py:54-72, kernels/pointnet2.metal:8-50);
 * dist = sqrt(d2), idx int32.  Requires M >= 3.
 */
void oracle_three_nn(const float *unknown, const float *known, int64_t B,
                     int64_t N, int64_t M, float *dist, int32_t *idx) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t bn = 0; bn < B * N; ++bn) {
        int64_t b = bn / N;
        const float *u = unknown + 3 * bn;
        const float *k = known + 3 * M * b;
        float bd[3] = {0.f, 0.f, 0.f};
        int64_t bi[3] = {-1, -1, -1};
        for (int64_t j = 0; j < M; ++j) {
            float d = sqdist3(u, k + 3 * j);
            int64_t s = 3;
            while (s > 0 && (bi[s - 1] < 0 || tn_before(d, j, bd[s - 1], bi[s - 1]))) --s;
            if (s >= 3) continue;
            for (int64_t t = 2; t > s; --t) { bd[t] = bd[t - 1]; bi[t] = bi[t - 1]; }
            bd[s] = d;
            bi[s] = j;
        }
        for (int t = 0; t < 3; ++t) {
            dist[3 * bn + t] = sqrtf(bd[t]);
            idx[3 * bn + t] = (int32_t)bi[t];
        }
    }
}

/* out[b,c,n] = (f[i0]*w0 + f[i1]*w1) + f[i2]*w2 (kernels/pointnet2.metal:52-71). */
void oracle_three_interpolate(const float *features, const int64_t *indices,
                              const float *weights, int64_t B, int64_t C,
                              int64_t M, int64_t N, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t bc = 0; bc < B * C; ++bc) {
        int64_t b = bc / C;
        const float *f = features + M * bc;
        for (int64_t n = 0; n < N; ++n) {
            const int64_t *ix = indices + 3 * (N * b + n);
            const float *w = weights + 3 * (N * b + n);
            float a = f[ix[0]] * w[0];
            float b1 = f[ix[1]] * w[1];
            float c1 = f[ix[2]] * w[2];
            out[N * bc + n] = (a + b1) + c1;
        }
    }
}

/* grad_features[b,c,i_t] += g[b,c,n] * w[b,n,t] accumulated in double
 * (pointnet2.py:150-188 backward; the reference's float CAS order is
 * nondeterministic, so parity is to a tolerance). */
void oracle_three_interpolate_backward(const float *grad_out, const int64_t *indices,
                                       const float *weights, int64_t B, int64_t C,
                                       int64_t M, int64_t N, double *grad_features) {
#pragma omp parallel for schedule(static)
    for (int64_t bc = 0; bc < B * C; ++bc) {
        int64_t b = bc / C;
        double *g = grad_features + M * bc;
        for (int64_t m = 0; m < M; ++m) g[m] = 0.0;
        for (int64_t n = 0; n < N; ++n) {
            const int64_t *ix = indices + 3 * (N * b + n);
            const float *w = weights + 3 * (N * b + n);
            float go = grad_out[N * bc + n];
            for (int t = 0; t < 3; ++t) g[ix[t]] += (double)(go * w[t]);
        }
    }
}

/* ------------------------------------------------- PointNet++ grouping */

/* out[b,c,p] = features[b,c,idx[b,p]]: compat.py:62-73 (gather_operation and
 * grouping_operation are torch.gather along the point axis; grouping reads
 * its (B, npoint, nsample) index flat). */
void oracle_group_points(const float *features, const int64_t *idx, int64_t B, int64_t C,
                         int64_t N, int64_t P, float *out) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < C; ++c)
            for (int64_t p = 0; p < P; ++p)
                out[(b * C + c) * P + p] = features[(b * C + c) * N + idx[b * P + p]];
}

/* The gradient of that gather, grad_features[b,c,idx[b,p]] += grad_out[b,c,p]
 * in float, p ascending: torch.gather's scatter-add backward as a
 * sequential loop. */
void oracle_group_points_backward(const float *grad_out, const int64_t *idx, int64_t B, int64_t C,
                                  int64_t N, int64_t P, float *grad_features) {
    for (int64_t i = 0; i < B * C * N; ++i) grad_features[i] = 0.0f;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < C; ++c)
            for (int64_t p = 0; p < P; ++p)
                grad_features[(b * C + c) * N + idx[b * P + p]] += grad_out[(b * C + c) * P + p];
}

/* The set-abstraction grouping of tests/test_pointnet2_e2e.py:36-45:
 * channels 0-2 = grouping_operation(xyz^T, idx) - new_xyz^T[..., None] (one
 * float subtraction), channels 3.. = grouping_operation(features, idx),
 * concatenated: out (B, 3+C, M, S) for xyz (B,N,3), centres (B,M,3),
 * features (B,C,N), idx (B,M,S). */
void oracle_group_points_rel(const float *xyz, const float *centres, const float *features,
                             const int64_t *idx, int64_t B, int64_t C, int64_t N, int64_t M,
                             int64_t S, float *out) {
    const int64_t P = M * S, CT = C + 3;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t p = 0; p < P; ++p) {
            const int64_t j = idx[b * P + p], m = p / S;
            for (int a = 0; a < 3; ++a)
                out[(b * CT + a) * P + p] = xyz[(b * N + j) * 3 + a] - centres[(b * M + m) * 3 + a];
            for (int64_t c = 0; c < C; ++c)
                out[(b * CT + 3 + c) * P + p] = features[(b * C + c) * N + j];
        }
}

/* -------------------------------------------------------------- Chamfer */

/*
 * Nearest reference per query (K = 1) under squared L2 (norm 2) or L1
 * (norm 1), first minimum index on ties: chamfer.py:161-212 (tiles in
 * increasing index order keep the old winner on ties) and
 * kernels/chamfer_nn.metal:13-226 (3-D order ((dx^2)+dy^2)+dz^2 with
 * d = query - ref; D != 3 sequential accumulation; L1 sums |d|).  The first
 * valid reference is taken even when its distance overflows to inf.
 * Rows at or beyond query_lengths[b], and rows of an empty reference cloud,
 * are (0, -1).
 */
#define CHAMFER_BODY(T, ABS)                                                        \
    for (int64_t bq = 0; bq < B * Q; ++bq) {                                        \
        int64_t b = bq / Q, qi = bq % Q;                                            \
        int64_t nref = rlen[b];                                                     \
        if (qi >= qlen[b] || nref <= 0) { dist[bq] = 0; idx[bq] = -1; continue; }   \
        const T *qp = q + D * bq;                                                   \
        const T *rp = r + D * R * b;                                                \
        T best = 0; int64_t bi = -1;                                                \
        for (int64_t j = 0; j < nref; ++j) {                                        \
            const T *x = rp + D * j;                                                \
            T d;                                                                    \
            if (norm == 1) {                                                        \
                d = ABS(qp[0] - x[0]);                                              \
                for (int64_t t = 1; t < D; ++t) d = d + ABS(qp[t] - x[t]);          \
            } else {                                                                \
                T f = qp[0] - x[0];                                                 \
                d = f * f;                                                          \
                for (int64_t t = 1; t < D; ++t) { T e = qp[t] - x[t]; T s = e * e; d = d + s; } \
            }                                                                       \
            if (bi < 0 || d < best) { best = d; bi = j; }                           \
        }                                                                           \
        dist[bq] = best; idx[bq] = bi;                                              \
    }

void oracle_chamfer_nearest_f32(const float *q, const float *r, const int64_t *qlen,
                                const int64_t *rlen, int64_t B, int64_t Q, int64_t R,
                                int64_t D, int norm, float *dist, int64_t *idx) {
#pragma omp parallel for schedule(dynamic, 64)
    CHAMFER_BODY(float, fabsf)
}

void oracle_chamfer_nearest_f64(const double *q, const double *r, const int64_t *qlen,
                                const int64_t *rlen, int64_t B, int64_t Q, int64_t R,
                                int64_t D, int norm, double *dist, int64_t *idx) {
#pragma omp parallel for schedule(dynamic, 64)
    CHAMFER_BODY(double, fabs)
}
