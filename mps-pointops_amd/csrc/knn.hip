// Exact k-nearest-neighbour search for gfx950.
//
// Two designs.  Dense 3-D queries with K <= 32 use knn3_lane_kernel (one lane
// per query, described with the kernel below; for clouds of up to 8192
// references it can start from a per-query limit taken from the query's
// Morton neighbours, see knn_window_prep_kernel).  Everything else (K up to 256,
// D != 3, flat/ragged batches) uses the wave-per-query kernels:
//
// One wave per query.  Lane l scans reference j = 64*c + l of chunk c; the
// current best K keys (squared distance, index) form a sorted list spread
// over the wave: slot s lives in lane s % 64 of register s / 64 (K <= 256).
// A reference is a candidate when its key is before the K-th entry; the wave
// ballots the candidates and inserts them one by one (rank by ballot
// popcount, shift by one lane with DPP wave_shr).  Keys order by distance then
// index, so the result is independent of visit order; chunks are visited with
// a stride coprime to the chunk count (as kernels/knn.metal:12-17 does) so
// that spatially sorted clouds do not insert on every chunk.
//
// Variants (template DIM3 / FLAT):
//   dense 3-D   kernels/knn.metal:32-140 semantics: NaN distances never match,
//               unfilled slots are (inf, 2^32-1);
//   dense D-dim kernels/feature_knn.metal:51-164: non-finite queries and
//               distances never match, unfilled slots (inf, -1);
//   flat        kernels/flat_search.metal:44-154 and feature_knn.metal:166-199:
//               segment by binary search on ptr_y, global indices, -1 padding.
#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kKnnThreads = 256;
constexpr int kKnnWaves = kKnnThreads / kWave;
constexpr int kMaxK = 256;

// Sequential squared L2 in D dimensions: s = d0^2; s = s + dt^2 (dt = r - q).
__device__ __forceinline__ float sqdist_nd(const float* __restrict__ r, const float* __restrict__ q,
                                           int D) {
    const float first = r[0] - q[0];
    float s = first * first;
    for (int t = 1; t < D; ++t) {
        const float delta = r[t] - q[t];
        const float term = delta * delta;
        s = s + term;
    }
    return s;
}

__device__ __forceinline__ int64_t segment_of(const int64_t* __restrict__ ptr, int64_t batch,
                                              int64_t q) {
    int64_t lo = 0, hi = batch;
    while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (ptr[mid + 1] <= q) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

__device__ __forceinline__ uint32_t gcd_u32(uint32_t a, uint32_t b) {
    while (b != 0) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// Chunk stride ~ golden ratio * chunks, bumped until coprime to chunks.
__device__ __forceinline__ uint32_t visit_stride(uint32_t chunks) {
    if (chunks <= 2) return 1;
    uint32_t s = static_cast<uint32_t>(static_cast<double>(chunks) * 0.6180339887498949 + 0.5) % chunks;
    if (s == 0) s = 1;
    while (gcd_u32(s, chunks) != 1) {
        s = (s + 1) % chunks;
        if (s == 0) s = 1;
    }
    return s;
}

// Insert candidate (cd, ci) into the wave-distributed sorted list.
template <int SLOTS>
__device__ __forceinline__ void list_insert(float (&ld)[SLOTS], int (&li)[SLOTS], int K, int lane,
                                            float cd, int ci) {
    int pos = 0;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        const int s = r * kWave + lane;
        pos += __popcll(ballot(s < K && before(ld[r], li[r], cd, ci)));
    }
    int carry_d = 0, carry_i = 0;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        const int s = r * kWave + lane;
        // Lane 63 of the previous register moves to lane 0 of this one.
        const int next_carry_d = readlane(f2i(ld[r]), kWave - 1);
        const int next_carry_i = readlane(li[r], kWave - 1);
        const float shifted_d = i2f(wave_shr1(f2i(ld[r]), carry_d));
        const int shifted_i = wave_shr1(li[r], carry_i);
        if (s > pos) {
            ld[r] = shifted_d;
            li[r] = shifted_i;
        } else if (s == pos) {
            ld[r] = cd;
            li[r] = ci;
        }
        carry_d = next_carry_d;
        carry_i = next_carry_i;
    }
}

template <int SLOTS>
__device__ __forceinline__ void list_tail(const float (&ld)[SLOTS], const int (&li)[SLOTS], int K,
                                          float& td, int& ti) {
    const int r_last = (K - 1) / kWave;
    const int l_last = (K - 1) % kWave;
    int d = 0, i = 0;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        if (r == r_last) {
            d = readlane(f2i(ld[r]), l_last);
            i = readlane(li[r], l_last);
        }
    }
    td = i2f(d);
    ti = i;
}

// One wave: scan n references and keep the K best keys.
template <int SLOTS, bool DIM3, bool FINITE_ONLY>
__device__ __forceinline__ void scan_refs(const float* __restrict__ qp, const float* __restrict__ rp,
                                          int n, int D, int K, int lane, float (&ld)[SLOTS],
                                          int (&li)[SLOTS]) {
    float td = INFINITY;
    int ti = -1;  // 0xFFFFFFFF: every real index is before it
    const uint32_t chunks = (static_cast<uint32_t>(n) + kWave - 1) / kWave;
    if (chunks == 0) return;
    float qx = 0.f, qy = 0.f, qz = 0.f;
    if (DIM3) {
        qx = qp[0];
        qy = qp[1];
        qz = qp[2];
    }
    const uint32_t stride = visit_stride(chunks);
    uint32_t chunk = 0;
    for (uint32_t c = 0; c < chunks; ++c) {
        const int j = static_cast<int>(chunk * kWave) + lane;
        chunk += stride;
        if (chunk >= chunks) chunk -= chunks;
        float d = INFINITY;
        bool valid = j < n;
        if (valid) {
            if (DIM3) {
                const float* r = rp + 3 * static_cast<int64_t>(j);
                d = sqdist3(r[0], r[1], r[2], qx, qy, qz);
            } else {
                d = sqdist_nd(rp + static_cast<int64_t>(j) * D, qp, D);
            }
            if (FINITE_ONLY) valid = isfinite(d);
        }
        uint64_t pending = ballot(valid && before(d, j, td, ti));
        while (pending != 0) {
            const int src = __builtin_ctzll(pending);
            pending &= pending - 1;
            const float cd = i2f(readlane(f2i(d), src));
            const int ci = readlane(j, src);
            if (!before(cd, ci, td, ti)) continue;  // an earlier insert raised the bar
            list_insert<SLOTS>(ld, li, K, lane, cd, ci);
            list_tail<SLOTS>(ld, li, K, td, ti);
        }
    }
}

template <int SLOTS, bool DIM3>
__global__ __launch_bounds__(kKnnThreads) void knn_dense_kernel(
    const float* __restrict__ query, const float* __restrict__ ref, float* __restrict__ out_dist,
    int64_t* __restrict__ out_idx, int64_t B, int64_t M, int64_t N, int D, int K) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kKnnWaves + uniform(threadIdx.x / kWave);
    if (row >= B * M) return;  // whole wave leaves; only wave-level sync below
    const int64_t b = row / M;
    const float* qp = query + row * D;
    const float* rp = ref + b * N * D;
    float ld[SLOTS];
    int li[SLOTS];
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        ld[r] = INFINITY;
        li[r] = -1;
    }
    bool query_ok = true;
    if (!DIM3) {
        for (int t = 0; t < D; ++t) query_ok = query_ok && isfinite(qp[t]);
    }
    if (query_ok) scan_refs<SLOTS, DIM3, !DIM3>(qp, rp, static_cast<int>(N), D, K, lane, ld, li);
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        const int s = r * kWave + lane;
        if (s < K) {
            out_dist[row * K + s] = sqrtf(ld[r]);
            // 3-D keeps the reference kernel's (inf, UINT_MAX) padding.
            out_idx[row * K + s] = DIM3 ? static_cast<int64_t>(static_cast<uint32_t>(li[r]))
                                        : (li[r] < 0 ? int64_t(-1) : int64_t(li[r]));
        }
    }
}

template <int SLOTS, bool DIM3>
__global__ __launch_bounds__(kKnnThreads) void knn_flat_kernel(
    const float* __restrict__ y, const float* __restrict__ x, const int64_t* __restrict__ ptr_y,
    const int64_t* __restrict__ ptr_x, int64_t* __restrict__ out, int64_t Q, int64_t batch, int D,
    int K) {
    const int lane = lane_id();
    const int64_t q = static_cast<int64_t>(blockIdx.x) * kKnnWaves + uniform(threadIdx.x / kWave);
    if (q >= Q) return;
    const int64_t b = segment_of(ptr_y, batch, q);
    const int64_t lo = ptr_x[b];
    const int n = static_cast<int>(ptr_x[b + 1] - lo);
    const float* qp = y + q * D;
    float ld[SLOTS];
    int li[SLOTS];
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        ld[r] = INFINITY;
        li[r] = -1;
    }
    bool query_ok = true;
    for (int t = 0; t < D; ++t) query_ok = query_ok && isfinite(qp[t]);
    if (query_ok) scan_refs<SLOTS, DIM3, true>(qp, x + lo * D, n, D, K, lane, ld, li);
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
        const int s = r * kWave + lane;
        if (s < K) out[q * K + s] = li[r] < 0 ? int64_t(-1) : lo + li[r];
    }
}

// ------------------------------------------------------------------------
// Small-K 3-D kNN (K <= KMAX <= 32): one lane per query.
//
// A block serves 64 queries of one cloud (lane = query); its 4 waves split
// the references into 4 contiguous ranges and each wave keeps, per lane, the
// best KMAX keys of its range; the 4 partial lists are merged at the end.
// Every lane of a wave reads the same reference, so references come through
// uniform (scalar) loads.  Keys are the squared distance's bit pattern:
// non-negative floats and +inf order like unsigned integers and NaN patterns
// are larger, so `bits(d) < tau`, with tau = key of the K-th entry
// (0x7F800001 while the list has free slots), admits exactly the references
// that beat the K-th entry under the (distance, index) order of the reference
// kernel -- a range is visited in index order, so an equal distance never
// beats an entry already kept, and NaN never enters.  Admitted references go
// to a per-lane LDS buffer ([slot][lane], conflict free); when any lane's
// buffer is full, and at the end, each lane merges it into its sorted register
// list.
constexpr int kLaneWaves = 4;
constexpr int kLaneThreads = kLaneWaves * kWave;
constexpr int kLaneCap = 32;  // buffered candidates per lane (merged at half)
constexpr uint32_t kEmptyKey = 0x7F800001u;

// Median of three unsigned ints (one v_med3_u32).
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <int KMAX>
__device__ __forceinline__ uint32_t kth_key(const uint32_t (&lk)[KMAX], int K) {
    if (K == KMAX) return lk[KMAX - 1];
    uint32_t t = 0;
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
        if (s == K - 1) t = lk[s];
    return t;
}

// Insert this lane's `cnt` buffered candidates (in index order) into its
// sorted list; the wave loops while any lane has entries left.
template <int KMAX>
__device__ __forceinline__ void lane_merge(uint32_t (&lk)[KMAX], int (&li)[KMAX], uint32_t& tau,
                                           int K, const uint2* buf, int lane, int cnt) {
    for (int e = 0;; ++e) {
        const bool has = e < cnt;
        if (ballot(has) == 0) break;
        // A lane with nothing to insert inserts the no-op key 0xFFFFFFFF
        // (never below a slot), so the network runs without branches.
        // Row e < max(cnt) <= CAP is inside the buffer for every lane; the
        // K-th key may have tightened since buffering.
        const uint2 c = buf[e * kWave + lane];
        const bool take = has && c.x < tau;
        const uint32_t ck = take ? c.x : 0xFFFFFFFFu;
        const int cj = static_cast<int>(c.y);
        if (ballot(take) == 0) continue;
        // Slots after the insertion point move down one place; `here` means
        // the candidate goes before slot s, `prev` before slot s - 1.  On a
        // sorted list the new key of slot s is med3(ck, lk[s-1], lk[s]).
        bool here = ck < lk[KMAX - 1];
#pragma unroll
        for (int s = KMAX - 1; s > 0; --s) {
            const bool prev = ck < lk[s - 1];
            lk[s] = med3_u32(ck, lk[s - 1], lk[s]);
            li[s] = prev ? li[s - 1] : (here ? cj : li[s]);
            here = prev;
        }
        lk[0] = min(ck, lk[0]);
        li[0] = here ? cj : li[0];
        tau = kth_key<KMAX>(lk, K);
    }
}

// Publish each wave's sorted list ([slot][lane] in lds[wave]) and merge the
// NW lists of every lane in wave 0, writing K (sqrt distance, index)
// pairs at row `row`.  Unfilled slots get (inf, empty_index).  The merge
// keeps every list's head in registers as a 64-bit (key, index) value, so
// a step is NW - 1 compares and one LDS read (the next entry of the list
// it took from) instead of NW dependent reads.
template <int KMAX, int NW, int CAP>
__device__ __forceinline__ void lane_publish_and_merge(
    uint2 (&lds)[NW][KMAX > CAP ? KMAX : CAP][kWave], const uint32_t (&lk)[KMAX],
    const int (&li)[KMAX], int K, int wave, int lane, bool active, int64_t row,
    float* __restrict__ out_dist, int64_t* __restrict__ out_idx, int64_t empty_index) {
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
        if (s < K) lds[wave][s][lane] = make_uint2(lk[s], static_cast<uint32_t>(li[s]));
    __syncthreads();
    if (wave != 0 || !active) return;
    auto pack = [](uint2 v) { return (static_cast<uint64_t>(v.x) << 32) | v.y; };
    constexpr uint64_t kPast = ~uint64_t(0);  // after a list's K-th entry
    uint64_t head[NW];
    int next[NW];  // slot of each list's following entry
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        head[w] = pack(lds[w][0][lane]);
        next[w] = 1;
    }
    for (int s = 0; s < K; ++s) {
        uint64_t best = head[0];
        int from = 0;
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const bool less = head[w] < best;  // distinct (key, index) pairs
            best = less ? head[w] : best;
            from = less ? w : from;
        }
        int h = next[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) h = from == w ? next[w] : h;
        const uint64_t fresh = h < K ? pack(lds[from][h][lane]) : kPast;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            head[w] = from == w ? fresh : head[w];
            next[w] = from == w ? h + 1 : next[w];
        }
        const uint32_t key = static_cast<uint32_t>(best >> 32);
        const int index = static_cast<int>(static_cast<uint32_t>(best));
        const bool empty = index < 0;
        out_dist[row + s] = empty ? INFINITY : sqrtf(i2f(static_cast<int>(key)));
        out_idx[row + s] = empty ? empty_index : static_cast<int64_t>(index);
    }
}

// ------------------------------------------------------------------------
// Starting limit from Morton neighbours (clouds of up to 8192 references).
//
// knn_window_prep_kernel (one workgroup per cloud) counting-sorts the
// references by a 16 x 16 x 16 Morton cell of the finite references'
// bounding box and writes their coordinates in that order, with the grid
// (box and cell starts); it reads no query, so it can run before the queries
// exist.  In knn3_lane_kernel every query takes a "home": the middle of its
// cell's range in the sorted order (or where the cell would start), and
// then, per query, the window
// of r*K sorted references around its home (r = min(8, N/K)) in K strided
// groups {w0 + g + j*K : j < r}; wave w takes the c groups g = w mod NW and
// the c-th smallest key among their c*r references, and the limit is the
// largest of these over the waves: every wave has c distinct references at
// or below it, K in all, so the query's K-th neighbour is no further (the
// c-th smallest of a union is at most the largest of its c group minima,
// the limit taken before).  Only references with keys at or below it are
// admitted from the start, which spares most of the list merging that a
// full list would otherwise cost before it tightens.
constexpr int kWindowPrepThreads = 1024;
constexpr int kWindowMaxRefs = 8192;
constexpr int kWindowMaxQueries = 16384;
constexpr int kWindowCells = 4096;  // 16^3 Morton cells
constexpr int kWindowGroups = 8;    // window references per group (r <= 8)
constexpr int kWindowChunk = 8;     // of which loaded at once

// Per cloud, the Morton grid of the sort: lo[3] and scale[3] (the first
// 8 words, as floats), then the cells' starts in the sorted order
// (kWindowCells + 1 ints).
constexpr int kWindowGridWords = 8 + ((kWindowCells + 1 + 63) & ~63);

struct WindowLayout {
    float4* sorted;  // [B][N]: coordinates in Morton order (w unused)
    int* grid;       // [B][kWindowGridWords]
};

__host__ __device__ inline size_t window_layout_bytes(int64_t B, int64_t M, int64_t N,
                                                      WindowLayout* out, char* base) {
    (void)M;
    const size_t sorted_bytes = (static_cast<size_t>(B * N) * sizeof(float4) + 255) & ~size_t(255);
    if (out != nullptr) {
        out->sorted = reinterpret_cast<float4*>(base);
        out->grid = reinterpret_cast<int*>(base + sorted_bytes);
    }
    return sorted_bytes + static_cast<size_t>(B * kWindowGridWords) * sizeof(int);
}

__device__ __forceinline__ uint32_t window_cell(float x, float y, float z, const float (&lo)[3],
                                                const float (&scale)[3]) {
    const float c3[3] = {x, y, z};
    uint32_t q[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        // fmaxf/fminf map NaN to cell 0 and infinities to the edge cells.
        q[a] = static_cast<uint32_t>(fminf(fmaxf((c3[a] - lo[a]) * scale[a], 0.f), 15.f));
    }
    return morton12(q[0], q[1], q[2]);
}

__global__ __launch_bounds__(kWindowPrepThreads) void knn_window_prep_kernel(
    const float* __restrict__ ref, WindowLayout L, int N) {
    constexpr int RPT = kWindowMaxRefs / kWindowPrepThreads;
    constexpr int CPT = kWindowCells / kWindowPrepThreads;  // cells per thread in the scan
    constexpr int NWV = kWindowPrepThreads / kWave;
    __shared__ int cell_off[kWindowCells + 1];
    __shared__ float red[6][NWV];
    __shared__ int wave_sum[NWV];
    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    const int64_t b = blockIdx.x;
    const float* rp = ref + 3 * b * N;

    for (int c = tid; c <= kWindowCells; c += kWindowPrepThreads) cell_off[c] = 0;
    // The references are requested together, without branches (an index
    // past the end reads the last point again), so that every load is in
    // flight before the first wait.
    float px[RPT], py[RPT], pz[RPT];
    // Rounds k with no point at all are skipped (a uniform branch).
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        px[k] = py[k] = pz[k] = 0.f;
        if (k * kWindowPrepThreads >= N) continue;
        const int j = min(tid + k * kWindowPrepThreads, N - 1);
        px[k] = rp[3 * j];
        py[k] = rp[3 * j + 1];
        pz[k] = rp[3 * j + 2];
    }
    float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int j = tid + k * kWindowPrepThreads;
        if (j < N && isfinite(px[k]) && isfinite(py[k]) && isfinite(pz[k])) {
            mn[0] = fminf(mn[0], px[k]); mx[0] = fmaxf(mx[0], px[k]);
            mn[1] = fminf(mn[1], py[k]); mx[1] = fmaxf(mx[1], py[k]);
            mn[2] = fminf(mn[2], pz[k]); mx[2] = fmaxf(mx[2], pz[k]);
        }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        mn[a] = wave_min(mn[a]);
        mx[a] = wave_max(mx[a]);
    }
    if (lane == 0) {
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            red[a][wave] = mn[a];
            red[3 + a][wave] = mx[a];
        }
    }
    __syncthreads();  // box partials and cleared counters
    float lo[3], scale[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        float l = red[a][0], h = red[3 + a][0];
        for (int w = 1; w < NWV; ++w) {
            l = fminf(l, red[a][w]);
            h = fmaxf(h, red[3 + a][w]);
        }
        const float ext = h - l;  // no finite reference: -inf - inf, not >= 0
        lo[a] = ext >= 0.f ? l : 0.f;
        scale[a] = (ext > 0.f && ext < INFINITY) ? 16.f / ext : 0.f;
    }
    int cell[RPT], rank[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        cell[k] = rank[k] = 0;
        if (k * kWindowPrepThreads >= N) continue;
        const int j = tid + k * kWindowPrepThreads;
        cell[k] = static_cast<int>(window_cell(px[k], py[k], pz[k], lo, scale));
        rank[k] = j < N ? atomicAdd(&cell_off[cell[k]], 1) : 0;
    }
    __syncthreads();  // counts complete
    {
        int run = 0;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int v = cell_off[tid * CPT + c];
            cell_off[tid * CPT + c] = run;
            run += v;
        }
        int incl = run;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int up = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += up;
        }
        if (lane == kWave - 1) wave_sum[wave] = incl;
        __syncthreads();  // wave totals
        int before = incl - run;
        for (int w = 0; w < wave; ++w) before += wave_sum[w];
#pragma unroll
        for (int c = 0; c < CPT; ++c) cell_off[tid * CPT + c] += before;
        if (tid == kWindowPrepThreads - 1) cell_off[kWindowCells] = before + run;
    }
    __syncthreads();  // offsets complete
    float4* sorted = L.sorted + b * N;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int j = tid + k * kWindowPrepThreads;
        if (j < N) sorted[cell_off[cell[k]] + rank[k]] = make_float4(px[k], py[k], pz[k], 0.f);
    }
    // The grid, from which each query finds its home in the lane kernel.
    int* grid = L.grid + b * kWindowGridWords;
    if (tid < 3) {
        grid[tid] = f2i(lo[tid]);
        grid[3 + tid] = f2i(scale[tid]);
    }
    for (int c = tid; c <= kWindowCells; c += kWindowPrepThreads) grid[8 + c] = cell_off[c];
}

template <int KMAX, int NW, int CAP>
__global__ __launch_bounds__(NW * kWave) void knn3_lane_kernel(
    const float* __restrict__ query, const float* __restrict__ ref, float* __restrict__ out_dist,
    int64_t* __restrict__ out_idx, int64_t M, int64_t N, int K, const float4* __restrict__ sorted,
    const int* __restrict__ grid, int64_t QS) {
    // Per wave: the candidate buffer during the scan, then the final list.
    __shared__ uint2 lds[NW][KMAX > CAP ? KMAX : CAP][kWave];
    __shared__ uint32_t window_max[kWave];  // per lane: the Morton-window limit
    // Per lane and wave: the key of the wave's K-th entry, read by the other
    // waves (one lane's NW keys are contiguous: two 16-byte reads).
    constexpr int kTauRows = (NW + 3) / 4;
    __shared__ uint4 taus[kWave][kTauRows];
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x / kWave);
    const uint32_t per_cloud = static_cast<uint32_t>((M + kWave - 1) / kWave);
    const CloudBlock cb = cloud_block(per_cloud);
    const int64_t b = cb.b;
    const int64_t m = static_cast<int64_t>(cb.x) * kWave + lane;
    const bool active = m < M;
    const float* qp = query + 3 * (b * QS + (active ? m : 0));  // QS: rows between clouds
    const float qx = qp[0], qy = qp[1], qz = qp[2];
    const float* rp = ref + 3 * b * N;
    uint2* buf = &lds[wave][0][0];
    // Contiguous reference ranges in wave order, the first half of the waves
    // taking 17/16 of an even share (a multiple of 8): two waves share each
    // SIMD and the older is issued first, so with even ranges the younger
    // half finished its scan ~7 us later at N = 4096 and the rest waited.
    static_assert(NW % 2 == 0, "two halves of waves");
    constexpr int kHalf = NW / 2;
    const int64_t a = ((N * 17 + 16 * NW - 1) / (16 * NW) + 7) / 8 * 8;
    const int64_t split = min<int64_t>(N, a * kHalf);
    const int64_t b_span = (N - split + kHalf - 1) / kHalf;
    const int64_t lo = wave < kHalf ? min<int64_t>(N, wave * a) : min<int64_t>(N, split + (wave - kHalf) * b_span);
    const int64_t hi = wave < kHalf ? min<int64_t>(split, lo + a) : min<int64_t>(N, lo + b_span);

    uint32_t lk[KMAX];
    int li[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
        lk[s] = kEmptyKey;
        li[s] = -1;
    }
    uint32_t tau = active ? kEmptyKey : 0u;  // inactive lanes admit nothing
    uint32_t* my_tau = reinterpret_cast<uint32_t*>(&taus[lane][0]) + wave;
    *my_tau = tau;
    if (wave == 0) window_max[lane] = 0;
    __syncthreads();
    // Keys at or below the Morton-window limit (sorted != nullptr: set up by
    // knn_window_prep_kernel for this launch) are admitted from the start;
    // wave w takes the groups g = w mod NW.  Keys compare as unsigned: NaN
    // patterns are above +inf, and then nothing is excluded.
    uint32_t bound = kEmptyKey;
    if (sorted != nullptr) {
        const float4* sp = sorted + b * N;
        const int n = static_cast<int>(N);
        const int r = min(kWindowGroups, n / K);
        // The query's home: the middle of its Morton cell's range in the
        // sorted order.
        int h = 0;
        if (active) {
            const int* g = grid + b * kWindowGridWords;
            const float glo[3] = {i2f(g[0]), i2f(g[1]), i2f(g[2])};
            const float gsc[3] = {i2f(g[3]), i2f(g[4]), i2f(g[5])};
            const int c = static_cast<int>(window_cell(qx, qy, qz, glo, gsc));
            h = min((g[8 + c] + g[8 + c + 1]) / 2, n - 1);
        }
        const int w0 = min(max(h - r * K / 2, 0), n - r * K);
        // This wave's groups g = wave mod NW (c of them) hold c x r distinct
        // references; the c-th smallest of their keys bounds c of them, so
        // the largest over the waves bounds K distinct references.
        constexpr int CMAX = (KMAX + NW - 1) / NW;
        uint32_t least[CMAX];  // the wave's smallest keys, ascending
#pragma unroll
        for (int c = 0; c < CMAX; ++c) least[c] = 0xFFFFFFFFu;
        int groups = 0;
        for (int g = wave; g < K; g += NW) {
            ++groups;
#pragma unroll
            for (int j0 = 0; j0 < kWindowGroups; j0 += kWindowChunk) {
                if (j0 >= r) break;
                float vx[kWindowChunk], vy[kWindowChunk], vz[kWindowChunk];
#pragma unroll
                for (int j = 0; j < kWindowChunk; ++j) {
                    const float* f = reinterpret_cast<const float*>(sp + w0 + g + min(j0 + j, r - 1) * K);
                    vx[j] = f[0];
                    vy[j] = f[1];
                    vz[j] = f[2];
                }
#pragma unroll
                for (int j = 0; j < kWindowChunk; ++j) {
                    // Clamped repeats of the last reference are not counted again.
                    const uint32_t key = j0 + j < r
                        ? static_cast<uint32_t>(f2i(sqdist3(vx[j], vy[j], vz[j], qx, qy, qz)))
                        : 0xFFFFFFFFu;
#pragma unroll
                    for (int c = CMAX - 1; c > 0; --c) least[c] = med3_u32(key, least[c - 1], least[c]);
                    least[0] = min(least[0], key);
                }
            }
        }
        uint32_t wmax = 0;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) wmax = groups == c + 1 ? least[c] : wmax;
        if (wmax != 0) atomicMax(&window_max[lane], wmax);
        __syncthreads();
        const uint32_t wm = window_max[lane];
        bound = wm < kEmptyKey ? wm + 1 : kEmptyKey;  // key < bound <=> key <= wm
    }
    // Admission limit: this wave's K-th key and the other waves' K-th keys
    // (read without synchronisation: they only decrease, so a stale value is
    // a looser but still valid limit; this wave's own published key is never
    // below its current one).  A lower range holds smaller indices, so an
    // equal key from a higher range cannot beat its K-th entry, while an equal
    // key from a lower range can beat a higher range's K-th entry.
    auto limit = [&]() {
        uint32_t t[4 * kTauRows];
#pragma unroll
        for (int v = 0; v < kTauRows; ++v) {
            const uint4 q4 = taus[lane][v];
            t[4 * v] = q4.x;
            t[4 * v + 1] = q4.y;
            t[4 * v + 2] = q4.z;
            t[4 * v + 3] = q4.w;
        }
        uint32_t lim = min(tau, bound);
#pragma unroll
        for (int w = 0; w < NW; ++w) lim = min(lim, t[w] + static_cast<uint32_t>(w > wave));
        return lim;
    };
    int cnt = 0;
    uint32_t lim = min(tau, bound);
    auto visit = [&](float rx, float ry, float rz, int j) {
        const uint32_t key = static_cast<uint32_t>(f2i(sqdist3(rx, ry, rz, qx, qy, qz)));
        if (key < lim) {  // rare once the lists fill: the masked store is skipped
            buf[cnt * kWave + lane] = make_uint2(key, static_cast<uint32_t>(j));
            ++cnt;
        }
    };
    constexpr int kRefBatch = 8;
    // After a batch: merge once a lane's buffer could not take another batch.
    auto drain = [&]() {
        if (ballot(cnt > CAP - kRefBatch) != 0) {
            lane_merge<KMAX>(lk, li, tau, K, buf, lane, cnt);
            cnt = 0;
            *my_tau = tau;
        }
    };
    // Batches of kRefBatch references through uniform (scalar) loads; the
    // shared limit is refreshed every second batch.
    // The next batch is requested after the limit is read, so its scalar
    // loads are in flight while this batch is scanned.
    int j0 = static_cast<int>(lo);
    const int jhi = static_cast<int>(hi);
    float cur[3 * kRefBatch];
    if (j0 + kRefBatch <= jhi) {
        const float* r = rp + 3 * static_cast<int64_t>(j0);
#pragma unroll
        for (int t = 0; t < 3 * kRefBatch; ++t) cur[t] = r[t];
    }
    for (int batch = 0; j0 + kRefBatch <= jhi; j0 += kRefBatch, ++batch) {
        lim = (batch & 1) ? min(lim, tau) : limit();
        float nxt[3 * kRefBatch];
        const int jn = min(j0 + kRefBatch, jhi - kRefBatch);  // stays inside the range
        const float* r = rp + 3 * static_cast<int64_t>(jn);
#pragma unroll
        for (int t = 0; t < 3 * kRefBatch; ++t) nxt[t] = r[t];
#pragma unroll
        for (int u = 0; u < kRefBatch; ++u) visit(cur[3 * u], cur[3 * u + 1], cur[3 * u + 2], j0 + u);
        drain();
#pragma unroll
        for (int t = 0; t < 3 * kRefBatch; ++t) cur[t] = nxt[t];
    }
    for (; j0 < jhi; ++j0) {
        const float* r = rp + 3 * static_cast<int64_t>(j0);
        lim = limit();
        visit(r[0], r[1], r[2], j0);
        drain();
    }
    lane_merge<KMAX>(lk, li, tau, K, buf, lane, cnt);

    lane_publish_and_merge<KMAX, NW, CAP>(lds, lk, li, K, wave, lane, active, (b * QS + m) * K, out_dist,
                                 out_idx, static_cast<int64_t>(0xFFFFFFFFu));
}

// Feature-space kNN, K <= KMAX <= 32, D a multiple of 4 up to 128: one lane
// per query, the scheme of knn3_lane_kernel (4 waves split the references into
// 4 contiguous ranges, per-lane sorted lists, shared admission limits).  The
// query stays in VGPRs; each wave streams its range through a wave-private
// 4 KiB LDS tile (the next tile is loaded into registers while the current
// one is scanned) and reads each reference with broadcast LDS loads.
// Semantics of kernels/feature_knn.metal:51-164: a non-finite query matches
// nothing, non-finite distances never match (keys below the bits of +inf
// only), unfilled slots are (inf, -1).  The distance is the sequential
// s = d0^2; s = s + dt^2 with dt = r - q.
constexpr int kFeatTileFloats = 1024;
constexpr uint32_t kInfKey = 0x7F800000u;

template <int KMAX, int D>
__global__ __launch_bounds__(kLaneThreads) void knn_feat_lane_kernel(
    const float* __restrict__ query, const float* __restrict__ ref, float* __restrict__ out_dist,
    int64_t* __restrict__ out_idx, int64_t M, int64_t N, int K) {
    static_assert(D % 4 == 0 && D <= 128, "feature width");
    constexpr int TR = kFeatTileFloats / D;                // references per tile
    constexpr int PER_LANE = kFeatTileFloats / kWave / 4;  // float4 loads per lane per tile
    constexpr int kGroup = 8;                              // references between drains
    static_assert(TR % kGroup == 0, "tile holds whole groups");
    __shared__ uint2 lds[kLaneWaves][KMAX > kLaneCap ? KMAX : kLaneCap][kWave];
    __shared__ uint32_t taus[kLaneWaves][kWave];
    __shared__ float4 tiles[kLaneWaves][kFeatTileFloats / 4];
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x / kWave);
    const CloudBlock cb = cloud_block(static_cast<uint32_t>((M + kWave - 1) / kWave));
    const int64_t b = cb.b;
    const int64_t m = static_cast<int64_t>(cb.x) * kWave + lane;
    const bool active = m < M;
    const float4* qp = reinterpret_cast<const float4*>(query + D * (b * M + (active ? m : 0)));
    float q[D];
    bool ok = active;
#pragma unroll
    for (int t = 0; t < D / 4; ++t) {
        const float4 v = qp[t];
        q[4 * t] = v.x;
        q[4 * t + 1] = v.y;
        q[4 * t + 2] = v.z;
        q[4 * t + 3] = v.w;
    }
#pragma unroll
    for (int t = 0; t < D; ++t) ok = ok && isfinite(q[t]);
    const float* rp = ref + D * b * N;
    uint2* buf = &lds[wave][0][0];
    float4* tile = tiles[wave];
    const int64_t span = (N + kLaneWaves - 1) / kLaneWaves;
    const int64_t lo = wave * span;
    const int64_t hi = min<int64_t>(N, lo + span);

    uint32_t lk[KMAX];
    int li[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
        lk[s] = kInfKey;
        li[s] = -1;
    }
    uint32_t tau = ok ? kInfKey : 0u;  // admits finite keys only; nothing for bad queries
    taus[wave][lane] = tau;
    __syncthreads();
    auto limit = [&]() {
        uint32_t lim = tau;
#pragma unroll
        for (int w = 0; w < kLaneWaves; ++w) {
            if (w == wave) continue;
            const uint32_t t = taus[w][lane];
            lim = min(lim, w < wave ? t : t + 1u);
        }
        return lim;
    };
    // Load the tile of references starting at t0 into registers (zeros past hi).
    auto fetch = [&](int64_t t0, float4 (&pf)[PER_LANE]) {
        const int64_t valid = max<int64_t>(0, min<int64_t>(TR, hi - t0)) * D / 4;
        const float4* src = reinterpret_cast<const float4*>(rp + D * t0);
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) {
            const int e = i * kWave + lane;
            pf[i] = e < valid ? src[e] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    int cnt = 0;
    float4 pf[PER_LANE];
    if (lo < hi) fetch(lo, pf);
    for (int64_t t0 = lo; t0 < hi; t0 += TR) {
        // Publish the prefetched tile to this wave's LDS and fetch the next.
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) tile[i * kWave + lane] = pf[i];
        __builtin_amdgcn_wave_barrier();
        if (t0 + TR < hi) fetch(t0 + TR, pf);
        const int nref = static_cast<int>(min<int64_t>(TR, hi - t0));
        for (int g0 = 0; g0 < nref; g0 += kGroup) {
            const uint32_t lim = limit();
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                if (g0 + u >= nref) break;  // uniform
                const float4* r = tile + (g0 + u) * (D / 4);
                float sd = 0.f;
#pragma unroll
                for (int t = 0; t < D / 4; ++t) {
                    const float4 v = r[t];  // same address in every lane: broadcast
                    const float d0 = v.x - q[4 * t], d1 = v.y - q[4 * t + 1];
                    const float d2 = v.z - q[4 * t + 2], d3 = v.w - q[4 * t + 3];
                    sd = t == 0 ? d0 * d0 : sd + d0 * d0;
                    sd = sd + d1 * d1;
                    sd = sd + d2 * d2;
                    sd = sd + d3 * d3;
                }
                const uint32_t key = static_cast<uint32_t>(f2i(sd));
                if (key < lim) {
                    buf[cnt * kWave + lane] = make_uint2(key, static_cast<uint32_t>(t0 + g0 + u));
                    ++cnt;
                }
            }
            if (ballot(cnt > kLaneCap - kGroup) != 0) {
                lane_merge<KMAX>(lk, li, tau, K, buf, lane, cnt);
                cnt = 0;
                taus[wave][lane] = tau;
            }
        }
    }
    lane_merge<KMAX>(lk, li, tau, K, buf, lane, cnt);
    lane_publish_and_merge<KMAX, kLaneWaves, kLaneCap>(lds, lk, li, K, wave, lane, active,
                                                      (b * M + m) * K, out_dist, out_idx, -1);
}

template <int KMAX, int D>
hipError_t launch_feat_lane(const float* query, const float* ref, float* dist, int64_t* idx,
                            int64_t B, int64_t M, int64_t N, int K, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>((M + kWave - 1) / kWave * B));  // cloud_block order
    hipLaunchKernelGGL((knn_feat_lane_kernel<KMAX, D>), grid, dim3(kLaneThreads), 0, stream, query,
                       ref, dist, idx, M, N, K);
    return hipGetLastError();
}

template <int KMAX>
hipError_t launch_lane(const float* query, const float* ref, float* dist, int64_t* idx, int64_t B,
                       int64_t M, int64_t N, int K, hipStream_t stream,
                       const WindowLayout* window = nullptr, int64_t QS = 0) {
    const dim3 grid(static_cast<uint32_t>((M + kWave - 1) / kWave * B));  // cloud_block order
    // Small lists: 8 waves per 64 queries (more waves in flight, 16-entry
    // buffers); K up to 32: 4 waves with 32-entry buffers.
    constexpr int NW = KMAX <= 16 ? 8 : 4;
    constexpr int CAP = KMAX <= 16 ? 16 : 32;
    hipLaunchKernelGGL((knn3_lane_kernel<KMAX, NW, CAP>), grid, dim3(NW * kWave), 0, stream, query,
                       ref, dist, idx, M, N, K, window ? window->sorted : nullptr,
                       window ? window->grid : nullptr, QS > 0 ? QS : M);
    return hipGetLastError();
}

template <bool DIM3>
hipError_t launch_dense(const float* query, const float* ref, float* dist, int64_t* idx, int64_t B,
                        int64_t M, int64_t N, int D, int K, hipStream_t stream) {
    const bool lane_grid_ok = (M + kWave - 1) / kWave * B <= INT32_MAX;
    if (DIM3 && K <= 32 && lane_grid_ok) {
        if (K <= 8) return launch_lane<8>(query, ref, dist, idx, B, M, N, K, stream);
        if (K <= 16) return launch_lane<16>(query, ref, dist, idx, B, M, N, K, stream);
        return launch_lane<32>(query, ref, dist, idx, B, M, N, K, stream);
    }
    const bool aligned = (reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(ref)) % 16 == 0;
    if (!DIM3 && D == 64 && K <= 32 && aligned && lane_grid_ok) {
        if (K <= 8) return launch_feat_lane<8, 64>(query, ref, dist, idx, B, M, N, K, stream);
        if (K <= 16) return launch_feat_lane<16, 64>(query, ref, dist, idx, B, M, N, K, stream);
        return launch_feat_lane<32, 64>(query, ref, dist, idx, B, M, N, K, stream);
    }
    if (!DIM3 && D == 128 && K <= 32 && aligned && lane_grid_ok) {
        if (K <= 8) return launch_feat_lane<8, 128>(query, ref, dist, idx, B, M, N, K, stream);
        if (K <= 16) return launch_feat_lane<16, 128>(query, ref, dist, idx, B, M, N, K, stream);
        return launch_feat_lane<32, 128>(query, ref, dist, idx, B, M, N, K, stream);
    }
    const int64_t rows = B * M;
    const dim3 grid(static_cast<uint32_t>((rows + kKnnWaves - 1) / kKnnWaves));
    const dim3 block(kKnnThreads);
    if (K <= 64)
        hipLaunchKernelGGL((knn_dense_kernel<1, DIM3>), grid, block, 0, stream, query, ref, dist, idx,
                           B, M, N, D, K);
    else if (K <= 128)
        hipLaunchKernelGGL((knn_dense_kernel<2, DIM3>), grid, block, 0, stream, query, ref, dist, idx,
                           B, M, N, D, K);
    else
        hipLaunchKernelGGL((knn_dense_kernel<4, DIM3>), grid, block, 0, stream, query, ref, dist, idx,
                           B, M, N, D, K);
    return hipGetLastError();
}

template <bool DIM3>
hipError_t launch_flat(const float* y, const float* x, const int64_t* ptr_y, const int64_t* ptr_x,
                       int64_t* out, int64_t Q, int64_t batch, int D, int K, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>((Q + kKnnWaves - 1) / kKnnWaves));
    const dim3 block(kKnnThreads);
    if (K <= 64)
        hipLaunchKernelGGL((knn_flat_kernel<1, DIM3>), grid, block, 0, stream, y, x, ptr_y, ptr_x, out,
                           Q, batch, D, K);
    else if (K <= 128)
        hipLaunchKernelGGL((knn_flat_kernel<2, DIM3>), grid, block, 0, stream, y, x, ptr_y, ptr_x, out,
                           Q, batch, D, K);
    else
        hipLaunchKernelGGL((knn_flat_kernel<4, DIM3>), grid, block, 0, stream, y, x, ptr_y, ptr_x, out,
                           Q, batch, D, K);
    return hipGetLastError();
}

bool grid_ok(int64_t rows) { return (rows + kKnnWaves - 1) / kKnnWaves <= INT32_MAX; }

}  // namespace


}  // namespace pointops

namespace pointops {

// The windowed kNN (D = 3, K <= 32) over M query rows per cloud whose rows --
// queries and both outputs -- lie QS rows apart (M consecutive centres of a
// (B, QS, 3) tensor and of its (B, QS, K) outputs).  `workspace` holds
// pointops_knn3_windowed_workspace_bytes(B, M, N) bytes.
// The windowed search in two launches: knn3_window_sort (the references of
// every cloud in Morton order, and the grid, into `workspace`; it depends on
// the references only) and knn3_windowed_rows (the queries -- M rows per
// cloud lying QS rows apart -- over a workspace the sort has filled for the
// same references, B and N).
hipError_t knn3_window_sort(const float* ref, void* workspace, int64_t B, int64_t M, int64_t N,
                            hipStream_t stream) {
    if (B < 1 || B > INT32_MAX || N < 1 || N > kWindowMaxRefs || workspace == nullptr)
        return hipErrorInvalidValue;
    WindowLayout L;
    window_layout_bytes(B, M, N, &L, static_cast<char*>(workspace));
    hipLaunchKernelGGL(knn_window_prep_kernel, dim3(static_cast<uint32_t>(B)),
                       dim3(kWindowPrepThreads), 0, stream, ref, L, static_cast<int>(N));
    return hipGetLastError();
}

hipError_t knn3_windowed_rows(const float* query, const float* ref, float* dist, int64_t* idx,
                              void* workspace, int64_t B, int64_t M, int64_t QS, int64_t N,
                              int64_t K, hipStream_t stream) {
    if (B < 1 || B > INT32_MAX || M < 1 || QS < M || K < 1 || K > 32 || K > N ||
        N > kWindowMaxRefs || M > kWindowMaxQueries || workspace == nullptr ||
        (M + kWave - 1) / kWave * B > INT32_MAX)
        return hipErrorInvalidValue;
    WindowLayout L;
    window_layout_bytes(B, M, N, &L, static_cast<char*>(workspace));
    const int k = static_cast<int>(K);
    if (K <= 8) return launch_lane<8>(query, ref, dist, idx, B, M, N, k, stream, &L, QS);
    if (K <= 16) return launch_lane<16>(query, ref, dist, idx, B, M, N, k, stream, &L, QS);
    return launch_lane<32>(query, ref, dist, idx, B, M, N, k, stream, &L, QS);
}

}  // namespace pointops

using namespace pointops;

extern "C" {

hipError_t pointops_knn3(const float* query, const float* ref, float* dist, int64_t* idx, int64_t B,
                         int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0 || K < 0 || K > kMaxK || K > N) return hipErrorInvalidValue;
    if (B == 0 || M == 0 || K == 0) return hipSuccess;
    if (N > INT32_MAX - kWave || !grid_ok(B * M)) return hipErrorInvalidValue;
    return launch_dense<true>(query, ref, dist, idx, B, M, N, 3, static_cast<int>(K), stream);
}

size_t pointops_knn3_windowed_workspace_bytes(int64_t B, int64_t M, int64_t N) {
    if (B <= 0 || M <= 0 || N <= 0) return 0;
    return window_layout_bytes(B, M, N, nullptr, nullptr);
}

hipError_t pointops_knn3_windowed(const float* query, const float* ref, float* dist, int64_t* idx,
                                  void* workspace, int64_t B, int64_t M, int64_t N, int64_t K,
                                  hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0 || K < 0 || K > 32 || K > N) return hipErrorInvalidValue;
    if (B == 0 || M == 0 || K == 0) return hipSuccess;
    if (N > kWindowMaxRefs || M > kWindowMaxQueries || workspace == nullptr || B > INT32_MAX ||
        (M + kWave - 1) / kWave * B > INT32_MAX)
        return hipErrorInvalidValue;
    const hipError_t err = knn3_window_sort(ref, workspace, B, M, N, stream);
    if (err != hipSuccess) return err;
    return knn3_windowed_rows(query, ref, dist, idx, workspace, B, M, M, N, K, stream);
}

hipError_t pointops_knn_feat(const float* query, const float* ref, float* dist, int64_t* idx,
                             int64_t B, int64_t M, int64_t N, int64_t D, int64_t K,
                             hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0 || D < 1 || K < 0 || K > kMaxK || K > N) return hipErrorInvalidValue;
    if (B == 0 || M == 0 || K == 0) return hipSuccess;
    if (N > INT32_MAX - kWave || D > INT32_MAX || !grid_ok(B * M)) return hipErrorInvalidValue;
    return launch_dense<false>(query, ref, dist, idx, B, M, N, static_cast<int>(D),
                               static_cast<int>(K), stream);
}

hipError_t pointops_knn_flat(const float* y, const float* x, const int64_t* ptr_y,
                             const int64_t* ptr_x, int64_t* out, int64_t Q, int64_t batch,
                             int64_t D, int64_t K, hipStream_t stream) {
    if (Q < 0 || batch < 0 || D < 1 || K < 0 || K > kMaxK) return hipErrorInvalidValue;
    if (Q == 0 || K == 0) return hipSuccess;
    if (batch == 0 || D > INT32_MAX || !grid_ok(Q)) return hipErrorInvalidValue;
    if (D == 3)
        return launch_flat<true>(y, x, ptr_y, ptr_x, out, Q, batch, 3, static_cast<int>(K), stream);
    return launch_flat<false>(y, x, ptr_y, ptr_x, out, Q, batch, static_cast<int>(D),
                              static_cast<int>(K), stream);
}

}  // extern "C"
