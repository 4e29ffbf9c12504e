// Exact 3-D kNN over a uniform grid, for large clouds (K <= 32).
//
// The result is the brute-force one of kernels/knn.metal:32-140 (neighbours
// sorted by float32 squared distance, then index; NaN distances never match;
// unfilled slots (inf, 2^32-1)); the grid only decides which references are
// examined.  Every comparison uses the (key, index) pair, key = bits of the
// squared distance, so the visit order does not matter.
//
// Per batch, in a caller-provided workspace:
//   1. grid_bounds_kernel: partial bounding boxes of the finite references
//      and counts of references with a non-finite coordinate; from them
//      (grid_params) a cell side for about grid_per_cell(K) references per
//      cell;
//   2. counting sort (count with ranks, two-pass tiled scan, scatter) of the
//      references by cell (x fastest), the non-finite ones in an overflow
//      cell after the last, and of the queries by 2 x 2 x 2 block of cells;
//   3. knn3_grid_kernel: one lane per query, 64 consecutive queries of the
//      sorted order (neighbours in space) per wave.  Each lane scans the
//      3 x 3 x 3 box of cells around its own query and stops once its K-th
//      squared distance is below that of the nearest unscanned cell face,
//      less a slack for float rounding (box_bound), else grows the box by
//      that face.  A non-finite query or a batch with non-finite
//      references lists the wave's queries, a walk that needs more than
//      kGridMaxGrow faces its own query, for a linear pass in the same call
//      (knn3_lane_listed: the brute-force lane kernel over the listed rows).
#include <algorithm>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kGridPrepThreads = 256;
constexpr int kGridBoundBlocks = 256;  // bounding-box partials per batch, at most
constexpr int kGridScanTile = 8 * kGridPrepThreads;
constexpr int kGridMaxDim = 1024;
constexpr int kGridSearchWaves = 4;
constexpr int kGridCap = 16;  // buffered candidates per lane
constexpr int kGridMaxGrow = 24;  // box faces a lane may add before the wave scans everything
// Nearest mode: box faces a lane may add before its query is left to the
// fill pass (measured best of 4-24).
constexpr int kGridNearestGrow = 6;
constexpr int kGridQueriesPerWave = kWave / 4;  // one quad of lanes per query
constexpr uint32_t kGridMatchLimit = 0x7F800001u;  // keys below: finite or +inf

struct alignas(16) GridParams {
    float lo[3];
    float inv_h;
    int dims[3];
    int cells;
    int nonfinite;
    int pad[7];
};
static_assert(sizeof(GridParams) == 64, "workspace layout");

// Cell capacity of one batch's grid (the overflow cell comes after it).
__host__ __device__ inline int64_t grid_cell_cap(int64_t N) { return N / 2 > 64 ? N / 2 : 64; }

// References per cell the grid aims at for K neighbours: the 3 x 3 x 3 box
// around a query then holds about 27 of them and, for evenly spread points,
// almost always the K nearest (the ball of radius one cell side holds about
// 4.2 of them).
__host__ __device__ inline double grid_per_cell(int K) { return K * 0.4 > 3.0 ? K * 0.4 : 3.0; }

struct GridLayout {
    int* control;    // 64 words: control[0] is the ball query's device-side choice
    const int* gate; // null, or control: the build and ball search skip when *gate == 0
    GridParams* params;
    float* partial;  // [B][kGridBoundBlocks][8]: bounding-box partials
    int* ref_off;    // [B][stride]: cell counts, then offsets
    int* q_off;      // [B][stride]
    int* tile_sum;   // [B][2][tiles]: per-tile totals of the two scans
    int* ref_rank;   // [B][N]: rank of each reference within its cell
    int* q_rank;     // [B][M]
    float4* sorted;  // [B][N]: x, y, z, index bits
    int* q_order;    // [B][M]
    int64_t stride;  // cap + 2 rounded up to whole 16-byte words
    int64_t tiles;   // scan tiles per array
};

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

__host__ __device__ inline size_t grid_layout_bytes(int64_t B, int64_t M, int64_t N,
                                                    GridLayout* out, char* base) {
    const int64_t stride = (grid_cell_cap(N) + 2 + 3) & ~int64_t(3);
    const int64_t tiles = (stride + kGridScanTile - 1) / kGridScanTile;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    const size_t p_ctrl = take(64 * sizeof(int));
    const size_t p_params = take(static_cast<size_t>(B) * sizeof(GridParams));
    const size_t p_part = take(static_cast<size_t>(B) * kGridBoundBlocks * 8 * sizeof(float));
    const size_t p_roff = take(static_cast<size_t>(B * stride) * sizeof(int));
    const size_t p_qoff = take(static_cast<size_t>(B * stride) * sizeof(int));
    const size_t p_tsum = take(static_cast<size_t>(B * 2 * tiles) * sizeof(int));
    const size_t p_rrank = take(static_cast<size_t>(B * N) * sizeof(int));
    const size_t p_qrank = take(static_cast<size_t>(B * M) * sizeof(int));
    const size_t p_sorted = take(static_cast<size_t>(B * N) * sizeof(float4));
    const size_t p_qord = take(static_cast<size_t>(B * M) * sizeof(int));
    if (out != nullptr) {
        out->control = reinterpret_cast<int*>(base + p_ctrl);
        out->gate = nullptr;
        out->params = reinterpret_cast<GridParams*>(base + p_params);
        out->partial = reinterpret_cast<float*>(base + p_part);
        out->ref_off = reinterpret_cast<int*>(base + p_roff);
        out->q_off = reinterpret_cast<int*>(base + p_qoff);
        out->tile_sum = reinterpret_cast<int*>(base + p_tsum);
        out->ref_rank = reinterpret_cast<int*>(base + p_rrank);
        out->q_rank = reinterpret_cast<int*>(base + p_qrank);
        out->sorted = reinterpret_cast<float4*>(base + p_sorted);
        out->q_order = reinterpret_cast<int*>(base + p_qord);
        out->stride = stride;
        out->tiles = tiles;
    }
    return o;
}

// True when the call's device-side choice went to the index-order search:
// the grid's sort and search then return at once.
__device__ __forceinline__ bool grid_gated_off(const GridLayout& L) {
    return L.gate != nullptr && *L.gate == 0;
}

__device__ __forceinline__ bool finite3(float x, float y, float z) {
    return isfinite(x) && isfinite(y) && isfinite(z);
}

__device__ __forceinline__ int cell_axis(float v, float lo, float inv_h, int dim) {
    const float t = floorf((v - lo) * inv_h);
    return static_cast<int>(fminf(fmaxf(t, 0.f), static_cast<float>(dim - 1)));
}

// Query order key: the 2 x 2 x 2 block of cells holding the point (blocks
// in x-fastest order), so that 64 consecutive queries form a compact group;
// non-finite queries go to block 0.  Keys stay below the cell count.
__device__ __forceinline__ int query_key(const GridParams& P, float x, float y, float z) {
    if (!finite3(x, y, z)) return 0;
    const int bx = cell_axis(x, P.lo[0], P.inv_h, P.dims[0]) >> 1;
    const int by = cell_axis(y, P.lo[1], P.inv_h, P.dims[1]) >> 1;
    const int bz = cell_axis(z, P.lo[2], P.inv_h, P.dims[2]) >> 1;
    const int nbx = (P.dims[0] + 1) >> 1, nby = (P.dims[1] + 1) >> 1;
    return bx + nbx * (by + nby * bz);
}

// Cell of a point; non-finite points go to the overflow cell `cells`.
__device__ __forceinline__ int cell_of(const GridParams& P, float x, float y, float z) {
    if (!finite3(x, y, z)) return P.cells;
    const int cx = cell_axis(x, P.lo[0], P.inv_h, P.dims[0]);
    const int cy = cell_axis(y, P.lo[1], P.inv_h, P.dims[1]);
    const int cz = cell_axis(z, P.lo[2], P.inv_h, P.dims[2]);
    return cx + P.dims[0] * (cy + P.dims[1] * cz);
}

// Per (block, batch): zero a share of the two count arrays and reduce a
// share of the references to a bounding-box partial (min xyz, max xyz, count
// of references with a non-finite coordinate).
__global__ __launch_bounds__(kGridPrepThreads) void grid_bounds_kernel(const float* __restrict__ ref,
                                                                       GridLayout L, int64_t N) {
    __shared__ float red[7][kGridPrepThreads / kWave];
    const int64_t b = blockIdx.y;
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kGridPrepThreads + tid;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kGridPrepThreads;
    for (int64_t e = first; e < L.stride; e += step) {
        L.ref_off[b * L.stride + e] = 0;
        L.q_off[b * L.stride + e] = 0;
    }
    const float* r = ref + 3 * b * N;
    float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
    int bad = 0;
    for (int64_t j = first; j < N; j += step) {
        const float x = r[3 * j], y = r[3 * j + 1], z = r[3 * j + 2];
        if (finite3(x, y, z)) {
            mn[0] = fminf(mn[0], x); mx[0] = fmaxf(mx[0], x);
            mn[1] = fminf(mn[1], y); mx[1] = fmaxf(mx[1], y);
            mn[2] = fminf(mn[2], z); mx[2] = fmaxf(mx[2], z);
        } else {
            ++bad;
        }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float wmn = wave_min(mn[a]), wmx = wave_max(mx[a]);
        if (lane == 0) {
            red[a][wave] = wmn;
            red[3 + a][wave] = wmx;
        }
    }
    int nb = bad;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) nb += __shfl_xor(nb, d);
    if (lane == 0) red[6][wave] = i2f(nb);
    __syncthreads();
    if (tid >= 8) return;
    float v;
    if (tid < 6) {
        v = red[tid][0];
        for (int w = 1; w < kGridPrepThreads / kWave; ++w)
            v = tid < 3 ? fminf(v, red[tid][w]) : fmaxf(v, red[tid][w]);
    } else if (tid == 6) {
        int t = 0;
        for (int w = 0; w < kGridPrepThreads / kWave; ++w) t += f2i(red[6][w]);
        v = i2f(t);
    } else {
        v = 0.f;
    }
    L.partial[(b * kGridBoundBlocks + blockIdx.x) * 8 + tid] = v;
}

// Run by the first wave of a workgroup: combine batch b's `parts` partials
// into the bounding box of its finite references and choose the grid; lane 0
// stores it to *out.
__device__ void grid_params(const GridLayout& L, int64_t b, int64_t N, int parts, int K,
                            float hmin, GridParams* out) {
    const int lane = threadIdx.x;
    float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
    int nonfinite = 0;
    for (int i = lane; i < parts; i += kWave) {
        const float* t = L.partial + (b * kGridBoundBlocks + i) * 8;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            mn[a] = fminf(mn[a], t[a]);
            mx[a] = fmaxf(mx[a], t[3 + a]);
        }
        nonfinite += f2i(t[6]);
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        mn[a] = wave_min(mn[a]);
        mx[a] = wave_max(mx[a]);
    }
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) nonfinite += __shfl_xor(nonfinite, d);
    if (lane != 0) return;
    float lo[3], ext[3];
    bool any = true;
    for (int a = 0; a < 3; ++a) {
        any = any && mn[a] <= mx[a];
        lo[a] = any ? mn[a] : 0.f;
        ext[a] = any ? mx[a] - mn[a] : 0.f;
    }
    GridParams P;
    const int64_t cap = grid_cell_cap(N);
    const float emax = fmaxf(fmaxf(ext[0], ext[1]), ext[2]);
    float hside = 1.f;
    if (any && emax > 0.f && emax < INFINITY) {
        const float thin = emax * 1e-3f;
        const double vol = static_cast<double>(fmaxf(ext[0], thin)) * fmaxf(ext[1], thin) *
                           fmaxf(ext[2], thin);
        const double target = fmax(1.0, fmin(static_cast<double>(cap),
                                             static_cast<double>(N) / grid_per_cell(K)));
        hside = static_cast<float>(cbrt(vol / target));
        if (!(hside > 0.f)) hside = emax;
        if (hside < hmin) hside = hmin;  // a caller's smallest useful cell (ball radius)
    }
    int dims[3] = {1, 1, 1};
    bool fits = false;
    for (int it = 0; it < 200 && !fits; ++it) {
        int64_t total = 1;
        for (int a = 0; a < 3; ++a) {
            const float t = ext[a] / hside;
            dims[a] = (t < static_cast<float>(kGridMaxDim - 1)) ? static_cast<int>(t) + 1 : kGridMaxDim;
            total *= dims[a];
        }
        fits = total <= cap;
        hside *= 1.25f;
    }
    if (!fits) {  // extents too large for float cell arithmetic: one cell
        dims[0] = dims[1] = dims[2] = 1;
        hside = 1.f;
    } else {
        hside /= 1.25f;
    }
    for (int a = 0; a < 3; ++a) {
        P.lo[a] = lo[a];
        P.dims[a] = dims[a];
    }
    P.inv_h = 1.f / hside;
    P.cells = dims[0] * dims[1] * dims[2];
    P.nonfinite = nonfinite;
    for (int i = 0; i < 7; ++i) P.pad[i] = 0;
    *out = P;
}

// Workgroups [0, ref_blocks) of a count or scatter launch cover the
// references of batch blockIdx.y, the rest its queries.
struct PrepItem {
    const float* pts;
    int64_t n, j;
    bool queries;
};
__device__ __forceinline__ PrepItem prep_item(const float* ref, const float* query, int64_t N,
                                              int64_t M, uint32_t ref_blocks) {
    const bool queries = blockIdx.x >= ref_blocks;
    const int64_t blk = queries ? blockIdx.x - ref_blocks : blockIdx.x;
    return {queries ? query : ref, queries ? M : N, blk * kGridPrepThreads + threadIdx.x, queries};
}

// Cell counts of the references and the queries (by query_key); each point
// keeps its rank among the points of its cell.  Every workgroup derives the
// grid from the bounding-box partials (the same arithmetic, so the same
// grid); the first of each batch stores it for the later kernels.
__global__ __launch_bounds__(kGridPrepThreads) void grid_count_kernel(const float* __restrict__ ref,
                                                                      const float* __restrict__ query,
                                                                      GridLayout L, int64_t N, int64_t M,
                                                                      uint32_t ref_blocks, int parts,
                                                                      int K, float hmin) {
    if (grid_gated_off(L)) return;  // uniform, before any barrier
    __shared__ GridParams shared_params;
    const int64_t b = blockIdx.y;
    if (threadIdx.x < kWave) grid_params(L, b, N, parts, K, hmin, &shared_params);
    __syncthreads();
    const GridParams P = shared_params;
    if (blockIdx.x == 0 && threadIdx.x == 0) L.params[b] = P;
    const PrepItem it = prep_item(ref, query, N, M, ref_blocks);
    if (it.j >= it.n) return;
    const float* p = it.pts + 3 * (b * it.n + it.j);
    const int c = it.queries ? query_key(P, p[0], p[1], p[2]) : cell_of(P, p[0], p[1], p[2]);
    const int rank = atomicAdd((it.queries ? L.q_off : L.ref_off) + b * L.stride + c, 1);
    (it.queries ? L.q_rank : L.ref_rank)[b * it.n + it.j] = rank;
}

// Sum of `v` over a workgroup of kGridPrepThreads threads (every thread gets
// it); `red` holds one int per wave.
__device__ __forceinline__ int block_sum(int v, int* red) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) v += __shfl_xor(v, d);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) red[wave] = v;
    __syncthreads();
    int t = 0;
#pragma unroll
    for (int w = 0; w < kGridPrepThreads / kWave; ++w) t += red[w];
    return t;
}

// The scans cover entries [0, cells + 2) of a batch's count array (the
// overflow cell is entry `cells`; entry cells + 1 stays 0 and receives the
// total), in tiles of kGridScanTile entries, 8 per thread.  blockIdx.y is
// the batch, blockIdx.z 1 for the queries' array.
__device__ __forceinline__ int scan_entries(const GridLayout& L, int64_t b) {
    return L.params[b].cells + 2;
}

__device__ __forceinline__ void load8(const int* a, int at, int count, int (&v)[8]) {
    if (at + 8 <= count) {
        const int4 x = *reinterpret_cast<const int4*>(a + at);
        const int4 y = *reinterpret_cast<const int4*>(a + at + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = at + u < count ? a[at + u] : 0;
    }
}

// Pass 1: the total of each tile.
__global__ __launch_bounds__(kGridPrepThreads) void grid_tile_sum_kernel(GridLayout L) {
    if (grid_gated_off(L)) return;
    __shared__ int red[kGridPrepThreads / kWave];
    const int64_t b = blockIdx.y;
    const bool queries = blockIdx.z != 0;
    const int count = scan_entries(L, b);
    const int t0 = blockIdx.x * kGridScanTile;
    if (t0 >= count) return;  // whole workgroup
    const int* a = (queries ? L.q_off : L.ref_off) + b * L.stride;
    int v[8];
    load8(a, t0 + threadIdx.x * 8, count, v);
    int s = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
    s = block_sum(s, red);
    if (threadIdx.x == 0) L.tile_sum[(b * 2 + queries) * L.tiles + blockIdx.x] = s;
}

// Pass 2: exclusive offsets of each tile's entries, in place, after the
// totals of the tiles before it.
__global__ __launch_bounds__(kGridPrepThreads) void grid_tile_scan_kernel(GridLayout L) {
    if (grid_gated_off(L)) return;
    __shared__ int red[kGridPrepThreads / kWave];
    __shared__ int wsum[kGridPrepThreads / kWave];
    const int64_t b = blockIdx.y;
    const bool queries = blockIdx.z != 0;
    const int count = scan_entries(L, b);
    const int t0 = blockIdx.x * kGridScanTile;
    if (t0 >= count) return;  // whole workgroup
    int* a = (queries ? L.q_off : L.ref_off) + b * L.stride;
    const int* ts = L.tile_sum + (b * 2 + queries) * L.tiles;
    int before = 0;
    for (int t = threadIdx.x; t < static_cast<int>(blockIdx.x); t += kGridPrepThreads) before += ts[t];
    before = block_sum(before, red);
    const int at = t0 + threadIdx.x * 8;
    int v[8];
    load8(a, at, count, v);
    int mine = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) mine += v[u];
    // Inclusive scan of the per-thread totals within the wave, then across
    // the waves of the workgroup.
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    int inc = mine;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(inc, d);
        if (lane >= d) inc += o;
    }
    if (lane == kWave - 1) wsum[wave] = inc;
    __syncthreads();
    int run = before + inc - mine;
    for (int w = 0; w < wave; ++w) run += wsum[w];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int c = v[u];
        v[u] = run;
        run += c;
    }
    if (at + 8 <= count) {
        *reinterpret_cast<int4*>(a + at) = make_int4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<int4*>(a + at + 4) = make_int4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (at + u < count) a[at + u] = v[u];
    }
}

// Place every point at its cell's offset plus its rank: the references with
// their index in the sorted array, the queries' indices in q_order.
__global__ __launch_bounds__(kGridPrepThreads) void grid_scatter_kernel(const float* __restrict__ ref,
                                                                        const float* __restrict__ query,
                                                                        GridLayout L, int64_t N, int64_t M,
                                                                        uint32_t ref_blocks) {
    if (grid_gated_off(L)) return;
    const PrepItem it = prep_item(ref, query, N, M, ref_blocks);
    if (it.j >= it.n) return;
    const int64_t b = blockIdx.y;
    const GridParams P = L.params[b];
    const float* p = it.pts + 3 * (b * it.n + it.j);
    const float x = p[0], y = p[1], z = p[2];
    if (it.queries) {
        const int q = L.q_off[b * L.stride + query_key(P, x, y, z)] + L.q_rank[b * M + it.j];
        L.q_order[b * M + q] = static_cast<int>(it.j);
    } else {
        const int q = L.ref_off[b * L.stride + cell_of(P, x, y, z)] + L.ref_rank[b * N + it.j];
        L.sorted[b * N + q] = make_float4(x, y, z, i2f(static_cast<int>(it.j)));
    }
}

// Composite neighbour word: key (bits of the squared distance) in the high
// half, reference index in the low half, so that one unsigned 64-bit compare
// orders by distance, then index.
__device__ __forceinline__ uint64_t grid_word(uint32_t key, uint32_t ix) {
    return (static_cast<uint64_t>(key) << 32) | ix;
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(dpp<CTRL>(static_cast<int>(static_cast<uint32_t>(v))));
    const uint32_t hi = static_cast<uint32_t>(dpp<CTRL>(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

constexpr int kDppQuadPrev = 0x90;  // quad_perm [0,0,1,2]: lane j <- lane j - 1
constexpr int quad_bcast(int j) { return j * 0x55; }  // quad_perm [j,j,j,j]

// A query's neighbour list is shared by the four lanes of its quad: an
// ascending list of 4S words of which lane j holds ranks S*j .. S*j + S - 1.
// Insert v (the same word on the four lanes); the last word drops out.  A v
// not below the last word changes nothing.  Called with the whole wave
// active (DPP reads neighbouring lanes).
template <int S>
__device__ __forceinline__ void quad_insert(uint64_t (&slot)[S], uint64_t v, int qi) {
    const uint64_t pl = dpp64<kDppQuadPrev>(slot[S - 1]);  // rank S*j - 1
    bool lt[S];
#pragma unroll
    for (int s = 0; s < S; ++s) lt[s] = v < slot[s];
    const bool ltp = qi != 0 && v < pl;
#pragma unroll
    for (int s = S - 1; s > 0; --s) slot[s] = lt[s - 1] ? slot[s - 1] : (lt[s] ? v : slot[s]);
    slot[0] = ltp ? pl : (lt[0] ? v : slot[0]);
}

// Insert lane J's word of each quad into that quad's list.
template <int J, int S>
__device__ __forceinline__ void quad_insert_from(uint64_t (&slot)[S], uint64_t tau, uint64_t mine,
                                                 int qi) {
    const uint64_t v = dpp64<quad_bcast(J)>(mine);
    if (ballot(v < tau) != 0) quad_insert<S>(slot, v, qi);
}

// Insert every lane's `cnt` buffered candidates into its quad's list, one
// source lane of the quad at a time; tau = the list's last word on all four
// lanes (refreshed once per buffer row: a stale tau only lets a no-op insert
// through).  Whole wave active.
template <int S>
__device__ __forceinline__ void quad_merge(uint64_t (&slot)[S], uint64_t& tau, const uint2* buf,
                                           int lane, int cnt) {
    const int qi = lane & 3;
    for (int e = 0;; ++e) {
        const bool has = e < cnt;
        if (ballot(has) == 0) break;
        const uint2 c = buf[e * kWave + lane];  // row e < max(cnt) <= kGridCap
        const uint64_t mine = has ? grid_word(c.x, c.y) : ~0ull;
        if (ballot(mine < tau) == 0) continue;
        quad_insert_from<0, S>(slot, tau, mine, qi);
        quad_insert_from<1, S>(slot, tau, mine, qi);
        quad_insert_from<2, S>(slot, tau, mine, qi);
        quad_insert_from<3, S>(slot, tau, mine, qi);
        tau = dpp64<quad_bcast(3)>(slot[S - 1]);
    }
}

// The cells a lane has scanned always form a box bl[a] <= cell[a] <= bh[a].
// It starts as the 3 x 3 x 3 box around the query's cell (clipped to the
// grid) and grows one face at a time by a slab of cells one cell thick.
// Scan units are segments, flat cell ranges [c0, c1] within one x-row:
//   face -1  the starting box: its nine x-rows, the query's own row first;
//   face 0/1 the x = bl[0] / x = bh[0] slab: one cell per (y, z);
//   face 2/3 the y = bl[1] / y = bh[1] slab: one x-row per z;
//   face 4/5 the z = bl[2] / z = bh[2] slab: one x-row per y.
struct GridBox {
    int bl[3], bh[3];
};

__device__ __forceinline__ int box_segments(const GridBox& X, int face) {
    const int ny = X.bh[1] - X.bl[1] + 1, nz = X.bh[2] - X.bl[2] + 1;
    return face < 0 ? 9 : (face < 2 ? ny * nz : (face < 4 ? nz : ny));
}

// Segment g of `face`; false when it lies outside the grid (only rows of the
// starting box can).
__device__ __forceinline__ bool box_segment(const GridParams& P, const GridBox& X,
                                            const int (&c)[3], int face, int g, int& c0,
                                            int& c1) {
    int x0 = X.bl[0], x1 = X.bh[0], y, z;
    if (face < 0) {
        const int t = g == 0 ? 4 : (g <= 4 ? g - 1 : g);
        y = c[1] + t % 3 - 1;
        z = c[2] + t / 3 - 1;
        if (y < 0 || y >= P.dims[1] || z < 0 || z >= P.dims[2]) return false;
    } else if (face < 2) {
        const int ny = X.bh[1] - X.bl[1] + 1;
        x0 = x1 = (face & 1) ? X.bh[0] : X.bl[0];
        y = X.bl[1] + g % ny;
        z = X.bl[2] + g / ny;
    } else if (face < 4) {
        y = (face & 1) ? X.bh[1] : X.bl[1];
        z = X.bl[2] + g;
    } else {
        y = X.bl[1] + g;
        z = (face & 1) ? X.bh[2] : X.bl[2];
    }
    const int row = P.dims[0] * (y + P.dims[1] * z);
    c0 = row + x0;
    c1 = row + x1;
    return true;
}

// Distance from query q to the box face `f` (2a: low side of axis a, 2a + 1:
// high side), +inf for a face on the grid's edge (references beyond an edge
// are clamped into the edge cell, so none lie outside it).
__device__ __forceinline__ float face_distance(const GridParams& P, float h, const float (&q)[3],
                                               const GridBox& X, int f) {
    const int a = f >> 1;
    if (f & 1)
        return X.bh[a] < P.dims[a] - 1
                   ? (P.lo[a] + static_cast<float>(X.bh[a] + 1) * h) - q[a]
                   : INFINITY;
    return X.bl[a] > 0 ? q[a] - (P.lo[a] + static_cast<float>(X.bl[a]) * h) : INFINITY;
}

// Lower bound on the distance from q to every finite reference outside the
// box: the nearest face, less a slack of 2^-18 of the grid's coordinate
// magnitude, far above the float rounding of the faces and of the cell
// assignment floor((v - lo) * inv_h).  +inf when the box is the whole grid.
__device__ __forceinline__ float box_bound(const GridParams& P, float h, const float (&q)[3],
                                           const GridBox& X) {
    float b = INFINITY;
#pragma unroll
    for (int f = 0; f < 6; ++f) {
        const int a = f >> 1;
        const float slack = (fabsf(P.lo[a]) + static_cast<float>(P.dims[a]) * h) * 0x1p-18f;
        b = fminf(b, face_distance(P, h, q, X, f) - slack);
    }
    return b;
}

template <int S>
__global__ __launch_bounds__(kGridSearchWaves * kWave) void knn3_grid_kernel(
    const float* __restrict__ query, GridLayout L, float* __restrict__ out_dist,
    int64_t* __restrict__ out_idx, int64_t B, int64_t M, int64_t N, int K, int nearest,
    int* __restrict__ miss_count, int* __restrict__ miss_list) {
    constexpr int KMAX = 4 * S;
    __shared__ uint2 bufs[kGridSearchWaves][kGridCap][kWave];
    const int lane = lane_id();
    const int qi = lane & 3;
    const int wave = uniform(threadIdx.x / kWave);
    const int64_t groups = (M + kGridQueriesPerWave - 1) / kGridQueriesPerWave;
    // Consecutive query groups (neighbours in space) share an XCD and the
    // references they read stay in its L2.
    const int64_t gw = static_cast<int64_t>(xcd_local_block(blockIdx.x, gridDim.x)) * kGridSearchWaves + wave;
    if (gw >= B * groups) return;  // whole wave; no barriers in this kernel
    const int64_t b = gw / groups;
    const int64_t pos = (gw - b * groups) * kGridQueriesPerWave + (lane >> 2);
    const bool active = pos < M;
    const int m = active ? L.q_order[b * M + pos] : 0;
    const float* qp = query + 3 * (b * M + m);
    const float q[3] = {qp[0], qp[1], qp[2]};
    const GridParams P = L.params[b];
    const int* off = L.ref_off + b * L.stride;
    const float4* srt = L.sorted + b * N;
    uint2* buf = &bufs[wave][0][0];

    // With K < KMAX the first KMAX - K ranks hold zero words that every
    // candidate sorts after, so the K results are the last K ranks and tau
    // (the admission bound) is always the last rank.  Inactive quads hold
    // zeros and admit nothing.
    uint64_t slot[S];
#pragma unroll
    for (int s = 0; s < S; ++s) slot[s] = (active && S * qi + s >= KMAX - K) ? ~0ull : 0ull;
    uint64_t tau = active ? ~0ull : 0ull;
    int cnt = 0;

    // Admit references base, base + 4, ..., base + 28 into this lane's
    // buffer (the quad's lanes interleaved, so one load instruction covers 4
    // consecutive references per quad): slot u while 4u < n.
    auto admit8s = [&](const float4 (&r)[8], int n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t key = static_cast<uint32_t>(f2i(sqdist3(r[u].x, r[u].y, r[u].z, q[0], q[1], q[2])));
            const uint32_t ix = static_cast<uint32_t>(f2i(r[u].w));
            if (4 * u < n && key < kGridMatchLimit && grid_word(key, ix) < tau) {
                buf[cnt * kWave + lane] = make_uint2(key, ix);
                ++cnt;
            }
        }
    };
    auto drain = [&](bool extra) {
        if (ballot(cnt > kGridCap - 8 || extra) != 0) {
            quad_merge<S>(slot, tau, buf, lane, cnt);
            cnt = 0;
        }
    };

    const bool qfinite = finite3(q[0], q[1], q[2]);
    // Queries left to the linear pass: the whole wave when the batch has
    // non-finite references or the wave a non-finite query, else the quads
    // whose walk needs more faces than the mode allows.
    const bool full = P.nonfinite > 0 || ballot(active && !qfinite) != 0;
    bool listed = false;
    if (!full) {
        // The quad scans the box around its query, 32 references of its
        // current segment per step (lane j of the quad takes every fourth
        // from the j-th), with the bounds of the next
        // segment fetched one segment ahead; the four lanes keep identical
        // copies of the walk's state.  When the box is done the quad stops if
        // its K-th key is below the squared bound of everything outside;
        // otherwise it grows the box by its nearest face.  A quad that needs
        // more faces than its mode's limit is listed for the linear pass.
        const float h = 1.f / P.inv_h;
        int c[3];
        GridBox X;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            c[a] = cell_axis(q[a], P.lo[a], P.inv_h, P.dims[a]);
            X.bl[a] = max(c[a] - 1, 0);
            X.bh[a] = min(c[a] + 1, P.dims[a] - 1);
        }
        int face = -1, grow = 0, g = 0, p = 0, e = 0, np = 0, ne = 0;
        auto fetch = [&]() {
            int c0, c1;
            const bool ok = box_segment(P, X, c, face, g, c0, c1);
            np = ok ? off[c0] : 0;
            ne = ok ? off[c1 + 1] : 0;
        };
        bool done = !active, want = false;
        if (!done) fetch();
        for (;;) {
            drain(want);
            want = false;
            int qc = cnt | dpp<kDppQuadXor1>(cnt);
            qc |= dpp<kDppQuadXor2>(qc);
            while (!done && !want && p >= e) {  // uniform within each quad
                const int nseg = box_segments(X, face);
                if (g < nseg) {
                    p = np;
                    e = ne;
                    ++g;
                    if (g < nseg) fetch();
                    continue;
                }
                const float bnd = box_bound(P, h, q, X);
                const float kth = i2f(static_cast<int>(tau >> 32));
                if (!(bnd < INFINITY) ||
                    (tau != ~0ull && bnd > 0.f && kth < bnd * bnd * (1.f - 0x1p-20f))) {
                    done = true;
                } else if (qc != 0) {
                    want = true;  // merge first, then check again
                } else if (grow == (nearest ? kGridNearestGrow : kGridMaxGrow)) {
                    listed = true;
                    done = true;
                } else {
                    float best = INFINITY;
                    int bf = 0;
#pragma unroll
                    for (int f = 0; f < 6; ++f) {
                        const float d = face_distance(P, h, q, X, f);
                        if (d < best) {
                            best = d;
                            bf = f;
                        }
                    }
#pragma unroll
                    for (int a = 0; a < 3; ++a) {  // constant indices keep X in registers
                        X.bl[a] -= bf == 2 * a;
                        X.bh[a] += bf == 2 * a + 1;
                    }
                    face = bf;
                    ++grow;
                    g = 0;
                    fetch();
                }
            }
            if (ballot(!done) == 0) break;
            const bool has = p < e;
            const int base = has ? p + qi : 0, last = has ? e - 1 : 0;
            float4 rv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) rv[u] = srt[min(base + 4 * u, last)];
            admit8s(rv, has ? e - base : 0);
            if (has) p += 32;
        }
    }
    // A listed query goes to its cloud's list (one atomic per query), and the
    // linear pass of the same call writes its results.
    if (full) {
        if (active && qi == 3) miss_list[b * M + atomicAdd(&miss_count[b], 1)] = m;
        return;  // whole wave
    }
    quad_merge<S>(slot, tau, buf, lane, cnt);
    if (!active) return;
    if (listed) {
        if (qi == 3) miss_list[b * M + atomicAdd(&miss_count[b], 1)] = m;
        return;
    }
    const int64_t row = (b * M + m) * K;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int r = S * qi + s - (KMAX - K);
        if (r >= 0) {
            const uint32_t key = static_cast<uint32_t>(slot[s] >> 32);
            const float d2 = i2f(static_cast<int>(key));
            out_dist[row + r] = slot[s] == ~0ull ? INFINITY : (nearest ? d2 : sqrtf(d2));
            out_idx[row + r] = static_cast<int64_t>(static_cast<uint32_t>(slot[s]));
        }
    }
}

// Exact first-K ball query over the same grid (the result of
// pointops_ball_query_f32 without lengths: the K smallest indices j with
// fl32((dx^2 + dy^2) + dz^2) < r2, ascending, then (-1, 0) padding; a
// non-finite query or point never matches).  A quad of lanes per query scans
// every cell of the box that covers the query's ball -- [q - rb, q + rb] per
// axis, rb = sqrt(r2) (1 + 2^-10) plus a slack of 2^-20 of the coordinate
// magnitude, wider than every point with d < r2 given float rounding, and
// cell assignment is monotone in the coordinate -- keeping an ascending list
// of (index, distance bits) words spread over the quad as in the kNN search.
// A reference whose index is not below the list's K-th is skipped before
// its distance is computed.  Non-finite references sit in the overflow cell,
// which no box reaches; they could not match anyway.
template <int S>
__global__ __launch_bounds__(kGridSearchWaves * kWave) void ball3_grid_kernel(
    const float* __restrict__ query, GridLayout L, int64_t* __restrict__ out_idx,
    float* __restrict__ out_dist, int64_t B, int64_t M, int64_t N, int K, float r2) {
    if (grid_gated_off(L)) return;
    constexpr int KMAX = 4 * S;
    __shared__ uint2 bufs[kGridSearchWaves][kGridCap][kWave];
    const int lane = lane_id();
    const int qi = lane & 3;
    const int wave = uniform(threadIdx.x / kWave);
    const int64_t groups = (M + kGridQueriesPerWave - 1) / kGridQueriesPerWave;
    const int64_t gw = static_cast<int64_t>(xcd_local_block(blockIdx.x, gridDim.x)) * kGridSearchWaves + wave;
    if (gw >= B * groups) return;  // whole wave; no barriers in this kernel
    const int64_t b = gw / groups;
    const int64_t pos = (gw - b * groups) * kGridQueriesPerWave + (lane >> 2);
    const bool active = pos < M;
    const int m = active ? L.q_order[b * M + pos] : 0;
    const float* qp = query + 3 * (b * M + m);
    const float q[3] = {qp[0], qp[1], qp[2]};
    const GridParams P = L.params[b];
    const int* off = L.ref_off + b * L.stride;
    const float4* srt = L.sorted + b * N;
    uint2* buf = &bufs[wave][0][0];
    const bool live = active && finite3(q[0], q[1], q[2]) && r2 > 0.f;

    uint64_t slot[S];
#pragma unroll
    for (int s = 0; s < S; ++s) slot[s] = (live && S * qi + s >= KMAX - K) ? ~0ull : 0ull;
    uint64_t tau = live ? ~0ull : 0ull;
    int cnt = 0;
    auto admit8s = [&](const float4 (&r)[8], int n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t ix = static_cast<uint32_t>(f2i(r[u].w));
            if (4 * u < n && grid_word(ix, 0u) < tau) {
                const float d = sqdist3(r[u].x, r[u].y, r[u].z, q[0], q[1], q[2]);
                if (d < r2) {
                    buf[cnt * kWave + lane] = make_uint2(ix, static_cast<uint32_t>(f2i(d)));
                    ++cnt;
                }
            }
        }
    };

    const float h = 1.f / P.inv_h;
    int c0[3], c1[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float slack = (fabsf(q[a]) + fabsf(P.lo[a]) + static_cast<float>(P.dims[a]) * h) * 0x1p-20f;
        const float rb = sqrtf(r2) * (1.f + 0x1p-10f) + slack;
        c0[a] = cell_axis(q[a] - rb, P.lo[a], P.inv_h, P.dims[a]);
        c1[a] = cell_axis(q[a] + rb, P.lo[a], P.inv_h, P.dims[a]);
    }
    const int ny = c1[1] - c0[1] + 1, nseg = ny * (c1[2] - c0[2] + 1);
    int g = 0, p = 0, e = 0, np = 0, ne = 0;
    auto fetch = [&]() {
        const int y = c0[1] + g % ny, z = c0[2] + g / ny;
        const int row = P.dims[0] * (y + P.dims[1] * z);
        np = off[row + c0[0]];
        ne = off[row + c1[0] + 1];
    };
    bool done = !live;
    if (!done) fetch();
    for (;;) {
        if (ballot(cnt > kGridCap - 8) != 0) {
            quad_merge<S>(slot, tau, buf, lane, cnt);
            cnt = 0;
        }
        while (!done && p >= e) {  // uniform within each quad
            if (g < nseg) {
                p = np;
                e = ne;
                ++g;
                if (g < nseg) fetch();
            } else {
                done = true;
            }
        }
        if (ballot(!done) == 0) break;
        const bool has = p < e;
        const int base = has ? p + qi : 0, last = has ? e - 1 : 0;
        float4 rv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) rv[u] = srt[min(base + 4 * u, last)];
        admit8s(rv, has ? e - base : 0);
        if (has) p += 32;
    }
    quad_merge<S>(slot, tau, buf, lane, cnt);
    if (!active) return;
    const int64_t row = (b * M + m) * K;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int r = S * qi + s - (KMAX - K);
        if (r >= 0) {
            const bool empty = !live || slot[s] == ~0ull;
            out_idx[row + r] = empty ? -1 : static_cast<int64_t>(slot[s] >> 32);
            out_dist[row + r] = empty ? 0.f : i2f(static_cast<int>(static_cast<uint32_t>(slot[s])));
        }
    }
}

// Device-side choice of the ball query between the grid and the index-order
// scan, from the grid build's bounding-box partials: the expected points
// per ball, lambda = N (4/3) pi r^3 / V with V the smallest per-cloud box
// volume (each side at least 2r; float32 products), against sqrt(N K / 6.4):
// the grid examines about 6.4 lambda points per query, the index-order scan
// stops after about N K / lambda.  Writes 1 (grid) or 0 to *choice.  One
// workgroup; wave w reduces the partials of batches w, w + NW, ...
constexpr int kGateThreads = 1024;

__global__ __launch_bounds__(kGateThreads) void ball_grid_choice_kernel(GridLayout L, int64_t B,
                                                                        int64_t N, int parts, int K,
                                                                        float radius_sq,
                                                                        int* __restrict__ choice) {
    constexpr int NW = kGateThreads / kWave;
    __shared__ float wave_vol[NW];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const double radius = sqrt(static_cast<double>(radius_sq));
    const float side = static_cast<float>(2.0 * radius);
    float vmin = INFINITY;
    for (int64_t b = wave; b < B; b += NW) {
        float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
        for (int i = lane; i < parts; i += kWave) {
            const float* t = L.partial + (b * kGridBoundBlocks + i) * 8;
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                mn[a] = fminf(mn[a], t[a]);
                mx[a] = fmaxf(mx[a], t[3 + a]);
            }
        }
        float vol = 1.f;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            // No finite point: max - min = -inf, so the side is 2r.
            vol = vol * fmaxf(wave_max(mx[a]) - wave_min(mn[a]), side);
        }
        vmin = fminf(vmin, vol);
    }
    if (lane == 0) wave_vol[wave] = vmin;
    __syncthreads();
    if (threadIdx.x != 0) return;
    float v = wave_vol[0];
    for (int w = 1; w < NW; ++w) v = fminf(v, wave_vol[w]);
    bool grid = false;
    if (radius_sq > 0.f && radius_sq < INFINITY && v > 0.f && v < INFINITY) {
        constexpr double kPi = 3.14159265358979323846;
        const double per_ball =
            static_cast<double>(N) * (4.0 / 3.0) * kPi * radius * radius * radius / v;
        grid = per_ball < sqrt(static_cast<double>(N) * K / 6.4);
    }
    *choice = grid ? 1 : 0;
}

// Nearest mode's second pass over each cloud's list of the queries the grid
// search left (their nearest reference is several cells away): one
// workgroup per 64 listed queries, lane = query, 8 waves splitting the
// references (batches of 8 read with wide scalar loads, the next batch
// requested before the current one is scanned), the best (squared distance,
// smallest index) per wave combined in LDS.  Workgroups past the list's end
// return at once.
constexpr int kFillThreads = 512;

__global__ void grid_zero_kernel(int* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(kFillThreads) void nearest_fill_kernel(
    const float* __restrict__ query, const float* __restrict__ ref,
    const int* __restrict__ miss_count, const int* __restrict__ miss_list,
    float* __restrict__ dist2, int64_t* __restrict__ idx, int64_t M, int64_t N) {
    constexpr int NWF = kFillThreads / kWave;
    __shared__ int keys[NWF][kWave];
    __shared__ int ids[NWF][kWave];
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x / kWave);
    const int64_t groups = (M + kWave - 1) / kWave;
    const int64_t b = blockIdx.x / groups;
    const int64_t first = (blockIdx.x - b * groups) * kWave;
    const int64_t count = miss_count[b];
    if (first >= count) return;  // uniform over the workgroup, before any barrier
    const bool active = first + lane < count;
    const int64_t row = b * M + miss_list[b * M + (active ? first + lane : first)];
    const float qx = query[3 * row], qy = query[3 * row + 1], qz = query[3 * row + 2];
    const float* rp = ref + 3 * b * N;
    const int64_t per = (N + NWF - 1) / NWF;
    const int64_t lo = min(N, wave * per), hi = min(N, lo + per);
    int best = 0x7FFFFFFF, bi = 0;
    const int64_t hi8 = lo + ((hi - lo) & ~int64_t(7));
    float cur[24], nxt[24];
    if (lo < hi8) {
#pragma unroll
        for (int t = 0; t < 24; ++t) cur[t] = rp[3 * lo + t];
    }
    for (int64_t j = lo; j < hi8; j += 8) {  // ascending: the first minimum is kept
        if (j + 8 < hi8) {
#pragma unroll
            for (int t = 0; t < 24; ++t) nxt[t] = rp[3 * (j + 8) + t];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int key = f2i(sqdist3(cur[3 * u], cur[3 * u + 1], cur[3 * u + 2], qx, qy, qz));
            if (key < best) {
                best = key;
                bi = static_cast<int>(j + u);
            }
        }
#pragma unroll
        for (int t = 0; t < 24; ++t) cur[t] = nxt[t];
    }
    for (int64_t j = hi8; j < hi; ++j) {
        const int key = f2i(sqdist3(rp[3 * j], rp[3 * j + 1], rp[3 * j + 2], qx, qy, qz));
        if (key < best) {
            best = key;
            bi = static_cast<int>(j);
        }
    }
    keys[wave][lane] = best;
    ids[wave][lane] = bi;
    __syncthreads();
    if (wave != 0 || !active) return;
    int k = keys[0][lane], i = ids[0][lane];
#pragma unroll
    for (int w = 1; w < NWF; ++w) {
        const int kk = keys[w][lane], ii = ids[w][lane];
        if (kk < k || (kk == k && ii < i)) {
            k = kk;
            i = ii;
        }
    }
    dist2[row] = i2f(k);
    idx[row] = i;
}

}  // namespace
}  // namespace pointops

using namespace pointops;

namespace {

// Bounding-box partials per batch (grid_bounds_kernel), their count per batch.
int grid_partial_count(int64_t N) {
    return static_cast<int>(std::min<int64_t>(kGridBoundBlocks, (N + 4095) / 4096));
}

// The five build launches shared by the kNN and ball-query searches; with
// `choice` (ball query only) the device-side choice runs after the bounds and
// L.gate must point at it.
void grid_build(const float* query, const float* ref, const GridLayout& L, int64_t B, int64_t M,
                int64_t N, int K, float hmin, hipStream_t stream, int* choice = nullptr,
                float radius_sq = 0.f) {
    const uint32_t nb = static_cast<uint32_t>(B);
    const uint32_t ref_blocks = static_cast<uint32_t>((N + kGridPrepThreads - 1) / kGridPrepThreads);
    const uint32_t q_blocks = static_cast<uint32_t>((M + kGridPrepThreads - 1) / kGridPrepThreads);
    const dim3 point_grid(ref_blocks + q_blocks, nb);
    const dim3 scan_grid(static_cast<uint32_t>(L.tiles), nb, 2);
    const int parts = grid_partial_count(N);
    const dim3 prep(kGridPrepThreads);
    hipLaunchKernelGGL(grid_bounds_kernel, dim3(static_cast<uint32_t>(parts), nb), prep, 0, stream,
                       ref, L, N);
    if (choice != nullptr)
        hipLaunchKernelGGL(ball_grid_choice_kernel, dim3(1), dim3(kGateThreads), 0, stream, L, B, N,
                           parts, K, radius_sq, choice);
    hipLaunchKernelGGL(grid_count_kernel, point_grid, prep, 0, stream, ref, query, L, N, M, ref_blocks,
                       parts, K, hmin);
    hipLaunchKernelGGL(grid_tile_sum_kernel, scan_grid, prep, 0, stream, L);
    hipLaunchKernelGGL(grid_tile_scan_kernel, scan_grid, prep, 0, stream, L);
    hipLaunchKernelGGL(grid_scatter_kernel, point_grid, prep, 0, stream, ref, query, L, N, M, ref_blocks);
}

// Search launch shape: 16 queries per wave, kGridSearchWaves waves per
// workgroup, a multiple of 8 workgroups for the XCD-local deal.
bool grid_search_grid(int64_t B, int64_t M, dim3& grid) {
    const int64_t waves = B * ((M + kGridQueriesPerWave - 1) / kGridQueriesPerWave);
    const int64_t blocks = ((waves + kGridSearchWaves - 1) / kGridSearchWaves + 7) / 8 * 8;
    if (blocks > INT32_MAX) return false;
    grid = dim3(static_cast<uint32_t>(blocks));
    return true;
}

}  // namespace

extern "C" {

size_t pointops_knn3_grid_workspace_bytes(int64_t B, int64_t M, int64_t N) {
    if (B <= 0 || M <= 0 || N <= 0) return 0;
    return grid_layout_bytes(B, M, N, nullptr, nullptr);
}

hipError_t pointops_knn3_grid(const float* query, const float* ref, float* dist, int64_t* idx,
                              void* workspace, int64_t B, int64_t M, int64_t N, int64_t K,
                              hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0 || K < 0 || K > 32 || K > N) return hipErrorInvalidValue;
    if (B == 0 || M == 0 || K == 0) return hipSuccess;
    if (N >= (int64_t(1) << 31) - 64 || M >= (int64_t(1) << 31) - 64 || B > 65535 ||
        workspace == nullptr || (M + kWave - 1) / kWave * B > INT32_MAX)
        return hipErrorInvalidValue;
    dim3 grid;
    if (!grid_search_grid(B, M, grid)) return hipErrorInvalidValue;
    GridLayout L;
    grid_layout_bytes(B, M, N, &L, static_cast<char*>(workspace));
    grid_build(query, ref, L, B, M, N, static_cast<int>(K), 0.f, stream);
    // The build's scan totals and query ranks are dead once the queries are
    // placed: they hold the per-cloud counts and lists of listed queries.
    int* miss_count = L.tile_sum;  // B * 2 * tiles >= B ints
    int* miss_list = L.q_rank;     // B * M ints
    hipLaunchKernelGGL(grid_zero_kernel, dim3(static_cast<uint32_t>((B + 255) / 256)), dim3(256), 0,
                       stream, miss_count, B);
    const dim3 block(kGridSearchWaves * kWave);
    const int k = static_cast<int>(K);
    if (K <= 4)
        hipLaunchKernelGGL((knn3_grid_kernel<1>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0, miss_count, miss_list);
    else if (K <= 8)
        hipLaunchKernelGGL((knn3_grid_kernel<2>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0, miss_count, miss_list);
    else if (K <= 16)
        hipLaunchKernelGGL((knn3_grid_kernel<4>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0, miss_count, miss_list);
    else
        hipLaunchKernelGGL((knn3_grid_kernel<8>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0, miss_count, miss_list);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return knn3_lane_listed(query, ref, dist, idx, B, M, N, k, miss_count, miss_list, stream);
}

hipError_t pointops_nearest3_grid(const float* query, const float* ref, float* dist2,
                                  int64_t* idx, void* workspace, int64_t B, int64_t M, int64_t N,
                                  hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || M == 0) return hipSuccess;
    if (N == 0 || N >= (int64_t(1) << 31) - 64 || M >= (int64_t(1) << 31) - 64 || B > 65535 ||
        workspace == nullptr || B * ((M + kWave - 1) / kWave) > INT32_MAX)
        return hipErrorInvalidValue;
    dim3 grid;
    if (!grid_search_grid(B, M, grid)) return hipErrorInvalidValue;
    GridLayout L;
    grid_layout_bytes(B, M, N, &L, static_cast<char*>(workspace));
    grid_build(query, ref, L, B, M, N, 1, 0.f, stream);
    // The build's scan totals and query ranks are dead once the queries are
    // placed: they hold the per-cloud counts and lists of far queries.
    int* miss_count = L.tile_sum;  // B * 2 * tiles >= B ints
    int* miss_list = L.q_rank;     // B * M ints
    hipLaunchKernelGGL(grid_zero_kernel, dim3(static_cast<uint32_t>((B + 255) / 256)), dim3(256), 0,
                       stream, miss_count, B);
    hipLaunchKernelGGL((knn3_grid_kernel<1>), grid, dim3(kGridSearchWaves * kWave), 0, stream, query,
                       L, dist2, idx, B, M, N, 1, 1, miss_count, miss_list);
    const int64_t fill_blocks = B * ((M + kWave - 1) / kWave);
    hipLaunchKernelGGL(nearest_fill_kernel, dim3(static_cast<uint32_t>(fill_blocks)),
                       dim3(kFillThreads), 0, stream, query, ref, miss_count, miss_list, dist2, idx,
                       M, N);
    return hipGetLastError();
}

size_t pointops_ball_query_grid_workspace_bytes(int64_t B, int64_t Q, int64_t P) {
    return pointops_knn3_grid_workspace_bytes(B, Q, P);
}

}  // extern "C"

namespace {

// The grid ball query; with `choose`, its sort and search are skipped on the
// device unless ball_grid_choice_kernel picks them, and the index-order
// kernel runs otherwise.
hipError_t ball_query_grid(const float* queries, const float* points, int64_t* idx, float* dist2,
                           void* workspace, int64_t B, int64_t Q, int64_t P, int64_t K,
                           float radius_sq, bool choose, hipStream_t stream) {
    if (B < 0 || Q < 0 || P < 0 || K < 0 || K > 64) return hipErrorInvalidValue;
    if (B == 0 || Q == 0 || K == 0) return hipSuccess;
    if (P == 0 || P >= (int64_t(1) << 31) - 64 || Q >= (int64_t(1) << 31) - 64 || B > 65535 ||
        workspace == nullptr)
        return hipErrorInvalidValue;
    dim3 grid;
    if (!grid_search_grid(B, Q, grid)) return hipErrorInvalidValue;
    GridLayout L;
    grid_layout_bytes(B, Q, P, &L, static_cast<char*>(workspace));
    if (choose) L.gate = L.control;
    const float hmin = (radius_sq > 0.f && radius_sq < INFINITY) ? sqrtf(radius_sq) : 0.f;
    grid_build(queries, points, L, B, Q, P, static_cast<int>(K), hmin, stream,
               choose ? L.control : nullptr, radius_sq);
    const dim3 block(kGridSearchWaves * kWave);
    const int k = static_cast<int>(K);
    if (K <= 4)
        hipLaunchKernelGGL((ball3_grid_kernel<1>), grid, block, 0, stream, queries, L, idx, dist2, B, Q, P, k, radius_sq);
    else if (K <= 8)
        hipLaunchKernelGGL((ball3_grid_kernel<2>), grid, block, 0, stream, queries, L, idx, dist2, B, Q, P, k, radius_sq);
    else if (K <= 16)
        hipLaunchKernelGGL((ball3_grid_kernel<4>), grid, block, 0, stream, queries, L, idx, dist2, B, Q, P, k, radius_sq);
    else if (K <= 32)
        hipLaunchKernelGGL((ball3_grid_kernel<8>), grid, block, 0, stream, queries, L, idx, dist2, B, Q, P, k, radius_sq);
    else
        hipLaunchKernelGGL((ball3_grid_kernel<16>), grid, block, 0, stream, queries, L, idx, dist2, B, Q, P, k, radius_sq);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess || !choose) return err;
    return ball_query_f32_unless(queries, points, idx, dist2, B, Q, P, K, radius_sq, L.control,
                                 stream);
}

}  // namespace

extern "C" {

hipError_t pointops_ball_query_grid_f32(const float* queries, const float* points, int64_t* idx,
                                        float* dist2, void* workspace, int64_t B, int64_t Q,
                                        int64_t P, int64_t K, float radius_sq, hipStream_t stream) {
    return ball_query_grid(queries, points, idx, dist2, workspace, B, Q, P, K, radius_sq, false,
                           stream);
}

size_t pointops_ball_query_auto_workspace_bytes(int64_t B, int64_t Q, int64_t P) {
    return pointops_knn3_grid_workspace_bytes(B, Q, P);
}

hipError_t pointops_ball_query_auto_f32(const float* queries, const float* points, int64_t* idx,
                                        float* dist2, void* workspace, int64_t B, int64_t Q,
                                        int64_t P, int64_t K, float radius_sq, hipStream_t stream) {
    return ball_query_grid(queries, points, idx, dist2, workspace, B, Q, P, K, radius_sq, true,
                           stream);
}

}  // extern "C"
