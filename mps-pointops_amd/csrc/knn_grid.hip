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
//      kGridMaxGrow faces its own query;
//   4. grid_list_kernel: the listed queries compacted in sorted-position
//      order, and the bounding box of every chunk of kChunkRefs sorted
//      references;
//   5. knn3_listed_kernel: a linear pass over the listed queries, 64 per
//      workgroup, that skips the chunks whose box is farther from every lane
//      than an upper bound on its K-th distance.
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
constexpr int kGridMaxGrow = 8;  // box faces a quad may add before its query is listed (measured best of 4-24)
// Nearest mode: box faces a lane may add before its query is left to the
// fill pass (measured best of 4-24).
constexpr int kGridNearestGrow = 6;
constexpr int kGridQueriesPerWave = kWave / 4;  // one quad of lanes per query
constexpr uint32_t kGridMatchLimit = 0x7F800001u;  // keys below: finite or +inf
// Listed queries (those the search leaves to a linear pass) are compacted in
// tiles of query positions; the linear pass prunes chunks of kChunkRefs
// consecutive sorted references by their bounding boxes.
constexpr int64_t kListTileMin = 2048;
constexpr int64_t kListTilesMax = 1024;
constexpr int kChunkRefs = 256;
constexpr int kSuperChunks = 16;
constexpr int kCountSortMin = 4;  // equal-cell neighbour pairs that make a count wave sort

struct alignas(16) GridParams {
    float lo[3];
    float inv_h;
    int dims[3];
    int cells;
    int nonfinite;
    int morton;  // query order: Morton blocks (1) or x-fastest blocks (0)
    int pad[6];
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
    int* list_total; // [B]: listed queries per cloud (the search raises it to 1 first)
    int* list_tiles; // [B][ltiles]: listed queries per tile of query positions
    int* list;       // [B][M]: listed query rows in sorted-position order
    float4* boxes;   // [B][chunks][2]: bounding box of each chunk of sorted references
    float4* supers;  // [B][supers][2]: bounding box of each kSuperChunks chunks
    int64_t stride;  // cap + 2 rounded up to whole 16-byte words
    int64_t tiles;   // scan tiles per array
    int64_t ltile;   // query positions per list tile (a multiple of kListTileMin)
    int64_t ltiles;  // list tiles per cloud (at most kListTilesMax)
    int64_t chunks;  // reference chunks per cloud
    int64_t nsupers; // chunk groups per cloud
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
    const int64_t ltile = kListTileMin * ((M + kListTileMin * kListTilesMax - 1) / (kListTileMin * kListTilesMax));
    const int64_t ltiles = (M + ltile - 1) / ltile;
    const int64_t chunks = (N + kChunkRefs - 1) / kChunkRefs;
    const size_t p_ltot = take(static_cast<size_t>(B + B * ltiles) * sizeof(int));
    const size_t p_list = take(static_cast<size_t>(B * M) * sizeof(int));
    const size_t p_box = take(static_cast<size_t>(B * chunks) * 2 * sizeof(float4));
    const int64_t supers = (chunks + kSuperChunks - 1) / kSuperChunks;
    const size_t p_sup = take(static_cast<size_t>(B * supers) * 2 * sizeof(float4));
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
        out->list_total = reinterpret_cast<int*>(base + p_ltot);
        out->list_tiles = out->list_total + B;
        out->list = reinterpret_cast<int*>(base + p_list);
        out->boxes = reinterpret_cast<float4*>(base + p_box);
        out->supers = reinterpret_cast<float4*>(base + p_sup);
        out->stride = stride;
        out->tiles = tiles;
        out->ltile = ltile;
        out->ltiles = ltiles;
        out->chunks = chunks;
        out->nsupers = supers;
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

// Query order key: the 2 x 2 x 2 block of cells holding the point, so that
// 64 consecutive queries form a compact group.  With P.morton the blocks go
// in Morton order (the bits of the three block coordinates interleaved from
// the lowest, an axis dropping out once its bits are used) scaled into
// [0, cells) by a monotone map -- the tighter groups the kNN linear pass
// prunes with; otherwise in x-fastest order, whose strips share the x-rows
// of cells the ball search reads.  Non-finite queries go to key 0.
__device__ __forceinline__ int query_key(const GridParams& P, float x, float y, float z) {
    if (!finite3(x, y, z)) return 0;
    const float v[3] = {x, y, z};
    uint32_t k = 0;
    int o = 0;
    int c[3], w[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        c[a] = cell_axis(v[a], P.lo[a], P.inv_h, P.dims[a]) >> 1;
        const int nb = (P.dims[a] + 1) >> 1;
        w[a] = nb > 1 ? 32 - __clz(nb - 1) : 0;
    }
    if (!P.morton) {
        const int nbx = (P.dims[0] + 1) >> 1, nby = (P.dims[1] + 1) >> 1;
        return c[0] + nbx * (c[1] + nby * c[2]);
    }
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            if (bit < w[a]) {
                k |= ((static_cast<uint32_t>(c[a]) >> bit) & 1u) << o;
                ++o;
            }
        }
    }
    return static_cast<int>((static_cast<uint64_t>(k) * static_cast<uint64_t>(P.cells)) >> o);
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
    P.morton = 0;
    for (int i = 0; i < 6; ++i) P.pad[i] = 0;
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
                                                                      int K, float hmin, int morton) {
    if (grid_gated_off(L)) return;  // uniform, before any barrier
    __shared__ GridParams shared_params;
    const int64_t b = blockIdx.y;
    if (threadIdx.x < kWave) grid_params(L, b, N, parts, K, hmin, &shared_params);
    if (threadIdx.x == 0) shared_params.morton = morton;
    __syncthreads();
    const GridParams P = shared_params;
    if (blockIdx.x == 0 && threadIdx.x == 0) L.params[b] = P;
    const PrepItem it = prep_item(ref, query, N, M, ref_blocks);
    const bool valid = it.j < it.n;
    int c = -1;
    if (valid) {
        const float* p = it.pts + 3 * (b * it.n + it.j);
        c = it.queries ? query_key(P, p[0], p[1], p[2]) : cell_of(P, p[0], p[1], p[2]);
    }
    // A wave whose neighbouring lanes often share a cell (at least
    // kCountSortMin pairs: clustered or spatially ordered input) sorts its
    // (cell, lane) pairs (bitonic network over the 64 lanes; absent points
    // last), so that each run of equal cells takes one atomic for its length
    // and every lane of the run its offset in it -- such points otherwise
    // queue thousands of atomics on a few cells.  Other waves take one atomic
    // per point.
    const int lane = lane_id();
    int* counts = (it.queries ? L.q_off : L.ref_off) + b * L.stride;
    const int before = __shfl_up(c, 1);
    if (__popcll(ballot(valid && lane > 0 && before == c)) < kCountSortMin) {
        if (valid) (it.queries ? L.q_rank : L.ref_rank)[b * it.n + it.j] = atomicAdd(counts + c, 1);
        return;
    }
    uint32_t key = valid ? static_cast<uint32_t>(c) : 0xFFFFFFFFu;
    int from = lane;
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t ok = static_cast<uint32_t>(__shfl_xor(static_cast<int>(key), stride));
            const int of = __shfl_xor(from, stride);
            const bool up = (lane & size) == 0;
            const bool low = (lane & stride) == 0;
            // (key, from) pairs are distinct, so the order is strict.
            const bool less = ok < key || (ok == key && of < from);
            const bool take = low == up ? less : !less;
            key = take ? ok : key;
            from = take ? of : from;
        }
    }
    const bool real = key != 0xFFFFFFFFu;
    const uint32_t prev = static_cast<uint32_t>(__shfl_up(static_cast<int>(key), 1));
    const uint64_t heads = ballot(real && (lane == 0 || prev != key));
    const uint64_t reals = ballot(real);
    int base = 0;
    if (real && ((heads >> lane) & 1)) {
        const uint64_t above = heads & ~((2ull << lane) - 1);  // heads after this one
        const int end = above != 0 ? __builtin_ctzll(above) : __popcll(reals);
        base = atomicAdd(counts + key, end - lane);
    }
    const uint64_t upto = heads & ((2ull << lane) - 1);  // 2 << 63 wraps to 0: all lanes
    const int head = upto != 0 ? 63 - __builtin_clzll(upto) : 0;
    const int rank = __shfl(base, head) + (lane - head);
    // Back to the lane that holds the point.
    const int mine = __builtin_amdgcn_ds_permute(from * 4, rank);
    if (valid) (it.queries ? L.q_rank : L.ref_rank)[b * it.n + it.j] = mine;
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
    int64_t* __restrict__ out_idx, int64_t B, int64_t M, int64_t N, int K, int nearest) {
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
    const int64_t pos0 = (gw - b * groups) * kGridQueriesPerWave;
    const int64_t pos = pos0 + (lane >> 2);
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
    // Every query's mark at its sorted position (in q_rank, dead since the
    // scatter): its row when listed, else -1.  The wave adds its listed count
    // to its positions' tile (a wave's 16 positions never straddle one) and
    // raises the cloud's flag; the list pass compacts the marks in position
    // order, so neighbours in space stay together, and the linear pass of the
    // same call writes the listed queries' results.
    listed = listed || full;
    const uint64_t lm = ballot(active && listed && qi == 3);
    if (lm != 0 && lane == 0) {
        atomicAdd(&L.list_tiles[b * L.ltiles + pos0 / L.ltile], __popcll(lm));
        L.list_total[b] = 1;
    }
    if (active && qi == 3) L.q_rank[b * M + pos] = listed ? m : -1;
    if (full) return;  // whole wave
    quad_merge<S>(slot, tau, buf, lane, cnt);
    if (!active || listed) return;
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
    const int64_t pos0 = (gw - b * groups) * kGridQueriesPerWave;
    const int64_t pos = pos0 + (lane >> 2);
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

// After the search, per cloud with listed queries: blocks [0, ltiles)
// compact the marks of their tile of query positions into L.list, in
// position order after the listed queries of the tiles before (block 0 also
// stores the cloud's total); with `boxes`, blocks from ltiles on give each
// wave one chunk of kChunkRefs sorted references, or one group of
// kSuperChunks chunks, and store its bounding box (lo, hi), or (-inf, +inf)
// when it holds a non-finite coordinate.
// Clouds with nothing listed return at once.
constexpr int kListWaves = kGridPrepThreads / kWave;
constexpr int kListRounds = 8;  // ballots per wave per pass: 2048 positions per block pass

__global__ __launch_bounds__(kGridPrepThreads) void grid_list_kernel(GridLayout L, int64_t N,
                                                                     int64_t M) {
    const int64_t b = blockIdx.y;
    if (L.list_total[b] == 0) return;  // uniform, before any barrier (1 or the total: both nonzero)
    __shared__ int red[kListWaves];
    __shared__ int counts[kListRounds][kListWaves];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    if (blockIdx.x >= L.ltiles) {
        // Boxes: waves [0, chunks) take one chunk each, the next nsupers one
        // group of kSuperChunks chunks each.
        const int64_t w = (blockIdx.x - L.ltiles) * kListWaves + wave;
        const bool group = w >= L.chunks;
        const int64_t c = group ? w - L.chunks : w;
        if (c >= (group ? L.nsupers : L.chunks)) return;  // whole wave; no barriers below
        const int64_t span = group ? int64_t(kChunkRefs) * kSuperChunks : kChunkRefs;
        const float4* srt = L.sorted + b * N + c * span;
        const int n = static_cast<int>(min<int64_t>(span, N - c * span));
        float lo[3] = {INFINITY, INFINITY, INFINITY}, hi[3] = {-INFINITY, -INFINITY, -INFINITY};
        bool bad = false;
        for (int t = lane; t < n; t += kWave) {
            const float4 r = srt[t];
            const float v[3] = {r.x, r.y, r.z};
            bad = bad || !finite3(r.x, r.y, r.z);
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                lo[a] = isfinite(v[a]) ? fminf(lo[a], v[a]) : lo[a];
                hi[a] = isfinite(v[a]) ? fmaxf(hi[a], v[a]) : hi[a];
            }
        }
        const bool any_bad = ballot(bad) != 0;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            lo[a] = any_bad ? -INFINITY : wave_min(lo[a]);
            hi[a] = any_bad ? INFINITY : wave_max(hi[a]);
        }
        if (lane == 0) {
            float4* box = group ? L.supers + 2 * (b * L.nsupers + c) : L.boxes + 2 * (b * L.chunks + c);
            box[0] = make_float4(lo[0], lo[1], lo[2], 0.f);
            box[1] = make_float4(hi[0], hi[1], hi[2], 0.f);
        }
        return;
    }
    const int64_t tile = blockIdx.x;
    const int* tc = L.list_tiles + b * L.ltiles;
    if (tile == 0) {
        int t = 0;
        for (int64_t i = threadIdx.x; i < L.ltiles; i += kGridPrepThreads) t += tc[i];
        t = block_sum(t, red);
        if (threadIdx.x == 0) L.list_total[b] = t;
    }
    if (tc[tile] == 0) return;  // uniform over the workgroup
    int before = 0;
    for (int64_t i = threadIdx.x; i < tile; i += kGridPrepThreads) before += tc[i];
    before = block_sum(before, red);
    const int* mark = L.q_rank + b * M;
    int* out = L.list + b * M;
    const int64_t end = min(M, (tile + 1) * L.ltile);
    // Positions p0 + u * 256 + threadIdx.x, u < kListRounds: the list order
    // is (u, wave, lane), which is position order.
    for (int64_t p0 = tile * L.ltile; p0 < end; p0 += kListRounds * kGridPrepThreads) {
        int v[kListRounds];
        uint64_t bal[kListRounds];
#pragma unroll
        for (int u = 0; u < kListRounds; ++u) {
            const int64_t p = p0 + u * kGridPrepThreads + threadIdx.x;
            v[u] = p < end ? mark[p] : -1;
            bal[u] = ballot(v[u] >= 0);
        }
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < kListRounds; ++u) counts[u][wave] = __popcll(bal[u]);
        }
        __syncthreads();
        int acc = 0;
        int off[kListRounds];
#pragma unroll
        for (int u = 0; u < kListRounds; ++u) {
            off[u] = 0;
#pragma unroll
            for (int w = 0; w < kListWaves; ++w) {
                off[u] = w == wave ? acc : off[u];
                acc += counts[u][w];
            }
        }
#pragma unroll
        for (int u = 0; u < kListRounds; ++u)
            if (v[u] >= 0) out[before + off[u] + lanes_below(bal[u])] = v[u];
        before += acc;
        __syncthreads();  // counts is rewritten by the next pass
    }
}

// Insert this lane's `cnt` buffered (key, index) candidates into its list
// of 64-bit words, ascending (KMAX - K zero words first, so the K-th entry
// is the last slot); the wave loops while any lane has entries left.
template <int KMAX>
__device__ __forceinline__ void word_merge(uint64_t (&slot)[KMAX], const uint2* buf, int lane,
                                           int cnt) {
    for (int e = 0;; ++e) {
        const bool has = e < cnt;
        if (ballot(has) == 0) break;
        const uint2 c = buf[e * kWave + lane];  // row e < max(cnt): inside the buffer
        const uint64_t w = has ? grid_word(c.x, c.y) : ~0ull;
        bool here = w < slot[KMAX - 1];
        if (ballot(here) == 0) continue;
#pragma unroll
        for (int s = KMAX - 1; s > 0; --s) {
            const bool prev = w < slot[s - 1];
            slot[s] = prev ? slot[s - 1] : (here ? w : slot[s]);
            here = prev;
        }
        slot[0] = here ? w : slot[0];
    }
}

// The linear pass over the listed queries (64 consecutive entries of a
// cloud's list per workgroup, neighbours in space), pruned by the chunk
// boxes of grid_list_kernel.  The chunks c = wave (mod kListedWaves) belong to
// wave `wave`.  First every wave bounds each lane's K-th key from above:
// all references of a chunk of at least K lie within the distance to the
// box's far corner, and the smallest such bound over the chunks is shared
// in LDS.  Then a wave scans a chunk unless, for every lane, the distance
// to the box exceeds both that bound and the smallest K-th key of the
// waves' lists.  Both bounds are computed with the distance arithmetic on
// the per-axis gaps fl(lo - q), fl(q - hi) (float subtraction and the sum of
// squares are monotone, so every reference in the box has a key at or above
// the near bound and at or below the far one), then widened by 2^-20 to
// cover fused or unfused products.  Each lane keeps an ascending list of
// (key, index) words, so the chunks' order does not matter, and the waves'
// lists are merged at the end.  A non-finite query scans every chunk.
constexpr int kListedWaves = 4;
constexpr int kListedCap = 16;  // buffered candidates per lane
constexpr int kListedBatch = 8;

template <int KMAX>
__global__ __launch_bounds__(kListedWaves * kWave) void knn3_listed_kernel(
    const float* __restrict__ query, GridLayout L, float* __restrict__ out_dist,
    int64_t* __restrict__ out_idx, int64_t M, int64_t N, int K) {
    constexpr int NW = kListedWaves;
    constexpr int ROWS = KMAX > kListedCap ? KMAX : kListedCap;
    __shared__ uint2 lds[NW][ROWS][kWave];
    __shared__ uint32_t far_bits[kWave];
    __shared__ uint4 taus[kWave];  // per lane: the K-th key of each wave's list
    static_assert(NW == 4, "one 16-byte word of K-th keys per lane");
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x / kWave);
    const int64_t per_cloud = (M + kWave - 1) / kWave;
    const int64_t b = blockIdx.x / per_cloud;
    const int64_t first = (blockIdx.x - b * per_cloud) * kWave;
    const int64_t count = L.list_total[b];
    if (first >= count) return;  // uniform over the workgroup, before any barrier
    const bool active = first + lane < count;
    const int m = L.list[b * M + (active ? first + lane : first)];
    const float* qp = query + 3 * (b * M + m);
    const float qx = qp[0], qy = qp[1], qz = qp[2];
    const bool qfin = finite3(qx, qy, qz);
    const float4* box = L.boxes + 2 * b * L.chunks;
    const float4* srt = L.sorted + b * N;
    uint2* buf = &lds[wave][0][0];
    uint32_t* my_tau = reinterpret_cast<uint32_t*>(&taus[lane]) + wave;
    if (wave == 0) far_bits[lane] = 0x7F800000u;
    *my_tau = 0xFFFFFFFFu;
    __syncthreads();
    // This wave's groups g = wave + NW i, i < mine (kSuperChunks chunks
    // each), visited 64 at a time: lane l loads the box of the l-th, and the
    // wave reads them in turn with readlane; a group some lane still needs
    // has its chunk boxes loaded the same way (lane u: chunk u).
    const float4* gbox = L.supers + 2 * b * L.nsupers;
    const int64_t mine = L.nsupers > wave ? (L.nsupers - wave + NW - 1) / NW : 0;
    auto rl = [](float v, int t) { return i2f(readlane(f2i(v), t)); };
    // Squared distance from the query to box t of (lo, hi), computed as the
    // references' keys are on the per-axis gaps, then lowered by 2^-20.
    auto near_key = [&](const float4& lo, const float4& hi, int t) {
        const float gx = qx - __builtin_amdgcn_fmed3f(qx, rl(lo.x, t), rl(hi.x, t));
        const float gy = qy - __builtin_amdgcn_fmed3f(qy, rl(lo.y, t), rl(hi.y, t));
        const float gz = qz - __builtin_amdgcn_fmed3f(qz, rl(lo.z, t), rl(hi.z, t));
        return __float_as_uint(sqdist3(gx, gy, gz, 0.f, 0.f, 0.f) * (1.f - 0x1p-20f));
    };

    // Upper bound: the nearest far corner over the chunks of at least K.  A
    // group nearer to no lane than its current bound cannot lower it (every
    // chunk's far corner is at least the group's near distance).
    {
        float far = INFINITY;
        for (int64_t i0 = 0; i0 < mine; i0 += kWave) {
            const int64_t g = wave + NW * min<int64_t>(i0 + lane, mine - 1);
            const float4 glo = gbox[2 * g], ghi = gbox[2 * g + 1];
            const int nb = static_cast<int>(min<int64_t>(kWave, mine - i0));
            for (int t = 0; t < nb; ++t) {
                const uint32_t gn = near_key(glo, ghi, t);
                if (ballot(active && qfin && __uint_as_float(gn) < far) == 0) continue;
                const int64_t c0 = (wave + NW * (i0 + t)) * kSuperChunks;
                const int nc = static_cast<int>(min<int64_t>(kSuperChunks, L.chunks - c0));
                const int64_t cl = c0 + min(lane, nc - 1);
                const float4 lo = box[2 * cl], hi = box[2 * cl + 1];
                for (int u = 0; u < nc; ++u) {
                    // Chunk u's box: the larger of |fl(lo - q)|, |fl(hi - q)| per axis.
                    const float ax = fmaxf(fabsf(rl(lo.x, u) - qx), fabsf(rl(hi.x, u) - qx));
                    const float ay = fmaxf(fabsf(rl(lo.y, u) - qy), fabsf(rl(hi.y, u) - qy));
                    const float az = fmaxf(fabsf(rl(lo.z, u) - qz), fabsf(rl(hi.z, u) - qz));
                    const float d = sqdist3(ax, ay, az, 0.f, 0.f, 0.f);
                    if (N - (c0 + u) * kChunkRefs >= K) far = fminf(far, d);
                }
            }
        }
        far *= 1.f + 0x1p-20f;
        if (active && qfin && far < INFINITY) atomicMin(&far_bits[lane], __float_as_uint(far));
    }
    __syncthreads();
    const uint32_t farkey = qfin ? min(far_bits[lane], 0x7F800000u) : 0x7F800000u;

    uint64_t slot[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) slot[s] = (active && s >= KMAX - K) ? ~0ull : 0ull;
    // Exclusive admission limit on keys: at or below the far bound and every
    // wave's K-th key (a key above another wave's K-th cannot be among the
    // K; an equal key can, with a smaller index).  Inactive lanes admit
    // nothing.  Other waves' keys are read without synchronisation: they only
    // decrease, so a stale one is a looser but valid limit.
    auto limit = [&]() -> uint32_t {
        const uint4 t = taus[lane];
        const uint32_t k = min(min(farkey, min(t.x, t.y)), min(t.z, t.w));
        return active ? k + 1u : 0u;
    };
    int cnt = 0;
    uint32_t lim = limit();
    auto drain = [&]() {
        if (ballot(cnt > kListedCap - kListedBatch) != 0) {
            word_merge<KMAX>(slot, buf, lane, cnt);
            cnt = 0;
            *my_tau = static_cast<uint32_t>(slot[KMAX - 1] >> 32);
        }
    };
    // One chunk's references through uniform (scalar) loads, a batch ahead;
    // a batch whose keys are all at or above every lane's limit costs no
    // buffer traffic.
    auto scan_chunk = [&](int64_t j0) {
        const int n = static_cast<int>(min<int64_t>(kChunkRefs, N - j0));
        const float4* cp = srt + j0;
        float4 cur[kListedBatch];
#pragma unroll
        for (int u = 0; u < kListedBatch; ++u) cur[u] = cp[min(u, n - 1)];
        for (int r0 = 0; r0 < n; r0 += kListedBatch) {
            const int rn = r0 + kListedBatch < n ? r0 + kListedBatch : r0;
            float4 nxt[kListedBatch];
#pragma unroll
            for (int u = 0; u < kListedBatch; ++u) nxt[u] = cp[min(rn + u, n - 1)];
            uint32_t key[kListedBatch];
            uint32_t least = 0xFFFFFFFFu;
#pragma unroll
            for (int u = 0; u < kListedBatch; ++u) {
                key[u] = r0 + u < n
                    ? static_cast<uint32_t>(f2i(sqdist3(cur[u].x, cur[u].y, cur[u].z, qx, qy, qz)))
                    : 0xFFFFFFFFu;
                least = min(least, key[u]);
            }
            if (ballot(least < lim) != 0) {
#pragma unroll
                for (int u = 0; u < kListedBatch; ++u) {
                    if (key[u] < lim) {
                        buf[cnt * kWave + lane] = make_uint2(key[u], static_cast<uint32_t>(f2i(cur[u].w)));
                        ++cnt;
                    }
                }
                drain();
                lim = limit();
            }
#pragma unroll
            for (int u = 0; u < kListedBatch; ++u) cur[u] = nxt[u];
        }
    };
    // Scan every chunk of a needed group that some lane needs: its box nearer
    // than the lane's limit (or a non-finite query).
    auto needed = [&](uint32_t nk) { return ballot(active && (!qfin || nk < lim)) != 0; };
    for (int64_t i0 = 0; i0 < mine; i0 += kWave) {
        const int64_t g = wave + NW * min<int64_t>(i0 + lane, mine - 1);
        const float4 glo = gbox[2 * g], ghi = gbox[2 * g + 1];
        const int nb = static_cast<int>(min<int64_t>(kWave, mine - i0));
        for (int t = 0; t < nb; ++t) {
            lim = limit();
            if (!needed(near_key(glo, ghi, t))) continue;
            const int64_t c0 = (wave + NW * (i0 + t)) * kSuperChunks;
            const int nc = static_cast<int>(min<int64_t>(kSuperChunks, L.chunks - c0));
            const int64_t cl = c0 + min(lane, nc - 1);
            const float4 lo = box[2 * cl], hi = box[2 * cl + 1];
            for (int k = 0; k < nc; ++k)
                if (needed(near_key(lo, hi, k))) scan_chunk((c0 + k) * kChunkRefs);
        }
    }
    word_merge<KMAX>(slot, buf, lane, cnt);

    // Merge the waves' lists: wave 0 keeps every list's head in registers.
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
        if (s >= KMAX - K)
            lds[wave][s - (KMAX - K)][lane] =
                make_uint2(static_cast<uint32_t>(slot[s] >> 32), static_cast<uint32_t>(slot[s]));
    __syncthreads();
    if (wave != 0 || !active) return;
    auto word_at = [&](int w, int s) {
        const uint2 v = lds[w][s][lane];
        return grid_word(v.x, v.y);
    };
    uint64_t head[NW];
    int next[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        head[w] = word_at(w, 0);
        next[w] = 1;
    }
    const int64_t row = (b * M + m) * K;
    for (int s = 0; s < K; ++s) {
        uint64_t best = head[0];
        int from = 0;
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const bool less = head[w] < best;
            best = less ? head[w] : best;
            from = less ? w : from;
        }
        int h = next[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) h = from == w ? next[w] : h;
        const uint64_t fresh = h < K ? word_at(from, h) : ~0ull;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            head[w] = from == w ? fresh : head[w];
            next[w] = from == w ? h + 1 : next[w];
        }
        const float d2 = i2f(static_cast<int>(static_cast<uint32_t>(best >> 32)));
        out_dist[row + s] = best == ~0ull ? INFINITY : sqrtf(d2);
        out_idx[row + s] = static_cast<int64_t>(static_cast<uint32_t>(best));
    }
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
                int64_t N, int K, float hmin, int morton, hipStream_t stream,
                int* choice = nullptr, float radius_sq = 0.f) {
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
                       parts, K, hmin, morton);
    hipLaunchKernelGGL(grid_tile_sum_kernel, scan_grid, prep, 0, stream, L);
    hipLaunchKernelGGL(grid_tile_scan_kernel, scan_grid, prep, 0, stream, L);
    hipLaunchKernelGGL(grid_scatter_kernel, point_grid, prep, 0, stream, ref, query, L, N, M, ref_blocks);
}

// Listed-query counts and flags to zero before the search.
void grid_list_zero(const GridLayout& L, int64_t B, hipStream_t stream) {
    const int64_t n = B + B * L.ltiles;
    hipLaunchKernelGGL(grid_zero_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                       stream, L.list_total, n);
}

// The list pass after the search: compaction, and the chunk boxes when the
// linear pass prunes by them.
void grid_list(const GridLayout& L, int64_t B, int64_t M, int64_t N, bool boxes, hipStream_t stream) {
    const int64_t box_blocks = boxes ? (L.chunks + L.nsupers + kListWaves - 1) / kListWaves : 0;
    hipLaunchKernelGGL(grid_list_kernel, dim3(static_cast<uint32_t>(L.ltiles + box_blocks),
                                              static_cast<uint32_t>(B)),
                       dim3(kGridPrepThreads), 0, stream, L, N, M);
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
    grid_build(query, ref, L, B, M, N, static_cast<int>(K), 0.f, 1, stream);
    grid_list_zero(L, B, stream);
    const dim3 block(kGridSearchWaves * kWave);
    const int k = static_cast<int>(K);
    if (K <= 4)
        hipLaunchKernelGGL((knn3_grid_kernel<1>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0);
    else if (K <= 8)
        hipLaunchKernelGGL((knn3_grid_kernel<2>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0);
    else if (K <= 16)
        hipLaunchKernelGGL((knn3_grid_kernel<4>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0);
    else
        hipLaunchKernelGGL((knn3_grid_kernel<8>), grid, block, 0, stream, query, L, dist, idx, B, M, N, k, 0);
    grid_list(L, B, M, N, true, stream);
    const dim3 listed(static_cast<uint32_t>(B * ((M + kWave - 1) / kWave)));
    const dim3 lblock(kListedWaves * kWave);
    if (K <= 8)
        hipLaunchKernelGGL((knn3_listed_kernel<8>), listed, lblock, 0, stream, query, L, dist, idx, M, N, k);
    else if (K <= 16)
        hipLaunchKernelGGL((knn3_listed_kernel<16>), listed, lblock, 0, stream, query, L, dist, idx, M, N, k);
    else
        hipLaunchKernelGGL((knn3_listed_kernel<32>), listed, lblock, 0, stream, query, L, dist, idx, M, N, k);
    return hipGetLastError();
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
    grid_build(query, ref, L, B, M, N, 1, 0.f, 1, stream);
    grid_list_zero(L, B, stream);
    hipLaunchKernelGGL((knn3_grid_kernel<1>), grid, dim3(kGridSearchWaves * kWave), 0, stream, query,
                       L, dist2, idx, B, M, N, 1, 1);
    grid_list(L, B, M, N, false, stream);
    const int64_t fill_blocks = B * ((M + kWave - 1) / kWave);
    hipLaunchKernelGGL(nearest_fill_kernel, dim3(static_cast<uint32_t>(fill_blocks)),
                       dim3(kFillThreads), 0, stream, query, ref, L.list_total, L.list, dist2, idx,
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
    grid_build(queries, points, L, B, Q, P, static_cast<int>(K), hmin, 0, stream,
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
