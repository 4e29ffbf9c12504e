// PointNet++ feature propagation for gfx950: three_nn and three_interpolate.
//
// three_nn: one lane per unknown point, 4 waves splitting the known points,
// which arrive through uniform (scalar) loads.  The three best keys are kept
// in registers; a key is the squared distance's bit pattern (non-negative
// floats order like unsigned integers) with NaN mapped above +inf, and known
// points are visited in index order with a strict `<`, which reproduces the
// stable argsort of pointnet2.py:54-72 (NaN last, ties by index) and the
// strict cascade of kernels/pointnet2.metal:24-43.
//
// three_interpolate: out[b,c,n] = (f[i0]*w0 + f[i1]*w1) + f[i2]*w2
// (kernels/pointnet2.metal:52-71).  When a group of feature rows fits LDS
// (M <= 16384) a block stages CG rows of one batch and gathers from LDS.
// Larger M falls back to one lane per (b, n) over 4 channels, gathering from
// memory.  The backward sums g*w_t per known point in (n, t) order from a
// per-batch CSR of the entries (deterministic, no float atomics) where the
// shape allows, else accumulates into LDS rows with LDS float atomics, or
// into memory with hardware float atomics.
#include <algorithm>

#include "csr_sort.hpp"
#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

// three_nn with one lane per unknown point and NW waves per 64 unknowns, each
// wave scanning a contiguous range of the known points through uniform
// (scalar) loads in batches of 8, the next batch requested before the current
// one is tested.  Keys are min(bits(d), 0x7FC00000): non-negative floats and
// +inf keep their order and every NaN (computed NaNs are quiet, so their
// bits are at least 0x7FC00000 or negative) becomes one key above +inf.  A lane's three best keys stay sorted in
// registers (strict `<` in index order); the NW partial lists are merged in
// range order with the same strict `<`, which keeps ties in index order.
constexpr uint32_t kNanKey = 0x7FC00000u;

template <int NW>
__global__ __launch_bounds__(NW * kWave) void three_nn_lane_kernel(
    const float* __restrict__ unknown, const float* __restrict__ known, float* __restrict__ dist,
    int32_t* __restrict__ idx, int64_t N, int64_t M) {
    __shared__ uint32_t pub_k[NW][3][kWave];
    __shared__ int pub_i[NW][3][kWave];
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x / kWave);
    const CloudBlock cb = cloud_block(static_cast<uint32_t>((N + kWave - 1) / kWave));
    const int64_t b = cb.b;
    const int64_t n = static_cast<int64_t>(cb.x) * kWave + lane;
    const bool active = n < N;
    const float* up = unknown + 3 * (b * N + (active ? n : 0));
    const float ux = up[0], uy = up[1], uz = up[2];
    const float* kp = known + 3 * b * M;
    const int span = static_cast<int>((M + NW - 1) / NW);
    const int lo = wave * span;
    const int hi = static_cast<int>(min<int64_t>(M, static_cast<int64_t>(lo) + span));
    uint32_t k0 = 0xFFFFFFFFu, k1 = 0xFFFFFFFFu, k2 = active ? 0xFFFFFFFFu : 0u;
    int i0 = -1, i1 = -1, i2 = -1;
    auto visit = [&](float rx, float ry, float rz, int j) {
        const uint32_t k = min(static_cast<uint32_t>(f2i(sqdist3(ux, uy, uz, rx, ry, rz))), kNanKey);
        if (k < k2) {  // rare once three are kept: the masked update is skipped
            const bool b0 = k < k0, b1 = k < k1;
            i2 = b1 ? i1 : j;
            i1 = b0 ? i0 : (b1 ? j : i1);
            i0 = b0 ? j : i0;
            k2 = max(k, k1);
            k1 = b0 ? k0 : (b1 ? k : k1);
            k0 = min(k, k0);
        }
    };
    constexpr int kBatch = 8;
    int j0 = lo;
    float cur[3 * kBatch];
    if (j0 + kBatch <= hi) {
#pragma unroll
        for (int t = 0; t < 3 * kBatch; ++t) cur[t] = kp[3 * static_cast<int64_t>(j0) + t];
    }
    for (; j0 + kBatch <= hi; j0 += kBatch) {
        float nxt[3 * kBatch];
        const int jn = min(j0 + kBatch, hi - kBatch);  // stays inside the range
#pragma unroll
        for (int t = 0; t < 3 * kBatch; ++t) nxt[t] = kp[3 * static_cast<int64_t>(jn) + t];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) visit(cur[3 * u], cur[3 * u + 1], cur[3 * u + 2], j0 + u);
#pragma unroll
        for (int t = 0; t < 3 * kBatch; ++t) cur[t] = nxt[t];
    }
    for (; j0 < hi; ++j0) {
        const float* r = kp + 3 * static_cast<int64_t>(j0);
        visit(r[0], r[1], r[2], j0);
    }
    pub_k[wave][0][lane] = k0;
    pub_k[wave][1][lane] = k1;
    pub_k[wave][2][lane] = k2;
    pub_i[wave][0][lane] = i0;
    pub_i[wave][1][lane] = i1;
    pub_i[wave][2][lane] = i2;
    __syncthreads();
    if (wave != 0 || !active) return;
#pragma unroll
    for (int w = 1; w < NW; ++w) {
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const uint32_t k = pub_k[w][s][lane];
            const int j = pub_i[w][s][lane];
            if (k < k2) {
                const bool b0 = k < k0, b1 = k < k1;
                i2 = b1 ? i1 : j;
                i1 = b0 ? i0 : (b1 ? j : i1);
                i0 = b0 ? j : i0;
                k2 = max(k, k1);
                k1 = b0 ? k0 : (b1 ? k : k1);
                k0 = min(k, k0);
            }
        }
    }
    const int64_t o = 3 * (b * N + n);
    dist[o] = sqrtf(i2f(static_cast<int>(k0)));
    dist[o + 1] = sqrtf(i2f(static_cast<int>(k1)));
    dist[o + 2] = sqrtf(i2f(static_cast<int>(k2)));
    idx[o] = i0;
    idx[o + 1] = i1;
    idx[o + 2] = i2;
}

constexpr int kTiThreads = 256;
constexpr int kTiChannels = 4;  // channels per lane

__global__ __launch_bounds__(kTiThreads) void three_interpolate_kernel(
    const float* __restrict__ features, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, float* __restrict__ out, int64_t C, int64_t M, int64_t N) {
    const int64_t b = blockIdx.z;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kTiThreads + threadIdx.x;
    if (n >= N) return;
    const int64_t tri = 3 * (b * N + n);
    const int32_t a0 = idx[tri], a1 = idx[tri + 1], a2 = idx[tri + 2];
    const float w0 = weights[tri], w1 = weights[tri + 1], w2 = weights[tri + 2];
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kTiChannels;
#pragma unroll
    for (int cc = 0; cc < kTiChannels; ++cc) {
        const int64_t c = c0 + cc;
        if (c >= C) break;
        const float* f = features + (b * C + c) * M;
        const float x = f[a0] * w0;
        const float y = f[a1] * w1;
        const float z = f[a2] * w2;
        out[(b * C + c) * N + n] = (x + y) + z;
    }
}

__global__ __launch_bounds__(kTiThreads) void three_interpolate_backward_kernel(
    const float* __restrict__ grad_out, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, float* __restrict__ grad_features, int64_t C, int64_t M,
    int64_t N) {
    const int64_t b = blockIdx.z;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kTiThreads + threadIdx.x;
    if (n >= N) return;
    const int64_t tri = 3 * (b * N + n);
    const int32_t a0 = idx[tri], a1 = idx[tri + 1], a2 = idx[tri + 2];
    const float w0 = weights[tri], w1 = weights[tri + 1], w2 = weights[tri + 2];
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kTiChannels;
#pragma unroll
    for (int cc = 0; cc < kTiChannels; ++cc) {
        const int64_t c = c0 + cc;
        if (c >= C) break;
        const float g = grad_out[(b * C + c) * N + n];
        float* gf = grad_features + (b * C + c) * M;
        unsafeAtomicAdd(gf + a0, g * w0);
        unsafeAtomicAdd(gf + a1, g * w1);
        unsafeAtomicAdd(gf + a2, g * w2);
    }
}

// LDS-staged variants (M <= kTiLdsFloats / CG): one block per (batch,
// group of CG channels, slice of the unknowns).  The CG feature rows are
// staged in LDS with coalesced loads, so the three gathers per output hit LDS
// instead of the vector-memory path, and the index/weight triplets are read
// once per channel group.  Backward accumulates into LDS rows with LDS float
// atomics and writes each row once (no global atomics): the block covers all
// unknowns of its (batch, channel group).
constexpr int kTiLdsFloats = 16384;  // 64 KiB of dynamic LDS
constexpr int kTiSlices = 1;         // unknown-slices per (batch, channel group) in the forward
// Backward: one block covers all unknowns of its (batch, channel group), so it
// is wide to keep enough loads and LDS atomics in flight.
constexpr int kTiBwdThreads = 1024;

// Copy `count` floats from global memory to LDS with float4 loads, eight in
// flight per thread (the source is 16-byte aligned when count % 4 == 0).
__device__ __forceinline__ void stage_rows(float* __restrict__ dst, const float* __restrict__ src,
                                           int64_t count) {
    constexpr int kInFlight = 8;
    if (count % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0) {
        const int64_t n4 = count / 4;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        float4* d4 = reinterpret_cast<float4*>(dst);
        for (int64_t e0 = threadIdx.x; e0 < n4; e0 += kInFlight * kTiThreads) {
            float4 v[kInFlight];
#pragma unroll
            for (int u = 0; u < kInFlight; ++u) {
                const int64_t e = e0 + u * kTiThreads;
                v[u] = e < n4 ? s4[e] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < kInFlight; ++u) {
                const int64_t e = e0 + u * kTiThreads;
                if (e < n4) d4[e] = v[u];
            }
        }
    } else {
        for (int64_t e = threadIdx.x; e < count; e += kTiThreads) dst[e] = src[e];
    }
}

template <int CG>
__global__ __launch_bounds__(kTiThreads) void three_interpolate_lds_kernel(
    const float* __restrict__ features, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, float* __restrict__ out, int64_t C, int64_t M, int64_t N) {
    extern __shared__ float rows[];  // CG x M
    const int64_t b = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CG;
    const int cg = static_cast<int>(min<int64_t>(CG, C - c0));
    stage_rows(rows, features + (b * C + c0) * M, cg * M);  // cg consecutive rows
    __syncthreads();
    const int64_t per = (N + kTiSlices - 1) / kTiSlices;
    const int64_t n_lo = blockIdx.z * per, n_hi = min<int64_t>(N, n_lo + per);
    for (int64_t n = n_lo + threadIdx.x; n < n_hi; n += kTiThreads) {
        const int64_t tri = 3 * (b * N + n);
        const int32_t a0 = idx[tri], a1 = idx[tri + 1], a2 = idx[tri + 2];
        const float w0 = weights[tri], w1 = weights[tri + 1], w2 = weights[tri + 2];
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
            if (cc >= cg) break;
            const float* f = rows + cc * M;
            const float x = f[a0] * w0;
            const float y = f[a1] * w1;
            const float z = f[a2] * w2;
            out[(b * C + c0 + cc) * N + n] = (x + y) + z;
        }
    }
}

template <int CG>
__global__ __launch_bounds__(kTiBwdThreads) void three_interpolate_backward_lds_kernel(
    const float* __restrict__ grad_out, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, float* __restrict__ grad_features, int64_t C, int64_t M,
    int64_t N) {
    extern __shared__ float acc[];  // CG x M
    const int64_t b = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CG;
    const int cg = static_cast<int>(min<int64_t>(CG, C - c0));
    for (int64_t e = threadIdx.x; e < cg * M; e += kTiBwdThreads) acc[e] = 0.f;
    __syncthreads();
    for (int64_t n = threadIdx.x; n < N; n += kTiBwdThreads) {
        const int64_t tri = 3 * (b * N + n);
        const int32_t a0 = idx[tri], a1 = idx[tri + 1], a2 = idx[tri + 2];
        const float w0 = weights[tri], w1 = weights[tri + 1], w2 = weights[tri + 2];
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
            if (cc >= cg) break;
            const float g = grad_out[(b * C + c0 + cc) * N + n];
            float* a = acc + cc * M;
            atomicAdd(a + a0, g * w0);
            atomicAdd(a + a1, g * w1);
            atomicAdd(a + a2, g * w2);
        }
    }
    __syncthreads();
    float* dst = grad_features + (b * C + c0) * M;
    for (int64_t e = threadIdx.x; e < cg * M; e += kTiBwdThreads) dst[e] = acc[e];
}

// Backward as a gather, for M <= 1024 known points and 3N < 65536 entries:
// the workgroup of (batch, group of CG channels) buckets the batch's 3N
// (unknown, slot) entries by known index in LDS (counting sort; 16-bit entry
// ids), sorts each bucket by entry id, then streams grad_out through LDS in
// tiles of NT unknowns x CG channels; thread m consumes its bucket's entries
// of the tile in (n, t) order -- the order of a sequential scatter loop, so
// the result is deterministic -- and writes each gradient element once.  No
// float atomics (LDS float atomics serialise at about one lane per 3 cycles).
constexpr int kTiGatherThreads = 1024;
constexpr int kTiGatherTile = 256;  // unknowns per staged tile
constexpr int kTiGatherChannels = 16;
// LDS for the entry list: 64 KiB minus the scan arrays and the tile.
constexpr int kTiGatherListBytes =
    65536 - (2 * kTiGatherThreads + 1) * 4 - kTiGatherChannels * kTiGatherTile * 4;

template <int CG>
__global__ __launch_bounds__(kTiGatherThreads) void three_interpolate_backward_gather_kernel(
    const float* __restrict__ grad_out, const int32_t* __restrict__ idx,
    const float* __restrict__ weights, float* __restrict__ grad_features, int64_t C, int64_t M,
    int64_t N) {
    constexpr int T = kTiGatherThreads;
    constexpr int NT = kTiGatherTile;
    extern __shared__ uint16_t list[];  // 3N entry ids, bucketed by known index
    __shared__ int start[T + 1];
    __shared__ int cursor[T];
    __shared__ float tile[CG][NT];
    const int tid = threadIdx.x;
    const int m_count = static_cast<int>(M);
    const int n_count = static_cast<int>(N);
    const int e_count = 3 * n_count;
    const int64_t b = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CG;
    const int cg = static_cast<int>(min<int64_t>(CG, C - c0));
    const int32_t* ib = idx + 3 * b * N;
    const float* wb = weights + 3 * b * N;
    const float* gb = grad_out + (b * C + c0) * N;

    cursor[tid] = 0;
    __syncthreads();
    // Indices outside [0, M) contribute nothing (the callers validate them).
    for (int e = tid; e < e_count; e += T) {
        const int a = ib[e];
        if (static_cast<unsigned>(a) < static_cast<unsigned>(m_count)) atomicAdd(&cursor[a], 1);
    }
    __syncthreads();
    // Exclusive scan of the T counts (Hillis-Steele over start[1..T]).
    const int own = cursor[tid];
    start[tid + 1] = own;
    if (tid == 0) start[0] = 0;
    __syncthreads();
    for (int off = 1; off < T; off <<= 1) {
        const int v = tid >= off ? start[tid + 1 - off] : 0;
        __syncthreads();
        start[tid + 1] += v;
        __syncthreads();
    }
    cursor[tid] = start[tid + 1] - own;  // == start[tid]
    __syncthreads();
    for (int e = tid; e < e_count; e += T) {
        const int a = ib[e];
        if (static_cast<unsigned>(a) < static_cast<unsigned>(m_count))
            list[atomicAdd(&cursor[a], 1)] = static_cast<uint16_t>(e);
    }
    __syncthreads();
    const int p0 = start[tid], p1 = start[tid + 1];
    for (int p = p0 + 1; p < p1; ++p) {  // insertion sort: buckets are short
        const uint16_t v = list[p];
        int q = p - 1;
        while (q >= p0 && list[q] > v) {
            list[q + 1] = list[q];
            --q;
        }
        list[q + 1] = v;
    }
    float acc[CG];
#pragma unroll
    for (int cc = 0; cc < CG; ++cc) acc[cc] = 0.f;
    int p = p0;
    for (int t0 = 0; t0 < n_count; t0 += NT) {
        __syncthreads();  // the previous tile (and the sorts) are done
        for (int k = tid; k < CG * NT; k += T) {
            const int cc = k / NT, j = k % NT;
            tile[cc][j] = (cc < cg && t0 + j < n_count) ? gb[static_cast<int64_t>(cc) * N + t0 + j]
                                                        : 0.f;
        }
        __syncthreads();
        const int e_end = 3 * min(t0 + NT, n_count);
        for (; p < p1; ++p) {
            const int e = list[p];
            if (e >= e_end) break;
            const float w = wb[e];
            const float* col = &tile[0][e / 3 - t0];
#pragma unroll
            for (int cc = 0; cc < CG; ++cc) acc[cc] = acc[cc] + col[cc * NT] * w;
        }
    }
    if (tid < m_count) {
#pragma unroll
        for (int cc = 0; cc < CG; ++cc)
            if (cc < cg) grad_features[(b * C + c0 + cc) * M + tid] = acc[cc];
    }
}

// Backward over a CSR of the entries, for M <= 4096 known points and
// N <= 4096 unknowns (N a multiple of 4), with a caller workspace:
//   three_interp_csr_kernel (per batch, R workgroups, each owning the known
//   indices of one residue class mod R): csr_sort_class, a counting sort of
//   the entry ids e = 3n + t by known index m = idx[b,n,t] in LDS, each
//   bucket in ascending order, written with the entries' weights.
//   three_interp_backward_csr_kernel (one workgroup per batch and block of
//   kTiCsrBlock channels): stages the batch's CSR once (ids, starts and each
//   entry's weight, gathered by id), then walks its channels CG at a time
//   with the CG rows of grad_out double-buffered in LDS (the next rows' loads
//   are in flight while the current ones are summed).  Thread m sums
//   grad_out[c, e/3] * w over its list in order -- the order of a sequential
//   scatter loop into a zero-filled array, so the result is deterministic --
//   and writes every element once (zero for a known point no entry selects).
//   No atomics on the gradients.
constexpr int kTiCsrThreads = 1024;
constexpr int kTiCsrMaxM = 4096;
constexpr int kTiCsrMaxN = 4096;
constexpr int kTiCsrBlock = 16;                    // channels per gather workgroup
constexpr int kTiCsrLdsBytes = 160 * 1024 - 1024;  // gather LDS budget
constexpr int kTiCsrStage = 8;                     // 16-byte chunks a thread stages at once
constexpr int kTiCsrRegEntries = 16;               // list entries a gather thread keeps in registers
constexpr int kTiCsrRanges = 8;                    // build workgroups per batch at most

// Per batch, each array is padded to whole 16-byte chunks, so that a batch's
// part starts 16-byte aligned.
struct TiCsr {
    int* start;      // [B][sstride]: bucket starts, M+1 used
    float* weight;   // [B][wstride]: w[e] in list order, 3N used
    uint16_t* list;  // [B][lstride]: entry ids by known index, ascending, 3N used
    uint16_t* key;   // [B][lstride]: the known index of each list position
    int sstride, wstride, lstride;
};

__host__ __device__ inline size_t ti_csr_bytes(int64_t B, int64_t M, int64_t N, TiCsr* out,
                                               char* base) {
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t ss = (M + 1 + 3) & ~int64_t(3), ws = (3 * N + 3) & ~int64_t(3),
                  ls = (3 * N + 7) & ~int64_t(7);
    const size_t start_bytes = up(static_cast<size_t>(B * ss) * sizeof(int));
    const size_t weight_bytes = up(static_cast<size_t>(B * ws) * sizeof(float));
    const size_t list_bytes = up(static_cast<size_t>(B * ls) * sizeof(uint16_t));
    if (out != nullptr) {
        out->start = reinterpret_cast<int*>(base);
        out->weight = reinterpret_cast<float*>(base + start_bytes);
        out->list = reinterpret_cast<uint16_t*>(base + start_bytes + weight_bytes);
        out->key = reinterpret_cast<uint16_t*>(base + start_bytes + weight_bytes + list_bytes);
        out->sstride = static_cast<int>(ss);
        out->wstride = static_cast<int>(ws);
        out->lstride = static_cast<int>(ls);
    }
    return start_bytes + weight_bytes + 2 * list_bytes;
}

__global__ __launch_bounds__(kTiCsrThreads) void three_interp_csr_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ weights, TiCsr csr, int M, int N) {
    const int64_t b = blockIdx.x;
    // Entries e = 3n + t keyed by known index; every bucket in (n, t) order.
    constexpr int kMaxE = 3 * kTiCsrMaxN;
    csr_sort_class<kTiCsrThreads, kMaxE, kTiCsrMaxM, kMaxE, int32_t, true, false>(
        idx + b * 3 * N, weights + b * 3 * N, 3 * N, M, static_cast<int>(blockIdx.y),
        static_cast<int>(gridDim.y), csr.start + b * csr.sstride, csr.list + b * csr.lstride,
        csr.weight + b * csr.wstride, csr.key + b * csr.lstride);
}

// Copies up to kTiCsrStage 16-byte chunks per thread from three consecutive
// source ranges [0, e0), [e0, e1), [e1, e2) of chunk indices into LDS chunks
// dst[...], every load issued before the first store.
__device__ __forceinline__ void stage3(float4* __restrict__ dst, const float4* __restrict__ s0,
                                       const float4* __restrict__ s1,
                                       const float4* __restrict__ s2, int e0, int e1, int e2) {
    if (e2 <= 0) return;
    constexpr int kHalf = kTiCsrStage / 2;  // two arrays: a longer one goes to scratch
    float4 va[kHalf], vb[kHalf];
    auto chunk = [&](int u) {  // past the end: the last chunk again, not stored
        const int i = min(static_cast<int>(threadIdx.x) + u * kTiCsrThreads, e2 - 1);
        return *(i < e0 ? s0 + i : i < e1 ? s1 + (i - e0) : s2 + (i - e1));  // s2 unused if e1 == e2
    };
#pragma unroll
    for (int u = 0; u < kHalf; ++u) va[u] = chunk(u);
#pragma unroll
    for (int u = 0; u < kHalf; ++u) vb[u] = chunk(kHalf + u);
    // Keeps the scheduler from sinking each load down to its store.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kTiCsrStage; ++u) {
        const int i = threadIdx.x + u * kTiCsrThreads;
        if (i < e2) dst[i] = u < kHalf ? va[u] : vb[u - kHalf];
    }
}

// LDS bytes of the gather for CG channels per step: weights [3N], ids
// [lstride], starts [sstride], two row buffers [CG][N].
__host__ __device__ inline int64_t csr_lds_bytes(int cg, int64_t M, int64_t N) {
    const int64_t ss = (M + 1 + 3) & ~int64_t(3), ls = (3 * N + 7) & ~int64_t(7);
    const int64_t ws = (3 * N + 3) & ~int64_t(3);
    return 4 * ws + 2 * ls + 4 * ss + 2 * 4 * cg * N;
}

template <int CG>
__global__ __launch_bounds__(kTiCsrThreads) void three_interp_backward_csr_kernel(
    const float* __restrict__ grad_out, const float* __restrict__ weights, TiCsr csr,
    float* __restrict__ grad_features, int64_t C, int M, int N) {
    static_assert(CG == 1 || CG == 2 || CG == 4, "channels per step");
    extern __shared__ float4 lds4[];
    const int w_chunks = csr.wstride / 4, l_chunks = csr.lstride / 8, s_chunks = csr.sstride / 4;
    const int r_chunks = CG * N / 4;  // one row buffer: [N][CG] floats, channels interleaved
    float* wl = reinterpret_cast<float*>(lds4);
    uint16_t* list = reinterpret_cast<uint16_t*>(lds4 + w_chunks);
    int* start = reinterpret_cast<int*>(lds4 + w_chunks + l_chunks);
    float4* const rb0 = lds4 + w_chunks + l_chunks + s_chunks;  // row buffers
    float4* const rb1 = rb0 + r_chunks;
    const int64_t b = blockIdx.y;
    const int64_t c_lo = static_cast<int64_t>(blockIdx.x) * kTiCsrBlock;
    const int cb = static_cast<int>(min<int64_t>(kTiCsrBlock, C - c_lo));
    const int steps = (cb + CG - 1) / CG;
    const int tid = threadIdx.x;
    const int n_chunks = N / 4;  // <= kTiCsrThreads: one 4-unknown chunk per thread
    const float4* gsrc = reinterpret_cast<const float4*>(grad_out + (b * C + c_lo) * N);
    // A step's rows for this thread's chunk: CG float4 (zero past the block).
    // Two steps are in flight in registers (x: the next step, y: the one
    // after) while the current one is summed from LDS.
    struct Rows {
        float4 r0, r1, r2, r3;
    };
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    Rows x{zero4, zero4, zero4, zero4}, y = x;
    auto fetch = [&](int g, Rows& to) {
        const int cg = min(CG, cb - g * CG);
        if (tid >= n_chunks) return;
        const float4* src = gsrc + static_cast<int64_t>(g) * CG * n_chunks + tid;
        to.r0 = src[0];
        if (CG > 1) to.r1 = cg > 1 ? src[n_chunks] : zero4;
        if (CG > 2) to.r2 = cg > 2 ? src[2 * n_chunks] : zero4;
        if (CG > 3) to.r3 = cg > 3 ? src[3 * n_chunks] : zero4;
    };
    auto put = [&](const Rows& v, float4* dst) {  // unknowns 4*tid .. 4*tid+3, CG channels each
        if (tid >= n_chunks) return;
        if (CG == 1) {
            dst[tid] = v.r0;
        } else if (CG == 2) {
            dst[2 * tid] = make_float4(v.r0.x, v.r1.x, v.r0.y, v.r1.y);
            dst[2 * tid + 1] = make_float4(v.r0.z, v.r1.z, v.r0.w, v.r1.w);
        } else {
            dst[4 * tid] = make_float4(v.r0.x, v.r1.x, v.r2.x, v.r3.x);
            dst[4 * tid + 1] = make_float4(v.r0.y, v.r1.y, v.r2.y, v.r3.y);
            dst[4 * tid + 2] = make_float4(v.r0.z, v.r1.z, v.r2.z, v.r3.z);
            dst[4 * tid + 3] = make_float4(v.r0.w, v.r1.w, v.r2.w, v.r3.w);
        }
    };
    // Prologue, one round trip: weights, ids and starts (contiguous in LDS,
    // in that order) and step 0's rows; steps 1 and 2 requested behind them.
    fetch(0, x);
    stage3(lds4, reinterpret_cast<const float4*>(csr.weight + b * csr.wstride),
           reinterpret_cast<const float4*>(csr.list + b * csr.lstride),
           reinterpret_cast<const float4*>(csr.start + b * csr.sstride), w_chunks,
           w_chunks + l_chunks, w_chunks + l_chunks + s_chunks);
    put(x, rb0);
    if (steps > 1) fetch(1, x);
    if (steps > 2) fetch(2, y);
    __syncthreads();
    // When every thread has one known point (M <= threads), its first
    // kTiCsrRegEntries entries (row offset and weight) stay in registers for
    // all steps; the rest of a longer list is read from LDS.  Otherwise every
    // entry is read from LDS.
    constexpr int kReg = kTiCsrRegEntries;
    const bool one_each = M <= kTiCsrThreads;
    const int m0 = tid;
    const int pb = (one_each && m0 < M) ? start[m0] : 0;
    const int pe = (one_each && m0 < M) ? start[m0 + 1] : 0;
    int ek[kReg];
    float wk[kReg];
#pragma unroll
    for (int k = 0; k < kReg; ++k) {
        const int q = min(pb + k, max(pe - 1, pb));  // an unused slot repeats a valid one
        ek[k] = (pe > pb ? list[q] / 3 : 0) * CG;
        wk[k] = pe > pb ? wl[q] : 0.f;
    }
    for (int g = 0; g < steps; ++g) {
        const float* rows = reinterpret_cast<const float*>((g & 1) ? rb1 : rb0);
        const int cg = min(CG, cb - g * CG);
        const int64_t c0 = c_lo + static_cast<int64_t>(g) * CG;
        if (one_each) {
            if (m0 < M) {
                float acc[CG];
#pragma unroll
                for (int cc = 0; cc < CG; ++cc) acc[cc] = 0.f;
#pragma unroll
                for (int k = 0; k < kReg; ++k) {
                    const bool ok = pb + k < pe;
#pragma unroll
                    for (int cc = 0; cc < CG; ++cc) {
                        const float t = rows[ek[k] + cc] * wk[k];
                        acc[cc] = ok ? acc[cc] + t : acc[cc];
                    }
                }
                // The rest of a long list: eight entries' reads at once (past
                // the end: the last entry again, not added), added in order.
                for (int p = pb + kReg; p < pe; p += 8) {
                    int off[8];
                    float w[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int q = min(p + u, pe - 1);
                        off[u] = (list[q] / 3) * CG;
                        w[u] = wl[q];
                    }
                    float v[8][CG];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
#pragma unroll
                        for (int cc = 0; cc < CG; ++cc) v[u][cc] = rows[off[u] + cc];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const bool ok = p + u < pe;
#pragma unroll
                        for (int cc = 0; cc < CG; ++cc) {
                            const float t = v[u][cc] * w[u];
                            acc[cc] = ok ? acc[cc] + t : acc[cc];
                        }
                    }
                }
#pragma unroll
                for (int cc = 0; cc < CG; ++cc)
                    if (cc < cg) grad_features[(b * C + c0 + cc) * M + m0] = acc[cc];
            }
        } else {
            for (int m = tid; m < M; m += kTiCsrThreads) {
                float acc[CG];
#pragma unroll
                for (int cc = 0; cc < CG; ++cc) acc[cc] = 0.f;
                const int p1 = start[m + 1];
                for (int p = start[m]; p < p1; ++p) {
                    const float* col = rows + (list[p] / 3) * CG;
                    const float w = wl[p];
#pragma unroll
                    for (int cc = 0; cc < CG; ++cc) acc[cc] = acc[cc] + col[cc] * w;
                }
#pragma unroll
                for (int cc = 0; cc < CG; ++cc)
                    if (cc < cg) grad_features[(b * C + c0 + cc) * M + m] = acc[cc];
            }
        }
        if (g + 1 < steps) {
            // Buffer (g+1)&1 last held step g-1, finished before the previous
            // barrier.
            put(x, ((g + 1) & 1) ? rb1 : rb0);
            x = y;
            if (g + 3 < steps) fetch(g + 3, y);
        }
        __syncthreads();
    }
}

// three_interp_csr_gather_kernel, the gather for M <= kTiCsrThreads known
// points: J workgroups per batch, each taking every J-th group of 4
// channels.  Thread t owns positions [12 t, 12 t + 12) of the batch's CSR
// (kTiPiece = 3 * kTiCsrMaxN / kTiCsrThreads), the same work in every lane
// however long the lists are, with each position's unknown index, weight
// and slot in registers for all channel groups.  The 4 rows of a group pass
// through one [N][4] LDS buffer (channels interleaved, so one 16-byte read
// serves a position's 4 channels), each group's rows requested two groups
// ahead into registers.  A thread sums the pieces of lists inside its
// range in list order; a list that crosses ranges is summed piece by piece,
// its first piece by the thread where it starts, which then adds the
// following threads' pieces in order.  So a known point's gradient is the
// sum of fl32(row * w) over its entries in (n, t) order, cut into pieces at
// every 12th CSR position of the batch, each piece summed from +0 in order
// and the pieces added in order.  The results go through LDS to coalesced
// stores; every element of grad_features is written once.
constexpr int kTiPiece = 3 * kTiCsrMaxN / kTiCsrThreads;

__global__ __launch_bounds__(kTiCsrThreads) void three_interp_csr_gather_kernel(
    const float* __restrict__ grad_out, TiCsr csr, float* __restrict__ grad_features, int64_t C,
    int M, int N, uint32_t J) {
    constexpr int T = kTiCsrThreads;
    constexpr int E = kTiPiece;
    constexpr int NK = kTiCsrMaxN / T;  // unknowns per thread when staging rows
    static_assert(E % 4 == 0 && E <= 32, "whole 8-byte id loads, one mask word");
    extern __shared__ float4 lds4[];
    // LDS: the rows [kTiCsrMaxN], then the slots: results [T] (M <= T),
    // continuation pieces [T], head pieces [T], a discard slot per thread [T].
    float4* const rows = lds4;
    float4* const slots = lds4 + kTiCsrMaxN;
    constexpr int kCont = T, kHead = 2 * T, kTrash = 3 * T;
    const CloudBlock cb = cloud_block(J);  // a 1-D launch of B J workgroups
    const int64_t b = cb.b;
    const int64_t j = cb.x;
    const int tid = threadIdx.x;
    const int64_t groups = (C + 3) / 4;
    const int64_t own = j < groups ? (groups - 1 - j) / J + 1 : 0;  // groups j, j + J, ...
    // This thread's positions q0 .. q0 + qn - 1 (the batch's CSR holds the
    // entries whose index lies in [0, M): start[M] of them).
    const int* st = csr.start + b * csr.sstride;
    const int total = st[M];
    const int q0 = tid * E;
    const int qn = max(0, min(E, total - q0));
    const int base = q0 < total ? q0 : 0;  // 3N % 12 == 0: the loads stay inside the list
    uint32_t ids[E / 2], pts[E / 2];
    float w[E];
    {
        const uint2* lp = reinterpret_cast<const uint2*>(csr.list + b * csr.lstride + base);
        const uint2* kp = reinterpret_cast<const uint2*>(csr.key + b * csr.lstride + base);
        const float4* wp = reinterpret_cast<const float4*>(csr.weight + b * csr.wstride + base);
#pragma unroll
        for (int u = 0; u < E / 4; ++u) {
            const uint2 l = lp[u], k = kp[u];
            const float4 v = wp[u];
            ids[2 * u] = l.x;
            ids[2 * u + 1] = l.y;
            pts[2 * u] = k.x;
            pts[2 * u + 1] = k.y;
            w[4 * u] = v.x;
            w[4 * u + 1] = v.y;
            w[4 * u + 2] = v.z;
            w[4 * u + 3] = v.w;
        }
    }
    const int before = q0 > 0 && q0 < total ? csr.key[b * csr.lstride + q0 - 1] : -1;
    const int after = q0 + qn < total ? csr.key[b * csr.lstride + q0 + qn] : -1;
    auto half = [](const uint32_t (&a)[E / 2], int u) {
        return static_cast<int>((u & 1) ? a[u >> 1] >> 16 : a[u >> 1] & 0xFFFFu);
    };
    // Entry ids become unknown indices (n = e / 3), 0 past my positions
    // (weight 0, never stored).
#pragma unroll
    for (int u = 0; u < E / 2; ++u) {
        const uint32_t lo = u * 2 < qn ? (ids[u] & 0xFFFFu) / 3 : 0;
        const uint32_t hi = u * 2 + 1 < qn ? (ids[u] >> 16) / 3 : 0;
        ids[u] = lo | (hi << 16);
    }
    // Per position: does a piece start here (bit u of `fresh`), and the slot
    // its running sum goes to (as in the grouping gather).
    uint32_t fresh = 0;
    uint32_t dest[E / 2];
    int head_m = -1;
    {
        const int first_m = qn > 0 ? half(pts, 0) : -1;
        const bool cont = qn > 0 && before == first_m;
#pragma unroll
        for (int u = 0; u < E; ++u) {
            const int m = half(pts, u);
            const int mm = u + 1 < qn ? half(pts, u + 1) : after;
            if (u < qn && (u == 0 || m != half(pts, u - 1))) fresh |= 1u << u;
            const bool mine_first = cont && m == first_m;  // a list begun before q0
            int d = kTrash + tid;
            if (u < qn && m != mm) {  // the list ends here
                d = mine_first ? kCont + tid : m;
            } else if (u + 1 == qn) {  // the list goes on past my range
                if (mine_first) {
                    d = kCont + tid;  // a middle piece
                } else {
                    d = kHead + tid;
                    head_m = m;
                }
            }
            if (u & 1) dest[u >> 1] |= static_cast<uint32_t>(d) << 16;
            else dest[u >> 1] = static_cast<uint32_t>(d);
        }
    }
    const int head_span = head_m >= 0 ? (st[head_m + 1] - (q0 + qn) + E - 1) / E : 0;
    // A group's rows, thread tid holding unknowns n = tid + k T (k < NK) of
    // its 4 channels, so that the LDS stores (one 16-byte [n][4] entry per
    // lane) go to consecutive addresses.  Every lane loads from inside the
    // batch (row and unknown clamped); what lies outside is zeroed.
    auto fetch = [&](int64_t s, float4 (&r)[NK]) {
        const int64_t c0 = 4 * (j + s * J);
        float v[4][NK];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const float* src = grad_out + (b * C + min(c0 + cc, C - 1)) * N;
#pragma unroll
            for (int k = 0; k < NK; ++k) v[cc][k] = src[min(tid + k * T, N - 1)];
        }
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            r[k] = make_float4(c0 < C ? v[0][k] : 0.f, c0 + 1 < C ? v[1][k] : 0.f,
                               c0 + 2 < C ? v[2][k] : 0.f, c0 + 3 < C ? v[3][k] : 0.f);
        }
    };
    float4 ra[NK], rb[NK];
    if (own > 0) fetch(0, ra);
    if (own > 1) fetch(1, rb);
    // Every result slot starts at 0: a known point with an empty list keeps
    // it, the others are rewritten for every group.
    if (tid < M) slots[tid] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t s = 0; s < own; ++s) {
        __syncthreads();  // every thread is done with the previous group's rows and slots
#pragma unroll
        for (int k = 0; k < NK; ++k)
            if (tid + k * T < N) rows[tid + k * T] = ra[k];
#pragma unroll
        for (int k = 0; k < NK; ++k) ra[k] = rb[k];
        __syncthreads();  // rows complete
        if (s + 2 < own) fetch(s + 2, rb);
        // Keeps the unpacked indices and slots from being hoisted out of the
        // group loop.
#pragma unroll
        for (int u = 0; u < E / 2; ++u) asm volatile("" : "+v"(ids[u]), "+v"(dest[u]));
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < E; ++u) {
            const float4 v = rows[half(ids, u)];
            const bool f = (fresh >> u) & 1u;
            // +0 + fl(row * w): a piece's first term, as the sequential loop
            // adds it to a zero-filled gradient.
            acc.x = (f ? 0.f : acc.x) + v.x * w[u];
            acc.y = (f ? 0.f : acc.y) + v.y * w[u];
            acc.z = (f ? 0.f : acc.z) + v.z * w[u];
            acc.w = (f ? 0.f : acc.w) + v.w * w[u];
            slots[half(dest, u)] = acc;
        }
        __syncthreads();  // pieces complete
        if (head_span > 0) {
            // The following threads' pieces, four reads in flight at a time
            // (past the span: the last piece again, not added).
            float4 v = slots[kHead + tid];
            for (int k0 = 1; k0 <= head_span; k0 += 4) {
                float4 c[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) c[k] = slots[kCont + tid + min(k0 + k, head_span)];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k0 + k <= head_span) {
                        v.x = v.x + c[k].x;
                        v.y = v.y + c[k].y;
                        v.z = v.z + c[k].z;
                        v.w = v.w + c[k].w;
                    }
            }
            slots[head_m] = v;
        }
        __syncthreads();  // results complete
        if (tid < M) {
            const int64_t c0 = 4 * (j + s * J);
            const float4 r = slots[tid];
            float* o = grad_features + (b * C + c0) * M + tid;
            o[0] = r.x;
            if (c0 + 1 < C) o[M] = r.y;
            if (c0 + 2 < C) o[2 * static_cast<int64_t>(M)] = r.z;
            if (c0 + 3 < C) o[3 * static_cast<int64_t>(M)] = r.w;
        }
    }
}

__host__ __device__ inline size_t csr_gather_lds_bytes() {
    return static_cast<size_t>(16 * (kTiCsrMaxN + 4 * kTiCsrThreads));
}

// Channels per step of the CSR gather: the largest CG in {4, 2, 1} whose
// LDS fits the budget (0: none).
int csr_channel_group(int64_t M, int64_t N) {
    for (int cg : {4, 2, 1})
        if (csr_lds_bytes(cg, M, N) <= kTiCsrLdsBytes) return cg;
    return 0;
}

// Channels per block so that CG rows of M floats fit the LDS budget (0: too big).
int lds_channel_group(int64_t M) {
    // At most 4 rows (16 KiB for M = 1024): more, smaller workgroups keep
    // more of HBM busy than 16-row groups do (4.4 against 3.6 TB/s at c2).
    for (int cg : {4, 2, 1})
        if (static_cast<int64_t>(cg) * M <= kTiLdsFloats) return cg;
    return 0;
}

template <int CG>
hipError_t launch_interp_lds(bool backward, const float* a, const int32_t* idx, const float* w,
                             float* o, int64_t B, int64_t C, int64_t M, int64_t N,
                             hipStream_t stream) {
    const size_t shmem = static_cast<size_t>(CG) * static_cast<size_t>(M) * sizeof(float);
    const uint32_t groups = static_cast<uint32_t>((C + CG - 1) / CG);
    if (backward)
        hipLaunchKernelGGL((three_interpolate_backward_lds_kernel<CG>),
                           dim3(groups, static_cast<uint32_t>(B), 1), dim3(kTiBwdThreads), shmem,
                           stream, a, idx, w, o, C, M, N);
    else
        hipLaunchKernelGGL((three_interpolate_lds_kernel<CG>),
                           dim3(groups, static_cast<uint32_t>(B), kTiSlices), dim3(kTiThreads), shmem,
                           stream, a, idx, w, o, C, M, N);
    return hipGetLastError();
}

hipError_t dispatch_interp_lds(bool backward, const float* a, const int32_t* idx, const float* w,
                               float* o, int64_t B, int64_t C, int64_t M, int64_t N,
                               hipStream_t stream) {
    switch (lds_channel_group(M)) {
        case 16: return launch_interp_lds<16>(backward, a, idx, w, o, B, C, M, N, stream);
        case 8: return launch_interp_lds<8>(backward, a, idx, w, o, B, C, M, N, stream);
        case 4: return launch_interp_lds<4>(backward, a, idx, w, o, B, C, M, N, stream);
        case 2: return launch_interp_lds<2>(backward, a, idx, w, o, B, C, M, N, stream);
        default: return launch_interp_lds<1>(backward, a, idx, w, o, B, C, M, N, stream);
    }
}

bool grid_fits(int64_t B, int64_t C, int64_t N) {
    return B <= 65535 && (C + kTiChannels - 1) / kTiChannels <= 65535 &&
           (N + kTiThreads - 1) / kTiThreads <= INT32_MAX;
}

}  // namespace
}  // namespace pointops

using namespace pointops;

extern "C" {

hipError_t pointops_three_nn(const float* unknown, const float* known, float* dist, int32_t* idx,
                             int64_t B, int64_t N, int64_t M, hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || M > INT32_MAX - 64) return hipErrorInvalidValue;
    if (B == 0 || N == 0) return hipSuccess;
    constexpr int NW = 4;
    const int64_t blocks = (N + kWave - 1) / kWave * B;
    if (M < 3 || blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((three_nn_lane_kernel<NW>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(NW * kWave), 0, stream, unknown, known, dist, idx, N, M);
    return hipGetLastError();
}

hipError_t pointops_three_interpolate(const float* features, const int32_t* idx,
                                      const float* weights, float* out, int64_t B, int64_t C,
                                      int64_t M, int64_t N, hipStream_t stream) {
    if (B < 0 || C < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || C == 0 || N == 0) return hipSuccess;
    if (M == 0 || !grid_fits(B, C, N)) return hipErrorInvalidValue;
    if (lds_channel_group(M) > 0)
        return dispatch_interp_lds(false, features, idx, weights, out, B, C, M, N, stream);
    const dim3 grid(static_cast<uint32_t>((N + kTiThreads - 1) / kTiThreads),
                    static_cast<uint32_t>((C + kTiChannels - 1) / kTiChannels),
                    static_cast<uint32_t>(B));
    hipLaunchKernelGGL(three_interpolate_kernel, grid, dim3(kTiThreads), 0, stream, features, idx,
                       weights, out, C, M, N);
    return hipGetLastError();
}

size_t pointops_three_interpolate_backward_workspace_bytes(int64_t B, int64_t M, int64_t N) {
    if (B <= 0 || M <= 0 || N <= 0) return 0;
    return ti_csr_bytes(B, M, N, nullptr, nullptr);
}

hipError_t pointops_three_interpolate_csr_build(const int32_t* idx, const float* weights,
                                               void* workspace, int64_t B, int64_t M, int64_t N,
                                               hipStream_t stream) {
    if (B < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || M == 0) return hipSuccess;
    if (N == 0 || M > kTiCsrMaxM || N > kTiCsrMaxN || N % 4 != 0 || workspace == nullptr ||
        B > 65535 || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return hipErrorInvalidValue;
    TiCsr csr;
    ti_csr_bytes(B, M, N, &csr, static_cast<char*>(workspace));
    // Workgroups per batch (a power of two, each owning the known indices of
    // one residue class): enough to cover the CUs.
    int64_t ranges = 1;
    while (ranges < kTiCsrRanges && ranges * B < 256) ranges *= 2;
    hipLaunchKernelGGL(three_interp_csr_kernel, dim3(static_cast<uint32_t>(B), static_cast<uint32_t>(ranges)),
                       dim3(kTiCsrThreads), 0, stream, idx, weights, csr, static_cast<int>(M),
                       static_cast<int>(N));
    return hipGetLastError();
}

hipError_t pointops_three_interpolate_backward_from_csr(const float* grad_out,
                                                        const void* workspace,
                                                        float* grad_features, int64_t B,
                                                        int64_t C, int64_t M, int64_t N,
                                                        hipStream_t stream) {
    if (B < 0 || C < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || C == 0 || M == 0) return hipSuccess;
    // grad_out rows are staged with 16-byte loads: N % 4 == 0, 16-byte aligned.
    if (N == 0 || M > kTiCsrMaxM || N > kTiCsrMaxN || N % 4 != 0 || workspace == nullptr ||
        B > 65535 || (C + kTiCsrBlock - 1) / kTiCsrBlock > INT32_MAX ||
        reinterpret_cast<uintptr_t>(grad_out) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return hipErrorInvalidValue;
    TiCsr csr;
    ti_csr_bytes(B, M, N, &csr, static_cast<char*>(const_cast<void*>(workspace)));
    const int m = static_cast<int>(M), n = static_cast<int>(N);
    if (M <= kTiCsrThreads) {
        // J workgroups per batch, enough to cover the CUs.
        const int64_t groups = (C + 3) / 4;
        const int64_t J = std::min<int64_t>(groups, std::max<int64_t>(1, (256 + B - 1) / B));
        if (B * J <= INT32_MAX) {
            hipLaunchKernelGGL(three_interp_csr_gather_kernel, dim3(static_cast<uint32_t>(B * J)),
                               dim3(kTiCsrThreads), csr_gather_lds_bytes(), stream, grad_out,
                               csr, grad_features, C, m, n, static_cast<uint32_t>(J));
            return hipGetLastError();
        }
    }
    const int cg = csr_channel_group(M, N);
    if (cg == 0) return hipErrorInvalidValue;
    const size_t shmem = static_cast<size_t>(csr_lds_bytes(cg, M, N));
    const dim3 grid(static_cast<uint32_t>((C + kTiCsrBlock - 1) / kTiCsrBlock),
                    static_cast<uint32_t>(B));
    switch (cg) {
        case 4:
            hipLaunchKernelGGL((three_interp_backward_csr_kernel<4>), grid, dim3(kTiCsrThreads), shmem,
                               stream, grad_out, nullptr, csr, grad_features, C, m, n);
            break;
        case 2:
            hipLaunchKernelGGL((three_interp_backward_csr_kernel<2>), grid, dim3(kTiCsrThreads), shmem,
                               stream, grad_out, nullptr, csr, grad_features, C, m, n);
            break;
        default:
            hipLaunchKernelGGL((three_interp_backward_csr_kernel<1>), grid, dim3(kTiCsrThreads), shmem,
                               stream, grad_out, nullptr, csr, grad_features, C, m, n);
    }
    return hipGetLastError();
}

hipError_t pointops_three_interpolate_backward_csr(const float* grad_out, const int32_t* idx,
                                                   const float* weights, float* grad_features,
                                                   void* workspace, int64_t B, int64_t C, int64_t M,
                                                   int64_t N, hipStream_t stream) {
    if (B < 0 || C < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || C == 0 || M == 0) return hipSuccess;
    if (N == 0 || M > kTiCsrMaxM || N > kTiCsrMaxN || N % 4 != 0 || workspace == nullptr ||
        B > 65535 || (C + kTiCsrBlock - 1) / kTiCsrBlock > INT32_MAX ||
        reinterpret_cast<uintptr_t>(grad_out) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(workspace) % 256 != 0 || csr_channel_group(M, N) == 0)
        return hipErrorInvalidValue;
    const hipError_t err =
        pointops_three_interpolate_csr_build(idx, weights, workspace, B, M, N, stream);
    if (err != hipSuccess) return err;
    return pointops_three_interpolate_backward_from_csr(grad_out, workspace, grad_features, B, C,
                                                        M, N, stream);
}

hipError_t pointops_three_interpolate_backward(const float* grad_out, const int32_t* idx,
                                               const float* weights, float* grad_features,
                                               int64_t B, int64_t C, int64_t M, int64_t N,
                                               hipStream_t stream) {
    if (B < 0 || C < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || C == 0 || N == 0) return hipSuccess;
    if (M == 0 || !grid_fits(B, C, N)) return hipErrorInvalidValue;
    if (M <= kTiGatherThreads && 3 * N * 2 <= kTiGatherListBytes) {
        constexpr int CG = kTiGatherChannels;
        const size_t shmem = static_cast<size_t>(3 * N) * sizeof(uint16_t);
        hipLaunchKernelGGL((three_interpolate_backward_gather_kernel<CG>),
                           dim3(static_cast<uint32_t>((C + CG - 1) / CG), static_cast<uint32_t>(B)),
                           dim3(kTiGatherThreads), shmem, stream, grad_out, idx, weights,
                           grad_features, C, M, N);
        return hipGetLastError();
    }
    if (lds_channel_group(M) > 0)
        return dispatch_interp_lds(true, grad_out, idx, weights, grad_features, B, C, M, N, stream);
    const dim3 grid(static_cast<uint32_t>((N + kTiThreads - 1) / kTiThreads),
                    static_cast<uint32_t>((C + kTiChannels - 1) / kTiChannels),
                    static_cast<uint32_t>(B));
    hipLaunchKernelGGL(three_interpolate_backward_kernel, grid, dim3(kTiThreads), 0, stream, grad_out,
                       idx, weights, grad_features, C, M, N);
    return hipGetLastError();
}

}  // extern "C"
