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
// (M <= 16384) a block stages CG rows of one batch and gathers from LDS; the
// backward accumulates g*w_t into LDS rows with LDS float atomics and writes
// each row once.  Larger M falls back to one lane per (b, n) over 4 channels,
// gathering from memory, with hardware float atomics in the backward.
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
#ifndef POINTOPS_TI_BWD_THREADS
#define POINTOPS_TI_BWD_THREADS 1024
#endif
// Backward: one block covers all unknowns of its (batch, channel group), so it
// is wide to keep enough loads and LDS atomics in flight.
constexpr int kTiBwdThreads = POINTOPS_TI_BWD_THREADS;

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
