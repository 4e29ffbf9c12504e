// Point gathers of PointNet++ set abstraction for gfx950.
//
// gather_operation and grouping_operation of the pointnet2_ops stand-in
// (compat.py:62-73: torch.gather along the point axis) are one operation on a
// flattened index: out[b,c,p] = features[b,c,idx[b,p]], with p over npoint
// (gather) or npoint * nsample (grouping).  The backward is the scatter-add
// of torch.gather's gradient, computed as a gather over the inverse index
// (deterministic, in increasing p).  group_points_rel_kernel fuses the set
// abstraction's grouping (tests/test_pointnet2_e2e.py:36-45, the step after
// ball query): channels 0-2 are the grouped xyz less the query centre
// (grouped_xyz - new_xyz, one float subtraction as in the reference layer),
// channels 3.. the grouped features, written once into the concatenated
// (B, 3+C, npoint, nsample) tensor instead of two gathers, a subtraction and
// a concatenation.
//
// Layout: one thread per output column (b, p) reads its index once and walks
// a block of channels; for a fixed channel, consecutive threads write
// consecutive p (coalesced), and the feature reads gather within one channel
// row, which stays in L2.  HBM traffic is the output plus one read of each
// feature row and of the index.  Indices outside [0, N) are clamped into it
// (the callers check the range first; the clamp keeps every access in
// bounds).
#include <algorithm>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kGroupThreads = 256;
constexpr int kGroupChannels = 16;  // channels per thread

template <typename I>
__device__ __forceinline__ int64_t group_index(const I* idx, int64_t at, int64_t N) {
    const int64_t j = static_cast<int64_t>(idx[at]);
    return j < 0 ? 0 : (j >= N ? N - 1 : j);
}

template <typename I>
__global__ __launch_bounds__(kGroupThreads) void group_points_kernel(
    const float* __restrict__ f, const I* __restrict__ idx, float* __restrict__ out, int64_t C,
    int64_t N, int64_t P) {
    const int64_t b = blockIdx.y;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kGroupThreads + threadIdx.x;
    if (p >= P) return;
    const int64_t j = group_index(idx, b * P + p, N);
    const int64_t c0 = static_cast<int64_t>(blockIdx.z) * kGroupChannels;
    const int64_t c1 = c0 + kGroupChannels < C ? c0 + kGroupChannels : C;
    const float* src = f + (b * C + c0) * N + j;
    float* dst = out + (b * C + c0) * P + p;
    for (int64_t c = c0; c < c1; ++c, src += N, dst += P) *dst = *src;
}

// Channels 0-2: xyz[b, j, a] - centre[b, p / S, a]; channels 3..: features.
template <typename I>
__global__ __launch_bounds__(kGroupThreads) void group_points_rel_kernel(
    const float* __restrict__ xyz, const float* __restrict__ centres, const float* __restrict__ f,
    const I* __restrict__ idx, float* __restrict__ out, int64_t C, int64_t N, int64_t M, int64_t S) {
    const int64_t b = blockIdx.y;
    const int64_t P = M * S;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kGroupThreads + threadIdx.x;
    if (p >= P) return;
    const int64_t j = group_index(idx, b * P + p, N);
    const int64_t CT = C + 3;
    int64_t c0 = static_cast<int64_t>(blockIdx.z) * kGroupChannels;
    const int64_t c1 = c0 + kGroupChannels < CT ? c0 + kGroupChannels : CT;
    float* dst = out + (b * CT + c0) * P + p;
    if (c0 < 3) {
        const float* q = xyz + (b * N + j) * 3;
        const float* m = centres + (b * M + p / S) * 3;
        for (; c0 < 3 && c0 < c1; ++c0, dst += P) *dst = q[c0] - m[c0];
    }
    if (c0 >= c1) return;  // also when there are no feature channels
    const float* src = f + (b * C + (c0 - 3)) * N + j;
    for (int64_t c = c0; c < c1; ++c, src += N, dst += P) *dst = *src;
}

// Backward: grad_features[b,c,n] = sum of grad_out[b,c,p] over the p with
// idx[b,p] = n, added in increasing p (the order of a sequential loop, so
// the result is deterministic) for points gathered at most 256 times; a
// point gathered more often sums in an unspecified order.  The inverse of the index is built per call
// in the workspace: per batch, counts of each point (the atomic return value
// is the entry's rank), an exclusive scan into offsets, placement of each p
// at offset + rank (in no particular order within a point), grad_out
// transposed to (B, P, C) so that one entry's channels are contiguous; then
// one wave per point walks its entries in increasing p
// (group_gather_grad_kernel), so every element of grad_features is written
// exactly once (no float atomics).
struct GroupInverse {
    int* off;     // [B][N + 1]: counts, then offsets
    int* rank;    // [B][P]
    int* list;    // [B][P]: p grouped by point
    float* gt;    // [B][P][C]: grad_out transposed, channels contiguous
};

__host__ __device__ inline size_t group_align(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

__host__ __device__ inline size_t group_inverse_bytes(int64_t B, int64_t C, int64_t N, int64_t P,
                                                      GroupInverse* out, char* base) {
    const size_t off = 0;
    const size_t rank = group_align(off + static_cast<size_t>(B * (N + 1)) * sizeof(int));
    const size_t list = group_align(rank + static_cast<size_t>(B * P) * sizeof(int));
    const size_t gt = group_align(list + static_cast<size_t>(B * P) * sizeof(int));
    const size_t end = group_align(gt + static_cast<size_t>(B * P * C) * sizeof(float));
    if (out != nullptr) {
        out->off = reinterpret_cast<int*>(base + off);
        out->rank = reinterpret_cast<int*>(base + rank);
        out->list = reinterpret_cast<int*>(base + list);
        out->gt = reinterpret_cast<float*>(base + gt);
    }
    return end;
}

// gt[b][p][c] = g[b*g_batch + c*P + p], through a 64 x 64 LDS tile (both
// sides coalesced).  blockIdx = (p tile, c tile, b).
constexpr int kGroupTile = 64;
__global__ __launch_bounds__(kGroupThreads) void group_transpose_kernel(
    const float* __restrict__ g, int64_t g_batch, float* __restrict__ gt, int64_t C, int64_t P) {
    __shared__ float tile[kGroupTile][kGroupTile + 1];
    const int64_t b = blockIdx.z;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kGroupTile;
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kGroupTile;
    const int tx = threadIdx.x % kGroupTile, ty = threadIdx.x / kGroupTile;
    for (int r = ty; r < kGroupTile; r += kGroupThreads / kGroupTile) {
        const int64_t c = c0 + r, p = p0 + tx;
        tile[r][tx] = (c < C && p < P) ? g[b * g_batch + c * P + p] : 0.f;
    }
    __syncthreads();
    for (int r = ty; r < kGroupTile; r += kGroupThreads / kGroupTile) {
        const int64_t p = p0 + r, c = c0 + tx;
        if (p < P && c < C) gt[(b * P + p) * C + c] = tile[tx][r];
    }
}

__global__ __launch_bounds__(kGroupThreads) void group_zero_kernel(int* __restrict__ a, int64_t n) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * kGroupThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kGroupThreads + threadIdx.x; i < n; i += step)
        a[i] = 0;
}

template <typename I>
__global__ __launch_bounds__(kGroupThreads) void group_count_kernel(const I* __restrict__ idx,
                                                                    GroupInverse V, int64_t N,
                                                                    int64_t P) {
    const int64_t b = blockIdx.y;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kGroupThreads + threadIdx.x;
    if (p >= P) return;
    const int64_t j = group_index(idx, b * P + p, N);
    V.rank[b * P + p] = atomicAdd(V.off + b * (N + 1) + j, 1);
}

// One workgroup per batch: exclusive scan of the N + 1 counts (the last is
// 0 and receives the total), each thread over a contiguous chunk.
constexpr int kGroupScanThreads = 1024;
__global__ __launch_bounds__(kGroupScanThreads) void group_scan_kernel(GroupInverse V, int64_t N) {
    __shared__ int part[kGroupScanThreads];
    int* a = V.off + static_cast<int64_t>(blockIdx.x) * (N + 1);
    const int64_t count = N + 1;
    const int tid = threadIdx.x;
    const int64_t per = (count + kGroupScanThreads - 1) / kGroupScanThreads;
    const int64_t lo = tid * per < count ? tid * per : count;
    const int64_t hi = lo + per < count ? lo + per : count;
    int run = 0;
    for (int64_t i = lo; i < hi; ++i) run += a[i];
    part[tid] = run;
    __syncthreads();
    for (int s = 1; s < kGroupScanThreads; s <<= 1) {
        const int v = tid >= s ? part[tid - s] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    run = part[tid] - run;
    for (int64_t i = lo; i < hi; ++i) {
        const int c = a[i];
        a[i] = run;
        run += c;
    }
}

template <typename I>
__global__ __launch_bounds__(kGroupThreads) void group_place_kernel(const I* __restrict__ idx,
                                                                    GroupInverse V, int64_t N,
                                                                    int64_t P) {
    const int64_t b = blockIdx.y;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kGroupThreads + threadIdx.x;
    if (p >= P) return;
    const int64_t j = group_index(idx, b * P + p, N);
    V.list[b * P + V.off[b * (N + 1) + j] + V.rank[b * P + p]] = static_cast<int>(p);
}

// One wave per (b, n, 64 channels), lane = channel: the wave walks the
// point's entries in increasing p -- each step takes the smallest entry
// above the previous one (a wave minimum over the entries, held four per lane
// for lists of up to 256) -- and adds that entry's gradient to every lane's
// channel.  Entries are distinct, so the walk visits each once, in order,
// without sorting the list.
constexpr int kGroupListRegs = 4;
__global__ __launch_bounds__(kGroupThreads) void group_gather_grad_kernel(
    GroupInverse V, float* __restrict__ gf, int64_t C, int64_t N, int64_t P, int64_t chunks) {
    const int lane = lane_id();
    const int64_t wid = static_cast<int64_t>(blockIdx.x) * (kGroupThreads / kWave) +
                        uniform(threadIdx.x / kWave);
    const int64_t b = blockIdx.y;
    if (wid >= N * chunks) return;  // whole wave
    const int64_t n = wid / chunks;
    const int64_t c = (wid - n * chunks) * kWave + lane;
    const bool live = c < C;
    const int lo = V.off[b * (N + 1) + n], hi = V.off[b * (N + 1) + n + 1];
    const int L = hi - lo;
    const int* l = V.list + b * P + lo;
    const float* gc = V.gt + b * P * C + (live ? c : 0);
    float acc = 0.f;
    int last = -1;
    if (L <= kGroupListRegs * kWave) {
        int e[kGroupListRegs];
#pragma unroll
        for (int r = 0; r < kGroupListRegs; ++r) {
            const int i = r * kWave + lane;
            e[r] = i < L ? l[i] : INT_MAX;
        }
        for (int t = 0; t < L; ++t) {
            int m = INT_MAX;
#pragma unroll
            for (int r = 0; r < kGroupListRegs; ++r) m = min(m, e[r] > last ? e[r] : INT_MAX);
            last = wave_min(m);
            acc = acc + gc[static_cast<int64_t>(last) * C];
        }
    } else {
        // A point gathered more than 256 times: its entries in list order
        // (the order the counting pass placed them, which varies between
        // runs), O(L) rather than an O(L^2) ordered walk.
        for (int i = 0; i < L; ++i) acc = acc + gc[static_cast<int64_t>(l[i]) * C];
    }
    if (live) gf[(b * C + c) * N + n] = acc;
}

bool group_grid(int64_t B, int64_t channels, int64_t P, dim3& grid) {
    const int64_t x = (P + kGroupThreads - 1) / kGroupThreads;
    const int64_t z = (channels + kGroupChannels - 1) / kGroupChannels;
    if (x > INT32_MAX || B > 65535 || z > 65535) return false;
    grid = dim3(static_cast<uint32_t>(x), static_cast<uint32_t>(B), static_cast<uint32_t>(z));
    return true;
}

}  // namespace
}  // namespace pointops

using namespace pointops;

extern "C" {

hipError_t pointops_group_points(const float* features, const void* idx, int idx_bits, float* out,
                                 int64_t B, int64_t C, int64_t N, int64_t P, hipStream_t stream) {
    if (B < 0 || C < 0 || N < 0 || P < 0 || (idx_bits != 32 && idx_bits != 64))
        return hipErrorInvalidValue;
    if (B == 0 || C == 0 || P == 0) return hipSuccess;
    dim3 grid;
    if (N == 0 || !group_grid(B, C, P, grid)) return hipErrorInvalidValue;
    if (idx_bits == 32)
        hipLaunchKernelGGL(group_points_kernel<int32_t>, grid, dim3(kGroupThreads), 0, stream,
                           features, static_cast<const int32_t*>(idx), out, C, N, P);
    else
        hipLaunchKernelGGL(group_points_kernel<int64_t>, grid, dim3(kGroupThreads), 0, stream,
                           features, static_cast<const int64_t*>(idx), out, C, N, P);
    return hipGetLastError();
}

size_t pointops_group_points_backward_workspace_bytes(int64_t B, int64_t C, int64_t N, int64_t P) {
    if (B <= 0 || C <= 0 || N <= 0 || P <= 0) return 0;
    return group_inverse_bytes(B, C, N, P, nullptr, nullptr);
}

hipError_t pointops_group_points_backward(const float* grad_out, int64_t grad_batch_stride,
                                          const void* idx, int idx_bits, float* grad_features,
                                          void* workspace, int64_t B, int64_t C, int64_t N,
                                          int64_t P, hipStream_t stream) {
    if (B < 0 || C < 0 || N < 0 || P < 0 || (idx_bits != 32 && idx_bits != 64) ||
        grad_batch_stride < C * P)
        return hipErrorInvalidValue;
    if (B == 0 || C == 0 || N == 0) return hipSuccess;
    dim3 pgrid, ngrid;
    if (P >= INT32_MAX || N >= INT32_MAX || workspace == nullptr || !group_grid(B, 1, P, pgrid) ||
        !group_grid(B, 1, N, ngrid) || N * ((C + kWave - 1) / kWave) / (kGroupThreads / kWave) >= INT32_MAX)
        return hipErrorInvalidValue;
    GroupInverse V;
    group_inverse_bytes(B, C, N, P, &V, static_cast<char*>(workspace));
    const int64_t zn = B * (N + 1);
    const int64_t zblocks = std::min<int64_t>((zn + kGroupThreads - 1) / kGroupThreads, 1 << 16);
    hipLaunchKernelGGL(group_zero_kernel, dim3(static_cast<uint32_t>(zblocks)), dim3(kGroupThreads),
                       0, stream, V.off, zn);
    if (P > 0) {
        if (idx_bits == 32)
            hipLaunchKernelGGL(group_count_kernel<int32_t>, pgrid, dim3(kGroupThreads), 0, stream,
                               static_cast<const int32_t*>(idx), V, N, P);
        else
            hipLaunchKernelGGL(group_count_kernel<int64_t>, pgrid, dim3(kGroupThreads), 0, stream,
                               static_cast<const int64_t*>(idx), V, N, P);
    }
    hipLaunchKernelGGL(group_scan_kernel, dim3(static_cast<uint32_t>(B)), dim3(kGroupScanThreads), 0,
                       stream, V, N);
    if (P > 0) {
        if (idx_bits == 32)
            hipLaunchKernelGGL(group_place_kernel<int32_t>, pgrid, dim3(kGroupThreads), 0, stream,
                               static_cast<const int32_t*>(idx), V, N, P);
        else
            hipLaunchKernelGGL(group_place_kernel<int64_t>, pgrid, dim3(kGroupThreads), 0, stream,
                               static_cast<const int64_t*>(idx), V, N, P);
    }
    const int64_t chunks = (C + kWave - 1) / kWave;
    const int64_t gblocks = (N * chunks + kGroupThreads / kWave - 1) / (kGroupThreads / kWave);
    if (P > 0) {
        const dim3 tgrid(static_cast<uint32_t>((P + kGroupTile - 1) / kGroupTile),
                         static_cast<uint32_t>((C + kGroupTile - 1) / kGroupTile),
                         static_cast<uint32_t>(B));
        hipLaunchKernelGGL(group_transpose_kernel, tgrid, dim3(kGroupThreads), 0, stream, grad_out,
                           grad_batch_stride, V.gt, C, P);
    }
    hipLaunchKernelGGL(group_gather_grad_kernel, dim3(static_cast<uint32_t>(gblocks), ngrid.y),
                       dim3(kGroupThreads), 0, stream, V, grad_features, C, N, P, chunks);
    return hipGetLastError();
}

hipError_t pointops_group_points_rel(const float* xyz, const float* centres, const float* features,
                                     const void* idx, int idx_bits, float* out, int64_t B,
                                     int64_t C, int64_t N, int64_t M, int64_t S,
                                     hipStream_t stream) {
    if (B < 0 || C < 0 || N < 0 || M < 0 || S < 0 || (idx_bits != 32 && idx_bits != 64) ||
        (C > 0 && features == nullptr))
        return hipErrorInvalidValue;
    if (B == 0 || M == 0 || S == 0) return hipSuccess;
    dim3 grid;
    if (N == 0 || M > INT64_MAX / S || !group_grid(B, C + 3, M * S, grid))
        return hipErrorInvalidValue;
    if (idx_bits == 32)
        hipLaunchKernelGGL(group_points_rel_kernel<int32_t>, grid, dim3(kGroupThreads), 0, stream,
                           xyz, centres, features, static_cast<const int32_t*>(idx), out, C, N, M, S);
    else
        hipLaunchKernelGGL(group_points_rel_kernel<int64_t>, grid, dim3(kGroupThreads), 0, stream,
                           xyz, centres, features, static_cast<const int64_t*>(idx), out, C, N, M, S);
    return hipGetLastError();
}

}  // extern "C"
