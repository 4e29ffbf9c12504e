// PointNet++ feature propagation for gfx950: three_nn and three_interpolate.
//
// three_nn: one lane per unknown point, the batch's known points staged
// through LDS in tiles (one float4 per point, broadcast reads).  The three
// best keys are kept in registers; a key is the squared distance's bit
// pattern (non-negative floats order like unsigned integers) with NaN mapped
// above +inf, and known points are visited in index order with a strict `<`,
// which reproduces the stable argsort of pointnet2.py:54-72 (NaN last, ties by
// index) and the strict cascade of kernels/pointnet2.metal:24-43.
//
// three_interpolate: out[b,c,n] = (f[i0]*w0 + f[i1]*w1) + f[i2]*w2
// (kernels/pointnet2.metal:52-71); one lane per (b, n) over a few channels so
// that the index/weight triplet is read once per channel group.  The backward
// adds g*w_t into grad_features with hardware float atomics.
#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kTnThreads = 256;
constexpr int kTnTile = 1024;  // known points per LDS tile (16 KiB)

__device__ __forceinline__ uint32_t sort_key(float d) {
    return (d != d) ? 0x7FC00000u : static_cast<uint32_t>(f2i(d));
}

__global__ __launch_bounds__(kTnThreads) void three_nn_kernel(const float* __restrict__ unknown,
                                                              const float* __restrict__ known,
                                                              float* __restrict__ dist,
                                                              int32_t* __restrict__ idx, int64_t N,
                                                              int64_t M) {
    __shared__ float4 tile[kTnTile];
    const int64_t b = blockIdx.y;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kTnThreads + threadIdx.x;
    const bool active = n < N;
    const float* up = unknown + 3 * (b * N + (active ? n : 0));
    const float ux = up[0], uy = up[1], uz = up[2];
    const float* kp = known + 3 * b * M;
    uint32_t k0 = 0xFFFFFFFFu, k1 = 0xFFFFFFFFu, k2 = 0xFFFFFFFFu;
    int i0 = -1, i1 = -1, i2 = -1;
    for (int64_t t0 = 0; t0 < M; t0 += kTnTile) {
        const int tn = static_cast<int>(min<int64_t>(kTnTile, M - t0));
        __syncthreads();
        for (int t = threadIdx.x; t < tn; t += kTnThreads) {
            const float* s = kp + 3 * (t0 + t);
            tile[t] = make_float4(s[0], s[1], s[2], 0.f);
        }
        __syncthreads();
        for (int t = 0; t < tn; ++t) {
            const float4 c = tile[t];
            const uint32_t k = sort_key(sqdist3(ux, uy, uz, c.x, c.y, c.z));
            const bool take = active && k < k2;
            if (ballot(take) == 0) continue;
            if (take) {
                const int j = static_cast<int>(t0) + t;
                if (k < k0) {
                    k2 = k1; i2 = i1;
                    k1 = k0; i1 = i0;
                    k0 = k;  i0 = j;
                } else if (k < k1) {
                    k2 = k1; i2 = i1;
                    k1 = k;  i1 = j;
                } else {
                    k2 = k;  i2 = j;
                }
            }
        }
    }
    if (active) {
        const int64_t o = 3 * (b * N + n);
        dist[o] = sqrtf(i2f(static_cast<int>(k0)));
        dist[o + 1] = sqrtf(i2f(static_cast<int>(k1)));
        dist[o + 2] = sqrtf(i2f(static_cast<int>(k2)));
        idx[o] = i0;
        idx[o + 1] = i1;
        idx[o + 2] = i2;
    }
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
    if (B < 0 || N < 0 || M < 0 || M > INT32_MAX) return hipErrorInvalidValue;
    if (B == 0 || N == 0) return hipSuccess;
    if (M < 3 || B > 65535 || (N + kTnThreads - 1) / kTnThreads > INT32_MAX)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<uint32_t>((N + kTnThreads - 1) / kTnThreads),
                    static_cast<uint32_t>(B));
    hipLaunchKernelGGL(three_nn_kernel, grid, dim3(kTnThreads), 0, stream, unknown, known, dist, idx,
                       N, M);
    return hipGetLastError();
}

hipError_t pointops_three_interpolate(const float* features, const int32_t* idx,
                                      const float* weights, float* out, int64_t B, int64_t C,
                                      int64_t M, int64_t N, hipStream_t stream) {
    if (B < 0 || C < 0 || M < 0 || N < 0) return hipErrorInvalidValue;
    if (B == 0 || C == 0 || N == 0) return hipSuccess;
    if (M == 0 || !grid_fits(B, C, N)) return hipErrorInvalidValue;
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
    const dim3 grid(static_cast<uint32_t>((N + kTiThreads - 1) / kTiThreads),
                    static_cast<uint32_t>((C + kTiChannels - 1) / kTiChannels),
                    static_cast<uint32_t>(B));
    hipLaunchKernelGGL(three_interpolate_backward_kernel, grid, dim3(kTiThreads), 0, stream, grad_out,
                       idx, weights, grad_features, C, M, N);
    return hipGetLastError();
}

}  // extern "C"
