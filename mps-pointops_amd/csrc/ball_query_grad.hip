// Backward of the dense first-K ball query for gfx950: the gradients of the
// squared distances d2[b, q, k] = |queries[b, q] - points[b, idx[b, q, k]]|^2
// with respect to both coordinate tensors (_ball_query_mps.py:168-203).
//
// Every valid slot (idx >= 0) contributes c = fl(2 g) * fl(q - p) per axis,
// g being the incoming gradient of that slot; padded slots contribute
// nothing (the reference masks them before multiplying, so NaN gradients in
// padded slots never reach the sums).  grad_queries[b, q] is the sum of the
// row's contributions (four strided partial sums, added in order);
// grad_points[b, j] is minus the sum of the contributions of the slots that
// hold j.  Both sums are taken in a fixed
// order, so the gradients are the same bits on every run (the reference's
// scatter_add accumulates with atomics in whatever order they land).
//
// Two launches:
//   ball_grad_rows_kernel: a quad of lanes per query row; lane l sums the
//     slots k = l (mod 4) in order, the quad adds its four sums in lane order;
//     writes the query gradient and the row's smallest and largest valid index.
//   ball_grad_points_kernel: one workgroup per (cloud, tile of kGradTile
//     points).  Wave w owns the w-th of kGradWaves contiguous segments of
//     rows and adds the contributions of its rows, in row order, into its own
//     LDS accumulators (a point occurs at most once per row, so the lanes of
//     one row never collide); the segments' sums are then added in segment
//     order.  In clouds of more than kGradDenseTiles tiles a row whose
//     index range misses the tile is skipped after its 8-byte range record,
//     so large clouds do not re-read every row per tile, and each wave loads
//     kGradBatch (row, 64-slot chunk) units before it adds the first; in
//     smaller clouds (where first-K hits span the whole index range) every
//     row is read and the next batch's loads are in flight while a batch is
//     added.
// Inputs are float32 or float16 coordinates (widened to float32, as the
// reference's .float()); gradients are float32.
#include <hip/hip_fp16.h>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kGradRowThreads = 256;
constexpr int kGradQuad = 4;     // lanes per query row
constexpr int kGradSlotBatch = 8;  // slots per lane loaded before the first is added
constexpr int kGradBatch = 8;    // (row, chunk) units per wave loaded before the first is added
constexpr int kGradWaves = 8;
constexpr int kGradThreads = kGradWaves * kWave;
constexpr int kGradTile = 512;  // points per workgroup: 48 KiB of accumulators
constexpr int kGradDenseTiles = 16;  // tiles per cloud up to which every tile reads every row

template <typename S>
__device__ __forceinline__ float widen(S v);
template <>
__device__ __forceinline__ float widen<float>(float v) { return v; }
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t v) {
    return __half2float(__ushort_as_half(v));
}

template <typename S>
__global__ __launch_bounds__(kGradRowThreads) void ball_grad_rows_kernel(
    const S* __restrict__ queries, const S* __restrict__ points, const int64_t* __restrict__ idx,
    const float* __restrict__ grad, float* __restrict__ grad_queries, int2* __restrict__ range,
    int64_t B, int64_t Q, int64_t P, int64_t K) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGradRowThreads + threadIdx.x;
    const int l = threadIdx.x % kGradQuad;
    // Rows past the end compute nothing but still take part in the quad sums.
    const int64_t row = min(gid / kGradQuad, B * Q - 1);
    const bool live = gid / kGradQuad < B * Q;
    const int64_t b = row / Q;
    const float qx = widen(queries[3 * row]), qy = widen(queries[3 * row + 1]),
                qz = widen(queries[3 * row + 2]);
    const int64_t* ri = idx + row * K;
    const float* rg = grad + row * K;
    const S* pb = points + 3 * b * P;
    float ax = 0.f, ay = 0.f, az = 0.f;
    int lo = INT_MAX, hi = -1;
    for (int64_t k0 = l; k0 < (live ? K : 0); k0 += kGradQuad * kGradSlotBatch) {
        int64_t j[kGradSlotBatch];
        float g2[kGradSlotBatch], px[kGradSlotBatch], py[kGradSlotBatch], pz[kGradSlotBatch];
#pragma unroll
        for (int u = 0; u < kGradSlotBatch; ++u) {
            const int64_t k = k0 + u * kGradQuad;
            j[u] = k < K ? ri[k] : -1;
            g2[u] = k < K ? rg[k] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kGradSlotBatch; ++u) {
            px[u] = py[u] = pz[u] = 0.f;
            if (j[u] >= 0 && j[u] < P) {  // else padding: no load
                const S* p = pb + 3 * j[u];
                px[u] = widen(p[0]);
                py[u] = widen(p[1]);
                pz[u] = widen(p[2]);
            }
        }
#pragma unroll
        for (int u = 0; u < kGradSlotBatch; ++u) {
            if (!(j[u] >= 0 && j[u] < P)) continue;
            const float g = 2.f * g2[u];
            ax = ax + g * (qx - px[u]);
            ay = ay + g * (qy - py[u]);
            az = az + g * (qz - pz[u]);
            lo = min(lo, static_cast<int>(j[u]));
            hi = max(hi, static_cast<int>(j[u]));
        }
    }
    // Quad sums in lane order: ((s0 + s1) + s2) + s3.
    const int base = (threadIdx.x % kWave) & ~(kGradQuad - 1);
    float sx = __shfl(ax, base, kWave), sy = __shfl(ay, base, kWave), sz = __shfl(az, base, kWave);
    int slo = __shfl(lo, base, kWave), shi = __shfl(hi, base, kWave);
#pragma unroll
    for (int t = 1; t < kGradQuad; ++t) {
        sx = sx + __shfl(ax, base + t, kWave);
        sy = sy + __shfl(ay, base + t, kWave);
        sz = sz + __shfl(az, base + t, kWave);
        slo = min(slo, __shfl(lo, base + t, kWave));
        shi = max(shi, __shfl(hi, base + t, kWave));
    }
    if (!live || l != 0) return;
    if (grad_queries != nullptr) {
        grad_queries[3 * row] = sx;
        grad_queries[3 * row + 1] = sy;
        grad_queries[3 * row + 2] = sz;
    }
    range[row] = make_int2(slo, shi);
}

template <typename S, bool DENSE>
__global__ __launch_bounds__(kGradThreads) void ball_grad_points_kernel(
    const S* __restrict__ queries, const S* __restrict__ points, const int64_t* __restrict__ idx,
    const float* __restrict__ grad, const int2* __restrict__ range, float* __restrict__ grad_points,
    int64_t Q, int64_t P, int64_t K, uint32_t tiles) {
    __shared__ float acc[kGradWaves][3][kGradTile];
    __shared__ float tile[3][kGradTile];
    const CloudBlock cb = cloud_block(tiles);
    const int64_t b = cb.b;
    const int64_t lo = static_cast<int64_t>(cb.x) * kGradTile;
    const int n = static_cast<int>(min<int64_t>(kGradTile, P - lo));
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const S* pb = points + 3 * b * P;
    for (int t = tid; t < kGradTile; t += kGradThreads) {
#pragma unroll
        for (int w = 0; w < kGradWaves; ++w) acc[w][0][t] = acc[w][1][t] = acc[w][2][t] = 0.f;
        const int64_t j = lo + min(t, n - 1);
#pragma unroll
        for (int c = 0; c < 3; ++c) tile[c][t] = widen(pb[3 * j + c]);
    }
    __syncthreads();
    const int64_t r0 = Q * wave / kGradWaves, r1 = Q * (wave + 1) / kGradWaves;
    const int tlo = static_cast<int>(lo), thi = static_cast<int>(lo) + n;  // [tlo, thi)
    // At least one chunk per row, so the unit walk advances (for K = 0 every
    // slot is masked).
    const int64_t chunks = K > kWave ? (K + kWave - 1) / kWave : 1;
    if constexpr (DENSE) {
        // Few tiles per cloud: every row is read by every tile anyway, so the
        // range records are not consulted.  Units (row q, slots [c * 64,
        // c * 64 + 64)) in row order, kGradBatch at a time; the next batch's
        // loads (from clamped addresses, masked at use) are in flight while
        // this batch is added.
        int64_t q = r0, c = 0;
        struct Batch {
            int64_t j[kGradBatch];
            float g[kGradBatch], x[kGradBatch], y[kGradBatch], z[kGradBatch];
            uint32_t live;  // bit d: unit d holds a slot of this lane
        };
        auto load = [&](Batch& t) {
            t.live = 0;
#pragma unroll
            for (int d = 0; d < kGradBatch; ++d) {
                const int64_t row = b * Q + min(q, r1 - 1);
                const int64_t k = c * kWave + lane;
                if (q < r1 && k < K) t.live |= 1u << d;
                const int64_t slot = row * K + min<int64_t>(k, K - 1);
                t.j[d] = idx[slot];
                t.g[d] = grad[slot];
                t.x[d] = widen(queries[3 * row]);
                t.y[d] = widen(queries[3 * row + 1]);
                t.z[d] = widen(queries[3 * row + 2]);
                if (q < r1 && ++c == chunks) {
                    c = 0;
                    ++q;
                }
            }
        };
        const int64_t batches = ((r1 - r0) * chunks + kGradBatch - 1) / kGradBatch;
        if (batches > 0 && K > 0) {
            Batch cur, nxt;
            load(cur);
            for (int64_t bt = 0; bt < batches; ++bt) {
                if (bt + 1 < batches) load(nxt);
#pragma unroll
                for (int d = 0; d < kGradBatch; ++d) {
                    const int64_t jd = (cur.live >> d) & 1u ? cur.j[d] : -1;
                    if (jd < tlo || jd >= thi) continue;
                    const int t = static_cast<int>(jd) - tlo;
                    const float g2 = 2.f * cur.g[d];
                    acc[wave][0][t] += g2 * (cur.x[d] - tile[0][t]);
                    acc[wave][1][t] += g2 * (cur.y[d] - tile[1][t]);
                    acc[wave][2][t] += g2 * (cur.z[d] - tile[2][t]);
                }
                cur = nxt;
            }
        }
    } else {
        // Units (row q, slots [c * 64, c * 64 + 64)) in row order; kGradBatch of
        // them are loaded, then added in order.
        int64_t q = r0, c = 0;
        while (q < r1) {
            int64_t rows[kGradBatch], ks[kGradBatch];
            bool use[kGradBatch];
            float ux[kGradBatch], uy[kGradBatch], uz[kGradBatch];
            // The units' range records and query rows (wave-uniform loads), all
            // requested before any is used; then the slots of the units in use.
    #pragma unroll
            for (int d = 0; d < kGradBatch; ++d) {
                use[d] = q < r1;
                rows[d] = b * Q + min(q, r1 - 1);
                ks[d] = c * kWave + lane;
                if (++c == chunks) {
                    c = 0;
                    ++q;
                }
            }
            int2 rr[kGradBatch];
    #pragma unroll
            for (int d = 0; d < kGradBatch; ++d) {
                rr[d] = range[rows[d]];
                ux[d] = widen(queries[3 * rows[d]]);
                uy[d] = widen(queries[3 * rows[d] + 1]);
                uz[d] = widen(queries[3 * rows[d] + 2]);
            }
            int64_t jj[kGradBatch];
            float gg[kGradBatch];
    #pragma unroll
            for (int d = 0; d < kGradBatch; ++d) {
                // Some slot of the row in the tile (wave-uniform), and a slot for this lane.
                const bool live = use[d] && !(rr[d].y < tlo || rr[d].x >= thi) && ks[d] < K;
                jj[d] = live ? idx[rows[d] * K + ks[d]] : -1;
                gg[d] = live ? grad[rows[d] * K + ks[d]] : 0.f;
            }
    #pragma unroll
            for (int d = 0; d < kGradBatch; ++d) {
                if (jj[d] < tlo || jj[d] >= thi) continue;
                const int t = static_cast<int>(jj[d]) - tlo;
                const float g2 = 2.f * gg[d];
                acc[wave][0][t] += g2 * (ux[d] - tile[0][t]);
                acc[wave][1][t] += g2 * (uy[d] - tile[1][t]);
                acc[wave][2][t] += g2 * (uz[d] - tile[2][t]);
            }
        }
    }
    __syncthreads();
    for (int t = tid; t < n; t += kGradThreads) {
        float* out = grad_points + 3 * (b * P + lo + t);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float s = acc[0][c][t];
#pragma unroll
            for (int w = 1; w < kGradWaves; ++w) s = s + acc[w][c][t];
            out[c] = -s;
        }
    }
}

template <typename S>
hipError_t launch_ball_grad(const S* queries, const S* points, const int64_t* idx,
                            const float* grad, float* grad_queries, float* grad_points,
                            void* workspace, int64_t B, int64_t Q, int64_t P, int64_t K,
                            hipStream_t stream) {
    if (B < 0 || Q < 0 || P < 0 || K < 0 || P >= INT32_MAX - kGradTile)
        return hipErrorInvalidValue;
    if (B == 0 || (grad_queries == nullptr && grad_points == nullptr)) return hipSuccess;
    const int64_t rows = B * Q;
    const int64_t tiles = (P + kGradTile - 1) / kGradTile;
    if ((rows * kGradQuad + kGradRowThreads - 1) / kGradRowThreads > INT32_MAX ||
        B * tiles > INT32_MAX)
        return hipErrorInvalidValue;
    if (rows > 0 && (queries == nullptr || workspace == nullptr ||
                     (K > 0 && (idx == nullptr || grad == nullptr)) ||
                     (P > 0 && points == nullptr)))
        return hipErrorInvalidValue;
    int2* range = static_cast<int2*>(workspace);
    if (rows > 0) {
        const int64_t threads = rows * kGradQuad;
        hipLaunchKernelGGL(ball_grad_rows_kernel<S>,
                           dim3(static_cast<uint32_t>((threads + kGradRowThreads - 1) / kGradRowThreads)),
                           dim3(kGradRowThreads), 0, stream, queries, points, idx, grad,
                           grad_queries, range, B, Q, P, K);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (grad_points == nullptr || tiles == 0) return hipSuccess;
    // Up to kGradDenseTiles tiles per cloud: every tile reads every row
    // (the dense loop, loads pipelined); beyond, rows missing a tile are
    // skipped after their range record.
    if (tiles <= kGradDenseTiles)
        hipLaunchKernelGGL((ball_grad_points_kernel<S, true>), dim3(static_cast<uint32_t>(B * tiles)),
                           dim3(kGradThreads), 0, stream, queries, points, idx, grad, range,
                           grad_points, Q, P, K, static_cast<uint32_t>(tiles));
    else
        hipLaunchKernelGGL((ball_grad_points_kernel<S, false>), dim3(static_cast<uint32_t>(B * tiles)),
                           dim3(kGradThreads), 0, stream, queries, points, idx, grad, range,
                           grad_points, Q, P, K, static_cast<uint32_t>(tiles));
    return hipGetLastError();
}

}  // namespace
}  // namespace pointops

using namespace pointops;

extern "C" {

size_t pointops_ball_query_backward_workspace_bytes(int64_t B, int64_t Q) {
    if (B <= 0 || Q <= 0) return 0;
    return static_cast<size_t>(B) * static_cast<size_t>(Q) * sizeof(int2);
}

hipError_t pointops_ball_query_backward_f32(const float* queries, const float* points,
                                            const int64_t* idx, const float* grad_dist2,
                                            float* grad_queries, float* grad_points,
                                            void* workspace, int64_t B, int64_t Q, int64_t P,
                                            int64_t K, hipStream_t stream) {
    return launch_ball_grad<float>(queries, points, idx, grad_dist2, grad_queries, grad_points,
                                   workspace, B, Q, P, K, stream);
}

hipError_t pointops_ball_query_backward_f16(const uint16_t* queries, const uint16_t* points,
                                            const int64_t* idx, const float* grad_dist2,
                                            float* grad_queries, float* grad_points,
                                            void* workspace, int64_t B, int64_t Q, int64_t P,
                                            int64_t K, hipStream_t stream) {
    return launch_ball_grad<uint16_t>(queries, points, idx, grad_dist2, grad_queries,
                                      grad_points, workspace, B, Q, P, K, stream);
}

}  // extern "C"
