// Chamfer nearest-neighbour search (K = 1) and its backward for gfx950.
//
// Forward: one lane per query row; the batch's reference points are staged
// through LDS in tiles and read with broadcasts, visited in index order.  The
// first reference is taken unconditionally (so an overflowed inf distance
// still yields a valid index) and later ones only with a strict `<`, which is
// the first-minimum rule of chamfer.py:161-212 and
// kernels/chamfer_nn.metal:13-226.  Distances: 3-D squared L2
// ((dx*dx) + dy*dy) + dz*dz with d = query - ref, L1 (|dx| + |dy|) + |dz|, and
// for D != 3 sequential accumulation over dimensions.  Rows at or beyond
// query_lengths[b], and all rows when the reference cloud is empty, are
// (0, -1).
//
// Backward (chamfer.py:227-294): gq = (q - ref[idx]) * (2 g) for squared L2,
// gq = (q > ref[idx] ? 1 : -1) * g for L1; grad_ref[idx] -= gq with hardware
// float atomics.
#include <type_traits>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kChThreads = 256;
constexpr int kChTile = 1024;

template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
    using type = float4;
    __device__ static float4 make(float x, float y, float z) { return make_float4(x, y, z, 0.f); }
};
template <>
struct Vec4<double> {
    using type = double4;
    __device__ static double4 make(double x, double y, double z) {
        return make_double4(x, y, z, 0.0);
    }
};

template <typename T, int NORM>
__device__ __forceinline__ T dist3(T qx, T qy, T qz, T rx, T ry, T rz) {
    const T dx = qx - rx;
    const T dy = qy - ry;
    const T dz = qz - rz;
    T d;
    if (NORM == 1) {
        d = fabs(dx);
        d = d + fabs(dy);
        d = d + fabs(dz);
    } else {
        d = dx * dx;
        d = d + dy * dy;
        d = d + dz * dz;
    }
    return d;
}

template <typename T, int NORM>
__global__ __launch_bounds__(kChThreads) void chamfer3_kernel(
    const T* __restrict__ query, const T* __restrict__ ref, const int64_t* __restrict__ qlen,
    const int64_t* __restrict__ rlen, T* __restrict__ out_dist, int64_t* __restrict__ out_idx,
    int64_t Q, int64_t R) {
    using V = typename Vec4<T>::type;
    __shared__ V tile[kChTile];
    const int64_t b = blockIdx.y;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kChThreads;
    const int64_t qi = first + threadIdx.x;
    const int64_t nq = qlen[b];
    const int64_t nr = rlen[b];
    const bool active = qi < Q && qi < nq && nr > 0;
    T qx = 0, qy = 0, qz = 0;
    if (active) {
        const T* qp = query + 3 * (b * Q + qi);
        qx = qp[0];
        qy = qp[1];
        qz = qp[2];
    }
    T best = 0;
    int bi = -1;
    // The whole block is padding or the reference cloud is empty: no scan.
    if (first < nq && nr > 0) {
        const T* rp = ref + 3 * b * R;
        for (int64_t t0 = 0; t0 < nr; t0 += kChTile) {
            const int tn = static_cast<int>(min<int64_t>(kChTile, nr - t0));
            __syncthreads();
            for (int t = threadIdx.x; t < tn; t += kChThreads) {
                const T* s = rp + 3 * (t0 + t);
                tile[t] = Vec4<T>::make(s[0], s[1], s[2]);
            }
            __syncthreads();
            int t = 0;
            if (t0 == 0) {
                const V c = tile[0];
                best = dist3<T, NORM>(qx, qy, qz, c.x, c.y, c.z);
                bi = 0;
                t = 1;
            }
            for (; t < tn; ++t) {
                const V c = tile[t];
                const T d = dist3<T, NORM>(qx, qy, qz, c.x, c.y, c.z);
                if (d < best) {
                    best = d;
                    bi = static_cast<int>(t0) + t;
                }
            }
        }
    }
    if (qi < Q) {
        const int64_t o = b * Q + qi;
        out_dist[o] = active ? best : T(0);
        out_idx[o] = active ? int64_t(bi) : int64_t(-1);
    }
}

// Generic D: sequential accumulation in increasing dimension order.
// Float 3-D variant: lane = query, the references come through uniform
// (scalar) loads in batches of 8 (no LDS tile, no barriers); same visiting
// order and first-minimum rule as chamfer3_kernel.
template <int NORM>
__global__ __launch_bounds__(kChThreads) void chamfer3_lane_kernel(
    const float* __restrict__ query, const float* __restrict__ ref,
    const int64_t* __restrict__ qlen, const int64_t* __restrict__ rlen,
    float* __restrict__ out_dist, int64_t* __restrict__ out_idx, int64_t Q, int64_t R) {
    constexpr int kBatch = 8;
    const int64_t b = blockIdx.y;
    const int64_t qi = static_cast<int64_t>(blockIdx.x) * kChThreads + threadIdx.x;
    const int64_t nq = qlen[b];
    const int64_t nr = rlen[b];
    const bool active = qi < Q && qi < nq && nr > 0;
    float qx = 0.f, qy = 0.f, qz = 0.f;
    if (active) {
        const float* qp = query + 3 * (b * Q + qi);
        qx = qp[0];
        qy = qp[1];
        qz = qp[2];
    }
    float best = 0.f;
    int bi = -1;
    if (ballot(active) != 0) {  // uniform: a wave of padding rows skips the scan
        const float* rp = ref + 3 * b * R;
        const int n = static_cast<int>(nr);
        best = dist3<float, NORM>(qx, qy, qz, rp[0], rp[1], rp[2]);  // first is always taken
        bi = 0;
        int j = 1;
        for (; j + kBatch <= n; j += kBatch) {
            float c[3 * kBatch];
            const float* r = rp + 3 * static_cast<int64_t>(j);
#pragma unroll
            for (int t = 0; t < 3 * kBatch; ++t) c[t] = r[t];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const float d = dist3<float, NORM>(qx, qy, qz, c[3 * u], c[3 * u + 1], c[3 * u + 2]);
                if (d < best) {
                    best = d;
                    bi = j + u;
                }
            }
        }
        for (; j < n; ++j) {
            const float* r = rp + 3 * static_cast<int64_t>(j);
            const float d = dist3<float, NORM>(qx, qy, qz, r[0], r[1], r[2]);
            if (d < best) {
                best = d;
                bi = j;
            }
        }
    }
    if (qi < Q) {
        const int64_t o = b * Q + qi;
        out_dist[o] = active ? best : 0.f;
        out_idx[o] = active ? int64_t(bi) : int64_t(-1);
    }
}

template <typename T, int NORM>
__global__ __launch_bounds__(kChThreads) void chamfer_nd_kernel(
    const T* __restrict__ query, const T* __restrict__ ref, const int64_t* __restrict__ qlen,
    const int64_t* __restrict__ rlen, T* __restrict__ out_dist, int64_t* __restrict__ out_idx,
    int64_t Q, int64_t R, int64_t D) {
    const int64_t b = blockIdx.y;
    const int64_t qi = static_cast<int64_t>(blockIdx.x) * kChThreads + threadIdx.x;
    if (qi >= Q) return;
    const int64_t o = b * Q + qi;
    const int64_t nr = rlen[b];
    if (qi >= qlen[b] || nr <= 0) {
        out_dist[o] = 0;
        out_idx[o] = -1;
        return;
    }
    const T* qp = query + o * D;
    const T* rp = ref + b * R * D;
    T best = 0;
    int64_t bi = -1;
    for (int64_t j = 0; j < nr; ++j) {
        const T* x = rp + j * D;
        const T f = qp[0] - x[0];
        T d = NORM == 1 ? fabs(f) : f * f;
        for (int64_t t = 1; t < D; ++t) {
            const T e = qp[t] - x[t];
            const T term = NORM == 1 ? fabs(e) : e * e;
            d = d + term;
        }
        if (bi < 0 || d < best) {
            best = d;
            bi = j;
        }
    }
    out_dist[o] = best;
    out_idx[o] = bi;
}

template <typename T, int NORM>
__global__ __launch_bounds__(kChThreads) void chamfer_backward_kernel(
    const T* __restrict__ query, const T* __restrict__ ref, const int64_t* __restrict__ idx,
    const T* __restrict__ grad, T* __restrict__ grad_query, T* __restrict__ grad_ref, int64_t Q,
    int64_t R, int64_t D, int64_t rows) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kChThreads + threadIdx.x;
    if (row >= rows) return;
    const int64_t i = idx[row];
    T* gq = grad_query + row * D;
    if (i < 0) {
        for (int64_t t = 0; t < D; ++t) gq[t] = T(0);
        return;
    }
    const int64_t b = row / Q;
    const T g = grad[row];
    const T scale = NORM == 1 ? g : T(2) * g;
    const T* qp = query + row * D;
    const T* rp = ref + (b * R + i) * D;
    T* gr = grad_ref + (b * R + i) * D;
    for (int64_t t = 0; t < D; ++t) {
        const T qv = qp[t], rv = rp[t];
        T v;
        if (NORM == 1) v = (qv > rv ? T(1) : T(-1)) * scale;
        else v = (qv - rv) * scale;
        gq[t] = v;
        unsafeAtomicAdd(gr + t, -v);
    }
}

template <typename T>
hipError_t launch_nearest(const T* q, const T* r, const int64_t* ql, const int64_t* rl, T* dist,
                          int64_t* idx, int64_t B, int64_t Q, int64_t R, int64_t D, int norm,
                          hipStream_t stream) {
    if (B < 0 || Q < 0 || R < 0 || D < 1 || (norm != 1 && norm != 2)) return hipErrorInvalidValue;
    if (B == 0 || Q == 0) return hipSuccess;
    if (B > 65535 || R > INT32_MAX || (Q + kChThreads - 1) / kChThreads > INT32_MAX)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<uint32_t>((Q + kChThreads - 1) / kChThreads),
                    static_cast<uint32_t>(B));
    const dim3 block(kChThreads);
    if (D == 3 && std::is_same<T, float>::value) {
        const float* qf = reinterpret_cast<const float*>(q);
        const float* rf = reinterpret_cast<const float*>(r);
        float* df = reinterpret_cast<float*>(dist);
        if (norm == 2)
            hipLaunchKernelGGL((chamfer3_lane_kernel<2>), grid, block, 0, stream, qf, rf, ql, rl, df,
                               idx, Q, R);
        else
            hipLaunchKernelGGL((chamfer3_lane_kernel<1>), grid, block, 0, stream, qf, rf, ql, rl, df,
                               idx, Q, R);
    } else if (D == 3) {
        if (norm == 2)
            hipLaunchKernelGGL((chamfer3_kernel<T, 2>), grid, block, 0, stream, q, r, ql, rl, dist, idx,
                               Q, R);
        else
            hipLaunchKernelGGL((chamfer3_kernel<T, 1>), grid, block, 0, stream, q, r, ql, rl, dist, idx,
                               Q, R);
    } else {
        if (norm == 2)
            hipLaunchKernelGGL((chamfer_nd_kernel<T, 2>), grid, block, 0, stream, q, r, ql, rl, dist,
                               idx, Q, R, D);
        else
            hipLaunchKernelGGL((chamfer_nd_kernel<T, 1>), grid, block, 0, stream, q, r, ql, rl, dist,
                               idx, Q, R, D);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t launch_backward(const T* q, const T* r, const int64_t* idx, const T* g, T* gq, T* gr,
                           int64_t B, int64_t Q, int64_t R, int64_t D, int norm,
                           hipStream_t stream) {
    if (B < 0 || Q < 0 || R < 0 || D < 1 || (norm != 1 && norm != 2)) return hipErrorInvalidValue;
    const int64_t rows = B * Q;
    if (rows == 0) return hipSuccess;
    const int64_t blocks = (rows + kChThreads - 1) / kChThreads;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    if (norm == 2)
        hipLaunchKernelGGL((chamfer_backward_kernel<T, 2>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kChThreads), 0, stream, q, r, idx, g, gq, gr, Q, R, D, rows);
    else
        hipLaunchKernelGGL((chamfer_backward_kernel<T, 1>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kChThreads), 0, stream, q, r, idx, g, gq, gr, Q, R, D, rows);
    return hipGetLastError();
}

}  // namespace
}  // namespace pointops

using namespace pointops;

extern "C" {

hipError_t pointops_chamfer_nearest_f32(const float* query, const float* ref,
                                        const int64_t* query_lengths, const int64_t* ref_lengths,
                                        float* dist, int64_t* idx, int64_t B, int64_t Q, int64_t R,
                                        int64_t D, int32_t norm, hipStream_t stream) {
    return launch_nearest<float>(query, ref, query_lengths, ref_lengths, dist, idx, B, Q, R, D, norm,
                                 stream);
}

hipError_t pointops_chamfer_nearest_f64(const double* query, const double* ref,
                                        const int64_t* query_lengths, const int64_t* ref_lengths,
                                        double* dist, int64_t* idx, int64_t B, int64_t Q, int64_t R,
                                        int64_t D, int32_t norm, hipStream_t stream) {
    return launch_nearest<double>(query, ref, query_lengths, ref_lengths, dist, idx, B, Q, R, D,
                                  norm, stream);
}

hipError_t pointops_chamfer_backward_f32(const float* query, const float* ref, const int64_t* idx,
                                         const float* grad_dist, float* grad_query,
                                         float* grad_ref, int64_t B, int64_t Q, int64_t R,
                                         int64_t D, int32_t norm, hipStream_t stream) {
    return launch_backward<float>(query, ref, idx, grad_dist, grad_query, grad_ref, B, Q, R, D, norm,
                                  stream);
}

hipError_t pointops_chamfer_backward_f64(const double* query, const double* ref,
                                         const int64_t* idx, const double* grad_dist,
                                         double* grad_query, double* grad_ref, int64_t B,
                                         int64_t Q, int64_t R, int64_t D, int32_t norm,
                                         hipStream_t stream) {
    return launch_backward<double>(query, ref, idx, grad_dist, grad_query, grad_ref, B, Q, R, D,
                                   norm, stream);
}

}  // extern "C"
