// First-K radius search for gfx950.
//
// One wave per query scans the candidate points in input order, 64 per block
// (lane l <-> point base + l).  A hit is fl32((dx^2 + dy^2) + dz^2) < r2 with
// the reference's separately rounded arithmetic (reference.py:83-121); NaN and
// overflowed distances never satisfy `<`.  The hits of a block take output
// slots found + rank, where rank is the number of hit lanes below (ballot +
// mbcnt), which keeps the first K hits in index order without atomics; the
// scan stops as soon as K hits are found and the remaining slots are padded.
// Dense batches (B <= 65535) stage the points through LDS: a workgroup of
// 8 waves (8 consecutive queries of one cloud) loads each 2048-point tile
// once for all of them (ball_query_lds_kernel).
//
//   dense: _ball_query_mps.py:122-166 / kernels/ball_query.metal:30-166
//          (query/point lengths, (idx -1, dist2 0) padding, f32 or f16 input)
//   flat:  _flat_search_mps.py:111-147 / kernels/flat_search.metal:171-275
//          (segments by ptr, global indices, -1 padding, optional exclusion of
//          index == query index before the cap)
#include <hip/hip_fp16.h>

#include <type_traits>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr int kBqThreads = 256;
constexpr int kBqWaves = kBqThreads / kWave;
constexpr int kBqDepth = 8;  // 64-point blocks in flight per wave (even)
// LDS-staged dense kernel: queries (waves) per workgroup and 64-point blocks
// per LDS tile (measured best of 2-16 waves and 8-48 blocks per tile).
constexpr int kBqLdsQueries = 8;
constexpr uint64_t kBqAllDone = 0x0101010101010101ull;  // every wave's done byte set
static_assert(kBqLdsQueries == 8, "the done bytes of a workgroup fill one 64-bit word");
// Element `slot` of a wave's output row, addressed by a 32-bit byte offset
// from the row's (wave-uniform) base, so that the store needs no 64-bit
// address arithmetic per lane.
template <typename T>
__device__ __forceinline__ T& row_at(T* base, uint32_t slot) {
    return *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + slot * static_cast<uint32_t>(sizeof(T)));
}
constexpr int kBqLdsDepth = 32;

template <typename S>
__device__ __forceinline__ float widen(S v);
template <>
__device__ __forceinline__ float widen<float>(float v) { return v; }
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t v) {
    return __half2float(__ushort_as_half(v));
}

template <typename S>
__global__ __launch_bounds__(kBqThreads) void ball_query_kernel(
    const S* __restrict__ queries, const S* __restrict__ points,
    const int64_t* __restrict__ query_lengths, const int64_t* __restrict__ point_lengths,
    int64_t* __restrict__ out_idx, float* __restrict__ out_dist, int64_t B, int64_t Q, int64_t P,
    int K, float r2) {
    const int lane = lane_id();
    const uint32_t blk = xcd_local_block(blockIdx.x, gridDim.x);
    const int64_t row = static_cast<int64_t>(blk) * kBqWaves + uniform(threadIdx.x / kWave);
    if (row >= B * Q) return;
    const int64_t b = row / Q;
    const int64_t qi = row - b * Q;
    int64_t* oi = out_idx + row * K;
    float* od = out_dist + row * K;
    int found = 0;
    const int64_t qlen = query_lengths != nullptr ? query_lengths[b] : Q;
    if (qi < qlen) {
        const int64_t plen = point_lengths != nullptr ? point_lengths[b] : P;
        const int n = static_cast<int>(plen < P ? plen : P);
        const S* qp = queries + 3 * row;
        const float qx = widen(qp[0]), qy = widen(qp[1]), qz = widen(qp[2]);
        const S* pp = points + 3 * b * P;
        // kBqDepth blocks of 64 points are loaded before the first is tested,
        // so one L2 round trip covers kBqDepth * 64 points.
        for (int base = 0; base < n && found < K; base += kBqDepth * kWave) {
            float vx[kBqDepth], vy[kBqDepth], vz[kBqDepth];
            // Loads are clamped into the cloud (not skipped) so that all of
            // them are in flight at once; lanes past n are masked below.
#pragma unroll
            for (int c = 0; c < kBqDepth; ++c) {
                const int jj = min(base + c * kWave + lane, n - 1);
                const S* pt = pp + 3 * static_cast<int64_t>(jj);
                vx[c] = widen(pt[0]);
                vy[c] = widen(pt[1]);
                vz[c] = widen(pt[2]);
            }
#pragma unroll
            for (int c = 0; c < kBqDepth; c += 2) {
                // Two blocks per round: straight-line tests, one branch.
                const int j0 = base + c * kWave + lane, j1 = j0 + kWave;
                const float d0 = sqdist3(qx, qy, qz, vx[c], vy[c], vz[c]);
                const float d1 = sqdist3(qx, qy, qz, vx[c + 1], vy[c + 1], vz[c + 1]);
                const bool h0 = j0 < n && d0 < r2;
                const bool h1 = j1 < n && d1 < r2;
                const uint64_t m0 = ballot(h0), m1 = ballot(h1);
                if ((m0 | m1) == 0) continue;
                const int s0 = found + lanes_below(m0);
                const int s1 = found + __popcll(m0) + lanes_below(m1);
                if (h0 && s0 < K) {
                    oi[s0] = j0;
                    od[s0] = d0;
                }
                if (h1 && s1 < K) {
                    oi[s1] = j1;
                    od[s1] = d1;
                }
                found += __popcll(m0) + __popcll(m1);
                if (found >= K) break;
            }
        }
        found = min(found, K);
    }
    for (int s = found + lane; s < K; s += kWave) {
        oi[s] = -1;
        od[s] = 0.f;
    }
}

// The same search with the candidate points staged through LDS: a workgroup
// serves NWQ consecutive queries of one cloud (one wave each), its threads
// load each tile of kBqDepth * 64 points once, and every wave tests its query
// against the tile.  The workgroup stops after the tile in which its last
// query reached K hits, so a tile is read from L2 once per NWQ queries.
// With `skip` set, every workgroup returns at once when *skip != 0 (another
// search of the same call, chosen on the device, writes the outputs).
// PN2: the pointnet2_ops output instead -- int32 indices only, unused slots
// repeating the query's first hit (all 0 without one) -- so that the
// grouping step needs no padding or conversion kernels.
template <typename S, int NWQ, bool PN2>
__global__ __launch_bounds__(NWQ * kWave) void ball_query_lds_kernel(
    const S* __restrict__ queries, const S* __restrict__ points,
    const int64_t* __restrict__ query_lengths, const int64_t* __restrict__ point_lengths,
    void* __restrict__ out_idx, float* __restrict__ out_dist, int64_t Q, int64_t P, int K,
    float r2, const int* __restrict__ skip, int64_t QS) {
    if (skip != nullptr && *skip != 0) return;  // uniform, before any barrier
    constexpr int kTile = kBqLdsDepth * kWave;
    constexpr int kPer = kTile / (NWQ * kWave);  // points each thread stages per tile
    static_assert(kPer * NWQ * kWave == kTile && kBqLdsDepth % 2 == 0, "tile shape");
    __shared__ float4 tile[kTile];
    __shared__ __align__(8) uint8_t done_flags[NWQ];  // one byte per wave, read as one word
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = uniform(tid / kWave);
    const int64_t b = blockIdx.y;
    const int64_t qi = static_cast<int64_t>(blockIdx.x) * NWQ + wave;
    const int64_t qlen = query_lengths != nullptr ? query_lengths[b] : Q;
    const int64_t plen = point_lengths != nullptr ? point_lengths[b] : P;
    const int n = static_cast<int>(plen < P ? plen : P);
    const bool live = qi < Q && qi < qlen;
    const int64_t row = b * QS + (qi < Q ? qi : 0);  // QS: rows between clouds (>= Q)
    float qx = 0.f, qy = 0.f, qz = 0.f;
    if (live) {
        const S* qp = queries + 3 * row;
        qx = widen(qp[0]);
        qy = widen(qp[1]);
        qz = widen(qp[2]);
    }
    int64_t* oi = static_cast<int64_t*>(out_idx) + row * K;
    int32_t* oi32 = static_cast<int32_t*>(out_idx) + row * K;
    float* od = PN2 ? nullptr : out_dist + row * K;
    const S* pp = points + 3 * b * P;
    // Points of the tile at `base` for this thread (clamped into the cloud;
    // points past n are masked in the test).
    float4 pf[kPer];
    auto fetch = [&](int base) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const S* pt = pp + 3 * static_cast<int64_t>(min(base + k * NWQ * kWave + tid, n - 1));
            pf[k] = make_float4(widen(pt[0]), widen(pt[1]), widen(pt[2]), 0.f);
        }
    };
    int found = 0;
    int first = 0;  // PN2: the query's first hit
    // d < r2 is impossible for r2 <= 0 (d is never negative) or NaN r2.
    bool done = !live || !(r2 > 0.f);
    if (n > 0) fetch(0);
    for (int base = 0; base < n; base += kTile) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) tile[k * NWQ * kWave + tid] = pf[k];
        __syncthreads();
        if (base + kTile < n) fetch(base + kTile);  // in flight during the scan
        // A full tile needs no bounds test (one instantiation each).
        auto scan = [&](auto full) {
#pragma unroll
            for (int c = 0; c < kBqLdsDepth; c += 2) {
                const float4 p0 = tile[c * kWave + lane];
                const float4 p1 = tile[(c + 1) * kWave + lane];
                const float d0 = sqdist3(qx, qy, qz, p0.x, p0.y, p0.z);
                const float d1 = sqdist3(qx, qy, qz, p1.x, p1.y, p1.z);
                // A full tile needs the point indices only where a hit is stored.
                const bool h0 = (decltype(full)::value || base + c * kWave + lane < n) && d0 < r2;
                const bool h1 = (decltype(full)::value || base + (c + 1) * kWave + lane < n) && d1 < r2;
                const uint64_t m0 = ballot(h0), m1 = ballot(h1);
                if ((m0 | m1) == 0) continue;
                const int j0 = base + c * kWave + lane, j1 = j0 + kWave;
                // Slots and indices are non-negative: unsigned, so that the
                // 64-bit addresses and index values need no sign extension.
                const uint32_t s0 = static_cast<uint32_t>(found + lanes_below(m0));
                const uint32_t s1 = static_cast<uint32_t>(found + __popcll(m0) + lanes_below(m1));
                const uint32_t uk = static_cast<uint32_t>(K);
                if constexpr (PN2) {
                    if (found == 0)
                        first = m0 != 0 ? base + c * kWave + static_cast<int>(__builtin_ctzll(m0))
                                        : base + (c + 1) * kWave + static_cast<int>(__builtin_ctzll(m1));
                    if (h0 && s0 < uk) row_at(oi32, s0) = j0;
                    if (h1 && s1 < uk) row_at(oi32, s1) = j1;
                } else {
                    if (h0 && s0 < uk) {
                        row_at(oi, s0) = static_cast<int64_t>(static_cast<uint32_t>(j0));
                        row_at(od, s0) = d0;
                    }
                    if (h1 && s1 < uk) {
                        row_at(oi, s1) = static_cast<int64_t>(static_cast<uint32_t>(j1));
                        row_at(od, s1) = d1;
                    }
                }
                found += __popcll(m0) + __popcll(m1);
                if (found >= K) break;
            }
        };
        if (!done) {
            if (base + kTile <= n) scan(std::true_type{});
            else scan(std::false_type{});
            done = found >= K;
        }
        if (lane == 0) done_flags[wave] = done ? 1 : 0;
        __syncthreads();  // flags written; every wave is past its reads of this tile
        if (*reinterpret_cast<const uint64_t*>(done_flags) == kBqAllDone) break;
    }
    if (qi >= Q) return;
    found = min(found, K);
    for (int s = found + lane; s < K; s += kWave) {
        if constexpr (PN2) {
            oi32[s] = first;  // 0 when nothing was found
        } else {
            oi[s] = -1;
            od[s] = 0.f;
        }
    }
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

template <typename S>
__global__ __launch_bounds__(kBqThreads) void radius_flat_kernel(
    const S* __restrict__ y, const S* __restrict__ x, const int64_t* __restrict__ ptr_y,
    const int64_t* __restrict__ ptr_x, int64_t* __restrict__ out, int64_t Q, int64_t batch, int K,
    float r2, int ignore_same_index) {
    const int lane = lane_id();
    const int64_t q = static_cast<int64_t>(blockIdx.x) * kBqWaves + uniform(threadIdx.x / kWave);
    if (q >= Q) return;
    const int64_t b = segment_of(ptr_y, batch, q);
    const int64_t lo = ptr_x[b], hi = ptr_x[b + 1];
    int64_t* o = out + q * K;
    int found = 0;
    if (r2 > 0.f) {
        const float qx = widen(y[3 * q]), qy = widen(y[3 * q + 1]), qz = widen(y[3 * q + 2]);
        for (int64_t base = lo; base < hi && found < K; base += kBqDepth * kWave) {
            float vx[kBqDepth], vy[kBqDepth], vz[kBqDepth];
#pragma unroll
            for (int c = 0; c < kBqDepth; ++c) {
                const int64_t jj = min<int64_t>(base + c * kWave + lane, hi - 1);
                const S* pt = x + 3 * jj;
                vx[c] = widen(pt[0]);
                vy[c] = widen(pt[1]);
                vz[c] = widen(pt[2]);
            }
#pragma unroll
            for (int c = 0; c < kBqDepth; ++c) {
                const int64_t j = base + c * kWave + lane;
                bool hit = false;
                if (j < hi && !(ignore_same_index && j == q))
                    hit = sqdist3(vx[c], vy[c], vz[c], qx, qy, qz) < r2;
                const uint64_t mask = ballot(hit);
                if (mask == 0) continue;
                const int slot = found + lanes_below(mask);
                if (hit && slot < K) o[slot] = j;
                found += __popcll(mask);
                if (found >= K) break;
            }
        }
        found = min(found, K);
    }
    for (int s = found + lane; s < K; s += kWave) o[s] = -1;
}

// `skip` (device word, may be null) is honoured by the LDS-staged kernel
// only, so a call with `skip` must fit it (B <= 65535).
template <typename S>
hipError_t launch_ball(const S* q, const S* p, const int64_t* ql, const int64_t* pl, int64_t* idx,
                       float* dist2, int64_t B, int64_t Q, int64_t P, int64_t K, float r2,
                       const int* skip, hipStream_t stream) {
    if (B < 0 || Q < 0 || P < 0 || K < 0 || K > INT32_MAX || P > INT32_MAX - kBqDepth * kWave)
        return hipErrorInvalidValue;
    if (B == 0 || Q == 0 || K == 0) return hipSuccess;
    constexpr int NWQ = kBqLdsQueries;
    const int64_t qblocks = (Q + NWQ - 1) / NWQ;
    if (B <= 65535 && qblocks <= INT32_MAX) {
        // Clouds are spread over all XCDs (blockIdx.x fastest), which
        // balances clouds of different scan lengths across them.
        hipLaunchKernelGGL((ball_query_lds_kernel<S, NWQ, false>),
                           dim3(static_cast<uint32_t>(qblocks), static_cast<uint32_t>(B)),
                           dim3(NWQ * kWave), 0, stream, q, p, ql, pl, idx, dist2, Q, P,
                           static_cast<int>(K), r2, skip, Q);
        return hipGetLastError();
    }
    if (skip != nullptr) return hipErrorInvalidValue;
    const int64_t blocks = (B * Q + kBqWaves - 1) / kBqWaves;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((ball_query_kernel<S>), dim3(static_cast<uint32_t>(blocks)), dim3(kBqThreads),
                       0, stream, q, p, ql, pl, idx, dist2, B, Q, P, static_cast<int>(K), r2);
    return hipGetLastError();
}

template <typename S>
hipError_t launch_radius(const S* y, const S* x, const int64_t* ptr_y, const int64_t* ptr_x,
                         int64_t* out, int64_t Q, int64_t batch, int64_t K, float r2, int ignore,
                         hipStream_t stream) {
    if (Q < 0 || batch < 0 || K < 0 || K > INT32_MAX) return hipErrorInvalidValue;
    if (Q == 0 || K == 0) return hipSuccess;
    const int64_t blocks = (Q + kBqWaves - 1) / kBqWaves;
    if (batch == 0 || blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((radius_flat_kernel<S>), dim3(static_cast<uint32_t>(blocks)), dim3(kBqThreads),
                       0, stream, y, x, ptr_y, ptr_x, out, Q, batch, static_cast<int>(K), r2,
                       ignore ? 1 : 0);
    return hipGetLastError();
}

}  // namespace

hipError_t ball_query_pn2(const float* queries, const float* points, int32_t* idx, int64_t B,
                          int64_t Q, int64_t P, int64_t K, float r2, hipStream_t stream) {
    if (B < 0 || Q < 0 || P < 0 || K < 0 || K > INT32_MAX || P > INT32_MAX - kBqDepth * kWave)
        return hipErrorInvalidValue;
    if (B == 0 || Q == 0 || K == 0) return hipSuccess;
    constexpr int NWQ = kBqLdsQueries;
    const int64_t qblocks = (Q + NWQ - 1) / NWQ;
    if (B > 65535 || qblocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((ball_query_lds_kernel<float, NWQ, true>),
                       dim3(static_cast<uint32_t>(qblocks), static_cast<uint32_t>(B)),
                       dim3(NWQ * kWave), 0, stream, queries, points, nullptr, nullptr, idx, nullptr,
                       Q, P, static_cast<int>(K), r2, nullptr, Q);
    return hipGetLastError();
}

hipError_t ball_query_f32_unless(const float* queries, const float* points, int64_t* idx,
                                 float* dist2, int64_t B, int64_t Q, int64_t P, int64_t K,
                                 float radius_sq, const int* skip, hipStream_t stream) {
    return launch_ball<float>(queries, points, nullptr, nullptr, idx, dist2, B, Q, P, K, radius_sq,
                              skip, stream);
}

}  // namespace pointops

namespace pointops {

// Ball queries of several radii around the same centres in one scan (the
// multi-scale grouping of a PointNet++ layer): the LDS-staged search of
// ball_query_lds_kernel, each pair's distance computed once and tested
// against every radius still short of its K hits.  A radius keeps its own
// first-K list in index order, so every output equals that radius's own
// search, bit for bit; the scan ends when every radius is done (or the
// cloud is).  Float32, no lengths; Q query rows per cloud lying QS rows
// apart, as in ball_query_rows_f32.
template <int NR>
__global__ __launch_bounds__(kBqLdsQueries * kWave) void ball_query_multi_kernel(
    const float* __restrict__ queries, const float* __restrict__ points, BallMulti out,
    int64_t Q, int64_t P, int64_t QS) {
    constexpr int NWQ = kBqLdsQueries;
    constexpr int kTile = kBqLdsDepth * kWave;
    constexpr int kPer = kTile / (NWQ * kWave);
    static_assert(kPer * NWQ * kWave == kTile && kBqLdsDepth % 2 == 0 && NR <= kBqMulti, "shape");
    __shared__ float4 tile[kTile];
    __shared__ __align__(8) uint8_t done_flags[NWQ];  // one byte per wave, read as one word
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = uniform(tid / kWave);
    const int64_t b = blockIdx.y;
    const int64_t qi = static_cast<int64_t>(blockIdx.x) * NWQ + wave;
    const int n = static_cast<int>(P);
    const bool live = qi < Q;
    const int64_t row = b * QS + (live ? qi : 0);
    float qx = 0.f, qy = 0.f, qz = 0.f;
    if (live) {
        qx = queries[3 * row];
        qy = queries[3 * row + 1];
        qz = queries[3 * row + 2];
    }
    int found[NR];
    bool fin[NR];  // wave-uniform: this radius needs no more points
    bool done = true;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        found[r] = 0;
        // d < r2 is impossible for r2 <= 0 (d is never negative) or NaN r2.
        fin[r] = !live || !(out.r2[r] > 0.f);
        done = done && fin[r];
    }
    const float* pp = points + 3 * b * P;
    float4 pf[kPer];
    auto fetch = [&](int base) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const float* pt = pp + 3 * static_cast<int64_t>(min(base + k * NWQ * kWave + tid, n - 1));
            pf[k] = make_float4(pt[0], pt[1], pt[2], 0.f);
        }
    };
    if (n > 0) fetch(0);
    for (int base = 0; base < n; base += kTile) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) tile[k * NWQ * kWave + tid] = pf[k];
        __syncthreads();
        if (base + kTile < n) fetch(base + kTile);  // in flight during the scan
        auto scan = [&](auto full) {
#pragma unroll
            for (int c = 0; c < kBqLdsDepth; c += 2) {
                const float4 p0 = tile[c * kWave + lane];
                const float4 p1 = tile[(c + 1) * kWave + lane];
                const float d0 = sqdist3(qx, qy, qz, p0.x, p0.y, p0.z);
                const float d1 = sqdist3(qx, qy, qz, p1.x, p1.y, p1.z);
                const bool in0 = decltype(full)::value || base + c * kWave + lane < n;
                const bool in1 = decltype(full)::value || base + (c + 1) * kWave + lane < n;
                bool all = true;
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    if (fin[r]) continue;
                    const bool h0 = in0 && d0 < out.r2[r];
                    const bool h1 = in1 && d1 < out.r2[r];
                    const uint64_t m0 = ballot(h0), m1 = ballot(h1);
                    if ((m0 | m1) != 0) {
                        // A full tile needs the point indices only here.
                        const int j0 = base + c * kWave + lane, j1 = j0 + kWave;
                        const uint32_t s0 = static_cast<uint32_t>(found[r] + lanes_below(m0));
                        const uint32_t s1 =
                            static_cast<uint32_t>(found[r] + __popcll(m0) + lanes_below(m1));
                        const uint32_t uk = static_cast<uint32_t>(out.k[r]);
                        int64_t* oi = out.idx[r] + row * out.k[r];
                        float* od = out.dist[r] + row * out.k[r];
                        if (h0 && s0 < uk) {
                            row_at(oi, s0) = static_cast<int64_t>(static_cast<uint32_t>(j0));
                            row_at(od, s0) = d0;
                        }
                        if (h1 && s1 < uk) {
                            row_at(oi, s1) = static_cast<int64_t>(static_cast<uint32_t>(j1));
                            row_at(od, s1) = d1;
                        }
                        found[r] += __popcll(m0) + __popcll(m1);
                        fin[r] = found[r] >= out.k[r];
                    }
                    all = all && fin[r];
                }
                if (all) break;
            }
        };
        if (!done) {
            if (base + kTile <= n) scan(std::true_type{});
            else scan(std::false_type{});
            done = true;
#pragma unroll
            for (int r = 0; r < NR; ++r) done = done && fin[r];
        }
        if (lane == 0) done_flags[wave] = done ? 1 : 0;
        __syncthreads();  // flags written; every wave is past its reads of this tile
        if (*reinterpret_cast<const uint64_t*>(done_flags) == kBqAllDone) break;
    }
    if (!live) return;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        int64_t* oi = out.idx[r] + row * out.k[r];
        float* od = out.dist[r] + row * out.k[r];
        for (int s = min(found[r], out.k[r]) + lane; s < out.k[r]; s += kWave) {
            oi[s] = -1;
            od[s] = 0.f;
        }
    }
}

// The multi-radius search over Q query rows per cloud lying QS rows apart
// (1 <= nr <= kBqMulti radii; every k >= 1).
hipError_t ball_query_multi_rows_f32(const float* q, const float* p, const BallMulti& out, int nr,
                                     int64_t B, int64_t Q, int64_t QS, int64_t P,
                                     hipStream_t stream) {
    constexpr int NWQ = kBqLdsQueries;
    const int64_t qblocks = (Q + NWQ - 1) / NWQ;
    if (nr < 1 || nr > kBqMulti || B < 1 || B > 65535 || Q < 1 || QS < Q || P < 0 ||
        P > INT32_MAX - kBqDepth * kWave || qblocks > INT32_MAX)
        return hipErrorInvalidValue;
    for (int r = 0; r < nr; ++r)
        if (out.k[r] < 1 || out.idx[r] == nullptr || out.dist[r] == nullptr) return hipErrorInvalidValue;
    const dim3 grid(static_cast<uint32_t>(qblocks), static_cast<uint32_t>(B));
    const dim3 block(NWQ * kWave);
    switch (nr) {
        case 1: hipLaunchKernelGGL(ball_query_multi_kernel<1>, grid, block, 0, stream, q, p, out, Q, P, QS); break;
        case 2: hipLaunchKernelGGL(ball_query_multi_kernel<2>, grid, block, 0, stream, q, p, out, Q, P, QS); break;
        case 3: hipLaunchKernelGGL(ball_query_multi_kernel<3>, grid, block, 0, stream, q, p, out, Q, P, QS); break;
        default: hipLaunchKernelGGL(ball_query_multi_kernel<4>, grid, block, 0, stream, q, p, out, Q, P, QS); break;
    }
    return hipGetLastError();
}

}  // namespace pointops

using namespace pointops;

extern "C" {

hipError_t pointops_ball_query_f32(const float* queries, const float* points,
                                   const int64_t* query_lengths, const int64_t* point_lengths,
                                   int64_t* idx, float* dist2, int64_t B, int64_t Q, int64_t P,
                                   int64_t K, float radius_sq, hipStream_t stream) {
    return launch_ball<float>(queries, points, query_lengths, point_lengths, idx, dist2, B, Q, P, K,
                              radius_sq, nullptr, stream);
}

hipError_t pointops_ball_query_multi_f32(const float* queries, const float* points, int64_t nball,
                                         const float* radii_sq, const int64_t* ks,
                                         int64_t* const* idx, float* const* dist2, int64_t B,
                                         int64_t Q, int64_t P, hipStream_t stream) {
    if (nball < 0 || nball > 8 || B < 0 || Q < 0 || P < 0 || P > INT32_MAX - kBqDepth * kWave ||
        (nball > 0 && (radii_sq == nullptr || ks == nullptr || idx == nullptr || dist2 == nullptr)))
        return hipErrorInvalidValue;
    for (int64_t r = 0; r < nball; ++r)
        if (ks[r] < 0 || ks[r] > INT32_MAX || (ks[r] > 0 && (idx[r] == nullptr || dist2[r] == nullptr)))
            return hipErrorInvalidValue;
    if (B == 0 || Q == 0) return hipSuccess;
    if (queries == nullptr || points == nullptr || B > 65535) return hipErrorInvalidValue;
    // The radii with K >= 1 in order, kBqMulti to a scan.
    BallMulti out{};
    int nr = 0;
    for (int64_t r = 0; r <= nball; ++r) {
        if (r < nball && ks[r] > 0) {
            out.idx[nr] = idx[r];
            out.dist[nr] = dist2[r];
            out.k[nr] = static_cast<int>(ks[r]);
            out.r2[nr] = radii_sq[r];
            ++nr;
        }
        if (nr == kBqMulti || (r == nball && nr > 0)) {
            const hipError_t err = ball_query_multi_rows_f32(queries, points, out, nr, B, Q, Q, P, stream);
            if (err != hipSuccess) return err;
            nr = 0;
        }
    }
    return hipSuccess;
}

hipError_t pointops_ball_query_pn2_f32(const float* queries, const float* points, int32_t* idx,
                                       int64_t B, int64_t Q, int64_t P, int64_t K, float radius_sq,
                                       hipStream_t stream) {
    return ball_query_pn2(queries, points, idx, B, Q, P, K, radius_sq, stream);
}

hipError_t pointops_ball_query_f16(const uint16_t* queries, const uint16_t* points,
                                   const int64_t* query_lengths, const int64_t* point_lengths,
                                   int64_t* idx, float* dist2, int64_t B, int64_t Q, int64_t P,
                                   int64_t K, float radius_sq, hipStream_t stream) {
    return launch_ball<uint16_t>(queries, points, query_lengths, point_lengths, idx, dist2, B, Q, P,
                                 K, radius_sq, nullptr, stream);
}

hipError_t pointops_radius_flat_f32(const float* y, const float* x, const int64_t* ptr_y,
                                    const int64_t* ptr_x, int64_t* out, int64_t Q, int64_t batch,
                                    int64_t K, float radius_sq, int32_t ignore_same_index,
                                    hipStream_t stream) {
    return launch_radius<float>(y, x, ptr_y, ptr_x, out, Q, batch, K, radius_sq, ignore_same_index,
                                stream);
}

hipError_t pointops_radius_flat_f16(const uint16_t* y, const uint16_t* x, const int64_t* ptr_y,
                                    const int64_t* ptr_x, int64_t* out, int64_t Q, int64_t batch,
                                    int64_t K, float radius_sq, int32_t ignore_same_index,
                                    hipStream_t stream) {
    return launch_radius<uint16_t>(y, x, ptr_y, ptr_x, out, Q, batch, K, radius_sq,
                                   ignore_same_index, stream);
}

}  // extern "C"
