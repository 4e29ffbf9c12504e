// Sampling and neighbourhood queries of a PointNet++ set-abstraction front end
// (FPS, then ball queries and kNN around the sampled centres), overlapped.
//
// The reference runs these as dependent calls: furthest_point_sample
// (ops.py:53-141), a gather of the centres, ball_query (ops.py:208-227) per
// radius and knn (ops.py:144-205).  Single-cloud FPS is sequential in its
// samples and occupies one CU per cloud (B CUs of 256), while the queries of
// a centre need only that centre.  Here FPS runs on `fps_stream` and
// publishes per-cloud progress every `chunk` samples; on `query_stream`, for
// each chunk of centres a one-workgroup gate kernel waits until every cloud
// has published the chunk, gathers its centres, and the ball queries of that
// chunk follow on the free CUs while FPS goes on.  kNN runs once, over all
// centres, after the last chunk: its lane kernel gives each workgroup 64
// queries against the whole cloud, so its duration does not shrink with the
// number of queries (measured at config 2: about 62 us for 128 centres per
// cloud, 86 us for 1024), and per-chunk launches would serialise that cost.  Results are those
// of the separate calls, bit for bit: the same kernels compute each query.
//
// The only waiting is the gate's bounded poll of the progress words; FPS
// waits on nothing, and its workgroups are resident before any chunk can be
// published, so the query kernels queued behind a gate cannot keep FPS from
// running.  A gate that gives up (kGateSpinLimit polls) sets *status and
// lets its chunk run on whatever the samples hold (indices clamped in
// bounds), so every launch ends.
#include <atomic>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {

hipError_t fps_dense_progress(const float* xyz, int64_t* out, int64_t B, int64_t N,
                              int64_t npoint, int64_t start, int skip, uint64_t* progress,
                              uint64_t tag, int64_t chunk, hipStream_t stream);
hipError_t ball_query_rows_f32(const float* q, const float* p, int64_t* idx, float* dist2,
                               int64_t B, int64_t Q, int64_t QS, int64_t P, int64_t K, float r2,
                               hipStream_t stream);
hipError_t knn3_windowed_rows(const float* query, const float* ref, float* dist, int64_t* idx,
                              void* workspace, int64_t B, int64_t M, int64_t QS, int64_t N,
                              int64_t K, hipStream_t stream);

namespace {

constexpr int kGateThreads = 256;
// Polls of one progress word before a gate gives up, each after a sleep of
// about 0.5 us: several seconds, against a few milliseconds for the longest
// FPS this path takes (8192 points).
constexpr uint32_t kGateSpinLimit = 1u << 24;
// Tags advance by 2^20 per call, above any chunk count (at most 8192).
constexpr int kTagShift = 20;
constexpr size_t kAlign = 256;

std::atomic<uint64_t> g_epoch{0};

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Waits until progress[b] >= target for every cloud b, then writes the
// centres of samples [m0, m1) of every cloud: centres[b, m] = xyz[b, samples[b, m]].
__global__ __launch_bounds__(kGateThreads) void pipeline_gate_kernel(
    const uint64_t* __restrict__ progress, uint64_t target, const float* __restrict__ xyz,
    const int64_t* samples, float* __restrict__ centres, uint32_t* __restrict__ status,
    int64_t B, int64_t N, int64_t npoint, int64_t m0, int64_t m1) {
    __shared__ int gave_up;
    if (threadIdx.x == 0) gave_up = 0;
    __syncthreads();
    for (int64_t b = threadIdx.x; b < B; b += kGateThreads) {
        uint32_t polls = 0;
        while (__hip_atomic_load(progress + b, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++polls > kGateSpinLimit) {
                gave_up = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(16);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (gave_up && threadIdx.x == 0) status[0] = 1u;
    const int64_t mc = m1 - m0;
    for (int64_t i = threadIdx.x; i < B * mc; i += kGateThreads) {
        const int64_t b = i / mc, m = m0 + i % mc;
        // Samples are read with agent-scope atomic loads: they were stored by
        // workgroups still running on other XCDs.
        int64_t j = __hip_atomic_load(samples + b * npoint + m, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
        j = j < 0 ? 0 : (j >= N ? N - 1 : j);
        const float* src = xyz + (b * N + j) * 3;
        float* dst = centres + (b * npoint + m) * 3;
        dst[0] = src[0];
        dst[1] = src[1];
        dst[2] = src[2];
    }
}

}  // namespace
}  // namespace pointops

using namespace pointops;

extern "C" {

size_t pointops_fps_query_pipeline_workspace_bytes(int64_t B, int64_t N, int64_t npoint,
                                                   int64_t chunk) {
    if (B <= 0 || N <= 0 || npoint <= 0 || chunk <= 0) return 0;
    return align_up(static_cast<size_t>(B) * sizeof(uint64_t)) +
           pointops_knn3_windowed_workspace_bytes(B, npoint, N);
}

hipError_t pointops_fps_query_pipeline_f32(
    const float* xyz, int64_t* samples, float* centres, int64_t nball, const float* radii_sq,
    const int64_t* ball_k, int64_t* const* ball_idx, float* const* ball_dist2, int64_t knn_k,
    float* knn_dist, int64_t* knn_idx, void* workspace, uint32_t* status, int64_t B, int64_t N,
    int64_t npoint, int64_t start_idx, int32_t skip_near_origin, int64_t chunk,
    hipStream_t fps_stream, hipStream_t query_stream) {
    if (xyz == nullptr || samples == nullptr || centres == nullptr || workspace == nullptr ||
        status == nullptr || B < 1 || B > 65535 || N < 1 || npoint < 1 || npoint > N ||
        chunk < 1 || nball < 0 || nball > 8 || knn_k < 0 || knn_k > 32 || knn_k > N ||
        (nball > 0 && (radii_sq == nullptr || ball_k == nullptr || ball_idx == nullptr ||
                       ball_dist2 == nullptr)) ||
        (knn_k > 0 && (knn_dist == nullptr || knn_idx == nullptr)))
        return hipErrorInvalidValue;
    for (int64_t r = 0; r < nball; ++r)
        if (ball_k[r] < 1 || ball_idx[r] == nullptr || ball_dist2[r] == nullptr)
            return hipErrorInvalidValue;
    const int64_t chunks = (npoint + chunk - 1) / chunk;
    if (chunks >= (int64_t(1) << kTagShift)) return hipErrorInvalidValue;
    uint64_t* progress = static_cast<uint64_t*>(workspace);
    char* knn_ws = static_cast<char*>(workspace) + align_up(static_cast<size_t>(B) * sizeof(uint64_t));
    // Progress words hold an earlier call's tag (smaller) or zero: every
    // target of this call lies above them.
    const uint64_t tag = (g_epoch.fetch_add(1) + 1) << kTagShift;
    hipError_t err = fps_dense_progress(xyz, samples, B, N, npoint, start_idx,
                                        skip_near_origin != 0, progress, tag, chunk, fps_stream);
    if (err != hipSuccess) return err;
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t m0 = c * chunk;
        const int64_t m1 = m0 + chunk < npoint ? m0 + chunk : npoint;
        const int64_t mc = m1 - m0;
        hipLaunchKernelGGL(pipeline_gate_kernel, dim3(1), dim3(kGateThreads), 0, query_stream,
                           progress, tag + static_cast<uint64_t>(c + 1), xyz, samples, centres,
                           status, B, N, npoint, m0, m1);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        for (int64_t r = 0; r < nball; ++r) {
            err = ball_query_rows_f32(centres + 3 * m0, xyz, ball_idx[r] + m0 * ball_k[r],
                                      ball_dist2[r] + m0 * ball_k[r], B, mc, npoint, N, ball_k[r],
                                      radii_sq[r], query_stream);
            if (err != hipSuccess) return err;
        }
    }
    if (knn_k > 0)  // after the last gate: every centre is in place
        return knn3_windowed_rows(centres, xyz, knn_dist, knn_idx, knn_ws, B, npoint, npoint, N,
                                  knn_k, query_stream);
    return hipSuccess;
}

}  // extern "C"
