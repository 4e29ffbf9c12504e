// Sampling and neighbourhood queries of a PointNet++ set-abstraction front end
// (FPS, then ball queries and kNN around the sampled centres), overlapped.
//
// The reference runs these as dependent calls: furthest_point_sample
// (ops.py:53-141), a gather of the centres, ball_query (ops.py:208-227) per
// radius and knn (ops.py:144-205).  Single-cloud FPS is sequential in its
// samples and occupies one CU per cloud (B CUs of 256), while the queries of
// a centre need only that centre.  Here FPS runs on `fps_stream` and
// stores each sample's index, and its coordinates in the workspace,
// publishing per-cloud progress every `chunk` samples; on `query_stream`,
// for each chunk of centres a gate kernel (one wave per cloud) waits until
// its cloud has published the chunk and copies the cloud's centres of the
// chunk (contiguous rows, not a gather through the indices), and the ball
// queries of that chunk follow on the free CUs while FPS goes on, every
// radius in one scan (ball_query_multi_kernel: each distance computed once,
// each radius's first-K list as its own search would build it).  kNN runs
// once, over all centres, after the last chunk: its lane kernel gives each
// workgroup 64 queries against the whole cloud, so its duration does not
// shrink with the number of queries (measured at config 2: about 62 us for
// 128 centres per cloud, 86 us for 1024), and per-chunk launches would
// serialise that cost.  Results are those of the separate calls, bit for
// bit: each query's distances and tests are the same.
//
// The only waiting is the gates' bounded poll of the progress words; FPS
// waits on nothing, and its workgroups are resident before any chunk can be
// published, so the query kernels queued behind a gate cannot keep FPS from
// running.
//
// Every call owns its progress words and status word: a clear kernel on
// `fps_stream` zeroes them, and `query_stream` waits (through an event) for
// that clear before its first gate, so a gate can only be satisfied by its
// own call's FPS.  Overlapping calls (on other streams, or queued back to
// back) need distinct workspaces; the Python wrapper allocates one per call.
// A gate wave that gives up (its poll budget spent, or a gate of the call
// gave up before it started) sets *status and writes NaN centres for its
// cloud's chunk, so those queries run on NaN centres: ball-query rows
// (0, -1) and kNN rows (inf, 2^32 - 1), the reference's results for a NaN
// query.  FPS only ever writes the workspace's copy, so nothing overwrites
// the NaN.  Every launch ends.
#include <cstdlib>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {

hipError_t fps_dense_progress(const float* xyz, int64_t* out, int64_t B, int64_t N,
                              int64_t npoint, int64_t start, int skip, uint64_t* progress,
                              uint64_t tag, int64_t chunk, float* centres, hipStream_t stream);
hipError_t knn3_window_sort(const float* ref, void* workspace, int64_t B, int64_t M, int64_t N,
                            hipStream_t stream);
hipError_t knn3_windowed_rows(const float* query, const float* ref, float* dist, int64_t* idx,
                              void* workspace, int64_t B, int64_t M, int64_t QS, int64_t N,
                              int64_t K, hipStream_t stream);

namespace {

constexpr int kGateThreads = 256;
// Reads of its cloud's progress word per gate wave before it gives up,
// each after a sleep of about 0.5 us: several
// seconds, against well under a second for the longest FPS this path takes
// (65535 clouds of 8192 points).
constexpr uint32_t kGateSpinLimit = 1u << 24;
constexpr size_t kAlign = 256;
constexpr int kMaxDevices = 64;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// kGateSpinLimit, or POINTOPS_PIPELINE_SPIN_LIMIT when set, read per call
// (0 makes every gate give up without reading a progress word: the host's
// way to exercise the give-up path while every kernel still ends).
uint32_t gate_spin_limit() {
    const char* env = std::getenv("POINTOPS_PIPELINE_SPIN_LIMIT");
    if (env == nullptr || *env == '\0') return kGateSpinLimit;
    return static_cast<uint32_t>(std::strtoul(env, nullptr, 10));
}

// Two events per host thread and device: `cleared` orders the query stream
// after the clear of the call's words, `done` orders the FPS stream after
// the call's last query.  An event may be recorded again once the waits on
// its previous record are enqueued, which happens before this call returns,
// so one pair per thread suffices.  They are never destroyed (no exit-time
// HIP calls).
struct CallEvents {
    hipEvent_t cleared = nullptr;
    hipEvent_t done = nullptr;
};
thread_local CallEvents tl_events[kMaxDevices];

hipError_t call_events(hipStream_t stream, CallEvents** out) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    int stream_device = device;
    err = hipStreamGetDevice(stream, &stream_device);
    if (err != hipSuccess) return err;
    if (stream_device != device || device < 0 || device >= kMaxDevices)
        return hipErrorInvalidDevice;
    CallEvents& ev = tl_events[device];
    if (ev.cleared == nullptr) {
        err = hipEventCreateWithFlags(&ev.cleared, hipEventDisableTiming);
        if (err != hipSuccess) return err;
    }
    if (ev.done == nullptr) {
        err = hipEventCreateWithFlags(&ev.done, hipEventDisableTiming);
        if (err != hipSuccess) return err;
    }
    *out = &ev;
    return hipSuccess;
}

// Zeroes the B progress words and the status word of one call.
__global__ __launch_bounds__(kGateThreads) void pipeline_clear_kernel(
    uint64_t* __restrict__ progress, uint32_t* __restrict__ status, int64_t B) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kGateThreads + threadIdx.x;
    if (i < B) progress[i] = 0;
    if (i == 0) status[0] = 0;
}

// One wave per cloud b: waits until progress[b] >= target, then writes the
// centres of samples [m0, m1) of cloud b, copied from the coordinates FPS
// stored in `staged` (B, npoint, 3) before publishing them (contiguous
// rows, every load in flight at once).  The wave reads the word at most
// `spin_limit` times; if it gives up, or an earlier gate of the call has
// (*status set), it sets *status and the cloud's chunk of centres is NaN.
constexpr int kGateRowFloats = 12;  // floats per lane per copy round

__global__ __launch_bounds__(kWave) void pipeline_gate_kernel(
    const uint64_t* __restrict__ progress, uint64_t target, const float* staged,
    float* __restrict__ centres, uint32_t* __restrict__ status, int64_t npoint, int64_t m0,
    int64_t m1, uint32_t spin_limit) {
    const int64_t b = blockIdx.x;
    const int lane = threadIdx.x;
    bool gave_up = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
    for (uint32_t polls = 0; !gave_up; ++polls) {
        if (polls >= spin_limit) {
            gave_up = true;
            break;
        }
        if (__hip_atomic_load(progress + b, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) >= target)
            break;
        __builtin_amdgcn_s_sleep(16);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (gave_up && lane == 0)
        __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t row = (m1 - m0) * 3;  // floats of the cloud's chunk
    const float* src = staged + (b * npoint + m0) * 3;
    float* dst = centres + (b * npoint + m0) * 3;
    for (int64_t i0 = lane; i0 < row; i0 += kGateRowFloats * kWave) {
        float v[kGateRowFloats];
#pragma unroll
        for (int u = 0; u < kGateRowFloats; ++u)
            v[u] = gave_up ? __builtin_nanf("") : src[min(i0 + u * kWave, row - 1)];
#pragma unroll
        for (int u = 0; u < kGateRowFloats; ++u)
            if (i0 + u * kWave < row) dst[i0 + u * kWave] = v[u];
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
           align_up(static_cast<size_t>(B * npoint * 3) * sizeof(float)) +
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
        if (ball_k[r] < 1 || ball_k[r] > INT32_MAX || ball_idx[r] == nullptr ||
            ball_dist2[r] == nullptr)
            return hipErrorInvalidValue;
    const int64_t chunks = (npoint + chunk - 1) / chunk;
    uint64_t* progress = static_cast<uint64_t*>(workspace);
    float* staged = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                             align_up(static_cast<size_t>(B) * sizeof(uint64_t)));
    char* knn_ws = reinterpret_cast<char*>(staged) +
                   align_up(static_cast<size_t>(B * npoint * 3) * sizeof(float));
    CallEvents* ev = nullptr;
    hipError_t err = call_events(fps_stream, &ev);
    if (err != hipSuccess) return err;
    const uint32_t limit = gate_spin_limit();
    // This call's words start at zero, after everything already on fps_stream.
    hipLaunchKernelGGL(pipeline_clear_kernel, dim3(static_cast<uint32_t>((B + kGateThreads - 1) / kGateThreads)),
                       dim3(kGateThreads), 0, fps_stream, progress, status, B);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if ((err = hipEventRecord(ev->cleared, fps_stream)) != hipSuccess) return err;
    if ((err = hipStreamWaitEvent(query_stream, ev->cleared, 0)) != hipSuccess) return err;
    err = fps_dense_progress(xyz, samples, B, N, npoint, start_idx, skip_near_origin != 0,
                             progress, 0, chunk, staged, fps_stream);
    if (err != hipSuccess) return err;
    // kNN's sort of the references needs the cloud only: it runs first on
    // the query stream, beside FPS.
    if (knn_k > 0) {
        err = knn3_window_sort(xyz, knn_ws, B, npoint, N, query_stream);
        if (err != hipSuccess) return err;
    }
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t m0 = c * chunk;
        const int64_t m1 = m0 + chunk < npoint ? m0 + chunk : npoint;
        const int64_t mc = m1 - m0;
        hipLaunchKernelGGL(pipeline_gate_kernel, dim3(static_cast<uint32_t>(B)), dim3(kWave), 0,
                           query_stream, progress, static_cast<uint64_t>(c + 1), staged, centres,
                           status, npoint, m0, m1, limit);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        // The radii in groups of up to kBqMulti, each group in one scan.
        for (int64_t r0 = 0; r0 < nball; r0 += kBqMulti) {
            const int nr = static_cast<int>(nball - r0 < kBqMulti ? nball - r0 : kBqMulti);
            BallMulti out{};
            for (int r = 0; r < nr; ++r) {
                out.idx[r] = ball_idx[r0 + r] + m0 * ball_k[r0 + r];
                out.dist[r] = ball_dist2[r0 + r] + m0 * ball_k[r0 + r];
                out.k[r] = static_cast<int>(ball_k[r0 + r]);
                out.r2[r] = radii_sq[r0 + r];
            }
            err = ball_query_multi_rows_f32(centres + 3 * m0, xyz, out, nr, B, mc, npoint, N,
                                            query_stream);
            if (err != hipSuccess) return err;
        }
    }
    if (knn_k > 0) {  // after the last gate: every centre is in place
        err = knn3_windowed_rows(centres, xyz, knn_dist, knn_idx, knn_ws, B, npoint, npoint, N,
                                 knn_k, query_stream);
        if (err != hipSuccess) return err;
    }
    // Work queued on fps_stream after this call sees every output.
    if ((err = hipEventRecord(ev->done, query_stream)) != hipSuccess) return err;
    return hipStreamWaitEvent(fps_stream, ev->done, 0);
}

}  // extern "C"
