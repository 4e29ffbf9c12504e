// Farthest point sampling for gfx950.
//
// Semantics (reference.py:27-58, kernels/fps.metal:19-107): sampling starts at
// `start`; each step takes the point whose running minimum squared distance
// to the sampled set is largest, ties to the smaller index; points with
// ((x*x + y*y) + z*z) < fl32(1e-3) are never picked when skip_near_origin is
// set (their running distance is -inf); if no point can be picked the step
// takes index 0.  A point with a NaN coordinate is never picked either: its
// running distance starts at -inf, as a NaN running distance never wins
// `m > best` in kernels/fps.metal:77-83 (reference.py:56-57's torch.minimum
// and argmax would instead let NaN win).
//
// Kernels:
//   fps_lead_kernel<P>      one workgroup per cloud of up to 4096 points:
//                           the tiled scheme below with the step chain taken
//                           by one leader wave and the tile updates applied
//                           by eight follower waves.
//   fps_tiled_kernel<P,T,PO> one workgroup per cloud of up to 8192 points
//                           (batched or ragged), its points and running
//                           distances in VGPRs, sorted into spatially compact
//                           64-point tiles so that a step updates only the
//                           tiles it can change; exact steps over 64
//                           published candidates between exchanges.
//   fps_global_kernel<T>    one workgroup per cloud for larger clouds of a
//                           batch: points re-read from L2, running distances
//                           in a caller-provided scratch array.
//   fps_lazy_kernel<P,T>    one cloud over up to 256 CUs (cooperative
//                           launch): each workgroup keeps its chunk in VGPRs;
//                           an exchange publishes every wave's best candidate
//                           and a bound, after which every workgroup takes
//                           exact steps over the candidates alone until the
//                           bound could be reached.
//   fps_stream_kernel<T>    the same exchange for clouds too large for the
//                           CUs' registers, the cloud streamed from HBM.
#include <hip/hip_cooperative_groups.h>

#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "pointops_common.hpp"
#include "pointops_hip.h"

namespace pointops {
namespace {

constexpr float kSkipThreshold = 1e-3f;  // torch.tensor(1e-3, dtype=float32)

__device__ __forceinline__ bool near_origin(float x, float y, float z) {
    float mag = x * x;
    mag = mag + y * y;
    mag = mag + z * z;
    return mag < kSkipThreshold;
}

// Initial running distance of a point: -inf for one that is never sampled
// (a NaN coordinate, as in kernels/fps.metal:77-83, where a NaN running
// distance never wins `m > best`; or near the origin when skip is set),
// +inf otherwise.  Every step's minimum keeps -inf, so such a point is
// never taken while another point of its cloud has a larger running
// distance (a taken point keeps 0).
__device__ __forceinline__ float initial_running(int skip, float x, float y, float z) {
    const bool nan = __builtin_isnan(x) || __builtin_isnan(y) || __builtin_isnan(z);
    return (nan || (skip && near_origin(x, y, z))) ? -INFINITY : INFINITY;
}

// Segment of workgroup b: dense clouds (ptr == nullptr) or ragged ones.
struct Segment {
    int64_t in_lo;   // first point of the cloud
    int64_t n;       // points in the cloud
    int64_t out_lo;  // first output slot
    int64_t cnt;     // samples to take
    int64_t start;   // local start index
    int64_t base;    // added to every emitted local index
};

__device__ __forceinline__ Segment segment_of(int b, const int64_t* ptr, const int64_t* out_ptr,
                                              const int64_t* starts, int64_t N, int64_t npoint,
                                              int64_t start) {
    Segment s;
    if (ptr != nullptr) {
        s.in_lo = ptr[b];
        s.n = ptr[b + 1] - s.in_lo;
        s.out_lo = out_ptr[b];
        s.cnt = out_ptr[b + 1] - s.out_lo;
        s.start = starts[b];
        s.base = s.in_lo;
    } else {
        s.in_lo = static_cast<int64_t>(b) * N;
        s.n = N;
        s.out_lo = static_cast<int64_t>(b) * npoint;
        s.cnt = npoint;
        s.start = start;
        s.base = 0;
    }
    return s;
}

// Block-wide argmax of (value, index) pairs held one per wave in `slots`:
// largest value, then smallest index.  Every thread gets the result.
template <int NW>
__device__ __forceinline__ int block_argmax(const int2* slots) {
    float best = i2f(slots[0].x);
    int bidx = slots[0].y;
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        const float v = i2f(slots[w].x);
        const int i = slots[w].y;
        if (v > best || (v == best && i < bidx)) {
            best = v;
            bidx = i;
        }
    }
    return bidx;
}

// One wave's candidate for a step: its largest running distance, the
// smallest point index holding it, and that point's coordinates.
struct alignas(16) WaveBest {
    int key;    // running distance bits
    int index;  // local point index
    float x, y, z;
    int pad[3];
};
// fps_tiled_kernel<P,T,PO>: the lazy single-workgroup FPS on a spatially
// sorted cloud, so that most per-step updates can be skipped.
//
// Setup: the cloud is counting-sorted in LDS by a 12-bit Morton key of its
// 16 x 16 x 16 cell (over the cloud's bounding box) and cut into tiles of 64
// consecutive sorted positions (lane = position % 64), so every tile holds
// 64 nearby points.  The first half of the waves hold PO tiles each, the
// others 2P - PO: two waves share a SIMD and the older one is issued first,
// so tile work moved to it shortens the run's critical wave.  Each point
// keeps its original index, which breaks every tie (largest running
// distance, then smallest index), so results do not depend on the sort.
// Lane s of every wave holds the bounding box of the wave's tile s.
//
// Steps are taken lazily: at an exchange every wave publishes its KC best
// points (largest running distance, then smallest index) and the (KC+1)-th
// largest running distance, its bound; every wave then holds the 64
// candidates, one per lane, and takes steps on its own (no barrier) while the
// chosen key is provably the argmax of the cloud -- always for the first
// step after an exchange (each wave published its maximum), afterwards while
// it is strictly above every bound (an unpublished running distance is at
// most its wave's bound, and distances only decrease).  Candidates are
// updated with the points' own arithmetic.  A step with centroid c and chosen key M (the
// largest running distance of the cloud) updates tile s only if
// lb(c, box_s) < M, where lb applies the update's own rounded operations
// to the per-axis gaps between c and the box: rounding is monotone, so lb
// is at most the rounded squared distance of every point in the box, and
// every running distance is at most M; a skipped tile therefore has no
// running distance that the update would lower.
template <int P, int T, int PO>
__global__ __launch_bounds__(T) void fps_tiled_kernel(const float* __restrict__ xyz,
                                                      const int64_t* __restrict__ ptr,
                                                      const int64_t* __restrict__ out_ptr,
                                                      const int64_t* __restrict__ starts,
                                                      int64_t* __restrict__ out, int64_t N,
                                                      int64_t npoint, int64_t start, int skip,
    uint64_t* __restrict__ progress, uint64_t tag, int64_t chunk, float* __restrict__ centres) {
    constexpr int NW = T / kWave;
    constexpr int KC = kWave / NW;  // candidates per wave
    constexpr int CAP = P * T;      // points per cloud at most
    constexpr int kCells = 4096;
    static_assert(KC * NW == kWave && KC + 1 <= kWave && P <= 16 && CAP <= 8192, "shape");
    static_assert(PO >= P && PO < 2 * P && PO <= 16 && NW % 2 == 0, "tile split");
    static_assert(kCells % T == 0, "cells per thread");
    // The sort's arrays, then (from the load of the tiles on) the points'
    // coordinates by sorted position, for the exchange's candidates.
    constexpr int kSortInts = kCells + CAP;
    constexpr int kBufVec = (kSortInts * 4 > CAP * 16 ? kSortInts * 4 : CAP * 16) / 16;
    __shared__ float4 buf[kBufVec];
    int* const cell_count = reinterpret_cast<int*>(buf);  // per-cell counts, then offsets
    int* const sorted_index = cell_count + kCells;         // sorted position -> local index
    float4* const spts = buf;                              // sorted position -> xyz
    __shared__ float red[6][NW];        // bounding-box partials
    __shared__ int wave_sum[NW];
    // Candidates and bounds, double-buffered by exchange parity: a wave
    // writes the next exchange's buffer only after the barrier that every
    // wave reaches after reading this one, so one barrier per exchange
    // suffices.
    __shared__ WaveBest cands[2][kWave];
    __shared__ int bounds[2][NW];

    const Segment seg = segment_of(blockIdx.x, ptr, out_ptr, starts, N, npoint, start);
    if (seg.cnt <= 0) return;  // uniform over the workgroup, before any barrier
    const float* p = xyz + 3 * seg.in_lo;
    int64_t* o = out + seg.out_lo;
    const int n = static_cast<int>(seg.n);
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int far0 = static_cast<int>(seg.start);
    // With `centres` set, sample s's coordinates also go to
    // centres[3 (out_lo + s) ..], copied from the cloud.
    float* const oc = centres != nullptr ? centres + 3 * seg.out_lo : nullptr;
    if (tid == 0) {
        o[0] = seg.base + far0;
        if (oc != nullptr && n > 0) {
            oc[0] = p[3 * far0];
            oc[1] = p[3 * far0 + 1];
            oc[2] = p[3 * far0 + 2];
        }
    }
    // With `progress` set, wave 0 publishes, once the samples [0, done) are
    // stored, tag + the number of whole `chunk`s among them (all of them once
    // done == seg.cnt) in word blockIdx.x: an agent-scope release fence over
    // the wave's stores, then one lane's store, so that a workgroup on any
    // XCD that reads the word with acquire ordering sees those samples.
    auto publish = [&](int64_t before, int64_t done) {
        if (progress == nullptr || wave != 0) return;
        const int64_t whole = (seg.cnt + chunk - 1) / chunk;
        const int64_t now = done >= seg.cnt ? whole : done / chunk;
        if (before >= 0 && now == (before >= seg.cnt ? whole : before / chunk)) return;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if (lane == 0)
            __hip_atomic_store(progress + blockIdx.x, tag + static_cast<uint64_t>(now),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (seg.cnt == 1 || n <= 0) {
        publish(-1, seg.cnt);
        return;
    }

    // ---- setup: bounding box, cells, counting sort
    for (int c = tid; c < kCells; c += T) cell_count[c] = 0;
    float lx[P], ly[P], lz[P];  // points t*P .. t*P+P-1 in index order
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int j = min(tid * P + k, n - 1);
        lx[k] = p[3 * j];
        ly[k] = p[3 * j + 1];
        lz[k] = p[3 * j + 2];
    }
    {
        float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int k = 0; k < P; ++k) {  // clamped duplicates do not change the box
            mn[0] = fminf(mn[0], lx[k]); mx[0] = fmaxf(mx[0], lx[k]);
            mn[1] = fminf(mn[1], ly[k]); mx[1] = fmaxf(mx[1], ly[k]);
            mn[2] = fminf(mn[2], lz[k]); mx[2] = fmaxf(mx[2], lz[k]);
        }
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            mn[a] = wave_min(mn[a]);
            mx[a] = wave_max(mx[a]);
        }
        if (lane == 0) {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                red[a][wave] = mn[a];
                red[3 + a][wave] = mx[a];
            }
        }
    }
    __syncthreads();  // box partials and cleared counters
    float lo[3], scale[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        float mn = red[a][0], mx = red[3 + a][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            mn = fminf(mn, red[a][w]);
            mx = fmaxf(mx, red[3 + a][w]);
        }
        lo[a] = mn;
        const float ext = mx - mn;
        scale[a] = (ext > 0.f && ext < INFINITY) ? 16.f / ext : 0.f;
    }
    int cell[P], rank[P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const float c3[3] = {lx[k], ly[k], lz[k]};
        uint32_t key = 0;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            // fmaxf/fminf also map NaN to cell 0 and infinities to the edges.
            const float f = fminf(fmaxf((c3[a] - lo[a]) * scale[a], 0.f), 15.f);
            const uint32_t q = static_cast<uint32_t>(f);
#pragma unroll
            for (int b = 0; b < 4; ++b) key |= ((q >> b) & 1u) << (3 * b + a);
        }
        cell[k] = static_cast<int>(key);
        rank[k] = (tid * P + k < n) ? atomicAdd(&cell_count[key], 1) : 0;
    }
    __syncthreads();  // counts complete
    {
        constexpr int CPT = kCells / T;  // cells per thread, scanned in place
        int run = 0;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int v = cell_count[tid * CPT + c];
            cell_count[tid * CPT + c] = run;
            run += v;
        }
        int incl = run;  // inclusive scan of the per-thread totals over the wave
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int up = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += up;
        }
        if (lane == kWave - 1) wave_sum[wave] = incl;
        __syncthreads();  // wave totals
        int before = incl - run;
        for (int w = 0; w < wave; ++w) before += wave_sum[w];
#pragma unroll
        for (int c = 0; c < CPT; ++c) cell_count[tid * CPT + c] += before;
    }
    __syncthreads();  // offsets complete
#pragma unroll
    for (int k = 0; k < P; ++k)
        if (tid * P + k < n) sorted_index[cell_count[cell[k]] + rank[k]] = tid * P + k;
    __syncthreads();  // permutation complete

    // ---- this thread's tile points, their indices and running distances
    const int my_tiles = wave < NW / 2 ? PO : 2 * P - PO;
    const int tile0 = wave < NW / 2 ? wave * PO : (NW / 2) * PO + (wave - NW / 2) * (2 * P - PO);
    constexpr int PA = PO <= 8 ? PO + 1 : PO;  // see fps_lazy_kernel
    float px[PA], py[PA], pz[PA], md[PO];
    int pcode[PA];  // local index << 13 | sorted position
#pragma unroll
    for (int k = 0; k < PA; ++k) {
        px[k] = py[k] = pz[k] = 0.f;
        pcode[k] = 0x7FFFFFFF;
    }
    float cx, cy, cz;
    {
        const int f = min(max(far0, 0), n - 1);
        cx = p[3 * f];
        cy = p[3 * f + 1];
        cz = p[3 * f + 2];
    }
    // Tile boxes; lanes without a tile, and tiles with no point of finite
    // coordinates on some axis, keep [+inf, +inf], which the step's box test
    // never selects.
    float blo[3] = {INFINITY, INFINITY, INFINITY}, bhi[3] = {INFINITY, INFINITY, INFINITY};
#pragma unroll
    for (int k = 0; k < PO; ++k) {
        const int q = (tile0 + k) * kWave + lane;
        const bool valid = k < my_tiles && q < n;
        const int j = valid ? sorted_index[q] : 0;
        px[k] = valid ? p[3 * j] : 0.f;
        py[k] = valid ? p[3 * j + 1] : 0.f;
        pz[k] = valid ? p[3 * j + 2] : 0.f;
        pcode[k] = valid ? (j << 13) | q : 0x7FFFFFFF;
        md[k] = !valid ? -INFINITY : initial_running(skip, px[k], py[k], pz[k]);
        md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], cx, cy, cz));
        // Box of tile k (padding excluded), kept in lane k.
        const float tlx = wave_min(valid ? px[k] : INFINITY), thx = wave_max(valid ? px[k] : -INFINITY);
        const float tly = wave_min(valid ? py[k] : INFINITY), thy = wave_max(valid ? py[k] : -INFINITY);
        const float tlz = wave_min(valid ? pz[k] : INFINITY), thz = wave_max(valid ? pz[k] : -INFINITY);
        if (lane == k && tlx <= thx && tly <= thy && tlz <= thz) {
            blo[0] = tlx; bhi[0] = thx;
            blo[1] = tly; bhi[1] = thy;
            blo[2] = tlz; bhi[2] = thz;
        }
    }

    __syncthreads();  // every sorted index has been read
#pragma unroll
    for (int k = 0; k < PO; ++k) {
        const int q = (tile0 + k) * kWave + lane;
        if (k < my_tiles && q < n) spts[q] = make_float4(px[k], py[k], pz[k], 0.f);
    }
    __syncthreads();  // coordinates by sorted position

    // ---- lazy steps
    // Tile updates run one step late (their scalar branches then test a
    // mask that is already in SGPRs): the centroid and mask of the step
    // before.  Steps read only the candidates, and every update is applied
    // before the next exchange reads the points.
    uint32_t pend = 0;
    float pfx = 0.f, pfy = 0.f, pfz = 0.f;
    auto apply_pending = [&]() {
#pragma unroll
        for (int k = 0; k < PO; ++k)
            if ((pend >> k) & 1u)
                md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], pfx, pfy, pfz));
        pend = 0;
    };
    int64_t step = 1;
    int parity = 0;
    while (step < seg.cnt) {
        // Exchange: this wave's KC best points (largest running distance,
        // then smallest index) and its bound, the (KC+1)-th.  Keys pack
        // (running distance bits ^ sign, ~code) into 64 bits, so one
        // unsigned compare orders them (0: no key).  Each lane keeps its two
        // largest keys; after a lane publishes its first, its second moves
        // up and the lane is marked in `unknown` (a wave-uniform mask), and
        // only if it wins again are its slots rescanned, below the key it
        // just published.  Candidate r collects in lane r; its coordinates
        // are read from LDS afterwards.
        auto top2 = [&](bool limited, uint64_t lim, uint64_t& a1, uint64_t& a2) {
            a1 = 0;
            a2 = 0;
#pragma unroll
            for (int k = 0; k < PO; ++k) {
                if (k >= my_tiles) break;  // wave-uniform
                const uint64_t key =
                    (static_cast<uint64_t>(static_cast<uint32_t>(f2i(md[k])) ^ 0x80000000u) << 32) |
                    static_cast<uint32_t>(~pcode[k]);
                const bool below = !limited || key < lim;
                const bool first = below && key > a1;
                const bool second = below && !first && key > a2;
                a2 = first ? a1 : (second ? key : a2);
                a1 = first ? key : a1;
            }
        };
        uint64_t h1, h2;
        top2(false, 0, h1, h2);
        uint64_t unknown = 0;
        int ck = 0, cc = 0x7FFFFFFF;
        int bound = 0;
#pragma unroll
        for (int r = 0; r <= KC; ++r) {
            const uint32_t hh = static_cast<uint32_t>(h1 >> 32);
            const uint32_t wv = wave_max_u32_l63(hh);
            const uint64_t at = ballot(hh == wv);
            int wl = static_cast<int>(__builtin_ctzll(at));
            uint32_t wlo;
            if (__popcll(at) > 1) {  // equal distances: the largest ~code (smallest index)
                wlo = wave_max_u32_l63(hh == wv ? static_cast<uint32_t>(h1) : 0u);
                wl = static_cast<int>(__builtin_ctzll(ballot(hh == wv && static_cast<uint32_t>(h1) == wlo)));
            } else {
                wlo = static_cast<uint32_t>(readlane(static_cast<int>(h1), wl));
            }
            if (r == KC) {
                bound = static_cast<int>(wv ^ 0x80000000u);
                break;
            }
            ck = writelane(ck, static_cast<int>(wv ^ 0x80000000u), r);
            cc = writelane(cc, static_cast<int>(~wlo), r);
            const bool won = lane == wl;
            if ((unknown >> wl) & 1u) {
                uint64_t n1, n2;
                top2(true, (static_cast<uint64_t>(wv) << 32) | wlo, n1, n2);
                h1 = won ? n1 : h1;
                h2 = won ? n2 : h2;
                unknown &= ~(uint64_t(1) << wl);
            } else {
                h1 = won ? h2 : h1;
                unknown |= uint64_t(1) << wl;
            }
        }
        if (lane < KC) {
            // Padding codes 0x7FFFFFFF: a published padding key never wins a
            // step, so any in-range position serves.
            const float4 c = spts[min(cc & 0x1FFF, CAP - 1)];
            WaveBest e;
            e.key = ck;
            e.index = cc >> 13;
            e.x = c.x;
            e.y = c.y;
            e.z = c.z;
            e.pad[0] = e.pad[1] = e.pad[2] = 0;
            cands[parity][wave * KC + lane] = e;
        }
        if (lane == 0) bounds[parity][wave] = bound;
        __syncthreads();
        const WaveBest mine = cands[parity][lane];
        int maxb_v = bounds[parity][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) maxb_v = max(maxb_v, bounds[parity][w]);
        parity ^= 1;
        int cmd = mine.key;
        const int cidx = mine.index;
        const float ccx = mine.x, ccy = mine.y, ccz = mine.z;
        // A later step of the run needs a key above every bound and above 0.
        // A taken candidate's key becomes its distance to itself, 0 -- or
        // stays +inf/-inf when a coordinate is not finite (the distance is
        // NaN) -- so with finite candidates none is taken twice in one run;
        // a non-finite candidate limits runs to one step.  One at -inf (a
        // NaN point, never sampled) does not: it can only be a run's first
        // step, after which no key is above 0.
        const bool odd = cmd >= 0 && !(isfinite(ccx) && isfinite(ccy) && isfinite(ccz));
        const int maxb = ballot(odd) ? INT_MAX : max(uniform(maxb_v), 0);
        // Steps of this run: at most `left`, counted in 32 bits.
        const int left = static_cast<int>(min<int64_t>(seg.cnt - step, int64_t(1) << 30));
        int taken = 0;
        // Step of this run at which each candidate was taken (-1: not
        // taken; at most once, see maxb); wave 0 stores the run's samples
        // after it.
        int when = -1;
        // One step with chosen key wv: the candidate holding it (smallest
        // index on a tie), its step recorded, the candidates updated, and
        // the tiles it may change queued for the next step.
        auto take = [&](int wv) {
            const uint64_t at_max = ballot(cmd == wv);
            int wl = static_cast<int>(__builtin_ctzll(at_max));
            if (__popcll(at_max) > 1) {  // ties (rare): the smallest index
                const int wneg = wave_max_i32_l63(cmd == wv ? -cidx : static_cast<int>(0x80000000u));
                wl = static_cast<int>(__builtin_ctzll(ballot(cmd == wv && -cidx == wneg)));
            }
            const float fx = i2f(readlane(f2i(ccx), wl));
            const float fy = i2f(readlane(f2i(ccy), wl));
            const float fz = i2f(readlane(f2i(ccz), wl));
            cmd = f2i(running_min(i2f(cmd), sqdist3(ccx, ccy, ccz, fx, fy, fz)));
            when = writelane(when, taken, wl);
            // Tiles whose box may hold a point nearer to the centroid than
            // the chosen (largest) running distance.  Per axis the gap is
            // f minus f clamped to the box: the rounded difference to the
            // nearer face (sign aside, which squaring drops), 0 inside.  A
            // non-finite centroid coordinate gives an infinite or NaN gap,
            // which selects no tile: such a centroid lowers no running
            // distance (every point's distance to it is +inf or NaN).
            const float M = i2f(wv);
            const float gx = fx - __builtin_amdgcn_fmed3f(fx, blo[0], bhi[0]);
            const float gy = fy - __builtin_amdgcn_fmed3f(fy, blo[1], bhi[1]);
            const float gz = fz - __builtin_amdgcn_fmed3f(fz, blo[2], bhi[2]);
            float lb = gx * gx;
            lb = lb + gy * gy;
            lb = lb + gz * gz;
            pend = static_cast<uint32_t>(ballot(lb < M));
            pfx = fx;
            pfy = fy;
            pfz = fz;
            ++taken;
        };
        take(wave_max_i32_l63(cmd));  // the first step after an exchange is exact
        while (taken < left) {
            const int wv = wave_max_i32_l63(cmd);
            if (pend) apply_pending();
            if (!(wv > maxb)) break;  // an unpublished point may tie or beat it
            take(wv);
        }
        if (pend) apply_pending();
        if (wave == 0 && when >= 0) {
            o[step + when] = seg.base + cidx;
            if (oc != nullptr) {
                oc[3 * (step + when)] = ccx;
                oc[3 * (step + when) + 1] = ccy;
                oc[3 * (step + when) + 2] = ccz;
            }
        }
        step += taken;
        publish(step - taken, step);
    }
}

// The boxes of a wave's PO tiles of 64 points (lane l holds point l of each
// tile, pcode 0x7FFFFFFF where it holds none), reduced together: the 6 PO
// minima (x, y, z and -x, -y, -z of every tile) are halved at each exchange
// 32, 16, ... lanes apart while their count is even (a lane keeps the half
// that its lane bit selects and folds in the partner's copy of it), and the
// 3 left are folded over the remaining exchanges.  Lane l then holds values
// 3 g .. 3 g + 2 of group g = l >> (5 - log2 PO): tile t's minima in group
// 2t, its negated maxima in group 2t + 1.  For PO = 8 that is 51 exchanges
// in place of 48 separate wave reductions.  Per lane, the box of tile
// lane % 16, or [+inf, +inf] where that tile does not exist or holds no
// point.
template <int V, int S>
__device__ __forceinline__ void fold_min(float* v, int lane) {
    if constexpr (S > 0) {
        if constexpr (V % 2 == 0 && V > 3) {
            constexpr int H = V / 2;
            const bool upper = (lane & S) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float send = upper ? v[i] : v[H + i];
                const float keep = upper ? v[H + i] : v[i];
                v[i] = fminf(keep, __shfl_xor(send, S, kWave));
            }
            fold_min<H, S / 2>(v, lane);
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) v[i] = fminf(v[i], __shfl_xor(v[i], S, kWave));
            fold_min<V, S / 2>(v, lane);
        }
    }
}

template <int PO>
__device__ __forceinline__ void tile_boxes(const float (&px)[PO], const float (&py)[PO],
                                           const float (&pz)[PO], const int (&pcode)[PO], int lane,
                                           float (&tlo)[3], float (&thi)[3]) {
    static_assert(PO == 1 || PO == 2 || PO == 4 || PO == 8, "tiles per wave: 1, 2, 4 or 8");
    float v[6 * PO];
#pragma unroll
    for (int k = 0; k < PO; ++k) {
        const bool valid = pcode[k] != 0x7FFFFFFF;
        v[6 * k] = valid ? px[k] : INFINITY;
        v[6 * k + 1] = valid ? py[k] : INFINITY;
        v[6 * k + 2] = valid ? pz[k] : INFINITY;
        v[6 * k + 3] = valid ? -px[k] : INFINITY;
        v[6 * k + 4] = valid ? -py[k] : INFINITY;
        v[6 * k + 5] = valid ? -pz[k] : INFINITY;
    }
    fold_min<6 * PO, kWave / 2>(v, lane);
    constexpr int shift = PO == 8 ? 2 : PO == 4 ? 3 : PO == 2 ? 4 : 5;
    const int t = lane & 15;
    const int src_lo = ((2 * t) << shift) & (kWave - 1);
    const int src_hi = ((2 * t + 1) << shift) & (kWave - 1);
    float lo[3], hi[3];
    bool has = t < PO;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        lo[a] = __shfl(v[a], src_lo, kWave);
        hi[a] = -__shfl(v[a], src_hi, kWave);
        has = has && lo[a] <= hi[a];
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        tlo[a] = has ? lo[a] : INFINITY;
        thi[a] = has ? hi[a] : INFINITY;
    }
}

// fps_lead_kernel<P>: the tiled FPS above with the step chain taken by one
// wave instead of all of them.
//
// Nine waves: eight followers (waves 0-7) hold the cloud's 64-point tiles
// (the setup, tiles and exchanges of fps_tiled_kernel with an even split, P
// tiles each) and the leader, wave 8, holds none.  After an exchange (every
// follower publishes its kLeadCand best points and its bound, the next
// largest running distance) the leader takes the exact steps of the run on
// its own over the 64 candidates: largest key, ties to the smallest index,
// the candidates updated with the points' own arithmetic, until the chosen
// key is no longer above every bound.  Its step loop is hand-scheduled
// gfx950 code (the chain is one wave's latency: wave maximum, ballot,
// readlanes, update), at raised priority.  Per step it publishes only the
// lane of the chosen candidate: four lanes are packed into a word, written
// into an LDS ring every 4 steps (and at the end of the run) with the chosen
// key of the block's first step, then the count of steps published.
//
// The followers follow the ring as it fills, a block of 4 steps at a time:
// lane l fetches the centroid of step l / 16 (this wave's copy of the
// candidates, by a lane permute) and tests tile l % 16's box against the
// block's first chosen key (keys only decrease, so it bounds the largest
// running distance of the block's later steps, and a tile it selects
// without need only takes a no-op minimum), so one ballot gives the tile
// masks of all four steps; then the masked tile updates.  Updates may be
// applied in any order before the next exchange, since running distances
// are minima.  At the end of a run follower 0 turns the ring's lanes into
// sample indices (64 per lane permute) and stores them, then publishes the
// progress words.  A run also ends after kLeadRing steps (the ring's size;
// the ring is rewritten only after the next exchange's barrier, which every
// follower reaches after reading it).  LDS ordering: one wave's LDS
// operations complete in issue order, so a follower that reads a published
// count (or the run's end) and then the ring sees the words the leader wrote
// before that count.
constexpr int kLeadWaves = 9;
constexpr int kLeadThreads = kLeadWaves * kWave;
constexpr int kLeadFollowers = 8;
constexpr int kLeadCand = 8;  // candidates per follower: the leader's 64 lanes
constexpr int kLeadRing = 256;

template <int P>
__global__ __launch_bounds__(kLeadThreads) void fps_lead_kernel(
    const float* __restrict__ xyz, const int64_t* __restrict__ ptr,
    const int64_t* __restrict__ out_ptr, const int64_t* __restrict__ starts,
    int64_t* __restrict__ out, int64_t N, int64_t npoint, int64_t start, int skip,
    uint64_t* __restrict__ progress, uint64_t tag, int64_t chunk, float* __restrict__ centres) {
    constexpr int NS = kLeadFollowers;  // followers; they also run the setup's sort
    constexpr int TS = NS * kWave;      // threads of the sort
    constexpr int NF = kLeadFollowers;
    constexpr int KC = kLeadCand;
    constexpr int CAP = P * TS;         // points per cloud at most
    constexpr int PO = P;               // tiles per follower
    constexpr int kCells = 4096;
    static_assert(KC * NF == kWave && KC + 1 <= kWave && P <= 16 && CAP <= 8192, "shape");
    static_assert(kCells % TS == 0, "cells per thread");
    // The sort's cell counts (then offsets), and the points by sorted
    // position (xyz, and the point's index in w), which the sort's scatter
    // writes directly.
    __shared__ int cell_count[kCells];
    __shared__ float4 spts[CAP];
    __shared__ float red[6][NS];
    __shared__ int wave_sum[NS];
    // The candidates: coordinates with the point index in w, and keys;
    // double-buffered by run parity, since followers read the table during
    // a run while followers that have finished it already extract the next.
    __shared__ float4 cand_pos[2][kWave];
    __shared__ int cand_key[2][kWave];
    __shared__ int bounds[NF];
    // Per 4 steps, a row of 64 words written by one conflict-free store of
    // the leader (lane l writes word l): the chosen candidate lanes (8 bits
    // per step, word 0) and the chosen key of the first of them (word 1);
    // the other words are padding.
    __shared__ uint32_t ring[kLeadRing / 4][kWave];
    // Word 0: steps published; word 1: the step at which the current run
    // ended (read together as one 8-byte value); words 2-63: padding that
    // the leader's other lanes write, so that its stores hit distinct
    // addresses.  Accessed with relaxed workgroup-scope atomics (plain LDS
    // reads and writes); compiler fences keep each wave's ring and mark
    // accesses in program order, which the LDS then keeps.
    __shared__ __align__(8) uint32_t marks[kWave];
    // Set by the leader at the end of a run when every sample is taken, in
    // the slot of the next iteration's parity: every wave reads it after the
    // next barrier, and the leader writes that slot again only two barriers
    // later.
    __shared__ int done[2];

    const Segment seg = segment_of(blockIdx.x, ptr, out_ptr, starts, N, npoint, start);
    if (seg.cnt <= 0) return;  // uniform over the workgroup, before any barrier
    const float* p = xyz + 3 * seg.in_lo;
    int64_t* o = out + seg.out_lo;
    const int n = static_cast<int>(seg.n);
    const int tid = threadIdx.x;
    const int wave = uniform(tid / kWave);  // known wave-uniform: scalar branches on it
    const int lane = tid % kWave;
    const bool leader = wave == NS;
    const bool sorter = wave < NS;
    const int fi = wave;  // follower number
    const bool follower = !leader;
    constexpr int kOutWave = 0;  // the first follower stores the samples
    const int far0 = static_cast<int>(seg.start);
    // With `centres` set, sample s's coordinates also go to
    // centres[3 (out_lo + s) ..], copied from the cloud.
    float* const oc = centres != nullptr ? centres + 3 * seg.out_lo : nullptr;
    if (wave == kOutWave && lane == 0) {
        o[0] = seg.base + far0;
        if (oc != nullptr && n > 0) {
            oc[0] = p[3 * far0];
            oc[1] = p[3 * far0 + 1];
            oc[2] = p[3 * far0 + 2];
        }
    }
    auto publish = [&](int64_t before, int64_t done_steps) {
        if (progress == nullptr || wave != kOutWave) return;
        const int64_t whole = (seg.cnt + chunk - 1) / chunk;
        const int64_t now = done_steps >= seg.cnt ? whole : done_steps / chunk;
        if (before >= 0 && now == (before >= seg.cnt ? whole : before / chunk)) return;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if (lane == 0)
            __hip_atomic_store(progress + blockIdx.x, tag + static_cast<uint64_t>(now),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (seg.cnt == 1 || n <= 0) {
        publish(-1, seg.cnt);
        return;
    }

    // ---- setup: the sort by waves 0-7
    if (sorter)
        for (int c = tid; c < kCells; c += TS) cell_count[c] = 0;
    // The cloud's coordinates, staged through the LDS (in the space that the
    // sorted points take later) by coalesced loads; sorting thread t then
    // takes points t, t + TS, ..., t + (P - 1) TS.
    float* const stage = reinterpret_cast<float*>(spts);
    static_assert(3 * CAP * sizeof(float) <= CAP * sizeof(float4), "the staged cloud fits");
    if (sorter) {
        float raw[3 * P];
#pragma unroll
        for (int m = 0; m < 3 * P; ++m) {
            const int f = tid + m * TS;
            raw[m] = f < 3 * n ? p[f] : 0.f;
        }
#pragma unroll
        for (int m = 0; m < 3 * P; ++m) {
            const int f = tid + m * TS;
            if (f < 3 * n) stage[f] = raw[m];
        }
    }
    if (tid == 0) {
        marks[0] = marks[1] = 1u;
        done[0] = done[1] = 0;
    }
    __syncthreads();  // staged coordinates, cleared counters, marks
    float lx[P], ly[P], lz[P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int j = min(tid + k * TS, n - 1);
        lx[k] = sorter ? stage[3 * j] : 0.f;
        ly[k] = sorter ? stage[3 * j + 1] : 0.f;
        lz[k] = sorter ? stage[3 * j + 2] : 0.f;
    }
    if (sorter) {
        // Minima of x, y, z and of -x, -y, -z, folded together: the minima
        // end in lane 0, the negated maxima in lane 32.
        float v[6];
        v[0] = v[1] = v[2] = v[3] = v[4] = v[5] = INFINITY;
#pragma unroll
        for (int k = 0; k < P; ++k) {
            v[0] = fminf(v[0], lx[k]); v[3] = fminf(v[3], -lx[k]);
            v[1] = fminf(v[1], ly[k]); v[4] = fminf(v[4], -ly[k]);
            v[2] = fminf(v[2], lz[k]); v[5] = fminf(v[5], -lz[k]);
        }
        fold_min<6, kWave / 2>(v, lane);
        if (lane == 0) {
#pragma unroll
            for (int a = 0; a < 3; ++a) red[a][wave] = v[a];
        }
        if (lane == kWave / 2) {
#pragma unroll
            for (int a = 0; a < 3; ++a) red[3 + a][wave] = -v[a];
        }
    }
    __syncthreads();  // box partials
    float lo[3], scale[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        float mn = red[a][0], mx = red[3 + a][0];
#pragma unroll
        for (int w = 1; w < NS; ++w) {
            mn = fminf(mn, red[a][w]);
            mx = fmaxf(mx, red[3 + a][w]);
        }
        lo[a] = mn;
        const float ext = mx - mn;
        scale[a] = (ext > 0.f && ext < INFINITY) ? 16.f / ext : 0.f;
    }
    int cell[P], rank[P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const float c3[3] = {lx[k], ly[k], lz[k]};
        uint32_t key = 0;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float f = fminf(fmaxf((c3[a] - lo[a]) * scale[a], 0.f), 15.f);
            const uint32_t q = static_cast<uint32_t>(f);
#pragma unroll
            for (int b = 0; b < 4; ++b) key |= ((q >> b) & 1u) << (3 * b + a);
        }
        cell[k] = static_cast<int>(key);
        rank[k] = (sorter && tid + k * TS < n) ? atomicAdd(&cell_count[key], 1) : 0;
    }
    __syncthreads();  // counts complete
    {
        constexpr int CPT = kCells / TS;
        int run = 0;
        if (sorter) {
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
                const int v = cell_count[tid * CPT + c];
                cell_count[tid * CPT + c] = run;
                run += v;
            }
        }
        int incl = run;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int up = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += up;
        }
        if (sorter && lane == kWave - 1) wave_sum[wave] = incl;
        __syncthreads();  // wave totals
        int before = incl - run;
        for (int w = 0; w < wave && w < NS; ++w) before += wave_sum[w];
        if (sorter) {
#pragma unroll
            for (int c = 0; c < CPT; ++c) cell_count[tid * CPT + c] += before;
        }
    }
    __syncthreads();  // offsets complete
    if (sorter) {
#pragma unroll
        for (int k = 0; k < P; ++k)
            if (tid + k * TS < n)
                spts[cell_count[cell[k]] + rank[k]] = make_float4(lx[k], ly[k], lz[k], i2f(tid + k * TS));
    }
    __syncthreads();  // permutation complete

    // ---- followers: their points, indices, running distances and boxes
    const int my_tiles = follower ? PO : 0;
    const int tile0 = fi * PO;
    float px[PO], py[PO], pz[PO], md[PO];
    int pcode[PO];
#pragma unroll
    for (int k = 0; k < PO; ++k) {
        px[k] = py[k] = pz[k] = 0.f;
        pcode[k] = 0x7FFFFFFF;
        md[k] = -INFINITY;
    }
    if (follower) {
        float cx, cy, cz;
        {
            const int f = min(max(far0, 0), n - 1);
            cx = p[3 * f];
            cy = p[3 * f + 1];
            cz = p[3 * f + 2];
        }
#pragma unroll
        for (int k = 0; k < PO; ++k) {
            const int q = (tile0 + k) * kWave + lane;  // < NF PO kWave = CAP
            const bool valid = k < my_tiles && q < n;
            const float4 s = spts[q];
            px[k] = valid ? s.x : 0.f;
            py[k] = valid ? s.y : 0.f;
            pz[k] = valid ? s.z : 0.f;
            pcode[k] = valid ? (f2i(s.w) << 13) | q : 0x7FFFFFFF;
            md[k] = !valid ? -INFINITY : initial_running(skip, px[k], py[k], pz[k]);
            md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], cx, cy, cz));
        }
    }
    // Per lane, the box of tile lane % 16 ([+inf, +inf] where that tile does
    // not exist or holds no point, which no test selects), and the shift of
    // step lane / 16's byte in a block's lanes.
    static_assert(PO <= 16, "a follower holds at most 16 tiles");
    float tlo[3], thi[3];
    tile_boxes<PO>(px, py, pz, pcode, lane, tlo, thi);
    const uint32_t lane_shift = 8u * static_cast<uint32_t>(lane >> 4);

    if (leader) __builtin_amdgcn_s_setprio(3);
    int64_t step = 1;
    int parity = 0;
    for (;;) {
        if (follower) {
            // Exchange: this follower's KC best points and its bound (the
            // (KC+1)-th), as in fps_tiled_kernel.
            auto top2 = [&](bool limited, uint64_t lim, uint64_t& a1, uint64_t& a2) {
                a1 = 0;
                a2 = 0;
#pragma unroll
                for (int k = 0; k < PO; ++k) {
                    if (k >= my_tiles) break;  // wave-uniform
                    const uint64_t key =
                        (static_cast<uint64_t>(static_cast<uint32_t>(f2i(md[k])) ^ 0x80000000u) << 32) |
                        static_cast<uint32_t>(~pcode[k]);
                    const bool below = !limited || key < lim;
                    const bool first = below && key > a1;
                    const bool second = below && !first && key > a2;
                    a2 = first ? a1 : (second ? key : a2);
                    a1 = first ? key : a1;
                }
            };
            uint64_t h1, h2;
            top2(false, 0, h1, h2);
            uint64_t unknown = 0;
            int ck = 0, cc = 0x7FFFFFFF;
            int bound = 0;
#pragma unroll
            for (int r = 0; r <= KC; ++r) {
                const uint32_t hh = static_cast<uint32_t>(h1 >> 32);
                const uint32_t wv = wave_max_u32_l63(hh);
                const uint64_t at = ballot(hh == wv);
                int wl = static_cast<int>(__builtin_ctzll(at));
                uint32_t wlo;
                if (__popcll(at) > 1) {
                    wlo = wave_max_u32_l63(hh == wv ? static_cast<uint32_t>(h1) : 0u);
                    wl = static_cast<int>(__builtin_ctzll(ballot(hh == wv && static_cast<uint32_t>(h1) == wlo)));
                } else {
                    wlo = static_cast<uint32_t>(readlane(static_cast<int>(h1), wl));
                }
                if (r == KC) {
                    bound = static_cast<int>(wv ^ 0x80000000u);
                    break;
                }
                ck = writelane(ck, static_cast<int>(wv ^ 0x80000000u), r);
                cc = writelane(cc, static_cast<int>(~wlo), r);
                const bool won = lane == wl;
                if ((unknown >> wl) & 1u) {
                    uint64_t n1, n2;
                    top2(true, (static_cast<uint64_t>(wv) << 32) | wlo, n1, n2);
                    h1 = won ? n1 : h1;
                    h2 = won ? n2 : h2;
                    unknown &= ~(uint64_t(1) << wl);
                } else {
                    h1 = won ? h2 : h1;
                    unknown |= uint64_t(1) << wl;
                }
            }
            if (lane < KC) {
                // Padding codes 0x7FFFFFFF: a published padding key never wins a
                // step, so any in-range position serves.
                const float4 c = spts[min(cc & 0x1FFF, CAP - 1)];
                cand_pos[parity][fi * KC + lane] = make_float4(c.x, c.y, c.z, i2f(cc >> 13));
                cand_key[parity][fi * KC + lane] = ck;
            }
            if (lane == 0) bounds[fi] = bound;
        }
        __syncthreads();  // candidates and bounds published; the last run applied
        if (done[parity]) break;  // uniform: written by the leader before this barrier
        const int64_t run_start = step;
        const float4 mine = cand_pos[parity][lane];  // w: the point index
        if (leader) {
            int maxb_v = bounds[0];
#pragma unroll
            for (int w = 1; w < NF; ++w) maxb_v = max(maxb_v, bounds[w]);
            int cmd = cand_key[parity][lane];
            const int cidx = f2i(mine.w);
            const float ccx = mine.x, ccy = mine.y, ccz = mine.z;
            // A later step of the run needs a key above every bound and
            // above 0.  A taken candidate's key becomes its distance to
            // itself, 0 -- or stays +inf/-inf when a coordinate is not
            // finite (the distance is NaN) -- so with finite candidates none
            // is taken twice in one run; a non-finite candidate limits runs
            // to one step.  One at -inf (a NaN point, never sampled) does
            // not: it can only be a run's first step, after which no key is
            // above 0.
            const bool odd = cmd >= 0 && !(isfinite(ccx) && isfinite(ccy) && isfinite(ccz));
            const int maxb = ballot(odd) ? INT_MAX : max(uniform(maxb_v), 0);
            const int64_t rest = seg.cnt - step;
            int rem = uniform(static_cast<int>(rest < kLeadRing ? rest : kLeadRing));  // steps left
            const uint32_t base = static_cast<uint32_t>(run_start);
            int taken = 0;
            // The candidates' LDS loads complete here, so that the loop's
            // waits never cover its own ring stores.
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            int wv = wave_max_i32_l63(cmd);  // the first step after an exchange is exact
            int block_key = wv;              // chosen key of the block's first step
            const int nidx = -cidx;
            const int imin = INT_MIN;
            uint32_t packed = 0, sh = 0;
            for (;;) {
                // Up to 4 steps (one block), as hand-scheduled gfx950 code:
                // the chosen candidate (the lowest lane holding the largest
                // key wv; on a tie, the smallest index by a second wave
                // maximum of -index), its coordinates by readlane, every
                // candidate's key lowered to its distance to them, the lane
                // packed into `packed`, then the next step's largest key by
                // the DPP reduction of wave_max_i32_l63.  It stops after 4
                // steps (st = 0, wv the next step's key), or when the run
                // ends (st = 1): no steps left, or the next key is not above
                // every bound.  The s_nop's give the wait states a DPP read
                // of a VALU result (2), a readlane of a DPP result (1) and a
                // VALU read of a readlane's SGPR (2) need.
                int st, wl, t, fx, fy, fz;
                uint64_t tt;
                float t0, t1, t2;
                int m;
                asm volatile(
                    "s_nop 1\n\t"
                    "s_mov_b32 %[sh], 0\n\t"
                    "s_mov_b32 %[pk], 0\n"
                    "1:\n\t"
                    "v_cmp_eq_u32_e32 vcc, %[wv], %[cmd]\n\t"
                    "s_ff1_i32_b64 %[wl], vcc\n\t"
                    "s_bcnt1_i32_b64 %[t], vcc\n\t"
                    "s_cmp_gt_u32 %[t], 1\n\t"
                    "s_cbranch_scc1 5f\n"
                    "2:\n\t"
                    "v_readlane_b32 %[fx], %[cx], %[wl]\n\t"
                    "v_readlane_b32 %[fy], %[cy], %[wl]\n\t"
                    "v_readlane_b32 %[fz], %[cz], %[wl]\n\t"
                    "s_lshl_b32 %[t], %[wl], %[sh]\n\t"
                    "v_subrev_f32_e32 %[t0], %[fx], %[cx]\n\t"
                    "v_subrev_f32_e32 %[t1], %[fy], %[cy]\n\t"
                    "v_subrev_f32_e32 %[t2], %[fz], %[cz]\n\t"
                    "s_or_b32 %[pk], %[pk], %[t]\n\t"
                    "v_mul_f32_e32 %[t0], %[t0], %[t0]\n\t"
                    "v_mul_f32_e32 %[t1], %[t1], %[t1]\n\t"
                    "v_mul_f32_e32 %[t2], %[t2], %[t2]\n\t"
                    "v_add_f32_e32 %[t0], %[t0], %[t1]\n\t"
                    "s_add_u32 %[sh], %[sh], 8\n\t"
                    "v_add_f32_e32 %[t0], %[t0], %[t2]\n\t"
                    "s_sub_u32 %[rem], %[rem], 1\n\t"
                    "v_min_f32_e32 %[cmd], %[cmd], %[t0]\n\t"
                    "s_cmp_eq_u32 %[rem], 0\n\t"
                    "s_cbranch_scc1 8f\n\t"
                    "v_max_i32_dpp %[m], %[cmd], %[cmd] quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_mirror row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
                    "s_nop 0\n\t"
                    "v_readlane_b32 %[wv], %[m], 63\n\t"
                    "s_cmp_le_i32 %[wv], %[maxb]\n\t"
                    "s_cbranch_scc1 8f\n\t"
                    "s_cmp_lt_u32 %[sh], 32\n\t"
                    "s_cbranch_scc1 1b\n\t"
                    "s_mov_b32 %[st], 0\n\t"
                    "s_branch 9f\n"
                    "5:\n\t"
                    "v_cndmask_b32_e32 %[m], %[imin], %[nidx], vcc\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_mirror row_mask:0xf bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
                    "s_nop 1\n\t"
                    "v_max_i32_dpp %[m], %[m], %[m] row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
                    "s_nop 0\n\t"
                    "v_readlane_b32 %[t], %[m], 63\n\t"
                    "s_nop 1\n\t"
                    "v_cmp_eq_u32_e64 %[tt], %[t], %[nidx]\n\t"
                    "s_and_b64 vcc, vcc, %[tt]\n\t"
                    "s_ff1_i32_b64 %[wl], vcc\n\t"
                    "s_branch 2b\n"
                    "8:\n\t"
                    "s_mov_b32 %[st], 1\n"
                    "9:\n\t"
                    "s_nop 1"
                    : [cmd] "+v"(cmd), [wv] "+s"(wv), [rem] "+s"(rem), [pk] "=&s"(packed),
                      [sh] "=&s"(sh), [st] "=&s"(st), [wl] "=&s"(wl), [t] "=&s"(t),
                      [fx] "=&s"(fx), [fy] "=&s"(fy), [fz] "=&s"(fz), [tt] "=&s"(tt),
                      [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [m] "=&v"(m)
                    : [cx] "v"(ccx), [cy] "v"(ccy), [cz] "v"(ccz), [nidx] "v"(nidx),
                      [imin] "v"(imin), [maxb] "s"(maxb)
                    : "vcc", "scc");
                taken += static_cast<int>(sh >> 3);
                if (st != 0) break;
                // A full block: its row, then the count.  Lane l writes word l
                // (distinct addresses, no conflicts).
                ring[(taken >> 2) - 1][lane] = lane == 0 ? packed : static_cast<uint32_t>(block_key);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the row is issued before the count
                __hip_atomic_store(&marks[lane == 0 ? 0 : lane + (lane == 1)], base + taken,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                block_key = wv;
            }
            // The last block's row (full or partial).
            ring[(taken - 1) >> 2][lane] = lane == 0 ? packed : static_cast<uint32_t>(block_key);
            step += taken;
            done[parity ^ 1] = step >= seg.cnt ? 1 : 0;  // read by every wave after the next barrier
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            // Count and end of the run (lanes 0 and 1 of one store: a follower
            // never sees an end beyond the count it reads with it).
            __hip_atomic_store(&marks[lane], lane < 2 ? base + taken : 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        } else if (follower) {
            // A block of up to 4 published steps, all box tests at once: lane
            // l takes tile l % 16 (a follower holds at most 16) and step
            // l / 16 of the block, whose centroid it fetches from this wave's
            // copy of the candidates by a lane permute; one ballot gives the
            // tile masks of the four steps (16 bits each), tested against
            // the block's first chosen key.  Then the masked updates (minima,
            // so their order does not matter), the centroid of step j read
            // from lane 16 j.
            auto block = [&](uint32_t lanes4, float M1, int cnt) {
                const int wl = static_cast<int>((lanes4 >> lane_shift) & 63u);
                const float cx = i2f(__builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.x)));
                const float cy = i2f(__builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.y)));
                const float cz = i2f(__builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.z)));
                const float gx = cx - __builtin_amdgcn_fmed3f(cx, tlo[0], thi[0]);
                const float gy = cy - __builtin_amdgcn_fmed3f(cy, tlo[1], thi[1]);
                const float gz = cz - __builtin_amdgcn_fmed3f(cz, tlo[2], thi[2]);
                float lb = gx * gx;
                lb = lb + gy * gy;
                lb = lb + gz * gz;
                uint64_t pend = ballot(lb < M1);
                if (cnt < 4) pend &= (uint64_t(1) << (16 * cnt)) - 1;
                if (pend == 0) return;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t pj = static_cast<uint32_t>(pend >> (16 * j)) & 0xFFFFu;
                    if (pj == 0) continue;
                    const float fx = i2f(readlane(f2i(cx), 16 * j));
                    const float fy = i2f(readlane(f2i(cy), 16 * j));
                    const float fz = i2f(readlane(f2i(cz), 16 * j));
#pragma unroll
                    for (int k = 0; k < PO; ++k)
                        if ((pj >> k) & 1u)
                            md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], fx, fy, fz));
                }
            };
            int a = 0;  // steps of this run applied (a multiple of 4 until the run ends)
            for (;;) {
                const uint64_t m = __hip_atomic_load(reinterpret_cast<uint64_t*>(marks), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);  // ring reads after the mark
                const int pub = uniform(static_cast<int>(m)) - static_cast<int>(run_start);
                const int end = uniform(static_cast<int>(m >> 32)) - static_cast<int>(run_start);
                // Whole blocks (counts published during a run are multiples of 4).
                while (a + 4 <= pub) {
                    const uint32_t* row = ring[a >> 2];
                    const uint32_t lanes4 = static_cast<uint32_t>(uniform(static_cast<int>(row[0])));
                    const float M1 = i2f(uniform(static_cast<int>(row[1])));
                    block(lanes4, M1, 4);
                    a += 4;
                }
                if (end > 0 && pub >= end) {
                    // The run's last, partial block.
                    if (a < end) {
                        const uint32_t* row = ring[a >> 2];
                        const uint32_t lanes4 = static_cast<uint32_t>(uniform(static_cast<int>(row[0])));
                        const float M1 = i2f(uniform(static_cast<int>(row[1])));
                        block(lanes4, M1, end - a);
                        a = end;
                    }
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (wave == kOutWave) {
                // The run's samples: lane i of a batch takes step c0 + i, its
                // chosen lane from the ring's bytes and that candidate's index
                // by a lane permute (all lanes take part).
                for (int c0 = 0; c0 < a; c0 += kWave) {
                    const int si = min(c0 + lane, a - 1);
                    const int wl = reinterpret_cast<const uint8_t*>(ring[si >> 2])[si & 3];
                    const int idx = __builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.w));
                    if (c0 + lane < a) o[run_start + c0 + lane] = seg.base + idx;
                    if (oc != nullptr) {
                        const int x = __builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.x));
                        const int y = __builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.y));
                        const int z = __builtin_amdgcn_ds_bpermute(wl << 2, f2i(mine.z));
                        if (c0 + lane < a) {
                            float* c = oc + 3 * (run_start + c0 + lane);
                            c[0] = i2f(x);
                            c[1] = i2f(y);
                            c[2] = i2f(z);
                        }
                    }
                }
            }
            step = run_start + a;
            publish(run_start, step);
        }
        parity ^= 1;
    }
}

template <int T>
__global__ __launch_bounds__(T) void fps_global_kernel(const float* __restrict__ xyz,
                                                       const int64_t* __restrict__ ptr,
                                                       const int64_t* __restrict__ out_ptr,
                                                       const int64_t* __restrict__ starts,
                                                       int64_t* __restrict__ out,
                                                       float* __restrict__ scratch, int64_t N,
                                                       int64_t npoint, int64_t start, int skip) {
    constexpr int NW = T / kWave;
    __shared__ int2 slots[2][NW];
    const Segment seg = segment_of(blockIdx.x, ptr, out_ptr, starts, N, npoint, start);
    if (seg.cnt <= 0) return;
    const float* p = xyz + 3 * seg.in_lo;
    float* md = scratch + seg.in_lo;
    int64_t* o = out + seg.out_lo;
    const int64_t n = seg.n;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;

    for (int64_t j = tid; j < n; j += T) {
        md[j] = initial_running(skip, p[3 * j], p[3 * j + 1], p[3 * j + 2]);
    }
    int64_t far = seg.start;
    for (int64_t step = 0; step < seg.cnt; ++step) {
        if (tid == 0) o[step] = seg.base + far;
        if (step + 1 == seg.cnt) break;
        const float cx = p[3 * far], cy = p[3 * far + 1], cz = p[3 * far + 2];
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int64_t j = tid; j < n; j += T) {
            const float d = sqdist3(p[3 * j], p[3 * j + 1], p[3 * j + 2], cx, cy, cz);
            const float m = fminf(md[j], d);
            md[j] = m;
            if (m > bv) {
                bv = m;
                bi = static_cast<int>(j);
            }
        }
        const float wv = wave_max(bv);
        const int wi = wave_min(bv == wv ? bi : INT_MAX);
        int2* buf = slots[step & 1];
        if (lane == 0) buf[wave] = make_int2(f2i(wv), wi);
        __syncthreads();
        const int win = block_argmax<NW>(buf);
        far = (win == INT_MAX) ? 0 : win;
    }
}
// ------------------------------------------------------------ large cloud
//
// Constants of the persistent large-cloud kernel below: one cloud over G <=
// kLargeMaxGrid co-resident workgroups (at most one per CU), cooperative
// launch; workgroup g owns points [g*chunk, g*chunk+chunk), thread t holds P
// consecutive ones in VGPRs.  Indices travel in 21 bits of the records.
// Polls are bounded: after kSpinLimit attempts (or when another workgroup
// has given up) the kernel raises the status word, workgroup 0 writes -1 to
// every output slot it has not written, and every workgroup returns, so no
// launch can hang and no slot is left unwritten.
constexpr int kLargeIdxBits = 21;
constexpr uint32_t kLargeIdxMask = (1u << kLargeIdxBits) - 1u;
constexpr int64_t kLargeMaxN = int64_t(1) << kLargeIdxBits;
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr int kLargeThreads = 256;
constexpr int kLargeMaxGrid = kLargeThreads;  // one polled record per thread (SoA stride)
// Every record is written to kLargeReplicas copies, and workgroup g polls copy
// g % kLargeReplicas, so each copy's cache lines are read by 1/kLargeReplicas
// of the pollers instead of all of them (one shared copy measured 4.8 us per
// exchange-free step on 1M points, 8 copies 3.6 us).
constexpr int kLargeReplicas = 8;

// True when this poller must stop: `limit` polls done, or another workgroup
// has already given up (checked every 64 polls).  Raises the shared status
// word.  Checked before each read, so limit 0 gives up at the first poll
// (the host-forced failure path of the tests; every wave still exits).
__device__ __forceinline__ bool poll_give_up(uint32_t* status, uint32_t spins, uint32_t limit) {
    if (spins >= limit ||
        ((spins & 63u) == 63u &&
         __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
        __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    return false;
}

// Lazy steps over an exchange's candidates (x, y, z and key bits in xyzk,
// the point index in idx, `count` of them), by one wave: lane l holds
// candidates l, l + 64, ... (CS per lane).  Each step takes the largest key
// (smallest index on ties) -- always for the first step, afterwards only
// while it is above `bound` -- updates the candidates' keys with the
// points' own arithmetic and calls on_step(centroid, index); at most
// max_steps steps.  Every wave of a workgroup runs the same steps on the
// same data.
template <int CS, typename OnStep>
__device__ __forceinline__ void lazy_candidate_run(const float4* xyzk, const uint32_t* idx, int count,
                                                   int bound, int lane, int max_steps, OnStep on_step) {
    float kx[CS], ky[CS], kz[CS];
    int kkey[CS];
    uint32_t knot[CS];  // ~index: larger for a smaller index
#pragma unroll
    for (int s = 0; s < CS; ++s) {
        const int id = s * kWave + lane;
        const float4 v = id < count ? xyzk[id] : make_float4(0.f, 0.f, 0.f, i2f(static_cast<int>(0x80000000u)));
        kx[s] = v.x;
        ky[s] = v.y;
        kz[s] = v.z;
        kkey[s] = f2i(v.w);
        knot[s] = ~(id < count ? idx[id] : 0xFFFFFFFFu);
    }
    for (int taken = 0; taken < max_steps; ++taken) {
        // This lane's best as one 64-bit value (key, then ~index), and its slot.
        uint64_t bk = 0;
        int bs = 0;
#pragma unroll
        for (int s = 0; s < CS; ++s) {
            const uint64_t k64 = (static_cast<uint64_t>(static_cast<uint32_t>(kkey[s]) ^ 0x80000000u) << 32) | knot[s];
            const bool better = k64 > bk;
            bk = better ? k64 : bk;
            bs = better ? s : bs;
        }
        const uint32_t hh = static_cast<uint32_t>(bk >> 32);
        const uint32_t wv = wave_max_u32_l63(hh);
        const uint64_t at = ballot(hh == wv);
        int wl = static_cast<int>(__builtin_ctzll(at));
        if (__popcll(at) > 1) {  // equal keys: the smallest index
            const uint32_t wlo = wave_max_u32_l63(hh == wv ? static_cast<uint32_t>(bk) : 0u);
            wl = static_cast<int>(__builtin_ctzll(ballot(hh == wv && static_cast<uint32_t>(bk) == wlo)));
        }
        const int key = static_cast<int>(wv ^ 0x80000000u);
        if (taken > 0 && !(key > bound)) break;  // an unpublished point may tie or beat it
        const int id = readlane(bs, wl) * kWave + wl;
        const float4 c = xyzk[id];
#pragma unroll
        for (int s = 0; s < CS; ++s)
            kkey[s] = f2i(running_min(i2f(kkey[s]), sqdist3(kx[s], ky[s], kz[s], c.x, c.y, c.z)));
        on_step(c, idx[id]);
    }
}

// The candidates a run can take: after the first step (which takes the
// largest key) a candidate is taken only while its key is above every
// bound, and keys only decrease, so those at or below `bound` that do not
// hold the largest key are dropped.  The live ones (at most kLazyLive) are
// copied, in candidate order, to live_xyzk / live_idx; returns their count
// (more than kLazyLive: the run keeps all candidates).
constexpr int kLazyLive = 2 * kWave;
template <int CW>
__device__ __forceinline__ int lazy_live_candidates(const float4* xyzk, const uint32_t* idx, int bound,
                                                    int lane, float4* live_xyzk, uint32_t* live_idx) {
    int maxkey = static_cast<int>(0x80000000u);
#pragma unroll
    for (int s = 0; s < CW; ++s) maxkey = max(maxkey, f2i(xyzk[s * kWave + lane].w));
    maxkey = wave_max_i32_l63(maxkey);
    int nlive = 0;
#pragma unroll
    for (int s = 0; s < CW; ++s) {
        const float4 v = xyzk[s * kWave + lane];
        const int key = f2i(v.w);
        const bool live = key > bound || key == maxkey;
        const uint64_t m = ballot(live);
        const int pos = nlive + lanes_below(m);
        if (live && pos < kLazyLive) {
            live_xyzk[pos] = v;
            live_idx[pos] = idx[s * kWave + lane];
        }
        nlive += __popcll(m);
    }
    return nlive;
}

// Runs the lazy steps over the live candidates when they fit 2 per lane,
// else over all CW per lane.
template <int CW, typename OnStep>
__device__ __forceinline__ void lazy_steps(const float4* xyzk, const uint32_t* idx, int bound, int lane,
                                           float4* live_xyzk, uint32_t* live_idx, int max_steps,
                                           OnStep on_step) {
    const int nlive = lazy_live_candidates<CW>(xyzk, idx, bound, lane, live_xyzk, live_idx);
    if (nlive <= kWave)
        lazy_candidate_run<1>(live_xyzk, live_idx, nlive, bound, lane, max_steps, on_step);
    else if (nlive <= kLazyLive)
        lazy_candidate_run<2>(live_xyzk, live_idx, nlive, bound, lane, max_steps, on_step);
    else
        lazy_candidate_run<CW>(xyzk, idx, CW * kWave, bound, lane, max_steps, on_step);
}

// fps_lazy_kernel<P,T>: the large-cloud FPS with an exchange every few steps
// instead of every step.  At an exchange every wave publishes its kLazyCand
// best points (running distance, index, xyz; largest distance first, smaller
// index first on ties) and the (kLazyCand+1)-th largest running distance of
// its points, its bound.  Every workgroup then reads all candidates and, on
// identical data, runs the same sequence of steps over the candidates alone:
// the first step after an exchange is exact (each wave's first candidate is
// its maximum, so the best candidate is the global maximum), and a later step
// is exact while the best candidate's distance is strictly above every
// bound, since an unpublished point's running distance is at most its wave's
// bound (distances only decrease).  Candidate distances are updated with the
// same arithmetic as the points.  The centroids chosen since the last
// exchange are applied to every workgroup's own points at the next exchange
// (a running minimum does not depend on the order).  Records carry a tag per
// 64-bit word and are double-buffered by exchange parity, in kLargeReplicas
// copies; polls are bounded.  Record of wave w (structure of arrays, stride
// kLazyMaxWaves words):
//   word 4c   = key << 32 | tag << 21 | idx   (candidate c: running distance
//                                              bits, 21-bit global index)
//   word 4c+1 = x_bits << 32 | tag,  4c+2 = y_bits << 32 | tag,
//   word 4c+3 = z_bits << 32 | tag,  last = bound_bits << 32 | tag
// The tag (exchange number mod 1024, bit 10 set) lets a reader tell a record
// of this exchange from one two exchanges back.
constexpr int kLazyCand = 1;          // candidates per wave
constexpr int kLazyMaxPending = 64;   // steps between exchanges at most
constexpr int kLazyRecWords = 4 * kLazyCand + 1;
constexpr int kLazyMaxWaves = kLargeMaxGrid * (kLargeThreads / kWave);
constexpr int64_t kLazyCopyWords = static_cast<int64_t>(kLazyRecWords) * kLazyMaxWaves;

template <int P, int T>
__global__ __launch_bounds__(T) void fps_lazy_kernel(
    const float* __restrict__ xyz, int64_t* __restrict__ out, uint64_t* __restrict__ records,
    uint32_t* __restrict__ status, int N, int64_t npoint, int start, int skip, int chunk,
    uint32_t spin_limit) {
    constexpr int NW = T / kWave;
    static_assert(NW <= 8 && P <= 32, "shape");
    constexpr int RPT = kLazyMaxWaves / T;  // records read per thread at most
    constexpr int CPT = RPT * kLazyCand;    // candidates held per thread at most
    constexpr int CW = kLazyMaxWaves * kLazyCand / kWave;  // candidates per lane in a run
    // The exchange's candidates (record r's candidate c at r * kLazyCand + c):
    // x, y, z and the key's bits; the index.
    __shared__ float4 cand_xyzk[kLazyMaxWaves * kLazyCand];
    __shared__ uint32_t cand_idx[kLazyMaxWaves * kLazyCand];
    __shared__ float4 live_xyzk[NW][kLazyLive];  // per wave: the run's live candidates
    __shared__ uint32_t live_idx[NW][kLazyLive];
    __shared__ int wave_bound[NW];
    __shared__ int abort_flag;

    const int G = gridDim.x;
    const int waves = G * NW;  // records per exchange
    const int g = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int lo = g * chunk;
    const int n = max(0, min(chunk, N - lo));
    const float* p = xyz + 3 * static_cast<int64_t>(lo);

    // Small P: one spare element so that px[os] is an indexed move, not a
    // select chain; P = 32 already is (and 33 floats would not stay in VGPRs).
    constexpr int PA = P <= 8 ? P + 1 : P;
    float px[PA], py[PA], pz[PA], md[P];
#pragma unroll
    for (int k = 0; k < PA; ++k) px[k] = py[k] = pz[k] = 0.f;
    if (n > 0) {
#pragma unroll
        for (int k = 0; k < P; ++k) {
            const int jj = min(tid * P + k, n - 1);
            px[k] = p[3 * jj];
            py[k] = p[3 * jj + 1];
            pz[k] = p[3 * jj + 2];
        }
    }
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int j = tid * P + k;
        const bool valid = j < n;
        px[k] = valid ? px[k] : 0.f;
        py[k] = valid ? py[k] : 0.f;
        pz[k] = valid ? pz[k] : 0.f;
        md[k] = !valid ? -INFINITY : initial_running(skip, px[k], py[k], pz[k]);
    }
    if (tid == 0) {
        abort_flag = 0;
        if (g == 0) out[0] = start;
    }
    {
        const float sx = xyz[3 * static_cast<int64_t>(start)];
        const float sy = xyz[3 * static_cast<int64_t>(start) + 1];
        const float sz = xyz[3 * static_cast<int64_t>(start) + 2];
#pragma unroll
        for (int k = 0; k < P; ++k) md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], sx, sy, sz));
    }
    int64_t step = 1;
    for (uint32_t exch = 0; step < npoint; ++exch) {
        __syncthreads();  // every wave is past the last run's reads of the candidates

        // This wave's kLazyCand best points and its bound, by repeated wave
        // maxima (first lane, then first slot, holding the maximum: the
        // smallest index).
        const int par = static_cast<int>(exch & 1);
        const uint32_t tag = (exch & 0x3FFu) | 0x400u;
        const int gw = g * NW + wave;
        uint64_t words[kLazyRecWords];
        uint32_t taken = 0;
#pragma unroll
        for (int r = 0; r <= kLazyCand; ++r) {
            int lm = static_cast<int>(0x80000000u), ls = 0;
#pragma unroll
            for (int k = P - 1; k >= 0; --k) {
                const int v = ((taken >> k) & 1u) ? static_cast<int>(0x80000000u) : f2i(md[k]);
                ls = v >= lm ? k : ls;
                lm = max(lm, v);
            }
            const int wv = wave_max_i32_l63(lm);
            const int wl = static_cast<int>(__builtin_ctzll(ballot(lm == wv)));
            const int os = readlane(ls, wl);
            if (r == kLazyCand) {
                words[4 * kLazyCand] = (static_cast<uint64_t>(static_cast<uint32_t>(wv)) << 32) | tag;
                break;
            }
            const uint32_t gidx = static_cast<uint32_t>(lo + (wave * kWave + wl) * P + os);
            const uint32_t bx = static_cast<uint32_t>(readlane(f2i(px[os]), wl));
            const uint32_t by = static_cast<uint32_t>(readlane(f2i(py[os]), wl));
            const uint32_t bz = static_cast<uint32_t>(readlane(f2i(pz[os]), wl));
            words[4 * r] = (static_cast<uint64_t>(static_cast<uint32_t>(wv)) << 32) |
                           (static_cast<uint64_t>(tag) << kLargeIdxBits) | (gidx & kLargeIdxMask);
            words[4 * r + 1] = (static_cast<uint64_t>(bx) << 32) | tag;
            words[4 * r + 2] = (static_cast<uint64_t>(by) << 32) | tag;
            words[4 * r + 3] = (static_cast<uint64_t>(bz) << 32) | tag;
            if (lane == wl) taken |= 1u << os;
        }
        // Lane r writes copy r; the bound word goes last.
        uint64_t* base = records + static_cast<int64_t>(par) * kLargeReplicas * kLazyCopyWords;
        if (lane < kLargeReplicas) {
            uint64_t* rec = base + lane * kLazyCopyWords + gw;
#pragma unroll
            for (int w = 0; w < kLazyRecWords; ++w)
                __hip_atomic_store(rec + static_cast<int64_t>(w) * kLazyMaxWaves, words[w],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }

        // Read every wave's record (copy g % kLargeReplicas).
        const uint64_t* copy = base + (g % kLargeReplicas) * kLazyCopyWords;
        int cmd[CPT], cidx[CPT];
        float cx_[CPT], cy_[CPT], cz_[CPT];
        int bmax = static_cast<int>(0x80000000u);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int rw = tid + j * T;
#pragma unroll
            for (int c = 0; c < kLazyCand; ++c) {
                cmd[j * kLazyCand + c] = static_cast<int>(0x80000000u);
                cidx[j * kLazyCand + c] = 0x7FFFFFFF;
                cx_[j * kLazyCand + c] = cy_[j * kLazyCand + c] = cz_[j * kLazyCand + c] = 0.f;
            }
            if (rw >= waves) continue;
            const uint64_t* q = copy + rw;
            for (uint32_t spins = 0;; ++spins) {
                if (poll_give_up(status, spins, spin_limit)) {
                    abort_flag = 1;
                    break;
                }
                const uint64_t wb = __hip_atomic_load(q + static_cast<int64_t>(kLazyRecWords - 1) * kLazyMaxWaves,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (static_cast<uint32_t>(wb) == tag) {
                    uint64_t rw_[kLazyRecWords - 1];
                    bool ok = true;
#pragma unroll
                    for (int w = 0; w < kLazyRecWords - 1; ++w) {
                        rw_[w] = __hip_atomic_load(q + static_cast<int64_t>(w) * kLazyMaxWaves,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const uint32_t t = (w % 4 == 0)
                                               ? static_cast<uint32_t>((rw_[w] >> kLargeIdxBits) & 0x7FFu)
                                               : static_cast<uint32_t>(rw_[w]);
                        ok = ok && t == tag;
                    }
                    if (ok) {
                        bmax = max(bmax, static_cast<int>(wb >> 32));
#pragma unroll
                        for (int c = 0; c < kLazyCand; ++c) {
                            cmd[j * kLazyCand + c] = static_cast<int>(rw_[4 * c] >> 32);
                            cidx[j * kLazyCand + c] = static_cast<int>(rw_[4 * c] & kLargeIdxMask);
                            cx_[j * kLazyCand + c] = i2f(static_cast<int>(rw_[4 * c + 1] >> 32));
                            cy_[j * kLazyCand + c] = i2f(static_cast<int>(rw_[4 * c + 2] >> 32));
                            cz_[j * kLazyCand + c] = i2f(static_cast<int>(rw_[4 * c + 3] >> 32));
                        }
                        break;
                    }
                }
            }
        }
        bmax = wave_max_i32_l63(bmax);
        if (lane == 0) wave_bound[wave] = bmax;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
#pragma unroll
            for (int c = 0; c < kLazyCand; ++c) {
                const int id = (tid + j * T) * kLazyCand + c;
                cand_xyzk[id] = make_float4(cx_[j * kLazyCand + c], cy_[j * kLazyCand + c],
                                            cz_[j * kLazyCand + c], i2f(cmd[j * kLazyCand + c]));
                cand_idx[id] = static_cast<uint32_t>(cidx[j * kLazyCand + c]);
            }
        }
        __syncthreads();
        if (abort_flag) {  // uniform: written before the barrier
            // Slots from `step` on were never written: mark them -1 so a
            // caller that misses the status word still sees the failure.
            if (g == 0)
                for (int64_t s = step + tid; s < npoint; s += T) out[s] = -1;
            return;
        }
        int bound = wave_bound[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) bound = max(bound, wave_bound[w]);

        // Steps over the candidates alone, by every wave on its own (no
        // barrier); each is applied at once to this thread's points.
        lazy_steps<CW>(cand_xyzk, cand_idx, bound, lane, live_xyzk[wave], live_idx[wave],
                       static_cast<int>(min<int64_t>(npoint - step, INT32_MAX)),
                       [&](const float4& c, uint32_t index) {
                           if (g == 0 && tid == 0) out[step] = index;
                           ++step;
#pragma unroll
                           for (int k = 0; k < P; ++k)
                               md[k] = running_min(md[k], sqdist3(px[k], py[k], pz[k], c.x, c.y, c.z));
                       });
    }
}

// fps_stream_kernel<T>: the same lazy exchange for clouds too large for the
// registers of the chip (more than 2^21 points; up to 2^32 - 1).  Workgroup
// g owns points [g*chunk, min(N, g*chunk + chunk)) and keeps their running
// distances in `md` (HBM, N floats, written on the first exchange): every
// exchange streams its chunk once -- coordinates and running distances in,
// the pending centroids applied, running distances out -- and each wave
// keeps, per lane, its largest running distance (smallest index on ties)
// with that point, and its second largest value.  The wave's candidate is
// the largest of its lanes' (smallest index on ties) and its bound the
// largest of the other lanes' maxima and the winner's second value, i.e. the
// largest running distance of every point it did not publish.  Records are
// those of fps_lazy_kernel (kLazyCand = 1) with the index split over two
// words: bits 0-20 beside the key, bits 21-31 beside x.
constexpr int kStreamUnroll = 8;  // points per thread per batch (two batches in flight)
constexpr int64_t kStreamMaxN = (int64_t(1) << 32) - 1;  // indices below 2^32 - 1

template <int T>
__global__ __launch_bounds__(T) void fps_stream_kernel(
    const float* __restrict__ xyz, float* __restrict__ md, int64_t* __restrict__ out,
    uint64_t* __restrict__ records, uint32_t* __restrict__ status, int64_t N, int64_t npoint,
    int64_t start, int skip, int64_t chunk, uint32_t spin_limit) {
    constexpr int NW = T / kWave;
    static_assert(NW <= 8 && kLazyCand == 1, "shape");
    constexpr int RPT = kLazyMaxWaves / T;  // records read per thread at most
    constexpr int CW = kLazyMaxWaves / kWave;  // candidates per lane in a run
    __shared__ float4 pend[kLazyMaxPending];
    __shared__ float4 cand_xyzk[kLazyMaxWaves];  // the exchange's candidates: x, y, z, key bits
    __shared__ uint32_t cand_idx[kLazyMaxWaves];
    __shared__ float4 live_xyzk[NW][kLazyLive];  // per wave: the run's live candidates
    __shared__ uint32_t live_idx[NW][kLazyLive];
    __shared__ int wave_bound[NW];
    __shared__ int abort_flag;

    const int G = gridDim.x;
    const int waves = G * NW;
    const int g = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int64_t lo = static_cast<int64_t>(g) * chunk;
    const int64_t hi = min(N, lo + chunk);
    if (tid == 0) {
        abort_flag = 0;
        pend[0] = make_float4(xyz[3 * start], xyz[3 * start + 1], xyz[3 * start + 2], 0.f);
        if (g == 0) out[0] = start;
    }
    int npend = 1;
    int64_t step = 1;
    for (uint32_t exch = 0; step < npoint; ++exch) {
        __syncthreads();  // pend[] complete; every wave is past the last run's reads
        // Stream the chunk: apply the pending centroids, keep this lane's
        // best point (running distance, index, xyz) and its second value.
        int bv = static_cast<int>(0x80000000u), sv = static_cast<int>(0x80000000u);
        uint32_t bi = 0xFFFFFFFFu;  // indices are below 2^32 - 1
        float bx = 0.f, by = 0.f, bz = 0.f;
        // Software-pipelined: the next batch's loads (clamped, so always in
        // bounds) are issued before the current batch is computed.
        constexpr int64_t kBatch = static_cast<int64_t>(kStreamUnroll) * T;
        float x[kStreamUnroll], y[kStreamUnroll], z[kStreamUnroll], m[kStreamUnroll];
        auto fetch = [&](int64_t j0, float (&fx)[kStreamUnroll], float (&fy)[kStreamUnroll],
                         float (&fz)[kStreamUnroll], float (&fm)[kStreamUnroll]) {
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u) {
                const int64_t j = min(j0 + static_cast<int64_t>(u) * T, hi - 1);
                fx[u] = xyz[3 * j];
                fy[u] = xyz[3 * j + 1];
                fz[u] = xyz[3 * j + 2];
                fm[u] = exch == 0 ? 0.f : md[j];
            }
        };
        if (lo + tid < hi) fetch(lo + tid, x, y, z, m);
        for (int64_t j0 = lo + tid; j0 < hi; j0 += kBatch) {
            float nx[kStreamUnroll], ny[kStreamUnroll], nz[kStreamUnroll], nm[kStreamUnroll];
            fetch(j0 + kBatch, nx, ny, nz, nm);
            float v[kStreamUnroll];
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u)
                v[u] = exch != 0 ? m[u] : initial_running(skip, x[u], y[u], z[u]);
            for (int i = 0; i < npend; ++i) {  // each centroid read once per batch
                const float4 c = pend[i];
#pragma unroll
                for (int u = 0; u < kStreamUnroll; ++u)
                    v[u] = running_min(v[u], sqdist3(x[u], y[u], z[u], c.x, c.y, c.z));
            }
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u) {
                const int64_t j = j0 + static_cast<int64_t>(u) * T;
                if (j >= hi) break;  // uniform per thread; j grows with u
                md[j] = v[u];
                const int key = f2i(v[u]);  // -inf orders below every distance
                // Indices grow along this thread's walk: strict `>` keeps the
                // smallest index among equal values.
                if (key > bv) {
                    sv = bv;
                    bv = key;
                    bi = static_cast<uint32_t>(j);
                    bx = x[u];
                    by = y[u];
                    bz = z[u];
                } else {
                    sv = max(sv, key);
                }
            }
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u) {
                x[u] = nx[u];
                y[u] = ny[u];
                z[u] = nz[u];
                m[u] = nm[u];
            }
        }
        npend = 0;

        // The wave's candidate (largest value, then smallest index) and bound.
        const int wv = wave_max_i32_l63(bv);
        const uint32_t ci = bv == wv ? bi : 0xFFFFFFFFu;
        const uint32_t gidx = ~wave_max_u32_l63(~ci);  // smallest index holding wv
        const int wl = static_cast<int>(__builtin_ctzll(ballot(bv == wv && ci == gidx)));
        const int other = lane == wl ? sv : bv;
        const int bound_w = wave_max_i32_l63(other);
        const uint32_t tag = (exch & 0x3FFu) | 0x400u;
        const int gw = g * NW + wave;
        uint64_t words[kLazyRecWords];
        words[0] = (static_cast<uint64_t>(static_cast<uint32_t>(wv)) << 32) |
                   (static_cast<uint64_t>(tag) << kLargeIdxBits) | (gidx & kLargeIdxMask);
        words[1] = (static_cast<uint64_t>(static_cast<uint32_t>(readlane(f2i(bx), wl))) << 32) |
                   (static_cast<uint64_t>(gidx >> kLargeIdxBits) << 11) | tag;
        words[2] = (static_cast<uint64_t>(static_cast<uint32_t>(readlane(f2i(by), wl))) << 32) | tag;
        words[3] = (static_cast<uint64_t>(static_cast<uint32_t>(readlane(f2i(bz), wl))) << 32) | tag;
        words[4] = (static_cast<uint64_t>(static_cast<uint32_t>(bound_w)) << 32) | tag;
        const int par = static_cast<int>(exch & 1);
        uint64_t* base = records + static_cast<int64_t>(par) * kLargeReplicas * kLazyCopyWords;
        if (lane < kLargeReplicas) {
            uint64_t* rec = base + lane * kLazyCopyWords + gw;
#pragma unroll
            for (int w = 0; w < kLazyRecWords; ++w)
                __hip_atomic_store(rec + static_cast<int64_t>(w) * kLazyMaxWaves, words[w],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }

        // Read every wave's record (copy g % kLargeReplicas).
        const uint64_t* copy = base + (g % kLargeReplicas) * kLazyCopyWords;
        int cmd[RPT];
        uint32_t cidx[RPT];
        float cx_[RPT], cy_[RPT], cz_[RPT];
        int bmax = static_cast<int>(0x80000000u);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int rw = tid + r * T;
            cmd[r] = static_cast<int>(0x80000000u);
            cidx[r] = 0xFFFFFFFFu;
            cx_[r] = cy_[r] = cz_[r] = 0.f;
            if (rw >= waves) continue;
            const uint64_t* q = copy + rw;
            for (uint32_t spins = 0;; ++spins) {
                if (poll_give_up(status, spins, spin_limit)) {
                    abort_flag = 1;
                    break;
                }
                const uint64_t wb = __hip_atomic_load(q + static_cast<int64_t>(kLazyRecWords - 1) * kLazyMaxWaves,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (static_cast<uint32_t>(wb) != tag) continue;
                uint64_t rw_[kLazyRecWords - 1];
#pragma unroll
                for (int w = 0; w < kLazyRecWords - 1; ++w)
                    rw_[w] = __hip_atomic_load(q + static_cast<int64_t>(w) * kLazyMaxWaves,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const bool ok = static_cast<uint32_t>((rw_[0] >> kLargeIdxBits) & 0x7FFu) == tag &&
                                (static_cast<uint32_t>(rw_[1]) & 0x7FFu) == tag &&
                                static_cast<uint32_t>(rw_[2]) == tag &&
                                static_cast<uint32_t>(rw_[3]) == tag;
                if (!ok) continue;
                bmax = max(bmax, static_cast<int>(wb >> 32));
                cmd[r] = static_cast<int>(rw_[0] >> 32);
                cidx[r] = static_cast<uint32_t>(rw_[0] & kLargeIdxMask) |
                          (((static_cast<uint32_t>(rw_[1]) >> 11) & 0x7FFu) << kLargeIdxBits);
                cx_[r] = i2f(static_cast<int>(rw_[1] >> 32));
                cy_[r] = i2f(static_cast<int>(rw_[2] >> 32));
                cz_[r] = i2f(static_cast<int>(rw_[3] >> 32));
                break;
            }
        }
        bmax = wave_max_i32_l63(bmax);
        if (lane == 0) wave_bound[wave] = bmax;
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            cand_xyzk[tid + r * T] = make_float4(cx_[r], cy_[r], cz_[r], i2f(cmd[r]));
            cand_idx[tid + r * T] = cidx[r];
        }
        __syncthreads();
        if (abort_flag) {  // uniform: written before the barrier
            if (g == 0)
                for (int64_t s = step + tid; s < npoint; s += T) out[s] = -1;
            return;
        }
        int bound = wave_bound[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) bound = max(bound, wave_bound[w]);

        // Steps over the candidates alone, by every wave on its own (no
        // barrier; wave 0 records the centroids for the next exchange).
        lazy_steps<CW>(cand_xyzk, cand_idx, bound, lane, live_xyzk[wave], live_idx[wave],
                       static_cast<int>(min<int64_t>(npoint - step, kLazyMaxPending - npend)),
                       [&](const float4& c, uint32_t index) {
                           if (g == 0 && tid == 0) out[step] = static_cast<int64_t>(index);
                           if (tid == 0) pend[npend] = make_float4(c.x, c.y, c.z, 0.f);
                           ++npend;
                           ++step;
                       });
    }
}

// ------------------------------------------------------------ dispatch

constexpr int kRegsThreads = 512;  // 8 waves: two per SIMD hide each other's reduction latency
constexpr int kRegsMaxPoints = 16 * kRegsThreads;  // 8192 points in VGPRs (P = 16)
constexpr int kGlobalThreads = 1024;

// Tiles per wave of the first half (the rest hold 2P - PO): 9 of 16 for
// P = 8 measured 1.5 % faster at N = 4096 than an even split, 10 and 12
// slower; other P keep the even split.
template <int P>
constexpr int kTilesFirstHalf = P == 8 ? 9 : P;

// The single-cloud kernel that runs P points per sorting thread: the
// leader/follower kernel up to 4096 points, the tiled kernel above (its
// follower tiles would not fit the registers of nine waves).
template <int P>
const void* dense_fps_kernel() {
    if constexpr (P <= 8) return reinterpret_cast<const void*>(&fps_lead_kernel<P>);
    else return reinterpret_cast<const void*>(&fps_tiled_kernel<P, kRegsThreads, kTilesFirstHalf<P>>);
}

template <int P>
hipError_t launch_regs(const float* xyz, const int64_t* ptr, const int64_t* out_ptr,
                       const int64_t* starts, int64_t* out, int64_t blocks, int64_t N,
                       int64_t npoint, int64_t start, int skip, hipStream_t stream,
                       uint64_t* progress = nullptr, uint64_t tag = 0, int64_t chunk = 1,
                       size_t reserve = 0, float* centres = nullptr) {
    if constexpr (P > 8) {
        hipLaunchKernelGGL((fps_tiled_kernel<P, kRegsThreads, kTilesFirstHalf<P>>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kRegsThreads), reserve, stream, xyz, ptr, out_ptr, starts, out, N, npoint,
                           start, skip, progress, tag, chunk, centres);
    } else {
        hipLaunchKernelGGL((fps_lead_kernel<P>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kLeadThreads), reserve, stream, xyz, ptr, out_ptr, starts, out, N, npoint,
                           start, skip, progress, tag, chunk, centres);
    }
    return hipGetLastError();
}

hipError_t launch_fps(const float* xyz, const int64_t* ptr, const int64_t* out_ptr,
                      const int64_t* starts, int64_t* out, float* scratch, int64_t blocks,
                      int64_t max_len, int64_t N, int64_t npoint, int64_t start, int skip,
                      hipStream_t stream) {
    if (max_len <= 1 * kRegsThreads)
        return launch_regs<1>(xyz, ptr, out_ptr, starts, out, blocks, N, npoint, start, skip, stream);
    if (max_len <= 2 * kRegsThreads)
        return launch_regs<2>(xyz, ptr, out_ptr, starts, out, blocks, N, npoint, start, skip, stream);
    if (max_len <= 4 * kRegsThreads)
        return launch_regs<4>(xyz, ptr, out_ptr, starts, out, blocks, N, npoint, start, skip, stream);
    if (max_len <= 8 * kRegsThreads)
        return launch_regs<8>(xyz, ptr, out_ptr, starts, out, blocks, N, npoint, start, skip, stream);
    if (max_len <= 16 * kRegsThreads)
        return launch_regs<16>(xyz, ptr, out_ptr, starts, out, blocks, N, npoint, start, skip, stream);
    if (scratch == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL((fps_global_kernel<kGlobalThreads>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(kGlobalThreads), 0, stream, xyz, ptr, out_ptr, starts, out, scratch,
                       N, npoint, start, skip);
    return hipGetLastError();
}

// The persistent large-cloud kernel for P points per thread.
template <int P>
const void* large_kernel() {
    return reinterpret_cast<const void*>(&fps_lazy_kernel<P, kLargeThreads>);
}

// Polls of one record before the large-cloud kernel gives up: kSpinLimit,
// or POINTOPS_FPS_SPIN_LIMIT when set (a diagnostic: 0 makes every call
// give up at its first exchange, which is how the failure path is tested).
uint32_t spin_limit() {
    const char* env = std::getenv("POINTOPS_FPS_SPIN_LIMIT");
    if (env == nullptr || *env == '\0') return kSpinLimit;
    return static_cast<uint32_t>(std::strtoul(env, nullptr, 10));
}

// The streaming kernel over one workgroup per CU (at most kLargeMaxGrid).
constexpr int kStreamThreads = kLargeThreads;

hipError_t launch_stream(const float* xyz, float* md, int64_t* out, uint64_t* records,
                         uint32_t* status, int64_t N, int64_t npoint, int64_t start, int skip,
                         int device, hipStream_t stream) {
    const void* kernel = reinterpret_cast<const void*>(&fps_stream_kernel<kStreamThreads>);
    int per_cu = 0, cus = 0;
    hipError_t err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kStreamThreads, 0);
    if (err != hipSuccess) return err;
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return err;
    if (per_cu < 1 || cus < 1) return hipErrorInvalidValue;
    int grid = min(cus, kLargeMaxGrid);
    int64_t chunk = (N + grid - 1) / grid;
    uint32_t limit = spin_limit();
    void* args[] = {(void*)&xyz, (void*)&md, (void*)&out, (void*)&records, (void*)&status,
                    (void*)&N, (void*)&npoint, (void*)&start, (void*)&skip, (void*)&chunk,
                    (void*)&limit};
    return hipLaunchCooperativeKernel(kernel, dim3(grid), dim3(kStreamThreads), args, 0, stream);
}

template <int P>
hipError_t launch_large(const float* xyz, int64_t* out, uint64_t* records, uint32_t* status,
                        int N, int64_t npoint, int start, int skip, int chunk, int grid,
                        hipStream_t stream) {
    uint32_t limit = spin_limit();
    void* args[] = {(void*)&xyz, (void*)&out, (void*)&records, (void*)&status, (void*)&N,
                    (void*)&npoint, (void*)&start, (void*)&skip, (void*)&chunk, (void*)&limit};
    return hipLaunchCooperativeKernel(large_kernel<P>(), dim3(grid), dim3(kLargeThreads), args, 0,
                                      stream);
}

// Status word (padded to 256 B) + 2 parities x copies x records.
constexpr size_t kLargeWorkspaceBytes =
    256 + static_cast<size_t>(2 * kLargeReplicas * kLazyCopyWords) * sizeof(uint64_t);

// Workspace of pointops_fps_large_noalloc (640 KiB per GPU, held until the
// process ends).  Host code never passes this name to a kernel: it is only a
// host-side handle, whose device address (one per GPU) comes from
// hipGetSymbolAddress in scratch_address().
static __device__ __align__(256) unsigned char scratch[kLargeWorkspaceBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU, once looked up

// Device address of `scratch` on `device` (the current device), looked up on
// the first call for that device.
hipError_t scratch_address(int device, void** out) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_ptr[device] == nullptr) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        if (p == nullptr) return hipErrorInvalidSymbol;
        scratch_ptr[device] = p;
    }
    *out = scratch_ptr[device];
    return hipSuccess;
}

// Zero-fill of n 64-bit words (a kernel, so the clear is an ordinary launch
// on the caller's stream rather than a memset node).
__global__ __launch_bounds__(256) void zero_words_kernel(uint64_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

template <int P>
int large_capacity(int device) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, large_kernel<P>(), kLargeThreads, 0) !=
        hipSuccess)
        return 0;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return 0;
    return min(per_cu, 1) * cus;  // at most one workgroup per CU
}

}  // namespace
}  // namespace pointops

namespace pointops {

// Dense FPS of B clouds of N <= 8192 points (fps_lead_kernel, or
// fps_tiled_kernel above 4096 points) that publishes per-cloud progress
// words: progress[b] = tag + the whole `chunk`s of samples of cloud b stored
// so far (all ceil(npoint / chunk) of them at the end).  With `centres` set,
// each sample's coordinates are stored too (B, npoint, 3), before the
// progress word that covers them.
// Dynamic LDS that, added to fps_tiled_kernel<P>'s own, takes all of a CU's
// LDS: no workgroup that uses LDS (every kernel queued beside a pipelined
// FPS does) can then share a CU with an FPS workgroup and take issue slots
// from its latency-bound steps.  0 if the attributes cannot be read.
template <int P>
size_t fps_reserve_lds() {
    static const size_t bytes = [] {
        hipFuncAttributes a{};
        int dev = 0, per_block = 0, per_cu = 0;
        const void* k = dense_fps_kernel<P>();
        if (hipFuncGetAttributes(&a, k) != hipSuccess || hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess)
            return size_t(0);
        const size_t cap = static_cast<size_t>(per_block < per_cu ? per_block : per_cu);
        const size_t mine = a.sharedSizeBytes;
        if (cap <= mine) return size_t(0);
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(cap - mine)) != hipSuccess)
            return size_t(0);
        return cap - mine;
    }();
    return bytes;
}

hipError_t fps_dense_progress(const float* xyz, int64_t* out, int64_t B, int64_t N,
                              int64_t npoint, int64_t start, int skip, uint64_t* progress,
                              uint64_t tag, int64_t chunk, float* centres, hipStream_t stream) {
    if (B < 1 || B > INT32_MAX || N < 1 || N > kRegsMaxPoints || npoint < 1 || npoint > N ||
        start < 0 || start >= N || chunk < 1 || progress == nullptr)
        return hipErrorInvalidValue;
    if (N <= 1 * kRegsThreads)
        return launch_regs<1>(xyz, nullptr, nullptr, nullptr, out, B, N, npoint, start, skip, stream,
                              progress, tag, chunk, fps_reserve_lds<1>(), centres);
    if (N <= 2 * kRegsThreads)
        return launch_regs<2>(xyz, nullptr, nullptr, nullptr, out, B, N, npoint, start, skip, stream,
                              progress, tag, chunk, fps_reserve_lds<2>(), centres);
    if (N <= 4 * kRegsThreads)
        return launch_regs<4>(xyz, nullptr, nullptr, nullptr, out, B, N, npoint, start, skip, stream,
                              progress, tag, chunk, fps_reserve_lds<4>(), centres);
    if (N <= 8 * kRegsThreads)
        return launch_regs<8>(xyz, nullptr, nullptr, nullptr, out, B, N, npoint, start, skip, stream,
                              progress, tag, chunk, fps_reserve_lds<8>(), centres);
    return launch_regs<16>(xyz, nullptr, nullptr, nullptr, out, B, N, npoint, start, skip, stream,
                           progress, tag, chunk, fps_reserve_lds<16>(), centres);
}

}  // namespace pointops

using namespace pointops;

extern "C" {

size_t pointops_fps_dense_scratch_bytes(int64_t B, int64_t N) {
    if (B <= 0 || N <= kRegsMaxPoints) return 0;
    return static_cast<size_t>(B) * static_cast<size_t>(N) * sizeof(float);
}

hipError_t pointops_fps_dense(const float* xyz, int64_t* out, void* scratch, int64_t B, int64_t N,
                              int64_t npoint, int64_t start_idx, int32_t skip_near_origin,
                              hipStream_t stream) {
    if (B < 0 || N < 0 || npoint < 0) return hipErrorInvalidValue;
    if (B == 0 || npoint == 0) return hipSuccess;
    if (N == 0 || start_idx < 0 || start_idx >= N || N > INT32_MAX - 1 || B > INT32_MAX)
        return hipErrorInvalidValue;
    if (xyz == nullptr || out == nullptr) return hipErrorInvalidValue;
    return launch_fps(xyz, nullptr, nullptr, nullptr, out, static_cast<float*>(scratch), B, N, N,
                      npoint, start_idx, skip_near_origin ? 1 : 0, stream);
}

size_t pointops_fps_flat_scratch_bytes(int64_t total_n, int64_t max_len) {
    if (max_len <= kRegsMaxPoints || total_n <= 0) return 0;
    return static_cast<size_t>(total_n) * sizeof(float);
}

hipError_t pointops_fps_flat(const float* x, const int64_t* ptr, const int64_t* out_ptr,
                             const int64_t* starts, int64_t* out, void* scratch, int64_t batch,
                             int64_t total_n, int64_t max_len, hipStream_t stream) {
    if (batch < 0 || total_n < 0 || max_len < 0 || max_len > INT32_MAX - 1 || batch > INT32_MAX)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (ptr == nullptr || out_ptr == nullptr || starts == nullptr) return hipErrorInvalidValue;
    return launch_fps(x, ptr, out_ptr, starts, out, static_cast<float*>(scratch), batch, max_len, 0,
                      0, 0, 0, stream);
}

size_t pointops_fps_large_workspace_bytes(int64_t N, int64_t npoint) {
    (void)npoint;
    if (N <= 0) return 0;
    if (N <= kLargeMaxN) return kLargeWorkspaceBytes;
    return kLargeWorkspaceBytes + static_cast<size_t>(N) * sizeof(float);  // running distances
}

}  // extern "C"

namespace pointops {
namespace {

// Checks shared by both large-cloud entry points; hipSuccess with *run = false
// when there is nothing to do.
hipError_t check_large(const float* xyz, const int64_t* out, int64_t N, int64_t npoint,
                       int64_t start_idx, int64_t max_n, bool* run) {
    *run = false;
    if (N < 0 || npoint < 0) return hipErrorInvalidValue;
    if (npoint == 0) return hipSuccess;
    if (N == 0 || N > max_n || start_idx < 0 || start_idx >= N) return hipErrorInvalidValue;
    if (xyz == nullptr || out == nullptr) return hipErrorInvalidValue;
    *run = true;
    return hipSuccess;
}

// Launches the persistent kernel with the smallest P (points per thread)
// whose grid fits one workgroup per CU and one polled record per thread.
// `workspace` holds kLargeWorkspaceBytes bytes, zero-filled.
hipError_t launch_large_any(const float* xyz, int64_t* out, void* workspace, int64_t N,
                            int64_t npoint, int64_t start_idx, int skip, int device,
                            hipStream_t stream) {
    auto* status = static_cast<uint32_t*>(workspace);
    auto* records = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + 256);
    if (N > kLargeMaxN) {  // running distances after the records
        auto* md = reinterpret_cast<float*>(static_cast<char*>(workspace) + kLargeWorkspaceBytes);
        return launch_stream(xyz, md, out, records, status, N, npoint, start_idx, skip, device,
                             stream);
    }
    const int n32 = static_cast<int>(N);
    const int s32 = static_cast<int>(start_idx);
    const int choices[] = {1, 2, 4, 8, 16, 32};
    for (int P : choices) {
        int cap = 0;
        switch (P) {
            case 1: cap = large_capacity<1>(device); break;
            case 2: cap = large_capacity<2>(device); break;
            case 4: cap = large_capacity<4>(device); break;
            case 8: cap = large_capacity<8>(device); break;
            case 16: cap = large_capacity<16>(device); break;
            default: cap = large_capacity<32>(device); break;
        }
        cap = min(cap, kLargeMaxGrid);
        const int64_t per_block = static_cast<int64_t>(P) * kLargeThreads;
        const int64_t need = (N + per_block - 1) / per_block;
        if (cap <= 0 || need > cap) continue;
        const int grid = static_cast<int>(need);
        const int chunk = static_cast<int>(per_block);
        switch (P) {
            case 1: return launch_large<1>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
            case 2: return launch_large<2>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
            case 4: return launch_large<4>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
            case 8: return launch_large<8>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
            case 16: return launch_large<16>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
            default: return launch_large<32>(xyz, out, records, status, n32, npoint, s32, skip, chunk, grid, stream);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace
}  // namespace pointops

extern "C" {

hipError_t pointops_fps_large(const float* xyz, int64_t* out, void* workspace, int64_t N,
                              int64_t npoint, int64_t start_idx, int32_t skip_near_origin,
                              hipStream_t stream) {
    bool run = false;
    hipError_t err = check_large(xyz, out, N, npoint, start_idx, kStreamMaxN, &run);
    if (err != hipSuccess || !run) return err;
    if (workspace == nullptr) return hipErrorInvalidValue;
    int device = 0;
    err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    return launch_large_any(xyz, out, workspace, N, npoint, start_idx, skip_near_origin ? 1 : 0,
                            device, stream);
}

hipError_t pointops_fps_large_noalloc(const float* xyz, int64_t* out, int64_t N, int64_t npoint,
                                      int64_t start_idx, int32_t skip_near_origin,
                                      hipStream_t stream) {
    bool run = false;
    hipError_t err = check_large(xyz, out, N, npoint, start_idx, kLargeMaxN, &run);
    if (err != hipSuccess || !run) return err;
    int device = 0;
    err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    void* ws = nullptr;
    err = scratch_address(device, &ws);
    if (err != hipSuccess) return err;
    // The previous call's records and status stay in the array: clear them.
    constexpr int64_t words = static_cast<int64_t>(kLargeWorkspaceBytes / sizeof(uint64_t));
    hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<uint32_t>((words + 255) / 256)),
                       dim3(256), 0, stream, static_cast<uint64_t*>(ws), words);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_large_any(xyz, out, ws, N, npoint, start_idx, skip_near_origin ? 1 : 0, device,
                            stream);
}

}  // extern "C"
