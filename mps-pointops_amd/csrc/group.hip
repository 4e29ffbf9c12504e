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

#include "csr_sort.hpp"
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
    const int nc = static_cast<int>(c0 + kGroupChannels < C ? kGroupChannels : C - c0);
    const float* src = f + (b * C + c0) * N + j;
    float* dst = out + (b * C + c0) * P + p;
    // Every channel's load in flight before the first store (channels past
    // the block read the last one again and are not stored).
    float v[kGroupChannels];
#pragma unroll
    for (int k = 0; k < kGroupChannels; ++k) v[k] = src[min(k, nc - 1) * N];
#pragma unroll
    for (int k = 0; k < kGroupChannels; ++k)
        if (k < nc) dst[k * P] = v[k];
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
    const int64_t c0 = static_cast<int64_t>(blockIdx.z) * kGroupChannels;
    const int nc = static_cast<int>(c0 + kGroupChannels < CT ? kGroupChannels : CT - c0);
    float* dst = out + (b * CT + c0) * P + p;
    // Channel c0 + k: relative xyz below 3, else feature c0 + k - 3.  Every
    // load is issued before the first store (channels past the block read a
    // valid one again and are not stored).
    // kx: the block's leading xyz channels (3 in the first block, whose c0
    // is 0, else none: kGroupChannels >= 3).
    const int kx = c0 == 0 ? 3 : 0;
    float v[kGroupChannels];
    if (nc > kx) {  // feature channels c0 + k - 3 for k in [kx, nc)
        const float* src = f + (b * C + c0 - 3) * N + j;
#pragma unroll
        for (int k = 0; k < kGroupChannels; ++k) v[k] = src[min(max(k, kx), nc - 1) * N];
    }
    if (kx > 0) {
        const float* q = xyz + (b * N + j) * 3;
        const float* m = centres + (b * M + p / S) * 3;
#pragma unroll
        for (int a = 0; a < 3; ++a) v[a] = q[a] - m[a];
    }
#pragma unroll
    for (int k = 0; k < kGroupChannels; ++k)
        if (k < nc) dst[k * P] = v[k];
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

// Backward over a per-batch CSR of the entries, for P <= 32768 entries and
// N <= 4096 points: group_csr_kernel (per batch up to kGroupCsrRanges
// workgroups, each owning the points of one residue class) sorts the
// entries p by their point idx[b,p] (csr_sort_class: ascending p within a
// point's list of up to 256, the scatter's order beyond);
// group_csr_grad_kernel (a few workgroups per batch, each taking every
// J-th channel): thread t owns positions [32 t, 32 t + 32) of the batch's
// CSR list -- the same amount of work in every lane, however long the
// lists are -- with, for all channels, one register per position holding
// the LDS byte offsets of the row element it reads and of the slot its
// running sum goes to.  A channel's grad_out row of P floats is staged in
// LDS (the next row requested into registers meanwhile, with non-temporal
// loads: each element is read once, and the rows -- larger than the
// caches -- would otherwise displace reused data); each thread sums the
// pieces of lists inside its range in list order, and a list that crosses
// ranges is summed piece by piece: its first piece by the thread where it
// starts, which then adds the following threads' pieces in order.  So a
// point's gradient is the sum of its entries in ascending p, cut into
// pieces at every 32nd list position of the batch, each piece summed from
// +0 in order and the pieces added in order.  The results go through LDS
// to coalesced stores; every element of grad_features is written once.
// No transpose, no atomics on the gradients.
constexpr int kGroupCsrThreads = 1024;
constexpr int kGroupCsrMaxP = 32768;
constexpr int kGroupCsrMaxN = 4096;
constexpr int kGroupCsrRanges = 8;       // build workgroups per batch at most
constexpr int kGroupCsrSorted = 256;     // lists up to this long are in ascending p
constexpr int kGroupGradThreads = 1024;  // the gather's workgroup: 32 list positions per thread
// The gather's LDS result slots, in floats: a channel's results, a
// continuation and a head piece per thread, and a padding slot (4 floats,
// so the row after them is 16-byte aligned).
__host__ __device__ constexpr int group_grad_slots(int threads) {
    return kGroupCsrMaxN + 2 * threads + 4;
}

struct GroupCsr {
    int* start;      // [B][sstride]: list starts, N + 1 used
    uint16_t* list;  // [B][lstride]: entries p by point
    uint16_t* key;   // [B][lstride]: the point of each list position
    int64_t sstride, lstride;
};

__host__ __device__ inline size_t group_csr_bytes(int64_t B, int64_t N, int64_t P, GroupCsr* out,
                                                  char* base) {
    const int64_t ss = (N + 1 + 63) & ~int64_t(63), ls = (P + 63) & ~int64_t(63);
    const size_t start_bytes = group_align(static_cast<size_t>(B * ss) * sizeof(int));
    const size_t list_bytes = group_align(static_cast<size_t>(B * ls) * sizeof(uint16_t));
    if (out != nullptr) {
        out->start = reinterpret_cast<int*>(base);
        out->list = reinterpret_cast<uint16_t*>(base + start_bytes);
        out->key = reinterpret_cast<uint16_t*>(base + start_bytes + list_bytes);
        out->sstride = ss;
        out->lstride = ls;
    }
    return start_bytes + 2 * list_bytes;
}

__host__ __device__ inline bool group_csr_fits(int64_t N, int64_t P) {
    return N >= 1 && N <= kGroupCsrMaxN && P >= 1 && P <= kGroupCsrMaxP;
}

template <typename I>
__global__ __launch_bounds__(kGroupCsrThreads) void group_csr_kernel(const I* __restrict__ idx,
                                                                     GroupCsr csr, int N, int P) {
    const int64_t b = blockIdx.x;
    // Indices outside [0, N) are clamped, as the forward gathers them.
    csr_sort_class<kGroupCsrThreads, kGroupCsrMaxP, kGroupCsrMaxN, kGroupCsrSorted, I, false, true>(
        idx + b * P, nullptr, P, N, static_cast<int>(blockIdx.y), static_cast<int>(gridDim.y),
        csr.start + b * csr.sstride, csr.list + b * csr.lstride, nullptr,
        csr.key + b * csr.lstride);
}

template <int T, bool VEC>
__global__ __launch_bounds__(T) void group_csr_grad_kernel(
    const float* __restrict__ g, int64_t g_batch, GroupCsr csr, float* __restrict__ gf, int64_t C,
    int N, int P, uint32_t J) {
    constexpr int E = kGroupCsrMaxP / T;    // list positions per thread
    constexpr int NPT = kGroupCsrMaxN / T;  // output points per thread
    constexpr int V = kGroupCsrMaxP / T;    // row floats per thread
    constexpr int B8 = 8;                   // positions per batch of LDS reads
    constexpr int kCont = kGroupCsrMaxN, kHead = kCont + T, kPad = kHead + T;
    constexpr uint32_t kRowByte = 4u * group_grad_slots(T);  // the row after the slots
    static_assert(E % B8 == 0 && V % 4 == 0 && E <= 64, "whole 16-byte loads");
    static_assert(kRowByte < 32768u && kRowByte % 16 == 0, "15-bit slot offsets, aligned row");
    __shared__ __align__(16) unsigned char group_lds[kRowByte + 4 * kGroupCsrMaxP];
    // LDS: the result slots -- a channel's results [N], continuation pieces
    // [T], head pieces [T] and a padding slot [4] -- then the row
    // [kGroupCsrMaxP].
    float* const slots = reinterpret_cast<float*>(group_lds);
    float* const row = reinterpret_cast<float*>(group_lds + kRowByte);
    const CloudBlock cb = cloud_block(J);  // a 1-D launch of B J workgroups
    const int64_t b = cb.b;
    const int64_t j = cb.x;
    const int tid = threadIdx.x;
    const int64_t own = j < C ? (C - 1 - j) / J + 1 : 0;  // channels j, j + J, ...
    const float* gb = g + b * g_batch;
    // A channel's row, read from inside it (chunks past P read the last
    // one again: row slots at or past P are stored but never read).
    auto fetch = [&](int64_t s, float (&r)[V]) {
        const float* src = gb + (j + s * J) * P;
        if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < V / 4; ++u) {
                const float4 v =
                    load_once(reinterpret_cast<const float4*>(src + min(4 * (u * T + tid), P - 4)));
                r[4 * u] = v.x;
                r[4 * u + 1] = v.y;
                r[4 * u + 2] = v.z;
                r[4 * u + 3] = v.w;
            }
        }
    };
    float rv[V];
    if (VEC && own > 0) fetch(0, rv);  // unaligned rows are read when needed instead
    // This thread's list positions q0 .. q0 + qn - 1: ids and points
    // (16-bit, two per register), the point just before q0 and the one just
    // after my range.
    const int q0 = tid * E;
    const int qn = max(0, min(E, P - q0));
    const int64_t lbase = b * csr.lstride + (q0 < P ? q0 : 0);  // lstride: whole 64-id blocks
    uint32_t ids[E / 2], pts[E / 2];
#pragma unroll
    for (int u = 0; u < E / 8; ++u) {
        const uint4 v = *reinterpret_cast<const uint4*>(csr.list + lbase + 8 * u);
        const uint4 k = *reinterpret_cast<const uint4*>(csr.key + lbase + 8 * u);
        ids[4 * u] = v.x;
        ids[4 * u + 1] = v.y;
        ids[4 * u + 2] = v.z;
        ids[4 * u + 3] = v.w;
        pts[4 * u] = k.x;
        pts[4 * u + 1] = k.y;
        pts[4 * u + 2] = k.z;
        pts[4 * u + 3] = k.w;
    }
    const int before = q0 > 0 && q0 < P ? csr.key[b * csr.lstride + q0 - 1] : -1;
    const int after = q0 + qn < P ? csr.key[b * csr.lstride + q0 + qn] : -1;
    auto half = [](const uint32_t (&a)[E / 2], int u) {
        return static_cast<int>((u & 1) ? a[u >> 1] >> 16 : a[u >> 1] & 0xFFFFu);
    };
    // Per position, two LDS byte offsets in one register: bits 15-31 the
    // row element it reads (4 x its id; row[0] past the end), bits 0-14
    // the slot its running sum goes to: the point's result slot where the
    // point's list ends inside my range and began inside it, my
    // continuation slot where my first piece (of a list begun before q0)
    // ends, my head slot where my last piece (of a list going on past my
    // range) ends -- my last position --, the padding slot past the end.
    // Positions inside a list also write my head slot: they come before my
    // head piece's write, if there is one, and the slot is read only then.
    // So a piece starts at position u exactly where position u - 1 wrote a
    // slot other than my head slot (or u = 0).
    uint32_t pos[E];
    int head_n = -1;  // the list my head piece begins (-1: none)
    const uint32_t head_byte = 4u * static_cast<uint32_t>(kHead + tid);
    {
        const int first_n = qn > 0 ? half(pts, 0) : -1;
        const bool cont = qn > 0 && before == first_n;
#pragma unroll
        for (int u = 0; u < E; ++u) {
            const int n = half(pts, u);
            const int nn = u + 1 < qn ? half(pts, u + 1) : after;
            const bool mine_first = cont && n == first_n;  // a list begun before q0
            int d = kHead + tid;  // inside a list
            if (u >= qn) {
                d = kPad;
            } else if (n != nn) {  // the list ends here
                d = mine_first ? kCont + tid : n;
            } else if (u + 1 == qn) {  // the list goes on past my range
                if (mine_first) {
                    d = kCont + tid;  // a middle piece
                } else {
                    head_n = n;
                }
            }
            const uint32_t id = u < qn ? static_cast<uint32_t>(half(ids, u)) : 0u;
            pos[u] = (4u * id) << 15 | 4u * static_cast<uint32_t>(d);
        }
    }
    // Following threads whose first pieces finish my head's list.
    const int head_span =
        head_n >= 0 ? (csr.start[b * csr.sstride + head_n + 1] - (q0 + qn) + E - 1) / E : 0;
    // Every result slot starts at 0: a point with an empty list keeps it,
    // the others are rewritten in every channel.
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int n = tid + i * T;
        if (n < N) slots[n] = 0.f;
    }
    for (int64_t s = 0; s < own; ++s) {
        __syncthreads();  // previous channel: row and results read
        if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < V / 4; ++u)
                *reinterpret_cast<float4*>(row + 4 * (u * T + tid)) =
                    make_float4(rv[4 * u], rv[4 * u + 1], rv[4 * u + 2], rv[4 * u + 3]);
        } else {
            const float* src = gb + (j + s * J) * P;
            for (int at = tid; at < P; at += T) row[at] = load_once(src + at);
        }
        __syncthreads();  // row complete
        if (VEC && s + 1 < own) fetch(s + 1, rv);
        // Keeps the unpacked offsets from being hoisted out of the channel
        // loop (twice the registers of the packed ones).
#pragma unroll
        for (int u = 0; u < E; ++u) asm volatile("" : "+v"(pos[u]));
        // The running sum in position order, restarted from +0 where a piece
        // starts, stored after every position to that position's slot.  The
        // next eight row reads are issued before the current eight are
        // summed (the row is not written in this phase).
        auto rd = [&](int u) {
            return *reinterpret_cast<const float*>(group_lds + kRowByte + (pos[u] >> 15));
        };
        float acc = 0.f;
        float va[B8], vb[B8];
#pragma unroll
        for (int u = 0; u < B8; ++u) va[u] = rd(u);
#pragma unroll
        for (int u8 = 0; u8 < E; u8 += B8) {
            if (u8 + B8 < E) {
#pragma unroll
                for (int u = 0; u < B8; ++u) vb[u] = rd(u8 + B8 + u);
            }
#pragma unroll
            for (int u = 0; u < B8; ++u) {
                const int q = u8 + u;
                const bool keep = q > 0 && (pos[q - 1] & 0x7FFFu) == head_byte;
                acc = (keep ? acc : 0.f) + va[u];  // +0 + x: a piece's first term
                *reinterpret_cast<float*>(group_lds + (pos[q] & 0x7FFFu)) = acc;
            }
#pragma unroll
            for (int u = 0; u < B8; ++u) va[u] = vb[u];
            __builtin_amdgcn_sched_barrier(0);  // eight positions at a time: few live values
        }
        __syncthreads();  // pieces complete
        if (head_span > 0) {
            // The following threads' pieces, eight reads in flight at a time
            // (past the span: the last piece again, not added).
            float v = slots[kHead + tid];
            for (int k0 = 1; k0 <= head_span; k0 += 8) {
                float w[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) w[k] = slots[kCont + tid + min(k0 + k, head_span)];
#pragma unroll
                for (int k = 0; k < 8; ++k) v = k0 + k <= head_span ? v + w[k] : v;
            }
            slots[head_n] = v;
        }
        __syncthreads();  // results complete
        const int64_t c = j + s * J;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
            const int n = tid + i * T;
            if (n < N) gf[(b * C + c) * N + n] = slots[n];
        }
    }
}

// LDS-staged grouping for clouds whose channel rows fit in LDS: one
// workgroup per (group of CG channels, batch, slice of the output columns)
// stages its batch's CG source rows -- feature rows, and for REL the
// coordinates for channels 0-2 -- with coalesced loads, then walks its
// columns: each column's index is read once (four columns per thread in
// flight) and its CG values come from LDS, so the gathers never touch L2;
// stores along p are coalesced and non-temporal (the output, S times the
// features, is larger than the caches and would displace the source rows).
// HBM traffic: the output, the source rows once per slice (L2 after the
// first) and the index once per channel group.
constexpr int kGroupLdsThreads = 512;
// Rows per workgroup: up to 32 KiB (measured at config 2's shape: 8 KiB
// rows, 2 per workgroup, 83 us; 1 row 104 us, 4 rows 94 us, 8 rows 134 us),
// or one row of up to 64 KiB.
constexpr int kGroupLdsBytes = 32 * 1024;
constexpr int kGroupLdsRowBytes = 64 * 1024;
constexpr int kGroupLdsCols = 4;           // output columns per thread per step

template <bool REL, int CG, typename I>
__global__ __launch_bounds__(kGroupLdsThreads) void group_lds_kernel(
    const float* __restrict__ xyz, const float* __restrict__ centres, const float* __restrict__ f,
    const I* __restrict__ idx, float* __restrict__ out, int64_t C, int64_t N, int64_t M,
    int64_t S) {
    constexpr int T = kGroupLdsThreads;
    constexpr int U = kGroupLdsCols;
    extern __shared__ float rows[];  // [CG][N]
    const int64_t CT = REL ? C + 3 : C;
    const int64_t P = M * S;
    const int64_t b = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CG;
    const int nc = static_cast<int>(c0 + CG < CT ? CG : CT - c0);
    const int tid = threadIdx.x;
    // Stage: row k is channel c0 + k; eight loads per thread in flight.
    for (int k = 0; k < nc; ++k) {
        const int64_t c = c0 + k;
        const bool coord = REL && c < 3;
        const float* src = coord ? xyz + b * N * 3 + c : f + (b * C + c - (REL ? 3 : 0)) * N;
        const int64_t stride = coord ? 3 : 1;
        float* dst = rows + static_cast<int64_t>(k) * N;
        for (int64_t n0 = 0; n0 < N; n0 += 8 * T) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = src[min(n0 + u * T + tid, N - 1) * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (n0 + u * T + tid < N) dst[n0 + u * T + tid] = v[u];
        }
    }
    __syncthreads();
    const int64_t per = (P + gridDim.z - 1) / gridDim.z;
    const int64_t p_lo = static_cast<int64_t>(blockIdx.z) * per;
    const int64_t p_hi = min(P, p_lo + per);
    const I* ib = idx + b * P;
    float* ob = out + (b * CT + c0) * P;
    for (int64_t p0 = p_lo + tid; p0 < p_hi; p0 += static_cast<int64_t>(U) * T) {
        int64_t j[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {  // clamped loads, all in flight
            const int64_t v = static_cast<int64_t>(ib[min(p0 + u * T, p_hi - 1)]);
            j[u] = v < 0 ? 0 : (v >= N ? N - 1 : v);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t p = p0 + u * T;
            if (p >= p_hi) break;
            // The first group's relative channels subtract the column's
            // centre (P < 2^31: 32-bit division, once per column).
            const float* ctr = nullptr;
            if (REL && c0 < 3)
                ctr = centres + (b * M + static_cast<uint32_t>(p) / static_cast<uint32_t>(S)) * 3;
#pragma unroll
            for (int k = 0; k < CG; ++k) {
                if (k >= nc) break;
                float v = rows[static_cast<int64_t>(k) * N + j[u]];
                if (REL && c0 + k < 3) v = v - ctr[c0 + k];
                store_once(ob + static_cast<int64_t>(k) * P + p, v);
            }
        }
    }
}

// Channels per workgroup of group_lds_kernel (0: rows of N floats do not fit).
int group_lds_channels(int64_t N) {
    const int64_t row = N * static_cast<int64_t>(sizeof(float));
    for (int cg : {8, 4, 2})
        if (cg * row <= kGroupLdsBytes) return cg;
    return row <= kGroupLdsRowBytes ? 1 : 0;
}

// Launches group_lds_kernel when the rows fit; returns false otherwise.
template <bool REL, typename I>
bool launch_group_lds(const float* xyz, const float* centres, const float* f, const I* idx,
                      float* out, int64_t B, int64_t C, int64_t N, int64_t M, int64_t S,
                      hipStream_t stream, hipError_t* err) {
    const int cg = group_lds_channels(N);
    const int64_t CT = REL ? C + 3 : C;
    const int64_t groups = cg > 0 ? (CT + cg - 1) / cg : 0;
    if (cg == 0 || B > 65535 || groups > INT32_MAX || M * S >= INT32_MAX) return false;
    // Slices of the columns: at least 2048 workgroups in all (eight per
    // resident slot, so the last round is a small part of the run), each
    // slice at least 2048 columns.
    const int64_t want = (2048 + groups * B - 1) / (groups * B);
    const int64_t slices = std::max<int64_t>(1, std::min<int64_t>({65535, want, (M * S + 2047) / 2048}));
    const dim3 grid(static_cast<uint32_t>(groups), static_cast<uint32_t>(B), static_cast<uint32_t>(slices));
    const size_t shmem = static_cast<size_t>(cg) * static_cast<size_t>(N) * sizeof(float);
    switch (cg) {
        case 8: hipLaunchKernelGGL((group_lds_kernel<REL, 8, I>), grid, dim3(kGroupLdsThreads), shmem, stream, xyz, centres, f, idx, out, C, N, M, S); break;
        case 4: hipLaunchKernelGGL((group_lds_kernel<REL, 4, I>), grid, dim3(kGroupLdsThreads), shmem, stream, xyz, centres, f, idx, out, C, N, M, S); break;
        case 2: hipLaunchKernelGGL((group_lds_kernel<REL, 2, I>), grid, dim3(kGroupLdsThreads), shmem, stream, xyz, centres, f, idx, out, C, N, M, S); break;
        default: hipLaunchKernelGGL((group_lds_kernel<REL, 1, I>), grid, dim3(kGroupLdsThreads), shmem, stream, xyz, centres, f, idx, out, C, N, M, S); break;
    }
    *err = hipGetLastError();
    return true;
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
    hipError_t err = hipSuccess;
    if (idx_bits == 32 ? launch_group_lds<false>(nullptr, nullptr, features, static_cast<const int32_t*>(idx),
                                                 out, B, C, N, P, 1, stream, &err)
                       : launch_group_lds<false>(nullptr, nullptr, features, static_cast<const int64_t*>(idx),
                                                 out, B, C, N, P, 1, stream, &err))
        return err;
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
    if (group_csr_fits(N, P)) return group_csr_bytes(B, N, P, nullptr, nullptr);
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
    if (workspace != nullptr && group_csr_fits(N, P) && B <= 65535 && C <= INT32_MAX) {
        GroupCsr csr;
        group_csr_bytes(B, N, P, &csr, static_cast<char*>(workspace));
        int64_t ranges = 1;  // workgroups per batch: a power of two covering the CUs
        while (ranges < kGroupCsrRanges && ranges * B < 256) ranges *= 2;
        const dim3 bgrid(static_cast<uint32_t>(B), static_cast<uint32_t>(ranges));
        const int n = static_cast<int>(N), p = static_cast<int>(P);
        if (idx_bits == 32)
            hipLaunchKernelGGL(group_csr_kernel<int32_t>, bgrid, dim3(kGroupCsrThreads), 0, stream,
                               static_cast<const int32_t*>(idx), csr, n, p);
        else
            hipLaunchKernelGGL(group_csr_kernel<int64_t>, bgrid, dim3(kGroupCsrThreads), 0, stream,
                               static_cast<const int64_t*>(idx), csr, n, p);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        // J workgroups per batch (every J-th channel each), enough to cover
        // the CUs; LDS: a row and the result slots.
        const int64_t J = std::min<int64_t>(C, std::max<int64_t>(1, (256 + B - 1) / B));
        constexpr int T = kGroupGradThreads;  // LDS: a row and the result slots (static)
        const dim3 ggrid(static_cast<uint32_t>(B * J));
        const uint32_t uj = static_cast<uint32_t>(J);
        const bool vec = P % 4 == 0 && grad_batch_stride % 4 == 0 &&
                         reinterpret_cast<uintptr_t>(grad_out) % 16 == 0;
        if (vec)
            hipLaunchKernelGGL((group_csr_grad_kernel<T, true>), ggrid, dim3(T), 0,
                               stream, grad_out, grad_batch_stride, csr, grad_features, C, n, p, uj);
        else
            hipLaunchKernelGGL((group_csr_grad_kernel<T, false>), ggrid, dim3(T), 0,
                               stream, grad_out, grad_batch_stride, csr, grad_features, C, n, p, uj);
        return hipGetLastError();
    }
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
    hipError_t err = hipSuccess;
    if (idx_bits == 32 ? launch_group_lds<true>(xyz, centres, features, static_cast<const int32_t*>(idx),
                                                out, B, C, N, M, S, stream, &err)
                       : launch_group_lds<true>(xyz, centres, features, static_cast<const int64_t*>(idx),
                                                out, B, C, N, M, S, stream, &err))
        return err;
    if (idx_bits == 32)
        hipLaunchKernelGGL(group_points_rel_kernel<int32_t>, grid, dim3(kGroupThreads), 0, stream,
                           xyz, centres, features, static_cast<const int32_t*>(idx), out, C, N, M, S);
    else
        hipLaunchKernelGGL(group_points_rel_kernel<int64_t>, grid, dim3(kGroupThreads), 0, stream,
                           xyz, centres, features, static_cast<const int64_t*>(idx), out, C, N, M, S);
    return hipGetLastError();
}

}  // extern "C"
