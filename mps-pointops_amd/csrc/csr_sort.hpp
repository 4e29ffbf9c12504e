// Counting sort of a batch's entries by key into a CSR, in LDS, shared by
// the deterministic backward passes (three_interpolate, grouping).
//
// R workgroups (R a power of two) share one batch: workgroup r owns the
// keys k with k % R == r, so that keys which are hot (many entries) spread
// over all of them.  Each reads all of the batch's keys (entry ids e <
// num_entries <= MAXE <= 65536, so ids fit in 16 bits), counts every key in
// LDS and scans the counts, which gives every bucket's start in the CSR;
// it writes the starts of its own keys and scatters only its own entries
// into an LDS copy of the CSR, then an entry's place in its bucket is the
// number of smaller ids there, so each bucket lists its ids in ascending
// order.  Buckets of up to kCsrSmall entries are ranked by the thread that
// holds each entry; longer ones by one wave per bucket, lane = entry, so no
// wave runs one long bucket's count while its other lanes hold short ones.
// A bucket of more than OMAX entries keeps the scatter's order instead (the
// count costs O(L^2)).  Entries go from their final place straight to
// memory.  Keys outside [0, num_keys) are dropped, or clamped into it with
// CLAMP; with W the entries' weights travel with their ids; with key_out
// non-null each list position also gets its key (num_keys <= 65536).
#pragma once

#include "pointops_common.hpp"

namespace pointops {

constexpr int kCsrSmall = 16;

// Number of ids below e in list[p0, p1): eight ids per 16-byte LDS read over
// the aligned chunks covering the range (callers size the list to a
// multiple of 8 entries, so the reads stay inside).
__device__ __forceinline__ int csr_rank(const uint16_t* list, int p0, int p1, int e) {
    int rank = 0;
    for (int q = p0 & ~7; q < p1; q += 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(&list[q]);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int id = static_cast<int>((w4[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            rank += (q + j >= p0 && q + j < p1 && id < e) ? 1 : 0;
        }
    }
    return rank;
}

template <int T, int MAXE, int MAXK, int OMAX, typename I, bool W, bool CLAMP>
__device__ __forceinline__ void csr_sort_class(const I* __restrict__ keys,
                                               const float* __restrict__ weights,
                                               int num_entries, int num_keys, int r, int R,
                                               int* __restrict__ start,
                                               uint16_t* __restrict__ list_out,
                                               float* __restrict__ weight_out,
                                               uint16_t* __restrict__ key_out = nullptr) {
    constexpr int EPT = MAXE / T;  // entries per thread
    constexpr int KPT = MAXK / T;  // keys per thread in the scan
    constexpr int NW = T / kWave;
    static_assert(EPT * T == MAXE && KPT * T == MAXK && MAXE <= 65536 && MAXE % 8 == 0 &&
                      MAXK <= 32768,
                  "shape");
    __shared__ int cursor[MAXK];                   // counts, then bucket ends
    __shared__ int first[MAXK];                    // bucket starts
    __shared__ __align__(16) uint16_t list[MAXE];  // own buckets, scatter order
    __shared__ int longs[MAXK];                    // own buckets ranked per wave
    __shared__ int n_longs;
    __shared__ int wave_sum[NW];
    const int tid = threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;
    // This thread's entries e = tid + k*T, all requested before the first use.
    int em[EPT];
    float ew[W ? EPT : 1];
#pragma unroll
    for (int k = 0; k < EPT; ++k) em[k] = static_cast<int>(keys[min(tid + k * T, num_entries - 1)]);
    if constexpr (W) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) ew[k] = weights[min(tid + k * T, num_entries - 1)];
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        int m = em[k];
        if constexpr (CLAMP) m = m < 0 ? 0 : (m >= num_keys ? num_keys - 1 : m);
        const bool valid = tid + k * T < num_entries &&
                           static_cast<unsigned>(m) < static_cast<unsigned>(num_keys);
        em[k] = valid ? m : -1;
    }
    for (int m = tid; m < MAXK; m += T) cursor[m] = 0;
    if (tid == 0) n_longs = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < EPT; ++k)
        if (em[k] >= 0) atomicAdd(&cursor[em[k]], 1);
    __syncthreads();
    // Exclusive scan of the counts: KPT consecutive keys per thread.
    int run = 0;
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
        const int v = cursor[tid * KPT + k];
        cursor[tid * KPT + k] = run;
        run += v;
    }
    int incl = run;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int up = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += up;
    }
    if (lane == kWave - 1) wave_sum[wave] = incl;
    __syncthreads();
    int before = incl - run;
    for (int w = 0; w < wave; ++w) before += wave_sum[w];
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
        const int m = tid * KPT + k;
        const int s = cursor[m] + before;
        cursor[m] = s;
        first[m] = s;
        if (m < num_keys && (m & (R - 1)) == r) start[m] = s;
    }
    if (tid == T - 1 && r == 0) start[num_keys] = before + run;
    __syncthreads();
    // Scatter this workgroup's entries; em[k] becomes key << 16 | position.
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (em[k] < 0 || (em[k] & (R - 1)) != r) {
            em[k] = -1;
            continue;
        }
        const int at = atomicAdd(&cursor[em[k]], 1);
        list[at] = static_cast<uint16_t>(tid + k * T);
        em[k] = (em[k] << 16) | at;
    }
    __syncthreads();
    // Own buckets longer than kCsrSmall (and at most OMAX) go to the waves.
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
        const int m = tid * KPT + k;
        const int len = cursor[m] - first[m];
        if ((m & (R - 1)) == r && len > kCsrSmall && len <= OMAX) longs[atomicAdd(&n_longs, 1)] = m;
    }
    // Entries of short (or beyond-OMAX) buckets: placed by their thread.
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (em[k] < 0) continue;
        const int e = tid + k * T;
        const int m = em[k] >> 16;
        const int p0 = first[m], p1 = cursor[m];
        if (p1 - p0 > kCsrSmall && p1 - p0 <= OMAX) continue;
        const int at = p1 - p0 <= kCsrSmall ? p0 + csr_rank(list, p0, p1, e) : (em[k] & 0xFFFF);
        list_out[at] = static_cast<uint16_t>(e);
        if (key_out != nullptr) key_out[at] = static_cast<uint16_t>(m);
        if constexpr (W) weight_out[at] = ew[k];
    }
    __syncthreads();  // the long-bucket list is complete
    const int nl = n_longs;
    for (int i = wave; i < nl; i += NW) {
        const int m = longs[i];
        const int p0 = first[m], p1 = cursor[m];
        for (int c = p0; c < p1; c += kWave) {  // lane = entry of the bucket
            const int q = c + lane;
            if (q < p1) {
                const int e = list[q];
                const int at = p0 + csr_rank(list, p0, p1, e);
                list_out[at] = static_cast<uint16_t>(e);
                if (key_out != nullptr) key_out[at] = static_cast<uint16_t>(m);
                if constexpr (W) weight_out[at] = weights[e];
            }
        }
    }
}

}  // namespace pointops
