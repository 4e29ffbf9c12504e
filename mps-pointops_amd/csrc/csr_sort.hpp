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
// order.  Buckets of up to kCsrSmall entries are sorted in registers by the
// thread that owns the key (a thread owns KPT consecutive keys, so a pass
// over keys replaces a pass over every entry of the batch); longer ones go
// to one wave per bucket, so no wave runs one long bucket's count while
// its other lanes hold short ones: up to 256 entries are sorted across the
// wave's lanes by a bitonic network, longer buckets ranked lane = entry.  A bucket of more
// than OMAX entries keeps the scatter's order instead (the count costs
// O(L^2)).  Entries go from their final place straight to memory.  Keys outside [0, num_keys) are dropped, or clamped into it with
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
    __shared__ int first[MAXK + 1];                // bucket starts, then the total
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
    if (tid == T - 1) {
        first[MAXK] = before + run;
        if (r == 0) start[num_keys] = before + run;
    }
    __syncthreads();
    // Scatter this workgroup's entries.  em[k] becomes key << 16 | position
    // for an entry of a bucket beyond OMAX (it stays at its scatter
    // position), -1 otherwise (its bucket is ordered below).
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (em[k] < 0 || (em[k] & (R - 1)) != r) {
            em[k] = -1;
            continue;
        }
        const int m = em[k];
        const int at = atomicAdd(&cursor[m], 1);
        list[at] = static_cast<uint16_t>(tid + k * T);
        em[k] = first[m + 1] - first[m] > OMAX ? (m << 16) | at : -1;
    }
    __syncthreads();
    auto put = [&](int at, int e, int m, float w) {
        list_out[at] = static_cast<uint16_t>(e);
        if (key_out != nullptr) key_out[at] = static_cast<uint16_t>(m);
        if constexpr (W) weight_out[at] = w;
    };
    // Own keys: buckets longer than kCsrSmall (and at most OMAX) go to the
    // waves; shorter ones are sorted here, each id placed at the number of
    // smaller ids of its bucket (ids are distinct).
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
        const int m = tid * KPT + k;
        if ((m & (R - 1)) != r) continue;
        const int p0 = first[m], len = first[m + 1] - p0;
        if (len > kCsrSmall) {
            if (len <= OMAX) longs[atomicAdd(&n_longs, 1)] = m;
            continue;
        }
        if (len == 0) continue;
        int v[kCsrSmall];
#pragma unroll
        for (int i = 0; i < kCsrSmall; ++i) v[i] = i < len ? static_cast<int>(list[p0 + i]) : 0x10000;
#pragma unroll
        for (int i = 0; i < kCsrSmall; ++i) {
            if (i >= len) break;
            int rank = 0;
#pragma unroll
            for (int j = 0; j < kCsrSmall; ++j) rank += v[j] < v[i] ? 1 : 0;
            put(p0 + rank, v[i], m, W ? weights[v[i]] : 0.f);
        }
    }
    // Entries of buckets beyond OMAX: at their scatter position.
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (em[k] < 0) continue;
        put(em[k] & 0xFFFF, tid + k * T, em[k] >> 16, W ? ew[k] : 0.f);
    }
    __syncthreads();  // the long-bucket list is complete
    const int nl = n_longs;
    // Buckets of up to 64 entries, four per wave at a time: one id per lane,
    // sorted across the wave by a bitonic network (ids are distinct; the
    // padding 0x10000 sorts last), the four sorts interleaved so that their
    // lane exchanges overlap; lane l then holds the l-th smallest id.
    constexpr int kSortsPerWave = 4;
    for (int i0 = wave * kSortsPerWave; i0 < nl; i0 += kSortsPerWave * NW) {
        int v[kSortsPerWave], ms[kSortsPerWave], ps[kSortsPerWave], ns[kSortsPerWave];
#pragma unroll
        for (int s = 0; s < kSortsPerWave; ++s) {
            ms[s] = i0 + s < nl ? longs[i0 + s] : 0;
            ps[s] = first[ms[s]];
            ns[s] = i0 + s < nl ? first[ms[s] + 1] - ps[s] : 0;
            if (ns[s] > kWave) ns[s] = 0;  // sorted below
            v[s] = lane < ns[s] ? static_cast<int>(list[ps[s] + lane]) : 0x10000;
        }
#pragma unroll
        for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {
                const bool low = ((lane & j) == 0) == ((lane & k) == 0);
#pragma unroll
                for (int s = 0; s < kSortsPerWave; ++s) {
                    const int o = __shfl_xor(v[s], j, kWave);
                    v[s] = low ? min(v[s], o) : max(v[s], o);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kSortsPerWave; ++s)
            if (lane < ns[s]) put(ps[s] + lane, v[s], ms[s], W ? weights[v[s]] : 0.f);
    }
    // Longer buckets, one wave each.  Up to 256 entries: four ids per lane
    // (element x = s * 64 + lane in register s), sorted by the same network
    // over 256 elements, whose exchanges 64 or more elements apart are
    // swaps between a lane's registers.  Beyond that: lane = entry, ranked
    // by its count of smaller ids.
    constexpr int kWideSort = 4;
    for (int i = wave; i < nl; i += NW) {
        const int m = longs[i];
        const int p0 = first[m], p1 = first[m + 1];
        const int len = p1 - p0;
        if (len <= kWave) continue;
        if (len <= kWideSort * kWave) {
            int v[kWideSort];
#pragma unroll
            for (int s = 0; s < kWideSort; ++s) {
                const int x = s * kWave + lane;
                v[s] = x < len ? static_cast<int>(list[p0 + x]) : 0x10000;
            }
#pragma unroll
            for (int k = 2; k <= kWideSort * kWave; k <<= 1) {
#pragma unroll
                for (int j = k >> 1; j > 0; j >>= 1) {
                    int o[kWideSort];
#pragma unroll
                    for (int s = 0; s < kWideSort; ++s)
                        o[s] = j >= kWave ? v[s ^ (j / kWave)] : __shfl_xor(v[s], j, kWave);
#pragma unroll
                    for (int s = 0; s < kWideSort; ++s) {
                        const int x = s * kWave + lane;
                        v[s] = (((x & j) == 0) == ((x & k) == 0)) ? min(v[s], o[s]) : max(v[s], o[s]);
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < kWideSort; ++s) {
                const int x = s * kWave + lane;
                if (x < len) put(p0 + x, v[s], m, W ? weights[v[s]] : 0.f);
            }
            continue;
        }
        for (int c = p0; c < p1; c += kWave) {
            const int q = c + lane;
            if (q < p1) {
                const int e = list[q];
                put(p0 + csr_rank(list, p0, p1, e), e, m, W ? weights[e] : 0.f);
            }
        }
    }
}

}  // namespace pointops
