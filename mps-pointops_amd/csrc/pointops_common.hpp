// Shared device helpers for the gfx950 neighbourhood-search kernels.
//
// Every kernel is compiled with -ffp-contract=off and without fast-math, so
// each float expression below is one IEEE binary32 operation rounded to
// nearest-even in the written order; denormals are preserved (no FTZ).  The
// squared distance is therefore bit-identical to the reference's separately
// rounded tensor ops ((dx*dx + dy*dy) + dz*dz), reference.py:21-24.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pointops {

constexpr int kWave = 64;

// 4-bit cell coordinates interleaved into a 12-bit Morton key: bit b of
// axis a goes to bit 3b + a (each coordinate's bits spread by two
// shift-or-mask rounds).
__device__ __forceinline__ uint32_t morton12(uint32_t x, uint32_t y, uint32_t z) {
    auto spread = [](uint32_t q) {
        q = (q | (q << 4)) & 0x0C3u;     // bits 0, 1 | 6, 7
        return (q | (q << 2)) & 0x249u;  // bits 0, 3, 6, 9
    };
    return spread(x) | (spread(y) << 1) | (spread(z) << 2);
}

__device__ __forceinline__ float sqdist3(float ax, float ay, float az, float bx, float by,
                                         float bz) {
    const float dx = ax - bx;
    const float dy = ay - by;
    const float dz = az - bz;
    float d = dx * dx;
    d = d + dy * dy;
    d = d + dz * dz;
    return d;
}

__device__ __forceinline__ int f2i(float v) { return __float_as_int(v); }
__device__ __forceinline__ float i2f(int v) { return __int_as_float(v); }

// Loads of data read exactly once (gradient rows streamed through LDS),
// marked non-temporal: they do not displace reused data from the caches.
__device__ __forceinline__ float4 load_once(const float4* p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float load_once(const float* p) { return __builtin_nontemporal_load(p); }
// Stores of outputs larger than the caches (the set-abstraction layer's
// grouped features), marked non-temporal for the same reason.
__device__ __forceinline__ void store_once(float* p, float v) { __builtin_nontemporal_store(v, p); }

// ---------------------------------------------------------------- DPP / SALU
// GFX9 DPP controls (row = 16 lanes).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppWaveShr1 = 0x138;     // lane l <- lane l-1; lane 0 keeps `old`

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}

// Shift the wave right by one lane: lane l gets v[l-1], lane 0 gets `fill`.
__device__ __forceinline__ int wave_shr1(int v, int fill) {
    return __builtin_amdgcn_update_dpp(fill, v, kDppWaveShr1, 0xF, 0xF, false);
}

__device__ __forceinline__ int readlane(int v, int lane) {
    return __builtin_amdgcn_readlane(v, lane);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// `old` with lane `lane` replaced by `value` (both wave-uniform): one
// v_writelane_b32 in place of a lane compare and a select.  The s_nop gives
// the four wait states a lane select written by a VALU instruction needs.
__device__ __forceinline__ int writelane(int old, int value, int lane) {
    asm("s_nop 3\n\tv_writelane_b32 %0, %1, m0" : "+v"(old) : "s"(value), "{m0}"(lane));
    return old;
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Lanes strictly below this lane whose bit is set in `mask`.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Maximum over the wave of a float with no NaN; every lane gets the result.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, i2f(dpp<kDppQuadXor1>(f2i(v))));
    v = fmaxf(v, i2f(dpp<kDppQuadXor2>(f2i(v))));
    v = fmaxf(v, i2f(dpp<kDppRowHalfMirror>(f2i(v))));
    v = fmaxf(v, i2f(dpp<kDppRowMirror>(f2i(v))));
    const float a = i2f(readlane(f2i(v), 0));
    const float b = i2f(readlane(f2i(v), 16));
    const float c = i2f(readlane(f2i(v), 32));
    const float d = i2f(readlane(f2i(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Minimum over the wave of a float with no NaN; every lane gets the result.
__device__ __forceinline__ float wave_min(float v) {
    v = fminf(v, i2f(dpp<kDppQuadXor1>(f2i(v))));
    v = fminf(v, i2f(dpp<kDppQuadXor2>(f2i(v))));
    v = fminf(v, i2f(dpp<kDppRowHalfMirror>(f2i(v))));
    v = fminf(v, i2f(dpp<kDppRowMirror>(f2i(v))));
    const float a = i2f(readlane(f2i(v), 0));
    const float b = i2f(readlane(f2i(v), 16));
    const float c = i2f(readlane(f2i(v), 32));
    const float d = i2f(readlane(f2i(v), 48));
    return fminf(fminf(a, b), fminf(c, d));
}

// Maximum over the wave of a signed int; every lane gets the result.
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, dpp<kDppQuadXor1>(v));
    v = max(v, dpp<kDppQuadXor2>(v));
    v = max(v, dpp<kDppRowHalfMirror>(v));
    v = max(v, dpp<kDppRowMirror>(v));
    const int a = readlane(v, 0);
    const int b = readlane(v, 16);
    const int c = readlane(v, 32);
    const int d = readlane(v, 48);
    return max(max(a, b), max(c, d));
}

// DPP move whose unwritten lanes read INT_MIN, the identity of max, so that
// max(v, dpp_or_lowest(v)) folds into one v_max_i32_dpp.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_or_lowest(int v) {
    return __builtin_amdgcn_update_dpp(static_cast<int>(0x80000000u), v, CTRL, ROW_MASK, 0xF,
                                       false);
}

// Maximum over the wave of a signed int, as a wave-uniform value: butterflies
// inside each row of 16, then row_bcast:15 / row_bcast:31 carry the row
// maxima up to lane 63.
__device__ __forceinline__ int wave_max_i32_l63(int v) {
    v = max(v, dpp_or_lowest<kDppQuadXor1>(v));
    v = max(v, dpp_or_lowest<kDppQuadXor2>(v));
    v = max(v, dpp_or_lowest<kDppRowHalfMirror>(v));
    v = max(v, dpp_or_lowest<kDppRowMirror>(v));
    v = max(v, dpp_or_lowest<0x142, 0xA>(v));  // row_bcast:15 into rows 1 and 3
    v = max(v, dpp_or_lowest<0x143, 0xC>(v));  // row_bcast:31 into rows 2 and 3
    return readlane(v, 63);
}

// DPP move whose unwritten lanes read 0, the identity of unsigned max.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}

// Maximum over the wave of an unsigned int, as a wave-uniform value (the
// row_bcast scheme of wave_max_i32_l63).
__device__ __forceinline__ uint32_t wave_max_u32_l63(uint32_t v) {
    v = max(v, dpp_or_zero<kDppQuadXor1>(v));
    v = max(v, dpp_or_zero<kDppQuadXor2>(v));
    v = max(v, dpp_or_zero<kDppRowHalfMirror>(v));
    v = max(v, dpp_or_zero<kDppRowMirror>(v));
    v = max(v, dpp_or_zero<0x142, 0xA>(v));  // row_bcast:15 into rows 1 and 3
    v = max(v, dpp_or_zero<0x143, 0xC>(v));  // row_bcast:31 into rows 2 and 3
    return static_cast<uint32_t>(readlane(static_cast<int>(v), 63));
}

// Maximum over each aligned group of 8 lanes, read from lane 0.
__device__ __forceinline__ int group8_max_i32(int v) {
    v = max(v, dpp_or_lowest<kDppQuadXor1>(v));
    v = max(v, dpp_or_lowest<kDppQuadXor2>(v));
    v = max(v, dpp_or_lowest<kDppRowHalfMirror>(v));
    return readlane(v, 0);
}

// fminf(m, d) for a running minimum m that is never NaN and a computed d
// (never a signalling NaN): in IEEE mode v_min_f32 returns the non-NaN
// operand, as fminf does.  Written as one instruction because the compiler
// otherwise canonicalises the loop-carried operand on every use.
__device__ __forceinline__ float running_min(float m, float d) {
    float r;
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(d));
    return r;
}

// Minimum over the wave of a signed int; every lane gets the result.
__device__ __forceinline__ int wave_min(int v) {
    v = min(v, dpp<kDppQuadXor1>(v));
    v = min(v, dpp<kDppQuadXor2>(v));
    v = min(v, dpp<kDppRowHalfMirror>(v));
    v = min(v, dpp<kDppRowMirror>(v));
    const int a = readlane(v, 0);
    const int b = readlane(v, 16);
    const int c = readlane(v, 32);
    const int d = readlane(v, 48);
    return min(min(a, b), min(c, d));
}

// (d, i) strictly before (e, j): smaller distance, then smaller index
// (the reference's kNN ordering, kernels/knn.metal:27-30).  NaN is never
// before anything.
__device__ __forceinline__ bool before(float d, int i, float e, int j) {
    return d < e || (d == e && static_cast<uint32_t>(i) < static_cast<uint32_t>(j));
}

// Map 32-bit block ids so that consecutive logical ids share an XCD: the
// hardware deals workgroups round-robin over the 8 XCDs, and neighbouring
// logical blocks touch the same cloud, so keeping them on one XCD keeps the
// cloud in that XCD's L2.
__device__ __forceinline__ uint32_t xcd_local_block(uint32_t hw, uint32_t nblocks) {
    constexpr uint32_t kXcds = 8;
    if (nblocks % kXcds != 0) return hw;
    const uint32_t per = nblocks / kXcds;
    return (hw % kXcds) * per + hw / kXcds;
}

// (block within its cloud, cloud) of a workgroup of a 1-D launch of
// per_cloud * B workgroups, dealt by xcd_local_block so that the workgroups
// of one cloud share an XCD (and its L2 copy of the cloud).
struct CloudBlock {
    uint32_t x;  // block within the cloud
    uint32_t b;  // cloud
};
__device__ __forceinline__ CloudBlock cloud_block(uint32_t per_cloud) {
    const uint32_t blk = xcd_local_block(blockIdx.x, gridDim.x);
    return {blk % per_cloud, blk / per_cloud};
}

// ball_query.hip: up to kBqMulti ball queries around the same centres in one
// scan (radius r: r2[r] as pointops_ball_query_f32 takes it, k[r] slots,
// outputs (B, QS, k[r]) written at the query rows).
constexpr int kBqMulti = 4;
struct BallMulti {
    int64_t* idx[kBqMulti];
    float* dist[kBqMulti];
    int k[kBqMulti];
    float r2[kBqMulti];
};
hipError_t ball_query_multi_rows_f32(const float* q, const float* p, const BallMulti& out, int nr,
                                     int64_t B, int64_t Q, int64_t QS, int64_t P,
                                     hipStream_t stream);

// ball_query.hip: the index-order float32 ball query without lengths (the
// LDS-staged kernel, B <= 65535), every workgroup returning at once when
// `skip` is non-null and *skip != 0 at launch time.
hipError_t ball_query_f32_unless(const float* queries, const float* points, int64_t* idx,
                                 float* dist2, int64_t B, int64_t Q, int64_t P, int64_t K,
                                 float radius_sq, const int* skip, hipStream_t stream);

}  // namespace pointops
