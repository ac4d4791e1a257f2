// Row operations of the x070 decode step shared by the row kernels
// (x070.hip) and the GEMV launches that form their input rows themselves
// (rwkvq.hip): layerNorm_ statistics (X070Generation.swift:511-514) and the
// token-shift lerp (tmixStep :214-239, cmixStep :303-308).  One copy of the
// arithmetic, so a row formed inside a GEMV launch is bitwise the row kernel's.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "wkv7_step.h"

namespace rwkv_x070 {

__device__ __forceinline__ float sum4(float4 a) { return (a.x + a.y) + (a.z + a.w); }

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const __half* p) {
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    const float2 a = __half22float2(*reinterpret_cast<const __half2*>(&raw.x));
    const float2 c = __half22float2(*reinterpret_cast<const __half2*>(&raw.y));
    return make_float4(a.x, a.y, c.x, c.y);
}

// Row kernels: a row of D is split over S workgroups of T threads (S = D/1024
// with T = 256 when 1024 divides D, else S = 1 with T = D/4); thread t of
// slice s writes the float4 chunk s·T + t.
__host__ __device__ inline void row_geometry(int64_t D, int& S, int& T, int& PS) {
    if (D % 1024 == 0) {
        T = 256;
        S = PS = (int)(D / 1024);
    } else {
        T = (int)(D / 4);
        S = PS = 1;
    }
}

// layerNorm_ (X070Generation.swift:511-514) statistics of a row of D floats
// (D % 256 == 0), formed by every wave on its own from the whole row: lane l
// takes the float4 chunks l + 64j (j < D/256) in order, each summed as
// (x + y) + (z + w); the 64 lane sums meet in wave_total's fixed butterfly.
// So every wave of every launch (row kernels and the GEMV launches that form
// their input rows) gets the same bits, with no LDS and no barrier.  The
// caller loads the first JH chunks with row_chunks ahead of its other loads
// (chunks past the row repeat the last one: no branch around a load); chunks
// beyond JH are read again here.
template <int JH, typename TY>
__device__ __forceinline__ void row_chunks(const TY* row, int D, int lane, float4 (&v)[JH]) {
    const int nj = D >> 8;
#pragma unroll
    for (int j = 0; j < JH; ++j) v[j] = load4(row + 4 * (lane + 64 * min(j, nj - 1)));
}

// (mean, sqrt(var + eps)): the mean, then the mean of squared deviations.
template <int JH, typename TY>
__device__ __forceinline__ float2 row_stats(const float4 (&v)[JH], const TY* row, int D, int lane, float eps) {
    const int nj = D >> 8;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < JH; ++j) s += j < nj ? sum4(v[j]) : 0.0f;
    for (int j = JH; j < nj; ++j) s += sum4(load4(row + 4 * (lane + 64 * j)));
    const float mean = rwkv_wkv::wave_total(s) / (float)D;
    auto sq = [mean](float4 x) {
        const float4 d = make_float4(x.x - mean, x.y - mean, x.z - mean, x.w - mean);
        return (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
    };
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < JH; ++j) q += j < nj ? sq(v[j]) : 0.0f;
    for (int j = JH; j < nj; ++j) q += sq(load4(row + 4 * (lane + 64 * j)));
    return make_float2(mean, sqrtf(rwkv_wkv::wave_total(q) / (float)D + eps));
}

__device__ __forceinline__ float4 ln_apply(float4 x, float2 md, float4 w, float4 b) {
    return make_float4((x.x - md.x) / md.y * w.x + b.x, (x.y - md.x) / md.y * w.y + b.y,
                       (x.z - md.x) / md.y * w.z + b.z, (x.w - md.x) / md.y * w.w + b.w);
}

// Token shift: xx = prev − xl; the lerp with coefficient q is xl + xx·q.
__device__ __forceinline__ float4 shift_delta(float4 prev, float4 xl) {
    return make_float4(prev.x - xl.x, prev.y - xl.y, prev.z - xl.z, prev.w - xl.w);
}
__device__ __forceinline__ float4 shift_lerp(float4 xl, float4 xx, float4 q) {
    return make_float4(xl.x + xx.x * q.x, xl.y + xx.y * q.y, xl.z + xx.z * q.z, xl.w + xx.w * q.w);
}

}  // namespace rwkv_x070
