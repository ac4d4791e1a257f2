// Row operations of the x070 decode step shared by the row kernels
// (x070.hip) and the GEMV launches that form their input rows themselves
// (rwkvq.hip): layerNorm_ statistics (X070Generation.swift:511-514) and the
// token-shift lerp (tmixStep :214-239, cmixStep :303-308).  One copy of the
// arithmetic, so a row formed inside a GEMV launch is bitwise the row kernel's.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "wkv7_step.h"

namespace rwkv_x070 {

// Sum over the workgroup: per-wave butterfly, then the wave totals in wave
// order; every thread gets the same value.  `red` (16 floats) is used once
// per kernel, so no barrier is needed before it is written.  Waves whose
// threads pass 0 add +0.0, which leaves the total unchanged.
__device__ __forceinline__ float block_total(float v, float* red) {
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = rwkv_wkv::wave_total(v);
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < nw; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float sum4(float4 a) { return (a.x + a.y) + (a.z + a.w); }

// Row kernels: a row of D is split over S workgroups of T threads (S = D/1024
// with T = 256 when 1024 divides D, else S = 1 with T = D/4); thread t of
// slice s writes the float4 chunk s·T + t.  Every workgroup forms the row's
// statistics itself from the whole row (PS = D/(4T) chunks per thread, the
// same order in every slice).
__host__ __device__ inline void row_geometry(int64_t D, int& S, int& T, int& PS) {
    if (D % 1024 == 0) {
        T = 256;
        S = PS = (int)(D / 1024);
    } else {
        T = (int)(D / 4);
        S = PS = 1;
    }
}

// layerNorm_ (X070Generation.swift:511-514): mean, then the mean of squared
// deviations; the row's (mean, sqrt(var + eps)).  Thread t < T holds chunks
// t + T·p (p < PS) in v; other threads pass `on` false and add nothing.
// A chunk left out adds +0.0 (no branch, so a caller's loads of v are not
// sunk past later ones); the sums are those of the chunks taken, in order.
template <int PS>
__device__ __forceinline__ float2 row_stats(const float4 (&v)[PS], int ps, bool on, int D, float eps, float* red) {
    float s = 0.0f;
#pragma unroll
    for (int p = 0; p < PS; ++p) {
        const float a = sum4(v[p]);
        s += (on && p < ps) ? a : 0.0f;
    }
    const float mean = block_total(s, red) / (float)D;   // red[0..15], then red[16..31]
    float q = 0.0f;
#pragma unroll
    for (int p = 0; p < PS; ++p) {
        const float4 d = make_float4(v[p].x - mean, v[p].y - mean, v[p].z - mean, v[p].w - mean);
        const float a = (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        q += (on && p < ps) ? a : 0.0f;
    }
    return make_float2(mean, sqrtf(block_total(q, red + 16) / (float)D + eps));
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
