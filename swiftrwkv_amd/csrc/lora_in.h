// Low-rank first layers of the x070 time mix (tmixStep, X070Generation.swift
// :256-276, the inner `lin` of the w / a / v / g branches), as device code
// shared by the standalone kernel (x070.hip) and the launch that runs it
// beside the fused r/k/v GEMV (rwkvq.hip).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "wkv7_step.h"

namespace rwkv_x070 {

// fp32 → fp16 (RNE) → fp32: the narrowing of `lin` for fp16 matrices.
__device__ __forceinline__ float f16_round(float x) { return __half2float(__float2half_rn(x)); }
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// The low-rank branch functions of the tmix core (decode) and of the parallel
// pass: exp2 of the scaled argument and the hardware reciprocal (each ~1 ulp;
// relative error of the result ~1e-6 over the branch outputs' range, against
// the IEEE sequences' ~30 dependent instructions).
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x)); }

// One wave computes one job = (input row n, matrix row j) of
// la[n, j] = act(lin(x_branch, Wcat[j])): rows of Wcat [rw + ra + rv + rg, D]
// are the w, a, v, g branches, inputs xmix [N, 4, D] rows w, a, v, g; tanh
// for w, sigmoid for g, none for a and v; the v branch is skipped without
// `with_v` (layer 0).  A lane takes 16-byte matrix slices lane·E + 64·E·q
// (E elements each) in ascending column order, BATCH loads in flight; the
// result does not depend on BATCH.  The caller guards job < RT·N.

// The branch of matrix row j.
__device__ __forceinline__ int lora_branch(int j, int rw, int ra, int rv) {
    return j < rw ? 0 : j < rw + ra ? 1 : j < rw + ra + rv ? 2 : 3;
}

// The matrix slices of a job's first chunk (columns lane·E + 64·E·q), for a
// caller that issues them before it forms the input row.
template <bool H16, int BATCH>
__device__ __forceinline__ void lora_in_first(int j, int lane, const void* __restrict__ Wcat, int D,
                                              uint4 (&first)[BATCH]) {
    constexpr int E = H16 ? 8 : 4;
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
        const int c = min(64 * E * q + lane * E, D - E);   // past the row: a valid slice, not used
        first[q] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(Wcat) +
                                                   ((int64_t)j * D + c) * (H16 ? 2 : 4));
    }
}

// One job given its branch's input row xin (global memory or LDS); with
// `first`, the first chunk's matrix slices are already loaded.
template <bool H16, int BATCH>
__device__ __forceinline__ void lora_in_row(int j, int n, int lane, const float* xin, const void* __restrict__ Wcat,
                                            float* __restrict__ la, int D, int RT, int br,
                                            const uint4 (*first)[BATCH] = nullptr) {
    float acc = 0.0f;
    constexpr int E = H16 ? 8 : 4;   // matrix elements per 16-byte load
    for (int c0 = 0; c0 < D; c0 += 64 * E * BATCH) {
        uint4 raw[BATCH];
        float4 xa[BATCH], xb[BATCH];
#pragma unroll
        for (int q = 0; q < BATCH; ++q) {
            const int c = c0 + 64 * E * q + lane * E;
            if (c < D) {   // D % 8 == 0
                const char* base = reinterpret_cast<const char*>(Wcat) + ((int64_t)j * D + c) * (H16 ? 2 : 4);
                raw[q] = (first && c0 == 0) ? (*first)[q] : *reinterpret_cast<const uint4*>(base);
                xa[q] = *reinterpret_cast<const float4*>(xin + c);
                if (H16) xb[q] = *reinterpret_cast<const float4*>(xin + c + 4);
            }
        }
#pragma unroll
        for (int q = 0; q < BATCH; ++q) {
            const int c = c0 + 64 * E * q + lane * E;
            if (c >= D) continue;
            if constexpr (H16) {
                const __half2* h = reinterpret_cast<const __half2*>(&raw[q]);
                const float xs[8] = {xa[q].x, xa[q].y, xa[q].z, xa[q].w, xb[q].x, xb[q].y, xb[q].z, xb[q].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float2 f = __half22float2(h[e]);
                    acc = fmaf(f16_round(xs[2 * e]), f.x, acc);
                    acc = fmaf(f16_round(xs[2 * e + 1]), f.y, acc);
                }
            } else {
                const float4 wv = *reinterpret_cast<const float4*>(&raw[q]);
                acc = fmaf(xa[q].x, wv.x, acc);
                acc = fmaf(xa[q].y, wv.y, acc);
                acc = fmaf(xa[q].z, wv.z, acc);
                acc = fmaf(xa[q].w, wv.w, acc);
            }
        }
    }
    float t = rwkv_wkv::wave_total(acc);
    if constexpr (H16) t = f16_round(t);
    if (br == 0) t = tanhf(t);
    else if (br == 3) t = sigmoidf_(t);
    if (lane == 0) la[(int64_t)n * RT + j] = t;
}

template <bool H16, int BATCH>
__device__ __forceinline__ void lora_in_job(int64_t job, int lane, const float* __restrict__ xmix,
                                            const void* __restrict__ Wcat, float* __restrict__ la, int D, int rw,
                                            int ra, int rv, int rg, int with_v) {
    const int RT = rw + ra + rv + rg;
    const int j = (int)(job % RT), n = (int)(job / RT);
    const int br = lora_branch(j, rw, ra, rv);
    if (br == 2 && !with_v) return;
    lora_in_row<H16, BATCH>(j, n, lane, xmix + ((int64_t)n * 4 + br) * D, Wcat, la, D, RT, br);
}

}  // namespace rwkv_x070
