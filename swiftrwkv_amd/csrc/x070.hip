// The x070 decode step around the WKV-7 / GEMV hot path, fp32 activations:
// layer norms (with the embedding row gather of the first), token shift and
// its lerps, the low-rank w / a / v / g branches, and the per-head tmix core
// (low-rank second layers, kk / k / v mixing, the WKV step and the tail).
//
// Reference: X070Generation.swift stepEager (:484-500), tmixStep (:201-296),
// cmixStep (:299-310), layerNorm_ (:505-515), l2normLast (:502-504).
// Low-rank products follow `lin` (:248-253): with fp16 matrices the input is
// rounded to fp16 and the product (fp32 accumulation) rounded to fp16, then
// widened back; with fp32 matrices the product is plain fp32.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.h"
#include "launch.h"
#include "lora_in.h"
#include "wkv7_step.h"
#include "x070_row.h"

namespace {
using namespace rwkv_wkv;
using namespace rwkv_x070;

constexpr int kRowMax = 8192;   // widest row of the row kernels


// v + (v of the DPP partner lane); CTRL quad_perm / row_half_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf,
                                                                       false));
}
// Sum over the 8 lanes 8j .. 8j+7 (lanes 1, 2 apart, then the other quad),
// the same bits in each of them.
__device__ __forceinline__ float sum8_lanes(float v) {
    v = dpp_add<0xB1>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);    // quad_perm [2,3,0,1]
    return dpp_add<0x141>(v);   // row_half_mirror
}

// Row kernels (row_geometry): all of a thread's loads are issued first.

// y[n] = LN(src(n)); src(n) = x[n] or, with `ids`, row ids[n] of the table x
// (fp32 or fp16); an id outside [0, rows) gives a NaN row.  Grid (S, N).
template <typename T, int JH>
__global__ __launch_bounds__(1024) void layer_norm_kernel(const T* __restrict__ x, const int32_t* ids, int64_t rows,
                                                          const float* __restrict__ w, const float* __restrict__ b,
                                                          float* __restrict__ y, int D, float eps) {
    const int n = blockIdx.y, T4 = blockDim.x;
    int64_t src = n;
    bool bad = false;
    if (ids) {
        const int32_t id = ids[n];
        bad = id < 0 || (int64_t)id >= rows;
        src = bad ? 0 : id;
    }
    const T* row = x + src * D;
    const int c = 4 * ((int)blockIdx.x * T4 + (int)threadIdx.x);
    float4 v[JH];
    row_chunks<JH>(row, D, threadIdx.x & 63, v);
    const float4 xo = load4(row + c), wv = load4(w + c), bv = load4(b + c);
    const float2 md = row_stats<JH>(v, row, D, threadIdx.x & 63, eps);
    const float nan = __builtin_nanf("");
    *reinterpret_cast<float4*>(y + (int64_t)n * D + c) = bad ? make_float4(nan, nan, nan, nan) : ln_apply(xo, md, wv, bv);
}

// The same rows for many rows (a parallel pass): one wave per row, four rows
// per workgroup.  The wave holds its whole row (JH >= D/256 chunks) and forms
// the statistics with row_stats, so every row is bitwise layer_norm_kernel's,
// while the row is read from memory once (layer_norm_kernel's D/256 waves per
// row each read the whole row for the statistics).  Grid N/4.
template <typename T, int JH>
__global__ __launch_bounds__(256) void layer_norm_rows_kernel(const T* __restrict__ x, const int32_t* ids,
                                                              int64_t rows, const float* __restrict__ w,
                                                              const float* __restrict__ b, float* __restrict__ y,
                                                              int N, int D, float eps) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (n >= N) return;   // whole waves; no barrier below
    int64_t src = n;
    bool bad = false;
    if (ids) {
        const int32_t id = ids[n];
        bad = id < 0 || (int64_t)id >= rows;
        src = bad ? 0 : id;
    }
    const T* row = x + src * D;
    float4 v[JH];
    row_chunks<JH>(row, D, lane, v);
    const float2 md = row_stats<JH>(v, row, D, lane, eps);
    const float nan = __builtin_nanf("");
    float* yr = y + (int64_t)n * D;
    const int nj = D >> 8;
    // a predicate, not a break: the loop unrolls and v stays in registers
    // (with a break the compiler indexed v at run time from scratch memory)
#pragma unroll
    for (int j = 0; j < JH; ++j) {
        if (j < nj) {
            const int c = 4 * (lane + 64 * j);
            *reinterpret_cast<float4*>(yr + c) =
                bad ? make_float4(nan, nan, nan, nan) : ln_apply(v[j], md, load4(w + c), load4(b + c));
        }
    }
}

// Rows from which rwkv_layer_norm takes layer_norm_rows_kernel (256
// workgroups of four rows).
constexpr int64_t kLnRowsMin = 1024;

// Token shift with its lerps (tmixStep :214-239, cmixStep :303-308) on the
// layer-normed row: xl = LN(x[n]); xx = prev[n] − xl; prev[n] ← xl;
// coefficient c gives xl + xx·coef[c].  NC = 6 (coefficients r, k, v, w, a, g):
// out0 [N, 3, D] ← (r, k, v), out1 [N, 4, D] ← (w, a, v, g), the low-rank
// branches' inputs; NC = 1: out0 [N, D].  Grid (S, N).
template <int NC, int JH>
__global__ __launch_bounds__(1024) void shift_mix_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ b, float* __restrict__ prev,
                                                         const float* __restrict__ coef, float* __restrict__ out0,
                                                         float* __restrict__ out1, int D, float eps) {
    const int n = blockIdx.y, T4 = blockDim.x;
    const float* row = x + (int64_t)n * D;
    const int c = 4 * ((int)blockIdx.x * T4 + (int)threadIdx.x);
    float4 v[JH], cv[NC];
    row_chunks<JH>(row, D, threadIdx.x & 63, v);
    const float4 xo = load4(row + c), wv = load4(w + c), bv = load4(b + c);
    const float4 pv = load4(prev + (int64_t)n * D + c);
#pragma unroll
    for (int k = 0; k < NC; ++k) cv[k] = load4(coef + (int64_t)k * D + c);
    const float2 md = row_stats<JH>(v, row, D, threadIdx.x & 63, eps);
    const float4 xl = ln_apply(xo, md, wv, bv);
    const float4 xx = shift_delta(pv, xl);
    *reinterpret_cast<float4*>(prev + (int64_t)n * D + c) = xl;
    constexpr int N0 = NC < 3 ? NC : 3;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const float4 m = shift_lerp(xl, xx, cv[k]);
        if (k < N0) *reinterpret_cast<float4*>(out0 + ((int64_t)n * N0 + k) * D + c) = m;
        // low-rank inputs: w, a, v, g ← coefficients 3, 4, 2, 5
        const int slot = k == 3 ? 0 : k == 4 ? 1 : k == 2 ? 2 : k == 5 ? 3 : -1;
        if (NC == 6 && slot >= 0) *reinterpret_cast<float4*>(out1 + ((int64_t)n * 4 + slot) * D + c) = m;
    }
}

// Widths the row kernels take (D % 256 == 0; D ≤ 4096 or 1024 | D ≤ 8192).
inline bool row_width_ok(int64_t D) { return D >= 256 && D % 256 == 0 && D <= kRowMax && (D <= 4096 || D % 1024 == 0); }

// ── low-rank first layers (tmixStep :256-276, the inner `lin` of each branch) ──
// One wave per (input row, matrix row): lora_in_job (lora_in.h).
template <bool H16>
__global__ __launch_bounds__(256) void lora_in_kernel(const float* __restrict__ xmix, const void* __restrict__ Wcat,
                                                      float* __restrict__ la, int N, int D, int rw, int ra, int rv,
                                                      int rg, int with_v) {
    const int64_t job = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (job >= (int64_t)(rw + ra + rv + rg) * N) return;   // uniform per wave
    lora_in_job<H16, 8>(job, threadIdx.x & 63, xmix, Wcat, la, D, rw, ra, rv, rg, with_v);
}

// ── the tmix core of one (input row, head) (tmixStep :256-296) ──
// Low-rank second layers for the head's 64 rows (outer `lin` + bias + the
// branch functions), kk = l2norm(k0·k_k), k = k0·(1 + (a − 1)·k_a), the value
// residual v + (v_first − v)·vv (layer 0: v_first ← v), the WKV step with
// (r, w, k, v, −kk, kk·a) on the state in place, and the tail
// ((GroupNorm(y)·lnw + lnb + Σ(r·k·r_k)·v)·gate) into out.  The step and tail
// are wkv7_step_tail_kernel's device code (same layout for the same N·H).
struct CoreArgs {
    const float* y_rkv;   // [N, 3D]: r | k0 | v0
    const float* la;      // [N, RT]
    const void* W2[4];    // w2 [D, rw], a2 [D, ra], v2 [D, rv], g2 [D, rg]
    int rank[4];
    const float* bias[3];   // w2, a2, v2 biases [D]
    const float *k_k, *k_a, *r_k, *lnw, *lnb;
    float* v_first;   // [N, D]
    float* state;     // [N, H, 64, 64]
    float* out;       // [N, D]
    const float* shift_src;   // nullable: shift_dst[n, :] ← shift_src[n, :] (the next token-shift row)
    float* shift_dst;
    int H, layer0;
    float eps;
};

template <bool R4, bool H16>
__global__ __launch_bounds__(R4 ? 1024 : 256) void tmix_core_kernel(CoreArgs A) {
    extern __shared__ float sm[];   // la row (RT) | w, a, vv, g (4 × 64) | y (64)
    const int RT = A.rank[0] + A.rank[1] + A.rank[2] + A.rank[3];
    float* lav = sm;
    float* br = sm + RT;
    float* ys = br + 4 * D;
    const int nh = blockIdx.x, n = nh / A.H, h = nh % A.H;
    const int Dm = A.H * D;
    const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane & 7, i0 = lane >> 3;
    constexpr int E = H16 ? 8 : 4;      // matrix elements per 16-byte load
    constexpr int CH = 8 * 8 * E;       // a chunk: 8 loads of each of a row's 8 lanes

    // ── loads that depend on nothing computed here, issued first ──
    const int blk = wave, l = lane;
    const int vrow = R4 ? step4_row(blk, l) : step16_row(blk, l);
    const int64_t ye = (int64_t)n * 3 * Dm + (int64_t)h * D;   // the head in the r block
    const int64_t he = (int64_t)h * D + l, vf0 = (int64_t)n * Dm + (int64_t)h * D;
    const float r = A.y_rkv[ye + l], k0 = A.y_rkv[ye + Dm + l];
    const float v0l = A.y_rkv[ye + 2 * Dm + l], v0r = A.y_rkv[ye + 2 * Dm + vrow];
    const float vfl = A.layer0 ? 0.0f : A.v_first[vf0 + l], vfr = A.layer0 ? 0.0f : A.v_first[vf0 + vrow];
    const float kkc = A.k_k[he], kac = A.k_a[he], rkc = A.r_k[he], lnwc = A.lnw[he], lnbc = A.lnb[he];
    float* st = A.state + (int64_t)nh * D * D;
    float S[R4 ? 4 : 16];
    if constexpr (R4) load_state4(st, blk, l, S);
    else load_state16(st, blk, l, S);

    // Low-rank second layers: 4 branches × 8 groups of 8 rows; a row's dot is
    // split over 8 lanes, then summed over them.  Job = branch·8 + group.
    struct Job {
        int b, i, off, rk;
        const char* wr;
        bool on;
    };
    // The branch is uniform per wave (read from the first lane) and the
    // job's matrix, rank and offset are selected among the kernel arguments,
    // not indexed: an indexed argument is a vector load whose result every
    // address below would have to wait for.
    auto job_of = [&](int job) {
        Job j;
        j.b = __builtin_amdgcn_readfirstlane(job >> 3);
        j.i = (job & 7) * 8 + i0;
        j.on = !(j.b == 2 && A.layer0);
        const int r0 = A.rank[0], r1 = A.rank[1], r2 = A.rank[2], r3 = A.rank[3];
        j.off = j.b == 0 ? 0 : j.b == 1 ? r0 : j.b == 2 ? r0 + r1 : r0 + r1 + r2;
        j.rk = j.b == 0 ? r0 : j.b == 1 ? r1 : j.b == 2 ? r2 : r3;
        const void* w = j.b == 0 ? A.W2[0] : j.b == 1 ? A.W2[1] : j.b == 2 ? A.W2[2] : A.W2[3];
        j.wr = reinterpret_cast<const char*>(w) + (int64_t)(h * D + j.i) * j.rk * (H16 ? 2 : 4);
        return j;
    };
    auto load_chunk = [&](const Job& j, int c0, uint4 (&raw)[8]) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int c = c0 + 8 * E * q + E * sub;
            if (c < j.rk) raw[q] = *reinterpret_cast<const uint4*>(j.wr + (int64_t)c * (H16 ? 2 : 4));
        }
    };
    // The low-rank inputs of two slices are read from LDS before their
    // products (16-byte reads; a row's last slices may read up to 127 floats
    // past its rank, inside the RT + 5·64 floats of LDS, values that are not
    // used); the products stay in column order.
    auto fma_chunk = [&](const Job& j, int c0, const uint4 (&raw)[8], float& acc) {
#pragma unroll
        for (int q0 = 0; q0 < 8; q0 += 2) {   // two slices' reads in flight at a time
            if (c0 + 8 * E * q0 >= j.rk) break;   // uniform: no slice from q0 on is taken
            float4 xa[2], xb[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int c = c0 + 8 * E * (q0 + u) + E * sub;
                xa[u] = *reinterpret_cast<const float4*>(lav + j.off + c);
                if constexpr (H16) xb[u] = *reinterpret_cast<const float4*>(lav + j.off + c + 4);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int q = q0 + u, c = c0 + 8 * E * q + E * sub;
                if (c >= j.rk) continue;
                if constexpr (H16) {
                    const __half2* hh = reinterpret_cast<const __half2*>(&raw[q]);
                    const float xs[8] = {xa[u].x, xa[u].y, xa[u].z, xa[u].w, xb[u].x, xb[u].y, xb[u].z, xb[u].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float2 f = __half22float2(hh[e]);
                        acc = fmaf(xs[2 * e], f.x, acc);
                        acc = fmaf(xs[2 * e + 1], f.y, acc);
                    }
                } else {
                    const float4 f = *reinterpret_cast<const float4*>(&raw[q]);
                    acc = fmaf(xa[u].x, f.x, acc);
                    acc = fmaf(xa[u].y, f.y, acc);
                    acc = fmaf(xa[u].z, f.z, acc);
                    acc = fmaf(xa[u].w, f.w, acc);
                }
            }
        }
    };
    // the row's bias (w, a, v branches), loaded with the job's first chunk
    auto bias_of = [&](const Job& j) {
        const float* bp = j.b == 0 ? A.bias[0] : j.b == 1 ? A.bias[1] : A.bias[2];
        return j.b < 3 ? bp[h * D + j.i] : 0.0f;
    };
    auto finish = [&](const Job& j, float acc, float bias) {
        acc = sum8_lanes(acc);
        if (sub == 0) {
            if constexpr (H16) acc = f16_round(acc);
            float t;
            if (j.b == 0) t = exp_fast(-0.606531f * sigmoid_fast(acc + bias));
            else if (j.b == 3) t = acc;
            else t = sigmoid_fast(acc + bias);
            br[j.b * D + j.i] = t;
        }
    };
    auto run_job = [&](const Job& j, const uint4 (&first)[8], float bias) {
        float acc = 0.0f;
        fma_chunk(j, 0, first, acc);
        for (int c0 = CH; c0 < j.rk; c0 += CH) {
            uint4 raw[8];
            load_chunk(j, c0, raw);
            fma_chunk(j, c0, raw, acc);
        }
        finish(j, acc, bias);
    };

    // sixteen waves: two jobs per wave, their first chunks in flight now
    Job jobs[R4 ? 2 : 1];
    uint4 pre[R4 ? 2 : 1][8];
    float bpre[R4 ? 2 : 1];
    if constexpr (R4) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            jobs[u] = job_of(wave + 16 * u);
            bpre[u] = 0.0f;
            if (jobs[u].on) {
                load_chunk(jobs[u], 0, pre[u]);
                bpre[u] = bias_of(jobs[u]);
            }
        }
    }
    for (int j = threadIdx.x; j < RT; j += blockDim.x) {
        const float t = A.la[(int64_t)n * RT + j];
        lav[j] = H16 ? f16_round(t) : t;
    }
    __syncthreads();
    if constexpr (R4) {
        // both jobs' products, then both branch functions in one straight
        // line, so the two dependent chains interleave
        float acc[2] = {0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (!jobs[u].on) continue;   // uniform per wave
            fma_chunk(jobs[u], 0, pre[u], acc[u]);
            for (int c0 = CH; c0 < jobs[u].rk; c0 += CH) {
                uint4 raw[8];
                load_chunk(jobs[u], c0, raw);
                fma_chunk(jobs[u], c0, raw, acc[u]);
            }
        }
        float t[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float a = sum8_lanes(acc[u]);
            if constexpr (H16) a = f16_round(a);
            const float sg = sigmoid_fast(a + bpre[u]);
            t[u] = jobs[u].b == 0 ? exp_fast(-0.606531f * sg) : jobs[u].b == 3 ? a : sg;
        }
        if (sub == 0) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
                if (jobs[u].on) br[jobs[u].b * D + jobs[u].i] = t[u];
        }
    } else {
        for (int job = wave; job < 32; job += nw) {
            const Job j = job_of(job);
            if (!j.on) continue;   // uniform per wave
            load_chunk(j, 0, pre[0]);
            run_job(j, pre[0], bias_of(j));
        }
    }
    __syncthreads();

    // ── kk, k, v, the WKV step and the tail ──
    const float kkr = k0 * kkc;
    const float kk = kkr / sqrtf(wave_total(kkr * kkr) + 1e-12f);
    const float av = br[D + l];
    const float k = k0 * (1.0f + (av - 1.0f) * kac);
    const float V = A.layer0 ? v0r : v0r + (vfr - v0r) * br[2 * D + vrow];
    const float W = br[l];
    float y;
    if constexpr (R4) y = head_step4_regs(S, st, blk, l, -kk, W, k, kk * av, r, V);
    else y = head_step16_regs(S, st, blk, l, -kk, W, k, kk * av, r, V);
    if ((R4 ? (l >> 2) : (l >> 4)) == 0) ys[vrow] = y;
    __syncthreads();
    if (blk == 0) {
        const float v = A.layer0 ? v0l : v0l + (vfl - v0l) * br[2 * D + l];
        if (A.layer0) A.v_first[vf0 + l] = v;
        A.out[(int64_t)n * Dm + he] = head_tail(ys[l], r, k, v, rkc, lnwc, lnbc, br[3 * D + l], A.eps);
        if (A.shift_dst) A.shift_dst[vf0 + l] = A.shift_src[vf0 + l];
    }
}

rwkv_status status_of(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        rwkv::set_error("%s: %s", what, hipGetErrorString(e));
        return RWKV_E_HIP;
    }
    rwkv::clear_error();
    rwkv::counters().x070++;
    return RWKV_OK;
}

}  // namespace

extern "C" {

rwkv_status rwkv_layer_norm(const void* x, rwkv_dtype x_dt, const int32_t* ids, int64_t rows, const float* w,
                            const float* b, float* y, int64_t N, int64_t D, float eps, void* stream) {
    RWKV_REQUIRE(N == 0 || (x && w && b && y), RWKV_E_NULL, "layer_norm: null buffer");
    RWKV_REQUIRE(x_dt == RWKV_F32 || x_dt == RWKV_F16, RWKV_E_DTYPE, "layer_norm: input dtype %d not f32/f16", (int)x_dt);
    RWKV_REQUIRE(N >= 0 && (N <= 65535 || (N >= kLnRowsMin && N <= INT32_MAX - 3)) && row_width_ok(D),
                 RWKV_E_SHAPE, "layer_norm: N=%lld D=%lld (D %% 256 == 0, D <= 4096 or a multiple of 1024 <= %d)",
                 (long long)N, (long long)D, kRowMax);
    RWKV_REQUIRE(!ids || rows >= 1, RWKV_E_SHAPE, "layer_norm: gather from a table of %lld rows", (long long)rows);
    if (N == 0) return RWKV_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (N >= kLnRowsMin) {
        const dim3 grid((unsigned)((N + 3) / 4)), block(256);
#define RWKV_LNR(TY, JV)                                                                                        \
    rwkv::launch(layer_norm_rows_kernel<TY, JV>, grid, block, st, reinterpret_cast<const TY*>(x), ids, rows, w, b, \
                 y, (int)N, (int)D, eps)
#define RWKV_LNR_P(TY)                \
    if (D <= 1024) RWKV_LNR(TY, 4);   \
    else if (D <= 2048) RWKV_LNR(TY, 8); \
    else if (D <= 4096) RWKV_LNR(TY, 16); \
    else RWKV_LNR(TY, 32);
        if (x_dt == RWKV_F16) {
            RWKV_LNR_P(__half)
        } else {
            RWKV_LNR_P(float)
        }
#undef RWKV_LNR_P
#undef RWKV_LNR
        return status_of("layer_norm launch");
    }
    int S, T, PS;
    row_geometry(D, S, T, PS);
    const dim3 grid((unsigned)S, (unsigned)N), block(T);
    // row chunks held per lane for the statistics: D/256 up to 8
#define RWKV_LN(TY, JV) \
    rwkv::launch(layer_norm_kernel<TY, JV>, grid, block, st, reinterpret_cast<const TY*>(x), ids, rows, w, b, y, (int)D, eps)
#define RWKV_LN_P(TY)            \
    if (D <= 1024) RWKV_LN(TY, 4); \
    else RWKV_LN(TY, 8);
    if (x_dt == RWKV_F16) {
        RWKV_LN_P(__half)
    } else {
        RWKV_LN_P(float)
    }
#undef RWKV_LN_P
#undef RWKV_LN
    return status_of("layer_norm launch");
}

rwkv_status rwkv_x070_shift_mix(const float* x, const float* lnw, const float* lnb, float* prev, const float* coef,
                                int nc, float* out0, float* out1, int64_t N, int64_t D, float eps, void* stream) {
    RWKV_REQUIRE(x && lnw && lnb && prev && coef && out0 && (nc <= 3 || out1), RWKV_E_NULL, "x070_shift_mix: null buffer");
    RWKV_REQUIRE(nc == 1 || nc == 6, RWKV_E_SHAPE, "x070_shift_mix: %d coefficients (1 or 6)", nc);
    RWKV_REQUIRE(N >= 1 && N <= 65535 && row_width_ok(D), RWKV_E_SHAPE,
                 "x070_shift_mix: N=%lld D=%lld (D %% 256 == 0, D <= 4096 or a multiple of 1024 <= %d)", (long long)N,
                 (long long)D, kRowMax);
    int S, T, PS;
    row_geometry(D, S, T, PS);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)S, (unsigned)N), block(T);
#define RWKV_SM(NCV, JV) \
    rwkv::launch(shift_mix_kernel<NCV, JV>, grid, block, st, x, lnw, lnb, prev, coef, out0, out1, (int)D, eps)
#define RWKV_SM_P(NCV)              \
    if (D <= 1024) RWKV_SM(NCV, 4); \
    else RWKV_SM(NCV, 8);
    if (nc == 6) {
        RWKV_SM_P(6)
    } else {
        RWKV_SM_P(1)
    }
#undef RWKV_SM_P
#undef RWKV_SM
    return status_of("x070_shift_mix launch");
}

rwkv_status rwkv_x070_lora_in(const float* xmix, const void* wcat, rwkv_dtype w_dt, int64_t rw, int64_t ra,
                              int64_t rv, int64_t rg, int with_v, float* la, int64_t N, int64_t D, void* stream) {
    RWKV_REQUIRE(xmix && wcat && la, RWKV_E_NULL, "x070_lora_in: null buffer");
    RWKV_REQUIRE(w_dt == RWKV_F16 || w_dt == RWKV_F32, RWKV_E_DTYPE, "x070_lora_in: matrix dtype %d not f16/f32",
                 (int)w_dt);
    RWKV_REQUIRE(rw >= 8 && ra >= 8 && rv >= 8 && rg >= 8 && rw % 8 == 0 && ra % 8 == 0 && rv % 8 == 0 && rg % 8 == 0 &&
                     rw + ra + rv + rg <= 8192,
                 RWKV_E_SHAPE, "x070_lora_in: ranks %lld/%lld/%lld/%lld (multiples of 8)", (long long)rw, (long long)ra,
                 (long long)rv, (long long)rg);
    RWKV_REQUIRE(N >= 1 && D >= 8 && D % 8 == 0 && D <= (1 << 20) && (rw + ra + rv + rg) * N <= INT32_MAX,
                 RWKV_E_SHAPE, "x070_lora_in: N=%lld D=%lld", (long long)N, (long long)D);
    const int64_t jobs = (rw + ra + rv + rg) * N;
    const dim3 grid((unsigned)((jobs + 3) / 4)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (w_dt == RWKV_F16)
        rwkv::launch(lora_in_kernel<true>, grid, block, st, xmix, wcat, la, (int)N, (int)D, (int)rw, (int)ra,
                     (int)rv, (int)rg, with_v);
    else
        rwkv::launch(lora_in_kernel<false>, grid, block, st, xmix, wcat, la, (int)N, (int)D, (int)rw, (int)ra,
                     (int)rv, (int)rg, with_v);
    return status_of("x070_lora_in launch");
}

rwkv_status rwkv_x070_tmix_core(const float* y_rkv, const float* la, const void* w2, const void* a2, const void* v2,
                                const void* g2, rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg,
                                const float* w2_bias, const float* a2_bias, const float* v2_bias, const float* k_k,
                                const float* k_a, const float* r_k, const float* lnx_w, const float* lnx_b,
                                float* v_first, int layer0, float* state, float* out, int64_t N, int64_t H, float eps,
                                const float* shift_src, float* shift_dst, void* stream) {
    RWKV_REQUIRE(y_rkv && la && w2 && a2 && g2 && w2_bias && a2_bias && k_k && k_a && r_k && lnx_w && lnx_b &&
                     v_first && state && out && (layer0 || (v2 && v2_bias)),
                 RWKV_E_NULL, "x070_tmix_core: null buffer");
    RWKV_REQUIRE((shift_src == nullptr) == (shift_dst == nullptr), RWKV_E_NULL,
                 "x070_tmix_core: shift_src and shift_dst are both set or both null");
    RWKV_REQUIRE(w_dt == RWKV_F16 || w_dt == RWKV_F32, RWKV_E_DTYPE, "x070_tmix_core: matrix dtype %d not f16/f32",
                 (int)w_dt);
    RWKV_REQUIRE(rw >= 8 && ra >= 8 && rv >= 8 && rg >= 8 && rw % 8 == 0 && ra % 8 == 0 && rv % 8 == 0 && rg % 8 == 0 &&
                     rw + ra + rv + rg <= 8192,
                 RWKV_E_SHAPE, "x070_tmix_core: ranks %lld/%lld/%lld/%lld (multiples of 8)", (long long)rw,
                 (long long)ra, (long long)rv, (long long)rg);
    RWKV_REQUIRE(N >= 1 && H >= 1 && N * H <= INT32_MAX && H * D <= (1 << 20), RWKV_E_SHAPE,
                 "x070_tmix_core: N=%lld H=%lld", (long long)N, (long long)H);
    CoreArgs A{};
    A.y_rkv = y_rkv;
    A.la = la;
    A.W2[0] = w2; A.W2[1] = a2; A.W2[2] = v2; A.W2[3] = g2;
    A.rank[0] = (int)rw; A.rank[1] = (int)ra; A.rank[2] = (int)rv; A.rank[3] = (int)rg;
    A.bias[0] = w2_bias; A.bias[1] = a2_bias; A.bias[2] = v2_bias;
    A.k_k = k_k; A.k_a = k_a; A.r_k = r_k; A.lnw = lnx_w; A.lnb = lnx_b;
    A.v_first = v_first; A.state = state; A.out = out;
    A.shift_src = shift_src; A.shift_dst = shift_dst;
    A.H = (int)H; A.layer0 = layer0 ? 1 : 0; A.eps = eps;
    const size_t lds = (size_t)(rw + ra + rv + rg + 5 * D) * 4;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)(N * H));
    const bool r4 = use_rows4(N * H), h16 = w_dt == RWKV_F16;
    if (r4 && h16) rwkv::launch_lds(tmix_core_kernel<true, true>, grid, dim3(1024), lds, st, A);
    else if (r4) rwkv::launch_lds(tmix_core_kernel<true, false>, grid, dim3(1024), lds, st, A);
    else if (h16) rwkv::launch_lds(tmix_core_kernel<false, true>, grid, dim3(256), lds, st, A);
    else rwkv::launch_lds(tmix_core_kernel<false, false>, grid, dim3(256), lds, st, A);
    return status_of("x070_tmix_core launch");
}

}  // extern "C"
