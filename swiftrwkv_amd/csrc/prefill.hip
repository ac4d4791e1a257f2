// The parallel (prefill) pass of the x070 block around its matrix products:
// the token shift over a whole sequence and the time-mix arithmetic between
// the projections / low-rank branches and the WKV-7 recurrence, for B rows of
// T tokens with right padding (Sources/RWKVGen/RWKVBlock.swift:145-264,
// rwkvTokenShift and rwkvTmixForward; BatchGenerate.swift:37-53).
//
// Rows are [B, T] flattened (n = b·T + t); row b holds lengths[b] real
// tokens, the rest is padding.  The padding is made neutral for the
// recurrence exactly as the reference does (w ← 1, k ← 0, b ← 0 at pad steps,
// RWKVBlock.swift:232-237): the state of a row stops at its last real token,
// whatever its neighbours or the amount of padding.  Outputs at pad positions
// are computed and left unused.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "common.h"
#include "launch.h"
#include "lora_in.h"
#include "wkv7_step.h"

namespace {

using rwkv_wkv::wave_total;
using rwkv_x070::exp_fast;
using rwkv_x070::sigmoid_fast;

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Token shift over the sequence with its lerps (rwkvTokenShift + the x_c
// lerps of rwkvTmixForward / rwkvCmixForward): for the layer-normed rows xl,
// prev_t = xl[t − 1] (t > 0) or the carried shift state prev_in[b] (zeros when
// NULL); m_c = xl + (prev_t − xl)·coef[c].  Coefficients [0, n0) go to y0
// (fp16 or fp32, element (n, c) at n·y0_row + c·y0_coef); with y1, the
// coefficients from y1_first on also go to y1 (fp32).  prev_out[b] ← xl[b, lengths[b] − 1] (the shift state of the row's
// last real token, gatherLast; may be prev_in).  One thread per 4 columns of one row.
// I32: the thread index and its divisions in 32 bits (fewer than 2^31
// threads; two 64-bit divisions per 4 columns cost more than the loads).
template <int NC, bool F16, bool I32>
__global__ __launch_bounds__(256) void seq_shift_kernel(const float* __restrict__ xl, const float* prev_in,
                                                        float* prev_out, const int32_t* __restrict__ lengths,
                                                        const float* __restrict__ coef, int n0, void* __restrict__ y0,
                                                        int64_t y0_row, int64_t y0_coef, float* __restrict__ y1,
                                                        int64_t y1_row, int64_t y1_coef, int y1_first, int T, int D,
                                                        int64_t total) {
    int64_t n;
    int c, b, t;
    if constexpr (I32) {
        const uint32_t gid = blockIdx.x * 256u + threadIdx.x, D4 = (uint32_t)(D >> 2);
        if (gid >= (uint32_t)total) return;
        const uint32_t n32 = gid / D4, b32 = n32 / (uint32_t)T;
        n = n32;
        c = (int)(gid - n32 * D4) * 4;
        b = (int)b32;
        t = (int)(n32 - b32 * (uint32_t)T);
    } else {
        const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (gid >= total) return;
        const int D4 = D >> 2;
        n = gid / D4;
        c = (int)(gid - n * D4) * 4;
        b = (int)(n / T);
        t = (int)(n - (int64_t)b * T);
    }
    const float4 x = ld4(xl + n * D + c);
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t > 0) p = ld4(xl + (n - 1) * D + c);
    else if (prev_in) p = ld4(prev_in + (int64_t)b * D + c);
    // the thread at t = 0 both reads the carried state and writes the new
    // one (xl of the row's last real token), so prev_out may be prev_in;
    // lengths past T read the row's last token (every read stays in the row)
    const int len = lengths ? min(lengths[b], T) : T;
    if (t == 0 && len > 0)
        *reinterpret_cast<float4*>(prev_out + (int64_t)b * D + c) = len == 1 ? x : ld4(xl + (n + len - 1) * D + c);
    const float4 xx = make_float4(p.x - x.x, p.y - x.y, p.z - x.z, p.w - x.w);
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const float4 q = ld4(coef + (int64_t)k * D + c);
        const float4 m = make_float4(x.x + xx.x * q.x, x.y + xx.y * q.y, x.z + xx.z * q.z, x.w + xx.w * q.w);
        if (k < n0) {
            const int64_t o = n * y0_row + k * y0_coef + c;
            if constexpr (F16) {
                __half2 h[2] = {__floats2half2_rn(m.x, m.y), __floats2half2_rn(m.z, m.w)};
                *reinterpret_cast<uint2*>(reinterpret_cast<__half*>(y0) + o) = *reinterpret_cast<uint2*>(h);
            } else {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(y0) + o) = m;
            }
        }
        if (y1 && k >= y1_first) *reinterpret_cast<float4*>(y1 + n * y1_row + k * y1_coef + c) = m;
    }
}

// The time-mix arithmetic between the projections and the WKV recurrence
// (rwkvTmixForward, RWKVBlock.swift:185-237), one wave per (row, head), lane
// = channel of the head.  Inputs: y_rkv [M, 3D] = r | k0 | v0 (the r/k/v
// projections), the low-rank second layers ww, aa, vv (pre-bias) [M, D]
// (vv NULL at layer 0).  Computes
//   w = exp(−0.606531·σ(ww + w_bias)), a = σ(aa + a_bias),
//   kk = l2norm(k0·k_k) over the head, k = k0·(1 + (a − 1)·k_a),
//   v = layer 0 ? v0 (v_first ← v0) : v0 + (v_first − v0)·σ(vv + v_bias),
// and writes the recurrence inputs r, w, k, v, a_w = −kk, b_w = kk·a [M, D]
// with pad steps neutral (w ← 1, k ← 0, b_w ← 0), plus k_bonus = k unmasked
// (the tail's bonus term uses it, RWKVBlock.swift:287-289).  The branch
// functions are the decode core's (exp2 / reciprocal based, ~1e-6).
__global__ __launch_bounds__(256) void seq_tmix_pre_kernel(
    const float* __restrict__ y_rkv, const float* __restrict__ ww, const float* __restrict__ aa,
    const float* __restrict__ vv, const float* __restrict__ w_bias, const float* __restrict__ a_bias,
    const float* __restrict__ v_bias, const float* __restrict__ k_k, const float* __restrict__ k_a,
    float* __restrict__ v_first, int layer0, const int32_t* __restrict__ lengths, float* __restrict__ r_o,
    float* __restrict__ w_o, float* __restrict__ k_o, float* __restrict__ v_o, float* __restrict__ a_o,
    float* __restrict__ b_o, float* __restrict__ kb_o, int T, int H, int64_t units) {
    // units < 2^30 (checked on the host): 32-bit index math
    const uint32_t unit = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (unit >= (uint32_t)units) return;   // uniform per wave
    const int lane = threadIdx.x & 63;
    const int D = H * 64;
    const uint32_t n32 = unit / (uint32_t)H, b32 = n32 / (uint32_t)T;
    const int64_t n = n32;
    const int h = (int)(unit - n32 * (uint32_t)H);
    const int ch = h * 64 + lane;
    const int b = (int)b32, t = (int)(n32 - b32 * (uint32_t)T);
    const bool real = t < (lengths ? lengths[b] : T);
    const int64_t e = n * D + ch;
    const float* yr = y_rkv + n * 3 * D;
    const float r = yr[ch], k0 = yr[D + ch], v0 = yr[2 * D + ch];
    const float w = exp_fast(-0.606531f * sigmoid_fast(ww[e] + w_bias[ch]));
    const float a = sigmoid_fast(aa[e] + a_bias[ch]);
    float v = v0;
    if (layer0) {
        v_first[e] = v0;
    } else {
        const float vf = v_first[e];
        v = v0 + (vf - v0) * sigmoid_fast(vv[e] + v_bias[ch]);
    }
    const float kkr = k0 * k_k[ch];
    const float kk = kkr / sqrtf(wave_total(kkr * kkr) + 1e-12f);
    const float k = k0 * (1.0f + (a - 1.0f) * k_a[ch]);
    r_o[e] = r;
    v_o[e] = v;
    a_o[e] = -kk;
    kb_o[e] = k;
    w_o[e] = real ? w : 1.0f;
    k_o[e] = real ? k : 0.0f;
    b_o[e] = real ? kk * a : 0.0f;
}

// ── the low-rank branches of the parallel pass (rwkvTmixForward,
// RWKVBlock.swift:185-226) on the matrix cores ──
// Each branch is two products: h = act(x·Aᵀ) (A [rank, D]; tanh for w,
// sigmoid for the gate, none for a and v), then h·Bᵀ (B [D, rank]).  The
// activations are fp32 and the matrices fp16 or fp32: fp16 values widen
// exactly, so these are fp32 products (MLX promotes the fp16 weight; no `lin`
// narrowing on this path).  One launch forms a stage of all branches: a job
// per branch (grid z), y = act(x·Wᵀ) for x [M, K] (row stride ldx), W [N, K].
// A workgroup of 4 waves computes a 64 × 64 tile of y; wave w the 32 × 32
// sub-tile (w >> 1, w & 1) as 2 × 2 tiles of v_mfma_f32_16x16x4_f32.  Four
// MFMAs take 16 K at a time: lane i + 16g provides A[row i][k0 + 4g + r] and
// B[k0 + 4g + r][col i] in MFMA r (the sum over k does not depend on which K
// slot carries which k), so each lane reads 16 contiguous bytes of an x row
// and 4 contiguous weights of a W row.  Sums in fp32, in a fixed order.
struct LoraJob {
    const float* x;
    const void* w;
    float* y;
    int N, K, ldx, ldy, act;   // act: 0 none, 1 tanh, 2 sigmoid
};
struct LoraJobs {
    LoraJob j[4];
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma4(float4 a, float4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
}

template <typename TW>
__device__ __forceinline__ float4 ldw4(const TW* p) {
    if constexpr (sizeof(TW) == 4) {
        return *reinterpret_cast<const float4*>(p);
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        const float2 a = __half22float2(*reinterpret_cast<const __half2*>(&u.x));
        const float2 c = __half22float2(*reinterpret_cast<const __half2*>(&u.y));
        return make_float4(a.x, a.y, c.x, c.y);
    }
}

// MT × NT tiles of 16 × 16 per wave; the four waves 2 × 2, so a workgroup
// covers (32·MT) rows × (32·NT) columns.
template <typename TW, int MT, int NT>
__global__ __launch_bounds__(256) void seq_lora_kernel(LoraJobs jobs, int M) {
    constexpr int BM = 32 * MT, BN = 32 * NT;
    const LoraJob J = jobs.j[blockIdx.z];
    if ((int)blockIdx.x * BN >= J.N) return;   // this job has fewer column tiles (uniform)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, i = lane & 15;
    const int row0 = (int)blockIdx.y * BM + 16 * MT * (wave >> 1), col0 = (int)blockIdx.x * BN + 16 * NT * (wave & 1);
    // rows / columns past the end read the last one (results not stored)
    const float* xr[MT];
    const TW* wr[NT];
#pragma unroll
    for (int t = 0; t < MT; ++t) xr[t] = J.x + (int64_t)min(row0 + 16 * t + i, M - 1) * J.ldx + 4 * g;
#pragma unroll
    for (int t = 0; t < NT; ++t)
        wr[t] = reinterpret_cast<const TW*>(J.w) + (int64_t)min(col0 + 16 * t + i, J.N - 1) * J.K + 4 * g;
    f32x4 acc[MT][NT];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    // one K step of 16 loaded ahead
    float4 xa[MT], wb[NT];
#pragma unroll
    for (int t = 0; t < MT; ++t) xa[t] = *reinterpret_cast<const float4*>(xr[t]);
#pragma unroll
    for (int t = 0; t < NT; ++t) wb[t] = ldw4(wr[t]);
    for (int k0 = 0; k0 < J.K; k0 += 16) {
        const int kn = min(k0 + 16, J.K - 16);   // the last step re-reads itself
        float4 xn[MT], wn[NT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xn[t] = *reinterpret_cast<const float4*>(xr[t] + kn);
#pragma unroll
        for (int t = 0; t < NT; ++t) wn[t] = ldw4(wr[t] + kn);
#pragma unroll
        for (int a = 0; a < MT; ++a)
#pragma unroll
            for (int b = 0; b < NT; ++b) acc[a][b] = mfma4(xa[a], wb[b], acc[a][b]);
#pragma unroll
        for (int t = 0; t < MT; ++t) xa[t] = xn[t];
#pragma unroll
        for (int t = 0; t < NT; ++t) wb[t] = wn[t];
    }
    // accumulator lane i + 16g: rows 4g + r, column i of each 16 × 16 tile
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b) {
            const int col = col0 + 16 * b + i;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + 16 * a + 4 * g + r;
                float v = acc[a][b][r];
                if (J.act == 1) v = tanhf(v);
                else if (J.act == 2) v = 1.0f / (1.0f + expf(-v));
                if (row < M && col < J.N) J.y[(int64_t)row * J.ldy + col] = v;
            }
        }
}

// Few rows (short prompts): the tiles above leave most of the GPU idle and
// each wave walks the whole K (768–4096 for the inner products) one step of
// loads ahead.  Here a workgroup computes a 32 × 32 tile of y and its four
// waves split K: wave q takes the K steps [q·S/4, (q+1)·S/4) of the S = K/16
// steps as 2 × 2 tiles of 16 × 16 (the MFMA lane layout of seq_lora_kernel),
// with groups of four steps loaded one group ahead in two register sets (fp16
// weights stay packed until their group is used).  The four partial tiles are
// summed through LDS in wave order, ((p0 + p1) + p2) + p3, then activated.
// Every output's arithmetic depends only on its row of x, its row of W and K.
template <typename TW>
struct LoraRaw {
    using T = float4;
};
template <>
struct LoraRaw<__half> {
    using T = uint2;
};

template <typename TW>
__device__ __forceinline__ typename LoraRaw<TW>::T ldraw(const TW* p) {
    return *reinterpret_cast<const typename LoraRaw<TW>::T*>(p);
}
__device__ __forceinline__ float4 widen(float4 v) { return v; }
__device__ __forceinline__ float4 widen(uint2 u) {
    const float2 a = __half22float2(*reinterpret_cast<const __half2*>(&u.x));
    const float2 c = __half22float2(*reinterpret_cast<const __half2*>(&u.y));
    return make_float4(a.x, a.y, c.x, c.y);
}

constexpr int64_t kLoraKsMaxRows = 512;

template <typename TW>
__global__ __launch_bounds__(256) void seq_lora_ks_kernel(LoraJobs jobs, int M) {
    using WR = typename LoraRaw<TW>::T;
    const LoraJob J = jobs.j[blockIdx.z];
    if ((int)blockIdx.x * 32 >= J.N) return;   // this job has fewer column tiles (uniform)
    __shared__ float red[4 * 16 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, i = lane & 15;
    const int row0 = (int)blockIdx.y * 32, col0 = (int)blockIdx.x * 32;
    // rows / columns past the end read the last one (results not stored)
    const float* xr[2];
    const TW* wr[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        xr[t] = J.x + (int64_t)min(row0 + 16 * t + i, M - 1) * J.ldx + 4 * g;
        wr[t] = reinterpret_cast<const TW*>(J.w) + (int64_t)min(col0 + 16 * t + i, J.N - 1) * J.K + 4 * g;
    }
    const int S = J.K >> 4;
    const int s0 = wave * S / 4, s1 = (wave + 1) * S / 4;
    f32x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    float4 xa[4][2], xb[4][2];
    WR wa[4][2], wb[4][2];
    // a group: steps s .. s + 3, the ones past s1 re-read step s1 − 1 and are
    // skipped when used (wave-uniform)
    auto load = [&](float4 (&x)[4][2], WR (&w)[4][2], int s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 16 * min(s + j, s1 - 1);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                x[j][t] = *reinterpret_cast<const float4*>(xr[t] + k);
                w[j][t] = ldraw(wr[t] + k);
            }
        }
    };
    auto use = [&](const float4 (&x)[4][2], const WR (&w)[4][2], int s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (s + j < s1) {
                const float4 w0 = widen(w[j][0]), w1 = widen(w[j][1]);
#pragma unroll
                for (int a = 0; a < 2; ++a) {
                    acc[a][0] = mfma4(x[j][a], w0, acc[a][0]);
                    acc[a][1] = mfma4(x[j][a], w1, acc[a][1]);
                }
            }
        }
    };
    if (s0 < s1) {
        load(xa, wa, s0);
        for (int s = s0; s < s1; s += 8) {
            if (s + 4 < s1) load(xb, wb, s + 4);
            use(xa, wa, s);
            if (s + 4 >= s1) break;
            if (s + 8 < s1) load(xa, wa, s + 8);
            use(xb, wb, s + 4);
        }
    }
    // partial tiles: red[wave][a][b][r][lane]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[((wave * 4 + a * 2 + b) * 4 + r) * 64 + lane] = acc[a][b][r];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = threadIdx.x + 256 * u;   // (a, b, r, lane) of the tile
        const int ln = e & 63, r = (e >> 6) & 3, b = (e >> 8) & 1, a = e >> 9;
        float v = red[e];
#pragma unroll
        for (int q = 1; q < 4; ++q) v += red[q * 1024 + e];
        const int row = row0 + 16 * a + 4 * (ln >> 4) + r, col = col0 + 16 * b + (ln & 15);
        if (J.act == 1) v = tanhf(v);
        else if (J.act == 2) v = 1.0f / (1.0f + expf(-v));
        if (row < M && col < J.N) J.y[(int64_t)row * J.ldy + col] = v;
    }
}

// ── long passes: the fp32 activations as two fp16 parts on the fp16 matrix cores ──
// The same y = act(x·Wᵀ) for fp16 W [N, K] with x [M, K] fp32 written
// x = hi + lo, hi = fp16(x), lo = fp16(x − hi) (x − hi is exact in fp32):
// hi·w and lo·w are exact in fp32 (11-bit significands) and both sum into
// one fp32 accumulator on v_mfma_f32_16x16x32_f16, at 2 fp16 MFMAs where the
// fp32 path takes 8 fp32 ones for the same products.  x enters with 22 of
// its 24 significant bits (error ≤ 2^-22·|x|; ≤ 2^-25 absolute where lo is
// an fp16 subnormal), below the fp32 sum's own rounding over these K; |x|
// must stay below 65504 (layer-normed rows and the branch activations are
// far below).  A workgroup of 4 waves computes a 128 × 128 tile of y in
// stages of 32 columns: hi, lo and W staged in LDS as 64-byte rows whose
// 16-byte chunk c sits at c ^ ((row >> 1) & 3) (8 consecutive rows read one
// chunk column from distinct banks; padded 80-byte rows counted 5.5
// conflict cycles per LDS instruction), wave w the 64 × 64 sub-tile
// (w >> 1, w & 1) as 4 × 4 accumulator tiles.  Two register sets alternate
// (the loop body is two stages), so a stage's loads are issued more than a
// stage before they are written to LDS.  Tiles run row block by row block,
// every job's column tiles of a row block together, the XCDs (workgroups
// x, x + 8, ...) each taking a contiguous run: a row block's activations
// are fetched into one L2, and every XCD gets its share of each job (the
// jobs' depths differ: 3 to 15 stages in the second launch at 7B-class
// width; job by job, the deep one landed on two XCDs and took 405 against
// 269 µs).
constexpr int LT = 128;    // tile rows = tile columns
constexpr int LK = 32;     // columns per stage

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

struct SplitJob {
    const float* x;
    const _Float16* w;
    float* y;
    int N, K, ldx, ldy, act;   // act: 0 none, 1 tanh, 2 sigmoid
};
struct SplitJobs {
    SplitJob j[4];
    int first[5];   // column tiles of jobs before j within a row block; first[4] = all of them
};

__device__ __forceinline__ int lswz(int row, int c) { return 8 * (c ^ ((row >> 1) & 3)); }

__global__ __launch_bounds__(256, 2) void lora_split_kernel(SplitJobs jobs, int M) {
    __shared__ __attribute__((aligned(16))) _Float16 sm[2][3][LT][LK];   // [buffer][hi, lo, W][row][column]
    const int per = jobs.first[4], total = ((M + LT - 1) / LT) * per;
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    const int t = xcd * (total >> 3) + min(xcd, total & 7) + loc;
    const int rb = t / per, rem = t - rb * per;
    int jb = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q) jb += rem >= jobs.first[q] ? 1 : 0;
    const SplitJob J = jobs.j[jb];
    const int n0 = (rem - jobs.first[jb]) * LT, m0 = rb * LT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, li = lane & 15;
    const int nst = J.K / LK;
    // staging: thread t → row t >> 1, chunks 2·(t & 1), +1 of the stage
    // (rows past the end read the last one; their results are not stored)
    const int sr = tid >> 1, sh = tid & 1;
    const float* xrow = J.x + (int64_t)min(m0 + sr, M - 1) * J.ldx + 16 * sh;
    const _Float16* wrow = J.w + (int64_t)min(n0 + sr, J.N - 1) * J.K + 16 * sh;
    struct Set {
        float4 a[4];
        uint4 b[2];
    };
    auto gload = [&](Set& s, int st) {
        st = min(st, nst - 1);
        const float4* p = reinterpret_cast<const float4*>(xrow + st * LK);
        const uint4* q = reinterpret_cast<const uint4*>(wrow + st * LK);
#pragma unroll
        for (int e = 0; e < 4; ++e) s.a[e] = p[e];
        s.b[0] = q[0];
        s.b[1] = q[1];
    };
    auto swrite = [&](int buf, const Set& s) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float v[8] = {s.a[2 * e].x, s.a[2 * e].y, s.a[2 * e].z, s.a[2 * e].w,
                                s.a[2 * e + 1].x, s.a[2 * e + 1].y, s.a[2 * e + 1].z, s.a[2 * e + 1].w};
            half8v hi, lo;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                hi[c] = (_Float16)v[c];
                lo[c] = (_Float16)(v[c] - (float)hi[c]);
            }
            const int off = lswz(sr, 2 * sh + e);
            *reinterpret_cast<half8v*>(&sm[buf][0][sr][off]) = hi;
            *reinterpret_cast<half8v*>(&sm[buf][1][sr][off]) = lo;
            *reinterpret_cast<uint4*>(&sm[buf][2][sr][off]) = s.b[e];
        }
    };
    const int wm = wave >> 1, wn = wave & 1;
    const int rc = lswz(li, gq);   // operand rows li + 16·tile: (row >> 1) & 3 = (li >> 1) & 3
    f32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto products = [&](int buf) {
        half8v bv[4], hv[4], lv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) bv[b] = *reinterpret_cast<const half8v*>(&sm[buf][2][64 * wn + 16 * b + li][rc]);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            hv[a] = *reinterpret_cast<const half8v*>(&sm[buf][0][64 * wm + 16 * a + li][rc]);
            lv[a] = *reinterpret_cast<const half8v*>(&sm[buf][1][64 * wm + 16 * a + li][rc]);
        }
        // W as the A operand: accumulator tile (a, b) holds y columns 16b + 4g + r
        // of row 16a + i in lane i + 16g, four consecutive columns per lane
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bv[b], hv[a], acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bv[b], lv[a], acc[a][b], 0, 0, 0);
            }
    };
    // buffer `buf` holds stage st; `ld` receives stage st + 2; `wr` (stage
    // st + 1, loaded a stage ago) goes to the other buffer
    auto stage = [&](int buf, Set& ld, int st, const Set& wr) {
        gload(ld, st + 2);
        __builtin_amdgcn_sched_barrier(0);
        products(buf);
        swrite(buf ^ 1, wr);
        __syncthreads();
    };
    Set sa, sb;
    gload(sa, 0);
    swrite(0, sa);
    gload(sa, 1);
    __syncthreads();
    int st = 0;
    for (; st + 1 < nst; st += 2) {
        stage(0, sb, st, sa);
        stage(1, sa, st + 1, sb);
    }
    if (st < nst) stage(0, sb, st, sa);   // an odd stage count: the last stage (its LDS write is unused)

    // lane i + 16g: row 16a + i, columns 16b + 4g .. +3 (N and ldy are
    // multiples of 16 and 4: a column group is wholly in or out)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int row = m0 + 64 * wm + 16 * a + li;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int col = n0 + 64 * wn + 16 * b + 4 * gq;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] = acc[a][b][r];
                if (J.act == 1) v[r] = tanhf(v[r]);
                else if (J.act == 2) v[r] = 1.0f / (1.0f + expf(-v[r]));
            }
            if (row < M && col < J.N)
                *reinterpret_cast<float4*>(J.y + (int64_t)row * J.ldy + col) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

// The two-part kernel takes long passes (M·D above 2^21) with fp16
// matrices, ranks and D multiples of 32; the fp32 kernel everything else.
bool lora_split_takes(int64_t M, int64_t D, rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg) {
    return w_dt == RWKV_F16 && M * D > ((int64_t)1 << 21) && D % 32 == 0 && rw % 32 == 0 && ra % 32 == 0 &&
           rv % 32 == 0 && rg % 32 == 0;
}

}  // namespace

extern "C" {

int rwkv_x070_seq_lora_split(int64_t M, int64_t D, rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg) {
    return lora_split_takes(M, D, w_dt, rw, ra, rv, rg);
}

rwkv_status rwkv_x070_seq_shift_mix(const float* xl, const float* prev_in, float* prev_out, const int32_t* lengths,
                                    const float* coef, int nc, int n0, void* y0, rwkv_dtype y0_dt, int64_t y0_row,
                                    int64_t y0_coef, float* y1, int64_t y1_row, int64_t y1_coef, int y1_first,
                                    int64_t B, int64_t T,
                                    int64_t D, void* stream) {
    RWKV_REQUIRE(xl && prev_out && coef && y0, RWKV_E_NULL, "x070_seq_shift_mix: null buffer");
    RWKV_REQUIRE(nc == 1 || nc == 6, RWKV_E_SHAPE, "x070_seq_shift_mix: %d coefficients (1 or 6)", nc);
    RWKV_REQUIRE(n0 >= 1 && n0 <= nc, RWKV_E_SHAPE, "x070_seq_shift_mix: n0 = %d", n0);
    RWKV_REQUIRE(y0_dt == RWKV_F32 || y0_dt == RWKV_F16, RWKV_E_DTYPE, "x070_seq_shift_mix: y0 must be f32 or f16");
    RWKV_REQUIRE(B >= 1 && T >= 1 && D >= 4 && D % 4 == 0 && B * T <= ((int64_t)1 << 26), RWKV_E_SHAPE,
                 "x070_seq_shift_mix: B=%lld T=%lld D=%lld", (long long)B, (long long)T, (long long)D);
    RWKV_REQUIRE(y0_row % 4 == 0 && y0_coef % 4 == 0 && (!y1 || (y1_row % 4 == 0 && y1_coef % 4 == 0)),
                 RWKV_E_SHAPE, "x070_seq_shift_mix: output strides must be multiples of 4");
    RWKV_REQUIRE(y1_first >= 0 && y1_first <= nc, RWKV_E_SHAPE, "x070_seq_shift_mix: y1_first = %d", y1_first);
    const int64_t total = B * T * (D / 4);
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool f16 = y0_dt == RWKV_F16;
    const bool i32 = total < INT32_MAX;
#define RWKV_SHIFT(NCV, F)                                                                                            \
    do {                                                                                                              \
        if (i32)                                                                                                      \
            rwkv::launch(seq_shift_kernel<NCV, F, true>, grid, block, s, xl, prev_in, prev_out, lengths, coef, n0,    \
                         y0, y0_row, y0_coef, y1, y1_row, y1_coef, y1_first, (int)T, (int)D, total);                  \
        else                                                                                                          \
            rwkv::launch(seq_shift_kernel<NCV, F, false>, grid, block, s, xl, prev_in, prev_out, lengths, coef, n0,   \
                         y0, y0_row, y0_coef, y1, y1_row, y1_coef, y1_first, (int)T, (int)D, total);                  \
    } while (0)
    if (nc == 6) {
        if (f16) RWKV_SHIFT(6, true);
        else RWKV_SHIFT(6, false);
    } else {
        if (f16) RWKV_SHIFT(1, true);
        else RWKV_SHIFT(1, false);
    }
#undef RWKV_SHIFT
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "x070_seq_shift_mix: launch failed");
    rwkv::counters().x070.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status rwkv_x070_seq_tmix_pre(const float* y_rkv, const float* ww, const float* aa, const float* vv,
                                   const float* w_bias, const float* a_bias, const float* v_bias, const float* k_k,
                                   const float* k_a, float* v_first, int layer0, const int32_t* lengths, float* r,
                                   float* w, float* k, float* v, float* a, float* b, float* k_bonus, int64_t B,
                                   int64_t T, int64_t H, void* stream) {
    RWKV_REQUIRE(y_rkv && ww && aa && w_bias && a_bias && k_k && k_a && v_first && r && w && k && v && a && b &&
                     k_bonus && (layer0 || (vv && v_bias)),
                 RWKV_E_NULL, "x070_seq_tmix_pre: null buffer");
    RWKV_REQUIRE(B >= 1 && T >= 1 && H >= 1 && B * T * H <= ((int64_t)1 << 30), RWKV_E_SHAPE,
                 "x070_seq_tmix_pre: B=%lld T=%lld H=%lld", (long long)B, (long long)T, (long long)H);
    const int64_t units = B * T * H;
    const dim3 grid((unsigned)((units + 3) / 4)), block(256);
    rwkv::launch(seq_tmix_pre_kernel, grid, block, reinterpret_cast<hipStream_t>(stream), y_rkv, ww, aa, vv, w_bias,
                 a_bias, v_bias, k_k, k_a, v_first, layer0, lengths, r, w, k, v, a, b, k_bonus, (int)T, (int)H, units);
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "x070_seq_tmix_pre: launch failed");
    rwkv::counters().x070.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status rwkv_x070_seq_lora(const float* mix, int64_t M, int64_t D, const void* wcat, const void* w2,
                               const void* a2, const void* v2, const void* g2, rwkv_dtype w_dt, int64_t rw,
                               int64_t ra, int64_t rv, int64_t rg, int with_v, float* la, float* ww, float* aa,
                               float* vv, float* gate, void* stream) {
    RWKV_REQUIRE(mix && wcat && w2 && a2 && g2 && la && ww && aa && gate && (!with_v || (v2 && vv)), RWKV_E_NULL,
                 "x070_seq_lora: null buffer");
    RWKV_REQUIRE(w_dt == RWKV_F16 || w_dt == RWKV_F32, RWKV_E_DTYPE, "x070_seq_lora: matrices f16 or f32 (dtype %d)",
                 (int)w_dt);
    RWKV_REQUIRE(M >= 1 && M <= ((int64_t)1 << 24) && D >= 16 && D % 16 == 0 && D <= ((int64_t)1 << 20) &&
                     M * D <= ((int64_t)1 << 31),
                 RWKV_E_SHAPE, "x070_seq_lora: M=%lld D=%lld (D %% 16 == 0)", (long long)M, (long long)D);
    RWKV_REQUIRE(rw >= 16 && ra >= 16 && rv >= 16 && rg >= 16 && rw % 16 == 0 && ra % 16 == 0 && rv % 16 == 0 &&
                     rg % 16 == 0 && rw + ra + rv + rg <= 8192,
                 RWKV_E_SHAPE, "x070_seq_lora: ranks %lld/%lld/%lld/%lld (multiples of 16)", (long long)rw,
                 (long long)ra, (long long)rv, (long long)rg);
    const int64_t RT = rw + ra + rv + rg;
    RWKV_REQUIRE(M * RT <= ((int64_t)1 << 31), RWKV_E_SHAPE, "x070_seq_lora: M·ranks too large");
    const int64_t es = w_dt == RWKV_F16 ? 2 : 4;
    const uintptr_t al = (uintptr_t)mix | (uintptr_t)la | (uintptr_t)wcat | (uintptr_t)w2 | (uintptr_t)a2 |
                         (uintptr_t)g2 | (uintptr_t)(with_v ? v2 : w2);
    RWKV_REQUIRE(al % 16 == 0, RWKV_E_SHAPE, "x070_seq_lora: buffers must be 16-byte aligned");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t md = M * D;
    // mix rows: coefficient order r, k, v, w, a, g (rwkv_x070_seq_shift_mix)
    const float* xin[4] = {mix + 3 * md, mix + 4 * md, mix + 2 * md, mix + 5 * md};
    const int64_t rk[4] = {rw, ra, rv, rg};
    const void* outer[4] = {w2, a2, v2, g2};
    float* dst[4] = {ww, aa, vv, gate};
    const int act[4] = {1, 0, 0, 2};
    // stage 1: la[:, branch] = act(x_branch · A_branchᵀ); stage 2: dst = la[:, branch] · B_branchᵀ
    LoraJobs s1{}, s2{};
    int n = 0;
    int64_t off = 0, maxn1 = 0;
    for (int b = 0; b < 4; ++b) {
        if (b == 2 && !with_v) {
            off += rk[b];
            continue;
        }
        s1.j[n] = LoraJob{xin[b], reinterpret_cast<const char*>(wcat) + off * D * es, la + off, (int)rk[b], (int)D,
                          (int)D, (int)RT, act[b]};
        s2.j[n] = LoraJob{la + off, outer[b], dst[b], (int)D, (int)rk[b], (int)RT, (int)D, 0};
        maxn1 = rk[b] > maxn1 ? rk[b] : maxn1;
        off += rk[b];
        ++n;
    }
    if (lora_split_takes(M, D, w_dt, rw, ra, rv, rg)) {
        const uintptr_t ao = (uintptr_t)ww | (uintptr_t)aa | (uintptr_t)gate | (uintptr_t)(with_v ? vv : ww);
        RWKV_REQUIRE(ao % 16 == 0, RWKV_E_SHAPE, "x070_seq_lora: outputs must be 16-byte aligned");
        SplitJobs t1{}, t2{};
        int c1 = 0, c2 = 0;
        for (int j = 0; j < 4; ++j) {
            t1.first[j] = c1;
            t2.first[j] = c2;
            if (j >= n) continue;   // fewer jobs: first[j] = all tiles, never selected
            const LoraJob& a = s1.j[j];
            const LoraJob& b = s2.j[j];
            t1.j[j] = SplitJob{a.x, reinterpret_cast<const _Float16*>(a.w), a.y, a.N, a.K, a.ldx, a.ldy, a.act};
            t2.j[j] = SplitJob{b.x, reinterpret_cast<const _Float16*>(b.w), b.y, b.N, b.K, b.ldx, b.ldy, b.act};
            c1 += (a.N + LT - 1) / LT;
            c2 += (b.N + LT - 1) / LT;
        }
        t1.first[4] = c1;
        t2.first[4] = c2;
        const int64_t mt = (M + LT - 1) / LT;
        RWKV_REQUIRE(mt * c2 < INT32_MAX, RWKV_E_SHAPE, "x070_seq_lora: too many tiles");
        rwkv::launch(lora_split_kernel, dim3((unsigned)(mt * c1)), dim3(256), st, t1, (int)M);
        rwkv::launch(lora_split_kernel, dim3((unsigned)(mt * c2)), dim3(256), st, t2, (int)M);
        RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "x070_seq_lora: launch failed");
        rwkv::counters().x070.fetch_add(2);
        rwkv::clear_error();
        return RWKV_OK;
    }
    // few rows: the K-split tiles (both stages, MI355X): 0.1B-wide (D 768) at
    // 128 rows 33 → 16 µs, 7B-class (D 4096) at 128 / 512 rows 158 → 56 /
    // 186 → 165 µs; from ~1024 rows on the 64 × 64 tiles below are as fast or
    // faster (D 2048, 1024 rows: 109 against 126 µs)
    if (M <= kLoraKsMaxRows) {
        const dim3 k1((unsigned)((maxn1 + 31) / 32), (unsigned)((M + 31) / 32), (unsigned)n);
        const dim3 k2((unsigned)((D + 31) / 32), (unsigned)((M + 31) / 32), (unsigned)n);
        if (w_dt == RWKV_F16) {
            rwkv::launch(seq_lora_ks_kernel<__half>, k1, dim3(256), st, s1, (int)M);
            rwkv::launch(seq_lora_ks_kernel<__half>, k2, dim3(256), st, s2, (int)M);
        } else {
            rwkv::launch(seq_lora_ks_kernel<float>, k1, dim3(256), st, s1, (int)M);
            rwkv::launch(seq_lora_ks_kernel<float>, k2, dim3(256), st, s2, (int)M);
        }
        RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "x070_seq_lora: launch failed");
        rwkv::counters().x070.fetch_add(2);
        rwkv::clear_error();
        return RWKV_OK;
    }
    // 2 × 2 tiles of 16 × 16 per wave (larger wave tiles measured faster only
    // at the long passes, which take the two-part kernel)
    constexpr int MT = 2, NT = 2;
    const dim3 grid1((unsigned)((maxn1 + 32 * NT - 1) / (32 * NT)), (unsigned)((M + 32 * MT - 1) / (32 * MT)), (unsigned)n);
    const dim3 grid2((unsigned)((D + 32 * NT - 1) / (32 * NT)), (unsigned)((M + 32 * MT - 1) / (32 * MT)), (unsigned)n);
    if (w_dt == RWKV_F16) {
        rwkv::launch(seq_lora_kernel<__half, MT, NT>, grid1, dim3(256), st, s1, (int)M);
        rwkv::launch(seq_lora_kernel<__half, MT, NT>, grid2, dim3(256), st, s2, (int)M);
    } else {
        rwkv::launch(seq_lora_kernel<float, MT, NT>, grid1, dim3(256), st, s1, (int)M);
        rwkv::launch(seq_lora_kernel<float, MT, NT>, grid2, dim3(256), st, s2, (int)M);
    }
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "x070_seq_lora: launch failed");
    rwkv::counters().x070.fetch_add(2);
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"
