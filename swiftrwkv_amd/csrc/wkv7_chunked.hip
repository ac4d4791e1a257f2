// WKV-7 forward in time chunks (a T-parallel formulation of the recurrence of
// Sources/RWKVKernel/WKV7.swift:213-220) for sequences with few (batch, head)
// rows, where the one-step-at-a-time kernel leaves the GPU idle.
//
// Per (b, h) and chunk of CH tokens with start state S0 (S[i, j]: value row
// i, key column j) the recurrence S_t = S_{t-1}(diag w_t + a_t b_tᵀ) + v_t k_tᵀ
// is affine in S0.  With L_t = Σ_{s≤t} log w_s (per column), the in-chunk
// sa_t = S_{t-1} a_t solve a unit lower-triangular system, and
//   Y  = G·S0ᵀ + E          (the chunk's outputs, y_t[i] = Y[t, i])
//   S' = S0·P + Q            (the state after the chunk)
// with, using R̃ = r ⊙ e^{L_t}, Ã = a ⊙ e^{L_{t-1}}, K̃ = k ⊙ e^{−L_s},
// B̃ = b ⊙ e^{−L_s}, K̂ = k ⊙ e^{L_end − L_s}, B̂ = b ⊙ e^{L_end − L_s}:
//   Mrk = R̃K̃ᵀ, Mrb = R̃B̃ᵀ (s ≤ t);  Mak = ÃK̃ᵀ, Mab = ÃB̃ᵀ (s < t)
//   T = (I − Mab)⁻¹,  W = T·Ã,  V̂ = T·Mak·V      (sa = W·S0ᵀ + V̂)
//   G = R̃ + Mrb·W,  E = Mrk·V + Mrb·V̂
//   P = diag(e^{L_end}) + WᵀB̂,  Q = VᵀK̂ + V̂ᵀB̂.
// Every decay factor of these products is ≤ 1 except e^{−L_s}; when a
// chunk's decay exceeds e^{40} in some column, its M matrices are formed from
// the pairwise factors e^{L_t − L_s} instead.  Pad steps past T are neutral
// (w = 1, everything else 0), the reference's own padding (WKV7.swift:121-133).
//
// Kernel 1 (one workgroup of 4 waves per (b, h, chunk), all chunks at once)
// forms P, Q, G, E into the workspace, every product a 16 × 16 tile of
// v_mfma_f32_16x16x4_f32.  T comes from its two 16 × 16 diagonal blocks
// (forward substitution) and T21 = T22·Mab21·T11.  After T, wave w owns the
// 16 state columns 16w..16w+15 and keeps its slabs of W, V̂ in registers:
// the accumulator layout of one product (lane: rows 4g..4g+3 of column i) is
// the B operand layout of the next when its K index runs as 16q + 4g + r.
// Kernel 2 (one workgroup per (b, h, 16 value rows)) walks the chunks in
// order: for its rows, S ← S·P + Q (wave w: state columns 16w..16w+15) and
// the outputs Y = G·Sᵀ + E (wave w: the K-quarter 16w..16w+15, summed across
// waves in LDS), with the operands of the next two chunks in flight.
//
// Results agree with the sequential kernels to fp32 rounding (not bitwise:
// the sums are taken in another order); the sequential kernels remain the
// path that keeps the reference's bitwise invariants.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.h"
#include "launch.h"

namespace {

constexpr int CH = 32;                             // tokens per chunk
constexpr int RS = 68;                             // LDS row stride of 64-wide rows (16-byte rows, 4-bank steps)
constexpr int MS = 36;                             // LDS row stride of the 32 × 32 matrices
constexpr int WS_CHUNK = 2 * 64 * 64 + 2 * CH * 64;   // P, Q, G, E floats per chunk
constexpr float kUnsafeDecay = 57.7f;              // 2^{±57.7} = e^{±40} keeps every scaled operand a normal float

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ f32x4 v4(float4 a) { return f32x4{a.x, a.y, a.z, a.w}; }
__device__ __forceinline__ float4 f4(float a, float b, float c, float d) { return make_float4(a, b, c, d); }
__device__ __forceinline__ float4& at4(float* p) { return *reinterpret_cast<float4*>(p); }

// Four K steps (k = k0 + r, r = 0..3) of one tile product.
__device__ __forceinline__ f32x4 mma4(float4 a, float4 b, f32x4 c) {
    c = mfma(a.x, b.x, c);
    c = mfma(a.y, b.y, c);
    c = mfma(a.z, b.z, c);
    return mfma(a.w, b.w, c);
}
__device__ __forceinline__ f32x4 mma4(float4 a, f32x4 b, f32x4 c) {
    return mma4(a, f4(b[0], b[1], b[2], b[3]), c);
}
__device__ __forceinline__ f32x4 mma4(f32x4 a, float4 b, f32x4 c) {
    return mma4(f4(a[0], a[1], a[2], a[3]), b, c);
}
__device__ __forceinline__ f32x4 mma4(f32x4 a, f32x4 b, f32x4 c) {
    return mma4(f4(a[0], a[1], a[2], a[3]), f4(b[0], b[1], b[2], b[3]), c);
}
// 2^x and log2(x) of the hardware (v_exp_f32, v_log_f32: 1 ulp); every
// argument here keeps them in the normal range.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float lg2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float4 ex2(float4 x) { return f4(ex2(x.x), ex2(x.y), ex2(x.z), ex2(x.w)); }
// Operand fetch for K block q (k = 16q + 4g + r): a row of M (k contiguous) or
// a column of M (k down the rows).
__device__ __forceinline__ float4 krow(const float* M, int ld, int row, int q, int g) {
    return at4(const_cast<float*>(M) + row * ld + 16 * q + 4 * g);
}
__device__ __forceinline__ float4 kcol(const float* M, int ld, int col, int q, int g) {
    const float* p = M + (16 * q + 4 * g) * ld + col;
    return f4(p[0], p[ld], p[2 * ld], p[3 * ld]);
}

template <typename TI>
__device__ __forceinline__ float4 load4w(const TI* p) {
    if constexpr (sizeof(TI) == 4) {
        return *reinterpret_cast<const float4*>(p);
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        const TI* h = reinterpret_cast<const TI*>(&u);
        return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    }
}

template <typename TI>
__global__ __launch_bounds__(256, 2) void wkv7_chunk_prep_kernel(const TI* __restrict__ r, const TI* __restrict__ w,
                                                                 const TI* __restrict__ k, const TI* __restrict__ v,
                                                                 const TI* __restrict__ a, const TI* __restrict__ b,
                                                                 float* __restrict__ ws, int T, int H, int NC) {
    __shared__ __attribute__((aligned(16))) float R[CH * RS], A[CH * RS], K[CH * RS], Bv[CH * RS];
    // one region, three lives: the per-block log-decay sums, then L (pairwise
    // branch only), then T = (I − Mab)⁻¹
    __shared__ __attribute__((aligned(16))) float Lx[CH * RS];
    __shared__ __attribute__((aligned(16))) float Mrk[CH * MS], Mrb[CH * MS], Mak[CH * MS], Mab[CH * MS];
    __shared__ float lam[64];
    float* const L = Lx;
    float* const Tm = Lx;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, i = lane & 15;
    const int cid = blockIdx.x;
    const int c = cid % NC, bh = cid / NC;
    const int h = bh % H, bb = bh / H;
    float* out = ws + (int64_t)cid * WS_CHUNK;
    // The workspace holds each chunk's P, Q, G, E in the scan's operand
    // order, so every load of the scan reads 1 KiB in one piece (lane
    // i + 16g of wave w, value-row slice s, tile q / tt):
    //   P[16q + 4g + r][16w + i] at (((w·4 + q)·4 + g)·16 + i)·4 + r
    //   Q[16s + 4g + r][16w + i] at (((s·4 + w)·4 + g)·16 + i)·4 + r
    //   G[16tt + i][16w + 4g + r] at (((w·2 + tt)·4 + g)·16 + i)·4 + r
    //   E[t][16s + i]             at (s·32 + t)·16 + i
    float* Pg = out;
    float* Qg = out + 4096;
    float* Gg = out + 8192;
    float* Eg = Gg + CH * 64;

    const int col = 16 * wave + i;   // this wave's slab of state / value columns (phases 4-6)

    // 1. inputs: thread (rb, j4) holds rows 2rb, 2rb + 1 of key columns j4..j4+3
    //    (neutral past T); V straight into this lane's operand registers
    const int rb = tid >> 4, j4 = (tid & 15) * 4;
    float4 rv[2], kv[2], av[2], bv[2], lw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int tg = c * CH + 2 * rb + u;
        rv[u] = kv[u] = av[u] = bv[u] = lw[u] = f4(0, 0, 0, 0);
        if (tg < T) {
            const int64_t off = (((int64_t)bb * T + tg) * H + h) * 64 + j4;
            rv[u] = load4w(r + off);
            const float4 wv = load4w(w + off);
            kv[u] = load4w(k + off);
            av[u] = load4w(a + off);
            bv[u] = load4w(b + off);
            lw[u] = f4(lg2(fmaxf(wv.x, 1e-35f)), lg2(fmaxf(wv.y, 1e-35f)), lg2(fmaxf(wv.z, 1e-35f)),
                       lg2(fmaxf(wv.w, 1e-35f)));
        }
    }
    float vreg[8];   // V[16q + 4g + u][col], q = 0..1
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int tg = c * CH + 16 * (e >> 2) + 4 * g + (e & 3);
        vreg[e] = tg < T ? (float)v[(((int64_t)bb * T + tg) * H + h) * 64 + col] : 0.0f;
    }

    // 2. L_t = Σ_{s≤t} log2 w_s (every decay factor below is a power of 2):
    //    two-row sums, then each thread's prefix over the earlier row pairs
    at4(&Lx[rb * 64 + j4]) = f4(lw[0].x + lw[1].x, lw[0].y + lw[1].y, lw[0].z + lw[1].z, lw[0].w + lw[1].w);
    __syncthreads();
    float4 pre = f4(0, 0, 0, 0), tot = pre;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float4 x = at4(&Lx[q * 64 + j4]);
        if (q < rb) pre = f4(pre.x + x.x, pre.y + x.y, pre.z + x.z, pre.w + x.w);
        tot = f4(tot.x + x.x, tot.y + x.y, tot.z + x.z, tot.w + x.w);
    }
    if (rb == 0) at4(&lam[j4]) = ex2(tot);
    // every wave holds all 64 columns' totals, formed in the same order by
    // every thread, so a wave vote gives each wave the same answer
    const int unsafe_cols = (-tot.x > kUnsafeDecay) | (-tot.y > kUnsafeDecay) | (-tot.z > kUnsafeDecay) |
                            (-tot.w > kUnsafeDecay);
    const bool unsafe = __ballot(unsafe_cols) != 0;
    const float4 L0 = f4(pre.x + lw[0].x, pre.y + lw[0].y, pre.z + lw[0].z, pre.w + lw[0].w);
    const float4 L1 = f4(L0.x + lw[1].x, L0.y + lw[1].y, L0.z + lw[1].z, L0.w + lw[1].w);

    // 3. the four CH × CH matrices
    const int t0 = 2 * rb;
    if (!unsafe) {
        // R̃ = r 2^{L_t}, Ã = a 2^{L_{t−1}}, K̃ = k 2^{−L_t}, B̃ = b 2^{−L_t}
        const float4 e0 = ex2(L0), e1 = ex2(L1), em = ex2(pre);
        const float4 i0 = ex2(f4(-L0.x, -L0.y, -L0.z, -L0.w)), i1 = ex2(f4(-L1.x, -L1.y, -L1.z, -L1.w));
        auto mul = [](float4 x, float4 y) { return f4(x.x * y.x, x.y * y.y, x.z * y.z, x.w * y.w); };
        at4(&R[t0 * RS + j4]) = mul(rv[0], e0);
        at4(&R[(t0 + 1) * RS + j4]) = mul(rv[1], e1);
        at4(&A[t0 * RS + j4]) = mul(av[0], em);
        at4(&A[(t0 + 1) * RS + j4]) = mul(av[1], e0);
        at4(&K[t0 * RS + j4]) = mul(kv[0], i0);
        at4(&K[(t0 + 1) * RS + j4]) = mul(kv[1], i1);
        at4(&Bv[t0 * RS + j4]) = mul(bv[0], i0);
        at4(&Bv[(t0 + 1) * RS + j4]) = mul(bv[1], i1);
        __syncthreads();
        // wave w forms matrix w: X·Yᵀ over the 64 key columns, tiles (0,0), (1,0), (1,1)
        const float* X = wave < 2 ? R : A;
        const float* Y = (wave & 1) ? Bv : K;
        float* M = wave == 0 ? Mrk : wave == 1 ? Mrb : wave == 2 ? Mak : Mab;
        f32x4 d00 = zero4(), d10 = zero4(), d11 = zero4();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 x0 = krow(X, RS, i, q, g), x1 = krow(X, RS, 16 + i, q, g);
            const float4 y0 = krow(Y, RS, i, q, g), y1 = krow(Y, RS, 16 + i, q, g);
            d00 = mma4(x0, y0, d00);
            d10 = mma4(x1, y0, d10);
            d11 = mma4(x1, y1, d11);
        }
        const bool strict = wave >= 2;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int t = 4 * g + u;   // row within the tile; the lane's column is i
            const bool keep = strict ? i < t : i <= t;
            M[t * MS + i] = keep ? d00[u] : 0.0f;
            M[(16 + t) * MS + i] = d10[u];
            M[(16 + t) * MS + 16 + i] = keep ? d11[u] : 0.0f;
        }
    } else {
        __syncthreads();   // the row-pair sums (Lx) are read above; L reuses them
        at4(&R[t0 * RS + j4]) = rv[0];
        at4(&R[(t0 + 1) * RS + j4]) = rv[1];
        at4(&A[t0 * RS + j4]) = av[0];
        at4(&A[(t0 + 1) * RS + j4]) = av[1];
        at4(&K[t0 * RS + j4]) = kv[0];
        at4(&K[(t0 + 1) * RS + j4]) = kv[1];
        at4(&Bv[t0 * RS + j4]) = bv[0];
        at4(&Bv[(t0 + 1) * RS + j4]) = bv[1];
        at4(&L[t0 * RS + j4]) = L0;
        at4(&L[(t0 + 1) * RS + j4]) = L1;
        for (int e = tid; e < CH * MS; e += 256) Mak[e] = Mab[e] = Mrk[e] = Mrb[e] = 0.0f;
        __syncthreads();
        for (int p = tid; p < CH * (CH + 1) / 2; p += 256) {
            int t = (int)((sqrtf(8.0f * p + 1.0f) - 1.0f) * 0.5f);
            while ((t + 1) * (t + 2) / 2 <= p) ++t;
            while (t * (t + 1) / 2 > p) --t;
            const int s = p - t * (t + 1) / 2;
            float rk = 0.f, rb_ = 0.f, ak = 0.f, ab = 0.f;
            for (int j = 0; j < 64; ++j) {
                const float ls = L[s * RS + j];
                const float e1 = exp2f(L[t * RS + j] - ls);
                const float e0 = t > 0 ? exp2f(L[(t - 1) * RS + j] - ls) : 0.0f;
                rk += R[t * RS + j] * K[s * RS + j] * e1;
                rb_ += R[t * RS + j] * Bv[s * RS + j] * e1;
                ak += A[t * RS + j] * K[s * RS + j] * e0;
                ab += A[t * RS + j] * Bv[s * RS + j] * e0;
            }
            Mrk[t * MS + s] = rk;
            Mrb[t * MS + s] = rb_;
            if (s < t) {
                Mak[t * MS + s] = ak;
                Mab[t * MS + s] = ab;
            }
        }
        __syncthreads();
        // R̃, Ã, K̂ = k 2^{L_end − L_s}, B̂ likewise, with factors ≤ 1
        for (int e = tid; e < CH * 64; e += 256) {
            const int t = e >> 6, j = e & 63;
            const float d = exp2f(L[(CH - 1) * RS + j] - L[t * RS + j]);
            K[t * RS + j] *= d;
            Bv[t * RS + j] *= d;
            R[t * RS + j] *= exp2f(L[t * RS + j]);
            A[t * RS + j] *= t > 0 ? exp2f(L[(t - 1) * RS + j]) : 1.0f;
        }
    }
    __syncthreads();

    // 4. K̂ = K̃ 2^{L_end}, B̂ likewise (scaled branch); T11 and T22 on the
    //    matrix cores; each wave its slab of Z = Mak·V
    if (!unsafe) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float4 lm = at4(&lam[j4]);
            float4& kk = at4(&K[(t0 + u) * RS + j4]);
            float4& bq = at4(&Bv[(t0 + u) * RS + j4]);
            kk = f4(kk.x * lm.x, kk.y * lm.y, kk.z * lm.z, kk.w * lm.w);
            bq = f4(bq.x * lm.x, bq.y * lm.y, bq.z * lm.z, bq.w * lm.w);
        }
    }
    if (wave < 2) {
        // N = the strictly lower diagonal block o of Mab, N^16 = 0, so
        // (I − N)⁻¹ = (I + N⁸)(I + N⁴)(I + N²)(I + N).  An accumulator
        // (lane i + 16g: rows 4g..4g+3 of column i) is the B operand of a
        // product and, read as a transpose, its A operand; so the powers are
        // formed with their transposes and every product stays in registers.
        const int o = 16 * wave;
        const float4 nA = at4(&Mab[(o + i) * MS + o + 4 * g]);                   // N[i][4g + r]
        const float4 nB = f4(Mab[(o + 4 * g) * MS + o + i], Mab[(o + 4 * g + 1) * MS + o + i],
                             Mab[(o + 4 * g + 2) * MS + o + i], Mab[(o + 4 * g + 3) * MS + o + i]);   // N[4g + r][i]
        const f32x4 n2 = mma4(nA, nB, zero4());     // N²
        const f32x4 n2t = mma4(nB, nA, zero4());    // (N²)ᵀ
        const f32x4 n4t = mma4(n2, n2t, zero4());   // (N⁴)ᵀ
        const f32x4 n4 = mma4(n2t, n2, zero4());    // N⁴
        const f32x4 n8t = mma4(n4, n4t, zero4());   // (N⁸)ᵀ
        f32x4 x = {nB.x + (4 * g == i ? 1.0f : 0.0f), nB.y + (4 * g + 1 == i ? 1.0f : 0.0f),
                   nB.z + (4 * g + 2 == i ? 1.0f : 0.0f), nB.w + (4 * g + 3 == i ? 1.0f : 0.0f)};   // I + N
        x = mma4(n2t, x, x);   // (I + N²)·x
        x = mma4(n4t, x, x);   // (I + N⁴)·x
        x = mma4(n8t, x, x);   // (I + N⁸)·x
#pragma unroll
        for (int u = 0; u < 4; ++u) Tm[(o + 4 * g + u) * MS + o + i] = x[u];
    }
    const float4 v0 = f4(vreg[0], vreg[1], vreg[2], vreg[3]), v1 = f4(vreg[4], vreg[5], vreg[6], vreg[7]);
    f32x4 z0 = mma4(krow(Mak, MS, i, 0, g), v0, zero4());
    f32x4 z1 = mma4(krow(Mak, MS, 16 + i, 1, g), v1, mma4(krow(Mak, MS, 16 + i, 0, g), v0, zero4()));
    __syncthreads();

    // 5. T21 = T22 · (Mab21 · T11)
    if (wave == 0) {
        f32x4 x = mma4(krow(Mab, MS, 16 + i, 0, g), kcol(Tm, MS, i, 0, g), zero4());
        f32x4 t21 = mma4(at4(&Tm[(16 + i) * MS + 16 + 4 * g]), x, zero4());
#pragma unroll
        for (int u = 0; u < 4; ++u) Tm[(16 + 4 * g + u) * MS + i] = t21[u];
    }
    __syncthreads();

    // 6. per wave, its slab: W, V̂ (registers), G, E → workspace, P and Q rows
    f32x4 w0, w1, h0, h1;
    {
        const float4 a0 = kcol(A, RS, col, 0, g), a1 = kcol(A, RS, col, 1, g);
        const float4 t00 = krow(Tm, MS, i, 0, g), t10 = krow(Tm, MS, 16 + i, 0, g), t11 = krow(Tm, MS, 16 + i, 1, g);
        w0 = mma4(t00, a0, zero4());
        w1 = mma4(t11, a1, mma4(t10, a0, zero4()));
        h0 = mma4(t00, z0, zero4());
        h1 = mma4(t11, z1, mma4(t10, z0, zero4()));
    }
    {
        // Gᵀ slab (rows: this wave's key columns, columns: tokens) = R̃ᵀ + Wᵀ·Mrbᵀ
        f32x4 gt0 = mma4(w0, krow(Mrb, MS, i, 0, g), v4(krow(R, RS, i, wave, g)));
        f32x4 gt1 = mma4(w1, krow(Mrb, MS, 16 + i, 1, g),
                         mma4(w0, krow(Mrb, MS, 16 + i, 0, g), v4(krow(R, RS, 16 + i, wave, g))));
        at4(Gg + (((wave * 2 + 0) * 4 + g) * 16 + i) * 4) = f4(gt0[0], gt0[1], gt0[2], gt0[3]);
        at4(Gg + (((wave * 2 + 1) * 4 + g) * 16 + i) * 4) = f4(gt1[0], gt1[1], gt1[2], gt1[3]);
        // E slab = Mrk·V + Mrb·V̂
        const float4 rb0 = krow(Mrb, MS, i, 0, g), rb10 = krow(Mrb, MS, 16 + i, 0, g),
                     rb11 = krow(Mrb, MS, 16 + i, 1, g);
        f32x4 e0 = mma4(krow(Mrk, MS, i, 0, g), v0, mma4(rb0, h0, zero4()));
        f32x4 e1 = mma4(krow(Mrk, MS, 16 + i, 0, g), v0, mma4(rb10, h0, zero4()));
        e1 = mma4(krow(Mrk, MS, 16 + i, 1, g), v1, mma4(rb11, h1, e1));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            Eg[(wave * 32 + 4 * g + u) * 16 + i] = e0[u];
            Eg[(wave * 32 + 16 + 4 * g + u) * 16 + i] = e1[u];
        }
    }
    {
        const float4 vt0 = v0, vt1 = v1;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int j = 16 * jt + i;
            const float4 b0 = kcol(Bv, RS, j, 0, g), b1 = kcol(Bv, RS, j, 1, g);
            const float4 k0 = kcol(K, RS, j, 0, g), k1 = kcol(K, RS, j, 1, g);
            f32x4 p = zero4();
            if (jt == wave) {
#pragma unroll
                for (int u = 0; u < 4; ++u) p[u] = 4 * g + u == i ? lam[j] : 0.0f;
            }
            p = mma4(w1, b1, mma4(w0, b0, p));
            f32x4 qq = mma4(vt1, k1, mma4(vt0, k0, zero4()));
            qq = mma4(h1, b1, mma4(h0, b0, qq));
            // P[16 wave + 4g + u][j] and Q[16 wave + 4g + u][j] in the scan's operand order
            at4(Pg + (((jt * 4 + wave) * 4 + g) * 16 + i) * 4) = f4(p[0], p[1], p[2], p[3]);
            at4(Qg + (((wave * 4 + jt) * 4 + g) * 16 + i) * 4) = f4(qq[0], qq[1], qq[2], qq[3]);
        }
    }
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for its
// global loads in flight (the operand prefetch).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Where the scan's stores for steps past T go (never read).
__device__ float g_scan_sink[512];

// Operands of one chunk for one lane of the scan's state waves (wave w < 4:
// state columns 16w..16w+15, value-row slice sl, lane i + 16g) and of its
// output waves (wave 4 + w: the K quarter 16w..16w+15 of the outputs).
struct StateOps {
    float4 p[4];    // P[16q + 4g + r][16w + i], q = 0..3
    float4 q;       // Q[16 sl + 4g + r][16w + i]
};
struct OutOps {
    float4 gk[2];   // G[16tt + i][16w + 4g + r], tt = 0..1
    float2 e;       // E[token][row], this thread's two outputs
};

__device__ __forceinline__ void load_state_ops(StateOps& o, const float* base, int c, int w, int g, int i, int slice) {
    const float* P = base + (int64_t)c * WS_CHUNK;
    const float* Q = P + 4096;
#pragma unroll
    for (int q = 0; q < 4; ++q) o.p[q] = *reinterpret_cast<const float4*>(P + (((w * 4 + q) * 4 + g) * 16 + i) * 4);
    o.q = *reinterpret_cast<const float4*>(Q + (((slice * 4 + w) * 4 + g) * 16 + i) * 4);
}

__device__ __forceinline__ void load_out_ops(OutOps& o, const float* base, int c, int w, int g, int i, int slice,
                                             int ot, int orow) {
    const float* G = base + (int64_t)c * WS_CHUNK + 8192;
    const float* E = G + CH * 64;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
        o.gk[tt] = *reinterpret_cast<const float4*>(G + (((w * 2 + tt) * 4 + g) * 16 + i) * 4);
    o.e = *reinterpret_cast<const float2*>(E + (slice * 32 + ot) * 16 + orow);
}

constexpr int YS = 36;   // LDS row stride of the partial outputs [wave][row][token] (conflict-free writes)

// Kernel 2: the chunks in order for 16 value rows of one (b, h), with 8
// waves.  Phase p (one barrier each): the state waves form
// S_{p+1} = S_p·P_p + Q_p (wave w: state columns 16w..16w+15, 16 MFMAs); the
// output waves, on the same SIMDs, form the partial outputs of chunk p from
// the same S_p (wave 4 + w: the K quarter 16w..16w+15 for all 32 tokens, 8
// MFMAs) and emit chunk p − 1's outputs from the partials of the previous
// phase.  The output waves' products fill the matrix pipe while the state
// chain waits for LDS and the barrier.  S and the partial outputs are
// double-buffered in LDS.
__global__ __launch_bounds__(512) void wkv7_chunk_scan_kernel(const float* ws,
                                                              const float* __restrict__ h_in, float* __restrict__ out,
                                                              float* __restrict__ h_out, int T, int H, int NC, int BH) {
    __shared__ __attribute__((aligned(16))) float S[2][16 * RS];
    __shared__ __attribute__((aligned(16))) float Sspare[16 * RS];   // state of phantom chunks (never read)
    __shared__ __attribute__((aligned(16))) float Yp[2][4 * 16 * YS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    // workgroups are dealt to the 8 XCDs round-robin (id mod 8); the four
    // row slices of a head get ids congruent mod 8, so they share one L2 and
    // each chunk's P and G come from HBM once.  The grid is padded to whole
    // groups of 8 heads.
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    const int slice = loc & 3, bh = (loc >> 2) * 8 + xcd;
    if (bh >= BH) return;
    const int h = bh % H, bb = bh / H;
    const int i0 = slice * 16;
    const int64_t hoff = (int64_t)bh * 4096;
    for (int e = tid; e < 16 * 64; e += 512) {
        const int ii = e >> 6, j = e & 63;
        S[0][ii * RS + j] = h_in ? h_in[hoff + (i0 + ii) * 64 + j] : 0.0f;
    }
    const float* base = ws + (int64_t)bh * NC * WS_CHUNK;
    const int w = wave & 3;

    if (wave < 4) {
        // state waves
        const int col = 16 * w + li;
        auto phase = [&](int p, StateOps& o) {
            const float* Sc = S[p & 1];
            float* Sn = p < NC ? S[(p & 1) ^ 1] : Sspare;
            float4 av[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) av[q] = at4(const_cast<float*>(Sc) + li * RS + 16 * q + 4 * g);
            f32x4 acc0 = {o.q.x, o.q.y, o.q.z, o.q.w}, acc1 = zero4();
            acc0 = mma4(av[0], o.p[0], acc0);
            acc1 = mma4(av[1], o.p[1], acc1);
            acc0 = mma4(av[2], o.p[2], acc0);
            acc1 = mma4(av[3], o.p[3], acc1);
            // the loads of chunk p + 3 into this slot, issued between the products
            load_state_ops(o, base, min(p + 3, NC - 1), w, g, li, slice);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);   // loads
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) Sn[(4 * g + r) * RS + col] = acc0[r] + acc1[r];
            lds_barrier();
        };
        // operands three chunks ahead; indexes past the end re-read the last
        // chunk.  Issued in chunk order: the loop-head wait count is formed
        // from the prologue too, so interleaved prologue loads would make
        // every iteration wait for the loads it has just issued.
        StateOps o0, o1, o2;
        load_state_ops(o0, base, 0, w, g, li, slice);
        asm volatile("" ::: "memory");
        load_state_ops(o1, base, min(1, NC - 1), w, g, li, slice);
        asm volatile("" ::: "memory");
        load_state_ops(o2, base, min(2, NC - 1), w, g, li, slice);
        asm volatile("" ::: "memory");
        lds_barrier();
        for (int p = 0; p <= NC; p += 3) {
            phase(p, o0);
            phase(p + 1, o1);
            phase(p + 2, o2);
        }
    } else {
        // output waves: this thread's two outputs of a chunk are token ot,
        // rows orow and orow + 1; chunk c's start at out0 + c·cstride
        const int u = tid - 256;
        const int ot = u >> 3, orow = (u & 7) * 2;
        float* const out0 = out + (((int64_t)bb * T + ot) * H + h) * 64 + i0 + orow;
        const int64_t cstride = (int64_t)CH * H * 64;
        // phase p: chunk p's partials from `cur`, chunk p − 1's outputs from
        // `prev`'s E, then `prev` is reloaded with chunk p + 2
        auto phase = [&](int p, const OutOps& cur, OutOps& prev) {
            const float* Sc = S[p & 1];
            float* Y = Yp[p & 1];
            const float* Ye = Yp[(p & 1) ^ 1];
            const float4 aw = at4(const_cast<float*>(Sc) + li * RS + 16 * w + 4 * g);   // the K quarter
            float y[2] = {prev.e.x, prev.e.y};
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                y[0] += Ye[(ww * 16 + orow) * YS + ot];
                y[1] += Ye[(ww * 16 + orow + 1) * YS + ot];
            }
            const f32x4 y0 = mma4(aw, cur.gk[0], zero4());
            const f32x4 y1 = mma4(aw, cur.gk[1], zero4());
            // chunk p − 1's outputs; steps past T (the phantom chunk −1 and
            // chunks past NC) store to a sink
            const int t = (p - 1) * CH + ot;
            float* dst = (unsigned)t < (unsigned)T ? out0 + (int64_t)(p - 1) * cstride : g_scan_sink + 2 * u;
            *reinterpret_cast<float2*>(dst) = make_float2(y[0], y[1]);
            load_out_ops(prev, base, min(p + 2, NC - 1), w, g, li, slice, ot, orow);
            // partial Yᵀ[row 4g + r][token 16 tt + li] of this wave's K quarter
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                Y[(w * 16 + 4 * g + r) * YS + li] = y0[r];
                Y[(w * 16 + 4 * g + r) * YS + 16 + li] = y1[r];
            }
            lds_barrier();
        };
        OutOps o0, o1, o2;
        load_out_ops(o0, base, 0, w, g, li, slice, ot, orow);
        asm volatile("" ::: "memory");
        load_out_ops(o1, base, min(1, NC - 1), w, g, li, slice, ot, orow);
        asm volatile("" ::: "memory");
        o2.gk[0] = o2.gk[1] = make_float4(0.f, 0.f, 0.f, 0.f);
        o2.e = make_float2(0.f, 0.f);
        lds_barrier();
        for (int p = 0; p <= NC; p += 3) {
            phase(p, o0, o2);
            phase(p + 1, o1, o0);
            phase(p + 2, o2, o1);
        }
    }
    const float* Sf = S[NC & 1];
    for (int e = tid; e < 16 * 64; e += 512) {
        const int ii = e >> 6, j = e & 63;
        h_out[hoff + (i0 + ii) * 64 + j] = Sf[ii * RS + j];
    }
}

template <typename TI>
rwkv_status run_chunked(const void* r, const void* w, const void* k, const void* v, const void* a, const void* b,
                        const float* h_in, float* out, float* h_out, float* ws, int B, int T, int H, hipStream_t s) {
    const int NC = (T + CH - 1) / CH;
    rwkv::launch(wkv7_chunk_prep_kernel<TI>, dim3((unsigned)(B * H * NC)), dim3(256), s, (const TI*)r, (const TI*)w,
                 (const TI*)k, (const TI*)v, (const TI*)a, (const TI*)b, ws, T, H, NC);
    rwkv::launch(wkv7_chunk_scan_kernel, dim3((unsigned)((B * H + 7) / 8 * 32)), dim3(512), s, (const float*)ws, h_in,
                 out, h_out, T, H, NC, B * H);
    return hipGetLastError() == hipSuccess ? RWKV_OK : RWKV_E_HIP;
}

}  // namespace

// Device scratch of the entry point that allocates nothing
// (rwkv_wkv7_seq_fwd_chunked_static): 64 MiB, the workspace of at most 1365
// (batch row, head, 32-token chunk) triples.  Every GPU the library runs on
// holds its own copy until the process ends.  Host code never names the array
// as an address: it uses the pointer hipGetSymbolAddress returns for the
// current device.
constexpr int64_t kScratchBytes = (int64_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device.
rwkv_status scratch_on_current_device(void** out) {
    int dev = -1;
    RWKV_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, RWKV_E_HIP,
                 "wkv7_seq_fwd_chunked_static: no current HIP device (or device index %d >= %d)", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        RWKV_REQUIRE(e == hipSuccess && p, RWKV_E_HIP, "wkv7_seq_fwd_chunked_static: hipGetSymbolAddress: %s",
                     hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return RWKV_OK;
}

rwkv_status seq_fwd_chunked(const char* who, const void* r, const void* w, const void* k, const void* v,
                            const void* a, const void* b, rwkv_dtype in_dt, const float* h_in, float* out,
                            float* h_out, int64_t B, int64_t T, int64_t H, void* workspace, int64_t workspace_bytes,
                            void* stream) {
    RWKV_REQUIRE(r && w && k && v && a && b && out && h_out && workspace, RWKV_E_NULL, "%s: null buffer", who);
    RWKV_REQUIRE(rwkv::dtype_ok(in_dt), RWKV_E_DTYPE, "%s: dtype %d", who, (int)in_dt);
    RWKV_REQUIRE(B >= 1 && T >= 1 && H >= 1 && B * H * ((T + CH - 1) / CH) <= INT32_MAX && (B * H + 7) / 8 * 32 <= INT32_MAX &&
                     B * T <= INT32_MAX && B * T * H * 64 < ((int64_t)1 << 40),
                 RWKV_E_SHAPE, "%s: B=%lld T=%lld H=%lld", who, (long long)B, (long long)T, (long long)H);
    const uintptr_t al = (uintptr_t)r | (uintptr_t)w | (uintptr_t)k | (uintptr_t)v | (uintptr_t)a | (uintptr_t)b |
                         (uintptr_t)h_in | (uintptr_t)out | (uintptr_t)h_out | (uintptr_t)workspace;
    RWKV_REQUIRE(al % 16 == 0, RWKV_E_SHAPE, "%s: every buffer must be 16-byte aligned", who);
    const int64_t need = B * H * ((T + CH - 1) / CH) * (int64_t)WS_CHUNK * 4;
    RWKV_REQUIRE(workspace_bytes >= need, RWKV_E_SHAPE, "%s: workspace %lld bytes, needs %lld", who,
                 (long long)workspace_bytes, (long long)need);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    float* ws = reinterpret_cast<float*>(workspace);
    rwkv_status st;
    if (in_dt == RWKV_F32) st = run_chunked<float>(r, w, k, v, a, b, h_in, out, h_out, ws, (int)B, (int)T, (int)H, s);
    else if (in_dt == RWKV_BF16)
        st = run_chunked<__hip_bfloat16>(r, w, k, v, a, b, h_in, out, h_out, ws, (int)B, (int)T, (int)H, s);
    else st = run_chunked<__half>(r, w, k, v, a, b, h_in, out, h_out, ws, (int)B, (int)T, (int)H, s);
    RWKV_REQUIRE(st == RWKV_OK, st, "%s: launch failed", who);
    rwkv::counters().seq_chunked.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

}  // namespace

extern "C" {

int64_t rwkv_wkv7_chunked_workspace(int64_t B, int64_t T, int64_t H) {
    if (B < 1 || T < 1 || H < 1) return 0;
    return B * H * ((T + CH - 1) / CH) * (int64_t)WS_CHUNK * 4;
}

rwkv_status rwkv_wkv7_seq_fwd_chunked(const void* r, const void* w, const void* k, const void* v, const void* a,
                                      const void* b, rwkv_dtype in_dt, const float* h_in, float* out, float* h_out,
                                      int64_t B, int64_t T, int64_t H, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
    return seq_fwd_chunked("wkv7_seq_fwd_chunked", r, w, k, v, a, b, in_dt, h_in, out, h_out, B, T, H, workspace,
                           workspace_bytes, stream);
}

rwkv_status rwkv_wkv7_seq_fwd_chunked_static(const void* r, const void* w, const void* k, const void* v,
                                             const void* a, const void* b, rwkv_dtype in_dt, const float* h_in,
                                             float* out, float* h_out, int64_t B, int64_t T, int64_t H,
                                             void* stream) {
    const char* who = "wkv7_seq_fwd_chunked_static";
    RWKV_REQUIRE(B >= 1 && T >= 1 && H >= 1, RWKV_E_SHAPE, "%s: B=%lld T=%lld H=%lld", who, (long long)B,
                 (long long)T, (long long)H);
    // compared by division: no product below can overflow, whatever B, T, H
    const int64_t max_chunks = kScratchBytes / ((int64_t)WS_CHUNK * 4);
    const int64_t chunks = (T - 1) / CH + 1;
    RWKV_REQUIRE(B <= max_chunks && H <= max_chunks && B * H <= max_chunks && chunks <= max_chunks / (B * H),
                 RWKV_E_SHAPE,
                 "%s: B=%lld H=%lld ceil(T/32)=%lld exceed the static scratch (B·H·ceil(T/32) <= %lld chunks of "
                 "48 KiB, 64 MiB); use rwkv_wkv7_seq_fwd_chunked with a workspace",
                 who, (long long)B, (long long)H, (long long)chunks, (long long)max_chunks);
    void* ptr = nullptr;
    const rwkv_status st = scratch_on_current_device(&ptr);
    if (st != RWKV_OK) return st;
    return seq_fwd_chunked(who, r, w, k, v, a, b, in_dt, h_in, out, h_out, B, T, H, ptr, kScratchBytes, stream);
}

}  // extern "C"
