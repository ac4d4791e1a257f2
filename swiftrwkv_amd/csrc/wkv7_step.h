// Device code of the WKV-7 kernels: the DPP step blocks and row sums of the
// two forward layouts, the layout choice, and the decode step and tmix tail
// of one head.  Kernels that call the same functions here compute the same
// bits (the forward kernels' T = 1 path performs the same operations).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rwkv_wkv {

constexpr int D = 64;   // WKV7_HEAD_SIZE

// ─────────────────────────────── DPP / lane-swap helpers ───────────────────────────────
// row_newbcast:c broadcasts lane c of every 16-lane row to the whole row.  The
// compiler does not fold a DPP move into an FMA, so the fused forms are written
// as inline assembly.  Every block starts with `s_nop 1`: the two wait states a
// VALU write of a broadcast source needs before its DPP read.
#define RWKV_BC(n) " row_newbcast:" #n " row_mask:0xf bank_mask:0xf\n\t"

// Sum of the four column-group partials of a row (lanes l, l^16, l^32, l^48),
// associated as (g0+g1)+(g2+g3) in every lane, so all four hold the same bits.
__device__ __forceinline__ float rowsum4(float x) {
    float a = x, b = x;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    const float s = a + b;
    float c = s, d = s;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
    return c + d;
}

// Forward update of 8 state elements (columns c0..c0+7 of the lane's group):
//   n = k·v ; n += b·sa ; n += w·S          (new state, one rounding per FMA)
//   y += r·n ; p += a'·n                    (a' = next step's a)
// Issued stage by stage over the 8 elements, so neighbouring instructions are
// independent (the y and p chains alternate).
#define RWKV_MUL(c, N) "v_mul_f32_dpp %[" N "], %[K], %[vv]" RWKV_BC(c)
#define RWKV_FB(c, N) "v_fmac_f32_dpp %[" N "], %[B], %[sa]" RWKV_BC(c)
#define RWKV_FW(c, S, N) "v_fmac_f32_dpp %[" N "], %[W], %[" S "]" RWKV_BC(c)
#define RWKV_YP(c, N) "v_fmac_f32_dpp %[y], %[R], %[" N "]" RWKV_BC(c) "v_fmac_f32_dpp %[p], %[A], %[" N "]" RWKV_BC(c)
#define RWKV_UPD8(c0, c1, c2, c3, c4, c5, c6, c7)                                                              \
    RWKV_MUL(c0, "n0") RWKV_MUL(c1, "n1") RWKV_MUL(c2, "n2") RWKV_MUL(c3, "n3")                                 \
    RWKV_MUL(c4, "n4") RWKV_MUL(c5, "n5") RWKV_MUL(c6, "n6") RWKV_MUL(c7, "n7")                                 \
    RWKV_FB(c0, "n0") RWKV_FB(c1, "n1") RWKV_FB(c2, "n2") RWKV_FB(c3, "n3")                                     \
    RWKV_FB(c4, "n4") RWKV_FB(c5, "n5") RWKV_FB(c6, "n6") RWKV_FB(c7, "n7")                                     \
    RWKV_FW(c0, "s0", "n0") RWKV_FW(c1, "s1", "n1") RWKV_FW(c2, "s2", "n2") RWKV_FW(c3, "s3", "n3")             \
    RWKV_FW(c4, "s4", "n4") RWKV_FW(c5, "s5", "n5") RWKV_FW(c6, "s6", "n6") RWKV_FW(c7, "s7", "n7")             \
    RWKV_YP(c0, "n0") RWKV_YP(c1, "n1") RWKV_YP(c2, "n2") RWKV_YP(c3, "n3")                                     \
    RWKV_YP(c4, "n4") RWKV_YP(c5, "n5") RWKV_YP(c6, "n6") RWKV_YP(c7, "n7")

#define RWKV_UPD_OPERANDS(S, N, o)                                                                              \
    : [n0] "=&v"(N[o + 0]), [n1] "=&v"(N[o + 1]), [n2] "=&v"(N[o + 2]), [n3] "=&v"(N[o + 3]),                    \
      [n4] "=&v"(N[o + 4]), [n5] "=&v"(N[o + 5]), [n6] "=&v"(N[o + 6]), [n7] "=&v"(N[o + 7]), [y] "+v"(y),        \
      [p] "+v"(p)                                                                                                 \
    : [s0] "v"(S[o + 0]), [s1] "v"(S[o + 1]), [s2] "v"(S[o + 2]), [s3] "v"(S[o + 3]), [s4] "v"(S[o + 4]),         \
      [s5] "v"(S[o + 5]), [s6] "v"(S[o + 6]), [s7] "v"(S[o + 7]), [K] "v"(K), [B] "v"(B), [W] "v"(W), [R] "v"(R), \
      [A] "v"(A), [vv] "v"(vv), [sa] "v"(sa)

__device__ __forceinline__ void fwd_update16(const float (&S)[16], float (&N)[16], float K, float B, float W,
                                             float R, float A, float vv, float sa, float& y, float& p) {
    asm("s_nop 1\n\t" RWKV_UPD8(0, 1, 2, 3, 4, 5, 6, 7) RWKV_UPD_OPERANDS(S, N, 0));
    asm("s_nop 1\n\t" RWKV_UPD8(8, 9, 10, 11, 12, 13, 14, 15) RWKV_UPD_OPERANDS(S, N, 8));
}

// p += Σ_c a_c·S_c over the lane's 16 columns (the first step's sa partial).
#define RWKV_DOT(c, S) "v_fmac_f32_dpp %[p], %[A], %[" S "]" RWKV_BC(c)
__device__ __forceinline__ void fwd_dot16(const float (&S)[16], float A, float& p) {
    asm("s_nop 1\n\t"
        RWKV_DOT(0, "s0") RWKV_DOT(1, "s1") RWKV_DOT(2, "s2") RWKV_DOT(3, "s3")
        RWKV_DOT(4, "s4") RWKV_DOT(5, "s5") RWKV_DOT(6, "s6") RWKV_DOT(7, "s7")
        : [p] "+v"(p)
        : [s0] "v"(S[0]), [s1] "v"(S[1]), [s2] "v"(S[2]), [s3] "v"(S[3]), [s4] "v"(S[4]), [s5] "v"(S[5]),
          [s6] "v"(S[6]), [s7] "v"(S[7]), [A] "v"(A));
    asm("s_nop 1\n\t"
        RWKV_DOT(8, "s0") RWKV_DOT(9, "s1") RWKV_DOT(10, "s2") RWKV_DOT(11, "s3")
        RWKV_DOT(12, "s4") RWKV_DOT(13, "s5") RWKV_DOT(14, "s6") RWKV_DOT(15, "s7")
        : [p] "+v"(p)
        : [s0] "v"(S[8]), [s1] "v"(S[9]), [s2] "v"(S[10]), [s3] "v"(S[11]), [s4] "v"(S[12]), [s5] "v"(S[13]),
          [s6] "v"(S[14]), [s7] "v"(S[15]), [A] "v"(A));
}

// Four-row layout (small B·H): lane l holds value row 4·blk + (l & 3) and key
// columns 4g..4g+3, g = l >> 2; the four lanes of a quad share g and hold
// elements 4g..4g+3 of each step vector, broadcast with DPP quad_perm.
#define RWKV_QB(c) " quad_perm:[" #c "," #c "," #c "," #c "] row_mask:0xf bank_mask:0xf\n\t"
#define RWKV_QMUL(c, N) "v_mul_f32_dpp %[" N "], %[K], %[vv]" RWKV_QB(c)
#define RWKV_QFB(c, N) "v_fmac_f32_dpp %[" N "], %[B], %[sa]" RWKV_QB(c)
#define RWKV_QFW(c, S, N) "v_fmac_f32_dpp %[" N "], %[W], %[" S "]" RWKV_QB(c)
#define RWKV_QYP(c, N) "v_fmac_f32_dpp %[y], %[R], %[" N "]" RWKV_QB(c) "v_fmac_f32_dpp %[p], %[A], %[" N "]" RWKV_QB(c)

// The forward update of the lane's 4 state elements (the same FMA sequence per
// element as fwd_update16).
__device__ __forceinline__ void fwd_update4(const float (&S)[4], float (&N)[4], float K, float B, float W, float R,
                                            float A, float vv, float sa, float& y, float& p) {
    asm("s_nop 1\n\t"
        RWKV_QMUL(0, "n0") RWKV_QMUL(1, "n1") RWKV_QMUL(2, "n2") RWKV_QMUL(3, "n3")
        RWKV_QFB(0, "n0") RWKV_QFB(1, "n1") RWKV_QFB(2, "n2") RWKV_QFB(3, "n3")
        RWKV_QFW(0, "s0", "n0") RWKV_QFW(1, "s1", "n1") RWKV_QFW(2, "s2", "n2") RWKV_QFW(3, "s3", "n3")
        RWKV_QYP(0, "n0") RWKV_QYP(1, "n1") RWKV_QYP(2, "n2") RWKV_QYP(3, "n3")
        : [n0] "=&v"(N[0]), [n1] "=&v"(N[1]), [n2] "=&v"(N[2]), [n3] "=&v"(N[3]), [y] "+v"(y), [p] "+v"(p)
        : [s0] "v"(S[0]), [s1] "v"(S[1]), [s2] "v"(S[2]), [s3] "v"(S[3]), [K] "v"(K), [B] "v"(B), [W] "v"(W),
          [R] "v"(R), [A] "v"(A), [vv] "v"(vv), [sa] "v"(sa));
}

// p += Σ_c a_c·S_c over the lane's 4 columns.
__device__ __forceinline__ void fwd_dot4(const float (&S)[4], float A, float& p) {
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %[p], %[A], %[s0]" RWKV_QB(0) "v_fmac_f32_dpp %[p], %[A], %[s1]" RWKV_QB(1)
        "v_fmac_f32_dpp %[p], %[A], %[s2]" RWKV_QB(2) "v_fmac_f32_dpp %[p], %[A], %[s3]" RWKV_QB(3)
        : [p] "+v"(p)
        : [s0] "v"(S[0]), [s1] "v"(S[1]), [s2] "v"(S[2]), [s3] "v"(S[3]), [A] "v"(A));
}

// Sum of a value row's 16 column-group partials (lanes l & 3 + 4g): within a
// 16-lane DPP row the lanes 8 and then 4 apart (row_ror), then across the
// four DPP rows (rowsum4).  Every lane of the row ends with the same bits.
__device__ __forceinline__ float rowsum16(float x) {
    float t, u;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "=&v"(t) : "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:4 row_mask:0xf bank_mask:0xf" : "=&v"(u) : "v"(t));
    return rowsum4(u);
}

// rowsum4 / rowsum16 of two independent values with their instructions
// interleaved (the same operations per value, so the same bits): the next
// step's sa and the last step's y are reduced together, which hides the
// latency of each chain's dependent steps.
#define RWKV_SWAP_PAIR(OP)                        \
    "v_mov_b32 %[b0], %[x0]\n\t"                 \
    "v_mov_b32 %[b1], %[x1]\n\t"                 \
    "s_nop 1\n\t"                                \
    OP " %[x0], %[b0]\n\t"                       \
    OP " %[x1], %[b1]\n\t"                       \
    "v_add_f32 %[x0], %[x0], %[b0]\n\t"          \
    "v_add_f32 %[x1], %[x1], %[b1]\n\t"
__device__ __forceinline__ void rowsum4_pair(float& x0, float& x1) {
    float b0, b1;
    asm("s_nop 1\n\t" RWKV_SWAP_PAIR("v_permlane16_swap_b32") RWKV_SWAP_PAIR("v_permlane32_swap_b32")
        : [x0] "+v"(x0), [x1] "+v"(x1), [b0] "=&v"(b0), [b1] "=&v"(b1));
}
__device__ __forceinline__ void rowsum16_pair(float& x0, float& x1) {
    float b0, b1;
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %[b0], %[x0], %[x0] row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %[b1], %[x1], %[x1] row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_add_f32_dpp %[x0], %[b0], %[b0] row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %[x1], %[b1], %[b1] row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
        RWKV_SWAP_PAIR("v_permlane16_swap_b32") RWKV_SWAP_PAIR("v_permlane32_swap_b32")
        : [x0] "+v"(x0), [x1] "+v"(x1), [b0] "=&v"(b0), [b1] "=&v"(b1));
}

// Layout choice, a function of B·H only (so every entry point agrees bitwise
// for a given batch and head count): four rows per wave while sixteen would
// leave the chip with fewer waves than SIMDs (1,024).
__host__ __device__ constexpr bool use_rows4(int64_t BH) { return BH < 256; }

// Sum over the 64 lanes of a full wave, the same bits in every lane: within
// each 16-lane DPP row the lanes 8, 4, 2 and 1 apart (row_ror; each lane's
// partner pairs the same values, so the row's lanes agree), then across the
// four rows (rowsum4).  DPP and lane swaps only — no LDS round trips.
__device__ __forceinline__ float wave_total(float x) {
    float t, u;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "=&v"(t) : "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:4 row_mask:0xf bank_mask:0xf" : "=&v"(u) : "v"(t));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:2 row_mask:0xf bank_mask:0xf" : "=&v"(t) : "v"(u));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:1 row_mask:0xf bank_mask:0xf" : "=&v"(u) : "v"(t));
    return rowsum4(u);
}

// ── decode: the T = 1 step of one head and the tmix tail ──
// Lane l of every layout holds element l of the step vectors a, w, k, b, r
// and the v of its own value row.  `hin` / `hout`: the head's state [64, 64]
// (hin NULL = zeros; may alias).  Returns the row's y (in every lane of the
// row); the forward kernels' T = 1 path performs the same operations.

// Sixteen-row layout, wave `blk` of four: rows 16·blk + (l & 15), columns
// 16·(l >> 4) .. +15.
__device__ __forceinline__ int step16_row(int blk, int l) { return 16 * blk + (l & 15); }
__device__ __forceinline__ void load_state16(const float* __restrict__ hin, int blk, int l, float (&S)[16]) {
    if (hin) {
        const float4* src = reinterpret_cast<const float4*>(hin + (int64_t)step16_row(blk, l) * D + 16 * (l >> 4));
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float4 f = src[m];
            S[4 * m] = f.x; S[4 * m + 1] = f.y; S[4 * m + 2] = f.z; S[4 * m + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) S[c] = 0.0f;
    }
}
__device__ __forceinline__ float head_step16_regs(const float (&S)[16], float* __restrict__ hout, int blk, int l,
                                                  float A, float W, float K, float Bv, float R, float V) {
    float N[16];
    float p = 0.0f;
    fwd_dot16(S, A, p);
    const float sa = rowsum4(p);
    float y = 0.0f;
    p = 0.0f;
    fwd_update16(S, N, K, Bv, W, R, A, V, sa, y, p);
    y = rowsum4(y);
    float4* dst = reinterpret_cast<float4*>(hout + (int64_t)step16_row(blk, l) * D + 16 * (l >> 4));
#pragma unroll
    for (int m = 0; m < 4; ++m) dst[m] = make_float4(N[4 * m], N[4 * m + 1], N[4 * m + 2], N[4 * m + 3]);
    return y;
}
__device__ __forceinline__ float head_step16(const float* __restrict__ hin, float* __restrict__ hout, int blk, int l,
                                             float A, float W, float K, float Bv, float R, float V) {
    float S[16];
    load_state16(hin, blk, l, S);
    return head_step16_regs(S, hout, blk, l, A, W, K, Bv, R, V);
}

// Four-row layout, wave `blk` of sixteen: rows 4·blk + (l & 3), columns
// 4·(l >> 2) .. +3.
__device__ __forceinline__ int step4_row(int blk, int l) { return 4 * blk + (l & 3); }
__device__ __forceinline__ void load_state4(const float* __restrict__ hin, int blk, int l, float (&S)[4]) {
    if (hin) {
        const float4 f = *reinterpret_cast<const float4*>(hin + (int64_t)step4_row(blk, l) * D + 4 * (l >> 2));
        S[0] = f.x; S[1] = f.y; S[2] = f.z; S[3] = f.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) S[c] = 0.0f;
    }
}
__device__ __forceinline__ float head_step4_regs(const float (&S)[4], float* __restrict__ hout, int blk, int l,
                                                 float A, float W, float K, float Bv, float R, float V) {
    float N[4];
    float p = 0.0f;
    fwd_dot4(S, A, p);
    const float sa = rowsum16(p);
    float y = 0.0f;
    p = 0.0f;
    fwd_update4(S, N, K, Bv, W, R, A, V, sa, y, p);
    y = rowsum16(y);
    *reinterpret_cast<float4*>(hout + (int64_t)step4_row(blk, l) * D + 4 * (l >> 2)) = make_float4(N[0], N[1], N[2], N[3]);
    return y;
}
__device__ __forceinline__ float head_step4(const float* __restrict__ hin, float* __restrict__ hout, int blk, int l,
                                            float A, float W, float K, float Bv, float R, float V) {
    float S[4];
    load_state4(hin, blk, l, S);
    return head_step4_regs(S, hout, blk, l, A, W, K, Bv, R, V);
}

// The tmix tail of element l of one head (S = 64): wkv x, r, k, v, g of the
// element, rk / lnw / lnb of the head; wkv_tail_kernel's operation sequence.
__device__ __forceinline__ float head_tail(float x, float r, float k, float v, float rk, float lnw, float lnb,
                                           float g, float eps) {
    const float mean = wave_total(0.0f + x) / (float)D;
    const float dd = x - mean;
    const float inv = 1.0f / sqrtf(wave_total(fmaf(dd, dd, 0.0f)) / (float)D + eps);
    const float dp = wave_total(fmaf(r * k, rk, 0.0f));
    const float nrm = (x - mean) * inv;
    const float yo = fmaf(dp, v, fmaf(nrm, lnw, lnb));
    return yo * g;
}

}  // namespace rwkv_wkv
