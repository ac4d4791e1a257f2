// Batched sb6 4-bit GEMV on the matrix cores: y[n, row] = Σ_c W[row, c]·x[n, c]
// for 2…32 inputs, the weights streamed once for all of them
// (RwkvqSb6GEMV.swift:159-190 per input row; the batch the reference runs as
// one launch per row, BatchGenerate.swift:58-90).
//
// A 32-column unit of a row carries 4-bit codes c and the block scales
// s = half(qs·d), m = half(qm·dm): w = c·s + m, so per unit
//   y += s·Σ c·x + m·Σ x.
// Σ c·x runs on v_mfma_f32_16x16x32_bf16: the codes are exact in bf16 and
// each input splits exactly into three bf16 parts (x = x1 + x2 + x3, 24
// significant bits), so the three products per unit are exact and only the
// fp32 accumulation rounds.  The A operand is 16 inputs × the unit's 32
// columns, the B operand the unit's codes of 16 rows, the accumulator lane
// i + 16g holds inputs 4g..4g+3 of row i — the lane's own row, whose two
// scales it folds in fp32 after the three MFMAs.  Results agree with the
// one-input VALU kernel to fp32 rounding (the sums are taken in another
// order), not bitwise.
//
// K3 layout: a unit's 16 bytes hold column c in the low nibble of byte c and
// column c + 16 in the high nibble (c < 16).  Lane g of a row takes bytes
// 4g..4g+3: its eight k slots are columns 4g..4g+3 (low nibbles) and
// 16+4g..16+4g+3 (high nibbles); the staged inputs use the same slot order.
// A nibble byte 0000nnnn read as fp8 E4M3 is n·2⁻⁹, so
// v_cvt_scalef32_pk_bf16_fp8 with scale 2⁹ turns two code bytes into two
// exact bf16 codes.
//
// Workgroup = 4 waves × RT tiles of 16 rows, over KW units (a K slice):
// the inputs of the slice are staged once in LDS as bf16 parts and unit
// sums, the weights of every (row, unit) are read once, all in flight
// before the staging.  K slices write fp32 partials [KS][N][OUT]; a second
// kernel sums them in slice order and applies the epilogue (store, add to
// y, relu²), so the result does not depend on scheduling.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int KW_MAX = 16;   // units per workgroup
constexpr int KS_MAX = 128;  // K slices (IN ≤ 16384 at 4 units per slice)

__device__ __forceinline__ float f16f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}
__device__ __forceinline__ float hround(float x) { return (float)(_Float16)x; }

struct BatchArgs {
    const float* x;      // [N, NK, IN]
    const uint32_t* q;   // K3 nibbles: [OUT, NU] units of 4 dwords
    const uint16_t* sm;  // [OUT, NU] (qs u8, qm i8)
    const uint32_t* dd;  // [OUT, NU/8] (d, dm) fp16
    const uint16_t* ts;  // T16 layout: s and m per (row, unit), fp16 (the codes in q)
    const uint16_t* tm;
    float* part;         // [KS, N, OUT]
    int N, OUT, IN, out_per, KS;
    int NK;    // fused matrices (OUT / out_per), each with its own input row
    int NRG;   // row groups (64·RT rows) per fused matrix
    int G;     // workgroups per (K slice, matrix), each a run of NRG / G row groups
};

// Exchanges between the 16-lane rows of a wave (rows = g): permlane16_swap
// trades the odd rows of its first operand with the even rows of its
// second, permlane32_swap rows 2-3 of the first with rows 0-1 of the second.
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// r_d of row g ← r_g of row d (a 4×4 transpose of dwords across the rows).
__device__ __forceinline__ void transpose4(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    swap16(r0, r1);
    swap16(r2, r3);
    swap32(r0, r2);
    swap32(r1, r3);
}

// Eight codes of one lane (its dword of the unit) as bf16, in slot order.
__device__ __forceinline__ bf16x8 codes_bf16(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The inputs of a K slice (KW units from u0, input row `mat` of each of N
// inputs) for the A operand.  Issued first (L2 hits): job → (input n, lane
// group gg, unit uu), the four gg of one (n, uu) in lanes n, n + 16, n + 32,
// n + 48 of one wave.
template <int NTL, int KW>
struct SliceInputs {
    static constexpr int JOBS = (KW * NTL * 64 + 255) / 256;   // jobs per thread
    float4 xa[JOBS], xb[JOBS];

    __device__ __forceinline__ void issue(const BatchArgs& A, int mat, int u0, int tid) {
        const int lane = tid & 63;
#pragma unroll
        for (int k = 0; k < JOBS; ++k) {
            const int blk = (tid + 256 * k) >> 6;
            const int n = (lane & 15) + 16 * (blk % NTL), gg = lane >> 4, uu = blk / NTL;
            xa[k] = xb[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (n < A.N) {
                const float* src = A.x + ((int64_t)n * A.NK + mat) * A.IN + (u0 + uu) * 32;
                xa[k] = *reinterpret_cast<const float4*>(src + 4 * gg);
                xb[k] = *reinterpret_cast<const float4*>(src + 16 + 4 * gg);
            }
        }
    }

    // bf16 parts in A-operand order into Xp[uu][t][part][lane] (16 bytes =
    // a lane's eight bf16 slots) and the unit sums Xs[uu][n]
    __device__ __forceinline__ void stage(uint4* Xp, float* Xs, int tid) const {
        constexpr int NI = 16 * NTL;
        const int lane = tid & 63;
#pragma unroll
        for (int k = 0; k < JOBS; ++k) {
            const int blk = (tid + 256 * k) >> 6;
            const int n = (lane & 15) + 16 * (blk % NTL), gg = lane >> 4, uu = blk / NTL;
            const float4 a = xa[k], b = xb[k];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            bf16x8 p1, p2, p3;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const __bf16 h1 = (__bf16)v[e];
                const float r1 = v[e] - (float)h1;
                const __bf16 h2 = (__bf16)r1;
                p1[e] = h1;
                p2[e] = h2;
                p3[e] = (__bf16)(r1 - (float)h2);
            }
            uint4* dst = Xp + ((uu * NTL + (n >> 4)) * 3) * 64 + gg * 16 + (n & 15);
            dst[0] = __builtin_bit_cast(uint4, p1);
            dst[64] = __builtin_bit_cast(uint4, p2);
            dst[128] = __builtin_bit_cast(uint4, p3);
            // Σ of the unit's 32 columns: the first and the second 16, each
            // over the four lane groups (butterfly: every lane gets the same sums)
            float h0 = a.x + a.y + a.z + a.w, h1 = b.x + b.y + b.z + b.w;
            h0 += __shfl_xor(h0, 16);
            h1 += __shfl_xor(h1, 16);
            h0 += __shfl_xor(h0, 32);
            h1 += __shfl_xor(h1, 32);
            if (gg == 0) Xs[uu * NI + n] = h0 + h1;
        }
    }
};

// The weights of one pipeline step: a group of 4 units (4 × 32 columns) of the
// wave's RT row tiles.  Lane g of row i loads unit g of the group whole
// (16 bytes); a 4×4 transpose across the four 16-lane rows later leaves lane
// g with dword g of every unit, the k slots its B operand needs.  The scales
// of a row group's whole K slice come with its first step: lane g of row i
// holds those of the slice's unit group g (qs, qm of its 4 units and the
// super-block's d, dm), and step q takes them from lane q of the row.
template <int RT>
struct StepBuf {
    uint32_t cw[RT][4];
    uint2 smv[RT];
    uint32_t ddv[RT];
};

template <int NTL, int RT, int KW>
__global__ __launch_bounds__(256) void sb6_gemv_mfma_kernel(BatchArgs A) {
    constexpr int NI = 16 * NTL;     // inputs of the launch, padded to whole tiles
    constexpr int NB = 4;            // weight buffers: NB − 1 steps in flight while one is multiplied
    constexpr int QPR = KW / 4;      // steps (unit groups) per row group
    constexpr int LQ = QPR == 4 ? 2 : QPR == 2 ? 1 : 0;
    static_assert(NB % QPR == 0, "ring slots must map to fixed unit groups");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // Xp[uu][t][part][lane]: 16 bytes = the lane's eight bf16 slots;  Xs[uu][n]: unit sums
    uint4* Xp = reinterpret_cast<uint4*>(smem);
    float* Xs = reinterpret_cast<float*>(smem + (size_t)KW * NTL * 3 * 64 * 16);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, i = lane & 15;
    // workgroup → (K slice, fused matrix, run of row groups of that matrix):
    // the slice's inputs are staged once and every row group of the run
    // streams through them
    const int ks = (int)blockIdx.x % A.KS, rest = (int)blockIdx.x / A.KS;
    const int mat = rest % A.NK, j = rest / A.NK;
    const int rg_lo = (int)((int64_t)j * A.NRG / A.G), rg_hi = (int)((int64_t)(j + 1) * A.NRG / A.G);
    const int NU = A.IN >> 5, NSB = NU >> 3;
    const int u0 = ks * KW;                          // NU % KW == 0: every slice is whole
    const int S = (rg_hi - rg_lo) << LQ;             // steps of every wave
    const int64_t mrow0 = (int64_t)mat * A.out_per;  // first row of the fused matrix
    if (S <= 0) return;   // (G ≤ NRG gives every workgroup a row group)

    // Issue order: the slice's inputs (L2 hits), then the first NB − 1 steps'
    // weights (HBM).  Loads complete in issue order, so the staging waits
    // only for the inputs.
    SliceInputs<NTL, KW> xin;
    xin.issue(A, mat, u0, tid);

    // Addresses: a uniform base per step (row group, unit group) plus a
    // per-lane 32-bit byte offset fixed for the whole kernel (the lane's row
    // within the row group, its unit of the group), so a load costs no VALU
    // address arithmetic.  Rows need no clamp: a matrix's rows are exactly
    // NRG row groups of 64·RT.
    const int gs = min(g, QPR - 1);   // the unit group whose scales lane g loads
    uint32_t oc[RT], os[RT], od[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t rl = (uint32_t)((wave * RT + rt) * 16 + i);
        oc[rt] = (rl * NU + g) * 16;
        os[rt] = (rl * NU + 4 * gs) * 2;
        od[rt] = (rl * NSB + ((u0 + 4 * gs) >> 3) - (u0 >> 3)) * 4;
    }
    // step s = (row group rg_lo + (s >> LQ), unit group s & (QPR − 1)); a step
    // past the last loads the last one again (unused), so every load is
    // issued unconditionally and the waits count statically.  Ring slot SLOT
    // always holds unit group SLOT % QPR (NB and the loop step are multiples
    // of QPR), so only the slots of unit group 0 load scales.
    auto load = [&](StepBuf<RT>& b, int s, auto slot) {
        constexpr int SLOT = decltype(slot)::value;
        s = min(s, S - 1);
        const int rg = rg_lo + (s >> LQ), ug = u0 + 4 * (SLOT % QPR);
        const int64_t rb = mrow0 + (int64_t)rg * 64 * RT;
        const char* qb = reinterpret_cast<const char*>(A.q) + (rb * NU + ug) * 16;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint4 w = *reinterpret_cast<const uint4*>(qb + oc[rt]);
            b.cw[rt][0] = w.x; b.cw[rt][1] = w.y; b.cw[rt][2] = w.z; b.cw[rt][3] = w.w;
        }
        if constexpr (SLOT % QPR == 0) {
            const char* sb = reinterpret_cast<const char*>(A.sm) + (rb * NU + u0) * 2;
            const char* db = reinterpret_cast<const char*>(A.dd) + (rb * NSB + (u0 >> 3)) * 4;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                b.smv[rt] = *reinterpret_cast<const uint2*>(sb + os[rt]);
                b.ddv[rt] = *reinterpret_cast<const uint32_t*>(db + od[rt]);
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    // every wave's input loads go out before any wave's weight loads, so the
    // staging does not wait behind the weights in the CU's memory queue
    __builtin_amdgcn_s_barrier();
    StepBuf<RT> b0, b1, b2, b3;
    load(b0, 0, S0{});
    load(b1, 1, S1{});
    load(b2, 2, S2{});

    xin.stage(Xp, Xs, tid);
    __syncthreads();

    f32x4 acc[RT][NTL];
    uint2 smc[RT];     // the current row group's scales (lane g: unit group g)
    uint32_t ddc[RT];
    // one step: the group's 4 units of the wave's RT row tiles; a row group's
    // partials are stored after its last unit group
    auto step = [&](StepBuf<RT>& b, int s, auto slot) {
        constexpr int Q = decltype(slot)::value % QPR;
        if (s >= S) return;   // uniform
        if constexpr (Q == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                smc[rt] = b.smv[rt];
                ddc[rt] = b.ddv[rt];
#pragma unroll
                for (int t = 0; t < NTL; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float dsc[RT], dmc[RT];
        uint32_t sq[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            transpose4(b.cw[rt][0], b.cw[rt][1], b.cw[rt][2], b.cw[rt][3]);
            const uint32_t dq = __shfl(ddc[rt], i + 16 * Q);
            sq[rt][0] = __shfl(smc[rt].x, i + 16 * Q);
            sq[rt][1] = __shfl(smc[rt].y, i + 16 * Q);
            dsc[rt] = f16f(dq);
            dmc[rt] = f16f(dq >> 16);
        }
        // the units in pairs: both units' A operands, then the 2·RT·NTL
        // independent product chains, then their folds
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            bf16x8 ap[2][NTL][3];
            float4 xs[2][NTL];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int uu = 4 * Q + 2 * kp + k2;
#pragma unroll
                for (int t = 0; t < NTL; ++t) {
#pragma unroll
                    for (int p = 0; p < 3; ++p)
                        ap[k2][t][p] = __builtin_bit_cast(bf16x8, Xp[((uu * NTL + t) * 3 + p) * 64 + lane]);
                    xs[k2][t] = *reinterpret_cast<const float4*>(Xs + uu * NI + t * 16 + 4 * g);
                }
            }
            bf16x8 bc[2][RT];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) bc[k2][rt] = codes_bf16(b.cw[rt][2 * kp + k2]);
            f32x4 d[2][RT][NTL];
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int t = 0; t < NTL; ++t)
                            d[k2][rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                ap[k2][t][p], bc[k2][rt], p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[k2][rt][t], 0, 0, 0);
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const uint32_t smr = (sq[rt][kp] >> (16 * k2)) & 0xffffu;
                    const float sv = hround((float)(smr & 0xffu) * dsc[rt]);
                    const float mv = hround((float)(int8_t)(smr >> 8) * dmc[rt]);
#pragma unroll
                    for (int t = 0; t < NTL; ++t) {
                        const float xsv[4] = {xs[k2][t].x, xs[k2][t].y, xs[k2][t].z, xs[k2][t].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[rt][t][e] = fmaf(mv, xsv[e], fmaf(sv, d[k2][rt][t][e], acc[rt][t][e]));
                    }
                }
            }
        }
        if constexpr (Q == QPR - 1) {
            // partials of this K slice: lane holds inputs 4g..4g+3 (+16t) of its row
            const int64_t rbase = mrow0 + (int64_t)(rg_lo + (s >> LQ)) * 64 * RT + wave * RT * 16 + i;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < NTL; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int n = t * 16 + 4 * g + e;
                        if (n < A.N)
                            A.part[((int64_t)ks * A.N + n) * A.OUT + rbase + rt * 16] = acc[rt][t][e];
                    }
        }
    };
    // a ring of NB buffers: the load for step s + NB − 1 goes out before step s
    for (int s = 0; s < S; s += NB) {
        load(b3, s + 3, S3{});
        step(b0, s, S0{});
        load(b0, s + 4, S0{});
        step(b1, s + 1, S1{});
        load(b1, s + 5, S1{});
        step(b2, s + 2, S2{});
        load(b2, s + 6, S2{});
        step(b3, s + 3, S3{});
    }
}

// ---------------------------------------------------------------------------
// T16 layout: the same weights permuted for this kernel's loads, and the unit
// scales precomputed (rwkv_sb6_t16_pack).  Per 16-row tile (rows 16r..16r+15)
// and group of 4 units (4G..4G+3), in tile order [r][G]:
//   codes  1 KiB: the 16 bytes at offset (g·16 + i)·16 are dword g of units
//          4G..4G+3 of row 16r + i (a K3 unit's dword g: columns 4g..4g+3 in
//          the low nibbles, 16+4g.. in the high ones), so lane i + 16g of one
//          16-byte load per lane holds its B-operand slots of all four units;
//   s      [16 rows][4 units] fp16: s = half(qs·d), the value the K3 kernels
//          round per unit;
//   m      [16 rows][8] bf16: m = half(qm·dm) as two exact bf16 parts, the
//          four units' high parts, then their low parts (m = hi + lo).
// One step's codes are 1 KiB contiguous per row tile (8 whole cache lines,
// where a K3 load touches 16 rows' half lines), its scales 128 bytes.
//
// The m·Σx term of every unit runs on the matrix cores once per row group:
// A = the slice's unit sums Σx [16 inputs × 16 units] in three bf16 parts,
// B = m [16 units × 16 rows] in its two bf16 parts, six
// v_mfma_f32_16x16x16_bf16 into the row group's accumulator; per unit only
// acc += s·(Σ c·x) stays on the VALU.
template <int RT>
struct T16Buf {
    uint32_t cw[RT][4];   // codes: dword g of the group's units 0..3, row i
    uint2 sv[RT];         // s of the group's 4 units, row i
    uint4 mv[RT];         // m (bf16 hi ×4, lo ×4) of the slice's unit group g, row i (first step of a row group)
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <int NTL, int RT, int KW>
__global__ __launch_bounds__(256) void sb6_t16_gemv_mfma_kernel(BatchArgs A) {
    constexpr int NI = 16 * NTL;
    constexpr int NB = 4;
    constexpr int QPR = KW / 4;
    constexpr int LQ = QPR == 4 ? 2 : QPR == 2 ? 1 : 0;
    static_assert(NB % QPR == 0, "ring slots must map to fixed unit groups");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint4* Xp = reinterpret_cast<uint4*>(smem);
    float* Xs = reinterpret_cast<float*>(smem + (size_t)KW * NTL * 3 * 64 * 16);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, i = lane & 15;
    const int ks = (int)blockIdx.x % A.KS, rest = (int)blockIdx.x / A.KS;
    const int mat = rest % A.NK, j = rest / A.NK;
    const int rg_lo = (int)((int64_t)j * A.NRG / A.G), rg_hi = (int)((int64_t)(j + 1) * A.NRG / A.G);
    const int NU = A.IN >> 5, NG = NU >> 2;
    const int u0 = ks * KW;
    const int S = (rg_hi - rg_lo) << LQ;
    const int64_t mrow0 = (int64_t)mat * A.out_per;
    if (S <= 0) return;

    SliceInputs<NTL, KW> xin;
    xin.issue(A, mat, u0, tid);

    // per-lane byte offsets within a row group (row tile tt = wave·RT + rt)
    const int gs = min(g, QPR - 1);
    uint32_t oc[RT], os[RT], om[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t tt = (uint32_t)(wave * RT + rt);
        oc[rt] = tt * NG * 1024 + lane * 16;
        os[rt] = tt * NG * 128 + i * 8;
        om[rt] = tt * NG * 256 + gs * 256 + i * 16;
    }
    auto load = [&](T16Buf<RT>& b, int s, auto slot) {
        constexpr int SLOT = decltype(slot)::value;
        s = min(s, S - 1);
        const int64_t rtile = (mrow0 + (int64_t)(rg_lo + (s >> LQ)) * 64 * RT) >> 4;
        const int64_t tile = rtile * NG + (u0 >> 2) + SLOT % QPR;
        const char* qb = reinterpret_cast<const char*>(A.q) + tile * 1024;
        const char* sb = reinterpret_cast<const char*>(A.ts) + tile * 128;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint4 w = *reinterpret_cast<const uint4*>(qb + oc[rt]);
            b.cw[rt][0] = w.x; b.cw[rt][1] = w.y; b.cw[rt][2] = w.z; b.cw[rt][3] = w.w;
            b.sv[rt] = *reinterpret_cast<const uint2*>(sb + os[rt]);
        }
        if constexpr (SLOT % QPR == 0) {
            const char* mb = reinterpret_cast<const char*>(A.tm) + (rtile * NG + (u0 >> 2)) * 256;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) b.mv[rt] = *reinterpret_cast<const uint4*>(mb + om[rt]);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    __builtin_amdgcn_s_barrier();
    T16Buf<RT> b0, b1, b2, b3;
    load(b0, 0, S0{});
    load(b1, 1, S1{});
    load(b2, 2, S2{});
    xin.stage(Xp, Xs, tid);
    __syncthreads();

    // A operand of the m·Σx products: lane (i, g) = input i (+16t), units
    // 4g..4g+3 of the slice (zero past KW), three exact bf16 parts
    bf16x4 a2[NTL][3];
#pragma unroll
    for (int t = 0; t < NTL; ++t)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int uu = 4 * g + kk;
            const float v = uu < KW ? Xs[uu * NI + t * 16 + i] : 0.0f;
            const __bf16 h1 = (__bf16)v;
            const float r1 = v - (float)h1;
            const __bf16 h2 = (__bf16)r1;
            a2[t][0][kk] = h1;
            a2[t][1][kk] = h2;
            a2[t][2][kk] = (__bf16)(r1 - (float)h2);
        }

    f32x4 acc[RT][NTL];
    auto step = [&](T16Buf<RT>& b, int s, auto slot) {
        constexpr int Q = decltype(slot)::value % QPR;
        if (s >= S) return;   // uniform
        if constexpr (Q == 0) {
            // the row group's m·Σx over the whole slice (units past KW have A = 0)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const bf16x4 bh = __builtin_bit_cast(bf16x4, make_uint2(b.mv[rt].x, b.mv[rt].y));
                const bf16x4 bl = __builtin_bit_cast(bf16x4, make_uint2(b.mv[rt].z, b.mv[rt].w));
#pragma unroll
                for (int t = 0; t < NTL; ++t) {
                    f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int pa = 0; pa < 3; ++pa) {
                        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a2[t][pa], bh, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a2[t][pa], bl, c, 0, 0, 0);
                    }
                    acc[rt][t] = c;
                }
            }
        }
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            bf16x8 ap[2][NTL][3];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int uu = 4 * Q + 2 * kp + k2;
#pragma unroll
                for (int t = 0; t < NTL; ++t)
#pragma unroll
                    for (int p = 0; p < 3; ++p)
                        ap[k2][t][p] = __builtin_bit_cast(bf16x8, Xp[((uu * NTL + t) * 3 + p) * 64 + lane]);
            }
            bf16x8 bc[2][RT];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) bc[k2][rt] = codes_bf16(b.cw[rt][2 * kp + k2]);
            f32x4 d[2][RT][NTL];
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int t = 0; t < NTL; ++t)
                            d[k2][rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                ap[k2][t][p], bc[k2][rt], p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[k2][rt][t], 0, 0, 0);
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const float sv = f16f((kp == 0 ? b.sv[rt].x : b.sv[rt].y) >> (16 * k2));
#pragma unroll
                    for (int t = 0; t < NTL; ++t)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[rt][t][e] = fmaf(sv, d[k2][rt][t][e], acc[rt][t][e]);
                }
        }
        if constexpr (Q == QPR - 1) {
            const int64_t rbase = mrow0 + (int64_t)(rg_lo + (s >> LQ)) * 64 * RT + wave * RT * 16 + i;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < NTL; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int n = t * 16 + 4 * g + e;
                        if (n < A.N)
                            A.part[((int64_t)ks * A.N + n) * A.OUT + rbase + rt * 16] = acc[rt][t][e];
                    }
        }
    };
    for (int s = 0; s < S; s += NB) {
        load(b3, s + 3, S3{});
        step(b0, s, S0{});
        load(b0, s + 4, S0{});
        step(b1, s + 1, S1{});
        load(b1, s + 5, S1{});
        step(b2, s + 2, S2{});
        load(b2, s + 6, S2{});
        step(b3, s + 3, S3{});
    }
}

// Row-owned kernel over T16 weights, for matrices whose K slices would
// leave too little work per workgroup (a few units of a few row groups) and
// a second launch to sum them: one workgroup per (RT 16-row tiles, 16-input
// tile), its W waves splitting K (wave w takes unit groups w, w + W, …) and
// loading their inputs straight into A-operand registers (no LDS staging: no
// other wave reads them).  The W accumulators are summed in LDS in wave
// order and the epilogue applied in the same launch; no workspace.  Per
// unit the MFMAs give Σ c·x (B = the codes, per row tile) and Σ x (B = ones,
// shared by the row tiles) of the lane's four inputs, so
// acc += s·Σ c·x + m·Σ x is two fmas per accumulator element.
template <int RT>
struct RowBuf {
    uint4 cw[RT];      // codes: dword g of the group's units 0..3, row i of row tile rt
    uint2 sv[RT];      // s of the 4 units, row i
    uint4 mv[RT];      // m of the 4 units (bf16 high ×4, low ×4), row i
    float4 xa[4], xb[4];   // input i of the tile, unit uu: columns 4g..4g+3 and 16+4g..16+4g+3
};

// RT row tiles per workgroup share its waves' inputs, their bf16 parts and
// unit sums.  SG > 0: every wave has at most SG unit groups (K ≤ SG·W
// groups), all loaded up front, no loop (SG = 1 leaves few enough registers
// for several workgroups per CU); SG = 0: any K, two groups in flight.
template <int W, int SG, int RT>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(SG == 1 ? 4 : 1)))
void sb6_t16_gemv_rows_kernel(BatchArgs A, float* __restrict__ y, int ep) {
    __shared__ f32x4 red[W][RT][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, i = lane & 15;
    const int64_t rtile0 = (int64_t)blockIdx.x * RT;
    const int64_t row0 = rtile0 * 16;
    const int n0 = 16 * (int)blockIdx.y, NL = min(16, A.N - n0);   // inputs of this tile
    const int mat = (int)(row0 / A.out_per);   // (out_per % (16·RT) == 0: one matrix)
    const int NG = A.IN >> 7;
    const int S = wave < NG ? (NG - 1 - wave) / W + 1 : 0;   // unit groups of this wave
    // inputs past the tile's last read that one, never stored
    const float* xrow = A.x + ((int64_t)(n0 + min(i, NL - 1)) * A.NK + mat) * A.IN + 4 * g;
    auto load = [&](RowBuf<RT>& b, int s) {
        s = min(s, S - 1);
        const int q = wave + s * W;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int64_t tile = (rtile0 + rt) * NG + q;
            b.cw[rt] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(A.q) + tile * 1024 + lane * 16);
            b.sv[rt] = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(A.ts) + tile * 128 + i * 8);
            b.mv[rt] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(A.tm) + tile * 256 + i * 16);
        }
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) {
            const float* src = xrow + (4 * q + uu) * 32;
            b.xa[uu] = *reinterpret_cast<const float4*>(src);
            b.xb[uu] = *reinterpret_cast<const float4*>(src + 16);
        }
    };
    f32x4 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const __bf16 one = (__bf16)1.0f;
    const bf16x8 ones = bf16x8{one, one, one, one, one, one, one, one};
    auto step = [&](const RowBuf<RT>& b) {
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) {
            const float4 xa = b.xa[uu], xb = b.xb[uu];
            const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            bf16x8 ap[3];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const __bf16 h1 = (__bf16)v[e];
                const float r1 = v[e] - (float)h1;
                const __bf16 h2 = (__bf16)r1;
                ap[0][e] = h1;
                ap[1][e] = h2;
                ap[2][e] = (__bf16)(r1 - (float)h2);
            }
            const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
            f32x4 sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[0], ones, z, 0, 0, 0);
            sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[1], ones, sx, 0, 0, 0);
            sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[2], ones, sx, 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint32_t cw[4] = {b.cw[rt].x, b.cw[rt].y, b.cw[rt].z, b.cw[rt].w};
                const uint32_t mw[4] = {b.mv[rt].x, b.mv[rt].y, b.mv[rt].z, b.mv[rt].w};
                const bf16x8 bc = codes_bf16(cw[uu]);
                const uint32_t s2 = uu < 2 ? b.sv[rt].x : b.sv[rt].y;
                const float sv = f16f(s2 >> (16 * (uu & 1)));
                // m = high + low bf16 parts, exact in fp32
                const uint32_t mh = mw[uu >> 1] >> (16 * (uu & 1)), ml = mw[2 + (uu >> 1)] >> (16 * (uu & 1));
                const float mu = __uint_as_float(mh << 16) + __uint_as_float(ml << 16);
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[0], bc, z, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[1], bc, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[2], bc, d, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[rt][e] = fmaf(mu, sx[e], fmaf(sv, d[e], acc[rt][e]));
            }
        }
    };
    if constexpr (SG == 1) {
        if (S == 1) {
            RowBuf<RT> b0;
            load(b0, 0);
            step(b0);
        }
    } else if constexpr (SG == 2) {
        if (S == 2) {
            RowBuf<RT> b0, b1;
            load(b0, 0);
            load(b1, 1);
            step(b0);
            step(b1);
        } else if (S == 1) {
            RowBuf<RT> b0;
            load(b0, 0);
            step(b0);
        }
    } else if (S == 1) {
        RowBuf<RT> b0;
        load(b0, 0);
        step(b0);
    } else if (S > 1) {
        // two buffers, the next group's loads in flight while one is
        // multiplied; loads past the last group reload it (clamped, unused),
        // so the waits count statically
        RowBuf<RT> b0, b1;
        load(b0, 0);
        for (int s = 0; s < S; s += 2) {
            load(b1, s + 1);
            step(b0);
            load(b0, s + 2);
            if (s + 1 < S) step(b1);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) red[wave][rt][lane] = acc[rt];
    __syncthreads();
    // output (row tile rt, input n, row r): lane r + 16·(n / 4), component
    // n mod 4; waves summed in order
    const float* rf = reinterpret_cast<const float*>(&red[0][0][0]);
    for (int o = tid; o < 256 * RT; o += 64 * W) {
        const int r = o & 15, n = (o >> 4) & 15, rt = o >> 8;
        if (n < NL) {
            const int off = (rt * 64 + r + 16 * (n >> 2)) * 4 + (n & 3);
            float v = rf[off];
#pragma unroll
            for (int w = 1; w < W; ++w) v += rf[w * RT * 256 + off];
            float* yo = y + (int64_t)(n0 + n) * A.OUT + row0 + rt * 16 + r;
            if (ep == 1) {
                v = *yo + v;
            } else if (ep == 2) {
                v = fmaxf(v, 0.0f);
                v = v * v;
            }
            *yo = v;
        }
    }
}

// K3 → T16: one thread per (row, unit).
__global__ __launch_bounds__(256) void sb6_t16_pack_kernel(const uint4* __restrict__ qblk,
                                                           const uint16_t* __restrict__ qsqm,
                                                           const uint32_t* __restrict__ ddm, int64_t OUT, int NU,
                                                           uint4* __restrict__ tq, uint16_t* __restrict__ ts,
                                                           uint16_t* __restrict__ tm) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= OUT * NU) return;
    const int64_t row = e / NU;
    const int u = (int)(e - row * NU), NG = NU >> 2, NSB = NU >> 3;
    const int64_t tile = (row >> 4) * NG + (u >> 2);
    const int ri = (int)(row & 15), g = u & 3;
    const uint4 q = qblk[e];
    const uint32_t qd[4] = {q.x, q.y, q.z, q.w};
    uint32_t* tqw = reinterpret_cast<uint32_t*>(tq) + tile * 256;
#pragma unroll
    for (int d = 0; d < 4; ++d) tqw[(d * 16 + ri) * 4 + g] = qd[d];   // dword d of unit g → lane (ri, d), slot g
    const uint32_t sm = qsqm[e], dd = ddm[row * NSB + (u >> 3)];
    const _Float16 sv = (_Float16)((float)(sm & 0xffu) * f16f(dd));
    const float mv = (float)(_Float16)((float)(int8_t)(sm >> 8) * f16f(dd >> 16));
    const __bf16 mh = (__bf16)mv, ml = (__bf16)(mv - (float)mh);   // exact: 11 significant bits
    ts[tile * 64 + ri * 4 + g] = __builtin_bit_cast(uint16_t, sv);
    tm[tile * 128 + ri * 8 + g] = __builtin_bit_cast(uint16_t, mh);
    tm[tile * 128 + ri * 8 + 4 + g] = __builtin_bit_cast(uint16_t, ml);
}

// y[n, row] = epilogue(Σ_ks part[ks, n, row]), slices in order; V
// consecutive outputs per thread (V = 4 where y is 16-byte aligned).  Eight
// slices' loads in flight at a time, issued unconditionally (a slice past
// the last reloads the last, unused) so the waits count statically.
template <int V>
__global__ __launch_bounds__(256) void sb6_gemv_mfma_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                                   int64_t NO, int KS, int ep) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
    if (e >= NO) return;
    vec t;
    for (int k0 = 0; k0 < KS; k0 += 8) {
        vec p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = *reinterpret_cast<const vec*>(part + (int64_t)min(k0 + k, KS - 1) * NO + e);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k0 + k < KS) t = (k0 + k == 0) ? p[k] : t + p[k];
    }
    vec* yo = reinterpret_cast<vec*>(y + e);
    if (ep == 1) {
        t = *yo + t;
    } else if (ep == 2) {
#pragma unroll
        for (int c = 0; c < V; ++c) {
            const float r = fmaxf(t[c], 0.0f);
            t[c] = r * r;
        }
    }
    *yo = t;
}

struct BatchPlan {
    int NTL, RT, KW, KS, NK, NRG, G;
    size_t lds;
    int64_t ws_bytes;
    int64_t grid() const { return (int64_t)KS * NK * G; }
};

// Workgroups resident on the chip at once (two per CU at ≤ 80 KB of LDS),
// and the tile count below which K slices are narrowed (each slice adds a
// partial sum per output to write and reduce: 4096x4096 x16 at 256 tiles of
// 16 units 9.9 µs, at 512 of 8 units 11.8 µs).
constexpr int kResident = 2 * 256;
constexpr int kMinTiles = 256;

// Tiles of 32 rows per wave (16 for 17-32 inputs, or where a fused matrix's
// rows are not a multiple of 128) and K slices of 16 (8 for 17-32 inputs) units, halved
// while (slices × matrices × row groups) < kMinTiles, so that small matrices
// still fill the chip.  The row groups of a (slice, matrix) pair are dealt to
// G workgroups in equal runs, G chosen so the grid is about kResident.
bool plan_batch(int64_t N, int64_t OUT, int64_t IN, int64_t out_per, BatchPlan& p) {
    if (N < 2 || N > 32 || OUT < 16 || OUT % 16 || IN < 256 || IN % 256 || out_per < 64 || out_per % 64 ||
        OUT % out_per)
        return false;
    p.NTL = N <= 16 ? 1 : 2;
    // two row tiles per wave for ≤ 16 inputs; one for 17–32, whose two input
    // tiles already double the registers per row (1024x4096 x32 11.7 → 9.6 µs)
    p.RT = p.NTL == 1 && out_per % 128 == 0 ? 2 : 1;
    p.NK = (int)(OUT / out_per);
    const int64_t NU = IN / 32;
    auto tiles = [&](int RT, int KW) { return (out_per / (64 * RT)) * p.NK * ((NU + KW - 1) / KW); };
    p.KW = p.NTL == 1 ? KW_MAX : KW_MAX / 2;   // ≤ 49 KiB of LDS
    while (p.KW > 4 && (NU % p.KW || tiles(p.RT, p.KW) < kMinTiles)) p.KW >>= 1;
    if (p.RT == 2 && tiles(p.RT, p.KW) < kMinTiles / 2) p.RT = 1;
    p.NRG = (int)(out_per / (64 * p.RT));
    p.KS = (int)((NU + p.KW - 1) / p.KW);
    const int64_t pairs = (int64_t)p.KS * p.NK;
    const int64_t g0 = std::max<int64_t>(1, std::min<int64_t>(p.NRG, (kResident + pairs - 1) / pairs));
    const int64_t run = (p.NRG + g0 - 1) / g0;   // row groups per workgroup
    p.G = (int)((p.NRG + run - 1) / run);
    p.lds = (size_t)p.KW * p.NTL * 3 * 64 * 16 + (size_t)p.KW * 16 * p.NTL * 4;
    p.ws_bytes = (int64_t)p.KS * N * OUT * 4;
    return p.KS <= KS_MAX && p.grid() <= INT32_MAX;
}

// The row-owned kernel: 4, 8 or 16 waves per (16-row, 16-input) tile with
// at most two unit groups each up to K = 4096 (beyond, 8 waves that loop),
// two or four row tiles per workgroup once one per workgroup would be more
// workgroups than CUs.  Taken by the T16 entry up to 2^24 weights for
// K ≤ 3072, and for K ≤ 4096 where its grid is one round of up to 64
// workgroups or pairs of row tiles, where it measured faster per call than
// K slices plus their reduction (graph-timed: 1024x1024 x32 4.2 vs 6.5 µs,
// 4096x1024 x32 5.6 vs 8.9, 12288x1024 x32 9.9 vs 14.5, 6144x2048 x16 8.4
// vs 10.4, 3072x3072 x16 8.3 vs 10.3, 4096x4096 x32 12.9 vs 16.4,
// 1024x4096 x8 8.1 vs 8.9); elsewhere every workgroup's conversion of its
// whole K into bf16 parts outweighs the saved launch (1024x4096 x32 10.1 vs
// 9.4, 4096x4096 x16 10.9 vs 9.5, 16384x2048 x16 15.6 vs 13.9, 65536x768 x8
// 20.3 vs 17.6).
constexpr int64_t kRowsPair = 257;
constexpr int64_t kRowsQuad = 1024;

bool rows_kernel_taken(int64_t N, int64_t OUT, int64_t IN) {
    const int64_t w = OUT * IN, wg = (OUT / 16) * ((N + 15) / 16);
    if (IN > 4096 || w > ((int64_t)1 << 24)) return false;
    return IN <= 3072 || wg <= 64 || wg >= kRowsPair;
}

rwkv_status launch_rows(BatchArgs a, int64_t N, float* y, int64_t OUT, int64_t IN, int64_t out_per, int epilogue,
                        void* stream, const char* who) {
    BatchPlan p;
    RWKV_REQUIRE(epilogue >= 0 && epilogue <= 2, RWKV_E_SHAPE, "%s: epilogue %d", who, epilogue);
    RWKV_REQUIRE(plan_batch(N, OUT, IN, out_per, p), RWKV_E_SHAPE,
                 "%s: N=%lld OUT=%lld IN=%lld out_per=%lld (2 <= N <= 32, IN %% 256 == 0, "
                 "out_per %% 64 == 0 dividing OUT)",
                 who, (long long)N, (long long)OUT, (long long)IN, (long long)out_per);
    RWKV_REQUIRE(OUT * (IN / 32) * 16 < ((int64_t)1 << 40) && OUT / 16 <= INT32_MAX, RWKV_E_SHAPE,
                 "%s: matrix too large", who);
    RWKV_REQUIRE((uintptr_t)a.x % 16 == 0 && (uintptr_t)y % 4 == 0, RWKV_E_SHAPE, "%s: x must be 16-byte aligned",
                 who);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    a.N = (int)N;
    a.OUT = (int)OUT;
    a.IN = (int)IN;
    a.out_per = (int)out_per;
    a.NK = (int)(OUT / out_per);
    const int64_t NT = (N + 15) / 16, NG = IN / 128;
    // two row tiles per workgroup once one per workgroup would be more
    // workgroups than CUs, four (K ≤ 1024) from 1024 (8192x1024 x32 6.8 vs
    // 7.4 µs, 16384x1024 x32 10.5 vs 13.5; 4096x1024 x32 6.6 vs 5.5)
    const int64_t wg = (OUT / 16) * NT;
    const int RT = NG <= 8 && wg >= kRowsQuad ? 4 : wg >= kRowsPair ? 2 : 1;
    const dim3 grid((unsigned)(OUT / (16 * RT)), (unsigned)NT);
#define RWKV_ROWS(WV, SGV)                                                                          \
    if (RT == 2)                                                                                    \
        rwkv::launch(sb6_t16_gemv_rows_kernel<WV, SGV, 2>, grid, dim3(64 * (WV)), st, a, y, epilogue); \
    else                                                                                            \
        rwkv::launch(sb6_t16_gemv_rows_kernel<WV, SGV, 1>, grid, dim3(64 * (WV)), st, a, y, epilogue)
    if (NG <= 4) {
        if (RT == 4) rwkv::launch(sb6_t16_gemv_rows_kernel<4, 1, 4>, grid, dim3(256), st, a, y, epilogue);
        else RWKV_ROWS(4, 1);
    } else if (NG <= 8) {
        if (RT == 4) rwkv::launch(sb6_t16_gemv_rows_kernel<8, 1, 4>, grid, dim3(512), st, a, y, epilogue);
        else RWKV_ROWS(8, 1);
    } else if (NG <= 16) {
        RWKV_ROWS(16, 1);
    } else if (NG <= 32) {
        RWKV_ROWS(16, 2);
    } else {
        RWKV_ROWS(8, 0);
    }
#undef RWKV_ROWS
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "%s: launch failed", who);
    rwkv::counters().sb6_batch.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status launch_batch(BatchArgs a, bool t16, int64_t N, float* y, int64_t OUT, int64_t IN, int64_t out_per,
                         int epilogue, void* workspace, int64_t workspace_bytes, void* stream, const char* who) {
    RWKV_REQUIRE(epilogue >= 0 && epilogue <= 2, RWKV_E_SHAPE, "%s: epilogue %d", who, epilogue);
    BatchPlan p;
    RWKV_REQUIRE(plan_batch(N, OUT, IN, out_per, p), RWKV_E_SHAPE,
                 "%s: N=%lld OUT=%lld IN=%lld out_per=%lld (2 <= N <= 32, IN %% 256 == 0, "
                 "out_per %% 64 == 0 dividing OUT)",
                 who, (long long)N, (long long)OUT, (long long)IN, (long long)out_per);
    RWKV_REQUIRE(OUT * (IN / 32) * 16 < ((int64_t)1 << 40), RWKV_E_SHAPE, "%s: matrix too large", who);
    RWKV_REQUIRE(((uintptr_t)a.x | (uintptr_t)workspace) % 16 == 0 && (uintptr_t)y % 4 == 0, RWKV_E_SHAPE,
                 "%s: x and the workspace must be 16-byte aligned", who);
    RWKV_REQUIRE(workspace_bytes >= p.ws_bytes, RWKV_E_SHAPE, "%s: workspace %lld bytes, needs %lld", who,
                 (long long)workspace_bytes, (long long)p.ws_bytes);
    if (t16 && rows_kernel_taken(N, OUT, IN))
        return launch_rows(a, N, y, OUT, IN, out_per, epilogue, stream, who);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    a.part = (float*)workspace;
    a.N = (int)N;
    a.OUT = (int)OUT;
    a.IN = (int)IN;
    a.out_per = (int)out_per;
    a.KS = p.KS;
    a.NK = p.NK;
    a.NRG = p.NRG;
    a.G = p.G;
    const dim3 grid((unsigned)p.grid()), block(256);
    bool launched = false;
#define RWKV_MB(NTLV, RTV, KWV)                                                                  \
    if (p.NTL == NTLV && p.RT == RTV && p.KW == KWV) {                                           \
        if (t16)                                                                                 \
            rwkv::launch_lds(sb6_t16_gemv_mfma_kernel<NTLV, RTV, KWV>, grid, block, p.lds, st, a); \
        else                                                                                     \
            rwkv::launch_lds(sb6_gemv_mfma_kernel<NTLV, RTV, KWV>, grid, block, p.lds, st, a);     \
        launched = true;                                                                         \
    }
    RWKV_MB(1, 2, 16);
    RWKV_MB(1, 2, 8);
    RWKV_MB(1, 2, 4);
    RWKV_MB(1, 1, 16);
    RWKV_MB(1, 1, 8);
    RWKV_MB(1, 1, 4);
    RWKV_MB(2, 2, 8);
    RWKV_MB(2, 2, 4);
    RWKV_MB(2, 1, 8);
    RWKV_MB(2, 1, 4);
#undef RWKV_MB
    RWKV_REQUIRE(launched, RWKV_E_UNSUPPORTED, "%s: no kernel variant for NTL %d RT %d KW %d", who, p.NTL, p.RT,
                 p.KW);
    const int64_t NO = N * OUT;
    if ((uintptr_t)y % 16 == 0)   // NO % 16 == 0 (OUT % 16 == 0)
        rwkv::launch(sb6_gemv_mfma_reduce_kernel<4>, dim3((unsigned)((NO / 4 + 255) / 256)), dim3(256), st,
                     (const float*)workspace, y, NO, p.KS, epilogue);
    else
        rwkv::launch(sb6_gemv_mfma_reduce_kernel<1>, dim3((unsigned)((NO + 255) / 256)), dim3(256), st,
                     (const float*)workspace, y, NO, p.KS, epilogue);
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "%s: launch failed", who);
    rwkv::counters().sb6_batch.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

}  // namespace

extern "C" {

int rwkv_sb6_gemv_batch_applies(int64_t N, int64_t OUT, int64_t IN, int xbits, int64_t out_per) {
    BatchPlan p;
    return xbits == 0 && plan_batch(N, OUT, IN, out_per, p) ? 1 : 0;
}

int rwkv_sb6_gemv_batch_t16_launches(int64_t N, int64_t OUT, int64_t IN, int64_t out_per) {
    BatchPlan p;
    if (!plan_batch(N, OUT, IN, out_per, p)) return 0;
    return rows_kernel_taken(N, OUT, IN) ? 1 : 2;
}

int64_t rwkv_sb6_gemv_batch_workspace(int64_t N, int64_t OUT, int64_t IN, int64_t out_per) {
    BatchPlan p;
    return plan_batch(N, OUT, IN, out_per, p) ? p.ws_bytes : 0;
}

rwkv_status rwkv_sb6_gemv_batch(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                                const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, int64_t out_per,
                                int epilogue, void* workspace, int64_t workspace_bytes, void* stream) {
    RWKV_REQUIRE(x && qblk && qsqm && ddm && y && workspace, RWKV_E_NULL, "sb6_gemv_batch: null buffer");
    RWKV_REQUIRE(xbits == 0, RWKV_E_UNSUPPORTED, "sb6_gemv_batch: 4-bit codes only (xbits %d)", xbits);
    RWKV_REQUIRE((uintptr_t)qblk % 16 == 0 && (uintptr_t)ddm % 4 == 0 && (uintptr_t)qsqm % 8 == 0, RWKV_E_SHAPE,
                 "sb6_gemv_batch: qblk must be 16-byte aligned, qsqm 8-byte, ddm 4-byte");
    BatchArgs a{x, (const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm, nullptr, nullptr};
    return launch_batch(a, false, N, y, OUT, IN, out_per, epilogue, workspace, workspace_bytes, stream,
                        "sb6_gemv_batch");
}

rwkv_status rwkv_sb6_t16_pack(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t OUT, int64_t IN,
                              uint8_t* tq, uint16_t* ts, uint16_t* tm, void* stream) {
    RWKV_REQUIRE(qblk && qsqm && ddm && tq && ts && tm, RWKV_E_NULL, "sb6_t16_pack: null buffer");
    RWKV_REQUIRE(OUT >= 16 && OUT % 16 == 0 && IN >= 256 && IN % 256 == 0 && OUT * (IN / 32) < INT32_MAX * 256LL,
                 RWKV_E_SHAPE, "sb6_t16_pack: OUT=%lld IN=%lld (OUT %% 16 == 0, IN %% 256 == 0)", (long long)OUT,
                 (long long)IN);
    RWKV_REQUIRE((uintptr_t)qblk % 16 == 0 && (uintptr_t)tq % 16 == 0 && (uintptr_t)qsqm % 2 == 0 &&
                     (uintptr_t)ddm % 4 == 0 && (uintptr_t)ts % 2 == 0 && (uintptr_t)tm % 2 == 0,
                 RWKV_E_SHAPE, "sb6_t16_pack: qblk and tq must be 16-byte aligned, ddm 4-byte");
    const int64_t units = OUT * (IN / 32);
    rwkv::launch(sb6_t16_pack_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256),
                 reinterpret_cast<hipStream_t>(stream), (const uint4*)qblk, (const uint16_t*)qsqm,
                 (const uint32_t*)ddm, OUT, (int)(IN / 32), (uint4*)tq, ts, tm);
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "sb6_t16_pack: launch failed");
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status rwkv_sb6_gemv_batch_t16(const float* x, int64_t N, const uint8_t* tq, const uint16_t* ts,
                                    const uint16_t* tm, float* y, int64_t OUT, int64_t IN, int64_t out_per,
                                    int epilogue, void* workspace, int64_t workspace_bytes, void* stream) {
    RWKV_REQUIRE(x && tq && ts && tm && y && workspace, RWKV_E_NULL, "sb6_gemv_batch_t16: null buffer");
    RWKV_REQUIRE((uintptr_t)tq % 16 == 0 && (uintptr_t)ts % 8 == 0 && (uintptr_t)tm % 16 == 0, RWKV_E_SHAPE,
                 "sb6_gemv_batch_t16: tq and tm must be 16-byte aligned, ts 8-byte");
    BatchArgs a{x, (const uint32_t*)tq, nullptr, nullptr, ts, tm};
    return launch_batch(a, true, N, y, OUT, IN, out_per, epilogue, workspace, workspace_bytes, stream,
                        "sb6_gemv_batch_t16");
}

rwkv_status rwkv_sb6_gemv_batch_t16_rows(const float* x, int64_t N, const uint8_t* tq, const uint16_t* ts,
                                         const uint16_t* tm, float* y, int64_t OUT, int64_t IN, int64_t out_per,
                                         int epilogue, void* stream) {
    RWKV_REQUIRE(x && tq && ts && tm && y, RWKV_E_NULL, "sb6_gemv_batch_t16_rows: null buffer");
    RWKV_REQUIRE((uintptr_t)tq % 16 == 0 && (uintptr_t)ts % 8 == 0 && (uintptr_t)tm % 16 == 0, RWKV_E_SHAPE,
                 "sb6_gemv_batch_t16_rows: tq and tm must be 16-byte aligned, ts 8-byte");
    BatchArgs a{x, (const uint32_t*)tq, nullptr, nullptr, ts, tm};
    return launch_rows(a, N, y, OUT, IN, out_per, epilogue, stream, "sb6_gemv_batch_t16_rows");
}

}  // extern "C"
