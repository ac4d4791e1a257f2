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
    float* part;         // [KS, N, OUT]
    int N, OUT, IN, out_per, KW, KS, NRG;
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

template <int NTL, int RT, int KW>
__global__ __launch_bounds__(256) void sb6_gemv_mfma_kernel(BatchArgs A) {
    constexpr int NI = 16 * NTL;   // inputs of the launch, padded to whole tiles
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // Xp[uu][t][part][lane]: 16 bytes = the lane's eight bf16 slots;  Xs[uu][n]: unit sums
    uint4* Xp = reinterpret_cast<uint4*>(smem);
    float* Xs = reinterpret_cast<float*>(smem + (size_t)KW * NTL * 3 * 64 * 16);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, i = lane & 15;
    // Workgroups are dealt to the 8 XCDs round-robin (id mod 8).  The K
    // slices of a row group get consecutive ids of one XCD, so the workgroups
    // that read a row's slices run side by side on one L2 (whole rows come
    // from HBM together); the grid is padded to groups of 8 row groups.
    const int xcd = (int)blockIdx.x & 7, loc = (int)blockIdx.x >> 3;
    const int ks = loc % A.KS, rg = (loc / A.KS) * 8 + xcd;
    if (rg >= A.NRG) return;
    const int row0 = rg * 64 * RT;
    const int NU = A.IN >> 5, NSB = NU >> 3, NK = A.OUT / A.out_per;
    const int xi = row0 / A.out_per;   // the input row every row of this workgroup reads
    const int u0 = ks * KW;
    const int nu = min(KW, NU - u0);

    // Issue order: the slice's inputs (L2 hits), then the weights of the
    // wave's rows (HBM).  Loads complete in issue order, so the staging below
    // waits only for the inputs, and each group of four units is transposed
    // and multiplied as soon as its own weights are in.
    constexpr int JOBS = 4;   // staging jobs per thread: KW·NI·4 ≤ 1024
    float4 xa[JOBS], xb[JOBS];
#pragma unroll
    for (int k = 0; k < JOBS; ++k) {
        const int job = tid + 256 * k;
        const int n = job % NI, gg = (job / NI) & 3, uu = job / (NI * 4);
        xa[k] = xb[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (uu < nu && n < A.N) {
            const float* src = A.x + ((int64_t)n * NK + xi) * A.IN + (u0 + uu) * 32;
            xa[k] = *reinterpret_cast<const float4*>(src + 4 * gg);
            xb[k] = *reinterpret_cast<const float4*>(src + 16 + 4 * gg);
        }
    }
    // lane g of row i loads whole units 4q + g (16 bytes each) and the row's
    // scales; a 4×4 transpose across the four 16-lane rows later leaves lane
    // g with dword g of every unit, the k slots its B operand needs
    int rows[RT];
    const uint4* qr[RT];
    const uint2* sr[RT];
    uint32_t cw[RT][KW], smv[RT][KW / 2], ddv[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        rows[rt] = row0 + (wave * RT + rt) * 16 + i;
        const int64_t row = min(rows[rt], A.OUT - 1);
        qr[rt] = reinterpret_cast<const uint4*>(A.q) + row * NU + u0;
        sr[rt] = reinterpret_cast<const uint2*>(A.sm + row * NU + u0);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) ddv[rt][sb] = A.dd[row * NSB + min((u0 >> 3) + sb, NSB - 1)];
    }
    // unit groups in the order they are used, every row tile's share of a
    // group together
#pragma unroll
    for (int q = 0; q < KW / 4; ++q) {
        if (4 * q < nu) {   // nu is a multiple of 4: uniform
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint2 sv = sr[rt][q];
                smv[rt][2 * q] = sv.x; smv[rt][2 * q + 1] = sv.y;
                const uint4 w = qr[rt][4 * q + g];
                cw[rt][4 * q] = w.x; cw[rt][4 * q + 1] = w.y; cw[rt][4 * q + 2] = w.z; cw[rt][4 * q + 3] = w.w;
            }
        }
    }

    // the slice's inputs: bf16 parts in A-operand order, and per-lane-slot
    // partial sums Xq[uu][gg][n] (the first and the second 16 columns) that
    // the sum pass below adds up
    float2* Xq = reinterpret_cast<float2*>(Xs + KW * NI);
#pragma unroll
    for (int k = 0; k < JOBS; ++k) {
        const int job = tid + 256 * k;
        const int n = job % NI, gg = (job / NI) & 3, uu = job / (NI * 4);
        if (uu >= nu) continue;   // (a guard, not a loop exit: the loops stay fully unrolled)
        const float4 a = xa[k], b = xb[k];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        bf16x8 p1, p2, p3;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const __bf16 h1 = (__bf16)v[j];
            const float r1 = v[j] - (float)h1;
            const __bf16 h2 = (__bf16)r1;
            p1[j] = h1;
            p2[j] = h2;
            p3[j] = (__bf16)(r1 - (float)h2);
        }
        uint4* dst = Xp + ((uu * NTL + (n >> 4)) * 3) * 64 + gg * 16 + (n & 15);
        dst[0] = __builtin_bit_cast(uint4, p1);
        dst[64] = __builtin_bit_cast(uint4, p2);
        dst[128] = __builtin_bit_cast(uint4, p3);
        Xq[(uu * 4 + gg) * NI + n] = make_float2(a.x + a.y + a.z + a.w, b.x + b.y + b.z + b.w);
    }
    __syncthreads();
    for (int job = tid; job < nu * NI; job += 256) {
        const int n = job % NI, uu = job / NI;
        float h0 = 0.0f, h1 = 0.0f;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            const float2 q = Xq[(uu * 4 + gg) * NI + n];
            h0 += q.x;
            h1 += q.y;
        }
        Xs[uu * NI + n] = h0 + h1;
    }
    __syncthreads();

    float dsc[RT][2], dmc[RT][2];   // the super-block scales d, dm
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            dsc[rt][sb] = f16f(ddv[rt][sb]);
            dmc[rt][sb] = f16f(ddv[rt][sb] >> 16);
        }
    f32x4 acc[RT][NTL];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < NTL; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int uu = 0; uu < KW; ++uu) {
        // nu < KW only in a row's last, partial slice; a guard rather than a
        // loop exit keeps the loop unrolled, so the per-unit registers are
        // addressed by constants (an exit left it rolled, with every cw / smv
        // access an indexed register move)
        if (uu >= nu) continue;   // uniform
        if (uu % 4 == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) transpose4(cw[rt][uu], cw[rt][uu + 1], cw[rt][uu + 2], cw[rt][uu + 3]);
        }
        bf16x8 ap[NTL][3];
        float4 xs[NTL];
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
#pragma unroll
            for (int p = 0; p < 3; ++p) ap[t][p] = __builtin_bit_cast(bf16x8, Xp[((uu * NTL + t) * 3 + p) * 64 + lane]);
            xs[t] = *reinterpret_cast<const float4*>(Xs + uu * NI + t * 16 + 4 * g);
        }
        const int sb = uu >> 3;   // u0 is a multiple of KW ∈ {4, 8, 16}
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const bf16x8 bc = codes_bf16(cw[rt][uu]);
            const uint32_t smr = (smv[rt][uu >> 1] >> (16 * (uu & 1))) & 0xffffu;
            const float s = hround((float)(smr & 0xffu) * dsc[rt][sb]);
            const float m = hround((float)(int8_t)(smr >> 8) * dmc[rt][sb]);
#pragma unroll
            for (int t = 0; t < NTL; ++t) {
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[t][0], bc, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[t][1], bc, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[t][2], bc, d, 0, 0, 0);
                const float xsv[4] = {xs[t].x, xs[t].y, xs[t].z, xs[t].w};
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[rt][t][r] = fmaf(m, xsv[r], fmaf(s, d[r], acc[rt][t][r]));
            }
        }
    }

    // partials of this K slice: lane holds inputs 4g..4g+3 (+16t) of its row
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (rows[rt] >= A.OUT) continue;
#pragma unroll
        for (int t = 0; t < NTL; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = t * 16 + 4 * g + r;
                if (n < A.N) A.part[((int64_t)ks * A.N + n) * A.OUT + rows[rt]] = acc[rt][t][r];
            }
    }
}

// y[n, row] = epilogue(Σ_ks part[ks, n, row]), slices in order.
__global__ __launch_bounds__(256) void sb6_gemv_mfma_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                                   int64_t NO, int KS, int ep) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= NO) return;
    // eight slices in flight at a time, summed in slice order
    float t = 0.0f;
    for (int k0 = 0; k0 < KS; k0 += 8) {
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = k0 + k < KS ? part[(int64_t)(k0 + k) * NO + e] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k0 + k < KS) t = (k0 + k == 0) ? p[k] : t + p[k];
    }
    if (ep == 1) {
        t = y[e] + t;
    } else if (ep == 2) {
        t = fmaxf(t, 0.0f);
        t = t * t;
    }
    y[e] = t;
}

struct BatchPlan {
    int NTL, RT, KW, KS, NRG;
    size_t lds;
    int64_t ws_bytes;
};

// Tiles of 32 rows per wave (16 for fused matrices whose groups would
// straddle two matrices) and K slices of 16 (8 for 17-32 inputs) units, halved
// until the grid holds ≥ 512 workgroups (the inputs are staged once per
// workgroup, so wider slices and taller groups read them fewer times; measured
// at 7B-class shapes × 16: 4096x4096 15.5 → 12.6 µs against the earlier
// 1024, the larger matrices within 2 %).
bool plan_batch(int64_t N, int64_t OUT, int64_t IN, int64_t out_per, BatchPlan& p) {
    if (N < 2 || N > 32 || OUT < 16 || OUT % 16 || IN < 256 || IN % 256 || out_per < 64 || out_per % 64 ||
        OUT % out_per)
        return false;
    p.NTL = N <= 16 ? 1 : 2;
    p.RT = out_per % 128 == 0 ? 2 : 1;
    const int64_t NU = IN / 32;
    auto grid = [&](int RT, int KW) {
        const int64_t nrg = (OUT + 64 * RT - 1) / (64 * RT), ks = (NU + KW - 1) / KW;
        return nrg * ks;
    };
    p.KW = p.NTL == 1 ? KW_MAX : KW_MAX / 2;   // ≤ 49 KiB of LDS: two or three workgroups per CU
    while (p.KW > 4 && grid(p.RT, p.KW) < 512) p.KW >>= 1;
    if (p.RT == 2 && grid(p.RT, p.KW) < 256) p.RT = 1;
    p.NRG = (int)((OUT + 64 * p.RT - 1) / (64 * p.RT));
    p.KS = (int)((NU + p.KW - 1) / p.KW);
    p.lds = (size_t)p.KW * p.NTL * 3 * 64 * 16 + (size_t)p.KW * 16 * p.NTL * 4 * (1 + 4 * 2);
    p.ws_bytes = (int64_t)p.KS * N * OUT * 4;
    return p.KS <= KS_MAX && (int64_t)(p.NRG + 7) / 8 * 8 * p.KS <= INT32_MAX;
}

}  // namespace

extern "C" {

int rwkv_sb6_gemv_batch_applies(int64_t N, int64_t OUT, int64_t IN, int xbits, int64_t out_per) {
    BatchPlan p;
    return xbits == 0 && plan_batch(N, OUT, IN, out_per, p) ? 1 : 0;
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
    RWKV_REQUIRE(epilogue >= 0 && epilogue <= 2, RWKV_E_SHAPE, "sb6_gemv_batch: epilogue %d", epilogue);
    BatchPlan p;
    RWKV_REQUIRE(plan_batch(N, OUT, IN, out_per, p), RWKV_E_SHAPE,
                 "sb6_gemv_batch: N=%lld OUT=%lld IN=%lld out_per=%lld (2 <= N <= 32, IN %% 256 == 0, "
                 "out_per %% 64 == 0 dividing OUT)",
                 (long long)N, (long long)OUT, (long long)IN, (long long)out_per);
    RWKV_REQUIRE(OUT * (IN / 32) * 16 < ((int64_t)1 << 40), RWKV_E_SHAPE, "sb6_gemv_batch: matrix too large");
    const uintptr_t al = (uintptr_t)x | (uintptr_t)qblk | (uintptr_t)workspace;
    RWKV_REQUIRE(al % 16 == 0 && (uintptr_t)ddm % 4 == 0 && (uintptr_t)qsqm % 8 == 0 && (uintptr_t)y % 4 == 0,
                 RWKV_E_SHAPE, "sb6_gemv_batch: x, qblk and the workspace must be 16-byte aligned, qsqm 8-byte");
    RWKV_REQUIRE(workspace_bytes >= p.ws_bytes, RWKV_E_SHAPE, "sb6_gemv_batch: workspace %lld bytes, needs %lld",
                 (long long)workspace_bytes, (long long)p.ws_bytes);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    BatchArgs a{x, (const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm, (float*)workspace,
                (int)N, (int)OUT, (int)IN, (int)out_per, p.KW, p.KS, p.NRG};
    const dim3 grid((unsigned)((p.NRG + 7) / 8 * 8 * p.KS)), block(256);
    bool launched = false;
#define RWKV_MB(NTLV, RTV, KWV)                                                        \
    if (p.NTL == NTLV && p.RT == RTV && p.KW == KWV) {                                 \
        rwkv::launch_lds(sb6_gemv_mfma_kernel<NTLV, RTV, KWV>, grid, block, p.lds, st, a); \
        launched = true;                                                               \
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
    RWKV_REQUIRE(launched, RWKV_E_UNSUPPORTED, "sb6_gemv_batch: no kernel variant for NTL %d RT %d KW %d", p.NTL, p.RT,
                 p.KW);
    const int64_t NO = N * OUT;
    rwkv::launch(sb6_gemv_mfma_reduce_kernel, dim3((unsigned)((NO + 255) / 256)), dim3(256), st,
                 (const float*)workspace, y, NO, p.KS, epilogue);
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "sb6_gemv_batch: launch failed");
    rwkv::counters().sb6_batch.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"
