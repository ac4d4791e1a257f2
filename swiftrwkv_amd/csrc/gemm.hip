// sb6 projections of a parallel (prefill) pass on the gfx950 matrix cores.
//
// The reference's long pass dequantises the whole matrix to the fp16 base
// type and runs an fp16 matmul, casting the result back to the input type
// (X070Backbone.baseMatmul, Sources/RWKVGen/X070Backbone.swift:337-356,
// 733-739; the dequant of RwkvqDequant.swift:116-140).  Here the dequant
// happens in the GEMM's operand path: no dense weight is written.  Per
// element the numbers are the reference's: the weight is
// fp16(fma(code, half(qs·d), half(qm·dm))) exactly as the dequant kernel
// stores it, the input is rounded to fp16, products accumulate in fp32 on
// v_mfma_f32_16x16x32_f16, and the sum is rounded to fp16 (the fp16 matmul's
// output) before the epilogue.
//
// Tiling.  A workgroup of 4 waves computes a 128 (input rows) × 128 (output
// features) tile in stages of 64 columns (two sb6 32-column units); two
// workgroups share a CU.  The input tile is staged in LDS as fp16
// (double-buffered; rows padded to 144 B so the 16 lanes of a row group read
// distinct banks).  Wave w owns 32 output features — its own weight rows,
// which no other wave of the workgroup reads — and all 128 input rows: 8 × 2
// tiles of 16 × 16 accumulators.  Each lane dequantises the 8 weights that
// are its MFMA B operand (row 16j + (lane & 15), columns 8·(lane >> 4) .. +7
// of a unit) straight from the K3 bytes (low or high nibbles of one 8-byte
// load), so a weight is decoded once per workgroup.  The next stage's input
// and weight bytes are loaded into registers before the current stage's
// products, so one barrier per stage separates LDS reuse.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (lane l, g = l >> 4, i = l & 15):
// A[m = i][k = 8g .. 8g+7], B[k = 8g .. 8g+7][n = i]; D[m = 4g + r][n = i],
// r = 0..3.

#include <hip/hip_runtime.h>

#include "launch.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;            // columns per stage: two sb6 units
constexpr int LDS_ROW = BK + 8;   // halves per staged row (144 B)

__device__ __forceinline__ float f16f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}
__device__ __forceinline__ float hround(float x) { return (float)(_Float16)x; }

struct GemmArgs {
    const void* x;        // inputs [groups][M][lda] (fp32 or fp16)
    int64_t lda, x_gstride;
    const uint8_t* qblk;  // sb6 4-bit K3: [N][IN/32·16]
    const uint8_t* qsqm;  // [N][IN/32·2]
    const uint16_t* ddm;  // [N][IN/256·2]
    void* y;              // [M][ldy]: fp32 (epilogues 0, 1) or fp16 (epilogue 2)
    int64_t ldy;
    int M, N, K, out_per;
};

// One unit's B operand: 8 fp16 weights of one row (`nib`: the 8 bytes whose
// low or high nibbles are this lane's columns), fp16(fma(code, s, m)) as the
// dequant kernel stores it.  A 4-bit code byte read as fp8 E4M3 is code·2^-9
// exactly, so two codes widen per instruction and s carries the 2^9.
__device__ __forceinline__ half8 dequant8(uint2 nib, int shift, uint32_t sm, uint32_t dd) {
    const float s = hround((float)(sm & 0xffu) * f16f(dd)) * 512.0f;
    const float m = hround((float)(int8_t)((sm >> 8) & 0xffu) * f16f(dd >> 16));
    const uint32_t c0 = (nib.x >> shift) & 0x0F0F0F0Fu, c1 = (nib.y >> shift) & 0x0F0F0F0Fu;
    const auto p0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c0, false), p1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c0, true);
    const auto p2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c1, false), p3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c1, true);
    half8 h;
    h[0] = (_Float16)fmaf(p0[0], s, m);
    h[1] = (_Float16)fmaf(p0[1], s, m);
    h[2] = (_Float16)fmaf(p1[0], s, m);
    h[3] = (_Float16)fmaf(p1[1], s, m);
    h[4] = (_Float16)fmaf(p2[0], s, m);
    h[5] = (_Float16)fmaf(p2[1], s, m);
    h[6] = (_Float16)fmaf(p3[0], s, m);
    h[7] = (_Float16)fmaf(p3[1], s, m);
    return h;
}

// A stage's weight bytes for one lane: NT row tiles × 2 units.
template <int NT>
struct BRaw {
    uint2 nib[NT][2];
    uint32_t sm[NT];   // qsqm of units (u, u+1): 2 bytes each
    uint32_t dd[NT];   // ddm of the super-block holding both units
};

// MT × 16 input rows × (4 waves × NT × 16) output features per workgroup.
// A stage's inputs: thread t stages row t / TPR, EPT consecutive columns.
template <typename TA, int EP, int MT, int NT>
__global__ __launch_bounds__(256, 2) void sb6_gemm_kernel(GemmArgs g) {
    constexpr int BM = 16 * MT, BN = 64 * NT;
    constexpr int TPR = 256 / BM;        // staging threads per row
    constexpr int EPT = BK / TPR;        // columns per staging thread
    constexpr int AV = EPT * sizeof(TA) / 16;   // 16-byte loads per staging thread
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM][LDS_ROW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gq = lane >> 4, li = lane & 15;
    // Workgroups are dealt to the 8 XCDs round-robin (id mod 8), each XCD with
    // its own L2: XCD x takes the input row-blocks m ≡ x (mod 8) and sweeps
    // every feature tile of one block before the next, so an input block is
    // fetched into one L2 only.  The grid is padded to whole groups of 8 row
    // blocks; a padding workgroup exits before any barrier.
    const int ntn = g.N / BN;
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    const int tile_n = loc % ntn, tile_m = xcd + 8 * (loc / ntn);
    if (tile_m * BM >= g.M) return;
    const int n0 = tile_n * BN;
    const int m0 = tile_m * BM;
    const int NU = g.K >> 5, NSB = g.K >> 8;
    const int nst = g.K / BK;

    // input rows of this tile come from the matrix group its output features belong to
    const TA* xg = reinterpret_cast<const TA*>(g.x) + (int64_t)(n0 / g.out_per) * g.x_gstride;
    const int srow = threadIdx.x / TPR, scol = (threadIdx.x % TPR) * EPT;
    const TA* xrow = xg + (int64_t)min(m0 + srow, g.M - 1) * g.lda + scol;

    const int nb = n0 + wave * (16 * NT) + li;   // weight row of tile j: nb + 16 j
    const int shift = (gq >> 1) * 4;
    const int nibo = 8 * (gq & 1);

    auto load_a = [&](int st) {
        uint4 a[AV];
        const uint4* p = reinterpret_cast<const uint4*>(xrow + st * BK);
#pragma unroll
        for (int e = 0; e < AV; ++e) a[e] = p[e];
        struct R { uint4 v[AV]; } r;
#pragma unroll
        for (int e = 0; e < AV; ++e) r.v[e] = a[e];
        return r;
    };
    auto store_a = [&](int buf, const auto& a) {
        _Float16* d = &As[buf][srow][scol];
        if constexpr (sizeof(TA) == 4) {
#pragma unroll
            for (int e = 0; e < AV / 2; ++e) {
                const uint4 p = a.v[2 * e], q = a.v[2 * e + 1];
                half8 h;
                h[0] = (_Float16)__uint_as_float(p.x); h[1] = (_Float16)__uint_as_float(p.y);
                h[2] = (_Float16)__uint_as_float(p.z); h[3] = (_Float16)__uint_as_float(p.w);
                h[4] = (_Float16)__uint_as_float(q.x); h[5] = (_Float16)__uint_as_float(q.y);
                h[6] = (_Float16)__uint_as_float(q.z); h[7] = (_Float16)__uint_as_float(q.w);
                *reinterpret_cast<half8*>(d + 8 * e) = h;
            }
        } else {
#pragma unroll
            for (int e = 0; e < AV; ++e) *reinterpret_cast<uint4*>(d + 8 * e) = a.v[e];
        }
    };
    auto load_b = [&](int st) {
        BRaw<NT> b;
        const int u = st * 2;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int64_t row = nb + 16 * j;
            const uint8_t* q = g.qblk + (row * NU + u) * 16 + nibo;
            b.nib[j][0] = *reinterpret_cast<const uint2*>(q);
            b.nib[j][1] = *reinterpret_cast<const uint2*>(q + 16);
            b.sm[j] = *reinterpret_cast<const uint32_t*>(g.qsqm + (row * NU + u) * 2);
            b.dd[j] = *reinterpret_cast<const uint32_t*>(g.ddm + (row * NSB + (u >> 3)) * 2);
        }
        return b;
    };
    auto dequant = [&](const BRaw<NT>& b, int q, half8* bop) {
#pragma unroll
        for (int j = 0; j < NT; ++j) bop[j] = dequant8(b.nib[j][q], shift, b.sm[j] >> (16 * q), b.dd[j]);
    };
    // MT × NT MFMAs of unit q of the staged buffer
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto products = [&](int buf, int q, const half8* bop) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const half8 aop = *reinterpret_cast<const half8*>(&As[buf][16 * i + li][32 * q + 8 * gq]);
#pragma unroll
            for (int j = 0; j < NT; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[j], acc[i][j], 0, 0, 0);
        }
    };

    auto ar = load_a(0);
    BRaw<NT> bcur = load_b(0);
    store_a(0, ar);
    half8 b0[NT], b1[NT];
    dequant(bcur, 0, b0);
    __syncthreads();

    // Per stage: the next stage's bytes are requested first; unit 0's
    // products run while unit 1 is decoded, unit 1's while the next stage's
    // unit 0 is (one MFMA, one VALU instruction, alternately).
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        const bool more = st + 1 < nst;
        BRaw<NT> bnxt = bcur;
        if (more) {
            ar = load_a(st + 1);
            bnxt = load_b(st + 1);
        }
        dequant(bcur, 1, b1);
        products(buf, 0, b0);
#pragma unroll
        for (int k = 0; k < MT * NT; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);   // one VALU
        }
        if (more) dequant(bnxt, 0, b0);
        products(buf, 1, b1);
#pragma unroll
        for (int k = 0; k < MT * NT; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
        }
        if (more) store_a(buf ^ 1, ar);
        bcur = bnxt;
        __syncthreads();
    }

    // epilogue: fp16 rounding of the product, then store / add / relu² (fp16)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + 16 * i + 4 * gq + r;
            if (row >= g.M) continue;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int64_t col = nb + 16 * j;
                const float v = hround(acc[i][j][r]);
                if constexpr (EP == 0) {
                    reinterpret_cast<float*>(g.y)[(int64_t)row * g.ldy + col] = v;
                } else if constexpr (EP == 1) {
                    float* p = reinterpret_cast<float*>(g.y) + (int64_t)row * g.ldy + col;
                    *p = *p + v;
                } else {
                    const float rl = fmaxf(v, 0.0f);
                    reinterpret_cast<_Float16*>(g.y)[(int64_t)row * g.ldy + col] = (_Float16)(rl * rl);
                }
            }
        }
    }
}

// One tile shape: 128 × 128 with two workgroups per CU measured fastest
// (larger tiles cost occupancy: at one wave per SIMD the stage's loads are
// not hidden).
template <typename TA, int EP>
void launch_gemm(const GemmArgs& g, hipStream_t s) {
    const int64_t blocks = (int64_t)((g.M + 8 * 128 - 1) / (8 * 128)) * 8 * (g.N / 128);
    rwkv::launch(sb6_gemm_kernel<TA, EP, 8, 2>, dim3((unsigned)blocks), dim3(256), s, g);
}

}  // namespace

extern "C" {

int rwkv_sb6_gemm_applies(int64_t OUT, int64_t IN, int xbits, int64_t out_per) {
    return xbits == 0 && OUT >= 128 && OUT % 128 == 0 && IN >= 256 && IN % 256 == 0 && out_per >= 128 &&
           out_per % 128 == 0 && OUT % out_per == 0 && OUT <= ((int64_t)1 << 30) && IN <= ((int64_t)1 << 24);
}

rwkv_status rwkv_sb6_gemm(const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda, int64_t x_group_stride,
                          const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, void* y, int64_t ldy,
                          int64_t OUT, int64_t IN, int xbits, int64_t out_per, int epilogue, void* stream) {
    RWKV_REQUIRE(x && qblk && qsqm && ddm && y, RWKV_E_NULL, "sb6_gemm: null buffer");
    RWKV_REQUIRE(x_dt == RWKV_F32 || x_dt == RWKV_F16, RWKV_E_DTYPE, "sb6_gemm: inputs must be f32 or f16");
    RWKV_REQUIRE(epilogue >= 0 && epilogue <= 2, RWKV_E_SHAPE, "sb6_gemm: epilogue %d", epilogue);
    RWKV_REQUIRE(rwkv_sb6_gemm_applies(OUT, IN, xbits, out_per), RWKV_E_UNSUPPORTED,
                 "sb6_gemm: 4-bit sb6 with OUT (%lld) and out_per (%lld) multiples of 128 and IN (%lld) of 256",
                 (long long)OUT, (long long)out_per, (long long)IN);
    RWKV_REQUIRE(M >= 1 && M <= ((int64_t)1 << 24), RWKV_E_SHAPE, "sb6_gemm: M (%lld) out of range", (long long)M);
    const int64_t groups = OUT / out_per;
    const int64_t xes = x_dt == RWKV_F32 ? 4 : 2;
    RWKV_REQUIRE(lda >= IN && lda % 8 == 0 && (groups == 1 || x_group_stride >= M * lda), RWKV_E_SHAPE,
                 "sb6_gemm: lda (%lld) must be >= IN and a multiple of 8; groups need x_group_stride >= M·lda",
                 (long long)lda);
    RWKV_REQUIRE(ldy >= OUT && (epilogue == 2 ? ldy % 2 == 0 : true), RWKV_E_SHAPE, "sb6_gemm: ldy (%lld) < OUT",
                 (long long)ldy);
    RWKV_REQUIRE((reinterpret_cast<uintptr_t>(x) % 16) == 0 && (x_group_stride * xes) % 16 == 0, RWKV_E_SHAPE,
                 "sb6_gemm: inputs must be 16-byte aligned");
    GemmArgs g{x, lda, x_group_stride, qblk, qsqm, ddm, y, ldy, (int)M, (int)OUT, (int)IN, (int)out_per};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool f16 = x_dt == RWKV_F16;
    switch (epilogue) {
        case 0: f16 ? launch_gemm<_Float16, 0>(g, s) : launch_gemm<float, 0>(g, s); break;
        case 1: f16 ? launch_gemm<_Float16, 1>(g, s) : launch_gemm<float, 1>(g, s); break;
        default: f16 ? launch_gemm<_Float16, 2>(g, s) : launch_gemm<float, 2>(g, s); break;
    }
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "sb6_gemm: launch failed");
    rwkv::counters().sb6_gemm.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"
