// Quantised projections of a parallel (prefill) pass on the gfx950 matrix
// cores: sb6 (4, 5 or 6-bit codes) and sym (8 or 6-bit codes).
//
// The reference's long pass dequantises the whole matrix to the fp16 base
// type and runs an fp16 matmul, casting the result back to the input type
// (X070Backbone.baseMatmul, Sources/RWKVGen/X070Backbone.swift:337-356,
// 733-739; the dequant of RwkvqDequant.swift:116-140 (sb6) and :350-388,
// 442-466 (sym, whose fp16 branch computes in half)).  Here the dequant
// happens in the GEMM's operand path (quant_gemm_kernel: no dense weight is
// written), or, for shapes with many output tiles, once per matrix into a
// workspace that dense_gemm_kernel then multiplies (below).  Per
// element the numbers are the reference's: the weight is exactly what the
// dequant kernels store in fp16 — sb6 fp16(fma(code, half(qs·d), half(qm·dm))),
// sym fp16((code − bias)·half(qs·d)) — the input is rounded to fp16, products
// accumulate in fp32 on v_mfma_f32_16x16x32_f16, and the sum is rounded to
// fp16 (the fp16 matmul's output) before the epilogue.
//
// Tiling.  A workgroup of 4 waves computes a 128 (input rows) × 128 (output
// features) tile in stages of 64 columns (two 32-column units); two
// workgroups share a CU.  The input tile is staged in LDS as fp16
// (double-buffered; rows padded to 144 B so the 16 lanes of a row group read
// distinct banks).  Wave w owns 32 output features — its own weight rows,
// which no other wave of the workgroup reads — and all 128 input rows: 8 × 2
// tiles of 16 × 16 accumulators.  Each lane dequantises the 8 weights that
// are its MFMA B operand (row 16j + (lane & 15), columns 8·(lane >> 4) .. +7
// of a unit) straight from the packed bytes, so a weight is decoded once per
// workgroup.  The next stage's input and weight bytes are loaded into
// registers before the current stage's products, so one barrier per stage
// separates LDS reuse.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (lane l, g = l >> 4, i = l & 15):
// A[m = i][k = 8g .. 8g+7], B[k = 8g .. 8g+7][n = i]; D[m = 4g + r][n = i],
// r = 0..3.

#include <hip/hip_runtime.h>

#include <algorithm>

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
    const uint8_t* q;     // codes: sb6 K3 qblk [N][IN/32·(16+4·xbits)], sym qblk (interleaved)
    const uint8_t* s1;    // sb6 qsqm [N][IN/32·2] / sym qs [N][IN/16]
    const uint16_t* s2;   // sb6 ddm [N][IN/256·2] / sym d [N][IN/256]
    void* y;              // [M][ldy]: fp32 (epilogues 0, 1) or fp16 (epilogue 2)
    int64_t ldy;
    int M, N, K, out_per;
    float* part;          // splits > 1: the fp32 partial sums [splits][M][N]
    int splits;           // K ranges the tile's stages are divided into
};

// The epilogue of one output: fp16 rounding of the fp32 sum (the fp16
// matmul's output), then store (fp32), add into y (fp32) or relu² (fp16).
template <int EP>
__device__ __forceinline__ void store_out(void* y, int64_t idx, float acc) {
    const float v = hround(acc);
    if constexpr (EP == 0) {
        reinterpret_cast<float*>(y)[idx] = v;
    } else if constexpr (EP == 1) {
        float* p = reinterpret_cast<float*>(y) + idx;
        *p = *p + v;
    } else {
        const float rl = fmaxf(v, 0.0f);
        reinterpret_cast<_Float16*>(y)[idx] = (_Float16)(rl * rl);
    }
}

// 4 bits → the low bit of 4 bytes (RwkvqSb6GEMV.swift:58-67 multiply spread).
__device__ __forceinline__ uint32_t spread4(uint32_t nib) { return (nib * 0x00204081u) & 0x01010101u; }

// Byte E of w as a float (v_cvt_f32_ubyteE).
template <int E>
__device__ __forceinline__ float ubyte(uint32_t w) {
    return (float)((w >> (8 * E)) & 0xffu);
}

// Eight code bytes (c0: columns 0..3, c1: 4..7 of the lane's 8) as
// fp16(fma(code, s, m)): the product and the sum are exact in fp32 for every
// format here, so the one rounding is the fp16 one.
__device__ __forceinline__ half8 bytes8_fma(uint32_t c0, uint32_t c1, float s, float m) {
    half8 h;
    h[0] = (_Float16)fmaf(ubyte<0>(c0), s, m);
    h[1] = (_Float16)fmaf(ubyte<1>(c0), s, m);
    h[2] = (_Float16)fmaf(ubyte<2>(c0), s, m);
    h[3] = (_Float16)fmaf(ubyte<3>(c0), s, m);
    h[4] = (_Float16)fmaf(ubyte<0>(c1), s, m);
    h[5] = (_Float16)fmaf(ubyte<1>(c1), s, m);
    h[6] = (_Float16)fmaf(ubyte<2>(c1), s, m);
    h[7] = (_Float16)fmaf(ubyte<3>(c1), s, m);
    return h;
}

// Weight formats.  A lane (row `row`, column group gq of 8) loads the bytes
// of its 8 columns of the stage's two units u, u + 1 (Raw) and decodes unit
// q ∈ {0, 1} into its B operand.
//
// sb6 (gs 32, super-block 8 units): unit = 16 B of nibbles (byte c: column c
// low, c + 16 high) ‖ 4 B qh ‖ 4 B qh2 (bit c: bit 4 / 5 of column c) for
// 4 + XB bit codes; qsqm (qs, qm − 31) per unit; ddm (d, dm) fp16 per
// super-block (the K3 layout, RwkvqFile.swift:189-212).
template <int XB>
struct Sb6W {
    static constexpr int UB = 16 + 4 * XB;
    struct Raw {
        uint2 nib[2];
        uint32_t hi[2][XB > 0 ? XB : 1];
        uint32_t sm;   // qsqm of units u, u + 1
        uint32_t dd;   // ddm of their super-block
    };
    __device__ static Raw load(const GemmArgs& g, int64_t row, int u, int gq) {
        const int NU = g.K >> 5, NSB = g.K >> 8;
        Raw r;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint8_t* b = g.q + (row * NU + u + q) * UB;
            // 4-byte aligned only for a 20-byte unit: two dword loads
            const uint32_t* w = reinterpret_cast<const uint32_t*>(b + 8 * (gq & 1));
            r.nib[q] = make_uint2(w[0], w[1]);
#pragma unroll
            for (int e = 0; e < XB; ++e) r.hi[q][e] = *reinterpret_cast<const uint32_t*>(b + 16 + 4 * e);
        }
        r.sm = *reinterpret_cast<const uint32_t*>(g.s1 + (row * NU + u) * 2);
        r.dd = *reinterpret_cast<const uint32_t*>(g.s2 + (row * NSB + (u >> 3)) * 2);
        return r;
    }
    __device__ static half8 dequant(const Raw& r, int q, int gq) {
        const uint32_t sm = r.sm >> (16 * q);
        const int shift = (gq >> 1) * 4;   // columns 16..31 in the high nibbles
        const uint32_t c0 = (r.nib[q].x >> shift) & 0x0F0F0F0Fu, c1 = (r.nib[q].y >> shift) & 0x0F0F0F0Fu;
        const float m = hround((float)(int8_t)((sm >> 8) & 0xffu) * f16f(r.dd >> 16));
        if constexpr (XB == 0) {
            // a 4-bit code byte read as fp8 E4M3 is code·2^-9 exactly: two
            // codes widen per instruction and s carries the 2^9
            const float s = hround((float)(sm & 0xffu) * f16f(r.dd)) * 512.0f;
            const auto p0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c0, false);
            const auto p1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c0, true);
            const auto p2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c1, false);
            const auto p3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)c1, true);
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
        } else {
            const float s = hround((float)(sm & 0xffu) * f16f(r.dd));
            uint32_t a = c0, b = c1;
#pragma unroll
            for (int e = 0; e < XB; ++e) {
                const uint32_t h8 = (r.hi[q][e] >> (8 * gq)) & 0xffu;   // bits of columns 8gq .. 8gq+7
                a |= spread4(h8 & 0xFu) << (4 + e);
                b |= spread4(h8 >> 4) << (4 + e);
            }
            return bytes8_fma(a, b, s, m);
        }
    }
};

// sym (gs = super-block = 16 columns, RwkvqFile.swift:437-449 interleave):
// 8-bit: 32 int8 codes per unit (byte c = column c); 6-bit: 24 B per unit —
// words 0..3 nibbles (register order l0, l1, h0, h1 | l2, l3, h2, h3: word
// 2·(c / 16) + (c / 4) % 2, low nibbles for c % 8 < 4), word 4 qh, word 5 qh2,
// codes stored + 32.  qs int8 per 16 columns, d fp16 per 256 columns;
// w = (code − bias)·half(qs·d).
template <int BITS>
struct SymW {
    static constexpr int UB = BITS == 8 ? 32 : 24;
    struct Raw {
        uint2 c[2];
        uint32_t hi[2][BITS == 8 ? 1 : 2];
        uint32_t qs;   // the four 16-column scales of units u, u + 1
        uint32_t d;    // super-block scale (fp16)
    };
    __device__ static Raw load(const GemmArgs& g, int64_t row, int u, int gq) {
        const int NU = g.K >> 5, NSB = g.K >> 8;
        Raw r;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint8_t* b = g.q + (row * NU + u + q) * UB;
            if constexpr (BITS == 8) {
                r.c[q] = *reinterpret_cast<const uint2*>(b + 8 * gq);
            } else {
                r.c[q] = *reinterpret_cast<const uint2*>(b + 8 * (gq >> 1));
                r.hi[q][0] = *reinterpret_cast<const uint32_t*>(b + 16);
                r.hi[q][1] = *reinterpret_cast<const uint32_t*>(b + 20);
            }
        }
        r.qs = *reinterpret_cast<const uint32_t*>(g.s1 + row * (g.K >> 4) + 2 * u);
        r.d = g.s2[row * NSB + (u >> 3)];
        return r;
    }
    __device__ static half8 dequant(const Raw& r, int q, int gq) {
        const float s = hround((float)(int8_t)((r.qs >> (8 * (2 * q + (gq >> 1)))) & 0xffu) * f16f(r.d));
        if constexpr (BITS == 8) {
            // int8 codes as unsigned bytes code + 128: (u − 128)·s exactly
            return bytes8_fma(r.c[q].x ^ 0x80808080u, r.c[q].y ^ 0x80808080u, s, -128.0f * s);
        } else {
            const int shift = (gq & 1) * 4;
            uint32_t a = (r.c[q].x >> shift) & 0x0F0F0F0Fu, b = (r.c[q].y >> shift) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t h8 = (r.hi[q][e] >> (8 * gq)) & 0xffu;
                a |= spread4(h8 & 0xFu) << (4 + e);
                b |= spread4(h8 >> 4) << (4 + e);
            }
            return bytes8_fma(a, b, s, -32.0f * s);
        }
    }
};

// MT × 16 input rows × (4 waves × NT × 16) output features per workgroup.
// A stage's inputs: thread t stages row t / TPR, EPT consecutive columns.
template <class F, typename TA, int EP, int MT, int NT>
__global__ __launch_bounds__(256, 2) void quant_gemm_kernel(GemmArgs g) {
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
    const int ntn = g.N / BN, S = g.splits;
    const int total = ((g.M + BM - 1) / BM) * ntn * S;
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    const int t = xcd * (total >> 3) + min(xcd, total & 7) + loc;   // the tile's place in (m, n, split) order
    const int kz = t % S, tile_n = (t / S) % ntn, tile_m = t / (S * ntn);
    const int n0 = tile_n * BN;
    const int m0 = tile_m * BM;
    const int nst = g.K / BK;
    const int st0 = (int)((int64_t)kz * nst / S), st1 = (int)((int64_t)(kz + 1) * nst / S);

    // input rows of this tile come from the matrix group its output features belong to
    const TA* xg = reinterpret_cast<const TA*>(g.x) + (int64_t)(n0 / g.out_per) * g.x_gstride;
    const int srow = threadIdx.x / TPR, scol = (threadIdx.x % TPR) * EPT;
    const TA* xrow = xg + (int64_t)min(m0 + srow, g.M - 1) * g.lda + scol;

    const int nb = n0 + wave * (16 * NT) + li;   // weight row of tile j: nb + 16 j

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
    using Raw = typename F::Raw;
    struct BRaw {
        Raw t[NT];
    };
    auto load_b = [&](int st) {
        BRaw b;
#pragma unroll
        for (int j = 0; j < NT; ++j) b.t[j] = F::load(g, nb + 16 * j, st * 2, gq);
        return b;
    };
    auto dequant = [&](const BRaw& b, int q, half8* bop) {
#pragma unroll
        for (int j = 0; j < NT; ++j) bop[j] = F::dequant(b.t[j], q, gq);
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

    auto ar = load_a(st0);
    BRaw bcur = load_b(st0);
    store_a(0, ar);
    half8 b0[NT], b1[NT];
    dequant(bcur, 0, b0);
    __syncthreads();

    // Per stage: the next stage's bytes are requested first; unit 0's
    // products run while unit 1 is decoded, unit 1's while the next stage's
    // unit 0 is (one MFMA, one VALU instruction, alternately).
    for (int st = st0; st < st1; ++st) {
        const int buf = (st - st0) & 1;
        const bool more = st + 1 < st1;
        BRaw bnxt = bcur;
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

    if (S > 1) {   // this K range's fp32 sums; gemm_split_reduce adds the ranges and applies the epilogue
        float* part = g.part + (int64_t)kz * g.M * g.N;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + 16 * i + 4 * gq + r;
                if (row >= g.M) continue;
#pragma unroll
                for (int j = 0; j < NT; ++j) part[(int64_t)row * g.N + nb + 16 * j] = acc[i][j][r];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + 16 * i + 4 * gq + r;
            if (row >= g.M) continue;
#pragma unroll
            for (int j = 0; j < NT; ++j) store_out<EP>(g.y, (int64_t)row * g.ldy + nb + 16 * j, acc[i][j][r]);
        }
    }
}

// ── dense fp16 weights ──
//
// y = epilogue(fp16(x · wᵀ)) for x [groups][M][lda] fp16 and w [N][K] fp16
// (rows K-contiguous): the long pass once the weight is fp16 — a dense fp16
// base, or a quantised one dequantised into a workspace (the quantised entry
// points do that for shapes with many output tiles: one dequant per matrix
// costs 10-35 µs against milliseconds of products at M ≥ 4096).
//
// A workgroup of 8 waves computes a 256 (input rows) × 256 (output features)
// tile in stages of 64 columns.  Both operands are staged in LDS as rows of
// 128 B whose 16-byte chunk c is stored at chunk c ^ (row & 7): the 8 lanes
// reading one chunk column of 8 consecutive rows (an MFMA operand) or
// writing 8 chunks of one row hit distinct banks.  Wave w takes input rows
// 128·(w & 1) .. +127 and features 64·(w >> 1) .. +63: 8 × 4 accumulator
// tiles of 16 × 16, 32 MFMAs per 32-column unit against 12 LDS operand reads
// (the fused kernel's waves: 16 MFMAs against 8).  Each thread moves 8
// chunks a stage (4 input rows, 4 weight rows) with buffer loads: one offset
// register per input row and one for the weights (the stage and the row
// group ride in the scalar offset), which leaves room at two waves per SIMD
// for two register sets.  The loop body is two stages, each set loaded
// during one stage's first unit and written to LDS during the next stage's
// second unit, so loads have more than a stage to land and no register is
// copied (a copy of a register whose load is in flight waits for the load).
// Loads, LDS writes and operand reads are spread between the MFMAs
// (sched_group_barrier): measured 0.42-0.51 of the fp16 peak at M = 8192
// against 0.38-0.43 with them grouped.
//
// Per output the products and their order are the fused kernel's
// (v_mfma_f32_16x16x32_f16 over the same 32-column units, first to last, the
// same lane layout), so with w = the fp16 weight the fused kernel decodes,
// the result is quant_gemm_kernel's bitwise.
constexpr int DT = 256;         // dense tile: input rows = output features
constexpr int DKS = 64;         // columns per stage
constexpr int DENSE_MIN_TILES = 128;   // dense route from this many 256 × 256 tiles

struct DenseArgs {
    const _Float16* x;    // [groups][M][lda]
    int64_t lda, x_gstride;
    const _Float16* w;    // [N][K]
    void* y;              // [M][ldy]
    int64_t ldy;
    int M, N, K, out_per;
};

template <int EP>
__global__ __launch_bounds__(512, 1) void dense_gemm_kernel(DenseArgs g) {
    __shared__ uint4 lds[2][2 * DT * 8];   // per stage: 256 input rows then 256 weight rows, 8 chunks each
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, li = lane & 15;
    // Tiles in groups of 4 row blocks × every feature block, feature-major
    // within a group; XCD x (workgroups x, x + 8, ...) takes a contiguous run
    // of that order, so the 32 workgroups an XCD holds at once share 4 input
    // row blocks and 8 weight blocks in its L2.
    const int ntm = (g.M + DT - 1) / DT, ntn = g.N / DT, total = ntm * ntn;
    const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3;
    const int t = xcd * (total >> 3) + min(xcd, total & 7) + loc;
    const int grp = t / (4 * ntn), first = 4 * grp, gm = min(4, ntm - first);
    const int rr = t - grp * 4 * ntn;
    const int m0 = (first + rr % gm) * DT, n0 = (rr / gm) * DT;
    const int nst = g.K / DKS;

    // staging: thread → chunk c of rows r0 + 64p (p < 4 input rows, clamped
    // to the last row; p >= 4 weight rows), offsets from the tile's first row
    const int c = tid & 7, r0 = tid >> 3;
    const int mrows = min(DT, g.M - m0);
    const _Float16* xt = g.x + (int64_t)(n0 / g.out_per) * g.x_gstride + (int64_t)m0 * g.lda;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(xt), 0, (int)(mrows * g.lda * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(g.w + (int64_t)n0 * g.K), 0, (int)((int64_t)DT * g.K * 2), 0x00020000);
    uint32_t xo[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) xo[p] = (uint32_t)((min(r0 + 64 * p, mrows - 1) * (int)g.lda + 8 * c) * 2);
    const uint32_t wo = (uint32_t)((r0 * g.K + 8 * c) * 2), wrow64 = (uint32_t)(64 * g.K * 2);
    const int dst0 = r0 * 8 + (c ^ (r0 & 7));   // row r0 + 64p: + 512p chunks, the same swizzle
    auto gload = [&](uint4 (&v)[8], int st) {
        const uint32_t so = (uint32_t)(min(st, nst - 1) * DKS * 2);
#pragma unroll
        for (int p = 0; p < 4; ++p)
            v[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[p], so, 0));
#pragma unroll
        for (int p = 0; p < 4; ++p)
            v[4 + p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, so + p * wrow64, 0));
    };
    auto swrite = [&](int buf, const uint4 (&v)[8]) {
#pragma unroll
        for (int p = 0; p < 8; ++p) lds[buf][dst0 + 512 * p] = v[p];
    };

    const int wm = wave & 1, wn = wave >> 1;
    f32x4 acc[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    // operand rows: li + 16·tile (row & 7 = li & 7 for every tile)
    const int ra = (128 * wm + li) * 8, rb = (DT + 64 * wn + li) * 8;
    // A 32-column unit: the B operands first, then the A operands (the
    // order the products use them)
    auto operands = [&](int buf, int kk, half8 (&av)[8], half8 (&bv)[4]) {
        const int ch = (4 * kk + gq) ^ (li & 7);
#pragma unroll
        for (int b = 0; b < 4; ++b) bv[b] = __builtin_bit_cast(half8, lds[buf][rb + 128 * b + ch]);
#pragma unroll
        for (int a = 0; a < 8; ++a) av[a] = __builtin_bit_cast(half8, lds[buf][ra + 128 * a + ch]);
    };
    auto products = [&](const half8 (&av)[8], const half8 (&bv)[4]) {
#pragma unroll
        for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[a], bv[b], acc[a][b], 0, 0, 0);
    };
    // One stage: its two units from LDS buffer `buf`.  The first unit's
    // products carry the loads of a later stage into `ld`, the second's the
    // LDS write of the next stage's chunks from `wr`: six operand reads up
    // front, then per A operand its four MFMAs, the read of the A operand two
    // ahead and one load or write (register use stays at 256, no spills).
    auto stage = [&](int buf, uint4 (&ld)[8], int ldst, const uint4 (&wr)[8]) {
        {
            half8 av[8], bv[4];
            operands(buf, 0, av, bv);
            gload(ld, ldst);
            products(av, bv);
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);   // DS reads
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);   // MFMA
                if (i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        {
            half8 av[8], bv[4];
            operands(buf, 1, av, bv);
            products(av, bv);
            swrite(buf ^ 1, wr);
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                if (i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };

    // nst is even; the last pair's loads repeat the last stage and its final
    // LDS write lands in a buffer no later stage reads
    uint4 va[8], vb[8];
    gload(va, 0);
    swrite(0, va);
    gload(va, 1);
    __syncthreads();
    for (int st = 0; st < nst; st += 2) {
        stage(0, vb, st + 2, va);
        stage(1, va, st + 3, vb);
    }

#pragma unroll
    for (int a = 0; a < 8; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + 128 * wm + 16 * a + 4 * gq + r;
            if (row >= g.M) continue;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                store_out<EP>(g.y, (int64_t)row * g.ldy + n0 + 64 * wn + 16 * b + li, acc[a][b][r]);
        }
    }
}

// The K ranges of a split launch summed in range order (a fixed order: the
// result does not depend on which workgroup finished first), then the
// epilogue of the one-range kernel: fp16 rounding, store / add / relu².
// Thread i takes 4 consecutive outputs of one row (N is a multiple of 128).
template <int EP>
__global__ __launch_bounds__(256) void gemm_split_reduce(const float* __restrict__ part, int S, int M, int N,
                                                         void* y, int64_t ldy) {
    const int64_t n4 = (int64_t)M * N / 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4* p = reinterpret_cast<const float4*>(part) + i;
    float4 a = p[0];
    for (int k = 1; k < S; ++k) {
        const float4 b = p[(int64_t)k * n4];
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    const int64_t row = 4 * i / N, col = 4 * i % N;
    const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) store_out<EP>(y, row * ldy + col + c, v[c]);
}

// K ranges per launch: one where the (row block, feature block) tiles
// already fill the chip; otherwise enough to reach about 384 workgroups
// (two per CU hold 512), each range at least 3 stages of 64 columns.  A
// tile's stages run one after another, each waiting on its loads (about
// 2 µs a stage at a few workgroups per XCD), so few tiles over a long K
// take K/64 such waits: 128 rows × 768 features × K 3072, 6 tiles, took
// 100 µs in one range.
int gemm_splits(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = ((M + 127) / 128) * (N / 128);
    if (tiles >= 160) return 1;
    const int64_t want = (384 + tiles - 1) / tiles, most = K / BK / 3;
    return (int)std::max<int64_t>(1, std::min(want, most));
}

// The dense kernel's shapes (x rows lda halves apart, group g at x + g·x_gstride).
bool dense_shape_ok(int64_t M, int64_t OUT, int64_t IN, int64_t out_per, int64_t lda) {
    return M >= 1 && M <= ((int64_t)1 << 24) && OUT >= DT && OUT % DT == 0 && OUT <= ((int64_t)1 << 30) &&
           out_per >= DT && out_per % DT == 0 && OUT % out_per == 0 && IN >= 2 * DKS && IN % (2 * DKS) == 0 &&
           lda >= IN && lda % 8 == 0 && (int64_t)DT * lda * 2 < ((int64_t)1 << 31) &&
           ((M + DT - 1) / DT) * (OUT / DT) < ((int64_t)1 << 31);
}

// The quantised entry points take the dense route (dequantise into the
// workspace, then dense_gemm_kernel) from DENSE_MIN_TILES tiles: half a round
// of the 256 CUs.  Below it the fused kernel's 128 × 128 tiles (and its K
// split) keep more CUs busy and no dequant is paid: 4096 rows × 1024 × 1024
// took 34 µs fused against 9.5 + 34 µs dequant + dense.
bool dense_prefers(int64_t M, int64_t OUT, int64_t IN) {
    return dense_shape_ok(M, OUT, IN, OUT, IN) && ((M + DT - 1) / DT) * (OUT / DT) >= DENSE_MIN_TILES;
}

int64_t gemm_workspace(int64_t M, int64_t N, int64_t K) {
    if (dense_prefers(M, N, K)) return N * K * 2;   // the fp16 weight
    const int S = gemm_splits(M, N, K);
    return S > 1 ? (int64_t)S * M * N * 4 : 0;
}

template <int EP>
void launch_dense_ep(const DenseArgs& g, hipStream_t s) {
    const int64_t tiles = (int64_t)((g.M + DT - 1) / DT) * (g.N / DT);
    rwkv::launch(dense_gemm_kernel<EP>, dim3((unsigned)tiles), dim3(512), s, g);
}

void launch_dense(const DenseArgs& g, int epilogue, hipStream_t s) {
    switch (epilogue) {
        case 0: launch_dense_ep<0>(g, s); break;
        case 1: launch_dense_ep<1>(g, s); break;
        default: launch_dense_ep<2>(g, s); break;
    }
}

// One tile shape: 128 × 128 with two workgroups per CU measured fastest
// (larger tiles cost occupancy: at one wave per SIMD the stage's loads are
// not hidden).
template <class F, typename TA, int EP>
void launch_gemm(const GemmArgs& g, hipStream_t s) {
    const int64_t blocks = (int64_t)((g.M + 127) / 128) * (g.N / 128) * g.splits;
    rwkv::launch(quant_gemm_kernel<F, TA, EP, 8, 2>, dim3((unsigned)blocks), dim3(256), s, g);
    if (g.splits > 1) {
        const int64_t n4 = (int64_t)g.M * g.N / 4;
        rwkv::launch(gemm_split_reduce<EP>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), s, g.part, g.splits,
                     g.M, g.N, g.y, g.ldy);
    }
}

template <class F>
void launch_gemm_ep(const GemmArgs& g, bool f16, int epilogue, hipStream_t s) {
    switch (epilogue) {
        case 0: f16 ? launch_gemm<F, _Float16, 0>(g, s) : launch_gemm<F, float, 0>(g, s); break;
        case 1: f16 ? launch_gemm<F, _Float16, 1>(g, s) : launch_gemm<F, float, 1>(g, s); break;
        default: f16 ? launch_gemm<F, _Float16, 2>(g, s) : launch_gemm<F, float, 2>(g, s); break;
    }
}

bool gemm_shape_ok(int64_t OUT, int64_t IN, int64_t out_per) {
    return OUT >= 128 && OUT % 128 == 0 && IN >= 256 && IN % 256 == 0 && out_per >= 128 && out_per % 128 == 0 &&
           OUT % out_per == 0 && OUT <= ((int64_t)1 << 30) && IN <= ((int64_t)1 << 24);
}

// Shared argument checks of the two entry points.
rwkv_status gemm_check(const char* who, const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda,
                       int64_t x_group_stride, int64_t ldy, int64_t OUT, int64_t IN, int64_t out_per, int epilogue) {
    RWKV_REQUIRE(x_dt == RWKV_F32 || x_dt == RWKV_F16, RWKV_E_DTYPE, "%s: inputs must be f32 or f16", who);
    RWKV_REQUIRE(epilogue >= 0 && epilogue <= 2, RWKV_E_SHAPE, "%s: epilogue %d", who, epilogue);
    RWKV_REQUIRE(M >= 1 && M <= ((int64_t)1 << 24), RWKV_E_SHAPE, "%s: M (%lld) out of range", who, (long long)M);
    const int64_t groups = OUT / out_per;
    const int64_t xes = x_dt == RWKV_F32 ? 4 : 2;
    RWKV_REQUIRE(lda >= IN && lda % 8 == 0 && (groups == 1 || x_group_stride >= M * lda), RWKV_E_SHAPE,
                 "%s: lda (%lld) must be >= IN and a multiple of 8; groups need x_group_stride >= M·lda", who,
                 (long long)lda);
    RWKV_REQUIRE(ldy >= OUT && (epilogue == 2 ? ldy % 2 == 0 : true), RWKV_E_SHAPE, "%s: ldy (%lld) < OUT", who,
                 (long long)ldy);
    RWKV_REQUIRE((reinterpret_cast<uintptr_t>(x) % 16) == 0 && (x_group_stride * xes) % 16 == 0, RWKV_E_SHAPE,
                 "%s: inputs must be 16-byte aligned", who);
    RWKV_REQUIRE(((M + 127) / 128) * (OUT / 128) <= ((int64_t)1 << 26), RWKV_E_SHAPE,
                 "%s: %lld x %lld outputs exceed one launch", who, (long long)M, (long long)OUT);
    return RWKV_OK;
}

// A caller's workspace: NULL, or at least rwkv_quant_gemm_workspace bytes,
// 16-byte aligned (checked before anything is launched).
rwkv_status gemm_workspace_check(const char* who, int64_t M, int64_t N, int64_t K, const void* workspace,
                                 int64_t workspace_bytes) {
    if (workspace == nullptr) return RWKV_OK;
    const int64_t need = gemm_workspace(M, N, K);
    RWKV_REQUIRE(workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 16 == 0, RWKV_E_SHAPE,
                 "%s: workspace of %lld bytes (16-byte aligned) needed, %lld given", who, (long long)need,
                 (long long)workspace_bytes);
    return RWKV_OK;
}

// The dense route of a quantised entry point: fp16 inputs, a workspace, and
// a shape the dense kernel takes with enough tiles.
bool take_dense(rwkv_dtype x_dt, int64_t M, int64_t OUT, int64_t IN, int64_t out_per, int64_t lda,
                const void* workspace) {
    return workspace != nullptr && x_dt == RWKV_F16 && dense_prefers(M, OUT, IN) &&
           dense_shape_ok(M, OUT, IN, out_per, lda);
}

// The fused launch's K ranges: several where the shape asks for them and the
// caller passed a workspace, one otherwise.
void gemm_split_args(GemmArgs& g, void* workspace) {
    g.part = nullptr;
    g.splits = 1;
    const int S = gemm_splits(g.M, g.N, g.K);
    if (workspace == nullptr || S == 1 || dense_prefers(g.M, g.N, g.K)) return;
    g.part = reinterpret_cast<float*>(workspace);
    g.splits = S;
}

}  // namespace

extern "C" {

int64_t rwkv_quant_gemm_workspace(int64_t M, int64_t OUT, int64_t IN) {
    if (M < 1 || M > ((int64_t)1 << 24) || OUT < 128 || OUT % 128 != 0 || IN < 256 || IN % 256 != 0) return 0;
    return gemm_workspace(M, OUT, IN);
}

int rwkv_sb6_gemm_applies(int64_t OUT, int64_t IN, int xbits, int64_t out_per) {
    return xbits >= 0 && xbits <= 2 && gemm_shape_ok(OUT, IN, out_per);
}

rwkv_status rwkv_sb6_gemm(const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda, int64_t x_group_stride,
                          const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, void* y, int64_t ldy,
                          int64_t OUT, int64_t IN, int xbits, int64_t out_per, int epilogue, void* workspace,
                          int64_t workspace_bytes, void* stream) {
    RWKV_REQUIRE(x && qblk && qsqm && ddm && y, RWKV_E_NULL, "sb6_gemm: null buffer");
    RWKV_REQUIRE(rwkv_sb6_gemm_applies(OUT, IN, xbits, out_per), RWKV_E_UNSUPPORTED,
                 "sb6_gemm: xbits %d (0..2), OUT (%lld) and out_per (%lld) multiples of 128, IN (%lld) of 256", xbits,
                 (long long)OUT, (long long)out_per, (long long)IN);
    rwkv_status c = gemm_check("sb6_gemm", x, x_dt, M, lda, x_group_stride, ldy, OUT, IN, out_per, epilogue);
    if (c != RWKV_OK) return c;
    c = gemm_workspace_check("sb6_gemm", M, OUT, IN, workspace, workspace_bytes);
    if (c != RWKV_OK) return c;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (take_dense(x_dt, M, OUT, IN, out_per, lda, workspace)) {
        c = rwkv_sb6_dequant(qblk, qsqm, ddm, workspace, RWKV_F16, OUT, IN, xbits, stream);
        if (c != RWKV_OK) return c;
        launch_dense(DenseArgs{reinterpret_cast<const _Float16*>(x), lda, x_group_stride,
                               reinterpret_cast<const _Float16*>(workspace), y, ldy, (int)M, (int)OUT, (int)IN,
                               (int)out_per},
                     epilogue, s);
    } else {
        GemmArgs g{x, lda, x_group_stride, qblk, qsqm, ddm, y, ldy, (int)M, (int)OUT, (int)IN, (int)out_per};
        gemm_split_args(g, workspace);
        const bool f16 = x_dt == RWKV_F16;
        if (xbits == 0) launch_gemm_ep<Sb6W<0>>(g, f16, epilogue, s);
        else if (xbits == 1) launch_gemm_ep<Sb6W<1>>(g, f16, epilogue, s);
        else launch_gemm_ep<Sb6W<2>>(g, f16, epilogue, s);
    }
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "sb6_gemm: launch failed");
    rwkv::counters().sb6_gemm.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

int rwkv_sym_gemm_applies(int64_t OUT, int64_t IN, int bits, int64_t out_per) {
    return (bits == 8 || bits == 6) && gemm_shape_ok(OUT, IN, out_per);
}

rwkv_status rwkv_sym_gemm(const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda, int64_t x_group_stride,
                          const uint8_t* qblk, const uint8_t* qs, const uint16_t* d, void* y, int64_t ldy,
                          int64_t OUT, int64_t IN, int bits, int64_t out_per, int epilogue, void* workspace,
                          int64_t workspace_bytes, void* stream) {
    RWKV_REQUIRE(x && qblk && qs && d && y, RWKV_E_NULL, "sym_gemm: null buffer");
    RWKV_REQUIRE(rwkv_sym_gemm_applies(OUT, IN, bits, out_per), RWKV_E_UNSUPPORTED,
                 "sym_gemm: %d-bit codes (8 or 6), OUT (%lld) and out_per (%lld) multiples of 128, IN (%lld) of 256",
                 bits, (long long)OUT, (long long)out_per, (long long)IN);
    rwkv_status c = gemm_check("sym_gemm", x, x_dt, M, lda, x_group_stride, ldy, OUT, IN, out_per, epilogue);
    if (c != RWKV_OK) return c;
    c = gemm_workspace_check("sym_gemm", M, OUT, IN, workspace, workspace_bytes);
    if (c != RWKV_OK) return c;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (take_dense(x_dt, M, OUT, IN, out_per, lda, workspace)) {
        c = rwkv_sym_dequant(qblk, qs, d, workspace, RWKV_F16, OUT, IN, bits, stream);
        if (c != RWKV_OK) return c;
        launch_dense(DenseArgs{reinterpret_cast<const _Float16*>(x), lda, x_group_stride,
                               reinterpret_cast<const _Float16*>(workspace), y, ldy, (int)M, (int)OUT, (int)IN,
                               (int)out_per},
                     epilogue, s);
    } else {
        GemmArgs g{x, lda, x_group_stride, qblk, qs, d, y, ldy, (int)M, (int)OUT, (int)IN, (int)out_per};
        gemm_split_args(g, workspace);
        const bool f16 = x_dt == RWKV_F16;
        if (bits == 8) launch_gemm_ep<SymW<8>>(g, f16, epilogue, s);
        else launch_gemm_ep<SymW<6>>(g, f16, epilogue, s);
    }
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "sym_gemm: launch failed");
    rwkv::counters().sym_gemm.fetch_add(1);
    rwkv::clear_error();
    return RWKV_OK;
}

int rwkv_f16_gemm_applies(int64_t M, int64_t OUT, int64_t IN, int64_t out_per) {
    return dense_shape_ok(M, OUT, IN, out_per, IN);
}

rwkv_status rwkv_f16_gemm(const void* x, int64_t M, int64_t lda, int64_t x_group_stride, const void* w, void* y,
                          int64_t ldy, int64_t OUT, int64_t IN, int64_t out_per, int epilogue, void* stream) {
    RWKV_REQUIRE(x && w && y, RWKV_E_NULL, "f16_gemm: null buffer");
    RWKV_REQUIRE(dense_shape_ok(M, OUT, IN, out_per, lda), RWKV_E_UNSUPPORTED,
                 "f16_gemm: M %lld, OUT (%lld) and out_per (%lld) multiples of 256, IN (%lld) of 128, lda (%lld) >= "
                 "IN and a multiple of 8",
                 (long long)M, (long long)OUT, (long long)out_per, (long long)IN, (long long)lda);
    rwkv_status c = gemm_check("f16_gemm", x, RWKV_F16, M, lda, x_group_stride, ldy, OUT, IN, out_per, epilogue);
    if (c != RWKV_OK) return c;
    RWKV_REQUIRE(reinterpret_cast<uintptr_t>(w) % 16 == 0, RWKV_E_SHAPE, "f16_gemm: weights must be 16-byte aligned");
    launch_dense(DenseArgs{reinterpret_cast<const _Float16*>(x), lda, x_group_stride,
                           reinterpret_cast<const _Float16*>(w), y, ldy, (int)M, (int)OUT, (int)IN, (int)out_per},
                 epilogue, reinterpret_cast<hipStream_t>(stream));
    RWKV_REQUIRE(hipGetLastError() == hipSuccess, RWKV_E_HIP, "f16_gemm: launch failed");
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"
