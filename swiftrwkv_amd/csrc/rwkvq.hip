// .rwkvq dequantisation and decode GEMV on gfx950.
//
// Formats (loader layouts, Sources/RWKVQuant/RwkvqFile.swift:183-212,437-449):
//   sb6 (block 32, super-block 8 blocks):
//     qblk[row, blk] = 16 B nibbles (byte c: column c low, column c+16 high)
//                      ‖ 4 B qh (bit c → bit 4 of column c) ‖ 4 B qh2 (bit 5)
//     qsqm[row, blk] = (qs u8, qm i8);   ddm[row, sb] = (d, dm) fp16
//     w = code·half(qs·d) + half(qm·dm), combined in fp32 (RwkvqDequant.swift:116-140)
//   sym (block 16, super-block 16 blocks):
//     8-bit: qblk = int8 codes [OUT, IN];  6-bit: per 32-column pair 16 B nibbles
//     (block-local: byte j of a block's 8 bytes holds column j low, j+8 high)
//     ‖ qh ‖ qh2, codes stored +32;  qs int8 [OUT, IN/16];  d fp16 [OUT, IN/256]
//     w = (q [−32])·half(qs·d) (RwkvqDequant.swift:350-388)
//
// GEMV (decode) mapping.  A row of IN columns is a sequence of NU "units"
// (sb6: one 32-column block; sym: 32 columns = 2 blocks).  G lanes (the largest
// power of two ≤ 64 dividing NU) cover one row; each lane owns the units
// g, g+G, ... of that row for every row it processes, so its x slice (32
// floats per unit) is loaded once into registers and reused across the RL
// consecutive rows assigned to it ("x-stationary").  Weight bytes are streamed
// exactly once: at fixed (unit, row) the G lanes read G consecutive units, so
// each wave-wide load covers whole 128-byte lines.  Codes are widened with
// byte→float conversions, dotted with x in fp32, and scaled once per block:
//   sb6:  Σ (q·s + m)·x = s·Σ q·x + m·Σ x      (RwkvqSb6GEMV.swift:118-144)
//   sym6: Σ (q−32)·s·x = s·(Σ q·x − 32·Σ x)    (RwkvqSymGEMV.swift:182-194)
// and the per-lane partial sums are reduced over the G lanes with a fixed
// butterfly.  N input rows (batched decode) share one weight pass (in tiles
// of NT ≤ 4 rows).  All sums have a fixed order: results are deterministic.

#include <hip/hip_runtime.h>

#include "launch.h"

namespace {

__device__ __forceinline__ float f16f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}
// fp32 → fp16 (RNE) → fp32, the `(half)` round trip of the reference kernels.
__device__ __forceinline__ float hround(float x) { return (float)(_Float16)x; }

// 4 bits → the low bit of 4 bytes (RwkvqSb6GEMV.swift:58-67 multiply spread).
__device__ __forceinline__ uint32_t spread4(uint32_t nib) { return (nib * 0x00204081u) & 0x01010101u; }

template <int DT>
__device__ __forceinline__ void store4(void* out, int64_t idx, float a, float b, float c, float d) {
    if constexpr (DT == RWKV_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + idx) = make_float4(a, b, c, d);
    } else {
        uint16_t h[4];
        float f[4] = {a, b, c, d};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (DT == RWKV_BF16) {
                uint32_t u = __float_as_uint(f[e]);
                h[e] = ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu))
                           ? (uint16_t)((u >> 16) | 0x40u)
                           : (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
            } else {
                h[e] = __builtin_bit_cast(uint16_t, (_Float16)f[e]);
            }
        }
        uint2 pk = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + idx) = pk;
    }
}

// ─────────────────────────────── sb6 dequant ───────────────────────────────
// One thread per (row, block, part): part p covers columns 4p..4p+3 of the
// block (p < 4: low nibbles of word p; p >= 4: high nibbles of word p-4), so 8
// consecutive threads write one block's 32 outputs contiguously.
template <int XB, int DT>
__global__ __launch_bounds__(256) void sb6_dequant_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qsqm, const uint16_t* __restrict__ ddm,
    void* __restrict__ out, int64_t OUT, int64_t IN) {
    constexpr int SUW = 4 + XB;  // 32-bit words per block
    const int64_t NB = IN >> 5, NSB = NB >> 3;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= OUT * NB * 8) return;
    const int p = (int)(gid & 7);
    const int64_t rb = gid >> 3;   // row * NB + blk
    const int64_t row = rb / NB, blk = rb - row * NB;
    const uint32_t* qb = reinterpret_cast<const uint32_t*>(qblk) + rb * SUW;
    const uint32_t wd = qb[p & 3];
    uint32_t q4 = (p < 4) ? (wd & 0x0F0F0F0Fu) : ((wd >> 4) & 0x0F0F0F0Fu);
    if constexpr (XB >= 1) q4 |= spread4((qb[4] >> (4 * p)) & 0xFu) << 4;
    if constexpr (XB >= 2) q4 |= spread4((qb[5] >> (4 * p)) & 0xFu) << 5;
    const uint16_t sm = reinterpret_cast<const uint16_t*>(qsqm)[rb];
    const uint32_t dd = reinterpret_cast<const uint32_t*>(ddm)[row * NSB + (blk >> 3)];
    const float s = hround((float)(sm & 0xffu) * f16f(dd));
    const float m = hround((float)(int8_t)(sm >> 8) * f16f(dd >> 16));
    store4<DT>(out, row * IN + blk * 32 + 4 * p,
               fmaf((float)(q4 & 0xffu), s, m), fmaf((float)((q4 >> 8) & 0xffu), s, m),
               fmaf((float)((q4 >> 16) & 0xffu), s, m), fmaf((float)(q4 >> 24), s, m));
}

// ─────────────────────────────── sym dequant ───────────────────────────────
// 8-bit: one thread per 4 columns.  6-bit: one thread per (pair, part p),
// part p = columns 4p..4p+3 of the pair in register order l0,l1,h0,h1,l2,l3,h2,h3.
template <int BITS, int DT>
__global__ __launch_bounds__(256) void sym_dequant_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d,
    void* __restrict__ out, int64_t OUT, int64_t IN) {
    const int64_t NB = IN >> 4, NSB = (NB + 15) >> 4;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= OUT * (IN >> 2)) return;
    const int64_t row = gid / (IN >> 2);
    const int64_t col = (gid - row * (IN >> 2)) * 4;
    const int64_t blk = col >> 4;
    const float s = hround((float)(int8_t)qs[row * NB + blk] * f16f(d[row * NSB + (blk >> 4)]));
    float f[4];
    if constexpr (BITS == 8) {
        const uint32_t wd = *reinterpret_cast<const uint32_t*>(qblk + row * IN + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = (float)(int8_t)(wd >> (8 * e)) * s;
    } else {
        const int64_t pair = col >> 5;
        const int p = (int)((col & 31) >> 2);
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(qblk + (row * (IN >> 5) + pair) * 24);
        const int hp = p >> 2, pm = p & 3;
        const uint32_t wd = qb[2 * hp + (pm & 1)];
        uint32_t q4 = (pm < 2) ? (wd & 0x0F0F0F0Fu) : ((wd >> 4) & 0x0F0F0F0Fu);
        q4 |= spread4((qb[4] >> (4 * p)) & 0xFu) << 4;
        q4 |= spread4((qb[5] >> (4 * p)) & 0xFu) << 5;
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = (float)((int)((q4 >> (8 * e)) & 0xffu) - 32) * s;
    }
    store4<DT>(out, row * IN + col, f[0], f[1], f[2], f[3]);
}

// ─────────────────────────────── GEMV ───────────────────────────────
// Decode 32 codes of one unit into bytes b[0..7] (4 codes per word, word m
// holds columns 4m..4m+3) then dot with x[0..31].
__device__ __forceinline__ float dot32_u8(const uint32_t (&q)[8], const float* x) {
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            d0 = fmaf((float)((q[m] >> (8 * e)) & 0xffu), x[4 * m + e], d0);
            d1 = fmaf((float)((q[m + 4] >> (8 * e)) & 0xffu), x[16 + 4 * m + e], d1);
        }
    }
    return d0 + d1;
}

template <int XB>
__device__ __forceinline__ void sb6_unit_codes(const uint32_t* __restrict__ qb, uint32_t (&q)[8]) {
    uint32_t wd[4 + XB];
#pragma unroll
    for (int m = 0; m < 4 + XB; ++m) wd[m] = qb[m];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        q[m] = wd[m] & 0x0F0F0F0Fu;              // columns 4m..4m+3
        q[m + 4] = (wd[m] >> 4) & 0x0F0F0F0Fu;   // columns 16+4m..16+4m+3
    }
    if constexpr (XB >= 1) {
#pragma unroll
        for (int m = 0; m < 8; ++m) q[m] |= spread4((wd[4] >> (4 * m)) & 0xFu) << 4;
    }
    if constexpr (XB >= 2) {
#pragma unroll
        for (int m = 0; m < 8; ++m) q[m] |= spread4((wd[5] >> (4 * m)) & 0xFu) << 5;
    }
}

__device__ __forceinline__ void load_x32(const float* __restrict__ xp, float (&xv)[32]) {
    const float4* p = reinterpret_cast<const float4*>(xp);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        float4 f = p[m];
        xv[4 * m] = f.x; xv[4 * m + 1] = f.y; xv[4 * m + 2] = f.z; xv[4 * m + 3] = f.w;
    }
}

struct GemvGeom {
    int G;     // lanes per row
    int R;     // row groups per wave (64 / G)
    int KU;    // units per lane (NU / G)
    int RL;    // consecutive rows per lane
    int WPB;   // waves per workgroup
};

// sb6: unit = 32-column block.
template <int XB, int RL, int NT>
__global__ __launch_bounds__(256) void sb6_gemv_kernel(
    const float* __restrict__ x, int N, const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qsqm,
    const uint16_t* __restrict__ ddm, float* __restrict__ y, int OUT, int IN, GemvGeom geo) {
    constexpr int SUW = 4 + XB;
    const int NB = IN >> 5, NSB = NB >> 3;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gi = lane / geo.G, g = lane - gi * geo.G;
    const int row0 = (blockIdx.x * geo.WPB + wave) * geo.R * RL + gi * RL;
    if (row0 >= OUT) return;   // whole lane idle (rows are assigned in RL-aligned groups)
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(qblk);
    const uint16_t* sm2 = reinterpret_cast<const uint16_t*>(qsqm);
    const uint32_t* dd2 = reinterpret_cast<const uint32_t*>(ddm);

    for (int n0 = 0; n0 < N; n0 += NT) {
        float acc[NT][RL];
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) acc[nn][rr] = 0.0f;
        for (int ku = 0; ku < geo.KU; ++ku) {
            const int blk = ku * geo.G + g;
            float xv[NT][32], xs[NT];
#pragma unroll
            for (int nn = 0; nn < NT; ++nn) {
                const int n = min(n0 + nn, N - 1);
                load_x32(x + (int64_t)n * IN + blk * 32, xv[nn]);
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int c = 0; c < 16; ++c) { s0 += xv[nn][c]; s1 += xv[nn][16 + c]; }
                xs[nn] = s0 + s1;
            }
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                const int row = row0 + rr;
                if (row < OUT) {
                    const int64_t rb = (int64_t)row * NB + blk;
                    uint32_t q[8];
                    sb6_unit_codes<XB>(qw + rb * SUW, q);
                    const uint32_t smv = sm2[rb];
                    const uint32_t dd = dd2[(int64_t)row * NSB + (blk >> 3)];
                    const float s = hround((float)(smv & 0xffu) * f16f(dd));
                    const float m = hround((float)(int8_t)(smv >> 8) * f16f(dd >> 16));
#pragma unroll
                    for (int nn = 0; nn < NT; ++nn) {
                        const float dv = dot32_u8(q, xv[nn]);
                        acc[nn][rr] = fmaf(m, xs[nn], fmaf(s, dv, acc[nn][rr]));
                    }
                }
            }
        }
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                float t = acc[nn][rr];
                for (int off = geo.G >> 1; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
                const int row = row0 + rr;
                if (g == 0 && row < OUT && n0 + nn < N) y[(int64_t)(n0 + nn) * OUT + row] = t;
            }
    }
}

// sym: unit = 32 columns (two 16-blocks).  Input row of output row `row` for
// input n is x[n·NK + row/out_per].
template <int BITS, int RL, int NT>
__global__ __launch_bounds__(256) void sym_gemv_kernel(
    const float* __restrict__ x, int N, const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qs,
    const uint16_t* __restrict__ d, float* __restrict__ y, int OUT, int IN, int out_per, GemvGeom geo) {
    const int NB = IN >> 4, NSB = IN >> 8, NU = IN >> 5;
    const int NK = OUT / out_per;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gi = lane / geo.G, g = lane - gi * geo.G;
    const int row0 = (blockIdx.x * geo.WPB + wave) * geo.R * RL + gi * RL;
    if (row0 >= OUT) return;
    const int xi = row0 / out_per;   // all RL rows of this lane share it (out_per % RL == 0)
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(qblk);
    const uint16_t* qs2 = reinterpret_cast<const uint16_t*>(qs);

    for (int n0 = 0; n0 < N; n0 += NT) {
        float acc[NT][RL];
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) acc[nn][rr] = 0.0f;
        for (int ku = 0; ku < geo.KU; ++ku) {
            const int u = ku * geo.G + g;
            float xv[NT][32], xs0[NT], xs1[NT];
#pragma unroll
            for (int nn = 0; nn < NT; ++nn) {
                const int n = min(n0 + nn, N - 1);
                load_x32(x + ((int64_t)n * NK + xi) * IN + u * 32, xv[nn]);
                if constexpr (BITS == 6) {
                    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                    for (int c = 0; c < 16; ++c) { s0 += xv[nn][c]; s1 += xv[nn][16 + c]; }
                    xs0[nn] = s0; xs1[nn] = s1;
                }
            }
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                const int row = row0 + rr;
                if (row < OUT) {
                    const uint32_t sc = qs2[(int64_t)row * (NB >> 1) + u];   // two int8 block scales
                    const float dsb = f16f(d[(int64_t)row * NSB + (u >> 3)]);
                    const float s0 = hround((float)(int8_t)(sc & 0xffu) * dsb);
                    const float s1 = hround((float)(int8_t)(sc >> 8) * dsb);
                    if constexpr (BITS == 8) {
                        const uint32_t* qb = qw + ((int64_t)row * IN + u * 32) / 4;
                        uint32_t wd[8];
#pragma unroll
                        for (int m = 0; m < 8; ++m) wd[m] = qb[m];
#pragma unroll
                        for (int nn = 0; nn < NT; ++nn) {
                            float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                            for (int m = 0; m < 4; ++m)
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    d0 = fmaf((float)(int8_t)(wd[m] >> (8 * e)), xv[nn][4 * m + e], d0);
                                    d1 = fmaf((float)(int8_t)(wd[m + 4] >> (8 * e)), xv[nn][16 + 4 * m + e], d1);
                                }
                            acc[nn][rr] = fmaf(s1, d1, fmaf(s0, d0, acc[nn][rr]));
                        }
                    } else {
                        const uint32_t* qb = qw + ((int64_t)row * NU + u) * 6;
                        uint32_t wd[6];
#pragma unroll
                        for (int m = 0; m < 6; ++m) wd[m] = qb[m];
                        // register order l0,l1,h0,h1 | l2,l3,h2,h3 → columns 4m..4m+3
                        uint32_t q[8];
                        q[0] = wd[0] & 0x0F0F0F0Fu;         q[1] = wd[1] & 0x0F0F0F0Fu;
                        q[2] = (wd[0] >> 4) & 0x0F0F0F0Fu;  q[3] = (wd[1] >> 4) & 0x0F0F0F0Fu;
                        q[4] = wd[2] & 0x0F0F0F0Fu;         q[5] = wd[3] & 0x0F0F0F0Fu;
                        q[6] = (wd[2] >> 4) & 0x0F0F0F0Fu;  q[7] = (wd[3] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                        for (int m = 0; m < 8; ++m) {
                            q[m] |= spread4((wd[4] >> (4 * m)) & 0xFu) << 4;
                            q[m] |= spread4((wd[5] >> (4 * m)) & 0xFu) << 5;
                        }
#pragma unroll
                        for (int nn = 0; nn < NT; ++nn) {
                            float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                            for (int m = 0; m < 4; ++m)
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    d0 = fmaf((float)((q[m] >> (8 * e)) & 0xffu), xv[nn][4 * m + e], d0);
                                    d1 = fmaf((float)((q[m + 4] >> (8 * e)) & 0xffu), xv[nn][16 + 4 * m + e], d1);
                                }
                            acc[nn][rr] = fmaf(s1, fmaf(-32.0f, xs1[nn], d1), fmaf(s0, fmaf(-32.0f, xs0[nn], d0), acc[nn][rr]));
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                float t = acc[nn][rr];
                for (int off = geo.G >> 1; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
                const int row = row0 + rr;
                if (g == 0 && row < OUT && n0 + nn < N) y[(int64_t)(n0 + nn) * OUT + row] = t;
            }
    }
}

// ─────────────────────────────── host side ───────────────────────────────
rwkv_status launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        rwkv::set_error("%s: %s", what, hipGetErrorString(e));
        return RWKV_E_HIP;
    }
    rwkv::clear_error();
    return RWKV_OK;
}

// Geometry for NU units per row and OUT rows: G lanes per row, RL rows per
// lane (dividing `rl_div`), waves per block shrunk until the grid reaches
// ~2 workgroups per CU when the matrix allows it.
GemvGeom pick_geom(int64_t OUT, int64_t NU, int64_t rl_div) {
    GemvGeom g{};
    int64_t G = NU & -NU;
    if (G > 64) G = 64;
    g.G = (int)G;
    g.R = 64 / g.G;
    g.KU = (int)(NU / G);
    g.RL = (rl_div % 4 == 0) ? 4 : (rl_div % 2 == 0) ? 2 : 1;
    g.WPB = 4;
    auto blocks = [&](const GemvGeom& q) { return (OUT + (int64_t)q.WPB * q.R * q.RL - 1) / ((int64_t)q.WPB * q.R * q.RL); };
    while (blocks(g) < 512 && (g.RL > 1 || g.WPB > 1)) {
        if (g.RL > 1) g.RL >>= 1;
        else g.WPB >>= 1;
    }
    return g;
}

int pick_nt(int64_t N) { return N >= 4 ? 4 : N >= 2 ? 2 : 1; }

}  // namespace

extern "C" {

rwkv_status rwkv_sb6_dequant(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, void* out,
                             rwkv_dtype out_dt, int64_t OUT, int64_t IN, int xbits, void* stream) {
    RWKV_REQUIRE(qblk && qsqm && ddm && out, RWKV_E_NULL, "sb6_dequant: null buffer");
    RWKV_REQUIRE(xbits >= 0 && xbits <= 2, RWKV_E_SHAPE, "sb6_dequant: xbits %d outside 0...2", xbits);
    RWKV_REQUIRE(rwkv::dtype_ok(out_dt), RWKV_E_DTYPE, "sb6_dequant: output dtype code %d", out_dt);
    RWKV_REQUIRE(OUT >= 1 && IN >= 256 && IN % 256 == 0, RWKV_E_SHAPE,
                 "sb6_dequant: IN (%lld) must be a positive multiple of 256 (block 32 x super-block 8)", (long long)IN);
    const int64_t total = OUT * (IN / 32) * 8;
    RWKV_REQUIRE(total / 256 < INT32_MAX, RWKV_E_SHAPE, "sb6_dequant: tensor too large");
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RWKV_DQ(XB, DT) rwkv::launch(sb6_dequant_kernel<XB, DT>, grid, block, st, qblk, qsqm, ddm, out, OUT, IN)
#define RWKV_DQ_DT(XB)                                  \
    switch (out_dt) {                                   \
        case RWKV_F32: RWKV_DQ(XB, RWKV_F32); break;    \
        case RWKV_BF16: RWKV_DQ(XB, RWKV_BF16); break;  \
        case RWKV_F16: RWKV_DQ(XB, RWKV_F16); break;    \
    }
    switch (xbits) {
        case 0: RWKV_DQ_DT(0) break;
        case 1: RWKV_DQ_DT(1) break;
        default: RWKV_DQ_DT(2) break;
    }
#undef RWKV_DQ_DT
#undef RWKV_DQ
    rwkv_status s = launch_status("sb6_dequant launch");
    if (s == RWKV_OK) rwkv::counters().sb6_dequant++;
    return s;
}

rwkv_status rwkv_sym_dequant(const uint8_t* qblk, const uint8_t* qs, const uint16_t* d, void* out,
                             rwkv_dtype out_dt, int64_t OUT, int64_t IN, int bits, void* stream) {
    RWKV_REQUIRE(qblk && qs && d && out, RWKV_E_NULL, "sym_dequant: null buffer");
    RWKV_REQUIRE(bits == 6 || bits == 8, RWKV_E_SHAPE, "sym_dequant: bits %d outside {6, 8}", bits);
    RWKV_REQUIRE(rwkv::dtype_ok(out_dt), RWKV_E_DTYPE, "sym_dequant: output dtype code %d", out_dt);
    RWKV_REQUIRE(OUT >= 1 && IN >= 16 && IN % (bits == 8 ? 16 : 32) == 0, RWKV_E_SHAPE,
                 "sym_dequant: IN (%lld) must be a positive multiple of %d", (long long)IN, bits == 8 ? 16 : 32);
    const int64_t total = OUT * (IN / 4);
    RWKV_REQUIRE(total / 256 < INT32_MAX, RWKV_E_SHAPE, "sym_dequant: tensor too large");
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RWKV_DQ(BITS, DT) rwkv::launch(sym_dequant_kernel<BITS, DT>, grid, block, st, qblk, qs, d, out, OUT, IN)
#define RWKV_DQ_DT(BITS)                                  \
    switch (out_dt) {                                     \
        case RWKV_F32: RWKV_DQ(BITS, RWKV_F32); break;    \
        case RWKV_BF16: RWKV_DQ(BITS, RWKV_BF16); break;  \
        case RWKV_F16: RWKV_DQ(BITS, RWKV_F16); break;    \
    }
    if (bits == 8) {
        RWKV_DQ_DT(8)
    } else {
        RWKV_DQ_DT(6)
    }
#undef RWKV_DQ_DT
#undef RWKV_DQ
    rwkv_status s = launch_status("sym_dequant launch");
    if (s == RWKV_OK) rwkv::counters().sym_dequant++;
    return s;
}

int rwkv_sb6_gemv_applies(int64_t OUT, int64_t IN, int xbits, int super_block, int64_t rows) {
    // rwkvqSb6GEMVConfig (RwkvqSb6GEMV.swift:39-43) and Applies (:159-164).
    int nsg = 4, rs = 4;
    if (OUT < 32768 && OUT >= 8192 && xbits == 0) { nsg = 2; rs = 2; }
    return xbits >= 0 && xbits <= 2 && super_block == 8 && rows == 1 && IN > 0 && IN % 256 == 0 && OUT > 0 &&
           OUT % (nsg * rs) == 0;
}

rwkv_status rwkv_sb6_gemv(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                          const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, void* stream) {
    RWKV_REQUIRE(x && qblk && qsqm && ddm && y, RWKV_E_NULL, "sb6_gemv: null buffer");
    RWKV_REQUIRE(xbits >= 0 && xbits <= 2, RWKV_E_SHAPE, "sb6_gemv: xbits %d outside 0...2", xbits);
    RWKV_REQUIRE(N >= 1 && N <= INT32_MAX, RWKV_E_SHAPE, "sb6_gemv: rows %lld", (long long)N);
    RWKV_REQUIRE(OUT >= 1 && OUT <= INT32_MAX && IN >= 256 && IN % 256 == 0 && IN <= (1 << 24), RWKV_E_SHAPE,
                 "sb6_gemv: shape %lldx%lld not taken (IN %% 256 == 0 required)", (long long)OUT, (long long)IN);
    const GemvGeom geo = pick_geom(OUT, IN / 32, OUT);
    const int64_t per_block = (int64_t)geo.WPB * geo.R * geo.RL;
    dim3 grid((unsigned)((OUT + per_block - 1) / per_block)), block(64 * geo.WPB);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int nt = pick_nt(N);
#define RWKV_GV(XB, RL, NT) \
    rwkv::launch(sb6_gemv_kernel<XB, RL, NT>, grid, block, st, x, (int)N, qblk, qsqm, ddm, y, (int)OUT, (int)IN, geo)
#define RWKV_GV_NT(XB, RL)                  \
    if (nt == 4) RWKV_GV(XB, RL, 4);        \
    else if (nt == 2) RWKV_GV(XB, RL, 2);   \
    else RWKV_GV(XB, RL, 1);
#define RWKV_GV_RL(XB)                                                       \
    if (geo.RL == 4) { RWKV_GV_NT(XB, 4) } else if (geo.RL == 2) { RWKV_GV_NT(XB, 2) } else { RWKV_GV_NT(XB, 1) }
    switch (xbits) {
        case 0: RWKV_GV_RL(0) break;
        case 1: RWKV_GV_RL(1) break;
        default: RWKV_GV_RL(2) break;
    }
#undef RWKV_GV_RL
#undef RWKV_GV_NT
#undef RWKV_GV
    rwkv_status s = launch_status("sb6_gemv launch");
    if (s == RWKV_OK) rwkv::counters().sb6_gemv++;
    return s;
}

int rwkv_sym_gemv_applies(int64_t OUT, int64_t IN, int bits, int64_t rows) {
    // rwkvqSymGEMVApplies (RwkvqSymGEMV.swift:213-218): NSG = RS = 4, NB_MAX = 4.
    return (bits == 6 || bits == 8) && IN > 0 && IN % 256 == 0 && OUT > 0 && OUT % 16 == 0 && rows >= 1 && rows <= 4;
}

rwkv_status rwkv_sym_gemv(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                          float* y, int64_t OUT, int64_t IN, int bits, int64_t out_per, void* stream) {
    RWKV_REQUIRE(x && qblk && qs && d && y, RWKV_E_NULL, "sym_gemv: null buffer");
    RWKV_REQUIRE(bits == 6 || bits == 8, RWKV_E_SHAPE, "sym_gemv: bits %d outside {6, 8}", bits);
    RWKV_REQUIRE(N >= 1 && N <= INT32_MAX, RWKV_E_SHAPE, "sym_gemv: rows %lld", (long long)N);
    RWKV_REQUIRE(OUT >= 1 && OUT <= INT32_MAX && IN >= 256 && IN % 256 == 0 && IN <= (1 << 24), RWKV_E_SHAPE,
                 "sym_gemv: shape %lldx%lld not taken (IN %% 256 == 0 required)", (long long)OUT, (long long)IN);
    RWKV_REQUIRE(out_per >= 1 && OUT % out_per == 0, RWKV_E_SHAPE,
                 "sym_gemv: %lld rows do not split into matrices of %lld", (long long)OUT, (long long)out_per);
    const GemvGeom geo = pick_geom(OUT, IN / 32, out_per);
    const int64_t per_block = (int64_t)geo.WPB * geo.R * geo.RL;
    dim3 grid((unsigned)((OUT + per_block - 1) / per_block)), block(64 * geo.WPB);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int nt = pick_nt(N);
#define RWKV_GV(BITS, RL, NT)                                                                                   \
    rwkv::launch(sym_gemv_kernel<BITS, RL, NT>, grid, block, st, x, (int)N, qblk, qs, d, y, (int)OUT, \
                       (int)IN, (int)out_per, geo)
#define RWKV_GV_NT(BITS, RL)                  \
    if (nt == 4) RWKV_GV(BITS, RL, 4);        \
    else if (nt == 2) RWKV_GV(BITS, RL, 2);   \
    else RWKV_GV(BITS, RL, 1);
#define RWKV_GV_RL(BITS)                                                                     \
    if (geo.RL == 4) { RWKV_GV_NT(BITS, 4) } else if (geo.RL == 2) { RWKV_GV_NT(BITS, 2) } else { RWKV_GV_NT(BITS, 1) }
    if (bits == 8) {
        RWKV_GV_RL(8)
    } else {
        RWKV_GV_RL(6)
    }
#undef RWKV_GV_RL
#undef RWKV_GV_NT
#undef RWKV_GV
    rwkv_status s = launch_status("sym_gemv launch");
    if (s == RWKV_OK) {
        if (out_per < OUT) rwkv::counters().sym_fused++;
        else rwkv::counters().sym_gemv++;
    }
    return s;
}

}  // extern "C"
