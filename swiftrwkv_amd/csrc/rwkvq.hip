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
// GEMV (decode) mapping.  A row of IN columns is a sequence of NU "units" of
// 32 columns (sb6: one block; sym: two blocks).  G lanes (the largest power of
// two ≤ 64 dividing NU) cover one row; a lane owns RL consecutive rows and, of
// each, the units g, g+G, ...  All of a lane's weight loads are issued before
// any is used (RL·KU loads of 16–32 B in flight per lane); meanwhile the
// workgroup stages its input rows in LDS (padded so the G lanes of a row group
// read distinct banks) together with per-unit input sums.  A unit's 32 inputs
// then stay in registers for the lane's RL rows ("x-stationary").  At fixed
// (unit, row) the G lanes read G consecutive units, so each wave-wide load
// covers whole 128-byte lines.  Codes are widened to fp32 (4-bit sb6 codes two
// per instruction through the fp8 converter), dotted with x in fp32, and
// scaled once per block:
//   sb6:  Σ (q·s + m)·x = s·Σ q·x + m·Σ x      (RwkvqSb6GEMV.swift:118-144)
//   sym6: Σ (q−32)·s·x = s·(Σ q·x − 32·Σ x)    (RwkvqSymGEMV.swift:182-194)
// and the per-lane partial sums are reduced over the G lanes with a fixed
// butterfly.  Up to 4 input rows (batched decode) share one weight pass; more
// rows are processed 4 at a time.  All sums have a fixed order: results are
// deterministic.

#include <hip/hip_runtime.h>

#include <type_traits>

#include <algorithm>

#include "launch.h"
#include "lora_in.h"
#include "x070_row.h"

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
// Four threads per (row, block): quarter q writes columns 8q..8q+7 as parts
// p = 2q, 2q + 1, part p covering columns 4p..4p+3 (p < 4: low nibbles of
// word p; p >= 4: high nibbles of word p-4) — so a wave's stores cover 16
// blocks contiguously.  Index math in 32 bits (rows × blocks × 4 < 2^31 is
// checked on the host): one thread per part with a 64-bit division each ran
// at 0.37 of HBM.
template <int DT>
__device__ __forceinline__ void store8(void* out, int64_t idx, const float (&f)[8]) {
    if constexpr (DT == RWKV_F32) {
        float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + idx);
        o[0] = make_float4(f[0], f[1], f[2], f[3]);
        o[1] = make_float4(f[4], f[5], f[6], f[7]);
    } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if constexpr (DT == RWKV_BF16) {
                const uint32_t u = __float_as_uint(f[e]);
                h[e] = ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu))
                           ? ((u >> 16) | 0x40u)
                           : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
            } else {
                h[e] = __builtin_bit_cast(uint16_t, (_Float16)f[e]);
            }
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + idx) =
            make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
}

template <int XB, int DT>
__global__ __launch_bounds__(256) void sb6_dequant_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qsqm, const uint16_t* __restrict__ ddm,
    void* __restrict__ out, int64_t OUT, int64_t IN) {
    constexpr int SUW = 4 + XB;  // 32-bit words per block
    const uint32_t NB = (uint32_t)(IN >> 5), NSB = NB >> 3;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    if (gid >= (uint32_t)OUT * NB * 4u) return;
    const uint32_t q = gid & 3u, rb = gid >> 2;   // quarter, row * NB + blk
    const uint32_t row = rb / NB, blk = rb - row * NB;
    const uint32_t* qb = reinterpret_cast<const uint32_t*>(qblk) + (int64_t)rb * SUW;
    const uint32_t w0 = qb[2 * (q & 1)], w1 = qb[2 * (q & 1) + 1];   // words of parts 2q, 2q + 1
    const uint32_t h1 = XB >= 1 ? qb[4] : 0u, h2 = XB >= 2 ? qb[5] : 0u;
    const uint16_t sm = reinterpret_cast<const uint16_t*>(qsqm)[rb];
    const uint32_t dd = reinterpret_cast<const uint32_t*>(ddm)[(int64_t)row * NSB + (blk >> 3)];
    const float s = hround((float)(sm & 0xffu) * f16f(dd));
    const float m = hround((float)(int8_t)(sm >> 8) * f16f(dd >> 16));
    float f[8];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int p = 2 * (int)q + e;
        const uint32_t wd = e ? w1 : w0;
        uint32_t q4 = (p < 4) ? (wd & 0x0F0F0F0Fu) : ((wd >> 4) & 0x0F0F0F0Fu);
        if constexpr (XB >= 1) q4 |= spread4((h1 >> (4 * p)) & 0xFu) << 4;
        if constexpr (XB >= 2) q4 |= spread4((h2 >> (4 * p)) & 0xFu) << 5;
        f[4 * e] = fmaf((float)(q4 & 0xffu), s, m);
        f[4 * e + 1] = fmaf((float)((q4 >> 8) & 0xffu), s, m);
        f[4 * e + 2] = fmaf((float)((q4 >> 16) & 0xffu), s, m);
        f[4 * e + 3] = fmaf((float)(q4 >> 24), s, m);
    }
    store8<DT>(out, (int64_t)row * IN + blk * 32 + 8 * q, f);
}

// ─────────────────────────────── sym dequant ───────────────────────────────
// 8-bit: one thread per 4 columns.  6-bit: one thread per (pair, part p),
// part p = columns 4p..4p+3 of the pair in register order l0,l1,h0,h1,l2,l3,h2,h3.
// With `ids` (n rows): output row o is matrix row ids[o] (the embedding row
// gather); an id outside [0, OUT) gives a row of NaN.  I32: the thread index
// and the row division in 32 bits (fewer than 2^31 threads; a 64-bit
// division per 4 outputs costs more than their loads).
template <int BITS, int DT, bool I32>
__global__ __launch_bounds__(256) void sym_dequant_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d,
    void* __restrict__ out, int64_t OUT, int64_t IN, const int32_t* __restrict__ ids, int64_t n) {
    const int64_t NB = IN >> 4, NSB = (NB + 15) >> 4;
    const int64_t rows = ids ? n : OUT;
    int64_t orow, col;
    if constexpr (I32) {
        const uint32_t gid = blockIdx.x * 256u + threadIdx.x, q = (uint32_t)(IN >> 2);
        if (gid >= (uint32_t)(rows * (IN >> 2))) return;
        const uint32_t o = gid / q;
        orow = o;
        col = (int64_t)(gid - o * q) * 4;
    } else {
        const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (gid >= rows * (IN >> 2)) return;
        orow = gid / (IN >> 2);
        col = (gid - orow * (IN >> 2)) * 4;
    }
    int64_t row = orow;
    if (ids) {
        row = ids[orow];
        if (row < 0 || row >= OUT) {
            const float nan = __int_as_float(0x7fc00000);
            store4<DT>(out, orow * IN + col, nan, nan, nan, nan);
            return;
        }
    }
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
    store4<DT>(out, orow * IN + col, f[0], f[1], f[2], f[3]);
}

// ─────────────────────────────── GEMV ───────────────────────────────
// Byte E of w as a float (v_cvt_f32_ubyteE).  Written out: for a masked word
// the compiler folds (w >> 8E) & 0xff into a bit-field extract + convert.
template <int E>
__device__ __forceinline__ float ubyte(uint32_t w) {
    float r;
    if constexpr (E == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (E == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (E == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
    return r;
}

__device__ __forceinline__ void bytes4(uint32_t w, float* c) {
    c[0] = ubyte<0>(w); c[1] = ubyte<1>(w); c[2] = ubyte<2>(w); c[3] = ubyte<3>(w);
}

// Four codes 0..15, one per byte, widened two per instruction as fp8 (E4M3)
// values: the byte 0000nnnn decodes to n·u with u = the value of byte 0x01
// (subnormals continue the first binade linearly), so c = code·u exactly.
__device__ __forceinline__ void nibbles4_fp8(uint32_t w, float* c) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    c[0] = lo[0]; c[1] = lo[1]; c[2] = hi[0]; c[3] = hi[1];
}

// Σ c[i]·x[i] over 32 columns as two 16-column chains, (cols 0..15) + (16..31).
__device__ __forceinline__ float dot32(const float (&c)[32], const float (&x)[32]) {
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        d0 = fmaf(c[i], x[i], d0);
        d1 = fmaf(c[16 + i], x[16 + i], d1);
    }
    return d0 + d1;
}

// Formats.  A unit is 32 columns of one row; `Raw` is what a lane loads for
// one (row, unit); `accumulate` adds the unit's contribution for NT inputs.
// xs[nn] = (Σ x cols 0..15, Σ x cols 16..31) of the unit.
template <int XB>
struct Sb6Fmt {
    static constexpr int WORDS = 4 + XB;
    static constexpr bool SUMS = true;
    static constexpr bool WIDE = XB > 0;   // codes wider than 4 bits: more registers per unit
    struct Ptr {
        const uint32_t* q;
        const uint16_t* sm;
        const uint32_t* dd;
    };
    struct Raw {
        uint32_t w[WORDS];
        uint32_t s0, s1;   // (qs, qm) pair; (d, dm) pair
    };
    // 32-bit byte offsets from the (uniform) buffer bases: the packed
    // matrix is below 4 GiB (checked by the host).
    __device__ static void load(const Ptr& p, int NU, uint32_t row, uint32_t u, Raw& r) {
        const uint32_t ru = row * (uint32_t)NU + u;
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(p.q) + ru * (WORDS * 4u));
#pragma unroll
        for (int m = 0; m < WORDS; ++m) r.w[m] = qb[m];
        r.s0 = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p.sm) + ru * 2u);
        r.s1 = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(p.dd) +
                                                  (row * (uint32_t)(NU >> 3) + (u >> 3)) * 4u);
    }
    // Codes of the unit; for XB == 0 they come out scaled by the fp8 unit u.
    __device__ static void codes(const Raw& r, float (&c)[32]) {
        if constexpr (XB == 0) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                nibbles4_fp8(r.w[m] & 0x0F0F0F0Fu, &c[4 * m]);
                nibbles4_fp8((r.w[m] >> 4) & 0x0F0F0F0Fu, &c[16 + 4 * m]);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                uint32_t q = (m < 4) ? (r.w[m] & 0x0F0F0F0Fu) : ((r.w[m - 4] >> 4) & 0x0F0F0F0Fu);
                q |= spread4((r.w[4] >> (4 * m)) & 0xFu) << 4;
                if constexpr (XB >= 2) q |= spread4((r.w[5] >> (4 * m)) & 0xFu) << 5;
                bytes4(q, &c[4 * m]);
            }
        }
    }
    // A unit decoded once for several inputs: codes and the two scales.
    // inv = 1/u for XB == 0 (a power of two: the scaled and the plain
    // computation round identically), 1 otherwise.
    struct Prep {
        float c[32];
        float s, m;
    };
    __device__ static void prep(const Raw& r, float inv, Prep& q) {
        codes(r, q.c);
        q.s = hround((float)(r.s0 & 0xffu) * f16f(r.s1)) * inv;
        q.m = hround((float)(int8_t)(r.s0 >> 8) * f16f(r.s1 >> 16));
    }
    __device__ static float apply(const Prep& q, const float (&xv)[32], const float (&xs)[2], float acc) {
        return fmaf(q.m, xs[0] + xs[1], fmaf(q.s, dot32(q.c, xv), acc));
    }
    template <int NT>
    __device__ static void accumulate(const Raw& r, float inv, const float (&xv)[NT][32], const float (&xs)[NT][2],
                                      float (&acc)[NT]) {
        Prep q;
        prep(r, inv, q);
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) acc[nn] = apply(q, xv[nn], xs[nn], acc[nn]);
    }
};

template <int BITS>
struct SymFmt {
    static constexpr int WORDS = BITS == 8 ? 8 : 6;
    static constexpr bool SUMS = BITS == 6;
    static constexpr bool WIDE = true;
    struct Ptr {
        const uint32_t* q;
        const uint16_t* qs;   // two int8 block scales per unit
        const uint16_t* d;
    };
    struct Raw {
        uint32_t w[WORDS];
        uint32_t s0, s1;   // two int8 block scales; super-block scale (fp16)
    };
    __device__ static void load(const Ptr& p, int NU, uint32_t row, uint32_t u, Raw& r) {
        const uint32_t ru = row * (uint32_t)NU + u;
        const uint32_t* qb = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(p.q) + ru * (WORDS * 4u));
#pragma unroll
        for (int m = 0; m < WORDS; ++m) r.w[m] = qb[m];
        r.s0 = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p.qs) + ru * 2u);
        r.s1 = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p.d) +
                                                  (row * (uint32_t)(NU >> 3) + (u >> 3)) * 2u);
    }
    struct Prep {
        float c[32];
        float s0, s1;   // block scales of columns 0..15 and 16..31
    };
    __device__ static void prep(const Raw& r, float, Prep& q) {
        const float dsb = f16f(r.s1);
        q.s0 = hround((float)(int8_t)(r.s0 & 0xffu) * dsb);
        q.s1 = hround((float)(int8_t)(r.s0 >> 8) * dsb);
        if constexpr (BITS == 8) {
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) q.c[4 * m + e] = (float)(int8_t)(r.w[m] >> (8 * e));
        } else {
            // register order l0,l1,h0,h1 | l2,l3,h2,h3 → columns 4m..4m+3; codes +32
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const uint32_t wd = r.w[(m >> 2) * 2 + (m & 1)];
                uint32_t q4 = (m & 2) ? ((wd >> 4) & 0x0F0F0F0Fu) : (wd & 0x0F0F0F0Fu);
                q4 |= spread4((r.w[4] >> (4 * m)) & 0xFu) << 4;
                q4 |= spread4((r.w[5] >> (4 * m)) & 0xFu) << 5;
                bytes4(q4, &q.c[4 * m]);
            }
        }
    }
    __device__ static float apply(const Prep& q, const float (&xv)[32], const float (&xs)[2], float acc) {
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            d0 = fmaf(q.c[i], xv[i], d0);
            d1 = fmaf(q.c[16 + i], xv[16 + i], d1);
        }
        if constexpr (BITS == 8) return fmaf(q.s1, d1, fmaf(q.s0, d0, acc));
        return fmaf(q.s1, fmaf(-32.0f, xs[1], d1), fmaf(q.s0, fmaf(-32.0f, xs[0], d0), acc));
    }
    template <int NT>
    __device__ static void accumulate(const Raw& r, float inv, const float (&xv)[NT][32], const float (&xs)[NT][2],
                                      float (&acc)[NT]) {
        Prep q;
        prep(r, inv, q);
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) acc[nn] = apply(q, xv[nn], xs[nn], acc[nn]);
    }
};

// Σ of v over each aligned group of G lanes (G a power of two ≤ 64), in every
// lane of the group: DPP butterflies within 16-lane rows (quad swaps, then the
// half-row and row mirrors pair disjoint halves), then lane swaps across rows.
template <int CTRL>
__device__ __forceinline__ float dpp_pair(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// v_l + v_(l^16) (v_l + v_(l^32)) from a lane swap across DPP rows (halves):
// each lane adds the same two values, so the sum is the xor-partner add's.
__device__ __forceinline__ float swap16_add(float v) {
    float a = v, b = v;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float swap32_add(float v) {
    float a = v, b = v;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float group_sum(float v, int G) {
    if (G >= 2) v += dpp_pair<0xB1>(v);    // quad_perm [1,0,3,2]
    if (G >= 4) v += dpp_pair<0x4E>(v);    // quad_perm [2,3,0,1]
    if (G >= 8) v += dpp_pair<0x141>(v);   // row_half_mirror
    if (G >= 16) v += dpp_pair<0x140>(v);  // row_mirror
    if (G >= 32) v = swap16_add(v);        // lanes l, l ^ 16
    if (G >= 64) v = swap32_add(v);        // lanes l, l ^ 32
    return v;
}

struct GemvGeom {
    int G;     // lanes per row (power of two)
    int LG;    // log2(G)
    int R;     // row groups per wave (64 / G)
    int NP;    // passes: a lane covers units (p·KU + ku)·G + g, p < NP, ku < KU
    int WPB;   // waves per workgroup
    int one_k; // fused groups: every row of a workgroup reads the same input row, staged alone
    int ep;    // epilogue: 0 store, 1 add to y (residual stream), 2 relu² of the result
    int xfirst;   // single input: inputs loaded before the weights (gemv_kernel<..., XF = true>)
    // with the store of output row `row` (one input, OUT = the copied width):
    // cp_dst[row] ← cp_src[row] (a state row handed on after every reader of
    // the old one has run); null: none
    const float* cp_src;
    float* cp_dst;
};

// A GEMV input row formed in the launch: LN(x) with (w, b), then the token
// shift lerp with the previous row `prev` and coefficient row `coef`
// (X070Generation.swift tmixStep :214-239 / cmixStep :303-308), in the row
// kernels' exact arithmetic (x070_row.h).  `xln` (nullable) receives LN(x)
// from one workgroup, for a later launch to store as the next `prev`.
struct LnMix {
    const float* x;
    const float* w;
    const float* b;
    const float* prev;
    const float* coef;   // coefficient rows; a fused group's matrix k uses row k
    float* xln;
    float eps;
};

// y[i] ← t, res + t (res = y[i], read before the product) or relu(t)², the
// separate operations' exact arithmetic.
__device__ __forceinline__ void store_out(float* __restrict__ y, int64_t i, float t, int ep, float res) {
    if (ep == 1) {
        t = res + t;
    } else if (ep == 2) {
        t = fmaxf(t, 0.0f);
        t = t * t;
    }
    y[i] = t;
}
__device__ __forceinline__ void store_out(float* __restrict__ y, int64_t i, float t, int ep) {
    store_out(y, i, t, ep, ep == 1 ? y[i] : 0.0f);
}

// Padded LDS row: column c at c + 4·(c / 32), so the G lanes of a row group
// reading G different units with ds_read_b128 hit distinct banks.
__host__ __device__ constexpr int xl_stride(int IN) { return IN + (IN >> 3); }

// y[n, row] = Σ_c W[row, c] · x[n·NK + row / out_per, c].  A lane owns RL
// consecutive rows and, for each, the units (p·KU + ku)·G + g; all RL·KU units
// of a pass are loaded before any is used, so every lane keeps RL·KU
// 16–32-byte loads in flight.  With `xl` the workgroup first stages its input
// rows (and per-unit sums) in LDS while those loads are outstanding, and the
// weights stay in registers across input tiles.
// The body of workgroup `bx` (gemv_kernel runs workgroup blockIdx.x; a fused
// launch may run it beside other work).
template <class F, int RL, int KU, int NT, bool XL, bool MULTI, bool XF, int LNC = 0>
__device__ __forceinline__ void gemv_body(int bx, const float* __restrict__ x, int N, typename F::Ptr P,
                                          float* __restrict__ y, int OUT, int IN, int out_per, GemvGeom geo,
                                          const LnMix& lm = LnMix{}) {
    extern __shared__ float lds[];
    const int NU = IN >> 5;
    const int NK = OUT / out_per;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // every launch of this body has 64·WPB threads; a constant instead of
    // blockDim.x, whose code-object-v5 read is a vector load that would queue
    // behind the weight loads
    const int nthr = 64 * geo.WPB;
    const int gi = lane >> geo.LG, g = lane & (geo.G - 1);
    const int row0 = (bx * geo.WPB + wave) * geo.R * RL + gi * RL;
    const bool live = row0 < OUT;
    const int xi = NK == 1 ? 0 : (live ? row0 : OUT - 1) / out_per;   // RL divides out_per
    float inv = 1.0f;
    if constexpr (std::is_same_v<F, Sb6Fmt<0>>) {
        // exact reciprocal of the fp8 unit (a power of two): negate the exponent
        inv = __uint_as_float(0x7F000000u - __float_as_uint(__builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0]));
    }

    using Raw = typename F::Raw;
    auto load_pass = [&](int p, Raw (&W)[RL][KU]) {
#pragma unroll
        for (int rr = 0; rr < RL; ++rr) {
            const uint32_t row = (uint32_t)min(row0 + rr, OUT - 1);
#pragma unroll
            for (int ku = 0; ku < KU; ++ku) F::load(P, NU, row, (uint32_t)((p * KU + ku) * geo.G + g), W[rr][ku]);
        }
    };
    const int XS = xl_stride(IN);
    const int NKs = geo.one_k ? 1 : NK;   // staged input rows per input
    const float* xsum = lds + NT * NKs * XS;
    // A single input staged weights-first (a launch of few workgroups, bound by
    // its round trips): each lane forms its units' Σx from the 32 inputs it
    // reads, instead of a sums pass and a barrier after the staging.
    constexpr bool LANE_SUMS = NT == 1 && !XF;
    auto compute_pass = [&](int p, const Raw (&W)[RL][KU], int n0, float (&acc)[NT][RL]) {
#pragma unroll
        for (int ku = 0; ku < KU; ++ku) {
            // One unit's inputs live at a time (scheduling barrier).
            if (ku) asm volatile("" ::: "memory");
            const int u = (p * KU + ku) * geo.G + g;
            float xv[NT][32], xs[NT][2];
#pragma unroll
            for (int nn = 0; nn < NT; ++nn) {
                if constexpr (XL) {
                    const int j = nn * NKs + (geo.one_k ? 0 : xi);
                    const float4* px = reinterpret_cast<const float4*>(lds + j * XS + u * 36);
#pragma unroll
                    for (int m = 0; m < 8; ++m) {
                        const float4 f = px[m];
                        xv[nn][4 * m] = f.x; xv[nn][4 * m + 1] = f.y; xv[nn][4 * m + 2] = f.z; xv[nn][4 * m + 3] = f.w;
                    }
                    if constexpr (F::SUMS) {
                        if constexpr (LANE_SUMS) {   // the staged sums' order: bitwise the same
                            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                            for (int c = 0; c < 16; ++c) { s0 += xv[nn][c]; s1 += xv[nn][16 + c]; }
                            xs[nn][0] = s0; xs[nn][1] = s1;
                        } else {
                            const float2 s = reinterpret_cast<const float2*>(xsum)[j * NU + u];
                            xs[nn][0] = s.x; xs[nn][1] = s.y;
                        }
                    }
                } else {
                    const int n = min(n0 + nn, N - 1);
                    const float4* px = reinterpret_cast<const float4*>(x + ((int64_t)n * NK + xi) * IN + u * 32);
#pragma unroll
                    for (int m = 0; m < 8; ++m) {
                        const float4 f = px[m];
                        xv[nn][4 * m] = f.x; xv[nn][4 * m + 1] = f.y; xv[nn][4 * m + 2] = f.z; xv[nn][4 * m + 3] = f.w;
                    }
                    if constexpr (F::SUMS) {
                        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                        for (int c = 0; c < 16; ++c) { s0 += xv[nn][c]; s1 += xv[nn][16 + c]; }
                        xs[nn][0] = s0; xs[nn][1] = s1;
                    }
                }
            }
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                float a[NT];
#pragma unroll
                for (int nn = 0; nn < NT; ++nn) a[nn] = acc[nn][rr];
                F::template accumulate<NT>(W[rr][ku], inv, xv, xs, a);
#pragma unroll
                for (int nn = 0; nn < NT; ++nn) acc[nn][rr] = a[nn];
            }
        }
    };
    // the residual of the add epilogue, read while the weights stream
    // (and the state row a copy epilogue hands on: read here, with the
    // weights in flight, not after the products)
    float cpv[RL];
    auto load_res = [&](float (&res)[NT][RL], int n0) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                const int row = row0 + rr;
                res[nn][rr] = (geo.ep == 1 && g == 0 && row < OUT && n0 + nn < N) ? y[(int64_t)(n0 + nn) * OUT + row]
                                                                                 : 0.0f;
            }
#pragma unroll
        for (int rr = 0; rr < RL; ++rr) {
            const int row = row0 + rr;
            cpv[rr] = (geo.cp_dst && g == 0 && row < OUT) ? geo.cp_src[row] : 0.0f;
        }
    };
    auto store = [&](float (&acc)[NT][RL], int n0, const float (&res)[NT][RL]) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                const float t = group_sum(acc[nn][rr], geo.G);
                const int row = row0 + rr;
                if (g == 0 && row < OUT && n0 + nn < N) {
                    store_out(y, (int64_t)(n0 + nn) * OUT + row, t, geo.ep, res[nn][rr]);
                    if (geo.cp_dst && n0 + nn == 0) geo.cp_dst[row] = cpv[rr];
                }
            }
    };

    auto zero = [&](float (&acc)[NT][RL]) {
#pragma unroll
        for (int nn = 0; nn < NT; ++nn)
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) acc[nn][rr] = 0.0f;
    };
    if constexpr (XL) {
        Raw W[RL][KU];
        float acc[NT][RL], res[NT][RL];
        const int rows = NT * NKs;   // one tile: N <= NT
        // matrix of the workgroup's rows when they all read one input row
        const int kwg = geo.one_k ? (int)(bx * geo.WPB * geo.R * RL) / out_per : 0;
        auto row_src = [&](int j) {   // staged row j
            const int nn = NKs == 1 ? j : j / NKs, k = geo.one_k ? kwg : j - nn * NK;
            return x + ((int64_t)min(nn, N - 1) * NK + k) * IN;
        };
        auto row_sums = [&]() {
            if constexpr (F::SUMS) {
                // sums[j][u][h] = x[j, 32u + 16h + 0..15], added in column order
                float* sums = lds + NT * NKs * XS;
#pragma unroll 1
                for (int j = 0; j < rows; ++j)
#pragma unroll 1
                    for (int i = threadIdx.x; i < NU * 2; i += nthr) {
                        const float4* px = reinterpret_cast<const float4*>(lds + j * XS + (i >> 1) * 36 + 16 * (i & 1));
                        float sum = 0.0f;
#pragma unroll
                        for (int m = 0; m < 4; ++m) {
                            const float4 f = px[m];
                            sum += f.x; sum += f.y; sum += f.z; sum += f.w;
                        }
                        sums[j * NU * 2 + i] = sum;
                    }
                __syncthreads();
            }
        };
        if constexpr (LNC > 0) {
            // The input row formed here: LN(x) and its token-shift lerp.  All
            // the row loads first (the lane's statistics chunks of the whole
            // row, row_chunks, then this thread's LNC staging chunks
            // e = tid + i·nthr), then the weights; one input row (rows == 1),
            // IN ≤ 4·LNC·nthr, LNC ≤ 2 and IN ≤ 4096 (checked by the host).
            using namespace rwkv_x070;
            const int IN4 = IN >> 2;
            float4 sv[8], xo[LNC], pv[LNC], cv[LNC], wv[LNC], bv[LNC];
            const float* coef = lm.coef + (int64_t)kwg * IN;
            row_chunks<8>(lm.x, IN, lane, sv);
#pragma unroll
            for (int i = 0; i < LNC; ++i) {
                const int e = min((int)threadIdx.x + i * nthr, IN4 - 1);
                xo[i] = *reinterpret_cast<const float4*>(lm.x + 4 * e);
                pv[i] = *reinterpret_cast<const float4*>(lm.prev + 4 * e);
                cv[i] = *reinterpret_cast<const float4*>(coef + 4 * e);
                wv[i] = *reinterpret_cast<const float4*>(lm.w + 4 * e);
                bv[i] = *reinterpret_cast<const float4*>(lm.b + 4 * e);
            }
            load_pass(0, W);
            load_res(res, 0);
            const float2 md = row_stats<8>(sv, lm.x, IN, lane, lm.eps);
            // chunks past the row repeat the last one (the same values to the
            // same addresses): no branch, so the row loads stay ahead of the
            // weight loads instead of being sunk behind them
#pragma unroll
            for (int i = 0; i < LNC; ++i) {
                const int e = min((int)threadIdx.x + i * nthr, IN4 - 1);
                const float4 xl = ln_apply(xo[i], md, wv[i], bv[i]);
                *reinterpret_cast<float4*>(lds + e * 4 + (e >> 3) * 4) = shift_lerp(xl, shift_delta(pv[i], xl), cv[i]);
                if (bx == 0 && lm.xln) *reinterpret_cast<float4*>(lm.xln + 4 * e) = xl;
            }
            __syncthreads();
            row_sums();
            __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (XF) {
            // Inputs first: the first XPRE float4 of each thread's share of
            // the staged rows are loaded before the weights.  Loads complete
            // in issue order, so the LDS stores then wait for these inputs,
            // not for the weights, and staging and sums run while the weights
            // stream (a bandwidth-bound launch's workgroups otherwise hold
            // their staging until their weights arrive).
            using v4 = float __attribute__((ext_vector_type(4)));
            const int IN4 = IN >> 2, total4 = rows * IN4;
            auto split = [&](int e, int& j, int& q) {   // float4 e → (row j, float4 q)
                if (rows == 1) {
                    j = 0; q = e;
                } else {
                    j = e / IN4; q = e - j * IN4;
                }
            };
            auto src4 = [&](int j, int q) { return reinterpret_cast<const v4*>(row_src(j)) + q; };
            auto dst4 = [&](int j, int q) { return reinterpret_cast<v4*>(lds + j * XS + q * 4 + (q >> 3) * 4); };
            constexpr int XPRE = 4;
            v4 xp[XPRE];
#pragma unroll
            for (int i = 0; i < XPRE; ++i) {
                const int e = (int)threadIdx.x + i * nthr;
                int j, q;
                split(e, j, q);
                v4 t = {};
                if (e < total4) t = *src4(j, q);
                xp[i] = t;
            }
            load_pass(0, W);
            load_res(res, 0);
#pragma unroll
            for (int i = 0; i < XPRE; ++i) {
                const int e = (int)threadIdx.x + i * nthr;
                if (e < total4) {
                    int j, q;
                    split(e, j, q);
                    *dst4(j, q) = xp[i];
                }
            }
#pragma unroll 1
            for (int e = (int)threadIdx.x + XPRE * nthr; e < total4; e += nthr) {
                int j, q;
                split(e, j, q);
                *dst4(j, q) = *src4(j, q);
            }
            __syncthreads();
            row_sums();
            // the weights' decode stays after the barriers
            __builtin_amdgcn_sched_barrier(0);
        } else {
            load_pass(0, W);   // in flight while the inputs are staged
            load_res(res, 0);
            const int step = nthr * 4;
#pragma unroll 1
            for (int j = 0; j < rows; ++j) {   // uniform
                const float* src = row_src(j);
#pragma unroll 1
                for (int c = (int)threadIdx.x * 4; c < IN; c += step)
                    *reinterpret_cast<float4*>(lds + j * XS + c + (c >> 5) * 4) =
                        *reinterpret_cast<const float4*>(src + c);
            }
            __syncthreads();
            if constexpr (!LANE_SUMS) row_sums();
        }
        zero(acc);
        if constexpr (MULTI) {
            for (int p = 0; p < geo.NP; ++p) {
                if (p + 1 < geo.NP) {
                    Raw Wn[RL][KU];
                    load_pass(p + 1, Wn);   // next pass in flight during this one
                    compute_pass(p, W, 0, acc);
#pragma unroll
                    for (int rr = 0; rr < RL; ++rr)
#pragma unroll
                        for (int ku = 0; ku < KU; ++ku) W[rr][ku] = Wn[rr][ku];
                } else {
                    compute_pass(p, W, 0, acc);
                }
            }
        } else {
            compute_pass(0, W, 0, acc);   // NP == 1
        }
        store(acc, 0, res);
    } else {
        for (int n0 = 0; n0 < N; n0 += NT) {
            float acc[NT][RL], res[NT][RL];
            load_res(res, n0);
            zero(acc);
            for (int p = 0; p < geo.NP; ++p) {
                Raw W[RL][KU];
                load_pass(p, W);
                compute_pass(p, W, n0, acc);
            }
            store(acc, n0, res);
        }
    }
}

template <class F, int RL, int KU, int NT, bool XL, bool MULTI, bool XF = false>
__global__ __launch_bounds__(NT == 1 ? 1024 : 256) void gemv_kernel(const float* __restrict__ x, int N, typename F::Ptr P,
                                                   float* __restrict__ y, int OUT, int IN, int out_per, GemvGeom geo) {
    gemv_body<F, RL, KU, NT, XL, MULTI, XF>((int)blockIdx.x, x, N, P, y, OUT, IN, out_per, geo);
}

// The fused r/k/v GEMV of an x070 layer (one input row, sb6 4-bit) and the
// layer's low-rank first layers (fp16 matrices) in one launch: both read only
// the token-shift mixes, and each alone leaves most of the GPU idle at small
// widths.  The first `lb` workgroups run one lora_in job per wave (the same
// arithmetic as lora_in_kernel), dispatched first so they overlap the GEMV
// when its workgroups fill the GPU; the rest are gemv_kernel's workgroups
// (the same code, so y is bitwise the separate launch's).
template <int RL, int KU, bool XF>
__global__ __launch_bounds__(1024) void rkv_lora_kernel(const float* __restrict__ x, typename Sb6Fmt<0>::Ptr P,
                                                        float* __restrict__ y, int OUT, int IN, int out_per,
                                                        GemvGeom geo, int lb, const float* __restrict__ xmix,
                                                        const void* __restrict__ wcat, float* __restrict__ la, int rw,
                                                        int ra, int rv, int rg, int with_v) {
    if ((int)blockIdx.x >= lb) {   // uniform per workgroup
        gemv_body<Sb6Fmt<0>, RL, KU, 1, true, false, XF>((int)blockIdx.x - lb, x, 1, P, y, OUT, IN, out_per, geo);
    } else {
        const int64_t job = (int64_t)blockIdx.x * geo.WPB + (threadIdx.x >> 6);
        if (job >= rw + ra + rv + rg) return;   // uniform per wave
        rwkv_x070::lora_in_job<true, 4>(job, threadIdx.x & 63, xmix, wcat, la, IN, rw, ra, rv, rg, with_v);
    }
}

// rkv_lora_kernel forming its inputs itself (LnMix: ln1, the token shift
// and its lerps) instead of reading the shift_mix launch's rows: a GEMV
// workgroup forms the r, k or v row of its matrix, a low-rank workgroup (its
// jobs are rows of one branch: ranks are multiples of 8, WPB divides 8) the
// w, a, v or g row in LDS.  Bitwise the shift_mix + rkv_lora pair.
template <int KU, int LNC>
__global__ __launch_bounds__(1024) void rkv_lora_ln_kernel(typename Sb6Fmt<0>::Ptr P, float* __restrict__ y, int OUT,
                                                           int IN, int out_per, GemvGeom geo, int lb, LnMix lm,
                                                           const void* __restrict__ wcat, float* __restrict__ la,
                                                           int rw, int ra, int rv, int rg, int with_v) {
    if ((int)blockIdx.x >= lb) {   // uniform per workgroup
        gemv_body<Sb6Fmt<0>, 1, KU, 1, true, false, true, LNC>((int)blockIdx.x - lb, lm.x, 1, P, y, OUT, IN, out_per,
                                                               geo, lm);
        return;
    }
    using namespace rwkv_x070;
    extern __shared__ float lds[];
    const int RT = rw + ra + rv + rg, nthr = 64 * geo.WPB, IN4 = IN >> 2;
    const int job = (int)blockIdx.x * geo.WPB + (threadIdx.x >> 6);
    const int br = lora_branch(min((int)blockIdx.x * geo.WPB, RT - 1), rw, ra, rv);   // uniform
    // the job's matrix row first (its first chunk; a wave past the jobs
    // reads row RT − 1), then the input row's loads
    uint4 first[4];
    lora_in_first<true, 4>(min(job, RT - 1), threadIdx.x & 63, wcat, IN, first);
    const float* coef = lm.coef + (int64_t)(br == 0 ? 3 : br == 1 ? 4 : br == 2 ? 2 : 5) * IN;
    float4 sv[8], xo[LNC], pv[LNC], cv[LNC], wv[LNC], bv[LNC];
    row_chunks<8>(lm.x, IN, threadIdx.x & 63, sv);
#pragma unroll
    for (int i = 0; i < LNC; ++i) {
        const int e = min((int)threadIdx.x + i * nthr, IN4 - 1);
        xo[i] = *reinterpret_cast<const float4*>(lm.x + 4 * e);
        pv[i] = *reinterpret_cast<const float4*>(lm.prev + 4 * e);
        cv[i] = *reinterpret_cast<const float4*>(coef + 4 * e);
        wv[i] = *reinterpret_cast<const float4*>(lm.w + 4 * e);
        bv[i] = *reinterpret_cast<const float4*>(lm.b + 4 * e);
    }
    const float2 md = row_stats<8>(sv, lm.x, IN, threadIdx.x & 63, lm.eps);
#pragma unroll
    for (int i = 0; i < LNC; ++i) {   // past the row: the last chunk again, no branch
        const int e = min((int)threadIdx.x + i * nthr, IN4 - 1);
        const float4 xl = ln_apply(xo[i], md, wv[i], bv[i]);
        reinterpret_cast<float4*>(lds)[e] = shift_lerp(xl, shift_delta(pv[i], xl), cv[i]);
    }
    __syncthreads();
    if (job >= RT || (br == 2 && !with_v)) return;   // uniform per wave
    lora_in_row<true, 4>(job, 0, threadIdx.x & 63, lds, wcat, la, IN, RT, br, &first);
}

// The ffn key GEMV (relu² epilogue) forming its input itself (LnMix: ln2,
// the token shift and its lerp); bitwise the shift_mix + GEMV pair.
template <int KU, int LNC>
__global__ __launch_bounds__(1024) void gemv_ln_kernel(typename Sb6Fmt<0>::Ptr P, float* __restrict__ y, int OUT,
                                                       int IN, GemvGeom geo, LnMix lm) {
    gemv_body<Sb6Fmt<0>, 1, KU, 1, true, false, true, LNC>((int)blockIdx.x, lm.x, 1, P, y, OUT, IN, OUT, geo, lm);
}

// Batches (N ≥ 2 inputs): NT inputs share one pass over the weights.  The
// lane → (row, unit) assignment, the per-unit arithmetic (F::prep / F::apply)
// and the group sums are those of gemv_kernel, so every output is bitwise
// what a single-input launch gives.  A unit's codes are decoded once for all
// NT inputs.  blockIdx.y selects the tile of NT inputs.  The inputs are
// staged in LDS a chunk of CP passes (CP·G units) at a time, so any IN fits
// and a workgroup reads each input element once; the next pass's weights are
// in flight during the current one.
template <class F, int RL, int NT>
__global__ __launch_bounds__(512) void gemv_batch_kernel(const float* __restrict__ x, int N, typename F::Ptr P,
                                                         float* __restrict__ y, int OUT, int IN, int out_per,
                                                         GemvGeom geo, int CP) {
    extern __shared__ float lds[];
    const int NU = IN >> 5;
    const int NK = OUT / out_per;
    {
        const int n0 = (int)blockIdx.y * NT;
        x += (int64_t)n0 * NK * IN;
        y += (int64_t)n0 * OUT;
        N = min(NT, N - n0);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gi = lane >> geo.LG, g = lane & (geo.G - 1);
    const int row0 = (blockIdx.x * geo.WPB + wave) * geo.R * RL + gi * RL;
    const int xi = NK == 1 ? 0 : min(row0, OUT - 1) / out_per;   // RL divides out_per
    float inv = 1.0f;
    if constexpr (std::is_same_v<F, Sb6Fmt<0>>) {
        inv = __uint_as_float(0x7F000000u - __float_as_uint(__builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0]));
    }
    // staged input rows: input nn, matrix k at nn·NK + k, or only the
    // workgroup's own matrix kwg (one_k) at nn
    const int NKs = geo.one_k ? 1 : NK;
    const int kwg = geo.one_k ? (int)(blockIdx.x * geo.WPB * geo.R * RL) / out_per : 0;
    const int rows = NT * NKs;
    const int CU = CP * geo.G;     // units per chunk
    const int XS = CU * 36;        // floats per staged row: units padded to 36 floats
    float* const sums = lds + rows * XS;   // [rows][CU][2]: Σ x of columns 0..15, 16..31

    using Raw = typename F::Raw;
    using Prep = typename F::Prep;
    auto load_pass = [&](int p, Raw (&W)[RL]) __attribute__((always_inline)) {
#pragma unroll
        for (int rr = 0; rr < RL; ++rr)
            F::load(P, NU, (uint32_t)min(row0 + rr, OUT - 1), (uint32_t)(p * geo.G + g), W[rr]);
    };
    auto stage = [&](int u0, int nu) __attribute__((always_inline)) {   // units u0 .. u0 + nu - 1
        const int q4 = nu * 8;   // float4 per staged row
        // a thread's float4 of column c4 for 8 rows at a time: 8 loads in flight
#pragma unroll 1
        for (int c4 = threadIdx.x; c4 < q4; c4 += blockDim.x) {
            const int c = c4 * 4, off = c + (c >> 5) * 4;
#pragma unroll 1
            for (int j0 = 0; j0 < rows; j0 += 8) {
                // staged row j = input nn, matrix k is x row j; rows of inputs
                // past N (their outputs are not stored) repeat the last row
                using f4 = float __attribute__((ext_vector_type(4)));
                f4 v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = NKs == 1 && NK > 1 ? min(j0 + e, N - 1) * NK + kwg : min(j0 + e, N * NK - 1);
                    v[e] = *reinterpret_cast<const f4*>(x + (int64_t)j * IN + u0 * 32 + c);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (j0 + e < rows) *reinterpret_cast<f4*>(lds + (j0 + e) * XS + off) = v[e];
            }
        }
        __syncthreads();
        if constexpr (F::SUMS) {
#pragma unroll 1
            for (int i = threadIdx.x; i < rows * nu * 2; i += blockDim.x) {
                const int j = i / (nu * 2), h = i - j * (nu * 2);   // h = 2·unit + half
                const float4* px = reinterpret_cast<const float4*>(lds + j * XS + (h >> 1) * 36 + 16 * (h & 1));
                float sum = 0.0f;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float4 f = px[m];
                    sum += f.x; sum += f.y; sum += f.z; sum += f.w;
                }
                sums[j * CU * 2 + h] = sum;
            }
            __syncthreads();
        }
    };

    float acc[NT][RL];
#pragma unroll
    for (int nn = 0; nn < NT; ++nn)
#pragma unroll
        for (int rr = 0; rr < RL; ++rr) acc[nn][rr] = 0.0f;
    Raw W[RL];
    load_pass(0, W);   // in flight while the first chunk is staged
    int u0 = 0;
#pragma unroll 1
    for (int p = 0; p < geo.NP; ++p) {
        if (p % CP == 0) {   // uniform across the workgroup
            if (p) __syncthreads();   // every wave is done with the previous chunk
            u0 = p * geo.G;
            stage(u0, min(CP, geo.NP - p) * geo.G);
        }
        Raw Wn[RL];
        if (p + 1 < geo.NP) load_pass(p + 1, Wn);
        Prep q[RL];
#pragma unroll
        for (int rr = 0; rr < RL; ++rr) F::prep(W[rr], inv, q[rr]);
        const int lu = p * geo.G + g - u0;
        // inputs nn + 1 are read from LDS while input nn is applied; the fence
        // (it consumes the accumulators and orders memory) keeps at most two
        // inputs' values live
        float xv[2][32], xs[2][2];
        auto read_x = [&](int nn, float (&v)[32], float (&sv)[2]) __attribute__((always_inline)) {
            const int j = nn * NKs + (geo.one_k ? 0 : xi);
            const float4* px = reinterpret_cast<const float4*>(lds + j * XS + lu * 36);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const float4 f = px[m];
                v[4 * m] = f.x; v[4 * m + 1] = f.y; v[4 * m + 2] = f.z; v[4 * m + 3] = f.w;
            }
            if constexpr (F::SUMS) {
                const float2 t = reinterpret_cast<const float2*>(sums)[j * CU + lu];
                sv[0] = t.x; sv[1] = t.y;
            } else {
                sv[0] = sv[1] = 0.0f;
            }
        };
        read_x(0, xv[0], xs[0]);
#pragma unroll
        for (int nn = 0; nn < NT; ++nn) {
            if (nn + 1 < NT) read_x(nn + 1, xv[(nn + 1) & 1], xs[(nn + 1) & 1]);
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) {
                acc[nn][rr] = F::apply(q[rr], xv[nn & 1], xs[nn & 1], acc[nn][rr]);
                asm volatile("" : "+v"(acc[nn][rr]) : : "memory");
            }
        }
        if (p + 1 < geo.NP) {
#pragma unroll
            for (int rr = 0; rr < RL; ++rr) W[rr] = Wn[rr];
        }
    }
#pragma unroll
    for (int nn = 0; nn < NT; ++nn)
#pragma unroll
        for (int rr = 0; rr < RL; ++rr) {
            const float t = group_sum(acc[nn][rr], geo.G);
            const int row = row0 + rr;
            if (g == 0 && row < OUT && nn < N) store_out(y, (int64_t)nn * OUT + row, t, geo.ep);
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

// LDS bytes a workgroup may use for staged inputs: a gfx950 workgroup can
// take the CU's whole 160 KB (e.g. the 14336-wide rows of a 7B-class FFN
// value matrix stage 68 KB; reading them from global memory per lane instead
// ran at 1.2 TB/s against 3.2 TB/s staged).
constexpr size_t kXlBudget = 160 * 1024;

struct GemvPlan {
    GemvGeom geo;
    int RL, KU, NT;
    bool xl;   // inputs staged in LDS (requires NP == 1)
    size_t lds;
    unsigned blocks;
};

// Geometry for an OUT × (32·NU) matrix, N inputs, NK input rows per input
// (fused groups), rows per lane dividing `rl_div`.  One input tile (N ≤ 1): G =
// the smallest power of two ≤ 64 dividing NU with at most 4 units per lane
// (fewer lanes per row: fewer reduction steps per weight), KU = the units per
// lane, and RL·KU up to 4 so each lane keeps several unit loads in flight;
// many small waves hide the memory latency better than few deep ones.  Four
// inputs per tile: KU = 1, RL ≤ 2 (registers).  The inputs go through LDS when one input
// tile covers them and they fit in the LDS budget; callers split larger batches.
GemvPlan plan_gemv(int64_t OUT, int64_t NU, int64_t rl_div, int64_t N, int64_t NK, bool sums, bool wide) {
    GemvPlan pl{};
    pl.NT = N >= 2 ? 4 : 1;
    int64_t G = NU & -NU;   // largest power of two dividing NU
    if (G > 64) G = 64;
    // (independent of the batch, so a row's result does not depend on it)
    while (G > 1 && NU / (G >> 1) <= 4) G >>= 1;
    pl.geo.G = (int)G;
    pl.geo.LG = __builtin_ctzll((unsigned long long)G);
    pl.geo.R = 64 / pl.geo.G;
    const int64_t per_lane = NU / G;
    // all of a lane's units in one pass (KU ≤ 4), else one unit per pass with
    // the next pass prefetched
    pl.KU = (pl.NT == 1 && per_lane <= 4) ? (int)per_lane : 1;
    const int KU = pl.KU;
    pl.geo.NP = (int)(per_lane / KU);
    // Rows per lane (the inputs of a unit stay in registers across them),
    // bounded by registers: RL·KU ≤ 4 (≤ 2 for wider codes), RL ≤ 2 with a
    // prefetched pass (1 for wider codes) or four inputs per tile.
    const int slots = pl.NT == 4 ? 2 : pl.geo.NP > 1 ? (wide ? 1 : 2) : (wide ? 2 : 4);
    pl.RL = (rl_div % 4 == 0 && 4 * KU <= slots) ? 4 : (rl_div % 2 == 0 && 2 * KU <= slots) ? 2 : 1;
    // Waves per workgroup share one staging of the inputs: 8 (one input row;
    // measured best between 4 and 16) while the grid keeps ≥ 256 workgroups,
    // at least 4 (fewer lose more to the staging than they gain in spread).
    pl.geo.WPB = pl.NT == 1 ? 8 : 4;
    auto blocks = [&]() {
        const int64_t per = (int64_t)pl.geo.WPB * pl.geo.R * pl.RL;
        return (OUT + per - 1) / per;
    };
    while (pl.geo.WPB > 4 && blocks() < 256) pl.geo.WPB >>= 1;
    pl.blocks = (unsigned)blocks();
    const int64_t IN = NU * 32;
    // a fused group's workgroups stage only their own matrix's input row when
    // their rows never straddle two matrices (out_per = rl_div)
    pl.geo.one_k = NK > 1 && rl_div % ((int64_t)pl.geo.WPB * pl.geo.R * pl.RL) == 0;
    const int64_t lds = (int64_t)pl.NT * (pl.geo.one_k ? 1 : NK) * (xl_stride((int)IN) + (sums ? NU * 2 : 0)) * 4;
    pl.xl = N <= pl.NT && lds <= (int64_t)kXlBudget;
    if (!pl.xl) {
        // inputs read from global memory: one row per lane keeps registers low
        pl.RL = 1;
        pl.blocks = (unsigned)blocks();
        pl.geo.one_k = 0;
    }
    pl.lds = pl.xl ? (size_t)lds : 0;
    // inputs loaded before the weights where the launch streams enough for
    // the staging latency to matter (a full grid or input rows of 2048 and
    // more: measured faster from 2 MB of weights on); a few workgroups of
    // short rows, bound by one memory round trip, issue their weights first
    pl.geo.xfirst = pl.xl && pl.NT == 1 && (pl.blocks >= 256 || IN >= 2048);
    return pl;
}

// Returns false when the plan names a variant that is not built.
template <class F>
bool launch_gemv(const GemvPlan& pl, hipStream_t st, const float* x, int N, typename F::Ptr P, float* y, int OUT,
                 int IN, int out_per) {
    const dim3 grid(pl.blocks), block(64 * pl.geo.WPB);
    bool launched = false;
    auto go = [&](auto kernel) {
        rwkv::launch_lds(kernel, grid, block, pl.lds, st, x, N, P, y, OUT, IN, out_per, pl.geo);
        launched = true;
    };
    // single input: the inputs-first variant where the plan asks for it
    auto go2 = [&](auto kernel, auto kernel_xfirst) {
        if (pl.geo.xfirst) go(kernel_xfirst);
        else go(kernel);
    };
    const bool multi = pl.geo.NP > 1;
    if (!pl.xl) {
        // inputs from global memory, one row per lane
        if (pl.NT == 4) go(gemv_kernel<F, 1, 1, 4, false, false>);
        else if (pl.KU == 1) go(gemv_kernel<F, 1, 1, 1, false, false>);
        else if (pl.KU == 2) go(gemv_kernel<F, 1, 2, 1, false, false>);
        else if (pl.KU == 3) go(gemv_kernel<F, 1, 3, 1, false, false>);
        else if (pl.KU == 4) go(gemv_kernel<F, 1, 4, 1, false, false>);
    } else if (pl.NT == 4) {
        // KU == 1, RL ≤ 2
        if (multi) {
            if (pl.RL == 2) go(gemv_kernel<F, 2, 1, 4, true, true>);
            else go(gemv_kernel<F, 1, 1, 4, true, true>);
        } else {
            if (pl.RL == 2) go(gemv_kernel<F, 2, 1, 4, true, false>);
            else go(gemv_kernel<F, 1, 1, 4, true, false>);
        }
    } else if (multi) {
        // KU == 1, RL ≤ 2 (1 for wider codes)
        if (pl.RL == 1) go2(gemv_kernel<F, 1, 1, 1, true, true>, gemv_kernel<F, 1, 1, 1, true, true, true>);
        else if constexpr (!F::WIDE) {
            if (pl.RL == 2) go2(gemv_kernel<F, 2, 1, 1, true, true>, gemv_kernel<F, 2, 1, 1, true, true, true>);
        }
    } else {
        // RL·KU ≤ 4 (≤ 2 for wider codes)
        if (pl.KU == 1) {
            if (pl.RL == 2) go2(gemv_kernel<F, 2, 1, 1, true, false>, gemv_kernel<F, 2, 1, 1, true, false, true>);
            else if (pl.RL == 1) go2(gemv_kernel<F, 1, 1, 1, true, false>, gemv_kernel<F, 1, 1, 1, true, false, true>);
            else if constexpr (!F::WIDE) {
                if (pl.RL == 4) go2(gemv_kernel<F, 4, 1, 1, true, false>, gemv_kernel<F, 4, 1, 1, true, false, true>);
            }
        } else if (pl.KU == 2) {
            if (pl.RL == 1) go2(gemv_kernel<F, 1, 2, 1, true, false>, gemv_kernel<F, 1, 2, 1, true, false, true>);
            else if constexpr (!F::WIDE) {
                if (pl.RL == 2) go2(gemv_kernel<F, 2, 2, 1, true, false>, gemv_kernel<F, 2, 2, 1, true, false, true>);
            }
        } else if (pl.KU == 3 && pl.RL == 1) {
            go2(gemv_kernel<F, 1, 3, 1, true, false>, gemv_kernel<F, 1, 3, 1, true, false, true>);
        } else if (pl.KU == 4 && pl.RL == 1) {
            go2(gemv_kernel<F, 1, 4, 1, true, false>, gemv_kernel<F, 1, 4, 1, true, false, true>);
        }
    }
    return launched;
}

constexpr int64_t kBatchLds = 160 * 1024;   // LDS of one gfx950 workgroup (and CU)

struct BatchPlan {
    GemvGeom geo;
    int RL, NT, CP;
    size_t lds;
    unsigned blocks;
};

// Batched geometry: G and the unit order are the single-input plan's (so the
// results match it bitwise), one unit per lane and pass.  NT = 8 / 4 / 2
// inputs per workgroup: 8 where one pass of staged inputs fits in half the
// LDS (two workgroups per CU; NT = 4 may take all of it) and the grid (row
// blocks × input tiles, at 4 waves per workgroup) keeps ≥ 1024 workgroups;
// else 4, or 2 for N ≤ 2 and for N ≤ 8 on a grid of < 1024 workgroups.
// A batch is bound by the FMAs, 32 per unit and input, and a grid of fewer
// workgroups leaves SIMDs idle; measured per projection at N = 8…32, this
// beats tiles of 16 inputs (0.4B FFN value × 32: 22.3 → 11.9 µs; 7B-class
// output projection × 16: 31.3 → 18.6 µs) and, at the 7B-class shapes with
// ≥ 1024 workgroups of 8 inputs, also tiles of 4; tiles of 2 win at N = 8
// (0.1B / 0.4B projections 5–20 % faster) but lose at N = 32 on the small
// grids (0.1B r/k/v × 32: 8.9 → 11.3 µs), where the decode of each unit is
// repeated per tile.  Then RL = 2 rows per lane
// where the rows allow and the grid stays ≥ 256 workgroups, and WPB = 8 waves
// under the same condition, else 4.  CP passes per chunk fill the LDS share.
bool plan_batch(int64_t OUT, int64_t NU, int64_t rl_div, int64_t N, int64_t NK, bool sums, BatchPlan& bp) {
    const GemvPlan one = plan_gemv(OUT, NU, rl_div, 1, NK, sums, false);
    bp.geo = one.geo;
    bp.geo.NP = (int)(NU / bp.geo.G);
    const int64_t per_row_pass = (int64_t)bp.geo.G * (36 + (sums ? 2 : 0)) * 4;   // bytes per input row, one pass
    auto blocks = [&](int wpb, int rl) {
        const int64_t per = (int64_t)wpb * bp.geo.R * rl;
        return (OUT + per - 1) / per;
    };
    auto tiles = [&](int nt) { return (N + nt - 1) / nt; };
    // A fused group's workgroups stage only their own matrix's input rows when
    // no workgroup straddles two matrices: workgroup rows (WPB·R·RL, powers
    // of two up to 8·R·2) divide rl_div (= out_per) whenever the largest does.
    bp.geo.one_k = NK > 1 && rl_div % (8 * (int64_t)bp.geo.R * 2) == 0;
    const int64_t NKs = bp.geo.one_k ? 1 : NK;
    bp.NT = N > 4 ? 8 : 4;
    if (bp.NT > 4 && (bp.NT * NKs * per_row_pass > kBatchLds / 2 || blocks(4, 1) * tiles(bp.NT) < 1024)) bp.NT = 4;
    if (bp.NT == 4 && (N <= 2 || (N <= 8 && blocks(4, 1) * tiles(4) < 1024))) bp.NT = 2;
    const int64_t pass_bytes = bp.NT * NKs * per_row_pass;
    if (pass_bytes > kBatchLds) return false;
    const int64_t budget = pass_bytes <= kBatchLds / 2 ? kBatchLds / 2 : kBatchLds;
    bp.CP = (int)std::min<int64_t>(bp.geo.NP, budget / pass_bytes);
    bp.lds = (size_t)(pass_bytes * bp.CP);
    bp.RL = (rl_div % 2 == 0 && blocks(4, 2) * tiles(bp.NT) >= 256) ? 2 : 1;
    bp.geo.WPB = blocks(8, bp.RL) * tiles(bp.NT) >= 256 ? 8 : 4;
    bp.blocks = (unsigned)blocks(bp.geo.WPB, bp.RL);
    return true;
}

template <class F>
bool launch_batch(const BatchPlan& bp, hipStream_t st, const float* x, int N, typename F::Ptr P, float* y, int OUT,
                  int IN, int out_per) {
    const dim3 grid(bp.blocks, (unsigned)((N + bp.NT - 1) / bp.NT)), block(64 * bp.geo.WPB);
#define RWKV_GB(RLV, NTV)                                                                                    \
    rwkv::launch_lds(gemv_batch_kernel<F, RLV, NTV>, grid, block, bp.lds, st, x, N, P, y, OUT, IN, out_per, \
                     bp.geo, bp.CP)
    if (bp.RL == 2) {
        if (bp.NT == 8) RWKV_GB(2, 8);
        else if (bp.NT == 4) RWKV_GB(2, 4);
        else RWKV_GB(2, 2);
    } else {
        if (bp.NT == 8) RWKV_GB(1, 8);
        else if (bp.NT == 4) RWKV_GB(1, 4);
        else RWKV_GB(1, 2);
    }
#undef RWKV_GB
    return true;
}

// One input: gemv_kernel.  Batches: one gemv_batch_kernel launch, a
// workgroup per (row block, tile of NT inputs).
template <class F>
bool run_gemv(int64_t OUT, int64_t IN, int64_t rl_div, int64_t N, int64_t NK, hipStream_t st, const float* x,
              typename F::Ptr P, float* y, int64_t out_per, int ep) {
    const int64_t NU = IN / 32;
    if (N >= 2) {
        BatchPlan bp;
        if (plan_batch(OUT, NU, rl_div, N, NK, F::SUMS, bp) && (N + bp.NT - 1) / bp.NT <= 65535) {
            bp.geo.ep = ep;
            return launch_batch<F>(bp, st, x, (int)N, P, y, (int)OUT, (int)IN, (int)out_per);
        }
    }
    GemvPlan all = plan_gemv(OUT, NU, rl_div, N, NK, F::SUMS, F::WIDE);
    all.geo.ep = ep;
    if (all.xl || N <= 4) return launch_gemv<F>(all, st, x, (int)N, P, y, (int)OUT, (int)IN, (int)out_per);
    GemvPlan tile = plan_gemv(OUT, NU, rl_div, 4, NK, F::SUMS, F::WIDE);
    tile.geo.ep = ep;
    if (!tile.xl) return launch_gemv<F>(all, st, x, (int)N, P, y, (int)OUT, (int)IN, (int)out_per);
    for (int64_t n0 = 0; n0 < N; n0 += 4) {
        const int64_t nn = N - n0 < 4 ? N - n0 : 4;
        GemvPlan pl = nn == 4 ? tile : plan_gemv(OUT, NU, rl_div, nn, NK, F::SUMS, F::WIDE);
        pl.geo.ep = ep;
        if (!launch_gemv<F>(pl, st, x + n0 * NK * IN, (int)nn, P, y + n0 * OUT, (int)OUT, (int)IN, (int)out_per))
            return false;
    }
    return true;
}

}  // namespace

extern "C" {

rwkv_status rwkv_sb6_dequant(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, void* out,
                             rwkv_dtype out_dt, int64_t OUT, int64_t IN, int xbits, void* stream) {
    RWKV_REQUIRE(qblk && qsqm && ddm && out, RWKV_E_NULL, "sb6_dequant: null buffer");
    RWKV_REQUIRE(xbits >= 0 && xbits <= 2, RWKV_E_SHAPE, "sb6_dequant: xbits %d outside 0...2", xbits);
    RWKV_REQUIRE(rwkv::dtype_ok(out_dt), RWKV_E_DTYPE, "sb6_dequant: output dtype code %d", out_dt);
    RWKV_REQUIRE(OUT >= 1 && IN >= 256 && IN % 256 == 0, RWKV_E_SHAPE,
                 "sb6_dequant: IN (%lld) must be a positive multiple of 256 (block 32 x super-block 8)", (long long)IN);
    const int64_t total = OUT * (IN / 32) * 4;   // four threads per (row, block)
    RWKV_REQUIRE(total < INT32_MAX, RWKV_E_SHAPE, "sb6_dequant: tensor too large");
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
    const bool i32 = total < INT32_MAX;
#define RWKV_DQ(BITS, DT)                                                                                             \
    if (i32)                                                                                                          \
        rwkv::launch(sym_dequant_kernel<BITS, DT, true>, grid, block, st, qblk, qs, d, out, OUT, IN,                  \
                     (const int32_t*)nullptr, (int64_t)0);                                                            \
    else                                                                                                              \
        rwkv::launch(sym_dequant_kernel<BITS, DT, false>, grid, block, st, qblk, qs, d, out, OUT, IN,                 \
                     (const int32_t*)nullptr, (int64_t)0)
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

rwkv_status rwkv_sym_rows(const int32_t* ids, int64_t n, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                          void* out, rwkv_dtype out_dt, int64_t OUT, int64_t IN, int bits, void* stream) {
    RWKV_REQUIRE((ids && out) || n == 0, RWKV_E_NULL, "sym_rows: null ids / output");
    RWKV_REQUIRE(qblk && qs && d, RWKV_E_NULL, "sym_rows: null buffer");
    RWKV_REQUIRE(bits == 6 || bits == 8, RWKV_E_SHAPE, "sym_rows: bits %d outside {6, 8}", bits);
    RWKV_REQUIRE(rwkv::dtype_ok(out_dt), RWKV_E_DTYPE, "sym_rows: output dtype code %d", out_dt);
    RWKV_REQUIRE(OUT >= 1 && IN >= 16 && IN % (bits == 8 ? 16 : 32) == 0 && n >= 0, RWKV_E_SHAPE,
                 "sym_rows: IN (%lld) must be a positive multiple of %d, n (%lld) >= 0", (long long)IN,
                 bits == 8 ? 16 : 32, (long long)n);
    RWKV_REQUIRE(OUT <= INT32_MAX && n * (IN / 4) / 256 < INT32_MAX, RWKV_E_SHAPE, "sym_rows: too large");
    if (n == 0) return RWKV_OK;
    const int64_t total = n * (IN / 4);
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool i32 = total < INT32_MAX;
#define RWKV_DQ(BITS, DT)                                                                                    \
    if (i32)                                                                                                 \
        rwkv::launch(sym_dequant_kernel<BITS, DT, true>, grid, block, st, qblk, qs, d, out, OUT, IN, ids, n); \
    else                                                                                                     \
        rwkv::launch(sym_dequant_kernel<BITS, DT, false>, grid, block, st, qblk, qs, d, out, OUT, IN, ids, n)
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
    rwkv_status s = launch_status("sym_rows launch");
    if (s == RWKV_OK) rwkv::counters().sym_rows++;
    return s;
}

int rwkv_sb6_gemv_applies(int64_t OUT, int64_t IN, int xbits, int super_block, int64_t rows) {
    // rwkvqSb6GEMVConfig (RwkvqSb6GEMV.swift:39-43) and Applies (:159-164).
    int nsg = 4, rs = 4;
    if (OUT < 32768 && OUT >= 8192 && xbits == 0) { nsg = 2; rs = 2; }
    return xbits >= 0 && xbits <= 2 && super_block == 8 && rows == 1 && IN > 0 && IN % 256 == 0 && OUT > 0 &&
           OUT % (nsg * rs) == 0;
}

}  // extern "C"

namespace {
rwkv_status sb6_gemv_args(const char* what, const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                          const uint16_t* ddm, const float* y, int64_t OUT, int64_t IN, int xbits, int64_t out_per,
                          int ep) {
    RWKV_REQUIRE(x && qblk && qsqm && ddm && y, RWKV_E_NULL, "%s: null buffer", what);
    RWKV_REQUIRE(ep >= 0 && ep <= 2, RWKV_E_SHAPE, "%s: epilogue %d outside 0...2", what, ep);
    RWKV_REQUIRE(xbits >= 0 && xbits <= 2, RWKV_E_SHAPE, "%s: xbits %d outside 0...2", what, xbits);
    RWKV_REQUIRE(N >= 1 && N <= INT32_MAX, RWKV_E_SHAPE, "%s: rows %lld", what, (long long)N);
    RWKV_REQUIRE(OUT >= 1 && OUT <= INT32_MAX && IN >= 256 && IN % 256 == 0 && IN <= (1 << 24), RWKV_E_SHAPE,
                 "%s: shape %lldx%lld not taken (IN %% 256 == 0 required)", what, (long long)OUT, (long long)IN);
    RWKV_REQUIRE(out_per >= 1 && OUT % out_per == 0, RWKV_E_SHAPE, "%s: %lld rows do not split into matrices of %lld",
                 what, (long long)OUT, (long long)out_per);
    RWKV_REQUIRE(OUT * (IN / 32) * (16 + 4 * xbits) < (int64_t(1) << 32), RWKV_E_SHAPE,
                 "%s: packed matrix of %lldx%lld exceeds 4 GiB", what, (long long)OUT, (long long)IN);
    return RWKV_OK;
}

rwkv_status sb6_gemv_impl(const char* what, const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                          const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, int64_t out_per,
                          void* stream, int ep = 0) {
    const rwkv_status a = sb6_gemv_args(what, x, N, qblk, qsqm, ddm, y, OUT, IN, xbits, out_per, ep);
    if (a != RWKV_OK) return a;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const Sb6Fmt<0>::Ptr P{(const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm};
    const int64_t NK = OUT / out_per;
    bool ok;
    switch (xbits) {
        case 0: ok = run_gemv<Sb6Fmt<0>>(OUT, IN, out_per, N, NK, st, x, P, y, out_per, ep); break;
        case 1: ok = run_gemv<Sb6Fmt<1>>(OUT, IN, out_per, N, NK, st, x, {P.q, P.sm, P.dd}, y, out_per, ep); break;
        default: ok = run_gemv<Sb6Fmt<2>>(OUT, IN, out_per, N, NK, st, x, {P.q, P.sm, P.dd}, y, out_per, ep); break;
    }
    RWKV_REQUIRE(ok, RWKV_E_UNSUPPORTED, "%s: no kernel variant for %lldx%lld", what, (long long)OUT, (long long)IN);
    return launch_status(what);
}
}  // namespace

extern "C" {

rwkv_status rwkv_sb6_gemv(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                          const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, void* stream) {
    const rwkv_status s = sb6_gemv_impl("sb6_gemv", x, N, qblk, qsqm, ddm, y, OUT, IN, xbits, OUT, stream);
    if (s == RWKV_OK) rwkv::counters().sb6_gemv++;
    return s;
}

rwkv_status rwkv_sb6_gemv_fused(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                                const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, int64_t out_per,
                                void* stream) {
    const rwkv_status s = sb6_gemv_impl("sb6_gemv_fused", x, N, qblk, qsqm, ddm, y, OUT, IN, xbits, out_per, stream);
    if (s == RWKV_OK) rwkv::counters().sb6_fused++;
    return s;
}

}  // extern "C"

namespace {
// rkv_lora_kernel for a single-pass plan of 3 or 4 units per lane (every
// r/k/v shape of the x070 presets); false where the plan is another.
bool launch_rkv_lora(const GemvPlan& pl, hipStream_t st, const float* x, Sb6Fmt<0>::Ptr P, float* y, int OUT, int IN,
                     int out_per, const float* xmix, const void* wcat, float* la, int rw, int ra, int rv, int rg,
                     int with_v) {
    if (pl.NT != 1 || !pl.xl || pl.geo.NP != 1 || pl.RL != 1 || (pl.KU != 3 && pl.KU != 4)) return false;
    const int RT = rw + ra + rv + rg;
    const int lb = (RT + pl.geo.WPB - 1) / pl.geo.WPB;   // lora_in workgroups
    const dim3 grid(pl.blocks + (unsigned)lb), block(64 * pl.geo.WPB);
#define RWKV_RL(KUV, XFV)                                                                                        \
    rwkv::launch_lds(rkv_lora_kernel<1, KUV, XFV>, grid, block, pl.lds, st, x, P, y, OUT, IN, out_per, pl.geo, \
                     lb, xmix, wcat, la, rw, ra, rv, rg, with_v)
    if (pl.KU == 4) {
        if (pl.geo.xfirst) RWKV_RL(4, true);
        else RWKV_RL(4, false);
    } else {
        if (pl.geo.xfirst) RWKV_RL(3, true);
        else RWKV_RL(3, false);
    }
#undef RWKV_RL
    return true;
}
}  // namespace

extern "C" {

rwkv_status rwkv_x070_rkv_lora(const float* x_rkv, const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                               float* y_rkv, int64_t OUT, int64_t IN, int xbits, int64_t out_per, const float* xmix,
                               const void* wcat, rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg,
                               int with_v, float* la, void* stream) {
    RWKV_REQUIRE(xmix && wcat && la, RWKV_E_NULL, "x070_rkv_lora: null low-rank buffer");
    RWKV_REQUIRE(w_dt == RWKV_F16 || w_dt == RWKV_F32, RWKV_E_DTYPE, "x070_rkv_lora: matrix dtype %d not f16/f32",
                 (int)w_dt);
    RWKV_REQUIRE(rw >= 8 && ra >= 8 && rv >= 8 && rg >= 8 && rw % 8 == 0 && ra % 8 == 0 && rv % 8 == 0 && rg % 8 == 0 &&
                     rw + ra + rv + rg <= 8192,
                 RWKV_E_SHAPE, "x070_rkv_lora: ranks %lld/%lld/%lld/%lld (multiples of 8)", (long long)rw,
                 (long long)ra, (long long)rv, (long long)rg);
    const rwkv_status a = sb6_gemv_args("x070_rkv_lora", x_rkv, 1, qblk, qsqm, ddm, y_rkv, OUT, IN, xbits, out_per, 0);
    if (a != RWKV_OK) return a;
    if (xbits == 0 && w_dt == RWKV_F16) {
        GemvPlan pl = plan_gemv(OUT, IN / 32, out_per, 1, OUT / out_per, true, false);
        pl.geo.ep = 0;
        const Sb6Fmt<0>::Ptr P{(const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm};
        if (launch_rkv_lora(pl, reinterpret_cast<hipStream_t>(stream), x_rkv, P, y_rkv, (int)OUT, (int)IN,
                            (int)out_per, xmix, wcat, la, (int)rw, (int)ra, (int)rv, (int)rg, with_v)) {
            const rwkv_status s = launch_status("x070_rkv_lora");
            if (s == RWKV_OK) {
                rwkv::counters().sb6_fused++;
                rwkv::counters().x070++;
            }
            return s;
        }
    }
    // other formats and plans: the two launches
    const rwkv_status s = rwkv_sb6_gemv_fused(x_rkv, 1, qblk, qsqm, ddm, y_rkv, OUT, IN, xbits, out_per, stream);
    if (s != RWKV_OK) return s;
    return rwkv_x070_lora_in(xmix, wcat, w_dt, rw, ra, rv, rg, with_v, la, 1, IN, stream);
}

}  // extern "C"

namespace {
// The plan of a GEMV that forms its input row in the launch: one input, one
// pass of 3 or 4 units per lane, one input row per workgroup, and the row
// (IN ≤ 4096, IN % 256 == 0) within four float4 per thread.  Forming the row
// costs registers (~90-104 VGPRs against 58: 4-5 waves per SIMD against 8),
// so only grids that still run in one round take it: at most 4096 waves, four
// per SIMD of the 256 CUs of a gfx950 (the 0.1B ... 1.5B shapes; at 7B-class
// widths the separate row launch is faster: 1.78 against 1.93 ms per token).
constexpr int64_t kLnWavesMax = 4 * 4 * 256;
bool ln_plan(int64_t OUT, int64_t IN, int64_t out_per, GemvPlan& pl) {
    if (IN < 256 || IN % 256 || IN > 4096 || out_per < 1 || OUT % out_per) return false;
    pl = plan_gemv(OUT, IN / 32, out_per, 1, OUT / out_per, true, false);
    return pl.NT == 1 && pl.xl && pl.geo.NP == 1 && pl.RL == 1 && (pl.KU == 3 || pl.KU == 4) &&
           (OUT == out_per || pl.geo.one_k) && IN <= 8 * 64 * pl.geo.WPB &&
           (int64_t)pl.blocks * pl.geo.WPB <= kLnWavesMax;
}
// float4 chunks of the row per thread (1 or 2; more would spill)
int ln_chunks(int64_t IN, const GemvPlan& pl) {
    return IN / 4 <= 64 * pl.geo.WPB ? 1 : 2;
}
// the value GEMV with the residual add and the state copy
bool value_plan(int64_t OUT, int64_t IN, GemvPlan& pl) {
    if (IN < 256 || IN % 256) return false;
    pl = plan_gemv(OUT, IN / 32, OUT, 1, 1, true, false);
    return pl.NT == 1;
}
}  // namespace

extern "C" {

int rwkv_x070_ln_fused_applies(int64_t D, int64_t F, int xbits) {
    GemvPlan a, b, c;
    return xbits == 0 && ln_plan(3 * D, D, D, a) && ln_plan(F, D, F, b) && value_plan(D, F, c) ? 1 : 0;
}

rwkv_status rwkv_x070_rkv_lora_ln(const float* x, const float* ln_w, const float* ln_b, const float* prev,
                                  const float* coef6, float eps, float* xln, const uint8_t* qblk, const uint8_t* qsqm,
                                  const uint16_t* ddm, float* y_rkv, int64_t D, int xbits, const void* wcat,
                                  rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg, int with_v,
                                  float* la, void* stream) {
    RWKV_REQUIRE(x && ln_w && ln_b && prev && coef6 && xln && wcat && la, RWKV_E_NULL, "x070_rkv_lora_ln: null buffer");
    RWKV_REQUIRE(w_dt == RWKV_F16, RWKV_E_DTYPE, "x070_rkv_lora_ln: low-rank matrices must be f16 (dtype %d)",
                 (int)w_dt);
    RWKV_REQUIRE(rw >= 8 && ra >= 8 && rv >= 8 && rg >= 8 && rw % 8 == 0 && ra % 8 == 0 && rv % 8 == 0 && rg % 8 == 0 &&
                     rw + ra + rv + rg <= 8192,
                 RWKV_E_SHAPE, "x070_rkv_lora_ln: ranks %lld/%lld/%lld/%lld (multiples of 8)", (long long)rw,
                 (long long)ra, (long long)rv, (long long)rg);
    const rwkv_status a = sb6_gemv_args("x070_rkv_lora_ln", x, 1, qblk, qsqm, ddm, y_rkv, 3 * D, D, xbits, D, 0);
    if (a != RWKV_OK) return a;
    GemvPlan pl;
    RWKV_REQUIRE(xbits == 0 && ln_plan(3 * D, D, D, pl), RWKV_E_UNSUPPORTED,
                 "x070_rkv_lora_ln: D=%lld xbits=%d not taken (rwkv_x070_ln_fused_applies)", (long long)D, xbits);
    pl.geo.ep = 0;
    const Sb6Fmt<0>::Ptr P{(const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm};
    const LnMix lm{x, ln_w, ln_b, prev, coef6, xln, eps};
    const int RT = (int)(rw + ra + rv + rg);
    const int lb = (RT + pl.geo.WPB - 1) / pl.geo.WPB;
    const dim3 grid(pl.blocks + (unsigned)lb), block(64 * pl.geo.WPB);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int ch = ln_chunks(D, pl);
#define RWKV_RLL(KUV, CHV)                                                                                         \
    if (pl.KU == KUV && ch == CHV)                                                                                 \
    rwkv::launch_lds(rkv_lora_ln_kernel<KUV, CHV>, grid, block, pl.lds, st, P, y_rkv, (int)(3 * D), (int)D, (int)D, \
                     pl.geo, lb, lm, wcat, la, (int)rw, (int)ra, (int)rv, (int)rg, with_v)
    RWKV_RLL(4, 1);
    RWKV_RLL(4, 2);
    RWKV_RLL(3, 1);
    RWKV_RLL(3, 2);
#undef RWKV_RLL
    const rwkv_status s = launch_status("x070_rkv_lora_ln");
    if (s == RWKV_OK) {
        rwkv::counters().sb6_fused++;
        rwkv::counters().x070++;
    }
    return s;
}

rwkv_status rwkv_x070_ffn_key_ln(const float* x, const float* ln_w, const float* ln_b, const float* prev,
                                 const float* coef, float eps, float* xln, const uint8_t* qblk, const uint8_t* qsqm,
                                 const uint16_t* ddm, float* hk, int64_t F, int64_t D, int xbits, void* stream) {
    RWKV_REQUIRE(x && ln_w && ln_b && prev && coef && xln, RWKV_E_NULL, "x070_ffn_key_ln: null buffer");
    const rwkv_status a = sb6_gemv_args("x070_ffn_key_ln", x, 1, qblk, qsqm, ddm, hk, F, D, xbits, F, 2);
    if (a != RWKV_OK) return a;
    GemvPlan pl;
    RWKV_REQUIRE(xbits == 0 && ln_plan(F, D, F, pl), RWKV_E_UNSUPPORTED,
                 "x070_ffn_key_ln: %lldx%lld xbits=%d not taken (rwkv_x070_ln_fused_applies)", (long long)F,
                 (long long)D, xbits);
    pl.geo.ep = 2;
    const Sb6Fmt<0>::Ptr P{(const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm};
    const LnMix lm{x, ln_w, ln_b, prev, coef, xln, eps};
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(pl.blocks), block(64 * pl.geo.WPB);
    const int ch = ln_chunks(D, pl);
#define RWKV_KL(KUV, CHV) \
    if (pl.KU == KUV && ch == CHV) rwkv::launch_lds(gemv_ln_kernel<KUV, CHV>, grid, block, pl.lds, st, P, hk, (int)F, (int)D, pl.geo, lm)
    RWKV_KL(4, 1);
    RWKV_KL(4, 2);
    RWKV_KL(3, 1);
    RWKV_KL(3, 2);
#undef RWKV_KL
    const rwkv_status s = launch_status("x070_ffn_key_ln");
    if (s == RWKV_OK) {
        rwkv::counters().sb6_gemv++;
        rwkv::counters().x070++;
    }
    return s;
}

rwkv_status rwkv_x070_ffn_value(const float* hk, const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                float* x, int64_t D, int64_t F, int xbits, const float* shift_src, float* shift_dst,
                                void* stream) {
    RWKV_REQUIRE((shift_src == nullptr) == (shift_dst == nullptr), RWKV_E_NULL,
                 "x070_ffn_value: shift_src and shift_dst are both set or both null");
    const rwkv_status a = sb6_gemv_args("x070_ffn_value", hk, 1, qblk, qsqm, ddm, x, D, F, xbits, D, 1);
    if (a != RWKV_OK) return a;
    GemvPlan pl;
    RWKV_REQUIRE(xbits == 0 && value_plan(D, F, pl), RWKV_E_UNSUPPORTED, "x070_ffn_value: %lldx%lld xbits=%d not taken",
                 (long long)D, (long long)F, xbits);
    pl.geo.ep = 1;
    pl.geo.cp_src = shift_src;
    pl.geo.cp_dst = shift_dst;
    const Sb6Fmt<0>::Ptr P{(const uint32_t*)qblk, (const uint16_t*)qsqm, (const uint32_t*)ddm};
    RWKV_REQUIRE(launch_gemv<Sb6Fmt<0>>(pl, reinterpret_cast<hipStream_t>(stream), hk, 1, P, x, (int)D, (int)F, (int)D),
                 RWKV_E_UNSUPPORTED, "x070_ffn_value: no kernel variant for %lldx%lld", (long long)D, (long long)F);
    const rwkv_status s = launch_status("x070_ffn_value");
    if (s == RWKV_OK) {
        rwkv::counters().sb6_gemv++;
        rwkv::counters().x070++;
    }
    return s;
}

int rwkv_sym_gemv_applies(int64_t OUT, int64_t IN, int bits, int64_t rows) {
    // rwkvqSymGEMVApplies (RwkvqSymGEMV.swift:213-218): NSG = RS = 4, NB_MAX = 4.
    return (bits == 6 || bits == 8) && IN > 0 && IN % 256 == 0 && OUT > 0 && OUT % 16 == 0 && rows >= 1 && rows <= 4;
}

}  // extern "C"

namespace {
rwkv_status sym_gemv_impl(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                          float* y, int64_t OUT, int64_t IN, int bits, int64_t out_per, void* stream, int ep) {
    RWKV_REQUIRE(x && qblk && qs && d && y, RWKV_E_NULL, "sym_gemv: null buffer");
    RWKV_REQUIRE(ep >= 0 && ep <= 2, RWKV_E_SHAPE, "sym_gemv: epilogue %d outside 0...2", ep);
    RWKV_REQUIRE(bits == 6 || bits == 8, RWKV_E_SHAPE, "sym_gemv: bits %d outside {6, 8}", bits);
    RWKV_REQUIRE(N >= 1 && N <= INT32_MAX, RWKV_E_SHAPE, "sym_gemv: rows %lld", (long long)N);
    RWKV_REQUIRE(OUT >= 1 && OUT <= INT32_MAX && IN >= 256 && IN % 256 == 0 && IN <= (1 << 24), RWKV_E_SHAPE,
                 "sym_gemv: shape %lldx%lld not taken (IN %% 256 == 0 required)", (long long)OUT, (long long)IN);
    RWKV_REQUIRE(out_per >= 1 && OUT % out_per == 0, RWKV_E_SHAPE,
                 "sym_gemv: %lld rows do not split into matrices of %lld", (long long)OUT, (long long)out_per);
    RWKV_REQUIRE(OUT * IN * bits / 8 < (int64_t(1) << 32), RWKV_E_SHAPE,
                 "sym_gemv: packed matrix of %lldx%lld exceeds 4 GiB", (long long)OUT, (long long)IN);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t NK = OUT / out_per;
    const bool ok = bits == 8 ? run_gemv<SymFmt<8>>(OUT, IN, out_per, N, NK, st, x, {(const uint32_t*)qblk, (const uint16_t*)qs, d}, y, out_per, ep)
                              : run_gemv<SymFmt<6>>(OUT, IN, out_per, N, NK, st, x, {(const uint32_t*)qblk, (const uint16_t*)qs, d}, y, out_per, ep);
    RWKV_REQUIRE(ok, RWKV_E_UNSUPPORTED, "sym_gemv: no kernel variant for %lldx%lld", (long long)OUT, (long long)IN);
    rwkv_status s = launch_status("sym_gemv launch");
    if (s == RWKV_OK) {
        if (out_per < OUT) rwkv::counters().sym_fused++;
        else rwkv::counters().sym_gemv++;
    }
    return s;
}
}  // namespace

extern "C" {

rwkv_status rwkv_sym_gemv(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                          float* y, int64_t OUT, int64_t IN, int bits, int64_t out_per, void* stream) {
    return sym_gemv_impl(x, N, qblk, qs, d, y, OUT, IN, bits, out_per, stream, 0);
}

rwkv_status rwkv_sym_gemv_ep(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                             float* y, int64_t OUT, int64_t IN, int bits, int epilogue, void* stream) {
    return sym_gemv_impl(x, N, qblk, qs, d, y, OUT, IN, bits, OUT, stream, epilogue);
}

rwkv_status rwkv_sb6_gemv_ep(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                             const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits, int epilogue,
                             void* stream) {
    const rwkv_status s = sb6_gemv_impl("sb6_gemv_ep", x, N, qblk, qsqm, ddm, y, OUT, IN, xbits, OUT, stream, epilogue);
    if (s == RWKV_OK) rwkv::counters().sb6_gemv++;
    return s;
}

}  // extern "C"
