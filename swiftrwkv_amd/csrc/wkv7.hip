// WKV-7 recurrence on gfx950: whole-sequence / chunk / training forward, the
// checkpointed backward, the one-token decode step and the tmix tail.
//
// Recurrence per (b, h), state S[i = value row, j = key column] (fp32):
//   sa_i = Σ_j S_ij a_j ;  S_ij ← w_j S_ij + v_i k_j + sa_i b_j ;  y_i = Σ_j S_ij r_j
// (Sources/RWKVKernel/WKV7.swift:207-224).
//
// Forward (one wave = 16 value rows × 64 key columns of one head, no LDS, no
// barrier).  Lane l owns row 16·blk + (l & 15) and the 16 key columns of
// column group g = l >> 4, holding those 16 state values in VGPRs for the
// whole sequence.  The 16 lanes of a DPP row share g, so each step vector
// (a, w, k, b, r) is held ONE value per lane (lane l keeps element 16g + (l & 15))
// and broadcast into the FMAs with DPP row_newbcast — a single global_load per
// vector per step, prefetched 8 steps ahead in a 16-slot register ring.  The
// four column-group partials of sa and y of a row (lanes l, l^16, l^32, l^48)
// are combined with v_permlane16_swap / v_permlane32_swap.  The next step's sa
// partial is accumulated inside the update loop, so a step is 5 FMAs per
// state element plus two lane swaps.
// The decode step, the chunk kernel and the training forward are this same
// kernel (T = 1 / emitted sa / emitted checkpoints), so they agree bitwise by
// construction (the reference's invariants WKV7SequenceTests,
// WKV7StateTests.swift:178-186, DecodeKernelTests.swift:27-39).
//
// Backward (column-owned, the scheme of ckptBwdKernelV2,
// WKV7Train.swift:234-339).  Eight waves per head: lane i owns key column i,
// wave q owns value rows J_q = [8q, 8q+8).  Instead of reconstructing earlier
// states by dividing by w (which re-amplifies the forward's rounding by up to
// 1/w^15), each 16-step chunk's states are recomputed forward from the
// previous checkpoint (or h_in) with the stored sa and the forward kernel's
// exact FMA sequence, so they are bitwise the forward's states.  The chunk is
// handled as two 8-step windows whose states are held in registers.  Step
// vectors are staged per chunk in LDS (coalesced loads issued one chunk
// ahead); dsa is the one quantity exchanged inside a step (one barrier per
// step); every output is summed over the eight waves from an LDS ring.
// Variant 1 is the reference's row-owned ckptBwdKernel (WKV7Train.swift:
// 99-205), which does divide by w: wkv7_bwd_rows_kernel below.
//
// All arithmetic is fp32 with a fixed summation order: launches are bitwise
// deterministic.

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "launch.h"
#include "wkv7_step.h"

namespace {

using namespace rwkv_wkv;
constexpr int CH = 16;  // WKV7_CHUNK

template <int DT>
__device__ __forceinline__ float load1(const void* __restrict__ p, int64_t off) {
    if constexpr (DT == RWKV_F32) return reinterpret_cast<const float*>(p)[off];
    uint16_t h = reinterpret_cast<const uint16_t*>(p)[off];
    if constexpr (DT == RWKV_BF16) return __uint_as_float((uint32_t)h << 16);
    return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ __forceinline__ void store1(void* __restrict__ p, int64_t off, float x) {
    if constexpr (DT == RWKV_F32) {
        reinterpret_cast<float*>(p)[off] = x;
    } else if constexpr (DT == RWKV_BF16) {
        uint32_t u = __float_as_uint(x);
        uint16_t h;
        if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) h = (uint16_t)((u >> 16) | 0x40u);
        else h = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        reinterpret_cast<uint16_t*>(p)[off] = h;
    } else {
        reinterpret_cast<uint16_t*>(p)[off] = __builtin_bit_cast(uint16_t, (_Float16)x);
    }
}

// ─────────────────────────────── forward ───────────────────────────────
// Grid: 4 workgroups of one wave per (b, h); workgroup 4·(b·H + h) + blk owns
// value rows 16·blk .. 16·blk + 15.  Offsets inside one (b, h) sequence are
// 32-bit (the host checks T·H·64·4 < 2^32), so loads use an SGPR base.
template <int DT>
struct FwdIn {
    using E = typename std::conditional<DT == RWKV_F32, float, uint16_t>::type;
    const E* a;
    const E* w;
    const E* k;
    const E* b;
    const E* r;
    const E* v;
    __device__ __forceinline__ static float cvt(E x) {
        if constexpr (DT == RWKV_F32) return x;
        else if constexpr (DT == RWKV_BF16) return __uint_as_float((uint32_t)x << 16);
        else return (float)__builtin_bit_cast(_Float16, x);
    }
};

template <int DT, bool EMIT_SA, bool EMIT_CK>
__global__ __launch_bounds__(64) void wkv7_fwd_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ h_in, float* __restrict__ out, float* __restrict__ h_out,
    float* __restrict__ sa_out, float* __restrict__ ckpt, int T, int H) {
    using In = FwdIn<DT>;
    using E = typename In::E;
    const int l = threadIdx.x;
    const int ri = l & 15, g = l >> 4;
    // Workgroups are dealt round-robin to the 8 XCDs (each with its own L2):
    // when the grid allows, the four waves of a head get ids congruent mod 8,
    // so they share one XCD and each step vector is fetched from HBM once.
    int bh, blk;
    if ((gridDim.x & 31) == 0) {
        const int id = blockIdx.x, xcd = id & 7, slot = id >> 3;
        bh = (slot >> 2) * 8 + xcd;
        blk = slot & 3;
    } else {
        bh = blockIdx.x >> 2;
        blk = blockIdx.x & 3;
    }
    const int bi = bh / H, hi = bh - bi * H;
    const int row = 16 * blk + ri;
    const uint32_t vidx = 16 * g + ri;   // step-vector element this lane broadcasts
    const uint32_t strideT = (uint32_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;
    const int64_t sbase = (int64_t)bh * D * D + (int64_t)row * D + 16 * g;
    const int NC = T / CH;
    In in{reinterpret_cast<const E*>(a) + base0, reinterpret_cast<const E*>(w) + base0,
          reinterpret_cast<const E*>(k) + base0, reinterpret_cast<const E*>(b) + base0,
          reinterpret_cast<const E*>(r) + base0, reinterpret_cast<const E*>(v) + base0};
    float* const outp = out + base0;
    float* const sap = EMIT_SA ? sa_out + base0 : nullptr;

    float S[2][16];
    if (h_in) {
        const float4* src = reinterpret_cast<const float4*>(h_in + sbase);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float4 f = src[m];
            S[0][4 * m] = f.x; S[0][4 * m + 1] = f.y; S[0][4 * m + 2] = f.z; S[0][4 * m + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) S[0][c] = 0.0f;
    }

    // ring slot: a, w, k, b, r (broadcast sources), v (own row), as raw elements
    E ring[CH][6];
    // Buffer addressing: a descriptor per input (SGPRs), the per-lane part a
    // fixed VGPR offset, the per-step part a scalar offset — no per-load VALU.
    const uint32_t esz = (uint32_t)sizeof(E);
    const uint32_t span = (uint32_t)T * strideT * esz - (uint32_t)hi * D * esz;   // bytes from this head's base
    const uint32_t voff = vidx * esz, roff = (uint32_t)row * esz;
    auto rsrc = [&](const void* p, uint32_t n) { return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000); };
    const __amdgpu_buffer_rsrc_t ra = rsrc(in.a, span), rw = rsrc(in.w, span), rk_ = rsrc(in.k, span),
                                 rb = rsrc(in.b, span), rr = rsrc(in.r, span), rv = rsrc(in.v, span);
    auto ld = [&](__amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t so) -> E {
        if constexpr (sizeof(E) == 2) return (E)__builtin_amdgcn_raw_buffer_load_b16(rs, vo, so, 0);
        else return __builtin_bit_cast(E, __builtin_amdgcn_raw_buffer_load_b32(rs, vo, so, 0));
    };
    auto fetch = [&](E (&slot)[6], int t) __attribute__((always_inline)) {
        const uint32_t so = (uint32_t)min(t, T - 1) * strideT * esz;
        slot[0] = ld(ra, voff, so);
        slot[1] = ld(rw, voff, so);
        slot[2] = ld(rk_, voff, so);
        slot[3] = ld(rb, voff, so);
        slot[4] = ld(rr, voff, so);
        slot[5] = ld(rv, roff, so);
    };
    const uint32_t ospan = (uint32_t)T * strideT * 4u - (uint32_t)hi * D * 4u;
    const __amdgpu_buffer_rsrc_t ro_ = rsrc(outp, ospan), rs_ = rsrc(EMIT_SA ? sap : outp, ospan);
    const uint32_t orow = (uint32_t)row * 4u;
#pragma unroll
    for (int s = 0; s < 8; ++s) fetch(ring[s], s);

    float p = 0.0f;
    fwd_dot16(S[0], In::cvt(ring[0][0]), p);
    float y = 0.0f;   // partial y of the previous step, reduced and stored one step late

    // one step at chunk position s (compile-time) and time t
    auto step = [&](auto sc, int t, int c) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        // Steps stay in program order (no store sinking / load hoisting across
        // them), so every wait for a prefetched value is a small exact count.
        __builtin_amdgcn_sched_barrier(0);
        fetch(ring[(s + 8) & (CH - 1)], t + 8);
        float sa = p;
        rowsum4_pair(sa, y);   // sa of step t, y of step t - 1
        // y of step t - 1 (at t = 0 a placeholder at row 0, overwritten next
        // step); the four lanes of a row store the same bits
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro_, orow,
                                              (uint32_t)max(t - 1, 0) * strideT * 4u, 0);
        y = 0.0f;
        p = 0.0f;
        const E* sl = ring[s];
        fwd_update16(S[s & 1], S[(s + 1) & 1], In::cvt(sl[2]), In::cvt(sl[3]), In::cvt(sl[1]), In::cvt(sl[4]),
                     In::cvt(ring[(s + 1) & (CH - 1)][0]), In::cvt(sl[5]), sa, y, p);
        const uint32_t so = (uint32_t)t * strideT * 4u;
        if constexpr (EMIT_SA) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sa), rs_, orow, so, 0);
        if constexpr (EMIT_CK && s == CH - 1) {
            float4* dst = reinterpret_cast<float4*>(ckpt + ((int64_t)bh * NC + c) * D * D + (int64_t)row * D + 16 * g);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                dst[m] = make_float4(S[0][4 * m], S[0][4 * m + 1], S[0][4 * m + 2], S[0][4 * m + 3]);
        }
    };
    auto body = [&](int c, int n) __attribute__((always_inline)) {
        const int t0 = c * CH;
        [&]<int... s>(std::integer_sequence<int, s...>) {
            ((n > s ? step(std::integral_constant<int, s>{}, t0 + s, c) : void()), ...);
        }(std::make_integer_sequence<int, CH>{});
    };
    auto body_full = [&](int c) __attribute__((always_inline)) {
        const int t0 = c * CH;
        [&]<int... s>(std::integer_sequence<int, s...>) {
            (step(std::integral_constant<int, s>{}, t0 + s, c), ...);
        }(std::make_integer_sequence<int, CH>{});
    };
    // Branch-free chunks.  The first one is peeled so the loop is entered
    // with the same outstanding loads and stores as its back edge: the wait
    // counts at the loop head stay exact instead of draining everything.
    if (NC > 0) body_full(0);
    for (int c = 1; c < NC; ++c) body_full(c);
    const int tail = T - NC * CH;
    if (tail) body(NC, tail);
    y = rowsum4(y);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro_, orow, (uint32_t)(T - 1) * strideT * 4u, 0);

    float4* dst = reinterpret_cast<float4*>(h_out + sbase);
    if (tail & 1) {
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[m] = make_float4(S[1][4 * m], S[1][4 * m + 1], S[1][4 * m + 2], S[1][4 * m + 3]);
    } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[m] = make_float4(S[0][4 * m], S[0][4 * m + 1], S[0][4 * m + 2], S[0][4 * m + 3]);
    }
}

// Forward, four-row layout: 16 workgroups of one wave per (b, h); workgroup
// 16·(b·H + h) + blk owns value rows 4·blk .. 4·blk + 3.  Each lane loads
// element l of the step vectors (a 256-byte coalesced row per vector and
// step) and its row's v; otherwise the step is wkv7_fwd_kernel's.
template <int DT, bool EMIT_SA, bool EMIT_CK>
__global__ __launch_bounds__(64) void wkv7_fwd4_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ h_in, float* __restrict__ out, float* __restrict__ h_out,
    float* __restrict__ sa_out, float* __restrict__ ckpt, int T, int H) {
    using In = FwdIn<DT>;
    using E = typename In::E;
    const int l = threadIdx.x;
    const int ri = l & 3, g = l >> 2;
    // the sixteen waves of a head on one XCD when the grid allows
    int bh, blk;
    if ((gridDim.x & 127) == 0) {
        const int id = blockIdx.x, xcd = id & 7, slot = id >> 3;
        bh = (slot >> 4) * 8 + xcd;
        blk = slot & 15;
    } else {
        bh = blockIdx.x >> 4;
        blk = blockIdx.x & 15;
    }
    const int bi = bh / H, hi = bh - bi * H;
    const int row = 4 * blk + ri;
    const uint32_t strideT = (uint32_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;
    const int64_t sbase = (int64_t)bh * D * D + (int64_t)row * D + 4 * g;
    const int NC = T / CH;
    In in{reinterpret_cast<const E*>(a) + base0, reinterpret_cast<const E*>(w) + base0,
          reinterpret_cast<const E*>(k) + base0, reinterpret_cast<const E*>(b) + base0,
          reinterpret_cast<const E*>(r) + base0, reinterpret_cast<const E*>(v) + base0};
    float* const outp = out + base0;
    float* const sap = EMIT_SA ? sa_out + base0 : nullptr;

    float S[2][4];
    if (h_in) {
        const float4 f = *reinterpret_cast<const float4*>(h_in + sbase);
        S[0][0] = f.x; S[0][1] = f.y; S[0][2] = f.z; S[0][3] = f.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) S[0][c] = 0.0f;
    }

    E ring[CH][6];
    const uint32_t esz = (uint32_t)sizeof(E);
    const uint32_t span = (uint32_t)T * strideT * esz - (uint32_t)hi * D * esz;
    const uint32_t voff = (uint32_t)l * esz, roff = (uint32_t)row * esz;
    auto rsrc = [&](const void* p, uint32_t n) { return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000); };
    const __amdgpu_buffer_rsrc_t ra = rsrc(in.a, span), rw = rsrc(in.w, span), rk_ = rsrc(in.k, span),
                                 rb = rsrc(in.b, span), rr = rsrc(in.r, span), rv = rsrc(in.v, span);
    auto ld = [&](__amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t so) -> E {
        if constexpr (sizeof(E) == 2) return (E)__builtin_amdgcn_raw_buffer_load_b16(rs, vo, so, 0);
        else return __builtin_bit_cast(E, __builtin_amdgcn_raw_buffer_load_b32(rs, vo, so, 0));
    };
    auto fetch = [&](E (&slot)[6], int t) __attribute__((always_inline)) {
        const uint32_t so = (uint32_t)min(t, T - 1) * strideT * esz;
        slot[0] = ld(ra, voff, so);
        slot[1] = ld(rw, voff, so);
        slot[2] = ld(rk_, voff, so);
        slot[3] = ld(rb, voff, so);
        slot[4] = ld(rr, voff, so);
        slot[5] = ld(rv, roff, so);
    };
    const uint32_t ospan = (uint32_t)T * strideT * 4u - (uint32_t)hi * D * 4u;
    const __amdgpu_buffer_rsrc_t ro_ = rsrc(outp, ospan), rs_ = rsrc(EMIT_SA ? sap : outp, ospan);
    const uint32_t orow = (uint32_t)row * 4u;
#pragma unroll
    for (int st = 0; st < 8; ++st) fetch(ring[st], st);

    float p = 0.0f;
    fwd_dot4(S[0], In::cvt(ring[0][0]), p);
    float y = 0.0f;   // partial y of the previous step, reduced and stored one step late

    auto step = [&](auto sc, int t, int c) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        __builtin_amdgcn_sched_barrier(0);
        fetch(ring[(s + 8) & (CH - 1)], t + 8);
        float sa = p;
        rowsum16_pair(sa, y);
        // y of step t - 1 (at t = 0 a placeholder at row 0, overwritten next
        // step); the sixteen lanes of a row store the same bits
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro_, orow,
                                              (uint32_t)max(t - 1, 0) * strideT * 4u, 0);
        y = 0.0f;
        p = 0.0f;
        const E* sl = ring[s];
        fwd_update4(S[s & 1], S[(s + 1) & 1], In::cvt(sl[2]), In::cvt(sl[3]), In::cvt(sl[1]), In::cvt(sl[4]),
                    In::cvt(ring[(s + 1) & (CH - 1)][0]), In::cvt(sl[5]), sa, y, p);
        const uint32_t so = (uint32_t)t * strideT * 4u;
        if constexpr (EMIT_SA) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sa), rs_, orow, so, 0);
        if constexpr (EMIT_CK && s == CH - 1) {
            *reinterpret_cast<float4*>(ckpt + ((int64_t)bh * NC + c) * D * D + (int64_t)row * D + 4 * g) =
                make_float4(S[0][0], S[0][1], S[0][2], S[0][3]);
        }
    };
    auto body = [&](int c, int n) __attribute__((always_inline)) {
        const int t0 = c * CH;
        [&]<int... s>(std::integer_sequence<int, s...>) {
            ((n > s ? step(std::integral_constant<int, s>{}, t0 + s, c) : void()), ...);
        }(std::make_integer_sequence<int, CH>{});
    };
    auto body_full = [&](int c) __attribute__((always_inline)) {
        const int t0 = c * CH;
        [&]<int... s>(std::integer_sequence<int, s...>) {
            (step(std::integral_constant<int, s>{}, t0 + s, c), ...);
        }(std::make_integer_sequence<int, CH>{});
    };
    if (NC > 0) body_full(0);
    for (int c = 1; c < NC; ++c) body_full(c);
    const int tail = T - NC * CH;
    if (tail) body(NC, tail);
    y = rowsum16(y);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro_, orow, (uint32_t)(T - 1) * strideT * 4u, 0);

    const int fs = tail & 1;
    *reinterpret_cast<float4*>(h_out + sbase) = make_float4(S[fs][0], S[fs][1], S[fs][2], S[fs][3]);
}

// ─────────────────────────────── backward ───────────────────────────────
constexpr int BQ = 8;     // waves per head
constexpr int BJ = 8;     // value rows per wave
constexpr int NVEC = 8;   // staged step vectors: r w k v a b dy sa
constexpr int NOUT = 6;   // dr dw dk db dv da
constexpr int WIN = 8;    // steps per register window (two per chunk)

#define RWKV_BC8(n) RWKV_BC(n)

// 8-wide broadcast helpers: lane l holds element 8q + (l & 7) of a step vector
// over the wave's rows; row_newbcast:jj reads row jj of the wave's block.
// (1) recompute: n_jj = v_j·k_i ; n_jj += sa_j·b_i      (then n += w_i·S in C++)
#define RWKV_RC(jj) \
    "v_mul_f32_dpp %[n" #jj "], %[V], %[ki]" RWKV_BC(jj) "v_fmac_f32_dpp %[n" #jj "], %[SA], %[bi]" RWKV_BC(jj)
__device__ __forceinline__ void bwd_recompute8(const float (&S)[BJ], float (&N)[BJ], float V, float SA, float ki,
                                               float bi, float wi) {
    asm("s_nop 1\n\t" RWKV_RC(0) RWKV_RC(1) RWKV_RC(2) RWKV_RC(3) RWKV_RC(4) RWKV_RC(5) RWKV_RC(6) RWKV_RC(7)
        : [n0] "=&v"(N[0]), [n1] "=&v"(N[1]), [n2] "=&v"(N[2]), [n3] "=&v"(N[3]), [n4] "=&v"(N[4]),
          [n5] "=&v"(N[5]), [n6] "=&v"(N[6]), [n7] "=&v"(N[7])
        : [V] "v"(V), [SA] "v"(SA), [ki] "v"(ki), [bi] "v"(bi));
#pragma unroll
    for (int jj = 0; jj < BJ; ++jj) N[jj] = fmaf(wi, S[jj], N[jj]);
}

// (2) first half of a reverse step, 4 rows at a time:
//   dr += dy_j·S_j ; dT_j += dy_j·r_i ; dR_j += r_j·dy_i
#define RWKV_B1(jj, e)                                              \
    "v_fmac_f32_dpp %[dr], %[DY], %[sa" #e "]" RWKV_BC(jj)          \
    "v_fmac_f32_dpp %[t" #e "], %[DY], %[ri]" RWKV_BC(jj)           \
    "v_fmac_f32_dpp %[u" #e "], %[R], %[dyi]" RWKV_BC(jj)
#define RWKV_B1_BLOCK(j0, j1, j2, j3, o)                                                                  \
    asm("s_nop 1\n\t" RWKV_B1(j0, 0) RWKV_B1(j1, 1) RWKV_B1(j2, 2) RWKV_B1(j3, 3)                          \
        : [dr] "+v"(pdr), [t0] "+v"(dT[o]), [t1] "+v"(dT[o + 1]), [t2] "+v"(dT[o + 2]), [t3] "+v"(dT[o + 3]), \
          [u0] "+v"(dR[o]), [u1] "+v"(dR[o + 1]), [u2] "+v"(dR[o + 2]), [u3] "+v"(dR[o + 3])               \
        : [sa0] "v"(Sa[o]), [sa1] "v"(Sa[o + 1]), [sa2] "v"(Sa[o + 2]), [sa3] "v"(Sa[o + 3]), [DY] "v"(DY),  \
          [R] "v"(R), [ri] "v"(ri), [dyi] "v"(dyi))
// (3) dk += v_j·dT_j ; db += sa_j·dT_j ; dv += k_j·dR_j ; dsa += b_j·dR_j
#define RWKV_B2(jj, e)                                              \
    "v_fmac_f32_dpp %[dk], %[V], %[t" #e "]" RWKV_BC(jj)            \
    "v_fmac_f32_dpp %[db], %[SA], %[t" #e "]" RWKV_BC(jj)           \
    "v_fmac_f32_dpp %[dv], %[K], %[u" #e "]" RWKV_BC(jj)            \
    "v_fmac_f32_dpp %[ds], %[B], %[u" #e "]" RWKV_BC(jj)
#define RWKV_B2_BLOCK(j0, j1, j2, j3, o)                                                                  \
    asm("s_nop 1\n\t" RWKV_B2(j0, 0) RWKV_B2(j1, 1) RWKV_B2(j2, 2) RWKV_B2(j3, 3)                          \
        : [dk] "+v"(pdk), [db] "+v"(pdb), [dv] "+v"(pdv), [ds] "+v"(pds)                                   \
        : [t0] "v"(dT[o]), [t1] "v"(dT[o + 1]), [t2] "v"(dT[o + 2]), [t3] "v"(dT[o + 3]), [u0] "v"(dR[o]),    \
          [u1] "v"(dR[o + 1]), [u2] "v"(dR[o + 2]), [u3] "v"(dR[o + 3]), [V] "v"(V), [SA] "v"(SA), [K] "v"(K), \
          [B] "v"(B))
// (4) da += dsa_j·Sp_j ; dR_j ← a_j·dsa_i + w_j·dR_j ; dT_j ← dsa_j·a_i (+ w_i·dT_j in C++)
#define RWKV_B3(jj, e)                                              \
    "v_fmac_f32_dpp %[da], %[DS], %[sp" #e "]" RWKV_BC(jj)          \
    "v_mul_f32_dpp %[nu" #e "], %[A], %[dsi]" RWKV_BC(jj)           \
    "v_fmac_f32_dpp %[nu" #e "], %[W], %[u" #e "]" RWKV_BC(jj)      \
    "v_mul_f32_dpp %[nt" #e "], %[DS], %[ai]" RWKV_BC(jj)
#define RWKV_B3_BLOCK(j0, j1, j2, j3, o)                                                                      \
    asm("s_nop 1\n\t" RWKV_B3(j0, 0) RWKV_B3(j1, 1) RWKV_B3(j2, 2) RWKV_B3(j3, 3)                              \
        : [da] "+v"(pda), [nu0] "=&v"(nR[o]), [nu1] "=&v"(nR[o + 1]), [nu2] "=&v"(nR[o + 2]),                  \
          [nu3] "=&v"(nR[o + 3]), [nt0] "=&v"(nT[o]), [nt1] "=&v"(nT[o + 1]), [nt2] "=&v"(nT[o + 2]),           \
          [nt3] "=&v"(nT[o + 3])                                                                               \
        : [sp0] "v"(Sp[o]), [sp1] "v"(Sp[o + 1]), [sp2] "v"(Sp[o + 2]), [sp3] "v"(Sp[o + 3]), [u0] "v"(dR[o]), \
          [u1] "v"(dR[o + 1]), [u2] "v"(dR[o + 2]), [u3] "v"(dR[o + 3]), [DS] "v"(DS), [A] "v"(A), [W] "v"(W),  \
          [dsi] "v"(dsa_i), [ai] "v"(ai))

// Σ over the 8 waves' partials p[0..7] of one column (stride D floats), pairwise.
__device__ __forceinline__ float sum8(const float* p) {
    const float x0 = p[0], x1 = p[D], x2 = p[2 * D], x3 = p[3 * D];
    const float x4 = p[4 * D], x5 = p[5 * D], x6 = p[6 * D], x7 = p[7 * D];
    return ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7));
}

// Variant 2, the default.
template <int DT, int GT>
__global__ __launch_bounds__(512) void wkv7_bwd_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ h_in, const float* __restrict__ ckpt, const float* __restrict__ sa,
    const float* __restrict__ dout, const float* __restrict__ dhout, void* __restrict__ g_dr,
    void* __restrict__ g_dw, void* __restrict__ g_dk, void* __restrict__ g_dv, void* __restrict__ g_da,
    void* __restrict__ g_db, float* __restrict__ dh_in, int T, int H) {
    __shared__ float stage[2][NVEC][CH][D];        // step vectors of a chunk, fp32
    // Per-wave partials, column-contiguous so a wave's 64 lanes write 64
    // consecutive words (no bank conflicts); summed over the 8 waves per column.
    __shared__ float dsa_part[2][BQ][D];           // [parity][wave][column]
    __shared__ float ring[3][NOUT][BQ][D];         // output partials of the last steps

    const int tid = threadIdx.x;
    const int i = tid & 63;                                    // key column
    const int q = __builtin_amdgcn_readfirstlane(tid >> 6);    // value rows 8q .. 8q+7
    const int jl = 8 * q + (i & 7);                            // row this lane broadcasts
    const int bh = blockIdx.x;
    const int bi = bh / H, hi = bh - bi * H;
    const int64_t strideT = (int64_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;
    const int64_t hb = (int64_t)bh * D * D;
    const int NC = T / CH;
    const void* const vec_src[6] = {r, w, k, v, a, b};
    void* const outs[NOUT] = {g_dr, g_dw, g_dk, g_db, g_dv, g_da};

    // chunk staging: thread covers 16 floats of the chunk's 8 × 16 × 64 block
    float stg[16];
    auto stage_load = [&](int c) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            const int idx = tid + 512 * m;            // (vec, step, elem)
            const int vi = idx >> 10, st = (idx >> 6) & 15, e = idx & 63;
            const int64_t off = base0 + (int64_t)(c * CH + st) * strideT + e;
            if (vi < 6) {
                switch (vi) {
                    case 0: stg[m] = load1<DT>(r, off); break;
                    case 1: stg[m] = load1<DT>(w, off); break;
                    case 2: stg[m] = load1<DT>(k, off); break;
                    case 3: stg[m] = load1<DT>(v, off); break;
                    case 4: stg[m] = load1<DT>(a, off); break;
                    default: stg[m] = load1<DT>(b, off); break;
                }
            } else {
                stg[m] = (vi == 6 ? dout : sa)[off];
            }
        }
    };
    auto stage_store = [&](int c) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            const int idx = tid + 512 * m;
            stage[c & 1][idx >> 10][(idx >> 6) & 15][idx & 63] = stg[m];
        }
    };
    (void)vec_src;

    float dT[BJ], dR[BJ];   // dS[J_q, i] (column copy) and dS[i, J_q] (row copy)
    if (dhout) {
#pragma unroll
        for (int jj = 0; jj < BJ; ++jj) dT[jj] = dhout[hb + (int64_t)(8 * q + jj) * D + i];
        const float4* src = reinterpret_cast<const float4*>(dhout + hb + (int64_t)i * D + 8 * q);
        const float4 f0 = src[0], f1 = src[1];
        dR[0] = f0.x; dR[1] = f0.y; dR[2] = f0.z; dR[3] = f0.w;
        dR[4] = f1.x; dR[5] = f1.y; dR[6] = f1.z; dR[7] = f1.w;
    } else {
#pragma unroll
        for (int jj = 0; jj < BJ; ++jj) { dT[jj] = 0.0f; dR[jj] = 0.0f; }
    }

    stage_load(NC - 1);
    stage_store(NC - 1);
    int u = 0;   // reverse step counter (parity of dsa_part, ring slot)

    // Outputs of reverse step uu (time tt): 6 × 64 sums of 8 partials, 48 per
    // wave so every wave carries the same share between two barriers.
    const int fidx = q * (NOUT * D / BQ) + i;   // output index owned by this lane (i < 48)
    const int fo = fidx >> 6, fcol = fidx & 63;
    auto flush = [&](int uu, int tt) {
        if (i < NOUT * D / BQ)
            store1<GT>(outs[fo], base0 + (int64_t)tt * strideT + fcol, sum8(&ring[uu % 3][fo][0][fcol]));
    };

    for (int c = NC - 1; c >= 0; --c) {
        __syncthreads();   // chunk c staged; every read of the other buffer is done
        if (c > 0) stage_load(c - 1);
        float (*st)[CH][D] = stage[c & 1];

        float Sst[BJ];     // state before the chunk
        if (c > 0) {
            const float* ck = ckpt + (hb * NC) + (int64_t)(c - 1) * D * D;
#pragma unroll
            for (int jj = 0; jj < BJ; ++jj) Sst[jj] = ck[(int64_t)(8 * q + jj) * D + i];
        } else if (h_in) {
#pragma unroll
            for (int jj = 0; jj < BJ; ++jj) Sst[jj] = h_in[hb + (int64_t)(8 * q + jj) * D + i];
        } else {
#pragma unroll
            for (int jj = 0; jj < BJ; ++jj) Sst[jj] = 0.0f;
        }

#pragma unroll
        for (int half = 1; half >= 0; --half) {
            // states of the window: hist[m] = state before step WIN·half + m
            float hist[WIN + 1][BJ];
            float S0[BJ];
#pragma unroll
            for (int jj = 0; jj < BJ; ++jj) S0[jj] = Sst[jj];
            if (half == 1) {
#pragma unroll
                for (int s = 0; s < WIN; ++s) {
                    float N[BJ];
                    bwd_recompute8(S0, N, st[3][s][jl], st[7][s][jl], st[2][s][i], st[5][s][i], st[1][s][i]);
#pragma unroll
                    for (int jj = 0; jj < BJ; ++jj) S0[jj] = N[jj];
                }
            }
#pragma unroll
            for (int jj = 0; jj < BJ; ++jj) hist[0][jj] = S0[jj];
#pragma unroll
            for (int m = 0; m < WIN; ++m) {
                const int s = WIN * half + m;
                bwd_recompute8(hist[m], hist[m + 1], st[3][s][jl], st[7][s][jl], st[2][s][i], st[5][s][i],
                               st[1][s][i]);
            }
            // step vectors: own column i and broadcast row jl; the next step's
            // are read before this step's barrier so they are ready after it
            struct StepVec {
                float ri, wi, ai, dyi, R, W, K, V, A, B, DY, SA;
            };
            auto load_vec = [&](int s) __attribute__((always_inline)) {
                return StepVec{st[0][s][i], st[1][s][i], st[4][s][i], st[6][s][i], st[0][s][jl], st[1][s][jl],
                               st[2][s][jl], st[3][s][jl], st[4][s][jl], st[5][s][jl], st[6][s][jl], st[7][s][jl]};
            };
            StepVec cur = load_vec(WIN * half + WIN - 1);
#pragma unroll
            for (int m = WIN - 1; m >= 0; --m, ++u) {
                const int s = WIN * half + m;
                const int t = c * CH + s;
                const float (&Sa)[BJ] = hist[m + 1];
                const float (&Sp)[BJ] = hist[m];
                const float ri = cur.ri, wi = cur.wi, ai = cur.ai, dyi = cur.dyi;
                const float R = cur.R, W = cur.W, K = cur.K, V = cur.V;
                const float A = cur.A, B = cur.B, DY = cur.DY, SA = cur.SA;
                float pdr = 0.0f, pdk = 0.0f, pdb = 0.0f, pdv = 0.0f, pds = 0.0f, pdw = 0.0f, pda = 0.0f;
                RWKV_B1_BLOCK(0, 1, 2, 3, 0);
                RWKV_B1_BLOCK(4, 5, 6, 7, 4);
                {
                    float w0 = 0.0f, w1 = 0.0f;
#pragma unroll
                    for (int jj = 0; jj < BJ; jj += 2) { w0 = fmaf(dT[jj], Sp[jj], w0); w1 = fmaf(dT[jj + 1], Sp[jj + 1], w1); }
                    pdw = w0 + w1;
                }
                RWKV_B2_BLOCK(0, 1, 2, 3, 0);
                RWKV_B2_BLOCK(4, 5, 6, 7, 4);
                const int par = u & 1, slot = u % 3;
                dsa_part[par][q][i] = pds;
                ring[slot][0][q][i] = pdr;
                ring[slot][1][q][i] = pdw;
                ring[slot][2][q][i] = pdk;
                ring[slot][3][q][i] = pdb;
                ring[slot][4][q][i] = pdv;
                StepVec nxt = cur;
                if (m > 0) nxt = load_vec(s - 1);
                __syncthreads();
                const float dsa_i = sum8(&dsa_part[par][0][i]);
                const float DS = __shfl(dsa_i, jl, 64);   // dsa of row 8q + (i & 7)
                float nR[BJ], nT[BJ];
                RWKV_B3_BLOCK(0, 1, 2, 3, 0);
                RWKV_B3_BLOCK(4, 5, 6, 7, 4);
#pragma unroll
                for (int jj = 0; jj < BJ; ++jj) {
                    dR[jj] = nR[jj];
                    dT[jj] = fmaf(wi, dT[jj], nT[jj]);
                }
                ring[slot][5][q][i] = pda;
                if (u > 0) flush(u - 1, t + 1);
                cur = nxt;
            }
        }
        if (c > 0) stage_store(c - 1);
    }
    __syncthreads();
    flush(u - 1, 0);
    float4* dst = reinterpret_cast<float4*>(dh_in + hb + (int64_t)i * D + 8 * q);
    dst[0] = make_float4(dR[0], dR[1], dR[2], dR[3]);
    dst[1] = make_float4(dR[4], dR[5], dR[6], dR[7]);
}

// ─────────────────────────────── backward, row-owned (variant 1) ───────────────────────────────
// The scheme of ckptBwdKernel (WKV7Train.swift:99-205): one wave per (b, h),
// lane i owns value row i of the state S and of its gradient C = dL/dS, both
// in VGPRs.  Each chunk starts from the state after it (the checkpoint) and
// walks its steps backward, recovering the state before a step by dividing
// by w: S_{t-1} = (S_t − v kᵀ − sa bᵀ) ⊘ w.  Per step (t descending)
//   C += dy rᵀ;  dsa = C b;  dv = C k
//   dr = S_tᵀ dy;  dw = Σ_i C ⊙ S_{t-1};  dk = Cᵀ v;  da = S_{t-1}ᵀ dsa;  db = Cᵀ sa
//   C ← C diag(w) + dsa aᵀ
// The column sums (over the lanes' rows, in row order) go through one LDS
// transpose per step: every lane writes its row of the five products as a
// column, lane j sums row j (16-byte reads).  A chunk's step vectors (and 1/w) are staged in LDS;
// the next chunk's values and checkpoint row are loaded while this one runs.
// Dividing by w amplifies the forward's rounding by up to Π 1/w over a chunk,
// the reason the default (variant 2) recomputes the states instead.
constexpr int kBwdRowsTS = D + 4;   // LDS row stride of the transposed products (16-byte rows)
constexpr int kBwdRowsLds = (CH * 8 * D + 5 * D * kBwdRowsTS) * 4;   // bytes of LDS

template <int DT, int GT>
__global__ __launch_bounds__(64) void wkv7_bwd_rows_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ h_ckpt, const float* __restrict__ sa, const float* __restrict__ d_out,
    const float* __restrict__ d_h_out, void* __restrict__ dr, void* __restrict__ dw, void* __restrict__ dk,
    void* __restrict__ dv, void* __restrict__ da, void* __restrict__ db, float* __restrict__ dh_in, int T, int H) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* sv = lds;                   // [CH][8][64]: r, w, k, a, b, 1/w, v, sa of the chunk's steps
    float* acc = lds + CH * 8 * D;     // [5][64][68]: the five products transposed (column j of lane i's row at [j][i])
    constexpr int TS = kBwdRowsTS, AS = D * TS;   // row stride, floats per product matrix
    const int i = threadIdx.x;
    const int bh = blockIdx.x, bi = bh / H, hi = bh - bi * H;
    const int NC = T / CH;
    auto elem = [&](int c, int t) { return (((int64_t)bi * T + (int64_t)c * CH + t) * H + hi) * D + i; };
    const int64_t hb = (int64_t)bh * D * D + (int64_t)i * D;

    float C[D], hr[D];
#pragma unroll
    for (int q = 0; q < D / 4; ++q) {
        const float4 f = d_h_out ? reinterpret_cast<const float4*>(d_h_out + hb)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        C[4 * q] = f.x; C[4 * q + 1] = f.y; C[4 * q + 2] = f.z; C[4 * q + 3] = f.w;
    }
    // the chunk's per-lane values: r, w, k, a, b, v, sa, dy per step, and its
    // checkpoint row; fetched one chunk ahead (clamped at chunk 0: its values
    // again, unused)
    float pf[CH][8];
    float4 ph[D / 4];
    auto fetch = [&](int c) {
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            const int64_t e = elem(c, t);
            pf[t][0] = load1<DT>(r, e);
            pf[t][1] = load1<DT>(w, e);
            pf[t][2] = load1<DT>(k, e);
            pf[t][3] = load1<DT>(a, e);
            pf[t][4] = load1<DT>(b, e);
            pf[t][5] = load1<DT>(v, e);
            pf[t][6] = sa[e];
            pf[t][7] = d_out[e];
        }
        const float4* src = reinterpret_cast<const float4*>(h_ckpt + ((int64_t)bh * NC + c) * D * D + (int64_t)i * D);
#pragma unroll
        for (int q = 0; q < D / 4; ++q) ph[q] = src[q];
    };
    fetch(NC - 1);
    for (int c = NC - 1; c >= 0; --c) {
        float dyc[CH];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            float* V = sv + t * 8 * D;
            V[0 * D + i] = pf[t][0];
            V[1 * D + i] = pf[t][1];
            V[2 * D + i] = pf[t][2];
            V[3 * D + i] = pf[t][3];
            V[4 * D + i] = pf[t][4];
            V[5 * D + i] = 1.0f / pf[t][1];
            V[6 * D + i] = pf[t][5];
            V[7 * D + i] = pf[t][6];
            dyc[t] = pf[t][7];
        }
#pragma unroll
        for (int q = 0; q < D / 4; ++q) {
            hr[4 * q] = ph[q].x; hr[4 * q + 1] = ph[q].y; hr[4 * q + 2] = ph[q].z; hr[4 * q + 3] = ph[q].w;
        }
        fetch(max(c - 1, 0));
        __syncthreads();
#pragma unroll 1
        for (int t = CH - 1; t >= 0; --t) {
            const float* V = sv + t * 8 * D;
            // the step vectors are the same for every lane: 16-byte broadcast reads
            const float4* V4 = reinterpret_cast<const float4*>(V);
            auto vec = [&](int q, int j4) { return V4[q * (D / 4) + j4]; };
            const float dy = dyc[t], vi = V[6 * D + i], sai = V[7 * D + i];
#pragma unroll
            for (int j4 = 0; j4 < D / 4; ++j4) {
                const float4 rr = vec(0, j4);
                C[4 * j4] = fmaf(dy, rr.x, C[4 * j4]);
                C[4 * j4 + 1] = fmaf(dy, rr.y, C[4 * j4 + 1]);
                C[4 * j4 + 2] = fmaf(dy, rr.z, C[4 * j4 + 2]);
                C[4 * j4 + 3] = fmaf(dy, rr.w, C[4 * j4 + 3]);
            }
            float dsa = 0.0f, dvv = 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < D / 4; ++j4) {
                const float4 bb = vec(4, j4), kk = vec(2, j4);
                dsa = fmaf(C[4 * j4], bb.x, dsa);
                dvv = fmaf(C[4 * j4], kk.x, dvv);
                dsa = fmaf(C[4 * j4 + 1], bb.y, dsa);
                dvv = fmaf(C[4 * j4 + 1], kk.y, dvv);
                dsa = fmaf(C[4 * j4 + 2], bb.z, dsa);
                dvv = fmaf(C[4 * j4 + 2], kk.z, dvv);
                dsa = fmaf(C[4 * j4 + 3], bb.w, dsa);
                dvv = fmaf(C[4 * j4 + 3], kk.w, dvv);
            }
            const int64_t e = elem(c, t);
            store1<GT>(dv, e, dvv);
            float* col = acc + i;   // lane i writes element i of every transposed row
#pragma unroll
            for (int j4 = 0; j4 < D / 4; ++j4) {
                const float4 kk = vec(2, j4), bb = vec(4, j4), iw = vec(5, j4);
                const float kv[4] = {kk.x, kk.y, kk.z, kk.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w};
                const float wv[4] = {iw.x, iw.y, iw.z, iw.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int j = 4 * j4 + u;
                    col[j * TS] = dy * hr[j];
                    hr[j] = (hr[j] - vi * kv[u] - sai * bv[u]) * wv[u];
                    col[AS + j * TS] = C[j] * hr[j];
                    col[2 * AS + j * TS] = C[j] * vi;
                    col[3 * AS + j * TS] = dsa * hr[j];
                    col[4 * AS + j * TS] = sai * C[j];
                }
            }
            __syncthreads();
            // column i of each product is row i of its transpose: 16-byte
            // reads, summed over the lanes' rows in order
            float gs[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < 5; ++m) {
                const float4* tr = reinterpret_cast<const float4*>(acc + m * AS + i * TS);
#pragma unroll
                for (int s4 = 0; s4 < D / 4; ++s4) {
                    const float4 f = tr[s4];
                    gs[m] += f.x;
                    gs[m] += f.y;
                    gs[m] += f.z;
                    gs[m] += f.w;
                }
            }
            store1<GT>(dr, e, gs[0]);
            store1<GT>(dw, e, gs[1]);
            store1<GT>(dk, e, gs[2]);
            store1<GT>(da, e, gs[3]);
            store1<GT>(db, e, gs[4]);
#pragma unroll
            for (int j4 = 0; j4 < D / 4; ++j4) {
                const float4 ww = vec(1, j4), aa = vec(3, j4);
                C[4 * j4] = fmaf(C[4 * j4], ww.x, dsa * aa.x);
                C[4 * j4 + 1] = fmaf(C[4 * j4 + 1], ww.y, dsa * aa.y);
                C[4 * j4 + 2] = fmaf(C[4 * j4 + 2], ww.z, dsa * aa.z);
                C[4 * j4 + 3] = fmaf(C[4 * j4 + 3], ww.w, dsa * aa.w);
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int q = 0; q < D / 4; ++q)
        reinterpret_cast<float4*>(dh_in + hb)[q] = make_float4(C[4 * q], C[4 * q + 1], C[4 * q + 2], C[4 * q + 3]);
}

// ─────────────────────────────── tmix tail ───────────────────────────────

// y·g rounded to fp32, then converted to TO: for fp16 the fp32 output's
// value rounded once more.  The empty asm keeps the fp32 product: without it
// the compiler folds multiply and conversion into one v_fma_mixlo_f16, which
// rounds the exact product straight to fp16.
template <typename TO>
__device__ __forceinline__ TO tail_out(float y, float g) {
    float o = y * g;
    asm("" : "+v"(o));
    return (TO)o;
}

// One wave per (row, head), four to a workgroup; the output fp32, or fp16
// (TO = _Float16: the rounding the fp16 long pass of o_proj applies to its
// input, so the projection reads the same values from half the bytes).
template <typename TO>
__global__ __launch_bounds__(256) void wkv_tail_kernel(
    const float* __restrict__ wkv, const float* __restrict__ r, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ rk, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const float* __restrict__ g, TO* __restrict__ out,
    int NH, int H, int S, float eps) {
    const int tg = blockIdx.x * 4 + (threadIdx.x >> 6);   // row * H + head
    if (tg >= NH) return;   // whole waves; no barrier below
    const int h = tg % H;
    const int64_t base = (int64_t)tg * S, hb = (int64_t)h * S;
    const int lane = threadIdx.x & 63;
    if (S == 64) {
        // one element per lane, every load issued up front; the operations
        // of the loops below for their single pass, so the same bits
        const int64_t i = base + lane, j = hb + lane;
        const float wv = wkv[i], rv = r[i], kv = k[i], vv = v[i], gv = g[i];
        const float rkv = rk[j], lw = lnw[j], lb = lnb[j];
        float t1 = 0.0f;
        t1 += wv;
        const float mean = wave_total(t1) / 64.0f;
        const float d = wv - mean;
        const float inv = 1.0f / sqrtf(wave_total(fmaf(d, d, 0.0f)) / 64.0f + eps);
        const float dp = wave_total(fmaf(rv * kv, rkv, 0.0f));
        const float y = fmaf(dp, vv, fmaf((wv - mean) * inv, lw, lb));
        out[i] = tail_out<TO>(y, gv);
        return;
    }
    float s1 = 0.0f;
    for (int e = lane; e < S; e += 64) s1 += wkv[base + e];
    const float mean = wave_total(s1) / (float)S;
    float s2 = 0.0f;
    for (int e = lane; e < S; e += 64) {
        const float d = wkv[base + e] - mean;
        s2 = fmaf(d, d, s2);
    }
    const float inv = 1.0f / sqrtf(wave_total(s2) / (float)S + eps);
    float dp = 0.0f;
    for (int e = lane; e < S; e += 64) dp = fmaf(r[base + e] * k[base + e], rk[hb + e], dp);
    dp = wave_total(dp);
    for (int e = lane; e < S; e += 64) {
        const float nrm = (wkv[base + e] - mean) * inv;
        const float y = fmaf(dp, v[base + e], fmaf(nrm, lnw[hb + e], lnb[hb + e]));
        out[base + e] = tail_out<TO>(y, g[base + e]);
    }
}

// ─────────────────────────────── decode: step + tail in one launch ───────────────────────────────
// One workgroup per (row, head): four waves (sixteen-row layout) or sixteen
// (four-row layout, B·H < 256), each the T = 1 path of the forward kernel for
// its rows (head_step16 / head_step4: the same operations, so state and wkv
// are bitwise those of rwkv_wkv7_step); the head's 64 wkv values meet in LDS
// and wave 0 applies the tail with wkv_tail_kernel's operation sequence for
// S = 64 (head_tail).
template <bool R4>
__global__ __launch_bounds__(R4 ? 1024 : 256) void wkv7_step_tail_kernel(
    const float* __restrict__ r, const float* __restrict__ w, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ h_in, float* __restrict__ h_out, const float* __restrict__ rk,
    const float* __restrict__ lnw, const float* __restrict__ lnb, const float* __restrict__ g,
    float* __restrict__ wkv_out, float* __restrict__ out, int H, float eps) {
    __shared__ float ys[D];
    const int blk = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int bh = blockIdx.x;
    const int hi = bh % H;
    const int64_t base0 = (int64_t)bh * D;   // [B, H, 64]
    const int64_t hb = (int64_t)bh * D * D;
    const int row = R4 ? step4_row(blk, l) : step16_row(blk, l);
    const float A = a[base0 + l], W = w[base0 + l], K = k[base0 + l], Bv = b[base0 + l];
    const float R = r[base0 + l], V = v[base0 + row];
    const float* hin = h_in ? h_in + hb : nullptr;
    float S[R4 ? 4 : 16];
    if constexpr (R4) load_state4(hin, blk, l, S);
    else load_state16(hin, blk, l, S);
    // the tail's other inputs (wave 0; r and k of column l are R and K) do not
    // depend on the step: loaded with the state, not after the barrier
    const int64_t e = base0 + l, he = (int64_t)hi * D + l;
    float tv = 0.0f, trk = 0.0f, tlnw = 0.0f, tlnb = 0.0f, tg = 0.0f;
    if (blk == 0) {   // uniform per wave
        tv = v[e];
        trk = rk[he];
        tlnw = lnw[he];
        tlnb = lnb[he];
        tg = g[e];
    }
    float y;
    if constexpr (R4) y = head_step4_regs(S, h_out + hb, blk, l, A, W, K, Bv, R, V);
    else y = head_step16_regs(S, h_out + hb, blk, l, A, W, K, Bv, R, V);
    if ((R4 ? (l >> 2) : (l >> 4)) == 0) {
        ys[row] = y;
        if (wkv_out) wkv_out[base0 + row] = y;
    }
    __syncthreads();
    if (blk == 0) out[e] = head_tail(ys[l], R, K, tv, trk, tlnw, tlnb, tg, eps);
}

// ─────────────────────────────── host dispatch ───────────────────────────────
rwkv_status launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        rwkv::set_error("%s: %s", what, hipGetErrorString(e));
        return RWKV_E_HIP;
    }
    rwkv::clear_error();
    return RWKV_OK;
}

template <bool SA, bool CK>
rwkv_status launch_fwd(const void* r, const void* w, const void* k, const void* v, const void* a, const void* b,
                       rwkv_dtype dt, const float* h_in, float* out, float* h_out, float* sa_out, float* ck,
                       int64_t B, int64_t T, int64_t H, void* stream) {
    const bool rows4 = use_rows4(B * H);
    dim3 grid((unsigned)(B * H * (rows4 ? 16 : 4))), block(64);   // one wave per 4 / 16 value rows
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RWKV_FWD(DTV)                                                                                        \
    if (rows4)                                                                                               \
        rwkv::launch(wkv7_fwd4_kernel<DTV, SA, CK>, grid, block, st, r, w, k, v, a, b, h_in, out, h_out, sa_out, \
                     ck, (int)T, (int)H);                                                                    \
    else                                                                                                     \
        rwkv::launch(wkv7_fwd_kernel<DTV, SA, CK>, grid, block, st, r, w, k, v, a, b, h_in, out, h_out, sa_out,  \
                     ck, (int)T, (int)H)
    switch (dt) {
        case RWKV_F32: RWKV_FWD(RWKV_F32); break;
        case RWKV_BF16: RWKV_FWD(RWKV_BF16); break;
        case RWKV_F16: RWKV_FWD(RWKV_F16); break;
    }
#undef RWKV_FWD
    return launch_status("wkv7 forward launch");
}

rwkv_status check_wkv_common(const void* r, const void* w, const void* k, const void* v, const void* a,
                             const void* b, int dt, int64_t B, int64_t T, int64_t H) {
    RWKV_REQUIRE(r && w && k && v && a && b, RWKV_E_NULL, "wkv7: r/w/k/v/a/b must be non-null");
    RWKV_REQUIRE(rwkv::dtype_ok(dt), RWKV_E_DTYPE, "wkv7: input dtype code %d not in {f32, bf16, f16}", dt);
    RWKV_REQUIRE(B >= 1 && H >= 1, RWKV_E_SHAPE, "wkv7: B (%lld) and H (%lld) must be >= 1", (long long)B, (long long)H);
    RWKV_REQUIRE(T >= 1, RWKV_E_SHAPE, "wkv7: T (%lld) must be >= 1", (long long)T);
    RWKV_REQUIRE(B * H * 4 <= INT32_MAX && T * H * 64 * 4 < ((int64_t)1 << 32) && B * T * H * 64 <= (int64_t)1 << 46,
                 RWKV_E_SHAPE, "wkv7: B·T·H too large (one sequence must stay under 2^32 bytes)");
    return RWKV_OK;
}

}  // namespace

extern "C" {

int rwkv_wkv7_head_size(void) { return D; }
int rwkv_wkv7_chunk(void) { return CH; }

rwkv_status rwkv_wkv7_seq_fwd(const void* r, const void* w, const void* k, const void* v, const void* a,
                              const void* b, rwkv_dtype in_dt, const float* h_in, float* out, float* h_out,
                              int64_t B, int64_t T, int64_t H, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, T, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(out && h_out, RWKV_E_NULL, "wkv7_seq_fwd: out and h_out must be non-null");
    s = launch_fwd<false, false>(r, w, k, v, a, b, in_dt, h_in, out, h_out, nullptr, nullptr, B, T, H, stream);
    if (s == RWKV_OK) rwkv::counters().seq_fwd++;
    return s;
}

rwkv_status rwkv_wkv7_chunk_fwd(const void* r, const void* w, const void* k, const void* v, const void* a,
                                const void* b, rwkv_dtype in_dt, const float* h_in, float* out, float* h_out,
                                float* sa_out, int64_t B, int64_t T, int64_t H, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, T, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(T == CH, RWKV_E_SHAPE, "wkv7_chunk_fwd: T (%lld) must equal CHUNK %d", (long long)T, CH);
    RWKV_REQUIRE(h_in && out && h_out && sa_out, RWKV_E_NULL, "wkv7_chunk_fwd: h_in/out/h_out/sa_out must be non-null");
    s = launch_fwd<true, false>(r, w, k, v, a, b, in_dt, h_in, out, h_out, sa_out, nullptr, B, T, H, stream);
    if (s == RWKV_OK) rwkv::counters().chunk_fwd++;
    return s;
}

rwkv_status rwkv_wkv7_train_fwd(const void* r, const void* w, const void* k, const void* v, const void* a,
                                const void* b, rwkv_dtype in_dt, const float* h_in, float* out, float* h_out,
                                float* sa_out, float* h_ckpt, int64_t B, int64_t T, int64_t H, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, T, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(T % CH == 0, RWKV_E_SHAPE, "wkv7_train_fwd: T (%lld) must be a multiple of CHUNK %d", (long long)T, CH);
    RWKV_REQUIRE(out && h_out && sa_out && h_ckpt, RWKV_E_NULL, "wkv7_train_fwd: out/h_out/sa_out/h_ckpt must be non-null");
    s = launch_fwd<true, true>(r, w, k, v, a, b, in_dt, h_in, out, h_out, sa_out, h_ckpt, B, T, H, stream);
    if (s == RWKV_OK) rwkv::counters().train_fwd++;
    return s;
}

rwkv_status rwkv_wkv7_step(const void* r, const void* w, const void* k, const void* v, const void* a,
                           const void* b, rwkv_dtype in_dt, const float* h_in, float* out, float* h_out,
                           int64_t B, int64_t H, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, 1, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(out && h_out, RWKV_E_NULL, "wkv7_step: out and h_out must be non-null");
    s = launch_fwd<false, false>(r, w, k, v, a, b, in_dt, h_in, out, h_out, nullptr, nullptr, B, 1, H, stream);
    if (s == RWKV_OK) rwkv::counters().step++;
    return s;
}

rwkv_status rwkv_wkv7_train_bwd(const void* r, const void* w, const void* k, const void* v, const void* a,
                                const void* b, rwkv_dtype in_dt, const float* h_in, const float* h_ckpt,
                                const float* sa, const float* d_out, const float* d_h_out, void* dr, void* dw,
                                void* dk, void* dv, void* da, void* db, rwkv_dtype g_dt, float* dh_in, int64_t B,
                                int64_t T, int64_t H, int variant, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, T, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(T % CH == 0, RWKV_E_SHAPE, "wkv7_train_bwd: T (%lld) must be a multiple of CHUNK %d", (long long)T, CH);
    RWKV_REQUIRE(h_ckpt && sa && d_out && dr && dw && dk && dv && da && db && dh_in, RWKV_E_NULL,
                 "wkv7_train_bwd: checkpoints, sa, d_out, gradients and dh_in must be non-null");
    RWKV_REQUIRE(rwkv::dtype_ok(g_dt), RWKV_E_DTYPE, "wkv7_train_bwd: gradient dtype code %d not in {f32, bf16, f16}", g_dt);
    RWKV_REQUIRE(variant == 1 || variant == 2, RWKV_E_UNSUPPORTED, "wkv7_train_bwd: variant %d not in {1, 2}", variant);
    dim3 grid((unsigned)(B * H)), block(512);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RWKV_BWD_LAUNCH(DT, GT)                                                                          \
    rwkv::launch(wkv7_bwd_kernel<DT, GT>, grid, block, st, r, w, k, v, a, b, h_in, h_ckpt, sa, \
                       d_out, d_h_out, dr, dw, dk, dv, da, db, dh_in, (int)T, (int)H)
#define RWKV_BWD_GT(DT)                                         \
    switch (g_dt) {                                                  \
        case RWKV_F32: RWKV_BWD_LAUNCH(DT, RWKV_F32); break;   \
        case RWKV_BF16: RWKV_BWD_LAUNCH(DT, RWKV_BF16); break; \
        case RWKV_F16: RWKV_BWD_LAUNCH(DT, RWKV_F16); break;   \
    }
#define RWKV_BWD_DT()                                  \
    switch (in_dt) {                                      \
        case RWKV_F32: RWKV_BWD_GT(RWKV_F32); break;   \
        case RWKV_BF16: RWKV_BWD_GT(RWKV_BF16); break; \
        case RWKV_F16: RWKV_BWD_GT(RWKV_F16); break;   \
    }
#define RWKV_ROWS_LAUNCH(DT, GT)                                                                              \
    rwkv::launch_lds(wkv7_bwd_rows_kernel<DT, GT>, dim3((unsigned)(B * H)), dim3(64), (size_t)kBwdRowsLds, st, r, \
                     w, k, v, a, b, h_ckpt, sa, d_out, d_h_out, dr, dw, dk, dv, da, db, dh_in, (int)T, (int)H)
#define RWKV_ROWS_GT(DT)                                           \
    switch (g_dt) {                                                \
        case RWKV_F32: RWKV_ROWS_LAUNCH(DT, RWKV_F32); break;   \
        case RWKV_BF16: RWKV_ROWS_LAUNCH(DT, RWKV_BF16); break; \
        case RWKV_F16: RWKV_ROWS_LAUNCH(DT, RWKV_F16); break;   \
    }
    if (variant == 2) {
        RWKV_BWD_DT()
    } else {
        switch (in_dt) {
            case RWKV_F32: RWKV_ROWS_GT(RWKV_F32); break;
            case RWKV_BF16: RWKV_ROWS_GT(RWKV_BF16); break;
            case RWKV_F16: RWKV_ROWS_GT(RWKV_F16); break;
        }
    }
#undef RWKV_ROWS_GT
#undef RWKV_ROWS_LAUNCH
#undef RWKV_BWD_DT
#undef RWKV_BWD_GT
#undef RWKV_BWD_LAUNCH
    s = launch_status("wkv7 backward launch");
    if (s == RWKV_OK) rwkv::counters().train_bwd++;
    return s;
}

rwkv_status rwkv_wkv7_step_tail(const float* r, const float* w, const float* k, const float* v, const float* a,
                                const float* b, const float* h_in, float* h_out, const float* rk, const float* lnw,
                                const float* lnb, const float* g, float* wkv_out, float* out, int64_t B, int64_t H,
                                float eps, void* stream) {
    RWKV_REQUIRE(r && w && k && v && a && b && h_out && rk && lnw && lnb && g && out, RWKV_E_NULL,
                 "wkv7_step_tail: null buffer");
    RWKV_REQUIRE(B >= 1 && H >= 1 && B * H <= INT32_MAX, RWKV_E_SHAPE, "wkv7_step_tail: bad B (%lld) / H (%lld)",
                 (long long)B, (long long)H);
    if (use_rows4(B * H))
        rwkv::launch(wkv7_step_tail_kernel<true>, dim3((unsigned)(B * H)), dim3(1024),
                     reinterpret_cast<hipStream_t>(stream), r, w, k, v, a, b, h_in, h_out, rk, lnw, lnb, g, wkv_out,
                     out, (int)H, eps);
    else
        rwkv::launch(wkv7_step_tail_kernel<false>, dim3((unsigned)(B * H)), dim3(256),
                     reinterpret_cast<hipStream_t>(stream), r, w, k, v, a, b, h_in, h_out, rk, lnw, lnb, g, wkv_out,
                     out, (int)H, eps);
    rwkv_status s = launch_status("wkv7_step_tail launch");
    if (s == RWKV_OK) rwkv::counters().step_tail++;
    return s;
}

int rwkv_wkv_tail_applies(int64_t S) { return S > 0 && S % 32 == 0; }

rwkv_status rwkv_wkv_tail_to(const float* wkv, const float* r, const float* k, const float* v, const float* rk,
                             const float* lnw, const float* lnb, const float* g, void* out, rwkv_dtype out_dt,
                             int64_t N, int64_t H, int64_t S, float eps, void* stream) {
    RWKV_REQUIRE(wkv && r && k && v && rk && lnw && lnb && g && out, RWKV_E_NULL, "wkv_tail: null buffer");
    RWKV_REQUIRE(out_dt == RWKV_F32 || out_dt == RWKV_F16, RWKV_E_DTYPE, "wkv_tail: output dtype %d not f32/f16",
                 (int)out_dt);
    RWKV_REQUIRE(rwkv_wkv_tail_applies(S), RWKV_E_SHAPE, "wkv_tail: S=%lld is not a multiple of 32", (long long)S);
    RWKV_REQUIRE(N >= 1 && H >= 1 && N * H <= INT32_MAX - 3 && S <= 1 << 20, RWKV_E_SHAPE, "wkv_tail: bad N/H/S");
    const dim3 grid((unsigned)((N * H + 3) / 4)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (out_dt == RWKV_F16)
        rwkv::launch(wkv_tail_kernel<_Float16>, grid, block, st, wkv, r, k, v, rk, lnw, lnb, g,
                     reinterpret_cast<_Float16*>(out), (int)(N * H), (int)H, (int)S, eps);
    else
        rwkv::launch(wkv_tail_kernel<float>, grid, block, st, wkv, r, k, v, rk, lnw, lnb, g,
                     reinterpret_cast<float*>(out), (int)(N * H), (int)H, (int)S, eps);
    rwkv_status s = launch_status("wkv_tail launch");
    if (s == RWKV_OK) rwkv::counters().tail++;
    return s;
}

rwkv_status rwkv_wkv_tail(const float* wkv, const float* r, const float* k, const float* v, const float* rk,
                          const float* lnw, const float* lnb, const float* g, float* out, int64_t N, int64_t H,
                          int64_t S, float eps, void* stream) {
    return rwkv_wkv_tail_to(wkv, r, k, v, rk, lnw, lnb, g, out, RWKV_F32, N, H, S, eps, stream);
}

}  // extern "C"
