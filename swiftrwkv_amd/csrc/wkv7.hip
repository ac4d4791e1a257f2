// WKV-7 recurrence on gfx950: whole-sequence / chunk / training forward, the
// checkpointed backward, the one-token decode step and the tmix tail.
//
// Recurrence per (b, h), state S[i = value row, j = key column] (fp32):
//   sa_i = Σ_j S_ij a_j ;  S_ij ← w_j S_ij + v_i k_j + sa_i b_j ;  y_i = Σ_j S_ij r_j
// (Sources/RWKVKernel/WKV7.swift:207-224).
//
// Forward work split (one 256-thread workgroup per (b, h)):
//   wave q (0..3) owns key columns J_q = [16q, 16q+16); lane i owns value row i.
//   Each lane keeps its 16 state values in VGPRs for the whole sequence.  The
//   per-step vectors a/w/k/b/r restricted to J_q are the same for all 64 lanes
//   of a wave, so they are read with wave-uniform (scalar) loads and used as
//   SGPR operands: no LDS fan-out of the step vectors.  The only exchange per
//   step is sa: four partial sums per row through LDS (double-buffered by step
//   parity, one barrier per step).  The four partial y's go to an LDS ring
//   that is summed and stored (coalesced) once every 16 steps.
//   The step kernel, the chunk kernel and the training forward are this same
//   kernel with T = 1 / emitted sa / emitted checkpoints, so they agree
//   bitwise by construction (the reference's own invariants:
//   WKV7SequenceTests, WKV7StateTests.swift:178-186, DecodeKernelTests.swift:27-39).
//
// Backward (variant 2, column-owned like ckptBwdKernelV2, WKV7Train.swift:234-339):
//   lane i owns key column i; wave q owns value rows J_q.  A lane holds
//   S[J_q, i], dS[J_q, i] and the row copy dS[i, J_q], so dr/dw/dk/db/da are
//   in-lane partial dots over J_q and dv/dsa are in-lane partial dots of the
//   row copy.  dsa is the one quantity exchanged within the step; every output
//   is summed over the four waves through an LDS ring, 4 steps at a time.
//
// All arithmetic is fp32 with fixed summation order, so every launch is
// bitwise deterministic.

#include <hip/hip_runtime.h>

#include "common.h"

namespace {

constexpr int D = 64;   // WKV7_HEAD_SIZE
constexpr int CH = 16;  // WKV7_CHUNK
constexpr int NQ = 4;   // waves per workgroup
constexpr int JW = 16;  // key columns (fwd) / value rows (bwd) per wave

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float f16_lo(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

// 16 consecutive elements starting at element `off` (off % 16 == 0), widened
// to fp32.  Called with wave-uniform addresses, so the compiler can use scalar
// loads.
template <int DT>
__device__ __forceinline__ void load16(const void* __restrict__ p, int64_t off, float (&o)[JW]) {
    if constexpr (DT == RWKV_F32) {
        const float* q = reinterpret_cast<const float*>(p) + off;
#pragma unroll
        for (int c = 0; c < JW; ++c) o[c] = q[c];
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(p) + off);
#pragma unroll
        for (int c = 0; c < JW / 2; ++c) {
            uint32_t u = q[c];
            if constexpr (DT == RWKV_BF16) {
                o[2 * c] = bf16_lo(u);
                o[2 * c + 1] = bf16_hi(u);
            } else {
                o[2 * c] = f16_lo(u);
                o[2 * c + 1] = f16_hi(u);
            }
        }
    }
}

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

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// ─────────────────────────────── forward ───────────────────────────────
template <int DT, bool EMIT_SA, bool EMIT_CK>
__global__ __launch_bounds__(256) void wkv7_fwd_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ h_in, float* __restrict__ out, float* __restrict__ h_out,
    float* __restrict__ sa_out, float* __restrict__ ckpt, int T, int H) {
    __shared__ float4 sa_part[2][D];      // [step parity][row] = partial sa of waves 0..3
    __shared__ float4 y_ring[2][CH][D];   // [chunk parity][step][row] = partial y of waves 0..3

    const int i = threadIdx.x & 63;
    const int q = wave_id();
    const int bh = blockIdx.x;
    const int bi = bh / H, hi = bh - bi * H;
    const int64_t sbase = (int64_t)bh * D * D + (int64_t)i * D + JW * q;   // S[i, J_q]
    const int64_t strideT = (int64_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;                  // (bi, t=0, hi, 0)
    const int NC = T / CH;

    float S[JW];
    if (h_in) {
        const float4* src = reinterpret_cast<const float4*>(h_in + sbase);
#pragma unroll
        for (int c = 0; c < JW / 4; ++c) {
            float4 f = src[c];
            S[4 * c] = f.x; S[4 * c + 1] = f.y; S[4 * c + 2] = f.z; S[4 * c + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < JW; ++c) S[c] = 0.0f;
    }

    const int nchunks = (T + CH - 1) / CH;
    for (int c = 0; c < nchunks; ++c) {
        const int t0 = c * CH;
        const int n = min(CH, T - t0);
        const int half = c & 1;
        float vreg[CH];
#pragma unroll
        for (int s = 0; s < CH; ++s) vreg[s] = (s < n) ? load1<DT>(v, base0 + (int64_t)(t0 + s) * strideT + i) : 0.0f;

#pragma unroll
        for (int s = 0; s < CH; ++s) {
            if (s < n) {
                const int t = t0 + s;
                const int64_t bt = base0 + (int64_t)t * strideT;
                float av[JW];
                load16<DT>(a, bt + JW * q, av);
                float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
                for (int j = 0; j < JW; j += 2) {
                    p0 = fmaf(S[j], av[j], p0);
                    p1 = fmaf(S[j + 1], av[j + 1], p1);
                }
                reinterpret_cast<float*>(&sa_part[t & 1][i])[q] = p0 + p1;
                float wv[JW], kv[JW], bv[JW], rv[JW];
                load16<DT>(w, bt + JW * q, wv);
                load16<DT>(k, bt + JW * q, kv);
                load16<DT>(b, bt + JW * q, bv);
                load16<DT>(r, bt + JW * q, rv);
                __syncthreads();
                const float4 pp = sa_part[t & 1][i];
                const float sa = (pp.x + pp.y) + (pp.z + pp.w);
                if (EMIT_SA && q == 0) sa_out[bt + i] = sa;
                const float vv = vreg[s];
                float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
                for (int j = 0; j < JW; j += 2) {
                    S[j] = fmaf(wv[j], S[j], fmaf(sa, bv[j], vv * kv[j]));
                    S[j + 1] = fmaf(wv[j + 1], S[j + 1], fmaf(sa, bv[j + 1], vv * kv[j + 1]));
                    y0 = fmaf(S[j], rv[j], y0);
                    y1 = fmaf(S[j + 1], rv[j + 1], y1);
                }
                reinterpret_cast<float*>(&y_ring[half][s][i])[q] = y0 + y1;
                if (EMIT_CK && s == CH - 1) {
                    float4* dst = reinterpret_cast<float4*>(ckpt + ((int64_t)bh * NC + c) * D * D + (int64_t)i * D + JW * q);
#pragma unroll
                    for (int m = 0; m < JW / 4; ++m) dst[m] = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
                }
            }
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < n * D; idx += NQ * 64) {
            const int s = idx >> 6, row = idx & 63;
            const float4 p = y_ring[half][s][row];
            out[base0 + (int64_t)(t0 + s) * strideT + row] = (p.x + p.y) + (p.z + p.w);
        }
    }
    float4* dst = reinterpret_cast<float4*>(h_out + sbase);
#pragma unroll
    for (int m = 0; m < JW / 4; ++m) dst[m] = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
}

// ─────────────────────────────── backward (column-owned) ───────────────────────────────
constexpr int BG = 4;   // steps per output flush
constexpr int NOUT = 6; // dr, dw, dk, db, dv, da

template <int DT, int GT>
__global__ __launch_bounds__(256) void wkv7_bwd_v2_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ ckpt, const float* __restrict__ sa, const float* __restrict__ dout,
    const float* __restrict__ dhout, void* __restrict__ g_dr, void* __restrict__ g_dw,
    void* __restrict__ g_dk, void* __restrict__ g_dv, void* __restrict__ g_da, void* __restrict__ g_db,
    float* __restrict__ dh_in, int T, int H) {
    __shared__ float4 dsa_part[2][D];           // [parity][column i] partial dsa (rows of waves 0..3)
    __shared__ float4 ring[2][BG][NOUT][D];     // [group parity][slot][output][column]

    const int i = threadIdx.x & 63;   // key column owned by this lane
    const int q = wave_id();          // value rows J_q
    const int bh = blockIdx.x;
    const int bi = bh / H, hi = bh - bi * H;
    const int64_t strideT = (int64_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;
    const int NC = T / CH;
    const int64_t hb = (int64_t)bh * D * D;

    float sT[JW], dT[JW], dR[JW];   // S[J_q, i], dS[J_q, i], dS[i, J_q]
    if (dhout) {
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) dT[jj] = dhout[hb + (int64_t)(JW * q + jj) * D + i];
        const float4* src = reinterpret_cast<const float4*>(dhout + hb + (int64_t)i * D + JW * q);
#pragma unroll
        for (int m = 0; m < JW / 4; ++m) {
            float4 f = src[m];
            dR[4 * m] = f.x; dR[4 * m + 1] = f.y; dR[4 * m + 2] = f.z; dR[4 * m + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) { dT[jj] = 0.0f; dR[jj] = 0.0f; }
    }

    void* const outs[NOUT] = {g_dr, g_dw, g_dk, g_db, g_dv, g_da};
    int step = 0;   // reverse-step counter
    for (int c = NC - 1; c >= 0; --c) {
        const float* ck = ckpt + (hb * NC) + (int64_t)c * D * D;
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) sT[jj] = ck[(int64_t)(JW * q + jj) * D + i];

        for (int s = CH - 1; s >= 0; --s, ++step) {
            const int t = c * CH + s;
            const int64_t bt = base0 + (int64_t)t * strideT;
            const int grp = step / BG, slot = step - grp * BG, gh = grp & 1;
            const float ri = load1<DT>(r, bt + i), wi = load1<DT>(w, bt + i), ki = load1<DT>(k, bt + i);
            const float ai = load1<DT>(a, bt + i), bI = load1<DT>(b, bt + i), dyi = dout[bt + i];

            float dyj[JW], saj[JW], vj[JW], rj[JW];
            load16<RWKV_F32>(dout, bt + JW * q, dyj);
            load16<RWKV_F32>(sa, bt + JW * q, saj);
            load16<DT>(v, bt + JW * q, vj);
            load16<DT>(r, bt + JW * q, rj);

            // dr_i = Σ_j S_ji dy_j  (state after the step)
            float e0 = 0.0f, e1 = 0.0f;
#pragma unroll
            for (int jj = 0; jj < JW; jj += 2) { e0 = fmaf(sT[jj], dyj[jj], e0); e1 = fmaf(sT[jj + 1], dyj[jj + 1], e1); }
            const float pdr = e0 + e1;
            // S_ji ← (S_ji − v_j k_i − sa_j b_i) / w_i ;  dS += dy ⊗ r
            const float iw = 1.0f / wi;
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                sT[jj] = fmaf(-saj[jj], bI, fmaf(-vj[jj], ki, sT[jj])) * iw;
                dT[jj] = fmaf(ri, dyj[jj], dT[jj]);
                dR[jj] = fmaf(dyi, rj[jj], dR[jj]);
            }
            float kj[JW], bj[JW];
            load16<DT>(k, bt + JW * q, kj);
            load16<DT>(b, bt + JW * q, bj);
            float w0 = 0, w1 = 0, k0 = 0, k1 = 0, b0 = 0, b1 = 0, v0 = 0, v1 = 0, s0 = 0, s1 = 0;
#pragma unroll
            for (int jj = 0; jj < JW; jj += 2) {
                w0 = fmaf(dT[jj], sT[jj], w0);       w1 = fmaf(dT[jj + 1], sT[jj + 1], w1);
                k0 = fmaf(dT[jj], vj[jj], k0);       k1 = fmaf(dT[jj + 1], vj[jj + 1], k1);
                b0 = fmaf(dT[jj], saj[jj], b0);      b1 = fmaf(dT[jj + 1], saj[jj + 1], b1);
                v0 = fmaf(dR[jj], kj[jj], v0);       v1 = fmaf(dR[jj + 1], kj[jj + 1], v1);
                s0 = fmaf(dR[jj], bj[jj], s0);       s1 = fmaf(dR[jj + 1], bj[jj + 1], s1);
            }
            reinterpret_cast<float*>(&dsa_part[step & 1][i])[q] = s0 + s1;
            reinterpret_cast<float*>(&ring[gh][slot][0][i])[q] = pdr;
            reinterpret_cast<float*>(&ring[gh][slot][1][i])[q] = w0 + w1;
            reinterpret_cast<float*>(&ring[gh][slot][2][i])[q] = k0 + k1;
            reinterpret_cast<float*>(&ring[gh][slot][3][i])[q] = b0 + b1;
            reinterpret_cast<float*>(&ring[gh][slot][4][i])[q] = v0 + v1;
            float wj[JW], aj[JW];
            load16<DT>(w, bt + JW * q, wj);
            load16<DT>(a, bt + JW * q, aj);
            __syncthreads();
            const float4 pp = dsa_part[step & 1][i];
            const float dsa_i = (pp.x + pp.y) + (pp.z + pp.w);
            float dsaj[JW];
#pragma unroll
            for (int jj = 0; jj < JW; ++jj)
                dsaj[jj] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsa_i), JW * q + jj));
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int jj = 0; jj < JW; jj += 2) { a0 = fmaf(sT[jj], dsaj[jj], a0); a1 = fmaf(sT[jj + 1], dsaj[jj + 1], a1); }
            reinterpret_cast<float*>(&ring[gh][slot][5][i])[q] = a0 + a1;
            // dS_ij ← dS_ij w_j + dsa_i a_j   (row copy and column copy)
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                dR[jj] = fmaf(dR[jj], wj[jj], dsa_i * aj[jj]);
                dT[jj] = fmaf(dT[jj], wi, ai * dsaj[jj]);
            }
            if (slot == BG - 1 || t == 0) {
                __syncthreads();
                const int nslot = slot + 1;
                for (int idx = threadIdx.x; idx < nslot * NOUT * D; idx += NQ * 64) {
                    const int sl = idx / (NOUT * D);
                    const int rem = idx - sl * NOUT * D;
                    const int o = rem >> 6, col = rem & 63;
                    const float4 p = ring[gh][sl][o][col];
                    const int tt = t + (slot - sl);   // slot sl of this group is time t + (slot - sl)
                    store1<GT>(outs[o], base0 + (int64_t)tt * strideT + col, (p.x + p.y) + (p.z + p.w));
                }
            }
        }
    }
    float4* dst = reinterpret_cast<float4*>(dh_in + hb + (int64_t)i * D + JW * q);
#pragma unroll
    for (int m = 0; m < JW / 4; ++m) dst[m] = make_float4(dR[4 * m], dR[4 * m + 1], dR[4 * m + 2], dR[4 * m + 3]);
}

// ─────────────────────────────── backward (row-owned, variant 1) ───────────────────────────────
// Lane i owns value row i; wave q owns key columns J_q (the forward's split).
// Row quantities (dv, dsa) are in-lane partial dots; column quantities (dr,
// dk, db, dw, da) are reduced over the 64 rows of a wave with a butterfly and
// then over the four waves through LDS.  Same math as variant 2, different
// summation order (the reference's v1 / v2 pair, WKV7Train.swift:99-205).
__device__ __forceinline__ float wave_sum64(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

template <int DT, int GT>
__global__ __launch_bounds__(256) void wkv7_bwd_v1_kernel(
    const void* __restrict__ r, const void* __restrict__ w, const void* __restrict__ k,
    const void* __restrict__ v, const void* __restrict__ a, const void* __restrict__ b,
    const float* __restrict__ ckpt, const float* __restrict__ sa, const float* __restrict__ dout,
    const float* __restrict__ dhout, void* __restrict__ g_dr, void* __restrict__ g_dw,
    void* __restrict__ g_dk, void* __restrict__ g_dv, void* __restrict__ g_da, void* __restrict__ g_db,
    float* __restrict__ dh_in, int T, int H) {
    __shared__ float rowpart[2][2][D][NQ];   // [parity][dv, dsa][row][wave]
    __shared__ float colsum[NOUT][D];        // per-step column sums (dr, dk, db, dw, da) by column

    const int i = threadIdx.x & 63;   // value row
    const int q = wave_id();          // key columns J_q
    const int bh = blockIdx.x;
    const int bi = bh / H, hi = bh - bi * H;
    const int64_t strideT = (int64_t)H * D;
    const int64_t base0 = ((int64_t)bi * T * H + hi) * D;
    const int NC = T / CH;
    const int64_t sb = (int64_t)bh * D * D + (int64_t)i * D + JW * q;

    float Sr[JW], dS[JW];   // S[i, J_q], dS[i, J_q]
    if (dhout) {
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) dS[jj] = dhout[sb + jj];
    } else {
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) dS[jj] = 0.0f;
    }
    int step = 0;
    for (int c = NC - 1; c >= 0; --c) {
        const float* ck = ckpt + (int64_t)bh * NC * D * D + (int64_t)c * D * D + (int64_t)i * D + JW * q;
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) Sr[jj] = ck[jj];
        for (int s = CH - 1; s >= 0; --s, ++step) {
            const int t = c * CH + s;
            const int64_t bt = base0 + (int64_t)t * strideT;
            const float dyi = dout[bt + i], vi = load1<DT>(v, bt + i), sai = sa[bt + i];
            float rj[JW], kj[JW], bj[JW], wj[JW], aj[JW];
            load16<DT>(r, bt + JW * q, rj);
            load16<DT>(k, bt + JW * q, kj);
            load16<DT>(b, bt + JW * q, bj);
            load16<DT>(w, bt + JW * q, wj);
            load16<DT>(a, bt + JW * q, aj);
            float pv = 0.0f, ps = 0.0f;
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                dS[jj] = fmaf(dyi, rj[jj], dS[jj]);
                pv = fmaf(dS[jj], kj[jj], pv);
                ps = fmaf(dS[jj], bj[jj], ps);
            }
            rowpart[step & 1][0][i][q] = pv;
            rowpart[step & 1][1][i][q] = ps;
            // column sums over the 64 rows of this wave, for the columns J_q
            float cdr[JW], cdk[JW], cdb[JW];
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                cdr[jj] = wave_sum64(Sr[jj] * dyi);
                cdk[jj] = wave_sum64(dS[jj] * vi);
                cdb[jj] = wave_sum64(dS[jj] * sai);
            }
            __syncthreads();
            const float dsa_i = (rowpart[step & 1][1][i][0] + rowpart[step & 1][1][i][1]) +
                                (rowpart[step & 1][1][i][2] + rowpart[step & 1][1][i][3]);
            const float dv_i = (rowpart[step & 1][0][i][0] + rowpart[step & 1][0][i][1]) +
                               (rowpart[step & 1][0][i][2] + rowpart[step & 1][0][i][3]);
            float cdw[JW], cda[JW];
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                const float prev = (fmaf(-sai, bj[jj], fmaf(-vi, kj[jj], Sr[jj]))) / wj[jj];
                Sr[jj] = prev;
                cdw[jj] = wave_sum64(prev * dS[jj]);
                cda[jj] = wave_sum64(prev * dsa_i);
                dS[jj] = fmaf(dS[jj], wj[jj], dsa_i * aj[jj]);
            }
            if (i < JW) {
                // lane jj of wave q publishes the sums of column 16q + jj
#pragma unroll
                for (int jj = 0; jj < JW; ++jj) {
                    if (i == jj) {
                        colsum[0][JW * q + jj] = cdr[jj];
                        colsum[1][JW * q + jj] = cdk[jj];
                        colsum[2][JW * q + jj] = cdb[jj];
                        colsum[3][JW * q + jj] = cdw[jj];
                        colsum[4][JW * q + jj] = cda[jj];
                    }
                }
            }
            __syncthreads();
            if (q == 0) {
                store1<GT>(g_dr, bt + i, colsum[0][i]);
                store1<GT>(g_dk, bt + i, colsum[1][i]);
                store1<GT>(g_db, bt + i, colsum[2][i]);
                store1<GT>(g_dw, bt + i, colsum[3][i]);
                store1<GT>(g_da, bt + i, colsum[4][i]);
                store1<GT>(g_dv, bt + i, dv_i);
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) dh_in[sb + jj] = dS[jj];
}

// ─────────────────────────────── tmix tail ───────────────────────────────
__device__ __forceinline__ float wave_total(float x) {
    x = wave_sum64(x);
    return __shfl(x, 0, 64);   // one lane's association for everybody
}

__global__ __launch_bounds__(64) void wkv_tail_kernel(
    const float* __restrict__ wkv, const float* __restrict__ r, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ rk, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const float* __restrict__ g, float* __restrict__ out,
    int H, int S, float eps) {
    const int tg = blockIdx.x;          // row * H + head
    const int h = tg % H;
    const int64_t base = (int64_t)tg * S, hb = (int64_t)h * S;
    const int lane = threadIdx.x;
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
        out[base + e] = y * g[base + e];
    }
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
    dim3 grid((unsigned)(B * H)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (dt) {
        case RWKV_F32:
            hipLaunchKernelGGL((wkv7_fwd_kernel<RWKV_F32, SA, CK>), grid, block, 0, st, r, w, k, v, a, b, h_in, out, h_out, sa_out, ck, (int)T, (int)H);
            break;
        case RWKV_BF16:
            hipLaunchKernelGGL((wkv7_fwd_kernel<RWKV_BF16, SA, CK>), grid, block, 0, st, r, w, k, v, a, b, h_in, out, h_out, sa_out, ck, (int)T, (int)H);
            break;
        case RWKV_F16:
            hipLaunchKernelGGL((wkv7_fwd_kernel<RWKV_F16, SA, CK>), grid, block, 0, st, r, w, k, v, a, b, h_in, out, h_out, sa_out, ck, (int)T, (int)H);
            break;
    }
    return launch_status("wkv7 forward launch");
}

rwkv_status check_wkv_common(const void* r, const void* w, const void* k, const void* v, const void* a,
                             const void* b, int dt, int64_t B, int64_t T, int64_t H) {
    RWKV_REQUIRE(r && w && k && v && a && b, RWKV_E_NULL, "wkv7: r/w/k/v/a/b must be non-null");
    RWKV_REQUIRE(rwkv::dtype_ok(dt), RWKV_E_DTYPE, "wkv7: input dtype code %d not in {f32, bf16, f16}", dt);
    RWKV_REQUIRE(B >= 1 && H >= 1, RWKV_E_SHAPE, "wkv7: B (%lld) and H (%lld) must be >= 1", (long long)B, (long long)H);
    RWKV_REQUIRE(T >= 1, RWKV_E_SHAPE, "wkv7: T (%lld) must be >= 1", (long long)T);
    RWKV_REQUIRE(B * H <= INT32_MAX && T <= INT32_MAX && B * T * H * 64 <= (int64_t)1 << 46, RWKV_E_SHAPE,
                 "wkv7: B·T·H too large");
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
                                const void* b, rwkv_dtype in_dt, const float* h_ckpt, const float* sa,
                                const float* d_out, const float* d_h_out, void* dr, void* dw, void* dk,
                                void* dv, void* da, void* db, rwkv_dtype g_dt, float* dh_in, int64_t B,
                                int64_t T, int64_t H, int variant, void* stream) {
    rwkv_status s = check_wkv_common(r, w, k, v, a, b, in_dt, B, T, H);
    if (s != RWKV_OK) return s;
    RWKV_REQUIRE(T % CH == 0, RWKV_E_SHAPE, "wkv7_train_bwd: T (%lld) must be a multiple of CHUNK %d", (long long)T, CH);
    RWKV_REQUIRE(h_ckpt && sa && d_out && dr && dw && dk && dv && da && db && dh_in, RWKV_E_NULL,
                 "wkv7_train_bwd: checkpoints, sa, d_out, gradients and dh_in must be non-null");
    RWKV_REQUIRE(rwkv::dtype_ok(g_dt), RWKV_E_DTYPE, "wkv7_train_bwd: gradient dtype code %d not in {f32, bf16, f16}", g_dt);
    RWKV_REQUIRE(variant == 1 || variant == 2, RWKV_E_UNSUPPORTED, "wkv7_train_bwd: variant %d not in {1, 2}", variant);
    dim3 grid((unsigned)(B * H)), block(256);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define RWKV_BWD_LAUNCH(KER, DT, GT)                                                                          \
    hipLaunchKernelGGL((KER<DT, GT>), grid, block, 0, st, r, w, k, v, a, b, h_ckpt, sa, d_out, d_h_out, dr, dw, \
                       dk, dv, da, db, dh_in, (int)T, (int)H)
#define RWKV_BWD_GT(KER, DT)                                 \
    switch (g_dt) {                                          \
        case RWKV_F32: RWKV_BWD_LAUNCH(KER, DT, RWKV_F32); break;   \
        case RWKV_BF16: RWKV_BWD_LAUNCH(KER, DT, RWKV_BF16); break; \
        case RWKV_F16: RWKV_BWD_LAUNCH(KER, DT, RWKV_F16); break;   \
    }
#define RWKV_BWD_DT(KER)                                 \
    switch (in_dt) {                                     \
        case RWKV_F32: RWKV_BWD_GT(KER, RWKV_F32); break;   \
        case RWKV_BF16: RWKV_BWD_GT(KER, RWKV_BF16); break; \
        case RWKV_F16: RWKV_BWD_GT(KER, RWKV_F16); break;   \
    }
    if (variant == 2) {
        RWKV_BWD_DT(wkv7_bwd_v2_kernel)
    } else {
        RWKV_BWD_DT(wkv7_bwd_v1_kernel)
    }
#undef RWKV_BWD_DT
#undef RWKV_BWD_GT
#undef RWKV_BWD_LAUNCH
    s = launch_status("wkv7 backward launch");
    if (s == RWKV_OK) rwkv::counters().train_bwd++;
    return s;
}

int rwkv_wkv_tail_applies(int64_t S) { return S > 0 && S % 32 == 0; }

rwkv_status rwkv_wkv_tail(const float* wkv, const float* r, const float* k, const float* v, const float* rk,
                          const float* lnw, const float* lnb, const float* g, float* out, int64_t N, int64_t H,
                          int64_t S, float eps, void* stream) {
    RWKV_REQUIRE(wkv && r && k && v && rk && lnw && lnb && g && out, RWKV_E_NULL, "wkv_tail: null buffer");
    RWKV_REQUIRE(rwkv_wkv_tail_applies(S), RWKV_E_SHAPE, "wkv_tail: S=%lld is not a multiple of 32", (long long)S);
    RWKV_REQUIRE(N >= 1 && H >= 1 && N * H <= INT32_MAX && S <= 1 << 20, RWKV_E_SHAPE, "wkv_tail: bad N/H/S");
    hipLaunchKernelGGL(wkv_tail_kernel, dim3((unsigned)(N * H)), dim3(64), 0, reinterpret_cast<hipStream_t>(stream),
                       wkv, r, k, v, rk, lnw, lnb, g, out, (int)H, (int)S, eps);
    rwkv_status s = launch_status("wkv_tail launch");
    if (s == RWKV_OK) rwkv::counters().tail++;
    return s;
}

}  // extern "C"
