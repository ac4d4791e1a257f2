/*
 * oracle.c — CPU restatement of the SwiftRWKV WKV-7 + .rwkvq hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the reference
 * results are compared with (or, for cpu_baseline, as the timed CPU
 * restatement).  The product path in
 * swiftrwkv_amd/ never calls it.
 *
 * Every function names the reference lines (Sources/... in RafaelUI/SwiftRWKV)
 * whose behaviour it restates.  How each is pinned (closed forms, invariants,
 * numpy/torch conversions, the in-repo KAT, finite differences) is listed in
 * tests/test_oracle.py; no function here is "parity unpinned" except the
 * encoder, which lives in the product library, not here.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  fp32 code is
 * compiled without FMA contraction so "a*b + c" rounds twice, as written.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 64          /* WKV7_HEAD_SIZE, Sources/RWKVKernel/WKV7.swift:7 */
#define CHUNK 16      /* WKV7_CHUNK,     Sources/RWKVKernel/WKV7.swift:8 */

/* ───────────────────────── half / bfloat16 conversions ─────────────────────────
 * IEEE binary16 with round-to-nearest-even, subnormals kept.  Metal's `(half)x`
 * (RwkvqDequant.swift:130-131, RwkvqSb6GEMV.swift:135-136) and MLX's
 * asType(.float16) are RNE conversions; pinned against numpy.float16. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) {                       /* inf / nan */
        if (mant) return (uint16_t)(sign | 0x7e00u | (mant >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t r = mant >> 13, rem = mant & 0x1fffu;
        uint32_t h = ((uint32_t)e << 10) | r;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) h += 1;   /* carry may reach inf */
        return (uint16_t)(sign | h);
    }
    if (exp == 0) return (uint16_t)sign;     /* f32 subnormal: far below half range */
    uint32_t sig = mant | 0x800000u;         /* 24-bit significand */
    int32_t shift = 14 - e;                  /* value in units of 2^-24 = sig >> shift */
    if (shift > 24) return (uint16_t)sign;
    uint32_t r = sig >> shift, rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r += 1;
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, x;
    if (exp == 0) {
        if (mant == 0) x = sign;
        else {                               /* subnormal: renormalise */
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (exp == 31) x = sign | 0x7f800000u | (mant << 13);
    else x = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    float f; memcpy(&f, &x, 4); return f;
}

/* bfloat16, RNE (MLX asType(.bfloat16), Metal bfloat16_t; RwkvqDequant.swift:139). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t b) { uint32_t x = (uint32_t)b << 16; float f; memcpy(&f, &x, 4); return f; }

void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]); }
void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]); }
void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]); }

static inline float hround(float v) { return orc_f16_to_f32(orc_f32_to_f16(v)); }

/* ───────────────────────────── WKV-7 forward ─────────────────────────────
 * Follows the per-row loop of wkv7_seq (Sources/RWKVKernel/WKV7.swift:207-224),
 * identical to wkv7_fwd (:33-47) and the train forward (WKV7Train.swift:61-87):
 *   sa  = Σ_dk h[dv,dk]·a[dk]           (sequential dk loop)
 *   h   = w[dk]·h + v[dv]·k[dk] + sa·b[dk]
 *   y   = Σ_dk h[dv,dk]·r[dk]
 * Layout: inputs [B,T,H,64]; state [B,H,64(dv),64(dk)] (WKV7Step.swift:23-24).
 * sa_out [B,T,H,64] and ckpt [B,H,T/16,64,64] (state after each 16-step chunk,
 * WKV7Train.swift:84-86) are optional.  fp32 throughout, no contraction. */
void orc_wkv7_fwd_f32(const float* r, const float* w, const float* k, const float* v,
                      const float* a, const float* b, const float* h_in,
                      float* out, float* h_out, float* sa_out, float* ckpt,
                      int B, int T, int H, int nthreads) {
    int NC = T / CHUNK;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    #pragma omp parallel for collapse(3) num_threads(nthreads) schedule(static)
#endif
    for (int bi = 0; bi < B; bi++)
    for (int hi = 0; hi < H; hi++)
    for (int dv = 0; dv < D; dv++) {
        float h[D];
        int64_t hb = ((int64_t)(bi * H + hi) * D + dv) * D;
        for (int j = 0; j < D; j++) h[j] = h_in ? h_in[hb + j] : 0.0f;
        for (int t = 0; t < T; t++) {
            int64_t base = ((int64_t)(bi * T + t) * H + hi) * D;
            float sa = 0.0f;
            for (int j = 0; j < D; j++) sa += h[j] * a[base + j];
            if (sa_out) sa_out[base + dv] = sa;
            float vv = v[base + dv];
            for (int j = 0; j < D; j++) h[j] = w[base + j] * h[j] + vv * k[base + j] + sa * b[base + j];
            float y = 0.0f;
            for (int j = 0; j < D; j++) y += h[j] * r[base + j];
            out[base + dv] = y;
            if (ckpt && (t % CHUNK) == CHUNK - 1 && NC > 0) {
                int64_t cb = (((int64_t)(bi * H + hi) * NC + t / CHUNK) * D + dv) * D;
                for (int j = 0; j < D; j++) ckpt[cb + j] = h[j];
            }
        }
        if (h_out) for (int j = 0; j < D; j++) h_out[hb + j] = h[j];
    }
}

/* Same recurrence in fp64 (the tolerance anchor for every fp32 path). */
void orc_wkv7_fwd_f64(const double* r, const double* w, const double* k, const double* v,
                      const double* a, const double* b, const double* h_in,
                      double* out, double* h_out, double* sa_out, int B, int T, int H) {
#ifdef _OPENMP
    #pragma omp parallel for collapse(3) schedule(static)
#endif
    for (int bi = 0; bi < B; bi++)
    for (int hi = 0; hi < H; hi++)
    for (int dv = 0; dv < D; dv++) {
        double h[D];
        int64_t hb = ((int64_t)(bi * H + hi) * D + dv) * D;
        for (int j = 0; j < D; j++) h[j] = h_in ? h_in[hb + j] : 0.0;
        for (int t = 0; t < T; t++) {
            int64_t base = ((int64_t)(bi * T + t) * H + hi) * D;
            double sa = 0.0;
            for (int j = 0; j < D; j++) sa += h[j] * a[base + j];
            if (sa_out) sa_out[base + dv] = sa;
            double vv = v[base + dv];
            for (int j = 0; j < D; j++) h[j] = w[base + j] * h[j] + vv * k[base + j] + sa * b[base + j];
            double y = 0.0;
            for (int j = 0; j < D; j++) y += h[j] * r[base + j];
            out[base + dv] = y;
        }
        if (h_out) for (int j = 0; j < D; j++) h_out[hb + j] = h[j];
    }
}

/* ───────────────────────────── WKV-7 backward (fp64) ─────────────────────────────
 * Analytic reverse pass of the recurrence above.  The equations are those of
 * ckptBwdKernelV2 (Sources/RWKVKernel/WKV7Train.swift:276-325) and of the v1
 * kernel (:147-192):
 *   dS += dy ⊗ r;  dr_j = Σ_i S_ij dy_i;  dv_i = Σ_j dS_ij k_j;  dsa_i = Σ_j dS_ij b_j
 *   dk_j = Σ_i dS_ij v_i;  db_j = Σ_i dS_ij sa_i
 *   dw_j = Σ_i S⁻_ij dS_ij;  da_j = Σ_i S⁻_ij dsa_i;  dS_ij ← dS_ij w_j + dsa_i a_j
 * with S⁻ the state before the step.  Here every state is STORED by an fp64
 * forward (no division by w), so this is the exact-arithmetic anchor the
 * kernels' reconstruct-by-division is measured against.  Loss convention of
 * WKV7TrainKernelTests.swift:46-52: cotangents d_out [B,T,H,64] and d_h_out
 * [B,H,64,64] (nullable ⇒ 0).  Outputs dr..db [B,T,H,64], dh_in [B,H,64,64]. */
void orc_wkv7_bwd_f64(const double* r, const double* w, const double* k, const double* v,
                      const double* a, const double* b, const double* h_in,
                      const double* d_out, const double* d_h_out,
                      double* dr, double* dw, double* dk, double* dv, double* da, double* db,
                      double* dh_in, int B, int T, int H) {
#ifdef _OPENMP
    #pragma omp parallel for collapse(2) schedule(dynamic)
#endif
    for (int bi = 0; bi < B; bi++)
    for (int hi = 0; hi < H; hi++) {
        double* S = (double*)malloc(sizeof(double) * (size_t)(T + 1) * D * D);
        double* SA = (double*)malloc(sizeof(double) * (size_t)T * D);
        double dS[D][D], dsa[D];
        int64_t hb = (int64_t)(bi * H + hi) * D * D;
        for (int i = 0; i < D * D; i++) S[i] = h_in ? h_in[hb + i] : 0.0;
        for (int t = 0; t < T; t++) {
            int64_t base = ((int64_t)(bi * T + t) * H + hi) * D;
            const double* Sp = S + (size_t)t * D * D;
            double* Sn = S + (size_t)(t + 1) * D * D;
            for (int i = 0; i < D; i++) {
                double sa = 0.0;
                for (int j = 0; j < D; j++) sa += Sp[i * D + j] * a[base + j];
                SA[t * D + i] = sa;
                for (int j = 0; j < D; j++)
                    Sn[i * D + j] = w[base + j] * Sp[i * D + j] + v[base + i] * k[base + j] + sa * b[base + j];
            }
        }
        for (int i = 0; i < D; i++) for (int j = 0; j < D; j++) dS[i][j] = d_h_out ? d_h_out[hb + i * D + j] : 0.0;
        for (int t = T - 1; t >= 0; t--) {
            int64_t base = ((int64_t)(bi * T + t) * H + hi) * D;
            const double* Sp = S + (size_t)t * D * D;
            const double* Sc = S + (size_t)(t + 1) * D * D;
            const double* dy = d_out + base;
            for (int i = 0; i < D; i++) for (int j = 0; j < D; j++) dS[i][j] += dy[i] * r[base + j];
            for (int j = 0; j < D; j++) {
                double s_dr = 0, s_dk = 0, s_db = 0, s_dw = 0;
                for (int i = 0; i < D; i++) {
                    s_dr += Sc[i * D + j] * dy[i];
                    s_dk += dS[i][j] * v[base + i];
                    s_db += dS[i][j] * SA[t * D + i];
                    s_dw += Sp[i * D + j] * dS[i][j];
                }
                dr[base + j] = s_dr; dk[base + j] = s_dk; db[base + j] = s_db; dw[base + j] = s_dw;
            }
            for (int i = 0; i < D; i++) {
                double s_dv = 0, s_dsa = 0;
                for (int j = 0; j < D; j++) { s_dv += dS[i][j] * k[base + j]; s_dsa += dS[i][j] * b[base + j]; }
                dv[base + i] = s_dv; dsa[i] = s_dsa;
            }
            for (int j = 0; j < D; j++) {
                double s_da = 0;
                for (int i = 0; i < D; i++) s_da += Sp[i * D + j] * dsa[i];
                da[base + j] = s_da;
            }
            for (int i = 0; i < D; i++) for (int j = 0; j < D; j++) dS[i][j] = dS[i][j] * w[base + j] + dsa[i] * a[base + j];
        }
        for (int i = 0; i < D; i++) for (int j = 0; j < D; j++) dh_in[hb + i * D + j] = dS[i][j];
        free(S); free(SA);
    }
}

/* ───────────────────────────── tmix tail ─────────────────────────────
 * wkv_tail (Sources/RWKVKernel/WKV7DecodeKernels.swift:124-156), in fp64:
 *   mean = Σ x / S;  var = Σ (x-mean)² / S   (two passes)
 *   inv  = 1/sqrt(var + eps);  dp = Σ r·k·rk
 *   out  = ((x-mean)·inv·lnw + lnb + dp·v)·g
 * wkv, r, k, v, g, out: [N, H·S];  rk, lnw, lnb: [H·S]. */
void orc_wkv_tail_f64(const float* wkv, const float* r, const float* k, const float* v,
                      const float* rk, const float* lnw, const float* lnb, const float* g,
                      double* out, int N, int H, int S, double eps) {
    for (int n = 0; n < N; n++)
    for (int h = 0; h < H; h++) {
        int64_t base = ((int64_t)n * H + h) * S, hb = (int64_t)h * S;
        double s1 = 0; for (int i = 0; i < S; i++) s1 += wkv[base + i];
        double mean = s1 / S;
        double s2 = 0; for (int i = 0; i < S; i++) { double d = wkv[base + i] - mean; s2 += d * d; }
        double inv = 1.0 / sqrt(s2 / S + eps);
        double dp = 0; for (int i = 0; i < S; i++) dp += (double)r[base + i] * k[base + i] * rk[hb + i];
        for (int i = 0; i < S; i++) {
            double nrm = (wkv[base + i] - mean) * inv;
            double y = nrm * lnw[hb + i] + lnb[hb + i] + dp * v[base + i];
            out[base + i] = y * g[base + i];
        }
    }
}

/* ───────────────────────────── .rwkvq: unpack / repack ─────────────────────────────
 * rwkvqUnpack6x8 (Sources/RWKVQuant/RwkvqFile.swift:171-181): 6 bytes → 8 values
 * of 6 bits, LSB-first, in two 3-byte chunks of 4 values. */
void orc_unpack6x8(const uint8_t* in, int64_t n_groups, int32_t* out) {
    for (int64_t g = 0; g < n_groups; g++) {
        for (int c = 0; c < 2; c++) {
            int32_t x0 = in[g * 6 + c * 3], x1 = in[g * 6 + c * 3 + 1], x2 = in[g * 6 + c * 3 + 2];
            out[g * 8 + c * 4 + 0] = x0 & 0x3f;
            out[g * 8 + c * 4 + 1] = ((x0 >> 6) | (x1 << 2)) & 0x3f;
            out[g * 8 + c * 4 + 2] = ((x1 >> 4) | (x2 << 4)) & 0x3f;
            out[g * 8 + c * 4 + 3] = (x2 >> 2) & 0x3f;
        }
    }
}

/* rwkvqSb6ToK3 (RwkvqFile.swift:189-212).  Disk layout → K3 interleave:
 *   qblk[row, blk] = codes_packed[16] ‖ qh[4] (xbits≥1) ‖ qh2[4] (xbits≥2)
 *   qsqm[row, blk] = (qs, (qm_stored − 31) mod 256)
 *   ddm [row, sb]  = (d, dm) as two fp16
 * disk: codes_packed [OUT, NB*16], qh/qh2 [OUT, NB*4] (nullable), gw_qsqm
 * [OUT, NSB, 12], gw_d / gw_dm [OUT, NSB] fp16 bits.  gs = 32, sb = 8. */
void orc_sb6_to_k3(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2,
                   const uint8_t* gw_qsqm, const uint16_t* gw_d, const uint16_t* gw_dm,
                   int64_t OUT, int64_t IN,
                   uint8_t* qblk, uint8_t* qsqm, uint16_t* ddm) {
    int64_t NB = IN / 32, NSB = NB / 8;
    int xbits = (qh ? 1 : 0) + (qh2 ? 1 : 0);
    int64_t SU = 16 + 4 * xbits;
    for (int64_t row = 0; row < OUT; row++) {
        for (int64_t blk = 0; blk < NB; blk++) {
            uint8_t* dst = qblk + (row * NB + blk) * SU;
            memcpy(dst, codes_packed + (row * NB + blk) * 16, 16);
            if (qh) memcpy(dst + 16, qh + (row * NB + blk) * 4, 4);
            if (qh2) memcpy(dst + 16 + (qh ? 4 : 0), qh2 + (row * NB + blk) * 4, 4);
        }
        for (int64_t sb = 0; sb < NSB; sb++) {
            int32_t qs[8], qm[8];
            const uint8_t* src = gw_qsqm + (row * NSB + sb) * 12;
            orc_unpack6x8(src, 1, qs);
            orc_unpack6x8(src + 6, 1, qm);
            for (int i = 0; i < 8; i++) {
                qsqm[(row * NB + sb * 8 + i) * 2 + 0] = (uint8_t)qs[i];
                qsqm[(row * NB + sb * 8 + i) * 2 + 1] = (uint8_t)((qm[i] - 31 + 256) % 256);
            }
            ddm[(row * NSB + sb) * 2 + 0] = gw_d[row * NSB + sb];
            ddm[(row * NSB + sb) * 2 + 1] = gw_dm[row * NSB + sb];
        }
    }
}

/* sym 6-bit interleave (RwkvqFile.swift:437-449): per pair of 16-blocks,
 * codes_packed[16] ‖ qh[4] ‖ qh2[4]  → qblk [OUT, IN/32*24]. */
void orc_sym_interleave(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2,
                        int64_t OUT, int64_t IN, uint8_t* qblk) {
    int64_t NP = IN / 32;
    for (int64_t row = 0; row < OUT; row++)
        for (int64_t p = 0; p < NP; p++) {
            uint8_t* dst = qblk + (row * NP + p) * 24;
            memcpy(dst, codes_packed + (row * NP + p) * 16, 16);
            memcpy(dst + 16, qh + (row * NP + p) * 4, 4);
            memcpy(dst + 20, qh2 + (row * NP + p) * 4, 4);
        }
}

/* ───────────────────────────── .rwkvq: dequant ─────────────────────────────
 * sb6 (RwkvqDequant.swift:116-140): code c of block blk:
 *   nib byte j (j<16): low nibble → column j, high nibble → column j+16
 *   qh bit c → bit 4 of column c; qh2 bit c → bit 5
 *   s = half(qs·d);  m = half(int8(qm)·dm);  w = float(code)·float(s) + float(m)
 * Output stored as fp32 (out_dt 0), bf16 (1) or fp16 (2) from the fp32 value. */
static float sb6_weight(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                        int64_t row, int64_t col, int64_t NB, int64_t NSB, int xbits) {
    int64_t SU = 16 + 4 * xbits, blk = col / 32;
    int c = (int)(col % 32);
    const uint8_t* qb = qblk + (row * NB + blk) * SU;
    int code = c < 16 ? (qb[c] & 0xf) : (qb[c - 16] >> 4);
    if (xbits >= 1) {
        uint32_t hb; memcpy(&hb, qb + 16, 4);
        code |= (int)((hb >> c) & 1u) << 4;
    }
    if (xbits >= 2) {
        uint32_t hb2; memcpy(&hb2, qb + 20, 4);
        code |= (int)((hb2 >> c) & 1u) << 5;
    }
    uint8_t qs = qsqm[(row * NB + blk) * 2], qmb = qsqm[(row * NB + blk) * 2 + 1];
    int8_t qm = (int8_t)qmb;
    int64_t sb = blk / 8;
    float d = orc_f16_to_f32(ddm[(row * NSB + sb) * 2]), dm = orc_f16_to_f32(ddm[(row * NSB + sb) * 2 + 1]);
    float s = hround((float)qs * d);
    float mn = hround((float)qm * dm);
    return (float)code * s + mn;
}

static void store_dt(void* out, int64_t idx, float val, int out_dt) {
    if (out_dt == 0) ((float*)out)[idx] = val;
    else if (out_dt == 1) ((uint16_t*)out)[idx] = orc_f32_to_bf16(val);
    else ((uint16_t*)out)[idx] = orc_f32_to_f16(val);
}

void orc_sb6_dequant(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                     int64_t OUT, int64_t IN, int xbits, void* out, int out_dt) {
    int64_t NB = IN / 32, NSB = NB / 8;
    for (int64_t row = 0; row < OUT; row++)
        for (int64_t col = 0; col < IN; col++)
            store_dt(out, row * IN + col, sb6_weight(qblk, qsqm, ddm, row, col, NB, NSB, xbits), out_dt);
}

/* sym (RwkvqDequant.swift:350-388 kernel; :442-466 rwkvqDequantSymReference):
 *   s = half(int8(qs[blk])·d[blk/16]);  8-bit: w = int8(code)·s;
 *   6-bit: pair of blocks, byte j of each 8-byte half: low nibble → col j,
 *   high → col j+8 (block-local); qh/qh2 bit c → bits 4/5 of pair column c;
 *   w = (q − 32)·s.  The product is exact in fp32, so the fp16 branch (half
 *   multiply) equals fp16 of the fp32 value.  d is [OUT, ceil(NB/16)]. */
static float sym_weight(const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                        int64_t row, int64_t col, int64_t IN, int bits) {
    int64_t NB = IN / 16, NSB = (NB + 15) / 16, blk = col / 16;
    float q;
    if (bits == 8) q = (float)(int8_t)qblk[row * IN + col];
    else {
        int64_t NP = IN / 32, p = col / 32;
        int c = (int)(col % 32), half = c / 16, j = c % 16;
        const uint8_t* qb = qblk + (row * NP + p) * 24;
        int code = j < 8 ? (qb[half * 8 + j] & 0xf) : (qb[half * 8 + j - 8] >> 4);
        uint32_t hb, hb2; memcpy(&hb, qb + 16, 4); memcpy(&hb2, qb + 20, 4);
        code |= (int)((hb >> c) & 1u) << 4;
        code |= (int)((hb2 >> c) & 1u) << 5;
        q = (float)(code - 32);
    }
    float s = hround((float)(int8_t)qs[row * NB + blk] * orc_f16_to_f32(d[row * NSB + blk / 16]));
    return q * s;
}

void orc_sym_dequant(const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                     int64_t OUT, int64_t IN, int bits, void* out, int out_dt) {
    for (int64_t row = 0; row < OUT; row++)
        for (int64_t col = 0; col < IN; col++)
            store_dt(out, row * IN + col, sym_weight(qblk, qs, d, row, col, IN, bits), out_dt);
}

/* ───────────────────────────── .rwkvq: GEMV (fp64 anchor) ─────────────────────────────
 * y[n, o] = Σ_i W[o, i] · x[n·NK + o/out_per, i], W the dequantised fp32 weights
 * (sb6: RwkvqSb6GEMV.swift:118-144; sym: RwkvqSymGEMV.swift:126-199, fused
 * rows pick their input as xi = row/OUT_PER, :105-106).  Accumulated in fp64. */
void orc_sb6_gemv_f64(const float* x, int N, const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                      int64_t OUT, int64_t IN, int xbits, double* y) {
    int64_t NB = IN / 32, NSB = NB / 8;
#ifdef _OPENMP
    #pragma omp parallel for schedule(static)
#endif
    for (int64_t o = 0; o < OUT; o++) {
        for (int n = 0; n < N; n++) {
            double acc = 0;
            for (int64_t i = 0; i < IN; i++) acc += (double)sb6_weight(qblk, qsqm, ddm, o, i, NB, NSB, xbits) * x[(int64_t)n * IN + i];
            y[(int64_t)n * OUT + o] = acc;
        }
    }
}

void orc_sym_gemv_f64(const float* x, int N, const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                      int64_t OUT, int64_t IN, int bits, int64_t out_per, double* y) {
    int64_t NK = OUT / out_per;
#ifdef _OPENMP
    #pragma omp parallel for schedule(static)
#endif
    for (int64_t o = 0; o < OUT; o++) {
        for (int n = 0; n < N; n++) {
            const float* xr = x + ((int64_t)n * NK + o / out_per) * IN;
            double acc = 0;
            for (int64_t i = 0; i < IN; i++) acc += (double)sym_weight(qblk, qs, d, o, i, IN, bits) * xr[i];
            y[(int64_t)n * OUT + o] = acc;
        }
    }
}

/* ───────────────────────────── CPU baseline (timed by bench.py) ─────────────────────────────
 * The reference's non-kernel projection path: dequantize(key, .float32) then
 * fp32 x·Wᵀ (RwkvqSidecar.swift:243-325 → X070Backbone.swift:733-739).  Rows are
 * dequantised into a per-thread fp32 buffer and dotted in fp32; OpenMP over
 * output rows with `nthreads` threads. */
void orc_cpu_sb6_dequant_matvec(const float* x, const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                int64_t OUT, int64_t IN, int xbits, float* y, int nthreads) {
    int64_t NB = IN / 32, NSB = NB / 8;
#ifdef _OPENMP
    #pragma omp parallel num_threads(nthreads)
#endif
    {
        float* wrow = (float*)malloc(sizeof(float) * (size_t)IN);
#ifdef _OPENMP
        #pragma omp for schedule(static)
#endif
        for (int64_t o = 0; o < OUT; o++) {
            for (int64_t i = 0; i < IN; i++) wrow[i] = sb6_weight(qblk, qsqm, ddm, o, i, NB, NSB, xbits);
            float acc = 0.0f;
            for (int64_t i = 0; i < IN; i++) acc += x[i] * wrow[i];
            y[o] = acc;
        }
        free(wrow);
    }
}

/* One decode step of the WKV recurrence on the CPU (B rows, T = 1), the MLX-op
 * step (WKV7Step.swift:120-122) restated; OpenMP over (b, h, dv). */
void orc_cpu_wkv7_step(const float* r, const float* w, const float* k, const float* v,
                       const float* a, const float* b, float* h, float* out, int B, int H, int nthreads) {
#ifdef _OPENMP
    #pragma omp parallel for collapse(3) num_threads(nthreads) schedule(static)
#endif
    for (int bi = 0; bi < B; bi++)
    for (int hi = 0; hi < H; hi++)
    for (int dv = 0; dv < D; dv++) {
        int64_t base = ((int64_t)bi * H + hi) * D;
        float* hr = h + (base + dv) * D;
        float sa = 0.0f;
        for (int j = 0; j < D; j++) sa += hr[j] * a[base + j];
        float y = 0.0f;
        for (int j = 0; j < D; j++) { hr[j] = hr[j] * w[base + j] + v[base + dv] * k[base + j] + sa * b[base + j]; y += hr[j] * r[base + j]; }
        out[base + dv] = y;
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
