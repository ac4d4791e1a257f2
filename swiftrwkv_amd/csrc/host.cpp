// Host-side (CPU) part of the C ABI: status strings and the thread-local last
// error, launch counters, the .rwkvq disk→loader byte permutations, the
// encoders, and the memory-mapped safetensors container.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "container.h"

namespace rwkv {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

Counters& counters() {
    static Counters c;
    return c;
}

static thread_local TimingEvents g_timing{nullptr, nullptr};

TimingEvents take_timing() {
    const TimingEvents t = g_timing;
    g_timing = {nullptr, nullptr};
    return t;
}

// IEEE binary16 with round-to-nearest-even (host copy; used by the encoders).
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t r = mant >> 13, rem = mant & 0x1fffu, h = ((uint32_t)e << 10) | r;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) h += 1;
        return (uint16_t)(sign | h);
    }
    if (exp == 0) return (uint16_t)sign;
    uint32_t sig = mant | 0x800000u;
    int32_t shift = 14 - e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t r = sig >> shift, rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r += 1;
    return (uint16_t)(sign | r);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, x;
    if (exp == 0) {
        if (mant == 0) x = sign;
        else {
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (exp == 31) x = sign | 0x7f800000u | (mant << 13);
    else x = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

static inline float hround(float v) { return f16_to_f32(f32_to_f16(v)); }

// Static row partition over `nthreads` std::threads (1 = inline).
template <class F>
static void parallel_rows(int64_t n, int nthreads, F&& body) {
    if (nthreads <= 1 || n < 2) {
        for (int64_t r = 0; r < n; ++r) body(r);
        return;
    }
    const int nt = (int)std::min<int64_t>(nthreads, n);
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (int t = 0; t < nt; ++t)
        pool.emplace_back([&, t] {
            for (int64_t r = n * t / nt; r < n * (t + 1) / nt; ++r) body(r);
        });
    for (auto& th : pool) th.join();
}

}  // namespace rwkv

using rwkv::set_error;

// ─────────────────────────────── status / counters ───────────────────────────────
extern "C" {

int rwkv_abi_version(void) { return RWKV_HIP_ABI_VERSION; }

const char* rwkv_status_string(rwkv_status s) {
    switch (s) {
        case RWKV_OK: return "ok";
        case RWKV_E_SHAPE: return "shape";
        case RWKV_E_DTYPE: return "dtype";
        case RWKV_E_UNSUPPORTED: return "unsupported";
        case RWKV_E_FORMAT: return "format";
        case RWKV_E_HIP: return "hip";
        case RWKV_E_NULL: return "null";
        case RWKV_E_IO: return "io";
    }
    return "unknown";
}

const char* rwkv_last_error(void) { return rwkv::g_last_error.c_str(); }

rwkv_status rwkv_time_next_launch(void* start_event, void* stop_event) {
    RWKV_REQUIRE((start_event == nullptr) == (stop_event == nullptr), RWKV_E_NULL,
                 "time_next_launch: give both events or neither");
    rwkv::g_timing = {start_event, stop_event};
    rwkv::clear_error();
    return RWKV_OK;
}

void rwkv_get_counters(rwkv_counters* out) {
    if (!out) return;
    auto& c = rwkv::counters();
    out->seq_fwd = c.seq_fwd.load();
    out->chunk_fwd = c.chunk_fwd.load();
    out->train_fwd = c.train_fwd.load();
    out->train_bwd = c.train_bwd.load();
    out->step = c.step.load();
    out->tail = c.tail.load();
    out->sb6_dequant = c.sb6_dequant.load();
    out->sym_dequant = c.sym_dequant.load();
    out->sb6_gemv = c.sb6_gemv.load();
    out->sym_gemv = c.sym_gemv.load();
    out->sym_fused = c.sym_fused.load();
    out->step_tail = c.step_tail.load();
    out->sb6_fused = c.sb6_fused.load();
    out->sym_rows = c.sym_rows.load();
    out->x070 = c.x070.load();
    out->sb6_gemm = c.sb6_gemm.load();
    out->seq_chunked = c.seq_chunked.load();
    out->sb6_batch = c.sb6_batch.load();
    out->sym_gemm = c.sym_gemm.load();
}

void rwkv_reset_counters(void) {
    auto& c = rwkv::counters();
    for (auto* a : {&c.seq_fwd, &c.chunk_fwd, &c.train_fwd, &c.train_bwd, &c.step, &c.tail, &c.sb6_dequant,
                    &c.sym_dequant, &c.sb6_gemv, &c.sym_gemv, &c.sym_fused, &c.step_tail, &c.sb6_fused,
                    &c.sym_rows, &c.x070, &c.sb6_gemm, &c.seq_chunked, &c.sb6_batch, &c.sym_gemm})
        a->store(0);
}

// ─────────────────────────────── disk → loader layouts ───────────────────────────────
// rwkvqUnpack6x8 (Sources/RWKVQuant/RwkvqFile.swift:171-181).
rwkv_status rwkv_unpack6x8(const uint8_t* in, int64_t n_groups, int32_t* out) {
    RWKV_REQUIRE(in && out, RWKV_E_NULL, "unpack6x8: null buffer");
    RWKV_REQUIRE(n_groups >= 0, RWKV_E_SHAPE, "unpack6x8: negative group count");
    for (int64_t g = 0; g < n_groups; ++g) {
        const uint8_t* b = in + g * 6;
        int32_t* o = out + g * 8;
        for (int c = 0; c < 2; ++c) {
            const uint32_t chunk = (uint32_t)b[3 * c] | ((uint32_t)b[3 * c + 1] << 8) | ((uint32_t)b[3 * c + 2] << 16);
            for (int e = 0; e < 4; ++e) o[4 * c + e] = (int32_t)((chunk >> (6 * e)) & 0x3fu);
        }
    }
    rwkv::clear_error();
    return RWKV_OK;
}

// rwkvqSb6ToK3 (RwkvqFile.swift:189-212): bytes are moved, never recomputed.
rwkv_status rwkv_sb6_to_k3(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2,
                           const uint8_t* gw_qsqm, const uint16_t* gw_d, const uint16_t* gw_dm, int64_t OUT,
                           int64_t IN, uint8_t* qblk, uint8_t* qsqm, uint16_t* ddm) {
    RWKV_REQUIRE(codes_packed && gw_qsqm && gw_d && gw_dm && qblk && qsqm && ddm, RWKV_E_NULL, "sb6_to_k3: null buffer");
    RWKV_REQUIRE(!(qh2 && !qh), RWKV_E_FORMAT, "sb6_to_k3: qh2 without qh");
    RWKV_REQUIRE(OUT >= 1 && IN >= 256 && IN % 256 == 0, RWKV_E_SHAPE, "sb6_to_k3: IN (%lld) must be a multiple of 256",
                 (long long)IN);
    const int64_t NB = IN / 32, NSB = NB / 8;
    const int xbits = (qh ? 1 : 0) + (qh2 ? 1 : 0);
    const int64_t SU = 16 + 4 * xbits;
    for (int64_t row = 0; row < OUT; ++row) {
        for (int64_t blk = 0; blk < NB; ++blk) {
            uint8_t* dst = qblk + (row * NB + blk) * SU;
            std::memcpy(dst, codes_packed + (row * NB + blk) * 16, 16);
            if (qh) std::memcpy(dst + 16, qh + (row * NB + blk) * 4, 4);
            if (qh2) std::memcpy(dst + 20, qh2 + (row * NB + blk) * 4, 4);
        }
        for (int64_t sb = 0; sb < NSB; ++sb) {
            int32_t v[16];
            rwkv_unpack6x8(gw_qsqm + (row * NSB + sb) * 12, 2, v);   // 8 qs then 8 stored qm
            for (int e = 0; e < 8; ++e) {
                qsqm[(row * NB + sb * 8 + e) * 2] = (uint8_t)v[e];
                qsqm[(row * NB + sb * 8 + e) * 2 + 1] = (uint8_t)((v[8 + e] - 31 + 256) & 0xff);
            }
            ddm[(row * NSB + sb) * 2] = gw_d[row * NSB + sb];
            ddm[(row * NSB + sb) * 2 + 1] = gw_dm[row * NSB + sb];
        }
    }
    rwkv::clear_error();
    return RWKV_OK;
}

// sym 6-bit interleave (RwkvqFile.swift:437-449).
rwkv_status rwkv_sym_interleave(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2, int64_t OUT,
                                int64_t IN, uint8_t* qblk) {
    RWKV_REQUIRE(codes_packed && qh && qh2 && qblk, RWKV_E_NULL, "sym_interleave: null buffer");
    RWKV_REQUIRE(OUT >= 1 && IN >= 32 && IN % 32 == 0, RWKV_E_SHAPE, "sym_interleave: IN (%lld) must be a multiple of 32",
                 (long long)IN);
    const int64_t NP = IN / 32;
    for (int64_t rp = 0; rp < OUT * NP; ++rp) {
        uint8_t* dst = qblk + rp * 24;
        std::memcpy(dst, codes_packed + rp * 16, 16);
        std::memcpy(dst + 16, qh + rp * 4, 4);
        std::memcpy(dst + 20, qh2 + rp * 4, 4);
    }
    rwkv::clear_error();
    return RWKV_OK;
}

// ─────────────────────────────── encoders ───────────────────────────────
// Not part of the reference (it reads files written by the external
// rwkv-quant).  Round-to-nearest-even everywhere; the decoder arithmetic
// (half(qs·d), half(qm·dm)) is reproduced so codes are chosen against the
// scales the kernels will actually use.
static void pack6x4(const int32_t* v, uint8_t* out3) {
    const uint32_t chunk = (uint32_t)(v[0] & 63) | ((uint32_t)(v[1] & 63) << 6) | ((uint32_t)(v[2] & 63) << 12) |
                           ((uint32_t)(v[3] & 63) << 18);
    out3[0] = (uint8_t)chunk;
    out3[1] = (uint8_t)(chunk >> 8);
    out3[2] = (uint8_t)(chunk >> 16);
}

static inline int32_t rne_clamp(float x, int32_t lo, int32_t hi) {
    if (!(x == x)) return 0;
    float r = std::nearbyint(x);
    if (r < (float)lo) return lo;
    if (r > (float)hi) return hi;
    return (int32_t)r;
}

rwkv_status rwkvq_encode_sb6(const float* w, int64_t OUT, int64_t IN, int bits, uint8_t* codes_packed, uint8_t* qh,
                             uint8_t* qh2, uint8_t* gw_qsqm, uint16_t* gw_d, uint16_t* gw_dm, int nthreads) {
    RWKV_REQUIRE(w && codes_packed && gw_qsqm && gw_d && gw_dm, RWKV_E_NULL, "encode_sb6: null buffer");
    RWKV_REQUIRE(bits >= 4 && bits <= 6, RWKV_E_SHAPE, "encode_sb6: bits %d outside 4...6", bits);
    RWKV_REQUIRE((bits < 5 || qh) && (bits < 6 || qh2), RWKV_E_NULL, "encode_sb6: bit-plane buffers missing");
    RWKV_REQUIRE(OUT >= 1 && IN >= 256 && IN % 256 == 0, RWKV_E_SHAPE, "encode_sb6: IN must be a multiple of 256");
    const int64_t NB = IN / 32, NSB = NB / 8;
    const int32_t qmax = (1 << bits) - 1;
    rwkv::parallel_rows(OUT, nthreads, [&](int64_t row) {
        const float* wr = w + row * IN;
        for (int64_t sb = 0; sb < NSB; ++sb) {
            float sblk[8], mblk[8];
            float smax = 0.0f, mabs = 0.0f;
            for (int e = 0; e < 8; ++e) {
                const float* wb = wr + (sb * 8 + e) * 32;
                float mn = wb[0], mx = wb[0];
                for (int c = 1; c < 32; ++c) { mn = std::min(mn, wb[c]); mx = std::max(mx, wb[c]); }
                sblk[e] = (mx - mn) / (float)qmax;
                mblk[e] = mn;
                smax = std::max(smax, sblk[e]);
                mabs = std::max(mabs, std::fabs(mn));
            }
            const uint16_t d16 = rwkv::f32_to_f16(smax / 63.0f), dm16 = rwkv::f32_to_f16(mabs / 31.0f);
            const float d = rwkv::f16_to_f32(d16), dm = rwkv::f16_to_f32(dm16);
            gw_d[row * NSB + sb] = d16;
            gw_dm[row * NSB + sb] = dm16;
            int32_t qs[8], qms[8];
            for (int e = 0; e < 8; ++e) {
                qs[e] = d > 0.0f ? rne_clamp(sblk[e] / d, 0, 63) : 0;
                const int32_t qm = dm > 0.0f ? rne_clamp(mblk[e] / dm, -31, 32) : 0;
                qms[e] = qm + 31;
                const float s = rwkv::hround((float)qs[e] * d), m = rwkv::hround((float)qm * dm);
                const int64_t blk = sb * 8 + e;
                const float* wb = wr + blk * 32;
                int32_t q[32];
                for (int c = 0; c < 32; ++c) q[c] = s > 0.0f ? rne_clamp((wb[c] - m) / s, 0, qmax) : 0;
                uint8_t* cp = codes_packed + (row * NB + blk) * 16;
                for (int c = 0; c < 16; ++c) cp[c] = (uint8_t)((q[c] & 0xf) | ((q[c + 16] & 0xf) << 4));
                if (bits >= 5) {
                    uint32_t hb = 0;
                    for (int c = 0; c < 32; ++c) hb |= (uint32_t)((q[c] >> 4) & 1) << c;
                    std::memcpy(qh + (row * NB + blk) * 4, &hb, 4);
                }
                if (bits >= 6) {
                    uint32_t hb2 = 0;
                    for (int c = 0; c < 32; ++c) hb2 |= (uint32_t)((q[c] >> 5) & 1) << c;
                    std::memcpy(qh2 + (row * NB + blk) * 4, &hb2, 4);
                }
            }
            uint8_t* dst = gw_qsqm + (row * NSB + sb) * 12;
            pack6x4(qs, dst);
            pack6x4(qs + 4, dst + 3);
            pack6x4(qms, dst + 6);
            pack6x4(qms + 4, dst + 9);
        }
    });
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status rwkvq_encode_sym(const float* w, int64_t OUT, int64_t IN, int bits, uint8_t* codes, uint8_t* codes_packed,
                             uint8_t* qh, uint8_t* qh2, uint8_t* gw_qs, uint16_t* gw_d, int nthreads) {
    RWKV_REQUIRE(w && gw_qs && gw_d, RWKV_E_NULL, "encode_sym: null buffer");
    RWKV_REQUIRE(bits == 6 || bits == 8, RWKV_E_SHAPE, "encode_sym: bits %d outside {6, 8}", bits);
    RWKV_REQUIRE(bits == 8 ? codes != nullptr : (codes_packed && qh && qh2), RWKV_E_NULL, "encode_sym: code buffers missing");
    RWKV_REQUIRE(OUT >= 1 && IN >= 256 && IN % 256 == 0, RWKV_E_SHAPE, "encode_sym: IN must be a multiple of 256");
    const int64_t NB = IN / 16, NSB = NB / 16;
    const float qden = bits == 8 ? 127.0f : 31.0f;
    const int32_t lo = bits == 8 ? -128 : -32, hi = bits == 8 ? 127 : 31;
    rwkv::parallel_rows(OUT, nthreads, [&](int64_t row) {
        const float* wr = w + row * IN;
        std::vector<int32_t> q(IN);
        for (int64_t sb = 0; sb < NSB; ++sb) {
            float sblk[16], smax = 0.0f;
            for (int e = 0; e < 16; ++e) {
                const float* wb = wr + (sb * 16 + e) * 16;
                float amax = 0.0f;
                for (int c = 0; c < 16; ++c) amax = std::max(amax, std::fabs(wb[c]));
                sblk[e] = amax / qden;
                smax = std::max(smax, sblk[e]);
            }
            const uint16_t d16 = rwkv::f32_to_f16(smax / 127.0f);
            const float d = rwkv::f16_to_f32(d16);
            gw_d[row * NSB + sb] = d16;
            for (int e = 0; e < 16; ++e) {
                const int64_t blk = sb * 16 + e;
                const int32_t qsv = d > 0.0f ? rne_clamp(sblk[e] / d, -128, 127) : 0;
                gw_qs[row * NB + blk] = (uint8_t)(int8_t)qsv;
                const float s = rwkv::hround((float)qsv * d);
                for (int c = 0; c < 16; ++c) q[blk * 16 + c] = s != 0.0f ? rne_clamp(wr[blk * 16 + c] / s, lo, hi) : 0;
            }
        }
        if (bits == 8) {
            for (int64_t c = 0; c < IN; ++c) codes[row * IN + c] = (uint8_t)(int8_t)q[c];
        } else {
            const int64_t NP = IN / 32;
            for (int64_t p = 0; p < NP; ++p) {
                const int32_t* qp = q.data() + p * 32;
                uint8_t* cp = codes_packed + (row * NP + p) * 16;
                uint32_t hb = 0, hb2 = 0;
                for (int half = 0; half < 2; ++half)
                    for (int j = 0; j < 8; ++j) {
                        const int32_t lo4 = qp[16 * half + j] + 32, hi4 = qp[16 * half + j + 8] + 32;
                        cp[8 * half + j] = (uint8_t)((lo4 & 0xf) | ((hi4 & 0xf) << 4));
                    }
                for (int c = 0; c < 32; ++c) {
                    const int32_t st = qp[c] + 32;
                    hb |= (uint32_t)((st >> 4) & 1) << c;
                    hb2 |= (uint32_t)((st >> 5) & 1) << c;
                }
                std::memcpy(qh + (row * NP + p) * 4, &hb, 4);
                std::memcpy(qh2 + (row * NP + p) * 4, &hb2, 4);
            }
        }
    });
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"

// ─────────────────────────────── safetensors container ───────────────────────────────
using rwkv::Entry;
using rwkv::JParser;
using rwkv::JVal;
using rwkv::dtype_bytes;

extern "C" {

rwkv_status rwkvq_open(const char* path, rwkvq_file** out) {
    RWKV_REQUIRE(path && out, RWKV_E_NULL, "rwkvq_open: null argument");
    *out = nullptr;
    int fd = ::open(path, O_RDONLY);
    RWKV_REQUIRE(fd >= 0, RWKV_E_IO, "%s: no such file", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        set_error("%s: not a regular file", path);
        return RWKV_E_IO;
    }
    const size_t size = (size_t)st.st_size;
    if (size < 8) {
        ::close(fd);
        set_error("%s: file shorter than the safetensors header", path);
        return RWKV_E_FORMAT;
    }
    void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    RWKV_REQUIRE(map != MAP_FAILED, RWKV_E_IO, "%s: mmap failed", path);
    std::unique_ptr<rwkvq_file, void (*)(rwkvq_file*)> f(new rwkvq_file, rwkvq_close);
    f->map = map;
    f->size = size;
    const uint8_t* bytes = static_cast<const uint8_t*>(map);
    // torch.save zip (the pickle container of the previous era), RwkvqFile.swift:62-69
    RWKV_REQUIRE(!(bytes[0] == 0x50 && bytes[1] == 0x4B && bytes[2] == 0x03 && bytes[3] == 0x04), RWKV_E_FORMAT,
                 "%s: this is a pickle container (torch.save zip), not safetensors", path);
    uint64_t n = 0;
    for (int e = 0; e < 8; ++e) n |= (uint64_t)bytes[e] << (8 * e);
    RWKV_REQUIRE(n > 0 && n <= (uint64_t)(size - 8), RWKV_E_FORMAT, "%s: header length %llu outside the file", path,
                 (unsigned long long)n);
    const int64_t base = 8 + (int64_t)n;
    JParser jp{reinterpret_cast<const char*>(bytes + 8), reinterpret_cast<const char*>(bytes + base), {}};
    JVal root;
    RWKV_REQUIRE(jp.value(root, 0), RWKV_E_FORMAT, "%s: bad safetensors header (%s)", path, jp.err.c_str());
    RWKV_REQUIRE(root.kind == JVal::Obj, RWKV_E_FORMAT, "%s: safetensors header is not an object", path);
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            // a metadata value that is not a string map is ignored as a whole
            bool all_str = kv.second.kind == JVal::Obj;
            if (all_str)
                for (auto& m : kv.second.obj) all_str = all_str && m.second.kind == JVal::Str;
            if (all_str)
                for (auto& m : kv.second.obj) f->metadata[m.first] = m.second.s;
            continue;
        }
        const JVal& d = kv.second;
        const JVal *dt = nullptr, *shape = nullptr, *off = nullptr;
        if (d.kind == JVal::Obj)
            for (auto& m : d.obj) {
                if (m.first == "dtype") dt = &m.second;
                else if (m.first == "shape") shape = &m.second;
                else if (m.first == "data_offsets") off = &m.second;
            }
        RWKV_REQUIRE(dt && dt->kind == JVal::Str && shape && shape->kind == JVal::Arr && off && off->kind == JVal::Arr &&
                         off->arr.size() == 2,
                     RWKV_E_FORMAT, "%s: incomplete entry for buffer %s", path, kv.first.c_str());
        Entry e;
        e.name = kv.first;
        e.dtype = dt->s;
        const int64_t esz = dtype_bytes(e.dtype);
        RWKV_REQUIRE(esz > 0, RWKV_E_FORMAT, "%s: dtype %s of buffer %s is not supported", path, e.dtype.c_str(),
                     e.name.c_str());
        // Every product and sum below is checked: a header is untrusted input,
        // and a wrapped size would let an entry point past the mapping.
        int64_t count = 1;
        bool wrapped = false;
        for (auto& s : shape->arr) {
            RWKV_REQUIRE(s.kind == JVal::Num && s.is_int && s.i >= 0, RWKV_E_FORMAT, "%s: bad shape of %s", path,
                         e.name.c_str());
            e.shape.push_back(s.i);
            wrapped = wrapped || __builtin_mul_overflow(count, s.i, &count);
        }
        int64_t nbytes = 0;
        wrapped = wrapped || __builtin_mul_overflow(count, esz, &nbytes);
        RWKV_REQUIRE(!wrapped, RWKV_E_FORMAT, "%s: the shape of %s overflows 64-bit sizes", path, e.name.c_str());
        RWKV_REQUIRE(off->arr[0].kind == JVal::Num && off->arr[0].is_int && off->arr[1].kind == JVal::Num &&
                         off->arr[1].is_int,
                     RWKV_E_FORMAT, "%s: bad data_offsets of %s", path, e.name.c_str());
        e.begin = off->arr[0].i;
        e.end = off->arr[1].i;
        const int64_t payload = (int64_t)size - base;   // > 0: base <= size was checked above
        RWKV_REQUIRE(e.begin >= 0 && e.end >= e.begin && e.end <= payload && e.end - e.begin == nbytes,
                     RWKV_E_FORMAT, "%s: buffer %s offsets [%lld, %lld] disagree with its shape and dtype %s", path,
                     e.name.c_str(), (long long)e.begin, (long long)e.end, e.dtype.c_str());
        e.begin += base;
        e.end += base;
        f->entries.push_back(std::move(e));
    }
    std::sort(f->entries.begin(), f->entries.end(), [](const Entry& a, const Entry& b) { return a.name < b.name; });
    madvise(map, size, MADV_WILLNEED);
    *out = f.release();
    rwkv::clear_error();
    return RWKV_OK;
}

void rwkvq_close(rwkvq_file* f) {
    if (!f) return;
    if (f->map) munmap(f->map, f->size);
    delete f;
}

int64_t rwkvq_count(const rwkvq_file* f) { return f ? (int64_t)f->entries.size() : 0; }

rwkv_status rwkvq_entry(const rwkvq_file* f, int64_t i, const char** name, const char** dtype, int* ndim,
                        const int64_t** shape, const void** data, int64_t* nbytes) {
    RWKV_REQUIRE(f, RWKV_E_NULL, "rwkvq_entry: null file");
    RWKV_REQUIRE(i >= 0 && i < (int64_t)f->entries.size(), RWKV_E_SHAPE, "rwkvq_entry: index %lld out of range",
                 (long long)i);
    const Entry& e = f->entries[(size_t)i];
    if (name) *name = e.name.c_str();
    if (dtype) *dtype = e.dtype.c_str();
    if (ndim) *ndim = (int)e.shape.size();
    if (shape) *shape = e.shape.data();
    if (data) *data = static_cast<const uint8_t*>(f->map) + e.begin;
    if (nbytes) *nbytes = e.end - e.begin;
    return RWKV_OK;
}

const char* rwkvq_metadata(const rwkvq_file* f, const char* key) {
    if (!f || !key) return nullptr;
    auto it = f->metadata.find(key);
    return it == f->metadata.end() ? nullptr : it->second.c_str();
}

}  // extern "C"
