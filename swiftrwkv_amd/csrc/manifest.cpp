// The .rwkvq manifest: the JSON held in the safetensors `__metadata__` under
// "rwkvq", checked as a whole against the container's buffer table before any
// byte is read, and the repacks of sb6 / sym matrices straight from the
// mapped file into the loader layouts the kernels read.
//
// The format is the reference's (Sources/RWKVQuant/RwkvqFile.swift:254-492,
// RwkvqSidecar.swift:60-99); the checks are organised here as one table per
// layout — which buffers it reads, their element size and exact element count
// or shape as a function of (OUT, IN) — driven by one generic loop, so every
// buffer a kernel will later index is known to be complete.  A file that
// passes cannot make a repack or a kernel read outside a buffer.

#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "container.h"

using rwkv::Entry;
using rwkv::JVal;

namespace {

enum Field { F_DENSE, F_CODES, F_CODES_PACKED, F_QH, F_QH2, F_QSQM, F_D, F_DM, F_QS, F_SCALE, F_MIN, F_RTN_SCALE,
             F_OUTLIERS, F_COUNT };
const char* const kField[F_COUNT] = {"dense", "codes", "codes_packed", "gw_qh", "gw_qh2", "gw_qsqm", "gw_d",
                                     "gw_dm", "gw_qs", "gw_scale", "gw_min", "scale", "outlier_indices"};

struct Tensor {
    std::string key;
    int kind = RWKVQ_DENSE;
    std::vector<int64_t> shape;
    int bits = 16, xbits = 0, gs = 0, sb = 0;
    bool transposed = false, packed = false;
    int64_t outliers = 0;
    const Entry* buf[F_COUNT] = {};
};

// A buffer a layout reads: element size in bytes (0 = any), and either an
// exact shape, an element count, or neither (presence only).
struct Want {
    Field field;
    int elem;
    std::vector<int64_t> dims;
    int64_t count;
};

const JVal* member(const JVal& obj, const char* name) {
    if (obj.kind != JVal::Obj) return nullptr;
    for (auto& kv : obj.obj)
        if (kv.first == name) return &kv.second;
    return nullptr;
}

int64_t int_or(const JVal& obj, const char* name, int64_t dflt) {
    const JVal* v = member(obj, name);
    return (v && v->kind == JVal::Num && v->is_int) ? v->i : dflt;
}

// World checkpoints keep att.{w,a,v,g}{1,2} as [in, out] (RwkvqFileTests.swift:123-127).
bool raw_lora_world(const std::string& key) {
    std::vector<std::string> part;
    size_t s = 0;
    for (;;) {
        size_t e = key.find('.', s);
        part.push_back(key.substr(s, e == std::string::npos ? std::string::npos : e - s));
        if (e == std::string::npos) break;
        s = e + 1;
    }
    return part.size() == 4 && part[0] == "blocks" && part[2] == "att" && part[3].size() == 2 &&
           std::strchr("wavg", part[3][0]) && (part[3][1] == '1' || part[3][1] == '2');
}

void put_dims(int64_t* dst, int* n, const std::vector<int64_t>& src) {
    *n = (int)std::min<size_t>(src.size(), 4);
    for (int e = 0; e < *n; ++e) dst[e] = src[(size_t)e];
}

struct Checker {
    const rwkvq_file* f;
    rwkvq_finding* out;

    rwkv_status malformed(const std::string& tensor, const char* fmt, ...) __attribute__((format(printf, 3, 4))) {
        char msg[768];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, sizeof msg, fmt, ap);
        va_end(ap);
        if (out) {
            out->kind = RWKVQ_FINDING_MALFORMED;
            std::snprintf(out->tensor, sizeof out->tensor, "%s", tensor.c_str());
        }
        rwkv::set_error("%s", msg);
        return RWKV_E_FORMAT;
    }

    rwkv_status missing(const Tensor& t, Field fld) {
        if (out) {
            out->kind = RWKVQ_FINDING_MISSING_BUFFER;
            std::snprintf(out->tensor, sizeof out->tensor, "%s", t.key.c_str());
            std::snprintf(out->buffer, sizeof out->buffer, "%s", kField[fld]);
        }
        rwkv::set_error("%s reads buffer %s::%s, which the file does not hold", t.key.c_str(), t.key.c_str(),
                        kField[fld]);
        return RWKV_E_FORMAT;
    }

    rwkv_status mismatch(const Tensor& t, Field fld, const std::vector<int64_t>& want, const Entry& got) {
        if (out) {
            out->kind = RWKVQ_FINDING_SHAPE;
            std::snprintf(out->tensor, sizeof out->tensor, "%s", t.key.c_str());
            std::snprintf(out->buffer, sizeof out->buffer, "%s", kField[fld]);
            put_dims(out->expected, &out->n_expected, want);
            put_dims(out->got, &out->n_got, got.shape);
        }
        std::string w, g;
        for (int64_t x : want) w += (w.empty() ? "" : ", ") + std::to_string(x);
        for (int64_t x : got.shape) g += (g.empty() ? "" : ", ") + std::to_string(x);
        rwkv::set_error("%s::%s: the layout needs [%s] (%s), the file holds [%s] of %s", t.key.c_str(), kField[fld],
                        w.c_str(), want.size() == 1 ? "elements" : "shape", g.c_str(), got.dtype.c_str());
        return RWKV_E_FORMAT;
    }

    bool has(const Tensor& t, Field fld) const { return rwkvq_find(f, t.key + "::" + kField[fld]) != nullptr; }

    // The scalar rules of each layout, the variant the present buffers select,
    // and the table of buffers that variant reads.
    rwkv_status layout(Tensor& t, const JVal& m, std::vector<Want>& wants) {
        const int64_t n_blocks = int_or(m, "n_blocks", 0);
        const bool two_d = t.shape.size() == 2;
        const int64_t OUT = two_d ? t.shape[0] : 0, IN = two_d ? t.shape[1] : 0;
        switch (t.kind) {
            case RWKVQ_DENSE:
                wants.push_back({F_DENSE, 0, {}, -1});
                return RWKV_OK;
            case RWKVQ_RTN:
                t.packed = has(t, F_CODES_PACKED);
                wants.push_back({t.packed ? F_CODES_PACKED : F_CODES, 0, {}, -1});
                wants.push_back({F_RTN_SCALE, 0, {}, -1});
                if (const Entry* o = rwkvq_find(f, t.key + "::" + kField[F_OUTLIERS]))
                    t.outliers = o->shape.empty() ? 0 : o->shape[0];
                return RWKV_OK;
            case RWKVQ_ASYM: {
                if (!two_d || t.gs <= 0)
                    return malformed(t.key, "%s: an asym entry needs a 2-D shape and gw_gs > 0", t.key.c_str());
                const int64_t nb = (IN + t.gs - 1) / t.gs;   // a short last block has its own scale
                if (n_blocks > 0 && n_blocks != nb)
                    return malformed(t.key, "%s: n_blocks = %lld in the manifest, the shape has %lld blocks",
                                     t.key.c_str(), (long long)n_blocks, (long long)nb);
                wants.push_back({F_SCALE, 0, {}, OUT * nb});
                wants.push_back({F_CODES, 0, {}, OUT * IN});
                wants.push_back({F_MIN, 0, {}, OUT * nb});
                return RWKV_OK;
            }
            case RWKVQ_SB6: {
                if (!two_d || t.gs != 32 || t.sb != 8 || IN % 256 != 0 || OUT < 1)
                    return malformed(t.key,
                                     "%s: sb6 is decoded with blocks of 32 columns in super-blocks of 8 and IN a "
                                     "multiple of 256; the manifest has gw_gs = %d, gw_sb = %d and %d-D shape "
                                     "[%lld, %lld]",
                                     t.key.c_str(), t.gs, t.sb, (int)t.shape.size(), (long long)OUT, (long long)IN);
                if (n_blocks > 0 && n_blocks != IN / 32)
                    return malformed(t.key, "%s: n_blocks = %lld in the manifest, the shape has %lld blocks",
                                     t.key.c_str(), (long long)n_blocks, (long long)(IN / 32));
                const bool qh = has(t, F_QH), qh2 = has(t, F_QH2);
                if (qh2 && !qh)
                    return malformed(t.key, "%s: a second high-bit plane (gw_qh2) without the first", t.key.c_str());
                t.xbits = (int)qh + (int)qh2;
                if (t.bits != 4 + t.xbits)
                    return malformed(t.key, "%s: %d-bit codes need %d high-bit planes; the file has %d bit planes",
                                     t.key.c_str(), t.bits, t.bits - 4, t.xbits);
                wants.push_back({F_QSQM, 1, {OUT, IN / 256, 12}, -1});
                wants.push_back({F_CODES_PACKED, 1, {}, OUT * IN / 2});
                wants.push_back({F_D, 2, {}, OUT * (IN / 256)});
                wants.push_back({F_DM, 2, {}, OUT * (IN / 256)});
                if (qh) wants.push_back({F_QH, 1, {}, OUT * IN / 8});
                if (qh2) wants.push_back({F_QH2, 1, {}, OUT * IN / 8});
                return RWKV_OK;
            }
            case RWKVQ_SYM: {
                if (!two_d || t.gs != 16 || t.sb != 16 || IN % 16 != 0 || OUT < 1)
                    return malformed(t.key,
                                     "%s: sym is decoded with blocks of 16 columns in super-blocks of 16 and IN a "
                                     "multiple of 16; the manifest has gw_gs = %d, gw_sb = %d and %d-D shape "
                                     "[%lld, %lld]",
                                     t.key.c_str(), t.gs, t.sb, (int)t.shape.size(), (long long)OUT, (long long)IN);
                if (n_blocks > 0 && n_blocks != IN / 16)
                    return malformed(t.key, "%s: n_blocks = %lld in the manifest, the shape has %lld blocks",
                                     t.key.c_str(), (long long)n_blocks, (long long)(IN / 16));
                // the code width follows from which code buffer exists
                const bool eight = has(t, F_CODES);
                if (eight && t.bits != 8)
                    return malformed(t.key, "%s: a codes buffer (8-bit sym) but bits = %d in the manifest",
                                     t.key.c_str(), t.bits);
                if (!eight && (t.bits != 6 || IN % 32 != 0))
                    return malformed(t.key, "%s: packed sym codes need bits = 6 and IN %% 32 == 0 (bits = %d, IN = %lld)",
                                     t.key.c_str(), t.bits, (long long)IN);
                wants.push_back({F_QS, 1, {OUT, IN / 16}, -1});
                // one scale per 256 columns: a width off the super-block has no d layout
                wants.push_back({F_D, 2, {OUT, IN % 256 ? -1 : IN / 256}, -1});
                if (eight) {
                    wants.push_back({F_CODES, 1, {}, OUT * IN});
                } else {
                    wants.push_back({F_CODES_PACKED, 1, {}, OUT * IN / 2});
                    wants.push_back({F_QH, 1, {}, OUT * IN / 8});
                    wants.push_back({F_QH2, 1, {}, OUT * IN / 8});
                }
                return RWKV_OK;
            }
        }
        return malformed(t.key, "%s: unknown layout", t.key.c_str());
    }

    rwkv_status buffers(Tensor& t, const std::vector<Want>& wants) {
        for (const Want& w : wants) {
            const Entry* e = rwkvq_find(f, t.key + "::" + kField[w.field]);
            if (!e) return missing(t, w.field);
            const int64_t esz = rwkv::dtype_bytes(e->dtype);
            const int64_t n = esz > 0 ? (e->end - e->begin) / esz : -1;
            const bool elem_ok = w.elem == 0 || esz == w.elem;
            if (!w.dims.empty()) {
                if (!elem_ok || e->shape != w.dims) return mismatch(t, w.field, w.dims, *e);
            } else if (w.count >= 0) {
                if (!elem_ok || n != w.count) return mismatch(t, w.field, {w.count}, *e);
            }
            t.buf[w.field] = e;
        }
        return RWKV_OK;
    }

    rwkv_status tensor(const std::string& key, const JVal& m, const std::string& naming, Tensor& t) {
        t.key = key;
        const JVal* shape = member(m, "shape");
        const JVal* kind = member(m, "kind");
        if (!shape || shape->kind != JVal::Arr || !kind || kind->kind != JVal::Str)
            return malformed(key, "%s: a manifest entry needs a shape and a kind", key.c_str());
        for (auto& s : shape->arr) {
            if (s.kind != JVal::Num || !s.is_int || s.i < 0)
                return malformed(key, "%s: the shape holds a value that is not a size", key.c_str());
            t.shape.push_back(s.i);
        }
        static const std::pair<const char*, int> kinds[] = {
            {"dense", RWKVQ_DENSE}, {"sb6", RWKVQ_SB6}, {"sym", RWKVQ_SYM}, {"asym", RWKVQ_ASYM}, {"rtn", RWKVQ_RTN}};
        t.kind = -1;
        for (auto& k : kinds)
            if (kind->s == k.first) t.kind = k.second;
        if (t.kind < 0) return malformed(key, "%s: unknown layout \"%s\"", key.c_str(), kind->s.c_str());
        t.bits = (int)int_or(m, "bits", 16);
        t.gs = (int)int_or(m, "gw_gs", 0);
        t.sb = (int)int_or(m, "gw_sb", 0);
        const JVal* tr = member(m, "transposed");
        t.transposed = (tr && tr->kind == JVal::Bool) ? tr->b : (naming == "world" && raw_lora_world(key));
        if (t.shape.size() == 2 && (t.shape[0] > (int64_t)1 << 31 || t.shape[1] > (int64_t)1 << 31))
            return malformed(key, "%s: a matrix side above 2^31", key.c_str());
        std::vector<Want> wants;
        rwkv_status st = layout(t, m, wants);
        return st != RWKV_OK ? st : buffers(t, wants);
    }
};

}  // namespace

struct rwkvq_manifest {
    std::vector<Tensor> tensors;   // sorted by key
    std::string naming;
    int format_version = 0;
    int64_t n_layer = 0, n_embd = 0, head_size = 64, vocab_size = 0;
};

const Entry* rwkvq_find(const rwkvq_file* f, const std::string& name) {
    auto it = std::lower_bound(f->entries.begin(), f->entries.end(), name,
                               [](const Entry& e, const std::string& n) { return e.name < n; });
    return (it != f->entries.end() && it->name == name) ? &*it : nullptr;
}

namespace {

const Tensor* tensor_at(const rwkvq_manifest* m, int64_t i) {
    return (m && i >= 0 && i < (int64_t)m->tensors.size()) ? &m->tensors[(size_t)i] : nullptr;
}

// Rows [r0, r1) of a matrix per thread; a large matrix is split over up to 8.
template <class F>
void over_rows(int64_t rows, int64_t bytes, F&& body) {
    const int nt = bytes < ((int64_t)8 << 20) ? 1 : (int)std::min<int64_t>(8, rows);
    if (nt <= 1) {
        body(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    for (int k = 0; k < nt; ++k) pool.emplace_back([&, k] { body(rows * k / nt, rows * (k + 1) / nt); });
    for (auto& th : pool) th.join();
}

const uint8_t* bytes_of(const rwkvq_file* f, const Entry* e) {
    return e ? static_cast<const uint8_t*>(f->map) + e->begin : nullptr;
}

}  // namespace

extern "C" {

rwkv_status rwkvq_manifest_read(const rwkvq_file* f, int max_format_version, rwkvq_manifest** out,
                                rwkvq_finding* finding) {
    if (finding) std::memset(finding, 0, sizeof *finding);
    RWKV_REQUIRE(f && out, RWKV_E_NULL, "rwkvq_manifest_read: null argument");
    *out = nullptr;
    Checker ck{f, finding};
    auto meta = f->metadata.find("rwkvq");
    JVal root;
    if (meta != f->metadata.end()) {
        rwkv::JParser jp{meta->second.data(), meta->second.data() + meta->second.size(), {}};
        if (!jp.value(root, 0)) root = JVal{};
    }
    if (root.kind != JVal::Obj)
        return ck.malformed("", "not an .rwkvq file: __metadata__ holds no rwkvq manifest object");
    const JVal* fmt = member(root, "format");
    if (!fmt || fmt->kind != JVal::Str || fmt->s != "rwkvq")
        return ck.malformed("", "the manifest's format is not \"rwkvq\"");
    std::unique_ptr<rwkvq_manifest> m(new rwkvq_manifest);
    m->format_version = (int)int_or(root, "format_version", 0);
    if (m->format_version > max_format_version)
        return ck.malformed("", "format_version %d is newer than this reader's %d", m->format_version,
                            max_format_version);
    const JVal* tensors = member(root, "tensors");
    if (!tensors || tensors->kind != JVal::Obj) return ck.malformed("", "the manifest has no \"tensors\" object");
    const JVal* naming = member(root, "naming");
    m->naming = (naming && naming->kind == JVal::Str) ? naming->s : "world";
    m->n_layer = int_or(root, "n_layer", 0);
    m->n_embd = int_or(root, "n_embd", 0);
    m->head_size = int_or(root, "head_size", 64);
    m->vocab_size = int_or(root, "vocab_size", 0);
    m->tensors.reserve(tensors->obj.size());
    for (auto& kv : tensors->obj) {
        Tensor t;
        rwkv_status st = ck.tensor(kv.first, kv.second, m->naming, t);
        if (st != RWKV_OK) return st;
        m->tensors.push_back(std::move(t));
    }
    std::sort(m->tensors.begin(), m->tensors.end(), [](const Tensor& a, const Tensor& b) { return a.key < b.key; });
    for (size_t i = 1; i < m->tensors.size(); ++i)
        if (m->tensors[i].key == m->tensors[i - 1].key)
            return ck.malformed(m->tensors[i].key, "%s: listed twice in the manifest", m->tensors[i].key.c_str());
    *out = m.release();
    rwkv::clear_error();
    return RWKV_OK;
}

void rwkvq_manifest_free(rwkvq_manifest* m) { delete m; }

int64_t rwkvq_manifest_count(const rwkvq_manifest* m) { return m ? (int64_t)m->tensors.size() : 0; }

rwkv_status rwkvq_manifest_model(const rwkvq_manifest* m, rwkvq_model* out) {
    RWKV_REQUIRE(m && out, RWKV_E_NULL, "rwkvq_manifest_model: null argument");
    out->format_version = m->format_version;
    out->naming = m->naming.c_str();
    out->n_layer = m->n_layer;
    out->n_embd = m->n_embd;
    out->head_size = m->head_size;
    out->vocab_size = m->vocab_size;
    return RWKV_OK;
}

rwkv_status rwkvq_manifest_tensor(const rwkvq_manifest* m, int64_t i, rwkvq_tensor* out) {
    RWKV_REQUIRE(m && out, RWKV_E_NULL, "rwkvq_manifest_tensor: null argument");
    const Tensor* t = tensor_at(m, i);
    RWKV_REQUIRE(t, RWKV_E_SHAPE, "rwkvq_manifest_tensor: index %lld out of range", (long long)i);
    std::memset(out, 0, sizeof *out);
    out->key = t->key.c_str();
    out->kind = t->kind;
    out->ndim = (int)std::min<size_t>(t->shape.size(), 8);
    for (int e = 0; e < out->ndim; ++e) out->shape[e] = t->shape[(size_t)e];
    out->bits = t->bits;
    out->xbits = t->xbits;
    out->group_size = t->gs;
    out->super_block = t->sb;
    out->transposed = t->transposed;
    out->packed = t->packed;
    out->outliers = t->outliers;
    return RWKV_OK;
}

rwkv_status rwkvq_read_sb6(const rwkvq_file* f, const rwkvq_manifest* m, int64_t i, uint8_t* qblk, uint8_t* qsqm,
                           uint16_t* ddm) {
    RWKV_REQUIRE(f && m && qblk && qsqm && ddm, RWKV_E_NULL, "rwkvq_read_sb6: null argument");
    const Tensor* t = tensor_at(m, i);
    RWKV_REQUIRE(t && t->kind == RWKVQ_SB6, RWKV_E_SHAPE, "rwkvq_read_sb6: entry %lld is not an sb6 matrix",
                 (long long)i);
    const int64_t OUT = t->shape[0], IN = t->shape[1], NB = IN / 32, NSB = IN / 256;
    const int64_t SU = 16 + 4 * t->xbits;
    const uint8_t* codes = bytes_of(f, t->buf[F_CODES_PACKED]);
    const uint8_t* qh = bytes_of(f, t->buf[F_QH]);
    const uint8_t* qh2 = bytes_of(f, t->buf[F_QH2]);
    const uint8_t* packed_scales = bytes_of(f, t->buf[F_QSQM]);
    const uint8_t* d = bytes_of(f, t->buf[F_D]);
    const uint8_t* dm = bytes_of(f, t->buf[F_DM]);
    std::atomic<int> st{RWKV_OK};
    over_rows(OUT, OUT * NB * SU, [&](int64_t r0, int64_t r1) {
        // the fp16 scales may sit at any byte offset of the file: copy them aligned
        std::vector<uint16_t> dd((size_t)((r1 - r0) * NSB)), ddmm(dd.size());
        std::memcpy(dd.data(), d + r0 * NSB * 2, dd.size() * 2);
        std::memcpy(ddmm.data(), dm + r0 * NSB * 2, ddmm.size() * 2);
        rwkv_status s = rwkv_sb6_to_k3(codes + r0 * NB * 16, qh ? qh + r0 * NB * 4 : nullptr,
                                       qh2 ? qh2 + r0 * NB * 4 : nullptr, packed_scales + r0 * NSB * 12, dd.data(),
                                       ddmm.data(), r1 - r0, IN, qblk + r0 * NB * SU, qsqm + r0 * NB * 2,
                                       ddm + r0 * NSB * 2);
        if (s != RWKV_OK) st = s;
    });
    if (st.load() != RWKV_OK) {
        rwkv::set_error("%s: repack failed", t->key.c_str());
        return (rwkv_status)st.load();
    }
    rwkv::clear_error();
    return RWKV_OK;
}

rwkv_status rwkvq_read_sym(const rwkvq_file* f, const rwkvq_manifest* m, int64_t i, uint8_t* qblk, uint8_t* qs,
                           uint16_t* d) {
    RWKV_REQUIRE(f && m && qblk && qs && d, RWKV_E_NULL, "rwkvq_read_sym: null argument");
    const Tensor* t = tensor_at(m, i);
    RWKV_REQUIRE(t && t->kind == RWKVQ_SYM, RWKV_E_SHAPE, "rwkvq_read_sym: entry %lld is not a sym matrix",
                 (long long)i);
    const int64_t OUT = t->shape[0], IN = t->shape[1];
    std::memcpy(qs, bytes_of(f, t->buf[F_QS]), (size_t)(OUT * IN / 16));
    std::memcpy(d, bytes_of(f, t->buf[F_D]), (size_t)(OUT * (IN / 256) * 2));
    if (t->bits == 8) {
        std::memcpy(qblk, bytes_of(f, t->buf[F_CODES]), (size_t)(OUT * IN));
        rwkv::clear_error();
        return RWKV_OK;
    }
    const uint8_t* codes = bytes_of(f, t->buf[F_CODES_PACKED]);
    const uint8_t* qh = bytes_of(f, t->buf[F_QH]);
    const uint8_t* qh2 = bytes_of(f, t->buf[F_QH2]);
    const int64_t NP = IN / 32;
    std::atomic<int> st{RWKV_OK};
    over_rows(OUT, OUT * NP * 24, [&](int64_t r0, int64_t r1) {
        rwkv_status s = rwkv_sym_interleave(codes + r0 * NP * 16, qh + r0 * NP * 4, qh2 + r0 * NP * 4, r1 - r0, IN,
                                            qblk + r0 * NP * 24);
        if (s != RWKV_OK) st = s;
    });
    if (st.load() != RWKV_OK) {
        rwkv::set_error("%s: repack failed", t->key.c_str());
        return (rwkv_status)st.load();
    }
    rwkv::clear_error();
    return RWKV_OK;
}

}  // extern "C"
