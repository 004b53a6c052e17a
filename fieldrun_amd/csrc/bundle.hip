// bundle.hip — the fieldrun bundle reader (host code) and its uploads.
//
// Restates Bundle::load (/root/reference/src/bundle.rs:314-376) for this
// path: `<stem>.fieldrun.json` is the manifest (FORMAT.md: "format" ==
// "fieldrun-bundle", "version" == 1, "arch", "config", optional "config_f",
// "eos" and "store", and "arrays": {name, dtype (default "f32"), shape,
// offset, bytes, optional group}); `<stem>.fieldrun.bin` is the blob, mapped
// read-only and viewed by offset.  A manifest the reference would refuse
// (other format or version, an array past the end of the blob) is
// FRQ_ERR_FORMAT; an absent array is FRQ_ERR_MISSING (378-380).  Uploads
// take the stored precision straight to the device: i8 (in, out) with its
// f16 __scale (the transpose of 345-355 runs on the device), i4 (out, in)
// packed with f16 (out, ceil(in/g)) scales (356-360, group default 32),
// rowi8 with its f16 row scales upcast as arr1o does (921-933), and 2-D
// f16 / f32 tables.  The MoE expert bank of a layer gathers the expert
// arrays by the names qwen3moe / gemma4 use ({p}experts.{e}.gate / .up /
// .down, or .gate_up / .down; src/qwen3moe.rs:148-152, src/gemma4.rs:
// 174-181).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "frq_internal.h"

namespace {

// ---- a small JSON reader: the manifest's values, depth-limited ----------------
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    bool is_int = false;  // an integer literal (no fraction or exponent)
    long long i = 0;
    double d = 0.0;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
    const JVal* get(const char* k) const {
        if (kind != Obj) return nullptr;
        for (const auto& kv : o)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* e;
    int depth = 0;
    std::string err;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    static void put_utf8(std::string& out, unsigned cp) {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18)); out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned& v) {
        if (e - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string& out) {
        if (p >= e || *p != '"') return fail("expected a string");
        ++p;
        while (p < e && *p != '"') {
            if ((unsigned char)*p < 0x20) return fail("control character in a string");
            if (*p != '\\') { out += *p++; continue; }
            if (++p >= e) return fail("truncated escape");
            const char c = *p++;
            switch (c) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        unsigned lo;
                        if (!hex4(lo)) return false;
                        if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= e) return fail("unterminated string");
        ++p;
        return true;
    }
    bool num(JVal& v) {
        const char* s0 = p;
        if (p < e && *p == '-') ++p;
        bool frac = false;
        while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
            if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
            ++p;
        }
        const std::string t(s0, p);
        if (t.empty() || t == "-") return fail("bad number");
        char* end = nullptr;
        v.kind = JVal::Num;
        v.d = std::strtod(t.c_str(), &end);
        if (*end) return fail("bad number");
        if (!frac) {
            errno = 0;
            v.i = std::strtoll(t.c_str(), &end, 10);
            v.is_int = !*end && errno == 0;
        }
        return true;
    }
    bool value(JVal& v) {
        ws();
        if (p >= e) return fail("unexpected end of manifest");
        if (++depth > 200) return fail("manifest nested too deeply");
        bool ok = true;
        const char c = *p;
        if (c == '{') {
            v.kind = JVal::Obj;
            ++p;
            ws();
            if (p < e && *p == '}') ++p;
            else
                for (;;) {
                    std::pair<std::string, JVal> kv;
                    ws();
                    if (!str(kv.first)) { ok = false; break; }
                    ws();
                    if (p >= e || *p != ':') { ok = fail("expected ':'"); break; }
                    ++p;
                    if (!value(kv.second)) { ok = false; break; }
                    v.o.push_back(std::move(kv));
                    ws();
                    if (p < e && *p == ',') { ++p; continue; }
                    if (p < e && *p == '}') { ++p; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
        } else if (c == '[') {
            v.kind = JVal::Arr;
            ++p;
            ws();
            if (p < e && *p == ']') ++p;
            else
                for (;;) {
                    JVal x;
                    if (!value(x)) { ok = false; break; }
                    v.a.push_back(std::move(x));
                    ws();
                    if (p < e && *p == ',') { ++p; continue; }
                    if (p < e && *p == ']') { ++p; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
        } else if (c == '"') {
            v.kind = JVal::Str;
            ok = str(v.s);
        } else if (c == 't' && e - p >= 4 && !std::strncmp(p, "true", 4)) {
            v.kind = JVal::Bool; v.b = true; p += 4;
        } else if (c == 'f' && e - p >= 5 && !std::strncmp(p, "false", 5)) {
            v.kind = JVal::Bool; v.b = false; p += 5;
        } else if (c == 'n' && e - p >= 4 && !std::strncmp(p, "null", 4)) {
            v.kind = JVal::Null; p += 4;
        } else {
            ok = num(v);
        }
        --depth;
        return ok;
    }
};

// A non-negative integer field (the reference's usize).
bool as_size(const JVal* v, size_t& out) {
    if (!v || v->kind != JVal::Num || !v->is_int || v->i < 0) return false;
    out = (size_t)v->i;
    return true;
}

struct ArrSpec {
    std::string dtype = "f32";
    std::vector<size_t> shape;
    size_t offset = 0, bytes = 0, group = 0;  // group 0: none
};

}  // namespace

struct frq_bundle {
    std::string arch;
    std::vector<long long> config, eos;
    std::vector<double> config_f;
    std::unordered_map<std::string, ArrSpec> arrays;
    const uint8_t* blob = nullptr;
    size_t blob_bytes = 0;
    void* map = nullptr;
    size_t map_bytes = 0;
    ~frq_bundle() {
        if (map) munmap(map, map_bytes);
    }
};

namespace {

int open_manifest(frq_bundle& b, const std::string& stem) {
    using frq::set_error;
    const std::string jpath = stem + ".fieldrun.json", bpath = stem + ".fieldrun.bin";
    std::string text;
    {
        const int fd = ::open(jpath.c_str(), O_RDONLY);
        if (fd < 0) return set_error(FRQ_ERR_ARG, "cannot open " + jpath + ": " + std::strerror(errno));
        char buf[1 << 16];
        for (;;) {
            const ssize_t r = ::read(fd, buf, sizeof buf);
            if (r < 0) {
                ::close(fd);
                return set_error(FRQ_ERR_ARG, "cannot read " + jpath);
            }
            if (r == 0) break;
            text.append(buf, (size_t)r);
        }
        ::close(fd);
    }
    JVal root;
    JParser jp{text.data(), text.data() + text.size()};
    if (!jp.value(root)) return set_error(FRQ_ERR_FORMAT, jpath + ": " + jp.err);
    jp.ws();
    if (jp.p != jp.e) return set_error(FRQ_ERR_FORMAT, jpath + ": trailing characters after the manifest");
    const JVal* fmt = root.get("format");
    const JVal* ver = root.get("version");
    size_t version = 0;
    const std::string fs = (fmt && fmt->kind == JVal::Str) ? fmt->s : std::string("?");
    if (!fmt || fmt->kind != JVal::Str || !as_size(ver, version) || fs != "fieldrun-bundle" || version != 1)
        return set_error(FRQ_ERR_FORMAT, "unsupported bundle: " + fs + " v" +
                                             (ver && ver->kind == JVal::Num ? std::to_string((long long)ver->d) : "?") +
                                             " (this fieldrun reads fieldrun-bundle v1)");
    const JVal* arch = root.get("arch");
    const JVal* config = root.get("config");
    const JVal* arrays = root.get("arrays");
    if (!arch || arch->kind != JVal::Str || !config || config->kind != JVal::Arr || !arrays ||
        arrays->kind != JVal::Arr)
        return set_error(FRQ_ERR_FORMAT, jpath + ": manifest needs arch, config and arrays");
    b.arch = arch->s;
    for (const JVal& v : config->a) {
        if (v.kind != JVal::Num || !v.is_int) return set_error(FRQ_ERR_FORMAT, jpath + ": config must be integers");
        b.config.push_back(v.i);
    }
    if (const JVal* cf = root.get("config_f")) {
        if (cf->kind != JVal::Arr) return set_error(FRQ_ERR_FORMAT, jpath + ": config_f must be a list");
        for (const JVal& v : cf->a) {
            if (v.kind != JVal::Num) return set_error(FRQ_ERR_FORMAT, jpath + ": config_f must be numbers");
            b.config_f.push_back(v.d);
        }
    }
    if (const JVal* eos = root.get("eos")) {
        if (eos->kind != JVal::Arr) return set_error(FRQ_ERR_FORMAT, jpath + ": eos must be a list");
        for (const JVal& v : eos->a) {
            if (v.kind != JVal::Num || !v.is_int) return set_error(FRQ_ERR_FORMAT, jpath + ": eos must be integers");
            b.eos.push_back(v.i);
        }
    }
    // the blob, mapped read-only
    const int fd = ::open(bpath.c_str(), O_RDONLY);
    if (fd < 0) return set_error(FRQ_ERR_ARG, "cannot open " + bpath + ": " + std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return set_error(FRQ_ERR_ARG, "cannot stat " + bpath);
    }
    b.blob_bytes = (size_t)st.st_size;
    if (b.blob_bytes) {
        b.map = mmap(nullptr, b.blob_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
        if (b.map == MAP_FAILED) {
            b.map = nullptr;
            ::close(fd);
            return set_error(FRQ_ERR_ARG, "cannot map " + bpath);
        }
        b.map_bytes = b.blob_bytes;
        b.blob = static_cast<const uint8_t*>(b.map);
    }
    ::close(fd);
    for (const JVal& a : arrays->a) {
        const JVal* name = a.get("name");
        const JVal* shape = a.get("shape");
        ArrSpec sp;
        if (!name || name->kind != JVal::Str || !shape || shape->kind != JVal::Arr ||
            !as_size(a.get("offset"), sp.offset) || !as_size(a.get("bytes"), sp.bytes))
            return set_error(FRQ_ERR_FORMAT, jpath + ": an array entry needs name, shape, offset and bytes");
        if (const JVal* dt = a.get("dtype")) {
            if (dt->kind != JVal::Str) return set_error(FRQ_ERR_FORMAT, jpath + ": dtype must be a string");
            sp.dtype = dt->s;
        }
        for (const JVal& d : shape->a) {
            size_t x;
            if (!as_size(&d, x)) return set_error(FRQ_ERR_FORMAT, jpath + ": shape of " + name->s + " must be sizes");
            sp.shape.push_back(x);
        }
        if (const JVal* g = a.get("group"))
            if (g->kind != JVal::Null && !as_size(g, sp.group))
                return set_error(FRQ_ERR_FORMAT, jpath + ": group of " + name->s + " must be a size");
        if (sp.offset > b.blob_bytes || sp.bytes > b.blob_bytes - sp.offset)
            return set_error(FRQ_ERR_FORMAT, name->s + ": bytes [" + std::to_string(sp.offset) + ", +" +
                                                 std::to_string(sp.bytes) + ") beyond the blob (" +
                                                 std::to_string(b.blob_bytes) + " bytes)");
        b.arrays[name->s] = std::move(sp);
    }
    return FRQ_OK;
}

const ArrSpec* find(const frq_bundle* b, const std::string& name) {
    const auto it = b->arrays.find(name);
    if (it == b->arrays.end()) {
        frq::set_error(FRQ_ERR_MISSING, "missing array " + name);
        return nullptr;
    }
    return &it->second;
}

// Product of the dims, false when it overflows size_t (a crafted manifest
// could otherwise wrap it onto the array's byte count).
bool prod(const std::vector<size_t>& s, size_t* out) {
    size_t n = 1;
    for (size_t x : s)
        if (__builtin_mul_overflow(n, x, &n)) return false;
    *out = n;
    return true;
}

// Bytes of an (n, ceil(k/g)) f16 table, false on overflow.
bool group_table_bytes(size_t n, size_t k, size_t g, size_t* out) {
    return g && !__builtin_mul_overflow(n, k / g + (k % g != 0), out) && !__builtin_mul_overflow(*out, (size_t)2, out);
}

// The array, checked to be `dt` with `ndim` dims and `bytes` of content.
const ArrSpec* need(const frq_bundle* b, const std::string& name, const char* dt, size_t ndim) {
    const ArrSpec* s = find(b, name);
    if (!s) return nullptr;
    if (s->dtype != dt || s->shape.size() != ndim) {
        frq::set_error(FRQ_ERR_FORMAT, name + ": expected a " + std::to_string(ndim) + "-D " + dt + " array");
        return nullptr;
    }
    size_t want = 0;
    bool ok = prod(s->shape, &want);
    if (!std::strcmp(dt, "f16")) ok = ok && !__builtin_mul_overflow(want, (size_t)2, &want);
    else if (!std::strcmp(dt, "f32")) ok = ok && !__builtin_mul_overflow(want, (size_t)4, &want);
    else if (!std::strcmp(dt, "i4") || !std::strcmp(dt, "q4a"))
        ok = ok && !__builtin_mul_overflow(s->shape[0], s->shape[1] / 2 + (s->shape[1] & 1), &want);
    if (!ok) {
        frq::set_error(FRQ_ERR_FORMAT, name + ": shape overflows the address space");
        return nullptr;
    }
    if (s->bytes != want) {
        frq::set_error(FRQ_ERR_FORMAT, name + ": " + std::to_string(s->bytes) + " bytes for its shape (" +
                                           std::to_string(want) + " expected)");
        return nullptr;
    }
    return s;
}

std::vector<float> upcast(const frq_bundle* b, const ArrSpec* s) {
    const size_t n = s->bytes / 2;
    std::vector<float> v(n);
    const uint8_t* p = b->blob + s->offset;
    for (size_t i = 0; i < n; ++i) v[i] = frq::h2f_host((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    return v;
}

// The f16 words of an array (the blob is little-endian, so is the host).
const uint16_t* f16_words(const frq_bundle* b, const ArrSpec* s, std::vector<uint16_t>& copy) {
    const uint8_t* p = b->blob + s->offset;
    if (((uintptr_t)p & 1) == 0) return reinterpret_cast<const uint16_t*>(p);
    copy.resize(s->bytes / 2);
    std::memcpy(copy.data(), p, s->bytes);
    return copy.data();
}

}  // namespace

extern "C" {

int frq_bundle_open(const char* stem, frq_bundle** out) {
    if (!stem || !out) return frq::set_error(FRQ_ERR_ARG, "frq_bundle_open: null stem or out");
    *out = nullptr;
    frq_bundle* b = new (std::nothrow) frq_bundle;
    if (!b) return frq::set_error(FRQ_ERR_ARG, "out of host memory");
    if (int rc = open_manifest(*b, stem)) {
        delete b;
        return rc;
    }
    *out = b;
    return FRQ_OK;
}

void frq_bundle_close(frq_bundle* b) { delete b; }

int frq_bundle_header(const frq_bundle* b, char* arch, size_t arch_cap, int64_t* config, size_t* n_config,
                      double* config_f, size_t* n_config_f) {
    if (!b) return frq::set_error(FRQ_ERR_ARG, "null bundle");
    if (arch && arch_cap) {
        const size_t n = b->arch.size() < arch_cap - 1 ? b->arch.size() : arch_cap - 1;
        std::memcpy(arch, b->arch.data(), n);
        arch[n] = 0;
    }
    if (n_config) {
        const size_t cap = *n_config;
        for (size_t i = 0; config && i < cap && i < b->config.size(); ++i) config[i] = b->config[i];
        *n_config = b->config.size();
    }
    if (n_config_f) {
        const size_t cap = *n_config_f;
        for (size_t i = 0; config_f && i < cap && i < b->config_f.size(); ++i) config_f[i] = b->config_f[i];
        *n_config_f = b->config_f.size();
    }
    return FRQ_OK;
}

int frq_bundle_array(const frq_bundle* b, const char* name, char* dtype, size_t dtype_cap, size_t* shape,
                     size_t* ndim, size_t* group, const void** data, size_t* bytes) {
    if (!b || !name) return frq::set_error(FRQ_ERR_ARG, "null bundle or name");
    const ArrSpec* s = find(b, name);
    if (!s) return FRQ_ERR_MISSING;
    if (dtype && dtype_cap) {
        const size_t n = s->dtype.size() < dtype_cap - 1 ? s->dtype.size() : dtype_cap - 1;
        std::memcpy(dtype, s->dtype.data(), n);
        dtype[n] = 0;
    }
    if (ndim) {
        const size_t cap = *ndim;
        for (size_t i = 0; shape && i < cap && i < s->shape.size(); ++i) shape[i] = s->shape[i];
        *ndim = s->shape.size();
    }
    if (group) *group = s->group;
    if (data) *data = b->blob ? b->blob + s->offset : nullptr;
    if (bytes) *bytes = s->bytes;
    return FRQ_OK;
}

static frq_w* bundle_weight(frq_ctx* ctx, const frq_bundle* b, const char* name) {
    if (!b || !name) {
        frq::set_error(FRQ_ERR_ARG, "null bundle or name");
        return nullptr;
    }
    const ArrSpec* s = find(b, name);
    if (!s) return nullptr;
    const std::string nm(name), sn = nm + "__scale";
    const uint8_t* data = b->blob ? b->blob + s->offset : nullptr;
    std::vector<uint16_t> tmp;
    if (s->dtype == "i8") {
        if (!need(b, nm, "i8", 2)) return nullptr;
        const ArrSpec* sc = need(b, sn, "f16", 1);
        if (!sc) return nullptr;
        const size_t k = s->shape[0], n = s->shape[1];
        if (sc->shape[0] != n) {
            frq::set_error(FRQ_ERR_FORMAT, sn + ": one scale per output column expected");
            return nullptr;
        }
        return frq_upload_i8_bundle(ctx, reinterpret_cast<const int8_t*>(data), f16_words(b, sc, tmp), k, n);
    }
    if (s->dtype == "i4") {
        if (!need(b, nm, "i4", 2)) return nullptr;
        const size_t n = s->shape[0], k = s->shape[1], g = s->group ? s->group : 32;
        const ArrSpec* sc = find(b, sn);
        if (!sc) return nullptr;
        size_t want = 0;
        if (sc->dtype != "f16" || !group_table_bytes(n, k, g, &want) || sc->bytes != want) {
            frq::set_error(FRQ_ERR_FORMAT, sn + ": f16 (out, ceil(in/group)) scales expected");
            return nullptr;
        }
        return frq_upload_i4(ctx, data, f16_words(b, sc, tmp), n, k, g);
    }
    if (s->dtype == "q4a") {  // Bundle::load 361-364 (group default 64); __scale and __min per mm (803-804)
        if (!need(b, nm, "q4a", 2)) return nullptr;
        const size_t n = s->shape[0], k = s->shape[1], g = s->group ? s->group : 64;
        const std::string mn = nm + "__min";
        const ArrSpec* sc = find(b, sn);
        if (!sc) return nullptr;
        const ArrSpec* mi = find(b, mn);
        if (!mi) return nullptr;
        size_t want = 0;
        if (sc->dtype != "f16" || !group_table_bytes(n, k, g, &want) || sc->bytes != want || mi->dtype != "f16" ||
            mi->bytes != want) {
            frq::set_error(FRQ_ERR_FORMAT, nm + ": f16 (out, ceil(in/group)) __scale and __min expected");
            return nullptr;
        }
        std::vector<uint16_t> tmp2;
        return frq_upload_q4a(ctx, data, f16_words(b, sc, tmp), f16_words(b, mi, tmp2), n, k, g);
    }
    if (s->dtype == "rowi8") {
        if (!need(b, nm, "rowi8", 2)) return nullptr;
        const ArrSpec* sc = need(b, sn, "f16", 1);
        if (!sc) return nullptr;
        if (sc->shape[0] != s->shape[0]) {
            frq::set_error(FRQ_ERR_FORMAT, sn + ": one scale per row expected");
            return nullptr;
        }
        const std::vector<float> scale = upcast(b, sc);
        return frq_upload_rows(ctx, FRQ_DT_ROWI8, data, scale.data(), s->shape[0], s->shape[1]);
    }
    if (s->dtype == "f16" || s->dtype == "f32") {
        if (!need(b, nm, s->dtype.c_str(), 2)) return nullptr;
        return frq_upload_rows(ctx, s->dtype == "f16" ? FRQ_DT_F16 : FRQ_DT_F32, data, nullptr, s->shape[0],
                               s->shape[1]);
    }
    frq::set_error(FRQ_ERR_DTYPE, nm + ": no device upload for dtype " + s->dtype);
    return nullptr;
}

static frq_moe_w* bundle_moe(frq_ctx* ctx, const frq_bundle* b, const char* prefix, size_t n_exp, int act) {
    if (!b || !prefix || !n_exp || (act != FRQ_ACT_SILU && act != FRQ_ACT_GELU_TANH)) {
        frq::set_error(FRQ_ERR_ARG, "frq_bundle_moe: null bundle / prefix, no experts or unknown act");
        return nullptr;
    }
    const std::string p(prefix);
    const bool silu_ = act == FRQ_ACT_SILU;
    // the bank's dtype is the first expert's (expert_f32's arms, src/bundle.rs:408-452)
    const std::string g0 = p + "experts.0." + (silu_ ? "gate" : "gate_up");
    const ArrSpec* s0 = find(b, g0);
    if (!s0) return nullptr;
    const std::string dt = s0->dtype;
    int dtype;
    if (dt == "i8") dtype = FRQ_DT_I8;
    else if (dt == "i4") dtype = FRQ_DT_I4;
    else if (dt == "q4a") dtype = FRQ_DT_Q4A;
    else if (dt == "f16") dtype = FRQ_DT_F16;
    else if (dt == "f32") dtype = FRQ_DT_F32;
    else {
        frq::set_error(FRQ_ERR_DTYPE, g0 + ": expert dtype " + dt + " unsupported");  // :452
        return nullptr;
    }
    const bool q = dtype == FRQ_DT_I4 || dtype == FRQ_DT_Q4A;
    if (!need(b, g0, dt.c_str(), 2)) return nullptr;
    // i8 / f16 / f32 store (in, out), i4 / q4a (out, in) (src/convert.rs:174-260)
    const size_t d = q ? s0->shape[1] : s0->shape[0], gwid = q ? s0->shape[0] : s0->shape[1];
    if (!silu_ && gwid % 2) {
        frq::set_error(FRQ_ERR_FORMAT, g0 + ": gate_up width must be even");
        return nullptr;
    }
    const size_t mi = silu_ ? gwid : gwid / 2;
    // i4 / q4a group: the manifest's, else the loader's defaults (32 / 64, src/bundle.rs:422, 435)
    const size_t g = q ? (s0->group ? s0->group : (dtype == FRQ_DT_I4 ? 32 : 64)) : 0;
    std::vector<const void*> gate(n_exp), up(n_exp, nullptr), down(n_exp);
    std::vector<const uint16_t*> gs(n_exp, nullptr), us(n_exp, nullptr), ds(n_exp, nullptr);
    std::vector<const uint16_t*> gm(n_exp, nullptr), um(n_exp, nullptr), dm(n_exp, nullptr);
    // one expert matrix of logical (in, out), its siblings checked against it
    auto take = [&](const std::string& nm, size_t in, size_t out, const void*& w, const uint16_t*& sc,
                    const uint16_t*& mn) {
        const ArrSpec* a = need(b, nm, dt.c_str(), 2);
        if (!a) return false;
        const size_t r0 = q ? out : in, r1 = q ? in : out;
        if (a->shape[0] != r0 || a->shape[1] != r1 || (q && (a->group ? a->group : g) != g)) {
            frq::set_error(FRQ_ERR_FORMAT, nm + ": shape or group differs from the other experts'");
            return false;
        }
        w = b->blob + a->offset;
        if (dtype == FRQ_DT_F16 || dtype == FRQ_DT_F32) return true;
        const size_t ns = dtype == FRQ_DT_I8 ? out : out * ((in + g - 1) / g);
        for (int which = 0; which < (dtype == FRQ_DT_Q4A ? 2 : 1); ++which) {
            const std::string sn = nm + (which ? "__min" : "__scale");
            const ArrSpec* c = need(b, sn, "f16", dtype == FRQ_DT_I8 ? 1 : 2);
            if (!c) return false;
            if (c->bytes != 2 * ns) {
                frq::set_error(FRQ_ERR_FORMAT, sn + ": " + std::to_string(ns) + " f16 values expected");
                return false;
            }
            (which ? mn : sc) = reinterpret_cast<const uint16_t*>(b->blob + c->offset);
        }
        return true;
    };
    for (size_t e = 0; e < n_exp; ++e) {
        const std::string pe = p + "experts." + std::to_string(e) + ".";
        if (silu_) {
            if (!take(pe + "gate", d, mi, gate[e], gs[e], gm[e]) || !take(pe + "up", d, mi, up[e], us[e], um[e]))
                return nullptr;
        } else if (!take(pe + "gate_up", d, 2 * mi, gate[e], gs[e], gm[e])) {
            return nullptr;
        }
        if (!take(pe + "down", mi, d, down[e], ds[e], dm[e])) return nullptr;
    }
    return frq_moe_upload(ctx, dtype, n_exp, d, mi, act, g, gate.data(), gs.data(), gm.data(),
                          silu_ ? up.data() : nullptr, us.data(), um.data(), down.data(), ds.data(), dm.data());
}
int frq_bundle_weight(frq_ctx* ctx, const frq_bundle* b, const char* name, frq_w** out) {
    if (!out) return frq::set_error(FRQ_ERR_ARG, "frq_bundle_weight: null out");
    *out = bundle_weight(ctx, b, name);
    return *out ? FRQ_OK : frq::last_code();
}

int frq_bundle_moe(frq_ctx* ctx, const frq_bundle* b, const char* prefix, size_t n_exp, int act,
                   frq_moe_w** out) {
    if (!out) return frq::set_error(FRQ_ERR_ARG, "frq_bundle_moe: null out");
    *out = bundle_moe(ctx, b, prefix, n_exp, act);
    return *out ? FRQ_OK : frq::last_code();
}

}  // extern "C"
