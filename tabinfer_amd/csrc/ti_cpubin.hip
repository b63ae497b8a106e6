// ti_cpubin.hip — reader of the `.cpu.bin` weight container of the native ternary engine
// (spec native/docs/FORMAT.md; the reference reader is native/crates/n2-core/src/binfmt.rs:
// 104-257, the packer native/tools/pack_bin.py). Host code only: it parses and validates
// the container into host memory; ti_bonsai_load uploads its tensors to the GPU.
//
//   offset 0      u32 le header_len
//   offset 4      header_len bytes of UTF-8 JSON: {"G": 64, "tensors": {name: {...}}}
//   4+header_len  the blob; every offset in the header is blob-relative
//
// Tensor kinds: "tern" (N, K, codesOff, codesLen, scalesOff, scalesLen: Q2_0_g64 codes
// and f32 scales), "embed_f16" (shape, off, len: f16 bit patterns), "f32" (shape, off,
// len). The rules the reference enforces are enforced here, each with the same failure:
// a header that overruns the file, a header that is not UTF-8 / JSON, G != 64, a missing
// `tensors` object or `kind`, an unknown kind, K % G != 0, codesLen != N*K/4, scalesLen !=
// N*(K/G)*4, and any byte range that overruns the blob; f32 ranges must be whole f32s at
// 4-byte-aligned offsets. The blob is held in its own 16-byte-aligned allocation, so an
// odd header length does not misalign it (binfmt.rs:55-78).
#include "ti_host.h"
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) --------------------
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0.0;
    bool integral = false;       // the number was written without fraction or exponent
    unsigned long long u = 0;    // its value when integral and non-negative
    bool neg = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;   // in file order
    const JVal* get(const char* k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* end;
    std::string err;
    int depth = 0;

    const char* begin;

    bool fail(const char* what) {
        if (err.empty()) {
            char b[128];
            snprintf(b, sizeof b, "%s at byte %ld", what, (long)(p - begin));
            err = b;
        }
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* s) {
        size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    static void put_utf8(std::string& o, unsigned cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
        else { o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
    }
    bool hex4(unsigned* v) {
        if (end - p < 4) return fail("truncated \\u escape");
        *v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (unsigned)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& o) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        while (p < end && *p != '"') {
            unsigned char c = (unsigned char)*p++;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') { o += (char)c; continue; }
            if (p >= end) return fail("truncated escape");
            char e = *p++;
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {       // surrogate pair
                        unsigned lo;
                        if (!lit("\\u") || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool number(JVal& v) {
        const char* s = p;
        if (p < end && *p == '-') p++;
        if (p >= end || *p < '0' || *p > '9') return fail("bad number");
        while (p < end && *p >= '0' && *p <= '9') p++;
        bool integral = true;
        if (p < end && *p == '.') { integral = false; p++; while (p < end && *p >= '0' && *p <= '9') p++; }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            p++;
            if (p < end && (*p == '+' || *p == '-')) p++;
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        std::string t(s, p);
        v.kind = JVal::NUM;
        v.num = strtod(t.c_str(), nullptr);
        v.neg = t[0] == '-';
        v.integral = integral;
        if (integral && !v.neg) {
            errno = 0;
            v.u = strtoull(t.c_str(), nullptr, 10);
            if (errno == ERANGE) v.integral = false;
        }
        return true;
    }
    bool value(JVal& v) {
        if (++depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end of the header");
        bool ok = true;
        if (*p == '{') {
            p++;
            v.kind = JVal::OBJ;
            ws();
            if (p < end && *p == '}') p++;
            else
                for (;;) {
                    ws();
                    std::string k;
                    if (!string(k)) { ok = false; break; }
                    ws();
                    if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
                    p++;
                    v.obj.emplace_back(k, JVal());
                    if (!value(v.obj.back().second)) { ok = false; break; }
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == '}') { p++; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
        } else if (*p == '[') {
            p++;
            v.kind = JVal::ARR;
            ws();
            if (p < end && *p == ']') p++;
            else
                for (;;) {
                    v.arr.emplace_back();
                    if (!value(v.arr.back())) { ok = false; break; }
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == ']') { p++; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
        } else if (*p == '"') {
            v.kind = JVal::STR;
            ok = string(v.str);
        } else if (lit("true")) { v.kind = JVal::BOOL; v.num = 1; }
        else if (lit("false")) { v.kind = JVal::BOOL; }
        else if (lit("null")) { v.kind = JVal::NUL; }
        else ok = number(v);
        depth--;
        return ok;
    }
};

bool valid_utf8(const unsigned char* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        unsigned c = s[i];
        int extra = c < 0x80 ? 0 : (c >> 5) == 6 ? 1 : (c >> 4) == 14 ? 2 : (c >> 3) == 30 ? 3 : -1;
        if (extra < 0 || i + extra >= n) return false;
        for (int k = 1; k <= extra; k++)
            if ((s[i + k] & 0xC0) != 0x80) return false;
        i += extra + 1;
    }
    return true;
}

}  // namespace

struct ti_cpubin {
    int G = 64;
    struct Tensor {
        std::string name;
        int kind;                 // TI_CPUBIN_TERN / _EMBED_F16 / _F32
        long long N = 0, K = 0, codes_off = 0, codes_len = 0, scales_off = 0, scales_len = 0;
        std::vector<long long> shape;
        long long off = 0, len = 0;
    };
    std::vector<Tensor> tensors;   // sorted by name (the reference keeps a BTreeMap)
    std::unique_ptr<uint8_t[], void (*)(void*)> blob{nullptr, free};
    size_t blob_len = 0;

    const Tensor* find(const char* name) const {
        for (auto& t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

// IEEE binary16 bits -> its value (exact in f32): sign * m * 2^(e - 25) with the implicit
// bit for normals, m * 2^-24 for subnormals, infinities and NaNs kept.
static float f16_value(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    const float sign = (h & 0x8000) ? -1.0f : 1.0f;
    if (e == 31) return m ? __builtin_nanf("") : sign * __builtin_inff();
    return sign * (e ? ldexpf((float)(1024 + m), e - 25) : ldexpf((float)m, -24));
}

static const char* kind_name(int k) {
    return k == TI_CPUBIN_TERN ? "tern" : k == TI_CPUBIN_EMBED_F16 ? "embed_f16" : "f32";
}

// usize_field / usize_array of the reference (binfmt.rs via json.rs): a non-negative integer
static int usize_field(const JVal& t, const char* name, const char* key, long long* out) {
    const JVal* v = t.get(key);
    if (!v) return ti_fail(TI_ERR_INVALID, "%s: missing `%s`", name, key);
    if (v->kind != JVal::NUM || !v->integral || v->neg || v->u > (1ull << 62))
        return ti_fail(TI_ERR_INVALID, "%s: `%s` is not a non-negative integer", name, key);
    *out = (long long)v->u;
    return TI_OK;
}

// Parse and validate a whole container held in memory (Container::from_bytes / assemble /
// validate, binfmt.rs:136-257); the blob is copied into an aligned allocation.
static int cpubin_assemble(const uint8_t* hdr, size_t hdr_len, ti_cpubin* c) {
    if (!valid_utf8(hdr, hdr_len)) return ti_fail(TI_ERR_INVALID, "header is not valid UTF-8");
    JParser jp{reinterpret_cast<const char*>(hdr), reinterpret_cast<const char*>(hdr) + hdr_len, {}, 0,
               reinterpret_cast<const char*>(hdr)};
    JVal root;
    if (!jp.value(root)) return ti_fail(TI_ERR_INVALID, "header JSON: %s", jp.err.c_str());
    jp.ws();
    if (jp.p != jp.end) return ti_fail(TI_ERR_INVALID, "header JSON: trailing characters");
    if (root.kind != JVal::OBJ) return ti_fail(TI_ERR_INVALID, "header JSON: not an object");
    long long G = 64;
    if (root.get("G")) {
        int rc = usize_field(root, "header", "G", &G);
        if (rc) return rc;
    }
    if (G != 64) return ti_fail(TI_ERR_INVALID, "container group size G=%lld but the kernels are built for G=64", G);
    c->G = (int)G;
    const JVal* tens = root.get("tensors");
    if (!tens || tens->kind != JVal::OBJ) return ti_fail(TI_ERR_INVALID, "header has no `tensors` object");
    std::map<std::string, ti_cpubin::Tensor> byname;
    for (auto& kv : tens->obj) {
        const char* name = kv.first.c_str();
        const JVal& t = kv.second;
        const JVal* kind = t.kind == JVal::OBJ ? t.get("kind") : nullptr;
        if (!kind || kind->kind != JVal::STR) return ti_fail(TI_ERR_INVALID, "%s: missing `kind`", name);
        ti_cpubin::Tensor x;
        x.name = kv.first;
        int rc = 0;
        if (kind->str == "tern") {
            x.kind = TI_CPUBIN_TERN;
            if ((rc = usize_field(t, name, "N", &x.N)) || (rc = usize_field(t, name, "K", &x.K))) return rc;
            if (x.K % G != 0) return ti_fail(TI_ERR_INVALID, "%s: K=%lld is not a multiple of G=%lld", name, x.K, G);
            if ((rc = usize_field(t, name, "codesLen", &x.codes_len)) || (rc = usize_field(t, name, "scalesLen", &x.scales_len)))
                return rc;
            // the declared byte counts against the shape: a packer/reader disagreement
            // fails here, at load, instead of as plausible garbage at inference (the products
            // in checked arithmetic: N and K may each be up to 2^62)
            long long nk = 0, ng4 = 0;
            if (__builtin_mul_overflow(x.N, x.K, &nk) || __builtin_mul_overflow(x.N, (x.K / G) * 4, &ng4))
                return ti_fail(TI_ERR_INVALID, "%s: N=%lld x K=%lld overflows the byte counts", name, x.N, x.K);
            if (x.codes_len != nk / 4)
                return ti_fail(TI_ERR_INVALID, "%s: codesLen=%lld but N*K/4=%lld", name, x.codes_len, nk / 4);
            if (x.scales_len != ng4)
                return ti_fail(TI_ERR_INVALID, "%s: scalesLen=%lld but N*(K/G)*4=%lld", name, x.scales_len, ng4);
            if ((rc = usize_field(t, name, "codesOff", &x.codes_off)) || (rc = usize_field(t, name, "scalesOff", &x.scales_off)))
                return rc;
        } else if (kind->str == "embed_f16" || kind->str == "f32") {
            x.kind = kind->str == "f32" ? TI_CPUBIN_F32 : TI_CPUBIN_EMBED_F16;
            const JVal* sh = t.get("shape");
            if (!sh) return ti_fail(TI_ERR_INVALID, "%s: missing `shape`", name);
            if (sh->kind != JVal::ARR) return ti_fail(TI_ERR_INVALID, "%s: `shape` is not an array", name);
            for (auto& d : sh->arr) {
                if (d.kind != JVal::NUM || !d.integral || d.neg || d.u > (1ull << 40))
                    return ti_fail(TI_ERR_INVALID, "%s: `shape` holds a value that is not a non-negative integer", name);
                x.shape.push_back((long long)d.u);
            }
            if ((rc = usize_field(t, name, "off", &x.off)) || (rc = usize_field(t, name, "len", &x.len))) return rc;
        } else {
            return ti_fail(TI_ERR_INVALID, "%s: unknown kind `%s`", name, kind->str.c_str());
        }
        byname[x.name] = x;
    }
    for (auto& kv : byname) c->tensors.push_back(kv.second);
    // every declared byte range lies inside the blob (binfmt.rs:229-250)
    const long long blob = (long long)c->blob_len;
    auto inside = [&](const ti_cpubin::Tensor& t, long long off, long long len) -> int {
        // off and len are each in [0, 2^62]: compare without forming a sum that could wrap
        if (off > blob || len > blob - off)
            return ti_fail(TI_ERR_INVALID, "%s: range at %lld of %lld bytes overruns the %lld-byte blob", t.name.c_str(), off,
                           len, blob);
        return TI_OK;
    };
    for (auto& t : c->tensors) {
        int rc;
        if (t.kind == TI_CPUBIN_TERN) {
            if ((rc = inside(t, t.codes_off, t.codes_len)) || (rc = inside(t, t.scales_off, t.scales_len))) return rc;
        } else if ((rc = inside(t, t.off, t.len))) {
            return rc;
        }
    }
    return TI_OK;
}

extern "C" int ti_cpubin_parse(const void* data, size_t bytes, ti_cpubin** out) {
    TI_REQUIRE(out && (data || !bytes), "ti_cpubin_parse: null argument");
    *out = nullptr;
    const uint8_t* d = static_cast<const uint8_t*>(data);
    if (bytes < 4) return ti_fail(TI_ERR_INVALID, "file is too short to contain a header length");
    const size_t hl = (size_t)d[0] | ((size_t)d[1] << 8) | ((size_t)d[2] << 16) | ((size_t)d[3] << 24);
    if (4 + hl > bytes) return ti_fail(TI_ERR_INVALID, "header length %zu overruns the file (%zu bytes)", hl, bytes);
    std::unique_ptr<ti_cpubin> c(new ti_cpubin());
    c->blob_len = bytes - 4 - hl;
    c->blob.reset(static_cast<uint8_t*>(aligned_alloc(16, (c->blob_len + 15) / 16 * 16 + 16)));
    if (!c->blob) return ti_fail(TI_ERR_OOM, "ti_cpubin_parse: host allocation of %zu bytes failed", c->blob_len);
    memcpy(c->blob.get(), d + 4 + hl, c->blob_len);
    int rc = cpubin_assemble(d + 4, hl, c.get());
    if (rc) return rc;
    *out = c.release();
    return TI_OK;
}

extern "C" int ti_cpubin_open(const char* path, ti_cpubin** out) {
    TI_REQUIRE(path && out, "ti_cpubin_open: null argument");
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) return ti_fail(TI_ERR_INVALID, "%s: cannot open", path);
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
    if (fseeko(f, 0, SEEK_END) != 0) return ti_fail(TI_ERR_INVALID, "%s: cannot seek", path);
    const long long total = (long long)ftello(f);
    rewind(f);
    uint8_t lb[4];
    if (total < 4 || fread(lb, 1, 4, f) != 4) return ti_fail(TI_ERR_INVALID, "file is too short to contain a header length");
    const size_t hl = (size_t)lb[0] | ((size_t)lb[1] << 8) | ((size_t)lb[2] << 16) | ((size_t)lb[3] << 24);
    if (4 + (long long)hl > total) return ti_fail(TI_ERR_INVALID, "header length %zu overruns the file (%lld bytes)", hl, total);
    std::vector<uint8_t> hdr(hl);
    if (hl && fread(hdr.data(), 1, hl, f) != hl) return ti_fail(TI_ERR_INVALID, "%s: short read", path);
    std::unique_ptr<ti_cpubin> c(new ti_cpubin());
    c->blob_len = (size_t)(total - 4 - (long long)hl);
    // the blob streams straight into its own aligned allocation (no whole-file copy)
    c->blob.reset(static_cast<uint8_t*>(aligned_alloc(16, (c->blob_len + 15) / 16 * 16 + 16)));
    if (!c->blob) return ti_fail(TI_ERR_OOM, "ti_cpubin_open: host allocation of %zu bytes failed", c->blob_len);
    if (c->blob_len && fread(c->blob.get(), 1, c->blob_len, f) != c->blob_len) return ti_fail(TI_ERR_INVALID, "%s: short read", path);
    int rc = cpubin_assemble(hdr.data(), hl, c.get());
    if (rc) return rc;
    *out = c.release();
    return TI_OK;
}

extern "C" int ti_cpubin_close(ti_cpubin* c) {
    delete c;
    return TI_OK;
}

extern "C" int ti_cpubin_summary(const ti_cpubin* c, int* group_size, int* n_tensors, size_t* blob_bytes) {
    TI_REQUIRE(c, "ti_cpubin_summary: null container");
    if (group_size) *group_size = c->G;
    if (n_tensors) *n_tensors = (int)c->tensors.size();
    if (blob_bytes) *blob_bytes = c->blob_len;
    return TI_OK;
}

extern "C" int ti_cpubin_name(const ti_cpubin* c, int i, const char** name) {
    TI_REQUIRE(c && name && i >= 0 && i < (int)c->tensors.size(), "ti_cpubin_name: bad index");
    *name = c->tensors[i].name.c_str();
    return TI_OK;
}

extern "C" int ti_cpubin_tensor(const ti_cpubin* c, const char* name, ti_cpubin_tensor_info* info) {
    TI_REQUIRE(c && name && info, "ti_cpubin_tensor: null argument");
    const ti_cpubin::Tensor* t = c->find(name);
    if (!t) return ti_fail(TI_ERR_INVALID, "%s: not in container", name);
    memset(info, 0, sizeof *info);
    info->kind = t->kind;
    const uint8_t* b = c->blob.get();
    if (t->kind == TI_CPUBIN_TERN) {
        info->N = t->N;
        info->K = t->K;
        info->data = b + t->codes_off;
        info->data_bytes = (size_t)t->codes_len;
        info->scales = b + t->scales_off;
        info->scale_bytes = (size_t)t->scales_len;
        if (t->scales_off % 4) return ti_fail(TI_ERR_INVALID, "f32 range is not 4-byte aligned: a header offset is misaligned");
    } else {
        info->ndim = (int)t->shape.size() < 4 ? (int)t->shape.size() : 4;
        for (int i = 0; i < info->ndim; i++) info->shape[i] = t->shape[i];
        info->data = b + t->off;
        info->data_bytes = (size_t)t->len;
        if (t->kind == TI_CPUBIN_F32) {
            if (t->len % 4) return ti_fail(TI_ERR_INVALID, "%lld bytes is not a whole number of f32", t->len);
            if (t->off % 4) return ti_fail(TI_ERR_INVALID, "f32 range is not 4-byte aligned: a header offset is misaligned");
        }
    }
    return TI_OK;
}

// embed_row (binfmt.rs:321-342): row `row` of an embed_f16 tensor as f32 (exact).
extern "C" int ti_cpubin_embed_row(const ti_cpubin* c, const char* name, long long row, float* dst, int dim) {
    TI_REQUIRE(c && name && dst, "ti_cpubin_embed_row: null argument");
    const ti_cpubin::Tensor* t = c->find(name);
    if (!t) return ti_fail(TI_ERR_INVALID, "%s: not in container", name);
    if (t->kind != TI_CPUBIN_EMBED_F16) return ti_fail(TI_ERR_INVALID, "%s: expected `embed_f16`, found `%s`", name, kind_name(t->kind));
    if (t->shape.empty()) return ti_fail(TI_ERR_INVALID, "embedding has no shape");
    const long long d = t->shape.back();
    if (dim != d) return ti_fail(TI_ERR_INVALID, "dst is %d long, embedding dim is %lld", dim, d);
    // row < len / (2 d) without forming a product that could overflow (row is the caller's)
    if (d <= 0 || row < 0 || (unsigned long long)row >= (unsigned long long)t->len / (2ull * (unsigned long long)d))
        return ti_fail(TI_ERR_INVALID, "row %lld is out of range for %s", row, name);
    const uint8_t* s = c->blob.get() + t->off + row * d * 2;
    for (long long i = 0; i < d; i++) dst[i] = f16_value((uint16_t)(s[2 * i] | (s[2 * i + 1] << 8)));
    return TI_OK;
}
