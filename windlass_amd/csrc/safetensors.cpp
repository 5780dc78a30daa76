// safetensors.cpp — the checkpoint reader of safetensors.h and its C ABI
// (wl_st_open / wl_st_close / wl_st_last_error / wl_st_count / wl_st_name /
// wl_st_info / wl_st_read). Reference: src/safetensors_io.cuh:89-230.
#include "safetensors.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <unordered_set>

#include "../../include/windlass_moe.h"

namespace wl {
namespace json {

const Value* Value::get(const std::string& key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

namespace {

struct Parser {
    const char* p;
    const char* b;
    const char* e;
    std::string* err;

    bool fail(const char* what) {
        char buf[160];
        snprintf(buf, sizeof(buf), "JSON: %s at byte %zu", what, (size_t)(p - b));
        *err = buf;
        return false;
    }
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(e - p) < n || memcmp(p, w, n) != 0) return false;
        p += n;
        return true;
    }
    static void utf8(uint32_t cp, std::string& s) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t* v) {
        if (e - p < 4) return fail("short \\u escape");
        uint32_t x = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            x <<= 4;
            if (c >= '0' && c <= '9') x |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') x |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') x |= (uint32_t)(c - 'A' + 10);
            else return fail("bad hex digit in \\u escape");
        }
        *v = x;
        return true;
    }
    bool string(std::string* s) {
        if (p >= e || *p != '"') return fail("expected a string");
        p++;
        s->clear();
        while (true) {
            if (p >= e) return fail("unterminated string");
            const unsigned char c = (unsigned char)*p++;
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                *s += (char)c;
                continue;
            }
            if (p >= e) return fail("unterminated escape");
            const char x = *p++;
            switch (x) {
                case '"': *s += '"'; break;
                case '\\': *s += '\\'; break;
                case '/': *s += '/'; break;
                case 'b': *s += '\b'; break;
                case 'f': *s += '\f'; break;
                case 'n': *s += '\n'; break;
                case 'r': *s += '\r'; break;
                case 't': *s += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
                        uint32_t lo;
                        if (e - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone high surrogate");
                        p += 2;
                        if (!hex4(&lo)) return false;
                        if (lo < 0xDC00 || lo >= 0xE000) return fail("bad low surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone low surrogate");
                    }
                    utf8(cp, *s);
                    break;
                }
                default: return fail("bad escape");
            }
        }
    }
    bool number(Value* v) {
        const char* s = p;
        bool neg = false, frac = false;
        if (p < e && *p == '-') {
            neg = true;
            p++;
        }
        if (p >= e || *p < '0' || *p > '9') return fail("bad number");
        if (*p == '0') {
            p++;
        } else {
            while (p < e && *p >= '0' && *p <= '9') p++;
        }
        if (p < e && *p == '.') {
            frac = true;
            p++;
            if (p >= e || *p < '0' || *p > '9') return fail("bad fraction");
            while (p < e && *p >= '0' && *p <= '9') p++;
        }
        if (p < e && (*p == 'e' || *p == 'E')) {
            frac = true;
            p++;
            if (p < e && (*p == '+' || *p == '-')) p++;
            if (p >= e || *p < '0' || *p > '9') return fail("bad exponent");
            while (p < e && *p >= '0' && *p <= '9') p++;
        }
        v->kind = Value::Num;
        v->s.assign(s, p - s);
        v->is_uint = false;
        if (!neg && !frac) {
            uint64_t x = 0;
            bool ok = true;
            for (const char* q = s; q < p; q++) {
                const uint64_t d = (uint64_t)(*q - '0');
                if (x > (UINT64_MAX - d) / 10) {
                    ok = false;
                    break;
                }
                x = x * 10 + d;
            }
            v->is_uint = ok;
            v->u = ok ? x : 0;
        }
        return true;
    }
    bool value(Value* v, int depth) {
        if (depth > 64) return fail("nesting deeper than 64");
        ws();
        if (p >= e) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            p++;
            v->kind = Value::Obj;
            ws();
            if (p < e && *p == '}') {
                p++;
                return true;
            }
            std::unordered_set<std::string> seen;  // an index's weight_map has ~10^5 keys
            while (true) {
                ws();
                std::string k;
                if (!string(&k)) return false;
                if (!seen.insert(k).second) return fail("duplicate key");
                ws();
                if (p >= e || *p != ':') return fail("expected ':'");
                p++;
                v->obj.emplace_back(std::move(k), Value());
                if (!value(&v->obj.back().second, depth + 1)) return false;
                ws();
                if (p < e && *p == ',') {
                    p++;
                    continue;
                }
                if (p < e && *p == '}') {
                    p++;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            p++;
            v->kind = Value::Arr;
            ws();
            if (p < e && *p == ']') {
                p++;
                return true;
            }
            while (true) {
                v->arr.emplace_back();
                if (!value(&v->arr.back(), depth + 1)) return false;
                ws();
                if (p < e && *p == ',') {
                    p++;
                    continue;
                }
                if (p < e && *p == ']') {
                    p++;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v->kind = Value::Str;
            return string(&v->s);
        }
        if (lit("true")) {
            v->kind = Value::Bool;
            v->b = true;
            return true;
        }
        if (lit("false")) {
            v->kind = Value::Bool;
            return true;
        }
        if (lit("null")) {
            v->kind = Value::Null;
            return true;
        }
        return number(v);
    }
};

}  // namespace

bool parse(const char* text, size_t n, Value* out, std::string* err) {
    Parser ps{text, text, text + n, err};
    *out = Value();
    if (!ps.value(out, 0)) return false;
    ps.ws();
    if (ps.p != ps.e) return ps.fail("trailing characters");
    return true;
}

}  // namespace json

uint32_t st_dtype_size(const std::string& d) {
    static const std::map<std::string, uint32_t> sizes = {
        {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"F8_E8M0", 1}, {"I16", 2},
        {"U16", 2},  {"F16", 2}, {"BF16", 2}, {"I32", 4},    {"U32", 4},     {"F32", 4},     {"I64", 8},
        {"U64", 8},  {"F64", 8}};
    auto it = sizes.find(d);
    return it == sizes.end() ? 0u : it->second;
}

}  // namespace wl

namespace {

constexpr uint64_t kMaxHeader = 100ull << 20;  // the format's own bound on a header (100 MB)
constexpr uint32_t kMaxDims = 8;

std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    return buf;
}

wl_status pread_all(int fd, void* dst, uint64_t n, uint64_t off, std::string* err, const std::string& what) {
    uint8_t* d = (uint8_t*)dst;
    uint64_t got = 0;
    while (got < n) {
        uint64_t want = n - got;
        if (want > (1ull << 30)) want = 1ull << 30;
        const ssize_t r = ::pread(fd, d + got, (size_t)want, (off_t)(off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            *err = fmt("read of %s: %s after %llu of %llu bytes", what.c_str(), r < 0 ? strerror(errno) : "end of file",
                       (unsigned long long)got, (unsigned long long)n);
            return WL_ERR_IO;
        }
        got += (uint64_t)r;
    }
    return WL_OK;
}

wl_status read_text(const std::string& path, std::string* out, std::string* err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        *err = fmt("cannot open %s: %s", path.c_str(), strerror(errno));
        return WL_ERR_IO;
    }
    struct stat s;
    wl_status st = WL_OK;
    if (fstat(fd, &s) != 0) {
        *err = fmt("stat %s: %s", path.c_str(), strerror(errno));
        st = WL_ERR_IO;
    } else if ((uint64_t)s.st_size > kMaxHeader) {
        *err = fmt("%s is %lld bytes, larger than an index can be", path.c_str(), (long long)s.st_size);
        st = WL_ERR_FORMAT;
    } else {
        out->resize((size_t)s.st_size);
        st = pread_all(fd, &(*out)[0], (uint64_t)s.st_size, 0, err, path);
    }
    ::close(fd);
    return st;
}

// A shard file name from the index: relative, no ".." component.
bool safe_name(const std::string& f) {
    if (f.empty() || f[0] == '/') return false;
    size_t i = 0;
    while (i <= f.size()) {
        const size_t j = f.find('/', i);
        const std::string part = f.substr(i, j == std::string::npos ? std::string::npos : j - i);
        if (part == "..") return false;
        if (j == std::string::npos) break;
        i = j + 1;
    }
    return true;
}

// Reads the header of `sh` (already open) into `out`: every tensor it
// declares, with its byte range checked against the file.
wl_status read_header(wl_st::Shard& sh, uint32_t shard_i, std::unordered_map<std::string, wl_st::Tensor>* out,
                 std::string* err) {
    uint8_t len8[8];
    if (sh.size < 8) {
        *err = fmt("%s: %llu bytes, too short for a safetensors header", sh.path.c_str(), (unsigned long long)sh.size);
        return WL_ERR_FORMAT;
    }
    wl_status rs = pread_all(sh.fd, len8, 8, 0, err, sh.path);
    if (rs != WL_OK) return rs;
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | len8[i];
    if (n > kMaxHeader || 8 + n > sh.size) {
        *err = fmt("%s: header length %llu does not fit the file (%llu bytes)", sh.path.c_str(), (unsigned long long)n,
                   (unsigned long long)sh.size);
        return WL_ERR_FORMAT;
    }
    std::string hdr((size_t)n, '\0');
    if (n && (rs = pread_all(sh.fd, &hdr[0], n, 8, err, sh.path)) != WL_OK) return rs;
    sh.base = 8 + n;
    wl::json::Value root;
    std::string jerr;
    if (!wl::json::parse(hdr.data(), hdr.size(), &root, &jerr)) {
        *err = sh.path + " header: " + jerr;
        return WL_ERR_FORMAT;
    }
    if (root.kind != wl::json::Value::Obj) {
        *err = sh.path + " header: not a JSON object";
        return WL_ERR_FORMAT;
    }
    const uint64_t data = sh.size - sh.base;
    for (const auto& kv : root.obj) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        const wl::json::Value& v = kv.second;
        const wl::json::Value* dt = v.get("dtype");
        const wl::json::Value* shp = v.get("shape");
        const wl::json::Value* off = v.get("data_offsets");
        if (!dt || dt->kind != wl::json::Value::Str || !shp || shp->kind != wl::json::Value::Arr || !off ||
            off->kind != wl::json::Value::Arr || off->arr.size() != 2 || !off->arr[0].is_uint || !off->arr[1].is_uint) {
            *err = fmt("%s: tensor %s lacks a string dtype, a shape array or two integer data_offsets", sh.path.c_str(),
                       name.c_str());
            return WL_ERR_FORMAT;
        }
        wl_st::Tensor t;
        t.shard = shard_i;
        t.dtype = dt->s;
        if (shp->arr.size() > kMaxDims) {
            *err = fmt("%s: tensor %s has %zu dimensions (at most %u)", sh.path.c_str(), name.c_str(), shp->arr.size(),
                       kMaxDims);
            return WL_ERR_FORMAT;
        }
        unsigned __int128 elems = 1;
        for (const auto& d : shp->arr) {
            if (!d.is_uint) {
                *err = fmt("%s: tensor %s has a non-integer dimension", sh.path.c_str(), name.c_str());
                return WL_ERR_FORMAT;
            }
            t.shape.push_back(d.u);
            elems *= d.u;
            if (elems > ((unsigned __int128)1 << 64)) elems = (unsigned __int128)1 << 64;
        }
        const uint64_t beg = off->arr[0].u, end = off->arr[1].u;
        if (end < beg || end > data) {
            *err = fmt("%s: tensor %s data_offsets [%llu, %llu] outside the %llu data bytes", sh.path.c_str(),
                       name.c_str(), (unsigned long long)beg, (unsigned long long)end, (unsigned long long)data);
            return WL_ERR_FORMAT;
        }
        const uint32_t es = wl::st_dtype_size(t.dtype);
        if (es && elems * es != (unsigned __int128)(end - beg)) {
            *err = fmt("%s: tensor %s holds %llu bytes, its %s shape needs %llu", sh.path.c_str(), name.c_str(),
                       (unsigned long long)(end - beg), t.dtype.c_str(), (unsigned long long)(elems * es));
            return WL_ERR_FORMAT;
        }
        t.offset = sh.base + beg;
        t.nbytes = end - beg;
        (*out)[name] = std::move(t);
    }
    return WL_OK;
}

wl_status open_shard(wl_st::Shard& sh, std::string* err) {
    sh.fd = ::open(sh.path.c_str(), O_RDONLY);
    if (sh.fd < 0) {
        *err = fmt("cannot open shard %s: %s", sh.path.c_str(), strerror(errno));
        return WL_ERR_IO;
    }
    struct stat s;
    if (fstat(sh.fd, &s) != 0) {
        *err = fmt("stat %s: %s", sh.path.c_str(), strerror(errno));
        return WL_ERR_IO;
    }
    sh.size = (uint64_t)s.st_size;
    return WL_OK;
}

thread_local std::string t_open_err;

}  // namespace

wl_st::~wl_st() {
    for (Shard& s : shards)
        if (s.fd >= 0) ::close(s.fd);
}

const wl_st::Tensor* wl_st::find(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
}

wl_status wl_st::open(const std::string& path, bool allow_missing) {
    struct stat s;
    if (::stat(path.c_str(), &s) != 0) {
        err = fmt("cannot open %s: %s", path.c_str(), strerror(errno));
        return WL_ERR_IO;
    }
    std::string single;
    if (S_ISREG(s.st_mode)) {
        single = path;
        root = path.substr(0, path.rfind('/') == std::string::npos ? 0 : path.rfind('/'));
    } else {
        root = path;
        const std::string idx = path + "/model.safetensors.index.json";
        if (::access(idx.c_str(), F_OK) == 0) {
            std::string text;
            wl_status rs = read_text(idx, &text, &err);
            if (rs != WL_OK) return rs;
            wl::json::Value v;
            std::string jerr;
            if (!wl::json::parse(text.data(), text.size(), &v, &jerr)) {
                err = idx + ": " + jerr;
                return WL_ERR_FORMAT;
            }
            const wl::json::Value* wm = v.get("weight_map");
            if (!wm || wm->kind != wl::json::Value::Obj) {
                err = idx + ": no weight_map object";
                return WL_ERR_FORMAT;
            }
            // shard file -> tensor names it holds, shards in first-seen order
            std::vector<std::string> order;
            std::unordered_map<std::string, std::vector<std::string>> of;
            for (const auto& kv : wm->obj) {
                if (kv.second.kind != wl::json::Value::Str || !safe_name(kv.second.s)) {
                    err = fmt("%s: tensor %s maps to no usable shard file name", idx.c_str(), kv.first.c_str());
                    return WL_ERR_FORMAT;
                }
                auto it = of.find(kv.second.s);
                if (it == of.end()) {
                    order.push_back(kv.second.s);
                    it = of.emplace(kv.second.s, std::vector<std::string>()).first;
                }
                it->second.push_back(kv.first);
            }
            for (const std::string& f : order) {
                Shard sh;
                sh.file = f;
                sh.path = root + "/" + f;
                if (::access(sh.path.c_str(), F_OK) != 0 && allow_missing) {
                    shards.push_back(sh);  // absent: its tensors are never entered
                    continue;
                }
                const uint32_t si = (uint32_t)shards.size();
                shards.push_back(sh);
                Shard& cur = shards.back();
                if ((rs = open_shard(cur, &err)) != WL_OK) return rs;
                std::unordered_map<std::string, Tensor> hdr;
                if ((rs = read_header(cur, si, &hdr, &err)) != WL_OK) return rs;
                for (const std::string& n : of[f]) {
                    auto it = hdr.find(n);
                    if (it == hdr.end()) {
                        err = fmt("tensor %s is missing from %s", n.c_str(), f.c_str());
                        return WL_ERR_FORMAT;
                    }
                    tensors[n] = std::move(it->second);
                }
            }
        } else {
            single = path + "/model.safetensors";
            if (::access(single.c_str(), F_OK) != 0) {
                err = fmt("%s has neither model.safetensors.index.json nor model.safetensors", path.c_str());
                return WL_ERR_IO;
            }
        }
    }
    if (!single.empty()) {
        Shard sh;
        sh.file = single.substr(single.rfind('/') == std::string::npos ? 0 : single.rfind('/') + 1);
        sh.path = single;
        shards.push_back(sh);
        wl_status rs = open_shard(shards.back(), &err);
        if (rs == WL_OK) rs = read_header(shards.back(), 0, &tensors, &err);
        if (rs != WL_OK) return rs;
    }
    names.reserve(tensors.size());
    for (const auto& kv : tensors) names.push_back(kv.first);
    std::sort(names.begin(), names.end());
    return WL_OK;
}

wl_status wl_st::read(const Tensor& t, uint64_t off, uint64_t n, void* dst, const std::string& name) {
    if (off > t.nbytes || n > t.nbytes - off) {
        err = fmt("range [%llu, +%llu) outside tensor %s (%llu bytes)", (unsigned long long)off, (unsigned long long)n,
                  name.c_str(), (unsigned long long)t.nbytes);
        return WL_ERR_INVALID;
    }
    return pread_all(shards[t.shard].fd, dst, n, t.offset + off, &err, name);
}

extern "C" {

wl_status wl_st_open(const char* path, int32_t allow_missing_shards, wl_st** out) {
    if (!out) return WL_ERR_INVALID;
    *out = nullptr;
    if (!path) {
        t_open_err = "path is null";
        return WL_ERR_INVALID;
    }
    wl_st* st = new (std::nothrow) wl_st();
    if (!st) {
        t_open_err = "out of host memory";
        return WL_ERR_OOM;
    }
    const wl_status rs = st->open(path, allow_missing_shards != 0);
    if (rs != WL_OK) {
        t_open_err = st->err;
        delete st;
        return rs;
    }
    *out = st;
    return WL_OK;
}

void wl_st_close(wl_st* st) { delete st; }

const char* wl_st_last_error(const wl_st* st) { return st ? st->err.c_str() : t_open_err.c_str(); }

uint32_t wl_st_count(const wl_st* st) { return st ? (uint32_t)st->names.size() : 0u; }

const char* wl_st_name(const wl_st* st, uint32_t i) {
    return (st && i < st->names.size()) ? st->names[i].c_str() : nullptr;
}

wl_status wl_st_info(const wl_st* st, const char* name, wl_st_tensor* out) {
    if (!st || !name || !out) return WL_ERR_INVALID;
    const wl_st::Tensor* t = st->find(name);
    if (!t) return WL_ERR_NOT_FOUND;
    memset(out, 0, sizeof(*out));
    snprintf(out->dtype, sizeof(out->dtype), "%s", t->dtype.c_str());
    out->ndim = (uint32_t)t->shape.size();
    for (uint32_t i = 0; i < out->ndim; i++) out->shape[i] = t->shape[i];
    out->nbytes = t->nbytes;
    out->file_offset = t->offset;
    out->shard = t->shard;
    return WL_OK;
}

wl_status wl_st_read(wl_st* st, const char* name, void* h_dst, size_t capacity) {
    if (!st) return WL_ERR_INVALID;
    if (!name || !h_dst) {
        st->err = "name and destination are required";
        return WL_ERR_INVALID;
    }
    const wl_st::Tensor* t = st->find(name);
    if (!t) {
        st->err = fmt("tensor %s is not in the checkpoint", name);
        return WL_ERR_NOT_FOUND;
    }
    if (capacity < t->nbytes) {
        st->err = fmt("tensor %s has %llu bytes, the destination holds %zu", name, (unsigned long long)t->nbytes,
                      capacity);
        return WL_ERR_INVALID;
    }
    return st->read(*t, 0, t->nbytes, h_dst, name);
}

}  // extern "C"
