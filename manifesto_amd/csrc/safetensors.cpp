// safetensors.cpp — SafeTensors index and reads (weights/reader.go:14-109)
// and the streaming loader that feeds tensors from the file through the
// backend's pinned staging ring onto the device.
//
// The header is parsed by a small JSON reader written for this format (an
// object of objects of strings, integer arrays and a string map); it accepts
// any JSON value where the format allows one and ignores what it does not
// use, like the reference's encoding/json decoding into TensorMeta.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/mfh_safetensors.h"
#include "backend_internal.hpp"
#include "common.hpp"

namespace mfh {
namespace {

// ---- a JSON value reader ------------------------------------------------------

struct Json {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    std::string text;  // string value, or the number's literal
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;
};

struct Parser {
    const char* p;
    const char* end;
    std::string error;
    int depth = 0;

    bool fail_at(const char* what)
    {
        if (error.empty()) error = what;
        return false;
    }
    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* word)
    {
        size_t n = std::strlen(word);
        if ((size_t)(end - p) < n || std::memcmp(p, word, n) != 0) return false;
        p += n;
        return true;
    }
    static void utf8(std::string& out, unsigned cp)
    {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) out += (char)(0xc0 | (cp >> 6)), out += (char)(0x80 | (cp & 0x3f));
        else if (cp < 0x10000)
            out += (char)(0xe0 | (cp >> 12)), out += (char)(0x80 | ((cp >> 6) & 0x3f)), out += (char)(0x80 | (cp & 0x3f));
        else
            out += (char)(0xf0 | (cp >> 18)), out += (char)(0x80 | ((cp >> 12) & 0x3f)),
                out += (char)(0x80 | ((cp >> 6) & 0x3f)), out += (char)(0x80 | (cp & 0x3f));
    }
    bool hex4(unsigned* v)
    {
        if (end - p < 4) return fail_at("truncated \\u escape");
        *v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (unsigned)(c - 'A' + 10);
            else return fail_at("bad \\u escape");
        }
        return true;
    }
    // One UTF-8 sequence at p as Go's utf8.DecodeRune reads it: a malformed
    // or overlong sequence, a surrogate or a value past U+10FFFF is U+FFFD
    // and takes one byte.
    unsigned rune()
    {
        const unsigned char* u = reinterpret_cast<const unsigned char*>(p);
        const size_t left = (size_t)(end - p);
        const unsigned b0 = u[0];
        auto cont = [&](size_t i, unsigned lo, unsigned hi) { return i < left && u[i] >= lo && u[i] <= hi; };
        if (b0 < 0x80) {
            p += 1;
            return b0;
        }
        if (b0 >= 0xc2 && b0 <= 0xdf && cont(1, 0x80, 0xbf)) {
            p += 2;
            return ((b0 & 0x1f) << 6) | (u[1] & 0x3f);
        }
        if (b0 >= 0xe0 && b0 <= 0xef) {
            const unsigned lo = b0 == 0xe0 ? 0xa0 : 0x80, hi = b0 == 0xed ? 0x9f : 0xbf;
            if (cont(1, lo, hi) && cont(2, 0x80, 0xbf)) {
                p += 3;
                return ((b0 & 0x0f) << 12) | ((u[1] & 0x3f) << 6) | (u[2] & 0x3f);
            }
        }
        if (b0 >= 0xf0 && b0 <= 0xf4) {
            const unsigned lo = b0 == 0xf0 ? 0x90 : 0x80, hi = b0 == 0xf4 ? 0x8f : 0xbf;
            if (cont(1, lo, hi) && cont(2, 0x80, 0xbf) && cont(3, 0x80, 0xbf)) {
                p += 4;
                return ((b0 & 0x07) << 18) | ((u[1] & 0x3f) << 12) | ((u[2] & 0x3f) << 6) | (u[3] & 0x3f);
            }
        }
        p += 1;
        return 0xfffd;
    }
    // A string as encoding/json unquotes it: invalid UTF-8 and unpaired
    // surrogate escapes become U+FFFD rather than errors.
    bool string(std::string& out)
    {
        if (p >= end || *p != '"') return fail_at("expected a string");
        p++;
        while (p < end && *p != '"') {
            unsigned char c = (unsigned char)*p;
            if (c < 0x20) return fail_at("control character in a string");
            if (c >= 0x80) {
                utf8(out, rune());
                continue;
            }
            p++;
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p >= end) return fail_at("truncated escape");
            char e = *p++;
            switch (e) {
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
                if (!hex4(&cp)) return false;
                if (cp >= 0xd800 && cp < 0xe000) {
                    // a high surrogate and a low one escaped right after it
                    // make one code point; any other surrogate is U+FFFD and
                    // the escape after it is read on its own
                    const char* save = p;
                    unsigned lo = 0;
                    if (cp < 0xdc00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        std::string err;
                        std::swap(err, error);
                        if (!hex4(&lo)) lo = 0;
                        std::swap(err, error);
                    }
                    if (lo >= 0xdc00 && lo < 0xe000) cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    else {
                        p = save;
                        cp = 0xfffd;
                    }
                }
                utf8(out, cp);
                break;
            }
            default: return fail_at("bad escape");
            }
        }
        if (p >= end) return fail_at("unterminated string");
        p++;
        return true;
    }
    // -?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?, as JSON (and Go's
    // scanner) has it
    bool number(Json& v)
    {
        const char* s = p;
        auto digits = [&] {
            const char* d = p;
            while (p < end && *p >= '0' && *p <= '9') p++;
            return p > d;
        };
        if (p < end && *p == '-') p++;
        if (p < end && *p == '0') p++;
        else if (!(p < end && *p >= '1' && *p <= '9') || !digits()) return fail_at("bad number");
        if (p < end && *p == '.') {
            p++;
            if (!digits()) return fail_at("bad number");
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            p++;
            if (p < end && (*p == '+' || *p == '-')) p++;
            if (!digits()) return fail_at("bad number");
        }
        v.kind = Json::kNumber;
        v.text.assign(s, p);
        return true;
    }
    bool value(Json& v)
    {
        if (++depth > 64) return fail_at("nesting too deep");
        ws();
        if (p >= end) return fail_at("unexpected end of header");
        bool ok;
        if (*p == '{') {
            v.kind = Json::kObject;
            p++;
            ws();
            ok = true;
            if (p < end && *p == '}') p++;
            else
                for (;;) {
                    std::string key;
                    ws();
                    if (!string(key)) return false;
                    ws();
                    if (p >= end || *p++ != ':') return fail_at("expected ':'");
                    Json item;
                    if (!value(item)) return false;
                    v.members.emplace_back(std::move(key), std::move(item));
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        p++;
                        break;
                    }
                    return fail_at("expected ',' or '}'");
                }
        } else if (*p == '[') {
            v.kind = Json::kArray;
            p++;
            ws();
            ok = true;
            if (p < end && *p == ']') p++;
            else
                for (;;) {
                    Json item;
                    if (!value(item)) return false;
                    v.items.push_back(std::move(item));
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        p++;
                        break;
                    }
                    return fail_at("expected ',' or ']'");
                }
        } else if (*p == '"') {
            v.kind = Json::kString;
            ok = string(v.text);
        } else if (lit("true") || lit("false")) {
            v.kind = Json::kBool;
            ok = true;
        } else if (lit("null")) {
            v.kind = Json::kNull;
            ok = true;
        } else {
            ok = number(v);
        }
        depth--;
        return ok;
    }
};

bool to_int64(const Json& v, int64_t* out)
{
    if (v.kind != Json::kNumber || v.text.find_first_of(".eE") != std::string::npos) return false;
    errno = 0;
    char* e = nullptr;
    long long x = std::strtoll(v.text.c_str(), &e, 10);
    if (errno || *e) return false;
    *out = x;
    return true;
}

// dtype.Parse (dtype/dtype.go:242-287).
int parse_dtype(const std::string& name)
{
    std::string n;
    size_t b = 0, e = name.size();
    while (b < e && std::isspace((unsigned char)name[b])) b++;
    while (e > b && std::isspace((unsigned char)name[e - 1])) e--;
    for (size_t i = b; i < e; i++) {
        char c = name[i];
        if (c == '_' || c == '-') continue;
        n += (char)std::toupper((unsigned char)c);
    }
    static const std::map<std::string, int> kNames = {
        {"F64", kFloat64}, {"FLOAT64", kFloat64}, {"DOUBLE", kFloat64},
        {"F32", kFloat32}, {"FLOAT32", kFloat32}, {"FLOAT", kFloat32}, {"SINGLE", kFloat32},
        {"F16", kFloat16}, {"FLOAT16", kFloat16}, {"HALF", kFloat16},
        {"BF16", kBFloat16}, {"BFLOAT16", kBFloat16}, {"BRAINFLOAT16", kBFloat16},
        {"F8E4M3", kF8E4M3}, {"FP8E4M3", kF8E4M3}, {"FLOAT8E4M3", kF8E4M3},
        {"F8E5M2", kF8E5M2}, {"FP8E5M2", kF8E5M2}, {"FLOAT8E5M2", kF8E5M2},
        {"I64", kInt64}, {"INT64", kInt64}, {"LONG", kInt64},
        {"I32", kInt32}, {"INT32", kInt32}, {"INT", kInt32},
        {"I16", kInt16}, {"INT16", kInt16}, {"SHORT", kInt16},
        {"I8", kInt8}, {"INT8", kInt8}, {"BYTE", kInt8},
        {"I4", kInt4}, {"INT4", kInt4},
        {"U64", kUint64}, {"UINT64", kUint64}, {"ULONG", kUint64},
        {"U32", kUint32}, {"UINT32", kUint32}, {"UINT", kUint32},
        {"U16", kUint16}, {"UINT16", kUint16}, {"USHORT", kUint16},
        {"U8", kUint8}, {"UINT8", kUint8}, {"UBYTE", kUint8},
        {"BOOL", kBool}, {"BOOLEAN", kBool}, {"B1", kBool},
        {"C64", kComplex64}, {"COMPLEX64", kComplex64}, {"C128", kComplex128}, {"COMPLEX128", kComplex128},
    };
    auto it = kNames.find(n);
    return it == kNames.end() ? kInvalid : it->second;
}

bool key_is(const std::string& key, const char* field)  // encoding/json matches field names case-insensitively
{
    if (key.size() != std::strlen(field)) return false;
    for (size_t i = 0; i < key.size(); i++)
        if (std::tolower((unsigned char)key[i]) != field[i]) return false;
    return true;
}

struct Entry {
    std::string name;
    std::string dtype_name;
    int dtype = kInvalid;
    std::vector<int64_t> shape;
    int64_t begin = 0, end = 0;
};

int read_full(int fd, void* dst, size_t len, int64_t at)
{
    char* p = static_cast<char*>(dst);
    while (len > 0) {
        ssize_t n = ::pread(fd, p, len, (off_t)at);
        if (n < 0) {
            if (errno == EINTR) continue;
            return -errno;
        }
        if (n == 0) return -1;  // end of file
        p += n;
        len -= (size_t)n;
        at += n;
    }
    return 0;
}

}  // namespace
}  // namespace mfh

struct mfh_safetensors {
    int fd = -1;
    std::string path;
    int64_t data_base = 0;
    int64_t file_size = 0;
    std::vector<mfh::Entry> entries;
    std::map<std::string, size_t> by_name;
};

namespace mfh {
namespace {

int index_file(mfh_safetensors& f)
{
    uint8_t len_bytes[8];
    int rc = read_full(f.fd, len_bytes, 8, 0);
    if (rc) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors index: %s", rc == -1 ? "unexpected EOF" : std::strerror(-rc));
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; i--) header_len = (header_len << 8) | len_bytes[i];
    if (header_len > (uint64_t)f.file_size - 8 || header_len > (1ull << 31))
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors index: unexpected EOF (header of %llu bytes)",
                    (unsigned long long)header_len);
    std::string header(header_len, '\0');
    rc = read_full(f.fd, &header[0], header_len, 8);
    if (rc) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors index: unexpected EOF");
    Parser ps{header.data(), header.data() + header.size(), "", 0};
    Json root;
    bool ok = ps.value(root);
    ps.ws();
    if (ok && ps.p != ps.end) ok = ps.fail_at("trailing data after the header object");
    if (!ok) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors index: %s", ps.error.c_str());
    // a null header unmarshals into an empty map, anything else but an
    // object is a type error
    if (root.kind != Json::kObject && root.kind != Json::kNull)
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors index: header is not an object");
    // Each entry decodes as json.Unmarshal fills TensorMeta
    // (weights/reader.go:13-17,64-68): null anywhere leaves the field as it
    // was, unknown fields are ignored, data_offsets fills [2]int64 (missing
    // elements zero, extra ones skipped), and a value of the wrong type is an
    // error.
    for (auto& kv : root.members) {
        if (kv.first == "__metadata__") continue;
        const Json& meta = kv.second;
        if (meta.kind != Json::kObject && meta.kind != Json::kNull)
            return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors tensor \"%s\": not an object", kv.first.c_str());
        Entry e;
        e.name = kv.first;
        for (auto& field : meta.members) {
            const Json& v = field.second;
            if (v.kind == Json::kNull) {
                if (key_is(field.first, "shape")) e.shape.clear();  // a nil slice
                continue;
            }
            if (key_is(field.first, "dtype")) {
                if (v.kind != Json::kString)
                    return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors tensor \"%s\": dtype is not a string", e.name.c_str());
                e.dtype_name = v.text;
                e.dtype = parse_dtype(v.text);
            } else if (key_is(field.first, "shape")) {
                if (v.kind != Json::kArray)
                    return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors tensor \"%s\": shape is not an array", e.name.c_str());
                e.shape.clear();
                for (const Json& d : v.items) {
                    int64_t x = 0;
                    if (d.kind != Json::kNull && !to_int64(d, &x))
                        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors tensor \"%s\": shape holds a non-integer",
                                    e.name.c_str());
                    e.shape.push_back(x);
                }
            } else if (key_is(field.first, "data_offsets")) {
                int64_t* slot[2] = {&e.begin, &e.end};
                if (v.kind != Json::kArray)
                    return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors tensor \"%s\": data_offsets is not an array",
                                e.name.c_str());
                for (size_t i = 0; i < 2; i++) {
                    if (i >= v.items.size()) *slot[i] = 0;
                    else if (v.items[i].kind != Json::kNull && !to_int64(v.items[i], slot[i]))
                        return fail(MFH_ERR_INVALID_ARGUMENT,
                                    "safetensors tensor \"%s\": data_offsets holds a non-integer", e.name.c_str());
                }
            }
        }
        auto it = f.by_name.find(e.name);
        if (it != f.by_name.end()) f.entries[it->second] = std::move(e);  // a repeated key keeps the last value
        else {
            f.by_name[e.name] = f.entries.size();
            f.entries.push_back(std::move(e));
        }
    }
    f.data_base = (int64_t)header_len + 8;
    return MFH_OK;
}

const Entry* find(const mfh_safetensors* f, const char* name)
{
    if (!f || !name) return nullptr;
    auto it = f->by_name.find(name);
    return it == f->by_name.end() ? nullptr : &f->entries[it->second];
}

// The byte range of an entry inside the file, checked like ReadAt would.
int entry_range(const mfh_safetensors& f, const Entry& e, int64_t* at, size_t* len)
{
    if (e.end < e.begin || e.begin < 0)
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": bad data_offsets [%lld, %lld]", e.name.c_str(),
                    (long long)e.begin, (long long)e.end);
    // compared against the bytes after the header first, so that offsets
    // near INT64_MAX cannot overflow the sums below
    if (e.end > f.file_size - f.data_base)
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": unexpected EOF", e.name.c_str());
    *at = f.data_base + e.begin;
    *len = (size_t)(e.end - e.begin);
    return MFH_OK;
}

struct FileSource : Source {
    int fd;
    int64_t base;
    std::string name;
    int read(void* dst, size_t offset, size_t len) override
    {
        int rc = read_full(fd, dst, len, base + (int64_t)offset);
        if (rc) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": %s", name.c_str(),
                            rc == -1 ? "unexpected EOF" : std::strerror(-rc));
        return MFH_OK;
    }
};

// One-element scale tensor as f32.
int read_scalar(const mfh_safetensors& f, const Entry& e, float* out)
{
    int64_t at;
    size_t len;
    MFH_TRY(entry_range(f, e, &at, &len));
    uint8_t buf[4] = {0, 0, 0, 0};
    const int size = dtype_size(e.dtype);
    if ((e.dtype != kFloat32 && e.dtype != kFloat16 && e.dtype != kBFloat16) || len != (size_t)size)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "safetensors: scale \"%s\" is not one F32/F16/BF16 value", e.name.c_str());
    if (read_full(f.fd, buf, len, at)) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": unexpected EOF", e.name.c_str());
    uint32_t bits;
    if (e.dtype == kFloat32) bits = buf[0] | (buf[1] << 8) | (buf[2] << 16) | ((uint32_t)buf[3] << 24);
    else if (e.dtype == kBFloat16) bits = (uint32_t)(buf[0] | (buf[1] << 8)) << 16;
    else {
        // binary16 -> binary32, exact
        const uint32_t h = buf[0] | (buf[1] << 8), sign = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1f, m = h & 0x3ff;
        if (ex == 0x1f) bits = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u);
        else if (ex) bits = sign | ((ex + 112) << 23) | (m << 13);
        else if (!m) bits = sign;
        else {
            int s = 0;
            uint32_t mm = m;
            while (!(mm & 0x400)) mm <<= 1, s++;
            bits = sign | ((uint32_t)(113 - s) << 23) | ((mm & 0x3ff) << 13);
        }
    }
    std::memcpy(out, &bits, 4);
    return MFH_OK;
}

}  // namespace
}  // namespace mfh

using namespace mfh;

extern "C" {

int mfh_safetensors_open(const char* path, mfh_safetensors** file)
{
    if (!file || !path) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_safetensors_open: path and out-pointer are required");
    *file = nullptr;
    auto f = std::make_unique<mfh_safetensors>();
    f->path = path;
    f->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "open %s: %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(f->fd, &st) != 0) {
        int e = errno;
        ::close(f->fd);
        return fail(MFH_ERR_INVALID_ARGUMENT, "stat %s: %s", path, std::strerror(e));
    }
    f->file_size = (int64_t)st.st_size;
    int rc = index_file(*f);
    if (rc != MFH_OK) {
        ::close(f->fd);
        return rc;
    }
    *file = f.release();
    return MFH_OK;
}

int mfh_safetensors_close(mfh_safetensors* file)
{
    if (!file) return MFH_OK;
    if (file->fd >= 0) ::close(file->fd);
    delete file;
    return MFH_OK;
}

int64_t mfh_safetensors_data_base(const mfh_safetensors* file) { return file ? file->data_base : -1; }
int32_t mfh_safetensors_count(const mfh_safetensors* file) { return file ? (int32_t)file->entries.size() : -1; }

int mfh_safetensors_entry(const mfh_safetensors* file, int32_t index, mfh_safetensors_meta* meta, int64_t* dims,
                          int32_t cap)
{
    if (!file || index < 0 || index >= (int32_t)file->entries.size() || !meta)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_safetensors_entry: no entry %d", (int)index);
    const Entry& e = file->entries[index];
    meta->name = e.name.c_str();
    meta->dtype_name = e.dtype_name.c_str();
    meta->dtype = (uint8_t)e.dtype;
    meta->rank = (int32_t)e.shape.size();
    meta->begin = e.begin;
    meta->end = e.end;
    for (int32_t i = 0; dims && i < cap && i < meta->rank; i++) dims[i] = e.shape[i];
    return MFH_OK;
}

int32_t mfh_safetensors_find(const mfh_safetensors* file, const char* name)
{
    if (!file || !name) return -1;
    auto it = file->by_name.find(name);
    return it == file->by_name.end() ? -1 : (int32_t)it->second;
}

int mfh_safetensors_read(const mfh_safetensors* file, const char* name, void* dst, size_t dst_bytes, size_t* n_bytes)
{
    const Entry* e = find(file, name);
    if (!e) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors: missing tensor \"%s\"", name ? name : "");
    int64_t at;
    size_t len;
    MFH_TRY(entry_range(*file, *e, &at, &len));
    if (n_bytes) *n_bytes = len;
    if (!dst) return MFH_OK;  // size query
    if (dst_bytes < len)
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": destination holds %zu bytes, need %zu", name,
                    dst_bytes, len);
    int rc = read_full(file->fd, dst, len, at);
    if (rc) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors read \"%s\": %s", name,
                        rc == -1 ? "unexpected EOF" : std::strerror(-rc));
    return MFH_OK;
}

}  // extern "C"

namespace {

int load(const mfh_safetensors* file, const char* name, mfh_backend* backend, const char* scale_name, int64_t group,
         bool wait, mfh_tensor** tensor)
{
    if (tensor) *tensor = nullptr;
    const Entry* e = find(file, name);
    if (!e) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors: missing tensor \"%s\"", name ? name : "");
    int64_t at;
    size_t len;
    MFH_TRY(entry_range(*file, *e, &at, &len));
    const bool as_is = e->dtype == kFloat32 || e->dtype == kFloat16 || e->dtype == kBFloat16;
    const bool fp8 = e->dtype == kF8E4M3 || e->dtype == kF8E5M2;
    if (!as_is && !fp8 && e->dtype != kInt4)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "safetensors: tensor \"%s\" has dtype \"%s\", which the backend does not "
                    "load (F32, F16, BF16, F8_E4M3, F8_E5M2, I4)", e->name.c_str(), e->dtype_name.c_str());
    Plan p;
    p.src = e->dtype;
    p.out = as_is ? e->dtype : kBFloat16;
    FileSource src;
    src.fd = file->fd;
    src.base = at;
    src.name = e->name;
    const Entry* se = scale_name ? find(file, scale_name) : nullptr;
    if (scale_name && !se) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors: missing tensor \"%s\"", scale_name);
    if (se && as_is)
        return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\" is %s, which is stored as written; a scale "
                    "(\"%s\") applies only to F8_E4M3, F8_E5M2 and I4 tensors", e->name.c_str(), e->dtype_name.c_str(),
                    se->name.c_str());
    if (se && fp8) MFH_TRY(read_scalar(*file, *se, &p.scale));
    FileSource scales;
    if (se && e->dtype == kInt4) {
        if (group <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "safetensors: group must be positive, got %lld", (long long)group);
        if (se->dtype != kFloat32 && se->dtype != kFloat16 && se->dtype != kBFloat16)
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "safetensors: scales \"%s\" are not F32/F16/BF16", se->name.c_str());
        int64_t elements;
        std::vector<int64_t> dims;
        MFH_TRY(make_shape(e->shape.data(), (int32_t)e->shape.size(), &dims, &elements));
        int64_t s_at;
        size_t s_len;
        MFH_TRY(entry_range(*file, *se, &s_at, &s_len));
        const int64_t groups = elements / group + (elements % group != 0);
        const size_t ssize = (size_t)dtype_size(se->dtype);
        const size_t need = (uint64_t)groups <= SIZE_MAX / ssize ? (size_t)groups * ssize : SIZE_MAX;
        if (s_len != need)
            return fail(MFH_ERR_SHAPE_MISMATCH, "safetensors: scales \"%s\" hold %zu bytes, %lld elements in groups of "
                        "%lld need %zu", se->name.c_str(), s_len, (long long)elements, (long long)group, need);
        // streamed from the file chunk by chunk beside the nibbles they scale
        scales.fd = file->fd;
        scales.base = s_at;
        scales.name = se->name;
        p.scales = &scales;
        p.scale_dt = se->dtype;
        p.group = group;
    }
    return upload_from(backend, e->shape.data(), (int32_t)e->shape.size(), p, src, len, wait, tensor);
}

}  // namespace

extern "C" {

int mfh_safetensors_load(const mfh_safetensors* file, const char* name, mfh_backend* backend, const char* scale_name,
                         int64_t group, mfh_tensor** tensor)
{
    return load(file, name, backend, scale_name, group, true, tensor);
}

int mfh_safetensors_load_async(const mfh_safetensors* file, const char* name, mfh_backend* backend,
                               const char* scale_name, int64_t group, mfh_tensor** tensor)
{
    return load(file, name, backend, scale_name, group, false, tensor);
}

}  // extern "C"
