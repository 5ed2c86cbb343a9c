// w4file.cpp -- reading and checking prepacked-W4 files (w4file.hpp).
//
// The reference stores nothing: its int4 weights live in caller memory as
// [K/2, N] bytes plus fp32 scales (quant.hpp:52-59), and its plan lists
// safetensors loaders for later (PLAN.md:326-333).  This reader treats a file
// as untrusted input: every length, offset and size in the header is checked
// in 64-bit unsigned arithmetic against the file's real size before any
// buffer is sized from it, and allocation failure is a status, not an
// exception.
#include "w4file.hpp"

#include <sys/stat.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <new>

#include "longhorn_hip.h"
#include "w4layout.hpp"

namespace lhq {
namespace {

constexpr const char* kFormat = "lhq-w4-prepacked";
constexpr const char* kVersion = "1";
constexpr const char* kLayout = "w4-tile16x128-v1";
constexpr uint64_t kMaxHeader = 1 << 20;  // bytes of JSON a valid file can need, with room to spare

int fail_with(std::string& err, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    err = buf;
    return code;
}

#define W4_REQUIRE(cond, ...) \
    do {                      \
        if (!(cond)) return fail_with(err, LHQ_ERR_INVALID, __VA_ARGS__); \
    } while (0)
#define W4_SUPPORTED(cond, ...) \
    do {                        \
        if (!(cond)) return fail_with(err, LHQ_ERR_UNSUPPORTED, __VA_ARGS__); \
    } while (0)

// --- a strict JSON subset: objects, arrays, strings, non-negative integers
struct Json {
    enum Kind { OBJ, ARR, STR, INT } kind = INT;
    std::map<std::string, Json> obj;
    std::vector<Json> arr;
    std::string str;
    uint64_t num = 0;
};

struct Parser {
    const char* p;
    const char* end;
    std::string err;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool fail(const char* what) {
        if (err.empty()) err = what;
        return false;
    }
    bool lit(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    bool string(std::string& out) {
        ws();
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            const unsigned char c = static_cast<unsigned char>(*p);
            if (c < 0x20) return fail("control character in a string");
            if (c == '\\') {
                if (++p >= end) return fail("truncated escape");
                switch (*p) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (end - p < 5) return fail("truncated \\u escape");
                        unsigned v = 0;
                        for (int i = 1; i <= 4; ++i) {
                            const char h = p[i];
                            v = v * 16 + static_cast<unsigned>(h >= '0' && h <= '9'   ? h - '0'
                                                               : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                                               : h >= 'A' && h <= 'F' ? h - 'A' + 10
                                                                                      : 99);
                            if ((h < '0' || h > '9') && (h < 'a' || h > 'f') && (h < 'A' || h > 'F'))
                                return fail("bad \\u escape");
                        }
                        if (v >= 0x80) return fail("non-ASCII \\u escape");  // no such field in this format
                        out += static_cast<char>(v);
                        p += 4;
                        break;
                    }
                    default: return fail("bad escape");
                }
                ++p;
            } else {
                out += static_cast<char>(c);
                ++p;
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 8) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("truncated header");
        bool ok;
        if (*p == '{') {
            ++p;
            v.kind = Json::OBJ;
            ok = true;
            if (!lit('}')) {
                do {
                    std::string key;
                    Json item;
                    if (!string(key) || !lit(':') || !value(item)) {
                        ok = false;
                        break;
                    }
                    if (v.obj.count(key)) {
                        ok = fail("duplicate key");
                        break;
                    }
                    v.obj.emplace(std::move(key), std::move(item));
                } while (lit(','));
                if (ok && !lit('}')) ok = fail("expected '}'");
            }
        } else if (*p == '[') {
            ++p;
            v.kind = Json::ARR;
            ok = true;
            if (!lit(']')) {
                do {
                    Json item;
                    if (!value(item)) {
                        ok = false;
                        break;
                    }
                    v.arr.push_back(std::move(item));
                } while (lit(','));
                if (ok && !lit(']')) ok = fail("expected ']'");
            }
        } else if (*p == '"') {
            v.kind = Json::STR;
            ok = string(v.str);
        } else if (*p >= '0' && *p <= '9') {
            v.kind = Json::INT;
            uint64_t n = 0;
            while (p < end && *p >= '0' && *p <= '9') {
                const uint64_t d = static_cast<uint64_t>(*p - '0');
                if (n > (UINT64_MAX - d) / 10) return fail("integer overflow");
                n = n * 10 + d;
                ++p;
            }
            if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return fail("non-integer number");
            v.num = n;
            ok = true;
        } else {
            ok = fail("unexpected character");
        }
        --depth;
        return ok;
    }
};

std::string hex64(uint64_t v) {
    char b[17];
    snprintf(b, sizeof(b), "%016llx", static_cast<unsigned long long>(v));
    return b;
}

bool get_int_field(const std::map<std::string, Json>& meta, const char* key, int& out) {
    auto it = meta.find(key);
    if (it == meta.end() || it->second.kind != Json::STR || it->second.str.empty() || it->second.str.size() > 10)
        return false;
    long long v = 0;
    for (char c : it->second.str) {
        if (c < '0' || c > '9') return false;
        v = v * 10 + (c - '0');
    }
    if (v <= 0 || v > 0x7fffffff) return false;
    out = static_cast<int>(v);
    return true;
}

int read_file(const char* who, const char* path, W4File& f, std::string& err) {
    W4_REQUIRE(path, "%s: null path", who);
    std::unique_ptr<FILE, int (*)(FILE*)> fp(std::fopen(path, "rb"), &std::fclose);
    W4_REQUIRE(fp, "%s: cannot open %s: %s", who, path, std::strerror(errno));
    struct stat st {};
    W4_REQUIRE(fstat(fileno(fp.get()), &st) == 0 && S_ISREG(st.st_mode) && st.st_size >= 0,
               "%s: %s: not a regular file", who, path);
    const uint64_t file_size = static_cast<uint64_t>(st.st_size);
    uint8_t len8[8];
    W4_REQUIRE(std::fread(len8, 1, 8, fp.get()) == 8, "%s: %s: truncated (no header length)", who, path);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | len8[i];
    W4_REQUIRE(hlen >= 2 && hlen <= kMaxHeader && hlen <= file_size - 8, "%s: %s: header length %llu out of range",
               who, path, static_cast<unsigned long long>(hlen));
    std::string header(hlen, '\0');
    W4_REQUIRE(std::fread(&header[0], 1, hlen, fp.get()) == hlen, "%s: %s: truncated header", who, path);
    Parser ps{header.data(), header.data() + header.size(), {}};
    Json root;
    const bool parsed = ps.value(root);
    ps.ws();
    W4_REQUIRE(parsed && ps.p == ps.end && root.kind == Json::OBJ, "%s: %s: malformed header (%s)", who, path,
               ps.err.empty() ? "trailing bytes" : ps.err.c_str());
    auto mit = root.obj.find("__metadata__");
    W4_REQUIRE(mit != root.obj.end() && mit->second.kind == Json::OBJ, "%s: %s: no __metadata__", who, path);
    const auto& meta = mit->second.obj;
    for (const auto& kv : meta)
        W4_REQUIRE(kv.second.kind == Json::STR, "%s: %s: metadata value of %s is not a string", who, path,
                   kv.first.c_str());
    auto str = [&](const char* k) -> const std::string* {
        auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second.str;
    };
    W4_REQUIRE(str("format") && *str("format") == kFormat, "%s: %s: not a prepacked W4 file (format)", who, path);
    W4_SUPPORTED(str("version") && *str("version") == kVersion, "%s: %s: version %s, this library reads %s", who,
                 path, str("version") ? str("version")->c_str() : "(none)", kVersion);
    W4_SUPPORTED(str("layout") && *str("layout") == kLayout, "%s: %s: layout %s, this library reads %s", who, path,
                 str("layout") ? str("layout")->c_str() : "(none)", kLayout);
    int K = 0, N = 0, G = 0;
    W4_REQUIRE(get_int_field(meta, "K", K) && get_int_field(meta, "N", N) && get_int_field(meta, "group_size", G),
               "%s: %s: K, N, group_size must be positive decimal strings", who, path);
    const bool asym = root.obj.count("zeros") != 0;
    if (int s = w4_dims(who, K, N, G, asym ? 1 : 0, f.d, err)) return s;
    W4_REQUIRE(root.obj.size() == (asym ? 4u : 3u), "%s: %s: unexpected tensors in the file", who, path);
    // The data section the dims imply must be exactly what the file holds:
    // checked before any buffer is sized from the header's claims.
    const uint64_t total = static_cast<uint64_t>(f.d.qbytes) + static_cast<uint64_t>(f.d.sbytes) +
                           static_cast<uint64_t>(f.d.zbytes);
    const uint64_t data_bytes = file_size - 8 - hlen;
    W4_REQUIRE(data_bytes == total, "%s: %s: data section is %llu bytes, the header implies %llu", who, path,
               static_cast<unsigned long long>(data_bytes), static_cast<unsigned long long>(total));

    // Each tensor's [begin, end) is checked as unsigned 64-bit values against
    // the data section before it becomes an offset.
    auto tensor = [&](const char* name, const char* dtype, int64_t bytes, int64_t elem, int64_t& off) -> int {
        auto it = root.obj.find(name);
        W4_REQUIRE(it != root.obj.end() && it->second.kind == Json::OBJ, "%s: %s: no tensor %s", who, path, name);
        const auto& t = it->second.obj;
        auto dt = t.find("dtype");
        auto sh = t.find("shape");
        auto of = t.find("data_offsets");
        W4_REQUIRE(dt != t.end() && dt->second.kind == Json::STR && dt->second.str == dtype, "%s: %s: %s must be %s",
                   who, path, name, dtype);
        W4_REQUIRE(sh != t.end() && sh->second.kind == Json::ARR && sh->second.arr.size() == 1 &&
                       sh->second.arr[0].kind == Json::INT &&
                       sh->second.arr[0].num == static_cast<uint64_t>(bytes / elem),
                   "%s: %s: %s must have shape [%lld]", who, path, name, static_cast<long long>(bytes / elem));
        W4_REQUIRE(of != t.end() && of->second.kind == Json::ARR && of->second.arr.size() == 2 &&
                       of->second.arr[0].kind == Json::INT && of->second.arr[1].kind == Json::INT,
                   "%s: %s: %s has no data_offsets pair", who, path, name);
        const uint64_t b = of->second.arr[0].num, e = of->second.arr[1].num;
        W4_REQUIRE(b <= e && e <= total && e - b == static_cast<uint64_t>(bytes),
                   "%s: %s: %s data_offsets [%llu, %llu) do not span %lld bytes inside the %llu-byte data section",
                   who, path, name, static_cast<unsigned long long>(b), static_cast<unsigned long long>(e),
                   static_cast<long long>(bytes), static_cast<unsigned long long>(total));
        off = static_cast<int64_t>(b);
        return LHQ_OK;
    };
    if (int s = tensor("qweight", "U8", f.d.qbytes, 1, f.q_off)) return s;
    if (int s = tensor("scales", asym ? "F16" : "F32", f.d.sbytes, asym ? 2 : 4, f.s_off)) return s;
    if (asym)
        if (int s = tensor("zeros", "U32", f.d.zbytes, 4, f.z_off)) return s;
    // the tensors tile the data section without overlap (each lies inside it)
    struct Span {
        int64_t off, len;
    } spans[3] = {{f.q_off, f.d.qbytes}, {f.s_off, f.d.sbytes}, {asym ? f.z_off : 0, f.d.zbytes}};
    for (int i = 0; i < 3; ++i)
        for (int j = i + 1; j < 3; ++j)
            if (spans[i].len && spans[j].len)
                W4_REQUIRE(spans[i].off + spans[i].len <= spans[j].off || spans[j].off + spans[j].len <= spans[i].off,
                           "%s: %s: tensors overlap", who, path);
    f.bytes.resize(static_cast<size_t>(total));
    W4_REQUIRE(std::fread(f.bytes.data(), 1, f.bytes.size(), fp.get()) == f.bytes.size() &&
                   std::fgetc(fp.get()) == EOF,
               "%s: %s: data section shorter or longer than its %llu bytes", who, path,
               static_cast<unsigned long long>(total));
    const std::string* sum = str("fnv1a64");
    W4_REQUIRE(sum && *sum == hex64(fnv1a64(f.bytes.data(), f.bytes.size())),
               "%s: %s: checksum mismatch (file damaged)", who, path);
    return LHQ_OK;
}

}  // namespace

uint64_t fnv1a64(const uint8_t* p, size_t n) {
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

int w4_dims(const char* who, int K, int N, int G, int fp16_scales, W4Dims& d, std::string& err) {
    W4_REQUIRE(w4_dims_ok(K, N, G), "%s: bad dims K=%d N=%d G=%d", who, K, N, G);
    // the group sizes every W4A16 GEMM entry point takes: a file holding
    // another would load and then fail at its first use
    W4_SUPPORTED(G == 32 || G == 64 || G % 128 == 0, "%s: group_size %d: the W4A16 GEMMs take 32, 64 or a multiple of 128",
                 who, G);
    d.K = K;
    d.N = N;
    d.G = G;
    d.asym = fp16_scales != 0;
    d.qbytes = lhq_w4_qweight_bytes(K, N);
    d.sbytes = lhq_w4_scales_bytes(K, N, G, d.asym ? 1 : 0);
    d.zbytes = d.asym ? lhq_w4_zeros_bytes(K, N, G) : 0;
    W4_REQUIRE(d.qbytes > 0 && d.sbytes > 0 && (d.zbytes > 0 || !d.asym) &&
                   d.qbytes <= INT64_MAX / 4 && d.sbytes <= INT64_MAX / 4 && d.zbytes <= INT64_MAX / 4,
               "%s: K=%d N=%d G=%d give a layout too large to address", who, K, N, G);
    return LHQ_OK;
}

int w4file_read(const char* who, const char* path, W4File& f, std::string& err) {
    try {
        return read_file(who, path, f, err);
    } catch (const std::bad_alloc&) {
        f.bytes = std::vector<uint8_t>();
        return fail_with(err, LHQ_ERR_INVALID, "%s: %s: out of host memory while reading", who, path ? path : "");
    }
}

std::string w4file_header(const W4Dims& d, uint64_t checksum) {
    auto tens = [](const char* name, const char* dtype, int64_t elems, int64_t off, int64_t bytes) {
        return std::string("\"") + name + "\":{\"dtype\":\"" + dtype + "\",\"shape\":[" + std::to_string(elems) +
               "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + bytes) + "]}";
    };
    std::string h = "{\"__metadata__\":{\"format\":\"" + std::string(kFormat) + "\",\"version\":\"" + kVersion +
                    "\",\"layout\":\"" + kLayout + "\",\"K\":\"" + std::to_string(d.K) + "\",\"N\":\"" +
                    std::to_string(d.N) + "\",\"group_size\":\"" + std::to_string(d.G) + "\",\"fnv1a64\":\"" +
                    hex64(checksum) + "\"}," + tens("qweight", "U8", d.qbytes, 0, d.qbytes) + "," +
                    tens("scales", d.asym ? "F16" : "F32", d.sbytes / (d.asym ? 2 : 4), d.qbytes, d.sbytes);
    if (d.asym) h += "," + tens("zeros", "U32", d.zbytes / 4, d.qbytes + d.sbytes, d.zbytes);
    h += "}";
    while ((8 + h.size()) % 8) h += ' ';  // the data section starts 8-byte aligned
    return h;
}

}  // namespace lhq
