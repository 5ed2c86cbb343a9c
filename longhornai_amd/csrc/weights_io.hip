// weights_io.hip -- prepacked W4 weights on disk: a versioned safetensors
// file and its loader (host code only).
//
// The reference stores nothing: its int4 weights live in caller memory as
// [K/2, N] bytes plus fp32 scales (quant.hpp:52-59), and its plan lists
// safetensors loaders for later (PLAN.md:326-333).  The GPU layout
// (include/longhorn_hip.h, "prepacked weight layouts") costs a prepack pass
// per matrix; this file keeps the prepacked form so a model loads straight
// into it.
//
// File = safetensors: an 8-byte little-endian header length, a JSON header,
// then the raw tensors.  Tensors: "qweight" U8 [Nt*Kt*1024], "scales" F16 or
// F32 [Nt*NG*16], "zeros" U32 [Nt*NG8*16] (asymmetric only).  Metadata (all
// strings, as safetensors requires): format = "lhq-w4-prepacked",
// version = "1", layout = "w4-tile16x128-v1", K, N, group_size, and
// fnv1a64 = 16 hex digits of FNV-1a (64-bit) over the data section.  The
// loader checks every field, every size and the checksum before anything
// reaches the device.
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"

namespace lhq {
namespace {

constexpr const char* kFormat = "lhq-w4-prepacked";
constexpr const char* kVersion = "1";
constexpr const char* kLayout = "w4-tile16x128-v1";
constexpr uint64_t kMaxHeader = 1 << 20;  // bytes of JSON a valid file can need, with room to spare

uint64_t fnv1a64(const uint8_t* p, size_t n) {
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

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

struct W4Dims {
    int K, N, G;
    bool asym;
    int64_t qbytes, sbytes, zbytes;
};

int dims_of(const char* who, int K, int N, int G, int fp16, W4Dims& d) {
    LHQ_REQUIRE(K > 0 && N > 0 && G > 0 && K % G == 0 && K % 2 == 0, "%s: bad dims K=%d N=%d G=%d", who, K, N, G);
    d.K = K;
    d.N = N;
    d.G = G;
    d.asym = fp16 != 0;
    d.qbytes = lhq_w4_qweight_bytes(K, N);
    d.sbytes = lhq_w4_scales_bytes(K, N, G, fp16 ? 1 : 0);
    d.zbytes = d.asym ? lhq_w4_zeros_bytes(K, N, G) : 0;
    return LHQ_OK;
}

std::string hex64(uint64_t v) {
    char b[17];
    snprintf(b, sizeof(b), "%016llx", static_cast<unsigned long long>(v));
    return b;
}

// A whole file read into memory, parsed and checked.
struct W4File {
    std::vector<uint8_t> bytes;
    size_t data_off = 0;
    W4Dims d{};
    int64_t q_off = 0, s_off = 0, z_off = 0;
};

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

int read_w4_file(const char* who, const char* path, W4File& f) {
    LHQ_REQUIRE(path, "%s: null path", who);
    std::unique_ptr<FILE, int (*)(FILE*)> fp(std::fopen(path, "rb"), &std::fclose);
    LHQ_REQUIRE(fp, "%s: cannot open %s: %s", who, path, std::strerror(errno));
    uint8_t len8[8];
    LHQ_REQUIRE(std::fread(len8, 1, 8, fp.get()) == 8, "%s: %s: truncated (no header length)", who, path);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | len8[i];
    LHQ_REQUIRE(hlen >= 2 && hlen <= kMaxHeader, "%s: %s: header length %llu out of range", who, path,
                static_cast<unsigned long long>(hlen));
    std::string header(hlen, '\0');
    LHQ_REQUIRE(std::fread(&header[0], 1, hlen, fp.get()) == hlen, "%s: %s: truncated header", who, path);
    Parser ps{header.data(), header.data() + header.size(), {}};
    Json root;
    const bool parsed = ps.value(root);
    ps.ws();
    LHQ_REQUIRE(parsed && ps.p == ps.end && root.kind == Json::OBJ, "%s: %s: malformed header (%s)", who, path,
                ps.err.empty() ? "trailing bytes" : ps.err.c_str());
    auto mit = root.obj.find("__metadata__");
    LHQ_REQUIRE(mit != root.obj.end() && mit->second.kind == Json::OBJ, "%s: %s: no __metadata__", who, path);
    const auto& meta = mit->second.obj;
    for (const auto& kv : meta)
        LHQ_REQUIRE(kv.second.kind == Json::STR, "%s: %s: metadata value of %s is not a string", who, path,
                    kv.first.c_str());
    auto str = [&](const char* k) -> const std::string* {
        auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second.str;
    };
    LHQ_REQUIRE(str("format") && *str("format") == kFormat, "%s: %s: not a prepacked W4 file (format)", who, path);
    LHQ_SUPPORTED(str("version") && *str("version") == kVersion, "%s: %s: version %s, this library reads %s", who,
                  path, str("version") ? str("version")->c_str() : "(none)", kVersion);
    LHQ_SUPPORTED(str("layout") && *str("layout") == kLayout, "%s: %s: layout %s, this library reads %s", who, path,
                  str("layout") ? str("layout")->c_str() : "(none)", kLayout);
    int K = 0, N = 0, G = 0;
    LHQ_REQUIRE(get_int_field(meta, "K", K) && get_int_field(meta, "N", N) && get_int_field(meta, "group_size", G),
                "%s: %s: K, N, group_size must be positive decimal strings", who, path);

    auto tensor = [&](const char* name, const char* dtype, int64_t bytes, int64_t elem, int64_t& off) -> int {
        auto it = root.obj.find(name);
        LHQ_REQUIRE(it != root.obj.end() && it->second.kind == Json::OBJ, "%s: %s: no tensor %s", who, path, name);
        const auto& t = it->second.obj;
        auto dt = t.find("dtype");
        auto sh = t.find("shape");
        auto of = t.find("data_offsets");
        LHQ_REQUIRE(dt != t.end() && dt->second.kind == Json::STR && dt->second.str == dtype, "%s: %s: %s must be %s",
                    who, path, name, dtype);
        LHQ_REQUIRE(sh != t.end() && sh->second.kind == Json::ARR && sh->second.arr.size() == 1 &&
                        sh->second.arr[0].kind == Json::INT &&
                        sh->second.arr[0].num == static_cast<uint64_t>(bytes / elem),
                    "%s: %s: %s must have shape [%lld]", who, path, name, static_cast<long long>(bytes / elem));
        LHQ_REQUIRE(of != t.end() && of->second.kind == Json::ARR && of->second.arr.size() == 2 &&
                        of->second.arr[0].kind == Json::INT && of->second.arr[1].kind == Json::INT &&
                        of->second.arr[1].num >= of->second.arr[0].num &&
                        of->second.arr[1].num - of->second.arr[0].num == static_cast<uint64_t>(bytes),
                    "%s: %s: %s data_offsets do not span %lld bytes", who, path, name, static_cast<long long>(bytes));
        off = static_cast<int64_t>(of->second.arr[0].num);
        return LHQ_OK;
    };
    const bool asym = root.obj.count("zeros") != 0;
    if (int st = dims_of(who, K, N, G, asym ? 1 : 0, f.d)) return st;
    LHQ_REQUIRE(f.d.sbytes > 0, "%s: %s: unsupported group_size %d", who, path, G);
    LHQ_REQUIRE(root.obj.size() == (asym ? 4u : 3u), "%s: %s: unexpected tensors in the file", who, path);
    if (int st = tensor("qweight", "U8", f.d.qbytes, 1, f.q_off)) return st;
    if (int st = tensor("scales", asym ? "F16" : "F32", f.d.sbytes, asym ? 2 : 4, f.s_off)) return st;
    if (asym)
        if (int st = tensor("zeros", "U32", f.d.zbytes, 4, f.z_off)) return st;

    // data section: exactly the tensors, without overlap
    const int64_t total = f.d.qbytes + f.d.sbytes + f.d.zbytes;
    struct Span {
        int64_t off, len;
    } spans[3] = {{f.q_off, f.d.qbytes}, {f.s_off, f.d.sbytes}, {asym ? f.z_off : 0, f.d.zbytes}};
    for (int i = 0; i < 3; ++i)
        for (int j = i + 1; j < 3; ++j)
            if (spans[i].len && spans[j].len)
                LHQ_REQUIRE(spans[i].off + spans[i].len <= spans[j].off || spans[j].off + spans[j].len <= spans[i].off,
                            "%s: %s: tensors overlap", who, path);
    for (const Span& sp : spans) LHQ_REQUIRE(sp.off + sp.len <= total, "%s: %s: tensor past the data", who, path);
    f.bytes.resize(static_cast<size_t>(total) + 1);
    const size_t got = std::fread(f.bytes.data(), 1, f.bytes.size(), fp.get());
    LHQ_REQUIRE(got == static_cast<size_t>(total), "%s: %s: data section is %zu bytes, expected %lld", who, path,
                got, static_cast<long long>(total));
    f.bytes.resize(static_cast<size_t>(total));
    const std::string* sum = str("fnv1a64");
    LHQ_REQUIRE(sum && *sum == hex64(fnv1a64(f.bytes.data(), f.bytes.size())),
                "%s: %s: checksum mismatch (file damaged)", who, path);
    return LHQ_OK;
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_w4_save(const char* path, const uint8_t* qweight, const void* scales, const uint32_t* zeros, int K, int N,
                int G, int fp16_scales, void* stream) {
    W4Dims d{};
    if (int st = dims_of("w4_save", K, N, G, fp16_scales, d)) return st;
    LHQ_REQUIRE(d.sbytes > 0, "w4_save: group_size %d does not divide K=%d", G, K);
    LHQ_REQUIRE(path && qweight && scales && (zeros || !d.asym), "w4_save: null pointer");
    std::vector<uint8_t> data(static_cast<size_t>(d.qbytes + d.sbytes + d.zbytes));
    hipStream_t s = as_stream(stream);
    hipError_t e = hipMemcpyAsync(data.data(), qweight, d.qbytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(data.data() + d.qbytes, scales, d.sbytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && d.asym)
        e = hipMemcpyAsync(data.data() + d.qbytes + d.sbytes, zeros, d.zbytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return set_error(LHQ_ERR_HIP, "w4_save: copy to host: %s", hipGetErrorString(e));

    auto tens = [](const char* name, const char* dtype, int64_t elems, int64_t off, int64_t bytes) {
        return std::string("\"") + name + "\":{\"dtype\":\"" + dtype + "\",\"shape\":[" + std::to_string(elems) +
               "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + bytes) + "]}";
    };
    std::string h = "{\"__metadata__\":{\"format\":\"" + std::string(kFormat) + "\",\"version\":\"" + kVersion +
                    "\",\"layout\":\"" + kLayout + "\",\"K\":\"" + std::to_string(K) + "\",\"N\":\"" +
                    std::to_string(N) + "\",\"group_size\":\"" + std::to_string(G) + "\",\"fnv1a64\":\"" +
                    hex64(fnv1a64(data.data(), data.size())) + "\"}," + tens("qweight", "U8", d.qbytes, 0, d.qbytes) +
                    "," + tens("scales", d.asym ? "F16" : "F32", d.sbytes / (d.asym ? 2 : 4), d.qbytes, d.sbytes);
    if (d.asym) h += "," + tens("zeros", "U32", d.zbytes / 4, d.qbytes + d.sbytes, d.zbytes);
    h += "}";
    while ((8 + h.size()) % 8) h += ' ';  // the data section starts 8-byte aligned
    uint8_t len8[8];
    for (int i = 0; i < 8; ++i) len8[i] = static_cast<uint8_t>(static_cast<uint64_t>(h.size()) >> (8 * i));

    std::unique_ptr<FILE, int (*)(FILE*)> fp(std::fopen(path, "wb"), &std::fclose);
    LHQ_REQUIRE(fp, "w4_save: cannot create %s: %s", path, std::strerror(errno));
    const bool ok = std::fwrite(len8, 1, 8, fp.get()) == 8 && std::fwrite(h.data(), 1, h.size(), fp.get()) == h.size() &&
                    std::fwrite(data.data(), 1, data.size(), fp.get()) == data.size();
    const int closed = std::fclose(fp.release());
    LHQ_REQUIRE(ok && closed == 0, "w4_save: writing %s failed", path);
    return LHQ_OK;
}

int lhq_w4_file_info(const char* path, int* K, int* N, int* group_size, int* fp16_scales) {
    W4File f;
    if (int st = read_w4_file("w4_file_info", path, f)) return st;
    if (K) *K = f.d.K;
    if (N) *N = f.d.N;
    if (group_size) *group_size = f.d.G;
    if (fp16_scales) *fp16_scales = f.d.asym ? 1 : 0;
    return LHQ_OK;
}

int lhq_w4_load(const char* path, uint8_t* qweight, void* scales, uint32_t* zeros, int K, int N, int G,
                int fp16_scales, void* stream) {
    W4File f;
    if (int st = read_w4_file("w4_load", path, f)) return st;
    LHQ_REQUIRE(f.d.K == K && f.d.N == N && f.d.G == G && f.d.asym == (fp16_scales != 0),
                "w4_load: %s holds K=%d N=%d G=%d %s, the caller asked for K=%d N=%d G=%d %s", path, f.d.K, f.d.N,
                f.d.G, f.d.asym ? "asymmetric" : "symmetric", K, N, G, fp16_scales ? "asymmetric" : "symmetric");
    LHQ_REQUIRE(qweight && scales && (zeros || !f.d.asym), "w4_load: null pointer");
    hipStream_t s = as_stream(stream);
    hipError_t e = hipMemcpyAsync(qweight, f.bytes.data() + f.q_off, f.d.qbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(scales, f.bytes.data() + f.s_off, f.d.sbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && f.d.asym)
        e = hipMemcpyAsync(zeros, f.bytes.data() + f.z_off, f.d.zbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host copy is freed on return
    if (e != hipSuccess) return set_error(LHQ_ERR_HIP, "w4_load: copy to device: %s", hipGetErrorString(e));
    return LHQ_OK;
}

}  // extern "C"
