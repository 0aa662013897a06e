// mnb_pack.cpp -- weight files: .wdmlpack packages and ONNX models holding
// int4 MatMulNBits triplets, opened read-only by memory mapping and handed to
// mnb_weight_create without a host copy of the packed nibbles.
//
// Reference behaviour followed (paths relative to the reference root):
//   MP  = directml-model-package/src/main/java/com/aresstack/windirectml/modelpack
//   INF = directml-inference/src/main/java/com/aresstack/windirectml/inference
//   Q2W = INF/qwen/Qwen2Weights.java
//   container header, manifest and payload ranges   MP/WdmlPackWriter.java:55-66, 114-177, 254-259
//   manifest root checks and value coercions        MP/WdmlPackManifest.java:35-68, 108-176
//   tensor directory and per-tensor payload ranges  MP/WdmlPackReader.java:37-96
//   Phi-3 role triplets                             INF/phi3/Phi3RuntimePackage.java:35-46, 132-152
//   Qwen payload packages (runtimeGraph nodes)      INF/qwen/QwenWdmlPackModelSource.java:59-185
//   ONNX graph, initializers, external references   directml-windows-bindings/.../windows/OnnxModelReader.java:183-600,
//                                                   Q2W:1809-1938 (external refs), Q2W:495-545 (node map)
//   triplet resolution and zero-point layouts       Q2W:936-976, 986-1121, 1576-1611, 2063-2131
//
// Every failure is the reference's IOException: status MNB_ERR_IO and its text.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "mnb_internal.h"

namespace {

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "file formats are little-endian");

struct IoError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

std::string fmt(const char *f, ...) {
    va_list ap;
    va_start(ap, f);
    va_list ap2;
    va_copy(ap2, ap);
    const int n = vsnprintf(nullptr, 0, f, ap);
    va_end(ap);
    std::string s(n > 0 ? (size_t)n : 0, '\0');
    if (n > 0) vsnprintf(&s[0], (size_t)n + 1, f, ap2);
    va_end(ap2);
    return s;
}

[[noreturn]] void io_error(const std::string &m) { throw IoError(m); }

void copy_bytes(void *dst, const void *src, size_t n) {  // memcpy that accepts n == 0 with null pointers
    if (n) memcpy(dst, src, n);
}

std::string dims_text(const std::vector<int64_t> &d) {  // java.util.Arrays.toString(long[])
    std::string s = "[";
    for (size_t i = 0; i < d.size(); ++i) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

// ---------------------------------------------------------------------------
// read-only file mapping
// ---------------------------------------------------------------------------
struct MappedFile {
    std::string path;
    const uint8_t *data = nullptr;
    int64_t size = 0;

    explicit MappedFile(const std::string &p) : path(p) {
        const int fd = ::open(p.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) io_error(fmt("Cannot open %s: %s", p.c_str(), strerror(errno)));
        struct stat st;
        if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
            ::close(fd);
            io_error("Not a regular file: " + p);
        }
        size = (int64_t)st.st_size;
        if (size > 0) {
            void *m = mmap(nullptr, (size_t)size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) {
                const int e = errno;
                ::close(fd);
                io_error(fmt("Cannot map %s: %s", p.c_str(), strerror(e)));
            }
            data = (const uint8_t *)m;
        }
        ::close(fd);
    }
    ~MappedFile() {
        if (data) munmap((void *)data, (size_t)size);
    }
    MappedFile(const MappedFile &) = delete;
    MappedFile &operator=(const MappedFile &) = delete;
};

bool file_exists(const std::string &p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string dir_of(const std::string &p) {
    const size_t k = p.find_last_of('/');
    if (k == std::string::npos) return ".";
    return k == 0 ? "/" : p.substr(0, k);
}

// ---------------------------------------------------------------------------
// JSON (the manifest): a small recursive-descent reader
// ---------------------------------------------------------------------------
struct Json {
    enum Kind : uint8_t { Null, Bool, Int, Real, Str, Arr, Obj };
    Kind kind = Null;
    bool b = false;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;  // members in file order

    // A later duplicate key replaces an earlier one, as in a map.
    const Json *get(const std::string &k) const {
        if (kind != Obj) return nullptr;
        for (auto it = o.rbegin(); it != o.rend(); ++it)
            if (it->first == k) return &it->second;
        return nullptr;
    }
};

class JsonReader {
public:
    JsonReader(const char *p, size_t n, const char *what = "wdmlpack manifest") : b_(p), p_(p), e_(p + n), what_(what) {}

    Json document() {
        ws();
        Json v = value(0);
        ws();
        if (p_ != e_) err("trailing characters after the document");
        return v;
    }

private:
    const char *b_, *p_, *e_;
    const char *what_;

    [[noreturn]] void err(const char *what) {
        io_error(fmt("Invalid %s JSON at byte %lld: %s", what_, (long long)(p_ - b_), what));
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(e_ - p_) >= n && memcmp(p_, w, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    Json value(int depth) {
        if (depth > 256) err("nesting too deep");
        if (p_ >= e_) err("unexpected end of input");
        Json v;
        switch (*p_) {
        case '{':
            ++p_;
            v.kind = Json::Obj;
            ws();
            if (p_ < e_ && *p_ == '}') {
                ++p_;
                return v;
            }
            for (;;) {
                ws();
                if (p_ >= e_ || *p_ != '"') err("expected a string key");
                std::string k = str();
                ws();
                if (p_ >= e_ || *p_ != ':') err("expected ':'");
                ++p_;
                ws();
                v.o.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    return v;
                }
                err("expected ',' or '}'");
            }
        case '[':
            ++p_;
            v.kind = Json::Arr;
            ws();
            if (p_ < e_ && *p_ == ']') {
                ++p_;
                return v;
            }
            for (;;) {
                ws();
                v.a.push_back(value(depth + 1));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    return v;
                }
                err("expected ',' or ']'");
            }
        case '"':
            v.kind = Json::Str;
            v.s = str();
            return v;
        case 't':
            if (!lit("true")) err("invalid literal");
            v.kind = Json::Bool;
            v.b = true;
            return v;
        case 'f':
            if (!lit("false")) err("invalid literal");
            v.kind = Json::Bool;
            return v;
        case 'n':
            if (!lit("null")) err("invalid literal");
            return v;
        default:
            return number();
        }
    }
    static void put_utf8(std::string &s, uint32_t c) {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    uint32_t hex4() {
        if (e_ - p_ < 4) err("truncated \\u escape");
        uint32_t c = 0;
        for (int k = 0; k < 4; ++k) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
            else err("invalid \\u escape");
        }
        return c;
    }
    std::string str() {
        ++p_;  // opening quote
        std::string s;
        for (;;) {
            if (p_ >= e_) err("unterminated string");
            const char c = *p_++;
            if (c == '"') return s;
            if ((unsigned char)c < 0x20) err("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= e_) err("unterminated escape");
            const char x = *p_++;
            switch (x) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t c1 = hex4();
                if (c1 >= 0xD800 && c1 < 0xDC00 && e_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                    const char *save = p_;
                    p_ += 2;
                    const uint32_t c2 = hex4();
                    if (c2 >= 0xDC00 && c2 < 0xE000) c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    else p_ = save;
                }
                put_utf8(s, c1);
                break;
            }
            default: err("invalid escape");
            }
        }
    }
    Json number() {
        const char *st = p_;
        bool real = false;
        if (p_ < e_ && *p_ == '-') ++p_;
        if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) err("unexpected character");
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < e_ && *p_ == '.') {
            real = true;
            ++p_;
            if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) err("invalid number");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            real = true;
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) err("invalid number");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string text(st, (size_t)(p_ - st));
        Json v;
        v.s = text;
        if (!real) {
            errno = 0;
            char *end = nullptr;
            const long long x = strtoll(text.c_str(), &end, 10);
            if (errno == 0 && end && *end == '\0') {
                v.kind = Json::Int;
                v.i = x;
                v.d = (double)x;
                return v;
            }
        }
        v.kind = Json::Real;
        v.d = strtod(text.c_str(), nullptr);
        return v;
    }
};

// Java's narrowing of a double to long / int: NaN -> 0, saturating.
int64_t java_d2l(double d) {
    if (std::isnan(d)) return 0;
    if (d >= 9.2233720368547758e18) return std::numeric_limits<int64_t>::max();
    if (d <= -9.2233720368547758e18) return std::numeric_limits<int64_t>::min();
    return (int64_t)d;
}
int32_t java_d2i(double d) {
    if (std::isnan(d)) return 0;
    if (d >= 2147483647.0) return std::numeric_limits<int32_t>::max();
    if (d <= -2147483648.0) return std::numeric_limits<int32_t>::min();
    return (int32_t)d;
}

// Long.parseLong / Integer.parseInt: optional sign, decimal digits only.
bool java_parse_long(const std::string &s, int64_t lo, int64_t hi, int64_t &out) {
    size_t k = 0;
    bool neg = false;
    if (k < s.size() && (s[k] == '-' || s[k] == '+')) neg = s[k++] == '-';
    if (k == s.size()) return false;
    unsigned __int128 acc = 0;
    for (; k < s.size(); ++k) {
        if (s[k] < '0' || s[k] > '9') return false;
        acc = acc * 10 + (unsigned)(s[k] - '0');
        if (acc > ((unsigned __int128)1 << 64)) return false;
    }
    const __int128 v = neg ? -(__int128)acc : (__int128)acc;
    if (v < lo || v > hi) return false;
    out = (int64_t)v;
    return true;
}

bool is_blank(const std::string &s) {
    for (char c : s)
        if (!(c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v')) return false;
    return true;
}

// WdmlPackManifest.intValue / longValue / stringValue / dimsValue (MP/WdmlPackManifest.java:125-176)
int32_t int_value(const Json *v, int32_t def) {
    if (!v) return def;
    if (v->kind == Json::Int) return (int32_t)(uint32_t)(uint64_t)v->i;  // Number.intValue of a Long
    if (v->kind == Json::Real) return java_d2i(v->d);
    if (v->kind == Json::Str && !is_blank(v->s)) {
        int64_t x;
        return java_parse_long(v->s, std::numeric_limits<int32_t>::min(), std::numeric_limits<int32_t>::max(), x)
                   ? (int32_t)x
                   : def;
    }
    return def;
}
int64_t long_value(const Json *v, int64_t def) {
    if (!v) return def;
    if (v->kind == Json::Int) return v->i;
    if (v->kind == Json::Real) return java_d2l(v->d);
    if (v->kind == Json::Str && !is_blank(v->s)) {
        int64_t x;
        return java_parse_long(v->s, std::numeric_limits<int64_t>::min(), std::numeric_limits<int64_t>::max(), x)
                   ? x
                   : def;
    }
    return def;
}
std::string string_value(const Json *v) { return v && v->kind == Json::Str ? v->s : std::string(); }
std::vector<int64_t> dims_value(const Json *v) {
    std::vector<int64_t> d;
    if (!v || v->kind != Json::Arr) return d;
    for (const Json &e : v->a) {
        int64_t x = 0;
        if (e.kind == Json::Int || e.kind == Json::Real) x = long_value(&e, 0);
        else if (e.kind == Json::Str && !is_blank(e.s)) x = long_value(&e, 0);
        d.push_back(x);
    }
    return d;
}
// String.valueOf(Object) of a manifest value, for messages.
std::string value_text(const Json *v) {
    if (!v || v->kind == Json::Null) return "null";
    switch (v->kind) {
    case Json::Bool: return v->b ? "true" : "false";
    case Json::Int:
    case Json::Real:
    case Json::Str: return v->s;
    case Json::Arr: return "[...]";
    default: return "{...}";
    }
}

std::vector<std::string> string_list(const Json *v) {  // RuntimeModelPackage.stringList: String.valueOf(item)
    std::vector<std::string> out;
    if (!v || v->kind != Json::Arr) return out;
    for (const Json &e : v->a) out.push_back(e.kind == Json::Str ? e.s : value_text(&e));
    return out;
}
// ---------------------------------------------------------------------------
// protobuf wire format (ONNX), lenient the way the reference reader is:
// a length that runs past its buffer is clamped to it.
// ---------------------------------------------------------------------------
struct Pb {
    const uint8_t *p, *end;

    bool more() const { return p < end; }
    uint64_t varint() {
        uint64_t r = 0;
        int sh = 0;
        while (p < end) {
            const uint8_t b = *p++;
            if (sh < 64) r |= (uint64_t)(b & 0x7F) << sh;
            if (!(b & 0x80)) return r;
            sh += 7;
        }
        return r;
    }
    Pb sub() {  // a length-delimited field, clamped to this buffer
        const uint64_t n = varint();
        const uint8_t *s = p;
        p = n > (uint64_t)(end - p) ? end : p + n;
        return Pb{s, p};
    }
    std::string str() {
        Pb s = sub();
        return std::string((const char *)s.p, (size_t)(s.end - s.p));
    }
    uint32_t fixed32() {
        uint32_t v = 0;
        if (end - p >= 4) memcpy(&v, p, 4);
        p = end - p >= 4 ? p + 4 : end;
        return v;
    }
    void skip(uint32_t wt) {
        switch (wt) {
        case 0: varint(); break;
        case 1: p = end - p >= 8 ? p + 8 : end; break;
        case 2: sub(); break;
        case 5: p = end - p >= 4 ? p + 4 : end; break;
        default: throw std::runtime_error(fmt("Unknown wire type: %u", wt));
        }
    }
};

constexpr int32_t kOnnxFloat = 1, kOnnxUint8 = 2, kOnnxInt8 = 3, kOnnxInt32 = 6, kOnnxInt64 = 7, kOnnxFloat16 = 10,
                  kOnnxBfloat16 = 16;

const char *onnx_type_name(int32_t t) {  // Q2W:2133-2143
    switch (t) {
    case kOnnxFloat: return "FLOAT";
    case kOnnxFloat16: return "FLOAT16";
    case kOnnxUint8: return "UINT8";
    case kOnnxInt8: return "INT8";
    case kOnnxInt32: return "INT32";
    case kOnnxInt64: return "INT64";
    case kOnnxBfloat16: return "BFLOAT16";
    default: return "UNKNOWN";
    }
}

// One tensor of a source, in the two views the reference keeps: an external
// reference (offset/length into the external data file) or inline data
// (raw bytes, or float values for FLOAT tensors).
struct Tensor {
    std::string name;
    int32_t dtype = 0;
    std::vector<int64_t> dims;
    bool external = false;
    int64_t ext_offset = 0, ext_length = 0;
    const uint8_t *raw = nullptr;  // inline raw bytes (in the mapping, or in `owned`)
    int64_t raw_len = 0;
    std::vector<uint8_t> owned;
    std::vector<float> floats;  // inline FLOAT values (float_data, or raw_data of a FLOAT tensor)

    bool has_inline() const { return !floats.empty() || raw_len > 0; }
};

struct Node {
    std::string op_type;
    std::vector<std::string> inputs, outputs;
};

// TensorProto (OnnxModelReader.java:403-578 for inline data, Q2W:1862-1938 for
// the external reference).
Tensor parse_tensor(Pb m, const uint8_t *file_end) {
    Tensor t;
    int32_t location = 0;
    const uint8_t *raw = nullptr;
    int64_t raw_len = -1;
    bool have_floats = false;
    std::vector<int64_t> i32;
    bool have_i32 = false;
    auto kv_entry = [&](Pb e) {
        std::string k, v;
        bool hk = false, hv = false;
        while (e.more()) {
            const uint64_t tag = e.varint();
            const uint32_t f = (uint32_t)(tag >> 3), wt = (uint32_t)(tag & 7);
            if (f == 1 && wt == 2) k = e.str(), hk = true;
            else if (f == 2 && wt == 2) v = e.str(), hv = true;
            else e.skip(wt);
        }
        if (!(hk && hv)) return;
        int64_t x;
        if (k == "offset" && java_parse_long(v, INT64_MIN, INT64_MAX, x)) t.ext_offset = x;
        if (k == "length" && java_parse_long(v, INT64_MIN, INT64_MAX, x)) t.ext_length = x;
    };
    while (m.more()) {
        const uint64_t tag = m.varint();
        const uint32_t f = (uint32_t)(tag >> 3), wt = (uint32_t)(tag & 7);
        switch (f) {
        case 1:  // dims
            if (wt == 2) {
                Pb d = m.sub();
                while (d.more()) t.dims.push_back((int64_t)d.varint());
            } else if (wt == 0) {
                t.dims.push_back((int64_t)m.varint());
            } else {
                m.skip(wt);
            }
            break;
        case 2:  // data_type
            if (wt == 0) t.dtype = (int32_t)m.varint();
            else m.skip(wt);
            break;
        case 4:  // float_data
            if (wt == 2) {
                Pb d = m.sub();
                t.floats.clear();
                while (d.end - d.p >= 4) {
                    const uint32_t u = d.fixed32();
                    float x;
                    memcpy(&x, &u, 4);
                    t.floats.push_back(x);
                }
                have_floats = true;
            } else if (wt == 5) {
                const uint32_t u = m.fixed32();
                float x;
                memcpy(&x, &u, 4);
                t.floats.assign(1, x);
                have_floats = true;
            } else {
                m.skip(wt);
            }
            break;
        case 5:  // int32_data
            if (wt == 2) {
                Pb d = m.sub();
                i32.clear();
                while (d.more()) i32.push_back((int64_t)d.varint());
                have_i32 = true;
            } else if (wt == 0) {
                i32.push_back((int64_t)m.varint());
                have_i32 = true;
            } else {
                m.skip(wt);
            }
            break;
        case 8:  // name
            if (wt == 2) t.name = m.str();
            else m.skip(wt);
            break;
        case 9:  // raw_data: a length beyond the file marks an external-data stub
            if (wt == 2) {
                const uint64_t n = m.varint();
                if (n > (uint64_t)(file_end - m.p)) {
                    m.p = m.end;
                } else {
                    raw = m.p;
                    raw_len = (int64_t)n;
                    m.p = m.p + n > m.end ? m.end : m.p + n;
                }
            } else {
                m.skip(wt);
            }
            break;
        case 13:  // external_data entries
            if (wt == 2) kv_entry(m.sub());
            else m.skip(wt);
            break;
        case 14:  // data_location (an entry in some writers)
            if (wt == 0) location = (int32_t)m.varint();
            else if (wt == 2) kv_entry(m.sub());
            else m.skip(wt);
            break;
        case 15:
            if (wt == 0) location = (int32_t)m.varint();
            else m.skip(wt);
            break;
        default:
            m.skip(wt);
        }
    }
    if (location == 1) {
        t.external = !t.name.empty();
        t.floats.clear();
        return t;
    }
    if (have_floats) return t;
    t.floats.clear();
    if (raw_len >= 0 && t.dtype == kOnnxFloat) {
        t.floats.resize((size_t)(raw_len / 4));
        copy_bytes(t.floats.data(), raw, t.floats.size() * 4);
    } else if (raw_len >= 0) {
        t.raw = raw;
        t.raw_len = raw_len;
    } else if (have_i32) {
        if (t.dtype == kOnnxInt8 || t.dtype == kOnnxUint8) {
            for (int64_t v : i32) t.owned.push_back((uint8_t)v);
        } else if (t.dtype == kOnnxInt32) {
            for (int64_t v : i32) {
                const uint32_t u = (uint32_t)v;
                for (int k = 0; k < 4; ++k) t.owned.push_back((uint8_t)(u >> (8 * k)));
            }
        } else if (t.dtype == kOnnxFloat16) {
            for (int64_t v : i32) {
                t.owned.push_back((uint8_t)v);
                t.owned.push_back((uint8_t)(v >> 8));
            }
        }
        t.raw = t.owned.data();
        t.raw_len = (int64_t)t.owned.size();
    }
    return t;
}

Node parse_node(Pb m) {
    Node n;
    while (m.more()) {
        const uint64_t tag = m.varint();
        const uint32_t f = (uint32_t)(tag >> 3), wt = (uint32_t)(tag & 7);
        if (f == 1 && wt == 2) n.inputs.push_back(m.str());
        else if (f == 2 && wt == 2) n.outputs.push_back(m.str());
        else if (f == 4 && wt == 2) n.op_type = m.str();
        else m.skip(wt);
    }
    return n;
}

// ---------------------------------------------------------------------------
// the reference's fp16 -> fp32 widening of scales (P3W:665-683, Q2W:1730-1743):
// exact for normal values, inf and NaN; a subnormal m*2^-24 becomes the fp32
// product (m*2^-136) * 2^-14, i.e. m*2^-150 rounded to nearest even.
// P3W = INF/phi3/Phi3Weights.java
// ---------------------------------------------------------------------------
float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
float ref_fp16_to_fp32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) & 1u, e = (uint32_t)(h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bits_f32(s << 31);
        volatile float sub = bits_f32((s << 31) | (m << 13));  // kept as an fp32 multiply
        return sub * (1.0f / 16384.0f);
    }
    if (e == 31) return bits_f32((s << 31) | 0x7F800000u | (m << 13));
    return bits_f32((s << 31) | ((e - 15 + 127) << 23) | (m << 13));
}

int java_round_f(float v) {  // Math.round(float): floor(v + 1/2), NaN -> 0, saturating
    if (std::isnan(v)) return 0;
    const double r = std::floor((double)v + 0.5);
    if (r >= 2147483647.0) return std::numeric_limits<int>::max();
    if (r <= -2147483648.0) return std::numeric_limits<int>::min();
    return (int)r;
}

void put_nibble(std::vector<uint8_t> &buf, int64_t i, int v) {
    uint8_t &b = buf[(size_t)(i / 2)];
    b = (i & 1) ? (uint8_t)((b & 0x0F) | ((v & 0xF) << 4)) : (uint8_t)((b & 0xF0) | (v & 0xF));
}
int get_nibble(const uint8_t *buf, int64_t i) { return (i & 1) ? buf[i / 2] >> 4 : buf[i / 2] & 0xF; }

// A resolved weight triplet: the reference's QuantizedWeight.
struct Triplet {
    int32_t N = 0, K = 0, bs = 0, kb = 0;
    const uint8_t *q = nullptr;
    int64_t q_bytes = 0;
    std::vector<float> scales;
    int32_t scale_dtype = kOnnxFloat;
    const uint8_t *zp = nullptr;
    int64_t zp_bytes = 0;
    std::vector<uint8_t> zp_owned;
    bool zp_implicit = false;
};

}  // namespace

// ---------------------------------------------------------------------------
// the pack
// ---------------------------------------------------------------------------
struct mnb_pack {
    int32_t kind = 0;
    std::unique_ptr<MappedFile> file;      // the package or the model
    std::unique_ptr<MappedFile> ext_file;  // ONNX external data
    // Phi-3 packages and Qwen payload packages: the tensor directory
    std::unordered_map<std::string, Tensor> tensors;
    // ONNX: external references and inline initializers, looked up in that order
    std::unordered_map<std::string, Tensor> ext_refs;
    std::unordered_map<std::string, Tensor> inline_tensors;
    std::vector<std::string> names;  // weights in file order
    // graph sources: weight name -> {qweight, scales, zero points ("" when absent)}
    std::unordered_map<std::string, std::vector<std::string>> triplets;

    const Tensor *find_ext(const std::string &n) const {
        auto it = ext_refs.find(n);
        return it == ext_refs.end() ? nullptr : &it->second;
    }
    const Tensor *find_inline(const std::string &n) const {
        auto it = inline_tensors.find(n);
        return it == inline_tensors.end() ? nullptr : &it->second;
    }
};

namespace {

// --- wdmlpack container -----------------------------------------------------
constexpr int64_t kHeaderSize = 64;
constexpr int32_t kPackVersion = 1;
constexpr int32_t kFlagManifestOnly = 1;

struct PackHeader {
    int32_t version = 0, flags = 0;
    int64_t manifest_off = 0, manifest_len = 0, dir_off = 0, dir_len = 0, payload_off = 0, payload_len = 0;
    bool payload_included() const { return payload_off > 0 && payload_len > 0 && !(flags & kFlagManifestOnly); }
};

template <class T>
T le(const uint8_t *p) {
    T v;
    memcpy(&v, p, sizeof v);
    return v;
}

void validate_range(const char *label, int64_t off, int64_t len, int64_t file_size, int64_t min_off) {
    int64_t end = 0;
    if (off < min_off || len < 0 || __builtin_add_overflow(off, len, &end) || end > file_size)
        io_error(fmt("Invalid wdmlpack %s range: offset=%lld, length=%lld, fileSize=%lld", label, (long long)off,
                     (long long)len, (long long)file_size));
}

PackHeader read_header(const MappedFile &f) {
    if (f.size < kHeaderSize) io_error("Invalid wdmlpack: file is smaller than header: " + f.path);
    std::string magic;
    for (int k = 0; k < 8; ++k) magic += (f.data[k] < 0x80) ? (char)f.data[k] : '?';  // US-ASCII decoding
    if (magic != "WDMLPACK") io_error("Invalid wdmlpack magic: " + magic);
    PackHeader h;
    h.version = le<int32_t>(f.data + 8);
    if (h.version != kPackVersion) io_error(fmt("Unsupported wdmlpack version: %d", h.version));
    h.flags = le<int32_t>(f.data + 12);
    h.manifest_off = le<int64_t>(f.data + 16);
    h.manifest_len = le<int64_t>(f.data + 24);
    h.dir_off = le<int64_t>(f.data + 32);
    h.dir_len = le<int64_t>(f.data + 40);
    h.payload_off = le<int64_t>(f.data + 48);
    h.payload_len = le<int64_t>(f.data + 56);
    validate_range("manifest", h.manifest_off, h.manifest_len, f.size, kHeaderSize);
    if (h.payload_off != 0 || h.payload_len != 0) validate_range("payload", h.payload_off, h.payload_len, f.size, kHeaderSize);
    return h;
}

Json read_manifest(const MappedFile &f, const PackHeader &h) {
    if (h.manifest_len > std::numeric_limits<int32_t>::max())
        io_error(fmt("wdmlpack manifest is too large to parse: %lld bytes", (long long)h.manifest_len));
    Json root = JsonReader((const char *)f.data + h.manifest_off, (size_t)h.manifest_len).document();
    if (root.kind != Json::Obj) io_error("Invalid wdmlpack manifest: the root is not a JSON object");
    return root;
}

bool payload_included(const Json &root) {
    const Json *v = root.get("payloadIncluded");
    return v && v->kind == Json::Bool && v->b;
}
bool runtime_loadable(const Json &root) {
    const Json *v = root.get("runtimeLoadable");
    return !(v && v->kind == Json::Bool) || v->b;
}

void validate_root(const Json &root, const PackHeader &h) {
    const Json *format = root.get("format");
    if (!(format && format->kind == Json::Str && format->s == "wdmlpack"))
        io_error("Invalid wdmlpack manifest format: " + value_text(format));
    const int32_t version = int_value(root.get("version"), -1);
    if (version != kPackVersion) io_error(fmt("Unsupported wdmlpack manifest version: %d", version));
    const bool pi = payload_included(root);
    if (pi && !h.payload_included())
        io_error("wdmlpack manifest says payloadIncluded=true but the container header has no payload");
    if (!pi && h.payload_included()) io_error("wdmlpack container has payload but manifest says payloadIncluded=false");
}

// RuntimeTensorCatalog of a payload package (MP/WdmlPackReader.java:37-96):
// every named directory entry, with its payload range checked.
void map_payload_tensors(mnb_pack &pk, const Json &root, const PackHeader &h) {
    const Json *dir = root.get("tensors");
    if (!dir || dir->kind != Json::Arr) io_error("Invalid wdmlpack: missing tensors directory");
    const MappedFile &f = *pk.file;
    for (const Json &e : dir->a) {
        if (e.kind != Json::Obj) continue;
        Tensor t;
        t.name = string_value(e.get("name"));
        if (is_blank(t.name)) continue;
        t.dtype = int_value(e.get("dataType"), 0);
        t.dims = dims_value(e.get("dims"));
        const int64_t byte_len = long_value(e.get("byteLength"), 0);
        const int64_t off = long_value(e.get("payloadOffset"), -1);
        const int64_t len = long_value(e.get("payloadLength"), byte_len);
        if (off >= 0 && len > 0) {
            int64_t start = 0, end = 0;
            if (__builtin_add_overflow(h.payload_off, off, &start) || __builtin_add_overflow(start, len, &end) ||
                end > h.payload_off + h.payload_len || end > f.size)
                io_error(fmt("Invalid wdmlpack tensor payload range for %s: offset=%lld, length=%lld", t.name.c_str(),
                             (long long)off, (long long)len));
            t.raw = f.data + start;
            t.raw_len = len;
        }
        std::string key = t.name;
        pk.tensors[key] = std::move(t);
    }
}

// --- Phi-3 packages (Phi3RuntimePackage.java:35-46, 132-152) ---------------
const std::string kQweight = ".qweight", kScales = ".scales", kZeropoints = ".zeropoints";

const Tensor &phi3_require(const mnb_pack &pk, const std::string &name) {
    auto it = pk.tensors.find(name);
    if (it == pk.tensors.end() || it->second.raw_len <= 0) io_error("Phi-3 wdmlpack is missing payload tensor: " + name);
    return it->second;
}

void open_phi3(mnb_pack &pk, const Json &root) {
    if (!payload_included(root) || !runtime_loadable(root))
        io_error("Phi-3 wdmlpack is not a runtime-loadable payload package: " + pk.file->path);
    const Json *dir = root.get("tensors");
    if (dir && dir->kind == Json::Arr)
        for (const Json &e : dir->a) {
            const std::string n = string_value(e.get("name"));
            if (n.size() > kQweight.size() && n.compare(n.size() - kQweight.size(), kQweight.size(), kQweight) == 0) {
                const std::string role = n.substr(0, n.size() - kQweight.size());
                bool seen = false;
                for (const std::string &r : pk.names) seen |= r == role;
                if (!seen) pk.names.push_back(role);
            }
        }
}

Triplet resolve_phi3(const mnb_pack &pk, const std::string &role) {
    const Tensor &q = phi3_require(pk, role + kQweight);
    if (q.dims.size() != 3)
        io_error(fmt("Phi-3 qweight '%s' must encode dims [N,K,blockSize], got %zu dims", role.c_str(), q.dims.size()));
    const Tensor &zp = phi3_require(pk, role + kZeropoints);
    const Tensor &sc = phi3_require(pk, role + kScales);
    Triplet t;
    t.N = (int32_t)q.dims[0];
    t.K = (int32_t)q.dims[1];
    t.bs = (int32_t)q.dims[2];
    t.kb = t.bs != 0 ? t.K / t.bs : 0;
    t.q = q.raw;
    t.q_bytes = q.raw_len;
    t.scales.resize((size_t)(sc.raw_len / 4));
    copy_bytes(t.scales.data(), sc.raw, t.scales.size() * 4);
    t.scale_dtype = kOnnxFloat;
    t.zp = zp.raw;
    t.zp_bytes = zp.raw_len;
    return t;
}

// --- graph sources: ONNX models and Qwen payload packages ------------------
void add_matmul_nodes(mnb_pack &pk, const std::vector<Node> &nodes) {  // Q2W:534-545
    for (const Node &n : nodes) {
        if (n.op_type != "MatMulNBits") continue;
        if (n.outputs.empty() || n.inputs.size() < 3)
            io_error(fmt("MatMulNBits node has %zu inputs and %zu outputs; expected at least 3 inputs and 1 output",
                         n.inputs.size(), n.outputs.size()));
        const std::string &out = n.outputs[0];
        // An empty name marks an omitted optional input in ONNX.
        std::vector<std::string> names = {n.inputs[1], n.inputs[2], n.inputs.size() > 3 ? n.inputs[3] : std::string()};
        if (!pk.triplets.count(out)) pk.names.push_back(out);
        pk.triplets[out] = std::move(names);
    }
}

bool find_dtype(const mnb_pack &pk, const std::string &name, int32_t &dtype) {  // Q2W:2119-2131
    if (const Tensor *e = pk.find_ext(name)) {
        dtype = e->dtype;
        return true;
    }
    const Tensor *t = pk.find_inline(name);
    if (t && t->has_inline()) {
        dtype = t->dtype;
        return true;
    }
    return false;
}

void require_dtype(const mnb_pack &pk, const std::string &name, const char *kind, int32_t a, int32_t b) {
    int32_t dt = 0;
    if (!find_dtype(pk, name, dt)) io_error(std::string("Required ") + kind + " tensor not found: " + name);
    if (dt != a && dt != b)
        io_error(fmt("Tensor '%s' has unsupported data type %s (%d)", name.c_str(), onnx_type_name(dt), dt));
}

void validate_graph_types(const mnb_pack &pk) {  // Q2W:2063-2080
    if (pk.ext_refs.empty() && pk.inline_tensors.empty())
        io_error("No ONNX tensor initializers found in selected model file");
    for (const std::string &w : pk.names) {
        const std::vector<std::string> &t = pk.triplets.at(w);
        require_dtype(pk, t[0], "quantized weight", kOnnxUint8, kOnnxInt8);
        require_dtype(pk, t[1], "quantized scale", kOnnxFloat16, kOnnxFloat);
        if (!t[2].empty()) require_dtype(pk, t[2], "quantized zero-point", kOnnxUint8, kOnnxInt8);
    }
}

struct RawView {
    const uint8_t *data = nullptr;
    int64_t len = 0;
    std::vector<int64_t> dims;
    int32_t dtype = 0;
};

const uint8_t *ext_bytes(const mnb_pack &pk, const Tensor &e) {
    if (!pk.ext_file) io_error("External tensor data is unavailable for " + e.name);
    int64_t end = 0;
    if (e.ext_offset < 0 || e.ext_length < 0 || __builtin_add_overflow(e.ext_offset, e.ext_length, &end) ||
        end > pk.ext_file->size)
        io_error(fmt("External tensor %s lies outside %s: offset=%lld, length=%lld, fileSize=%lld", e.name.c_str(),
                     pk.ext_file->path.c_str(), (long long)e.ext_offset, (long long)e.ext_length,
                     (long long)pk.ext_file->size));
    return pk.ext_file->data + e.ext_offset;
}

bool resolve_raw(const mnb_pack &pk, const std::string &name, RawView &v) {  // Q2W:1576-1592
    if (const Tensor *e = pk.find_ext(name)) {
        v.data = ext_bytes(pk, *e);
        v.len = e->ext_length;
        v.dims = e->dims;
        v.dtype = e->dtype;
        return true;
    }
    const Tensor *t = pk.find_inline(name);
    if (t && t->raw_len > 0) {
        v.data = t->raw;
        v.len = t->raw_len;
        v.dims = t->dims;
        v.dtype = t->dtype;
        return true;
    }
    return false;
}

void widen_fp16(const uint8_t *p, int64_t count, std::vector<float> &out) {
    out.resize((size_t)count);
    for (int64_t i = 0; i < count; ++i) out[(size_t)i] = ref_fp16_to_fp32(le<uint16_t>(p + 2 * i));
}

bool resolve_float(const mnb_pack &pk, const std::string &name, std::vector<float> &out, int32_t &dtype) {
    if (const Tensor *e = pk.find_ext(name)) {  // Q2W:1683-1695
        const uint8_t *p = ext_bytes(pk, *e);
        dtype = e->dtype;
        if (e->dtype == kOnnxFloat16) {
            widen_fp16(p, e->ext_length / 2, out);
        } else if (e->dtype == kOnnxFloat) {
            out.resize((size_t)(e->ext_length / 4));
            copy_bytes(out.data(), p, out.size() * 4);
        } else {
            io_error(fmt("Unsupported tensor data type for %s: %s (%d). Supported: FLOAT16, FLOAT", name.c_str(),
                         onnx_type_name(e->dtype), e->dtype));
        }
        return true;
    }
    const Tensor *t = pk.find_inline(name);
    if (!(t && t->has_inline())) return false;
    dtype = t->dtype;
    if (t->dtype == kOnnxFloat) {  // Q2W:1612-1630
        if (!t->floats.empty()) {
            out = t->floats;
            return true;
        }
        if (t->raw_len > 0) {
            out.resize((size_t)(t->raw_len / 4));
            copy_bytes(out.data(), t->raw, out.size() * 4);
            return true;
        }
    } else if (t->dtype == kOnnxFloat16 && t->raw_len > 0) {
        widen_fp16(t->raw, t->raw_len / 2, out);
        return true;
    }
    io_error(fmt("Unsupported inline tensor data for %s: %s (%d)", name.c_str(), onnx_type_name(t->dtype), t->dtype));
}

// Zero points -> the flat nibble stream (Q2W:986-1112).
void zp_repack_row_padded(const uint8_t *src, int64_t len, const std::string &name, int64_t rows, int64_t bpr,
                          int64_t row_bytes, Triplet &t) {
    const int64_t expected = rows * row_bytes;
    if (len < expected)
        io_error(fmt("Zero-point tensor %s is truncated: %lld bytes, expected at least %lld", name.c_str(),
                     (long long)len, (long long)expected));
    t.zp_owned.assign((size_t)((rows * bpr + 1) / 2), 0);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < bpr; ++b) put_nibble(t.zp_owned, r * bpr + b, get_nibble(src, r * row_bytes * 2 + b));
}

void zp_pack_unpacked(const uint8_t *src, int64_t len, const std::string &name, int64_t count, Triplet &t) {
    if (len < count)
        io_error(fmt("Zero-point tensor %s is truncated: %lld values, expected %lld", name.c_str(), (long long)len,
                     (long long)count));
    t.zp_owned.assign((size_t)((count + 1) / 2), 0);
    for (int64_t i = 0; i < count; ++i) put_nibble(t.zp_owned, i, src[i] & 0xF);
}

// No zero-point tensor: every zero point is 8, the stream 0x88... (Q2W:1107-1112).
void set_default_zero_points(Triplet &t, int64_t count) {
    t.zp_owned.assign((size_t)((count + 1) / 2), 0x88);
    t.zp = t.zp_owned.data();
    t.zp_bytes = (int64_t)t.zp_owned.size();
    t.zp_implicit = true;
}

void resolve_zero_points(const mnb_pack &pk, const std::string &name, Triplet &t) {
    const int64_t rows = t.N, bpr = t.kb, count = rows * bpr;
    int32_t dtype = 0;
    if (name.empty() || !find_dtype(pk, name, dtype)) {
        set_default_zero_points(t, count);
        return;
    }
    if (dtype == kOnnxFloat || dtype == kOnnxFloat16) {  // Q2W:1002-1008, 1092-1105
        std::vector<float> v;
        int32_t dt = 0;
        if (!resolve_float(pk, name, v, dt)) {
            set_default_zero_points(t, count);
            return;
        }
        if ((int64_t)v.size() < count)
            io_error(fmt("Zero-point tensor %s is truncated: %zu values, expected %lld", name.c_str(), v.size(),
                         (long long)count));
        t.zp_owned.assign((size_t)((count + 1) / 2), 0);
        for (int64_t i = 0; i < count; ++i) {
            const int r = java_round_f(v[(size_t)i]);
            put_nibble(t.zp_owned, i, r < 0 ? 0 : (r > 15 ? 15 : r));
        }
    } else {
        RawView z;
        if (!resolve_raw(pk, name, z)) {
            set_default_zero_points(t, count);
            return;
        }
        const int64_t flat_bytes = (count + 1) / 2, row_bytes = (bpr + 1) / 2, row_total = rows * row_bytes;
        if (z.dims.size() == 2 && z.dims[0] == rows && z.dims[1] == row_bytes) {
            zp_repack_row_padded(z.data, z.len, name, rows, bpr, row_bytes, t);
        } else if (z.dims.size() == 2 && z.dims[0] == rows && z.dims[1] == bpr) {
            zp_pack_unpacked(z.data, z.len, name, count, t);
        } else if (z.len == row_total && row_total != flat_bytes) {
            zp_repack_row_padded(z.data, z.len, name, rows, bpr, row_bytes, t);
        } else if (z.len == flat_bytes) {
            t.zp = z.data;
            t.zp_bytes = z.len;
            return;
        } else if (z.len == count) {
            zp_pack_unpacked(z.data, z.len, name, count, t);
        } else {
            io_error(fmt("Unexpected zero-point layout for %s: dims=%s, bytes=%lld, expected packed row layout [%lld, "
                         "%lld], flat packed bytes %lld, or unpacked [%lld, %lld]",
                         name.c_str(), dims_text(z.dims).c_str(), (long long)z.len, (long long)rows,
                         (long long)row_bytes, (long long)flat_bytes, (long long)rows, (long long)bpr));
        }
    }
    t.zp = t.zp_owned.data();
    t.zp_bytes = (int64_t)t.zp_owned.size();
}

Triplet resolve_graph(const mnb_pack &pk, const std::string &weight) {  // Q2W:936-976
    const std::vector<std::string> &names = pk.triplets.at(weight);
    const std::string &qn = names[0], &sn = names[1];
    RawView q;
    const bool have_q = resolve_raw(pk, qn, q);
    Triplet t;
    const bool have_s = resolve_float(pk, sn, t.scales, t.scale_dtype);
    if (!have_q) io_error("Quantized weight not found: " + qn);
    if (!have_s) io_error("Scale not found: " + sn);
    if (q.dims.size() < 3)
        io_error("Unexpected dimensions for quantized weight " + qn + ": " + dims_text(q.dims) +
                 ", expected [N, blocks, packedBlock]");
    // Dimensions that are not positive 32-bit values, or more blocks than the
    // packed bytes hold, are refused before anything is sized from them.
    const int64_t lim = std::numeric_limits<int32_t>::max();
    if (q.dims[0] < 1 || q.dims[1] < 1 || q.dims[2] < 1 || q.dims[0] > lim || q.dims[1] > lim || q.dims[2] > lim / 2 ||
        q.dims[1] * q.dims[2] * 2 > lim)
        io_error("Unexpected dimensions for quantized weight " + qn + ": " + dims_text(q.dims) +
                 ", expected [N, blocks, packedBlock]");
    if (q.len / q.dims[0] / q.dims[1] < q.dims[2])
        io_error(fmt("Quantized weight %s holds %lld bytes, fewer than its dims %s need", qn.c_str(), (long long)q.len,
                     dims_text(q.dims).c_str()));
    t.N = (int32_t)q.dims[0];
    t.kb = (int32_t)q.dims[1];
    t.bs = (int32_t)(q.dims[2] * 2);
    t.K = t.kb * t.bs;
    if ((int64_t)t.scales.size() != (int64_t)t.N * t.kb)
        io_error(fmt("Unexpected scale tensor size for %s: %zu, expected %lld for quantized weight %s", sn.c_str(),
                     t.scales.size(), (long long)t.N * t.kb, qn.c_str()));
    t.q = q.data;
    t.q_bytes = q.len;
    resolve_zero_points(pk, names[2], t);
    return t;
}

Triplet resolve(const mnb_pack &pk, const char *name) {
    if (!name) io_error("weight name must not be null");
    const std::string n(name);
    if (pk.kind == MNB_PACK_PHI3) {
        bool known = false;
        for (const std::string &r : pk.names) known |= r == n;
        if (!known) io_error("Phi-3 wdmlpack is missing payload tensor: " + n + kQweight);
        return resolve_phi3(pk, n);
    }
    if (!pk.triplets.count(n)) io_error("Quantized weight not found: " + n);
    return resolve_graph(pk, n);
}

// --- ONNX model -------------------------------------------------------------
void open_onnx(mnb_pack &pk) {
    const MappedFile &f = *pk.file;
    std::vector<Node> nodes;
    bool have_graph = false;
    Pb m{f.data, f.data + f.size};
    const uint8_t *file_end = f.data + f.size;
    try {
        while (m.more()) {  // ModelProto
            const uint64_t tag = m.varint();
            const uint32_t fld = (uint32_t)(tag >> 3), wt = (uint32_t)(tag & 7);
            if (fld == 7 && wt == 2) {  // graph
                Pb g = m.sub();
                have_graph = true;
                nodes.clear();
                pk.ext_refs.clear();
                pk.inline_tensors.clear();
                while (g.more()) {
                    const uint64_t gt = g.varint();
                    const uint32_t gf = (uint32_t)(gt >> 3), gw = (uint32_t)(gt & 7);
                    if (gf == 1 && gw == 2) {
                        nodes.push_back(parse_node(g.sub()));
                    } else if (gf == 5 && gw == 2) {
                        Tensor t = parse_tensor(g.sub(), file_end);
                        if (t.external) {
                            Tensor ref;
                            ref.name = t.name;
                            ref.dtype = t.dtype;
                            ref.dims = t.dims;
                            ref.external = true;
                            ref.ext_offset = t.ext_offset;
                            ref.ext_length = t.ext_length;
                            pk.ext_refs[t.name] = std::move(ref);
                        }
                        std::string key = t.name;
                        pk.inline_tensors[key] = std::move(t);
                    } else {
                        g.skip(gw);
                    }
                }
            } else {
                m.skip(wt);
            }
        }
    } catch (const std::runtime_error &e) {
        if (dynamic_cast<const IoError *>(&e)) throw;
        io_error(fmt("Failed to parse ONNX model '%s' at byte offset %lld of %lld (%s)", f.path.c_str(),
                     (long long)(m.p - f.data), (long long)f.size, e.what()));
    }
    if (!have_graph) io_error("No graph found in ONNX model");
    add_matmul_nodes(pk, nodes);
    if (!pk.ext_refs.empty()) {
        const std::string dir = dir_of(f.path);
        std::string data = dir + "/model.onnx_data";
        if (!file_exists(data)) data = dir + "/model.onnx.data";
        if (!file_exists(data))
            io_error("Required file missing: model.onnx_data (or model.onnx.data) (looked in " + dir + ")");
        pk.ext_file.reset(new MappedFile(data));
    }
    pk.kind = MNB_PACK_ONNX;
    validate_graph_types(pk);
}

// --- Qwen packages (QwenWdmlPackModelSource.java:59-185) ------------------
std::string lower(std::string s) {
    for (char &c : s) c = (char)((c >= 'A' && c <= 'Z') ? c - 'A' + 'a' : c);
    return s;
}

void open_qwen2(mnb_pack &pk, const Json &root, const PackHeader &h) {
    if (!runtime_loadable(root))
        io_error("wdmlpack package is import-only and not runtime-loadable yet: " + string_value(root.get("runtimeLoadMode")));
    if (!payload_included(root)) {
        // manifest-only: the tensors live in the source ONNX model (QWS:76-86,
        // WdmlPackManifest.java:89-100, RuntimeModelPackage.java:112-123)
        const Json *src = root.get("source");
        if (!src || src->kind != Json::Obj) io_error("Invalid wdmlpack: missing source metadata");
        std::string cand = string_value(src->get("relativePath"));
        if (is_blank(cand)) cand = string_value(src->get("fileName"));
        if (is_blank(cand)) cand = "model.onnx";
        if (cand.empty() || cand[0] == '/' || cand == ".." || cand.rfind("../", 0) == 0 ||
            cand.find("/../") != std::string::npos || (cand.size() >= 3 && cand.compare(cand.size() - 3, 3, "/..") == 0))
            io_error("Invalid wdmlpack source path escapes model directory: " + cand);
        const std::string path = dir_of(pk.file->path) + "/" + cand;
        if (!file_exists(path)) io_error("wdmlpack source is missing: " + path);
        const int64_t expected = long_value(src->get("sizeBytes"), -1);
        std::unique_ptr<MappedFile> onnx(new MappedFile(path));
        if (expected >= 0 && expected != onnx->size)
            io_error(fmt("wdmlpack source size mismatch for %s: manifest=%lld, actual=%lld",
                         cand.substr(cand.find_last_of('/') + 1).c_str(), (long long)expected, (long long)onnx->size));
        pk.file = std::move(onnx);
        open_onnx(pk);
        return;
    }
    map_payload_tensors(pk, root, h);
    for (auto &kv : pk.tensors) pk.inline_tensors[kv.first] = kv.second;
    std::vector<Node> nodes;
    const Json *g = root.get("runtimeGraph");
    const Json *list = g ? g->get("nodes") : nullptr;
    if (list && list->kind == Json::Arr)
        for (const Json &e : list->a) {
            if (e.kind != Json::Obj) continue;
            Node n;
            n.op_type = string_value(e.get("opType"));
            n.inputs = string_list(e.get("inputs"));
            n.outputs = string_list(e.get("outputs"));
            if (!is_blank(n.op_type)) nodes.push_back(std::move(n));
        }
    add_matmul_nodes(pk, nodes);
    pk.kind = MNB_PACK_QWEN2;
    validate_graph_types(pk);
}

void open_wdmlpack(mnb_pack &pk) {
    const PackHeader h = read_header(*pk.file);
    const Json root = read_manifest(*pk.file, h);
    validate_root(root, h);
    const Json *arch = root.get("architecture");
    if (arch && arch->kind == Json::Str && arch->s == "phi3") {
        pk.kind = MNB_PACK_PHI3;
        open_phi3(pk, root);
        map_payload_tensors(pk, root, h);
        return;
    }
    const Json *model = root.get("model");
    const Json *march = model ? model->get("architecture") : nullptr;
    if (model && model->kind == Json::Obj && lower(value_text(march)) == "qwen2") {
        open_qwen2(pk, root, h);
        return;
    }
    io_error("Unsupported wdmlpack architecture: " + value_text(march ? march : arch) +
             " (this loader reads architecture phi3 and model.architecture qwen2): " + pk.file->path);
}

// --- SafeTensors container (SafeTensorsReader.java:84-277) -----------------
// An 8-byte little-endian header length, a JSON directory {name: {dtype,
// shape, data_offsets}, "__metadata__": ...}, then the tensor bytes.  The
// reference checks each entry in this order and with these messages.
int32_t st_bytes_per_element(const std::string &dt) {  // SafeTensorsReader.java:248-256
    if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    if (dt == "I8" || dt == "U8" || dt == "BOOL") return 1;
    io_error("Unsupported SafeTensors dtype: " + dt);
}

int32_t st_onnx_type(const std::string &dt) {  // SafeTensorsReader.java:258-276
    static const std::pair<const char *, int32_t> kTypes[] = {
        {"F32", 1}, {"U8", 2}, {"I8", 3}, {"I32", 6}, {"I64", 7}, {"F16", 10}, {"BF16", 16},
        {"BOOL", 9}, {"F64", 11}, {"I16", 5}, {"U16", 4}, {"U32", 12}, {"U64", 13}};
    for (const auto &t : kTypes)
        if (dt == t.first) return t.second;
    io_error("Unsupported SafeTensors dtype: " + dt);
}

std::string base_name(const std::string &p) {
    const size_t s = p.find_last_of('/');
    return s == std::string::npos ? p : p.substr(s + 1);
}

// Jackson's canConvertToLong: integers that fit 64 bits, and reals inside the
// long range (converted by truncation, as asLong does).
bool st_long_array(const Json *v, std::vector<int64_t> &out) {
    out.clear();
    for (const Json &e : v->a) {
        if (e.kind == Json::Int) {
            out.push_back(e.i);
        } else if (e.kind == Json::Real && e.d >= -9223372036854775808.0 && e.d <= 9223372036854775807.0) {
            out.push_back(java_d2l(e.d));
        } else {
            return false;
        }
    }
    return true;
}

void open_safetensors(mnb_pack &pk) {
    const MappedFile &f = *pk.file;
    const std::string fname = base_name(f.path);
    if (f.size < 8) io_error("Invalid SafeTensors file: too small: " + f.path);
    const int64_t hlen = le<int64_t>(f.data);
    if (hlen < 2 || hlen > f.size - 8) io_error(fmt("Invalid SafeTensors header length for %s: %lld", fname.c_str(), (long long)hlen));
    if (8 + hlen > 2147483647LL) io_error(fmt("SafeTensors header too large for current reader: %lld", (long long)hlen));
    const Json root = JsonReader((const char *)f.data + 8, (size_t)hlen, "SafeTensors header").document();
    const int64_t base = 8 + hlen;
    pk.kind = MNB_PACK_SAFETENSORS;
    if (root.kind != Json::Obj) return;   // a directory that is not an object lists no tensors
    // members in file order; a repeated name keeps its first position and its last value
    std::vector<std::string> order;
    std::unordered_map<std::string, const Json *> entry;
    for (const auto &m : root.o) {
        if (!entry.count(m.first)) order.push_back(m.first);
        entry[m.first] = &m.second;
    }
    for (const std::string &name : order) {
        if (name == "__metadata__") continue;
        const Json &node = *entry[name];
        if (node.kind != Json::Obj) io_error("Invalid SafeTensors tensor entry for " + name + " in " + fname);
        const Json *dt = node.get("dtype");
        if (!dt || dt->kind != Json::Str)
            io_error("Invalid SafeTensors tensor " + name + " in " + fname + ": missing textual dtype");
        std::string dtype = dt->s;
        for (char &c : dtype) c = (char)toupper((unsigned char)c);
        std::vector<int64_t> shape, offsets;
        for (const char *field : {"shape", "data_offsets"}) {
            const Json *v = node.get(field);
            if (!v || v->kind != Json::Arr)
                io_error("Invalid SafeTensors tensor " + name + " in " + fname + ": missing array " + field);
            if (!st_long_array(v, strcmp(field, "shape") == 0 ? shape : offsets))
                io_error("Invalid SafeTensors tensor " + name + " in " + fname + ": non-integer " + field);
        }
        if (offsets.size() != 2) io_error("Invalid SafeTensors data_offsets for " + name + " in " + fname);
        const int64_t begin = offsets[0], end = offsets[1];
        if (begin < 0 || end < begin)
            io_error(fmt("Invalid SafeTensors data range for %s: [%lld, %lld]", name.c_str(), (long long)begin,
                         (long long)end));
        int64_t abs_begin = 0, abs_end = 0;
        if (__builtin_add_overflow(base, begin, &abs_begin) || __builtin_add_overflow(base, end, &abs_end) ||
            abs_end > f.size)
            io_error(fmt("SafeTensors data range for %s escapes file bounds: [%lld, %lld] fileSize=%lld", name.c_str(),
                         (long long)begin, (long long)end, (long long)f.size));
        int64_t elements = 1;
        for (int64_t d : shape) {
            if (d < 0)
                io_error(fmt("Invalid negative dimension for SafeTensors tensor %s in %s: %lld", name.c_str(),
                             fname.c_str(), (long long)d));
            if (__builtin_mul_overflow(elements, d, &elements)) io_error("long overflow");
        }
        int64_t expected = 0;
        if (__builtin_mul_overflow(elements, (int64_t)st_bytes_per_element(dtype), &expected)) io_error("long overflow");
        if (expected != end - begin)
            io_error(fmt("SafeTensors byte length mismatch for %s in %s: expected %lld bytes from dtype/shape, got %lld",
                         name.c_str(), fname.c_str(), (long long)expected, (long long)(end - begin)));
        Tensor t;
        t.name = name;
        t.dtype = st_onnx_type(dtype);
        t.dims = shape;
        t.raw = f.data + abs_begin;
        t.raw_len = end - begin;
        pk.names.push_back(name);
        pk.inline_tensors[name] = std::move(t);
    }
}

// Runs one entry point's body: IoError -> MNB_ERR_IO with its text, host
// allocation failure -> MNB_ERR_OUT_OF_MEMORY.
template <class F>
int32_t guarded(F &&body) {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return mnb::report(MNB_ERR_OUT_OF_MEMORY, "out of host memory while reading the weight file");
    } catch (const std::exception &e) {
        return mnb::report(MNB_ERR_IO, e.what());
    }
}

int32_t copy_name(const std::string &n, char *buf, int64_t cap, int64_t *length) {
    if (length) *length = (int64_t)n.size();
    if (buf && cap > 0) {
        const size_t k = std::min((size_t)(cap - 1), n.size());
        memcpy(buf, n.data(), k);
        buf[k] = '\0';
    }
    return MNB_OK;
}

}  // namespace

extern "C" {

int32_t mnb_pack_open(const char *path, mnb_pack **out) {
    if (!out) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!path) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "path must not be null");
    return guarded([&] {
        std::unique_ptr<mnb_pack> pk(new mnb_pack());
        pk->file.reset(new MappedFile(path));
        const std::string p(path);
        auto ends_with = [&](const std::string &ext) {
            return p.size() >= ext.size() && p.compare(p.size() - ext.size(), ext.size(), ext) == 0;
        };
        if (ends_with(".wdmlpack") || (pk->file->size >= 8 && memcmp(pk->file->data, "WDMLPACK", 8) == 0))
            open_wdmlpack(*pk);
        else if (ends_with(".safetensors"))
            open_safetensors(*pk);
        else
            open_onnx(*pk);
        *out = pk.release();
        return MNB_OK;
    });
}

int32_t mnb_pack_close(mnb_pack *pack) {
    delete pack;
    return MNB_OK;
}

int32_t mnb_pack_kind(const mnb_pack *pack, int32_t *kind) {
    if (!pack || !kind) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack and kind must not be null");
    *kind = pack->kind;
    return MNB_OK;
}

int32_t mnb_pack_weight_count(const mnb_pack *pack, int32_t *count) {
    if (!pack || !count) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack and count must not be null");
    *count = (int32_t)pack->names.size();
    return MNB_OK;
}

int32_t mnb_pack_weight_name(const mnb_pack *pack, int32_t index, char *buf, int64_t cap, int64_t *length) {
    if (!pack) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack must not be null");
    if (index < 0 || (size_t)index >= pack->names.size())
        return mnb::report(MNB_ERR_INVALID_ARGUMENT,
                           fmt("weight index %d out of range [0, %zu)", index, pack->names.size()).c_str());
    return copy_name(pack->names[(size_t)index], buf, cap, length);
}

int32_t mnb_pack_find_projection(const mnb_pack *pack, int32_t layer, const char *projection, char *buf, int64_t cap,
                                 int64_t *length) {
    if (!pack || !projection) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack and projection must not be null");
    const std::string prefix = "layers." + std::to_string(layer);
    for (const std::string &n : pack->names) {
        if (pack->kind == MNB_PACK_SAFETENSORS) break;   // dense tensors only: no quantized weights
        if (n.find(prefix) != std::string::npos && n.find(projection) != std::string::npos)
            return copy_name(n, buf, cap, length);
    }
    return mnb::report(MNB_ERR_IO, fmt("Quantized weight not found for layer %d %s", layer, projection).c_str());
}

int32_t mnb_pack_weight_info(const mnb_pack *pack, const char *name, mnb_triplet_info *out) {
    if (!pack || !out) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack and out must not be null");
    return guarded([&] {
        const Triplet t = resolve(*pack, name);
        mnb_triplet_info i{};
        i.N = t.N;
        i.K = t.K;
        i.block_size = t.bs;
        i.blocks_per_row = t.kb;
        i.q_bytes = t.q_bytes;
        i.scale_count = (int64_t)t.scales.size();
        i.zp_bytes = t.zp_bytes;
        i.zp_implicit = t.zp_implicit ? 1 : 0;
        i.scale_dtype = t.scale_dtype;
        *out = i;
        return MNB_OK;
    });
}

int32_t mnb_pack_read_weight(const mnb_pack *pack, const char *name, uint8_t *q, int64_t q_cap, float *scales,
                             int64_t scale_cap, uint8_t *zp, int64_t zp_cap) {
    if (!pack || !q || !scales) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack, q and scales must not be null");
    return guarded([&] {
        const Triplet t = resolve(*pack, name);
        const int64_t zb = t.zp_bytes;
        if (q_cap < t.q_bytes || scale_cap < (int64_t)t.scales.size() || zp_cap < zb || (zb > 0 && !zp))
            return mnb::report(MNB_ERR_INVALID_ARGUMENT,
                               fmt("buffers too small for %s: need q %lld, scales %zu, zero points %lld bytes", name,
                                   (long long)t.q_bytes, t.scales.size(), (long long)zb)
                                   .c_str());
        copy_bytes(q, t.q, (size_t)t.q_bytes);
        copy_bytes(scales, t.scales.data(), t.scales.size() * 4);
        if (zb > 0) memcpy(zp, t.zp, (size_t)zb);
        return MNB_OK;
    });
}

int32_t mnb_pack_tensor_info(const mnb_pack *pack, const char *name, int32_t *dtype, int64_t *dims, int32_t dims_cap,
                             int32_t *ndims) {
    if (!pack || !name || !dtype || !ndims)
        return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack, name, dtype and ndims must not be null");
    return guarded([&] {
        const Tensor *t = pack->find_ext(name);
        if (!t) t = pack->find_inline(name);
        if (!t) {
            auto it = pack->tensors.find(name);
            if (it != pack->tensors.end()) t = &it->second;
        }
        if (!t) io_error(std::string("Tensor not found: ") + name);
        *dtype = t->dtype;
        *ndims = (int32_t)t->dims.size();
        for (int32_t i = 0; i < *ndims && i < dims_cap && dims; ++i) dims[i] = t->dims[(size_t)i];
        return MNB_OK;
    });
}

int32_t mnb_pack_weight_quantize(mnb_context *ctx, const mnb_pack *pack, const char *name, int32_t rows, int32_t cols,
                                 int32_t block_size, mnb_weight **out) {
    if (!out) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!pack || !name) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack and name must not be null");
    std::vector<float> data;
    const int32_t rr = guarded([&] {
        const Tensor *t = pack->find_ext(name);
        if (!t) t = pack->find_inline(name);
        if (!t) io_error(std::string("Tensor not found: ") + name);
        // Qwen2Weights.validateMatrixShape (Q2W:1637-1642)
        if (!(t->dims.size() == 2 && t->dims[0] == rows && t->dims[1] == cols)) {
            std::string d = "[";
            for (size_t i = 0; i < t->dims.size(); ++i) d += (i ? ", " : "") + std::to_string(t->dims[i]);
            io_error(fmt("Unexpected dimensions for %s: %s], expected [%d, %d]", name, d.c_str(), rows, cols));
        }
        // the embedding table's values: FLOAT as stored, FLOAT16 through the
        // reference's fp16ToFp32 (Q2W:200-270, 599-704); other types refused
        int32_t dt = 0;
        if (!resolve_float(*pack, name, data, dt)) io_error(std::string("Tensor has no data: ") + name);
        if ((int64_t)data.size() != (int64_t)rows * cols)
            io_error(fmt("Tensor %s holds %zu values, expected %lld", name, data.size(), (long long)rows * cols));
        return MNB_OK;
    });
    if (rr != MNB_OK) return rr;
    const int32_t rc = mnb_weight_quantize(ctx, data.data(), MNB_F32, rows, cols, block_size, MNB_HOST_MEMORY, out);
    if (rc != MNB_OK) {
        const std::string msg = std::string(name) + ": " + mnb_last_error();
        return mnb::report(rc, msg.c_str());
    }
    return MNB_OK;
}

int32_t mnb_pack_weight_create(mnb_context *ctx, const mnb_pack *pack, const char *name, mnb_weight **out) {
    if (!out) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!pack) return mnb::report(MNB_ERR_INVALID_ARGUMENT, "pack must not be null");
    Triplet t;
    const int32_t rr = guarded([&] {
        t = resolve(*pack, name);
        return MNB_OK;
    });
    if (rr != MNB_OK) return rr;
    // A stream of all-8 nibbles is the implicit zero point.
    const int64_t blocks = (int64_t)t.N * (t.bs > 0 ? (t.K + t.bs - 1) / t.bs : 0);
    bool all8 = t.zp_implicit;
    if (!all8 && t.zp && blocks > 0 && t.zp_bytes >= (blocks + 1) / 2) {
        all8 = true;
        for (int64_t i = 0; i < blocks && all8; ++i) all8 = get_nibble(t.zp, i) == 8;
    }
    const int32_t rc = mnb_weight_create(ctx, t.N, t.K, t.bs, 4, t.q, t.q_bytes, t.scales.data(), MNB_F32,
                                         (int64_t)t.scales.size(), all8 ? nullptr : t.zp, all8 ? 0 : t.zp_bytes,
                                         all8 ? MNB_ZP_NONE : MNB_ZP_FLAT, 0, out);
    if (rc != MNB_OK) {
        const std::string msg = std::string(name) + ": " + mnb_last_error();
        return mnb::report(rc, msg.c_str());
    }
    return MNB_OK;
}

}  // extern "C"
