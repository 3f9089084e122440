// MLX checkpoint loader (include/qmr_checkpoint.h): safetensors shards with
// MLX affine quantisation metadata, memory-mapped and validated once at open,
// then read per matrix into host arrays or uploaded straight into device
// buffers (the codes go from the mapped shard to HBM without a host copy).
//
// Behaviour follows the reference's Checkpoint (src/weights.rs:32-486,
// 569-738) and Matrix::load (src/engine.rs:48-135): the same validation,
// name canonicalisation, quantisation lookup, exact metadata expansion and
// error texts. The model-level parts of that Checkpoint (ModelConfig
// validation, norm sanitising, conv layouts, vectors) are not on the matrix
// path and are not restated here.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <optional>
#include <set>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/qmr_checkpoint.h"
#include "contract.hpp"

namespace {

using qmr::Error;

[[noreturn]] void fail(const std::string &message) { throw Error{QMR_ERR_INVALID, message}; }

void ensure(bool ok, const std::string &message) {
    if (!ok) fail(message);
}

template <typename F>
int guarded(F &&f) {
    try {
        qmr::clear_error();
        return f();
    } catch (const Error &e) {
        return qmr::record_error(e.code, e.message);
    } catch (const std::bad_alloc &) {
        return qmr::record_error(QMR_ERR_INVALID, "host allocation failed");
    } catch (const std::exception &e) {
        return qmr::record_error(QMR_ERR_INVALID, e.what());
    }
}

bool starts_with(const std::string &s, const char *p) { return s.compare(0, std::strlen(p), p) == 0; }

bool ends_with(const std::string &s, const char *p) {
    const size_t n = std::strlen(p);
    return s.size() >= n && s.compare(s.size() - n, n, p) == 0;
}

// ---- JSON ----------------------------------------------------------------
// RFC 8259 values. Safetensors headers are parsed with duplicate keys
// rejected at every depth (the reference's StrictJson, src/weights.rs:493-566);
// config and index files keep the last duplicate, as serde_json::Value does.

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool boolean = false;
    bool is_u64 = false;  // a non-negative integer literal that fits in 64 bits
    uint64_t u64 = 0;
    std::string str;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;

    const Json *get(const std::string &key) const {
        if (kind != Object) return nullptr;
        for (auto it = members.rbegin(); it != members.rend(); ++it)
            if (it->first == key) return &it->second;
        return nullptr;
    }
    std::optional<uint64_t> as_u64() const {
        if (kind == Number && is_u64) return u64;
        return std::nullopt;
    }
    const std::string *as_str() const { return kind == String ? &str : nullptr; }
};

class JsonParser {
  public:
    JsonParser(const char *p, size_t n, bool strict) : p_(p), end_(p + n), strict_(strict) {}

    Json parse_document() {
        validate_utf8();
        skip_ws();
        Json v = value(0);
        skip_ws();
        if (p_ != end_) error("trailing characters");
        return v;
    }

  private:
    const char *p_;
    const char *end_;
    bool strict_;

    [[noreturn]] void error(const char *what) { fail(std::string("invalid JSON: ") + what); }

    void validate_utf8() {
        const auto *s = reinterpret_cast<const unsigned char *>(p_);
        const auto *e = reinterpret_cast<const unsigned char *>(end_);
        while (s < e) {
            const unsigned c = *s;
            size_t n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
            if (n == 0 || size_t(e - s) < n) error("invalid UTF-8");
            uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1f) : n == 3 ? (c & 0x0f) : (c & 0x07);
            for (size_t i = 1; i < n; ++i) {
                if ((s[i] & 0xc0) != 0x80) error("invalid UTF-8");
                cp = (cp << 6) | (s[i] & 0x3f);
            }
            static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
            if (cp < kMin[n] || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) error("invalid UTF-8");
            s += n;
        }
    }

    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }

    bool literal(const char *word) {
        const size_t n = std::strlen(word);
        if (size_t(end_ - p_) >= n && std::memcmp(p_, word, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }

    Json value(int depth) {
        if (depth > 128) error("recursion limit exceeded");
        if (p_ == end_) error("unexpected end");
        Json v;
        switch (*p_) {
            case '{': object(v, depth); break;
            case '[': array(v, depth); break;
            case '"':
                v.kind = Json::String;
                v.str = string();
                break;
            case 't':
                if (!literal("true")) error("expected value");
                v.kind = Json::Bool;
                v.boolean = true;
                break;
            case 'f':
                if (!literal("false")) error("expected value");
                v.kind = Json::Bool;
                break;
            case 'n':
                if (!literal("null")) error("expected value");
                break;
            default: number(v); break;
        }
        return v;
    }

    void object(Json &v, int depth) {
        v.kind = Json::Object;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == '}') {
            ++p_;
            return;
        }
        std::set<std::string> seen;
        for (;;) {
            skip_ws();
            if (p_ == end_ || *p_ != '"') error("expected key");
            std::string key = string();
            if (strict_ && !seen.insert(key).second) fail("invalid JSON: duplicate key " + key);
            skip_ws();
            if (p_ == end_ || *p_ != ':') error("expected ':'");
            ++p_;
            skip_ws();
            Json member = value(depth + 1);
            v.members.emplace_back(std::move(key), std::move(member));
            skip_ws();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return;
            }
            error("expected ',' or '}'");
        }
    }

    void array(Json &v, int depth) {
        v.kind = Json::Array;
        ++p_;
        skip_ws();
        if (p_ < end_ && *p_ == ']') {
            ++p_;
            return;
        }
        for (;;) {
            skip_ws();
            v.items.push_back(value(depth + 1));
            skip_ws();
            if (p_ < end_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return;
            }
            error("expected ',' or ']'");
        }
    }

    unsigned hex4() {
        if (end_ - p_ < 4) error("truncated escape");
        unsigned v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= unsigned(c - '0');
            else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
            else error("invalid escape");
        }
        return v;
    }

    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += char(cp);
        } else if (cp < 0x800) {
            out += char(0xc0 | (cp >> 6));
            out += char(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += char(0xe0 | (cp >> 12));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        } else {
            out += char(0xf0 | (cp >> 18));
            out += char(0x80 | ((cp >> 12) & 0x3f));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        }
    }

    std::string string() {
        ++p_;  // opening quote
        std::string out;
        for (;;) {
            if (p_ == end_) error("unterminated string");
            const char c = *p_++;
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) error("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ == end_) error("unterminated string");
            const char e = *p_++;
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
                    uint32_t cp = hex4();
                    if (cp >= 0xdc00 && cp <= 0xdfff) error("lone trailing surrogate");
                    if (cp >= 0xd800 && cp <= 0xdbff) {
                        if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') error("lone leading surrogate");
                        p_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xdc00 || lo > 0xdfff) error("invalid surrogate pair");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: error("invalid escape");
            }
        }
    }

    void number(Json &v) {
        const char *start = p_;
        bool negative = false, integral = true;
        if (p_ < end_ && *p_ == '-') {
            negative = true;
            ++p_;
        }
        if (p_ == end_ || *p_ < '0' || *p_ > '9') error("expected value");
        if (*p_ == '0') {
            ++p_;
            if (p_ < end_ && *p_ >= '0' && *p_ <= '9') error("leading zero");
        } else {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const char *int_end = p_;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') error("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') error("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.kind = Json::Number;
        if (integral && !negative) {
            uint64_t u = 0;
            bool fits = true;
            for (const char *q = start; q < int_end; ++q) {
                if (__builtin_mul_overflow(u, uint64_t(10), &u) ||
                    __builtin_add_overflow(u, uint64_t(*q - '0'), &u)) {
                    fits = false;
                    break;
                }
            }
            v.is_u64 = fits;
            v.u64 = fits ? u : 0;
        }
    }
};

Json parse_json(const char *p, size_t n, bool strict) { return JsonParser(p, n, strict).parse_document(); }

std::string read_file(const std::string &path) {
    FILE *f = std::fopen(path.c_str(), "rb");
    ensure(f != nullptr, "cannot read " + path + ": " + std::strerror(errno));
    std::string data;
    char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) data.append(buf, n);
    const bool err = std::ferror(f) != 0;
    std::fclose(f);
    ensure(!err, "cannot read " + path);
    return data;
}

bool file_exists(const std::string &path) {
    struct stat st;
    return ::stat(path.c_str(), &st) == 0;
}

// ---- names ---------------------------------------------------------------

// canonical_name (src/weights.rs:458-472).
std::string canonical_name(const std::string &name) {
    if (starts_with(name, "model.language_model.")) return "model." + name.substr(21);
    if (starts_with(name, "language_model.model.")) return "model." + name.substr(21);
    if (starts_with(name, "language_model.")) {
        std::string rest = name.substr(15);
        return starts_with(rest, "lm_head") ? rest : "model." + rest;
    }
    return name;
}

// weight_key (src/weights.rs:474-486).
std::string weight_key(const std::string &name) {
    std::string key = canonical_name(name);
    if (ends_with(key, ".weight") || ends_with(key, ".scales") || ends_with(key, ".biases") ||
        ends_with(key, ".A_log") || ends_with(key, ".dt_bias"))
        return key;
    return key + ".weight";
}

// validate_shard_name (src/weights.rs:447-456): one normal path component
// ending in ".safetensors".
void validate_shard_name(const std::string &f) {
    ensure(!f.empty() && f.find('/') == std::string::npos && f != "." && f != ".." &&
               ends_with(f, ".safetensors"),
           "unsafe shard filename " + f);
}

// ---- quantisation --------------------------------------------------------

struct QuantSpec {
    uint32_t bits = 0;
    size_t group = 0;
};

// parse_quant_spec (src/weights.rs:711-738).
QuantSpec parse_quant_spec(const Json &v) {
    const Json *mode = v.get("mode");
    const std::string m = mode && mode->as_str() ? *mode->as_str() : "affine";
    ensure(m == "affine", "unsupported quantization mode " + m);
    const Json *bits_v = v.get("bits");
    ensure(bits_v && bits_v->as_u64(), "missing quantization bits");
    const uint64_t bits = *bits_v->as_u64();
    ensure(bits <= UINT32_MAX, "quantization bits out of range");
    ensure(bits == 4 || bits == 8, "unsupported quantization bit width " + std::to_string(bits));
    const Json *group_v = v.get("group_size");
    ensure(group_v && group_v->as_u64(), "missing quantization group size");
    const uint64_t group = *group_v->as_u64();
    ensure(group > 0 && group % (32 / bits) == 0, "invalid quantization group size");
    return QuantSpec{uint32_t(bits), size_t(group)};
}

// ---- safetensors ---------------------------------------------------------

struct Tensor {
    size_t file = 0;
    size_t offset = 0;  // absolute byte offset in the mapped file
    size_t length = 0;
    std::vector<size_t> shape;
    std::string dtype;
};

struct Mapping {
    void *base = nullptr;
    size_t length = 0;
    Mapping() = default;
    Mapping(const Mapping &) = delete;
    Mapping &operator=(const Mapping &) = delete;
    ~Mapping() {
        if (base) ::munmap(base, length);
    }
    const unsigned char *bytes() const { return static_cast<const unsigned char *>(base); }
};

std::unique_ptr<Mapping> map_file(const std::string &path, const std::string &label) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    ensure(fd >= 0, "open " + label + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        fail("map " + label + ": " + std::strerror(errno));
    }
    auto m = std::make_unique<Mapping>();
    m->length = size_t(st.st_size);
    if (m->length > 0) {
        void *p = ::mmap(nullptr, m->length, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            fail("map " + label + ": " + std::strerror(errno));
        }
        m->base = p;
    }
    ::close(fd);
    return m;
}

size_t item_size(const std::string &name, const std::string &dtype) {
    if (dtype == "F16" || dtype == "BF16") return 2;
    if (dtype == "F32" || dtype == "U32" || dtype == "I32") return 4;
    if (dtype == "F64" || dtype == "I64" || dtype == "U64") return 8;
    if (dtype == "U8" || dtype == "I8" || dtype == "BOOL") return 1;
    fail(name + ": unsupported dtype " + dtype);
}

// parse_safetensors (src/weights.rs:569-677).
std::vector<std::pair<std::string, Tensor>> parse_safetensors(const Mapping &m, const std::string &label) {
    auto ctx = [&](const std::string &msg) { return "parse " + label + ": " + msg; };
    ensure(m.length >= 8, ctx("safetensors header truncated"));
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | m.bytes()[i];
    ensure(header_len <= 100000000ull, ctx("safetensors header exceeds 100 MB"));
    const size_t data_start = 8 + size_t(header_len);
    ensure(data_start <= m.length, ctx("safetensors header truncated"));
    Json header;
    try {
        header = parse_json(reinterpret_cast<const char *>(m.bytes()) + 8, size_t(header_len), true);
    } catch (const Error &e) {
        fail(ctx("invalid safetensors JSON header: " + e.message));
    }
    ensure(header.kind == Json::Object, ctx("safetensors header is not an object"));
    if (const Json *meta = header.get("__metadata__")) {
        ensure(meta->kind == Json::Object, ctx("invalid safetensors metadata"));
        for (const auto &kv : meta->members)
            ensure(kv.second.kind == Json::String, ctx("invalid safetensors metadata value"));
    }
    std::vector<std::pair<std::string, Tensor>> out;
    std::vector<std::pair<size_t, size_t>> ranges;
    for (const auto &kv : header.members) {
        const std::string &name = kv.first;
        if (name == "__metadata__") continue;
        const Json &v = kv.second;
        const Json *dt = v.get("dtype");
        ensure(dt && dt->as_str(), ctx(name + ": missing dtype"));
        const size_t isz = item_size(ctx(name), *dt->as_str());
        const Json *shape_v = v.get("shape");
        ensure(shape_v && shape_v->kind == Json::Array, ctx(name + ": missing shape"));
        Tensor t;
        size_t count = 1;
        for (const Json &d : shape_v->items) {
            ensure(d.as_u64().has_value(), ctx("invalid tensor dimension"));
            const uint64_t n = *d.as_u64();
            ensure(n <= SIZE_MAX, ctx("tensor dimension overflow"));
            ensure(n > 0, ctx("zero tensor dimension"));
            t.shape.push_back(size_t(n));
            ensure(!__builtin_mul_overflow(count, size_t(n), &count), ctx(name + ": tensor element count overflow"));
        }
        size_t length = 0;
        ensure(!__builtin_mul_overflow(count, isz, &length), ctx(name + ": tensor byte length overflow"));
        const Json *offs = v.get("data_offsets");
        ensure(offs && offs->kind == Json::Array, ctx(name + ": missing data offsets"));
        ensure(offs->items.size() == 2, ctx(name + ": invalid data offsets"));
        ensure(offs->items[0].as_u64().has_value(), ctx("invalid start offset"));
        ensure(offs->items[1].as_u64().has_value(), ctx("invalid end offset"));
        const uint64_t start = *offs->items[0].as_u64(), end = *offs->items[1].as_u64();
        ensure(end >= start && end - start == length, ctx(name + ": byte length mismatch"));
        size_t abs_end = 0;
        ensure(end <= SIZE_MAX && !__builtin_add_overflow(data_start, size_t(end), &abs_end),
               ctx("tensor offset overflow"));
        ensure(abs_end <= m.length, ctx(name + ": tensor exceeds file"));
        ranges.emplace_back(size_t(start), size_t(end));
        t.offset = data_start + size_t(start);
        t.length = length;
        t.dtype = *dt->as_str();
        out.emplace_back(name, std::move(t));
    }
    std::sort(ranges.begin(), ranges.end());
    size_t indexed_until = 0;
    for (const auto &r : ranges) {
        ensure(r.first == indexed_until, ctx("safetensors data ranges overlap or leave holes"));
        indexed_until = r.second;
    }
    ensure(indexed_until == m.length - data_start, ctx("safetensors data has unindexed trailing bytes"));
    return out;
}

// ---- value conversions ---------------------------------------------------

// Exact IEEE binary16 -> binary32 (every F16 value, subnormals included, is a
// binary32 value).
float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1f, mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        bits = sign;
    } else {
        // Subnormal: mant * 2^-24, normalised.
        int e = 113;
        uint32_t m = mant;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            --e;
        }
        bits = sign | (uint32_t(e) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_f32(uint16_t h) {
    const uint32_t bits = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// binary32 -> binary16 with round-to-nearest, ties to even, for finite values
// of magnitude at most 65504 (the callers reject everything else first).
uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    const uint32_t e = ax >> 23;
    if (ax >= 0x38800000u) {  // >= 2^-14: a normal binary16
        uint32_t h = ((e - 112u) << 10) | ((ax >> 13) & 0x3ffu);
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // a carry moves into the exponent
        return uint16_t(sign | h);
    }
    if (ax <= 0x33000000u) return sign;  // <= 2^-25: rounds to zero (2^-25 ties to even zero)
    // Subnormal binary16: units of 2^-24. The value is m * 2^(e - 150).
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;  // 14..24
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1;
    return uint16_t(sign | h);
}

}  // namespace

// ---- the checkpoint ------------------------------------------------------

struct qmr_checkpoint {
    // Everything Checkpoint::matrix decides before it reads values
    // (src/weights.rs:292-337 for packed, 338-340 for dense).
    struct Resolved {
        std::string key;
        const Tensor *w = nullptr;
        const Tensor *s = nullptr;
        const Tensor *b = nullptr;
        qmr_matrix_info info{};
    };

    std::vector<std::unique_ptr<Mapping>> files;
    std::unordered_map<std::string, Tensor> tensors;
    std::optional<QuantSpec> quant_default;
    std::unordered_map<std::string, std::optional<QuantSpec>> quant_overrides;
    bool tie_word_embeddings = false;

    // Checkpoint::tensor (src/weights.rs:397-410).
    const Tensor &tensor(const std::string &key) const {
        if (tie_word_embeddings && key == "lm_head.weight" && !tensors.count(key)) {
            auto it = tensors.find("model.embed_tokens.weight");
            ensure(it != tensors.end(), "tied output embedding is missing");
            return it->second;
        }
        auto it = tensors.find(key);
        ensure(it != tensors.end(), "missing tensor " + key);
        return it->second;
    }

    const unsigned char *bytes(const Tensor &t) const { return files[t.file]->bytes() + t.offset; }

    // Checkpoint::float_values (src/weights.rs:427-445).
    void float_values(const Tensor &t, float *out) const {
        const unsigned char *b = bytes(t);
        if (t.dtype == "F32") {
            std::memcpy(out, b, t.length);
        } else if (t.dtype == "F16" || t.dtype == "BF16") {
            const bool f16 = t.dtype == "F16";
            const size_t n = t.length / 2;
            for (size_t i = 0; i < n; ++i) {
                const uint16_t h = uint16_t(b[2 * i] | (b[2 * i + 1] << 8));
                out[i] = f16 ? f16_to_f32(h) : bf16_to_f32(h);
            }
        } else {
            fail("tensor dtype " + t.dtype + " is not floating point");
        }
    }

    static size_t elements(const Tensor &t) {
        size_t n = 1;
        for (size_t d : t.shape) n *= d;
        return n;
    }

    // Checkpoint::quant_values (src/weights.rs:416-425), shape part.
    const Tensor &quant_tensor(const std::string &key, size_t rows, size_t groups) const {
        const Tensor &t = tensor(key);
        ensure(t.shape.size() == 2 && t.shape[0] == rows && t.shape[1] == groups, key + " shape mismatch");
        ensure(t.dtype == "F32" || t.dtype == "F16" || t.dtype == "BF16",
               "tensor dtype " + t.dtype + " is not floating point");
        return t;
    }

    // Checkpoint::quant_values: the values, all finite.
    void quant_values(const std::string &key, const Tensor &t, float *out) const {
        float_values(t, out);
        const size_t n = elements(t);
        bool finite = true;
        for (size_t i = 0; i < n; ++i) finite &= std::isfinite(out[i]);
        ensure(finite, key + " contains non-finite values");
    }

    Resolved resolve(const std::string &name) const {
        Resolved r;
        r.key = weight_key(name);
        r.w = &tensor(r.key);
        ensure(r.w->shape.size() == 2, "matrix " + r.key + " must be rank 2");
        r.info.rows = r.w->shape[0];
        std::snprintf(r.info.dtype, sizeof r.info.dtype, "%s", r.w->dtype.c_str());
        if (r.w->dtype == "U32") {
            ensure(ends_with(r.key, ".weight"), "packed matrix name");
            const std::string module = r.key.substr(0, r.key.size() - 7);
            auto ov = quant_overrides.find(module);
            const std::optional<QuantSpec> q = ov != quant_overrides.end() ? ov->second : quant_default;
            ensure(q.has_value(), "packed matrix lacks quantization metadata");
            ensure(q->bits == 4 || q->bits == 8, "unsupported packed bit width");
            ensure(q->group > 0 && q->group % (32 / q->bits) == 0, "invalid quantization group size");
            const size_t words_per_group = q->group / (32 / q->bits);
            ensure(r.w->shape[1] % words_per_group == 0, "packed width not divisible by group width");
            const size_t groups = r.w->shape[1] / words_per_group;
            size_t cols = 0;
            ensure(!__builtin_mul_overflow(groups, q->group, &cols), "packed matrix width overflow");
            r.s = &quant_tensor(module + ".scales", r.info.rows, groups);
            r.b = &quant_tensor(module + ".biases", r.info.rows, groups);
            r.info.packed = 1;
            r.info.cols = cols;
            r.info.bits = q->bits;
            r.info.group_size = q->group;
            std::snprintf(r.info.metadata_dtype, sizeof r.info.metadata_dtype, "%s", r.s->dtype.c_str());
        } else {
            ensure(r.w->dtype == "F32" || r.w->dtype == "F16" || r.w->dtype == "BF16",
                   "tensor dtype " + r.w->dtype + " is not floating point");
            r.info.packed = 0;
            r.info.cols = r.w->shape[1];
            r.info.bits = 16;
            r.info.group_size = 0;
            r.info.metadata_dtype[0] = '\0';
        }
        return r;
    }

    // Dense values as F16 bits (src/weights.rs:338-350).
    void dense_values(const Resolved &r, uint16_t *out) const {
        const size_t n = elements(*r.w);
        std::vector<float> v(n);
        float_values(*r.w, v.data());
        bool in_range = true;
        for (size_t i = 0; i < n; ++i) in_range &= std::fabs(v[i]) <= 65504.0f;  // false for NaN too
        ensure(in_range, "matrix " + r.key + " exceeds F16 range");
        for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(v[i]);
    }
};

namespace {

// parse_quantization (src/weights.rs:679-709).
void parse_quantization(const Json *value, qmr_checkpoint &cp) {
    if (!value) return;
    ensure(value->kind == Json::Object, "invalid quantization metadata");
    if (value->get("bits") || value->get("group_size")) cp.quant_default = parse_quant_spec(*value);
    std::set<std::string> seen;
    for (const auto &kv : value->members) {
        const std::string &key = kv.first;
        if (key == "bits" || key == "group_size" || key == "mode") continue;
        std::optional<QuantSpec> spec;
        if (kv.second.kind == Json::Bool) {
            if (kv.second.boolean) spec = cp.quant_default;
        } else if (kv.second.kind == Json::Object) {
            spec = parse_quant_spec(kv.second);
        } else {
            fail("invalid quantization entry " + key);
        }
        const std::string canonical = canonical_name(key);
        ensure(seen.insert(canonical).second, "duplicate quantization entry " + canonical);
        cp.quant_overrides[canonical] = spec;
    }
}

// serde_json::Value keeps the last of duplicate keys; the config and index
// files are read that way (only safetensors headers are strict).
Json dedup_last(const Json &v) {
    Json out = v;
    if (v.kind == Json::Object) {
        out.members.clear();
        for (const auto &kv : v.members) {
            bool later = false;
            for (const auto &other : v.members)
                if (&other > &kv && other.first == kv.first) later = true;
            if (!later) out.members.emplace_back(kv.first, dedup_last(kv.second));
        }
    } else if (v.kind == Json::Array) {
        for (auto &item : out.items) item = dedup_last(item);
    }
    return out;
}

std::string real_path(const std::string &p) {
    char buf[PATH_MAX];
    ensure(::realpath(p.c_str(), buf) != nullptr, "cannot resolve " + p + ": " + std::strerror(errno));
    return buf;
}

std::unique_ptr<qmr_checkpoint> open_checkpoint(const std::string &dir) {
    struct stat st;
    ensure(::stat(dir.c_str(), &st) == 0 && S_ISDIR(st.st_mode), "checkpoint path must be a directory");
    const std::string config_text = read_file(dir + "/config.json");
    const Json config = dedup_last(parse_json(config_text.data(), config_text.size(), false));
    auto cp = std::make_unique<qmr_checkpoint>();
    const Json *quant = config.get("quantization");
    if (!quant) quant = config.get("quantization_config");
    parse_quantization(quant, *cp);
    // ModelConfig::from_json (src/config.rs:145-149): text_config first, then the root.
    const Json *text = config.get("text_config");
    const Json *tie = text ? text->get("tie_word_embeddings") : nullptr;
    if (!tie) tie = config.get("tie_word_embeddings");
    cp->tie_word_embeddings = tie && tie->kind == Json::Bool && tie->boolean;

    std::vector<std::string> filenames;
    std::optional<std::unordered_map<std::string, std::string>> weight_map;
    const std::string index_path = dir + "/model.safetensors.index.json";
    if (file_exists(index_path)) {
        const std::string text_idx = read_file(index_path);
        Json index;
        try {
            index = dedup_last(parse_json(text_idx.data(), text_idx.size(), false));
        } catch (const Error &e) {
            fail("invalid safetensors index: " + e.message);
        }
        const Json *map = index.get("weight_map");
        ensure(map && map->kind == Json::Object, "missing safetensors weight_map");
        ensure(!map->members.empty(), "empty safetensors index");
        std::set<std::string> names;
        weight_map.emplace();
        for (const auto &kv : map->members) {
            ensure(kv.second.kind == Json::String, "invalid shard filename");
            validate_shard_name(kv.second.str);
            names.insert(kv.second.str);
            (*weight_map)[kv.first] = kv.second.str;
        }
        filenames.assign(names.begin(), names.end());
    } else {
        DIR *d = ::opendir(dir.c_str());
        ensure(d != nullptr, "cannot list " + dir + ": " + std::strerror(errno));
        while (const dirent *e = ::readdir(d)) {
            const std::string n = e->d_name;
            if (ends_with(n, ".safetensors")) filenames.push_back(n);
        }
        ::closedir(d);
        std::sort(filenames.begin(), filenames.end());
        ensure(filenames.size() == 1, "expected one safetensors file or an index");
    }

    const std::string root = real_path(dir) + "/";
    std::set<std::string> seen_index_names;
    for (const std::string &filename : filenames) {
        validate_shard_name(filename);
        const std::string path = dir + "/" + filename;
        ensure(starts_with(real_path(path), root.c_str()), "safetensors shard escapes checkpoint directory");
        cp->files.push_back(map_file(path, filename));
        const size_t file_id = cp->files.size() - 1;
        for (auto &entry : parse_safetensors(*cp->files.back(), filename)) {
            if (weight_map) {
                auto it = weight_map->find(entry.first);
                ensure(it != weight_map->end() && it->second == filename,
                       "tensor " + entry.first + " missing or mapped to wrong shard");
                seen_index_names.insert(entry.first);
            }
            entry.second.file = file_id;
            const std::string canonical = canonical_name(entry.first);
            ensure(cp->tensors.emplace(canonical, std::move(entry.second)).second,
                   "duplicate canonical tensor " + canonical);
        }
    }
    if (weight_map) ensure(seen_index_names.size() == weight_map->size(), "index names missing from shards");
    return cp;
}

void release_matrix(qmr_matrix *m) {
    if (!m) return;
    if (m->weight) qmr_buffer_release(m->weight);
    if (m->scales) qmr_buffer_release(m->scales);
    if (m->biases) qmr_buffer_release(m->biases);
    m->weight = m->scales = m->biases = nullptr;
}

void upload(qmr_device *device, const void *data, size_t bytes, qmr_buffer **out) {
    // Large arrays go through the pinned staging path.
    const int rc = bytes >= (size_t(32) << 20) ? qmr::upload_staged(device, data, bytes, out)
                                               : qmr_buffer_upload(device, data, bytes, out);
    if (rc != QMR_OK) throw Error{QMR_ERR_DEVICE, qmr_last_error()};
}

// A packed matrix's codes, scales and biases through one staged pipeline.
void upload_matrix(qmr_device *device, const void *w, size_t w_bytes, const void *s, const void *b,
                   size_t meta_bytes, qmr_matrix *m) {
    const qmr::StagedView views[3] = {{w, w_bytes}, {s, meta_bytes}, {b, meta_bytes}};
    qmr_buffer *out[3] = {nullptr, nullptr, nullptr};
    if (qmr::upload_staged_views(device, views, 3, out) != QMR_OK) throw Error{QMR_ERR_DEVICE, qmr_last_error()};
    m->weight = out[0];
    m->scales = out[1];
    m->biases = out[2];
}

// Whether n BF16 values are all finite (the exponent field not all ones).
bool bf16_all_finite(const unsigned char *p, size_t n) {
    uint16_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        uint16_t v;
        std::memcpy(&v, p + 2 * i, 2);
        bad |= uint16_t((v & 0x7F80u) == 0x7F80u);
    }
    return bad == 0;
}

}  // namespace

using Resolved = qmr_checkpoint::Resolved;

extern "C" {

int qmr_checkpoint_open(const char *dir, qmr_checkpoint **out) {
    return guarded([&]() -> int {
        ensure(dir != nullptr && out != nullptr, "qmr_checkpoint_open: null argument");
        *out = nullptr;
        *out = open_checkpoint(dir).release();
        return QMR_OK;
    });
}

void qmr_checkpoint_close(qmr_checkpoint *checkpoint) { delete checkpoint; }

size_t qmr_checkpoint_tensor_count(const qmr_checkpoint *checkpoint) {
    return checkpoint ? checkpoint->tensors.size() : 0;
}

int qmr_checkpoint_contains(const qmr_checkpoint *checkpoint, const char *name) {
    if (!checkpoint || !name) return 0;
    const std::string key = weight_key(name);
    return checkpoint->tensors.count(key) ||
                   (checkpoint->tie_word_embeddings && key == "lm_head.weight" &&
                    checkpoint->tensors.count("model.embed_tokens.weight"))
               ? 1
               : 0;
}

int qmr_checkpoint_matrix_info(const qmr_checkpoint *checkpoint, const char *name, qmr_matrix_info *info) {
    return guarded([&]() -> int {
        ensure(checkpoint && name && info, "qmr_checkpoint_matrix_info: null argument");
        *info = checkpoint->resolve(name).info;
        return QMR_OK;
    });
}

int qmr_checkpoint_matrix(const qmr_checkpoint *checkpoint, const char *name, uint32_t *weights, float *scales,
                          float *biases) {
    return guarded([&]() -> int {
        ensure(checkpoint && name && weights && scales && biases, "qmr_checkpoint_matrix: null argument");
        const auto r = checkpoint->resolve(name);
        ensure(r.info.packed == 1, "matrix " + r.key + " is not packed");
        checkpoint->quant_values(r.key.substr(0, r.key.size() - 7) + ".scales", *r.s, scales);
        checkpoint->quant_values(r.key.substr(0, r.key.size() - 7) + ".biases", *r.b, biases);
        std::memcpy(weights, checkpoint->bytes(*r.w), r.w->length);  // little-endian host
        return QMR_OK;
    });
}

int qmr_checkpoint_dense(const qmr_checkpoint *checkpoint, const char *name, uint16_t *values) {
    return guarded([&]() -> int {
        ensure(checkpoint && name && values, "qmr_checkpoint_dense: null argument");
        const auto r = checkpoint->resolve(name);
        ensure(r.info.packed == 0, "matrix " + r.key + " is packed");
        checkpoint->dense_values(r, values);
        return QMR_OK;
    });
}

int qmr_matrix_load(qmr_device *device, const qmr_checkpoint *checkpoint, const char *name, size_t rows,
                    size_t cols, qmr_matrix *out) {
    qmr_matrix m{};
    const int rc = guarded([&]() -> int {
        ensure(device && checkpoint && name && out, "qmr_matrix_load: null argument");
        std::memset(out, 0, sizeof *out);
        Resolved r;
        try {
            r = checkpoint->resolve(name);
        } catch (const Error &e) {
            throw Error{e.code, std::string("loading ") + name + ": " + e.message};
        }
        ensure(r.info.rows == rows && r.info.cols == cols,
               std::string(name) + ": expected [" + std::to_string(rows) + "," + std::to_string(cols) + "], got [" +
                   std::to_string(r.info.rows) + "," + std::to_string(r.info.cols) + "]");
        m.rows = rows;
        m.cols = cols;
        m.bits = r.info.bits;
        m.group = r.info.group_size;
        if (!r.info.packed) {
            std::vector<uint16_t> v(rows * cols);
            checkpoint->dense_values(r, v.data());
            ensure(v.size() * 2 < qmr::device_free_bytes(device),
                   "model exceeds the device's free memory; use packed 4-bit weights");
            upload(device, v.data(), v.size() * 2, &m.weight);
        } else if (r.s->dtype == "BF16" && r.b->dtype == "BF16" &&
                   std::strcmp(qmr_metadata_mode(device), "bf16") == 0 &&
                   qmr_supported_bf16_quantization(m.bits, m.group)) {
            // BF16 metadata for a device that keeps BF16: expanding each value
            // to FP32 and compacting it back (qmr_compact_metadata) returns the
            // stored bit pattern for every finite value, so the mapped bytes
            // are uploaded as they are once no value is Inf or NaN.
            const size_t n = qmr_checkpoint::elements(*r.s);
            const std::string module = r.key.substr(0, r.key.size() - 7);
            ensure(r.w->length + 2 * n * 2 < qmr::device_free_bytes(device),
                   "model exceeds the device's free memory; use packed 4-bit weights");
            // The finiteness checks run on another thread while the arrays
            // upload; a non-finite value releases the buffers and fails the
            // load with the check's message, as before any upload.
            const unsigned char *sp = checkpoint->bytes(*r.s);
            const unsigned char *bp = checkpoint->bytes(*r.b);
            bool s_ok = true, b_ok = true;
            std::thread check([&] {
                s_ok = bf16_all_finite(sp, n);
                b_ok = bf16_all_finite(bp, n);
            });
            try {
                upload_matrix(device, checkpoint->bytes(*r.w), r.w->length, sp, bp, n * 2, &m);
            } catch (...) {
                check.join();
                throw;
            }
            check.join();
            ensure(s_ok, module + ".scales contains non-finite values");
            ensure(b_ok, module + ".biases contains non-finite values");
            qmr_record_compacted_metadata(device, uint64_t(n) * 2 * 2);
            m.metadata_bf16 = 1;
        } else {
            const size_t n = qmr_checkpoint::elements(*r.s);
            std::vector<float> s(n), b(n);
            const std::string module = r.key.substr(0, r.key.size() - 7);
            checkpoint->quant_values(module + ".scales", *r.s, s.data());
            checkpoint->quant_values(module + ".biases", *r.b, b.data());
            std::vector<uint16_t> s16(n), b16(n);
            const bool compacted = qmr_compact_metadata(device, m.bits, m.group, s.data(), b.data(), n, s16.data(),
                                                        b16.data()) == 1;
            const size_t meta_bytes = compacted ? 2 * n * 2 : 2 * n * 4;
            ensure(r.w->length + meta_bytes < qmr::device_free_bytes(device),
                   "model exceeds the device's free memory; use packed 4-bit weights");
            if (compacted) {
                upload_matrix(device, checkpoint->bytes(*r.w), r.w->length, s16.data(), b16.data(), n * 2, &m);
                qmr_record_compacted_metadata(device, uint64_t(n) * 2 * 2);
            } else {
                upload_matrix(device, checkpoint->bytes(*r.w), r.w->length, s.data(), b.data(), n * 4, &m);
            }
            m.metadata_bf16 = compacted ? 1 : 0;
        }
        *out = m;
        return QMR_OK;
    });
    if (rc != QMR_OK) release_matrix(&m);
    return rc;
}

void qmr_matrix_release(qmr_matrix *matrix) { release_matrix(matrix); }

}  // extern "C"
