// checkpoint.hip — host-side checkpoint readers behind include/dmx_ckpt.h
// (no device code).
//
// Two containers, the ones `load_weights` accepts
// (crates/demucs-core/src/demucs/weights.rs:30-88); the readers are this
// build's own and share only the file formats with the reference's
// (crates/demucs-core/src/safetensors.rs, crates/demucs-core/src/ckpt/):
//   * safetensors: tensors of any listed element type become f32, and the
//     model config comes from the "kwargs" metadata entry when present
//     (HtdemucsConfig::from_kwargs_json, config.rs:150-215);
//   * torch.save zips: "<root>/data.pkl" (a pickle), "<root>/data/<key>" (one
//     raw blob per storage) and "<root>/byteorder". The pickle is evaluated
//     symbolically (PickleMachine): calls are recorded, never made, and the
//     tensors are recognised in the finished tree by their rebuild calls.
//     The state dict is the top-level dict or its "model_state_dict" /
//     "state_dict" / "state" entry, the keys demucs' packages and training
//     checkpoints use (crates/demucs-core/src/ckpt/mod.rs:232-256).
// Tensors are kept sorted by name, each contiguous row-major f32.
#include <algorithm>
#include <array>
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <fstream>
#include <map>
#include <memory>
#include <vector>

#include "../../include/dmx.h"
#include "../../include/dmx_ckpt.h"
#include "common.h"

namespace dmx {
namespace {

constexpr int ERR_CHECKPOINT = 9;  // Error::Checkpoint / Error::Pickle
constexpr int ERR_IO = 10;         // Error::Io

[[noreturn]] void bad(const std::string &msg) { throw Error(ERR_CHECKPOINT, msg); }

// ----- a small JSON reader (objects keep their key order) -----

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    bool integral = false;  // the literal had no fraction or exponent
    int64_t inum = 0;       // its value when integral
    std::string str;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;

    const Json *get(const std::string &k) const {
        for (const auto &m : members)
            if (m.first == k) return &m.second;
        return nullptr;
    }
};

class JsonReader {
  public:
    JsonReader(const char *p, size_t n) : p_(p), end_(p + n) {}
    Json parse_document() {
        Json v = value(0);
        ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

  private:
    const char *p_, *end_;

    [[noreturn]] void fail(const char *what) { bad(std::string("JSON: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool eat(const char *lit) {
        const size_t n = std::strlen(lit);
        if ((size_t)(end_ - p_) >= n && std::memcmp(p_, lit, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xc0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += (char)(0xe0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        } else {
            out += (char)(0xf0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3f));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("truncated \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        if (p_ >= end_ || *p_ != '"') fail("expected a string");
        ++p_;
        std::string out;
        while (true) {
            if (p_ >= end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if ((unsigned char)c < 0x20) fail("control character in a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= end_) fail("unterminated escape");
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
                    if (cp >= 0xd800 && cp < 0xdc00) {  // a surrogate pair
                        if (!eat("\\u")) fail("lone high surrogate");
                        const uint32_t lo = hex4();
                        if (lo < 0xdc00 || lo >= 0xe000) fail("bad low surrogate");
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    } else if (cp >= 0xdc00 && cp < 0xe000) {
                        fail("lone low surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        return out;
    }
    Json number() {
        const char *start = p_;
        bool integral = true;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad number");
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string text(start, p_);
        Json v;
        v.kind = Json::Number;
        v.num = std::strtod(text.c_str(), nullptr);
        if (integral) {
            errno = 0;
            const long long i = std::strtoll(text.c_str(), nullptr, 10);
            v.integral = errno == 0;
            v.inum = i;
        }
        return v;
    }
    Json value(int depth) {
        if (depth > 256) fail("nesting too deep");
        ws();
        if (p_ >= end_) fail("unexpected end");
        Json v;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Object;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return v;
            }
            while (true) {
                ws();
                std::string k = string();
                ws();
                if (p_ >= end_ || *p_ != ':') fail("expected ':'");
                ++p_;
                v.members.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return v;
                }
                fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Json::Array;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return v;
            }
            while (true) {
                v.items.push_back(value(depth + 1));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return v;
                }
                fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::String;
            v.str = string();
            return v;
        }
        if (eat("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return v;
        }
        if (eat("false")) {
            v.kind = Json::Bool;
            return v;
        }
        if (eat("null")) return v;
        return number();
    }
};

Json parse_json(const char *p, size_t n) { return JsonReader(p, n).parse_document(); }

// ----- element decoding -----

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    float v;
    if (exp == 0) {
        v = std::ldexp((float)man, -24);  // zero and subnormals
    } else if (exp == 0x1f) {
        v = man ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
    } else {
        uint32_t bits = ((exp + 112) << 23) | (man << 13);
        std::memcpy(&v, &bits, 4);
    }
    if (sign) v = -v;
    return v;
}

enum class DType { F32, F16, BF16, F64, U8, I8, I16, I32, I64, Bool };

int dtype_size(DType t) {
    switch (t) {
        case DType::F32: case DType::I32: return 4;
        case DType::F16: case DType::BF16: case DType::I16: return 2;
        case DType::F64: case DType::I64: return 8;
        default: return 1;
    }
}

template <class T>
T load_as(const uint8_t *p, bool big) {
    uint8_t b[sizeof(T)];
    for (size_t i = 0; i < sizeof(T); ++i) b[i] = big ? p[sizeof(T) - 1 - i] : p[i];
    T v;
    std::memcpy(&v, b, sizeof(T));
    return v;
}

// n elements of type t at p -> f32.
void decode(const uint8_t *p, size_t n, DType t, bool big, float *out) {
    for (size_t i = 0; i < n; ++i) {
        const uint8_t *e = p + i * dtype_size(t);
        switch (t) {
            case DType::F32: out[i] = load_as<float>(e, big); break;
            case DType::F64: out[i] = (float)load_as<double>(e, big); break;
            case DType::F16: out[i] = half_to_float(load_as<uint16_t>(e, big)); break;
            case DType::BF16: {
                const uint32_t bits = (uint32_t)load_as<uint16_t>(e, big) << 16;
                std::memcpy(&out[i], &bits, 4);
                break;
            }
            case DType::U8: case DType::Bool: out[i] = (float)e[0]; break;
            case DType::I8: out[i] = (float)(int8_t)e[0]; break;
            case DType::I16: out[i] = (float)load_as<int16_t>(e, big); break;
            case DType::I32: out[i] = (float)load_as<int32_t>(e, big); break;
            case DType::I64: out[i] = (float)load_as<int64_t>(e, big); break;
        }
    }
}

// ----- the checkpoint object -----

struct Tensor {
    std::vector<int64_t> shape;
    std::vector<float> data;
};

}  // namespace
}  // namespace dmx

struct dmx_checkpoint {
    std::map<std::string, dmx::Tensor> tensors;
    std::map<std::string, std::string> metadata;
    dmx_config config;
    std::vector<dmx_tensor> view;  // dmx_tensor entries over `tensors`, by name
};

namespace dmx {
namespace {

void finish(dmx_checkpoint &c) {
    c.view.clear();
    for (auto &kv : c.tensors) {
        if (kv.second.shape.size() > 4) bad(kv.first + ": more than 4 dimensions");
        dmx_tensor t{};
        t.name = kv.first.c_str();
        t.data = kv.second.data.data();
        t.ndim = (int32_t)kv.second.shape.size();
        for (size_t d = 0; d < kv.second.shape.size(); ++d) t.shape[d] = kv.second.shape[d];
        c.view.push_back(t);
    }
}

// Element count of a shape; at most 2^36 elements (256 GiB of f32).
uint64_t checked_product(const std::vector<int64_t> &shape, const std::string &name) {
    constexpr uint64_t limit = (uint64_t)1 << 36;
    uint64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) bad(name + ": negative dimension");
        if (d && n > limit / (uint64_t)d) bad(name + ": too many elements");
        n *= (uint64_t)d;
    }
    return n;
}

// kwargs (config.rs:77-145): each known key overrides the default; unknown keys
// are ignored; `segment` is a number or {numerator, denominator}.
void config_from_kwargs(const Json &kw, dmx_config &cfg) {
    if (kw.kind != Json::Object) throw Error(2, "checkpoint kwargs are not a JSON object");
    auto uint_field = [&](const char *key, int32_t &dst) {
        const Json *v = kw.get(key);
        if (!v || v->kind == Json::Null) return;
        if (v->kind != Json::Number || !v->integral || v->inum < 0 || v->inum > INT32_MAX)
            throw Error(2, std::string("checkpoint kwargs: `") + key + "` is not an unsigned integer");
        dst = (int32_t)v->inum;
    };
    auto float_field = [&](const char *key, double &dst) {
        const Json *v = kw.get(key);
        if (!v || v->kind == Json::Null) return;
        if (v->kind != Json::Number) throw Error(2, std::string("checkpoint kwargs: `") + key + "` is not a number");
        dst = v->num;
    };
    if (const Json *v = kw.get("sources"); v && v->kind != Json::Null) {
        if (v->kind != Json::Array) throw Error(2, "checkpoint kwargs: `sources` is not a list");
        for (const Json &s : v->items)
            if (s.kind != Json::String) throw Error(2, "checkpoint kwargs: `sources` holds a non-string");
        cfg.sources = (int32_t)v->items.size();
    }
    uint_field("audio_channels", cfg.audio_channels);
    uint_field("samplerate", cfg.samplerate);
    if (const Json *v = kw.get("segment"); v && v->kind != Json::Null) {
        if (v->kind == Json::Number) {
            cfg.segment = v->num;
        } else if (v->kind == Json::Object && v->get("numerator") && v->get("denominator") &&
                   v->get("numerator")->kind == Json::Number && v->get("denominator")->kind == Json::Number) {
            const double den = v->get("denominator")->num;
            cfg.segment = den == 0.0 ? std::nan("") : v->get("numerator")->num / den;
        } else {
            throw Error(2, "checkpoint kwargs: `segment` is neither a number nor a fraction");
        }
    }
    uint_field("channels", cfg.channels);
    uint_field("growth", cfg.growth);
    uint_field("nfft", cfg.nfft);
    uint_field("depth", cfg.depth);
    uint_field("stride", cfg.stride);
    uint_field("kernel_size", cfg.kernel_size);
    uint_field("context", cfg.context);
    float_field("freq_emb", cfg.freq_emb);
    float_field("emb_scale", cfg.emb_scale);
    if (const Json *v = kw.get("cac"); v && v->kind != Json::Null) {
        if (v->kind != Json::Bool) throw Error(2, "checkpoint kwargs: `cac` is not a boolean");
        cfg.cac = v->b ? 1 : 0;
    }
    uint_field("bottom_channels", cfg.bottom_channels);
    uint_field("t_layers", cfg.t_layers);
    uint_field("t_heads", cfg.t_heads);
    float_field("t_hidden_scale", cfg.t_hidden_scale);
    float_field("t_max_period", cfg.t_max_period);
    float_field("t_weight_pos_embed", cfg.t_weight_pos_embed);
}

// ----- safetensors -----
// An 8-byte little-endian header size h, then h bytes of JSON that map each
// tensor name to {"dtype", "shape", "data_offsets": [begin, end)} (offsets
// into the data section after the header), plus an optional "__metadata__"
// object of strings. Every entry is checked before any tensor is decoded.

struct StEntry {
    std::string name;
    DType type;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
};

// Element types by their safetensors spelling (all widen to f32).
const std::map<std::string, DType> &st_types() {
    static const std::map<std::string, DType> types = {
        {"BOOL", DType::Bool}, {"U8", DType::U8},   {"I8", DType::I8},   {"I16", DType::I16}, {"I32", DType::I32},
        {"I64", DType::I64},   {"F16", DType::F16}, {"BF16", DType::BF16}, {"F32", DType::F32}, {"F64", DType::F64}};
    return types;
}

[[noreturn]] void st_fail(const std::string &tensor, const std::string &what) {
    bad("safetensors tensor `" + tensor + "`: " + what);
}

// A list of non-negative integers under `key` of a header entry.
std::vector<int64_t> st_ints(const Json &entry, const char *key, const std::string &tensor) {
    const Json *v = entry.get(key);
    if (!v || v->kind != Json::Array) st_fail(tensor, std::string("its header entry lacks a `") + key + "` list");
    std::vector<int64_t> out;
    for (const Json &x : v->items) {
        if (x.kind != Json::Number || !x.integral || x.inum < 0)
            st_fail(tensor, std::string("`") + key + "` holds a value that is not a non-negative integer");
        out.push_back(x.inum);
    }
    return out;
}

std::string shape_text(const std::vector<int64_t> &shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

StEntry st_entry(const std::string &name, const Json &e, uint64_t data_bytes) {
    if (e.kind != Json::Object) st_fail(name, "its header entry is not an object");
    StEntry t;
    t.name = name;
    const Json *dt = e.get("dtype");
    if (!dt || dt->kind != Json::String) st_fail(name, "its header entry lacks a `dtype` string");
    const auto ty = st_types().find(dt->str);
    if (ty == st_types().end()) st_fail(name, "element type `" + dt->str + "` is not one this reader widens to f32");
    t.type = ty->second;
    t.shape = st_ints(e, "shape", name);
    const std::vector<int64_t> span = st_ints(e, "data_offsets", name);
    if (span.size() != 2) st_fail(name, "`data_offsets` must be the pair [begin, end]");
    t.begin = (uint64_t)span[0];
    t.end = (uint64_t)span[1];
    if (t.begin > t.end || t.end > data_bytes)
        st_fail(name, "its bytes [" + std::to_string(t.begin) + ", " + std::to_string(t.end) + ") lie beyond the " +
                          std::to_string(data_bytes) + "-byte data section");
    const uint64_t need = checked_product(t.shape, name) * (uint64_t)dtype_size(t.type);
    if (t.end - t.begin != need)
        st_fail(name, "shape " + shape_text(t.shape) + " of " + dt->str + " takes " + std::to_string(need) +
                          " bytes, but its entry spans " + std::to_string(t.end - t.begin));
    return t;
}

void parse_safetensors(const uint8_t *bytes, size_t len, dmx_checkpoint &c) {
    if (len < 8)
        bad("safetensors: " + std::to_string(len) + " bytes cannot hold the 8-byte header size that starts the file");
    const uint64_t header_bytes = load_as<uint64_t>(bytes, false);
    if (header_bytes > len - 8)
        bad("safetensors: the header size field announces " + std::to_string(header_bytes) + " bytes, but only " +
            std::to_string(len - 8) + " follow it");
    const Json header = parse_json(reinterpret_cast<const char *>(bytes) + 8, (size_t)header_bytes);
    if (header.kind != Json::Object) bad("safetensors: the header is not a JSON object");
    const uint8_t *data = bytes + 8 + header_bytes;
    const uint64_t data_bytes = len - 8 - header_bytes;
    std::vector<StEntry> entries;
    for (const auto &m : header.members) {
        if (m.first == "__metadata__") {
            if (m.second.kind != Json::Object) bad("safetensors: `__metadata__` is not an object");
            for (const auto &kv : m.second.members)
                if (kv.second.kind == Json::String) c.metadata[kv.first] = kv.second.str;
            continue;
        }
        entries.push_back(st_entry(m.first, m.second, data_bytes));
    }
    for (const StEntry &e : entries) {
        Tensor t;
        t.shape = e.shape;
        t.data.resize((e.end - e.begin) / (uint64_t)dtype_size(e.type));
        decode(data + e.begin, t.data.size(), e.type, false, t.data.data());
        if (!c.tensors.emplace(e.name, std::move(t)).second) bad("safetensors: tensor `" + e.name + "` is listed twice");
    }
    const auto kw = c.metadata.find("kwargs");
    if (kw != c.metadata.end()) config_from_kwargs(parse_json(kw->second.data(), kw->second.size()), c.config);
}

// ----- zip (stored entries; torch.save writes no compression) -----

struct ZipEntry {
    uint64_t offset = 0, size = 0, csize = 0;
    uint16_t method = 0;
};

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)rd16(p) | (uint32_t)rd16(p + 2) << 16; }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | (uint64_t)rd32(p + 4) << 32; }

std::map<std::string, ZipEntry> zip_directory(const uint8_t *z, size_t len) {
    if (len < 22) bad("not a zip archive (too short)");
    // End of central directory: the last "PK\5\6" within 64 KiB + 22 of the end.
    size_t eocd = SIZE_MAX;
    const size_t lo = len > 22 + 65535 ? len - 22 - 65535 : 0;
    for (size_t i = len - 22 + 1; i-- > lo;)
        if (rd32(z + i) == 0x06054b50) {
            eocd = i;
            break;
        }
    if (eocd == SIZE_MAX) bad("not a zip archive (no end-of-central-directory record)");
    uint64_t count = rd16(z + eocd + 10), cd_size = rd32(z + eocd + 12), cd_off = rd32(z + eocd + 16);
    if (eocd >= 20 && rd32(z + eocd - 20) == 0x07064b50) {  // zip64 locator
        const uint64_t e64 = rd64(z + eocd - 20 + 8);
        if (e64 + 56 > len || rd32(z + e64) != 0x06064b50) bad("zip64 end-of-central-directory record is corrupt");
        count = rd64(z + e64 + 32);
        cd_size = rd64(z + e64 + 40);
        cd_off = rd64(z + e64 + 48);
    }
    if (cd_off > len || cd_size > len - cd_off) bad("zip central directory lies outside the file");
    std::map<std::string, ZipEntry> dir;
    size_t p = cd_off;
    for (uint64_t i = 0; i < count; ++i) {
        if (p + 46 > len || rd32(z + p) != 0x02014b50) bad("zip central directory entry is corrupt");
        ZipEntry e;
        e.method = rd16(z + p + 10);
        e.csize = rd32(z + p + 20);
        e.size = rd32(z + p + 24);
        const uint16_t nlen = rd16(z + p + 28), xlen = rd16(z + p + 30), clen = rd16(z + p + 32);
        e.offset = rd32(z + p + 42);
        if (p + 46 + (size_t)nlen + xlen + clen > len) bad("zip central directory entry is truncated");
        std::string name(reinterpret_cast<const char *>(z + p + 46), nlen);
        // zip64 extra field: the 64-bit values, in order, of the fields that read 0xffffffff.
        const uint8_t *x = z + p + 46 + nlen, *xend = x + xlen;
        while (x + 4 <= xend) {
            const uint16_t id = rd16(x), sz = rd16(x + 2);
            if (x + 4 + sz > xend) break;
            if (id == 1) {
                const uint8_t *q = x + 4, *qend = x + 4 + sz;
                if (e.size == 0xffffffffu && q + 8 <= qend) e.size = rd64(q), q += 8;
                if (e.csize == 0xffffffffu && q + 8 <= qend) e.csize = rd64(q), q += 8;
                if (e.offset == 0xffffffffu && q + 8 <= qend) e.offset = rd64(q), q += 8;
            }
            x += 4 + sz;
        }
        dir[name] = e;
        p += 46 + (size_t)nlen + xlen + clen;
    }
    return dir;
}

// The bytes of one stored entry.
std::pair<const uint8_t *, uint64_t> zip_data(const uint8_t *z, size_t len, const ZipEntry &e,
                                              const std::string &name) {
    if (e.method != 0) bad("archive entry " + name + " is compressed (method " + std::to_string(e.method) +
                           "); torch.save archives are stored uncompressed");
    if (e.offset + 30 > len || rd32(z + e.offset) != 0x04034b50) bad("archive entry " + name + ": bad local header");
    const uint64_t start = e.offset + 30 + rd16(z + e.offset + 26) + rd16(z + e.offset + 28);
    if (start > len || e.size > len - start) bad("archive entry " + name + " lies outside the file");
    return {z + start, e.size};
}

// ----- pickles, evaluated symbolically -----
// torch.save stores the state dict as a pickle: a small stack program whose
// objects are made by calling importable functions
// (torch._utils._rebuild_tensor_v2, collections.OrderedDict, ...) and whose
// storages are named by "persistent ids" that point at archive entries. This
// reader runs the stack program without importing or calling anything: a
// call leaves an `Apply` node holding the callee's dotted name and its
// arguments, a persistent id leaves a `Persistent` node, and the tensors are
// recognised afterwards by walking the finished tree (torch_tensor below).
// Opcode numbers and meanings are those of the pickle format (CPython's
// Lib/pickle.py and pickletools); torch writes protocol 2.

struct PNode;
using PNodeRef = std::shared_ptr<PNode>;

struct PNode {
    enum class Shape : uint8_t { Nil, Truth, Whole, Real, Text, Raw, Row, Table, Name, Apply, Persistent };
    Shape shape = Shape::Nil;
    bool tuple = false;                                // Row: a tuple rather than a list
    int64_t whole = 0;                                 // Truth (0 or 1), Whole
    double real = 0.0;                                 // Real
    std::string text;                                  // Text, Raw; Name: "module.qualname"
    std::vector<PNodeRef> row;                         // Row items; Apply, Persistent: the arguments
    std::vector<std::pair<PNodeRef, PNodeRef>> table;  // Table entries; Apply: items stored into the result
    PNodeRef callee, state;                            // Apply: the Name called, and the state BUILD gave it
};

PNodeRef node(PNode::Shape shape) {
    auto n = std::make_shared<PNode>();
    n->shape = shape;
    return n;
}

class PickleMachine {
  public:
    PickleMachine(const uint8_t *p, size_t n) : begin_(p), at_(p), end_(p + n) {}

    PNodeRef evaluate() {
        while (!result_) {
            op_at_ = (size_t)(at_ - begin_);
            if (at_ == end_) fail("the data ends before a STOP opcode");
            const uint8_t op = byte();
            const Step step = steps()[op];
            if (!step) {
                char hex[8];
                std::snprintf(hex, sizeof hex, "0x%02x", op);
                fail(std::string("opcode ") + hex + " is not one this reader runs");
            }
            (this->*step)(op);
        }
        return result_;
    }

  private:
    using Step = void (PickleMachine::*)(uint8_t);

    // One handler per opcode byte; bytes without one are refused.
    static const std::array<Step, 256> &steps() {
        static const std::array<Step, 256> table = [] {
            std::array<Step, 256> t{};
            auto on = [&t](std::initializer_list<uint8_t> ops, Step s) {
                for (uint8_t o : ops) t[o] = s;
            };
            on({0x80}, &PickleMachine::proto);
            on({0x95}, &PickleMachine::frame);
            on({'.'}, &PickleMachine::stop);
            on({'N', 0x88, 0x89}, &PickleMachine::constant);
            on({'K', 'M', 'J'}, &PickleMachine::binary_int);
            on({0x8a, 0x8b}, &PickleMachine::long_int);
            on({'I', 'L'}, &PickleMachine::text_int);
            on({'G'}, &PickleMachine::binary_float);
            on({'F'}, &PickleMachine::text_float);
            on({0x8c, 'X', 0x8d, 'U', 'T'}, &PickleMachine::sized_text);
            on({'C', 'B', 0x8e, 0x96}, &PickleMachine::sized_bytes);
            on({'V', 'S'}, &PickleMachine::line_text);
            on({'(', }, &PickleMachine::mark);
            on({'0', '1', '2'}, &PickleMachine::stack_op);
            on({')', 't', 0x85, 0x86, 0x87}, &PickleMachine::make_tuple);
            on({']', 'l', 0x8f, 0x91}, &PickleMachine::make_list);
            on({'a', 'e', 0x90}, &PickleMachine::append);
            on({'}', 'd'}, &PickleMachine::make_dict);
            on({'s', 'u'}, &PickleMachine::set_items);
            on({'p', 'q', 'r', 0x94}, &PickleMachine::memo_put);
            on({'g', 'h', 'j'}, &PickleMachine::memo_get);
            on({'c', 0x93}, &PickleMachine::global);
            on({'R', 0x81, 0x92}, &PickleMachine::apply);
            on({'b'}, &PickleMachine::build);
            on({'P', 'Q'}, &PickleMachine::persistent);
            return t;
        }();
        return table;
    }

    // ---- input ----
    [[noreturn]] void fail(const std::string &what) const {
        bad("pickle, opcode at byte " + std::to_string(op_at_) + ": " + what);
    }
    const uint8_t *span(uint64_t n) {
        if (n > (uint64_t)(end_ - at_)) fail("the data ends " + std::to_string(n - (uint64_t)(end_ - at_)) +
                                             " bytes short of this opcode's argument");
        const uint8_t *p = at_;
        at_ += n;
        return p;
    }
    uint8_t byte() { return *span(1); }
    uint64_t unsigned_le(int bytes) {
        const uint8_t *p = span((uint64_t)bytes);
        uint64_t v = 0;
        for (int i = bytes - 1; i >= 0; --i) v = v << 8 | p[i];
        return v;
    }
    std::string line() {
        const uint8_t *nl = static_cast<const uint8_t *>(std::memchr(at_, '\n', (size_t)(end_ - at_)));
        if (!nl) fail("a text argument has no terminating newline");
        std::string s(reinterpret_cast<const char *>(at_), (size_t)(nl - at_));
        at_ = nl + 1;
        return s;
    }
    int64_t decimal(std::string t) {
        while (!t.empty() && (t.back() == 'L' || t.back() == ' ' || t.back() == '\r')) t.pop_back();
        errno = 0;
        char *stop = nullptr;
        const long long v = std::strtoll(t.c_str(), &stop, 10);
        if (t.empty() || *stop || errno) fail("`" + t + "` is not a 64-bit decimal integer");
        return (int64_t)v;
    }

    // ---- the value stack ----
    void push(PNodeRef n) { stack_.push_back(std::move(n)); }
    PNodeRef pop() {
        if (stack_.size() <= floor()) fail("the stack has no value above the last mark");
        PNodeRef n = std::move(stack_.back());
        stack_.pop_back();
        return n;
    }
    PNodeRef &top() {
        if (stack_.size() <= floor()) fail("the stack has no value above the last mark");
        return stack_.back();
    }
    size_t floor() const { return marks_.empty() ? 0 : marks_.back(); }
    std::vector<PNodeRef> pop_to_mark() {
        if (marks_.empty()) fail("no mark is set");
        const size_t m = marks_.back();
        marks_.pop_back();
        std::vector<PNodeRef> items(std::make_move_iterator(stack_.begin() + (ptrdiff_t)m),
                                    std::make_move_iterator(stack_.end()));
        stack_.resize(m);
        return items;
    }
    PNodeRef whole(int64_t v, PNode::Shape shape = PNode::Shape::Whole) {
        PNodeRef n = node(shape);
        n->whole = v;
        return n;
    }
    PNodeRef text(std::string s, PNode::Shape shape = PNode::Shape::Text) {
        PNodeRef n = node(shape);
        n->text = std::move(s);
        return n;
    }
    // The dict entries of a Table, or of the Apply result SETITEM(S) fill.
    std::vector<std::pair<PNodeRef, PNodeRef>> &entries_of(PNode &target) {
        if (target.shape != PNode::Shape::Table && target.shape != PNode::Shape::Apply)
            fail("items are stored into something that is neither a dict nor a constructed object");
        return target.table;
    }

    // ---- steps ----
    void proto(uint8_t) {
        if (byte() > 5) fail("protocol above 5");
    }
    void frame(uint8_t) { span(8); }  // frames only group the opcodes that follow
    void stop(uint8_t) { result_ = pop(); }  // whatever lies below the result is dropped, as CPython does
    void constant(uint8_t op) {
        if (op == 'N')
            push(node(PNode::Shape::Nil));
        else
            push(whole(op == 0x88 ? 1 : 0, PNode::Shape::Truth));
    }
    void binary_int(uint8_t op) {
        if (op == 'K') push(whole((int64_t)unsigned_le(1)));
        if (op == 'M') push(whole((int64_t)unsigned_le(2)));
        if (op == 'J') push(whole((int64_t)(int32_t)(uint32_t)unsigned_le(4)));
    }
    void long_int(uint8_t op) {  // two's complement, little-endian, of the given length
        const uint64_t n = op == 0x8a ? unsigned_le(1) : unsigned_le(4);
        if (n > 8) fail("an integer of " + std::to_string(n) + " bytes does not fit 64 bits");
        uint64_t v = n ? unsigned_le((int)n) : 0;
        if (n && n < 8 && (v >> (8 * n - 1)) & 1) v |= ~(uint64_t)0 << (8 * n);
        push(whole((int64_t)v));
    }
    void text_int(uint8_t op) {
        std::string t = line();
        // In protocol 0 the text "01" / "00" of INT spells True / False.
        if (op == 'I' && (t == "01" || t == "00"))
            push(whole(t == "01" ? 1 : 0, PNode::Shape::Truth));
        else
            push(whole(decimal(t)));
    }
    void binary_float(uint8_t) {
        PNodeRef n = node(PNode::Shape::Real);
        n->real = load_as<double>(span(8), true);
        push(n);
    }
    void text_float(uint8_t) {
        PNodeRef n = node(PNode::Shape::Real);
        n->real = std::strtod(line().c_str(), nullptr);
        push(n);
    }
    void sized_text(uint8_t op) {
        const uint64_t n = op == 0x8c || op == 'U' ? unsigned_le(1) : op == 0x8d ? unsigned_le(8) : unsigned_le(4);
        push(text(std::string(reinterpret_cast<const char *>(span(n)), (size_t)n)));
    }
    void sized_bytes(uint8_t op) {
        const uint64_t n = op == 'C' ? unsigned_le(1) : op == 'B' ? unsigned_le(4) : unsigned_le(8);
        push(text(std::string(reinterpret_cast<const char *>(span(n)), (size_t)n), PNode::Shape::Raw));
    }
    void line_text(uint8_t op) {
        std::string t = line();
        // STRING carries a quoted literal; only plain text inside the quotes is kept.
        if (op == 'S' && t.size() >= 2 && (t[0] == '\'' || t[0] == '"') && t.back() == t[0]) t = t.substr(1, t.size() - 2);
        push(text(t));
    }
    void mark(uint8_t) { marks_.push_back(stack_.size()); }
    void stack_op(uint8_t op) {
        if (op == '0') pop();
        if (op == '1') pop_to_mark();
        if (op == '2') push(top());
    }
    void make_tuple(uint8_t op) {
        PNodeRef n = node(PNode::Shape::Row);
        n->tuple = true;
        if (op == 't') {
            n->row = pop_to_mark();
        } else if (op != ')') {
            const int k = op - 0x84;  // TUPLE1..3
            n->row.resize((size_t)k);
            for (int i = k - 1; i >= 0; --i) n->row[(size_t)i] = pop();
        }
        push(n);
    }
    void make_list(uint8_t op) {  // lists, and sets read as lists
        PNodeRef n = node(PNode::Shape::Row);
        if (op == 'l' || op == 0x91) n->row = pop_to_mark();
        push(n);
    }
    void append(uint8_t op) {
        std::vector<PNodeRef> items;
        if (op == 'a')
            items.push_back(pop());
        else
            items = pop_to_mark();
        PNode &list = *top();
        if (list.shape != PNode::Shape::Row || list.tuple) fail("items are appended to something that is not a list");
        list.row.insert(list.row.end(), items.begin(), items.end());
    }
    void make_dict(uint8_t op) {
        PNodeRef n = node(PNode::Shape::Table);
        if (op == 'd') {
            std::vector<PNodeRef> kv = pop_to_mark();
            if (kv.size() % 2) fail("a dict is built from an odd number of values");
            for (size_t i = 0; i < kv.size(); i += 2) n->table.emplace_back(kv[i], kv[i + 1]);
        }
        push(n);
    }
    void set_items(uint8_t op) {
        std::vector<PNodeRef> kv;
        if (op == 's') {
            PNodeRef v = pop(), k = pop();
            kv = {k, v};
        } else {
            kv = pop_to_mark();
            if (kv.size() % 2) fail("SETITEMS is given an odd number of values");
        }
        auto &dst = entries_of(*top());
        for (size_t i = 0; i < kv.size(); i += 2) dst.emplace_back(kv[i], kv[i + 1]);
    }
    void memo_put(uint8_t op) {
        const uint64_t slot = op == 'q' ? unsigned_le(1) : op == 'r' ? unsigned_le(4) : op == 'p'
                                                                              ? (uint64_t)decimal(line())
                                                                              : (uint64_t)memo_.size();
        memo_[slot] = top();
    }
    void memo_get(uint8_t op) {
        const uint64_t slot = op == 'h' ? unsigned_le(1) : op == 'j' ? unsigned_le(4) : (uint64_t)decimal(line());
        const auto it = memo_.find(slot);
        if (it == memo_.end()) fail("memo slot " + std::to_string(slot) + " is read before it is written");
        push(it->second);
    }
    void global(uint8_t op) {
        std::string module, qualname;
        if (op == 'c') {
            module = line();
            qualname = line();
        } else {
            PNodeRef q = pop(), m = pop();
            if (m->shape != PNode::Shape::Text || q->shape != PNode::Shape::Text)
                fail("STACK_GLOBAL needs two strings");
            module = m->text;
            qualname = q->text;
        }
        push(text(module + "." + qualname, PNode::Shape::Name));  // a name only, never resolved
    }
    void apply(uint8_t op) {
        PNodeRef kwargs = op == 0x92 ? pop() : nullptr;  // NEWOBJ_EX: cls, args, kwargs
        PNodeRef args = pop(), callee = pop();
        if (callee->shape != PNode::Shape::Name) fail("a call whose callee is not a global name");
        if (args->shape != PNode::Shape::Row) fail("a call whose arguments are not a tuple");
        PNodeRef n = node(PNode::Shape::Apply);
        n->callee = callee;
        n->row = args->row;
        if (kwargs && kwargs->shape == PNode::Shape::Table) n->table = kwargs->table;
        push(n);
    }
    void build(uint8_t) {
        PNodeRef state = pop();
        PNode &target = *top();
        if (target.shape == PNode::Shape::Apply) target.state = state;  // other targets keep no state
    }
    void persistent(uint8_t op) {
        PNodeRef n = node(PNode::Shape::Persistent);
        if (op == 'Q') {
            PNodeRef id = pop();
            if (id->shape != PNode::Shape::Row) fail("a persistent id that is not a tuple");
            n->row = id->row;
        } else {
            n->row = repr_tuple(line());
        }
        push(n);
    }
    // PERSID carries the id as the text of a Python tuple, e.g.
    // ('storage', <class 'torch.FloatStorage'>, '0', 'cpu', 2): quoted
    // strings, <class '...'> names and decimal integers are read.
    std::vector<PNodeRef> repr_tuple(const std::string &t) {
        std::vector<PNodeRef> items;
        size_t i = t.find('(');
        if (i == std::string::npos) fail("a text persistent id that is not a tuple");
        ++i;
        while (i < t.size() && t[i] != ')') {
            while (i < t.size() && (t[i] == ' ' || t[i] == ',')) ++i;
            if (i >= t.size() || t[i] == ')') break;
            if (t[i] == '\'' || t[i] == '"') {
                const size_t close = t.find(t[i], i + 1);
                if (close == std::string::npos) fail("an unterminated string in a persistent id");
                items.push_back(text(t.substr(i + 1, close - i - 1)));
                i = close + 1;
            } else if (t.compare(i, 8, "<class '") == 0) {
                const size_t close = t.find("'>", i + 8);
                if (close == std::string::npos) fail("an unterminated class name in a persistent id");
                items.push_back(text(t.substr(i + 8, close - i - 8), PNode::Shape::Name));
                i = close + 2;
            } else {
                const size_t stop = t.find_first_of(",)", i);
                items.push_back(whole(decimal(t.substr(i, stop == std::string::npos ? std::string::npos : stop - i))));
                i = stop == std::string::npos ? t.size() : stop;
            }
        }
        return items;
    }

    const uint8_t *begin_, *at_, *end_;
    size_t op_at_ = 0;
    std::vector<PNodeRef> stack_;
    std::vector<size_t> marks_;
    std::map<uint64_t, PNodeRef> memo_;
    PNodeRef result_;
};

// ----- torch's objects in an evaluated pickle -----

// A storage's element type from its class name ("torch.HalfStorage") or
// dtype name ("torch.float16"): the part between "torch." and "Storage",
// lower-cased, names the element type.
bool torch_element_type(std::string s, DType &t) {
    std::transform(s.begin(), s.end(), s.begin(), [](unsigned char ch) { return (char)std::tolower(ch); });
    if (s.rfind("torch.", 0) == 0) s.erase(0, 6);
    if (s.size() > 7 && s.compare(s.size() - 7, 7, "storage") == 0) s.erase(s.size() - 7);
    static const std::map<std::string, DType> types = {
        {"bool", DType::Bool},   {"byte", DType::U8},      {"uint8", DType::U8},    {"char", DType::I8},
        {"int8", DType::I8},     {"short", DType::I16},    {"int16", DType::I16},   {"int", DType::I32},
        {"int32", DType::I32},   {"long", DType::I64},     {"int64", DType::I64},   {"half", DType::F16},
        {"float16", DType::F16}, {"bfloat16", DType::BF16}, {"float", DType::F32},  {"float32", DType::F32},
        {"double", DType::F64},  {"float64", DType::F64}};
    const auto it = types.find(s);
    if (it == types.end()) return false;
    t = it->second;
    return true;
}

struct TorchStorage {
    DType type = DType::F32;
    std::string key;  // archive entry <root>/data/<key>
    int64_t numel = 0;
};

struct TorchTensor {
    TorchStorage storage;
    int64_t offset = 0;
    std::vector<int64_t> size, stride;
};

bool is_call(const PNode &n, const char *name) {
    return n.shape == PNode::Shape::Apply && n.callee && n.callee->text == name;
}

std::vector<int64_t> whole_list(const PNode &n, const std::string &what) {
    if (n.shape != PNode::Shape::Row) bad("torch tensor: " + what + " is not a tuple");
    std::vector<int64_t> out;
    for (const PNodeRef &x : n.row) {
        if (x->shape != PNode::Shape::Whole) bad("torch tensor: " + what + " holds a value that is not an integer");
        out.push_back(x->whole);
    }
    return out;
}

// The storage a persistent id ("storage", <storage class>, key, location,
// numel) points at.
TorchStorage torch_storage(const PNode &id) {
    if (id.shape != PNode::Shape::Persistent || id.row.size() < 5 || id.row[0]->shape != PNode::Shape::Text ||
        id.row[0]->text != "storage")
        bad("torch tensor: its storage is not a (\"storage\", class, key, location, size) reference");
    const PNode &cls = *id.row[1], &key = *id.row[2], &numel = *id.row[4];
    TorchStorage s;
    if (cls.shape != PNode::Shape::Name || !torch_element_type(cls.text, s.type))
        bad("torch tensor: storage class `" + cls.text + "` has no element type this reader knows");
    if (key.shape != PNode::Shape::Text) bad("torch tensor: the storage key is not a string");
    if (numel.shape != PNode::Shape::Whole || numel.whole < 0) bad("torch tensor: the storage size is not a count");
    s.key = key.text;
    s.numel = numel.whole;
    return s;
}

// A dense tensor value: _rebuild_tensor(_v2)(storage, offset, size, stride,
// ...), possibly wrapped in _rebuild_parameter(tensor, requires_grad, hooks).
// Returns false for every other value.
bool torch_tensor(const PNode &n, TorchTensor &t) {
    if (is_call(n, "torch._utils._rebuild_parameter") || is_call(n, "torch._utils._rebuild_parameter_with_state"))
        return !n.row.empty() && torch_tensor(*n.row[0], t);
    if (!is_call(n, "torch._utils._rebuild_tensor_v2") && !is_call(n, "torch._utils._rebuild_tensor")) return false;
    if (n.row.size() < 4) bad("torch tensor: the rebuild call has fewer than four arguments");
    t.storage = torch_storage(*n.row[0]);
    if (n.row[1]->shape != PNode::Shape::Whole || n.row[1]->whole < 0)
        bad("torch tensor: the storage offset is not a count");
    t.offset = n.row[1]->whole;
    t.size = whole_list(*n.row[2], "the size");
    t.stride = whole_list(*n.row[3], "the stride");
    if (t.size.size() != t.stride.size()) bad("torch tensor: size and stride have different lengths");
    return true;
}

// Torch's rebuild functions this reader does not read (sparse, quantized,
// meta, ...): a state-dict entry made by one of them is an error, not skipped.
bool unreadable_torch_tensor(const PNode &n) {
    return n.shape == PNode::Shape::Apply && n.callee && n.callee->text.rfind("torch._utils._rebuild_", 0) == 0;
}

// The (key, value) entries of a mapping: a dict, or an OrderedDict call
// (given its items as an argument, filled by SETITEMS, or both).
bool mapping_entries(const PNode &n, std::vector<std::pair<PNodeRef, PNodeRef>> &out) {
    out.clear();
    if (n.shape == PNode::Shape::Table) {
        out = n.table;
        return true;
    }
    if (!is_call(n, "collections.OrderedDict")) return false;
    if (!n.row.empty()) {
        const PNode &items = *n.row[0];
        if (items.shape == PNode::Shape::Table) {
            out = items.table;
        } else if (items.shape == PNode::Shape::Row) {
            for (const PNodeRef &pair : items.row) {
                if (pair->shape != PNode::Shape::Row || pair->row.size() != 2)
                    bad("checkpoint: an OrderedDict item is not a (key, value) pair");
                out.emplace_back(pair->row[0], pair->row[1]);
            }
        } else {
            bad("checkpoint: OrderedDict is built from a value that holds no items");
        }
    }
    out.insert(out.end(), n.table.begin(), n.table.end());
    return true;
}

bool holds_a_tensor(const std::vector<std::pair<PNodeRef, PNodeRef>> &entries) {
    TorchTensor t;
    for (const auto &kv : entries)
        if (torch_tensor(*kv.second, t)) return true;
    return false;
}

// The state dict of a checkpoint: the top-level mapping itself, or its
// "model_state_dict", "state_dict" or "state" entry (a training checkpoint or
// a demucs package around it) -- whichever first holds a tensor.
std::vector<std::pair<PNodeRef, PNodeRef>> find_state_dict(const PNode &top) {
    std::vector<std::pair<PNodeRef, PNodeRef>> entries, inner;
    if (!mapping_entries(top, entries)) bad("checkpoint: the pickled object is not a dict");
    for (const char *wrapper : {"model_state_dict", "state_dict", "state"})
        for (const auto &kv : entries)
            if (kv.first->shape == PNode::Shape::Text && kv.first->text == wrapper &&
                mapping_entries(*kv.second, inner) && holds_a_tensor(inner))
                return inner;
    if (holds_a_tensor(entries)) return entries;
    bad("checkpoint: neither the pickled dict nor a model_state_dict / state_dict / state entry of it holds a tensor");
}

// A tensor's values as f32, read through its size and stride from the
// storage's bytes.
Tensor gather(const std::string &name, const TorchTensor &t, const uint8_t *blob, uint64_t blob_bytes, bool big) {
    const int es = dtype_size(t.storage.type);
    if (blob_bytes % (uint64_t)es) bad("checkpoint: storage " + t.storage.key + " is not a whole number of elements");
    if ((uint64_t)t.storage.numel > blob_bytes / (uint64_t)es)
        bad("checkpoint: storage " + t.storage.key + " is declared with " + std::to_string(t.storage.numel) +
            " elements but its entry holds " + std::to_string(blob_bytes / (uint64_t)es));
    Tensor out;
    out.shape = t.size;
    const uint64_t n = checked_product(out.shape, name);
    out.data.resize(n);
    if (n == 0) return out;
    // Highest storage index the view touches: offset + sum (size_d - 1) stride_d.
    int64_t last = t.offset;
    for (size_t d = 0; d < t.size.size(); ++d) {
        if (t.stride[d] < 0) bad("checkpoint: tensor `" + name + "` has a negative stride");
        if (t.size[d] > 1 && t.stride[d] > (std::numeric_limits<int64_t>::max() - last) / (t.size[d] - 1))
            bad("checkpoint: tensor `" + name + "` reaches past the end of its storage");
        last += (t.size[d] - 1) * t.stride[d];
    }
    if (last >= t.storage.numel) bad("checkpoint: tensor `" + name + "` reaches past the end of its storage");
    // Row-major walk; the innermost dimension is decoded as one strided run.
    const size_t rank = t.size.size();
    const int64_t inner = rank ? t.size[rank - 1] : 1, inner_stride = rank ? t.stride[rank - 1] : 1;
    std::vector<int64_t> idx(rank ? rank - 1 : 0, 0);
    for (uint64_t at_out = 0; at_out < n; at_out += (uint64_t)inner) {
        int64_t base = t.offset;
        for (size_t d = 0; d + 1 < rank; ++d) base += idx[d] * t.stride[d];
        if (inner_stride == 1) {
            decode(blob + (uint64_t)base * es, (size_t)inner, t.storage.type, big, &out.data[at_out]);
        } else {
            for (int64_t i = 0; i < inner; ++i)
                decode(blob + (uint64_t)(base + i * inner_stride) * es, 1, t.storage.type, big, &out.data[at_out + i]);
        }
        for (size_t d = idx.size(); d-- > 0;) {
            if (++idx[d] < t.size[d]) break;
            idx[d] = 0;
        }
    }
    return out;
}

// A torch.save archive: "<root>/data.pkl", one "<root>/data/<key>" entry per
// storage, and "<root>/byteorder" ("little" when absent).
void parse_torch_zip(const uint8_t *z, size_t len, dmx_checkpoint &c) {
    const auto dir = zip_directory(z, len);
    const std::string suffix = "/data.pkl";
    auto pkl = dir.end();
    for (auto it = dir.begin(); it != dir.end(); ++it)
        if (it->first.size() > suffix.size() &&
            it->first.compare(it->first.size() - suffix.size(), suffix.size(), suffix) == 0) {
            pkl = it;
            break;
        }
    if (pkl == dir.end()) bad("checkpoint: the archive has no `<root>/data.pkl` entry; it is not a torch.save file");
    const std::string root = pkl->first.substr(0, pkl->first.size() - suffix.size());
    bool big = false;
    if (const auto bo = dir.find(root + "/byteorder"); bo != dir.end()) {
        const auto d = zip_data(z, len, bo->second, bo->first);
        big = std::string(reinterpret_cast<const char *>(d.first), (size_t)d.second).rfind("big", 0) == 0;
    }
    const auto program = zip_data(z, len, pkl->second, pkl->first);
    const PNodeRef top = PickleMachine(program.first, (size_t)program.second).evaluate();
    for (const auto &kv : find_state_dict(*top)) {
        if (kv.first->shape != PNode::Shape::Text) bad("checkpoint: a state-dict key is not a string");
        const std::string &name = kv.first->text;
        TorchTensor t;
        if (!torch_tensor(*kv.second, t)) {
            if (unreadable_torch_tensor(*kv.second))
                bad("checkpoint: tensor `" + name + "` is stored by " + kv.second->callee->text +
                    ", which this reader does not read (only dense tensors)");
            const PNode::Shape sh = kv.second->shape;
            if (sh == PNode::Shape::Nil || sh == PNode::Shape::Apply || sh == PNode::Shape::Name) continue;
            bad("checkpoint: state-dict entry `" + name + "` is a plain value, not a tensor");
        }
        const auto blob = dir.find(root + "/data/" + t.storage.key);
        if (blob == dir.end()) bad("checkpoint: the archive lacks the storage entry " + root + "/data/" + t.storage.key);
        const auto bytes = zip_data(z, len, blob->second, blob->first);
        c.tensors[name] = gather(name, t, bytes.first, bytes.second, big);
    }
}

std::vector<uint8_t> read_file(const char *path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw Error(ERR_IO, std::string(path) + ": cannot open");
    const std::streamsize n = f.tellg();
    f.seekg(0);
    std::vector<uint8_t> bytes((size_t)std::max<std::streamsize>(n, 0));
    if (n > 0 && !f.read(reinterpret_cast<char *>(bytes.data()), n)) throw Error(ERR_IO, std::string(path) + ": read failed");
    return bytes;
}

bool is_torch_extension(const char *path) {
    std::string p(path);
    const size_t dot = p.find_last_of('.'), slash = p.find_last_of('/');
    if (dot == std::string::npos || (slash != std::string::npos && dot < slash)) return false;
    std::string ext = p.substr(dot + 1);
    std::transform(ext.begin(), ext.end(), ext.begin(), [](unsigned char ch) { return (char)std::tolower(ch); });
    return ext == "th" || ext == "pth" || ext == "pt";
}

int load_into(const uint8_t *bytes, size_t len, int torch_zip, dmx_checkpoint **out) {
    auto c = std::make_unique<dmx_checkpoint>();
    dmx_config_default(&c->config);
    if (torch_zip)
        parse_torch_zip(bytes, len, *c);
    else
        parse_safetensors(bytes, len, *c);
    finish(*c);
    *out = c.release();
    return 0;
}

}  // namespace
}  // namespace dmx

extern "C" {

int dmx_checkpoint_load(const char *path, dmx_checkpoint **out) {
    if (!path || !out) {
        dmx::last_error_slot() = "dmx_checkpoint_load: null argument";
        return DMX_ERR_ARGUMENT;
    }
    *out = nullptr;
    return dmx::guarded([&] {
        const std::vector<uint8_t> bytes = dmx::read_file(path);
        try {
            dmx::load_into(bytes.data(), bytes.size(), dmx::is_torch_extension(path) ? 1 : 0, out);
        } catch (const dmx::Error &e) {
            throw dmx::Error(e.code, std::string(path) + ": " + e.what());
        }
    });
}

int dmx_checkpoint_from_bytes(const void *bytes, size_t len, int torch_zip, dmx_checkpoint **out) {
    if ((!bytes && len) || !out) {
        dmx::last_error_slot() = "dmx_checkpoint_from_bytes: null argument";
        return DMX_ERR_ARGUMENT;
    }
    *out = nullptr;
    return dmx::guarded([&] { dmx::load_into(static_cast<const uint8_t *>(bytes), len, torch_zip, out); });
}

void dmx_checkpoint_free(dmx_checkpoint *c) { delete c; }

size_t dmx_checkpoint_count(const dmx_checkpoint *c) { return c ? c->view.size() : 0; }

const dmx_tensor *dmx_checkpoint_tensors(const dmx_checkpoint *c) { return c && !c->view.empty() ? c->view.data() : nullptr; }

const char *dmx_checkpoint_metadata(const dmx_checkpoint *c, const char *key) {
    if (!c || !key) return nullptr;
    auto it = c->metadata.find(key);
    return it == c->metadata.end() ? nullptr : it->second.c_str();
}

size_t dmx_checkpoint_metadata_count(const dmx_checkpoint *c) { return c ? c->metadata.size() : 0; }

const char *dmx_checkpoint_metadata_key(const dmx_checkpoint *c, size_t i) {
    if (!c || i >= c->metadata.size()) return nullptr;
    auto it = c->metadata.begin();
    std::advance(it, (long)i);
    return it->first.c_str();
}

int dmx_checkpoint_config(const dmx_checkpoint *c, dmx_config *out) {
    if (!c || !out) {
        dmx::last_error_slot() = "dmx_checkpoint_config: null argument";
        return DMX_ERR_ARGUMENT;
    }
    *out = c->config;
    return DMX_OK;
}

int dmx_config_from_kwargs(const char *json, dmx_config *out) {
    if (!json || !out) {
        dmx::last_error_slot() = "dmx_config_from_kwargs: null argument";
        return DMX_ERR_ARGUMENT;
    }
    return dmx::guarded([&] {
        dmx_config cfg;
        dmx_config_default(&cfg);
        try {
            dmx::config_from_kwargs(dmx::parse_json(json, std::strlen(json)), cfg);
        } catch (const dmx::Error &e) {
            // JSON syntax errors are config errors here (from_kwargs_json, config.rs:151-152).
            throw dmx::Error(2, std::string("checkpoint kwargs are not valid: ") + e.what());
        }
        *out = cfg;
    });
}

}  // extern "C"
