// checkpoint.hip — host-side checkpoint readers behind include/dmx_ckpt.h
// (no device code).
//
// Two containers, as `load_weights` (crates/demucs-core/src/demucs/weights.rs:30-88)
// accepts them:
//   * safetensors (crates/demucs-core/src/safetensors.rs:38-139): u64 LE header
//     length, a JSON header {name: {dtype, shape, data_offsets}, "__metadata__":
//     {str: str}}, then the data; tensors of any listed dtype become f32, and the
//     model config comes from the "kwargs" metadata entry when present
//     (HtdemucsConfig::from_kwargs_json, config.rs:150-215);
//   * torch.save zips (crates/demucs-core/src/ckpt/mod.rs:43-120): "<root>/data.pkl"
//     (a pickle), "<root>/data/<key>" (one raw blob per storage) and
//     "<root>/byteorder". The pickle is read by a data-only interpreter
//     (ckpt/pickle.rs:140-460 models the same opcodes): it builds lists, dicts and
//     tuples, and recognises torch's tensor-rebuild and OrderedDict reductions by
//     name; every other reduction becomes an opaque value. Nothing named in the
//     file is imported or called. The state dict is the top-level dict or its
//     "model_state_dict" / "state_dict" / "state" entry (mod.rs:232-256).
// Tensors are kept sorted by name, each contiguous row-major f32.
#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cmath>
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

bool safetensors_dtype(const std::string &s, DType &t) {
    static const std::pair<const char *, DType> table[] = {
        {"F32", DType::F32}, {"F64", DType::F64}, {"F16", DType::F16}, {"BF16", DType::BF16},
        {"I64", DType::I64}, {"I32", DType::I32}, {"I16", DType::I16}, {"I8", DType::I8},
        {"U8", DType::U8},   {"BOOL", DType::Bool}};
    for (const auto &e : table)
        if (s == e.first) {
            t = e.second;
            return true;
        }
    return false;
}

// Storage class ("HalfStorage") or dtype ("torch.float16", "float16") spellings.
bool torch_dtype(std::string s, DType &t) {
    std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::tolower(c); });
    if (s.rfind("torch.", 0) == 0) s = s.substr(6);
    static const std::pair<const char *, DType> table[] = {
        {"floatstorage", DType::F32},  {"float", DType::F32},    {"float32", DType::F32},
        {"halfstorage", DType::F16},   {"half", DType::F16},     {"float16", DType::F16},
        {"bfloat16storage", DType::BF16}, {"bfloat16", DType::BF16},
        {"doublestorage", DType::F64}, {"double", DType::F64},   {"float64", DType::F64},
        {"bytestorage", DType::U8},    {"uint8", DType::U8},     {"charstorage", DType::I8},
        {"int8", DType::I8},           {"shortstorage", DType::I16}, {"int16", DType::I16},
        {"intstorage", DType::I32},    {"int32", DType::I32},    {"longstorage", DType::I64},
        {"int64", DType::I64},         {"boolstorage", DType::Bool}, {"bool", DType::Bool}};
    for (const auto &e : table)
        if (s == e.first) {
            t = e.second;
            return true;
        }
    return false;
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

void parse_safetensors(const uint8_t *bytes, size_t len, dmx_checkpoint &c) {
    if (len < 8) bad("safetensors file is shorter than its header length");
    uint64_t hlen;
    std::memcpy(&hlen, bytes, 8);  // little-endian host
    if (hlen > len - 8)
        bad("safetensors header claims " + std::to_string(hlen) + " bytes but the file holds " + std::to_string(len));
    const Json header = parse_json(reinterpret_cast<const char *>(bytes) + 8, (size_t)hlen);
    if (header.kind != Json::Object) bad("safetensors header is not an object");
    const uint8_t *data = bytes + 8 + hlen;
    const uint64_t data_len = len - 8 - hlen;
    for (const auto &m : header.members) {
        const std::string &name = m.first;
        const Json &e = m.second;
        if (name == "__metadata__") {
            for (const auto &kv : e.members)
                if (kv.second.kind == Json::String) c.metadata[kv.first] = kv.second.str;
            continue;
        }
        const Json *dt = e.get("dtype"), *sh = e.get("shape"), *off = e.get("data_offsets");
        if (!dt || dt->kind != Json::String) bad(name + ": no dtype");
        if (!sh || sh->kind != Json::Array) bad(name + ": no shape");
        if (!off || off->kind != Json::Array) bad(name + ": no data_offsets");
        if (off->items.size() != 2) bad(name + ": malformed data_offsets");
        DType t;
        if (!safetensors_dtype(dt->str, t)) bad(name + ": unsupported safetensors dtype " + dt->str);
        Tensor tensor;
        for (const Json &d : sh->items) {
            if (d.kind != Json::Number || !d.integral || d.inum < 0) bad(name + ": bad shape entry");
            tensor.shape.push_back(d.inum);
        }
        for (const Json &o : off->items)
            if (o.kind != Json::Number || !o.integral || o.inum < 0) bad(name + ": bad data offset");
        const uint64_t begin = (uint64_t)off->items[0].inum, stop = (uint64_t)off->items[1].inum;
        if (stop < begin || stop > data_len)
            bad(name + ": data range [" + std::to_string(begin) + ", " + std::to_string(stop) + ") is outside the " +
                std::to_string(data_len) + " data bytes");
        const uint64_t n = checked_product(tensor.shape, name);
        if (stop - begin != n * (uint64_t)dtype_size(t))
            bad(name + ": " + std::to_string(stop - begin) + " data bytes do not match " + std::to_string(n) +
                " elements of " + dt->str);
        tensor.data.resize(n);
        decode(data + begin, n, t, false, tensor.data.data());
        c.tensors[name] = std::move(tensor);
    }
    auto kw = c.metadata.find("kwargs");
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

// ----- the pickle interpreter -----

struct PVal;
using PRef = std::shared_ptr<PVal>;

struct StorageRef {
    DType dtype = DType::F32;
    std::string key;
    int64_t numel = 0;
};
struct TensorRef {
    StorageRef storage;
    int64_t offset = 0;
    bool dense = false;  // false: a sparse layout (not supported)
    std::vector<int64_t> size, stride;
};

struct PVal {
    enum Kind { None, Bool, Int, Float, Str, Bytes, Tuple, List, Dict, Global, Storage, Tensor, Opaque } kind = None;
    int64_t i = 0;
    double f = 0.0;
    std::string s, s2;  // Str / Bytes / Opaque: s; Global: module s, name s2
    std::vector<PRef> items;
    std::vector<std::pair<PRef, PRef>> dict;
    StorageRef storage;
    TensorRef tensor;
};

PRef mk(PVal::Kind k) {
    auto v = std::make_shared<PVal>();
    v->kind = k;
    return v;
}

class Unpickler {
  public:
    Unpickler(const uint8_t *p, size_t n) : p_(p), end_(p + n) {}

    PRef run() {
        while (true) {
            const uint8_t op = u8();
            switch (op) {
                case 0x80: u8(); break;                     // PROTO
                case '.': return pop();                     // STOP
                case 0x95: take(8); break;                  // FRAME
                case '(': marks_.push_back(stack_.size()); break;  // MARK
                case ')': push(mk(PVal::Tuple)); break;    // EMPTY_TUPLE
                case ']': push(mk(PVal::List)); break;     // EMPTY_LIST
                case '}': push(mk(PVal::Dict)); break;     // EMPTY_DICT
                case 'N': push(mk(PVal::None)); break;     // NONE
                case 0x88: push_bool(true); break;         // NEWTRUE
                case 0x89: push_bool(false); break;        // NEWFALSE
                case 'K': push_int(u8()); break;           // BININT1
                case 'M': push_int(rd16(take(2))); break;  // BININT2
                case 'J': push_int((int32_t)rd32(take(4))); break;  // BININT
                case 'I': {                                // INT (text)
                    std::string t = line();
                    while (!t.empty() && (t.back() == 'L' || t.back() == ' ')) t.pop_back();
                    if (t == "01") push_bool(true);
                    else if (t == "00") push_bool(false);
                    else push_int(parse_int(t));
                    break;
                }
                case 0x8a: push_int(long_le(take(u8()), 0)); break;  // LONG1
                case 0x8b: {                                          // LONG4
                    const uint32_t n = rd32(take(4));
                    push_int(long_le(take(n), n));
                    break;
                }
                case 'F': {  // FLOAT (text)
                    auto v = mk(PVal::Float);
                    v->f = std::strtod(line().c_str(), nullptr);
                    push(v);
                    break;
                }
                case 'G': {  // BINFLOAT, big-endian
                    auto v = mk(PVal::Float);
                    v->f = load_as<double>(take(8), true);
                    push(v);
                    break;
                }
                case 'X': push_str(PVal::Str, rd32(take(4))); break;      // BINUNICODE
                case 0x8c: push_str(PVal::Str, u8()); break;             // SHORT_BINUNICODE
                case 0x8d: push_str(PVal::Str, rd64(take(8))); break;    // BINUNICODE8
                case 'C': push_str(PVal::Bytes, u8()); break;            // SHORT_BINBYTES
                case 'B': push_str(PVal::Bytes, rd32(take(4))); break;   // BINBYTES
                case 0x8e: push_str(PVal::Bytes, rd64(take(8))); break;  // BINBYTES8
                case 't': {  // TUPLE
                    auto v = mk(PVal::Tuple);
                    v->items = pop_mark();
                    push(v);
                    break;
                }
                case 0x85: case 0x86: case 0x87: {  // TUPLE1..3
                    const int n = op - 0x84;
                    auto v = mk(PVal::Tuple);
                    if (stack_.size() < (size_t)n) fail("stack underflow");
                    v->items.assign(stack_.end() - n, stack_.end());
                    stack_.resize(stack_.size() - n);
                    push(v);
                    break;
                }
                case 'l': {  // LIST
                    auto v = mk(PVal::List);
                    v->items = pop_mark();
                    push(v);
                    break;
                }
                case 'a': {  // APPEND
                    PRef item = pop();
                    top(PVal::List, "APPEND")->items.push_back(item);
                    break;
                }
                case 'e': {  // APPENDS
                    auto items = pop_mark();
                    auto &dst = top(PVal::List, "APPENDS")->items;
                    dst.insert(dst.end(), items.begin(), items.end());
                    break;
                }
                case 'd': {  // DICT
                    auto v = mk(PVal::Dict);
                    v->dict = pairs(pop_mark());
                    push(v);
                    break;
                }
                case 's': {  // SETITEM
                    PRef val = pop(), key = pop();
                    top(PVal::Dict, "SETITEM")->dict.emplace_back(key, val);
                    break;
                }
                case 'u': {  // SETITEMS
                    auto kv = pairs(pop_mark());
                    auto &dst = top(PVal::Dict, "SETITEMS")->dict;
                    dst.insert(dst.end(), kv.begin(), kv.end());
                    break;
                }
                case 'c': {  // GLOBAL: a name only, never resolved
                    auto v = mk(PVal::Global);
                    v->s = line();
                    v->s2 = line();
                    push(v);
                    break;
                }
                case 0x93: {  // STACK_GLOBAL
                    PRef name = pop(), module = pop();
                    auto v = mk(PVal::Global);
                    v->s = text(module);
                    v->s2 = text(name);
                    push(v);
                    break;
                }
                case 'q': memoize(u8()); break;          // BINPUT
                case 'r': memoize(rd32(take(4))); break;  // LONG_BINPUT
                case 0x94: memoize(memo_.size()); break;  // MEMOIZE
                case 'p': memoize((uint64_t)parse_int(line())); break;  // PUT
                case 'h': push(recall(u8())); break;                  // BINGET
                case 'j': push(recall(rd32(take(4)))); break;         // LONG_BINGET
                case 'g': push(recall((uint64_t)parse_int(line()))); break;  // GET
                case 'Q': push(persistent(pop())); break;             // BINPERSID
                case 'P': {                                           // PERSID (text)
                    auto v = mk(PVal::Opaque);
                    v->s = "PERSID(" + line() + ")";
                    push(v);
                    break;
                }
                case 'R': {  // REDUCE
                    PRef args = pop(), fn = pop();
                    push(reduce(fn, args));
                    break;
                }
                case 0x81: {  // NEWOBJ
                    PRef args = pop(), cls = pop();
                    push(reduce(cls, args));
                    break;
                }
                case 0x92: {  // NEWOBJ_EX
                    pop();
                    PRef args = pop(), cls = pop();
                    push(reduce(cls, args));
                    break;
                }
                case 'b': pop(); break;  // BUILD: object state (OrderedDict metadata, ...) is not needed
                case '0': pop(); break;  // POP
                case '1': pop_mark(); break;  // POP_MARK
                case '2': push(top_any()); break;  // DUP
                default: {
                    char buf[64];
                    std::snprintf(buf, sizeof buf, "unsupported pickle opcode 0x%02x at offset %zu", op,
                                  (size_t)(p_ - start_) - 1);
                    bad(buf);
                }
            }
        }
    }

  private:
    const uint8_t *p_, *end_, *start_ = p_;
    std::vector<PRef> stack_;
    std::vector<size_t> marks_;
    std::map<uint64_t, PRef> memo_;

    [[noreturn]] void fail(const std::string &m) { bad("pickle: " + m); }
    const uint8_t *take(uint64_t n) {
        if (n > (uint64_t)(end_ - p_)) fail("truncated stream");
        const uint8_t *q = p_;
        p_ += n;
        return q;
    }
    uint8_t u8() { return *take(1); }
    std::string line() {
        const uint8_t *q = p_;
        while (q < end_ && *q != '\n') ++q;
        if (q >= end_) fail("unterminated line");
        std::string s(reinterpret_cast<const char *>(p_), q - p_);
        p_ = q + 1;
        while (!s.empty() && (s.back() == '\r' || s.back() == ' ')) s.pop_back();
        return s;
    }
    int64_t parse_int(const std::string &t) {
        char *e = nullptr;
        errno = 0;
        const long long v = std::strtoll(t.c_str(), &e, 10);
        if (t.empty() || *e || errno) fail("bad integer literal `" + t + "`");
        return v;
    }
    int64_t long_le(const uint8_t *b, uint64_t n) {
        if (n == 0) return 0;
        if (n > 8) fail("integer literal of " + std::to_string(n) + " bytes exceeds 64 bits");
        uint8_t buf[8];
        std::memset(buf, (b[n - 1] & 0x80) ? 0xff : 0x00, 8);
        std::memcpy(buf, b, n);
        return load_as<int64_t>(buf, false);
    }
    void push(PRef v) { stack_.push_back(std::move(v)); }
    void push_int(int64_t x) {
        auto v = mk(PVal::Int);
        v->i = x;
        push(v);
    }
    void push_bool(bool x) {
        auto v = mk(PVal::Bool);
        v->i = x;
        push(v);
    }
    void push_str(PVal::Kind k, uint64_t n) {
        auto v = mk(k);
        const uint8_t *q = take(n);
        v->s.assign(reinterpret_cast<const char *>(q), n);
        push(v);
    }
    PRef pop() {
        if (stack_.empty()) fail("stack underflow");
        PRef v = stack_.back();
        stack_.pop_back();
        return v;
    }
    PRef top_any() {
        if (stack_.empty()) fail("stack underflow");
        return stack_.back();
    }
    PVal *top(PVal::Kind k, const char *op) {
        if (stack_.empty() || stack_.back()->kind != k) fail(std::string(op) + " on the wrong kind of object");
        return stack_.back().get();
    }
    std::vector<PRef> pop_mark() {
        if (marks_.empty()) fail("MARK stack underflow");
        const size_t m = marks_.back();
        marks_.pop_back();
        if (m > stack_.size()) fail("MARK past the stack");
        std::vector<PRef> out(stack_.begin() + m, stack_.end());
        stack_.resize(m);
        return out;
    }
    std::vector<std::pair<PRef, PRef>> pairs(const std::vector<PRef> &v) {
        if (v.size() % 2) fail("odd number of items in a dict");
        std::vector<std::pair<PRef, PRef>> out;
        for (size_t i = 0; i < v.size(); i += 2) out.emplace_back(v[i], v[i + 1]);
        return out;
    }
    void memoize(uint64_t idx) { memo_[idx] = top_any(); }
    PRef recall(uint64_t idx) {
        auto it = memo_.find(idx);
        if (it == memo_.end()) fail("memo has no entry " + std::to_string(idx));
        return it->second;
    }
    static std::string text(const PRef &v) {
        if (v->kind != PVal::Str && v->kind != PVal::Bytes) bad("pickle: expected a string");
        return v->s;
    }
    static int64_t integer(const PRef &v) {
        if (v->kind != PVal::Int && v->kind != PVal::Bool) bad("pickle: expected an integer");
        return v->i;
    }
    static const std::vector<PRef> &seq(const PRef &v) {
        if (v->kind != PVal::Tuple && v->kind != PVal::List) bad("pickle: expected a tuple");
        return v->items;
    }

    // ('storage', <class or dtype name>, key, location, numel)
    PRef persistent(const PRef &pid) {
        const auto &it = seq(pid);
        if (it.size() < 5 || it[0]->kind != PVal::Str || it[0]->s != "storage") fail("unsupported persistent id");
        DType t;
        const std::string cls = it[1]->kind == PVal::Global ? it[1]->s2 : text(it[1]);
        if (!torch_dtype(cls, t)) fail("unknown storage type " + cls);
        auto v = mk(PVal::Storage);
        v->storage.dtype = t;
        v->storage.key = text(it[2]);
        v->storage.numel = integer(it[4]);
        if (v->storage.numel < 0) fail("negative storage size");
        return v;
    }

    PRef reduce(const PRef &fn, const PRef &args) {
        if (fn->kind != PVal::Global) fail("REDUCE with a callable that is not a global name");
        const std::string &mod = fn->s, &name = fn->s2;
        if (mod == "collections" && name == "OrderedDict") {
            const auto &a = seq(args);
            auto d = mk(PVal::Dict);
            if (a.empty()) return d;
            if (a[0]->kind == PVal::Dict) {
                d->dict = a[0]->dict;
            } else if (a[0]->kind == PVal::List || a[0]->kind == PVal::Tuple) {
                for (const PRef &kv : a[0]->items) {
                    const auto &p = seq(kv);
                    if (p.size() != 2) fail("OrderedDict item is not a pair");
                    d->dict.emplace_back(p[0], p[1]);
                }
            } else {
                fail("OrderedDict from an unsupported value");
            }
            return d;
        }
        if (mod == "torch._utils" &&
            (name == "_rebuild_tensor_v2" || name == "_rebuild_tensor" || name == "_rebuild_tensor_v3")) {
            const auto &a = seq(args);
            if (a.size() < 4) fail("_rebuild_tensor with too few arguments");
            if (a[0]->kind != PVal::Storage) fail("_rebuild_tensor without a storage");
            auto v = mk(PVal::Tensor);
            v->tensor.storage = a[0]->storage;
            v->tensor.offset = integer(a[1]);
            if (v->tensor.offset < 0) fail("negative storage offset");
            if (a[2]->kind == PVal::Tuple && a[3]->kind == PVal::Tuple) {
                v->tensor.dense = true;
                for (const PRef &d : a[2]->items) v->tensor.size.push_back(integer(d));
                for (const PRef &d : a[3]->items) v->tensor.stride.push_back(integer(d));
                if (v->tensor.size.size() != v->tensor.stride.size()) fail("size and stride ranks differ");
            }
            return v;
        }
        if (mod == "torch._utils" && (name == "_rebuild_parameter" || name == "_rebuild_parameter_with_state")) {
            const auto &a = seq(args);
            if (a.empty()) fail("_rebuild_parameter without arguments");
            return a[0];
        }
        auto v = mk(PVal::Opaque);
        v->s = mod + "." + name;
        return v;
    }
};

bool looks_like_state_dict(const PVal &d) {
    for (const auto &kv : d.dict)
        if (kv.second->kind == PVal::Tensor && kv.second->tensor.dense) return true;
    return false;
}

void parse_torch_zip(const uint8_t *z, size_t len, dmx_checkpoint &c) {
    const auto dir = zip_directory(z, len);
    std::string root;
    bool found = false;
    for (const auto &e : dir) {
        const std::string &n = e.first;
        if (n.size() >= 9 && n.compare(n.size() - 9, 9, "/data.pkl") == 0) {
            root = n.substr(0, n.size() - 9);
            found = true;
            break;
        }
    }
    if (!found) bad("archive contains no `<root>/data.pkl`; is this a torch.save file?");
    bool big = false;
    if (auto bo = dir.find(root + "/byteorder"); bo != dir.end()) {
        auto d = zip_data(z, len, bo->second, bo->first);
        std::string s(reinterpret_cast<const char *>(d.first), d.second);
        while (!s.empty() && (s.back() == '\n' || s.back() == ' ' || s.back() == '\r')) s.pop_back();
        big = s == "big";
    }
    auto pk = dir.find(root + "/data.pkl");
    auto pkd = zip_data(z, len, pk->second, pk->first);
    const PRef top = Unpickler(pkd.first, pkd.second).run();
    if (top->kind != PVal::Dict) bad("checkpoint top level is not a dict");
    const PVal *state = nullptr;
    for (const char *key : {"model_state_dict", "state_dict", "state"}) {
        for (const auto &kv : top->dict)
            if (kv.first->kind == PVal::Str && kv.first->s == key && kv.second->kind == PVal::Dict &&
                looks_like_state_dict(*kv.second)) {
                state = kv.second.get();
                break;
            }
        if (state) break;
    }
    if (!state && looks_like_state_dict(*top)) state = top.get();
    if (!state) bad("checkpoint has no tensor state dict (looked for model_state_dict/state_dict/state)");
    for (const auto &kv : state->dict) {
        if (kv.first->kind != PVal::Str) bad("state dict key is not a string");
        const std::string &name = kv.first->s;
        const PVal &v = *kv.second;
        if (v.kind == PVal::None || v.kind == PVal::Opaque) continue;
        if (v.kind != PVal::Tensor) bad("state dict entry `" + name + "` is not a tensor");
        if (!v.tensor.dense) bad("tensor `" + name + "` is sparse, which is not supported");
        const TensorRef &t = v.tensor;
        auto se = dir.find(root + "/data/" + t.storage.key);
        if (se == dir.end()) bad("missing archive entry " + root + "/data/" + t.storage.key);
        auto blob = zip_data(z, len, se->second, se->first);
        const int es = dtype_size(t.storage.dtype);
        if (blob.second % es) bad("storage " + t.storage.key + " length is not a multiple of its element size");
        const uint64_t avail = blob.second / es;
        if ((uint64_t)t.storage.numel > avail)
            bad("storage " + t.storage.key + " holds " + std::to_string(avail) + " elements but is declared with " +
                std::to_string(t.storage.numel));
        Tensor out;
        out.shape = t.size;
        const uint64_t n = checked_product(out.shape, name);
        out.data.resize(n);
        bool contiguous = true;
        for (int64_t d = (int64_t)out.shape.size() - 1, acc = 1; d >= 0; acc *= out.shape[d], --d)
            if (out.shape[d] != 1 && t.stride[d] != acc) contiguous = false;
        if (contiguous) {
            if ((uint64_t)t.offset + n > (uint64_t)t.storage.numel) bad("tensor `" + name + "` reads past its storage");
            decode(blob.first + (uint64_t)t.offset * es, n, t.storage.dtype, big, out.data.data());
            c.tensors[name] = std::move(out);
            continue;
        }
        // Element (i_0..i_k) sits at offset + sum i_d stride_d of the storage.
        std::vector<int64_t> idx(out.shape.size(), 0);
        for (uint64_t e = 0; e < n; ++e) {
            int64_t at = t.offset;
            for (size_t d = 0; d < idx.size(); ++d) at += idx[d] * t.stride[d];
            if (at < 0 || (uint64_t)at >= (uint64_t)t.storage.numel) bad("tensor `" + name + "` reads past its storage");
            decode(blob.first + (uint64_t)at * es, 1, t.storage.dtype, big, &out.data[e]);
            for (size_t d = idx.size(); d-- > 0;) {
                if (++idx[d] < out.shape[d]) break;
                idx[d] = 0;
            }
        }
        c.tensors[name] = std::move(out);
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
