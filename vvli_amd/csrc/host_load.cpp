// host_load.cpp -- checkpoint loaders into the contiguous weight blob: the
// HF config.json / model.safetensors pair and GGUF v2/v3 files (F32, F16,
// BF16 tensors). Host-only; the blob they fill is what vvli_gpu_model_create
// copies to HBM.
//
// Behaviour follows the reference loaders:
//   Config.fromJson            src/llm.zig:98-145, helpers :1527-1577
//   Config.fromGguf            src/llm.zig:153-193, helpers :1511-1525
//   gguf.parse / File lookups  src/gguf.zig:148-178, 234-354
//   safetensors into the blob  src/llm.zig:923-1006, 1149-1226
//   GGUF into the blob         src/llm.zig:1008-1147
// The JSON reader, the GGUF reader and the copy loops are written for this
// library; only the formats, tensor names, defaults, dtype conversions and the
// order of the checks (which decides the error returned) are shared.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"
#include "vvli_host.h"

namespace vvli {
namespace {

// ---------------------------------------------------------------------------
// JSON values as the reference's std.json.Value sees them with numbers parsed:
// integer literals that fit int64 are Int, larger ones NumStr, anything with a
// fraction or exponent Float.
// ---------------------------------------------------------------------------
struct JVal {
    enum Kind { Null, Bool, Int, Float, NumStr, Str, Arr, Obj } kind = Null;
    bool b = false;
    int64_t i = 0;
    double f = 0.0;
    std::string s;                                    // Str, NumStr
    std::vector<JVal> items;                          // Arr
    std::vector<std::pair<std::string, JVal>> fields;  // Obj

    const JVal* get(const char* key) const {
        // The last duplicate wins, as with a hash-map insert.
        const JVal* hit = nullptr;
        for (const auto& kv : fields)
            if (kv.first == key) hit = &kv.second;
        return hit;
    }
};

class JsonReader {
  public:
    JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}

    // Whole-document parse; false on any syntax error or trailing bytes.
    bool document(JVal& out) {
        ws();
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

  private:
    static constexpr int kMaxDepth = 256;
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        size_t n = strlen(w);
        if (static_cast<size_t>(end_ - p_) < n || memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static int hexval(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    bool hex4(uint32_t& u) {
        if (end_ - p_ < 4) return false;
        u = 0;
        for (int k = 0; k < 4; ++k) {
            int h = hexval(p_[k]);
            if (h < 0) return false;
            u = u * 16 + static_cast<uint32_t>(h);
        }
        p_ += 4;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += static_cast<char>(cp);
        } else if (cp < 0x800) {
            s += static_cast<char>(0xc0 | (cp >> 6));
            s += static_cast<char>(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            s += static_cast<char>(0xe0 | (cp >> 12));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
            s += static_cast<char>(0x80 | (cp & 0x3f));
        } else {
            s += static_cast<char>(0xf0 | (cp >> 18));
            s += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
            s += static_cast<char>(0x80 | (cp & 0x3f));
        }
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_) {
            char c = *p_++;
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t u;
                    if (!hex4(u)) return false;
                    if (u >= 0xd800 && u < 0xdc00) {  // high surrogate: a low one must follow
                        uint32_t lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xdc00 || lo >= 0xe000) return false;
                        u = 0x10000 + ((u - 0xd800) << 10) + (lo - 0xdc00);
                    } else if (u >= 0xdc00 && u < 0xe000) {
                        return false;
                    }
                    put_utf8(s, u);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    bool number(JVal& v) {
        const char* b = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_) return false;
        if (*p_ == '0') {
            ++p_;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        } else {
            return false;
        }
        bool integer = true;
        if (p_ < end_ && *p_ == '.') {
            integer = false;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integer = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        std::string text(b, p_);
        if (integer) {
            errno = 0;
            char* stop = nullptr;
            long long x = strtoll(text.c_str(), &stop, 10);
            if (errno == ERANGE) {
                v.kind = JVal::NumStr;
                v.s = std::move(text);
            } else {
                v.kind = JVal::Int;
                v.i = x;
            }
        } else {
            v.kind = JVal::Float;
            v.f = strtod(text.c_str(), nullptr);
        }
        return true;
    }
    bool value(JVal& v, int depth) {
        if (depth > kMaxDepth || p_ >= end_) return false;
        switch (*p_) {
            case 'n': v.kind = JVal::Null; return lit("null");
            case 't': v.kind = JVal::Bool; v.b = true; return lit("true");
            case 'f': v.kind = JVal::Bool; v.b = false; return lit("false");
            case '"': v.kind = JVal::Str; return string(v.s);
            case '[': {
                ++p_;
                v.kind = JVal::Arr;
                ws();
                if (p_ < end_ && *p_ == ']') return ++p_, true;
                for (;;) {
                    v.items.emplace_back();
                    ws();
                    if (!value(v.items.back(), depth + 1)) return false;
                    ws();
                    if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                    if (p_ < end_ && *p_ == ']') return ++p_, true;
                    return false;
                }
            }
            case '{': {
                ++p_;
                v.kind = JVal::Obj;
                ws();
                if (p_ < end_ && *p_ == '}') return ++p_, true;
                for (;;) {
                    ws();
                    std::string key;
                    if (!string(key)) return false;
                    ws();
                    if (p_ >= end_ || *p_ != ':') return false;
                    ++p_;
                    ws();
                    v.fields.emplace_back(std::move(key), JVal());
                    if (!value(v.fields.back().second, depth + 1)) return false;
                    ws();
                    if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                    if (p_ < end_ && *p_ == '}') return ++p_, true;
                    return false;
                }
            }
            default: return number(v);
        }
    }
};

// jsonValueUsize (src/llm.zig:1571-1577): non-negative integers, or an
// integer literal too large for int64 that still parses as a 64-bit unsigned.
bool json_usize(const JVal& v, uint64_t& out) {
    if (v.kind == JVal::Int) {
        if (v.i < 0) return false;
        out = static_cast<uint64_t>(v.i);
        return true;
    }
    if (v.kind == JVal::NumStr) {
        if (v.s.empty() || v.s[0] == '-') return false;
        errno = 0;
        char* stop = nullptr;
        unsigned long long x = strtoull(v.s.c_str(), &stop, 10);
        if (errno == ERANGE || *stop != '\0') return false;
        out = x;
        return true;
    }
    return false;
}

// ---------------------------------------------------------------------------
// Config.fromJson
// ---------------------------------------------------------------------------
int u32_field(uint64_t v, const char* key, uint32_t& out) {
    if (v > 0xffffffffull) return set_error(VVLI_INVALID_CONFIG, "%s = %llu does not fit 32 bits", key,
                                             static_cast<unsigned long long>(v));
    out = static_cast<uint32_t>(v);
    return VVLI_OK;
}

int json_required_u32(const JVal& o, const char* key, uint32_t& out) {
    // getRequiredUsize (src/llm.zig:1527-1529): absent -> MissingJsonField,
    // present but not a usize -> InvalidConfig.
    const JVal* v = o.get(key);
    if (!v) return set_error(VVLI_MISSING_FIELD, "config.json lacks \"%s\"", key);
    uint64_t x;
    if (!json_usize(*v, x)) return set_error(VVLI_INVALID_CONFIG, "config.json \"%s\" is not a non-negative integer", key);
    return u32_field(x, key, out);
}

bool json_optional_usize(const JVal& o, const char* key, uint64_t& out) {
    const JVal* v = o.get(key);  // getOptionalUsize (:1531-1534): wrong type -> absent
    return v && json_usize(*v, out);
}

bool json_optional_f32(const JVal& o, const char* key, float& out) {
    // getOptionalF32 (:1545-1553).
    const JVal* v = o.get(key);
    if (!v) return false;
    if (v->kind == JVal::Int) { out = static_cast<float>(v->i); return true; }
    if (v->kind == JVal::Float) { out = static_cast<float>(v->f); return true; }
    if (v->kind == JVal::NumStr) {
        char* stop = nullptr;
        float x = strtof(v->s.c_str(), &stop);
        if (*stop != '\0') return false;
        out = x;
        return true;
    }
    return false;
}

bool json_optional_bool(const JVal& o, const char* key, bool& out) {
    const JVal* v = o.get(key);  // getOptionalBool (:1555-1561)
    if (!v || v->kind != JVal::Bool) return false;
    out = v->b;
    return true;
}

bool json_optional_token(const JVal& o, const char* key, uint64_t& out) {
    // getOptionalTokenId (:1536-1543): null -> absent, array -> first item.
    const JVal* v = o.get(key);
    if (!v || v->kind == JVal::Null) return false;
    if (v->kind == JVal::Arr) return !v->items.empty() && json_usize(v->items[0], out);
    return json_usize(*v, out);
}

int arch_from_name(const std::string& s, uint32_t& arch) {
    if (s == "llama") arch = VVLI_ARCH_LLAMA;
    else if (s == "mistral") arch = VVLI_ARCH_MISTRAL;
    else if (s == "olmoe") arch = VVLI_ARCH_OLMOE;
    else if (s == "qwen2") arch = VVLI_ARCH_QWEN2;
    else return set_error(VVLI_UNSUPPORTED_ARCH, "unsupported model architecture \"%s\"", s.c_str());
    return VVLI_OK;
}

const char* arch_prefix(uint32_t arch) {
    switch (arch) {  // Architecture.ggufPrefix, src/llm.zig:35-42
        case VVLI_ARCH_LLAMA: return "llama";
        case VVLI_ARCH_MISTRAL: return "mistral";
        case VVLI_ARCH_OLMOE: return "olmoe";
        default: return "qwen2";
    }
}

int config_from_json(const char* text, size_t len, uint32_t weight_kind, vvli_gpu_config& c) {
    JVal root;
    if (!JsonReader(text, len).document(root)) return set_error(VVLI_INVALID_FILE, "config.json is not valid JSON");
    if (root.kind != JVal::Obj) return set_error(VVLI_INVALID_CONFIG, "config.json is not an object");
    const JVal* mt = root.get("model_type");
    if (!mt || mt->kind != JVal::Str) return set_error(VVLI_MISSING_FIELD, "config.json lacks \"model_type\"");
    memset(&c, 0, sizeof(c));
    c.abi_version = VVLI_GPU_ABI_VERSION;
    c.weight_kind = weight_kind;
    int rc = arch_from_name(mt->s, c.arch);
    if (rc) return rc;
    uint64_t x = 0;
    if ((rc = json_required_u32(root, "num_attention_heads", c.heads))) return rc;
    if (json_optional_usize(root, "num_experts", x) && (rc = u32_field(x, "num_experts", c.num_experts))) return rc;
    if ((rc = json_required_u32(root, "vocab_size", c.vocab))) return rc;
    if ((rc = json_required_u32(root, "hidden_size", c.hidden))) return rc;
    if ((rc = json_required_u32(root, "intermediate_size", c.inter))) return rc;
    if ((rc = json_required_u32(root, "num_hidden_layers", c.layers))) return rc;
    c.kv_heads = c.heads;
    if (json_optional_usize(root, "num_key_value_heads", x) && (rc = u32_field(x, "num_key_value_heads", c.kv_heads)))
        return rc;
    if (json_optional_usize(root, "num_experts_per_tok", x) &&
        (rc = u32_field(x, "num_experts_per_tok", c.experts_per_tok)))
        return rc;
    c.qk_norm = c.arch == VVLI_ARCH_OLMOE;
    c.rope_layout = VVLI_ROPE_SPLIT_HALF;
    if ((rc = json_required_u32(root, "max_position_embeddings", c.max_pos))) return rc;
    c.rope_theta = 10000.0f;
    json_optional_f32(root, "rope_theta", c.rope_theta);
    c.rms_eps = 0.000001f;
    json_optional_f32(root, "rms_norm_eps", c.rms_eps);
    bool flag = false;
    c.tie = json_optional_bool(root, "tie_word_embeddings", flag) && flag;
    flag = c.arch == VVLI_ARCH_QWEN2;
    json_optional_bool(root, "attention_bias", flag);
    c.qkv_bias = flag;
    if (json_optional_token(root, "eos_token_id", x) && (rc = u32_field(x, "eos_token_id", c.eos_token_id))) return rc;
    if (json_optional_token(root, "pad_token_id", x) && (rc = u32_field(x, "pad_token_id", c.pad_token_id))) return rc;
    return validate_config(c, false);
}

// ---------------------------------------------------------------------------
// GGUF (src/gguf.zig): metadata table, tensor table, data start.
// ---------------------------------------------------------------------------
enum GType : uint32_t {
    G_U8 = 0, G_I8, G_U16, G_I16, G_U32, G_I32, G_F32, G_BOOL, G_STR, G_ARR, G_U64, G_I64, G_F64
};
enum : uint32_t { T_F32 = 0, T_F16 = 1, T_BF16 = 30 };

// Tensor type ids gguf.TensorType knows (src/gguf.zig:32-66); any other id is
// rejected while parsing, like its readEnum.
bool known_tensor_type(uint32_t t) {
    return t <= 3 || (t >= 6 && t <= 30) || t == 34 || t == 35 || t == 39;
}

struct GMeta {
    std::string key;
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned integers and bools
    int64_t i = 0;   // signed integers
    double f = 0;    // floats
    std::string s;
    uint32_t arr_type = 0;
    uint64_t arr_len = 0;
};

struct GTensor {
    std::string name;
    uint32_t ndim = 0;
    uint64_t dims[8] = {};
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct GFile {
    uint32_t version = 0;
    std::vector<GMeta> meta;
    std::vector<GTensor> tensors;
    uint64_t alignment = 32, data_start = 0;

    const GMeta* find(const char* key) const {
        for (const auto& m : meta)
            if (m.key == key) return &m;  // the first entry with the key, as File.metadataValue
        return nullptr;
    }
    const GTensor* tensor(const std::string& name) const {
        for (const auto& t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
    // File.usizeValue (src/gguf.zig:148-161).
    bool usize(const char* key, uint64_t& out) const {
        const GMeta* m = find(key);
        if (!m) return false;
        switch (m->type) {
            case G_U8: case G_U16: case G_U32: case G_U64: out = m->u; return true;
            case G_I8: case G_I16: case G_I32: case G_I64:
                if (m->i < 0) return false;
                out = static_cast<uint64_t>(m->i);
                return true;
            default: return false;
        }
    }
    // File.f32Value (src/gguf.zig:163-177).
    bool f32(const char* key, float& out) const {
        const GMeta* m = find(key);
        if (!m) return false;
        switch (m->type) {
            case G_F32: case G_F64: out = static_cast<float>(m->f); return true;
            case G_U8: case G_U16: case G_U32: case G_U64: out = static_cast<float>(m->u); return true;
            case G_I8: case G_I16: case G_I32: case G_I64: out = static_cast<float>(m->i); return true;
            default: return false;
        }
    }
};

class GReader {
  public:
    GReader(const uint8_t* b, size_t n) : b_(b), n_(n) {}
    size_t pos() const { return i_; }

    bool bytes(size_t len, const uint8_t** out) {
        if (len > n_ - i_) return false;
        *out = b_ + i_;
        i_ += len;
        return true;
    }
    template <typename T>
    bool num(T& v) {
        const uint8_t* p;
        if (!bytes(sizeof(T), &p)) return false;
        memcpy(&v, p, sizeof(T));  // little-endian host
        return true;
    }
    bool str(std::string* out) {
        uint64_t len;
        const uint8_t* p;
        if (!num(len) || !bytes(len, &p)) return false;
        if (out) out->assign(reinterpret_cast<const char*>(p), len);
        return true;
    }
    // One metadata value of a known type; arrays are walked, not stored
    // (readMetadataValue / skipMetadataValue, src/gguf.zig:317-353). Returns
    // VVLI_OK, VVLI_INVALID_FILE (truncated) or VVLI_UNSUPPORTED_METADATA.
    int value(uint32_t type, GMeta* m, int depth) {
        uint8_t u8; uint16_t u16; uint32_t u32; uint64_t u64;
        int8_t i8; int16_t i16; int32_t i32; int64_t i64;
        float f32; double f64;
        GMeta scratch;
        GMeta& o = m ? *m : scratch;
        switch (type) {
            case G_U8: if (!num(u8)) return trunc(); o.u = u8; return VVLI_OK;
            case G_BOOL: if (!num(u8)) return trunc(); o.u = u8 != 0; return VVLI_OK;
            case G_I8: if (!num(i8)) return trunc(); o.i = i8; return VVLI_OK;
            case G_U16: if (!num(u16)) return trunc(); o.u = u16; return VVLI_OK;
            case G_I16: if (!num(i16)) return trunc(); o.i = i16; return VVLI_OK;
            case G_U32: if (!num(u32)) return trunc(); o.u = u32; return VVLI_OK;
            case G_I32: if (!num(i32)) return trunc(); o.i = i32; return VVLI_OK;
            case G_F32: if (!num(f32)) return trunc(); o.f = f32; return VVLI_OK;
            case G_U64: if (!num(u64)) return trunc(); o.u = u64; return VVLI_OK;
            case G_I64: if (!num(i64)) return trunc(); o.i = i64; return VVLI_OK;
            case G_F64: if (!num(f64)) return trunc(); o.f = f64; return VVLI_OK;
            case G_STR: return str(m ? &o.s : nullptr) ? VVLI_OK : trunc();
            case G_ARR: {
                // Nested arrays recurse; the depth bound only stops a hostile
                // file from exhausting the stack (the format nests one level).
                if (depth >= 64) return set_error(VVLI_INVALID_FILE, "GGUF arrays nested deeper than 64");
                uint32_t it;
                uint64_t len;
                if (!num(it)) return trunc();
                if (it > G_F64) return set_error(VVLI_UNSUPPORTED_METADATA, "GGUF metadata type %u", it);
                if (!num(len)) return trunc();
                o.arr_type = it;
                o.arr_len = len;
                for (uint64_t k = 0; k < len; ++k) {
                    int rc = value(it, nullptr, depth + 1);
                    if (rc) return rc;
                }
                return VVLI_OK;
            }
            default: return set_error(VVLI_UNSUPPORTED_METADATA, "GGUF metadata type %u", type);
        }
    }
    int trunc() { return set_error(VVLI_INVALID_FILE, "GGUF ends inside its header (offset %zu)", i_); }

  private:
    const uint8_t* b_;
    size_t n_;
    size_t i_ = 0;
};

// gguf.parse, src/gguf.zig:234-284.
int gguf_parse(const uint8_t* bytes, size_t len, GFile& f) {
    GReader r(bytes, len);
    const uint8_t* magic;
    if (!r.bytes(4, &magic) || memcmp(magic, "GGUF", 4) != 0) return set_error(VVLI_INVALID_FILE, "not a GGUF file");
    if (!r.num(f.version)) return r.trunc();
    if (f.version < 2 || f.version > 3) return set_error(VVLI_UNSUPPORTED_VERSION, "GGUF version %u", f.version);
    uint64_t n_tensors, n_meta;
    if (!r.num(n_tensors) || !r.num(n_meta)) return r.trunc();
    // Every entry takes at least 12 bytes: a count beyond the file size is
    // truncation, caught before reserving memory for it.
    if (n_meta > len / 12 || n_tensors > len / 12) return r.trunc();
    f.meta.resize(n_meta);
    for (auto& m : f.meta) {
        if (!r.str(&m.key) || !r.num(m.type)) return r.trunc();
        if (m.type > G_F64) return set_error(VVLI_UNSUPPORTED_METADATA, "GGUF metadata type %u", m.type);
        int rc = r.value(m.type, &m, 0);
        if (rc) return rc;
    }
    f.tensors.resize(n_tensors);
    for (auto& t : f.tensors) {
        if (!r.str(&t.name) || !r.num(t.ndim)) return r.trunc();
        if (t.ndim == 0 || t.ndim > 8) return set_error(VVLI_INVALID_FILE, "tensor %s has %u dims", t.name.c_str(), t.ndim);
        for (uint32_t d = 0; d < t.ndim; ++d)
            if (!r.num(t.dims[d])) return r.trunc();
        if (!r.num(t.type)) return r.trunc();
        if (!known_tensor_type(t.type)) return set_error(VVLI_UNSUPPORTED_METADATA, "GGUF tensor type %u", t.type);
        if (!r.num(t.offset)) return r.trunc();
    }
    uint64_t a;
    f.alignment = f.usize("general.alignment", a) ? a : 32;
    if (f.alignment == 0) return set_error(VVLI_INVALID_FILE, "general.alignment is 0");
    const uint64_t idx = r.pos();
    if (idx > UINT64_MAX - (f.alignment - 1)) return set_error(VVLI_INVALID_FILE, "GGUF data start overflows");
    f.data_start = (idx + f.alignment - 1) / f.alignment * f.alignment;
    if (f.data_start > len) return set_error(VVLI_INVALID_FILE, "GGUF data start beyond the end of the file");
    return VVLI_OK;
}

int gguf_required_u32(const GFile& f, const char* prefix, const char* suffix, uint32_t& out) {
    std::string key = std::string(prefix) + "." + suffix;
    uint64_t v;
    if (!f.usize(key.c_str(), v)) return set_error(VVLI_MISSING_FIELD, "GGUF lacks %s", key.c_str());
    return u32_field(v, key.c_str(), out);
}

// Config.fromGguf, src/llm.zig:153-193.
int config_from_gguf(const GFile& f, uint32_t weight_kind, vvli_gpu_config& c) {
    const GMeta* a = f.find("general.architecture");
    if (!a || a->type != G_STR) return set_error(VVLI_MISSING_FIELD, "GGUF lacks general.architecture");
    memset(&c, 0, sizeof(c));
    c.abi_version = VVLI_GPU_ABI_VERSION;
    c.weight_kind = weight_kind;
    int rc = arch_from_name(a->s, c.arch);
    if (rc) return rc;
    const char* px = arch_prefix(c.arch);
    const GMeta* tok = f.find("tokenizer.ggml.tokens");
    if (!tok) return set_error(VVLI_MISSING_FIELD, "GGUF lacks tokenizer.ggml.tokens");
    if (tok->type != G_ARR) return set_error(VVLI_INVALID_CONFIG, "tokenizer.ggml.tokens is not an array");
    if ((rc = u32_field(tok->arr_len, "vocab", c.vocab))) return rc;
    if ((rc = gguf_required_u32(f, px, "attention.head_count", c.heads))) return rc;
    if ((rc = gguf_required_u32(f, px, "embedding_length", c.hidden))) return rc;
    if ((rc = gguf_required_u32(f, px, "feed_forward_length", c.inter))) return rc;
    if ((rc = gguf_required_u32(f, px, "block_count", c.layers))) return rc;
    c.kv_heads = c.heads;
    uint64_t x;
    std::string key = std::string(px) + ".attention.head_count_kv";
    if (f.usize(key.c_str(), x) && (rc = u32_field(x, key.c_str(), c.kv_heads))) return rc;
    c.rope_layout = VVLI_ROPE_INTERLEAVED;
    if ((rc = gguf_required_u32(f, px, "context_length", c.max_pos))) return rc;
    c.rope_theta = 10000.0f;
    f.f32((std::string(px) + ".rope.freq_base").c_str(), c.rope_theta);
    c.rms_eps = 0.000001f;
    f.f32((std::string(px) + ".attention.layer_norm_rms_epsilon").c_str(), c.rms_eps);
    c.tie = f.tensor("output.weight") == nullptr;
    c.qkv_bias = 0;
    if (f.usize("tokenizer.ggml.eos_token_id", x) && (rc = u32_field(x, "eos_token_id", c.eos_token_id))) return rc;
    if (f.usize("tokenizer.ggml.padding_token_id", x) && (rc = u32_field(x, "pad_token_id", c.pad_token_id))) return rc;
    return validate_config(c, false);
}

// ---------------------------------------------------------------------------
// Element conversions (src/llm.zig:791-803).
// ---------------------------------------------------------------------------
// IEEE binary16 -> binary32, exact for every input (the widening conversion
// loses nothing): normals rebias the exponent, subnormals are normalised,
// Inf/NaN keep sign and payload shifted into the wider mantissa.
float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        // value = man * 2^-24; shift the leading one into the implicit bit.
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while ((man & 0x400u) == 0);
        bits = sign | ((112u - static_cast<uint32_t>(e)) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

using SrcType = TensorSrc;
constexpr TensorSrc S_F32 = kSrcF32, S_F16 = kSrcF16, S_BF16 = kSrcBF16;

// Copies `n` elements of type `src` from `raw` into blob slice `dst`, converting
// to the blob's element type. Same-type copies are byte copies.
void convert_into(void* blob, uint32_t kind, size_t dst, const uint8_t* raw, SrcType src, size_t n) {
    if (kind == VVLI_WEIGHT_F32) {
        float* out = static_cast<float*>(blob) + dst;
        if (src == S_F32) {
            memcpy(out, raw, n * 4);
            return;
        }
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, raw + 2 * i, 2);
            out[i] = src == S_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
    } else {
        uint16_t* out = static_cast<uint16_t*>(blob) + dst;
        if (src == S_BF16) {
            memcpy(out, raw, n * 2);
            return;
        }
        if (src == S_F16) {
            for (size_t i = 0; i < n; ++i) {
                uint16_t h;
                memcpy(&h, raw + 2 * i, 2);
                out[i] = f32_to_bf16(f16_to_f32(h));
            }
        } else {
            for (size_t i = 0; i < n; ++i) {
                float v;
                memcpy(&v, raw + 4 * i, 4);
                out[i] = f32_to_bf16(v);
            }
        }
    }
}

bool mul_overflows(uint64_t a, uint64_t b, uint64_t& out) { return __builtin_mul_overflow(a, b, &out); }

// ---------------------------------------------------------------------------
// The tensor list both loaders walk, in OwnedModel.assignSlices order: the
// HF and llama.cpp names of each blob slice and its element count.
// ---------------------------------------------------------------------------
struct Slot {
    std::string hf, gguf;
    size_t offset, elems;
};

std::vector<Slot> slots(const vvli_gpu_config& c, const BlobLayout& L) {
    const size_t h = c.hidden, kv = kv_dim(c), inter = c.inter, vocab = c.vocab;
    std::vector<Slot> s;
    s.push_back({"model.embed_tokens.weight", "token_embd.weight", L.embed, vocab * h});
    for (uint32_t i = 0; i < c.layers; ++i) {
        const LayerSlices& l = L.layers[i];
        const std::string hp = "model.layers." + std::to_string(i) + ".";
        const std::string gp = "blk." + std::to_string(i) + ".";
        s.push_back({hp + "input_layernorm.weight", gp + "attn_norm.weight", l.input_norm, h});
        s.push_back({hp + "self_attn.q_proj.weight", gp + "attn_q.weight", l.q, h * h});
        if (c.qkv_bias) s.push_back({hp + "self_attn.q_proj.bias", "", l.q_bias, h});
        s.push_back({hp + "self_attn.k_proj.weight", gp + "attn_k.weight", l.k, kv * h});
        if (c.qkv_bias) s.push_back({hp + "self_attn.k_proj.bias", "", l.k_bias, kv});
        s.push_back({hp + "self_attn.v_proj.weight", gp + "attn_v.weight", l.v, kv * h});
        if (c.qkv_bias) s.push_back({hp + "self_attn.v_proj.bias", "", l.v_bias, kv});
        s.push_back({hp + "self_attn.o_proj.weight", gp + "attn_output.weight", l.o, h * h});
        s.push_back({hp + "post_attention_layernorm.weight", gp + "ffn_norm.weight", l.post_norm, h});
        s.push_back({hp + "mlp.gate_proj.weight", gp + "ffn_gate.weight", l.gate, inter * h});
        s.push_back({hp + "mlp.up_proj.weight", gp + "ffn_up.weight", l.up, inter * h});
        s.push_back({hp + "mlp.down_proj.weight", gp + "ffn_down.weight", l.down, h * inter});
    }
    s.push_back({"model.norm.weight", "output_norm.weight", L.final_norm, h});
    if (!c.tie) s.push_back({"lm_head.weight", "output.weight", L.lm_head, vocab * h});
    return s;
}

int check_target(const vvli_gpu_config* cfg, void* blob, size_t blob_elems, BlobLayout& L) {
    if (!cfg || !blob) return set_error(VVLI_NULL_ARG, "cfg or blob is NULL");
    // OwnedModel.init (src/llm.zig:424-446) rejects configs the dense runner
    // cannot hold before any tensor is read.
    int rc = validate_config(*cfg, true);
    if (rc) return rc;
    L = compute_layout(*cfg);
    if (blob_elems < L.total)
        return set_error(VVLI_INVALID_WEIGHT, "blob has %zu elements, layout needs %zu", blob_elems, L.total);
    return VVLI_OK;
}

void report(vvli_host_progress_fn fn, void* user, size_t done, size_t total, const char* name) {
    if (fn) fn(user, done, total, name);
}

// One safetensors entry (parseTensorInfo + copyTensorIntoWeight,
// src/llm.zig:1149-1218), checks in the reference's order.
int copy_safetensor(const JVal& tensors, const uint8_t* data, size_t data_len, const Slot& s, TensorPut put,
                    void* ctx) {
    const char* name = s.hf.c_str();
    const JVal* meta = tensors.get(name);
    if (!meta) return set_error(VVLI_MISSING_TENSOR, "safetensors lacks %s", name);
    if (meta->kind != JVal::Obj) return set_error(VVLI_INVALID_WEIGHT, "%s: entry is not an object", name);
    const JVal* dt = meta->get("dtype");
    if (!dt || dt->kind != JVal::Str) return set_error(VVLI_INVALID_WEIGHT, "%s: no dtype", name);
    SrcType src;
    if (dt->s == "F32") src = S_F32;
    else if (dt->s == "BF16") src = S_BF16;
    else return set_error(VVLI_UNSUPPORTED_DTYPE, "%s: dtype %s (F32 and BF16 are supported)", name, dt->s.c_str());
    const JVal* shape = meta->get("shape");
    if (!shape || shape->kind != JVal::Arr) return set_error(VVLI_INVALID_WEIGHT, "%s: no shape", name);
    const JVal* offs = meta->get("data_offsets");
    if (!offs || offs->kind != JVal::Arr || offs->items.size() != 2)
        return set_error(VVLI_INVALID_WEIGHT, "%s: data_offsets is not a pair", name);
    uint64_t start, end;
    if (!json_usize(offs->items[0], start) || !json_usize(offs->items[1], end))
        return set_error(VVLI_INVALID_CONFIG, "%s: data_offsets are not non-negative integers", name);
    // shapeElementCount: a dimension that is not a usize makes the count 0.
    uint64_t count = 1;
    for (const JVal& d : shape->items) {
        uint64_t x;
        if (!json_usize(d, x)) { count = 0; break; }
        if (mul_overflows(count, x, count)) { count = UINT64_MAX; break; }
    }
    if (count != s.elems)
        return set_error(VVLI_INVALID_WEIGHT, "%s: shape holds %llu elements, the model needs %zu", name,
                         static_cast<unsigned long long>(count), s.elems);
    if (end > data_len || end < start) return set_error(VVLI_INVALID_WEIGHT, "%s: data_offsets out of range", name);
    const size_t esz = src == S_F32 ? 4 : 2;
    if (end - start != s.elems * esz)
        return set_error(VVLI_INVALID_WEIGHT, "%s: %llu bytes for %zu %s elements", name,
                         static_cast<unsigned long long>(end - start), s.elems, dt->s.c_str());
    return put(ctx, s.offset, data + start, src, s.elems);
}

// One GGUF entry (copyGgufTensorIntoWeight + ggufTensorByteLen,
// src/llm.zig:1081-1147).
int copy_gguf_tensor(const GFile& f, const uint8_t* bytes, size_t len, const Slot& s, TensorPut put, void* ctx) {
    const char* name = s.gguf.c_str();
    const GTensor* t = f.tensor(s.gguf);
    if (!t) return set_error(VVLI_MISSING_TENSOR, "GGUF lacks %s", name);
    SrcType src;
    if (t->type == T_F32) src = S_F32;
    else if (t->type == T_F16) src = S_F16;
    else if (t->type == T_BF16) src = S_BF16;
    else return set_error(VVLI_UNSUPPORTED_DTYPE, "%s: GGUF tensor type %u (F32, F16 and BF16 are supported)", name, t->type);
    uint64_t count = 1;
    for (uint32_t d = 0; d < t->ndim; ++d)
        if (mul_overflows(count, t->dims[d], count)) { count = UINT64_MAX; break; }
    if (count != s.elems)
        return set_error(VVLI_INVALID_WEIGHT, "%s: dims hold %llu elements, the model needs %zu", name,
                         static_cast<unsigned long long>(count), s.elems);
    const uint64_t nbytes = count * (src == S_F32 ? 4 : 2);
    uint64_t start, end;
    if (__builtin_add_overflow(f.data_start, t->offset, &start) || __builtin_add_overflow(start, nbytes, &end) ||
        end > len)
        return set_error(VVLI_INVALID_WEIGHT, "%s: data lies beyond the end of the file", name);
    return put(ctx, s.offset, bytes + start, src, s.elems);
}

struct HostSink {
    void* blob;
    uint32_t kind;
};
int host_put(void* ctx, size_t dst, const uint8_t* raw, TensorSrc src, size_t n) {
    auto* h = static_cast<HostSink*>(ctx);
    convert_into(h->blob, h->kind, dst, raw, src, n);
    return VVLI_OK;
}

}  // namespace

int load_safetensors_into(const vvli_gpu_config& cfg, const void* bytes, size_t len, TensorPut put, void* ctx,
                          vvli_host_progress_fn progress, void* user) {
    // OwnedModel.init (src/llm.zig:424-446) rejects configs the dense runner
    // cannot hold before any tensor is read.
    int rc = validate_config(cfg, true);
    if (rc) return rc;
    if (!bytes) return set_error(VVLI_NULL_ARG, "bytes is NULL");
    const BlobLayout L = compute_layout(cfg);
    const uint8_t* b = static_cast<const uint8_t*>(bytes);
    if (len < 8) return set_error(VVLI_INVALID_WEIGHT, "safetensors file shorter than its 8-byte header length");
    uint64_t hlen;
    memcpy(&hlen, b, 8);
    if (hlen > len - 8) return set_error(VVLI_INVALID_WEIGHT, "safetensors header runs past the end of the file");
    JVal root;
    if (!JsonReader(reinterpret_cast<const char*>(b + 8), hlen).document(root))
        return set_error(VVLI_INVALID_FILE, "safetensors header is not valid JSON");
    if (root.kind != JVal::Obj) return set_error(VVLI_INVALID_WEIGHT, "safetensors header is not an object");
    const uint8_t* data = b + 8 + hlen;
    const size_t data_len = len - 8 - hlen;
    std::vector<Slot> list = slots(cfg, L);
    report(progress, user, 0, list.size(), "start");
    for (size_t k = 0; k < list.size(); ++k) {
        if ((rc = copy_safetensor(root, data, data_len, list[k], put, ctx))) return rc;
        report(progress, user, k + 1, list.size(), list[k].hf.c_str());
    }
    return VVLI_OK;
}

int load_gguf_into(const vvli_gpu_config& cfg, const void* bytes, size_t len, TensorPut put, void* ctx,
                   vvli_host_progress_fn progress, void* user) {
    int rc = validate_config(cfg, true);
    if (rc) return rc;
    if (!bytes) return set_error(VVLI_NULL_ARG, "bytes is NULL");
    // loadGgufIntoOwnedModel (src/llm.zig:1008-1011): GGUF files carry no
    // q/k/v bias tensors.
    if (cfg.qkv_bias) return set_error(VVLI_UNSUPPORTED_ARCH, "GGUF loading does not support q/k/v bias");
    GFile f;
    const uint8_t* b = static_cast<const uint8_t*>(bytes);
    if ((rc = gguf_parse(b, len, f))) return rc;
    const BlobLayout L = compute_layout(cfg);
    std::vector<Slot> list = slots(cfg, L);
    report(progress, user, 0, list.size(), "start");
    for (size_t k = 0; k < list.size(); ++k) {
        if ((rc = copy_gguf_tensor(f, b, len, list[k], put, ctx))) return rc;
        report(progress, user, k + 1, list.size(), list[k].gguf.c_str());
    }
    return VVLI_OK;
}

int gguf_config(const void* bytes, size_t len, uint32_t weight_kind, vvli_gpu_config& out) {
    if (!bytes) return set_error(VVLI_NULL_ARG, "bytes is NULL");
    GFile f;
    int rc = gguf_parse(static_cast<const uint8_t*>(bytes), len, f);
    if (rc) return rc;
    return config_from_gguf(f, weight_kind, out);
}

}  // namespace vvli

using namespace vvli;

extern "C" {

int vvli_host_config_from_json(const char* json, size_t len, uint32_t weight_kind, vvli_gpu_config* out) {
    if (!json || !out) return set_error(VVLI_NULL_ARG, "json or out is NULL");
    clear_error();
    vvli_gpu_config c;
    int rc = config_from_json(json, len, weight_kind, c);
    if (rc == VVLI_OK) *out = c;
    return rc;
}

int vvli_host_config_from_gguf(const void* bytes, size_t len, uint32_t weight_kind, vvli_gpu_config* out) {
    if (!bytes || !out) return set_error(VVLI_NULL_ARG, "bytes or out is NULL");
    clear_error();
    vvli_gpu_config c;
    const int rc = gguf_config(bytes, len, weight_kind, c);
    if (rc == VVLI_OK) *out = c;
    return rc;
}

int vvli_host_load_safetensors(const vvli_gpu_config* cfg, const void* bytes, size_t len, void* blob,
                               size_t blob_elems, vvli_host_progress_fn progress, void* user) {
    BlobLayout L;
    int rc = check_target(cfg, blob, blob_elems, L);
    if (rc) return rc;
    clear_error();
    // Alignment padding stays zero, like a freshly allocated OwnedModel.
    memset(blob, 0, L.total * elem_bytes(*cfg));
    HostSink sink{blob, cfg->weight_kind};
    return load_safetensors_into(*cfg, bytes, len, host_put, &sink, progress, user);
}

int vvli_host_load_gguf(const vvli_gpu_config* cfg, const void* bytes, size_t len, void* blob, size_t blob_elems,
                        vvli_host_progress_fn progress, void* user) {
    BlobLayout L;
    int rc = check_target(cfg, blob, blob_elems, L);
    if (rc) return rc;
    clear_error();
    memset(blob, 0, L.total * elem_bytes(*cfg));
    HostSink sink{blob, cfg->weight_kind};
    return load_gguf_into(*cfg, bytes, len, host_put, &sink, progress, user);
}

int vvli_host_map_file(const char* path, const void** data, size_t* len) {
    if (!path || !data || !len) return set_error(VVLI_NULL_ARG, "path, data or len is NULL");
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_error(VVLI_INVALID_FILE, "open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        int e = errno;
        close(fd);
        return set_error(VVLI_INVALID_FILE, "stat %s: %s", path, strerror(e));
    }
    if (st.st_size == 0) {
        close(fd);
        *data = nullptr;
        *len = 0;
        return set_error(VVLI_INVALID_FILE, "%s is empty", path);
    }
    void* p = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    int e = errno;
    close(fd);
    if (p == MAP_FAILED) return set_error(VVLI_INVALID_FILE, "mmap %s: %s", path, strerror(e));
    *data = p;
    *len = static_cast<size_t>(st.st_size);
    return VVLI_OK;
}

int vvli_host_unmap_file(const void* data, size_t len) {
    if (!data) return VVLI_OK;
    if (munmap(const_cast<void*>(data), len) != 0) return set_error(VVLI_INVALID_FILE, "munmap: %s", strerror(errno));
    return VVLI_OK;
}

float vvli_host_f16_to_f32(uint16_t bits) { return f16_to_f32(bits); }

}  // extern "C"
