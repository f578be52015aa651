// GGUF container and `det convert` (host code): reference crates/det/src/gguf.rs (reader, header writer),
// convert.rs (the conversion plan) and config.rs (qwen35 hyperparameters).  The linears are quantized on the GPU
// with det_quantize_rows (quantize.rs's rules, bit-identical), in row chunks.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>
#include "../../include/det_gguf.h"
#include "../../include/det_hip.h"

namespace {

thread_local std::string g_err;

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// ------------------------------------------------------------------ values (gguf.rs:9-76)
struct Value {
    uint32_t type = 0;
    uint64_t raw = 0;           // scalar bits, little-endian as stored (keeps F32/F64 payloads exact)
    std::string s;
    uint32_t elem = 0;          // array element type
    std::vector<Value> arr;
};

bool as_u64(const Value& v, uint64_t* out) {
    switch (v.type) {
    case DET_GGUF_U8: case DET_GGUF_U16: case DET_GGUF_U32: case DET_GGUF_U64: *out = v.raw; return true;
    case DET_GGUF_I8: { const int8_t x = (int8_t)v.raw; if (x < 0) return false; *out = (uint64_t)x; return true; }
    case DET_GGUF_I16: { const int16_t x = (int16_t)v.raw; if (x < 0) return false; *out = (uint64_t)x; return true; }
    case DET_GGUF_I32: { const int32_t x = (int32_t)v.raw; if (x < 0) return false; *out = (uint64_t)x; return true; }
    case DET_GGUF_I64: { const int64_t x = (int64_t)v.raw; if (x < 0) return false; *out = (uint64_t)x; return true; }
    default: return false;
    }
}
bool as_f64(const Value& v, double* out) {
    if (v.type == DET_GGUF_F32) { float f; uint32_t b = (uint32_t)v.raw; memcpy(&f, &b, 4); *out = f; return true; }
    if (v.type == DET_GGUF_F64) { memcpy(out, &v.raw, 8); return true; }
    uint64_t u;
    if (as_u64(v, &u)) { *out = (double)u; return true; }
    return false;
}
// Value::as_f32 (gguf.rs:35-41): F32 as is, F64 rounded, integers converted
bool as_f32(const Value& v, float* out) {
    if (v.type == DET_GGUF_F32) { uint32_t b = (uint32_t)v.raw; memcpy(out, &b, 4); return true; }
    if (v.type == DET_GGUF_F64) { double d; memcpy(&d, &v.raw, 8); *out = (float)d; return true; }
    uint64_t u;
    if (as_u64(v, &u)) { *out = (float)u; return true; }
    return false;
}
Value f32_value(float f) { Value v; v.type = DET_GGUF_F32; uint32_t b; memcpy(&b, &f, 4); v.raw = b; return v; }

// ------------------------------------------------------------------ tensor types (gguf.rs:79-158)
constexpr uint32_t T_F32 = 0, T_F16 = 1, T_BF16 = 30, T_DET4 = 0xDE04, T_DET6 = 0xDE06, T_DET8 = 0xDE08;
bool known_type(uint32_t t) { return t == T_F32 || t == T_F16 || t == T_BF16 || t == T_DET4 || t == T_DET6 || t == T_DET8; }
int det_bits(uint32_t t) { return t == T_DET4 ? 4 : t == T_DET6 ? 6 : t == T_DET8 ? 8 : 0; }
uint32_t det_type(int bits) { return bits == 4 ? T_DET4 : bits == 6 ? T_DET6 : T_DET8; }
uint64_t bytes_per_32(int bits) { return bits == 8 ? 32 : bits == 6 ? 24 : 16; }
uint64_t row_bytes(uint32_t t, uint64_t k) {
    if (t == T_F32) return 4 * k;
    if (t == T_F16 || t == T_BF16) return 2 * k;
    return k / 32 * bytes_per_32(det_bits(t)) + 4 + 2 * (k / 128);
}
std::string type_name(uint32_t t) {
    switch (t) {
    case T_F32: return "F32"; case T_F16: return "F16"; case T_BF16: return "BF16";
    case T_DET4: return "DET_W4"; case T_DET6: return "DET_W6"; case T_DET8: return "DET_W8";
    }
    static const char* names[31] = {"F32", "F16", "Q4_0", "Q4_1", "?4", "?5", "Q5_0", "Q5_1", "Q8_0", "Q8_1", "Q2_K",
                                    "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_K", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ1_S",
                                    "IQ4_NL", "IQ3_S", "IQ2_S", "IQ4_XS", "I8", "I16", "I32", "I64", "F64", "IQ1_M", "BF16"};
    return t < 31 ? names[t] : "type" + std::to_string(t);
}

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t bytes() const {
        uint64_t outer = 1;
        for (size_t i = 1; i < dims.size(); i++) outer *= dims[i];
        return row_bytes(type, dims[0]) * outer;
    }
    uint64_t elems() const { uint64_t n = 1; for (auto d : dims) n *= d; return n; }
};

std::string dims_str(const std::vector<uint64_t>& d) {
    std::string s = "[";
    for (size_t i = 0; i < d.size(); i++) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

// ------------------------------------------------------------------ reader (gguf.rs:192-359)
struct Cursor {
    const uint8_t* b;
    uint64_t n, pos = 0;
    const uint8_t* take(uint64_t k) {
        if (k > n - pos) throw Error("truncated GGUF header");
        const uint8_t* p = b + pos;
        pos += k;
        return p;
    }
    uint32_t u32() { uint32_t v; memcpy(&v, take(4), 4); return v; }
    uint64_t u64() { uint64_t v; memcpy(&v, take(8), 8); return v; }
    std::string str() { const uint64_t k = u64(); const uint8_t* p = take(k); return std::string((const char*)p, k); }
    Value value(uint32_t ty) {
        Value v;
        v.type = ty;
        switch (ty) {
        case DET_GGUF_U8: case DET_GGUF_I8: case DET_GGUF_BOOL: v.raw = *take(1); break;
        case DET_GGUF_U16: case DET_GGUF_I16: { uint16_t x; memcpy(&x, take(2), 2); v.raw = x; break; }
        case DET_GGUF_U32: case DET_GGUF_I32: case DET_GGUF_F32: v.raw = u32(); break;
        case DET_GGUF_U64: case DET_GGUF_I64: case DET_GGUF_F64: v.raw = u64(); break;
        case DET_GGUF_STR: v.s = str(); break;
        case DET_GGUF_ARRAY: {
            v.elem = u32();
            const uint64_t len = u64();
            v.arr.reserve(len < (1u << 20) ? len : (1u << 20));
            for (uint64_t j = 0; j < len; j++) v.arr.push_back(value(v.elem));
            break;
        }
        default: throw Error("unknown GGUF value type " + std::to_string(ty));
        }
        return v;
    }
};

struct Gguf {
    std::string path;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    std::vector<std::pair<std::string, Value>> kv;
    std::unordered_map<std::string, size_t> index;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> tindex;
    uint64_t data_start = 0, alignment = 32;

    ~Gguf() { if (map) munmap((void*)map, size); }

    static std::unique_ptr<Gguf> open(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) throw Error(path + ": " + strerror(errno));
        struct stat st;
        if (fstat(fd, &st) != 0) { ::close(fd); throw Error(path + ": " + strerror(errno)); }
        std::unique_ptr<Gguf> g(new Gguf());
        g->path = path;
        g->size = (uint64_t)st.st_size;
        if (g->size > 0) {
            void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p == MAP_FAILED) { ::close(fd); throw Error(path + ": mmap failed"); }
            g->map = (const uint8_t*)p;
        }
        ::close(fd);
        Cursor c{g->map, g->size};
        if (memcmp(c.take(4), "GGUF", 4) != 0) throw Error("not a GGUF file");
        const uint32_t version = c.u32();
        if (version != 3 && version != 2) throw Error("unsupported GGUF version " + std::to_string(version));
        const uint64_t n_tensors = c.u64(), n_kv = c.u64();
        for (uint64_t i = 0; i < n_kv; i++) {
            std::string key = c.str();
            const uint32_t ty = c.u32();
            g->kv.emplace_back(std::move(key), c.value(ty));
        }
        for (uint64_t i = 0; i < n_tensors; i++) {
            TensorInfo t;
            t.name = c.str();
            const uint32_t nd = c.u32();
            for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.u64());
            t.type = c.u32();
            t.offset = c.u64();
            g->tensors.push_back(std::move(t));
        }
        // the indexes keep the last of equal names (gguf.rs:244-253 collects into maps); general.alignment is the
        // first such key (gguf.rs:254-259)
        for (size_t i = 0; i < g->kv.size(); i++) g->index[g->kv[i].first] = i;
        for (size_t i = 0; i < g->tensors.size(); i++) g->tindex[g->tensors[i].name] = i;
        for (const auto& [k, v] : g->kv) {
            if (k != "general.alignment") continue;
            uint64_t a;
            if (as_u64(v, &a)) g->alignment = a;
            break;
        }
        if (g->alignment == 0) throw Error("general.alignment is zero");
        g->data_start = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
        for (const auto& t : g->tensors) {
            const bool ok = known_type(t.type) &&
                            ((!t.dims.empty() && t.dims[0] % 32 == 0) || t.type == T_F32 || t.type == T_F16 || t.type == T_BF16);
            if (!ok || t.dims.empty())
                throw Error("tensor " + t.name + " has unsupported type " + type_name(t.type) + " or shape " + dims_str(t.dims));
            if (t.dims.size() > 2 || g->data_start + t.offset + t.bytes() > g->size)
                throw Error("tensor " + t.name + " (" + dims_str(t.dims) + " at " + std::to_string(t.offset) + ") does not fit the file");
        }
        return g;
    }
    const Value* get(const std::string& key) const {
        auto it = index.find(key);
        return it == index.end() ? nullptr : &kv[it->second].second;
    }
    bool u64(const std::string& key, uint64_t* out) const { const Value* v = get(key); return v && as_u64(*v, out); }
    const TensorInfo* tensor(const std::string& name) const {
        auto it = tindex.find(name);
        return it == tindex.end() ? nullptr : &tensors[it->second];
    }
    const uint8_t* data(const TensorInfo& t) const { return map + data_start + t.offset; }
};

// ------------------------------------------------------------------ header writer (gguf.rs:361-418)
void put(std::vector<uint8_t>& o, const void* p, size_t n) { o.insert(o.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
void put_u32(std::vector<uint8_t>& o, uint32_t v) { put(o, &v, 4); }
void put_u64(std::vector<uint8_t>& o, uint64_t v) { put(o, &v, 8); }
void put_str(std::vector<uint8_t>& o, const std::string& s) { put_u64(o, s.size()); put(o, s.data(), s.size()); }
void put_value(std::vector<uint8_t>& o, const Value& v) {
    switch (v.type) {
    case DET_GGUF_U8: case DET_GGUF_I8: case DET_GGUF_BOOL: o.push_back((uint8_t)v.raw); break;
    case DET_GGUF_U16: case DET_GGUF_I16: { const uint16_t x = (uint16_t)v.raw; put(o, &x, 2); break; }
    case DET_GGUF_U32: case DET_GGUF_I32: case DET_GGUF_F32: put_u32(o, (uint32_t)v.raw); break;
    case DET_GGUF_U64: case DET_GGUF_I64: case DET_GGUF_F64: put_u64(o, v.raw); break;
    case DET_GGUF_STR: put_str(o, v.s); break;
    case DET_GGUF_ARRAY: {
        // the element type of an array is its first element's (0 when empty), as gguf.rs:383-391 writes it
        const uint32_t et = v.arr.empty() ? 0 : v.arr[0].type;
        put_u32(o, et);
        put_u64(o, v.arr.size());
        for (const auto& e : v.arr) {
            if (e.type != et) throw Error("mixed array element types");
            put_value(o, e);
        }
        break;
    }
    default: throw Error("unknown GGUF value type " + std::to_string(v.type));
    }
}
std::vector<uint8_t> write_header(const std::vector<std::pair<std::string, Value>>& kv, const std::vector<TensorInfo>& ts,
                                  uint64_t alignment) {
    std::vector<uint8_t> o;
    put(o, "GGUF", 4);
    put_u32(o, 3);
    put_u64(o, ts.size());
    put_u64(o, kv.size());
    for (const auto& [k, v] : kv) { put_str(o, k); put_u32(o, v.type); put_value(o, v); }
    for (const auto& t : ts) {
        put_str(o, t.name);
        put_u32(o, (uint32_t)t.dims.size());
        for (auto d : t.dims) put_u64(o, d);
        put_u32(o, t.type);
        put_u64(o, t.offset);
    }
    o.resize((o.size() + alignment - 1) / alignment * alignment, 0);
    return o;
}

// ------------------------------------------------------------------ conversion (convert.rs, config.rs)
// IEEE binary16 / bfloat16 to fp32, exactly (spec/tensor.rs:7-30, spec/prim.rs:199-201)
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1F, mant = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {                                        // subnormal: normalise
            uint32_t m = mant;
            int e = 127 - 15 + 1;
            while (!(m & 0x400)) { m <<= 1; e--; }
            bits = sign | ((uint32_t)e << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
float bf16_to_f32(uint16_t b) { const uint32_t bits = (uint32_t)b << 16; float f; memcpy(&f, &bits, 4); return f; }

// one row of a stored tensor as fp32 (spec/tensor.rs:73-104; det rows dequantize as (c * m) * q)
void dequant_row(uint32_t ty, const uint8_t* row, uint64_t k, float* out) {
    if (ty == T_F32) { memcpy(out, row, 4 * k); return; }
    if (ty == T_F16 || ty == T_BF16) {
        for (uint64_t i = 0; i < k; i++) {
            uint16_t h;
            memcpy(&h, row + 2 * i, 2);
            out[i] = ty == T_F16 ? f16_to_f32(h) : bf16_to_f32(h);
        }
        return;
    }
    const int bits = det_bits(ty);
    const uint64_t cb = k / 32 * bytes_per_32(bits);
    float c;
    memcpy(&c, row + cb, 4);
    for (uint64_t b = 0; b < k / 32; b++) {
        const uint8_t* p = row + b * bytes_per_32(bits);
        for (int j = 0; j < 32; j++) {
            int q;
            if (bits == 8) {
                q = (int8_t)p[j];
            } else {
                const int lo = j < 16 ? (p[j] & 15) : (p[j - 16] >> 4);
                q = bits == 4 ? lo - 8 : (lo | (((p[16 + (j % 8)] >> (2 * (j / 8))) & 3) << 4)) - 32;
            }
            uint16_t m;
            memcpy(&m, row + cb + 4 + 2 * ((b * 32 + j) / 128), 2);
            out[b * 32 + j] = (c * (float)m) * (float)q;
        }
    }
}

// a model possibly split over several files (convert.rs:12-67)
struct Source {
    std::vector<std::unique_ptr<Gguf>> parts;
    explicit Source(const std::string& path) {
        parts.push_back(Gguf::open(path));
        uint64_t count = 1;
        parts[0]->u64("split.count", &count);
        if (count > 1) {
            const size_t slash = path.find_last_of('/');
            const std::string dir = slash == std::string::npos ? "" : path.substr(0, slash + 1);
            const std::string name = slash == std::string::npos ? path : path.substr(slash + 1);
            const size_t marker = name.find("-00001-of-");
            if (marker == std::string::npos) throw Error("split GGUF without -00001-of- in its name");
            for (uint64_t i = 2; i <= count; i++) {
                char num[32];
                snprintf(num, sizeof num, "-%05llu-of-", (unsigned long long)i);
                parts.push_back(Gguf::open(dir + name.substr(0, marker) + num + name.substr(marker + 10)));
            }
        }
    }
    const Gguf& first() const { return *parts[0]; }
    std::pair<const Gguf*, const TensorInfo*> tensor(const std::string& name) const {
        for (const auto& g : parts)
            if (const TensorInfo* t = g->tensor(name)) return {g.get(), t};
        return {nullptr, nullptr};
    }
    std::pair<const Gguf*, const TensorInfo*> need(const std::string& name) const {
        auto r = tensor(name);
        if (!r.second) throw Error("missing tensor " + name);
        if (!known_type(r.second->type)) throw Error(name + ": unsupported source type");
        return r;
    }
    std::vector<float> f32s(const std::string& name) const {
        auto [g, t] = need(name);
        const uint64_t k = t->dims[0], rows = t->elems() / k, rb = row_bytes(t->type, k);
        std::vector<float> out(rows * k);
        const uint8_t* d = g->data(*t);
        for (uint64_t r = 0; r < rows; r++) dequant_row(t->type, d + r * rb, k, out.data() + r * k);
        return out;
    }
};

// qwen35 hyperparameters (config.rs:32-93)
struct Config {
    std::string arch;
    uint64_t hidden = 0, vocab = 0, n_heads = 0, n_kv = 0, head_dim = 0, rot_dim = 0, intermediate = 0;
    uint64_t gdn_k_heads = 0, gdn_v_heads = 0, gdn_dk = 0, gdn_dv = 0, conv_k = 0;
    double rope_theta = 0;
    float eps = 0;
    std::vector<bool> attention;      // per layer
    uint64_t conv_dim() const { return 2 * gdn_k_heads * gdn_dk + gdn_v_heads * gdn_dv; }
    uint64_t n_attention_layers() const { uint64_t n = 0; for (bool a : attention) n += a; return n; }

    static Config from(const Gguf& g) {
        Config c;
        const Value* a = g.get("general.architecture");
        if (!a || a->type != DET_GGUF_STR) throw Error("no general.architecture");
        c.arch = a->s;
        if (c.arch != "qwen35") throw Error("architecture " + c.arch + " is not supported (qwen35 only)");
        auto key = [&](const char* s) { return c.arch + "." + s; };
        auto u = [&](const char* s) {
            uint64_t v;
            if (!g.u64(key(s), &v)) throw Error("missing " + key(s));
            return v;
        };
        uint64_t nextn = 0;
        g.u64(key("nextn_predict_layers"), &nextn);
        const uint64_t n_layers = u("block_count") - nextn, interval = u("full_attention_interval");
        for (uint64_t i = 0; i < n_layers; i++) c.attention.push_back((i + 1) % interval == 0);
        if (const TensorInfo* t = g.tensor("token_embd.weight")) {
            c.vocab = t->dims.size() > 1 ? t->dims[1] : 1;
        } else {
            const Value* tok = g.get("tokenizer.ggml.tokens");
            if (!tok || tok->type != DET_GGUF_ARRAY) throw Error("no token_embd.weight and no tokenizer tokens");
            c.vocab = tok->arr.size();
        }
        c.gdn_dk = u("ssm.state_size");
        c.gdn_v_heads = u("ssm.time_step_rank");
        c.hidden = u("embedding_length");
        const Value* e = g.get(key("attention.layer_norm_rms_epsilon"));
        if (!e || !as_f32(*e, &c.eps)) throw Error("missing eps");
        c.n_heads = u("attention.head_count");
        c.n_kv = u("attention.head_count_kv");
        c.head_dim = u("attention.key_length");
        c.rot_dim = u("rope.dimension_count");
        float th;
        const Value* r = g.get(key("rope.freq_base"));
        if (!r || !as_f32(*r, &th)) throw Error("missing rope.freq_base");
        c.rope_theta = th;
        c.intermediate = u("feed_forward_length");
        c.gdn_k_heads = u("ssm.group_count");
        c.gdn_dv = u("ssm.inner_size") / c.gdn_v_heads;
        c.conv_k = u("ssm.conv_kernel");
        return c;
    }
};

// bit widths: a default and per-linear overrides, "6,output=8,ffn_down=8" (convert.rs:69-118)
struct Bits {
    int def = 6;
    std::vector<std::pair<std::string, int>> per;
    static Bits parse(const std::string& s) {
        Bits b;
        size_t start = 0;
        while (start <= s.size()) {
            size_t end = s.find(',', start);
            if (end == std::string::npos) end = s.size();
            std::string item = s.substr(start, end - start);
            const size_t a = item.find_first_not_of(" \t\n\r"), z = item.find_last_not_of(" \t\n\r");
            item = a == std::string::npos ? "" : item.substr(a, z - a + 1);
            start = end + 1;
            if (item.empty()) continue;
            const size_t eq = item.find('=');
            const std::string name = eq == std::string::npos ? "" : item.substr(0, eq);
            const std::string val = eq == std::string::npos ? item : item.substr(eq + 1);
            char* endp = nullptr;
            const long v = val.empty() ? -1 : strtol(val.c_str(), &endp, 10);
            if (val.empty() || *endp != '\0' || v < 0) throw Error("bad bit width \"" + val + "\"");
            if (v != 4 && v != 6 && v != 8) throw Error("bit width " + std::to_string(v) + " is not 4, 6 or 8");
            if (eq == std::string::npos) b.def = (int)v;
            else b.per.emplace_back(name, (int)v);
        }
        return b;
    }
    int of(const std::string& linear) const {
        for (const auto& [n, v] : per)
            if (n == linear) return v;
        return def;
    }
};
const char* DEFAULT_BITS = "6,output=8,ssm_alpha=8,ssm_beta=8";     // convert.rs:122
const char* V_SCALE_KEY = "det.v_scale";                             // model.rs:47-48
const float DEFAULT_V_SCALE = 1.0f / 1024.0f;

std::vector<uint64_t> identity(uint64_t n) { std::vector<uint64_t> p(n); for (uint64_t i = 0; i < n; i++) p[i] = i; return p; }
// perm[new] = old over width-element blocks of the v heads: new head h2 takes GGUF head (h2 % rep) * n_k + h2 / rep,
// whose k head is h2 / rep (convert.rs:149-161, SPEC §5.2)
std::vector<uint64_t> head_perm(uint64_t n_k, uint64_t n_v, uint64_t width, uint64_t offset, uint64_t total) {
    const uint64_t rep = n_v / n_k;
    std::vector<uint64_t> p = identity(total);
    for (uint64_t h2 = 0; h2 < n_v; h2++) {
        const uint64_t h = (h2 % rep) * n_k + h2 / rep;
        for (uint64_t j = 0; j < width; j++) p[offset + h2 * width + j] = offset + h * width + j;
    }
    return p;
}

enum class Gen { Copy, Vec, Quant, Rope };
struct Out {
    std::string name, src;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    Gen gen = Gen::Copy;
    int bits = 0;
    std::vector<uint64_t> rows, cols;   // Quant permutations (empty: none); Vec: the outer permutation in rows
    bool cos = false;
};

// det rows of w [n][k] quantized on the GPU in chunks of rows (det_quantize_rows is per row, so chunking is exact)
std::vector<uint8_t> quantize_on_gpu(const std::vector<float>& w, uint64_t n, uint64_t k, int bits) {
    const uint64_t rb = row_bytes(det_type(bits), k);
    std::vector<uint8_t> out(n * rb);
    const uint64_t chunk = std::max<uint64_t>(1, (256ull << 20) / (4 * k));
    float* dw = (float*)det_malloc(4 * k * std::min(chunk, n));
    uint8_t* dr = (uint8_t*)det_malloc(rb * std::min(chunk, n));
    if (!dw || !dr) throw Error("device allocation failed");
    for (uint64_t r0 = 0; r0 < n; r0 += chunk) {
        const uint64_t rows = std::min(chunk, n - r0);
        det_memcpy(dw, w.data() + r0 * k, 4 * k * rows, nullptr);
        det_quantize_rows(dw, (int)rows, (int)k, bits, dr, nullptr);
        det_memcpy(out.data() + r0 * rb, dr, rb * rows, nullptr);
    }
    det_sync();
    det_free(dw);
    det_free(dr);
    return out;
}

void convert(const std::string& src_path, const std::string& dst, const std::string& bits_spec, int64_t rope_positions) {
    const Source src(src_path);
    const Bits bits = Bits::parse(bits_spec);
    const Config cfg = Config::from(src.first());
    const uint64_t n_k = cfg.gdn_k_heads, n_v = cfg.gdn_v_heads, dk = cfg.gdn_dk, dv = cfg.gdn_dv;
    const uint64_t kd = n_k * dk, conv_dim = cfg.conv_dim();
    uint64_t n_pos = 32768;
    if (rope_positions > 0) n_pos = (uint64_t)rope_positions;
    else src.first().u64(cfg.arch + ".context_length", &n_pos);
    std::vector<Out> plan;
    auto copy = [&](const std::string& name) {
        auto [g, t] = src.need(name);
        Out o;
        o.name = o.src = name; o.dims = t->dims; o.type = t->type; o.gen = Gen::Copy;
        plan.push_back(o);
    };
    auto quant = [&](const std::string& name, std::vector<uint64_t> rows, std::vector<uint64_t> cols) {
        auto [g, t] = src.need(name);
        if (t->dims.size() < 2) throw Error(name + ": a linear must be 2-D");
        // the linear's name is the second-to-last dotted component: blk.3.ffn_down.weight -> ffn_down
        const size_t last = name.rfind('.');
        const size_t prev = last == std::string::npos || last == 0 ? std::string::npos : name.rfind('.', last - 1);
        const std::string linear = last == std::string::npos ? name : name.substr(prev == std::string::npos ? 0 : prev + 1,
                                                                                    last - (prev == std::string::npos ? 0 : prev + 1));
        Out o;
        o.name = o.src = name; o.dims = {t->dims[0], t->dims[1]}; o.bits = bits.of(linear);
        o.type = det_type(o.bits); o.gen = Gen::Quant; o.rows = std::move(rows); o.cols = std::move(cols);
        plan.push_back(o);
    };
    copy("token_embd.weight");
    copy("output_norm.weight");
    {
        const std::string head = src.tensor("output.weight").second ? "output.weight" : "token_embd.weight";
        auto [g, t] = src.need(head);
        Out o;
        o.name = "output.weight"; o.src = head; o.dims = {t->dims[0], t->dims.size() > 1 ? t->dims[1] : 1};
        o.bits = bits.of("output"); o.type = det_type(o.bits); o.gen = Gen::Quant;
        plan.push_back(o);
    }
    for (bool c : {true, false}) {
        Out o;
        o.name = c ? "rope_cos" : "rope_sin"; o.dims = {cfg.rot_dim / 2, n_pos}; o.type = T_F32; o.gen = Gen::Rope; o.cos = c;
        plan.push_back(o);
    }
    for (size_t i = 0; i < cfg.attention.size(); i++) {
        auto n = [&](const std::string& s) { return "blk." + std::to_string(i) + "." + s; };
        copy(n("attn_norm.weight"));
        copy(n("post_attention_norm.weight"));
        for (const char* s : {"ffn_gate", "ffn_up", "ffn_down"}) quant(n(std::string(s) + ".weight"), {}, {});
        if (cfg.attention[i]) {
            for (const char* s : {"attn_q", "attn_k", "attn_v", "attn_output"}) quant(n(std::string(s) + ".weight"), {}, {});
            copy(n("attn_q_norm.weight"));
            copy(n("attn_k_norm.weight"));
        } else {
            const std::vector<uint64_t> vrows = head_perm(n_k, n_v, dv, 2 * kd, conv_dim);
            const std::vector<uint64_t> heads = head_perm(n_k, n_v, 1, 0, n_v);
            quant(n("attn_qkv.weight"), vrows, {});
            quant(n("attn_gate.weight"), head_perm(n_k, n_v, dv, 0, n_v * dv), {});
            quant(n("ssm_alpha.weight"), heads, {});
            quant(n("ssm_beta.weight"), heads, {});
            quant(n("ssm_out.weight"), {}, head_perm(n_k, n_v, dv, 0, n_v * dv));
            const std::pair<const char*, const std::vector<uint64_t>*> vecs[3] = {
                {"ssm_conv1d.weight", &vrows}, {"ssm_a", &heads}, {"ssm_dt.bias", &heads}};
            for (const auto& [name, perm] : vecs) {
                auto [g, t] = src.need(n(name));
                Out o;
                o.name = o.src = n(name); o.dims = t->dims; o.type = T_F32; o.gen = Gen::Vec; o.rows = *perm;
                plan.push_back(o);
            }
            copy(n("ssm_norm.weight"));
        }
    }

    const uint64_t align = 32;
    std::vector<TensorInfo> infos;
    uint64_t offset = 0;
    for (const auto& o : plan) {
        TensorInfo t;
        t.name = o.name; t.dims = o.dims; t.type = o.type; t.offset = offset;
        offset = (offset + t.bytes() + align - 1) / align * align;
        infos.push_back(t);
    }
    std::vector<std::pair<std::string, Value>> kv;
    for (const auto& [k, v] : src.first().kv)
        if (k.rfind("split.", 0) != 0 && k != V_SCALE_KEY) kv.emplace_back(k, v);
    Value vs;
    vs.type = DET_GGUF_ARRAY;
    vs.elem = DET_GGUF_F32;
    vs.arr.assign(cfg.n_attention_layers() * cfg.n_kv, f32_value(DEFAULT_V_SCALE));
    kv.emplace_back(V_SCALE_KEY, vs);
    const std::vector<uint8_t> header = write_header(kv, infos, align);

    FILE* f = fopen(dst.c_str(), "wb");
    if (!f) throw Error(dst + ": " + strerror(errno));
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
    auto write = [&](const void* p, size_t n) {
        if (n && fwrite(p, 1, n, f) != n) throw Error(dst + ": write failed");
    };
    write(header.data(), header.size());
    uint64_t written = 0;
    const std::vector<uint8_t> zeros(align, 0);
    for (size_t i = 0; i < plan.size(); i++) {
        const Out& o = plan[i];
        std::vector<uint8_t> data;
        const uint8_t* p = nullptr;
        uint64_t bytes = 0;
        if (o.gen == Gen::Copy) {
            auto [g, t] = src.need(o.src);
            p = g->data(*t);
            bytes = t->bytes();
        } else if (o.gen == Gen::Vec) {
            const std::vector<float> v = src.f32s(o.src);
            const uint64_t inner = o.dims.size() > 1 ? o.dims[0] : 1, outer = v.size() / inner;
            if (o.rows.size() != outer) throw Error(o.src + ": permutation length");
            data.resize(v.size() * 4);
            for (uint64_t r = 0; r < outer; r++) memcpy(data.data() + r * inner * 4, v.data() + o.rows[r] * inner, inner * 4);
        } else if (o.gen == Gen::Quant) {
            const uint64_t k = o.dims[0], n = o.dims[1];
            std::vector<float> w = src.f32s(o.src);
            if (!o.rows.empty()) {
                if (o.rows.size() != n) throw Error(o.src + ": row permutation length");
                std::vector<float> pw(n * k);
                for (uint64_t r = 0; r < n; r++) memcpy(pw.data() + r * k, w.data() + o.rows[r] * k, k * 4);
                w.swap(pw);
            }
            if (!o.cols.empty()) {
                if (o.cols.size() != k) throw Error(o.src + ": column permutation length");
                std::vector<float> pw(n * k);
                for (uint64_t r = 0; r < n; r++)
                    for (uint64_t c = 0; c < k; c++) pw[r * k + c] = w[r * k + o.cols[c]];
                w.swap(pw);
            }
            if (k % 128 != 0) throw Error(o.src + ": K = " + std::to_string(k) + " is not a multiple of 128");
            fprintf(stderr, "  %s: %llu x %llu -> W%d\n", o.src.c_str(), (unsigned long long)n, (unsigned long long)k, o.bits);
            data = quantize_on_gpu(w, n, k, o.bits);
        } else {
            // rope tables [pos][rot / 2]: cos or sin of pos * theta^(-2 i / rot) in binary64, rounded to fp32
            const uint64_t half = cfg.rot_dim / 2;
            std::vector<double> inv(half);
            for (uint64_t j = 0; j < half; j++) inv[j] = pow(cfg.rope_theta, -(double)(2 * j) / (double)cfg.rot_dim);
            data.resize(n_pos * half * 4);
            float* d = (float*)data.data();
            for (uint64_t pos = 0; pos < n_pos; pos++)
                for (uint64_t j = 0; j < half; j++) {
                    const double a = (double)pos * inv[j];
                    d[pos * half + j] = (float)(o.cos ? cos(a) : sin(a));
                }
        }
        if (!p) { p = data.data(); bytes = data.size(); }
        if (written != infos[i].offset) throw Error(o.name + ": offset");
        write(p, bytes);
        written += bytes;
        const uint64_t pad = (written + align - 1) / align * align - written;
        write(zeros.data(), pad);
        written += pad;
    }
    fprintf(stderr, "wrote %s (%zu tensors, %.2f GB)\n", dst.c_str(), infos.size(), (header.size() + written) / 1e9);
}

template <class F>
auto guarded(F&& f, decltype(f()) fail) -> decltype(f()) {
    try {
        return f();
    } catch (const std::exception& e) {
        g_err = e.what();
        return fail;
    }
}

} // namespace

struct det_gguf {
    std::unique_ptr<Gguf> g;
};

extern "C" {

const char* det_gguf_last_error(void) { return g_err.c_str(); }

det_gguf* det_gguf_open(const char* path) {
    return guarded([&]() -> det_gguf* { auto* h = new det_gguf; h->g = Gguf::open(path); return h; }, nullptr);
}
void det_gguf_close(det_gguf* g) { delete g; }
uint64_t det_gguf_data_start(const det_gguf* g) { return g->g->data_start; }
uint64_t det_gguf_alignment(const det_gguf* g) { return g->g->alignment; }

uint64_t det_gguf_n_kv(const det_gguf* g) { return g->g->kv.size(); }
const char* det_gguf_kv_key(const det_gguf* g, uint64_t i) { return i < g->g->kv.size() ? g->g->kv[i].first.c_str() : nullptr; }
uint32_t det_gguf_kv_type(const det_gguf* g, uint64_t i) { return i < g->g->kv.size() ? g->g->kv[i].second.type : 0xFFFFFFFFu; }
int64_t det_gguf_find_kv(const det_gguf* g, const char* key) {
    auto it = g->g->index.find(key);
    return it == g->g->index.end() ? -1 : (int64_t)it->second;
}
int det_gguf_get_u64(const det_gguf* g, const char* key, uint64_t* out) { const Value* v = g->g->get(key); return v && as_u64(*v, out); }
int det_gguf_get_f32(const det_gguf* g, const char* key, float* out) { const Value* v = g->g->get(key); return v && as_f32(*v, out); }
const char* det_gguf_get_str(const det_gguf* g, const char* key) {
    const Value* v = g->g->get(key);
    return v && v->type == DET_GGUF_STR ? v->s.c_str() : nullptr;
}
int det_gguf_get_array(const det_gguf* g, const char* key, uint32_t* elem_type, uint64_t* len) {
    const Value* v = g->g->get(key);
    if (!v || v->type != DET_GGUF_ARRAY) return 0;
    if (elem_type) *elem_type = v->elem;
    if (len) *len = v->arr.size();
    return 1;
}
int det_gguf_array_u64(const det_gguf* g, const char* key, uint64_t j, uint64_t* out) {
    const Value* v = g->g->get(key);
    return v && v->type == DET_GGUF_ARRAY && j < v->arr.size() && as_u64(v->arr[j], out);
}
int det_gguf_array_f64(const det_gguf* g, const char* key, uint64_t j, double* out) {
    const Value* v = g->g->get(key);
    return v && v->type == DET_GGUF_ARRAY && j < v->arr.size() && as_f64(v->arr[j], out);
}
const char* det_gguf_array_str(const det_gguf* g, const char* key, uint64_t j) {
    const Value* v = g->g->get(key);
    if (!v || v->type != DET_GGUF_ARRAY || j >= v->arr.size() || v->arr[j].type != DET_GGUF_STR) return nullptr;
    return v->arr[j].s.c_str();
}

uint64_t det_gguf_n_tensors(const det_gguf* g) { return g->g->tensors.size(); }
int64_t det_gguf_find_tensor(const det_gguf* g, const char* name) {
    auto it = g->g->tindex.find(name);
    return it == g->g->tindex.end() ? -1 : (int64_t)it->second;
}
const char* det_gguf_tensor_name(const det_gguf* g, uint64_t i) { return i < g->g->tensors.size() ? g->g->tensors[i].name.c_str() : nullptr; }
uint32_t det_gguf_tensor_type(const det_gguf* g, uint64_t i) { return i < g->g->tensors.size() ? g->g->tensors[i].type : 0xFFFFFFFFu; }
int det_gguf_tensor_dims(const det_gguf* g, uint64_t i, uint64_t dims[4]) {
    if (i >= g->g->tensors.size()) return -1;
    const auto& d = g->g->tensors[i].dims;
    for (size_t j = 0; j < d.size() && j < 4; j++) dims[j] = d[j];
    return (int)d.size();
}
uint64_t det_gguf_tensor_offset(const det_gguf* g, uint64_t i) { return i < g->g->tensors.size() ? g->g->tensors[i].offset : 0; }
uint64_t det_gguf_tensor_bytes(const det_gguf* g, uint64_t i) { return i < g->g->tensors.size() ? g->g->tensors[i].bytes() : 0; }
const void* det_gguf_tensor_data(const det_gguf* g, uint64_t i) {
    return i < g->g->tensors.size() ? g->g->data(g->g->tensors[i]) : nullptr;
}

int det_convert(const char* src, const char* dst, const char* bits, int64_t rope_positions) {
    return guarded([&]() { convert(src, dst, bits ? bits : DEFAULT_BITS, rope_positions); return 0; }, -1);
}

} // extern "C"
