// The GGUF reader shared by the converter (gguf.hip) and the model runner (model.hip), host code: reference
// crates/det/src/gguf.rs (values, tensor types, reader), spec/tensor.rs (dequantization of a stored row) and
// config.rs (qwen35 hyperparameters).  Everything lives in an unnamed namespace, one copy per translation unit.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>
#include "../../include/det_gguf.h"

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

// ------------------------------------------------------------------ stored rows as fp32
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

} // namespace
