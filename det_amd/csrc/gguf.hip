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

#include "gguf_reader.h"

namespace {

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
