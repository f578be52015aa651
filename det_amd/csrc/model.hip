// The qwen35 model runner (host code): the reference's Model (crates/det/src/model.rs:164-548) and
// qwen35::forward (qwen35.rs:8-172) over det_hip.h's kernels, behind det_model.h.  Greedy picking only (the
// reference's temperature / top-k / top-p sampling is not part of this build).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <vector>
#include "common.h"
#include "gguf_reader.h"
#include "mixer_internal.h"
#include "gemm_internal.h"
#include "../../include/det_hip.h"
#include "../../include/det_model.h"

namespace {

constexpr float DEFAULT_V_SCALE = 1.0f / 1024.0f;      // model.rs:46-48
const char* const V_SCALE_KEY = "det.v_scale";

// one fused linear: consecutive tensors of one type and K, concatenated along N (their widths are the parts)
struct Lin {
    det_qlinear q{};
    std::vector<int> widths;
};
struct Proj { std::vector<Lin> lins; };

struct AttnL {
    Proj qkv, o;
    det_attn_layer layer{};
    det_kv_cache kv{};
};
struct GdnL {
    Proj qkvz, ab, out;
    det_gdn_layer layer{};
    det_gdn_state state{};
};
struct Layer {
    const float* attn_norm = nullptr;
    const float* ffn_norm = nullptr;
    Proj gu, down;
    bool attn = false;
    AttnL a;
    GdnL g;
};

} // namespace

struct det_model {
    std::unique_ptr<Gguf> g;
    Config c;
    hipStream_t st = nullptr;
    std::vector<void*> allocs;
    const TensorInfo* embed = nullptr;
    const float* final_norm = nullptr;
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    Proj lm_head;
    std::vector<Layer> layers;
    int max_ctx = 0, max_batch = 0, pos = 0;
    // activation buffers for max_batch tokens (model.rs:93-122)
    float *x, *sx, *qg, *k, *v, *o, *so, *qkv, *z, *a, *b, *on, *son, *gg, *u, *sh, *logits;
    int8_t *xq, *oq, *onq, *hq;
    uint16_t *mx, *mo, *mon, *mh;
    void* gdn_scratch = nullptr;
    void* attn_scratch = nullptr;
    int* pick = nullptr;
    std::vector<float> host_x;

    ~det_model() {
        if (st) (void)hipStreamSynchronize(st);     // teardown: a device error was reported where it happened
        for (void* p : allocs) det_free(p);
    }
    template <class T> T* alloc(size_t n) {
        void* p = det_malloc(std::max<size_t>(n * sizeof(T), 16));
        if (!p) throw Error("device allocation of " + std::to_string(n * sizeof(T)) + " bytes failed");
        allocs.push_back(p);
        return static_cast<T*>(p);
    }
    const TensorInfo& tensor(const std::string& name) const {
        const TensorInfo* t = g->tensor(name);
        if (!t) throw Error("missing tensor " + name);
        return *t;
    }
    // a float vector (any stored type, exactly dequantized) uploaded as fp32
    std::vector<float> host_vec(const std::string& name) const {
        const TensorInfo& t = tensor(name);
        std::vector<float> out(t.elems());
        const uint64_t k = t.dims[0], rows = t.elems() / k, rb = row_bytes(t.type, k);
        for (uint64_t r = 0; r < rows; r++) dequant_row(t.type, g->data(t) + r * rb, k, out.data() + r * k);
        return out;
    }
    float* upload(const std::vector<float>& h) {
        float* d = alloc<float>(h.size());
        det_memcpy(d, h.data(), h.size() * sizeof(float), st);
        return d;
    }
    float* vec(const std::string& name) { return upload(host_vec(name)); }

    // Backend::linear over tensors of one type and K (their rows concatenated along N), repacked on the device
    Lin linear(const std::vector<const TensorInfo*>& ts) {
        Lin L;
        const int bits = det_bits(ts[0]->type);
        if (!bits) throw Error(ts[0]->name + ": not a det linear (type " + type_name(ts[0]->type) + ")");
        const uint64_t K = ts[0]->dims[0], rb = row_bytes(ts[0]->type, K);
        uint64_t N = 0;
        for (const TensorInfo* t : ts) {
            if (t->dims.size() != 2) throw Error(t->name + ": not a matrix");
            L.widths.push_back((int)t->dims[1]);
            N += t->dims[1];
        }
        if (K % 128 || N > 0x7fffffff) throw Error(ts[0]->name + ": unsupported shape");
        void* rows = det_malloc(N * rb);
        if (!rows) throw Error("device allocation for " + ts[0]->name + " failed");
        uint64_t off = 0;
        for (const TensorInfo* t : ts) {
            det_memcpy(static_cast<uint8_t*>(rows) + off, g->data(*t), t->dims[1] * rb, st);
            off += t->dims[1] * rb;
        }
        size_t wb, cb, mb;
        det_linear_sizes((int)N, (int)K, bits, &wb, &cb, &mb);
        uint8_t* wq = alloc<uint8_t>(wb);
        float* cs = alloc<float>(cb / 4);
        uint16_t* ms = alloc<uint16_t>(mb / 2);
        det_linear_repack(static_cast<const uint8_t*>(rows), (int)N, (int)K, bits, wq, cs, ms, st);
        const hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) throw Error(std::string("weight repack failed on the device: ") + hipGetErrorString(e));
        det_free(rows);
        L.q = det_qlinear{wq, cs, ms, (int)N, (int)K, bits};
        return L;
    }
    // model.rs:180-197: consecutive tensors of one type and K share a linear
    Proj proj(const std::vector<std::string>& names) {
        std::vector<const TensorInfo*> infos;
        for (const auto& n : names) infos.push_back(&tensor(n));
        Proj p;
        size_t i = 0;
        while (i < infos.size()) {
            size_t j = i + 1;
            while (j < infos.size() && infos[j]->type == infos[i]->type && infos[j]->dims[0] == infos[i]->dims[0]) j++;
            p.lins.push_back(linear(std::vector<const TensorInfo*>(infos.begin() + i, infos.begin() + j)));
            i = j;
        }
        return p;
    }
    // Model::project (model.rs:416-440): one GEMM per linear, written whole or routed into its parts
    void project(const Proj& p, const int8_t* xq_, const float* sx_, const uint16_t* mx_, int t,
                 const std::vector<float*>& dsts) {
        size_t i = 0;
        for (const Lin& L : p.lins) {
            const int n = (int)L.widths.size();
            if (i + n > dsts.size() || n > 4) throw Error("projection parts do not match its outputs");
            if (n == 1) {
                det_gemm_ex(&L.q, xq_, sx_, mx_, t, dsts[i], 0, 0, nullptr, nullptr, st);
            } else {
                int offs[4];
                float* ds[4];
                int o = 0;
                for (int j = 0; j < n; j++) { offs[j] = o; ds[j] = dsts[i + j]; o += L.widths[j]; }
                det_gemm_ex(&L.q, xq_, sx_, mx_, t, nullptr, 0, n, offs, ds, st);
            }
            i += n;
        }
        if (i != dsts.size()) throw Error("projection parts do not match its outputs");
    }
};

namespace {

// model.rs:13-44: a NaN or infinity is outside the numerics' domain
void check_finite(const Gguf& g) {
    for (const TensorInfo& t : g.tensors) {
        const uint8_t* d = g.data(t);
        const uint64_t n = t.elems();
        bool bad = false;
        if (t.type == T_F32) {
            for (uint64_t i = 0; i < n && !bad; i++) { float f; memcpy(&f, d + 4 * i, 4); bad = !std::isfinite(f); }
        } else if (t.type == T_F16) {
            for (uint64_t i = 0; i < n && !bad; i++) bad = (d[2 * i + 1] & 0x7C) == 0x7C;
        } else if (t.type == T_BF16) {
            for (uint64_t i = 0; i < n && !bad; i++) bad = (d[2 * i + 1] & 0x7F) == 0x7F && (d[2 * i] & 0x80) != 0;
        } else {
            const uint64_t k = t.dims[0], rb = row_bytes(t.type, k), cb = k / 32 * bytes_per_32(det_bits(t.type));
            for (uint64_t r = 0; r < n / k && !bad; r++) { float c; memcpy(&c, d + r * rb + cb, 4); bad = !std::isfinite(c); }
        }
        if (bad) throw Error(t.name + ": non-finite value");
    }
}

det_model* load(const std::string& path, int max_ctx, int max_batch) {
    if (max_ctx < 1 || max_batch < 1) throw Error("max_ctx and max_batch must be positive");
    std::unique_ptr<det_model> m(new det_model());
    m->st = static_cast<hipStream_t>(det_hip_stream());
    try {
        m->g = Gguf::open(path);
    } catch (const Error& e) {
        throw Error(path + ": " + e.what());
    }
    const Gguf& g = *m->g;
    m->c = Config::from(g);
    const Config& c = m->c;
    check_finite(g);
    m->max_ctx = max_ctx;
    m->max_batch = max_batch;
    const TensorInfo& embed = m->tensor("token_embd.weight");
    if (!(embed.type == T_F32 || embed.type == T_F16 || embed.type == T_BF16) || embed.dims.size() != 2 ||
        embed.dims[0] != c.hidden || embed.dims[1] != c.vocab)
        throw Error("token_embd.weight: not a float [hidden][vocab] table");
    m->embed = &embed;
    if (c.hidden % 128 || c.intermediate % 128 || (c.n_heads * c.head_dim) % 128 || (c.gdn_v_heads * c.gdn_dv) % 128)
        throw Error("a linear input width is not a multiple of 128");
    if (c.conv_k != 4) throw Error("conv kernel " + std::to_string(c.conv_k) + " (4 supported)");
    m->final_norm = m->vec("output_norm.weight");
    const TensorInfo* rope = g.tensor("rope_cos");
    if (!rope) throw Error("no rope tables; run `det convert`");
    if (rope->dims.size() != 2 || rope->dims[1] < (uint64_t)max_ctx)
        throw Error("rope tables cover " + std::to_string(rope->dims.size() == 2 ? rope->dims[1] : 0) +
                    " positions, context " + std::to_string(max_ctx) + " requested");
    if (rope->dims[0] != c.rot_dim / 2) throw Error("rope tables do not have rot_dim / 2 columns");
    m->rope_cos = m->vec("rope_cos");
    m->rope_sin = m->vec("rope_sin");
    m->lm_head = m->proj({"output.weight"});
    // det.v_scale: n_attention_layers * n_kv positive finite floats, or the default (model.rs:219-243)
    const uint64_t n_attn = c.n_attention_layers();
    std::vector<float> v_scales;
    if (const Value* vs = g.get(V_SCALE_KEY); vs && vs->type == DET_GGUF_ARRAY) {
        for (const Value& e : vs->arr) {
            float f;
            if (!as_f32(e, &f) || !std::isfinite(f) || !(f > 0.0f)) { v_scales.clear(); v_scales.push_back(-1); break; }
            v_scales.push_back(f);
        }
        if (v_scales.size() != n_attn * c.n_kv)
            throw Error(std::string(V_SCALE_KEY) + ": expected " + std::to_string(n_attn * c.n_kv) + " positive floats");
    }
    const int n_h = (int)c.n_heads, n_kv = (int)c.n_kv, hd = (int)c.head_dim;
    const int n_k = (int)c.gdn_k_heads, n_v = (int)c.gdn_v_heads, dk = (int)c.gdn_dk, dv = (int)c.gdn_dv;
    const uint64_t cd = c.conv_dim();
    int attn_index = 0;
    for (size_t i = 0; i < c.attention.size(); i++) {
        const std::string b = "blk." + std::to_string(i) + ".";
        Layer L;
        L.attn = c.attention[i];
        if (L.attn) {
            std::vector<float> vs(n_kv, DEFAULT_V_SCALE), vi(n_kv);
            if (!v_scales.empty()) for (int h = 0; h < n_kv; h++) vs[h] = v_scales[(size_t)attn_index * n_kv + h];
            for (int h = 0; h < n_kv; h++) vi[h] = 1.0f / vs[h];
            attn_index++;
            L.a.qkv = m->proj({b + "attn_q.weight", b + "attn_k.weight", b + "attn_v.weight"});
            L.a.o = m->proj({b + "attn_output.weight"});
            L.a.layer = det_attn_layer{m->vec(b + "attn_q_norm.weight"), m->vec(b + "attn_k_norm.weight"), m->upload(vs),
                                       m->upload(vi)};
            L.a.kv = det_kv_cache{m->alloc<int8_t>((size_t)max_ctx * n_kv * hd), m->alloc<float>((size_t)max_ctx * n_kv),
                                  m->alloc<int16_t>((size_t)max_ctx * n_kv * hd), max_ctx, nullptr, nullptr};
        } else {
            std::vector<float> A = m->host_vec(b + "ssm_a");
            for (float& x : A) x = -x;                              // model.rs:282-296
            L.g.qkvz = m->proj({b + "attn_qkv.weight", b + "attn_gate.weight"});
            L.g.ab = m->proj({b + "ssm_alpha.weight", b + "ssm_beta.weight"});
            L.g.out = m->proj({b + "ssm_out.weight"});
            L.g.layer = det_gdn_layer{m->vec(b + "ssm_conv1d.weight"), m->upload(A), m->vec(b + "ssm_dt.bias"),
                                      m->vec(b + "ssm_norm.weight")};
            L.g.state = det_gdn_state{m->alloc<float>(3 * cd), m->alloc<float>((size_t)n_v * dk * dv)};
        }
        L.attn_norm = m->vec(b + "attn_norm.weight");
        L.ffn_norm = m->vec(b + "post_attention_norm.weight");
        L.gu = m->proj({b + "ffn_gate.weight", b + "ffn_up.weight"});
        L.down = m->proj({b + "ffn_down.weight"});
        m->layers.push_back(std::move(L));
    }
    const size_t mb = (size_t)max_batch, h = c.hidden, in = c.intermediate;
    m->x = m->alloc<float>(mb * h);
    m->xq = m->alloc<int8_t>(mb * h);
    m->sx = m->alloc<float>(mb);
    m->mx = m->alloc<uint16_t>(mb * h / 128);
    m->qg = m->alloc<float>(mb * n_h * 2 * hd);
    m->k = m->alloc<float>(mb * n_kv * hd);
    m->v = m->alloc<float>(mb * n_kv * hd);
    m->o = m->alloc<float>(mb * n_h * hd);
    m->oq = m->alloc<int8_t>(mb * n_h * hd);
    m->so = m->alloc<float>(mb);
    m->mo = m->alloc<uint16_t>(mb * n_h * hd / 128);
    m->qkv = m->alloc<float>(mb * cd);
    m->z = m->alloc<float>(mb * n_v * dv);
    m->a = m->alloc<float>(mb * n_v);
    m->b = m->alloc<float>(mb * n_v);
    m->on = m->alloc<float>(mb * n_v * dv);
    m->onq = m->alloc<int8_t>(mb * n_v * dv);
    m->son = m->alloc<float>(mb);
    m->mon = m->alloc<uint16_t>(mb * n_v * dv / 128);
    m->gg = m->alloc<float>(mb * in);
    m->u = m->alloc<float>(mb * in);
    m->hq = m->alloc<int8_t>(mb * in);
    m->sh = m->alloc<float>(mb);
    m->mh = m->alloc<uint16_t>(mb * in / 128);
    m->logits = m->alloc<float>(c.vocab);
    m->pick = m->alloc<int>(1);
    m->gdn_scratch = m->alloc<uint8_t>(det_gdn_scratch_bytes(max_batch, n_k, n_v, dk, dv));
    m->attn_scratch = m->alloc<uint8_t>(det_attn_scratch_bytes(max_batch, (int)m->c.n_heads, (int)m->c.head_dim));
    DET_CHECK(hipStreamSynchronize(m->st));
    return m.release();
}

// Model::embed_rows (model.rs:390-414): exact dequantization of the rows on the host, written into x
void embed_rows(det_model* m, const int* ids, int t) {
    const uint64_t h = m->c.hidden, rb = row_bytes(m->embed->type, h), rows = m->embed->dims[1];
    m->host_x.resize((size_t)t * h);
    for (int i = 0; i < t; i++) {
        if (ids[i] < 0 || (uint64_t)ids[i] >= rows)
            throw Error("token id " + std::to_string(ids[i]) + " is outside the embedding table (" + std::to_string(rows) + " rows)");
        dequant_row(m->embed->type, m->g->data(*m->embed) + (uint64_t)ids[i] * rb, h, m->host_x.data() + (size_t)i * h);
    }
    det_memcpy(m->x, m->host_x.data(), m->host_x.size() * sizeof(float), m->st);
}

// qwen35::forward (qwen35.rs:8-172) for t tokens at pos0; the logits of the last one into m->logits
void forward_layers(det_model* m, int pos0, int t) {
    const Config& c = m->c;
    const int h = (int)c.hidden, n_h = (int)c.n_heads, n_kv = (int)c.n_kv, hd = (int)c.head_dim;
    const int n_k = (int)c.gdn_k_heads, n_v = (int)c.gdn_v_heads, dk = (int)c.gdn_dk, dv = (int)c.gdn_dv;
    const float eps = c.eps;
    hipStream_t st = m->st;
    for (Layer& L : m->layers) {
        det_rmsnorm_quant(m->x, L.attn_norm, eps, t, h, nullptr, m->xq, m->sx, m->mx, st);
        if (L.attn) {
            m->project(L.a.qkv, m->xq, m->sx, m->mx, t, {m->qg, m->k, m->v});
            det_attention(&L.a.layer, &L.a.kv, m->qg, m->k, m->v, m->rope_cos, m->rope_sin, (int)c.rot_dim, eps, t, pos0,
                          n_h, n_kv, hd, m->o, m->attn_scratch, st);
            det_quant(m->o, t, n_h * hd, m->oq, m->so, m->mo, st);
            det_gemm_ex(&L.a.o.lins[0].q, m->oq, m->so, m->mo, t, m->x, 1, 0, nullptr, nullptr, st);
        } else {
            m->project(L.g.qkvz, m->xq, m->sx, m->mx, t, {m->qkv, m->z});
            // one token with det's default W8 a|b: the projection runs inside the GDN input stage (one launch less)
            const bool fuse_ab = t == 1 && L.g.ab.lins.size() == 1 && L.g.ab.lins[0].q.bits == 8 &&
                                 L.g.ab.lins[0].q.N == 2 * n_v && n_v / n_k <= 64;
            if (!fuse_ab) m->project(L.g.ab, m->xq, m->sx, m->mx, t, {m->a, m->b});
            det::gdn_run(&L.g.layer, &L.g.state, m->qkv, m->z, m->a, m->b, fuse_ab ? &L.g.ab.lins[0].q : nullptr, m->xq,
                         m->sx, m->mx, eps, t, n_k, n_v, dk, dv, m->on, m->gdn_scratch, st);
            det_quant(m->on, t, n_v * dv, m->onq, m->son, m->mon, st);
            det_gemm_ex(&L.g.out.lins[0].q, m->onq, m->son, m->mon, t, m->x, 1, 0, nullptr, nullptr, st);
        }
        det_rmsnorm_quant(m->x, L.ffn_norm, eps, t, h, nullptr, m->xq, m->sx, m->mx, st);
        // one token through one fused gate|up linear: the GEMV stores silu(g), and the quantization only multiplies
        const int ff = (int)c.intermediate;
        if (t == 1 && L.gu.lins.size() == 1 && L.gu.lins[0].widths.size() == 2 && ff % 128 == 0 && ff <= 32768) {
            const int offs[2] = {0, L.gu.lins[0].widths[0]};
            float* ds[2] = {m->gg, m->u};
            det::gemm_parts_silu0(&L.gu.lins[0].q, m->xq, m->sx, m->mx, 2, offs, ds, st);
            if (!det::mul_quant(m->gg, m->u, 1, ff, m->hq, m->sh, m->mh, st)) throw Error("mul_quant: unsupported row");
        } else {
            m->project(L.gu, m->xq, m->sx, m->mx, t, {m->gg, m->u});
            det_silu_mul_quant(m->gg, m->u, t, ff, nullptr, m->hq, m->sh, m->mh, st);
        }
        det_gemm_ex(&L.down.lins[0].q, m->hq, m->sh, m->mh, t, m->x, 1, 0, nullptr, nullptr, st);
    }
    // the last token's row only (qwen35.rs:157-170)
    det_rmsnorm_quant(m->x + (size_t)(t - 1) * h, m->final_norm, eps, 1, h, nullptr, m->xq, m->sx, m->mx, st);
    det_gemm_ex(&m->lm_head.lins[0].q, m->xq, m->sx, m->mx, 1, m->logits, 0, 0, nullptr, nullptr, st);
}

void forward(det_model* m, const int* ids, int t) {
    if (t < 1 || t > m->max_batch) throw Error("batch of " + std::to_string(t) + " tokens (1 to " + std::to_string(m->max_batch) + " allowed)");
    if ((long long)m->pos + t > m->max_ctx)
        throw Error(std::to_string(t) + " tokens at position " + std::to_string(m->pos) + " exceed the context of " + std::to_string(m->max_ctx));
    embed_rows(m, ids, t);
    forward_layers(m, m->pos, t);
    m->pos += t;
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

extern "C" {

const char* det_model_last_error(void) { return g_err.c_str(); }

det_model* det_model_load(const char* path, int max_ctx, int max_batch) {
    return guarded([&] { return load(path, max_ctx, max_batch); }, (det_model*)nullptr);
}

void det_model_free(det_model* m) { delete m; }
int det_model_vocab(const det_model* m) { return (int)m->c.vocab; }
int det_model_pos(const det_model* m) { return m->pos; }

void det_model_reset(det_model* m) {
    DET_CHECK(hipStreamSynchronize(m->st));
    m->pos = 0;
    const uint64_t cd = m->c.conv_dim();
    for (Layer& L : m->layers)
        if (!L.attn) {
            det_memset(L.g.state.conv_state, 0, 3 * cd * sizeof(float), m->st);
            det_memset(L.g.state.S, 0, m->c.gdn_v_heads * m->c.gdn_dk * m->c.gdn_dv * sizeof(float), m->st);
        }
}

int det_model_forward(det_model* m, const int* ids, int n) {
    return guarded([&] { forward(m, ids, n); return 0; }, -1);
}

int det_model_prefill(det_model* m, const int* ids, int n) {
    return guarded([&] {
        for (int i = 0; i < n; i += m->max_batch) forward(m, ids + i, std::min(m->max_batch, n - i));
        return 0;
    }, -1);
}

int det_model_logits(det_model* m, float* out) {
    return guarded([&] {
        det_memcpy(out, m->logits, m->c.vocab * sizeof(float), m->st);
        DET_CHECK(hipStreamSynchronize(m->st));
        return 0;
    }, -1);
}

int det_model_argmax(det_model* m) {
    return guarded([&] {
        det_argmax(m->logits, 1, (int)m->c.vocab, m->pick, m->st);
        int id = 0;
        det_memcpy(&id, m->pick, sizeof(int), m->st);
        DET_CHECK(hipStreamSynchronize(m->st));
        return id;
    }, -1);
}

int det_model_generate(det_model* m, const int* prompt, int n_prompt, int n_new, const int* stop, int n_stop, int* out) {
    return guarded([&] {
        for (int i = 0; i < n_prompt; i += m->max_batch) forward(m, prompt + i, std::min(m->max_batch, n_prompt - i));
        int n = 0;
        for (int i = 0; i < n_new; i++) {
            const int id = det_model_argmax(m);
            if (id < 0) throw Error(g_err);
            out[n++] = id;
            bool stopped = false;
            for (int s = 0; s < n_stop; s++) stopped |= stop[s] == id;
            if (stopped || i + 1 == n_new) break;
            forward(m, &id, 1);
        }
        return n;
    }, -1);
}

} // extern "C"
