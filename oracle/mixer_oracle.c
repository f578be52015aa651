/*
 * mixer_oracle.c -- CPU restatement of det's token mixers and the model-level ops around the GEMM
 * (TEST INFRASTRUCTURE ONLY: the checker, never the product; only tests/ load it).
 *
 * Restates crates/det/src/spec/layers.rs (rope, attention, Gated DeltaNet), spec/prim.rs:183-190 (l2norm),
 * spec/sample.rs:6-14 (argmax) and the Cpu backend's attention / gdn drivers (cpu.rs:212-383) op for op, in
 * scalar C compiled like det_oracle.c (-ffp-contract=off, no fast-math, default MXCSR).  Pinned independently in
 * tests/test_mixer_oracle_pins.py (closed forms on tiny heads, GQA mapping, causality, orientation of the state).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float ora_exp_f(float x);
float ora_sigmoid_f(float x);
float ora_softplus_f(float x);
float ora_silu_f(float x);
float ora_treesum(const float* x, int n);
float ora_fmax(float a, float b);
float ora_rint(float x);
float ora_quant_act_i8(const float* x, int n, int8_t* q);
void ora_rmsnorm(const float* x, const float* w, float eps, int n, float* y);

/* spec/prim.rs:183-190 l2norm: y = x * (1 / sqrt(treesum(x*x) + eps)) */
void ora_l2norm(const float* x, float eps, int n, float* y) {
    float* sq = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int i = 0; i < n; i++) sq[i] = x[i] * x[i];
    const float inv = 1.0f / sqrtf(ora_treesum(sq, n) + eps);
    free(sq);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv;
}

/* spec/layers.rs:5-13 rope: neox half split of the first 2 * half dims */
void ora_rope(float* x, const float* cs, const float* sn, int half) {
    for (int i = 0; i < half; i++) {
        const float a = x[i], b = x[i + half];
        x[i] = (a * cs[i]) - (b * sn[i]);
        x[i + half] = (b * cs[i]) + (a * sn[i]);
    }
}

/* spec/layers.rs:73-86 quant_v: clamp(rint(v * inv), -32767, 32767) */
void ora_quant_v(const float* v, float v_inv_scale, int n, int16_t* vq) {
    for (int i = 0; i < n; i++) {
        const float r = ora_rint(v[i] * v_inv_scale);
        vq[i] = r < -32767.0f ? -32767 : r > 32767.0f ? 32767 : (int16_t)r;
    }
}

/* spec/layers.rs:24-32 attn_score: (f32(dot_i8) * sq) * sk */
static float attn_score(const int8_t* qq, float sq, const int8_t* kq, float sk, int hd) {
    int32_t dot = 0;
    for (int i = 0; i < hd; i++) dot += (int32_t)qq[i] * (int32_t)kq[i];
    return ((float)dot * sq) * sk;
}

/* spec/layers.rs:36-69 attn_head: max by fmax fold from -inf, pq = rint(exp(s - mx) * 2^24) as i64,
 * den = sum pq, num[i] = sum pq * vq[i], o[i] = (f32(num[i]) / f32(den)) * v_scale.  Key j of the head is at
 * kq + j * stride, its scale at sk[j * sstride], its values at vq + j * stride. */
void ora_attn_head(const int8_t* qq, float sq, const int8_t* kq, const float* sk, const int16_t* vq, int nkeys,
                   int stride, int sstride, float v_scale, int hd, float* o) {
    float mx = -INFINITY;
    for (int j = 0; j < nkeys; j++) mx = ora_fmax(mx, attn_score(qq, sq, kq + (size_t)j * stride, sk[(size_t)j * sstride], hd));
    int64_t* num = (int64_t*)calloc((size_t)hd, sizeof(int64_t));
    int64_t den = 0;
    for (int j = 0; j < nkeys; j++) {
        const float s = attn_score(qq, sq, kq + (size_t)j * stride, sk[(size_t)j * sstride], hd);
        const int64_t pq = (int64_t)ora_rint(ora_exp_f(s - mx) * 16777216.0f);
        den += pq;
        const int16_t* vr = vq + (size_t)j * stride;
        for (int i = 0; i < hd; i++) num[i] += pq * (int64_t)vr[i];
    }
    for (int i = 0; i < hd; i++) o[i] = ((float)num[i] / (float)den) * v_scale;
    free(num);
}

/* cpu.rs:212-285 Cpu::attention.  kq[cap][n_kv][hd], sk[cap][n_kv], vq[cap][n_kv][hd]; qg[M][n_h][2 hd] (q | gate),
 * k, v [M][n_kv][hd]; rope tables [pos][rot / 2]; o[M][n_h][hd]. */
void ora_attention(const float* q_norm, const float* k_norm, const float* v_scale, const float* v_inv_scale,
                   int8_t* kq, float* sk, int16_t* vq, const float* qg, const float* k, const float* v,
                   const float* rope_cos, const float* rope_sin, int rot, float eps, int M, int pos0,
                   int n_h, int n_kv, int hd, float* o) {
    const int half = rot / 2, rep = n_h / n_kv;
    const float qscale = 1.0f / sqrtf((float)hd);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)hd);
    int8_t* qq = (int8_t*)malloc((size_t)hd);
    for (int t = 0; t < M; t++) {
        const int pos = pos0 + t;
        const float* rc = rope_cos + (size_t)pos * half;
        const float* rs = rope_sin + (size_t)pos * half;
        for (int h = 0; h < n_kv; h++) {
            const float* kr = k + ((size_t)t * n_kv + h) * hd;
            ora_rmsnorm(kr, k_norm, eps, hd, tmp);
            ora_rope(tmp, rc, rs, half);
            const size_t row = ((size_t)pos * n_kv + h) * hd;
            sk[(size_t)pos * n_kv + h] = ora_quant_act_i8(tmp, hd, kq + row);
            ora_quant_v(v + ((size_t)t * n_kv + h) * hd, v_inv_scale[h], hd, vq + row);
        }
        for (int h = 0; h < n_h; h++) {
            const float* qr = qg + ((size_t)t * n_h + h) * 2 * hd;
            const float* gate = qr + hd;
            ora_rmsnorm(qr, q_norm, eps, hd, tmp);
            ora_rope(tmp, rc, rs, half);
            for (int i = 0; i < hd; i++) tmp[i] = tmp[i] * qscale;
            const float sq = ora_quant_act_i8(tmp, hd, qq);
            const int kvh = h / rep;
            float* oh = o + ((size_t)t * n_h + h) * hd;
            ora_attn_head(qq, sq, kq + (size_t)kvh * hd, sk + kvh, vq + (size_t)kvh * hd, pos + 1, n_kv * hd, n_kv,
                          v_scale[kvh], hd, oh);
            for (int i = 0; i < hd; i++) oh[i] = oh[i] * ora_sigmoid_f(gate[i]);   /* layers.rs:64-69 attn_gate */
        }
    }
    free(tmp);
    free(qq);
}

/* spec/layers.rs:132-138 gdn_conv: ((w0 x0 + w1 x1) + w2 x2) + w3 x3, then silu */
float ora_gdn_conv(const float* win, const float* w) {
    float y = (w[0] * win[0]) + (w[1] * win[1]);
    y = y + (w[2] * win[2]);
    y = y + (w[3] * win[3]);
    return ora_silu_f(y);
}

/* spec/layers.rs:140-143 gdn_decay = exp(-(A * softplus(a + dt_bias))) */
float ora_gdn_decay(float a, float dt_bias, float a_coef) { return ora_exp_f(-(a_coef * ora_softplus_f(a + dt_bias))); }

/* spec/layers.rs:90-130 gdn_head_step over s[dk][dv] (row-major): per column j, S *= decay,
 * kv = treesum_i(S[i] k[i]), delta = (v_j - kv) beta, S[i] += k[i] delta, o_j = treesum_i(S[i] q[i]) */
void ora_gdn_head_step(float* s, int dk, int dv, const float* k, const float* q, const float* v, float beta,
                       float decay, float* o) {
    float* col = (float*)malloc(sizeof(float) * (size_t)dk);
    float* prod = (float*)malloc(sizeof(float) * (size_t)dk);
    for (int j = 0; j < dv; j++) {
        for (int i = 0; i < dk; i++) col[i] = s[(size_t)i * dv + j] * decay;
        for (int i = 0; i < dk; i++) prod[i] = col[i] * k[i];
        const float kv_mem = ora_treesum(prod, dk);
        const float delta = (v[j] - kv_mem) * beta;
        for (int i = 0; i < dk; i++) col[i] = col[i] + (k[i] * delta);
        for (int i = 0; i < dk; i++) s[(size_t)i * dv + j] = col[i];
        for (int i = 0; i < dk; i++) prod[i] = col[i] * q[i];
        o[j] = ora_treesum(prod, dk);
    }
    free(col);
    free(prod);
}

/* cpu.rs:287-383 Cpu::gdn (without the gin/gout export).  conv_w[conv_dim][4]; a_coef[n_v] (the negated ssm_a,
 * model.rs:282-296); conv_state[3][conv_dim] oldest first; S[n_v][dk][dv]; qkv[M][conv_dim]; z[M][n_v][dv];
 * a, b [M][n_v]; on[M][n_v][dv]. */
void ora_gdn(const float* conv_w, const float* a_coef, const float* dt_bias, const float* norm, float* conv_state,
             float* S, const float* qkv, const float* z, const float* a, const float* b, float eps, int M, int n_k,
             int n_v, int dk, int dv, float* on) {
    const int kd = n_k * dk, conv_dim = 2 * kd + n_v * dv, rep = n_v / n_k;
    const uint32_t qbits = 0x3DB504F3u;         /* spec/layers.rs:146 QSCALE_GDN = fp32(1/sqrt(128)) by its bits */
    float QSCALE;
    memcpy(&QSCALE, &qbits, 4);
    float* y = (float*)malloc(sizeof(float) * (size_t)conv_dim);
    float* q = (float*)malloc(sizeof(float) * (size_t)kd);
    float* kk = (float*)malloc(sizeof(float) * (size_t)kd);
    float* beta = (float*)malloc(sizeof(float) * (size_t)n_v);
    float* decay = (float*)malloc(sizeof(float) * (size_t)n_v);
    float* oh = (float*)malloc(sizeof(float) * (size_t)dv);
    float* yn = (float*)malloc(sizeof(float) * (size_t)dv);
    for (int t = 0; t < M; t++) {
        const float* xt = qkv + (size_t)t * conv_dim;
        for (int c = 0; c < conv_dim; c++) {
            const float win[4] = {conv_state[c], conv_state[conv_dim + c], conv_state[2 * conv_dim + c], xt[c]};
            y[c] = ora_gdn_conv(win, conv_w + (size_t)c * 4);
        }
        memmove(conv_state, conv_state + conv_dim, sizeof(float) * 2 * (size_t)conv_dim);
        memcpy(conv_state + 2 * (size_t)conv_dim, xt, sizeof(float) * (size_t)conv_dim);
        for (int h = 0; h < n_k; h++) {
            ora_l2norm(y + (size_t)h * dk, eps, dk, q + (size_t)h * dk);
            for (int i = 0; i < dk; i++) q[h * dk + i] = q[h * dk + i] * QSCALE;
            ora_l2norm(y + kd + (size_t)h * dk, eps, dk, kk + (size_t)h * dk);
        }
        const float* vv = y + 2 * kd;
        for (int h = 0; h < n_v; h++) {
            beta[h] = ora_sigmoid_f(b[(size_t)t * n_v + h]);
            decay[h] = ora_gdn_decay(a[(size_t)t * n_v + h], dt_bias[h], a_coef[h]);
        }
        for (int h = 0; h < n_v; h++) {
            const int kh = h / rep;
            ora_gdn_head_step(S + (size_t)h * dk * dv, dk, dv, kk + (size_t)kh * dk, q + (size_t)kh * dk,
                              vv + (size_t)h * dv, beta[h], decay[h], oh);
            ora_rmsnorm(oh, norm, eps, dv, yn);
            const size_t base = ((size_t)t * n_v + h) * dv;
            for (int j = 0; j < dv; j++) on[base + j] = yn[j] * ora_silu_f(z[base + j]);
        }
    }
    free(y); free(q); free(kk); free(beta); free(decay); free(oh); free(yn);
}

/* spec/sample.rs:6-14 argmax: the first index of the largest value (strict >) */
int ora_argmax(const float* x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}
