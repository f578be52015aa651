/*
 * det_oracle.c -- CPU restatement of det's quantized-linear path (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the checker, never the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  The shipped path is det_amd/libdet_hip.so, which never calls into it.
 *
 * Every function restates the reference (crates/det/src, Rust) op for op, in scalar C.  Build with
 * -ffp-contract=off and no fast-math, default MXCSR (round to nearest even, no FTZ/DAZ), so that every
 * float op is one IEEE binary32/binary64 op exactly as in the Rust.
 *
 * Pinning (how each function is checked independently of this restatement) is in tests/test_oracle_pins.py:
 *   ora_unpack_row / ora_pack        exhaustive pack->unpack identity + numpy restatement from docs/SPEC.md
 *   ora_quantize_row                 reference KAT (quantize.rs:108-140) invariants + numpy restatement
 *   ora_quant_act_i8g / _i8          closed-form rows, Rust cast semantics (NaN->0), numpy restatement
 *   ora_gemm_row / ora_gemm          brute-force exact integers (python ints) + exact RNE conversion
 *   ora_i64_to_f32                   python-integer RNE on crafted ties
 *   ora_rng_*                        reference xorshift64 (conformance.rs:35-59), fixed vectors
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 128

/* ---------------------------------------------------------------- scalar primitives (spec/prim.rs) */

/* spec/prim.rs:58-70 fmax: larger operand, -0 below +0, a NaN operand is returned. */
float ora_fmax(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    if (a > b || (a == b && signbit(b))) return a;
    return b;
}
/* spec/prim.rs:41-56 fmin */
float ora_fmin(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    if (a < b || (a == b && signbit(a))) return a;
    return b;
}
/* spec/prim.rs:72-76 rint: round half to even (default rounding mode). */
float ora_rint(float x) { return rintf(x); }

/* spec/prim.rs:193-195 absmax: fold of fmax(|v|) from +0. */
float ora_absmax(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) m = ora_fmax(m, fabsf(x[i]));
    return m;
}

/* Rust `v as i8` after the explicit clamp of spec/quant.rs:51-60: NaN -> 0. */
static int8_t clamp_i8(float v) {
    if (v < -127.0f) return -127;
    if (v > 127.0f) return 127;
    if (isnan(v)) return 0;
    return (int8_t)(int)v;
}
/* Rust `m as u16` for m already clamped to [1, 65535] or NaN (NaN -> 0). */
static uint16_t as_u16(float m) { return isnan(m) ? 0 : (uint16_t)(int)m; }

/* int64 -> fp32, round to nearest even (Rust `as`, i.e. cvtsi2ss under the default MXCSR). */
float ora_i64_to_f32(int64_t v) { return (float)v; }

/* spec/prim.rs:78-99 exp_f */
static const float EXP_P[6] = {(float)1.9875691500E-4, (float)1.3981999507E-3, (float)8.3334519073E-3,
                               (float)4.1665795894E-2, (float)1.6666665459E-1, (float)5.0000001201E-1};
float ora_exp_f(float x) {
    x = ora_fmin(x, 88.0f);
    if (x < -87.0f) return 0.0f;
    float n = floorf((x * (float)1.44269504088896341) + 0.5f);
    float r = x - (n * (float)0.693359375);
    r = r - (n * (float)-2.12194440e-4);
    float z = r * r;
    float y = EXP_P[0];
    for (int i = 1; i < 6; i++) y = (y * r) + EXP_P[i];
    y = (y * z) + r;
    y = y + 1.0f;
    int ni = (int)n;
    uint32_t sb = (uint32_t)((ni + 127) << 23);
    float scale;
    memcpy(&scale, &sb, 4);
    return y * scale;
}
/* spec/prim.rs:101-126 log_f */
static const float LOG_P[9] = {(float)7.0376836292E-2, (float)-1.1514610310E-1, (float)1.1676998740E-1,
                               (float)-1.2420140846E-1, (float)1.4249322787E-1, (float)-1.6668057665E-1,
                               (float)2.0000714765E-1, (float)-2.4999993993E-1, (float)3.3333331174E-1};
float ora_log_f(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    int e = (int)((b >> 23) & 0xFF) - 126;
    uint32_t mb = (b & 0x007FFFFFu) | 0x3F000000u;
    float m;
    memcpy(&m, &mb, 4);
    if (m < (float)0.707106781186547524) { e -= 1; m = (m + m) - 1.0f; } else { m = m - 1.0f; }
    float z = m * m;
    float y = LOG_P[0];
    for (int i = 1; i < 9; i++) y = (y * m) + LOG_P[i];
    y = y * m;
    y = y * z;
    float ef = (float)e;
    y = y + ((float)-2.12194440e-4 * ef);
    y = y + (-0.5f * z);
    float r = m + y;
    r = r + ((float)0.693359375 * ef);
    return r;
}
/* spec/prim.rs:128-137 softplus_f */
float ora_softplus_f(float x) {
    if (x > 20.0f) return x;
    if (x < -15.0f) return ora_exp_f(x);
    float xs = ora_fmin(x, 20.0f);
    return ora_log_f(1.0f + ora_exp_f(xs));
}
/* spec/prim.rs:139-145 sigmoid_f */
float ora_sigmoid_f(float x) {
    if (x < -80.0f) return ora_exp_f(x);
    float xs = ora_fmax(x, -80.0f);
    return 1.0f / (1.0f + ora_exp_f(-xs));
}
/* spec/prim.rs:147-149 silu_f */
float ora_silu_f(float x) { return x * ora_sigmoid_f(x); }

/* spec/prim.rs:154-170 treesum: balanced tree over x padded with +0 to the next power of two. */
float ora_treesum(const float* x, int n) {
    if (n <= 0) return 0.0f;
    int p = 1;
    while (p < n) p <<= 1;
    float* s = (float*)malloc(sizeof(float) * (size_t)p);
    for (int i = 0; i < p; i++) s[i] = i < n ? x[i] : 0.0f;
    for (int w = p; w > 1;) {
        w /= 2;
        for (int i = 0; i < w; i++) s[i] = s[2 * i] + s[2 * i + 1];
    }
    float r = s[0];
    free(s);
    return r;
}
/* spec/prim.rs:172-181 rmsnorm */
void ora_rmsnorm(const float* x, const float* w, float eps, int n, float* y) {
    float* sq = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int i = 0; i < n; i++) sq[i] = x[i] * x[i];
    float ss = ora_treesum(sq, n);
    free(sq);
    float mean = ss / (float)n;
    float inv = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) y[i] = (x[i] * inv) * w[i];
}

/* ---------------------------------------------------------------- activation quantization (spec/quant.rs) */

/* spec/quant.rs:8-16 quant_act_i8 (per row). Returns s. */
float ora_quant_act_i8(const float* x, int n, int8_t* q) {
    float amax = ora_absmax(x, n);
    float s = amax == 0.0f ? 1.0f : amax / 127.0f;
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) q[i] = clamp_i8(ora_rint(x[i] * inv));
    return s;
}

/* spec/quant.rs:21-49 quant_act_i8g (per row, per 128-group multipliers). Returns sx. */
float ora_quant_act_i8g(const float* x, int n, int8_t* q, uint16_t* mx) {
    int g = n / GROUP;
    float* s_g = (float*)malloc(sizeof(float) * (size_t)(g > 0 ? g : 1));
    for (int i = 0; i < g; i++) s_g[i] = ora_absmax(x + (size_t)i * GROUP, GROUP) / 127.0f;
    float smax = 0.0f;
    for (int i = 0; i < g; i++) smax = ora_fmax(smax, s_g[i]);
    float sx = smax == 0.0f ? 1.0f : smax / 65535.0f;
    for (int i = 0; i < g; i++) {
        float m = ora_rint(s_g[i] / sx);
        if (m < 1.0f) m = 1.0f;
        else if (m > 65535.0f) m = 65535.0f;
        mx[i] = as_u16(m);
        float eff = sx * (float)mx[i];
        float inv = 1.0f / eff;
        for (int k = 0; k < GROUP; k++) q[i * GROUP + k] = clamp_i8(ora_rint(x[i * GROUP + k] * inv));
    }
    free(s_g);
    return sx;
}

/* cpu.rs:130-140 Cpu::quant over M rows (mx == NULL selects quant_act_i8, as det_cuda.h:35-39). */
void ora_quant(const float* x, int M, int n, int8_t* xq, float* sx, uint16_t* mx) {
    for (int t = 0; t < M; t++) {
        const float* xr = x + (size_t)t * n;
        if (mx) sx[t] = ora_quant_act_i8g(xr, n, xq + (size_t)t * n, mx + (size_t)t * (n / GROUP));
        else sx[t] = ora_quant_act_i8(xr, n, xq + (size_t)t * n);
    }
}

/* cpu.rs:105-128 Cpu::rmsnorm_quant */
void ora_rmsnorm_quant(const float* x, const float* w, float eps, int M, int n, int8_t* xq, float* sx, uint16_t* mx) {
    float* y = (float*)malloc(sizeof(float) * (size_t)n);
    for (int t = 0; t < M; t++) {
        ora_rmsnorm(x + (size_t)t * n, w, eps, n, y);
        sx[t] = ora_quant_act_i8g(y, n, xq + (size_t)t * n, mx + (size_t)t * (n / GROUP));
    }
    free(y);
}

/* cpu.rs:187-211 Cpu::silu_mul_quant */
void ora_silu_mul_quant(const float* g, const float* u, int M, int n, int8_t* hq, float* sh, uint16_t* mh) {
    float* h = (float*)malloc(sizeof(float) * (size_t)n);
    for (int t = 0; t < M; t++) {
        for (int i = 0; i < n; i++) h[i] = ora_silu_f(g[(size_t)t * n + i]) * u[(size_t)t * n + i];
        sh[t] = ora_quant_act_i8g(h, n, hq + (size_t)t * n, mh + (size_t)t * (n / GROUP));
    }
    free(h);
}

/* ---------------------------------------------------------------- det rows (spec/tensor.rs) */

/* spec/tensor.rs:33-40 bytes_per_32 */
int ora_bytes_per_32(int bits) { return bits == 8 ? 32 : bits == 6 ? 24 : bits == 4 ? 16 : -1; }
/* spec/tensor.rs:49-55 det_row_bytes */
size_t ora_row_bytes(int bits, int k) { return (size_t)k / 32 * ora_bytes_per_32(bits) + 4 + (size_t)k / GROUP * 2; }

/* spec/tensor.rs:57-70 det_row: c and m of a row */
static void row_scales(const uint8_t* row, int bits, int k, float* c, uint16_t* m) {
    size_t nc = (size_t)k / 32 * ora_bytes_per_32(bits);
    memcpy(c, row + nc, 4);
    for (int g = 0; g < k / GROUP; g++) m[g] = (uint16_t)(row[nc + 4 + 2 * g] | (row[nc + 5 + 2 * g] << 8));
}

/* spec/quant.rs:63-97 unpack_row */
void ora_unpack_row(const uint8_t* p, int bits, int k, int8_t* out) {
    if (bits == 8) {
        for (int i = 0; i < k; i++) out[i] = (int8_t)p[i];
    } else if (bits == 4) {
        for (int blk = 0; blk < k / 32; blk++) {
            const uint8_t* b = p + blk * 16;
            for (int i = 0; i < 16; i++) {
                out[blk * 32 + i] = (int8_t)((b[i] & 0xF) - 8);
                out[blk * 32 + 16 + i] = (int8_t)((b[i] >> 4) - 8);
            }
        }
    } else if (bits == 6) {
        for (int blk = 0; blk < k / 32; blk++) {
            const uint8_t* ql = p + blk * 24;
            const uint8_t* qh = ql + 16;
            for (int i = 0; i < 32; i++) {
                int lo = i < 16 ? (ql[i] & 0xF) : (ql[i - 16] >> 4);
                int hi = (qh[i % 8] >> (2 * (i / 8))) & 3;
                out[blk * 32 + i] = (int8_t)((lo | (hi << 4)) - 32);
            }
        }
    } else {
        abort();
    }
}

/* quantize.rs:9-31 pack (n a multiple of 32) */
void ora_pack(const int8_t* codes, int n, int bits, uint8_t* out) {
    for (int blk = 0; blk < n / 32; blk++) {
        const int8_t* q = codes + blk * 32;
        if (bits == 8) {
            for (int i = 0; i < 32; i++) *out++ = (uint8_t)q[i];
        } else if (bits == 4) {
            for (int i = 0; i < 16; i++) *out++ = (uint8_t)((q[i] + 8) | ((q[i + 16] + 8) << 4));
        } else if (bits == 6) {
            uint8_t u[32];
            for (int i = 0; i < 32; i++) u[i] = (uint8_t)(q[i] + 32);
            for (int i = 0; i < 16; i++) *out++ = (uint8_t)((u[i] & 0xF) | ((u[i + 16] & 0xF) << 4));
            for (int i = 0; i < 8; i++)
                *out++ = (uint8_t)((u[i] >> 4) | ((u[i + 8] >> 4) << 2) | ((u[i + 16] >> 4) << 4) | ((u[i + 24] >> 4) << 6));
        } else {
            abort();
        }
    }
}

/* ---------------------------------------------------------------- GEMM (spec/quant.rs:102-117, cpu.rs:142-185) */

/* spec/quant.rs:102-117 gemm_row: exact int64 acc, then (f32(acc) * c) * sx.  mx == NULL means all ones. */
float ora_gemm_row(const int8_t* wq, float c, const uint16_t* m, const int8_t* xq, float sx, const uint16_t* mx, int k) {
    int64_t acc = 0;
    for (int g = 0; g < k / GROUP; g++) {
        int64_t part = 0;
        for (int i = g * GROUP; i < (g + 1) * GROUP; i++) part += (int64_t)wq[i] * (int64_t)xq[i];
        int64_t mult = (int64_t)m[g] * (mx ? (int64_t)mx[g] : 1);
        acc += mult * part;
    }
    return (ora_i64_to_f32(acc) * c) * sx;
}

/* Exact integer accumulator of one output (for pinning tests). */
int64_t ora_gemm_acc(const int8_t* wq, const uint16_t* m, const int8_t* xq, const uint16_t* mx, int k) {
    int64_t acc = 0;
    for (int g = 0; g < k / GROUP; g++) {
        int64_t part = 0;
        for (int i = g * GROUP; i < (g + 1) * GROUP; i++) part += (int64_t)wq[i] * (int64_t)xq[i];
        acc += (int64_t)m[g] * (mx ? (int64_t)mx[g] : 1) * part;
    }
    return acc;
}

/* cpu.rs:142-185 Cpu::gemm over det rows rows[N][row_bytes] with the GemmOut semantics of backend.rs:138-142:
 * accumulate != 0: y = y + v (one fp32 add); nparts > 1: column n in [offs[i], offs[i+1]) goes to
 * dsts[i][t][n - offs[i]] (offs[nparts] == N).  Parallel over rows (independent outputs). */
void ora_gemm(const uint8_t* rows, int N, int K, int bits, const int8_t* xq, const float* sx, const uint16_t* mx, int M,
              float* y, int accumulate, int nparts, const int* offs, float* const* dsts) {
    size_t rb = ora_row_bytes(bits, K);
    int G = K / GROUP;
#pragma omp parallel
    {
        int8_t* wq = (int8_t*)malloc((size_t)K);
        uint16_t* m = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)G);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            const uint8_t* row = rows + (size_t)n * rb;
            float c;
            row_scales(row, bits, K, &c, m);
            ora_unpack_row(row, bits, K, wq);
            for (int t = 0; t < M; t++) {
                float v = ora_gemm_row(wq, c, m, xq + (size_t)t * K, sx[t], mx ? mx + (size_t)t * G : NULL, K);
                if (nparts > 1) {
                    int i = 0;
                    while (i + 1 < nparts && n >= offs[i + 1]) i++;
                    int w = (i + 1 < nparts ? offs[i + 1] : N) - offs[i];
                    dsts[i][(size_t)t * w + (n - offs[i])] = v;
                } else {
                    float* p = y + (size_t)t * N + n;
                    *p = accumulate ? *p + v : v;
                }
            }
        }
        free(wq);
        free(m);
    }
}

/* ---------------------------------------------------------------- weight quantizer (quantize.rs) */

/* quantize.rs:33-55 group_scale: best of 11 scales base*(0.80+0.02*step) by sequential f64 squared error,
 * strict < (first wins); all-zero group -> 1.0 */
static double group_scale(const double* w, int n, double qmax) {
    double amax = 0.0;
    for (int i = 0; i < n; i++) amax = fmax(amax, fabs(w[i]));
    if (amax == 0.0) return 1.0;
    double base = amax / qmax;
    double best_err = INFINITY, best_s = base;
    for (int step = 0; step <= 10; step++) {
        double s = base * (0.80 + 0.02 * (double)step);
        double err = -0.0;
        for (int i = 0; i < n; i++) {
            double q = rint(w[i] / s);
            if (q < -qmax) q = -qmax;
            if (q > qmax) q = qmax;
            double d = q * s - w[i];
            err = err + d * d;
        }
        if (err < best_err) { best_err = err; best_s = s; }
    }
    return best_s;
}

/* quantize.rs:58-85 quantize_row: one det row [codes][c][m] from k weights. */
void ora_quantize_row(const float* w, int k, int bits, uint8_t* out) {
    int G = k / GROUP;
    double qmax = (double)((1 << (bits - 1)) - 1);
    double* wd = (double*)malloc(sizeof(double) * (size_t)k);
    double* sc = (double*)malloc(sizeof(double) * (size_t)G);
    int8_t* codes = (int8_t*)malloc((size_t)k);
    uint16_t* m = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)G);
    for (int i = 0; i < k; i++) wd[i] = (double)w[i];
    for (int g = 0; g < G; g++) sc[g] = group_scale(wd + (size_t)g * GROUP, GROUP, qmax);
    double smax = 0.0;
    for (int g = 0; g < G; g++) smax = fmax(smax, sc[g]);
    float c = (float)(smax / 65535.0);
    for (int g = 0; g < G; g++) {
        double v = rint(sc[g] / (double)c);
        if (v < 1.0) v = 1.0;
        if (v > 65535.0) v = 65535.0;
        m[g] = (uint16_t)v;
    }
    for (int g = 0; g < G; g++) {
        double eff = (double)c * (double)m[g];
        for (int i = g * GROUP; i < (g + 1) * GROUP; i++) {
            double q = rint(wd[i] / eff);
            if (q < -qmax) q = -qmax;
            if (q > qmax) q = qmax;
            codes[i] = (int8_t)q;
        }
    }
    size_t nc = (size_t)k / 32 * ora_bytes_per_32(bits);
    ora_pack(codes, k, bits, out);
    memcpy(out + nc, &c, 4);
    for (int g = 0; g < G; g++) { out[nc + 4 + 2 * g] = (uint8_t)(m[g] & 0xFF); out[nc + 5 + 2 * g] = (uint8_t)(m[g] >> 8); }
    free(wd); free(sc); free(codes); free(m);
}

/* quantize.rs:88-100 quantize_rows (rows are independent; parallel order is irrelevant) */
void ora_quantize_rows(const float* w, int n, int k, int bits, uint8_t* out) {
    size_t rb = ora_row_bytes(bits, k);
#pragma omp parallel for schedule(dynamic, 64)
    for (int r = 0; r < n; r++) ora_quantize_row(w + (size_t)r * k, k, bits, out + (size_t)r * rb);
}

/* ---------------------------------------------------------------- conformance RNG (conformance.rs:35-59) */

uint64_t ora_rng_next(uint64_t* s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}
float ora_rng_unit(uint64_t* s) { return (float)((double)(ora_rng_next(s) >> 11) / (double)(1ULL << 53) * 2.0 - 1.0); }
uint8_t ora_rng_byte(uint64_t* s) { return (uint8_t)(ora_rng_next(s) >> 56); }
uint64_t ora_rng_below(uint64_t* s, uint64_t n) { return ora_rng_next(s) % n; }
float ora_rng_denorm(uint64_t* s) {
    uint32_t b = (uint32_t)ora_rng_next(s) & 0x807FFFFFu;
    if ((b & 0x7FFFFFFFu) == 0) b |= 1;
    float f;
    memcpy(&f, &b, 4);
    return f;
}
void ora_rng_units(uint64_t* s, float* out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = ora_rng_unit(s); }

/* conformance.rs:104-120 fake_gguf: n det rows of random code bytes, c in [1e-8, 1e-6+1e-8), m in [1, 65535]. */
void ora_fake_rows(uint64_t* s, int bits, int n, int k, uint8_t* rows) {
    size_t rb = ora_row_bytes(bits, k), nc = (size_t)k / 32 * ora_bytes_per_32(bits);
    for (int r = 0; r < n; r++) {
        uint8_t* row = rows + (size_t)r * rb;
        for (size_t b = 0; b < nc; b++) row[b] = ora_rng_byte(s);
        float c = fabsf(ora_rng_unit(s)) * 1e-6f + 1e-8f;
        memcpy(row + nc, &c, 4);
        for (int g = 0; g < k / GROUP; g++) {
            uint16_t m = (uint16_t)(1 + ora_rng_below(s, 65535));
            row[nc + 4 + 2 * g] = (uint8_t)(m & 0xFF);
            row[nc + 5 + 2 * g] = (uint8_t)(m >> 8);
        }
    }
}

/* conformance.rs:147-156 acts: x[t][g*128+i] = unit * 10^-((g+t)%5) (before quantization). */
void ora_acts_x(uint64_t* s, int m, int k, float* x) {
    for (int t = 0; t < m; t++)
        for (int g = 0; g < k / GROUP; g++) {
            int e = (g + t) % 5;
            float p = 1.0f;
            for (int j = 0; j < e; j++) p = p * 10.0f;
            float scale = 1.0f / p;
            for (int i = 0; i < GROUP; i++) x[(size_t)t * k + g * GROUP + i] = ora_rng_unit(s) * scale;
        }
}
