// The token mixers of det's qwen35 forward and argmax: attention over the int8 / int16 KV cache, the Gated
// DeltaNet (conv, l2norm, recurrence, gated norm) and argmax.  Semantics are those of the reference backend
// (crates/det/src/cpu.rs:212-383 over spec/layers.rs, spec/prim.rs:154-190, spec/sample.rs:6-14); the C ABI is
// det_cuda.h:60-103's (det_attention, det_gdn, det_argmax).
//
// Every reduction the spec orders is reproduced in that order: treesum is a balanced tree over the row padded to a
// power of two (ping-pong LDS levels, or an in-register subtree per lane plus lane shuffles that combine the
// aligned subtrees in tree order); the attention max is an fmax fold (order-free) and its weighted sums are exact
// int64 integers (order-free).
#include <algorithm>
#include "common.h"
#include "mixer_internal.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

constexpr int RT = 256;          // threads of the row kernels

__device__ __forceinline__ int p2(int n) { int p = 1; while (p < n) p <<= 1; return p; }

__device__ __forceinline__ float wave_fmax(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmax_spec(v, __shfl_xor(v, o, 64));
    return v;
}

// spec/prim.rs:154-170 treesum of v[0..n) (squared when SQ) over the block; s, t: LDS scratch of p2(n) and
// p2(n) / 2 floats.  Every thread returns the sum; s and t are free again when it returns.
template <bool SQ>
__device__ float block_treesum(const float* v, int n, float* s, float* t) {
    const int p = p2(n);
    for (int i = threadIdx.x; i < p; i += blockDim.x) s[i] = i < n ? (SQ ? v[i] * v[i] : v[i]) : 0.0f;
    for (int w = p >> 1; w >= 1; w >>= 1) {
        __syncthreads();
        for (int i = threadIdx.x; i < w; i += blockDim.x) t[i] = s[2 * i] + s[2 * i + 1];
        float* u = s; s = t; t = u;
    }
    __syncthreads();
    const float r = s[0];
    __syncthreads();
    return r;
}

// order-free max of |v[0..n)| from 0 (spec/prim.rs:193-195); red: LDS of blockDim / 64 floats
__device__ float block_absmax(const float* v, int n, float* red) {
    float am = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) am = fmax_spec(am, __builtin_fabsf(v[i]));
    am = wave_fmax(am);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
    __syncthreads();
    am = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) am = fmax_spec(am, red[w]);
    __syncthreads();
    return am;
}

// spec/prim.rs:172-181 rmsnorm of x[0..n) in LDS, in place, weights w (global)
__device__ void block_rmsnorm(float* x, int n, const float* w, float eps, float* s, float* t) {
    const float ss = block_treesum<true>(x, n, s, t);
    const float inv = 1.0f / __builtin_sqrtf((ss / (float)n) + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = (x[i] * inv) * w[i];
    __syncthreads();
}

// spec/layers.rs:5-13 rope of x in LDS: thread i < half rotates the pair (x[i], x[i + half]), which no other
// thread touches
__device__ void block_rope(float* x, const float* cs, const float* sn, int half) {
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float a = x[i], b = x[i + half];
        x[i] = (a * cs[i]) - (b * sn[i]);
        x[i + half] = (b * cs[i]) + (a * sn[i]);
    }
    __syncthreads();
}

// spec/quant.rs:8-16 quant_act_i8 of x[0..n) (LDS) into q; returns s
__device__ float block_quant_i8(const float* x, int n, int8_t* q, float* red) {
    const float am = block_absmax(x, n, red);
    const float s = am == 0.0f ? 1.0f : am / 127.0f;
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) q[i] = (int8_t)clamp_i8(rint_(x[i] * inv));
    return s;
}

// ------------------------------------------------------------------ attention (cpu.rs:212-285)
// One workgroup per (token, kv head): k -> rmsnorm(k_norm) -> rope -> quant_act_i8 into kq / sk at row pos0 + t,
// v -> quant_v (spec/layers.rs:73-86) into vq.  LDS: x[hd], tree s[p], t[p / 2].
__device__ __forceinline__ void attn_kv_row(int kvrow, const float* __restrict__ k_norm, const float* __restrict__ v_inv_scale,
                                                int8_t* __restrict__ kq, float* __restrict__ sk, int16_t* __restrict__ vq,
                                                const float* __restrict__ k, const float* __restrict__ v,
                                                const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
                                                int half, float eps, int pos0, int n_kv, int hd) {
    extern __shared__ float lds[];
    __shared__ float red[RT / 64];
    float* x = lds;
    float* s = x + hd;
    float* t = s + p2(hd);
    const int tok = kvrow / n_kv, h = kvrow - tok * n_kv, pos = pos0 + tok;
    const size_t src = ((size_t)tok * n_kv + h) * hd;
    for (int i = threadIdx.x; i < hd; i += RT) x[i] = k[src + i];
    __syncthreads();
    block_rmsnorm(x, hd, k_norm, eps, s, t);
    block_rope(x, rope_cos + (size_t)pos * half, rope_sin + (size_t)pos * half, half);
    const size_t row = ((size_t)pos * n_kv + h) * hd;
    const float sc = block_quant_i8(x, hd, kq + row, red);
    if (threadIdx.x == 0) sk[(size_t)pos * n_kv + h] = sc;
    const float vi = v_inv_scale[h];
    for (int i = threadIdx.x; i < hd; i += RT) {
        const float r = rint_(v[src + i] * vi);
        vq[row + i] = (int16_t)(r < -32767.0f ? -32767 : r > 32767.0f ? 32767 : __builtin_isnan(r) ? 0 : (int)r);
    }
}

// The attention of a token and head over keys 0 .. pos of kv head h / rep (spec/layers.rs:24-69):
// s_j = (f32(dot(qq, kq_j)) * sq) * sk_j, mx = fmax fold of the s_j, pq_j = rint(exp(s_j - mx) * 2^24) as an
// integer, den = sum pq_j, num_i = sum pq_j vq_j[i], o_i = ((f32(num_i) / f32(den)) * v_scale) * sigmoid(gate_i).
// The max is order-free and the sums are exact integers, so the keys are split into chunks of CK, one workgroup
// each (grid x = chunk, grid y = token * n_h + head), and the chunks meet through device atomics:
//   k_attn_prep the cache rows of the new k and v (k_attn_kv's work) and the q rows: q -> rmsnorm(q_norm) -> rope
//              -> * 1/sqrt(hd) -> quant_act_i8 into scratch, clearing the head's max, den, num and chunk counter
//              (so no memset is needed and the launches can be captured);
//   k_attn_max  the chunk's scores and their max, merged by atomicMax on an order-preserving integer image;
//   k_attn_acc  the chunk's scores again (same integers, same fp32 ops), its pq_j, and the chunk's den and num
//              partials added by int64 atomics; for a few tokens the row's last chunk to count itself writes the
//              output, for a batch k_attn_fin does (waiting for the atomics in every workgroup costs more there).
// A score takes 16 lanes: lane l reads words l, l + 16, ... of the key row (coalesced) into v_dot4 sums, and the
// 16 partial sums meet by DPP exchanges (integers: any order).
struct AttnScratch {
    int8_t* qq;       // [M][n_h][hd]
    float* sq;        // [M][n_h]
    unsigned* mxo;    // [M][n_h] order-preserving image of the max
    long long* den;   // [M][n_h]
    long long* num;   // [M][n_h][hd]
    unsigned* cnt;    // [M][n_h] chunks of the row that have added their sums
    size_t bytes;
};
__host__ __device__ inline size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }
inline AttnScratch attn_layout(void* base, int M, int n_h, int hd) {
    AttnScratch S{};
    const size_t r = (size_t)M * n_h;
    char* p = static_cast<char*>(base);
    size_t off = 0;
    S.qq = reinterpret_cast<int8_t*>(p + off);     off += al256(r * hd);
    S.sq = reinterpret_cast<float*>(p + off);      off += al256(r * 4);
    S.mxo = reinterpret_cast<unsigned*>(p + off);  off += al256(r * 4);
    S.den = reinterpret_cast<long long*>(p + off); off += al256(r * 8);
    S.num = reinterpret_cast<long long*>(p + off); off += al256(r * hd * 8);
    S.cnt = reinterpret_cast<unsigned*>(p + off);  off += al256(r * 4);
    S.bytes = off;
    return S;
}
// fp32 total order of fmax_spec (-0 below +0; every NaN above everything, as one canonical NaN) as unsigned
// integers, 0 below every value
__device__ __forceinline__ unsigned f2ord(float f) {
    if (__builtin_isnan(f)) return 0xffffffffu;
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(unsigned u) {
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
__device__ __forceinline__ int sum16(int v) {       // every lane of an aligned 16-lane row gets the row's sum
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x141>(v);
    v += dpp_i<0x140>(v);
    return v;
}
constexpr int AQW = 16;     // max words (4 codes each) per lane of a score: hd <= 1024

__device__ __forceinline__ void attn_q_row(int qrow, const float* __restrict__ q_norm, const float* __restrict__ qg,
                                               const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
                                               int half, float eps, int pos0, int n_h, int hd, AttnScratch S) {
    extern __shared__ float lds[];
    __shared__ float red[RT / 64];
    const int p = p2(hd);
    float* x = lds;
    float* s = x + hd;
    float* t = s + p;
    const int row = qrow, tok = row / n_h, pos = pos0 + tok;
    const float* qr = qg + (size_t)row * 2 * hd;
    for (int i = threadIdx.x; i < hd; i += RT) x[i] = qr[i];
    __syncthreads();
    block_rmsnorm(x, hd, q_norm, eps, s, t);
    block_rope(x, rope_cos + (size_t)pos * half, rope_sin + (size_t)pos * half, half);
    const float qscale = 1.0f / __builtin_sqrtf((float)hd);
    for (int i = threadIdx.x; i < hd; i += RT) x[i] = x[i] * qscale;
    __syncthreads();
    const float sq = block_quant_i8(x, hd, S.qq + (size_t)row * hd, red);
    for (int i = threadIdx.x; i < hd; i += RT) S.num[(size_t)row * hd + i] = 0;
    if (threadIdx.x == 0) {
        S.sq[row] = sq;
        S.mxo[row] = 0u;
        S.den[row] = 0;
        S.cnt[row] = 0u;
    }
}

// the k rows, v rows and q rows of the call in one launch: workgroups 0 .. nkv - 1 take (token, kv head) rows,
// the rest (token, head) rows
__global__ void __launch_bounds__(RT) k_attn_prep(const float* __restrict__ k_norm, const float* __restrict__ v_inv_scale,
                                                  int8_t* __restrict__ kq, float* __restrict__ sk, int16_t* __restrict__ vq,
                                                  const float* __restrict__ k, const float* __restrict__ v,
                                                  const float* __restrict__ q_norm, const float* __restrict__ qg,
                                                  const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
                                                  int half, float eps, int pos0, int n_kv, int n_h, int hd, int nkv,
                                                  AttnScratch S) {
    if ((int)blockIdx.x < nkv) attn_kv_row(blockIdx.x, k_norm, v_inv_scale, kq, sk, vq, k, v, rope_cos, rope_sin, half, eps, pos0, n_kv, hd);
    else attn_q_row(blockIdx.x - nkv, q_norm, qg, rope_cos, rope_sin, half, eps, pos0, n_h, hd, S);
}

// scores of the chunk's keys for this thread's 16-lane row: calls f(key, score) on lane 0 of the row for every key
template <class F>
__device__ __forceinline__ void chunk_scores(const int8_t* __restrict__ kq, const float* __restrict__ sk,
                                             const AttnScratch& S, int row, int kvh, int n_kv, int hd, int j0, int j1,
                                             F&& f) {
    const int l16 = threadIdx.x & 15, kslot = threadIdx.x >> 4, hw = hd / 4;
    const int* qw = reinterpret_cast<const int*>(S.qq + (size_t)row * hd);
    int q[AQW];
#pragma unroll
    for (int u = 0; u < AQW; u++) q[u] = l16 + 16 * u < hw ? qw[l16 + 16 * u] : 0;
    const float sq = S.sq[row];
    for (int jb = j0; jb < j1; jb += RT / 16) {          // uniform trip count: every row takes part in the DPP sums
        const int j = jb + kslot;
        int dot = 0;
        if (j < j1) {
            const int* kw = reinterpret_cast<const int*>(kq + ((size_t)j * n_kv + kvh) * hd);
#pragma unroll
            for (int u = 0; u < AQW; u++)
                if (l16 + 16 * u < hw) dot = __builtin_amdgcn_sdot4(q[u], kw[l16 + 16 * u], dot, false);
        }
        dot = sum16(dot);
        if (j < j1 && l16 == 0) f(j, ((float)dot * sq) * sk[(size_t)j * n_kv + kvh]);
    }
}

template <int CK>
__global__ void __launch_bounds__(RT) k_attn_max(const int8_t* __restrict__ kq, const float* __restrict__ sk, int pos0,
                                                 int n_h, int n_kv, int hd, AttnScratch S) {
    __shared__ float red[RT / 64];
    const int row = blockIdx.y, tok = row / n_h, h = row - tok * n_h, kvh = h / (n_h / n_kv);
    const int nkeys = pos0 + tok + 1, j0 = blockIdx.x * CK;
    if (j0 >= nkeys) return;                              // uniform: the whole workgroup leaves
    float mx = -__builtin_inff();
    chunk_scores(kq, sk, S, row, kvh, n_kv, hd, j0, min(j0 + CK, nkeys), [&](int, float sj) { mx = fmax_spec(mx, sj); });
    mx = wave_fmax(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < RT / 64; w++) mx = fmax_spec(mx, red[w]);
        atomicMax(S.mxo + row, f2ord(mx));
    }
}

template <int CK, bool FIN>
__global__ void __launch_bounds__(RT) k_attn_acc(const int8_t* __restrict__ kq, const float* __restrict__ sk,
                                                 const int16_t* __restrict__ vq, int pos0, int n_h, int n_kv, int hd,
                                                 AttnScratch S, const float* __restrict__ v_scale,
                                                 const float* __restrict__ qg, float* __restrict__ o) {
    __shared__ int pqs[CK];
    __shared__ long long dens[RT / 64];
    __shared__ unsigned last;
    const int row = blockIdx.y, tok = row / n_h, h = row - tok * n_h, kvh = h / (n_h / n_kv);
    const int nkeys = pos0 + tok + 1, j0 = blockIdx.x * CK;
    if (j0 >= nkeys) return;
    const int j1 = min(j0 + CK, nkeys);
    const float mx = ord2f(S.mxo[row]);
    long long den = 0;
    chunk_scores(kq, sk, S, row, kvh, n_kv, hd, j0, j1, [&](int j, float sj) {
        const int pq = (int)rint_(exp_f(sj - mx) * 16777216.0f);   // 0 .. 2^24
        pqs[j - j0] = pq;
        den += pq;
    });
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) den += __shfl_xor(den, off, 64);
    if ((threadIdx.x & 63) == 0) dens[threadIdx.x >> 6] = den;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < RT / 64; w++) den += dens[w];
        atomicAdd(reinterpret_cast<unsigned long long*>(S.den + row), (unsigned long long)den);
    }
    const int nc = j1 - j0;
    const int16_t* vb = vq + ((size_t)j0 * n_kv + kvh) * hd;
    const size_t vstride = (size_t)n_kv * hd;
    for (int i = threadIdx.x; i < hd; i += RT) {
        long long acc = 0;
#pragma unroll 16
        for (int jj = 0; jj < nc; jj++) acc += (long long)pqs[jj] * (long long)vb[jj * vstride + i];
        atomicAdd(reinterpret_cast<unsigned long long*>(S.num + (size_t)row * hd + i), (unsigned long long)acc);
    }
    if (!FIN) return;
    // the row's last chunk to arrive writes the output (its sums are complete once every chunk's adds are performed)
    wait_performed();
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(S.cnt + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)((nkeys + CK - 1) / CK - 1);
    __syncthreads();
    if (!last) return;
    const float fden = i64_to_f(__hip_atomic_load(S.den + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const float vs = v_scale[kvh];
    const float* gate = qg + (size_t)row * 2 * hd + hd;
    for (int i = threadIdx.x; i < hd; i += RT) {
        const long long nm = __hip_atomic_load(S.num + (size_t)row * hd + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        o[(size_t)row * hd + i] = ((i64_to_f(nm) / fden) * vs) * sigmoid_f(gate[i]);
    }
}


// ---- row kernels of a batch, one wave per row: the row's n <= 64 EPT values sit in registers, EPT consecutive per
// lane, so the spec's treesum of squares is each lane's aligned subtree, then lane pairs (DPP, two shuffles); leaves
// past n (to the wave's 64 EPT) are +0 and squares are >= +0, so the root equals the tree over the padded row.
template <int EPT>
__device__ __forceinline__ float wave_sumsq(const float* v) {
    float r[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) r[k] = v[k] * v[k];
#pragma unroll
    for (int w2 = EPT >> 1; w2 >= 1; w2 >>= 1)
#pragma unroll
        for (int k = 0; k < w2; k++) r[k] = r[2 * k] + r[2 * k + 1];
    float t = lane_tree_sum<16>(r[0]);
    t = t + __shfl_xor(t, 16, 64);
    return t + __shfl_xor(t, 32, 64);
}
// k_attn_prep with a wave per row for hd = 64 EPT (EPT = 1, 2, 4): the row in registers, EPT consecutive values
// per lane; the RMSNorm sum by lane subtrees and DPP (the spec's tree: hd is a power of two), rope's partner
// values (i +- half, half a multiple of EPT) by a lane shuffle, the absmax by DPP.  Same operations as
// attn_kv_row / attn_q_row.
template <int EPT>
__device__ __forceinline__ float wave_absmax0(const float* v) {
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < EPT; k++) am = fmax_spec(am, __builtin_fabsf(v[k]));
    return wave_fmax(am);
}
template <int EPT>
__device__ __forceinline__ void wave_norm_rope(float* v, const float* __restrict__ nw, float eps, const float* cs,
                                               const float* sn, int half, int lane) {
    constexpr int HD = 64 * EPT;
    const float inv = 1.0f / __builtin_sqrtf((wave_sumsq<EPT>(v) / (float)HD) + eps);   // spec/prim.rs:172-181
#pragma unroll
    for (int k = 0; k < EPT; k++) v[k] = (v[k] * inv) * nw[lane * EPT + k];
    const int sh = half / EPT;                                   // lanes between i and i + half
    const bool lo = lane * EPT < half, hi = lane * EPT >= half && lane * EPT < 2 * half;
    const int src = lo ? lane + sh : hi ? lane - sh : lane;
#pragma unroll
    for (int k = 0; k < EPT; k++) {                              // spec/layers.rs:5-13
        const float pv = __shfl(v[k], src, 64);
        const int i = lane * EPT + k;
        if (lo) v[k] = (v[k] * cs[i]) - (pv * sn[i]);
        else if (hi) v[k] = (v[k] * cs[i - half]) + (pv * sn[i - half]);
    }
}
template <int EPT>
__global__ void __launch_bounds__(256) k_attn_prep_w(const float* __restrict__ k_norm, const float* __restrict__ v_inv_scale,
                                                     int8_t* __restrict__ kq, float* __restrict__ sk, int16_t* __restrict__ vq,
                                                     const float* __restrict__ k, const float* __restrict__ v,
                                                     const float* __restrict__ q_norm, const float* __restrict__ qg,
                                                     const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
                                                     int half, float eps, int pos0, int n_kv, int n_h, int nkv, int nrows,
                                                     AttnScratch S) {
    constexpr int HD = 64 * EPT;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= nrows) return;                          // whole waves; no barrier follows
    float x[EPT];
    if (row < nkv) {
        const int tok = row / n_kv, h = row - tok * n_kv, pos = pos0 + tok;
        const size_t src = ((size_t)tok * n_kv + h) * HD;
#pragma unroll
        for (int e = 0; e < EPT; e++) x[e] = k[src + lane * EPT + e];
        wave_norm_rope<EPT>(x, k_norm, eps, rope_cos + (size_t)pos * half, rope_sin + (size_t)pos * half, half, lane);
        const float am = wave_absmax0<EPT>(x);
        const float sc = am == 0.0f ? 1.0f : am / 127.0f, inv = 1.0f / sc;          // spec/quant.rs:8-16
        const size_t dst = ((size_t)pos * n_kv + h) * HD;
#pragma unroll
        for (int e = 0; e < EPT; e++) kq[dst + lane * EPT + e] = (int8_t)clamp_i8(rint_(x[e] * inv));
        if (lane == 0) sk[(size_t)pos * n_kv + h] = sc;
        const float vi = v_inv_scale[h];
#pragma unroll
        for (int e = 0; e < EPT; e++) {                                              // spec/layers.rs:73-86
            const float r = rint_(v[src + lane * EPT + e] * vi);
            vq[dst + lane * EPT + e] = (int16_t)(r < -32767.0f ? -32767 : r > 32767.0f ? 32767 : __builtin_isnan(r) ? 0 : (int)r);
        }
        return;
    }
    const int qrow = row - nkv, tok = qrow / n_h, pos = pos0 + tok;
    const float* qr = qg + (size_t)qrow * 2 * HD;
#pragma unroll
    for (int e = 0; e < EPT; e++) x[e] = qr[lane * EPT + e];
    wave_norm_rope<EPT>(x, q_norm, eps, rope_cos + (size_t)pos * half, rope_sin + (size_t)pos * half, half, lane);
    const float qscale = 1.0f / __builtin_sqrtf((float)HD);
#pragma unroll
    for (int e = 0; e < EPT; e++) x[e] = x[e] * qscale;
    const float am = wave_absmax0<EPT>(x);
    const float sq = am == 0.0f ? 1.0f : am / 127.0f, inv = 1.0f / sq;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        S.qq[(size_t)qrow * HD + lane * EPT + e] = (int8_t)clamp_i8(rint_(x[e] * inv));
        S.num[(size_t)qrow * HD + lane * EPT + e] = 0;
    }
    if (lane == 0) {
        S.sq[qrow] = sq;
        S.mxo[qrow] = 0u;
        S.den[qrow] = 0;
        S.cnt[qrow] = 0u;
    }
}

// ---- a batch on the matrix cores (k_attn_mma): the same integers and fp32 operations as k_attn_max / k_attn_acc.
// Workgroup = (32 output dims, 16 tokens, up to 4 q heads of one kv head: a wave each); keys in chunks of 64 staged
// in LDS and shared by the heads.  Scores: v_mfma_i32_16x16x64_i8 of the int8 q rows by the int8 key rows (exact
// int32 dots), then (f32(dot) * sq) * sk.  Pass 1 folds the row maxima (order-free); pass 2 recomputes the scores,
// forms pq = rint(exp(s - mx) * 2^24) and the exact products with the int16 values as digit products on the matrix
// core: pq = sum_a 2^(7 a) p_a with unsigned 7-bit p_0..p_2 and p_3 <= 8, v = sum_b 2^(7 b) v_b with balanced
// 7-bit v_0, v_1 in [-64, 63] and v_2 in [-2, 2], so num = sum_{a,b} 2^(7 (a + b)) (P_a V_b) with every P_a V_b an
// exact int32 sum (|p_a v_b| <= 127 * 64, fewer than 2^18 keys).  P reaches the A-operand layout through a
// wave-private LDS tile; V's digits are staged transposed ([dim][key]) so a lane's 16 keys are contiguous.
typedef int v4i_t __attribute__((ext_vector_type(4)));
constexpr int AM_T = 16, AM_KC = 64, AM_D = 32;
template <int CTRL>
__device__ __forceinline__ long long dpp_ll(long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(v & 0xffffffffll), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((long long)hi << 32) | (unsigned int)lo;
}
template <int HD>
__global__ void __launch_bounds__(256) k_attn_mma(const int8_t* __restrict__ kq, const float* __restrict__ sk,
                                                  const int16_t* __restrict__ vq, int pos0, int M, int n_h, int n_kv,
                                                  AttnScratch S, const float* __restrict__ v_scale,
                                                  const float* __restrict__ qg, float* __restrict__ o) {
    constexpr int KS = HD / 64;                       // 64-deep k steps of a score
    __shared__ __attribute__((aligned(16))) int8_t kc[AM_KC * HD];
    __shared__ float skc[AM_KC];
    __shared__ __attribute__((aligned(16))) int8_t vt[3][AM_D][AM_KC];
    __shared__ int ps[4][AM_T][AM_KC];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rep = n_h / n_kv, hgroups = (rep + 3) / 4;
    const int kvh = blockIdx.z / hgroups, hg = blockIdx.z - kvh * hgroups;
    const int hl = hg * 4 + w, h = kvh * rep + hl;
    const bool active = hl < rep;
    const int t0 = blockIdx.y * AM_T, d0 = blockIdx.x * AM_D;
    const int nk = pos0 + min(M, t0 + AM_T);          // keys any row of the block sees
    const int c16 = lane & 15, q4 = lane >> 4;
    // A operands of the q rows: lane holds row c16, k bytes [64 s + 16 q4, + 16)
    v4i_t qa[KS];
    {
        const int t = t0 + c16;
        const int8_t* qr = S.qq + ((size_t)t * n_h + (active ? h : 0)) * HD;
#pragma unroll
        for (int s2 = 0; s2 < KS; s2++)
            qa[s2] = (active && t < M) ? *reinterpret_cast<const v4i_t*>(qr + 64 * s2 + 16 * q4) : v4i_t{0, 0, 0, 0};
    }
    // C layout rows of this lane: i = 4 q4 + r
    float sqr[4];
    int posr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int t = t0 + 4 * q4 + r;
        const bool ok = active && t < M;
        sqr[r] = ok ? S.sq[(size_t)t * n_h + h] : 0.0f;
        posr[r] = ok ? pos0 + t : -1;                  // keys 0 .. posr are seen; none for a padding row
    }
    auto stage_k = [&](int j0) __attribute__((always_inline)) {
        for (int e = tid; e < AM_KC * (HD / 16); e += 256) {
            const int j = e / (HD / 16), c = e - j * (HD / 16);
            v4i_t v = {0, 0, 0, 0};
            if (j0 + j < nk) v = *reinterpret_cast<const v4i_t*>(kq + ((size_t)(j0 + j) * n_kv + kvh) * HD + 16 * c);
            *reinterpret_cast<v4i_t*>(kc + j * HD + 16 * c) = v;
        }
        for (int j = tid; j < AM_KC; j += 256) skc[j] = j0 + j < nk ? sk[(size_t)(j0 + j) * n_kv + kvh] : 0.0f;
    };
    // the 16 x 16 score tile of key columns ct * 16 .. + 15 of the staged chunk
    auto scores = [&](int ct) __attribute__((always_inline)) {
        v4i_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int s2 = 0; s2 < KS; s2++) {
            const v4i_t b = *reinterpret_cast<const v4i_t*>(kc + (ct * 16 + c16) * HD + 64 * s2 + 16 * q4);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[s2], b, acc, 0, 0, 0);
        }
        return acc;
    };
    // pass 1: row maxima
    float mx[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    for (int j0 = 0; j0 < nk; j0 += AM_KC) {
        __syncthreads();
        stage_k(j0);
        __syncthreads();
        if (!active) continue;
#pragma unroll
        for (int ct = 0; ct < AM_KC / 16; ct++) {
            const v4i_t acc = scores(ct);
            const int j = j0 + ct * 16 + c16;
            const float skj = skc[ct * 16 + c16];
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (j <= posr[r]) mx[r] = fmax_spec(mx[r], ((float)acc[r] * sqr[r]) * skj);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {                     // over the 16 lanes of the row group (order-free)
        mx[r] = fmax_spec(mx[r], dpp_f<0xB1>(mx[r]));
        mx[r] = fmax_spec(mx[r], dpp_f<0x4E>(mx[r]));
        mx[r] = fmax_spec(mx[r], dpp_f<0x141>(mx[r]));
        mx[r] = fmax_spec(mx[r], dpp_f<0x140>(mx[r]));
    }
    // pass 2: weights, den and the digit products
    v4i_t cacc[4][3][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 3; b++)
#pragma unroll
            for (int dt = 0; dt < 2; dt++) cacc[a][b][dt] = v4i_t{0, 0, 0, 0};
    long long den[4] = {0, 0, 0, 0};
    for (int j0 = 0; j0 < nk; j0 += AM_KC) {
        __syncthreads();
        stage_k(j0);
        for (int e = tid; e < AM_KC * AM_D; e += 256) {
            const int j = e / AM_D, d = e - j * AM_D;
            const int v = j0 + j < nk ? (int)vq[((size_t)(j0 + j) * n_kv + kvh) * HD + d0 + d] : 0;
            const int v0 = ((v + 64) & 127) - 64, r1 = (v - v0) >> 7;
            const int v1 = ((r1 + 64) & 127) - 64, v2 = (r1 - v1) >> 7;
            vt[0][d][j] = (int8_t)v0;
            vt[1][d][j] = (int8_t)v1;
            vt[2][d][j] = (int8_t)v2;
        }
        __syncthreads();
        if (!active) continue;
#pragma unroll
        for (int ct = 0; ct < AM_KC / 16; ct++) {
            const v4i_t acc = scores(ct);
            const int j = j0 + ct * 16 + c16;
            const float skj = skc[ct * 16 + c16];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int pq = 0;
                if (j <= posr[r]) pq = (int)rint_(exp_f(((float)acc[r] * sqr[r]) * skj - mx[r]) * 16777216.0f);
                den[r] += pq;
                ps[w][4 * q4 + r][ct * 16 + c16] = pq;
            }
        }
        // A operands of the weight digits: lane holds row c16, keys 16 q4 .. + 15 (the wave's own tile; its lanes'
        // writes above are complete before the reads: LDS operations of a wave are performed in order)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        v4i_t pa[4];
        {
            const int* pr = &ps[w][c16][16 * q4];
            uint32_t wd[4][4];
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                uint32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t pq = (uint32_t)pr[4 * k4 + k];
                    b0 |= (pq & 127u) << (8 * k);
                    b1 |= ((pq >> 7) & 127u) << (8 * k);
                    b2 |= ((pq >> 14) & 127u) << (8 * k);
                    b3 |= (pq >> 21) << (8 * k);
                }
                wd[0][k4] = b0; wd[1][k4] = b1; wd[2][k4] = b2; wd[3][k4] = b3;
            }
#pragma unroll
            for (int a = 0; a < 4; a++) pa[a] = v4i_t{(int)wd[a][0], (int)wd[a][1], (int)wd[a][2], (int)wd[a][3]};
        }
#pragma unroll
        for (int b = 0; b < 3; b++)
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                const v4i_t vb = *reinterpret_cast<const v4i_t*>(&vt[b][dt * 16 + c16][16 * q4]);
#pragma unroll
                for (int a = 0; a < 4; a++) cacc[a][b][dt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[a], vb, cacc[a][b][dt], 0, 0, 0);
            }
    }
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {                     // den over the row group's 16 lanes (exact)
        den[r] += dpp_ll<0xB1>(den[r]);
        den[r] += dpp_ll<0x4E>(den[r]);
        den[r] += dpp_ll<0x141>(den[r]);
        den[r] += dpp_ll<0x140>(den[r]);
    }
    const float vs = v_scale[kvh];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int t = t0 + 4 * q4 + r;
        if (t >= M) continue;
        const float fden = i64_to_f(den[r]);
        const float* gate = qg + ((size_t)t * n_h + h) * 2 * HD + HD;
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
            long long num = 0;
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 3; b++) num += (long long)cacc[a][b][dt][r] << (7 * (a + b));
            const int d = d0 + dt * 16 + c16;
            o[((size_t)t * n_h + h) * HD + d] = ((i64_to_f(num) / fden) * vs) * sigmoid_f(gate[d]);
        }
    }
}

// the output of a batch's rows once every chunk has added its sums (k_attn_acc<CK, false>)
__global__ void __launch_bounds__(RT) k_attn_fin(const float* __restrict__ v_scale, const float* __restrict__ qg,
                                                 int n_h, int n_kv, int hd, AttnScratch S, float* __restrict__ o) {
    const int row = blockIdx.x, h = row % n_h, kvh = h / (n_h / n_kv);
    const float fden = i64_to_f(S.den[row]), vs = v_scale[kvh];
    const float* gate = qg + (size_t)row * 2 * hd + hd;
    for (int i = threadIdx.x; i < hd; i += RT)
        o[(size_t)row * hd + i] = ((i64_to_f(S.num[(size_t)row * hd + i]) / fden) * vs) * sigmoid_f(gate[i]);
}

// ------------------------------------------------------------------ Gated DeltaNet (cpu.rs:287-383)
// conv + silu of every token's channels at once: window (t - 3, t - 2, t - 1, t), rows before the call from
// conv_state[3][cd] (oldest first).  grid (M, ceil(cd / RT)).
__global__ void __launch_bounds__(RT) k_gdn_conv(const float* __restrict__ conv_w, const float* __restrict__ conv_state,
                                                 const float* __restrict__ qkv, int cd, float* __restrict__ y) {
    const int tok = blockIdx.x, c = blockIdx.y * RT + threadIdx.x;
    if (c >= cd) return;
    float win[4];
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int u = tok - 3 + r;
        win[r] = u >= 0 ? qkv[(size_t)u * cd + c] : conv_state[(size_t)(3 + u) * cd + c];
    }
    win[3] = qkv[(size_t)tok * cd + c];
    const float* w = conv_w + (size_t)c * 4;
    float acc = (w[0] * win[0]) + (w[1] * win[1]);   // spec/layers.rs:132-138
    acc = acc + (w[2] * win[2]);
    acc = acc + (w[3] * win[3]);
    y[(size_t)tok * cd + c] = silu_f(acc);
}

// the conv window after the call: the last three inputs (rows of the old window when M < 3); one thread per
// channel reads its three old rows before writing
__global__ void __launch_bounds__(RT) k_gdn_conv_state(float* __restrict__ conv_state, const float* __restrict__ qkv,
                                                       int M, int cd) {
    const int c = blockIdx.x * RT + threadIdx.x;
    if (c >= cd) return;
    const float o0 = conv_state[c], o1 = conv_state[(size_t)cd + c], o2 = conv_state[2 * (size_t)cd + c];
    float nw[3];
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int u = M - 3 + r;                   // input index of new row r; old row u + 3 when u < 0
        nw[r] = u >= 0 ? qkv[(size_t)u * cd + c] : (u == -3 ? o0 : u == -2 ? o1 : o2);
    }
#pragma unroll
    for (int r = 0; r < 3; r++) conv_state[(size_t)r * cd + c] = nw[r];
}

// one workgroup per (token, k head): q = l2norm(conv q) * QSCALE, k = l2norm(conv k) (spec/prim.rs:183-190), and
// for the head's rep v heads beta = sigmoid(b), decay = exp(-(A softplus(a + dt_bias))) (spec/layers.rs:140-143)
__global__ void __launch_bounds__(RT) k_gdn_prep(const float* __restrict__ y, const float* __restrict__ A,
                                                 const float* __restrict__ dt_bias, const float* __restrict__ a,
                                                 const float* __restrict__ b, float eps, int n_k, int n_v, int dk, int cd,
                                                 float* __restrict__ qb, float* __restrict__ kb, float* __restrict__ bd) {
    extern __shared__ float lds[];
    float* x = lds;
    float* s = x + dk;
    float* t = s + p2(dk);
    const int tok = blockIdx.x / n_k, kh = blockIdx.x - tok * n_k, rep = n_v / n_k;
    const float qscale = __uint_as_float(0x3DB504F3u);            // spec/layers.rs:146
    for (int part = 0; part < 2; part++) {
        const float* src = y + (size_t)tok * cd + (size_t)part * n_k * dk + (size_t)kh * dk;
        for (int i = threadIdx.x; i < dk; i += RT) x[i] = src[i];
        __syncthreads();
        const float inv = 1.0f / __builtin_sqrtf(block_treesum<true>(x, dk, s, t) + eps);
        float* dst = (part == 0 ? qb : kb) + ((size_t)tok * n_k + kh) * dk;
        for (int i = threadIdx.x; i < dk; i += RT) dst[i] = part == 0 ? (x[i] * inv) * qscale : x[i] * inv;
        __syncthreads();
    }
    for (int i = threadIdx.x; i < rep; i += RT) {
        const int hv = kh * rep + i;
        const size_t ti = (size_t)tok * n_v + hv;
        bd[2 * ti] = sigmoid_f(b[ti]);
        bd[2 * ti + 1] = exp_f(-(A[hv] * softplus_f(a[ti] + dt_bias[hv])));
    }
}

// ---- row kernels of a batch, one wave per row (wave_sumsq above)
// k_gdn_prep with a wave per (token, k head): l2norm of q (times QSCALE) and of k, beta and decay of the rep v heads
template <int EPT>
__global__ void __launch_bounds__(256) k_gdn_prep_w(const float* __restrict__ y, const float* __restrict__ A,
                                                    const float* __restrict__ dt_bias, const float* __restrict__ a,
                                                    const float* __restrict__ b, float eps, int rows, int n_k, int n_v,
                                                    int dk, int cd, float* __restrict__ qb, float* __restrict__ kb,
                                                    float* __restrict__ bd) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;                           // whole waves: no barrier follows
    const int tok = row / n_k, kh = row - tok * n_k, rep = n_v / n_k;
    const float qscale = __uint_as_float(0x3DB504F3u);            // spec/layers.rs:146
    for (int part = 0; part < 2; part++) {
        const float* src = y + (size_t)tok * cd + (size_t)part * n_k * dk + (size_t)kh * dk;
        float v[EPT];
#pragma unroll
        for (int k = 0; k < EPT; k++) v[k] = lane * EPT + k < dk ? src[lane * EPT + k] : 0.0f;
        const float inv = 1.0f / __builtin_sqrtf(wave_sumsq<EPT>(v) + eps);     // spec/prim.rs:183-190
        float* dst = (part == 0 ? qb : kb) + ((size_t)tok * n_k + kh) * dk;
#pragma unroll
        for (int k = 0; k < EPT; k++)
            if (lane * EPT + k < dk) dst[lane * EPT + k] = part == 0 ? (v[k] * inv) * qscale : v[k] * inv;
    }
    for (int i = lane; i < rep; i += 64) {
        const int hv = kh * rep + i;
        const size_t ti = (size_t)tok * n_v + hv;
        bd[2 * ti] = sigmoid_f(b[ti]);
        bd[2 * ti + 1] = exp_f(-(A[hv] * softplus_f(a[ti] + dt_bias[hv])));
    }
}
// k_gdn_out with a wave per (token, v head): on = rmsnorm(o, norm) * silu(z)
template <int EPT>
__global__ void __launch_bounds__(256) k_gdn_out_w(const float* __restrict__ ob, const float* __restrict__ norm,
                                                   const float* __restrict__ z, float eps, int rows, int dv,
                                                   float* __restrict__ on) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = (size_t)row * dv;
    float v[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) v[k] = lane * EPT + k < dv ? ob[base + lane * EPT + k] : 0.0f;
    const float inv = 1.0f / __builtin_sqrtf((wave_sumsq<EPT>(v) / (float)dv) + eps);   // spec/prim.rs:172-181
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = lane * EPT + k;
        if (i < dv) on[base + i] = ((v[k] * inv) * norm[i]) * silu_f(z[base + i]);
    }
}

// balanced tree over the RB values of v (adjacent pairs level by level): the aligned subtree of the spec's tree
template <int RB>
__device__ __forceinline__ float reg_tree(float* v) {
#pragma unroll
    for (int w = RB >> 1; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; i++) v[i] = v[2 * i] + v[2 * i + 1];
    return v[0];
}

// The recurrence of one v head over the M tokens in order (spec/layers.rs:90-130).  Column j of S[h] (dk rows)
// is split over R adjacent lanes, lane r holding rows RB r .. RB r + RB - 1 (dk = R RB, a power of two), so a
// column's treesum is the lane's subtree, then log2(R) DPP levels that add the aligned subtrees in tree order
// (lane_tree_sum).  The columns evolve independently, so a head's dv columns are spread over blocks of
// CW = GT / R columns (grid y), one workgroup of GT threads each.  Tokens come in chunks of TC: a chunk's k, q (of
// the head's k head), its columns' v, beta and decay are loaded into registers while the previous chunk is
// computed from LDS, then written to the other of two LDS buffers (one barrier per chunk).  Inside a chunk the
// next token's operands are read from LDS before the current token is computed.
constexpr int GT = 256, GTC = 32;
template <int RB, int R>
__global__ void __launch_bounds__(GT) k_gdn_rec(float* __restrict__ S, const float* __restrict__ qb,
                                                const float* __restrict__ kb, const float* __restrict__ y,
                                                const float* __restrict__ bd, int M, int n_k, int n_v, int dv, int cd,
                                                float* __restrict__ ob, const float* __restrict__ norm,
                                                const float* __restrict__ z, float eps, float* __restrict__ on,
                                                unsigned* __restrict__ cnt) {
    constexpr int DK = R * RB, TC = GTC, CW = GT / R;
    __shared__ unsigned last;
    constexpr int LK = (TC * DK + GT - 1) / GT, LV = (TC * CW + GT - 1) / GT;
    constexpr int BUF = 2 * TC * DK + TC * CW + 2 * TC;           // floats of one buffer: k, q, v, (beta, decay)
    extern __shared__ float sm[];
    const int h = blockIdx.x, kh = h / (n_v / n_k), j0 = blockIdx.y * CW, tid = threadIdx.x;
    const int jl = tid / R, r = tid % R, j = j0 + jl;
    const bool live = j < dv;
    float col[RB];
    float* Sh = S + (size_t)h * DK * dv;
#pragma unroll
    for (int i = 0; i < RB; i++) col[i] = live ? Sh[(size_t)(r * RB + i) * dv + j] : 0.0f;
    const size_t vbase = (size_t)2 * n_k * DK + (size_t)h * dv;      // v of head h inside a token's conv outputs
    float rk[LK], rq[LK], rv[LV], rb = 0.0f;
    auto load = [&](int c0) __attribute__((always_inline)) {
        const int nt = min(TC, M - c0);
#pragma unroll
        for (int u = 0; u < LK; u++) {
            const int e = tid + u * GT, tt = e / DK, i = e - tt * DK;
            const size_t src = ((size_t)(c0 + tt) * n_k + kh) * DK + i;
            rk[u] = e < nt * DK ? kb[src] : 0.0f;
            rq[u] = e < nt * DK ? qb[src] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < LV; u++) {
            const int e = tid + u * GT, tt = e / CW, jj = e - tt * CW;
            rv[u] = e < nt * CW && j0 + jj < dv ? y[(size_t)(c0 + tt) * cd + vbase + j0 + jj] : 0.0f;
        }
        if (tid < 2 * nt) rb = bd[2 * ((size_t)(c0 + tid / 2) * n_v + h) + (tid & 1)];
    };
    auto store = [&](float* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < LK; u++) {
            const int e = tid + u * GT;
            if (e < TC * DK) { buf[e] = rk[u]; buf[TC * DK + e] = rq[u]; }
        }
#pragma unroll
        for (int u = 0; u < LV; u++) {
            const int e = tid + u * GT;
            if (e < TC * CW) buf[2 * TC * DK + e] = rv[u];
        }
        if (tid < 2 * TC) buf[2 * TC * DK + TC * CW + tid] = rb;
    };
    load(0);
    store(sm);
    __syncthreads();
    int cur = 0;
    for (int c0 = 0; c0 < M; c0 += TC) {
        const int nt = min(TC, M - c0);
        const bool more = c0 + TC < M;
        if (more) load(c0 + TC);
        const float* ks = sm + cur * BUF;
        const float* qs = ks + TC * DK;
        const float* vs = qs + TC * DK;
        const float* bt = vs + TC * CW;
        float kc[RB], qc[RB], beta, decay, vj;
        auto fetch = [&](int tt, float* kd, float* qd, float& be, float& de, float& vv) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < RB; i++) { kd[i] = ks[tt * DK + r * RB + i]; qd[i] = qs[tt * DK + r * RB + i]; }
            be = bt[2 * tt];
            de = bt[2 * tt + 1];
            vv = vs[tt * CW + jl];
        };
        fetch(0, kc, qc, beta, decay, vj);
        for (int tt = 0; tt < nt; tt++) {
            float kn[RB], qn[RB], bn, dn, vn;
            fetch(min(tt + 1, nt - 1), kn, qn, bn, dn, vn);
            float p[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) col[i] = col[i] * decay;
#pragma unroll
            for (int i = 0; i < RB; i++) p[i] = col[i] * kc[i];
            const float kv = lane_tree_sum<R>(reg_tree<RB>(p));
            const float delta = (vj - kv) * beta;
#pragma unroll
            for (int i = 0; i < RB; i++) col[i] = col[i] + (kc[i] * delta);
#pragma unroll
            for (int i = 0; i < RB; i++) p[i] = col[i] * qc[i];
            const float oj = lane_tree_sum<R>(reg_tree<RB>(p));
            if (live && r == 0) {
                float* dst = ob + ((size_t)(c0 + tt) * n_v + h) * dv + j;
                if (cnt) __hip_atomic_store(dst, oj, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else *dst = oj;
            }
#pragma unroll
            for (int i = 0; i < RB; i++) { kc[i] = kn[i]; qc[i] = qn[i]; }
            beta = bn;
            decay = dn;
            vj = vn;
        }
        if (more) store(sm + (cur ^ 1) * BUF);
        __syncthreads();
        cur ^= 1;
    }
    if (live) {
#pragma unroll
        for (int i = 0; i < RB; i++) Sh[(size_t)(r * RB + i) * dv + j] = col[i];
    }
    if (!cnt) return;
    // one token (cnt != NULL): the head's last column block to count itself runs the gated norm (k_gdn_out) on the
    // head's output, which every block stored with agent-scope stores that have been performed
    wait_performed();
    __syncthreads();
    if (tid == 0) last = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.y - 1;
    __syncthreads();
    if (!last) return;
    float* x = sm;
    float* s2 = x + dv;
    float* t2 = s2 + p2(dv);
    for (int i = tid; i < dv; i += GT) x[i] = __hip_atomic_load(ob + (size_t)h * dv + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    block_rmsnorm(x, dv, norm, eps, s2, t2);
    for (int i = tid; i < dv; i += GT) on[(size_t)h * dv + i] = x[i] * silu_f(z[(size_t)h * dv + i]);
}

// gated norm: on = rmsnorm(o, norm) * silu(z) per (token, v head)
__global__ void __launch_bounds__(RT) k_gdn_out(const float* __restrict__ ob, const float* __restrict__ norm,
                                                const float* __restrict__ z, float eps, int dv, float* __restrict__ on) {
    extern __shared__ float lds[];
    float* x = lds;
    float* s = x + dv;
    float* t = s + p2(dv);
    const size_t base = (size_t)blockIdx.x * dv;
    for (int i = threadIdx.x; i < dv; i += RT) x[i] = ob[base + i];
    __syncthreads();
    block_rmsnorm(x, dv, norm, eps, s, t);
    for (int i = threadIdx.x; i < dv; i += RT) on[base + i] = x[i] * silu_f(z[base + i]);
}

// ---- one decode token (M = 1): the input stage in one launch instead of three
// k_gdn_in1: one workgroup per k head: conv + silu of its q and k channels and of its rep v heads' v channels, the
// conv window update of those channels (each channel belongs to one workgroup, so its thread reads the old rows
// before writing the new ones), l2norm of q (times QSCALE) and k, and beta / decay of the rep v heads.  The same
// operations, in the same order, as k_gdn_conv, k_gdn_conv_state and k_gdn_prep.
__global__ void __launch_bounds__(RT) k_gdn_in1(const float* __restrict__ conv_w, float* __restrict__ conv_state,
                                                const float* __restrict__ qkv, const float* __restrict__ A,
                                                const float* __restrict__ dt_bias, const float* __restrict__ a,
                                                const float* __restrict__ b, float eps, int n_k, int n_v, int dk, int dv,
                                                int cd, float* __restrict__ y, float* __restrict__ qb,
                                                float* __restrict__ kb, float* __restrict__ bd, unsigned* __restrict__ cnt,
                                                det_qlinear ab, const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                const uint16_t* __restrict__ mx) {
    extern __shared__ float lds[];
    const int p = p2(dk);
    float* x = lds;                  // conv q [dk], then conv k [dk]
    float* s = x + 2 * dk;
    float* t = s + p;
    const int kh = blockIdx.x, rep = n_v / n_k, nch = 2 * dk + rep * dv;
    for (int e = threadIdx.x; e < nch; e += RT) {
        const int c = e < dk ? kh * dk + e
                    : e < 2 * dk ? n_k * dk + kh * dk + (e - dk)
                    : 2 * n_k * dk + kh * rep * dv + (e - 2 * dk);
        const float o0 = conv_state[c], o1 = conv_state[(size_t)cd + c], o2 = conv_state[2 * (size_t)cd + c];
        const float in = qkv[c];
        const float* w = conv_w + (size_t)c * 4;
        float acc = (w[0] * o0) + (w[1] * o1);       // spec/layers.rs:132-138
        acc = acc + (w[2] * o2);
        acc = acc + (w[3] * in);
        const float v = silu_f(acc);
        if (e < 2 * dk) x[e] = v;
        else y[c] = v;
        conv_state[c] = o1;
        conv_state[(size_t)cd + c] = o2;
        conv_state[2 * (size_t)cd + c] = in;
    }
    __syncthreads();
    const float qscale = __uint_as_float(0x3DB504F3u);            // spec/layers.rs:146
    for (int part = 0; part < 2; part++) {
        const float inv = 1.0f / __builtin_sqrtf(block_treesum<true>(x + part * dk, dk, s, t) + eps);
        float* dst = (part == 0 ? qb : kb) + (size_t)kh * dk;
        for (int i = threadIdx.x; i < dk; i += RT) dst[i] = part == 0 ? (x[i] * inv) * qscale : x[dk + i] * inv;
    }
    __shared__ float abv[2 * 64];
    if (ab.wq) {
        // the a|b projection of the token (a W8 linear of 2 n_v rows: a heads, then b heads), the same integers and
        // epilogue as det_gemm_ex: wave w takes the rows w, w + 4, ... of this k head's 2 rep; lane l the 16-code
        // chunks l, l + 64, ... of the row; each chunk's v_dot4 sum is scaled by its group's m * mx into int64
        const int G = ab.K / GROUP, lane = threadIdx.x & 63;
        for (int e = threadIdx.x >> 6; e < 2 * rep; e += RT / 64) {
            const int R = e < rep ? kh * rep + e : n_v + kh * rep + (e - rep), tile = R / 64, rr = R % 64;
            long long acc = 0;
            for (int ch = lane; ch < G * 8; ch += 64) {
                const int g = ch >> 3;
                const size_t tg = (size_t)tile * G + g;
                const int4 w4 = *reinterpret_cast<const int4*>(ab.wq + ((tg * 8 + (ch & 7)) * 64 + rr) * 16);
                const int4 x4 = *reinterpret_cast<const int4*>(xq + (size_t)ch * 16);
                int p = __builtin_amdgcn_sdot4(w4.x, x4.x, 0, false);
                p = __builtin_amdgcn_sdot4(w4.y, x4.y, p, false);
                p = __builtin_amdgcn_sdot4(w4.z, x4.z, p, false);
                p = __builtin_amdgcn_sdot4(w4.w, x4.w, p, false);
                mac_s32_u32(acc, p, (uint32_t)ab.m[tg * 64 + rr] * (mx ? (uint32_t)mx[g] : 1u));
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
            if (lane == 0) abv[e] = (i64_to_f(acc) * ab.c[R]) * sx[0];
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < rep; i += RT) {
        const int hv = kh * rep + i;
        cnt[hv] = 0u;                                 // the fused gated norm's arrival counter of v head hv
        const float av = ab.wq ? abv[i] : a[hv], bv = ab.wq ? abv[rep + i] : b[hv];
        bd[2 * hv] = sigmoid_f(bv);
        bd[2 * hv + 1] = exp_f(-(A[hv] * softplus_f(av + dt_bias[hv])));
    }
}

// ------------------------------------------------------------------ argmax (spec/sample.rs:6-14)
// The spec scans i = 1 .. V-1 and moves to i when l[i] > l[best]: the result is 0 when l[0] is NaN, else the lowest
// index of the largest non-NaN value, with -0 equal to +0.  That is the maximum of the 64-bit keys
// (order image of l[i] with -0 read as +0) << 32 | ~i, NaN keyed 0, so the rows' slices reduce in any order:
// k_argmax_part takes the max over a slice of AMX_SLICE values and merges it into acc[row] by atomicMax;
// k_argmax_fin decodes the key and leaves acc[row] at 0 for the next call.
constexpr int AMX_SLICE = 2048;
__device__ __forceinline__ unsigned long long amx_key(float v, int i) {
    if (__builtin_isnan(v)) return 0ull;
    const unsigned u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(~(unsigned)i);
}
__global__ void __launch_bounds__(RT) k_argmax_part(const float* __restrict__ logits, int V,
                                                    unsigned long long* __restrict__ acc) {
    __shared__ unsigned long long red[RT / 64];
    const float* l = logits + (size_t)blockIdx.y * V;
    const int i0 = blockIdx.x * AMX_SLICE + threadIdx.x;
    constexpr int PER = AMX_SLICE / RT;
    float v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) v[u] = i0 + u * RT < V ? l[i0 + u * RT] : __builtin_nanf("");
    unsigned long long k = 0;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const unsigned long long c = amx_key(v[u], i0 + u * RT);
        k = c > k ? c : k;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long c = __shfl_xor(k, off, 64);
        k = c > k ? c : k;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < RT / 64; w++) k = red[w] > k ? red[w] : k;
        if (k) atomicMax(acc + blockIdx.y, k);
    }
}
__global__ void k_argmax_fin(const float* __restrict__ logits, int M, int V, unsigned long long* __restrict__ acc,
                             int* __restrict__ out) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= M) return;
    const unsigned long long k = acc[row];
    acc[row] = 0ull;
    out[row] = (__builtin_isnan(logits[(size_t)row * V]) || k == 0ull) ? 0 : (int)~(unsigned)(k & 0xffffffffull);
}

// row accumulators of the argmax, zero between calls; library-owned, grown on demand
unsigned long long* g_amx = nullptr;
size_t g_amx_cap = 0;

size_t gdn_scratch_floats(int M, int n_k, int n_v, int dk, int dv) {
    const size_t cd = 2 * (size_t)n_k * dk + (size_t)n_v * dv;
    return (size_t)M * cd + 2 * (size_t)M * n_k * dk + 2 * (size_t)M * n_v + (size_t)M * n_v * dv + (size_t)n_v;
}

} // namespace

extern "C" {

size_t det_attn_scratch_bytes(int M, int n_h, int hd) {
    return attn_layout(nullptr, M < 1 ? 1 : M, n_h < 1 ? 1 : n_h, hd < 4 ? 4 : hd).bytes;
}

void det_attention(const det_attn_layer* L, const det_kv_cache* kv, const float* qg, const float* k, const float* v,
                   const float* rope_cos, const float* rope_sin, int rot, float eps, int M, int pos0, int n_h, int n_kv,
                   int hd, float* o, void* scratch, hipStream_t st) {
    if (M < 1) return;
    if (hd < 4 || hd > 4 * 16 * AQW || hd % 4) DET_FAIL("det_attention: head_dim %d (multiple of 4, at most 1024)", hd);
    if (n_kv < 1 || n_h < n_kv || n_h % n_kv) DET_FAIL("det_attention: %d heads over %d kv heads", n_h, n_kv);
    if (rot < 0 || rot > hd || rot % 2) DET_FAIL("det_attention: rot %d for head_dim %d", rot, hd);
    if (pos0 < 0 || (long long)pos0 + M > kv->capacity) DET_FAIL("det_attention: positions %d..%d exceed the cache of %d", pos0, pos0 + M - 1, kv->capacity);
    if (!scratch) DET_FAIL("det_attention: scratch of det_attn_scratch_bytes(M, n_h, hd) is required");
    if ((long long)M * n_h > 65535) DET_FAIL("det_attention: %d tokens x %d heads exceed the grid", M, n_h);
    int p = 1;
    while (p < hd) p <<= 1;
    const size_t lds_row = ((size_t)hd + p + p / 2) * 4;
    const AttnScratch S = attn_layout(scratch, M, n_h, hd);
    const int nrows = M * (n_kv + n_h), half = rot / 2;
    const int ept = hd == 256 ? 4 : hd == 128 ? 2 : hd == 64 ? 1 : 0;
    if (ept && half % ept == 0) {
        if (ept == 4) k_attn_prep_w<4><<<(nrows + 3) / 4, 256, 0, st>>>(L->k_norm, L->v_inv_scale, kv->kq, kv->sk, kv->vq, k, v, L->q_norm, qg,
                                                                       rope_cos, rope_sin, half, eps, pos0, n_kv, n_h, M * n_kv, nrows, S);
        else if (ept == 2) k_attn_prep_w<2><<<(nrows + 3) / 4, 256, 0, st>>>(L->k_norm, L->v_inv_scale, kv->kq, kv->sk, kv->vq, k, v, L->q_norm, qg,
                                                                            rope_cos, rope_sin, half, eps, pos0, n_kv, n_h, M * n_kv, nrows, S);
        else k_attn_prep_w<1><<<(nrows + 3) / 4, 256, 0, st>>>(L->k_norm, L->v_inv_scale, kv->kq, kv->sk, kv->vq, k, v, L->q_norm, qg,
                                                              rope_cos, rope_sin, half, eps, pos0, n_kv, n_h, M * n_kv, nrows, S);
    } else
    k_attn_prep<<<M * (n_kv + n_h), RT, lds_row, st>>>(L->k_norm, L->v_inv_scale, kv->kq, kv->sk, kv->vq, k, v, L->q_norm, qg,
                                                      rope_cos, rope_sin, rot / 2, eps, pos0, n_kv, n_h, hd, M * n_kv, S);
    DET_CHECK(hipGetLastError());
    // chunks of 32 keys for a few tokens (a decode step: many workgroups per head), 256 for a batch
    const int nkeys = pos0 + M;
    if (M <= 4) {
        const dim3 grid((nkeys + 31) / 32, M * n_h);
        k_attn_max<32><<<grid, RT, 0, st>>>(kv->kq, kv->sk, pos0, n_h, n_kv, hd, S);
        DET_CHECK(hipGetLastError());
        k_attn_acc<32, true><<<grid, RT, 0, st>>>(kv->kq, kv->sk, kv->vq, pos0, n_h, n_kv, hd, S, L->v_scale, qg, o);
    } else if (hd == 256 && (long long)nkeys < (1 << 18)) {
        // a batch: the matrix-core path (workgroups of 32 dims x 16 tokens x up to 4 heads of a kv head)
        const int rep = n_h / n_kv;
        const dim3 grid(hd / AM_D, (M + AM_T - 1) / AM_T, n_kv * ((rep + 3) / 4));
        k_attn_mma<256><<<grid, 256, 0, st>>>(kv->kq, kv->sk, kv->vq, pos0, M, n_h, n_kv, S, L->v_scale, qg, o);
    } else if (hd == 128 && (long long)nkeys < (1 << 18)) {
        const int rep = n_h / n_kv;
        const dim3 grid(hd / AM_D, (M + AM_T - 1) / AM_T, n_kv * ((rep + 3) / 4));
        k_attn_mma<128><<<grid, 256, 0, st>>>(kv->kq, kv->sk, kv->vq, pos0, M, n_h, n_kv, S, L->v_scale, qg, o);
    } else if (hd == 64 && (long long)nkeys < (1 << 18)) {
        const int rep = n_h / n_kv;
        const dim3 grid(hd / AM_D, (M + AM_T - 1) / AM_T, n_kv * ((rep + 3) / 4));
        k_attn_mma<64><<<grid, 256, 0, st>>>(kv->kq, kv->sk, kv->vq, pos0, M, n_h, n_kv, S, L->v_scale, qg, o);
    } else {
        const dim3 grid((nkeys + 255) / 256, M * n_h);
        k_attn_max<256><<<grid, RT, 0, st>>>(kv->kq, kv->sk, pos0, n_h, n_kv, hd, S);
        DET_CHECK(hipGetLastError());
        k_attn_acc<256, false><<<grid, RT, 0, st>>>(kv->kq, kv->sk, kv->vq, pos0, n_h, n_kv, hd, S, L->v_scale, qg, o);
        DET_CHECK(hipGetLastError());
        k_attn_fin<<<M * n_h, RT, 0, st>>>(L->v_scale, qg, n_h, n_kv, hd, S, o);
    }
    DET_CHECK(hipGetLastError());
}

size_t det_gdn_scratch_bytes(int M, int n_k, int n_v, int dk, int dv) {
    return gdn_scratch_floats(M < 1 ? 1 : M, n_k, n_v, dk, dv) * sizeof(float);
}

void det_gdn(const det_gdn_layer* L, det_gdn_state* S, const float* qkv, const float* z, const float* a, const float* b,
             float eps, int M, int n_k, int n_v, int dk, int dv, float* on, void* scratch, hipStream_t st) {
    det::gdn_run(L, S, qkv, z, a, b, nullptr, nullptr, nullptr, nullptr, eps, M, n_k, n_v, dk, dv, on, scratch, st);
}

} // extern "C"

namespace det {

void gdn_run(const det_gdn_layer* L, det_gdn_state* S, const float* qkv, const float* z, const float* a, const float* b,
             const det_qlinear* ab, const int8_t* xq, const float* sx, const uint16_t* mx, float eps, int M, int n_k,
             int n_v, int dk, int dv, float* on, void* scratch, hipStream_t st) {
    if (M < 1) return;
    if (n_k < 1 || n_v < n_k || n_v % n_k) DET_FAIL("det_gdn: %d v heads over %d k heads", n_v, n_k);
    if (dk < 4 || dk > 128 || (dk & (dk - 1))) DET_FAIL("det_gdn: dk %d (a power of two, 4 .. 128)", dk);
    if (dv < 1 || dv > 256) DET_FAIL("det_gdn: dv %d (at most 256)", dv);
    if (!scratch) DET_FAIL("det_gdn: scratch of det_gdn_scratch_bytes() is required");
    if (ab && (M != 1 || ab->bits != 8 || ab->N != 2 * n_v || n_v / n_k > 64 || !xq || !sx))
        DET_FAIL("det_gdn: the fused a|b projection needs one token, a W8 linear of 2 n_v rows and rep <= 64");
    const int cd = 2 * n_k * dk + n_v * dv;
    float* y = static_cast<float*>(scratch);
    float* qb = y + (size_t)M * cd;
    float* kb = qb + (size_t)M * n_k * dk;
    float* bd = kb + (size_t)M * n_k * dk;
    float* ob = bd + 2 * (size_t)M * n_v;
    unsigned* cnt = M == 1 ? reinterpret_cast<unsigned*>(ob + (size_t)M * n_v * dv) : nullptr;   // [n_v]
    if (M == 1) {
        // one decode token: conv, window update and prep in one launch
        int p = 1;
        while (p < dk) p <<= 1;
        k_gdn_in1<<<n_k, RT, ((size_t)2 * dk + p + p / 2) * 4, st>>>(L->conv, S->conv_state, qkv, L->A, L->dt_bias, a, b,
                                                                    eps, n_k, n_v, dk, dv, cd, y, qb, kb, bd, cnt,
                                                                    ab ? *ab : det_qlinear{}, xq, sx, mx);
        DET_CHECK(hipGetLastError());
    } else {
        k_gdn_conv<<<dim3(M, (cd + RT - 1) / RT), RT, 0, st>>>(L->conv, S->conv_state, qkv, cd, y);
        DET_CHECK(hipGetLastError());
        k_gdn_conv_state<<<(cd + RT - 1) / RT, RT, 0, st>>>(S->conv_state, qkv, M, cd);
        DET_CHECK(hipGetLastError());
        int p = 1;
        while (p < dk) p <<= 1;
        const int rows = M * n_k, wg = (rows + 3) / 4;
        (void)p;
        if (dk <= 64) k_gdn_prep_w<1><<<wg, 256, 0, st>>>(y, L->A, L->dt_bias, a, b, eps, rows, n_k, n_v, dk, cd, qb, kb, bd);
        else k_gdn_prep_w<2><<<wg, 256, 0, st>>>(y, L->A, L->dt_bias, a, b, eps, rows, n_k, n_v, dk, cd, qb, kb, bd);
        DET_CHECK(hipGetLastError());
    }
    // lanes per column: 16 (dk when dk < 16); blocks of GT / R columns, one workgroup each (grid y)
    const int R = dk < 16 ? dk : 16, CW = GT / R;
    const dim3 grid(n_v, (dv + CW - 1) / CW);
    const size_t rl = (size_t)2 * (2 * GTC * dk + GTC * CW + 2 * GTC) * sizeof(float);
    static bool attr = false;
    if (!attr) {
        const void* fs[] = {(const void*)k_gdn_rec<1, 4>, (const void*)k_gdn_rec<1, 8>, (const void*)k_gdn_rec<1, 16>,
                            (const void*)k_gdn_rec<2, 16>, (const void*)k_gdn_rec<4, 16>, (const void*)k_gdn_rec<8, 16>};
        for (const void* f : fs) DET_CHECK(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024));
        attr = true;
    }
    switch (dk) {
    case 4: k_gdn_rec<1, 4><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    case 8: k_gdn_rec<1, 8><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    case 16: k_gdn_rec<1, 16><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    case 32: k_gdn_rec<2, 16><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    case 64: k_gdn_rec<4, 16><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    default: k_gdn_rec<8, 16><<<grid, GT, rl, st>>>(S->S, qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, L->norm, z, eps, on, cnt); break;
    }
    DET_CHECK(hipGetLastError());
    if (cnt) return;                                  // one token: the recurrence's last block of each head ran the gated norm
    const int rows = M * n_v, wg = (rows + 3) / 4;
    if (dv <= 64) k_gdn_out_w<1><<<wg, 256, 0, st>>>(ob, L->norm, z, eps, rows, dv, on);
    else if (dv <= 128) k_gdn_out_w<2><<<wg, 256, 0, st>>>(ob, L->norm, z, eps, rows, dv, on);
    else k_gdn_out_w<4><<<wg, 256, 0, st>>>(ob, L->norm, z, eps, rows, dv, on);
    DET_CHECK(hipGetLastError());
}

} // namespace det

extern "C" {

void det_argmax(const float* logits, int M, int V, int* out, hipStream_t st) {
    if (M < 1) return;
    if (V < 1) DET_FAIL("det_argmax: V=%d", V);
    if (M > 65535) DET_FAIL("det_argmax: M=%d exceeds the grid", M);
    if ((size_t)M > g_amx_cap) {
        DET_CHECK(hipStreamSynchronize(st));     // earlier launches may still use the old buffer
        if (g_amx) DET_CHECK(hipFree(g_amx));
        g_amx_cap = std::max<size_t>(M, 256);
        DET_CHECK(hipMalloc(&g_amx, g_amx_cap * 8));
        DET_CHECK(hipMemset(g_amx, 0, g_amx_cap * 8));
        DET_CHECK(hipDeviceSynchronize());
    }
    k_argmax_part<<<dim3((V + AMX_SLICE - 1) / AMX_SLICE, M), RT, 0, st>>>(logits, V, g_amx);
    DET_CHECK(hipGetLastError());
    k_argmax_fin<<<(M + 255) / 256, 256, 0, st>>>(logits, M, V, g_amx, out);
    DET_CHECK(hipGetLastError());
}

} // extern "C"
