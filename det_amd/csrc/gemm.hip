// det quantized GEMM on gfx950 (MI355X), bit-exact to the spec (reference docs/SPEC.md:56-64,
// crates/det/src/spec/quant.rs:102-117):
//   acc[t][n] = sum_g ( m[n][g] * mx[t][g] ) * sum_{k in group g} wq[n][k] * xq[t][k]     (exact integers)
//   y[t][n]   = ((float)acc[t][n] * c[n]) * sx[t]                                          (RNE, 2 fp32 muls)
// The group partial fits int32 (|p| < 2^21), the multiplier uint32 (< 2^32) and acc int64 (< 2^61); every integer
// sum is associative, so tiling, split-K and atomics cannot change a result.
//
// Weights are read in the tiled layout det_linear_repack writes (det_hip.h): per 64-row tile and 128-group,
// GB/16 chunk planes of [64 rows][16 bytes], so one wave instruction loads 1 KB of contiguous bytes.
//
// Kernels (chosen by shape only, like the reference's gemm_bits, gemm.cu:1016-1023):
//   k_decode<BITS,MP> (M <= 8): one wave per (64-row tile, slice of groups).  Lane = output row; the lane streams
//       its row's packed groups with dwordx4 loads, unpacks to signed int8 words in registers, and dots them with
//       the activations (uniform across the wave, so they are scalar loads) with v_dot4c_i32_i8.  The int32 group
//       partial is scaled by m*mx into int64.  When the grid would not fill the chip the K range is split over
//       waves; the partial int64 sums meet in a self-cleaning device buffer with atomics and the last wave of a
//       tile runs the epilogue.
//   k_mfma<BITS,BM> (M > 8): 128-row x BM-token workgroup tile, 4 waves of (BM/2) x 64.  Per 128-group the
//       activation tile and the unpacked (signed int8) weight tile are staged in LDS; v_mfma_i32_32x32x32_i8 gives
//       the exact int32 group partials, which are scaled into int64 accumulators before the next group.
#include <string.h>
#include <algorithm>
#include "common.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ output routing (GemmOut, backend.rs:138-142)
struct Out {
    float* y;
    int acc, nparts;
    int offs[5];
    float* dst[4];
    __device__ __forceinline__ void store(int N, int t, int n, float v) const {
        float* p;
        if (nparts <= 1) {
            p = y + (size_t)t * N + n;
        } else {
            int i = 0;
#pragma unroll
            for (int j = 1; j < 4; j++) if (j < nparts && n >= offs[j]) i = j;
            p = dst[i] + (size_t)t * (offs[i + 1] - offs[i]) + (n - offs[i]);
        }
        *p = acc ? *p + v : v;
    }
};

// ------------------------------------------------------------------ code unpacking
// One 32-code block of the det format (spec §2): W8 = 8 words of int8; W4 = 4 words, byte i = u[i] | u[i+16] << 4
// with u = wq + 8; W6 = 4 words of low nibbles as W4 (u = wq + 32) then 2 words of 2-bit high parts, byte i =
// hi[i] | hi[i+8] << 2 | hi[i+16] << 4 | hi[i+24] << 6.  Output: 8 words of signed codes in k order.
// Unsigned bytes u in [0, 2^b) become signed u - OFF per byte as (u + 128 - OFF) ^ 0x80 (no carry between bytes).
template <int BITS> __device__ __forceinline__ void block_signed(const uint32_t* q, uint32_t* s);
template <> __device__ __forceinline__ void block_signed<8>(const uint32_t* q, uint32_t* s) {
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = q[j];
}
template <> __device__ __forceinline__ void block_signed<4>(const uint32_t* q, uint32_t* s) {
    constexpr uint32_t LM = 0x0F0F0F0Fu, ADD = 0x78787878u, X = 0x80808080u;   // 120 = 128 - 8
#pragma unroll
    for (int j = 0; j < 4; j++) {
        s[j] = ((q[j] & LM) + ADD) ^ X;
        s[j + 4] = (((q[j] >> 4) & LM) + ADD) ^ X;
    }
}
template <> __device__ __forceinline__ void block_signed<6>(const uint32_t* q, uint32_t* s) {
    constexpr uint32_t LM = 0x0F0F0F0Fu, HM = 0x30303030u, ADD = 0x60606060u, X = 0x80808080u;  // 96 = 128 - 32
    // codes 4j..4j+3: low nibble from word j % 4 (high half for j >= 4); the high pair sits at bit 2*(j/2 % 4)... of
    // high word (j & 1): codes c = 4j + b keep their pair in high byte (c % 8) at shift 2 * (c / 8)
    const uint32_t h0 = q[4], h1 = q[5];
    uint32_t u[8];
    u[0] = (q[0] & LM) | ((h0 << 4) & HM);
    u[1] = (q[1] & LM) | ((h1 << 4) & HM);
    u[2] = (q[2] & LM) | ((h0 << 2) & HM);
    u[3] = (q[3] & LM) | ((h1 << 2) & HM);
    u[4] = ((q[0] >> 4) & LM) | (h0 & HM);
    u[5] = ((q[1] >> 4) & LM) | (h1 & HM);
    u[6] = ((q[2] >> 4) & LM) | ((h0 >> 2) & HM);
    u[7] = ((q[3] >> 4) & LM) | ((h1 >> 2) & HM);
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = (u[j] + ADD) ^ X;
}

// int64 += int32 * uint32 (one 32x32->64 unsigned multiply-add and a sign fix of the high word)
__device__ __forceinline__ void mac_s32_u32(long long& acc, int p, uint32_t s) {
    unsigned long long r = (unsigned long long)(uint32_t)p * (unsigned long long)s + (unsigned long long)acc;
    r -= (unsigned long long)(s & (uint32_t)(p >> 31)) << 32;
    acc = (long long)r;
}

// ------------------------------------------------------------------ decode (M <= 8)
template <int BITS, int MP>
__global__ void __launch_bounds__(64) k_decode(const uint8_t* __restrict__ wq, const float* __restrict__ cs,
                                                const uint16_t* __restrict__ ms, int N, int K,
                                                const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                const uint16_t* __restrict__ mx, int M, Out out, int gps, int ks,
                                                unsigned long long* __restrict__ part, unsigned int* __restrict__ cnt) {
    constexpr int NC = group_bytes(BITS) / 16;     // 16-byte chunks per row-group
    const int lane = threadIdx.x;
    const int tile = blockIdx.x / ks, slice = blockIdx.x - tile * ks;
    const int G = K / GROUP;
    const int g0 = slice * gps, g1 = min(G, g0 + gps);
    long long acc[MP];
#pragma unroll
    for (int t = 0; t < MP; t++) acc[t] = 0;

    for (int g = g0; g < g1; g++) {
        const size_t tg = (size_t)tile * G + g;
        const uint4* src = reinterpret_cast<const uint4*>(wq + tg * NC * 1024) + lane;
        uint32_t q[NC * 4];
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src + c * 64));
            q[4 * c] = v.x; q[4 * c + 1] = v.y; q[4 * c + 2] = v.z; q[4 * c + 3] = v.w;
        }
        const uint32_t mm = ms[tg * 64 + lane];
        uint32_t w[32];
#pragma unroll
        for (int b = 0; b < 4; b++) block_signed<BITS>(q + b * (NC), w + 8 * b);
#pragma unroll
        for (int t = 0; t < MP; t++) {
            if (t < M) {
                const int* xr = reinterpret_cast<const int*>(xq + (size_t)t * K + (size_t)g * GROUP);
                int p = 0;
#pragma unroll
                for (int j = 0; j < 32; j++) p = __builtin_amdgcn_sdot4((int)w[j], xr[j], p, false);
                const uint32_t s = mm * (mx ? (uint32_t)mx[(size_t)t * G + g] : 1u);
                mac_s32_u32(acc[t], p, s);
            }
        }
    }

    const int n = tile * TILE_N + lane;
    if (ks == 1) {
        if (n < N) {
            const float c = cs[n];
#pragma unroll
            for (int t = 0; t < MP; t++)
                if (t < M) out.store(N, t, n, (i64_to_f(acc[t]) * c) * sx[t]);
        }
        return;
    }
    // split-K: exact int64 partial sums meet in part[t][Npad]; the last wave of the tile finishes and clears them
    const size_t npad = (size_t)gridDim.x / ks * TILE_N;
#pragma unroll
    for (int t = 0; t < MP; t++)
        if (t < M)
            __hip_atomic_fetch_add(part + (size_t)t * npad + n, (unsigned long long)acc[t], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    unsigned int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ks - 1);
    last = __shfl(last, 0, 64);
    if (!last) return;
    __threadfence();
    const float c = n < N ? cs[n] : 0.0f;
#pragma unroll
    for (int t = 0; t < MP; t++) {
        if (t < M) {
            const long long tot = (long long)__hip_atomic_exchange(part + (size_t)t * npad + n, 0ull, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_AGENT);
            if (n < N) out.store(N, t, n, (i64_to_f(tot) * c) * sx[t]);
        }
    }
    if (lane == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ MFMA GEMM (M > 8)
constexpr int MF_BN = 128;          // output rows n per workgroup (two 64-row tiles)
constexpr int MF_STR = 144;         // LDS row stride in bytes (128 codes + 16 pad)

template <int BITS, int BM>
__global__ void __launch_bounds__(256) k_mfma(const uint8_t* __restrict__ wq, const float* __restrict__ cs,
                                               const uint16_t* __restrict__ ms, int N, int K,
                                               const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                               const uint16_t* __restrict__ mx, int M, Out out) {
    constexpr int NC = group_bytes(BITS) / 16;
    constexpr int TM = BM / 64;                    // 32x32 tiles per wave along t
    __shared__ __attribute__((aligned(16))) int8_t As[BM * MF_STR];
    __shared__ __attribute__((aligned(16))) int8_t Bs[MF_BN * MF_STR];
    __shared__ uint32_t mxs[BM];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    const int n0 = blockIdx.x * MF_BN, t0 = blockIdx.y * BM;
    const int G = K / GROUP;
    const int tile0 = n0 / TILE_N;

    long long acc[TM][2][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    for (int g = 0; g < G; g++) {
        __syncthreads();
        // activations: BM rows x 128 bytes
#pragma unroll
        for (int i = 0; i < BM / 32; i++) {
            const int ch = tid + i * 256, tl = ch >> 3, kc = ch & 7;
            const int t = t0 + tl;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t < M) v = *reinterpret_cast<const uint4*>(xq + (size_t)t * K + (size_t)g * GROUP + kc * 16);
            *reinterpret_cast<uint4*>(As + tl * MF_STR + kc * 16) = v;
        }
        // weights: thread = (row r, half h) unpacks 64 codes
        {
            const int r = tid >> 1, h = tid & 1;
            const int tile = tile0 + (r >> 6), rr = r & 63;
            const uint4* src = reinterpret_cast<const uint4*>(wq + ((size_t)tile * G + g) * NC * 1024) + rr;
            uint32_t q[NC * 2];
#pragma unroll
            for (int c = 0; c < NC / 2; c++) {
                const uint4 v = src[(h * (NC / 2) + c) * 64];
                q[4 * c] = v.x; q[4 * c + 1] = v.y; q[4 * c + 2] = v.z; q[4 * c + 3] = v.w;
            }
            uint32_t w[16];
            block_signed<BITS>(q, w);
            block_signed<BITS>(q + NC, w + 8);
            uint4* dst = reinterpret_cast<uint4*>(Bs + r * MF_STR + h * 64);
#pragma unroll
            for (int c = 0; c < 4; c++) dst[c] = make_uint4(w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]);
        }
        if (tid < BM) {
            const int t = t0 + tid;
            mxs[tid] = (mx && t < M) ? (uint32_t)mx[(size_t)t * G + g] : 1u;
        }
        __syncthreads();

        v16i c[TM][2];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            v4i a[TM], b[2];
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const v4i*>(As + (wm * (BM / 2) + i * 32 + (lane & 31)) * MF_STR + s * 32 + (lane >> 5) * 16);
#pragma unroll
            for (int j = 0; j < 2; j++)
                b[j] = *reinterpret_cast<const v4i*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * MF_STR + s * 32 + (lane >> 5) * 16);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                    c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], s == 0 ? z : c[i][j], 0, 0, 0);
                }
        }
        // group scaling: element (row t, col n) of a 32x32 tile sits in lane (n % 32) + 32 * ((t / 4) % 2),
        // register 4 * (t / 8) + t % 4
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int nl = wn * 64 + j * 32 + (lane & 31);
            const uint32_t mm = ms[((size_t)(tile0 + (nl >> 6)) * G + g) * 64 + (nl & 63)];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int tl = wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    mac_s32_u32(acc[i][j][r], c[i][j][r], mm * mxs[tl]);
                }
        }
    }

#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float cn = cs[n];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = t0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t < M) out.store(N, t, n, (i64_to_f(acc[i][j][r]) * cn) * sx[t]);
            }
    }
}

// ------------------------------------------------------------------ load-time repack and quantizer
__global__ void k_repack(const uint8_t* __restrict__ rows, int N, int K, int bits, uint8_t* __restrict__ wq,
                         float* __restrict__ cs, uint16_t* __restrict__ ms, size_t nchunks) {
    const int G = K / GROUP, GB = group_bytes(bits), NC = GB / 16;
    const size_t rb = (size_t)K / 32 * bpl(bits) + 4 + 2 * (size_t)G;
    const size_t nc = (size_t)K / 32 * bpl(bits);
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < nchunks; idx += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(idx & 63);
        const size_t rest = idx >> 6;
        const int c = (int)(rest % NC);
        const size_t tg = rest / NC;
        const int g = (int)(tg % G);
        const size_t tile = tg / G;
        const size_t n = tile * TILE_N + r;
        uint8_t b[16];
        if (n < (size_t)N) {
            const uint8_t* s = rows + n * rb + (size_t)g * GB + c * 16;
#pragma unroll
            for (int i = 0; i < 16; i++) b[i] = s[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) b[i] = 0;
        }
        uint4 v;
        memcpy(&v, b, 16);
        reinterpret_cast<uint4*>(wq)[idx] = v;
        if (c == 0) {
            const uint8_t* s = rows + n * rb + nc;
            ms[tg * 64 + r] = n < (size_t)N ? (uint16_t)(s[4 + 2 * g] | (s[5 + 2 * g] << 8)) : 0;
            if (g == 0) {
                float cv = 0.0f;
                if (n < (size_t)N) { uint32_t u = s[0] | (s[1] << 8) | (s[2] << 16) | ((uint32_t)s[3] << 24); cv = __uint_as_float(u); }
                cs[n] = cv;
            }
        }
    }
}

// quantize.rs:33-55 group_scale (binary64; sequential squared-error sum; strict < keeps the first best)
__device__ double group_scale(const float* w, double qmax) {
    double amax = 0.0;
    for (int i = 0; i < GROUP; i++) amax = fmax(amax, fabs((double)w[i]));
    if (amax == 0.0) return 1.0;
    const double base = amax / qmax;
    double best_err = __builtin_inf(), best = base;
    for (int step = 0; step <= 10; step++) {
        const double s = base * (0.80 + 0.02 * (double)step);
        double err = -0.0;
        for (int i = 0; i < GROUP; i++) {
            const double v = (double)w[i];
            double q = __builtin_rint(v / s);
            q = q < -qmax ? -qmax : (q > qmax ? qmax : q);
            const double d = q * s - v;
            err = err + d * d;
        }
        if (err < best_err) { best_err = err; best = s; }
    }
    return best;
}

// quantize.rs:58-85 quantize_row, one workgroup per row, one thread per 128-group
__global__ void __launch_bounds__(256) k_quantize(const float* __restrict__ w, int K, int bits, uint8_t* __restrict__ rows) {
    __shared__ double sc[1024];
    __shared__ float c_s;
    const int G = K / GROUP, row = blockIdx.x;
    const float* wr = w + (size_t)row * K;
    const size_t rb = (size_t)K / 32 * bpl(bits) + 4 + 2 * (size_t)G, nc = (size_t)K / 32 * bpl(bits);
    uint8_t* out = rows + (size_t)row * rb;
    const double qmax = (double)((1 << (bits - 1)) - 1);
    for (int g = threadIdx.x; g < G; g += blockDim.x) sc[g] = group_scale(wr + g * GROUP, qmax);
    __syncthreads();
    if (threadIdx.x == 0) {
        double smax = 0.0;
        for (int g = 0; g < G; g++) smax = fmax(smax, sc[g]);
        const float c = (float)(smax / 65535.0);
        c_s = c;
        const uint32_t u = __float_as_uint(c);
        out[nc] = u & 0xFF; out[nc + 1] = (u >> 8) & 0xFF; out[nc + 2] = (u >> 16) & 0xFF; out[nc + 3] = u >> 24;
    }
    __syncthreads();
    const float c = c_s;
    for (int g = threadIdx.x; g < G; g += blockDim.x) {
        double mv = __builtin_rint(sc[g] / (double)c);
        mv = mv < 1.0 ? 1.0 : (mv > 65535.0 ? 65535.0 : mv);
        const uint32_t mg = (uint32_t)mv;
        out[nc + 4 + 2 * g] = mg & 0xFF;
        out[nc + 5 + 2 * g] = mg >> 8;
        const double eff = (double)c * (double)mg;
        for (int b = 0; b < 4; b++) {
            int q[32];
            for (int i = 0; i < 32; i++) {
                double v = __builtin_rint((double)wr[g * GROUP + b * 32 + i] / eff);
                v = v < -qmax ? -qmax : (v > qmax ? qmax : v);
                q[i] = (int)v;
            }
            uint8_t* o = out + ((size_t)g * 4 + b) * bpl(bits);
            if (bits == 8) {
                for (int i = 0; i < 32; i++) o[i] = (uint8_t)q[i];
            } else if (bits == 4) {
                for (int i = 0; i < 16; i++) o[i] = (uint8_t)((q[i] + 8) | ((q[i + 16] + 8) << 4));
            } else {
                for (int i = 0; i < 16; i++) o[i] = (uint8_t)(((q[i] + 32) & 0xF) | (((q[i + 16] + 32) & 0xF) << 4));
                for (int i = 0; i < 8; i++)
                    o[16 + i] = (uint8_t)(((q[i] + 32) >> 4) | (((q[i + 8] + 32) >> 4) << 2) | (((q[i + 16] + 32) >> 4) << 4) |
                                          (((q[i + 24] + 32) >> 4) << 6));
            }
        }
    }
}

// ------------------------------------------------------------------ host side
int g_num_cus = 0;
int g_decode_waves = 2048;      // target waves per decode launch (split-K below it)
int g_decode_max_m = 8;

// split-K buffers of k_decode: int64 partial sums [M][Npad] and per-tile arrival counters, zero between calls
unsigned long long* g_part = nullptr;
size_t g_part_cap = 0;          // elements
unsigned int* g_cnt = nullptr;
size_t g_cnt_cap = 0;
void* g_user_scratch = nullptr;
size_t g_user_scratch_bytes = 0;

void ensure_split_buffers(size_t part_elems, size_t tiles, hipStream_t st) {
    if (part_elems <= g_part_cap && tiles <= g_cnt_cap) return;
    DET_CHECK(hipStreamSynchronize(st));     // earlier launches may still use the old buffers
    if (part_elems > g_part_cap) {
        if (g_part) DET_CHECK(hipFree(g_part));
        g_part_cap = std::max(part_elems, (size_t)1 << 20);
        DET_CHECK(hipMalloc(&g_part, g_part_cap * 8));
        DET_CHECK(hipMemset(g_part, 0, g_part_cap * 8));
    }
    if (tiles > g_cnt_cap) {
        if (g_cnt) DET_CHECK(hipFree(g_cnt));
        g_cnt_cap = std::max(tiles, (size_t)1 << 14);
        DET_CHECK(hipMalloc(&g_cnt, g_cnt_cap * 4));
        DET_CHECK(hipMemset(g_cnt, 0, g_cnt_cap * 4));
    }
    DET_CHECK(hipDeviceSynchronize());
}

template <int BITS, int MP>
void launch_decode(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    const int G = L.K / GROUP;
    const int T = (L.N + TILE_N - 1) / TILE_N;
    int gps = G, ks = 1;
    if (T < g_decode_waves) {
        gps = (int)std::max<long long>(1, ((long long)T * G) / g_decode_waves);
        ks = (G + gps - 1) / gps;
    }
    unsigned long long* part = nullptr;
    unsigned int* cnt = nullptr;
    if (ks > 1) {
        ensure_split_buffers((size_t)M * T * TILE_N, (size_t)T, st);
        part = g_part;
        cnt = g_cnt;
    }
    k_decode<BITS, MP><<<T * ks, 64, 0, st>>>(L.wq, L.c, L.m, L.N, L.K, xq, sx, mx, M, y, gps, ks, part, cnt);
    DET_CHECK(hipGetLastError());
}

template <int BITS, int BM>
void launch_mfma(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    dim3 grid((L.N + MF_BN - 1) / MF_BN, (M + BM - 1) / BM);
    k_mfma<BITS, BM><<<grid, 256, 0, st>>>(L.wq, L.c, L.m, L.N, L.K, xq, sx, mx, M, y);
    DET_CHECK(hipGetLastError());
}

template <int BITS>
void gemm_bits(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    if (M <= g_decode_max_m) {
        if (M <= 1) launch_decode<BITS, 1>(L, xq, sx, mx, M, y, st);
        else if (M <= 2) launch_decode<BITS, 2>(L, xq, sx, mx, M, y, st);
        else if (M <= 4) launch_decode<BITS, 4>(L, xq, sx, mx, M, y, st);
        else launch_decode<BITS, 8>(L, xq, sx, mx, M, y, st);
    } else if (M <= 64) {
        launch_mfma<BITS, 64>(L, xq, sx, mx, M, y, st);
    } else {
        launch_mfma<BITS, 128>(L, xq, sx, mx, M, y, st);
    }
}

} // namespace

extern "C" {

void det_linear_sizes(int N, int K, int bits, size_t* wq_bytes, size_t* c_bytes, size_t* m_bytes) {
    if (K <= 0 || K % GROUP || N <= 0) DET_FAIL("det_linear_sizes: bad shape N=%d K=%d", N, K);
    if (bits != 4 && bits != 6 && bits != 8) DET_FAIL("det_linear_sizes: unsupported bits=%d", bits);
    const size_t T = ((size_t)N + TILE_N - 1) / TILE_N, G = (size_t)K / GROUP;
    if (wq_bytes) *wq_bytes = T * G * group_bytes(bits) * TILE_N;
    if (c_bytes) *c_bytes = T * TILE_N * 4;
    if (m_bytes) *m_bytes = T * G * TILE_N * 2;
}

void det_linear_repack(const uint8_t* rows, int N, int K, int bits, uint8_t* wq, float* c, uint16_t* m, hipStream_t st) {
    size_t wb;
    det_linear_sizes(N, K, bits, &wb, nullptr, nullptr);
    const size_t nchunks = wb / 16;
    const size_t blocks = std::min<size_t>((nchunks + 255) / 256, 65536);
    k_repack<<<(unsigned)blocks, 256, 0, st>>>(rows, N, K, bits, wq, c, m, nchunks);
    DET_CHECK(hipGetLastError());
}

void det_quantize_rows(const float* w, int N, int K, int bits, uint8_t* rows, hipStream_t st) {
    if (N < 1) return;
    if (K <= 0 || K % GROUP || K / GROUP > 1024) DET_FAIL("det_quantize_rows: bad K=%d", K);
    if (bits != 4 && bits != 6 && bits != 8) DET_FAIL("det_quantize_rows: unsupported bits=%d", bits);
    k_quantize<<<N, 64, 0, st>>>(w, K, bits, rows);
    DET_CHECK(hipGetLastError());
}

size_t det_gemm_scratch_bytes(int M, int K) { return (size_t)(M < 1 ? 1 : M) * (size_t)((K + 127) / 128) * sizeof(int); }
void det_gemm_set_scratch(void* p, size_t bytes) { g_user_scratch = p; g_user_scratch_bytes = p ? bytes : 0; }

void det_gemm_ex(const det_qlinear* Lp, const int8_t* xq, const float* sx, const uint16_t* mx, int M, float* y, int accumulate,
                 int nparts, const int* offs, float* const* dsts, hipStream_t st) {
    const det_qlinear L = *Lp;
    if (M < 1) return;
    if (L.K % GROUP != 0 || L.K <= 0 || L.N <= 0) DET_FAIL("det_gemm: bad shape N=%d K=%d", L.N, L.K);
    Out out;
    memset(&out, 0, sizeof out);
    out.y = y;
    out.acc = accumulate ? 1 : 0;
    if (nparts > 1) {
        if (nparts > 4) DET_FAIL("det_gemm: at most 4 output parts");
        if (offs[0] != 0) DET_FAIL("det_gemm: the first part must start at column 0");
        out.nparts = nparts;
        for (int i = 0; i < nparts; i++) { out.dst[i] = dsts[i]; out.offs[i] = offs[i]; }
        out.offs[nparts] = L.N;
    } else if (!y) {
        DET_FAIL("det_gemm: y == NULL");
    }
    if (L.bits != 4 && L.bits != 6 && L.bits != 8) DET_FAIL("det_gemm: unsupported bits=%d", L.bits);
    if (g_num_cus == 0) {
        int dev = 0;
        DET_CHECK(hipGetDevice(&dev));
        DET_CHECK(hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_decode_waves = 8 * g_num_cus;
    }
    switch (L.bits) {
        case 8: gemm_bits<8>(L, xq, sx, mx, M, out, st); break;
        case 6: gemm_bits<6>(L, xq, sx, mx, M, out, st); break;
        case 4: gemm_bits<4>(L, xq, sx, mx, M, out, st); break;
    }
}

void det_gemm(const det_qlinear* Lp, const int8_t* xq, const float* sx, const uint16_t* mx, int M, float* y, hipStream_t st) {
    det_gemm_ex(Lp, xq, sx, mx, M, y, 0, 0, nullptr, nullptr, st);
}

} // extern "C"
