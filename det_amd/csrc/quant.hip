// Activation quantization kernels: det_quant, det_rmsnorm_quant, det_silu_mul_quant.
// One workgroup (4 waves of 64) per row; the row is staged in LDS as fp32 so any n works with one code path.
// Semantics are those of the reference backend (crates/det/src/cpu.rs:105-140,187-211 over
// spec/quant.rs:8-49), including Rust's casts: a NaN multiplier (0/0 when sx underflows to 0) becomes 0 and a NaN
// code becomes 0.
#include <string.h>
#include "common.h"
#include "gemm_internal.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

// threads per row: 256 when many rows fill the device, 1024 for a few rows (a lone row's workgroup then has 16
// waves to overlap its latency-bound reductions); the results do not depend on the count
constexpr int QT_MANY = 256, QT_FEW = 1024, QT_FEW_MAX_ROWS = 64;

enum { MODE_QUANT = 0, MODE_RMSNORM = 1, MODE_SILU_MUL = 2, MODE_MUL = 3 };

__host__ __device__ __forceinline__ int p_of(int n) { int p = 1; while (p < n) p <<= 1; return p; }

// order-free max over the wave: DPP exchanges inside rows of 16 lanes, then two lane shuffles
__device__ __forceinline__ float wave_max(float v) {
    v = fmax_spec(v, dpp_f<0xB1>(v));
    v = fmax_spec(v, dpp_f<0x4E>(v));
    v = fmax_spec(v, dpp_f<0x141>(v));
    v = fmax_spec(v, dpp_f<0x140>(v));
    v = fmax_spec(v, __shfl_xor(v, 16, 64));
    return fmax_spec(v, __shfl_xor(v, 32, 64));
}

// balanced tree over the N values of r (adjacent pairs level by level)
template <int N>
__device__ __forceinline__ float tree_reg(float* r) {
#pragma unroll
    for (int w = N >> 1; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; i++) r[i] = r[2 * i] + r[2 * i + 1];
    return r[0];
}
// the subtree of squares of v over the aligned leaves [i0, i0 + E) (leaves past n are +0)
template <int E>
__device__ __forceinline__ float sq_subtree(const float* v, int n, int i0) {
    float r[E];
#pragma unroll
    for (int i = 0; i < E; i++) r[i] = i0 + i < n ? v[i0 + i] * v[i0 + i] : 0.0f;
    return tree_reg<E>(r);
}

// dynamic LDS: v[n] fp32 (the row after its producer op)
template <int MODE, int QT>
__global__ void __launch_bounds__(QT) k_quant(const float* __restrict__ a, const float* __restrict__ b, float eps, int n,
                                              float* __restrict__ y, int8_t* __restrict__ xq, float* __restrict__ sx,
                                              uint16_t* __restrict__ mx) {
    constexpr int QW = QT / 64;        // waves per row
    extern __shared__ float lds[];
    __shared__ float red[QW];
    __shared__ float sg[1024];
    float* v = lds;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const size_t off = (size_t)row * n;

    // LB elements per thread are loaded before any is used, so their latencies overlap
    constexpr int LB = 8;
    for (int i0 = tid; i0 < n; i0 += LB * QT) {
        float ra[LB], rb[LB];
#pragma unroll
        for (int u = 0; u < LB; u++) {
            const int i = i0 + u * QT;
            ra[u] = i < n ? a[off + i] : 0.0f;
            if (MODE == MODE_SILU_MUL) rb[u] = i < n ? b[off + i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < LB; u++) {
            const int i = i0 + u * QT;
            if (i < n) {
                float x = ra[u];
                if (MODE == MODE_SILU_MUL) {
                    x = silu_f(x) * rb[u];
                    if (y) y[off + i] = x;
                }
                v[i] = x;
            }
        }
    }
    if (MODE == MODE_RMSNORM) {
        // spec/prim.rs:172-181: ss = treesum(x*x) over the row padded with +0 to p = next power of two.  The
        // squares are >= +0, so the tree over max(p, QT) leaves (zeros past p) has the same root: its extra
        // levels only add +0.  Thread t sums the aligned leaves [t E, t E + E) as a subtree, the wave's lanes
        // combine theirs pairwise (DPP, then two shuffles), and the waves' subtrees meet in tree order.
        const int p = p_of(n), E = p > QT ? p / QT : 1;
        __syncthreads();
        float ts;
        switch (E) {
        case 1: ts = sq_subtree<1>(v, n, tid); break;
        case 2: ts = sq_subtree<2>(v, n, tid * 2); break;
        case 4: ts = sq_subtree<4>(v, n, tid * 4); break;
        case 8: ts = sq_subtree<8>(v, n, tid * 8); break;
        case 16: ts = sq_subtree<16>(v, n, tid * 16); break;
        default: ts = sq_subtree<32>(v, n, tid * 32); break;
        }
        ts = lane_tree_sum<16>(ts);
        ts = ts + __shfl_xor(ts, 16, 64);
        ts = ts + __shfl_xor(ts, 32, 64);
        if (lane == 0) red[wv] = ts;
        __syncthreads();
        float wsum[QW];
#pragma unroll
        for (int w = 0; w < QW; w++) wsum[w] = red[w];
        const float ss = tree_reg<QW>(wsum);
        __syncthreads();                                  // red is reused by the plain quantization below
        const float mean = ss / (float)n;
        const float inv = 1.0f / __builtin_sqrtf(mean + eps);
        for (int i0 = tid; i0 < n; i0 += LB * QT) {
            float rw[LB];
#pragma unroll
            for (int u = 0; u < LB; u++) rw[u] = i0 + u * QT < n ? b[i0 + u * QT] : 0.0f;
#pragma unroll
            for (int u = 0; u < LB; u++) {
                const int i = i0 + u * QT;
                if (i < n) {
                    const float t = (v[i] * inv) * rw[u];
                    v[i] = t;
                    if (y) y[off + i] = t;
                }
            }
        }
    }
    __syncthreads();
    if (!xq) return;

    if (mx) {
        // spec/quant.rs:21-49
        const int G = n / GROUP;
        for (int g = wv; g < G; g += QW) {
            const float am = wave_max(fmax_spec(__builtin_fabsf(v[g * GROUP + lane]), __builtin_fabsf(v[g * GROUP + 64 + lane])));
            if (lane == 0) sg[g] = am / 127.0f;
        }
        __syncthreads();
        float smax = 0.0f;                       // fmax fold, order-free: one wave reduction per wave
        for (int g = lane; g < G; g += 64) smax = fmax_spec(smax, sg[g]);
        smax = wave_max(smax);
        const float s = smax == 0.0f ? 1.0f : smax / 65535.0f;
        for (int g = wv; g < G; g += QW) {
            float m = rint_(sg[g] / s);
            if (m < 1.0f) m = 1.0f;
            else if (m > 65535.0f) m = 65535.0f;
            const unsigned int mi = __builtin_isnan(m) ? 0u : (unsigned int)m;
            const float inv = 1.0f / (s * (float)mi);
            int8_t* q = xq + off + g * GROUP;
            q[lane] = (int8_t)clamp_i8(rint_(v[g * GROUP + lane] * inv));
            q[64 + lane] = (int8_t)clamp_i8(rint_(v[g * GROUP + 64 + lane] * inv));
            if (lane == 0) mx[(size_t)row * G + g] = (uint16_t)mi;
        }
        if (tid == 0) sx[row] = s;
    } else {
        // spec/quant.rs:8-16 quant_act_i8 over the whole row
        float am = 0.0f;
        for (int i = tid; i < n; i += QT) am = fmax_spec(am, __builtin_fabsf(v[i]));
        am = wave_max(am);
        if (lane == 0) red[wv] = am;
        __syncthreads();
        am = 0.0f;
        for (int w = 0; w < QW; w++) am = fmax_spec(am, red[w]);
        const float s = am == 0.0f ? 1.0f : am / 127.0f;
        const float inv = 1.0f / s;
        for (int i = tid; i < n; i += QT) xq[off + i] = (int8_t)clamp_i8(rint_(v[i] * inv));
        if (tid == 0) sx[row] = s;
    }
}

// Group mode with every thread holding EPT consecutive values of the row in registers (threads = n / EPT <= 1024,
// one row per workgroup): the producer op, the RMSNorm sum, the group maxima (LPG = 128 / EPT lanes per group, DPP)
// and the quantization run on registers, with two barriers in all (the standalone k_quant stages the row in LDS and
// walks the groups wave by wave).  The operations are k_quant's: the RMSNorm sum is the spec's tree (a thread's
// EPT leaves are an aligned subtree, then lane pairs by DPP and shuffles, then the waves' subtrees in order on 16
// lanes, zero leaves past the row adding +0 to squares), the maxima are order-free.
template <int LPG>
__device__ __forceinline__ float group_max(float v) {
    if (LPG >= 2) v = fmax_spec(v, dpp_f<0xB1>(v));
    if (LPG >= 4) v = fmax_spec(v, dpp_f<0x4E>(v));
    if (LPG >= 8) v = fmax_spec(v, dpp_f<0x141>(v));
    if (LPG >= 16) v = fmax_spec(v, dpp_f<0x140>(v));
    return v;
}
template <int MODE, int EPT>
__global__ void __launch_bounds__(1024) k_qrow(const float* __restrict__ a, const float* __restrict__ b, float eps, int n,
                                               float* __restrict__ y, int8_t* __restrict__ xq, float* __restrict__ sx,
                                               uint16_t* __restrict__ mx) {
    constexpr int LPG = GROUP / EPT;
    __shared__ float red[16];
    __shared__ float sg[1024];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, G = n / GROUP;
    const int i0 = tid * EPT;
    const bool live = i0 < n;                          // n is a multiple of 128, so a thread is all in or all out
    const size_t off = (size_t)row * n + i0;
    float v[EPT], u[EPT];
    if (live) {
#pragma unroll
        for (int k = 0; k < EPT; k += 4) {
            const float4 t = *reinterpret_cast<const float4*>(a + off + k);
            v[k] = t.x; v[k + 1] = t.y; v[k + 2] = t.z; v[k + 3] = t.w;
            if (MODE != MODE_QUANT) {
                const float4 q = *reinterpret_cast<const float4*>(b + (MODE == MODE_RMSNORM ? (size_t)i0 : off) + k);
                u[k] = q.x; u[k + 1] = q.y; u[k + 2] = q.z; u[k + 3] = q.w;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < EPT; k++) { v[k] = 0.0f; u[k] = 0.0f; }
    }
    if (MODE == MODE_SILU_MUL) {
#pragma unroll
        for (int k = 0; k < EPT; k++) v[k] = silu_f(v[k]) * u[k];
    }
    if (MODE == MODE_MUL) {
#pragma unroll
        for (int k = 0; k < EPT; k++) v[k] = v[k] * u[k];
    }
    if (MODE == MODE_RMSNORM) {
        float sq[EPT];
#pragma unroll
        for (int k = 0; k < EPT; k++) sq[k] = v[k] * v[k];
        float ts = tree_reg<EPT>(sq);
        ts = lane_tree_sum<16>(ts);
        ts = ts + __shfl_xor(ts, 16, 64);
        ts = ts + __shfl_xor(ts, 32, 64);
        if (lane == 0) red[wv] = ts;
        __syncthreads();
        const int nw = (int)(blockDim.x >> 6);
        float w = lane < nw && lane < 16 ? red[lane] : 0.0f;
        w = lane_tree_sum<16>(w);
        const float ss = __shfl(w, 0, 64);
        const float inv = 1.0f / __builtin_sqrtf((ss / (float)n) + eps);
#pragma unroll
        for (int k = 0; k < EPT; k++) v[k] = (v[k] * inv) * u[k];
    }
    if (y && live) {
#pragma unroll
        for (int k = 0; k < EPT; k += 4) *reinterpret_cast<float4*>(y + off + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    }
    if (!xq) return;
    // spec/quant.rs:21-49
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < EPT; k++) am = fmax_spec(am, __builtin_fabsf(v[k]));
    am = group_max<LPG>(am);
    const int g = tid / LPG;
    if (live && tid % LPG == 0) sg[g] = am / 127.0f;
    __syncthreads();
    float smax = 0.0f;
    for (int j = lane; j < G; j += 64) smax = fmax_spec(smax, sg[j]);
    smax = wave_max(smax);
    const float s = smax == 0.0f ? 1.0f : smax / 65535.0f;
    if (!live) return;
    float m = rint_(sg[g] / s);
    if (m < 1.0f) m = 1.0f;
    else if (m > 65535.0f) m = 65535.0f;
    const unsigned int mi = __builtin_isnan(m) ? 0u : (unsigned int)m;
    const float inv = 1.0f / (s * (float)mi);
    uint32_t pk[EPT / 4];
#pragma unroll
    for (int k = 0; k < EPT; k += 4) {
        uint32_t wd = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) wd |= ((uint32_t)(uint8_t)(int8_t)clamp_i8(rint_(v[k + j] * inv))) << (8 * j);
        pk[k / 4] = wd;
    }
    uint32_t* qd = reinterpret_cast<uint32_t*>(xq + off);
#pragma unroll
    for (int k = 0; k < EPT / 4; k++) qd[k] = pk[k];
    if (tid % LPG == 0) mx[(size_t)row * G + g] = (uint16_t)mi;
    if (tid == 0) sx[row] = s;
}

// k_qrow when it applies: group mode, 16-byte aligned rows, n / EPT <= 1024 threads (EPT = 8 up to n = 8192, 16 up
// to 16384, 32 up to 32768).  Returns false to leave the call to k_quant.
template <int MODE>
bool launch_qrow(const float* a, const float* b, float eps, int M, int n, float* y, int8_t* xq, float* sx, uint16_t* mx,
                 hipStream_t st) {
    if (!mx || !xq || n % GROUP) return false;
    const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al(a) || (b && !al(b)) || (y && !al(y)) || !al(xq)) return false;
    const int ept = n <= 8192 ? 8 : n <= 16384 ? 16 : n <= 32768 ? 32 : 0;
    if (!ept) return false;
    const int threads = ((n / ept + 63) / 64) * 64;
    switch (ept) {
    case 8: k_qrow<MODE, 8><<<M, threads, 0, st>>>(a, b, eps, n, y, xq, sx, mx); break;
    case 16: k_qrow<MODE, 16><<<M, threads, 0, st>>>(a, b, eps, n, y, xq, sx, mx); break;
    default: k_qrow<MODE, 32><<<M, threads, 0, st>>>(a, b, eps, n, y, xq, sx, mx); break;
    }
    DET_CHECK(hipGetLastError());
    return true;
}

template <int MODE>
void launch(const float* a, const float* b, float eps, int M, int n, float* y, int8_t* xq, float* sx, uint16_t* mx,
            hipStream_t st, const char* who) {
    if (M < 1) return;
    if (n < 1) DET_FAIL("%s: bad n=%d", who, n);
    if (mx && (n % GROUP)) DET_FAIL("%s: group mode needs n %% 128 == 0 (n=%d)", who, n);
    if (n / GROUP > 1024) DET_FAIL("%s: n=%d exceeds 1024 groups", who, n);
    int p = 1;
    while (p < n) p <<= 1;
    if (MODE == MODE_RMSNORM && p > 8192) DET_FAIL("%s: unsupported n=%d", who, n);
    const size_t lds = (size_t)n * 4;
    if (lds > 150 * 1024) DET_FAIL("%s: row of n=%d does not fit in LDS", who, n);
    if (launch_qrow<MODE>(a, b, eps, M, n, y, xq, sx, mx, st)) return;
    static bool attr = false;
    if (!attr) {
        DET_CHECK(hipFuncSetAttribute((const void*)k_quant<MODE, QT_MANY>, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024));
        DET_CHECK(hipFuncSetAttribute((const void*)k_quant<MODE, QT_FEW>, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024));
        attr = true;
    }
    if (M <= QT_FEW_MAX_ROWS) k_quant<MODE, QT_FEW><<<M, QT_FEW, lds, st>>>(a, b, eps, n, y, xq, sx, mx);
    else k_quant<MODE, QT_MANY><<<M, QT_MANY, lds, st>>>(a, b, eps, n, y, xq, sx, mx);
    DET_CHECK(hipGetLastError());
}

} // namespace

extern "C" {

void det_quant(const float* x, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st) {
    if (!xq || !sx) DET_FAIL("det_quant: xq and sx are required");
    launch<MODE_QUANT>(x, nullptr, 0.0f, M, n, nullptr, xq, sx, mx, st, "det_quant");
}

void det_rmsnorm_quant(const float* x, const float* w, float eps, int M, int n, float* y, int8_t* xq, float* sx, uint16_t* mx,
                       hipStream_t st) {
    launch<MODE_RMSNORM>(x, w, eps, M, n, y, xq, sx, mx, st, "det_rmsnorm_quant");
}

void det_silu_mul_quant(const float* g, const float* u, int M, int n, float* h, int8_t* hq, float* sh, uint16_t* mh,
                        hipStream_t st) {
    launch<MODE_SILU_MUL>(g, u, 0.0f, M, n, h, hq, sh, mh, st, "det_silu_mul_quant");
}

} // extern "C"

namespace det {

bool mul_quant(const float* a, const float* b, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st) {
    if (M < 1) return true;
    return launch_qrow<MODE_MUL>(a, b, 0.0f, M, n, nullptr, xq, sx, mx, st);
}

} // namespace det

extern "C" {

void det_test_gemv_silu0(const det_qlinear* L, const int8_t* xq, const float* sx, const uint16_t* mx, int nparts,
                         const int* offs, float* const* dsts, hipStream_t st) {
    det::gemm_parts_silu0(L, xq, sx, mx, nparts, offs, dsts, st);
}

void det_test_mul_quant(const float* a, const float* b, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st) {
    if (!det::mul_quant(a, b, M, n, xq, sx, mx, st)) DET_FAIL("det_test_mul_quant: unsupported row of n=%d", n);
}

} // extern "C"
