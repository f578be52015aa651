// Device helpers shared by the GEMM kernels of gemm.hip (decode, M <= 64) and prefill.hip (M > 64).
#pragma once
#include <stdint.h>
#include "common.h"
#include "../../include/det_hip.h"

namespace det {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ output routing (GemmOut, backend.rs:138-142)
struct Out {
    float* y;
    int acc, nparts;
    int offs[5];
    float* dst[4];
    __device__ __forceinline__ float* ptr(int N, int t, int n) const {
        if (nparts <= 1) return y + (size_t)t * N + n;
        // selects, not an indexed load: a runtime index into dst/offs would put the struct in private memory
        float* d = dst[0];
        int lo = offs[0], hi = offs[1];
#pragma unroll
        for (int j = 1; j < 4; j++)
            if (j < nparts && n >= offs[j]) { d = dst[j]; lo = offs[j]; hi = offs[j + 1]; }
        return d + (size_t)t * (hi - lo) + (n - lo);
    }
    __device__ __forceinline__ void store(int N, int t, int n, float v) const {
        float* p = ptr(N, t, n);
        *p = acc ? *p + v : v;
    }
    // the same routing for the rows from token t on
    Out rows_from(int N, int t) const {
        Out o = *this;
        if (nparts <= 1) o.y = y + (size_t)t * N;
        for (int j = 0; j < 4 && j < nparts; j++) o.dst[j] = dst[j] + (size_t)t * (offs[j + 1] - offs[j]);
        return o;
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

// One 32-code block as unsigned codes u = wq + OFF (W4: 0..15, W6: 0..63), 8 words in k order.  These are valid
// non-negative int8 operands; the -OFF part of the codes is applied separately (on the MFMA, as x . (-OFF)).
template <int BITS> __device__ __forceinline__ void block_unsigned(const uint32_t* q, uint32_t* u);
template <> __device__ __forceinline__ void block_unsigned<4>(const uint32_t* q, uint32_t* u) {
    constexpr uint32_t LM = 0x0F0F0F0Fu;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        u[j] = q[j] & LM;
        u[j + 4] = (q[j] >> 4) & LM;
    }
}
template <> __device__ __forceinline__ void block_unsigned<6>(const uint32_t* q, uint32_t* u) {
    constexpr uint32_t LM = 0x0F0F0F0Fu, HM = 0x30303030u;
    const uint32_t h0 = q[4], h1 = q[5];
    u[0] = (q[0] & LM) | ((h0 << 4) & HM);
    u[1] = (q[1] & LM) | ((h1 << 4) & HM);
    u[2] = (q[2] & LM) | ((h0 << 2) & HM);
    u[3] = (q[3] & LM) | ((h1 << 2) & HM);
    u[4] = ((q[0] >> 4) & LM) | (h0 & HM);
    u[5] = ((q[1] >> 4) & LM) | (h1 & HM);
    u[6] = ((q[2] >> 4) & LM) | ((h0 >> 2) & HM);
    u[7] = ((q[3] >> 4) & LM) | ((h1 >> 2) & HM);
}
template <> __device__ __forceinline__ void block_unsigned<8>(const uint32_t* q, uint32_t* u) {
#pragma unroll
    for (int j = 0; j < 8; j++) u[j] = q[j];
}

// ------------------------------------------------------------------ global -> LDS copies
// Global -> LDS copy by the buffer unit (BYTES = 4 or 16 per lane, lane i's bytes land at lds + i * BYTES), written as
// inline assembly so that the compiler does not track it: with the builtin it cannot tell that later LDS reads touch
// other buffers and waits for every copy in flight before the first of them.  The caller waits (s_waitcnt vmcnt)
// and synchronises before reading the target.  `lds` must be wave-uniform; it travels in M0, which the asm takes as
// an operand (constraint {m0}), so that the compiler sets M0 itself and knows its value around every copy.
template <int BYTES>
__device__ __forceinline__ void dma_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff_, const void* lds) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(soff_);
    const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds);
    if (BYTES == 16)
        asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" :: "v"(voff), "s"(r), "s"(soff), "{m0}"(m0v) : "memory");
    else
        asm volatile("buffer_load_dword %0, %1, %2 offen lds" :: "v"(voff), "s"(r), "s"(soff), "{m0}"(m0v) : "memory");
}

// N (<= 4) copies of 16 bytes per lane under one M0 value: copy i reads the resource at voff[i] + soff + 1024 i and
// lands at lds + 1024 i + 16 lane (the instruction offset moves both addresses).  Changing M0 stalls until the copies
// issued before have consumed it, so each run sets it once.
template <int N>
__device__ __forceinline__ void dma16_run(__amdgpu_buffer_rsrc_t r, const uint32_t* voff, uint32_t soff_, const void* lds) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(soff_);      // uniform by construction; keep it scalar
    const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds);
    static_assert(N >= 1 && N <= 4, "at most 4 copies per run");
    if constexpr (N == 4)
        asm volatile("buffer_load_dwordx4 %0, %4, %6 offen lds\n\t"
                     "buffer_load_dwordx4 %1, %4, %6 offen offset:1024 lds\n\t"
                     "buffer_load_dwordx4 %2, %4, %6 offen offset:2048 lds\n\t"
                     "buffer_load_dwordx4 %3, %4, %6 offen offset:3072 lds"
                     :: "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "v"(voff[3]), "s"(r), "{m0}"(m0v), "s"(soff) : "memory");
    else if constexpr (N == 3)
        asm volatile("buffer_load_dwordx4 %0, %3, %5 offen lds\n\t"
                     "buffer_load_dwordx4 %1, %3, %5 offen offset:1024 lds\n\t"
                     "buffer_load_dwordx4 %2, %3, %5 offen offset:2048 lds"
                     :: "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "s"(r), "{m0}"(m0v), "s"(soff) : "memory");
    else if constexpr (N == 2)
        asm volatile("buffer_load_dwordx4 %0, %2, %4 offen lds\n\t"
                     "buffer_load_dwordx4 %1, %2, %4 offen offset:1024 lds"
                     :: "v"(voff[0]), "v"(voff[1]), "s"(r), "{m0}"(m0v), "s"(soff) : "memory");
    else
        asm volatile("buffer_load_dwordx4 %0, %1, %3 offen lds"
                     :: "v"(voff[0]), "s"(r), "{m0}"(m0v), "s"(soff) : "memory");
}
// four copies under one M0 through one resource, copy i at voff[i] + soff + 1024 i, landing at lds + 1024 i + 16 lane
__device__ __forceinline__ void dma16_run4v(__amdgpu_buffer_rsrc_t r, const uint32_t* voff, uint32_t soff_, const void* lds) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(soff_);
    const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds);
    asm volatile("buffer_load_dwordx4 %0, %4, %6 offen lds\n\t"
                 "buffer_load_dwordx4 %1, %4, %6 offen offset:1024 lds\n\t"
                 "buffer_load_dwordx4 %2, %4, %6 offen offset:2048 lds\n\t"
                 "buffer_load_dwordx4 %3, %4, %6 offen offset:3072 lds"
                 :: "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "v"(voff[3]), "s"(r), "{m0}"(m0v), "s"(soff) : "memory");
}
// four copies under one M0, copy i through resource r[i] at voff[i % 2] + soff + 1024 i, landing at
// lds + 1024 i + 16 lane
__device__ __forceinline__ void dma16_run4x(const __amdgpu_buffer_rsrc_t* r, uint32_t voff0, uint32_t voff1, uint32_t soff_,
                                            const void* lds) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(soff_);
    const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds);
    asm volatile("buffer_load_dwordx4 %0, %2, %7 offen lds\n\t"
                 "buffer_load_dwordx4 %1, %3, %7 offen offset:1024 lds\n\t"
                 "buffer_load_dwordx4 %0, %4, %7 offen offset:2048 lds\n\t"
                 "buffer_load_dwordx4 %1, %5, %7 offen offset:3072 lds"
                 :: "v"(voff0), "v"(voff1), "s"(r[0]), "s"(r[1]), "s"(r[2]), "s"(r[3]), "{m0}"(m0v), "s"(soff) : "memory");
}


// int64 -> fp32 (round to nearest even) for the epilogues: |v| < 2^52 is exact as a double (high word times 2^32
// plus the low word, one fma), and the double -> float conversion then rounds once; larger magnitudes take
// i64_to_f.
__device__ __forceinline__ float i64_to_f_fast(long long v) {
    const int hi = (int)(v >> 32);
    if ((uint32_t)(hi + (1 << 20)) < (1u << 21)) {       // -2^52 <= v < 2^52
        const double d = __builtin_fma((double)hi, 4294967296.0, (double)(uint32_t)v);
        return (float)d;
    }
    return i64_to_f(v);
}
// start value of every MFMA chain in the biased scaling: |p| <= 128 * 127 * 128 < 2^21, so p + B >= 0
constexpr uint32_t PF_BIAS = 1u << 21;
// a * b for a, b < 2^16 (m and mx).  Inline asm: the compiler turns __umul24 of operands it cannot bound into an
// AND and the quarter-rate v_mul_lo_u32.
__device__ __forceinline__ uint32_t mul_u24(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// prefill.hip: the prefill planes inside a linear's wq buffer, their load-time repack, and the GEMM for M > 64
// (returns false, having launched nothing, when the shape is outside what the kernel covers)
__attribute__((visibility("hidden"))) bool use_streamk();
__attribute__((visibility("hidden"))) size_t pf_offset(int N, int K, int bits);
__attribute__((visibility("hidden"))) void prefill_repack(const uint8_t* rows, int N, int K, int bits, uint8_t* wq, hipStream_t st);
__attribute__((visibility("hidden"))) bool prefill_gemm(const det_qlinear& L, const int8_t* xq, const float* sx,
                                                        const uint16_t* mx, int M, const Out& y, int cus, hipStream_t st);

} // namespace det
