// Shared device primitives of det's HIP path.  Every fp32 helper is exactly one IEEE binary32 operation in the
// op order of the spec (reference crates/det/src/spec/prim.rs); the library is compiled with -ffp-contract=off,
// denormals preserved and correctly rounded division/sqrt, so plain C operators are single IEEE ops.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#define DET_CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { \
    fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); abort(); } } while (0)

#define DET_FAIL(...) do { fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); abort(); } while (0)

namespace det {

constexpr int GROUP = 128;

// bytes per 32 codes (spec/tensor.rs:33-40) and per 128-group of one row
__host__ __device__ constexpr int bpl(int bits) { return bits == 8 ? 32 : bits == 6 ? 24 : 16; }
__host__ __device__ constexpr int group_bytes(int bits) { return 4 * bpl(bits); }
// tile geometry of the repacked layout: 64 rows per tile, 16-byte chunks
constexpr int TILE_N = 64;

// Hand-over between the workgroups of one launch (K-slices, split tiles, last-arriver epilogues): the producer writes
// its results with agent-scope atomic operations, which are performed at the device-coherent level instead of
// staying dirty in one XCD's L2; this wait blocks until every memory operation of the wave has been performed, and
// the memory clobber keeps the compiler from moving loads or stores across it.  Only then is the arrival counter
// bumped, and the consumer that sees the final count reads with agent-scope atomic loads.
// This is an ordering by completion, not a release/acquire pair of the language's memory model: on gfx950 an
// agent-scope release compiles to an L2 write-back (buffer_wbl2) and an acquire to an L2 invalidate, which measured
// tens of microseconds per split-K call, while every value handed over here is itself an agent-scope atomic.
__device__ __forceinline__ void wait_performed() { asm volatile("s_waitcnt 0" ::: "memory"); }

__device__ __forceinline__ float fmax_spec(float a, float b) {   // spec/prim.rs:58-70 (-0 below +0, NaN wins)
    if (__builtin_isnan(a) || __builtin_isnan(b)) return __builtin_isnan(a) ? a : b;
    if (a > b || (a == b && __builtin_signbit(b))) return a;
    return b;
}
__device__ __forceinline__ float fmin_spec(float a, float b) {   // spec/prim.rs:41-56
    if (__builtin_isnan(a) || __builtin_isnan(b)) return __builtin_isnan(a) ? a : b;
    if (a < b || (a == b && __builtin_signbit(a))) return a;
    return b;
}
__device__ __forceinline__ float rint_(float x) { return __builtin_rintf(x); }   // v_rndne_f32: ties to even

// Rust `v as i32` on an fp32 (saturating, NaN -> 0).
__device__ __forceinline__ int f2i_sat(float v) {
    if (__builtin_isnan(v)) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v < -2147483648.0f) return (int)0x80000000;
    return (int)v;
}
// spec/quant.rs:51-60 clamp_i8 on an already rounded value (NaN -> 0, as Rust `as i8`)
__device__ __forceinline__ int clamp_i8(float v) {
    if (v < -127.0f) return -127;
    if (v > 127.0f) return 127;
    if (__builtin_isnan(v)) return 0;
    return (int)v;
}

// int64 -> fp32 with round-to-nearest-even: shift the magnitude so that its leading one is bit 63, fold the low
// 32 bits into a sticky bit 0 of the high word, and let the hardware's u32 -> f32 conversion (round to nearest
// even) round that word; the sticky bit lies below the rounding position, so it only breaks exact ties, as the
// dropped bits would.  ldexp then restores the scale exactly.
__host__ __device__ __forceinline__ float i64_to_f(long long v) {
    const unsigned long long a = v < 0 ? 0ull - (unsigned long long)v : (unsigned long long)v;
    if (a == 0) return 0.0f;
    const int lz = __builtin_clzll(a);
    const unsigned long long nrm = a << lz;
    const unsigned int hi = (unsigned int)(nrm >> 32) | ((unsigned int)nrm != 0u ? 1u : 0u);
    const float f = __builtin_ldexpf((float)hi, 32 - lz);
    return v < 0 ? -f : f;
}

// int64 += int32 * uint32 (one 32x32->64 unsigned multiply-add and a sign fix of the high word)
__device__ __forceinline__ void mac_s32_u32(long long& acc, int p, uint32_t s) {
    unsigned long long r = (unsigned long long)(uint32_t)p * (unsigned long long)s + (unsigned long long)acc;
    r -= (unsigned long long)(s & (uint32_t)(p >> 31)) << 32;
    acc = (long long)r;
}

// ---- spec/prim.rs:78-149 transcendental op sequences (Cephes-derived, explicit fp32 ops; no libm).
// Constants are binary64 literals rounded once to binary32, as spec/prim.rs:4-35 writes them.
__device__ __forceinline__ float exp_f(float x) {
    x = fmin_spec(x, (float)88.0);
    if (x < (float)-87.0) return (float)0.0;
    const float n = __builtin_floorf((x * (float)1.44269504088896341) + (float)0.5);
    float r = x - (n * (float)0.693359375);
    r = r - (n * (float)-2.12194440e-4);
    const float z = r * r;
    float y = (float)1.9875691500E-4;
    y = (y * r) + (float)1.3981999507E-3;
    y = (y * r) + (float)8.3334519073E-3;
    y = (y * r) + (float)4.1665795894E-2;
    y = (y * r) + (float)1.6666665459E-1;
    y = (y * r) + (float)5.0000001201E-1;
    y = (y * z) + r;
    y = y + (float)1.0;
    const int ni = (int)n;
    const float scale = __uint_as_float((unsigned int)((ni + 127) << 23));
    return y * scale;
}
__device__ __forceinline__ float log_f(float x) {
    const unsigned int b = __float_as_uint(x);
    int e = (int)((b >> 23) & 0xFF) - 126;
    float m = __uint_as_float((b & 0x007FFFFFu) | 0x3F000000u);
    if (m < (float)0.707106781186547524) { e -= 1; m = (m + m) - (float)1.0; } else { m = m - (float)1.0; }
    const float z = m * m;
    float y = (float)7.0376836292E-2;
    y = (y * m) + (float)-1.1514610310E-1;
    y = (y * m) + (float)1.1676998740E-1;
    y = (y * m) + (float)-1.2420140846E-1;
    y = (y * m) + (float)1.4249322787E-1;
    y = (y * m) + (float)-1.6668057665E-1;
    y = (y * m) + (float)2.0000714765E-1;
    y = (y * m) + (float)-2.4999993993E-1;
    y = (y * m) + (float)3.3333331174E-1;
    y = y * m;
    y = y * z;
    const float ef = (float)e;
    y = y + ((float)-2.12194440e-4 * ef);
    y = y + ((float)-0.5 * z);
    float r = m + y;
    r = r + ((float)0.693359375 * ef);
    return r;
}
__device__ __forceinline__ float softplus_f(float x) {
    if (x > (float)20.0) return x;
    if (x < (float)-15.0) return exp_f(x);
    return log_f((float)1.0 + exp_f(fmin_spec(x, (float)20.0)));
}
__device__ __forceinline__ float sigmoid_f(float x) {
    if (x < (float)-80.0) return exp_f(x);
    return (float)1.0 / ((float)1.0 + exp_f(-fmax_spec(x, (float)-80.0)));
}
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }

// DPP lane exchange within a row of 16 lanes (ctrl: quad_perm 0xB1 = lane ^ 1, 0x4E = lane ^ 2; 0x141 row_half_mirror
// = lane 7 - i of its 8; 0x140 row_mirror = lane 15 - i of its 16)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum of the R adjacent lanes' subtree values (R = 1, 2, 4, 8 or 16, groups aligned to R), every lane of the group
// receiving it, added in the balanced tree's order: pairs of lanes, then pairs of pairs, ...  Each level adds the
// lower aligned half's value and the upper one's; fp32 addition commutes, so both halves compute the same sum.
// After level 2 a quad holds one value, so the half-mirror partner holds the other quad's; likewise the mirror
// partner after level 3.
template <int R>
__device__ __forceinline__ float lane_tree_sum(float v) {
    if (R >= 2) v = v + dpp_f<0xB1>(v);
    if (R >= 4) v = v + dpp_f<0x4E>(v);
    if (R >= 8) v = v + dpp_f<0x141>(v);
    if (R >= 16) v = v + dpp_f<0x140>(v);
    return v;
}

} // namespace det
