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
//   k_decode<BITS,MP> (M <= 16): 64-row tiles x K-slices, lane = output row.  Each wave streams one packed
//       128-group at a time with dwordx4 loads (all issued before any arithmetic) and unpacks them to signed int8 words in
//       registers.  M == 1: dots with the activations (scalar loads) by v_dot4c_i32_i8; 2 <= M <= 16: one
//       v_mfma_i32_32x32x32_i8 per 16 k-bytes carries the 64 rows x MP tokens.  The int32 group partial is scaled by
//       m*mx into int64; the waves of a workgroup add in LDS, the K-slices of a tile by int64 atomics.
//   k_decode_ms<BITS,TS> (16 < M <= 64): 64-row tiles x K-slices; a wave owns 32 rows x all MT = 32 TS tokens,
//       each lane half a row's packed group (no duplicate loads or unpacking); the activations come global -> LDS by
//       the buffer unit; one v_mfma_i32_32x32x32_i8 per 32 codes and token set; group scaling with two VALU ops per
//       output (biased partials, bias removed by digit-product MFMAs once per workgroup).
//   k_prefill2<BITS> (M > 64): 128-token x 64-row workgroup tiles, three workgroups per CU, activations copied
//       global -> LDS by the buffer unit, W4/W6 codes unpacked from registers a group ahead into a double-buffered
//       tile (one barrier per group), the same biased scaling.
#include <string.h>
#include <algorithm>
#include "common.h"
#include "gemm_internal.h"
#include "gemm_common.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

// ------------------------------------------------------------------ decode (M <= 16)
// Grid: T tiles x KS K-slices, one workgroup each, S waves per workgroup; wave w of slice k takes the groups
// g0(k) + w, g0(k) + w + S, ... (normally exactly one), issuing all its loads before any arithmetic.  The waves'
// exact int64 sums meet in LDS.  With KS > 1 every slice adds its sums into part[t][n] with int64 atomics, waits
// until they are performed, then counts itself in cnt[tile]; the workgroup that arrives last takes the totals by
// atomic exchange with 0, runs the epilogue and resets the counter, so part and cnt are zero again between calls.
// No workgroup waits for another.  Atomics are coherent across the XCDs' L2s, so no cache write-back is needed.
constexpr int DEC_MAXW = 16;
constexpr int DEC_GPW = 1;         // groups a wave keeps in flight at once (2 to 4 measured slower)
constexpr int DEC_MMA_MIN = 4;     // fewest tokens that take the matrix-core form

// MP >= 4 runs the dot products on the matrix core: per 16 k-bytes one v_mfma_i32_32x32x32_i8 with the weights as
// the B operand straight from the tile layout (lane l holds row l; column j of B is row j in the low k-half and row
// j + 32 in the high k-half) and the activations as A: row i < MP of A is token i in the low k-half (zero in the high
// one), row MP + i is token i in the high k-half (zero in the low one).  Element (i, j) of the 32 x 32 result
// (lane j + 32 * ((i / 4) % 2), register 4 * (i / 8) + i % 4) is then the partial sum of token i mod MP with weight
// row j + 32 * (i >= MP); registers r < MP carry every (row, token) pair of the tile once.
template <int MP>
__device__ __forceinline__ int dec_tok(int r, int lane) {
    if (MP < DEC_MMA_MIN) return r;
    const int i = 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
    return i >= MP ? i - MP : i;
}
template <int MP>
__device__ __forceinline__ int dec_row(int r, int lane) {
    if (MP < DEC_MMA_MIN) return lane;
    const int i = 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
    return (lane & 31) + (i >= MP ? 32 : 0);
}

template <int MP>
constexpr int dec_maxw() { return MP >= DEC_MMA_MIN ? 8 : DEC_MAXW; }     // the matrix-core form needs up to 256 VGPRs

// SILU0: the one-token gate|up projection stores silu_f(v) for the columns of part 0 (cpu.rs:187-211's silu of g)
template <bool SILU0>
__device__ __forceinline__ float dec_val(const Out& out, int n, float v) {
    if constexpr (SILU0) return n < out.offs[1] ? silu_f(v) : v;
    return v;
}

template <int BITS, int MP, bool SILU0 = false>
__global__ void __launch_bounds__(64 * dec_maxw<MP>()) k_decode(const uint8_t* __restrict__ wq, const float* __restrict__ cs,
                                                const uint16_t* __restrict__ ms, int N, int K,
                                                const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                const uint16_t* __restrict__ mx, int M, Out out, int KS,
                                                long long* __restrict__ part, unsigned int* __restrict__ cnt) {
    constexpr int NC = group_bytes(BITS) / 16;     // 16-byte chunks per row-group
    constexpr bool MMA = MP >= DEC_MMA_MIN;
    static_assert(MP <= 16, "at most 16 tokens");
    extern __shared__ long long red_dyn[];          // [S][MP][64] int64 partial sums
    __shared__ unsigned int last_s;
    const int lane = threadIdx.x & 63, S = blockDim.x >> 6;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);     // wave-uniform: activations come in by scalar loads
    const int tile = blockIdx.x / KS, ks = blockIdx.x - tile * KS;
    const int G = K / GROUP;
    const int gs = (G + KS - 1) / KS;              // groups per slice
    const int g0 = ks * gs, g1 = min(G, g0 + gs);
    long long acc[MP];
#pragma unroll
    for (int t = 0; t < MP; t++) acc[t] = 0;
    // the epilogue's row scales and token scales, loaded now so that their latency hides under the weight stream
    float csr[MP], sxr[MP];
#pragma unroll
    for (int r = 0; r < MP; r++) {
        const int t = dec_tok<MP>(r, lane), n = tile * TILE_N + dec_row<MP>(r, lane);
        csr[r] = n < N ? cs[n] : 0.0f;
        sxr[r] = t < M ? sx[t] : 0.0f;
    }
    // matrix-core path: the token whose activations this lane feeds into A (-1: none)
    const int ai = lane & 31;
    int atok = (lane < 32) ? (ai < MP ? ai : -1) : (ai >= MP && ai < 2 * MP ? ai - MP : -1);
    if (atok >= M) atok = -1;

    for (int gb = g0 + wv; gb < g1; gb += S * DEC_GPW) {
        uint32_t q[DEC_GPW][NC * 4];
        uint32_t mm[DEC_GPW][MMA ? 2 : 1];
        v4i xa[MMA ? DEC_GPW : 1][MMA ? 8 : 1];
        uint32_t mxa[DEC_GPW];
#pragma unroll
        for (int u = 0; u < DEC_GPW; u++) {          // every load of this batch before any arithmetic
            const int g = gb + u * S;
            if (g < g1) {
                const size_t tg = (size_t)tile * G + g;
                const v4i* src = reinterpret_cast<const v4i*>(wq + tg * NC * 1024) + lane;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const v4i v = __builtin_nontemporal_load(src + c * 64);
                    q[u][4 * c] = v.x; q[u][4 * c + 1] = v.y; q[u][4 * c + 2] = v.z; q[u][4 * c + 3] = v.w;
                }
                if constexpr (MMA) {
                    mm[u][0] = ms[tg * 64 + (lane & 31)];
                    mm[u][1] = ms[tg * 64 + (lane & 31) + 32];
                    const v4i z = {0, 0, 0, 0};
                    const v4i* xs = reinterpret_cast<const v4i*>(xq + (size_t)max(atok, 0) * K + (size_t)g * GROUP);
#pragma unroll
                    for (int c = 0; c < 8; c++) xa[u][c] = atok >= 0 ? xs[c] : z;
                    mxa[u] = atok < 0 ? 0u : (mx ? (uint32_t)mx[(size_t)atok * G + g] : 1u);
                } else {
                    mm[u][0] = ms[tg * 64 + lane];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < DEC_GPW; u++) {
            const int g = gb + u * S;
            if (g < g1) {
                uint32_t w[32];
#pragma unroll
                for (int b = 0; b < 4; b++) block_signed<BITS>(q[u] + b * NC, w + 8 * b);
                if constexpr (MMA) {
                    v16i d = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        const v4i bw = {(int)w[4 * c], (int)w[4 * c + 1], (int)w[4 * c + 2], (int)w[4 * c + 3]};
                        d = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[u][c], bw, d, 0, 0, 0);
                    }
                    // multipliers of token t: lane t feeds token t (t < MP), so read them across the wave
                    uint32_t mxt[MP];
#pragma unroll
                    for (int t = 0; t < MP; t++) mxt[t] = __builtin_amdgcn_readlane(mxa[u], t);
#pragma unroll
                    for (int r = 0; r < MP; r++) {
                        // token and row of register r in the low and high half of the wave (compile-time per half)
                        const int i0 = 8 * (r / 4) + (r % 4), i1 = i0 + 4;
                        const uint32_t mx0 = mxt[i0 >= MP ? i0 - MP : i0], mx1 = mxt[i1 >= MP ? i1 - MP : i1];
                        const uint32_t m0 = mm[u][i0 >= MP], m1 = mm[u][i1 >= MP];
                        const uint32_t sc = lane < 32 ? m0 * mx0 : m1 * mx1;
                        mac_s32_u32(acc[r], d[r], sc);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < MP; t++) {
                        if (t < M) {
                            const int* xr = reinterpret_cast<const int*>(xq + (size_t)t * K + (size_t)g * GROUP);
                            int p = 0;
#pragma unroll
                            for (int j = 0; j < 32; j++) p = __builtin_amdgcn_sdot4((int)w[j], xr[j], p, false);
                            const uint32_t sc = mm[u][0] * (mx ? (uint32_t)mx[(size_t)t * G + g] : 1u);
                            mac_s32_u32(acc[t], p, sc);
                        }
                    }
                }
            }
        }
    }
    // register r of this lane holds (token dec_tok(r), row dec_row(r)); tokens >= M are padding
    if (S == 1 && KS == 1) {
#pragma unroll
        for (int r = 0; r < MP; r++) {
            const int t = dec_tok<MP>(r, lane), n = tile * TILE_N + dec_row<MP>(r, lane);
            if (t < M && n < N) out.store(N, t, n, dec_val<SILU0>(out, n, (i64_to_f(acc[r]) * csr[r]) * sxr[r]));
        }
        return;
    }
    if (S > 1) {
#pragma unroll
        for (int r = 0; r < MP; r++) red_dyn[(wv * MP + r) * 64 + lane] = acc[r];
        __syncthreads();
    }
    // wave w finishes registers w, w + S, ... of the workgroup's sum
    const size_t npad = (size_t)(gridDim.x / KS) * TILE_N;
    long long tot[MP];
#pragma unroll
    for (int r = 0; r < MP; r++) {
        tot[r] = 0;
        const int t = dec_tok<MP>(r, lane), n = tile * TILE_N + dec_row<MP>(r, lane);
        if (r % S != wv) continue;
        long long v = 0;
        if (S > 1) for (int w = 0; w < S; w++) v += red_dyn[(w * MP + r) * 64 + lane];
        else v = acc[r];
        tot[r] = v;
        // every slice adds into the accumulator (device-coherent atomics: no cache write-back needed)
        if (KS > 1 && t < M) __hip_atomic_fetch_add(part + (size_t)t * npad + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (KS > 1) {
        wait_performed();             // this wave's adds have been performed
        __syncthreads();
        if (threadIdx.x == 0)
            last_s = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(KS - 1);
        __syncthreads();
        if (!last_s) return;
        // the last slice to arrive reads the sums, leaving the accumulator and the counter at zero for the next call
#pragma unroll
        for (int r = 0; r < MP; r++) {
            const int t = dec_tok<MP>(r, lane), n = tile * TILE_N + dec_row<MP>(r, lane);
            if (r % S != wv || t >= M) continue;
            tot[r] = __hip_atomic_exchange(part + (size_t)t * npad + n, 0LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (threadIdx.x == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int r = 0; r < MP; r++) {
        const int t = dec_tok<MP>(r, lane), n = tile * TILE_N + dec_row<MP>(r, lane);
        if (r % S == wv && t < M && n < N) out.store(N, t, n, dec_val<SILU0>(out, n, (i64_to_f(tot[r]) * csr[r]) * sxr[r]));
    }
}

// ------------------------------------------------------------------ decode, many tokens (16 < M <= 64)
// A workgroup of P (<= 4) wave pairs walks the groups g0 .. g1-1 of one tile's K-slice, pair p taking groups
// g0 + p, g0 + p + P, ... (one round = one group per pair); wave h of a pair owns weight rows 32 h .. 32 h + 31 of the
// tile for all MT = 32 TS tokens.  Lane l holds row 32 h + l % 32 and k-half e = l / 32 of the group: packed blocks
// 2 e and 2 e + 1 (whole chunk planes in every format), so no lane loads or unpacks what another lane does.  Per 32
// k-codes step s (0..3) the lane's B operand is its codes 64 e + 16 s .. + 15 and the A operand of lane l the same
// codes of token l % 32 (+ 32 ts), so one v_mfma_i32_32x32x32_i8 per step and token set gives the 32 x 32 (token,
// row) group partials in the standard layout: lane l keeps row 32 h + l % 32, register r token 8 (r / 4) + 4 e + r % 4.
// Scaling as in k_prefill2: each chain starts from B = 2^21 and U += (p + B) * (m * mx) (one v_mul_u32_u24, one
// v_mad_u64_u32).  B * S, S = sum_g m * mx, is removed once per workgroup: every round stages the 7-bit digits of its
// group's m (per row) and mx (per token) in LDS at the group's slot, and after the loop 9 digit-product MFMAs per 32
// slots give S for each 32 x 32 block exactly.
// The activations of a pair's group (MT rows of 128 bytes, chunk-swizzled) are copied global -> LDS by the buffer
// unit, half by each wave; the workgroup runs in lockstep (one barrier per round) with the next round's weight words
// and activations in flight while the current round computes (two LDS areas).  With P = 2 two workgroups share a CU,
// so one's prologue and epilogue overlap the other's rounds.  The waves' int64 sums meet in LDS (over the activation areas);
// with KS > 1 every slice stores its sums (agent-scope stores, coherent across the XCDs' L2s) into its own plane of
// `part`, counts itself in cnt[tile], and the last slice to arrive adds the other planes and writes the outputs.
constexpr int DMS_MAXP = 4;          // wave pairs per workgroup
constexpr int DMS_MAXSLOT = 96;      // groups per K-slice (digit slots in LDS)
// bytes of v (slots s0 .. s0 + 3) at or past slot n set to zero
__device__ __forceinline__ int mask_slots(int v, int s0, int n) {
    const int k = n - s0;
    return k >= 4 ? v : k <= 0 ? 0 : (int)((uint32_t)v & (0xffffffffu >> (32 - 8 * k)));
}
template <int BITS, int TS>
__global__ void __launch_bounds__(128 * DMS_MAXP) k_decode_ms(const uint8_t* __restrict__ wq, const float* __restrict__ cs,
                                                                const uint16_t* __restrict__ ms, int N, int K,
                                                                const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                                const uint16_t* __restrict__ mx, int M, Out out, int KS,
                                                                long long* __restrict__ part, unsigned int* __restrict__ cnt) {
    constexpr int NC = group_bytes(BITS) / 16;  // chunk planes per row-group; a k-half is NC / 2 of them
    constexpr int NH = NC / 2;
    constexpr int MT = 32 * TS;                 // tokens per launch
    constexpr int XB = MT * 128;                // bytes of one group's activations
    constexpr int NCP = MT / 16;                // 1 KB copies per wave per group (half the rows)
    // dynamic LDS: [2 areas][P pairs][MT rows][128] activations (later the int64 sums [MT][64]), then the digits
    // [3][64 rows][NS] of m and [3][MT][NS] of mx (NS = slots, a multiple of 32)
    extern __shared__ __attribute__((aligned(16))) int8_t xs_dyn[];
    __shared__ __attribute__((aligned(16))) uint32_t mxs_s[2 * DMS_MAXP][MT];   // each wave's token multipliers
    __shared__ float sxs_s[MT];
    __shared__ unsigned int last_s;
    const int lane = threadIdx.x & 63, W = blockDim.x >> 6, P = W >> 1;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // token block blockIdx.y: tokens t0 .. t0 + MT - 1 (the launch has ceil(M / MT) of them); from here on xq, sx,
    // mx and M describe the block's own tokens, and only the output rows and the K-slice buffers see t0
    const int tbk = blockIdx.y, t0 = tbk * MT;
    xq += (size_t)t0 * K;
    sx += t0;
    if (mx) mx += (size_t)t0 * (K / GROUP);
    M -= t0;
    const int pr = wv >> 1, hf = wv & 1;        // pair and row half of this wave
    const int e = lane >> 5, l32 = lane & 31, row = 32 * hf + l32;
    const int tile = blockIdx.x / KS, ks = blockIdx.x - tile * KS;
    const int G = K / GROUP;
    const int gs = (G + KS - 1) / KS;
    const int g0 = ks * gs, g1 = min(G, g0 + gs), ng = g1 - g0;
    const int NS = (gs + 31) & ~31;
    const int rounds = (gs + P - 1) / P;        // the same for every wave: each round ends at a barrier
    const int n = tile * TILE_N + lane;         // output row of this thread in the epilogue
    // epilogue operands, loaded now so that their latency hides under the rounds
    const float cn = n < N ? cs[n] : 0.0f;
    const float sxl = wv == 0 && lane < MT ? sx[min(lane, M - 1)] : 0.0f;
    unsigned long long U[TS][16];
#pragma unroll
    for (int t = 0; t < TS; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) U[t][r] = 0;
    const int tot_bytes = max(2 * P * XB, MT * TILE_N * 8);
    int8_t* wdig = xs_dyn + tot_bytes;           // [3][64][NS]
    int8_t* xdig = wdig + 3 * 64 * NS;           // [3][MT][NS]
    // activation copy c of this wave: row R = MT/2 hf + 8 c + lane / 8; LDS slot lane % 8 of row R holds chunk
    // (lane % 8) ^ ((R / 2) % 8).  Rows past M lie beyond the resource's range and read as zero.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, M * K, 0x00020000);
    uint32_t xvo[NCP];
#pragma unroll
    for (int c = 0; c < NCP; c++) {
        const int R = (MT / 2) * hf + 8 * c + (lane >> 3);
        xvo[c] = (uint32_t)(R * K + (((lane & 7) ^ ((R >> 1) & 7)) * 16)) - 1024u * (c & 3);
    }
    auto area = [&](int par) __attribute__((always_inline)) { return xs_dyn + (par * P + pr) * XB; };

    uint32_t q[NH * 4];
    uint32_t m_n = 0, mxl_n = 0;
    auto fetch = [&](int g, int8_t* xd) __attribute__((always_inline)) {
#pragma unroll
        for (int c0 = 0; c0 < NCP; c0 += 4) {
            if (NCP - c0 >= 4) dma16_run<4>(xr, xvo + c0, g * GROUP, xd + (MT / 2) * hf * 128 + c0 * 1024);
            else dma16_run<2>(xr, xvo + c0, g * GROUP, xd + (MT / 2) * hf * 128 + c0 * 1024);
        }
        const size_t tg = (size_t)tile * G + g;
        const v4i* src = reinterpret_cast<const v4i*>(wq + tg * NC * 1024 + (size_t)NH * e * 1024) + row;
#pragma unroll
        for (int c = 0; c < NH; c++) {
            const v4i v = __builtin_nontemporal_load(src + c * 64);
            q[4 * c] = v.x; q[4 * c + 1] = v.y; q[4 * c + 2] = v.z; q[4 * c + 3] = v.w;
        }
        m_n = ms[tg * 64 + row];
        mxl_n = lane < MT && lane < M ? (mx ? (uint32_t)mx[(size_t)lane * G + g] : 1u) : 0u;
    };
    v16i biasv;
#pragma unroll
    for (int r = 0; r < 16; r++) biasv[r] = (int)PF_BIAS;
    auto compute = [&](const int8_t* xd, const uint32_t* w, uint32_t mr, uint32_t mxl, int slot) __attribute__((always_inline)) {
        uint32_t* mxw = mxs_s[wv];
        if (lane < MT) mxw[lane] = mxl;          // read back below by this wave only (LDS operations stay in order)
        if (hf == 0 && lane < MT) {
            xdig[(0 * MT + lane) * NS + slot] = (int8_t)(mxl & 127);
            xdig[(1 * MT + lane) * NS + slot] = (int8_t)((mxl >> 7) & 127);
            xdig[(2 * MT + lane) * NS + slot] = (int8_t)(mxl >> 14);
        }
        if (e == 0) {
            wdig[(0 * 64 + row) * NS + slot] = (int8_t)(mr & 127);
            wdig[(1 * 64 + row) * NS + slot] = (int8_t)((mr >> 7) & 127);
            wdig[(2 * 64 + row) * NS + slot] = (int8_t)(mr >> 14);
        }
#pragma unroll
        for (int t = 0; t < TS; t++) {
            const int R = 32 * t + l32;          // this lane's A row (token)
            v16i d = biasv;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const v4i xa = *reinterpret_cast<const v4i*>(xd + R * 128 + (((4 * e + s) ^ ((R >> 1) & 7)) << 4));
                const v4i bw = {(int)w[4 * s], (int)w[4 * s + 1], (int)w[4 * s + 2], (int)w[4 * s + 3]};
                d = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, bw, d, 0, 0, 0);
            }
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const uint4 mv = *reinterpret_cast<const uint4*>(mxw + 32 * t + 8 * qq + 4 * e);
                const uint32_t mxv[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
                for (int j = 0; j < 4; j++)
                    U[t][4 * qq + j] += (unsigned long long)(uint32_t)d[4 * qq + j] * mul_u24(mr, mxv[j]);
            }
        }
    };

    int g = g0 + pr;
    if (g < g1) fetch(g, area(0));
    for (int it = 0; it < rounds; it++, g += P) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");     // this wave's copies and loads for round it have landed
        __syncthreads();                                      // ... and the other waves' copies
        uint32_t w[16];
#pragma unroll
        for (int b = 0; b < 2; b++) block_signed<BITS>(q + b * NC, w + 8 * b);
        const uint32_t mr = m_n, mxl = mxl_n;
        if (g + P < g1) fetch(g + P, area((it + 1) & 1));   // the next round's loads run under this compute
        if (g < g1) compute(area(it & 1), w, mr, mxl, g - g0);
    }
    if (wv == 0 && lane < MT) sxs_s[lane] = sxl;
    __syncthreads();                                          // digits staged, activation areas free
    // U -= B * S for block (row half hf, token set t) where t % P == pr:
    // S = sum_{i,j} 2^(7 (i + j)) D_ij, D_ij = sum over slots of digit i of mx times digit j of m
#pragma unroll
    for (int t = 0; t < TS; t++) {
        if (t % P != pr) continue;               // compile-time t: U is indexed by constants only
        for (int k0 = 0; k0 < NS; k0 += 32) {
            v4i A[3], Bd[3];
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const int4 av = *reinterpret_cast<const int4*>(xdig + (i * MT + 32 * t + l32) * NS + k0 + 16 * e);
                const int4 bv = *reinterpret_cast<const int4*>(wdig + (i * 64 + row) * NS + k0 + 16 * e);
                const int s0 = k0 + 16 * e;
                A[i][0] = mask_slots(av.x, s0, ng); A[i][1] = mask_slots(av.y, s0 + 4, ng);
                A[i][2] = mask_slots(av.z, s0 + 8, ng); A[i][3] = mask_slots(av.w, s0 + 12, ng);
                Bd[i][0] = mask_slots(bv.x, s0, ng); Bd[i][1] = mask_slots(bv.y, s0 + 4, ng);
                Bd[i][2] = mask_slots(bv.z, s0 + 8, ng); Bd[i][3] = mask_slots(bv.w, s0 + 12, ng);
            }
            const v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            const v16i d4 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[2], z, 0, 0, 0);
            v16i d3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[1], z, 0, 0, 0);
            d3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[2], d3, 0, 0, 0);
            v16i d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[0], z, 0, 0, 0);
            d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[1], d2, 0, 0, 0);
            d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[2], d2, 0, 0, 0);
            v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[0], z, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[1], d1, 0, 0, 0);
            const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[0], z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // d4 < 2^9, d3 < 2^15, d2, d1 < 2^20, d0 < 2^19 (32 slots): S = hi 2^14 + lo with
                // hi = (d4 2^7 + d3) 2^7 + d2 < 2^25 and lo = d1 2^7 + d0 < 2^28, one v_mad_u64_u32
                const uint32_t hi = ((((uint32_t)d4[r] << 7) + (uint32_t)d3[r]) << 7) + (uint32_t)d2[r];
                const uint32_t lo = ((uint32_t)d1[r] << 7) + (uint32_t)d0[r];
                const unsigned long long S = (unsigned long long)hi * 16384u + lo;
                U[t][r] -= S << 21;
            }
        }
    }
    // sums of the workgroup: tot[t][row], pair 0 writes, the others add
    long long* tot = reinterpret_cast<long long*>(xs_dyn);
    if (pr == 0) {
#pragma unroll
        for (int t = 0; t < TS; t++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                tot[(32 * t + 8 * (r >> 2) + 4 * e + (r & 3)) * 64 + row] = (long long)U[t][r];
    }
    __syncthreads();
    if (pr > 0) {
#pragma unroll
        for (int t = 0; t < TS; t++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                __hip_atomic_fetch_add(tot + (32 * t + 8 * (r >> 2) + 4 * e + (r & 3)) * 64 + row, (long long)U[t][r],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    // thread (wave w, lane) finishes tokens w + W i of row n (W = 2 or 4: at most MT / 2 of them), every load
    // before the first conversion, every conversion before the first store
    constexpr int EI = MT / 2;
    const int mt = min(M, MT);
    long long v[EI];
#pragma unroll
    for (int i = 0; i < EI; i++) {
        const int t = wv + W * i;
        v[i] = t < mt ? tot[t * 64 + lane] : 0;
    }
    if (KS > 1) {
        const size_t npad = (size_t)(gridDim.x / KS) * TILE_N;
        part += (size_t)tbk * KS * MT * npad;                  // this token block's planes
        cnt += (size_t)tbk * (gridDim.x / KS);                 // and counters
        long long* mine = part + (size_t)ks * MT * npad;
#pragma unroll
        for (int i = 0; i < EI; i++) {
            const int t = wv + W * i;
            if (t < mt) __hip_atomic_store(mine + (size_t)t * npad + n, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        wait_performed();             // this wave's stores have been performed
        __syncthreads();
        if (threadIdx.x == 0)
            last_s = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(KS - 1);
        __syncthreads();
        if (!last_s) return;
        for (int k = 0; k < KS; k++) {
            if (k == ks) continue;
            const long long* other = part + (size_t)k * MT * npad;
            long long o[EI];
#pragma unroll
            for (int i = 0; i < EI; i++) {
                const int t = wv + W * i;
                o[i] = t < mt ? __hip_atomic_load(other + (size_t)t * npad + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
            }
#pragma unroll
            for (int i = 0; i < EI; i++) v[i] += o[i];
        }
        if (threadIdx.x == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float f[EI];
#pragma unroll
    for (int i = 0; i < EI; i++) {
        const int t = wv + W * i;
        f[i] = (i64_to_f_fast(v[i]) * cn) * sxs_s[t < MT ? t : 0];
    }
    if (n >= N) return;
    if (!out.acc && out.nparts <= 1) {
#pragma unroll
        for (int i = 0; i < EI; i++) {
            const int t = wv + W * i;
            if (t < mt) out.y[(size_t)(t0 + t) * N + n] = f[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < EI; i++) {
            const int t = wv + W * i;
            if (t < mt) out.store(N, t0 + t, n, f[i]);
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
int g_decode_max_m = 16;
// The scratch registered with det_gemm_set_scratch (the reference's per-(token, group) activation-sum buffer,
// gemm.cu:913-936).  This backend's kernels need no caller scratch: the pointer is kept for the ABI only.
void* g_user_scratch = nullptr;
size_t g_user_scratch_bytes = 0;

// K-split buffers of k_decode: int64 accumulators part[MP][Npad] and per-tile arrival counters, zero between calls
// (the last workgroup of each tile clears what it used); library-owned, grown on demand.  Calls that overlap on
// different streams would share them: det runs every call on one in-order stream.  The zero-between-calls invariant
// holds only while every launch completes: a kernel that faults part-way leaves counts behind, which is why such a
// fault is fatal (det_sync and DET_CHECK abort) rather than something a caller recovers from and calls again.
// These buffers are the library's own and are not counted by det_allocated_bytes.
long long* g_part = nullptr;
size_t g_part_cap = 0;              // elements
unsigned int* g_cnt = nullptr;
size_t g_cnt_cap = 0;

void decode_buffers(size_t part_elems, size_t tiles, hipStream_t st) {
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

template <int BITS, int MP, bool SILU0 = false>
void launch_decode(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    const int G = L.K / GROUP;
    const int T = (L.N + TILE_N - 1) / TILE_N;
    // K-split only when the tiles cannot occupy half the CUs: the split's combine costs three dependent memory round
    // trips, which a launch that already fills the device does not repay.
    const int cus = g_decode_waves / 8;
    int KS = 1;
    if (2 * T < cus) KS = std::max(1, std::min((cus + T - 1) / T, (G + 3) / 4));
    const int gs = (G + KS - 1) / KS;
    int S = (g_decode_waves + T * KS - 1) / (T * KS);
    S = std::max(1, std::min(S, std::min(gs, std::min(dec_maxw<MP>(), 128 / MP))));     // LDS: S * MP * 512 <= 64 KB
    long long* part = nullptr;
    unsigned int* cnt = nullptr;
    if (KS > 1) {
        decode_buffers((size_t)MP * T * TILE_N, (size_t)T, st);
        part = g_part;
        cnt = g_cnt;
    }
    const size_t lds = S > 1 ? (size_t)S * MP * 64 * sizeof(long long) : 0;
    k_decode<BITS, MP, SILU0><<<T * KS, 64 * S, lds, st>>>(L.wq, L.c, L.m, L.N, L.K, xq, sx, mx, M, y, KS, part, cnt);
    DET_CHECK(hipGetLastError());
}

// K-slice partial sums of k_decode_ms and k_prefill2: part[KS][tokens][Npad] int64 (each slice stores its own
// plane, so nothing needs zeroing); library-owned, grown on demand
long long* g_part_ks = nullptr;
size_t g_part_ks_cap = 0;
long long* partial_buffer(size_t elems, hipStream_t st) {
    if (elems > g_part_ks_cap) {
        DET_CHECK(hipStreamSynchronize(st));     // earlier launches may still use the old buffer
        if (g_part_ks) DET_CHECK(hipFree(g_part_ks));
        g_part_ks_cap = std::max(elems, (size_t)1 << 20);
        DET_CHECK(hipMalloc(&g_part_ks, g_part_ks_cap * 8));
    }
    return g_part_ks;
}

// K-slices of k_decode_ms for `units` (tile, token block) pairs: until every CU has a workgroup, each slice keeping
// at least 16 groups (the slices' combine costs about as much as a few rounds) and at most DMS_MAXSLOT
int dms_slices(int units, int G) {
    const int cus = g_decode_waves / 8;
    int KS = units >= cus ? 1 : std::max(1, std::min((cus + units - 1) / units, G / 16));
    KS = std::max(KS, (G + DMS_MAXSLOT - 1) / DMS_MAXSLOT);
    const int gs = (G + KS - 1) / KS;
    return (G + gs - 1) / gs;                    // no empty slices
}

template <int BITS, int TS>
void launch_decode_ms(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    constexpr int MT = 32 * TS;
    const int G = L.K / GROUP;
    const int T = (L.N + TILE_N - 1) / TILE_N;
    const int NB = (M + MT - 1) / MT;            // token blocks (grid y)
    const int units = T * NB;
    const int cus = g_decode_waves / 8;
    const int KS = dms_slices(units, G);
    const int gs = (G + KS - 1) / KS;
    // four pairs when every workgroup has a CU of its own, else two (two workgroups share a CU, one's prologue and
    // epilogue overlapping the other's rounds)
    const int P = std::min(units * KS <= cus ? DMS_MAXP : 2, gs);
    long long* part = nullptr;
    unsigned int* cnt = nullptr;
    if (KS > 1) {
        part = partial_buffer((size_t)NB * KS * MT * T * TILE_N, st);
        decode_buffers(0, (size_t)units, st);    // arrival counters (shared with k_decode: zero between calls)
        cnt = g_cnt;
    }
    const int NS = (gs + 31) & ~31;
    const size_t lds = std::max((size_t)2 * P * MT * 128, (size_t)MT * TILE_N * 8) + (size_t)3 * (64 + MT) * NS;
    k_decode_ms<BITS, TS><<<dim3(T * KS, NB), 128 * P, lds, st>>>(L.wq, L.c, L.m, L.N, L.K, xq, sx, mx, M, y, KS, part, cnt);
    DET_CHECK(hipGetLastError());
}

template <int BITS>
void gemm_bits(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y, hipStream_t st) {
    if (M <= g_decode_max_m) {
        if (M <= 1) launch_decode<BITS, 1>(L, xq, sx, mx, M, y, st);
        else if (M <= 4) launch_decode<BITS, 4>(L, xq, sx, mx, M, y, st);
        else if (M <= 8) launch_decode<BITS, 8>(L, xq, sx, mx, M, y, st);
        else launch_decode<BITS, 16>(L, xq, sx, mx, M, y, st);
    } else if (M <= 64) {
        // 33..64 tokens: one 64-token block per tile, or two 32-token blocks (each unpacking the tile's codes for
        // half the tokens) when that gives more workgroups than the K-slices of the 64-token blocks do
        const int T = (L.N + TILE_N - 1) / TILE_N, G = L.K / GROUP;
        const bool split = M > 32 && 2 * T * dms_slices(2 * T, G) > T * dms_slices(T, G);
        if (M <= 32 || split) launch_decode_ms<BITS, 1>(L, xq, sx, mx, M, y, st);
        else launch_decode_ms<BITS, 2>(L, xq, sx, mx, M, y, st);
    } else if (!prefill_gemm(L, xq, sx, mx, M, y, g_decode_waves / 8, st)) {
        // shapes outside the prefill kernel (K >= 131072 or M * K >= 2^31): 16-token slices of the decode kernel
        const int G = L.K / GROUP;
        for (int t = 0; t < M; t += 16)
            launch_decode<BITS, 16>(L, xq + (size_t)t * L.K, sx + t, mx ? mx + (size_t)t * G : nullptr, std::min(16, M - t),
                                    y.rows_from(L.N, t), st);
    }
}

} // namespace

extern "C" {

void det_linear_sizes(int N, int K, int bits, size_t* wq_bytes, size_t* c_bytes, size_t* m_bytes) {
    if (K <= 0 || K % GROUP || N <= 0) DET_FAIL("det_linear_sizes: bad shape N=%d K=%d", N, K);
    if (bits != 4 && bits != 6 && bits != 8) DET_FAIL("det_linear_sizes: unsupported bits=%d", bits);
    // whole 128-row blocks (pairs of 64-row tiles): the prefill kernel reads weight tiles two at a time
    const size_t T = 2 * (((size_t)N + 2 * TILE_N - 1) / (2 * TILE_N)), G = (size_t)K / GROUP;
    // the decode tiles, then (only when the stream-K prefill kernel is selected) the prefill planes: the same size,
    // 32-row blocks of the same row pairs
    if (wq_bytes) *wq_bytes = (use_streamk() ? 2 : 1) * T * G * group_bytes(bits) * TILE_N;
    if (c_bytes) *c_bytes = T * TILE_N * 4;
    if (m_bytes) *m_bytes = T * G * TILE_N * 2;
}

void det_linear_repack(const uint8_t* rows, int N, int K, int bits, uint8_t* wq, float* c, uint16_t* m, hipStream_t st) {
    det_linear_sizes(N, K, bits, nullptr, nullptr, nullptr);     // validates the shape
    // the decode tiles only: k_repack also writes c and m for every tile it visits, and those planes cover the
    // decode tiles (the prefill planes that follow in wq are written by prefill_repack)
    const size_t nchunks = pf_offset(N, K, bits) / 16;
    const size_t blocks = std::min<size_t>((nchunks + 255) / 256, 65536);
    k_repack<<<(unsigned)blocks, 256, 0, st>>>(rows, N, K, bits, wq, c, m, nchunks);
    DET_CHECK(hipGetLastError());
    if (use_streamk()) prefill_repack(rows, N, K, bits, wq, st);
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

namespace det {

void gemm_parts_silu0(const det_qlinear* Lp, const int8_t* xq, const float* sx, const uint16_t* mx, int nparts,
                      const int* offs, float* const* dsts, hipStream_t st) {
    const det_qlinear L = *Lp;
    if (nparts < 2 || nparts > 4 || offs[0] != 0) DET_FAIL("det_gemm: silu of part 0 needs 2 to 4 parts from column 0");
    if (L.K % GROUP != 0 || L.K <= 0 || L.N <= 0) DET_FAIL("det_gemm: bad shape N=%d K=%d", L.N, L.K);
    if (L.bits != 4 && L.bits != 6 && L.bits != 8) DET_FAIL("det_gemm: unsupported bits=%d", L.bits);
    if (g_num_cus == 0) {
        int dev = 0;
        DET_CHECK(hipGetDevice(&dev));
        DET_CHECK(hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_decode_waves = 8 * g_num_cus;
    }
    Out out;
    memset(&out, 0, sizeof out);
    out.nparts = nparts;
    for (int i = 0; i < nparts; i++) { out.dst[i] = dsts[i]; out.offs[i] = offs[i]; }
    out.offs[nparts] = L.N;
    switch (L.bits) {                              // one token: the GEMV, whose epilogue goes through Out::store
        case 8: launch_decode<8, 1, true>(L, xq, sx, mx, 1, out, st); break;
        case 6: launch_decode<6, 1, true>(L, xq, sx, mx, 1, out, st); break;
        default: launch_decode<4, 1, true>(L, xq, sx, mx, 1, out, st); break;
    }
}

} // namespace det
