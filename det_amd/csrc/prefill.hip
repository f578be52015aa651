// det quantized GEMM for many tokens (M > 64) on gfx950 (MI355X), bit-exact to the spec (reference
// docs/SPEC.md:56-64, crates/det/src/spec/quant.rs:102-117):
//   acc[t][n] = sum_g ( m[n][g] * mx[t][g] ) * sum_{k in group g} wq[n][k] * xq[t][k]     (exact integers)
//   y[t][n]   = ((float)acc[t][n] * c[n]) * sx[t]
// The reference runs this shape on k_mma2 + k_xsum (kernels/cuda/gemm.cu:672-1023); the design here is this
// backend's own.
//
// Work: the output is cut into 128-token x 128-row tiles; a tile's 128-groups along K are its units.  A persistent
// grid of two workgroups per CU takes equal contiguous runs of units (stream-K), so every CU gets the same work
// whatever the tile count.  A tile split between workgroups is finished by the last one to arrive, which adds the
// others' exact int64 partial tiles.
//
// Workgroup: 4 waves; wave w owns 32 weight rows for all 128 tokens of the tile.  Per 128-group:
//   - the activations (128 tokens x 128 bytes) arrive in LDS by the buffer unit, two groups ahead (3 stages);
//   - each lane loads its row's codes for the group straight into registers (the prefill planes below), one group
//     ahead, and unpacks them with 1-2 VALU ops per 4 codes;
//   - 16 v_mfma_i32_32x32x32_i8 per wave: A = the wave's 32 rows of codes (registers), B = 32 tokens of activations
//     (LDS); the 32x32 result holds (row, token) with lane = token, register = row;
//   - group scaling into int64: U += (p + B) * (m * mx), one v_mul_u32_u24 and one v_mad_u64_u32 per element.
//     Every chain starts from the bias B = 2^21 so that p + B >= 0; the bias is removed every 32 groups from
//     S = sum_g m * mx, computed exactly on the matrix core from 7-bit digits staged in LDS (9 MFMAs per 32x32 block).
//
// Prefill planes (written by det_linear_repack after the decode tiles): per 32-row block b and group g, NP planes of
// [64 lanes][16 bytes].  Lane l = row b*32 + l%32, half h = l/32, holds the row's 64 codes c_i of k = 32*(i/16) +
// 16h + i%16 (i < 64): exactly the bytes of the MFMA A operand of the four 32-k steps, in a packing that unpacks to
// codes scaled by 2^SH (two's complement in the high bits of each byte):
//   W8 (NP 4, SH 0): the int8 codes.
//   W6 (NP 3, SH 2): per step three words D0..D2; byte j of Di = (c[4i+j] & 63) << 2 | spare, where the spare bits
//       of D0, D1, D2 are bits 5:4, 3:2, 1:0 of c[12+j].  Unpack: Di & 0xfcfcfcfc (i < 3) and the spares assembled.
//   W4 (NP 2, SH 4): per step two words; byte j of Ni = (c[8i+j] & 15) << 4 | (c[8i+4+j] & 15).  Unpack: Ni &
//       0xf0f0f0f0 and (Ni << 4) & 0xf0f0f0f0.
// Scaled codes keep |p| <= 128 * 127 * 128 < 2^21 at every width, and U = 2^SH * acc exactly.
#include <string.h>
#include <algorithm>
#include "common.h"
#include "gemm_common.h"
#include "gemm_internal.h"

namespace det {
namespace {

constexpr int PF_BM = 128;        // tokens per tile
constexpr int PF_BN = 128;        // rows per tile (four waves of 32)
constexpr int PF_STG = 3;         // activation stages in LDS
constexpr int PF_SLOTS = 32;      // groups per bias-correction batch
constexpr int PF_TILE = PF_BM * PF_BN;

template <int BITS> constexpr int pf_planes() { return BITS == 8 ? 4 : BITS == 6 ? 3 : 2; }
template <int BITS> constexpr int pf_shift() { return BITS == 8 ? 0 : BITS == 6 ? 2 : 4; }

// signed code of k (0 <= k < 128) in one row's packed 128-group of the det format (spec/quant.rs:63-97)
__device__ __forceinline__ int det_code(const uint8_t* grp, int bits, int k) {
    const int b = k >> 5, j = k & 31;
    if (bits == 8) return (int)(int8_t)grp[b * 32 + j];
    if (bits == 4) {
        const uint8_t v = grp[b * 16 + (j & 15)];
        return (j < 16 ? (v & 15) : (v >> 4)) - 8;
    }
    const uint8_t v = grp[b * 24 + (j & 15)];
    const int lo = j < 16 ? (v & 15) : (v >> 4);
    const int hi = (grp[b * 24 + 16 + (j & 7)] >> (2 * (j >> 3))) & 3;
    return (lo | hi << 4) - 32;
}

// One work item per (32-row block, group, lane): writes the lane's NP 16-byte words of the prefill planes.
__global__ void k_repack_pf(const uint8_t* __restrict__ rows, int N, int K, int bits, uint8_t* __restrict__ pw, size_t items) {
    const int G = K / GROUP, NP = bits == 8 ? 4 : bits == 6 ? 3 : 2;
    const size_t rb = (size_t)K / 32 * bpl(bits) + 4 + 2 * (size_t)G;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < items; idx += (size_t)gridDim.x * blockDim.x) {
        const int l = (int)(idx & 63), r = l & 31, h = l >> 5;
        const size_t bg = idx >> 6;
        const int g = (int)(bg % G);
        const size_t blk = bg / G;
        const size_t n = blk * 32 + r;
        int c[64];
#pragma unroll 4
        for (int i = 0; i < 64; i++)
            c[i] = n < (size_t)N ? det_code(rows + n * rb + (size_t)g * group_bytes(bits), bits, 32 * (i >> 4) + 16 * h + (i & 15)) : 0;
        uint32_t q[16];
        for (int s = 0; s < 4; s++) {
            const int* cs = c + 16 * s;
            if (bits == 8) {
                for (int d = 0; d < 4; d++)
                    q[4 * s + d] = (uint32_t)(cs[4 * d] & 255) | (uint32_t)(cs[4 * d + 1] & 255) << 8 |
                                   (uint32_t)(cs[4 * d + 2] & 255) << 16 | (uint32_t)(cs[4 * d + 3] & 255) << 24;
            } else if (bits == 6) {
                for (int i = 0; i < 3; i++) {
                    uint32_t wv = 0;
                    for (int j = 0; j < 4; j++) {
                        const int spare = (cs[12 + j] >> (4 - 2 * i)) & 3;
                        wv |= (uint32_t)(((cs[4 * i + j] & 63) << 2) | spare) << (8 * j);
                    }
                    q[3 * s + i] = wv;
                }
            } else {
                for (int i = 0; i < 2; i++) {
                    uint32_t wv = 0;
                    for (int j = 0; j < 4; j++)
                        wv |= (uint32_t)(((cs[8 * i + j] & 15) << 4) | (cs[8 * i + 4 + j] & 15)) << (8 * j);
                    q[2 * s + i] = wv;
                }
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(pw + bg * (size_t)NP * 1024) + l;
        for (int p = 0; p < NP; p++) dst[p * 64] = make_uint4(q[4 * p], q[4 * p + 1], q[4 * p + 2], q[4 * p + 3]);
    }
}

// the MFMA A operands of the four 32-k steps from a lane's prefill words (codes scaled by 2^SH)
template <int BITS> __device__ __forceinline__ void pf_unpack(const v4i* q, v4i* a);
template <> __device__ __forceinline__ void pf_unpack<8>(const v4i* q, v4i* a) {
    // the codes are the operands; copied by asm (the next group's loads reuse q while the MFMAs read a), so that the
    // copy stays behind the wait, which a plain assignment the compiler could place anywhere would not
    typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const u64x2 in = __builtin_bit_cast(u64x2, q[s]);
        unsigned long long lo, hi;
        asm volatile("v_mov_b64 %0, %2\n\tv_mov_b64 %1, %3" : "=v"(lo), "=v"(hi) : "v"(in.x), "v"(in.y));
        a[s] = __builtin_bit_cast(v4i, u64x2{lo, hi});
    }
}
template <> __device__ __forceinline__ void pf_unpack<6>(const v4i* q, v4i* a) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(q);
    constexpr uint32_t HI = 0xfcfcfcfcu, LO = 0x03030303u;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t d0 = w[3 * s], d1 = w[3 * s + 1], d2 = w[3 * s + 2];
        const uint32_t sp = ((((d0 & LO) << 2) | (d1 & LO)) << 2 | (d2 & LO)) << 2;
        a[s] = v4i{(int)(d0 & HI), (int)(d1 & HI), (int)(d2 & HI), (int)sp};
    }
}
template <> __device__ __forceinline__ void pf_unpack<4>(const v4i* q, v4i* a) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(q);
    constexpr uint32_t HI = 0xf0f0f0f0u;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t n0 = w[2 * s], n1 = w[2 * s + 1];
        a[s] = v4i{(int)(n0 & HI), (int)((n0 << 4) & HI), (int)(n1 & HI), (int)((n1 << 4) & HI)};
    }
}

// byte offset of chunk c (16 bytes) of token row r in a 128-byte-row activation stage; chunk position c ^ ((r/2) % 8)
// puts the 16 rows that one LDS cycle serves on 16 distinct 16-byte bank slots
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Loads issued as inline assembly, so that the compiler places no wait for them; every use of a destination comes
// after an explicit s_waitcnt that names the register (pf_wait), which also orders the use after the wait.
template <int OFF>
__device__ __forceinline__ void ld16(v4i& d, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:%4" : "=v"(d) : "v"(voff), "s"(r), "s"(soff), "i"(OFF) : "memory");
}
__device__ __forceinline__ void ld_u16(uint32_t& d, __amdgpu_buffer_rsrc_t r, uint32_t voff) {
    asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(d) : "v"(voff), "s"(r) : "memory");
}
// wait until at most KEEP vector-memory operations of this wave are outstanding, then hand the loaded registers to
// the code that follows: the asm claims to modify them, so no use of them can move above the wait.  This holds only
// if the registers reach the asm where the loads put them (a copy placed before the asm would read them early):
// every iteration of the group loop issues the same loads and waits the same way, so that no path merges loaded and
// not-loaded values, and tests/test_isa_waits.py proves it on the generated code.
template <int NP, int KEEP>
__device__ __forceinline__ void pf_wait(v4i* q, uint32_t& s) {
    if constexpr (NP == 4)
        asm volatile("s_waitcnt vmcnt(%5)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(s) : "i"(KEEP) : "memory");
    else if constexpr (NP == 3)
        asm volatile("s_waitcnt vmcnt(%4)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(s) : "i"(KEEP) : "memory");
    else
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(q[0]), "+v"(q[1]), "+v"(s) : "i"(KEEP) : "memory");
}
__device__ __forceinline__ void pf_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// store four consecutive outputs (columns n .. n + 3 of token t) through the output routing
__device__ __forceinline__ void store4(const Out& out, int N, int M, int t, int n, const float4& v) {
    if (t >= M) return;
    float* base;
    int lo = 0, width = N;
    if (out.nparts <= 1) {
        base = out.y;
    } else {
        base = out.dst[0];
        int hi = out.offs[1];
#pragma unroll
        for (int j = 1; j < 4; j++)
            if (j < out.nparts && n >= out.offs[j]) { base = out.dst[j]; lo = out.offs[j]; hi = out.offs[j + 1]; }
        width = hi - lo;
    }
    float* p = base + (size_t)t * width + (n - lo);
    const bool vec = n - lo + 4 <= width && ((n - lo) & 3) == 0 && (width & 3) == 0 && (((size_t)base & 15) == 0);
    if (vec) {
        float4* p4 = reinterpret_cast<float4*>(p);
        if (out.acc) {
            const float4 o = *p4;
            *p4 = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        } else {
            *p4 = v;
        }
        return;
    }
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (n + e < N) out.store(N, t, n + e, vv[e]);
}

// The WG that owns unit u of `total` units split evenly over P workgroups: u0(w) = floor(w * total / P).
__device__ __forceinline__ int pf_owner(long long u, long long total, int P) {
    return (int)(((u + 1) * P + total - 1) / total) - 1;
}

template <int BITS>
__global__ void __launch_bounds__(256, 2) k_prefill(const uint8_t* __restrict__ pw, const float* __restrict__ cs,
                                                     const uint16_t* __restrict__ ms, int N, int K,
                                                     const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                     const uint16_t* __restrict__ mx, int M, Out out, int nbt,
                                                     int tiles, int P, long long* __restrict__ part,
                                                     unsigned int* __restrict__ cnt) {
    constexpr int NP = pf_planes<BITS>(), SH = pf_shift<BITS>();
    __shared__ __attribute__((aligned(16))) int8_t As[PF_STG][PF_BM * 128];
    // multipliers by group parity: entries 0-127 m of the tile's rows, 128-255 mx of its tokens; thread tid stages
    // entry tid, so its slot address is a function of tid alone (no per-thread base register to keep alive)
    __shared__ __attribute__((aligned(16))) uint32_t sv_s[2][PF_BN + PF_BM];
    // their 7-bit digits for the bias removal, [digit][entry as in sv_s][group slot]
    __shared__ __attribute__((aligned(16))) uint8_t dig[3][PF_BN + PF_BM][PF_SLOTS];
    __shared__ unsigned int last_s;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K / GROUP;
    const int nbn = tiles / nbt;
    const long long total = (long long)tiles * G;
    // logical workgroup: consecutive ids on one XCD (workgroups are dealt to the 8 XCDs round robin), so the token
    // tiles that share a weight tile, and the workgroups that share a split tile, share an L2
    int w = blockIdx.x;
    if ((P & 7) == 0) w = (w & 7) * (P >> 3) + (w >> 3);
    const long long u0 = (long long)w * total / P, u1 = (long long)(w + 1) * total / P;

    v16i biasv;
#pragma unroll
    for (int r = 0; r < 16; r++) biasv[r] = (int)PF_BIAS;

    // staging role of this thread: waves 0-1 load m of tile row tid, waves 2-3 mx of tile token tid - 128
    const bool is_m = wv < 2;
    const int sidx = tid & 127;
    const bool x_one = !is_m && !mx;
    const __amdgpu_buffer_rsrc_t sres = is_m
        ? __builtin_amdgcn_make_buffer_rsrc((void*)ms, (short)0, nbn * 2 * G * 128, 0x00020000)
        : __builtin_amdgcn_make_buffer_rsrc((void*)(mx ? mx : ms), (short)0, mx ? M * G * 2 : 0, 0x00020000);
    const uint32_t sstride = is_m ? 128u : 2u;
    uint8_t* const dg = &dig[0][tid][0];                      // this thread's digit slots (planes 8 KB apart)
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, M * K, 0x00020000);
    // LDS byte offsets of this lane's B operands: token l32 (+ 32 j), chunk 2 s + h of the group
    uint32_t boff[4];
#pragma unroll
    for (int s = 0; s < 4; s++) boff[s] = (uint32_t)swz(l32, 2 * s + h);

    for (long long u = u0; u < u1;) {
        const int tile = (int)(u / G);
        const int ga = (int)(u - (long long)tile * G);
        const int gb = (int)std::min<long long>((long long)G, u1 - (long long)tile * G);
        u = (long long)tile * G + gb;
        const int nb = tile / nbt, tb = tile - nb * nbt;
        const int t0 = tb * PF_BM, n0 = nb * PF_BN;
        __syncthreads();                          // the previous fragment's readers of every LDS array are done

        unsigned long long U[4][16];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) U[j][r] = 0;

        // activations: copy i of wave wv takes tile tokens 32 wv + 8 i + lane / 8 into As[stage] + 4096 wv + 1024 i;
        // token row R's chunk c sits at position c ^ ((R / 2) % 8), so lane position p reads chunk p ^ (4 i + lane / 16)
        // % 8.  The copy's instruction offset 1024 i moves both addresses, so its per-lane offset is 1024 i short on
        // the global side; the range check (per-lane offset plus instruction offset against M rows) makes rows past
        // M read as zero.
        uint32_t avo[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            avo[i] = (uint32_t)(t0 + wv * 32 + 8 * i + (lane >> 3)) * (uint32_t)K - 1024u * i +
                     (uint32_t)(((lane & 7) ^ (((i & 1) << 2) | (lane >> 4))) * 16);
        auto issue_a = [&](int g, int stg) __attribute__((always_inline)) {
            dma16_run4v(xres, avo, g * GROUP, As[stg] + wv * 4096);
        };
        // codes: the wave's 32-row block
        const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(pw + (size_t)(nb * 4 + wv) * G * NP * 1024), (short)0, G * NP * 1024, 0x00020000);
        v4i qn[NP];
        auto issue_w = [&](int g) __attribute__((always_inline)) {
            const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)(g * NP * 1024));
            ld16<0>(qn[0], cr, lane * 16, soff);
            ld16<1024>(qn[1], cr, lane * 16, soff);
            if constexpr (NP > 2) ld16<2048>(qn[2], cr, lane * 16, soff);
            if constexpr (NP > 3) ld16<3072>(qn[3], cr, lane * 16, soff);
        };
        // multipliers: m of row n0 + sidx (layout [64-row tile][G][64]) or mx of token t0 + sidx
        const uint32_t s_vo = is_m ? (uint32_t)((((n0 + sidx) >> 6) * G * 64 + ((n0 + sidx) & 63)) * 2)
                                   : (uint32_t)((t0 + sidx) * G * 2);
        uint32_t sreg = 0;
        auto issue_s = [&](int g) __attribute__((always_inline)) { ld_u16(sreg, sres, s_vo + (uint32_t)g * sstride); };

        // prologue: group ga's multiplier into LDS; copies of ga and ga + 1, codes of ga.  Loads are issued for
        // every group position, the ones past the fragment's last group repeating that group (gl), so that every
        // iteration issues and waits alike: the group's wait always leaves exactly the newest four copies in flight.
        const int gl = gb - 1;
        issue_s(ga);
        pf_wait<NP, 0>(qn, sreg);
        uint32_t scur = x_one ? 1u : sreg;
        sv_s[0][tid] = scur;
        issue_a(ga, 0);
        issue_w(ga);
        issue_s(std::min(ga + 1, gl));
        issue_a(std::min(ga + 1, gl), 1);

        int stg = 0;
        for (int i = 0, g = ga; g < gb; i++, g++) {
            const int par = i & 1;
            // this group's copies, codes and the next group's multiplier have landed (the next group's copies may
            // still be in flight: they are the last four operations issued)
            pf_wait<NP, 4>(qn, sreg);
            __syncthreads();                      // ... in every wave; and group g - 1's readers are done
            const uint32_t snext = x_one ? 1u : sreg;
            if (g + 1 < gb) sv_s[par ^ 1][tid] = snext;
            const int slot = i & (PF_SLOTS - 1);
            if (slot == 0 && gb - g < PF_SLOTS) {  // a short last batch: clear this thread's slots
#pragma unroll
                for (int d = 0; d < 3; d++) {
                    uint4* p = reinterpret_cast<uint4*>(dg + d * (PF_BN + PF_BM) * PF_SLOTS);
                    p[0] = make_uint4(0, 0, 0, 0);
                    p[1] = make_uint4(0, 0, 0, 0);
                }
            }
            dg[slot] = (uint8_t)(scur & 127);
            dg[(PF_BN + PF_BM) * PF_SLOTS + slot] = (uint8_t)((scur >> 7) & 127);
            dg[2 * (PF_BN + PF_BM) * PF_SLOTS + slot] = (uint8_t)(scur >> 14);
            scur = snext;

            v4i a[4];
            pf_unpack<BITS>(qn, a);
            // loads for the next groups, the copies last (the wait above keeps exactly those in flight)
            issue_w(std::min(g + 1, gl));
            issue_s(std::min(g + 2, gl));
            issue_a(std::min(g + 2, gl), stg == 0 ? 2 : stg - 1);     // the stage group g - 1 used

            const int8_t* Ab = As[stg];
            uint32_t xm[4];
#pragma unroll
            for (int j = 0; j < 4; j++) xm[j] = sv_s[par][PF_BN + 32 * j + l32];
#pragma unroll
            for (int p = 0; p < 2; p++) {
                v16i d0 = biasv, d1 = biasv;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const v4i b0 = *reinterpret_cast<const v4i*>(Ab + boff[s] + 64 * p * 128);
                    const v4i b1 = *reinterpret_cast<const v4i*>(Ab + boff[s] + (64 * p + 32) * 128);
                    d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], b0, d0, 0, 0, 0);
                    d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], b1, d1, 0, 0, 0);
                }
                // element (row, token): lane = token, register 4 (row / 8) + row % 4 with (row / 4) % 2 = h
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const uint4 mq = *reinterpret_cast<const uint4*>(&sv_s[par][wv * 32 + 8 * q4 + 4 * h]);
                    const uint32_t mvv[4] = {mq.x, mq.y, mq.z, mq.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        U[2 * p][4 * q4 + e] += (unsigned long long)(uint32_t)d0[4 * q4 + e] * mul_u24(mvv[e], xm[2 * p]);
                        U[2 * p + 1][4 * q4 + e] += (unsigned long long)(uint32_t)d1[4 * q4 + e] * mul_u24(mvv[e], xm[2 * p + 1]);
                    }
                }
            }
            stg = stg == 2 ? 0 : stg + 1;

            // ---- bias removal every PF_SLOTS groups: S = sum_g m * mx from the digits v = d0 + 128 d1 + 16384 d2
            if (slot == PF_SLOTS - 1 || g + 1 == gb) {
                __syncthreads();                  // every thread's digits of this batch are in LDS
                v4i Ad[3];
#pragma unroll
                for (int d = 0; d < 3; d++) Ad[d] = *reinterpret_cast<const v4i*>(&dig[d][wv * 32 + l32][16 * h]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v4i Bd[3];
#pragma unroll
                    for (int d = 0; d < 3; d++) Bd[d] = *reinterpret_cast<const v4i*>(&dig[d][PF_BN + 32 * j + l32][16 * h]);
                    const v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                    // digit weights 2^28 (sum < 2^9), 2^21 (< 2^15), 2^14 (< 2^21), 2^7 (< 2^20): t stays below 2^32
                    v16i t = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[2], Bd[2], z, 0, 0, 0);
                    v16i e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[2], Bd[1], z, 0, 0, 0);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[1], Bd[2], e, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[2], Bd[0], z, 0, 0, 0);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[1], Bd[1], e, 0, 0, 0);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[0], Bd[2], e, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[1], Bd[0], z, 0, 0, 0);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[0], Bd[1], e, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
                    e = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ad[0], Bd[0], z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const unsigned long long S = ((unsigned long long)(uint32_t)t[r] << 7) + (uint32_t)e[r];
                        U[j][r] -= S << 21;
                    }
                }
            }
        }

        // the repeated loads of the last two iterations: their registers and LDS stage are free for reuse only once
        // they have landed, in every wave
        pf_drain();
        __syncthreads();

        // ---- a tile split between workgroups: every fragment but the last to arrive stores its exact partial
        // (agent-scope stores: coherent across the XCDs' L2s) and counts itself; the last adds the others
        if (ga != 0 || gb != G) {
            const long long tu = (long long)tile * G;
            const int wf = pf_owner(tu, total, P), wl = pf_owner(tu + G - 1, total, P);
            // slot of fragment (tile, workgroup v): 2 v for the workgroup's first fragment, 2 v + 1 for its last
            auto slot_of = [&](int v) __attribute__((always_inline)) {
                const int ft = (int)(((long long)v * total / P) / G);
                return (size_t)(2 * v + (ft == tile ? 0 : 1)) * PF_TILE;
            };
            long long* mine = part + slot_of(w);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    __hip_atomic_store(mine + ((wv * 4 + j) * 16 + r) * 64 + lane, (long long)U[j][r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            wait_performed();                      // this wave's stores have been performed
            __syncthreads();
            if (tid == 0)
                last_s = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(wl - wf);
            __syncthreads();
            if (!last_s) continue;
            for (int v = wf; v <= wl; v++) {
                if (v == w) continue;
                const long long* other = part + slot_of(v);
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        U[j][r] += (unsigned long long)__hip_atomic_load(other + ((wv * 4 + j) * 16 + r) * 64 + lane,
                                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }

        // ---- epilogue: y = (f32(acc) * c[n]) * sx[t], acc = U / 2^SH; transposed through a wave-private LDS tile
        // (32 tokens x 32 rows, rows padded to 36 floats) so that each store writes 4 consecutive columns
        float* Tt = reinterpret_cast<float*>(As[0]) + wv * (32 * 36);
        float cn[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int n = n0 + wv * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            cn[r] = n < N ? cs[n] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = t0 + 32 * j + l32;
            const float st = sx[min(t, M - 1)];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = 4 * q4 + e;
                    v[e] = (i64_to_f_fast((long long)U[j][r] >> SH) * cn[r]) * st;
                }
                *reinterpret_cast<float4*>(Tt + l32 * 36 + 8 * q4 + 4 * h) = make_float4(v[0], v[1], v[2], v[3]);
            }
            // the same wave reads back: LDS operations of one wave complete in order
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int tk = (lane >> 3) + 8 * k, c4 = (lane & 7) * 4;
                const float4 v = *reinterpret_cast<const float4*>(Tt + tk * 36 + c4);
                store4(out, N, M, t0 + 32 * j + tk, n0 + wv * 32 + c4, v);
            }
        }
    }
}

constexpr int P2_BM = 128;        // tokens per workgroup of k_prefill2

// ------------------------------------------------------------------ prefill, 128 x 64 tiles (M > 64)
// Workgroup tile 128 tokens x 64 rows (one weight tile), 4 waves of 32 tokens x 64 rows; up to three workgroups per
// CU (<= 168 VGPRs, <= 50 KB LDS), so a CU holds 12 waves whose MFMA chains, scaling and copy waits interleave.
// Per 128-group g (one round):
//   - every wave waits for its own copies and loads of round g and stages its multiplier; one barrier;
//   - W4/W6: each lane unpacks its 32-code block of group g + 1 (wave = block, lane = row; the packed bytes were
//     loaded into registers during the previous round) into the other half of the double-buffered signed tile Bs.
//     W8 needs no unpack: the MFMA reads its B operand straight from a double-buffered copy of the codes (tile
//     layout: plane c holds bytes 16 c .. 16 c + 15 of the 64 rows);
//   - the activations of group g + 1 are copied by the buffer unit into LDS (W8 also its codes), the multipliers
//     loaded into a register, W4/W6 group g + 2's packed block into registers;
//   - 8 v_mfma_i32_32x32x32_i8 (two chains from the bias B) and the scaling U += (p + B) * (m * mx).
// Group scaling with two VALU ops per (token, row, group): each group's MFMA chain starts from a constant
// accumulator B = 2^21, so the int32 result p + B is never negative (|p| <= 128*127*128 < 2^21) and
//     U += (p + B) * (m * mx)            (v_mul_u32_u24, v_mad_u64_u32; exact, U < 2^62)
// The bias is removed once per output, acc = U - B * S with S = sum_g m[n,g] * mx[t,g], computed exactly on the
// MFMA from unsigned 7-bit digits v = d0 + 128 d1 + 16384 d2 of m and mx, staged in LDS once per value:
//     S = sum_{i,j} 2^(7 (i + j)) D_ij,   D_ij = sum_g dx_i[t,g] dw_j[n,g]   (every D_ij >= 0, no offset terms).
template <int BITS>
__global__ void __launch_bounds__(256, 3) k_prefill2(const uint8_t* __restrict__ wq, const float* __restrict__ cs,
                                                      const uint16_t* __restrict__ ms, int N, int K,
                                                      const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                      const uint16_t* __restrict__ mx, int M,
                                                      Out out, int nbn, int nbt, int KS,
                                                      long long* __restrict__ part, unsigned int* __restrict__ cnt) {
    constexpr int NC = group_bytes(BITS) / 16;                 // 1 KB planes per tile-group
    constexpr int WB = NC * 1024;
    constexpr bool W8 = BITS == 8;    // W8: codes copied into a double-buffered staging tile the MFMA reads directly
    __shared__ __attribute__((aligned(16))) int8_t As[2][P2_BM * 128];
    __shared__ __attribute__((aligned(16))) int8_t Bp[2][W8 ? WB : 16];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][W8 ? 16 : TILE_N * 128];   // W4/W6: unpacked tiles
    __shared__ __attribute__((aligned(16))) uint32_t mxs[2][P2_BM];   // mx of the tile's tokens, per buffer
    __shared__ uint16_t mss[2][TILE_N];                                // m of the tile's rows, per buffer
    __shared__ unsigned int last_s;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wvu = __builtin_amdgcn_readfirstlane(wv);
    const int l32 = lane & 31, lh = lane >> 5;
    // XCD-aware order: consecutive workgroup ids go to different XCDs; each XCD gets a contiguous run of tiles,
    // token blocks innermost, so the token blocks that share a weight tile (and K-slice) share an L2
    int tile = blockIdx.x;
    const int total = nbn * nbt * KS;
    if ((total & 7) == 0) tile = (tile & 7) * (total >> 3) + (tile >> 3);
    const int nb = tile / (nbt * KS), rem = tile - nb * (nbt * KS), ks = rem / nbt, tb = rem - ks * nbt;
    const int t0 = tb * P2_BM, n0 = nb * TILE_N;
    const int G = K / GROUP;
    const int gs = (G + KS - 1) / KS;                          // groups of this workgroup's K-slice: [g0, g1)
    const int g0 = ks * gs, g1 = min(G, g0 + gs);

    unsigned long long U[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) U[j][r] = 0;
    v16i biasv;
#pragma unroll
    for (int r = 0; r < 16; r++) biasv[r] = (int)PF_BIAS;

    // activations: copy i of wave wv takes rows t0 + 32 wv + 8 i + lane / 8 into As + 4096 wv + 1024 i, row R's chunk
    // c at position c ^ ((R / 2) % 8); copy i reads through its own resource (based 8 i rows on, minus the 1 KB
    // instruction offset) whose range ends at row M, so rows past M read as zero
    __amdgpu_buffer_rsrc_t xr[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        xr[i] = __builtin_amdgcn_make_buffer_rsrc((void*)(xq + (size_t)i * 8 * K - 1024 * i), (short)0,
                                                  M > 8 * i ? (M - 8 * i) * K + 1024 * i : 0, 0x00020000);
    const uint32_t a_vo = (uint32_t)(t0 + wv * 32 + (lane >> 3)) * (uint32_t)K + (uint32_t)(((lane & 7) ^ (lane >> 4)) * 16);
    const uint32_t a_vo1 = a_vo ^ 64u;
    // W8 codes: the tile-group is WB contiguous bytes; wave w copies planes 2 w, 2 w + 1
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)(wq + (size_t)nb * G * WB), (short)0, G * WB, 0x00020000);
    const uint32_t w_vo[2] = {(uint32_t)lane * 16, (uint32_t)lane * 16};
    // W4/W6 codes: wave w = block b (32 codes), lane = row r: bytes BPL b .. BPL b + BPL - 1 of the row's group,
    // loaded into registers two groups ahead of their use (W4 plane b; W6 16 bytes of plane 3 (b / 2) + 2 (b % 2)
    // and 8 bytes of plane 3 (b / 2) + 1 at byte 8 (b % 2), the odd blocks' low words starting with the latter)
    const uint8_t* wcodes = wq + (size_t)nb * G * WB + lane * 16;
    uint32_t qn[6];
    auto load_w = [&](int g) __attribute__((always_inline)) {
        const uint8_t* p = wcodes + (size_t)g * WB;
        if constexpr (BITS == 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + wvu * 1024);
            qn[0] = v.x; qn[1] = v.y; qn[2] = v.z; qn[3] = v.w;
        } else if constexpr (BITS == 6) {
            const int pp = 3 * (wvu >> 1);
            const uint4 v = *reinterpret_cast<const uint4*>(p + (pp + 2 * (wvu & 1)) * 1024);
            const uint2 w = *reinterpret_cast<const uint2*>(p + (pp + 1) * 1024 + 8 * (wvu & 1));
            qn[0] = v.x; qn[1] = v.y; qn[2] = v.z; qn[3] = v.w; qn[4] = w.x; qn[5] = w.y;
        }
    };
    // unpack the registers' block into the signed tile bs (row lane, chunks 2 b and 2 b + 1); the W6 reorder of odd
    // blocks happens here, not at the load, so no wait for the load is placed early
    auto unpack_to = [&](int8_t* bs) __attribute__((always_inline)) {
        uint32_t o[8];
        if constexpr (BITS == 6) {
            const bool odd = wvu & 1;
            const uint32_t w6[6] = {odd ? qn[4] : qn[0], odd ? qn[5] : qn[1], odd ? qn[0] : qn[2],
                                    odd ? qn[1] : qn[3], odd ? qn[2] : qn[4], odd ? qn[3] : qn[5]};
            block_signed<6>(w6, o);
        } else {
            block_signed<W8 ? 4 : BITS>(qn, o);
        }
        *reinterpret_cast<uint4*>(bs + swz(lane, 2 * wvu)) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(bs + swz(lane, 2 * wvu + 1)) = make_uint4(o[4], o[5], o[6], o[7]);
    };
    // multipliers: thread tid < 128 loads mx[t0 + tid][g] (1 for tokens past M or without mx), 128 <= tid < 192
    // m[tile][g][tid - 128], by plain zero-extending loads (a 16-bit buffer load's result needs a mask, for which
    // the compiler can wait at once)
    const bool xm = tid < P2_BM, wm_ = tid >= P2_BM && tid < P2_BM + TILE_N;
    const bool x_one = xm && !(mx && t0 + tid < M);
    const bool s_load = (xm && !x_one) || wm_;
    const uint16_t* s_ptr = xm ? (x_one ? ms : mx + (size_t)(t0 + tid) * G) : ms + (size_t)nb * G * 64 + (wm_ ? tid - P2_BM : 0);
    const int s_stride = xm ? 1 : 64;
    uint32_t sreg = 1;

    auto issue_a = [&](int g) __attribute__((always_inline)) {
        dma16_run4x(xr, a_vo, a_vo1, g * GROUP, As[g & 1] + wvu * 4096);
    };
    auto issue_s = [&](int g) __attribute__((always_inline)) {
        if (s_load) sreg = s_ptr[(size_t)g * s_stride];
    };

    issue_a(g0);
    issue_s(g0);
    if constexpr (W8) {
        dma16_run<2>(wr, w_vo, g0 * WB + wvu * 2048, Bp[g0 & 1] + wvu * 2048);
    } else {
        load_w(g0);
        unpack_to(Bs[g0 & 1]);
        if (g0 + 1 < g1) load_w(g0 + 1);
    }
    for (int g = g0; g < g1; g++) {
        const int par = g & 1;
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(sreg) :: "memory");
        if (xm) mxs[par][tid] = x_one ? 1u : sreg;
        else if (wm_) mss[par][tid - P2_BM] = (uint16_t)sreg;
        __syncthreads();                      // group g's copies and unpacked codes are in place; group g - 1's
                                              // compute is done, so the other buffers are free
        if constexpr (!W8) {
            // group g + 1's codes (loaded during the previous round) into the other tile, before any new load is
            // issued (so the wait for those registers finds nothing newer outstanding)
            if (g + 1 < g1) unpack_to(Bs[(g + 1) & 1]);
        }
        if (g + 1 < g1) {
            issue_a(g + 1);
            issue_s(g + 1);
            if constexpr (W8) dma16_run<2>(wr, w_vo, (g + 1) * WB + wvu * 2048, Bp[(g + 1) & 1] + wvu * 2048);
            else if (g + 2 < g1) load_w(g + 2);
        }
        // MFMA over group g and scaling into U
        const int8_t* Ab = As[par];
        v16i d[2];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const v4i a = *reinterpret_cast<const v4i*>(Ab + swz(wv * 32 + l32, 2 * s + lh));
            v4i b0, b1;
            if constexpr (BITS == 8) {
                const int8_t* Bb = Bp[par] + (2 * s + lh) * 1024;
                b0 = *reinterpret_cast<const v4i*>(Bb + l32 * 16);
                b1 = *reinterpret_cast<const v4i*>(Bb + (32 + l32) * 16);
            } else {
                b0 = *reinterpret_cast<const v4i*>(Bs[par] + swz(l32, 2 * s + lh));
                b1 = *reinterpret_cast<const v4i*>(Bs[par] + swz(32 + l32, 2 * s + lh));
            }
            d[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b0, s == 0 ? biasv : d[0], 0, 0, 0);
            d[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b1, s == 0 ? biasv : d[1], 0, 0, 0);
        }
        // element (t, n): lane n % 32 + 32 ((t / 4) % 2), register 4 (t / 8) + t % 4 of chain n / 32
        const uint32_t m0 = mss[par][l32], m1 = mss[par][32 + l32];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint4 mv = *reinterpret_cast<const uint4*>(&mxs[par][wv * 32 + 8 * q4 + 4 * lh]);
            const uint32_t mxv[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                U[0][4 * q4 + e] += (unsigned long long)(uint32_t)d[0][4 * q4 + e] * mul_u24(m0, mxv[e]);
                U[1][4 * q4 + e] += (unsigned long long)(uint32_t)d[1][4 * q4 + e] * mul_u24(m1, mxv[e]);
            }
        }
    }

    // ---- bias correction: S = sum_g m * mx from 7-bit digits on the MFMA, 32 groups at a time, staged in As:
    // xd[i][t][32] of mx (128 tokens), wd[i][n][32] of m (64 rows)
    __syncthreads();                          // every wave is done with As
    int8_t* xd = As[0];                       // [3][128][32] = 12 KB
    int8_t* wd = As[1];                       // [3][64][32] = 6 KB
    float* sxs = reinterpret_cast<float*>(As[1] + 8192);
    if (tid < P2_BM) sxs[tid] = sx[min(t0 + tid, M - 1)];
    // thread tid stages 16 groups of token tid / 2 (half tid % 2); threads < 128 also 16 groups of row tid / 2
    const int sl = tid >> 1, sh = (tid & 1) * 16;
    const bool tok_ok = mx && t0 + sl < M;
    const uint16_t* mrow = mx + (size_t)(t0 + sl) * G;
    const uint16_t* wrow = ms + (size_t)nb * G * 64 + (sl & 63);
    auto digits4 = [](const uint32_t* v, uint32_t& w0, uint32_t& w1, uint32_t& w2) __attribute__((always_inline)) {
        const uint32_t p01 = v[0] | (v[1] << 16), p23 = v[2] | (v[3] << 16);
        w0 = __builtin_amdgcn_perm(p23 & 0x007f007fu, p01 & 0x007f007fu, 0x06040200u);
        w1 = __builtin_amdgcn_perm((p23 >> 7) & 0x007f007fu, (p01 >> 7) & 0x007f007fu, 0x06040200u);
        w2 = __builtin_amdgcn_perm((p23 >> 14) & 0x00030003u, (p01 >> 14) & 0x00030003u, 0x06040200u);
    };
    for (int k0 = g0; k0 < g1; k0 += 32) {
        uint32_t xv[16], wv_[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int g = k0 + sh + e;
            xv[e] = g < g1 ? (tok_ok ? (uint32_t)mrow[g] : 1u) : 0u;
            wv_[e] = g < g1 && tid < 2 * TILE_N ? (uint32_t)wrow[(size_t)g * 64] : 0u;
        }
        uint32_t xw[3][4], ww[3][4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            digits4(xv + 4 * q, xw[0][q], xw[1][q], xw[2][q]);
            digits4(wv_ + 4 * q, ww[0][q], ww[1][q], ww[2][q]);
        }
        if (k0 > g0) __syncthreads();         // the previous chunk's digit reads are done
#pragma unroll
        for (int d = 0; d < 3; d++) {
            *reinterpret_cast<uint4*>(xd + (d * P2_BM + sl) * 32 + sh) = make_uint4(xw[d][0], xw[d][1], xw[d][2], xw[d][3]);
            if (tid < 2 * TILE_N)
                *reinterpret_cast<uint4*>(wd + (d * TILE_N + sl) * 32 + sh) = make_uint4(ww[d][0], ww[d][1], ww[d][2], ww[d][3]);
        }
        __syncthreads();
        v4i A[3];
#pragma unroll
        for (int d = 0; d < 3; d++) A[d] = *reinterpret_cast<const v4i*>(xd + (d * P2_BM + wv * 32 + l32) * 32 + 16 * lh);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            v4i Bd[3];
#pragma unroll
            for (int d = 0; d < 3; d++) Bd[d] = *reinterpret_cast<const v4i*>(wd + (d * TILE_N + j * 32 + l32) * 32 + 16 * lh);
            const v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            // digit weights 2^28 (sum < 2^9), 2^21 (< 2^15), 2^14 (< 2^21), 2^7 (< 2^20): t stays below 2^32
            v16i t = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[2], z, 0, 0, 0);
            v16i e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[1], z, 0, 0, 0);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[2], e, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2], Bd[0], z, 0, 0, 0);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[1], e, 0, 0, 0);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[2], e, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1], Bd[0], z, 0, 0, 0);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[1], e, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) t[r] = (int)(((uint32_t)t[r] << 7) + (uint32_t)e[r]);
            e = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], Bd[0], z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const unsigned long long S = ((unsigned long long)(uint32_t)t[r] << 7) + (uint32_t)e[r];
                U[j][r] -= S << 21;
            }
        }
    }

    // ---- K-slices: every slice stores its exact int64 sums into its own plane of `part` (agent-scope stores,
    // coherent across the XCDs' L2s), waits until they are performed and counts itself in cnt[tile]; the slice
    // that arrives last adds the other planes and runs the epilogue, then resets the counter
    if (KS > 1) {
        const size_t npad = (size_t)nbn * TILE_N, mpad = (size_t)nbt * P2_BM;
        const int tcount = tb * nbn + nb;
        const int tr0 = t0 + wv * 32 + 4 * lh;                   // token of register 0; register r adds 8 (r / 4) + r % 4
        auto at = [&](int k, int j, int r) __attribute__((always_inline)) {
            return part + ((size_t)k * mpad + tr0 + 8 * (r >> 2) + (r & 3)) * npad + n0 + 32 * j + l32;
        };
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                __hip_atomic_store(at(ks, j, r), (long long)U[j][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_performed();             // this wave's stores have been performed
        __syncthreads();
        if (tid == 0)
            last_s = __hip_atomic_fetch_add(cnt + tcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(KS - 1);
        __syncthreads();
        if (!last_s) return;
        for (int k = 0; k < KS; k++) {
            if (k == ks) continue;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    U[j][r] += (unsigned long long)__hip_atomic_load(at(k, j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid == 0) __hip_atomic_store(cnt + tcount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // ---- epilogue: y = (f32(acc) * c[n]) * sx[t]; a tile routed whole to one plain output stores unchecked
    const bool full = t0 + P2_BM <= M && n0 + TILE_N <= N && out.nparts <= 1;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + 32 * j + l32;
        const float cn = n < N ? cs[n] : 0.0f;
        float v[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const float4 sv = *reinterpret_cast<const float4*>(sxs + wv * 32 + 8 * q4 + 4 * lh);
            const float svv[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) v[4 * q4 + e] = (i64_to_f_fast((long long)U[j][4 * q4 + e]) * cn) * svv[e];
        }
        const int tb = t0 + wv * 32 + 4 * lh;        // token of register 0; register r adds 8 (r / 4) + r % 4
        if (full) {
            float* yb = out.y + (size_t)tb * N + n;
            if (out.acc) {
                float old[16];
#pragma unroll
                for (int r = 0; r < 16; r++) old[r] = yb[(size_t)(8 * (r >> 2) + (r & 3)) * N];
#pragma unroll
                for (int r = 0; r < 16; r++) v[r] = old[r] + v[r];
            }
#pragma unroll
            for (int r = 0; r < 16; r++) yb[(size_t)(8 * (r >> 2) + (r & 3)) * N] = v[r];
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = tb + 8 * (r >> 2) + (r & 3);
                if (t < M && n < N) out.store(N, t, n, v[r]);
            }
        }
    }
}

// library-owned stream-K / K-slice buffers: partial tiles and per-tile arrival counters, the counters zero between
// calls (the finishing workgroup resets its tile's; a launch that fails part-way breaks this, and the library treats
// every kernel fault as fatal).  Not counted by det_allocated_bytes.
long long* g_pf_part = nullptr;
size_t g_pf_part_cap = 0;
unsigned int* g_pf_cnt = nullptr;
size_t g_pf_cnt_cap = 0;

void pf_buffers(size_t part_elems, size_t tiles, hipStream_t st) {
    if (part_elems <= g_pf_part_cap && tiles <= g_pf_cnt_cap) return;
    DET_CHECK(hipStreamSynchronize(st));       // earlier launches may still use the old buffers
    if (part_elems > g_pf_part_cap) {
        if (g_pf_part) DET_CHECK(hipFree(g_pf_part));
        g_pf_part_cap = part_elems;
        DET_CHECK(hipMalloc(&g_pf_part, g_pf_part_cap * 8));
    }
    if (tiles > g_pf_cnt_cap) {
        if (g_pf_cnt) DET_CHECK(hipFree(g_pf_cnt));
        g_pf_cnt_cap = std::max(tiles, (size_t)1 << 12);
        DET_CHECK(hipMalloc(&g_pf_cnt, g_pf_cnt_cap * 4));
        DET_CHECK(hipMemset(g_pf_cnt, 0, g_pf_cnt_cap * 4));
    }
    DET_CHECK(hipDeviceSynchronize());
}

template <int BITS>
void launch_prefill(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y,
                    int cus, hipStream_t st) {
    const int G = L.K / GROUP;
    const int nbn = (L.N + PF_BN - 1) / PF_BN, nbt = (M + PF_BM - 1) / PF_BM;
    const int tiles = nbn * nbt;
    const long long total = (long long)tiles * G;
    // two workgroups per CU, each at least 4 groups of work
    long long P = std::min<long long>(2LL * cus, std::max<long long>(1, total / 4));
    if (P > 8) P &= ~7LL;
    const bool split = total % P != 0 || (total / P) % G != 0;
    if (split) pf_buffers((size_t)2 * P * PF_TILE, (size_t)tiles, st);
    else pf_buffers(0, (size_t)tiles, st);
    const uint8_t* pw = L.wq + pf_offset(L.N, L.K, L.bits);
    k_prefill<BITS><<<(unsigned)P, 256, 0, st>>>(pw, L.c, L.m, L.N, L.K, xq, sx, mx, M, y, nbt, tiles, (int)P, g_pf_part, g_pf_cnt);
    DET_CHECK(hipGetLastError());
}

template <int BITS>
void launch_prefill2(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y,
                     int cus, hipStream_t st) {
    const int nbn = (L.N + TILE_N - 1) / TILE_N, nbt = (M + P2_BM - 1) / P2_BM;
    // K-slices when the tiles leave CUs idle: up to 1.5 workgroups per CU, each slice at least 16 groups (the
    // combine costs about as much as a few groups)
    const int G = L.K / GROUP, tiles = nbn * nbt;
    int KS = 1;
    if (2 * tiles < 3 * cus) KS = std::max(1, std::min((3 * cus + 2 * tiles - 1) / (2 * tiles), G / 16));
    const int gs = (G + KS - 1) / KS;
    KS = (G + gs - 1) / gs;                      // no empty slices
    if (KS > 1) pf_buffers((size_t)KS * nbt * P2_BM * nbn * TILE_N, (size_t)tiles, st);
    k_prefill2<BITS><<<tiles * KS, 256, 0, st>>>(L.wq, L.c, L.m, L.N, L.K, xq, sx, mx, M, y, nbn, nbt, KS,
                                                 KS > 1 ? g_pf_part : nullptr, KS > 1 ? g_pf_cnt : nullptr);
    DET_CHECK(hipGetLastError());
}

} // namespace

// Which kernel serves M > 64: the 128 x 64-tile kernel k_prefill2, or the stream-K kernel k_prefill when the
// environment sets DET_PREFILL=streamk (read once, so that a linear's layout and the kernel that reads it agree for
// the life of the process).  Only the stream-K kernel reads the prefill planes: without it they are neither
// reserved nor written.
bool use_streamk() {
    static const int v = [] {
        const char* e = getenv("DET_PREFILL");
        return e && !strcmp(e, "streamk") ? 1 : 0;
    }();
    return v != 0;
}

// byte offset of the prefill planes inside a linear's wq buffer (after the decode tiles)
size_t pf_offset(int N, int K, int bits) {
    const size_t T = 2 * (((size_t)N + 2 * TILE_N - 1) / (2 * TILE_N)), G = (size_t)K / GROUP;
    return T * G * group_bytes(bits) * TILE_N;
}

void prefill_repack(const uint8_t* rows, int N, int K, int bits, uint8_t* wq, hipStream_t st) {
    const size_t blocks32 = 4 * (((size_t)N + PF_BN - 1) / PF_BN), G = (size_t)K / GROUP;
    const size_t items = blocks32 * G * 64;
    const size_t grid = std::min<size_t>((items + 255) / 256, 65536);
    k_repack_pf<<<(unsigned)grid, 256, 0, st>>>(rows, N, K, bits, wq + pf_offset(N, K, bits), items);
    DET_CHECK(hipGetLastError());
}

bool prefill_gemm(const det_qlinear& L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, const Out& y,
                  int cus, hipStream_t st) {
    const int G = L.K / GROUP;
    // U = 2^SH acc must fit int64 (|acc| < G * 2^51) and 32-bit buffer offsets must cover the activations
    if (G >= 1024 || (long long)M * L.K >= (1LL << 31)) return false;
    if (use_streamk()) {
        switch (L.bits) {
            case 8: launch_prefill<8>(L, xq, sx, mx, M, y, cus, st); break;
            case 6: launch_prefill<6>(L, xq, sx, mx, M, y, cus, st); break;
            default: launch_prefill<4>(L, xq, sx, mx, M, y, cus, st); break;
        }
    } else {
        switch (L.bits) {
            case 8: launch_prefill2<8>(L, xq, sx, mx, M, y, cus, st); break;
            case 6: launch_prefill2<6>(L, xq, sx, mx, M, y, cus, st); break;
            default: launch_prefill2<4>(L, xq, sx, mx, M, y, cus, st); break;
        }
    }
    return true;
}

} // namespace det
