// det's x86-64 quantized GEMM, restated in C with AVX2 / AVX-VNNI intrinsics, for the CPU baseline that bench.py
// reports beside the GPU figure (TEST INFRASTRUCTURE: only bench.py's cpu_baseline leg and tests/ load it).
//
// The algorithm is the reference backend's (crates/det/src/x86/gemm.rs; dot products x86/simd.rs:50-71; the
// VNNI choice x86/mod.rs:41-52), kept alike because this file exists to time that algorithm:
//   - load-time repack into strips of 8 rows; per 16-k block the unsigned codes u = wq + OFF of the strip as four
//     32-byte operands (k-quad q: byte 4 r + j = u[r][4 q + j]), nibble-packed for W4 (2 loads) and W6 (3 loads),
//     then the strip's m[g][row] and c[row] (gemm.rs:1-9, 64-130);
//   - a work item is a pair of strips (16 rows) x up to 64 tokens; per 1024-k chunk the pair's codes are unpacked
//     once into an L1 scratch, then 4 tokens at a time: one 8-lane s32 accumulator per (token, strip) over a
//     128-group by vpdpbusd (AVX-VNNI) or vpmaddubsw + vpmaddwd (AVX2; W8 split into nibbles, since the 16-bit
//     pair sums saturate for u > 127), then p - OFF * sum(xq) times m * mx into int64 (gemm.rs:200-287);
//   - y = ((float)acc * c) * sx (the spec's epilogue; int64 -> float is cvtsi2ss, round to nearest even).
// The same source is compiled twice: XVNNI = 0 with -mavx2 (this unit also holds the repack and the entry point)
// and XVNNI = 1 with -mavx2 -mavxvnni, so no VEX vpdpbusd can appear in the AVX2 path.
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define XR 8          // rows per strip
#define XPAIR 16      // rows per work item
#define XBLK 16       // k per block
#define XKC 1024      // k per unpacked chunk
#define XTC 64        // tokens per work item
#define XGROUP 128

typedef struct {
    uint8_t* data;
    int n, k, bits, strips;
    size_t strip_bytes, m_off, c_off;
} ora_x86_lin;

static inline int xblock_bytes(int bits) { return bits == 8 ? 128 : bits == 6 ? 96 : 64; }

#if XVNNI
#define SUFFIX(f) f##_vnni
#else
#define SUFFIX(f) f##_avx2
#endif

// acc + sum over each lane's four byte pairs of u (unsigned) * x (signed)
static inline __m256i xdp(__m256i acc, __m256i u, __m256i x, int bits) {
#if XVNNI
    (void)bits;
    return _mm256_dpbusd_avx_epi32(acc, u, x);
#else
    const __m256i ones = _mm256_set1_epi16(1);
    if (bits == 8) {
        const __m256i nib = _mm256_set1_epi8(0x0F);
        const __m256i lo = _mm256_and_si256(u, nib), hi = _mm256_and_si256(_mm256_srli_epi16(u, 4), nib);
        const __m256i a = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, x), ones);
        const __m256i b = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, x), ones);
        return _mm256_add_epi32(acc, _mm256_add_epi32(a, _mm256_slli_epi32(b, 4)));
    }
    return _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_maddubs_epi16(u, x), ones));
#endif
}

// the four k-quad operands of one 16-k block of a strip
static inline void xunpack(const uint8_t* p, int bits, __m256i q[4]) {
    const __m256i l0 = _mm256_load_si256((const __m256i*)p), l1 = _mm256_load_si256((const __m256i*)(p + 32));
    if (bits == 8) {
        q[0] = l0; q[1] = l1;
        q[2] = _mm256_load_si256((const __m256i*)(p + 64)); q[3] = _mm256_load_si256((const __m256i*)(p + 96));
        return;
    }
    const __m256i nib = _mm256_set1_epi8(0x0F);
    q[0] = _mm256_and_si256(l0, nib);
    q[1] = _mm256_and_si256(_mm256_srli_epi16(l0, 4), nib);
    q[2] = _mm256_and_si256(l1, nib);
    q[3] = _mm256_and_si256(_mm256_srli_epi16(l1, 4), nib);
    if (bits == 6) {
        const __m256i h = _mm256_load_si256((const __m256i*)(p + 64)), two = _mm256_set1_epi8(0x30);
        q[0] = _mm256_or_si256(q[0], _mm256_and_si256(_mm256_slli_epi16(h, 4), two));
        q[1] = _mm256_or_si256(q[1], _mm256_and_si256(_mm256_slli_epi16(h, 2), two));
        q[2] = _mm256_or_si256(q[2], _mm256_and_si256(h, two));
        q[3] = _mm256_or_si256(q[3], _mm256_and_si256(_mm256_srli_epi16(h, 2), two));
    }
}

// p * mm as int64 for 8 lanes (s32 p, u32 mm): the even lanes and the odd lanes, an unsigned 32 x 32 product minus
// mm << 32 where p < 0
static inline void xmul(__m256i p, __m256i mm, __m256i* even, __m256i* odd) {
    const __m256i neg = _mm256_srai_epi32(p, 31);
    const __m256i fe = _mm256_slli_epi64(_mm256_and_si256(mm, neg), 32);
    const __m256i po = _mm256_srli_epi64(p, 32), mo = _mm256_srli_epi64(mm, 32), no = _mm256_srli_epi64(neg, 32);
    const __m256i fo = _mm256_slli_epi64(_mm256_and_si256(mo, no), 32);
    *even = _mm256_sub_epi64(_mm256_mul_epu32(p, mm), fe);
    *odd = _mm256_sub_epi64(_mm256_mul_epu32(po, mo), fo);
}

// T tokens from t over the unpacked chunk at kc0 (groups of it): acc[token][16] int64, lanes 0-3 of a strip are its
// even rows, 4-7 its odd rows
static inline void xtile(const ora_x86_lin* L, int pair, const int8_t* xq, const int32_t* xsum, const uint16_t* mx,
                         const uint8_t* scratch, int kc0, int groups, int t, int T, int64_t (*acc)[XPAIR], int t0) {
    const int k = L->k, G = k / XGROUP, off = 1 << (L->bits - 1), bits = L->bits;
    for (int gi = 0; gi < groups; gi++) {
        const int g = kc0 / XGROUP + gi;
        __m256i a[4][2];
        for (int tt = 0; tt < 4; tt++) a[tt][0] = a[tt][1] = _mm256_setzero_si256();
        for (int kq = 0; kq < XGROUP / 4; kq++) {
            const uint8_t* w = scratch + (size_t)((gi * (XGROUP / 4) + kq) * 2) * 32;
            const __m256i w0 = _mm256_load_si256((const __m256i*)w), w1 = _mm256_load_si256((const __m256i*)(w + 32));
            for (int tt = 0; tt < T; tt++) {
                int32_t xv;
                memcpy(&xv, xq + (size_t)(t + tt) * k + kc0 + gi * XGROUP + kq * 4, 4);
                const __m256i x = _mm256_set1_epi32(xv);
                a[tt][0] = xdp(a[tt][0], w0, x, bits);
                a[tt][1] = xdp(a[tt][1], w1, x, bits);
            }
        }
        __m256i m[2];
        for (int s = 0; s < 2; s++) {
            const uint16_t* mp = (const uint16_t*)(L->data + (size_t)(2 * pair + s) * L->strip_bytes + L->m_off) + (size_t)g * XR;
            m[s] = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i*)mp));
        }
        for (int tt = 0; tt < T; tt++) {
            const __m256i xs = _mm256_set1_epi32(off * xsum[(size_t)(t + tt) * G + g]);
            const __m256i mxv = _mm256_set1_epi32(mx ? mx[(size_t)(t + tt) * G + g] : 1);
            for (int s = 0; s < 2; s++) {
                __m256i even, odd;
                xmul(_mm256_sub_epi32(a[tt][s], xs), _mm256_mullo_epi32(m[s], mxv), &even, &odd);
                int64_t* dst = acc[t + tt - t0] + s * XR;
                _mm256_storeu_si256((__m256i*)dst, _mm256_add_epi64(_mm256_loadu_si256((const __m256i*)dst), even));
                _mm256_storeu_si256((__m256i*)(dst + 4), _mm256_add_epi64(_mm256_loadu_si256((const __m256i*)(dst + 4)), odd));
            }
        }
    }
}

void SUFFIX(ora_x86_item)(const ora_x86_lin* L, int pair, const int8_t* xq, const int32_t* xsum, const uint16_t* mx,
                          int t0, int t1, int64_t (*acc)[XPAIR], uint8_t* scratch) {
    const int k = L->k, bb = xblock_bytes(L->bits);
    for (int kc0 = 0; kc0 < k; kc0 += XKC) {
        const int kc = k - kc0 < XKC ? k - kc0 : XKC;
        for (int s = 0; s < 2; s++) {
            const uint8_t* codes = L->data + (size_t)(2 * pair + s) * L->strip_bytes + (size_t)(kc0 / XBLK) * bb;
            for (int b = 0; b < kc / XBLK; b++) {
                __m256i q[4];
                xunpack(codes + (size_t)b * bb, L->bits, q);
                for (int qi = 0; qi < 4; qi++) _mm256_store_si256((__m256i*)(scratch + (size_t)((b * 4 + qi) * 2 + s) * 32), q[qi]);
            }
        }
        int t = t0;
        for (; t + 4 <= t1; t += 4) xtile(L, pair, xq, xsum, mx, scratch, kc0, kc / XGROUP, t, 4, acc, t0);
        for (; t < t1; t++) xtile(L, pair, xq, xsum, mx, scratch, kc0, kc / XGROUP, t, 1, acc, t0);
    }
}

#if !XVNNI
#include <cpuid.h>
void ora_unpack_row(const uint8_t* p, int bits, int k, int8_t* out);
size_t ora_row_bytes(int bits, int k);
void ora_x86_item_vnni(const ora_x86_lin* L, int pair, const int8_t* xq, const int32_t* xsum, const uint16_t* mx,
                       int t0, int t1, int64_t (*acc)[XPAIR], uint8_t* scratch);

// AVX-VNNI (the VEX form det uses): CPUID leaf 7, sub-leaf 1, EAX bit 4
int ora_x86_has_vnni(void) {
    unsigned a, b, c, d;
    if (!__get_cpuid_count(7, 1, &a, &b, &c, &d)) return 0;
    return (a >> 4) & 1;
}

// repack det rows [n][row_bytes] into strips (gemm.rs:64-130); rows past n are zero codes with c = 0, m = 1
ora_x86_lin* ora_x86_repack(const uint8_t* rows, int n, int k, int bits) {
    ora_x86_lin* L = (ora_x86_lin*)calloc(1, sizeof(ora_x86_lin));
    const int bb = xblock_bytes(bits), G = k / XGROUP, off = 1 << (bits - 1);
    L->n = n; L->k = k; L->bits = bits;
    L->strips = (n + XPAIR - 1) / XPAIR * 2;
    L->m_off = (size_t)(k / XBLK) * bb;
    L->c_off = L->m_off + (size_t)G * XR * 2;
    L->strip_bytes = (L->c_off + XR * 4 + 63) / 64 * 64;
    L->data = (uint8_t*)aligned_alloc(64, (size_t)L->strips * L->strip_bytes);
    memset(L->data, 0, (size_t)L->strips * L->strip_bytes);
    const size_t rb = ora_row_bytes(bits, k), cb = (size_t)k / 32 * (bits == 8 ? 32 : bits == 6 ? 24 : 16);
#pragma omp parallel for schedule(dynamic, 4)
    for (int s = 0; s < L->strips; s++) {
        uint8_t* d = L->data + (size_t)s * L->strip_bytes;
        uint8_t* u = (uint8_t*)malloc((size_t)XR * k);
        int8_t* wq = (int8_t*)malloc(k);
        for (int r = 0; r < XR; r++) {
            const int row = s * XR + r;
            float c = 0.0f;
            if (row < n) {
                const uint8_t* src = rows + (size_t)row * rb;
                ora_unpack_row(src, bits, k, wq);
                for (int i = 0; i < k; i++) u[(size_t)r * k + i] = (uint8_t)(wq[i] + off);
                memcpy(&c, src + cb, 4);
                for (int g = 0; g < G; g++) memcpy(d + L->m_off + ((size_t)g * XR + r) * 2, src + cb + 4 + 2 * g, 2);
            } else {
                memset(u + (size_t)r * k, off, k);
                const uint16_t one = 1;
                for (int g = 0; g < G; g++) memcpy(d + L->m_off + ((size_t)g * XR + r) * 2, &one, 2);
            }
            memcpy(d + L->c_off + 4 * r, &c, 4);
        }
        for (int b = 0; b < k / XBLK; b++) {
            uint8_t* blk = d + (size_t)b * bb;
            for (int r = 0; r < XR; r++)
                for (int j = 0; j < 4; j++) {
                    uint8_t q[4];
                    for (int qi = 0; qi < 4; qi++) q[qi] = u[(size_t)r * k + b * XBLK + qi * 4 + j];
                    const int i = r * 4 + j;
                    if (bits == 8) {
                        for (int qi = 0; qi < 4; qi++) blk[qi * 32 + i] = q[qi];
                    } else {
                        blk[i] = (uint8_t)((q[0] & 15) | (q[1] & 15) << 4);
                        blk[32 + i] = (uint8_t)((q[2] & 15) | (q[3] & 15) << 4);
                        if (bits == 6) blk[64 + i] = (uint8_t)((q[0] >> 4) | (q[1] >> 4) << 2 | (q[2] >> 4) << 4 | (q[3] >> 4) << 6);
                    }
                }
        }
        free(u);
        free(wq);
    }
    return L;
}

void ora_x86_free(ora_x86_lin* L) {
    if (!L) return;
    free(L->data);
    free(L);
}

// y[M][n] = the GEMM (Write), over `threads` OpenMP threads (0: the runtime's default); vnni = 1 requires AVX-VNNI
void ora_x86_gemm(const ora_x86_lin* L, const int8_t* xq, const float* sx, const uint16_t* mx, int M, float* y,
                  int vnni, int threads) {
    const int k = L->k, n = L->n, G = k / XGROUP;
    int32_t* xsum = (int32_t*)malloc(sizeof(int32_t) * (size_t)M * G);
    for (size_t i = 0; i < (size_t)M * G; i++) {
        int s = 0;
        for (int j = 0; j < XGROUP; j++) s += xq[i * XGROUP + j];
        xsum[i] = s;
    }
    const int pairs = (n + XPAIR - 1) / XPAIR, tchunks = (M + XTC - 1) / XTC;
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
    {
        uint8_t* scratch = (uint8_t*)aligned_alloc(64, (size_t)XKC / 4 * 2 * 32);
        int64_t (*acc)[XPAIR] = (int64_t (*)[XPAIR])malloc(sizeof(int64_t) * XTC * XPAIR);
#pragma omp for schedule(dynamic, 1)
        for (int i = 0; i < pairs * tchunks; i++) {
            const int pair = i % pairs, tc = i / pairs;
            const int t0 = tc * XTC, t1 = (tc + 1) * XTC < M ? (tc + 1) * XTC : M;
            memset(acc, 0, sizeof(int64_t) * XTC * XPAIR);
            if (vnni) ora_x86_item_vnni(L, pair, xq, xsum, mx, t0, t1, acc, scratch);
            else ora_x86_item_avx2(L, pair, xq, xsum, mx, t0, t1, acc, scratch);
            for (int r = 0; r < XPAIR; r++) {
                const int row = pair * XPAIR + r;
                if (row >= n) break;
                const int lane = (r / XR) * XR + (r % 2) * 4 + (r % XR) / 2;
                float c;
                memcpy(&c, L->data + (size_t)(row / XR) * L->strip_bytes + L->c_off + (row % XR) * 4, 4);
                for (int t = t0; t < t1; t++) y[(size_t)t * n + row] = ((float)acc[t - t0][lane] * c) * sx[t];
            }
        }
        free(scratch);
        free(acc);
    }
    free(xsum);
}
#endif
