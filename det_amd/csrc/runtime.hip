// det HIP runtime: device init, tracked device buffers, synchronization, the primitive test hook.
// Mirrors the behaviour of the reference runtime (kernels/cuda/runtime.cu:83-127): det_malloc zero-fills and
// returns NULL on failure, det_free waits for pending work and aborts on a foreign pointer, det_sync aborts on a
// kernel error.  One in-order stream: the null stream.
#include <mutex>
#include <string.h>
#include <unordered_map>
#include "common.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

struct Ctx {
    int dev = 0;
    char name[256] = {0};
    std::mutex mu;
    std::unordered_map<void*, size_t> allocs;
    size_t allocated = 0;
};
Ctx* g = nullptr;
std::once_flag g_once;

void init_once() {
    g = new Ctx();
    DET_CHECK(hipGetDevice(&g->dev));
    hipDeviceProp_t p;
    DET_CHECK(hipGetDeviceProperties(&p, g->dev));
    snprintf(g->name, sizeof g->name, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
}
inline void ensure_init() { std::call_once(g_once, init_once); }

// ---- test hook kernels: op numbers as documented in det_hip.h
__global__ void k_prim(int op, const float* __restrict__ x, int n, float* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    const float w = x[n - 1 - i];
    float r = 0.0f;
    switch (op) {
        case 0: r = exp_f(v); break;
        case 1: r = log_f(v); break;
        case 2: r = softplus_f(v); break;
        case 3: r = sigmoid_f(v); break;
        case 4: r = silu_f(v); break;
        case 5: case 12: {
            if (i & 1) return;
            const unsigned long long lo = __float_as_uint(v), hi = __float_as_uint(x[i + 1]);
            const long long q = (long long)((hi << 32) | lo);
            r = op == 5 ? i64_to_f(q) : (float)q;
            break;
        }
        case 6: r = rint_(v); break;
        case 7: r = 1.0f / v; break;
        case 8: r = __builtin_sqrtf(v); break;
        case 9: r = v * w; break;
        case 10: r = v + w; break;
        case 13: r = (float)f2i_sat(rint_(v)); break;
        case 14: r = v / w; break;
        case 15: r = v - w; break;
        case 16: r = fmax_spec(v, w); break;
        default: r = v;
    }
    out[i] = r;
}

// spec treesum (spec/prim.rs:154-170) of each row of n <= 8192, padded with +0 to p = next power of two:
// each thread reduces 8 contiguous values as a local tree, then the p/8 partials are combined pairwise by
// ascending distance through LDS -- the same balanced tree.  Rows of p <= 8 run the tree in one thread.
__global__ void __launch_bounds__(1024) k_prim_treesum(const float* __restrict__ x, int n, float* __restrict__ out) {
    __shared__ float s[1024];
    const float* row = x + (size_t)blockIdx.x * n;
    const int t = threadIdx.x;
    int p = 1;
    while (p < n) p <<= 1;
    if (p <= 8) {
        if (t == 0) {
            float v[8];
            for (int i = 0; i < p; i++) v[i] = i < n ? row[i] : 0.0f;
            for (int w = p; w > 1;) { w >>= 1; for (int i = 0; i < w; i++) v[i] = v[2 * i] + v[2 * i + 1]; }
            out[blockIdx.x] = n > 0 ? v[0] : 0.0f;
        }
        return;
    }
    const int nt = p / 8;
    if (t < nt) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { const int idx = t * 8 + i; v[i] = idx < n ? row[idx] : 0.0f; }
        s[t] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    }
    __syncthreads();
    for (int d = 1; d < nt; d <<= 1) {
        float r = 0.0f;
        const bool act = t < nt && (t % (2 * d)) == 0;
        if (act) r = s[t] + s[t + d];
        __syncthreads();
        if (act) s[t] = r;
        __syncthreads();
    }
    if (t == 0) out[blockIdx.x] = s[0];
}

} // namespace

extern "C" {

int det_init(void) { ensure_init(); return g ? 0 : 1; }
const char* det_device_name(void) { ensure_init(); return g->name; }
void* det_hip_stream(void) { ensure_init(); return (void*)(hipStream_t)0; }

void* det_malloc(size_t bytes) {
    ensure_init();
    if (bytes == 0) bytes = 16;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        fprintf(stderr, "det_malloc(%zu) failed\n", bytes);
        return NULL;
    }
    DET_CHECK(hipMemsetAsync(p, 0, bytes, 0));
    std::lock_guard<std::mutex> lock(g->mu);
    g->allocs[p] = bytes;
    g->allocated += bytes;
    return p;
}

void det_free(void* p) {
    if (!p || !g) return;
    {
        std::lock_guard<std::mutex> lock(g->mu);
        auto it = g->allocs.find(p);
        if (it == g->allocs.end()) { fprintf(stderr, "det_free: %p is not a det_malloc pointer\n", p); abort(); }
        g->allocated -= it->second;
        g->allocs.erase(it);
    }
    DET_CHECK(hipDeviceSynchronize());   // pending work may still read the buffer
    DET_CHECK(hipFree(p));
}

size_t det_allocated_bytes(void) { return g ? g->allocated : 0; }

void det_sync(void) {
    ensure_init();
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) { fprintf(stderr, "det (hip) fatal: %s\n", hipGetErrorString(e)); abort(); }
}
void det_flush(void) {}

void det_memset(void* p, int value, size_t bytes, hipStream_t st) { DET_CHECK(hipMemsetAsync(p, value, bytes, st)); }
void det_memcpy(void* dst, const void* src, size_t bytes, hipStream_t st) {
    DET_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, st));
}

void det_test_prim(int op, const float* x, int M, int n, float* out, hipStream_t st) {
    if (op == 11) {
        if (n > 8192) { fprintf(stderr, "det_test_prim: treesum rows are limited to 8192 (n=%d)\n", n); abort(); }
        k_prim_treesum<<<M, 1024, 0, st>>>(x, n, out);
    } else {
        k_prim<<<(unsigned)(((size_t)M * n + 255) / 256), 256, 0, st>>>(op, x, (int)((size_t)M * n), out);
    }
    DET_CHECK(hipGetLastError());
}

} // extern "C"
