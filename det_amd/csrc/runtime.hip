// Runtime half of det's C ABI on HIP: the device, the buffers det_malloc hands out, synchronisation, copies and the
// elementwise primitive test hook.  The behaviour the ABI fixes (reference det_cuda.h:15-24, runtime.cu:83-128):
//   * det_malloc returns a zero-filled device buffer, or NULL (with a message) when the device cannot provide it;
//   * det_free accepts NULL (and anything before the first det_malloc or det_init), refuses (message, abort) a
//     pointer det_malloc did not return, and waits for the device before releasing, since launches still in flight
//     may read the buffer;
//   * det_sync waits for the device and aborts when a kernel failed;
//   * every operation runs on the null stream, det's one in-order stream.
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <string.h>
#include "common.h"
#include "../../include/det_hip.h"
using namespace det;

namespace {

// The process's view of the device: which one, what it is called, and every live det_malloc block (start address ->
// size), so that det_free can tell its own pointers from foreign ones and det_allocated_bytes can report the total.
class DeviceState {
public:
    static DeviceState& instance() {
        static DeviceState s;           // constructed on first use, once, even with concurrent first callers
        return s;
    }
    const char* label() const { return label_.c_str(); }

    void* allocate(size_t bytes) {
        const size_t want = bytes ? bytes : 1;            // a zero-byte request still gets a distinct block
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();                      // the failure is reported here, not by the next call
            fprintf(stderr, "det_malloc: %zu bytes not available on the device (%s)\n", bytes, hipGetErrorString(e));
            return nullptr;
        }
        DET_CHECK(hipMemsetAsync(p, 0, want, nullptr));
        std::lock_guard<std::mutex> hold(mu_);
        blocks_.emplace(reinterpret_cast<uintptr_t>(p), want);
        live_ += want;
        return p;
    }

    // false: p is not the start of a live block
    bool forget(void* p) {
        std::lock_guard<std::mutex> hold(mu_);
        const auto it = blocks_.find(reinterpret_cast<uintptr_t>(p));
        if (it == blocks_.end()) return false;
        live_ -= it->second;
        blocks_.erase(it);
        return true;
    }

    size_t live() {
        std::lock_guard<std::mutex> hold(mu_);
        return live_;
    }

private:
    DeviceState() {
        int dev = 0;
        DET_CHECK(hipGetDevice(&dev));
        hipDeviceProp_t prop;
        DET_CHECK(hipGetDeviceProperties(&prop, dev));
        label_ = std::string(prop.name) + " (" + prop.gcnArchName + ", " + std::to_string(prop.multiProcessorCount) +
                 " CUs)";
    }
    std::string label_;
    std::mutex mu_;
    std::map<uintptr_t, size_t> blocks_;
    size_t live_ = 0;
};

// set once the device state exists: det_free and det_allocated_bytes never create it.  Atomic: any thread may be
// the first to call device() while another reads the flag.
std::atomic<bool> g_touched{false};

DeviceState& device() {
    DeviceState& d = DeviceState::instance();
    g_touched.store(true, std::memory_order_release);
    return d;
}

// ---- det_test_prim: ops as numbered in det_hip.h.  Binary ops pair element i with element n - 1 - i.
__device__ float prim_one(int op, float a, float b) {
    switch (op) {
        case 0: return exp_f(a);
        case 1: return log_f(a);
        case 2: return softplus_f(a);
        case 3: return sigmoid_f(a);
        case 4: return silu_f(a);
        case 6: return rint_(a);
        case 7: return 1.0f / a;
        case 8: return __builtin_sqrtf(a);
        case 9: return a * b;
        case 10: return a + b;
        case 13: return (float)f2i_sat(rint_(a));
        case 14: return a / b;
        case 15: return a - b;
        case 16: return fmax_spec(a, b);
        default: return a;
    }
}

__global__ void k_prim_elementwise(int op, const float* __restrict__ x, int n, float* __restrict__ out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = prim_one(op, x[i], x[n - 1 - i]);
}

// ops 5 and 12: the int64 whose low / high 32 bits are the fp32 bit patterns x[2j] / x[2j + 1], converted to fp32
// into out[2j] (5: the library's RNE routine i64_to_f, 12: the compiler's conversion); odd entries are left as they are
__global__ void k_prim_int64(int op, const float* __restrict__ x, int pairs, float* __restrict__ out) {
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < pairs; j += gridDim.x * blockDim.x) {
        const unsigned long long bits = (unsigned long long)__float_as_uint(x[2 * j + 1]) << 32 | __float_as_uint(x[2 * j]);
        const long long v = (long long)bits;
        out[2 * j] = op == 5 ? i64_to_f(v) : (float)v;
    }
}

// op 11: the spec treesum (spec/prim.rs:154-170) of each row of n <= 8192, padded with +0 to p = next power of two:
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

// det_test_read: a plain streaming read, the measuring stick for the HBM-bound GEMV.  Workgroup b reads its
// contiguous share of the buffer with 16-byte nontemporal loads, four in flight per thread, and stores the xor of
// everything it read into sink[b] (so that no load can be dropped).
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) k_read(const v4u* __restrict__ p, size_t n16, unsigned* __restrict__ sink) {
    __shared__ unsigned red[256];
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t lo = (size_t)blockIdx.x * per, hi = lo + per < n16 ? lo + per : n16;
    unsigned acc = 0;
    size_t i = lo + threadIdx.x;
    for (; i + 3 * 256 < hi; i += 4 * 256) {
        v4u v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = __builtin_nontemporal_load(p + i + u * 256);
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < hi; i += 256) {
        const v4u v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned r = 0;
        for (int t = 0; t < 256; t++) r ^= red[t];
        sink[blockIdx.x] = r;
    }
}

unsigned grid_for(size_t items) { return (unsigned)std::min<size_t>((items + 255) / 256, 65535); }

} // namespace

extern "C" {

int det_init(void) { device(); return 0; }
const char* det_device_name(void) { return device().label(); }
void* det_hip_stream(void) { device(); return nullptr; }          // the null stream

void* det_malloc(size_t bytes) { return device().allocate(bytes); }

void det_free(void* p) {
    if (!p || !g_touched.load(std::memory_order_acquire)) return;     // nothing was ever allocated: nothing to release
    if (!device().forget(p)) {
        fprintf(stderr, "det_free: %p was not returned by det_malloc (or was freed already)\n", p);
        abort();
    }
    DET_CHECK(hipDeviceSynchronize());        // launches still in flight may read the block
    DET_CHECK(hipFree(p));
}

size_t det_allocated_bytes(void) { return g_touched.load(std::memory_order_acquire) ? device().live() : 0; }

void det_sync(void) {
    device();
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        fprintf(stderr, "det_sync: the device reported an error: %s\n", hipGetErrorString(e));
        abort();
    }
}

void det_flush(void) {}       // launches are submitted as they are made

void det_memset(void* p, int value, size_t bytes, hipStream_t st) { DET_CHECK(hipMemsetAsync(p, value, bytes, st)); }

void det_memcpy(void* dst, const void* src, size_t bytes, hipStream_t st) {
    DET_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, st));
}

void det_test_read(const void* p, size_t bytes, int blocks, unsigned* sink, hipStream_t st) {
    if (bytes % 16 || blocks < 1) DET_FAIL("det_test_read: bytes must be a multiple of 16 and blocks positive");
    k_read<<<blocks, 256, 0, st>>>(static_cast<const v4u*>(p), bytes / 16, sink);
    DET_CHECK(hipGetLastError());
}

void det_test_prim(int op, const float* x, int M, int n, float* out, hipStream_t st) {
    const size_t total = (size_t)M * n;
    if (op == 11) {
        if (n > 8192) { fprintf(stderr, "det_test_prim: treesum rows are limited to 8192 (n=%d)\n", n); abort(); }
        k_prim_treesum<<<M, 1024, 0, st>>>(x, n, out);
    } else if (op == 5 || op == 12) {
        k_prim_int64<<<grid_for(total / 2), 256, 0, st>>>(op, x, (int)(total / 2), out);
    } else {
        k_prim_elementwise<<<grid_for(total), 256, 0, st>>>(op, x, (int)total, out);
    }
    DET_CHECK(hipGetLastError());
}

} // extern "C"
