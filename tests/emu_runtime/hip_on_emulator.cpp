// Test infrastructure: a stand-in for the HIP runtime entry points libdet_hip.so calls, so that the library's own
// host code (argument checks, kernel choice, grids, buffer management) runs unchanged on a machine without a GPU,
// with every kernel launch handed to the instruction-level emulator (tests/gfx950_emu.py) through callbacks the
// Python side installs.  "Device" memory is host memory the callbacks allocate (numpy buffers the emulator knows),
// so copies and fills are plain memcpy / memset.  Loaded with RTLD_GLOBAL before the library, so that the
// library's references to these symbols bind here; the version script gives them the versions it asks for.
// Never part of the product: only tests/test_emulated_runtime.py builds and loads it.
#include <hip/hip_runtime_api.h>
#include <cstring>
#include <map>
#include <string>
#include <vector>

typedef int (*emu_launch_fn)(const char* name, unsigned gx, unsigned gy, unsigned gz, unsigned bx, unsigned by,
                             unsigned bz, void** args, size_t shared);
typedef void* (*emu_alloc_fn)(size_t bytes);
typedef int (*emu_release_fn)(void* p);

namespace {
emu_launch_fn g_launch = nullptr;
emu_alloc_fn g_alloc = nullptr;
emu_release_fn g_release = nullptr;
int g_cus = 256;
hipError_t g_error = hipSuccess;
std::map<const void*, std::string> g_kernels;          // host stub -> device symbol
struct Var { size_t size; void* dev; };
std::map<const void*, Var> g_vars;                     // host shadow of a __device__ variable -> its device copy
struct Config { dim3 grid, block; size_t shared; hipStream_t stream; };
std::vector<Config> g_configs;
void* g_fatbin_handle = nullptr;
}  // namespace

extern "C" {

void emu_install(emu_launch_fn launch, emu_alloc_fn alloc, emu_release_fn release, int cus) {
    g_launch = launch;
    g_alloc = alloc;
    g_release = release;
    g_cus = cus;
}

void** __hipRegisterFatBinary(const void*) { return &g_fatbin_handle; }
void __hipUnregisterFatBinary(void**) {}
void __hipRegisterFunction(void**, const void* host_function, char*, const char* device_name, unsigned int, uint3*,
                           uint3*, dim3*, dim3*, int*) {
    g_kernels[host_function] = device_name;
}

// __device__ variables: the size at registration; device memory (zeroed) on the first hipGetSymbolAddress
void __hipRegisterVar(void**, void* var, char*, char*, int, size_t size, int, int) { g_vars[var] = {size, nullptr}; }
hipError_t hipGetSymbolAddress(void** p, const void* symbol) {
    const auto it = g_vars.find(symbol);
    if (it == g_vars.end() || !g_alloc) return g_error = hipErrorInvalidSymbol;
    if (!it->second.dev) it->second.dev = g_alloc(it->second.size);
    *p = it->second.dev;
    return *p ? hipSuccess : (g_error = hipErrorOutOfMemory);
}

hipError_t __hipPushCallConfiguration(dim3 grid, dim3 block, size_t shared, hipStream_t stream) {
    g_configs.push_back({grid, block, shared, stream});
    return hipSuccess;
}
hipError_t __hipPopCallConfiguration(dim3* grid, dim3* block, size_t* shared, hipStream_t* stream) {
    if (g_configs.empty()) return hipErrorInvalidConfiguration;
    const Config c = g_configs.back();
    g_configs.pop_back();
    *grid = c.grid;
    *block = c.block;
    *shared = c.shared;
    *stream = c.stream;
    return hipSuccess;
}
hipError_t hipLaunchKernel(const void* f, dim3 grid, dim3 block, void** args, size_t shared, hipStream_t) {
    const auto it = g_kernels.find(f);
    if (it == g_kernels.end() || !g_launch) return g_error = hipErrorInvalidDeviceFunction;
    if (g_launch(it->second.c_str(), grid.x, grid.y, grid.z, block.x, block.y, block.z, args, shared) != 0)
        return g_error = hipErrorLaunchFailure;
    return hipSuccess;
}

hipError_t hipMalloc(void** p, size_t bytes) {
    *p = g_alloc ? g_alloc(bytes) : nullptr;
    return *p ? hipSuccess : (g_error = hipErrorOutOfMemory);
}
hipError_t hipFree(void* p) {
    if (p && g_release) g_release(p);
    return hipSuccess;
}
hipError_t hipMemset(void* p, int v, size_t n) { memset(p, v, n); return hipSuccess; }
hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t) { memset(p, v, n); return hipSuccess; }
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) { memmove(d, s, n); return hipSuccess; }
hipError_t hipDeviceSynchronize(void) { return g_error; }
hipError_t hipStreamSynchronize(hipStream_t) { return g_error; }
hipError_t hipGetLastError(void) { const hipError_t e = g_error; g_error = hipSuccess; return e; }
const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "error in the emulated runtime"; }
hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_tR0600* p, int) {
    memset(p, 0, sizeof *p);
    strcpy(p->name, "gfx950 instruction-level emulator");
    strcpy(p->gcnArchName, "gfx950");
    p->multiProcessorCount = g_cus;
    p->warpSize = 64;
    p->maxThreadsPerBlock = 1024;
    p->sharedMemPerBlock = 160 * 1024;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t attr, int) {
    *v = attr == hipDeviceAttributeMultiprocessorCount ? g_cus : attr == hipDeviceAttributeWarpSize ? 64 : 0;
    return hipSuccess;
}
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int) { return hipSuccess; }

}  // extern "C"
