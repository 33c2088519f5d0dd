// HIP runtime of the library: device 0, one non-blocking stream, and
// stream-ordered allocation from the device's default memory pool.
// Replaces gpt.c's kernels/src/cuda/runtime.cu:16-52 and Alloc.cu:9-20
// (no BLAS handle: the attention path uses no BLAS library).
#include <cstdint>
#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace {
hipStream_t g_stream = nullptr;
bool g_ready = false;
bool g_pool_alloc = false;  // device supports stream-ordered allocation
}  // namespace

hipStream_t gptc_stream_checked() {
    CHECK_ERROR(!g_ready, "The GPU runtime has not been initialised. Call runtime_init(CUDA) first.");
    return g_stream;
}

extern "C" void runtime_init_cuda(void) {
    if (g_ready) return;
    int count = 0;
    hipCheck(hipGetDeviceCount(&count));
    CHECK_ERROR(count < 1, "No HIP device is visible.");
    hipCheck(hipSetDevice(0));
    hipCheck(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    int pools = 0;
    hipCheck(hipDeviceGetAttribute(&pools, hipDeviceAttributeMemoryPoolsSupported, 0));
    g_pool_alloc = pools != 0;
    if (g_pool_alloc) {
        // Keep freed blocks in the pool: layers allocate and free their
        // activations every step, and returning them to the driver at each
        // synchronisation would turn every step into fresh mappings.
        hipMemPool_t pool;
        hipCheck(hipDeviceGetDefaultMemPool(&pool, 0));
        uint64_t keep = UINT64_MAX;
        hipCheck(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
    }
    g_ready = true;
}

extern "C" void runtime_destroy_cuda(void) {
    if (!g_ready) return;
    hipCheck(hipStreamSynchronize(g_stream));
    hipCheck(hipStreamDestroy(g_stream));
    g_stream = nullptr;
    g_ready = false;
}

extern "C" void synchronize_cuda(void) {
    hipCheck(hipStreamSynchronize(gptc_stream_checked()));
}

extern "C" void *gptc_stream(void) {
    return reinterpret_cast<void *>(gptc_stream_checked());
}

extern "C" void *alloc_cuda(const size_t nbytes) {
    hipStream_t s = gptc_stream_checked();
    void *ptr = nullptr;
    const size_t n = nbytes ? nbytes : 4;
    if (g_pool_alloc)
        hipCheck(hipMallocAsync(&ptr, n, s));
    else
        hipCheck(hipMalloc(&ptr, n));
    return ptr;
}

extern "C" void free_cuda(void *ptr) {
    if (ptr == nullptr) return;
    hipStream_t s = gptc_stream_checked();
    if (g_pool_alloc)
        hipCheck(hipFreeAsync(ptr, s));
    else
        hipCheck(hipFree(ptr));
}
