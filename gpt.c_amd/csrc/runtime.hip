// HIP runtime of the library: device 0, one non-blocking stream, and a
// stream-ordered caching allocator.  Replaces gpt.c's
// kernels/src/cuda/runtime.cu:16-52 and Alloc.cu:9-20.
//
// Allocation.  gpt.c's layers allocate and free their activations and
// gradients every step (hundreds of buffers per GPT-2 step).  hipFreeAsync
// on this stack can block the host for milliseconds (tens of ms seen for
// some frees in a GPT-2 step trace), which leaves the GPU idle.  So freed
// blocks are kept in a cache keyed by size class and handed to the next
// request of the same class.  Every launch, copy and fill of the library
// runs on its one stream, so a block reused after free_cuda() is only
// touched by work queued after everything that used it before: reuse needs
// no event or synchronisation.  Size classes: multiples of 512 B up to
// 1 MiB, multiples of 2 MiB above.  When the device runs out of memory the
// cache is returned to the device and the request retried once.
//
// Serials.  Every allocation of a block, and every write the library's
// tensor data ops make into it, gives the block a new serial: a host-side
// cache of something derived from a block's contents (the attention mask
// check) stays valid while the serial is unchanged.
//
// Shared blocks.  gptc_retain_cuda() adds an owner to a live block: two
// tensors can then hold one buffer (the attention layer keeps its output
// for the backward that way instead of copying it), and the block returns
// to the cache when the last owner frees it.
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>
#include "blas.hpp"
#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace {
hipStream_t g_stream = nullptr;
bool g_ready = false;
bool g_pool_alloc = false;  // device supports stream-ordered allocation

std::mutex g_alloc_mu;
struct LiveBlock {
    size_t cls;       // size class
    int refs;         // owners (1 + retains)
    uint64_t serial;  // changes at every allocation of the block and every library write into it
};
uint64_t g_serial = 0;
std::unordered_map<void *, LiveBlock> g_live;  // blocks in use
std::multimap<size_t, void *> g_cached;     // size class -> free block
size_t g_cached_bytes = 0;

size_t size_class(size_t n) {
    if (n == 0) n = 1;
    constexpr size_t kSmall = 512, kLarge = 2u << 20, kSplit = 1u << 20;
    return n <= kSplit ? (n + kSmall - 1) / kSmall * kSmall : (n + kLarge - 1) / kLarge * kLarge;
}

hipError_t device_alloc(void **p, size_t n) {
    return g_pool_alloc ? hipMallocAsync(p, n, g_stream) : hipMalloc(p, n);
}

void device_free(void *p) {
    if (g_pool_alloc)
        hipCheck(hipFreeAsync(p, g_stream));
    else
        hipCheck(hipFree(p));
}

// Return every cached block to the device (caller holds g_alloc_mu).
void release_cache() {
    for (auto &kv : g_cached) device_free(kv.second);
    g_cached.clear();
    g_cached_bytes = 0;
}
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
        // Blocks that do leave the cache stay in the driver's pool.
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
    gptc_blas_destroy();
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        release_cache();
    }
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
    gptc_stream_checked();
    const size_t cls = size_class(nbytes);
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_cached.find(cls);
    void *ptr = nullptr;
    if (it != g_cached.end()) {
        ptr = it->second;
        g_cached.erase(it);
        g_cached_bytes -= cls;
    } else {
        hipError_t err = device_alloc(&ptr, cls);
        if (err == hipErrorOutOfMemory && !g_cached.empty()) {
            (void)hipGetLastError();  // clear the failed allocation's error
            release_cache();
            hipCheck(hipStreamSynchronize(g_stream));
            err = device_alloc(&ptr, cls);
        }
        hipCheck(err);
    }
    g_live.emplace(ptr, LiveBlock{cls, 1, ++g_serial});
    return ptr;
}

uint64_t gptc_block_serial(const void *ptr) {
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_live.find(const_cast<void *>(ptr));
    return it == g_live.end() ? 0 : it->second.serial;
}

void gptc_block_written(const void *ptr) {
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_live.find(const_cast<void *>(ptr));
    if (it != g_live.end()) it->second.serial = ++g_serial;
}

extern "C" void gptc_retain_cuda(void *ptr) {
    REQUIRE_ARG(ptr);
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_live.find(ptr);
    CHECK_ERROR(it == g_live.end(), "gptc_retain_cuda: %p is not a live block of alloc_cuda.", ptr);
    ++it->second.refs;
}

extern "C" void free_cuda(void *ptr) {
    if (ptr == nullptr) return;
    gptc_stream_checked();
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) {  // not from alloc_cuda: hand it back directly
        device_free(ptr);
        return;
    }
    if (--it->second.refs > 0) return;  // another owner still holds the block
    g_cached.emplace(it->second.cls, ptr);
    g_cached_bytes += it->second.cls;
    g_live.erase(it);
}
