// Device tensor data ops (replaces gpt.c's kernels/src/cuda/Tensor.cu:9-130):
// fill / arange / copy kernels and the synchronous host <-> device moves.
// Grid-stride loops over 16-byte vectors; a launch uses at most 8 waves
// per CU worth of workgroups and lets each thread cover several vectors.
#include <cstdint>
#include <cstdlib>
#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace {

constexpr int kThreads = 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));

int grid_for(int64_t work) {
    int64_t g = (work + kThreads - 1) / kThreads;
    if (g > 256 * 8) g = 256 * 8;
    return g < 1 ? 1 : static_cast<int>(g);
}

// vec: dst is 16-byte aligned, so the body can use 16-byte stores.
__global__ __launch_bounds__(kThreads) void fill_kernel(float *__restrict__ dst, int64_t n, float value, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t n4 = vec ? n / 4 : 0;
    const f32x4 v = {value, value, value, value};
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride)
        reinterpret_cast<f32x4 *>(dst)[i] = v;
    for (int64_t i = 4 * n4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) dst[i] = value;
}

__global__ __launch_bounds__(kThreads) void arange_kernel(float *__restrict__ dst, int64_t n, int start, int steps) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        dst[i] = static_cast<float>(start + steps * static_cast<int>(i));
}

__global__ __launch_bounds__(kThreads) void copy_kernel(float *__restrict__ dst, const float *__restrict__ src, int64_t n,
                                                       bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t n4 = vec ? n / 4 : 0;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride)
        reinterpret_cast<f32x4 *>(dst)[i] = reinterpret_cast<const f32x4 *>(src)[i];
    for (int64_t i = 4 * n4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

void launch_fill(tensor_t *tensor, float value) {
    if (tensor->length == 0) return;
    gptc_block_written(tensor->t);
    const bool vec = (reinterpret_cast<uintptr_t>(tensor->t) & 15) == 0;
    fill_kernel<<<grid_for(tensor->length / 4 + 1), kThreads, 0, gptc_stream_checked()>>>(tensor->t, tensor->length, value, vec);
    hipCheck(hipGetLastError());
}

}  // namespace

extern "C" void move_tensor_to_host_cuda(tensor_t *tensor) {
    REQUIRE_ARG(tensor);
    CHECK_ERROR(tensor->t == NULL, "%s(): `tensor` has no data buffer.", __func__);
    if (tensor->device == CPU) return;
    hipStream_t s = gptc_stream_checked();
    const size_t nbytes = static_cast<size_t>(tensor->length) * sizeof(float);
    float *host = static_cast<float *>(alignedMallocCheck(64, nbytes ? nbytes : 64));
    hipCheck(hipMemcpyAsync(host, tensor->t, nbytes, hipMemcpyDeviceToHost, s));
    hipCheck(hipStreamSynchronize(s));
    free_cuda(tensor->t);
    tensor->t = host;
    tensor->device = CPU;
}

extern "C" void move_tensor_to_device_cuda(tensor_t *tensor) {
    REQUIRE_ARG(tensor);
    CHECK_ERROR(tensor->t == NULL, "%s(): `tensor` has no data buffer.", __func__);
    if (tensor->device == CUDA) return;
    hipStream_t s = gptc_stream_checked();
    const size_t nbytes = static_cast<size_t>(tensor->length) * sizeof(float);
    float *dev = static_cast<float *>(alloc_cuda(nbytes));
    hipCheck(hipMemcpyAsync(dev, tensor->t, nbytes, hipMemcpyHostToDevice, s));
    hipCheck(hipStreamSynchronize(s));
    free(tensor->t);
    tensor->t = dev;
    tensor->device = CUDA;
}

extern "C" void create_tensor_data_cuda(tensor_t *tensor) {
    REQUIRE_ARG(tensor);
    CHECK_ERROR(tensor->t != NULL, "%s(): the tensor already owns a data buffer (%p).", __func__, (void *)tensor->t);
    tensor->t = static_cast<float *>(alloc_cuda(static_cast<size_t>(tensor->length) * sizeof(float)));
}

extern "C" void zeros_tensor_data_cuda(tensor_t *tensor) {
    REQUIRE_ARG(tensor);
    if (!tensor->t) create_tensor_data_cuda(tensor);
    launch_fill(tensor, 0.0f);
}

extern "C" void ones_tensor_data_cuda(tensor_t *tensor) {
    REQUIRE_ARG(tensor);
    if (!tensor->t) create_tensor_data_cuda(tensor);
    launch_fill(tensor, 1.0f);
}

extern "C" void fill_tensor_data_cuda(tensor_t *tensor, const float value) {
    REQUIRE_ARG(tensor);
    if (!tensor->t) create_tensor_data_cuda(tensor);
    launch_fill(tensor, value);
}

extern "C" void arange_tensor_data_cuda(tensor_t *tensor, const int start, const int end, const int steps) {
    (void)end;
    REQUIRE_ARG(tensor);
    if (!tensor->t) create_tensor_data_cuda(tensor);
    if (tensor->length == 0) return;
    gptc_block_written(tensor->t);
    arange_kernel<<<grid_for(tensor->length), kThreads, 0, gptc_stream_checked()>>>(tensor->t, tensor->length, start, steps);
    hipCheck(hipGetLastError());
}

extern "C" void copy_tensor_data_cuda(tensor_t *dst, const tensor_t *src) {
    REQUIRE_ARG(dst);
    REQUIRE_ARG(src);
    CHECK_ERROR(dst->t == NULL, "%s(): `dst` has no data buffer.", __func__);
    CHECK_ERROR(src->t == NULL, "%s(): `src` has no data buffer.", __func__);
    CHECK_ERROR(src->length != dst->length, "tensor copy: source has %d elements, destination %d.", src->length, dst->length);
    if (src->length == 0) return;
    gptc_block_written(dst->t);
    const bool vec = ((reinterpret_cast<uintptr_t>(dst->t) | reinterpret_cast<uintptr_t>(src->t)) & 15) == 0;
    copy_kernel<<<grid_for(src->length / 4 + 1), kThreads, 0, gptc_stream_checked()>>>(dst->t, src->t, src->length, vec);
    hipCheck(hipGetLastError());
}
