// Fatal HIP error check (the reference's cudaCheck convention,
// kernels/src/cuda/cuda_common.h:61-68: print and exit(EXIT_FAILURE)).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

inline void hip_check(hipError_t err, const char *file, int line) {
    if (err != hipSuccess) {
        std::fprintf(stderr, "[HIP ERROR] at file %s:%d: %s\n", file, line, hipGetErrorString(err));
        std::fflush(stderr);
        std::exit(EXIT_FAILURE);
    }
}
#define hipCheck(err) hip_check((err), __FILE__, __LINE__)

// The one stream every launch, copy and allocation of the library uses
// (fatal if runtime_init_cuda() has not run).
hipStream_t gptc_stream_checked();

// The serial of the live alloc_cuda block starting at ptr (0 if it is none):
// new at each allocation of the block and at each write of the library's
// tensor data ops into it (gptc_block_written).
uint64_t gptc_block_serial(const void *ptr);
void gptc_block_written(const void *ptr);
