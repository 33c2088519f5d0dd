/*
 * runtime.h -- device runtime entry points of gpt.c
 * (/root/reference/include/runtime.h:7-9, src/runtime.c:4-14).
 *
 * runtime_init(CUDA) selects HIP device 0 and creates the single
 * non-blocking stream that every kernel, allocation and copy of this
 * library is ordered on.  synchronize(CUDA) waits for that stream.
 * For device == CPU all three are no-ops, as in the reference.
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

void runtime_init(const device_t device);
void runtime_destroy(const device_t device);
void synchronize(const device_t device);

#ifdef __cplusplus
}
#endif
