/* Host-side storage and data ops used by the dispatchers (internal). */
#pragma once

#include <stddef.h>
#include <stdlib.h>
#include "tensor.h"

void *alloc_cpu(const size_t nbytes, const size_t alignment);
void free_cpu(void *ptr);
void create_tensor_data_cpu(tensor_t *tensor);
void fill_tensor_data_cpu(tensor_t *tensor, const float value);
void arange_tensor_data_cpu(tensor_t *tensor, const int start, const int end, const int steps);
void copy_tensor_data_cpu(tensor_t *dst, const tensor_t *src);
