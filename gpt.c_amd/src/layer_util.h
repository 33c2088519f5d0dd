/*
 * Helpers shared by the layer objects: parameter lists, moves and
 * state loading across devices.
 */
#pragma once

#include <stdlib.h>
#include <string.h>
#include "dispatch.h"
#include "gpu_kernels.h"
#include "tensor.h"
#include "utils.h"

/* A second tensor_t over t's GPU storage: the block gains an owner
 * (gptc_retain_cuda) and returns to the allocator when both are freed.
 * Writes through either are seen by both.  Other tensors are copied. */
static inline tensor_t *share_tensor(const tensor_t *t) {
    if (t->device != CUDA || t->t == NULL) {
        tensor_t *c = create_tensor(t->shape, t->ndims, t->device);
        tensor_copy(c, t);
        return c;
    }
    tensor_t *s = (tensor_t *)mallocCheck(sizeof(tensor_t));
    memcpy(s, t, sizeof(tensor_t));
    gptc_retain_cuda(t->t);
    return s;
}

/* Move a tensor if it exists. */
static inline void move_opt(tensor_t *t, const device_t device) {
    if (t != NULL) t->to(t, device);
}

/* dst's data := src's data (equal lengths, any devices). */
static inline void load_param(tensor_t *dst, const tensor_t *src, const char *what) {
    CHECK_ERROR(dst == NULL || src == NULL, "Cannot load %s: missing tensor.", what);
    CHECK_ERROR(dst->length != src->length, "Cannot load %s. Expected a tensor of size %d, but got %d.", what,
                dst->length, src->length);
    if (dst->device == src->device) {
        copy_tensor_data_dispatch(dst, src);
        return;
    }
    tensor_t *tmp = create_tensor(src->shape, src->ndims, src->device);
    copy_tensor_data_dispatch(tmp, src);
    move_tensor_data_dispatch(tmp, dst->device);
    copy_tensor_data_dispatch(dst, tmp);
    free_tensor(tmp);
}

/* Append the n tensors of list (freed here) to out[*idx...]. */
static inline void append_list(tensor_t **out, int *idx, tensor_t **list, int n) {
    for (int i = 0; i < n; i++) out[(*idx)++] = list[i];
    free(list);
}

/* Leading dimensions of a (..., C) tensor with C replaced by c. */
static inline void shape_with_last(const tensor_t *t, int c, int *shape) {
    for (int i = 0; i < t->ndims; i++) shape[i] = t->shape[i];
    shape[t->ndims - 1] = c;
}
