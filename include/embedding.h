/*
 * embedding.h -- gpt.c's Embedding layer, unchanged interface
 * (/root/reference/include/embedding.h:34-59).  forward(ids) with float ids
 * returns (…, embedding_dim) rows of W and keeps ids as the cache;
 * backward(g) accumulates into dW, consumes g and the cache and returns
 * NULL, as the reference does.
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct embedding {
    tensor_t *W;
    tensor_t *dW;
    tensor_t *cache;

    tensor_t *(*forward)(struct embedding *, tensor_t *);
    tensor_t *(*backward)(struct embedding *, tensor_t *);
    void (*description)(const struct embedding *);
    int (*num_parameters)(const struct embedding *);
    void (*free_layer)(struct embedding *);
    void (*free_cache)(struct embedding *);
    tensor_t **(*parameters)(const struct embedding *);
    tensor_t **(*gradients)(const struct embedding *);
    void (*load_state_dict)(struct embedding *, tensor_t **);
    void (*to)(struct embedding *, const device_t);

    int num_embeddings;
    int embedding_dim;
    int _num_param_tensors;
    char __padding[4];
} __attribute__((aligned(64))) embedding_t;

embedding_t *Embedding(int num_embeddings, int embedding_dim);

#ifdef __cplusplus
}
#endif
