/*
 * loss.h -- gpt.c's CrossEntropyLoss, unchanged interface
 * (/root/reference/include/loss.h:34-50).  forward(logits, targets) returns
 * a 1-element tensor holding the mean loss; the logits are not consumed,
 * the targets are (they become cache[1]).  cache[0] holds the log-softmax.
 * backward(g) with g (B, T) returns dlogits (B, T, V) and consumes g and the
 * cache.
 */
#pragma once

#include "activation.h"
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cross_entropy_loss {
    softmax_t *softmax;
    tensor_t *cache[2];
    tensor_t *(*forward)(struct cross_entropy_loss *, tensor_t *, tensor_t *);
    tensor_t *(*backward)(struct cross_entropy_loss *, tensor_t *);
    void (*description)(const struct cross_entropy_loss *);
    int (*num_parameters)(const struct cross_entropy_loss *);
    void (*free_layer)(struct cross_entropy_loss *);
    void (*free_cache)(struct cross_entropy_loss *);
    void (*to)(struct cross_entropy_loss *, const device_t);
} __attribute__((aligned(64))) cross_entropy_loss_t;

cross_entropy_loss_t *CrossEntropyLoss(void);

#ifdef __cplusplus
}
#endif
