/*
 * dataloader.h -- gpt.c's token-file loader, unchanged interface
 * (/root/reference/include/dataloader.h:32-52).  The file is raw int32 token
 * ids (data/common.py:35-48).  next() returns (inputs, targets) as two new
 * host tensors of shape (batch_size, block_size): a window of
 * batch_size*block_size + 1 tokens, targets shifted by one.  Successive
 * windows advance by batch_size*block_size tokens and wrap to the start when
 * the next window would pass the end.  len() is the number of windows.
 */
#pragma once

#include <stdio.h>
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dataloader {
    int batch_size;
    int block_size;
    FILE *fp;
    int *batch;
    size_t _file_size;
    size_t _curr_fp_ptr;
    void (*next)(struct dataloader *, tensor_t **);
    int (*len)(struct dataloader *);
    void (*reset)(struct dataloader *);
    void (*free_layer)(struct dataloader *);
} __attribute__((aligned(64))) dataloader_t;

dataloader_t *DataLoader(const char *filename, const int batch_size, const int block_size);

#ifdef __cplusplus
}
#endif
