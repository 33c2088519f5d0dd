/*
 * Token-file loader (/root/reference/src/dataloader.c:14-101): raw int32 ids,
 * windows of batch*block + 1 tokens read with one fread, inputs and targets
 * (shifted by one) returned as host float tensors.
 */
#include <stdlib.h>
#include "dataloader.h"
#include "utils.h"

static void dataloader_next(dataloader_t *loader, tensor_t **batch);
static int dataloader_len(dataloader_t *loader);
static void dataloader_reset(dataloader_t *loader);
static void dataloader_free_layer(dataloader_t *loader);

dataloader_t *DataLoader(const char *filename, const int batch_size, const int block_size) {
    CHECK_ERROR(filename == NULL, "Expected *filename to be a const char pointer, but got NULL.");
    CHECK_ERROR(batch_size <= 0, "Expected batch_size to be a positive integer, but got %d.", batch_size);
    CHECK_ERROR(block_size <= 0, "Expected block_size to be a positive integer, but got %d.", block_size);
    dataloader_t *loader = (dataloader_t *)mallocCheck(sizeof(dataloader_t));
    loader->batch_size = batch_size;
    loader->block_size = block_size;
    loader->batch = NULL;
    loader->fp = fopenCheck(filename, "rb");
    loader->_curr_fp_ptr = 0;
    fseekCheck(loader->fp, 0, SEEK_END);
    loader->_file_size = (size_t)ftell(loader->fp);
    fseekCheck(loader->fp, 0, SEEK_SET);
    const size_t window = ((size_t)batch_size * block_size + 1) * sizeof(int);
    CHECK_ERROR(loader->_file_size < window,
                "File size (%zu) is too small for the batch_size (%d) and block_size (%d) given.", loader->_file_size,
                batch_size, block_size);
    loader->next = dataloader_next;
    loader->len = dataloader_len;
    loader->reset = dataloader_reset;
    loader->free_layer = dataloader_free_layer;
    return loader;
}

static void dataloader_next(dataloader_t *loader, tensor_t **batch) {
    CHECK_ERROR(loader == NULL, "Expected *loader to be a dataloader_t pointer, but got NULL.");
    CHECK_ERROR(batch == NULL, "Expected **batch to be a tensor_t pointer, but got NULL.");
    const size_t n = (size_t)loader->batch_size * loader->block_size;
    if (loader->batch == NULL) loader->batch = (int *)mallocCheck(sizeof(int) * (n + 1));
    if (loader->_curr_fp_ptr + (n + 1) * sizeof(int) > loader->_file_size) loader->_curr_fp_ptr = 0;
    fseekCheck(loader->fp, (long)loader->_curr_fp_ptr, SEEK_SET);
    freadCheck(loader->batch, sizeof(int), n + 1, loader->fp);
    loader->_curr_fp_ptr += n * sizeof(int);
    int shape[2] = {loader->batch_size, loader->block_size};
    tensor_t *inputs = create_tensor(shape, 2, CPU);
    tensor_t *targets = create_tensor(shape, 2, CPU);
    for (size_t i = 0; i < n; i++) {
        inputs->t[i] = (float)loader->batch[i];
        targets->t[i] = (float)loader->batch[i + 1];
    }
    batch[0] = inputs;
    batch[1] = targets;
}

static int dataloader_len(dataloader_t *loader) {
    CHECK_ERROR(loader == NULL, "Expected *loader to be a dataloader_t pointer, but got NULL.");
    return (int)(loader->_file_size / (((size_t)loader->batch_size * loader->block_size + 1) * sizeof(int)));
}

static void dataloader_reset(dataloader_t *loader) {
    CHECK_ERROR(loader == NULL, "Expected *loader to be a dataloader_t pointer, but got NULL.");
    loader->_curr_fp_ptr = 0;
}

static void dataloader_free_layer(dataloader_t *loader) {
    if (loader == NULL) return;
    if (loader->fp) fcloseCheck(loader->fp);
    free(loader->batch);
    free(loader);
}
