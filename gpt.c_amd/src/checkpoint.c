/*
 * GPT-2 checkpoint reader and writer (train_gpt.c:197-348, the format
 * model.py:246-283 writes); see include/checkpoint.h for the layout.
 */
#include <stdlib.h>
#include <string.h>
#include "checkpoint.h"
#include "utils.h"

gpt2_t *gptc_load_model(const char *path, size_t *steps) {
    FILE *fp = fopenCheck(path, "rb");
    int header[256];
    freadCheck(header, sizeof(int), 256, fp);
    CHECK_ERROR(header[0] != GPTC_CHECKPOINT_MAGIC, "Bad magic model file %s (got %d).", path, header[0]);
    GPT2Config_t cfg;
    cfg.block_size = header[1];
    cfg.vocab_size = header[2];
    cfg.n_layers = header[3];
    cfg.n_heads = header[4];
    cfg.n_embd = header[5];
    const int n_shape = header[6];
    CHECK_ERROR(cfg.block_size <= 0 || cfg.vocab_size <= 0 || cfg.n_layers < 0 || cfg.n_heads <= 0 ||
                    cfg.n_embd <= 0 || cfg.n_embd % cfg.n_heads != 0 || n_shape <= 0,
                "Corrupt model header in %s.", path);
    if (steps != NULL) *steps = (size_t)header[7];
    gpt2_t *model = GPT2(&cfg);
    int *shape_words = (int *)mallocCheck(sizeof(int) * (size_t)n_shape);
    freadCheck(shape_words, sizeof(int), (size_t)n_shape, fp);
    tensor_t **params = model->parameters(model);
    int idx = 0, p = 0;
    while (idx < n_shape) {
        CHECK_ERROR(p >= model->_num_param_tensors, "%s holds more tensors than the model's %d.", path,
                    model->_num_param_tensors);
        const int ndims = shape_words[idx];
        CHECK_ERROR(ndims < 1 || ndims > 8 || idx + 1 + ndims > n_shape, "Corrupt shape words in %s.", path);
        tensor_t *param = params[p];
        CHECK_ERROR(ndims != param->ndims, "Parameter %d: expected %d dims, file has %d.", p, param->ndims, ndims);
        for (int d = 0; d < ndims; d++)
            CHECK_ERROR(shape_words[idx + 1 + d] != param->shape[d],
                        "Parameter %d: dimension %d is %d in the model and %d in %s.", p, d, param->shape[d],
                        shape_words[idx + 1 + d], path);
        idx += ndims + 1;
        p++;
    }
    CHECK_ERROR(p != model->_num_param_tensors, "%s holds %d tensors; the model has %d.", path, p,
                model->_num_param_tensors);
    for (int i = 0; i < p; i++) {
        tensor_t *param = params[i];
        CHECK_ERROR(param->device != CPU, "gptc_load_model builds the model on the CPU.");
        freadCheck(param->t, sizeof(float), (size_t)param->length, fp);
    }
    free(params);
    free(shape_words);
    fcloseCheck(fp);
    return model;
}

void gptc_save_model(const char *path, const gpt2_t *model, const size_t steps) {
    CHECK_ERROR(model == NULL, "Expected *model to be of type gpt2_t. Got NULL.");
    tensor_t **params = model->parameters(model);
    int n_shape = 0;
    for (int i = 0; i < model->_num_param_tensors; i++) n_shape += params[i]->ndims + 1;
    int header[256];
    memset(header, 0, sizeof(header));
    header[0] = GPTC_CHECKPOINT_MAGIC;
    header[1] = model->block_size;
    header[2] = model->vocab_size;
    header[3] = model->n_layers;
    header[4] = model->n_heads;
    header[5] = model->n_embd;
    header[6] = n_shape;
    header[7] = (int)steps;
    int *shape_words = (int *)mallocCheck(sizeof(int) * (size_t)(n_shape > 0 ? n_shape : 1));
    int idx = 0;
    for (int i = 0; i < model->_num_param_tensors; i++) {
        shape_words[idx++] = params[i]->ndims;
        for (int d = 0; d < params[i]->ndims; d++) shape_words[idx++] = params[i]->shape[d];
    }
    FILE *fp = fopenCheck(path, "wb");
    CHECK_ERROR(fwrite(header, sizeof(int), 256, fp) != 256, "Failed to write %s.", path);
    CHECK_ERROR(fwrite(shape_words, sizeof(int), (size_t)n_shape, fp) != (size_t)n_shape, "Failed to write %s.", path);
    for (int i = 0; i < model->_num_param_tensors; i++) tensor_save(fp, params[i]);
    fcloseCheck(fp);
    free(shape_words);
    free(params);
}
