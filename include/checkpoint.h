/*
 * checkpoint.h -- gpt.c's GPT-2 checkpoint file (train_gpt.c:197-348,
 * model.py:246-283), whose reader and writer are static functions of
 * train_gpt.c / infer_gpt.c in gpt.c; here they are library calls.
 *
 * Layout (all little-endian int32 / float32):
 *   header[256]  [0] magic 20240415, [1] block_size, [2] vocab_size,
 *                [3] n_layers, [4] n_heads, [5] n_embd,
 *                [6] number of shape words, [7] training steps, rest 0;
 *   shape words  per parameter: ndims, then its dims;
 *   data         every parameter's floats, in GPT2.parameters() order
 *                (wte, wpe, per block ln1.W, ln1.b, qkv.W, qkv.b,
 *                c_proj.W, c_proj.b, ln2.W, ln2.b, c_fc.W, c_fc.b,
 *                mlp.c_proj.W, mlp.c_proj.b, then ln_f.W, ln_f.b).
 *
 * gptc_load_model(path, steps)  builds a GPT2 on the CPU from the file
 *                               (fatal on a bad magic or a shape mismatch);
 *                               *steps receives header[7] when steps != NULL.
 * gptc_save_model(path, model, steps)
 *                               writes the model (its parameters may live on
 *                               the GPU).
 */
#pragma once

#include <stddef.h>
#include "transformer.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GPTC_CHECKPOINT_MAGIC 20240415

gpt2_t *gptc_load_model(const char *path, size_t *steps);
void gptc_save_model(const char *path, const gpt2_t *model, const size_t steps);

#ifdef __cplusplus
}
#endif
