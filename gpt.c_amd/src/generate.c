/*
 * One-token GPT-2 step over per-layer K/V caches (include/generate.h).
 * gpt.c has no such step: infer_gpt.c:339-351 recomputes the whole window
 * through GPT2.forward (src/transformer.c:69-111) for every token.  This
 * computes the same model (src/block.c:54-90, src/self_attention.c:47-64,
 * src/mlp.c:46-57) for one position of each sequence:
 *   x = wte[id] + wpe[pos]
 *   per block: h = ln1(x); qkv = h Wqkv^T + b; a = attention over cached
 *              keys 0..pos (attention_decode_cuda_kernel, which also stores
 *              this token's k, v at pos); x2 = x + a Wproj^T + b;
 *              h2 = ln2(x2); f = gelu(h2 Wfc^T + b); x = x2 + f Wmproj^T + b
 *   logits = ln_f(x) wte^T
 * with the small-row kernels of gpu_kernels.h (each weight read once).
 * The step's activations live in the cache object and are reused.
 */
#include <stdlib.h>
#include "generate.h"
#include "gpu_kernels.h"
#include "utils.h"

enum { S_X, S_H, S_QKV, S_A, S_X2, S_MEAN, S_RSTD, S_F };

gptc_kv_cache_t *gptc_kv_cache_create(const gpt2_t *gpt, const int B, const int L) {
    CHECK_ERROR(gpt == NULL, "Expected *gpt to be a gpt2_t pointer, but got NULL.");
    CHECK_ERROR(B < 1 || B > 8, "The decode step takes 1 .. 8 sequences, but got B = %d.", B);
    CHECK_ERROR(L < 1 || L > gpt->block_size, "Expected 1 <= L <= block_size = %d, but got L = %d.", gpt->block_size, L);
    const int C = gpt->n_embd, H = gpt->n_heads, D = C / H;
    gptc_kv_cache_t *kv = (gptc_kv_cache_t *)mallocCheck(sizeof(gptc_kv_cache_t));
    kv->n_layers = gpt->n_layers;
    kv->B = B;
    kv->L = L;
    kv->k = (tensor_t **)mallocCheck(sizeof(tensor_t *) * (gpt->n_layers > 0 ? gpt->n_layers : 1));
    kv->v = (tensor_t **)mallocCheck(sizeof(tensor_t *) * (gpt->n_layers > 0 ? gpt->n_layers : 1));
    int cshape[4] = {B, H, L, D};
    for (int l = 0; l < gpt->n_layers; l++) {
        kv->k[l] = zeros(cshape, 4, CUDA);
        kv->v[l] = zeros(cshape, 4, CUDA);
    }
    int s_bc[3] = {B, 1, C}, s_b3c[3] = {B, 1, 3 * C}, s_b[1] = {B}, s_b4c[3] = {B, 1, 4 * C};
    kv->scratch[S_X] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_H] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_QKV] = create_tensor(s_b3c, 3, CUDA);
    kv->scratch[S_A] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_X2] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_MEAN] = create_tensor(s_b, 1, CUDA);
    kv->scratch[S_RSTD] = create_tensor(s_b, 1, CUDA);
    kv->scratch[S_F] = create_tensor(s_b4c, 3, CUDA);
    return kv;
}

void gptc_kv_cache_free(gptc_kv_cache_t *kv) {
    if (kv == NULL) return;
    for (int l = 0; l < kv->n_layers; l++) {
        free_tensor(kv->k[l]);
        free_tensor(kv->v[l]);
    }
    free(kv->k);
    free(kv->v);
    for (int i = 0; i < 8; i++) free_tensor(kv->scratch[i]);
    free(kv);
}

static void layer_norm_rows(const layer_norm_t *ln, const tensor_t *x, gptc_kv_cache_t *kv, tensor_t *y) {
    tensor_t *stats[2] = {kv->scratch[S_MEAN], kv->scratch[S_RSTD]};
    layer_norm_forward_cuda_kernel(ln->W, ln->b, x, ln->eps, stats, y);
}

tensor_t *gptc_gpt2_decode(gpt2_t *gpt, gptc_kv_cache_t *kv, const tensor_t *ids, const int pos) {
    CHECK_ERROR(gpt == NULL || kv == NULL || ids == NULL, "gptc_gpt2_decode: NULL model, cache or ids.");
    CHECK_ERROR(ids->device != CUDA || gpt->wte->W->device != CUDA, "gptc_gpt2_decode runs on the GPU: move the "
                "model and the ids there first.");
    CHECK_ERROR(ids->length != kv->B, "Expected %d ids (one per sequence), but got %d.", kv->B, ids->length);
    CHECK_ERROR(kv->n_layers != gpt->n_layers, "The cache was made for %d layers, the model has %d.", kv->n_layers,
                gpt->n_layers);
    CHECK_ERROR(pos < 0 || pos >= kv->L, "Expected 0 <= pos < L = %d, but got pos = %d.", kv->L, pos);
    tensor_t **s = kv->scratch;
    gptc_embed_token_cuda(gpt->wte->W, gpt->wpe->W, ids, pos, s[S_X]);
    for (int l = 0; l < gpt->n_layers; l++) {
        const block_t *blk = gpt->layers[l];
        const self_attention_t *sa = blk->attn;
        const mlp_t *mlp = blk->mlp;
        layer_norm_rows(blk->ln1, s[S_X], kv, s[S_H]);
        gptc_linear_rows_cuda(sa->qkv->W, sa->qkv->b, s[S_H], NULL, 0, s[S_QKV]);
        attention_decode_cuda_kernel(s[S_QKV], kv->k[l], kv->v[l], pos, gpt->n_heads, s[S_A]);
        gptc_linear_rows_cuda(sa->c_proj->W, sa->c_proj->b, s[S_A], s[S_X], 0, s[S_X2]);
        layer_norm_rows(blk->ln2, s[S_X2], kv, s[S_H]);
        gptc_linear_rows_cuda(mlp->c_fc->W, mlp->c_fc->b, s[S_H], NULL, 1, s[S_F]);
        gptc_linear_rows_cuda(mlp->c_proj->W, mlp->c_proj->b, s[S_F], s[S_X2], 0, s[S_X]);
    }
    layer_norm_rows(gpt->ln_f, s[S_X], kv, s[S_H]);
    int lshape[3] = {kv->B, 1, gpt->vocab_size};
    tensor_t *logits = create_tensor(lshape, 3, CUDA);
    gptc_linear_rows_cuda(gpt->wte->W, NULL, s[S_H], NULL, 0, logits);
    return logits;
}
