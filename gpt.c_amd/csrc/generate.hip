// One-token GPT-2 steps over per-layer K/V caches (include/generate.h).
// gpt.c has no such step: infer_gpt.c:339-351 recomputes the whole window
// through GPT2.forward (src/transformer.c:69-111) for every token.  This
// computes the same model (src/block.c:54-90, src/self_attention.c:47-64,
// src/mlp.c:46-57) for one position of each sequence:
//   x = wte[id] + wpe[pos]
//   per block: h = ln1(x); qkv = h Wqkv^T + b; a = attention over cached keys
//              0..pos (which also stores this token's k, v at pos);
//              x2 = x + a Wproj^T + b; h2 = ln2(x2); f = gelu(h2 Wfc^T + b);
//              x = x2 + f Wmproj^T + b
//   logits = ln_f(x) wte^T
// with the small-row kernels of decode_ops.hip: every weight is read once per
// token.  At B = 1 a step is about 90 short launches, so greedy generation
// (gptc_gpt2_generate) captures one step as a HIP graph with the position in
// device memory and replays it, instead of launching and waiting per token.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include "generate.h"
#include "gpu_kernels.h"
#include "ops_common.hpp"

using namespace gptc;

namespace {

enum { S_X, S_PART, S_QKV, S_A, S_X2, S_MEAN, S_RSTD, S_F };  // S_PART: split-key decode partials

// The blocks, ln_f and lm_head of one step, from s[S_X] to logits.  pos_dev
// set: the attention reads the position from device memory.
void step_body(gpt2_t *gpt, gptc_kv_cache_t *kv, int pos, const int *pos_dev, tensor_t *logits) {
    // Each LayerNorm is folded into the linear that consumes it (the row's
    // statistics are recomputed by each workgroup): 6 launches per block.
    tensor_t **s = kv->scratch;
    for (int l = 0; l < gpt->n_layers; l++) {
        const block_t *blk = gpt->layers[l];
        const self_attention_t *sa = blk->attn;
        const mlp_t *mlp = blk->mlp;
        ln_linear_rows(blk->ln1->W, blk->ln1->b, blk->ln1->eps, sa->qkv->W, sa->qkv->b, s[S_X], NULL, 0, s[S_QKV]);
        attention_decode_cached(s[S_QKV], kv->k[l], kv->v[l], pos, pos_dev, gpt->n_heads, s[S_A], s[S_PART]->t);
        gptc_linear_rows_cuda(sa->c_proj->W, sa->c_proj->b, s[S_A], s[S_X], 0, s[S_X2]);
        ln_linear_rows(blk->ln2->W, blk->ln2->b, blk->ln2->eps, mlp->c_fc->W, mlp->c_fc->b, s[S_X2], NULL, 1,
                       s[S_F]);
        gptc_linear_rows_cuda(mlp->c_proj->W, mlp->c_proj->b, s[S_F], s[S_X2], 0, s[S_X]);
    }
    ln_linear_rows(gpt->ln_f->W, gpt->ln_f->b, gpt->ln_f->eps, gpt->wte->W, NULL, s[S_X], NULL, 0, logits);
}

void check_model(const gpt2_t *gpt, const gptc_kv_cache_t *kv) {
    REQUIRE_ARG(gpt);
    REQUIRE_ARG(kv);
    CHECK_ERROR(gpt->wte->W->device != CUDA, "Generation runs on the GPU: move the model there first.");
    CHECK_ERROR(kv->n_layers != gpt->n_layers, "The cache was made for %d layers, the model has %d.", kv->n_layers,
                gpt->n_layers);
}

void drop_graph(gptc_kv_cache_t *kv) {
    if (kv->graph_exec != nullptr) hipCheck(hipGraphExecDestroy(static_cast<hipGraphExec_t>(kv->graph_exec)));
    kv->graph_exec = nullptr;
    free(kv->graph_key);
    kv->graph_key = nullptr;
    kv->graph_key_len = 0;
}

// Every value the captured step's launches take as an argument and that a
// caller can change between calls: the model object, each parameter's
// device address, the LayerNorm eps values, the shapes, the token buffer,
// prompt and total.  (The cache's own buffers are fixed for its lifetime.)
// Returns a malloc'd array of *len words.
unsigned long long *graph_key(const gpt2_t *gpt, const tensor_t *tokens, int prompt, int total, int *len) {
    const int np = gpt->_num_param_tensors;
    const int n = 8 + np + 2 * gpt->n_layers + 1;
    auto *key = static_cast<unsigned long long *>(mallocCheck(sizeof(unsigned long long) * n));
    int i = 0;
    auto bits = [](float f) {
        unsigned u;
        memcpy(&u, &f, sizeof(u));
        return static_cast<unsigned long long>(u);
    };
    key[i++] = reinterpret_cast<uintptr_t>(gpt);
    key[i++] = reinterpret_cast<uintptr_t>(tokens->t);
    key[i++] = static_cast<unsigned long long>(prompt);
    key[i++] = static_cast<unsigned long long>(total);
    key[i++] = static_cast<unsigned long long>(gpt->n_heads);
    key[i++] = static_cast<unsigned long long>(gpt->n_embd);
    key[i++] = static_cast<unsigned long long>(gpt->vocab_size);
    key[i++] = static_cast<unsigned long long>(np);
    tensor_t **params = gpt->parameters(gpt);
    for (int p = 0; p < np; p++) key[i++] = reinterpret_cast<uintptr_t>(params[p]->t);
    free(params);
    for (int l = 0; l < gpt->n_layers; l++) {
        key[i++] = bits(gpt->layers[l]->ln1->eps);
        key[i++] = bits(gpt->layers[l]->ln2->eps);
    }
    key[i++] = bits(gpt->ln_f->eps);
    *len = i;
    return key;
}

}  // namespace

extern "C" gptc_kv_cache_t *gptc_kv_cache_create(const gpt2_t *gpt, const int B, const int L) {
    REQUIRE_ARG(gpt);
    CHECK_ERROR(B < 1 || B > 8, "The decode step takes 1 .. 8 sequences, but got B = %d.", B);
    CHECK_ERROR(L < 1 || L > gpt->block_size, "Expected 1 <= L <= block_size = %d, but got L = %d.", gpt->block_size,
                L);
    const int C = gpt->n_embd, H = gpt->n_heads, D = C / H;
    gptc_kv_cache_t *kv = static_cast<gptc_kv_cache_t *>(mallocCheck(sizeof(gptc_kv_cache_t)));
    kv->n_layers = gpt->n_layers;
    kv->B = B;
    kv->L = L;
    const int nl = gpt->n_layers > 0 ? gpt->n_layers : 1;
    kv->k = static_cast<tensor_t **>(mallocCheck(sizeof(tensor_t *) * nl));
    kv->v = static_cast<tensor_t **>(mallocCheck(sizeof(tensor_t *) * nl));
    int cshape[4] = {B, H, L, D};
    for (int l = 0; l < gpt->n_layers; l++) {
        kv->k[l] = zeros(cshape, 4, CUDA);
        kv->v[l] = zeros(cshape, 4, CUDA);
    }
    int s_bc[3] = {B, 1, C}, s_b3c[3] = {B, 1, 3 * C}, s_b[1] = {B}, s_b4c[3] = {B, 1, 4 * C};
    int s_bv[3] = {B, 1, gpt->vocab_size};
    kv->scratch[S_X] = create_tensor(s_bc, 3, CUDA);
    int s_part[1] = {static_cast<int>(attention_decode_part_floats(B, H, L))};
    kv->scratch[S_PART] = create_tensor(s_part, 1, CUDA);
    kv->scratch[S_QKV] = create_tensor(s_b3c, 3, CUDA);
    kv->scratch[S_A] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_X2] = create_tensor(s_bc, 3, CUDA);
    kv->scratch[S_MEAN] = create_tensor(s_b, 1, CUDA);
    kv->scratch[S_RSTD] = create_tensor(s_b, 1, CUDA);
    kv->scratch[S_F] = create_tensor(s_b4c, 3, CUDA);
    kv->logits = create_tensor(s_bv, 3, CUDA);
    kv->pos_dev = static_cast<int *>(alloc_cuda(sizeof(int)));
    kv->graph_exec = nullptr;
    kv->graph_key = nullptr;
    kv->graph_key_len = 0;
    return kv;
}

extern "C" void gptc_kv_cache_free(gptc_kv_cache_t *kv) {
    if (kv == NULL) return;
    drop_graph(kv);
    for (int l = 0; l < kv->n_layers; l++) {
        free_tensor(kv->k[l]);
        free_tensor(kv->v[l]);
    }
    free(kv->k);
    free(kv->v);
    for (int i = 0; i < 8; i++) free_tensor(kv->scratch[i]);
    free_tensor(kv->logits);
    free_cuda(kv->pos_dev);
    free(kv);
}

extern "C" tensor_t *gptc_gpt2_decode(gpt2_t *gpt, gptc_kv_cache_t *kv, const tensor_t *ids, const int pos) {
    check_model(gpt, kv);
    CHECK_ERROR(ids == NULL || ids->device != CUDA, "Expected the ids as a GPU tensor.");
    CHECK_ERROR(ids->length != kv->B, "Expected %d ids (one per sequence), but got %d.", kv->B, ids->length);
    CHECK_ERROR(pos < 0 || pos >= kv->L, "Expected 0 <= pos < L = %d, but got pos = %d.", kv->L, pos);
    gptc_embed_token_cuda(gpt->wte->W, gpt->wpe->W, ids, pos, kv->scratch[S_X]);
    int lshape[3] = {kv->B, 1, gpt->vocab_size};
    tensor_t *logits = create_tensor(lshape, 3, CUDA);
    step_body(gpt, kv, pos, nullptr, logits);
    return logits;
}

extern "C" void gptc_gpt2_generate(gpt2_t *gpt, gptc_kv_cache_t *kv, tensor_t *tokens, const int prompt,
                                   const int total) {
    check_model(gpt, kv);
    CHECK_ERROR(tokens == NULL || tokens->device != CUDA, "Expected the token buffer as a GPU tensor.");
    CHECK_ERROR(tokens->ndims != 2 || tokens->shape[0] != kv->B || tokens->shape[1] != total,
                "Expected a (%d, %d) token buffer.", kv->B, total);
    CHECK_ERROR(prompt < 1 || prompt > total || total > kv->L,
                "Expected 1 <= prompt <= total <= L = %d, but got prompt %d, total %d.", kv->L, prompt, total);
    if (total == prompt) return;  // nothing to generate
    hipStream_t s = gptc_stream_checked();
    int key_len = 0;
    unsigned long long *key = graph_key(gpt, tokens, prompt, total, &key_len);
    const bool reuse = kv->graph_exec != nullptr && kv->graph_key_len == key_len &&
                       memcmp(kv->graph_key, key, sizeof(unsigned long long) * key_len) == 0;
    if (reuse) {
        free(key);
    } else {
        drop_graph(kv);
        // The captured step: every launch reads the position from kv->pos_dev.
        hipGraph_t graph;
        hipCheck(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        launch_embed_tokens_devpos(gpt->wte->W, gpt->wpe->W, tokens->t, kv->B, total, kv->pos_dev, kv->scratch[S_X]);
        step_body(gpt, kv, 0, kv->pos_dev, kv->logits);
        launch_argmax_next(kv->logits, tokens->t, total, kv->pos_dev, prompt, total);
        launch_advance_pos(kv->pos_dev);
        hipCheck(hipStreamEndCapture(s, &graph));
        hipGraphExec_t exec;
        hipCheck(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        hipCheck(hipGraphDestroy(graph));
        kv->graph_exec = exec;
        kv->graph_key = key;
        kv->graph_key_len = key_len;
    }
    // Position 0, then one replay per position 0 .. total-2 (each reads the
    // token at pos and writes the token at pos + 1 once past the prompt).
    const int zero = 0;
    hipCheck(hipMemcpyAsync(kv->pos_dev, &zero, sizeof(int), hipMemcpyHostToDevice, s));
    hipCheck(hipStreamSynchronize(s));  // `zero` lives on this frame
    for (int p = 0; p + 1 < total; ++p) hipCheck(hipGraphLaunch(static_cast<hipGraphExec_t>(kv->graph_exec), s));
}
