/*
 * gpu_kernels.h -- the C-ABI that this library exports for gpt.c's GPU
 * device.  Every symbol keeps the name, argument list and meaning of the
 * CUDA back end it replaces, so gpt.c's device dispatchers
 * (the files of kernels/src/core/) link against this library instead of
 * the CUDA objects without a source change.  Plain pointers and sizes only; errors
 * are fatal (print + exit(EXIT_FAILURE)), as in the reference.
 *
 * All device work is ordered on one non-blocking HIP stream created by
 * runtime_init_cuda().
 */
#pragma once

#include <stddef.h>
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime: replaces kernels/src/cuda/runtime.h:7-9 (runtime.cu:16-52) ---- */
void runtime_init_cuda(void);
void runtime_destroy_cuda(void);
void synchronize_cuda(void);

/* ---- stream-ordered allocation: replaces kernels/src/cuda/Alloc.h:10-12 ---- */
void *alloc_cuda(const size_t nbytes);
void free_cuda(void *ptr);
/* No counterpart in the reference: adds an owner to a block returned by
 * alloc_cuda, so that it survives until free_cuda has been called once per
 * owner (a tensor that shares another tensor's storage). */
void gptc_retain_cuda(void *ptr);

/* ---- tensor data ops: replace kernels/src/cuda/Tensor.h:9-17 ---- */
void move_tensor_to_host_cuda(tensor_t *tensor);
void move_tensor_to_device_cuda(tensor_t *tensor);
void create_tensor_data_cuda(tensor_t *tensor);
void zeros_tensor_data_cuda(tensor_t *tensor);
void ones_tensor_data_cuda(tensor_t *tensor);
void fill_tensor_data_cuda(tensor_t *tensor, const float value);
void arange_tensor_data_cuda(tensor_t *tensor, const int start, const int end, const int steps);
void copy_tensor_data_cuda(tensor_t *dst, const tensor_t *src);

/*
 * ---- causal self-attention: replaces kernels/src/cuda/Attention.h:9-22 ----
 *
 * attention_forward_cuda_kernel(input, mask, n_heads, cache, output)
 *   input  (B, T, 3C) qkv, device.  output (B, T, C), device, overwritten.
 *   mask   the layer's (block, block) lower-triangular buffer; block >= T is
 *          checked.  The kernel applies the causal rule key <= query from
 *          indices; the buffer itself is never read on the device.
 *   cache  four device tensors allocated by the caller.  Two layouts are
 *          accepted and told apart by cache[0]:
 *          - compact (this library's attention.c): cache[0] IS the input
 *            tensor (ownership passed to the layer), cache[1] (B, T, C)
 *            is the output's storage itself (attention.c shares it) or,
 *            when it is a buffer of its own, receives a copy of the
 *            output; cache[2] (B, H, T) receives the
 *            row log-sum-exp, cache[3] receives the backward state: the
 *            causal blocks of the probabilities (about B*H*T*T/2 floats)
 *            and their per-tile row maxima.  A cache[3] that is not a 1-D
 *            tensor of gptc_attention_state_floats() floats is re-pointed
 *            to one (stream-ordered free + alloc);
 *          - reference (gpt.c's unchanged attention.c:105-120): cache[0..2]
 *            (B, H, T, D) receive the permuted q, k, v exactly as gpt.c's
 *            CPU kernel writes them; cache[3], allocated (B, H, T, T), is
 *            re-pointed to a 1-D buffer holding the output copy, the
 *            log-sum-exp and the backward state (about half the size of
 *            the B*H*T*T probability matrix gpt.c keeps there).
 *   Supported head sizes: 1 <= D <= 1024 (D = C / n_heads; fatal before
 *   any launch otherwise).  D <= 128 runs the MFMA kernels, 128 < D <= 1024
 *   plain-FMA kernels that keep the LSE-only state.  The state must fit the
 *   int length of a tensor_t (checked, fatal otherwise).
 *
 * attention_backward_cuda_kernel(global_grad, cache, n_heads, dout)
 *   global_grad (B, T, C) upstream gradient (may be clobbered by the caller
 *   afterwards), cache as left by the forward, dout (B, T, 3C) receives
 *   dq | dk | dv.  Every element of dout is written (no accumulation), so
 *   dout need not be zeroed; a zeroed dout (gpt.c attention.c:142-143)
 *   gives the same result.  The backward consumes cache[3] (its dS
 *   overwrites the stored probabilities), as gpt.c's backward, which
 *   frees the cache right after (attention.c:147-155), permits; a second
 *   backward needs a new forward.  It allocates nothing per call: the work
 *   lists of its D = 64 kernels (a few KB per shape) are built and uploaded
 *   on the first backward of a shape and kept for the life of the process.
 */
void attention_forward_cuda_kernel(
    const tensor_t *input,
    const tensor_t *mask,
    const int n_heads,
    tensor_t **cache,
    tensor_t *output
);

void attention_backward_cuda_kernel(
    const tensor_t *global_grad,
    tensor_t **cache,
    const int n_heads,
    tensor_t *dout
);

/*
 * ---- the qkv Linear's bias folded into attention: no counterpart in the
 * reference (gpt.c's SelfAttention adds it in the Linear, self_attention.c:59,
 * and sums its gradient there, linear.c's backward) ----
 *
 * gptc_attention_forward_qkv_bias(input, bias, mask, n_heads, cache, output)
 *   As attention_forward_cuda_kernel with the compact cache layout, where
 *   input = x W^T holds the qkv Linear's product without its bias (3C): the
 *   D = 64 kernels add the bias as they load q, k and v (the 75 MB bias
 *   pass over the qkv activations at GPT-2 small's B=8 T=1024 disappears);
 *   other head sizes have it added to the input in place first.
 * gptc_attention_backward_qkv_bias(global_grad, cache, bias, n_heads, dout, db)
 *   As attention_backward_cuda_kernel after that forward, and db (3C) +=
 *   the column sums of dout (the bias gradient of the qkv Linear), formed
 *   from per-workgroup sums in the kernels' epilogues and added in a fixed
 *   order (deterministic).
 */
void gptc_attention_forward_qkv_bias(const tensor_t *input, const tensor_t *bias, const tensor_t *mask,
                                     const int n_heads, tensor_t **cache, tensor_t *output);
void gptc_attention_backward_qkv_bias(const tensor_t *global_grad, tensor_t **cache, const tensor_t *bias,
                                      const int n_heads, tensor_t *dout, tensor_t *db);

/*
 * gptc_gelu_forward_bias_cuda(input, bias, output)
 *   output = gelu(input + bias), bias per last-dim column.  No counterpart in
 *   the reference, whose MLP adds c_fc's bias in the Linear and then runs
 *   GELU (src/mlp.c): here the MLP's c_fc runs without it and this adds it
 *   on the way into GELU (one pass over the 8192 x 3072 activations at
 *   GPT-2 small's B=8 T=1024 instead of two).
 * gptc_gelu_backward_bias_cuda(global_grad, cache, bias, dout, db)
 *   dout = global_grad * gelu'(cache + bias) (written), and db += the column
 *   sums of dout, formed from per-workgroup partials as dout is written and
 *   added in a fixed order (deterministic): c_fc's bias gradient without a
 *   second pass over dout.
 */
void gptc_gelu_forward_bias_cuda(const tensor_t *input, const tensor_t *bias, tensor_t *output);
void gptc_gelu_backward_bias_cuda(const tensor_t *global_grad, const tensor_t *cache, const tensor_t *bias,
                                  tensor_t *dout, tensor_t *db);

/*
 * gptc_layer_norm_backward_set(global_grad, cache, W, dW, db, dout)
 *   As layer_norm_backward_cuda_kernel, but dout = dx instead of dout += dx
 *   (dout is not read).  No counterpart in the reference: gpt.c's LayerNorm
 *   layer zero-fills a new dout before the accumulating kernel
 *   (src/layer_norm.c:127-135); the layer here calls this and skips the fill
 *   and the read of the zeros (50 MB per call at GPT-2 small's B=8 T=1024).
 */
void gptc_layer_norm_backward_set(const tensor_t *global_grad, const tensor_t **cache, const tensor_t *W,
                                  tensor_t *dW, tensor_t *db, tensor_t *dout);

/*
 * ---- the rest of gpt.c's GPU back end (the other layers of the model) ----
 * Same names, arguments and meaning as the CUDA entry points they replace;
 * the semantics are those of gpt.c's CPU kernels (kernels/src/cpu/), which
 * the CUDA ones follow.  Rows are the product of all dimensions but the
 * last (B*T for gpt.c's (B, T, C) tensors).  Every device buffer is checked
 * against the shapes before a launch (fatal on mismatch).
 */

/* BLAS, replaces kernels/src/cuda/Tensor.h:18-36 (Tensor.cu:132-206).
 * Row-major, op = transpose when Trans* == 1.  The GEMMs are rocBLAS fp32
 * (the reference runs cuBLAS in TF32 on sm >= 80), without atomic split-K,
 * so results are deterministic.  saxpy requires incx, incy >= 1. */
void saxpy_cuda(
    const int n, const float alpha,
    const tensor_t *x, const int offsetx, const int incx,
    tensor_t *y, const int offsety, const int incy
);
void sgemm_cuda(
    const int TransA, const int TransB, const int M, const int N, const int K,
    const float alpha, const tensor_t *A, const int offsetA, const int lda,
    const tensor_t *B, const int offsetB, const int ldb,
    const float beta, tensor_t *C, const int offsetC, const int ldc
);
void sgemm_strided_batched_cuda(
    const int TransA, const int TransB, const int M, const int N, const int K,
    const float alpha, const tensor_t *A, const int lda, const int strideA,
    const tensor_t *B, const int ldb, const int strideB,
    const float beta, tensor_t *C, const int ldc, const int strideC, const int batch_count
);

/* Linear, replaces kernels/src/cuda/Linear.h:9-17 (cpu/Linear.c:4-80).
 * forward: output = input W^T (+ b).  backward: dout = global_grad W
 * (overwritten), dW += global_grad^T cache, db += column sums of global_grad
 * (deterministic two-pass sum). */
void linear_forward_cuda_kernel(const tensor_t *W, const tensor_t *b, const tensor_t *input, tensor_t *output);
void linear_backward_cuda_kernel(
    const tensor_t *global_grad, const tensor_t *cache, const tensor_t *W,
    tensor_t *dW, tensor_t *db, tensor_t *dout
);

/* LayerNorm, replaces kernels/src/cuda/LayerNorm.h:9-25 (cpu/LayerNorm.c:5-124).
 * cache[0] mean and cache[1] rstd (one per row), cache[2] the input.
 * backward: dout += dx, dW += ..., db += ... (accumulate, as the reference).
 * Up to 2048 features (fatal beyond). */
void layer_norm_forward_cuda_kernel(
    const tensor_t *W, const tensor_t *b, const tensor_t *input, const float eps,
    tensor_t **cache, tensor_t *output
);
void layer_norm_backward_cuda_kernel(
    const tensor_t *global_grad, const tensor_t **cache, const tensor_t *W,
    tensor_t *dW, tensor_t *db, tensor_t *dout
);

/* GELU (tanh form), replaces kernels/src/cuda/GeLU.h:9-15 (cpu/GeLU.c:7-42).
 * backward writes dout = global_grad * gelu'(cache). */
void gelu_forward_cuda_kernel(const tensor_t *input, tensor_t *output);
void gelu_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout);

/* Softmax over the last dimension, replaces kernels/src/cuda/Softmax.h:9-15
 * (cpu/Softmax.c:7-63).  cache = the forward's output. */
void softmax_forward_cuda_kernel(const tensor_t *input, tensor_t *output);
void softmax_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout);

/* Embedding, replaces kernels/src/cuda/Embedding.h:9-19 (cpu/Embedding.c:3-47).
 * Ids are floats truncated to int.  backward: dW[ids[i % len(ids)]] += g[i],
 * deterministic (rows of one id are added in row order by one wave).  Ids
 * outside [0, V): the forward writes a NaN row, the backward skips them. */
void embedding_forward_cuda_kernel(const tensor_t *W, const tensor_t *input, tensor_t *output);
void embedding_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dW);

/* Cross-entropy, replaces kernels/src/cuda/CrossEntropyLoss.h:9-20
 * (cpu/CrossEntropyLoss.c:7-97).  forward: cache[0] (B,T,V) receives the
 * log-softmax, output[0] the mean loss (a target outside [0, V) gives NaN).
 * backward: cache[1] = targets; dout (B,T,V) is overwritten with
 * (softmax - onehot(target)) * global_grad / (B*T). */
void cross_entropy_forward_cuda_kernel(
    const tensor_t *logits, const tensor_t *targets, tensor_t **cache, tensor_t *output
);
void cross_entropy_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t **cache, tensor_t *dout);

/* AdamW, replaces kernels/src/cuda/AdamW.h:9-24 (cpu/AdamW.c:5-58).
 * One launch per 36 tensors of the list. */
void step_adamW_cuda_kernel(
    tensor_t **parameters, tensor_t **gradients, tensor_t **m, tensor_t **v,
    const int n, const float lr, const float beta1, const float beta2,
    const float weight_decay, const float eps, const int step
);
void zero_grad_adamW_cuda_kernel(tensor_t **gradients, const int n);

/*
 * ---- KV-cache decode: no counterpart in the reference ----
 *
 * attention_decode_cuda_kernel(qkv, k_cache, v_cache, pos, n_heads, output)
 *   One generation step of causal self-attention with a KV cache.  gpt.c's
 *   inference loop (infer_gpt.c:339-351) has no cache: it runs the whole
 *   window through attention_forward_cuda_kernel for every new token and
 *   keeps one row.  This call returns that row directly.
 *   qkv      (B, 1, 3C) device: the new token's q | k | v (the c_attn row).
 *   k_cache, v_cache (B, H, L, D) device, the (B, H, T, D) layout of gpt.c's
 *            attention caches (attention.c:105-120): rows 0 .. pos-1 hold the
 *            earlier tokens' keys and values; this call writes the new
 *            token's k and v into row pos.  0 <= pos < L, pos < 8192.
 *   output   (B, 1, C) device: attention output of position pos, equal to row
 *            pos of the forward over tokens 0 .. pos.
 *   Head size 64 with 16-byte rows: one launch (one workgroup per (b, h))
 *   for pos < 512; past that a split-key launch over 64-key chunks and a
 *   merge launch, with a stream-ordered partials buffer.
 */
void attention_decode_cuda_kernel(
    const tensor_t *qkv,
    tensor_t *k_cache,
    tensor_t *v_cache,
    const int pos,
    const int n_heads,
    tensor_t *output
);

/*
 * attention_decode_noalloc_cuda_kernel(qkv, k_cache, v_cache, pos, n_heads, output)
 *   No counterpart in the reference.  For callers that cannot allocate
 *   device memory (code under HIP graph capture, tight serving loops,
 *   harnesses that forbid hipMalloc): the same step, arguments and results
 *   as attention_decode_cuda_kernel, but the partial softmax states of its
 *   split-key steps (head size 64, pos >= 512) go to a fixed device array
 *   (gptc_decode_noalloc_scratch_floats() floats, 4 MiB, one per GPU, held
 *   until the process ends) instead of a stream-ordered allocation; the call
 *   allocates and frees nothing.  A step needing more partials
 *   (B*H*ceil((pos+1)/64)*68 floats) is a fatal error.  Calls that overlap on
 *   one GPU share that array and race.  pos is a host argument: a graph
 *   capture of this call replays that position (and its split count), so
 *   each position needs its own capture (gptc_gpt2_generate reads the
 *   position from device memory instead).
 */
void attention_decode_noalloc_cuda_kernel(
    const tensor_t *qkv,
    tensor_t *k_cache,
    tensor_t *v_cache,
    const int pos,
    const int n_heads,
    tensor_t *output
);
long long gptc_decode_noalloc_scratch_floats(void);

/*
 * ---- extensions with no counterpart in the reference ----
 * gptc_stream(): the hipStream_t (as void*) every launch of this library is
 * ordered on; for callers that time or order their own work against it.
 *
 * gptc_set_kernel_events(events, 8): hipEvent_t handles (as void*) that the
 * attention entry points record on that stream around each kernel launch:
 * [0,1] the forward kernel, then the backward's [2,3] delta, [4,5] dk/dv
 * and [6,7] dq kernels.  They stay registered until the next call;
 * events == NULL stops the recording.  For per-kernel timing.
 *
 * gptc_attention_state_floats(B, T, C, n_heads): floats of the 1-D cache[3]
 * that the compact layout's forward expects (and otherwise re-points), so
 * that a layer can allocate it once at the right size.
 *
 * gptc_attention_block_schedule(BH, nqt, per_cu, cus, wg_start, items, cap,
 *                               max_cu_load, used_pairs)
 *   The work lists the D = 64 forward and dq kernels run for BH heads of nqt
 *   64-query blocks on a GPU of 8 XCDs x cus CUs keeping per_cu workgroups
 *   per CU (host computation only, for tests and tuning): workgroup w runs
 *   the blocks items[wg_start[w] .. wg_start[w+1]), each (bh << 12) | j.
 *   Returns the workgroup count (-1 when cap ints do not hold the table);
 *   max_cu_load receives the largest per-CU sum of block costs (j + 1.5
 *   tiles each), used_pairs 1 when the pairs construction was chosen.
 *
 * gptc_attention_block_schedule_pool(BH, nqt, per_cu, cus, wg_start, items,
 *                                    cap, pool_j0)
 *   The lists of the compact layout's D = 64 forward, which leaves the
 *   blocks j < *pool_j0 of every head to a pool that workgroups whose lists
 *   are done take from (*pool_j0 = 0: no pool, the lists hold every block).
 *   Same filling and return as gptc_attention_block_schedule.
 *
 * gptc_attention_key_schedule(BH, nqt, per_cu, cus, wg_start, items, cap,
 *                             est, nsplit)
 *   The work lists the D = 64 dk/dv kernel runs for BH heads of nqt 64-query
 *   tiles (128-key blocks kb = 0 .. ceil(nqt / 2) - 1, block kb reducing
 *   tiles 2kb .. nqt-1), on the same GPU description (host computation only,
 *   for tests and tuning): workgroup w runs items wg_start[w] ..
 *   wg_start[w+1]), item i being items[4i .. 4i+3] = (bh, kb, qa, qe), query
 *   tiles [qa, qe) of key block kb of head bh.  Blocks kb < *nsplit are cut
 *   into two items, the others are one.  Returns the workgroup count (-1 when
 *   cap ints do not hold the table); est receives the estimated time (tiles)
 *   the choice of nsplit minimised.
 */
/*
 * ---- one-token model step (KV-cache generation): no counterpart in gpt.c ----
 * gptc_linear_rows_cuda(W, b, x, residual, act, y)
 *   y = act(x W^T + b) + residual for x with 1 .. 8 rows (the decode step's
 *   activations); b and residual may be NULL; act 0 = none, 1 = GELU (the tanh
 *   form of kernels/src/cpu/GeLU.c).  Each weight row is read once.
 * gptc_embed_token_cuda(wte, wpe, ids, pos, out)
 *   out (B, C) = wte[ids] + wpe[pos]; ids outside [0, V) give NaN rows.
 * gptc_argmax_cuda(logits, ids)
 *   ids[r] = first index of the maximum of logits row r (greedy decoding).
 */
void gptc_linear_rows_cuda(const tensor_t *W, const tensor_t *b, const tensor_t *x, const tensor_t *residual,
                           const int act, tensor_t *y);
void gptc_embed_token_cuda(const tensor_t *wte, const tensor_t *wpe, const tensor_t *ids, const int pos,
                           tensor_t *out);
void gptc_argmax_cuda(const tensor_t *logits, tensor_t *ids);

void *gptc_stream(void);
void gptc_set_kernel_events(void **events, int n);
long long gptc_attention_state_floats(int B, int T, int C, int n_heads);

/*
 * gptc_attention_set_state_limit(floats): no counterpart in gpt.c.  The
 * largest backward state (in floats) the forward keeps with the probability
 * blocks of P'; a forward whose state would be larger keeps only the
 * log-sum-exp (O(T) per head) when head size 64 runs.  Its backward then
 * recomputes P in the dK/dV kernel (4 contractions there instead of 3) and
 * writes dS to a scratch the dQ kernel reads (see the scratch limit below);
 * same results to the stated tolerance.  Default and floats < 0: the int
 * length of a tensor_t.  0 makes every D = 64 forward keep the LSE-only state.
 * Returns the previous limit.  Applies to forwards that run after the call.
 */
long long gptc_attention_set_state_limit(long long floats);

/*
 * gptc_attention_set_scratch_limit(floats): no counterpart in gpt.c.  The
 * largest dS scratch (in floats) the backward of the LSE-only state
 * allocates, stream-ordered, for the duration of the call: the packed causal
 * blocks of as many whole heads as fit (T^2/2 floats per head, roughly),
 * the heads running in chunks of that many.  If not even one head fits, the
 * dQ kernel recomputes P and dP from the LSE too (7 contractions in all, no
 * scratch).  Default, floats < 0 and floats > 2^30: 2^30 floats (4 GiB).
 * Returns the previous limit.  Applies to backwards that run after the call.
 */
long long gptc_attention_set_scratch_limit(long long floats);
int gptc_attention_block_schedule(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items, int cap,
                                  double *max_cu_load, int *used_pairs);
int gptc_attention_block_schedule_pool(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items, int cap,
                                       int *pool_j0);
int gptc_attention_key_schedule(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items, int cap,
                                double *est, int *nsplit);

#ifdef __cplusplus
}
#endif
