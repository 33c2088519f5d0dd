"""Greedy generation loops on the library's GPT-2 (C4), for tests and bench.

window_generate  infer_gpt.c:313-408's context handling, with greedy argmax in
                 place of sample_mult (C4's rule): the token buffer starts as
                 EOT (50256) everywhere with the prompt in front; for each new
                 token the block_size window starting at start_index goes
                 through GPT2.forward, and row i-1 of the logits (block_size-1
                 once the window slides) picks token i.
kv_generate      the same tokens from one-token steps over per-layer K/V
                 caches (gptc_gpt2_decode): the prompt is decoded position by
                 position, then each new token is decoded at its position.
Both return the full token list (prompt + generated) and, when asked, the
logits rows that chose each generated token.
"""
import ctypes

import numpy as np

import gptc

EOT = 50256


def window_generate(rt, model, prompt, total, block_size, keep_logits=False):
    lib = rt.lib
    mult = -(-total // block_size)
    X = np.full(block_size * mult, EOT, np.float32)
    X[:len(prompt)] = prompt
    ids_out = rt.empty((1,))
    rows = []
    start = 0
    for i in range(len(prompt), total):
        start += 0 if i < block_size else 1
        win = rt.from_numpy(X[start:start + block_size].reshape(1, block_size))
        logits = model.forward(win)
        model.free_cache()  # frees the window (cached by wte) and the layer caches
        r = i - 1 if i < block_size else block_size - 1
        V = logits.contents.shape[2]
        row = rt.empty((1, 1, V))
        # logits[:, r, :] -> row (a device-side copy through a view of the row)
        view = gptc.Tensor()
        ctypes.memmove(ctypes.byref(view), logits, ctypes.sizeof(gptc.Tensor))
        base = ctypes.cast(logits.contents.t, ctypes.c_void_p).value
        view.t = ctypes.cast(base + 4 * r * V, ctypes.POINTER(ctypes.c_float))
        view.ndims, view.length = 3, V
        view.shape[0], view.shape[1], view.shape[2] = 1, 1, V
        lib.tensor_copy(row, ctypes.byref(view))
        lib.gptc_argmax_cuda(row, ids_out)
        if keep_logits:
            rows.append(rt.to_numpy(row)[0, 0])
        X[i] = rt.to_numpy(ids_out)[0]
        rt.free(row)
        rt.free(logits)
    return X[:total].astype(np.int64), rows


def graph_generate(rt, model, prompt, total, cache=None):
    """gptc_gpt2_generate: the whole greedy loop on the GPU (one captured step
    replayed per position), for one or more prompts of equal length.
    prompt: (P,) or (B, P) ids.  Returns the (B, total) or (total,) tokens."""
    p = np.asarray(prompt)
    single = p.ndim == 1
    p = p.reshape(1, -1) if single else p
    B, P = p.shape
    buf = np.zeros((B, total), np.float32)
    buf[:, :P] = p
    tokens = rt.from_numpy(buf)
    own = cache is None
    cache = cache or gptc.KVCache(rt, model, B, total)
    rt.lib.gptc_gpt2_generate(model.raw, cache.raw, tokens, P, total)
    out = rt.to_numpy(tokens).astype(np.int64)
    rt.free(tokens)
    if own:
        cache.free()
    return out[0] if single else out


def kv_generate(rt, model, prompt, total, block_size, keep_logits=False):
    lib = rt.lib
    cache = gptc.KVCache(rt, model, 1, total)
    tokens = list(int(t) for t in prompt)
    rows = []
    next_id = rt.empty((1,))
    for pos in range(total - 1):
        step_ids = rt.from_numpy(np.array([[tokens[pos]]], np.float32))
        logits = cache.decode(step_ids, pos)
        rt.free(step_ids)
        if pos + 1 >= len(prompt):
            lib.gptc_argmax_cuda(logits, next_id)
            if keep_logits:
                rows.append(rt.to_numpy(logits)[0, 0])
            tokens.append(int(rt.to_numpy(next_id)[0]))
        rt.free(logits)
    rt.free(next_id)
    cache.free()
    return np.array(tokens, np.int64), rows
