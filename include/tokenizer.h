/*
 * tokenizer.h -- gpt.c's GPT-2 token decoder, unchanged interface
 * (/root/reference/include/tokenizer.h:31-49).  tokenizer.bin
 * (tokenizer.py:12-40): 256 int32 header words (magic 20240415, vocab size,
 * EOT id), then per token one length byte (1 .. 255) and that many bytes.
 */
#pragma once

#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tokenizer {
    uint32_t vocab_size;
    int eot_token;
    char **token_map;
    void (*free_layer)(struct tokenizer *);
    char *(*decode)(struct tokenizer *, uint32_t token);
    void (*decode_tokens)(struct tokenizer *, uint32_t *tokens, size_t n, char *dest, size_t dest_n);
    uint32_t (*decode_length)(struct tokenizer *, uint32_t *tokens, size_t n);
} tokenizer_t;

/* Print a token's text, skipping single non-printable bytes. */
void safe_printf(const char *piece);
tokenizer_t *Tokenizer(const char *filename);

#ifdef __cplusplus
}
#endif
