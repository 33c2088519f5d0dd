/*
 * GPT-2 token decoder (/root/reference/src/tokenizer.c:16-114): reads
 * tokenizer.bin and maps ids to their byte strings.
 */
#include <ctype.h>
#include <stdlib.h>
#include <string.h>
#include "tokenizer.h"
#include "utils.h"

#define TOKENIZER_MAGIC 20240415

static void free_layer_tokenizer(tokenizer_t *tokenizer);
static char *decode_tokenizer(tokenizer_t *tokenizer, uint32_t token);
static void decode_tokens_tokenizer(tokenizer_t *tokenizer, uint32_t *tokens, size_t n, char *dest, size_t dest_n);
static uint32_t decode_length_tokenizer(tokenizer_t *tokenizer, uint32_t *tokens, size_t n);

tokenizer_t *Tokenizer(const char *filename) {
    FILE *file = fopenCheck(filename, "rb");
    uint32_t header[256];
    freadCheck(header, sizeof(uint32_t), 256, file);
    CHECK_ERROR(header[0] != TOKENIZER_MAGIC, "Bad magic number in %s file. Expected %d got %u\n", filename,
                TOKENIZER_MAGIC, header[0]);
    tokenizer_t *tokenizer = (tokenizer_t *)mallocCheck(sizeof(tokenizer_t));
    tokenizer->vocab_size = header[1];
    tokenizer->eot_token = (int)header[2];
    tokenizer->token_map = (char **)mallocCheck(sizeof(char *) * (tokenizer->vocab_size ? tokenizer->vocab_size : 1));
    for (uint32_t i = 0; i < tokenizer->vocab_size; i++) {
        unsigned char length;
        freadCheck(&length, sizeof(unsigned char), 1, file);
        CHECK_ERROR(length == 0, "Expected every token to be at least one byte. Got 0 for token %u\n", i);
        char *bytes = (char *)mallocCheck((size_t)length + 1);
        freadCheck(bytes, sizeof(char), length, file);
        bytes[length] = '\0';
        tokenizer->token_map[i] = bytes;
    }
    fcloseCheck(file);
    tokenizer->decode = decode_tokenizer;
    tokenizer->decode_tokens = decode_tokens_tokenizer;
    tokenizer->decode_length = decode_length_tokenizer;
    tokenizer->free_layer = free_layer_tokenizer;
    return tokenizer;
}

static void free_layer_tokenizer(tokenizer_t *tokenizer) {
    if (tokenizer == NULL) return;
    for (uint32_t i = 0; i < tokenizer->vocab_size; i++) free(tokenizer->token_map[i]);
    free(tokenizer->token_map);
    free(tokenizer);
}

static uint32_t decode_length_tokenizer(tokenizer_t *tokenizer, uint32_t *tokens, size_t n) {
    if (tokenizer == NULL || tokens == NULL) return 0;
    uint32_t length = 0;
    for (size_t i = 0; i < n; i++) length += (uint32_t)strlen(tokenizer->decode(tokenizer, tokens[i]));
    return length;
}

static char *decode_tokenizer(tokenizer_t *tokenizer, uint32_t token) {
    if (tokenizer == NULL) return NULL;
    CHECK_ERROR(token >= tokenizer->vocab_size, "Expected token to be less than vocab_size(%u). Got %u\n",
                tokenizer->vocab_size, token);
    return tokenizer->token_map[token];
}

/* Concatenation of the tokens' bytes into dest, truncated to dest_n - 1 bytes. */
static void decode_tokens_tokenizer(tokenizer_t *tokenizer, uint32_t *tokens, size_t n, char *dest, size_t dest_n) {
    if (tokenizer == NULL || tokens == NULL || dest == NULL || dest_n == 0) return;
    size_t idx = 0;
    for (size_t i = 0; i < n; i++) {
        const char *d = tokenizer->decode(tokenizer, tokens[i]);
        while (*d != '\0' && idx < dest_n - 1) dest[idx++] = *d++;
    }
    dest[idx] = '\0';
}

void safe_printf(const char *piece) {
    if (piece == NULL || piece[0] == '\0') return;
    if (piece[1] == '\0') {
        const unsigned char byte = (unsigned char)piece[0];
        if (!(isprint(byte) || isspace(byte))) return;
    }
    printf("%s", piece);
}
