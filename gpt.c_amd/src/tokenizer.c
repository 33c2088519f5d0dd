/*
 * GPT-2 token decoder behind gpt.c's Tokenizer API
 * (/root/reference/include/tokenizer.h:31-49).  File format, as written by
 * gpt.c's tokenizer.py:12-40: 256 little-endian int32 header words
 * (word 0 = 20240415, word 1 = vocabulary size, word 2 = end-of-text id),
 * then for every token id in order one length byte L (1 .. 255) followed
 * by L raw bytes.
 *
 * Design: the file is read with one fread into memory, validated while it
 * is walked once, and every token's bytes are copied into one arena of
 * NUL-terminated strings; token_map[i] points into that arena (one
 * allocation for the whole vocabulary instead of one per token, and
 * token_map[0] is the arena itself).
 */
#include <ctype.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include "tokenizer.h"
#include "utils.h"

enum { kHeaderWords = 256, kTokenizerMagic = 20240415 };

static char *tok_decode(tokenizer_t *tk, uint32_t id);
static void tok_decode_many(tokenizer_t *tk, uint32_t *ids, size_t n, char *dest, size_t dest_n);
static uint32_t tok_decoded_length(tokenizer_t *tk, uint32_t *ids, size_t n);
static void tok_release(tokenizer_t *tk);

/* The whole file in one heap buffer; *size receives its length. */
static unsigned char *slurp(const char *path, size_t *size) {
    FILE *fp = fopenCheck(path, "rb");
    fseekCheck(fp, 0, SEEK_END);
    const long end = ftell(fp);
    CHECK_ERROR(end < 0, "Tokenizer: cannot size '%s'.", path);
    fseekCheck(fp, 0, SEEK_SET);
    unsigned char *buf = (unsigned char *)mallocCheck((size_t)end + 1);
    if (end > 0) freadCheck(buf, 1, (size_t)end, fp);
    fcloseCheck(fp);
    *size = (size_t)end;
    return buf;
}

tokenizer_t *Tokenizer(const char *filename) {
    REQUIRE_ARG(filename);
    size_t size = 0;
    unsigned char *raw = slurp(filename, &size);
    CHECK_ERROR(size < kHeaderWords * sizeof(int32_t), "Tokenizer: '%s' is %zu bytes, shorter than its header.",
                filename, size);
    int32_t header[kHeaderWords];
    memcpy(header, raw, sizeof(header));
    CHECK_ERROR(header[0] != kTokenizerMagic, "Tokenizer: '%s' is not a tokenizer.bin file (word 0 is %d, not %d).",
                filename, header[0], kTokenizerMagic);
    CHECK_ERROR(header[1] < 0, "Tokenizer: '%s' declares a negative vocabulary (%d).", filename, header[1]);
    const uint32_t vocab = (uint32_t)header[1];

    /* One pass over the records: check that they fit the file and total
     * their bytes, so the arena is allocated once. */
    const unsigned char *rec = raw + sizeof(header), *end = raw + size;
    size_t arena_bytes = 0;
    for (uint32_t i = 0; i < vocab; i++) {
        CHECK_ERROR(rec >= end, "Tokenizer: '%s' ends before the record of token %u.", filename, i);
        const unsigned len = *rec;
        CHECK_ERROR(len == 0, "Tokenizer: token %u of '%s' has an empty byte string.", i, filename);
        CHECK_ERROR((size_t)(end - rec) < 1 + (size_t)len, "Tokenizer: '%s' ends inside the bytes of token %u.",
                    filename, i);
        arena_bytes += (size_t)len + 1;
        rec += 1 + len;
    }

    char *arena = (char *)mallocCheck(arena_bytes ? arena_bytes : 1);
    char **map = (char **)mallocCheck(sizeof(char *) * (vocab ? vocab : 1));
    rec = raw + sizeof(header);
    char *w = arena;
    for (uint32_t i = 0; i < vocab; i++) {
        const unsigned len = *rec++;
        memcpy(w, rec, len);
        w[len] = '\0';
        map[i] = w;
        w += len + 1;
        rec += len;
    }
    free(raw);

    tokenizer_t *tk = (tokenizer_t *)mallocCheck(sizeof(tokenizer_t));
    tk->vocab_size = vocab;
    tk->eot_token = header[2];
    tk->token_map = map;
    if (vocab == 0) map[0] = arena; /* keep the arena reachable for tok_release */
    tk->decode = tok_decode;
    tk->decode_tokens = tok_decode_many;
    tk->decode_length = tok_decoded_length;
    tk->free_layer = tok_release;
    return tk;
}

static char *tok_decode(tokenizer_t *tk, uint32_t id) {
    if (tk == NULL) return NULL;
    CHECK_ERROR(id >= tk->vocab_size, "Tokenizer: id %u is outside the vocabulary (size %u).", id, tk->vocab_size);
    return tk->token_map[id];
}

/* Total bytes of the decoded ids (no terminator). */
static uint32_t tok_decoded_length(tokenizer_t *tk, uint32_t *ids, size_t n) {
    if (tk == NULL || ids == NULL) return 0;
    size_t total = 0;
    for (size_t i = 0; i < n; i++) total += strlen(tok_decode(tk, ids[i]));
    return (uint32_t)total;
}

/* The ids' bytes concatenated into dest, cut to dest_n - 1 bytes, NUL-terminated. */
static void tok_decode_many(tokenizer_t *tk, uint32_t *ids, size_t n, char *dest, size_t dest_n) {
    if (tk == NULL || ids == NULL || dest == NULL || dest_n == 0) return;
    size_t used = 0;
    for (size_t i = 0; i < n && used + 1 < dest_n; i++) {
        const char *piece = tok_decode(tk, ids[i]);
        size_t len = strlen(piece);
        if (len > dest_n - 1 - used) len = dest_n - 1 - used;
        memcpy(dest + used, piece, len);
        used += len;
    }
    dest[used] = '\0';
}

static void tok_release(tokenizer_t *tk) {
    if (tk == NULL) return;
    free(tk->token_map[0]); /* the arena: token 0's string is its first entry */
    free(tk->token_map);
    free(tk);
}

/* A token made of one byte that is neither printable nor white space (a raw
 * control or partial UTF-8 byte) would garble the terminal: print nothing. */
static int lone_unprintable_byte(const char *piece) {
    const unsigned char c = (unsigned char)piece[0];
    return piece[1] == '\0' && !isprint(c) && !isspace(c);
}

void safe_printf(const char *piece) {
    if (piece == NULL || piece[0] == '\0' || lone_unprintable_byte(piece)) return;
    fputs(piece, stdout);
}
