/*
 * Token-stream reader behind gpt.c's DataLoader API
 * (/root/reference/include/dataloader.h:32-52; the file format is
 * data/common.py:35-48: raw little-endian int32 token ids, nothing else).
 *
 * Design: the whole file is mapped read-only once (mmap), so a batch is a
 * slice of the mapping converted to floats; there are no seeks or reads per
 * step and the page cache is shared with other processes reading the same
 * shard.  The behaviour seen through the API is gpt.c's:
 *   - next() hands out a window of n = batch*block + 1 consecutive ids:
 *     inputs are ids [s, s + n - 1), targets ids [s + 1, s + n), both as
 *     new (batch, block) host float tensors owned by the caller;
 *   - the window start then moves on by batch*block ids; when a window
 *     starting there would run past the last id, it restarts at id 0;
 *   - len() = floor(file bytes / (4 * n)), the number of whole windows;
 *   - reset() restarts at id 0.
 *
 * Field use of dataloader_t (the struct layout is gpt.c's, so that callers
 * compiled against gpt.c's header see the function pointers where they
 * expect them): `batch` points at the mapped ids, `_file_size` is the file
 * size in bytes, `_curr_fp_ptr` the byte offset of the next window, `fp`
 * is unused (NULL).
 */
#include <fcntl.h>
#include <stdint.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "dataloader.h"
#include "utils.h"

static size_t window_ids(const dataloader_t *dl) { return (size_t)dl->batch_size * (size_t)dl->block_size + 1; }

static void loader_next(dataloader_t *dl, tensor_t **out);
static int loader_len(dataloader_t *dl);
static void loader_reset(dataloader_t *dl);
static void loader_release(dataloader_t *dl);

dataloader_t *DataLoader(const char *filename, const int batch_size, const int block_size) {
    REQUIRE_ARG(filename);
    CHECK_ERROR(batch_size < 1 || block_size < 1, "DataLoader(%s): batch (%d) and block (%d) sizes must be >= 1.",
                filename, batch_size, block_size);

    const int fd = open(filename, O_RDONLY);
    CHECK_ERROR(fd < 0, "DataLoader: cannot open token file '%s'.", filename);
    struct stat info;
    CHECK_ERROR(fstat(fd, &info) != 0, "DataLoader: cannot stat '%s'.", filename);
    const size_t bytes = (size_t)info.st_size;
    const size_t need = ((size_t)batch_size * (size_t)block_size + 1) * sizeof(int32_t);
    CHECK_ERROR(bytes < need,
                "DataLoader: '%s' holds %zu bytes, fewer than one window of %d x %d + 1 token ids (%zu bytes).",
                filename, bytes, batch_size, block_size, need);

    void *map = mmap(NULL, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    CHECK_ERROR(map == MAP_FAILED, "DataLoader: cannot map '%s' (%zu bytes).", filename, bytes);
    close(fd); /* the mapping keeps the file's pages reachable */
    (void)madvise(map, bytes, MADV_SEQUENTIAL);

    dataloader_t *dl = (dataloader_t *)mallocCheck(sizeof(dataloader_t));
    dl->batch_size = batch_size;
    dl->block_size = block_size;
    dl->fp = NULL;
    dl->batch = (int *)map;
    dl->_file_size = bytes;
    dl->_curr_fp_ptr = 0;
    dl->next = loader_next;
    dl->len = loader_len;
    dl->reset = loader_reset;
    dl->free_layer = loader_release;
    return dl;
}

static void loader_next(dataloader_t *dl, tensor_t **out) {
    REQUIRE_ARG(dl);
    REQUIRE_ARG(out);
    const size_t n = window_ids(dl);
    const size_t total_ids = dl->_file_size / sizeof(int32_t);
    size_t start = dl->_curr_fp_ptr / sizeof(int32_t);
    if (start + n > total_ids) start = 0; /* the window would run past the end: wrap */

    const int32_t *ids = (const int32_t *)dl->batch + start;
    int shape[2] = {dl->batch_size, dl->block_size};
    tensor_t *inputs = create_tensor(shape, 2, CPU);
    tensor_t *targets = create_tensor(shape, 2, CPU);
    float *x = inputs->t, *y = targets->t;
    for (size_t i = 0; i + 1 < n; i++) {
        x[i] = (float)ids[i];
        y[i] = (float)ids[i + 1];
    }
    dl->_curr_fp_ptr = (start + n - 1) * sizeof(int32_t);
    out[0] = inputs;
    out[1] = targets;
}

static int loader_len(dataloader_t *dl) {
    REQUIRE_ARG(dl);
    return (int)(dl->_file_size / (window_ids(dl) * sizeof(int32_t)));
}

static void loader_reset(dataloader_t *dl) {
    REQUIRE_ARG(dl);
    dl->_curr_fp_ptr = 0;
}

static void loader_release(dataloader_t *dl) {
    if (dl == NULL) return;
    if (dl->batch != NULL) munmap(dl->batch, dl->_file_size);
    free(dl);
}
