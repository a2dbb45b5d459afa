/* io.c — the .ember loader (replaces src/io.c:30-96).
 *
 * The file is mapped read-only; the header and tensor table are validated so
 * that every pointer handed out lies inside the mapping.  Nothing is copied
 * here: the weights reach the GPU when a state is created (model.c), and the
 * device copy is cached on the model so several states share it.
 */
#define _DEFAULT_SOURCE
#include "ember.h"
#include "model_internal.h"
#include "util.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static EmberModel *load_fail(const char *why, void *base, size_t size, int fd) {
    fprintf(stderr, "ember: %s\n", why);
    if (base) munmap(base, size);
    if (fd >= 0) close(fd);
    return NULL;
}

EmberModel *ember_model_load(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return load_fail("cannot open model file", NULL, 0, -1);
    struct stat st;
    if (fstat(fd, &st) != 0 || (uint64_t)st.st_size < sizeof(EmberHeader))
        return load_fail("model file too small", NULL, 0, fd);
    const size_t size = (size_t)st.st_size;
    void *base = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (base == MAP_FAILED) return load_fail("mmap failed", NULL, 0, fd);
    const EmberHeader *h = base;
    const uint64_t fsize = size;
    if (memcmp(h->magic, "EMBR", 4) != 0 || h->version != EMBER_VERSION)
        return load_fail("bad magic or version", base, size, fd);
    if (h->n_tensors < 0 || h->dim <= 0 || h->n_layers <= 0 || h->vocab_size <= 0)
        return load_fail("header has non-positive dimensions", base, size, fd);
    if (h->tensor_table_offset > fsize || h->tensor_table_size > fsize - h->tensor_table_offset ||
        h->tensor_table_size < (uint64_t)h->n_tensors * sizeof(EmberTensor))
        return load_fail("tensor table out of bounds", base, size, fd);
    if (h->tokenizer_offset > fsize || h->tokenizer_size > fsize - h->tokenizer_offset)
        return load_fail("tokenizer blob out of bounds", base, size, fd);
    EmberModel *m = ember_xcalloc(1, sizeof *m, "EmberModel");
    m->fd = fd;
    m->size = size;
    m->base = base;
    m->hdr = h;
    m->table = (const EmberTensor *)(m->base + h->tensor_table_offset);
    madvise(base, size, MADV_WILLNEED);
    return m;
}

void ember_model_free(EmberModel *m) {
    if (!m) return;
    ember_model_release_device(m);
    munmap((void *)m->base, m->size);
    close(m->fd);
    free(m);
}

const EmberHeader *ember_model_header(const EmberModel *m) { return m->hdr; }

const EmberTensor *ember_model_tensor(const EmberModel *m, const char *name) {
    for (int i = 0; i < m->hdr->n_tensors; i++)
        if (strncmp(m->table[i].name, name, sizeof m->table[i].name) == 0) return &m->table[i];
    return NULL;
}

const void *ember_model_data(const EmberModel *m, const EmberTensor *t) {
    if (!t) return NULL;
    if (t->offset > m->size || t->nbytes > m->size - t->offset) {
        fprintf(stderr, "ember: tensor data out of bounds\n");
        return NULL;
    }
    return m->base + t->offset;
}
