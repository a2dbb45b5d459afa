/* io.c — opening .ember files (the surface of src/io.c:30-96, ember.h).
 *
 * File format (include/ember.h): a packed 256-byte EmberHeader at offset 0,
 * a table of n_tensors packed 88-byte EmberTensor entries at
 * tensor_table_offset, a tokenizer blob at tokenizer_offset, and tensor
 * payloads at the offsets their entries name.
 *
 * The header is first read with pread() into a local copy and validated
 * there, so a file that is not an .ember file is rejected before anything is
 * mapped.  A valid file is then mapped read-only as a whole; the model hands
 * out pointers into that mapping (the weights reach the GPU when a state is
 * created, model.c) and the device copy is cached on the model so several
 * states share it.  Every region the header names is checked against the
 * file size with overflow-safe arithmetic; tensor payloads are checked when
 * ember_model_data resolves them.  Failures return NULL after one
 * "ember: <path>: <reason>" line on stderr.
 */
#define _DEFAULT_SOURCE
#include "ember.h"
#include "model_internal.h"
#include "util.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* [off, off + len) lies inside a file of `size` bytes */
static int inside(uint64_t off, uint64_t len, uint64_t size) {
    return off <= size && len <= size - off;
}

/* Why the header cannot describe a usable model, or NULL if it can. */
static const char *header_problem(const EmberHeader *h, uint64_t size) {
    if (memcmp(h->magic, "EMBR", 4) != 0) return "not an .ember file (magic is not EMBR)";
    if (h->version != EMBER_VERSION) return "unsupported .ember format version";
    if (h->dim <= 0 || h->n_layers <= 0 || h->vocab_size <= 0 || h->n_tensors < 0)
        return "header declares a non-positive size";
    if (!inside(h->tensor_table_offset, h->tensor_table_size, size))
        return "tensor table extends past the end of the file";
    if (h->tensor_table_size / sizeof(EmberTensor) < (uint64_t)h->n_tensors)
        return "tensor table is shorter than its entry count";
    if (!inside(h->tokenizer_offset, h->tokenizer_size, size))
        return "tokenizer data extends past the end of the file";
    return NULL;
}

static EmberModel *reject(const char *path, const char *why, int fd) {
    fprintf(stderr, "ember: %s: %s\n", path, why);
    if (fd >= 0) close(fd);
    return NULL;
}

EmberModel *ember_model_load(const char *path) {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return reject(path, strerror(errno), -1);
    struct stat st;
    if (fstat(fd, &st) != 0) return reject(path, strerror(errno), fd);
    const uint64_t size = (uint64_t)st.st_size;
    EmberHeader h;
    if (size < sizeof h || pread(fd, &h, sizeof h, 0) != (ssize_t)sizeof h)
        return reject(path, "shorter than an .ember header", fd);
    const char *why = header_problem(&h, size);
    if (why) return reject(path, why, fd);
    void *map = mmap(NULL, (size_t)size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) return reject(path, strerror(errno), fd);
    (void)madvise(map, (size_t)size, MADV_WILLNEED);   /* the upload reads it all */
    EmberModel *m = ember_xcalloc(1, sizeof *m, "model");
    m->fd = fd;
    m->size = (size_t)size;
    m->base = map;
    m->hdr = map;
    m->table = (const EmberTensor *)((const uint8_t *)map + h.tensor_table_offset);
    return m;
}

void ember_model_free(EmberModel *m) {
    if (m == NULL) return;
    ember_model_release_device(m);
    (void)munmap((void *)m->base, m->size);
    (void)close(m->fd);
    free(m);
}

const EmberHeader *ember_model_header(const EmberModel *m) { return m->hdr; }

/* Entry names are NUL-padded to their 48 bytes and may fill all of them:
 * compare at most that many characters, stopping at the first NUL. */
static int same_name(const char field[48], const char *want) {
    for (int i = 0; i < 48; i++) {
        if (field[i] != want[i]) return 0;
        if (want[i] == '\0') return 1;
    }
    return 1;
}

const EmberTensor *ember_model_tensor(const EmberModel *m, const char *name) {
    const EmberTensor *t = m->table, *end = m->table + m->hdr->n_tensors;
    for (; t < end; t++)
        if (same_name(t->name, name)) return t;
    return NULL;
}

const void *ember_model_data(const EmberModel *m, const EmberTensor *t) {
    if (t == NULL) return NULL;
    if (!inside(t->offset, t->nbytes, m->size)) {
        fprintf(stderr, "ember: payload of tensor '%.48s' extends past the end of the file\n", t->name);
        return NULL;
    }
    return m->base + t->offset;
}
