/* util.c — the host library's failure convention and the allocation helpers
 * built on it.
 *
 * Convention (the reference's, src/util.h:13-20): a fatal condition prints
 * one line "ember: <reason>" on stderr and ends the process with status 1.
 * The message is formatted into a local buffer first, so it reaches stderr
 * as a single write even when other threads print.  Allocation sizes are
 * checked for overflow before the C library sees them; a zero-byte request
 * is served as a one-byte block, so success never returns NULL.
 */
#include "util.h"

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

void ember_die(const char *fmt, ...) {
    char line[1024];
    va_list ap;
    va_start(ap, fmt);
    const int n = vsnprintf(line, sizeof line, fmt, ap);
    va_end(ap);
    fprintf(stderr, "ember: %s%s\n", line, n >= (int)sizeof line ? " [...]" : "");
    fflush(stderr);
    exit(1);
}

/* A NULL from the C allocator is fatal; `what` names the object. */
static void *granted(void *p, size_t bytes, const char *what) {
    if (p == NULL) ember_die("allocation of %zu bytes for %s failed", bytes, what ? what : "(unnamed)");
    return p;
}

void *ember_xmalloc(size_t n, const char *what) {
    return granted(malloc(n > 0 ? n : 1), n, what);
}

void *ember_xcalloc(size_t count, size_t size, const char *what) {
    if (size != 0 && count > SIZE_MAX / size)
        ember_die("allocation of %zu elements of %zu bytes for %s overflows", count, size, what ? what : "(unnamed)");
    const size_t total = count * size;
    return granted(calloc(total > 0 ? total : 1, 1), total, what);
}

void *ember_xrealloc(void *p, size_t n, const char *what) {
    return granted(realloc(p, n > 0 ? n : 1), n, what);
}
