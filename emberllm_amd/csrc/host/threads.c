/* threads.c — the reference's pool entry points (src/threads.c:61-104,
 * src/kernels.h:71-83).  The forward pass runs on the GPU, whose launch grid
 * replaces the host pool, so these only record the requested count for
 * callers that print or query it. */
#include "ember.h"

static int g_nthreads = 1;

void ember_threads_init(int nthreads) { g_nthreads = nthreads < 1 ? 1 : nthreads; }
void ember_threads_shutdown(void) { g_nthreads = 1; }
int  ember_nthreads(void) { return g_nthreads; }
