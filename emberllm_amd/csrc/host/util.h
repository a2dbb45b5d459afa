/* util.h — fatal errors and checked allocation for the host library.
 * Error convention of the reference (src/util.h:13-20, util.c:8-34): print
 * "ember: <message>" to stderr and exit(1). */
#ifndef EMBER_HOST_UTIL_H
#define EMBER_HOST_UTIL_H

#include <stddef.h>
#include <stdint.h>

void  ember_die(const char *fmt, ...) __attribute__((noreturn, format(printf, 1, 2)));
void *ember_xmalloc(size_t n, const char *what);
void *ember_xcalloc(size_t count, size_t size, const char *what);
void *ember_xrealloc(void *p, size_t n, const char *what);

/* fp16 <-> fp32 conversions of the file format (src/kernels.c:25-68):
 * exact half->float; float->half rounds to nearest even, overflow -> inf. */
float    ember_half_to_float(uint16_t h);
uint16_t ember_float_to_half(float f);

/* Q8_0 / Q4_0 block quantizers (src/kernels.c:73-115); n % 32 == 0. */
void ember_quant_q8_row(const float *x, uint8_t *out, int n);
void ember_quant_q4_row(const float *x, uint8_t *out, int n);

#endif
