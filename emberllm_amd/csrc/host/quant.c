/* quant.c — fp16 conversion, the Q8_0 / Q4_0 block quantizers and the
 * offline requantizer.
 *
 * The quantizers must reproduce the reference bit for bit, since they make
 * the weight bytes the GPU streams (src/kernels.c:73-115):
 *   Q8_0: d = amax/127, inverse from the unrounded d, codes round half away
 *         from zero and clamp to +-127, d stored as fp16 (RNE).
 *   Q4_0: d = v/-8 with v the signed element of largest magnitude, codes
 *         (int)(x/d + 8.5) truncated and clamped to 0..15, element i in the
 *         low nibble and element i+16 in the high nibble of byte i.
 * ember_quantize_file follows the file rules of src/quant.c:26-125: 1-D
 * tensors stay F32, rows not divisible by 32 stay F32, already-quantized
 * tensors pass through, and in Q4_0 mode tok_embeddings / lm_head become
 * Q8_0.  Layout: tokenizer blob right after the header, table 8-aligned,
 * data region and every tensor 64-aligned (tools/convert.py:57-112).  The
 * blocks of every tensor to be quantized are encoded on the GPU in one
 * ehip_quantize_rows call (the same arithmetic as the row quantizers here);
 * without a GPU the call fails with a message, as state creation does.
 */
#define _DEFAULT_SOURCE
#include "ember.h"
#include "ehip.h"
#include "util.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

float ember_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float f;
    if (e == 0) {                 /* zero or subnormal: m * 2^-24, exact */
        f = (float)m * 5.9604644775390625e-8f;
        uint32_t bits; memcpy(&bits, &f, 4); bits |= sign; memcpy(&f, &bits, 4);
        return f;
    }
    uint32_t bits = e == 0x1fu ? (sign | 0x7f800000u | (m << 13))
                               : (sign | ((e + 112u) << 23) | (m << 13));
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ember_float_to_half(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* rounds past 65504, inf, NaN */
    if (a < 0x38800000u) {                                      /* below 2^-14: subnormal half */
        float g; memcpy(&g, &a, 4);
        return (uint16_t)(sign | (uint16_t)rintf(g * 16777216.0f));  /* RNE to a multiple of 2^-24 */
    }
    a += 0xfffu + ((a >> 13) & 1u);                             /* round the 13 dropped bits to even */
    return (uint16_t)(sign | ((a - 0x38000000u) >> 13));
}

void ember_quant_q8_row(const float *x, uint8_t *out, int n) {
    for (int b = 0; b < n / EMBER_Q_BLOCK; b++, out += 34) {
        const float *v = x + (size_t)b * EMBER_Q_BLOCK;
        float amax = 0.0f;
        for (int i = 0; i < EMBER_Q_BLOCK; i++) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
        const float d = amax / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = ember_float_to_half(d);
        memcpy(out, &dh, 2);
        for (int i = 0; i < EMBER_Q_BLOCK; i++) {
            /* the reference's (int)lroundf: NaN and infinite products give
             * LONG_MIN, whose int conversion is 0 (code 0, not -127) */
            int q = (int)lroundf(v[i] * inv);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            out[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

void ember_quant_q4_row(const float *x, uint8_t *out, int n) {
    for (int b = 0; b < n / EMBER_Q_BLOCK; b++, out += 18) {
        const float *v = x + (size_t)b * EMBER_Q_BLOCK;
        float amax = 0.0f, vmax = 0.0f;
        for (int i = 0; i < EMBER_Q_BLOCK; i++)
            if (fabsf(v[i]) > amax) { amax = fabsf(v[i]); vmax = v[i]; }
        const float d = vmax / -8.0f;
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = ember_float_to_half(d);
        memcpy(out, &dh, 2);
        for (int i = 0; i < EMBER_Q_BLOCK / 2; i++) {
            int lo = (int)(v[i] * inv + 8.5f), hi = (int)(v[i + 16] * inv + 8.5f);
            lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
            hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
            out[2 + i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

static uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

int ember_quantize_file(const char *in_path, const char *out_path, int target) {
    if (target != EMBER_DT_Q8_0 && target != EMBER_DT_Q4_0) {
        fprintf(stderr, "ember: quantize target must be q8_0 or q4_0\n");
        return 1;
    }
    EmberModel *m = ember_model_load(in_path);
    if (!m) return 1;
    const EmberHeader *h = ember_model_header(m);
    const EmberTensor *tab = (const EmberTensor *)((const uint8_t *)h + h->tensor_table_offset);
    const int n = h->n_tensors;
    EmberTensor *meta = ember_xcalloc((size_t)n, sizeof(EmberTensor), "quantize table");
    uint8_t **data = ember_xcalloc((size_t)n, sizeof(uint8_t *), "quantize data");
    EhipQuantJob *jobs = ember_xcalloc((size_t)n, sizeof(EhipQuantJob), "quantize jobs");
    int n_jobs = 0;
    for (int i = 0; i < n; i++) {
        const EmberTensor *t = &tab[i];
        const void *src = ember_model_data(m, t);
        const int rows = t->shape[0], cols = t->shape[1];
        const int quantize = t->dtype == EMBER_DT_F32 && t->ndim >= 2 && cols % EMBER_Q_BLOCK == 0;
        /* the fp32 rows the encoder reads must lie inside the tensor's payload */
        const int short_payload = quantize && (rows < 0 || cols < 0 ||
                                               (uint64_t)rows * (uint64_t)cols * 4u > t->nbytes);
        if (short_payload)
            fprintf(stderr, "ember: %s: tensor '%.48s' holds %llu bytes, fewer than its [%d, %d] fp32 shape\n",
                    in_path, t->name, (unsigned long long)t->nbytes, rows, cols);
        if (!src || short_payload) {
            for (int k = 0; k < i; k++) free(data[k]);
            free(data); free(meta); free(jobs);
            ember_model_free(m);
            return 1;
        }
        meta[i] = *t;
        int want = target;
        if (target == EMBER_DT_Q4_0 &&
            (!strcmp(t->name, "tok_embeddings") || !strcmp(t->name, "lm_head")))
            want = EMBER_DT_Q8_0;
        if (!quantize) {   /* passes through unchanged */
            data[i] = ember_xmalloc(t->nbytes, "tensor copy");
            memcpy(data[i], src, t->nbytes);
            continue;
        }
        const size_t bs = want == EMBER_DT_Q8_0 ? 34 : 18;
        const size_t rb = (size_t)(cols / EMBER_Q_BLOCK) * bs;
        meta[i].dtype = want;
        meta[i].nbytes = rb * (size_t)rows;
        data[i] = ember_xmalloc(meta[i].nbytes, "quantized tensor");
        jobs[n_jobs++] = (EhipQuantJob){ (const float *)src, rows, cols, want, data[i] };
    }
    int rc = 0;
    if (n_jobs > 0) {
        if (ehip_device_count() <= 0) {
            fprintf(stderr, "ember: no GPU is visible to the HIP runtime\n");
            rc = 1;
        } else if (ehip_quantize_rows(jobs, n_jobs) != 0) {
            fprintf(stderr, "ember: quantization failed: %s\n", ehip_last_error());
            rc = 1;
        }
    }
    free(jobs);
    if (rc) {
        for (int i = 0; i < n; i++) free(data[i]);
        free(data); free(meta);
        ember_model_free(m);
        return rc;
    }
    EmberHeader nh = *h;
    nh.tokenizer_offset = sizeof(EmberHeader);
    nh.tensor_table_offset = round_up(nh.tokenizer_offset + h->tokenizer_size, 8);
    nh.tensor_table_size = (uint64_t)n * sizeof(EmberTensor);
    nh.header_bytes = round_up(nh.tensor_table_offset + nh.tensor_table_size, 64);
    uint64_t cur = nh.header_bytes;
    for (int i = 0; i < n; i++) {
        cur = round_up(cur, 64);
        meta[i].offset = cur;
        cur += meta[i].nbytes;
    }
    FILE *f = fopen(out_path, "wb");
    if (!f) {
        fprintf(stderr, "ember: cannot write %s\n", out_path);
        rc = 1;
    } else {
        static const uint8_t zeros[64];
        uint64_t at = 0;
#define PUT(p, len) do { if (fwrite((p), 1, (len), f) != (size_t)(len)) rc = 1; at += (len); } while (0)
#define PAD_TO(o)   do { while (at < (o)) { uint64_t k = (o) - at > 64 ? 64 : (o) - at; PUT(zeros, k); } } while (0)
        PUT(&nh, sizeof nh);
        PUT((const uint8_t *)h + h->tokenizer_offset, h->tokenizer_size);
        PAD_TO(nh.tensor_table_offset);
        PUT(meta, sizeof(EmberTensor) * (size_t)n);
        PAD_TO(nh.header_bytes);
        for (int i = 0; i < n; i++) { PAD_TO(meta[i].offset); PUT(data[i], meta[i].nbytes); }
#undef PUT
#undef PAD_TO
        if (fclose(f) != 0) rc = 1;
        if (rc) fprintf(stderr, "ember: short write to %s\n", out_path);
        else fprintf(stderr, "quantized %s -> %s (%.1f MB)\n", in_path, out_path, cur / 1e6);
    }
    for (int i = 0; i < n; i++) free(data[i]);
    free(data); free(meta);
    ember_model_free(m);
    return rc;
}
