/* tokenizer.c — the two tokenizer blobs of the .ember format
 * (replaces src/tokenizer.c:176-420; host text processing, not on the GPU).
 *
 * EMBER_TOK_LLAMA_SP blob: int32 max_len, then per id {f32 score, i32 len,
 *   bytes}.  Encoding: optional BOS, a " " dummy prefix when the text is not
 *   empty, one piece per UTF-8 character (byte fallback to id byte+3), then
 *   repeatedly merge the adjacent pair whose concatenation is a piece with
 *   the highest score (leftmost on ties).  Decoding strips the leading space
 *   after BOS and turns "<0xNN>" into the raw byte.
 * EMBER_TOK_BYTE_BPE blob: u32 vocab, u32 merges, u32 specials; per id
 *   {u8 special, u32 len, bytes}; per merge {u32 len, a, u32 len, b}; per
 *   special {u32 id, u32 len, bytes}.  Encoding: special tokens matched
 *   first, the rest split by the reference's approximation of the GPT-4/Qwen
 *   pre-tokenizer, mapped through the GPT-2 byte<->unicode table and merged
 *   by lowest rank (leftmost on ties).  Decoding maps back to bytes.
 */
#define _DEFAULT_SOURCE
#include "ember.h"
#include "model_internal.h"
#include "util.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- string -> int table (open addressing, keys point into owned memory) */
typedef struct { const char *k; int n, v; } Slot;
typedef struct { Slot *s; uint32_t mask; } Table;

static uint32_t hash_bytes(const char *p, int n) {
    uint32_t h = 2166136261u;
    for (int i = 0; i < n; i++) { h ^= (unsigned char)p[i]; h *= 16777619u; }
    return h ^ (h >> 15);
}

static void table_init(Table *t, int entries) {
    uint32_t cap = 64;
    while (cap < (uint32_t)entries * 2u + 2u) cap <<= 1;
    t->s = ember_xcalloc(cap, sizeof(Slot), "tokenizer table");
    t->mask = cap - 1;
}

static void table_put(Table *t, const char *k, int n, int v) {
    for (uint32_t i = hash_bytes(k, n) & t->mask;; i = (i + 1) & t->mask) {
        Slot *s = &t->s[i];
        if (!s->k) { s->k = k; s->n = n; s->v = v; return; }
        if (s->n == n && !memcmp(s->k, k, (size_t)n)) { s->v = v; return; }
    }
}

static int table_get(const Table *t, const char *k, int n) {
    for (uint32_t i = hash_bytes(k, n) & t->mask;; i = (i + 1) & t->mask) {
        const Slot *s = &t->s[i];
        if (!s->k) return -1;
        if (s->n == n && !memcmp(s->k, k, (size_t)n)) return s->v;
    }
}

struct EmberTokenizer {
    int type, vocab, bos;
    /* SentencePiece-style */
    char **piece; int *plen; float *score; int max_len; Table pieces;
    char bytechar[256][2];
    /* byte-level BPE */
    const uint8_t **str; int *slen; uint8_t *special;
    Table ids, ranks; char *rank_keys;
    int n_special; const char **sp_str; int *sp_len, *sp_id;
    char b2u[256][4]; int b2u_len[256];
    int u2b[512];
    char dec[512];
};

static uint32_t rd32(const uint8_t **p) { uint32_t v; memcpy(&v, *p, 4); *p += 4; return v; }

static void load_sp(EmberTokenizer *t, const uint8_t *p) {
    t->max_len = (int)rd32(&p);
    t->piece = ember_xcalloc((size_t)t->vocab, sizeof(char *), "pieces");
    t->plen = ember_xcalloc((size_t)t->vocab, sizeof(int), "piece lengths");
    t->score = ember_xcalloc((size_t)t->vocab, sizeof(float), "scores");
    table_init(&t->pieces, t->vocab);
    for (int b = 0; b < 256; b++) { t->bytechar[b][0] = (char)b; t->bytechar[b][1] = 0; }
    for (int i = 0; i < t->vocab; i++) {
        uint32_t sc = rd32(&p);
        memcpy(&t->score[i], &sc, 4);
        int len = (int)rd32(&p);
        t->piece[i] = ember_xmalloc((size_t)len + 1, "piece");
        memcpy(t->piece[i], p, (size_t)len);
        t->piece[i][len] = 0;
        t->plen[i] = len;
        p += len;
        table_put(&t->pieces, t->piece[i], len, i);
    }
}

static int utf8_put(int cp, char *o) {
    if (cp < 0x80) { o[0] = (char)cp; return 1; }
    if (cp < 0x800) { o[0] = (char)(0xC0 | (cp >> 6)); o[1] = (char)(0x80 | (cp & 63)); return 2; }
    o[0] = (char)(0xE0 | (cp >> 12)); o[1] = (char)(0x80 | ((cp >> 6) & 63)); o[2] = (char)(0x80 | (cp & 63));
    return 3;
}

static int utf8_get(const char *s, int *cp) {
    const unsigned char c = (unsigned char)s[0];
    if (c < 0x80) { *cp = c; return 1; }
    if ((c & 0xE0) == 0xC0) { *cp = ((c & 31) << 6) | (s[1] & 63); return 2; }
    if ((c & 0xF0) == 0xE0) { *cp = ((c & 15) << 12) | ((s[1] & 63) << 6) | (s[2] & 63); return 3; }
    *cp = ((c & 7) << 18) | ((s[1] & 63) << 12) | ((s[2] & 63) << 6) | (s[3] & 63);
    return 4;
}

static void load_bpe(EmberTokenizer *t, const uint8_t *p) {
    /* GPT-2 table: printable latin-1 bytes map to themselves, the others to 256.. */
    int next = 256;
    for (int i = 0; i < 512; i++) t->u2b[i] = -1;
    for (int b = 0; b < 256; b++) {
        const int printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE);
        const int cp = printable ? b : next++;
        t->b2u_len[b] = utf8_put(cp, t->b2u[b]);
        t->u2b[cp] = b;
    }
    const uint32_t nv = rd32(&p), nm = rd32(&p), ns = rd32(&p);
    t->str = ember_xcalloc((size_t)t->vocab, sizeof(uint8_t *), "bpe strings");
    t->slen = ember_xcalloc((size_t)t->vocab, sizeof(int), "bpe lengths");
    t->special = ember_xcalloc((size_t)t->vocab, 1, "bpe specials");
    table_init(&t->ids, t->vocab);
    for (uint32_t i = 0; i < nv; i++) {
        const uint8_t sp = *p++;
        const int len = (int)rd32(&p);
        if ((int)i < t->vocab) {
            t->str[i] = p; t->slen[i] = len; t->special[i] = sp;
            if (len) table_put(&t->ids, (const char *)p, len, (int)i);
        }
        p += len;
    }
    /* merge keys "a\0b" packed into one owned buffer */
    const uint8_t *q = p;
    size_t total = 0;
    for (uint32_t i = 0; i < nm; i++) {
        uint32_t la = rd32(&q); q += la;
        uint32_t lb = rd32(&q); q += lb;
        total += la + lb + 1;
    }
    t->rank_keys = ember_xmalloc(total ? total : 1, "merge keys");
    table_init(&t->ranks, (int)nm);
    char *w = t->rank_keys;
    for (uint32_t i = 0; i < nm; i++) {
        uint32_t la = rd32(&p); memcpy(w, p, la); p += la; w[la] = 0;
        uint32_t lb = rd32(&p); memcpy(w + la + 1, p, lb); p += lb;
        table_put(&t->ranks, w, (int)(la + 1 + lb), (int)i);
        w += la + 1 + lb;
    }
    t->n_special = (int)ns;
    t->sp_str = ember_xcalloc(ns ? ns : 1, sizeof(char *), "specials");
    t->sp_len = ember_xcalloc(ns ? ns : 1, sizeof(int), "specials");
    t->sp_id = ember_xcalloc(ns ? ns : 1, sizeof(int), "specials");
    for (uint32_t i = 0; i < ns; i++) {
        t->sp_id[i] = (int)rd32(&p);
        t->sp_len[i] = (int)rd32(&p);
        t->sp_str[i] = (const char *)p;
        p += t->sp_len[i];
    }
}

EmberTokenizer *ember_tokenizer_new(const EmberModel *m) {
    const EmberHeader *h = ember_model_header(m);
    EmberTokenizer *t = ember_xcalloc(1, sizeof *t, "tokenizer");
    t->type = h->tokenizer_type;
    t->vocab = h->vocab_size;
    t->bos = h->bos_token_id;
    const uint8_t *blob = (const uint8_t *)h + h->tokenizer_offset;
    if (t->type == EMBER_TOK_BYTE_BPE) load_bpe(t, blob);
    else load_sp(t, blob);
    return t;
}

void ember_tokenizer_free(EmberTokenizer *t) {
    if (!t) return;
    if (t->piece) for (int i = 0; i < t->vocab; i++) free(t->piece[i]);
    free(t->piece); free(t->plen); free(t->score); free(t->pieces.s);
    free(t->str); free(t->slen); free(t->special); free(t->ids.s); free(t->ranks.s);
    free(t->rank_keys); free(t->sp_str); free(t->sp_len); free(t->sp_id);
    free(t);
}

/* ---------------------------------------------------------------- SP ---- */
static int sp_encode(EmberTokenizer *t, const char *text, int add_bos, int **out) {
    const size_t n_text = strlen(text);
    int *ids = ember_xmalloc(sizeof(int) * (n_text + 3), "token ids");
    int n = 0;
    if (add_bos) ids[n++] = t->bos;
    if (text[0]) { const int sp = table_get(&t->pieces, " ", 1); if (sp >= 0) ids[n++] = sp; }
    for (const char *c = text; *c;) {
        const unsigned char lead = (unsigned char)*c;
        int want = lead >= 0xF0 ? 4 : lead >= 0xE0 ? 3 : lead >= 0xC0 ? 2 : 1, got = 0;
        while (got < want && c[got]) got++;
        const int id = table_get(&t->pieces, c, got);
        if (id >= 0) ids[n++] = id;
        else for (int k = 0; k < got; k++) ids[n++] = (unsigned char)c[k] + 3;
        c += got;
    }
    char *buf = ember_xmalloc((size_t)t->max_len * 2 + 2, "merge buffer");
    for (;;) {
        float best = -1e30f;
        int at = -1, merged = -1;
        for (int i = 0; i + 1 < n; i++) {
            const int la = t->plen[ids[i]], lb = t->plen[ids[i + 1]];
            if (la + lb > t->max_len * 2) continue;
            memcpy(buf, t->piece[ids[i]], (size_t)la);
            memcpy(buf + la, t->piece[ids[i + 1]], (size_t)lb);
            const int id = table_get(&t->pieces, buf, la + lb);
            if (id >= 0 && t->score[id] > best) { best = t->score[id]; at = i; merged = id; }
        }
        if (at < 0) break;
        ids[at] = merged;
        memmove(&ids[at + 1], &ids[at + 2], sizeof(int) * (size_t)(n - at - 2));
        n--;
    }
    free(buf);
    *out = ids;
    return n;
}

static const char *sp_decode(EmberTokenizer *t, int prev, int tok) {
    if (tok < 0 || tok >= t->vocab) return "";
    const char *p = t->piece[tok];
    if (prev == t->bos && p[0] == ' ') p++;
    unsigned byte;
    if (sscanf(p, "<0x%02X>", &byte) == 1) return t->bytechar[byte & 255];
    return p;
}

/* --------------------------------------------------------------- BPE ---- */
static int is_ws(unsigned char c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n' || c == '\f' || c == '\v'; }
static int is_alpha(unsigned char c) { return ((c | 32) >= 'a' && (c | 32) <= 'z') || c >= 0x80; }
static int is_num(unsigned char c) { return c >= '0' && c <= '9'; }

/* Length of the next pre-token at s (n bytes left); the reference's regex
 * approximation (src/tokenizer.c:248-303). */
static int pretoken(const char *s, int n) {
    const unsigned char c0 = (unsigned char)s[0];
    if (c0 == '\'' && n >= 2) {                     /* contractions */
        const unsigned char c1 = (unsigned char)s[1] | 32;
        if (c1 == 's' || c1 == 't' || c1 == 'm' || c1 == 'd') return 2;
        if (n >= 3) {
            const unsigned char c2 = (unsigned char)s[2] | 32;
            if ((c1 == 'r' && c2 == 'e') || (c1 == 'v' && c2 == 'e') || (c1 == 'l' && c2 == 'l')) return 3;
        }
    }
    {   /* [^\r\n\p{L}\p{N}]?\p{L}+ */
        const int lead = c0 != '\r' && c0 != '\n' && !is_alpha(c0) && !is_num(c0);
        int i = (lead && n >= 2 && is_alpha((unsigned char)s[1])) ? 1 : 0;
        if (i < n && is_alpha((unsigned char)s[i])) {
            while (i < n && is_alpha((unsigned char)s[i])) i++;
            return i;
        }
    }
    if (is_num(c0)) return 1;                        /* one digit */
    {   /*  ?[^\s\p{L}\p{N}]+[\r\n]* */
        int i = c0 == ' ' ? 1 : 0;
        if (i < n) {
            const unsigned char c = (unsigned char)s[i];
            if (!is_ws(c) && !is_alpha(c) && !is_num(c)) {
                while (i < n && !is_ws((unsigned char)s[i]) && !is_alpha((unsigned char)s[i]) && !is_num((unsigned char)s[i])) i++;
                while (i < n && (s[i] == '\r' || s[i] == '\n')) i++;
                return i;
            }
        }
    }
    if (is_ws(c0)) {                                 /* whitespace runs */
        int j = 0, nl = -1;
        while (j < n && is_ws((unsigned char)s[j])) { if (s[j] == '\n' || s[j] == '\r') nl = j; j++; }
        if (nl >= 0) return nl + 1;
        if (j >= n) return j;
        return j > 1 ? j - 1 : 1;
    }
    return 1;
}

static int bpe_piece(EmberTokenizer *t, const char *bl, int len, int *out, int cap) {
    int start[512], size[512], ns = 0;
    for (int i = 0; i < len && ns < 512;) {
        int cp;
        const int adv = utf8_get(bl + i, &cp);
        start[ns] = i; size[ns] = adv; ns++;
        i += adv;
    }
    char key[512];
    for (;;) {
        int best = -1, best_rank = 0x7fffffff;
        for (int i = 0; i + 1 < ns; i++) {
            const int la = size[i], lb = size[i + 1];
            if (la + lb + 1 > (int)sizeof key) continue;
            memcpy(key, bl + start[i], (size_t)la);
            key[la] = 0;
            memcpy(key + la + 1, bl + start[i + 1], (size_t)lb);
            const int r = table_get(&t->ranks, key, la + lb + 1);
            if (r >= 0 && r < best_rank) { best_rank = r; best = i; }
        }
        if (best < 0) break;
        size[best] += size[best + 1];
        memmove(&start[best + 1], &start[best + 2], sizeof(int) * (size_t)(ns - best - 2));
        memmove(&size[best + 1], &size[best + 2], sizeof(int) * (size_t)(ns - best - 2));
        ns--;
    }
    int n = 0;
    for (int i = 0; i < ns && n < cap; i++) {
        const int id = table_get(&t->ids, bl + start[i], size[i]);
        if (id >= 0) out[n++] = id;
    }
    return n;
}

static int bpe_encode(EmberTokenizer *t, const char *text, int add_bos, int **out) {
    const int n_text = (int)strlen(text);
    int cap = n_text + 16, n = 0;
    int *ids = ember_xmalloc(sizeof(int) * (size_t)cap, "token ids");
    if (add_bos && t->bos >= 0) ids[n++] = t->bos;
    char *bl = ember_xmalloc((size_t)n_text * 4 + 8, "byte-level text");
    int piece_ids[512];
    for (int i = 0; i < n_text;) {
        int sp = -1;
        for (int k = 0; k < t->n_special && sp < 0; k++)
            if (t->sp_len[k] <= n_text - i && !memcmp(text + i, t->sp_str[k], (size_t)t->sp_len[k])) sp = k;
        if (sp >= 0) {
            if (n + 1 >= cap) { cap *= 2; ids = ember_xrealloc(ids, sizeof(int) * (size_t)cap, "token ids"); }
            ids[n++] = t->sp_id[sp];
            i += t->sp_len[sp];
            continue;
        }
        const int plen = pretoken(text + i, n_text - i);
        int bl_len = 0;
        for (int k = 0; k < plen; k++) {
            const unsigned char b = (unsigned char)text[i + k];
            memcpy(bl + bl_len, t->b2u[b], (size_t)t->b2u_len[b]);
            bl_len += t->b2u_len[b];
        }
        const int got = bpe_piece(t, bl, bl_len, piece_ids, 512);
        if (n + got >= cap) { cap = (n + got) * 2; ids = ember_xrealloc(ids, sizeof(int) * (size_t)cap, "token ids"); }
        memcpy(ids + n, piece_ids, sizeof(int) * (size_t)got);
        n += got;
        i += plen;
    }
    free(bl);
    *out = ids;
    return n;
}

static const char *bpe_decode(EmberTokenizer *t, int tok) {
    if (tok < 0 || tok >= t->vocab || !t->str[tok]) return "";
    const char *s = (const char *)t->str[tok];
    const int len = t->slen[tok];
    if (t->special[tok]) {
        const int k = len < 511 ? len : 511;
        memcpy(t->dec, s, (size_t)k);
        t->dec[k] = 0;
        return t->dec;
    }
    int o = 0;
    for (int i = 0; i < len && o < 511;) {
        int cp;
        i += utf8_get(s + i, &cp);
        const int b = (cp >= 0 && cp < 512) ? t->u2b[cp] : -1;
        t->dec[o++] = (char)(b >= 0 ? b : '?');
    }
    t->dec[o] = 0;
    return t->dec;
}

int ember_encode(EmberTokenizer *t, const char *text, int add_bos, int **out_ids) {
    return t->type == EMBER_TOK_BYTE_BPE ? bpe_encode(t, text, add_bos, out_ids)
                                         : sp_encode(t, text, add_bos, out_ids);
}

const char *ember_decode(EmberTokenizer *t, int prev_tok, int tok) {
    return t->type == EMBER_TOK_BYTE_BPE ? bpe_decode(t, tok) : sp_decode(t, prev_tok, tok);
}
